"""prana_amd — MI355X (gfx950) backend for the inference hot path of
pariharshyamu/Prana.

Host-side mirror of the reference's interface (prana-kernels / prana-model) over
the C ABI of libprana_hip (include/prana_hip.h): Matrix ~ Linear, Model ~
prana_model::Model, Cache ~ KvCache, and forward / prefill / forward_batch /
generate / generate_speculative with the reference's argument meanings.

All compute runs in the HIP library; there is no CPU fallback in this package.
"""
import ctypes as C

import numpy as np

from . import _lib
from ._lib import GenStats, PranaConfig, PranaError, check, check_synth, load, load_synth

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 8, 12, 14
GGML_NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q6_K: "Q6_K"}


def _ptr(a):
    return C.c_void_p(a.ctypes.data) if a is not None else None


def init():
    check(load().prana_init(0))


class DeviceArray:
    """A device buffer holding one numpy-typed array (test/bench plumbing)."""

    def __init__(self, shape, dtype):
        init()
        self.shape = tuple(shape) if isinstance(shape, (tuple, list)) else (shape,)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        p = C.c_void_p()
        check(load().prana_device_alloc(self.nbytes, C.byref(p)))
        self.ptr = p

    @classmethod
    def from_host(cls, a):
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        if d.nbytes:
            check(load().prana_memcpy_h2d(d.ptr, _ptr(a), d.nbytes))
        return d

    def to_host(self):
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            check(load().prana_memcpy_d2h(_ptr(out), self.ptr, self.nbytes))
        return out

    def free(self):
        if self.ptr is not None and self.ptr.value:
            load().prana_device_free(self.ptr)
        self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def ggml_nbytes(ggml_type, n_elems):
    return int(load().prana_ggml_nbytes(ggml_type, n_elems))


# Fixture encoders (libprana_synth.so, host code): synthetic weights for the
# tests and the benchmark. The product library only uploads tensor bytes.
def quantize_tensor(ggml_type, x):
    """Encode an f32 [rows, cols] array into ggml block bytes."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    out = np.zeros(ggml_nbytes(ggml_type, rows * cols), np.uint8)
    check_synth(load_synth().prana_quantize_tensor(ggml_type, _ptr(x), rows, cols, _ptr(out), out.nbytes))
    return out


def synth_normal(seed, sigma, n):
    out = np.empty(n, np.float32)
    check_synth(load_synth().prana_synth_normal(seed, sigma, _ptr(out), n))
    return out


def synth_tensor(ggml_type, rows, cols, seed, sigma):
    out = np.empty(ggml_nbytes(ggml_type, rows * cols), np.uint8)
    check_synth(load_synth().prana_synth_tensor(ggml_type, rows, cols, seed, sigma, _ptr(out), out.nbytes))
    return out


class Matrix:
    """A device-resident weight matrix (Linear / QuantMatrix / KQuantMatrix)."""

    def __init__(self, ggml_type, rows, cols, raw):
        init()
        raw = np.ascontiguousarray(raw)
        h = C.c_void_p()
        check(load().prana_mat_create(ggml_type, rows, cols, _ptr(raw), raw.nbytes, C.byref(h)))
        self.h, self.rows, self.cols, self.ggml_type = h, rows, cols, ggml_type

    @classmethod
    def q8_parts(cls, q, scales):
        """QuantMatrix::from_parts (matmul.rs:34-39)."""
        self = cls.__new__(cls)
        init()
        q = np.ascontiguousarray(q, np.int8)
        scales = np.ascontiguousarray(scales, np.float32)
        rows, cols = q.shape
        h = C.c_void_p()
        check(load().prana_mat_create_q8(rows, cols, _ptr(q), _ptr(scales), C.byref(h)))
        self.h, self.rows, self.cols, self.ggml_type = h, rows, cols, None
        return self

    def info(self):
        r, c, k, b = C.c_size_t(), C.c_size_t(), C.c_int(), C.c_size_t()
        check(load().prana_mat_info(self.h, C.byref(r), C.byref(c), C.byref(k), C.byref(b)))
        return {"rows": r.value, "cols": c.value, "kind": k.value, "stream_bytes": b.value}

    def apply(self, x):
        """Linear::apply over n token rows: x [n, cols] f32 -> [n, rows]."""
        x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
        n = x.shape[0]
        dx = DeviceArray.from_host(x)
        dout = DeviceArray((n, self.rows), np.float32)
        check(load().prana_matmul(self.h, dx.ptr, n, dout.ptr, None))
        return dout.to_host()

    def apply_prefill(self, q, sa, sums, x=None):
        """Linear::apply_prefill over already-quantized rows."""
        n = q.shape[0]
        dq, ds, dm = DeviceArray.from_host(q), DeviceArray.from_host(sa), DeviceArray.from_host(sums)
        dx = DeviceArray.from_host(x) if x is not None else None
        dout = DeviceArray((n, self.rows), np.float32)
        check(load().prana_matmul_prefill(self.h, dx.ptr if dx else None, dq.ptr, ds.ptr, dm.ptr, n, dout.ptr, None))
        return dout.to_host()

    def block_sums(self, q, sums):
        n = q.shape[0]
        terms = self.cols // 16 if self.ggml_type == Q6_K else self.cols // 32
        dq, dm = DeviceArray.from_host(q), DeviceArray.from_host(sums)
        dout = DeviceArray((n, self.rows, terms), np.int32)
        check(load().prana_matmul_block_sums(self.h, dq.ptr, dm.ptr, n, dout.ptr, None))
        return dout.to_host()

    def embed_rows(self, tokens, scale=1.0):
        t = DeviceArray.from_host(np.asarray(tokens, np.uint32))
        dout = DeviceArray((len(tokens), self.cols), np.float32)
        check(load().prana_embed_rows(self.h, t.ptr, len(tokens), scale, dout.ptr, None))
        return dout.to_host()

    def __del__(self):
        try:
            if getattr(self, "h", None) is not None:
                load().prana_mat_destroy(self.h)
                self.h = None
        except Exception:
            pass


# ---------------------------------------------------------------- kernels
def quantize_acts(x):
    """quantize_acts (matmul.rs:105-127) of each row of x."""
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    n, k = x.shape
    dx = DeviceArray.from_host(x)
    q, s, m = DeviceArray((n, k), np.int8), DeviceArray((n, k // 32), np.float32), DeviceArray((n, k // 32), np.int32)
    check(load().prana_quantize_acts(dx.ptr, n, k, q.ptr, s.ptr, m.ptr, None))
    return q.to_host(), s.to_host(), m.to_host()


def quantize_q8(w):
    """quantize_q8 (matmul.rs:61-84) of a dense f32 matrix: (q, scales)."""
    w = np.ascontiguousarray(np.atleast_2d(w), np.float32)
    rows, cols = w.shape
    dw = DeviceArray.from_host(w)
    q, s = DeviceArray((rows, cols), np.int8), DeviceArray((rows, cols // 32), np.float32)
    check(load().prana_quantize_q8(dw.ptr, rows, cols, q.ptr, s.ptr, None))
    return q.to_host(), s.to_host()


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    rows, dim = x.shape
    dx, dw, do = DeviceArray.from_host(x), DeviceArray.from_host(np.asarray(w, np.float32)), DeviceArray(x.shape,
                                                                                                     np.float32)
    check(load().prana_rmsnorm(dx.ptr, dw.ptr, rows, dim, eps, do.ptr, None))
    return do.to_host()


def _inplace(fn, x):
    x = np.ascontiguousarray(x, np.float32)
    d = DeviceArray.from_host(x)
    check(fn(d.ptr, x.size, None))
    return d.to_host()


def silu(x):
    return _inplace(load().prana_silu, x)


def gelu_tanh(x):
    return _inplace(load().prana_gelu_tanh, x)


def act_mul(g, u, gelu=False):
    """g = act(g) * u (infer.rs:193-199), act = silu or gelu_tanh."""
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    assert g.shape == u.shape
    dg, du = DeviceArray.from_host(g), DeviceArray.from_host(u)
    fn = load().prana_gelu_tanh_mul if gelu else load().prana_silu_mul
    check(fn(dg.ptr, du.ptr, g.size, None))
    return dg.to_host()


def add_bias(x, bias):
    """add_bias (infer.rs:73-79) on every row of x."""
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    b = np.ascontiguousarray(bias, np.float32)
    assert b.shape == (x.shape[1],)
    dx, db = DeviceArray.from_host(x), DeviceArray.from_host(b)
    check(load().prana_add_bias(dx.ptr, db.ptr, x.shape[0], x.shape[1], None))
    return dx.to_host()


def softmax(x):
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    d, o = DeviceArray.from_host(x), DeviceArray(x.shape, np.float32)
    check(load().prana_softmax(d.ptr, x.shape[0], x.shape[1], o.ptr, None))
    return o.to_host()


def expf(x):
    x = np.ascontiguousarray(x, np.float32)
    d, o = DeviceArray.from_host(x), DeviceArray(x.shape, np.float32)
    check(load().prana_expf(d.ptr, x.size, o.ptr, None))
    return o.to_host()


def tanhf(x):
    x = np.ascontiguousarray(x, np.float32)
    d, o = DeviceArray.from_host(x), DeviceArray(x.shape, np.float32)
    check(load().prana_tanhf(d.ptr, x.size, o.ptr, None))
    return o.to_host()


def rope(x, pos0, head_dim, theta, neox):
    """rope_interleaved / rope_neox on each row of x at positions pos0 + i."""
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    d = DeviceArray.from_host(x)
    fn = load().prana_rope_neox if neox else load().prana_rope_interleaved
    check(fn(d.ptr, x.shape[0], x.shape[1], pos0, head_dim, theta, None))
    return d.to_host()


def f32_to_f16(x):
    x = np.ascontiguousarray(x, np.float32)
    d, o = DeviceArray.from_host(x), DeviceArray(x.shape, np.uint16)
    check(load().prana_f32_to_f16(d.ptr, x.size, o.ptr, None))
    return o.to_host()


def f16_to_f32(h):
    h = np.ascontiguousarray(h, np.uint16)
    d, o = DeviceArray.from_host(h), DeviceArray(h.shape, np.float32)
    check(load().prana_f16_to_f32(d.ptr, h.size, o.ptr, None))
    return o.to_host()


def kv_write_f16(cache, first_row, kv_stride, src):
    """f16_kv_write on a host copy of the cache; returns the updated cache."""
    dc = DeviceArray.from_host(np.asarray(cache, np.uint16))
    ds = DeviceArray.from_host(np.asarray(src, np.float32))
    check(load().prana_kv_write_f16(dc.ptr, first_row, kv_stride, ds.ptr, ds.shape[0] if ds.shape else 0, None))
    return dc.to_host()


def attention_decode(q, kc, vc, pos, n_heads, n_kv_heads, head_dim):
    dq, dk, dv = (DeviceArray.from_host(np.asarray(q, np.float32)), DeviceArray.from_host(np.asarray(kc, np.uint16)),
                  DeviceArray.from_host(np.asarray(vc, np.uint16)))
    do = DeviceArray((n_heads * head_dim,), np.float32)
    check(load().prana_attention_decode(dq.ptr, dk.ptr, dv.ptr, pos, n_heads, n_kv_heads, head_dim, do.ptr, None))
    return do.to_host()


def attention_verify(q, kc, vc, pos0, seq, n_heads, n_kv_heads, head_dim):
    dq, dk, dv = (DeviceArray.from_host(np.asarray(q, np.float32)), DeviceArray.from_host(np.asarray(kc, np.uint16)),
                  DeviceArray.from_host(np.asarray(vc, np.uint16)))
    do = DeviceArray((seq, n_heads * head_dim), np.float32)
    check(load().prana_attention_verify(dq.ptr, dk.ptr, dv.ptr, pos0, seq, n_heads, n_kv_heads, head_dim, do.ptr,
                                        None))
    return do.to_host()


def attention_decode_splitk(q, kcs, vcs, pos, n_heads, n_kv_heads, head_dim):
    """Split-K flash decoding of len(pos) independent sequences: q [n_seq,
    n_heads*hd] f32, kcs / vcs lists of per-sequence f16 caches (host arrays or
    DeviceArrays), pos[i] the position of sequence i. Within 1e-4 relative of
    attention_decode; not bit-exact."""
    n = len(pos)
    dq = DeviceArray.from_host(np.asarray(q, np.float32).reshape(n, n_heads * head_dim))
    dk = [c if isinstance(c, DeviceArray) else DeviceArray.from_host(np.asarray(c, np.uint16)) for c in kcs]
    dv = [c if isinstance(c, DeviceArray) else DeviceArray.from_host(np.asarray(c, np.uint16)) for c in vcs]
    kp = (C.c_void_p * n)(*[c.ptr.value for c in dk])
    vp = (C.c_void_p * n)(*[c.ptr.value for c in dv])
    ps = (C.c_size_t * n)(*[int(p) for p in pos])
    do = DeviceArray((n, n_heads * head_dim), np.float32)
    check(load().prana_attention_decode_splitk(dq.ptr, kp, vp, ps, n, n_heads, n_kv_heads, head_dim, do.ptr, None))
    return do.to_host()


def attention_decode_splitk_noalloc(q, kcs, vcs, pos, n_heads, n_kv_heads, head_dim):
    """attention_decode_splitk through the allocation-free entry point (the
    library's fixed partial-state array); synchronises after the call."""
    n = len(pos)
    dq = DeviceArray.from_host(np.asarray(q, np.float32).reshape(n, n_heads * head_dim))
    dk = [c if isinstance(c, DeviceArray) else DeviceArray.from_host(np.asarray(c, np.uint16)) for c in kcs]
    dv = [c if isinstance(c, DeviceArray) else DeviceArray.from_host(np.asarray(c, np.uint16)) for c in vcs]
    kp = (C.c_void_p * n)(*[c.ptr.value for c in dk])
    vp = (C.c_void_p * n)(*[c.ptr.value for c in dv])
    ps = (C.c_size_t * n)(*[int(p) for p in pos])
    do = DeviceArray((n, n_heads * head_dim), np.float32)
    check(load().prana_attention_decode_splitk_noalloc(dq.ptr, kp, vp, ps, n, n_heads, n_kv_heads, head_dim, do.ptr,
                                                        None))
    check(load().prana_synchronize())
    return do.to_host()


def attention_prefill(q, k, v, seq, n_heads, n_kv_heads, head_dim):
    dq, dk, dv = (DeviceArray.from_host(np.asarray(q, np.float32)), DeviceArray.from_host(np.asarray(k, np.float32)),
                  DeviceArray.from_host(np.asarray(v, np.float32)))
    do = DeviceArray((seq, n_heads * head_dim), np.float32)
    check(load().prana_attention_prefill(dq.ptr, dk.ptr, dv.ptr, seq, n_heads, n_kv_heads, head_dim, do.ptr, None))
    return do.to_host()


def argmax(logits):
    x = np.ascontiguousarray(np.atleast_2d(logits), np.float32)
    d, o = DeviceArray.from_host(x), DeviceArray((x.shape[0],), np.uint32)
    check(load().prana_argmax(d.ptr, x.shape[0], x.shape[1], o.ptr, None))
    return o.to_host()


# ---------------------------------------------------------------- model
class Model:
    """prana_model::Model over device buffers; tensors attached by GGUF name."""

    def __init__(self, config, tensors=None):
        init()
        self.config = config
        self.cfg = PranaConfig(**config)
        h = C.c_void_p()
        check(load().prana_model_create(C.byref(self.cfg), C.byref(h)))
        self.h = h
        if tensors:
            for name, (ty, dims, raw) in tensors.items():
                self.set_tensor(name, ty, dims, raw)
            self.finalize()

    def set_tensor(self, name, ggml_type, dims, raw):
        raw = np.ascontiguousarray(raw)
        d = (C.c_uint64 * len(dims))(*dims)
        check(load().prana_model_set_tensor(self.h, name.encode(), ggml_type, d, len(dims), _ptr(raw), raw.nbytes))

    def finalize(self):
        check(load().prana_model_finalize(self.h))

    def stream_bytes(self):
        b = C.c_size_t()
        check(load().prana_model_stream_bytes(self.h, C.byref(b)))
        return b.value

    def cache(self, positions):
        return Cache(self, positions)

    def generate(self, prompt, steps, stops=()):
        prompt = np.asarray(prompt, np.uint32)
        stops = np.asarray(stops, np.uint32)
        out = np.zeros(max(steps, 1), np.uint32)
        n = C.c_size_t()
        st = GenStats()
        check(load().prana_generate(self.h, _ptr(prompt), len(prompt), steps, _ptr(stops) if len(stops) else None,
                                    len(stops), _ptr(out), C.byref(n), C.byref(st)))
        return out[: n.value].copy(), st

    def __del__(self):
        try:
            if getattr(self, "h", None) is not None:
                load().prana_model_destroy(self.h)
                self.h = None
        except Exception:
            pass


def _config_dict(cfg):
    return {name: getattr(cfg, name) for name, _ in PranaConfig._fields_}


class Gguf:
    """A parsed GGUF file (gguf.rs:140-264): metadata and tensor directory,
    read on the host by the library (the file is memory-mapped, not copied)."""

    def __init__(self, path=None, data=None):
        h = C.c_void_p()
        if (path is None) == (data is None):
            raise ValueError("give exactly one of path= or data=")
        if path is not None:
            check(load().prana_gguf_open(str(path).encode(), C.byref(h)))
        else:
            buf = np.frombuffer(bytes(data), np.uint8)
            check(load().prana_gguf_open_bytes(_ptr(buf) if buf.size else None, buf.size, C.byref(h)))
        self.h = h

    def counts(self):
        v, nt, nm = C.c_uint32(), C.c_size_t(), C.c_size_t()
        check(load().prana_gguf_counts(self.h, C.byref(v), C.byref(nt), C.byref(nm)))
        return v.value, nt.value, nm.value

    @staticmethod
    def _grow(call):
        """Caller-sized buffer, grown once to the size the library asks for."""
        n = C.c_size_t()
        rc = call(None, 0, C.byref(n))
        if rc != 0 and rc != _lib.ERR_SHORT_BUFFER:
            check(rc)
        buf = C.create_string_buffer(n.value + 1)
        check(call(buf, n.value + 1, C.byref(n)))
        return buf.raw[: n.value]

    def tensor_names(self):
        _, nt, _ = self.counts()
        return [self._grow(lambda b, c, n, i=i: load().prana_gguf_tensor_name(self.h, i, b, c, n)).decode()
                for i in range(nt)]

    def tensor_info(self, name):
        ty, nd, nb = C.c_int(), C.c_int(), C.c_size_t()
        dims = (C.c_uint64 * 8)()
        check(load().prana_gguf_tensor_info(self.h, name.encode(), C.byref(ty), dims, C.byref(nd), C.byref(nb)))
        return ty.value, [dims[i] for i in range(nd.value)], nb.value

    def tensor_bytes(self, name):
        p, nb = C.c_void_p(), C.c_size_t()
        check(load().prana_gguf_tensor_data(self.h, name.encode(), C.byref(p), C.byref(nb)))
        return C.string_at(p, nb.value) if nb.value else b""

    def tensor_f32(self, name):
        """Gguf::tensor_f32: any supported type decoded to f32."""
        n = C.c_size_t()
        rc = load().prana_gguf_tensor_f32(self.h, name.encode(), None, 0, C.byref(n))
        if rc != 0 and rc != _lib.ERR_SHORT_BUFFER:
            check(rc)
        out = np.empty(n.value, np.float32)
        check(load().prana_gguf_tensor_f32(self.h, name.encode(), _ptr(out), out.size, C.byref(n)))
        return out

    def meta_type(self, key):
        t, e = C.c_int(), C.c_int()
        check(load().prana_gguf_meta_type(self.h, key.encode(), C.byref(t), C.byref(e)))
        return t.value, e.value

    def meta_usize(self, key):
        v = C.c_uint64()
        check(load().prana_gguf_meta_u64(self.h, key.encode(), C.byref(v)))
        return v.value

    def meta_f32(self, key):
        v = C.c_float()
        check(load().prana_gguf_meta_f32(self.h, key.encode(), C.byref(v)))
        return v.value

    def meta_str(self, key):
        return self._grow(lambda b, c, n: load().prana_gguf_meta_str(self.h, key.encode(), b, c, n))

    def meta_array_len(self, key):
        n = C.c_size_t()
        check(load().prana_gguf_meta_array_len(self.h, key.encode(), C.byref(n)))
        return n.value

    def meta_array_str(self, key):
        return [self._grow(lambda b, c, n, i=i: load().prana_gguf_meta_array_str(self.h, key.encode(), i, b, c, n))
                for i in range(self.meta_array_len(key))]

    def _array(self, fn, key, dtype):
        n = C.c_size_t()
        rc = fn(self.h, key.encode(), None, 0, C.byref(n))
        if rc != 0 and rc != _lib.ERR_SHORT_BUFFER:
            check(rc)
        out = np.empty(n.value, dtype)
        check(fn(self.h, key.encode(), _ptr(out), out.size, C.byref(n)))
        return out

    def meta_array_f32(self, key):
        return self._array(load().prana_gguf_meta_array_f32, key, np.float32)

    def meta_array_i64(self, key):
        return self._array(load().prana_gguf_meta_array_i64, key, np.int64)

    def model_config(self):
        """The Config load (gguf.rs:340-425) would build from this file."""
        cfg = PranaConfig()
        check(load().prana_gguf_model_config(self.h, C.byref(cfg)))
        return _config_dict(cfg)

    def close(self):
        if getattr(self, "h", None) is not None:
            load().prana_gguf_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def load_gguf(source, precision="f32"):
    """gguf::load (gguf.rs:338-437) without the tokenizer: a finalized device
    Model from a GGUF path, raw bytes or an open Gguf. precision "f32" or "q8"."""
    prec = {"f32": 0, "q8": 1}[precision]
    g = source if isinstance(source, Gguf) else (Gguf(data=source) if isinstance(source, (bytes, bytearray))
                                                  else Gguf(path=source))
    init()
    h = C.c_void_p()
    check(load().prana_model_load_gguf(g.h, prec, C.byref(h)))
    cfg = PranaConfig()
    check(load().prana_model_config(h, C.byref(cfg)))
    m = Model.__new__(Model)
    m.h, m.cfg, m.config = h, cfg, _config_dict(cfg)
    return m


class Tokenizer:
    """prana-model's tokenizers (tokenizer.rs SentencePiece, bpe.rs byte-level
    BPE) in the library, host side. Build with from_gguf / from_llama2c."""

    def __init__(self, handle):
        self.h = handle
        k, n = C.c_int(), C.c_size_t()
        check(load().prana_tokenizer_info(self.h, C.byref(k), C.byref(n)))
        self.kind, self.vocab_size = ("spm", "bpe")[k.value], n.value

    @classmethod
    def from_gguf(cls, g):
        h = C.c_void_p()
        check(load().prana_tokenizer_from_gguf(g.h, C.byref(h)))
        return cls(h)

    @classmethod
    def from_llama2c(cls, data, vocab_size):
        buf = np.frombuffer(bytes(data), np.uint8)
        h = C.c_void_p()
        check(load().prana_tokenizer_from_llama2c(_ptr(buf) if buf.size else None, buf.size, vocab_size, C.byref(h)))
        return cls(h)

    @staticmethod
    def _text(text):
        b = text.encode() if isinstance(text, str) else bytes(text)
        return C.create_string_buffer(b, len(b) + 1), len(b)

    def _ids(self, call):
        n = C.c_size_t()
        rc = call(None, 0, C.byref(n))
        if rc != 0 and rc != _lib.ERR_SHORT_BUFFER:
            check(rc)
        out = (C.c_uint32 * max(n.value, 1))()
        check(call(out, n.value, C.byref(n)))
        return [out[i] for i in range(n.value)]

    def encode(self, text, bos, eos):
        b, n = self._text(text)
        return self._ids(lambda o, c, k: load().prana_tokenizer_encode(self.h, b, n, int(bos), int(eos), o, c, k))

    def encode_prompt(self, text):
        b, n = self._text(text)
        return self._ids(lambda o, c, k: load().prana_tokenizer_encode_prompt(self.h, b, n, o, c, k))

    def decode(self, prev, token):
        n = C.c_size_t()
        rc = load().prana_tokenizer_decode(self.h, prev, token, None, 0, C.byref(n))
        if rc != 0 and rc != _lib.ERR_SHORT_BUFFER:
            check(rc)
        buf = C.create_string_buffer(max(n.value, 1))
        check(load().prana_tokenizer_decode(self.h, prev, token, buf, n.value, C.byref(n)))
        return buf.raw[: n.value]

    def is_stop(self, token):
        v = C.c_int()
        check(load().prana_tokenizer_is_stop(self.h, token, C.byref(v)))
        return bool(v.value)

    def stop_ids(self):
        return self._ids(lambda o, c, k: load().prana_tokenizer_stop_ids(self.h, o, c, k))

    def __del__(self):
        try:
            if getattr(self, "h", None) is not None:
                load().prana_tokenizer_destroy(self.h)
                self.h = None
        except Exception:
            pass


def bpe_pre_tokenize(text):
    """BpeTokenizer::pre_tokenize (bpe.rs:96-139) as a list of strings."""
    b = text.encode()
    buf = C.create_string_buffer(b, len(b) + 1)
    n = C.c_size_t()
    rc = load().prana_bpe_pre_tokenize(buf, len(b), None, 0, C.byref(n))
    if rc != 0 and rc != _lib.ERR_SHORT_BUFFER:
        check(rc)
    bounds = (C.c_size_t * max(2 * n.value, 1))()
    check(load().prana_bpe_pre_tokenize(buf, len(b), bounds, 2 * n.value, C.byref(n)))
    return [b[bounds[2 * i]:bounds[2 * i + 1]].decode() for i in range(n.value)]


def generate_text(model, tokenizer, prompt, steps, sampler=None):
    """generate (infer.rs:696-771) from text: encode_prompt, decode with the
    tokenizer's stop ids, pieces as the reference streams them: (bytes,
    in_prompt) for every prompt transition and generated token."""
    ids = tokenizer.encode_prompt(prompt)
    if not ids:
        raise ValueError("prompt encoded to zero tokens")
    stops = tokenizer.stop_ids()
    if sampler is None:
        out, st = model.generate(ids, steps, stops)
    else:
        out, st = sampler.generate(model, ids, steps, stops)
    max_pos = min(model.config["seq_len"], len(ids) + steps)
    pieces = []
    if 1 < len(ids) <= max_pos:
        pieces += [(tokenizer.decode(a, b), True) for a, b in zip(ids[:-1], ids[1:])]
    elif len(ids) > max_pos:  # all teacher-forced, one step at a time, up to the window
        pieces += [(tokenizer.decode(ids[i], ids[i + 1]), True) for i in range(max_pos - 1)]
    prev = ids[-1]
    for t in out:
        pieces.append((tokenizer.decode(prev, int(t)), False))
        prev = int(t)
    return pieces, st


class Sampler:
    """Sampler (sampler.rs:6-71) on the device: greedy for temp <= 0, else
    temperature sampling with the xorshift64* stream of `seed`."""

    def __init__(self, temp, seed):
        h = C.c_void_p()
        check(load().prana_sampler_create(temp, seed, C.byref(h)))
        self.h, self.temp = h, float(temp)

    @property
    def state(self):
        v = C.c_uint64()
        check(load().prana_sampler_state(self.h, C.byref(v)))
        return v.value

    def next_f32(self):
        v = C.c_float()
        check(load().prana_sampler_next_f32(self.h, C.byref(v)))
        return v.value

    def sample(self, logits):
        init()
        x = DeviceArray.from_host(np.ascontiguousarray(logits, np.float32))
        t = C.c_uint32()
        check(load().prana_sampler_sample(self.h, x.ptr, int(np.prod(x.shape)), C.byref(t), None))
        return t.value

    def generate(self, model, prompt, steps, stops=()):
        prompt = np.asarray(prompt, np.uint32)
        stops = np.asarray(stops, np.uint32)
        out = np.zeros(max(steps, 1), np.uint32)
        n = C.c_size_t()
        st = GenStats()
        check(load().prana_generate_sampled(model.h, _ptr(prompt), len(prompt), steps,
                                            _ptr(stops) if len(stops) else None, len(stops), self.h, _ptr(out),
                                            C.byref(n), C.byref(st)))
        return out[: n.value].copy(), st

    def __del__(self):
        try:
            if getattr(self, "h", None) is not None:
                load().prana_sampler_destroy(self.h)
                self.h = None
        except Exception:
            pass


def sample_pick(probs, r):
    """The bucket walk (sampler.rs:29-36) over probs on the device for a given r."""
    p = DeviceArray.from_host(np.ascontiguousarray(probs, np.float32))
    o = DeviceArray((1,), np.uint32)
    check(load().prana_sample_pick(p.ptr, int(np.prod(p.shape)), r, o.ptr, None))
    return int(o.to_host()[0])


class GraphError(PranaError):
    """GraphError (prana-graph lib.rs:55-63): kind is "UnsetInput",
    "ShapeMismatch" or "NotF32"; node is the unset input or the failing node."""

    KINDS = {1: "UnsetInput", 2: "ShapeMismatch", 3: "NotF32"}

    def __init__(self, msg, code, kind, node):
        super().__init__(msg, code)
        self.kind, self.node = self.KINDS.get(kind, str(kind)), node


class Graph:
    """prana_graph::Graph (lib.rs:25-220) over device buffers: build nodes,
    bind inputs, execute, read outputs. Node ids are plain ints."""

    def __init__(self):
        init()
        h = C.c_void_p()
        check(load().prana_graph_create(C.byref(h)))
        self.h = h

    def _node(self, fn, *args):
        i = C.c_size_t()
        check(fn(self.h, *args, C.byref(i)))
        return i.value

    def input(self, n_tokens):
        return self._node(load().prana_graph_input, n_tokens)

    def matmul_f32(self, x, weight, k, n_rows):
        w = np.ascontiguousarray(weight, np.float32).ravel()
        if w.size != k * n_rows:
            raise ValueError("weight must hold n_rows * k values")
        return self._node(load().prana_graph_matmul_f32, x, _ptr(w), k, n_rows)

    def matmul_q8(self, x, q, scales):
        """A QuantMatrix by its parts (quantize_q8's q [rows, cols], scales [rows, cols/32])."""
        q = np.ascontiguousarray(q, np.int8)
        sc = np.ascontiguousarray(scales, np.float32)
        if sc.shape != (q.shape[0], q.shape[1] // 32):
            raise ValueError("scales must be [rows, cols/32]")
        return self._node(load().prana_graph_matmul_q8, x, q.shape[0], q.shape[1], _ptr(q), _ptr(sc))

    def rmsnorm(self, x, weight, dim, eps):
        w = np.ascontiguousarray(weight, np.float32)
        if w.size != dim:
            raise ValueError("weight must hold dim values")
        return self._node(load().prana_graph_rmsnorm, x, _ptr(w), dim, eps)

    def add(self, a, b):
        return self._node(load().prana_graph_add, a, b)

    def softmax(self, x):
        return self._node(load().prana_graph_softmax, x)

    def rope(self, x, n_heads, head_dim, theta_base):
        return self._node(load().prana_graph_rope, x, n_heads, head_dim, theta_base)

    def attention(self, q, k, v, n_heads, n_kv_heads, head_dim):
        return self._node(load().prana_graph_attention, q, k, v, n_heads, n_kv_heads, head_dim)

    def set_input(self, node, values, shape=None):
        """Tensor::from_f32(shape, values); a DeviceArray is copied on the device."""
        if isinstance(values, DeviceArray):
            shape = tuple(values.shape) if shape is None else tuple(shape)
            sh = (C.c_size_t * max(len(shape), 1))(*shape)
            check(load().prana_graph_set_input_device(self.h, node, values.ptr, sh, len(shape)))
            return
        v = np.ascontiguousarray(values, np.float32)
        shape = v.shape if shape is None else tuple(shape)
        if int(np.prod(shape)) != v.size:
            raise ValueError(f"shape {shape} does not match {v.size} values")
        sh = (C.c_size_t * max(len(shape), 1))(*shape)
        check(load().prana_graph_set_input(self.h, node, _ptr(v) if v.size else None, sh, len(shape)))

    def execute(self):
        kind, node = C.c_int(), C.c_size_t()
        rc = load().prana_graph_execute(self.h, C.byref(kind), C.byref(node))
        if rc != 0:
            msg = load().prana_last_error().decode(errors="replace")
            if kind.value:
                raise GraphError(msg, rc, kind.value, node.value)
            check(rc)

    def reset(self):
        check(load().prana_graph_reset(self.h))

    def shape(self, node):
        sh, nd = (C.c_size_t * 8)(), C.c_int()
        check(load().prana_graph_shape(self.h, node, sh, C.byref(nd)))
        return tuple(sh[i] for i in range(nd.value))

    def output_f32(self, node):
        n = C.c_size_t()
        rc = load().prana_graph_output_f32(self.h, node, None, 0, C.byref(n))
        if rc != 0 and rc != _lib.ERR_SHORT_BUFFER:
            check(rc)
        out = np.empty(n.value, np.float32)
        check(load().prana_graph_output_f32(self.h, node, _ptr(out), out.size, C.byref(n)))
        return out

    def __del__(self):
        try:
            if getattr(self, "h", None) is not None:
                load().prana_graph_destroy(self.h)
                self.h = None
        except Exception:
            pass


def gemv_profile(on, period=1):
    """Time every `period`-th decode-GEMV dispatch while on (dispatch timestamps)."""
    check(load().prana_gemv_profile(max(1, int(period)) if on else 0))


def gemv_profile_read(reset=True):
    n, s, b = C.c_size_t(), C.c_double(), C.c_double()
    check(load().prana_gemv_profile_read(C.byref(n), C.byref(s), C.byref(b), 1 if reset else 0))
    return n.value, s.value, b.value


def gemv_profile_shapes():
    """[(weight bytes per launch, timed launches, seconds)] since the last reset,
    ascending by bytes (read before gemv_profile_read(reset=True))."""
    n = C.c_size_t()
    check(load().prana_gemv_profile_shapes(0, None, None, None, C.byref(n)))
    cap = n.value
    b, l, s = (C.c_size_t * max(cap, 1))(), (C.c_size_t * max(cap, 1))(), (C.c_double * max(cap, 1))()
    check(load().prana_gemv_profile_shapes(cap, b, l, s, C.byref(n)))
    return [(int(b[i]), int(l[i]), float(s[i])) for i in range(min(cap, n.value))]


def generate_speculative(target, draft, prompt, steps, k, stops=()):
    prompt = np.asarray(prompt, np.uint32)
    stops = np.asarray(stops, np.uint32)
    out = np.zeros(max(steps, 1), np.uint32)
    n = C.c_size_t()
    st = GenStats()
    check(load().prana_generate_speculative(target.h, draft.h, _ptr(prompt), len(prompt), steps, k,
                                            _ptr(stops) if len(stops) else None, len(stops), _ptr(out), C.byref(n),
                                            C.byref(st)))
    return out[: n.value].copy(), st


class Cache:
    """KvCache::with_len (infer.rs:37-44)."""

    def __init__(self, model, positions):
        self.model = model
        h = C.c_void_p()
        check(load().prana_cache_create(model.h, positions, C.byref(h)))
        self.h = h
        self.len = min(positions, model.config["seq_len"])

    def forward(self, token, pos, need_logits=True):
        v = self.model.config["vocab_size"]
        logits = np.zeros(v, np.float32)
        check(load().prana_forward(self.model.h, self.h, int(token), pos, 1 if need_logits else 0, _ptr(logits)))
        return logits if need_logits else None

    def prefill(self, tokens):
        t = np.asarray(tokens, np.uint32)
        check(load().prana_prefill(self.model.h, self.h, _ptr(t), len(t)))

    def forward_batch(self, tokens, pos0):
        t = np.asarray(tokens, np.uint32)
        v = self.model.config["vocab_size"]
        logits = np.zeros((len(t), v), np.float32)
        check(load().prana_forward_batch(self.model.h, self.h, _ptr(t), len(t), pos0, _ptr(logits)))
        return logits

    def decode(self, token, pos, n_steps):
        """Greedy decode n_steps tokens feeding `token` at `pos` (ids stay on device)."""
        out = np.zeros(max(n_steps, 1), np.uint32)
        check(load().prana_decode(self.model.h, self.h, int(token), pos, n_steps, _ptr(out)))
        return out[:n_steps]

    def read(self, layer, which, rows):
        kv = self.model.config["n_kv_heads"] * self.model.config["head_dim"]
        out = np.zeros((rows, kv), np.uint16)
        check(load().prana_cache_read(self.h, layer, which, rows, _ptr(out)))
        return out

    def __del__(self):
        try:
            if getattr(self, "h", None) is not None:
                load().prana_cache_destroy(self.h)
                self.h = None
        except Exception:
            pass
