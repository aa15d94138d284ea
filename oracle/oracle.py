"""TEST INFRASTRUCTURE ONLY — ctypes binding of the CPU oracle
(oracle/prana_oracle.c, a C restatement of the reference's scalar tier).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")

_lib = None
c_size, c_int, c_float, c_vp = C.c_size_t, C.c_int, C.c_float, C.c_void_p


class PoConfig(C.Structure):
    _fields_ = [
        ("dim", c_size), ("hidden_dim", c_size), ("n_layers", c_size), ("n_heads", c_size),
        ("n_kv_heads", c_size), ("vocab_size", c_size), ("seq_len", c_size), ("head_dim", c_size),
        ("rope_theta", c_float), ("norm_eps", c_float), ("emb_scale", c_float),
        ("rope_neox", c_int), ("act", c_int),
    ]


class PoStats(C.Structure):
    _fields_ = [("prompt_tokens", c_size), ("generated_tokens", c_size), ("proposed", c_size), ("accepted", c_size)]


_SIGS = {
    "po_f16_to_f32": (c_float, [C.c_uint16]),
    "po_f32_to_f16": (C.c_uint16, [c_float]),
    "po_expf_bits": (None, [C.c_uint32, c_size, c_vp, c_int]),
    "po_tanhf_bits": (None, [C.c_uint32, c_size, c_vp, c_int]),
    "po_f16_to_f32_n": (None, [c_vp, c_size, c_vp]),
    "po_f32_to_f16_n": (None, [c_vp, c_size, c_vp]),
    "po_quantize_acts": (None, [c_vp, c_size, c_vp, c_vp, c_vp]),
    "po_quantize_q8": (None, [c_size, c_size, c_vp, c_vp, c_vp]),
    "po_dot_f32": (c_float, [c_vp, c_vp, c_size]),
    "po_dequant_q40_block": (None, [c_vp, c_vp]),
    "po_dequant_q4k_block": (None, [c_vp, c_vp]),
    "po_dequant_q6k_block": (None, [c_vp, c_vp]),
    "po_q4k_scale_min": (None, [c_int, c_vp, C.POINTER(c_float), C.POINTER(c_float)]),
    "po_mat_f32": (c_vp, [c_size, c_size, c_vp]),
    "po_mat_q8_parts": (c_vp, [c_size, c_size, c_vp, c_vp]),
    "po_mat_from_ggml": (c_vp, [c_int, c_size, c_size, c_vp, c_size]),
    "po_mat_free": (None, [c_vp]),
    "po_matmul": (None, [c_vp, c_vp, c_size, c_vp]),
    "po_matmul_prefill": (None, [c_vp, c_vp, c_vp, c_vp, c_vp, c_size, c_vp]),
    "po_mat_row_block_isums": (c_size, [c_vp, c_vp, c_vp, c_size, c_vp]),
    "po_mat_row_f32": (None, [c_vp, c_size, c_vp]),
    "po_set_threads": (None, [c_int]),
    "po_set_tier": (c_int, [c_int, c_int]),
    "po_tier_name": (C.c_char_p, []),
    "po_rmsnorm": (None, [c_vp, c_vp, c_size, c_size, c_float, c_vp]),
    "po_silu": (None, [c_vp, c_size]),
    "po_gelu_tanh": (None, [c_vp, c_size]),
    "po_softmax": (None, [c_vp, c_size, c_vp]),
    "po_rope": (None, [c_vp, c_size, c_size, c_size, c_float]),
    "po_rope_interleaved": (None, [c_vp, c_size, c_size, c_size, c_float]),
    "po_rope_neox": (None, [c_vp, c_size, c_size, c_size, c_float]),
    "po_f16_kv_write": (None, [c_vp, c_size, c_size, c_vp, c_size]),
    "po_attention_decode": (None, [c_vp, c_vp, c_vp, c_size, c_size, c_size, c_size, c_vp]),
    "po_attention_verify": (None, [c_vp, c_vp, c_vp, c_size, c_size, c_size, c_size, c_size, c_vp]),
    "po_attention": (None, [c_vp, c_vp, c_vp, c_size, c_size, c_size, c_size, c_vp]),
    "po_model_new": (c_vp, [C.POINTER(PoConfig)]),
    "po_model_free": (None, [c_vp]),
    "po_model_set_linear": (None, [c_vp, c_size, c_int, c_vp]),
    "po_model_set_vec": (None, [c_vp, c_size, c_int, c_vp, c_size]),
    "po_model_set_rms_final": (None, [c_vp, c_vp, c_size]),
    "po_model_set_embedding": (c_int, [c_vp, c_int, c_vp, c_size]),
    "po_model_set_wcls": (None, [c_vp, c_vp]),
    "po_cache_new": (c_vp, [c_vp, c_size]),
    "po_cache_free": (None, [c_vp]),
    "po_cache_k": (c_vp, [c_vp, c_size]),
    "po_cache_v": (c_vp, [c_vp, c_size]),
    "po_cache_len": (c_size, [c_vp]),
    "po_forward": (None, [c_vp, c_vp, C.c_uint32, c_size, c_int, c_vp]),
    "po_prefill": (None, [c_vp, c_vp, c_vp, c_size]),
    "po_forward_batch": (None, [c_vp, c_vp, c_vp, c_size, c_size, c_vp]),
    "po_argmax": (C.c_uint32, [c_vp, c_size]),
    "po_generate": (c_size, [c_vp, c_vp, c_size, c_size, c_vp, c_size, c_vp, C.POINTER(PoStats)]),
    "po_xorshift_seed": (C.c_uint64, [C.c_uint64]),
    "po_xorshift_next_f32": (c_float, [C.POINTER(C.c_uint64)]),
    "po_sample_pick": (C.c_uint32, [c_vp, c_size, c_float]),
    "po_sampler_sample": (C.c_uint32, [c_float, C.POINTER(C.c_uint64), c_vp, c_size]),
    "po_generate_sampled": (c_size, [c_vp, c_vp, c_size, c_size, c_vp, c_size, c_float, C.POINTER(C.c_uint64),
                                     c_vp]),
    "po_generate_speculative": (c_size, [c_vp, c_vp, c_vp, c_size, c_size, c_size, c_vp, c_size, c_vp,
                                         C.POINTER(PoStats)]),
}

SLOTS = {"attn_q": 0, "attn_k": 1, "attn_v": 2, "attn_output": 3, "ffn_gate": 4, "ffn_down": 5, "ffn_up": 6}
VSLOTS = {"attn_norm": 7, "ffn_norm": 8, "attn_q.bias": 9, "attn_k.bias": 10, "attn_v.bias": 11}


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        for n, (r, a) in _SIGS.items():
            f = getattr(L, n)
            f.restype = r
            f.argtypes = a
        _lib = L
        threads = int(os.environ.get("PRANA_ORACLE_THREADS", min(16, os.cpu_count() or 1)))
        L.po_set_threads(threads)
    return _lib


def P(a):
    return C.c_void_p(a.ctypes.data) if a is not None else None


def f16_to_f32(h):
    return lib().po_f16_to_f32(int(h))


def f32_to_f16(x):
    return lib().po_f32_to_f16(float(x))


def f16_to_f32_n(h):
    h = np.ascontiguousarray(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().po_f16_to_f32_n(P(h), h.size, P(out))
    return out


def f32_to_f16_n(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().po_f32_to_f16_n(P(x), x.size, P(out))
    return out


def expf_bits(base, n, threads=16):
    out = np.empty(n, np.float32)
    lib().po_expf_bits(base, n, P(out), threads)
    return out


def tanhf_bits(base, n, threads=16):
    out = np.empty(n, np.float32)
    lib().po_tanhf_bits(base, n, P(out), threads)
    return out


def quantize_acts(x):
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    n, k = x.shape
    q = np.zeros((n, k), np.int8)
    s = np.zeros((n, k // 32), np.float32)
    m = np.zeros((n, k // 32), np.int32)
    for t in range(n):
        lib().po_quantize_acts(P(x[t]), k, P(q[t]), P(s[t]), P(m[t]))
    return q, s, m


def quantize_q8(w):
    w = np.ascontiguousarray(w, np.float32)
    r, c = w.shape
    q = np.zeros((r, c), np.int8)
    s = np.zeros((r, c // 32), np.float32)
    lib().po_quantize_q8(r, c, P(w), P(q), P(s))
    return q, s


class Mat:
    def __init__(self, h, rows, cols):
        if not h:
            raise ValueError("oracle: matrix rejected (shape not block-aligned?)")
        self.h, self.rows, self.cols, self.owned = h, rows, cols, True

    @classmethod
    def from_ggml(cls, ty, rows, cols, raw):
        raw = np.ascontiguousarray(raw)
        return cls(lib().po_mat_from_ggml(ty, rows, cols, P(raw), raw.nbytes), rows, cols)

    @classmethod
    def f32(cls, w):
        w = np.ascontiguousarray(w, np.float32)
        return cls(lib().po_mat_f32(w.shape[0], w.shape[1], P(w)), w.shape[0], w.shape[1])

    @classmethod
    def q8_parts(cls, q, s):
        q = np.ascontiguousarray(q, np.int8)
        s = np.ascontiguousarray(s, np.float32)
        return cls(lib().po_mat_q8_parts(q.shape[0], q.shape[1], P(q), P(s)), q.shape[0], q.shape[1])

    def apply(self, x):
        x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
        out = np.zeros((x.shape[0], self.rows), np.float32)
        lib().po_matmul(self.h, P(x), x.shape[0], P(out))
        return out

    def apply_prefill(self, q, s, m, x=None):
        n = q.shape[0]
        out = np.zeros((n, self.rows), np.float32)
        xx = np.ascontiguousarray(x, np.float32) if x is not None else None
        lib().po_matmul_prefill(self.h, P(xx), P(np.ascontiguousarray(q)), P(np.ascontiguousarray(s)),
                                P(np.ascontiguousarray(m)), n, P(out))
        return out

    def row_isums(self, q, m, r, terms):
        out = np.zeros(terms, np.int32)
        n = lib().po_mat_row_block_isums(self.h, P(np.ascontiguousarray(q)), P(np.ascontiguousarray(m)), r, P(out))
        return out[:n]

    def row_f32(self, r):
        out = np.zeros(self.cols, np.float32)
        lib().po_mat_row_f32(self.h, r, P(out))
        return out

    def release(self):
        """Hand ownership to a model (po_model_set_linear frees it)."""
        self.owned = False
        return self.h

    def __del__(self):
        try:
            if self.owned and self.h:
                lib().po_mat_free(self.h)
        except Exception:
            pass


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    out = np.zeros_like(x)
    lib().po_rmsnorm(P(x), P(np.ascontiguousarray(w, np.float32)), x.shape[0], x.shape[1], eps, P(out))
    return out


def silu(x):
    x = np.array(x, np.float32, copy=True)
    lib().po_silu(P(x), x.size)
    return x


def gelu_tanh(x):
    x = np.array(x, np.float32, copy=True)
    lib().po_gelu_tanh(P(x), x.size)
    return x


def softmax(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros_like(x)
    lib().po_softmax(P(x), x.size, P(out))
    return out


def rope_interleaved(x, pos, head_dim, theta):
    x = np.array(x, np.float32, copy=True)
    lib().po_rope_interleaved(P(x), x.size, pos, head_dim, theta)
    return x


def rope_neox(x, pos, head_dim, theta):
    x = np.array(x, np.float32, copy=True)
    lib().po_rope_neox(P(x), x.size, pos, head_dim, theta)
    return x


def rope_batch(x, seq, n_heads, head_dim, theta):
    x = np.array(x, np.float32, copy=True)
    lib().po_rope(P(x), seq, n_heads, head_dim, theta)
    return x


def f16_kv_write(cache, first_row, kv_stride, src):
    cache = np.array(cache, np.uint16, copy=True)
    src = np.ascontiguousarray(src, np.float32)
    lib().po_f16_kv_write(P(cache), first_row, kv_stride, P(src), src.size)
    return cache


def attention_decode(q, kc, vc, pos, nh, nkv, hd):
    out = np.zeros(nh * hd, np.float32)
    lib().po_attention_decode(P(np.ascontiguousarray(q, np.float32)), P(np.ascontiguousarray(kc, np.uint16)),
                              P(np.ascontiguousarray(vc, np.uint16)), pos, nh, nkv, hd, P(out))
    return out


def attention_verify(q, kc, vc, pos0, seq, nh, nkv, hd):
    out = np.zeros((seq, nh * hd), np.float32)
    lib().po_attention_verify(P(np.ascontiguousarray(q, np.float32)), P(np.ascontiguousarray(kc, np.uint16)),
                              P(np.ascontiguousarray(vc, np.uint16)), pos0, seq, nh, nkv, hd, P(out))
    return out


def attention(q, k, v, seq, nh, nkv, hd):
    out = np.zeros((seq, nh * hd), np.float32)
    lib().po_attention(P(np.ascontiguousarray(q, np.float32)), P(np.ascontiguousarray(k, np.float32)),
                       P(np.ascontiguousarray(v, np.float32)), seq, nh, nkv, hd, P(out))
    return out


def argmax(v):
    v = np.ascontiguousarray(v, np.float32)
    return lib().po_argmax(P(v), v.size)


class Model:
    """The oracle model, built from the same {name: (ggml_type, dims, bytes)} as the GPU model."""

    def __init__(self, config, tensors):
        """tensors: {name: (ggml_type, dims, bytes)}; a matrix may also be a
        ready Mat (e.g. Mat.q8_parts of quantize_q8, Precision::Q8)."""
        self.config = config
        self.cfg = PoConfig(**config)
        self.h = lib().po_model_new(C.byref(self.cfg))
        for name, v in tensors.items():
            if isinstance(v, Mat):
                if name == "output.weight":
                    lib().po_model_set_wcls(self.h, v.release())
                else:
                    _, li, rest = name.split(".", 2)
                    lib().po_model_set_linear(self.h, int(li), SLOTS[rest[: -len(".weight")]], v.release())
                continue
            ty, dims, raw = v
            raw = np.ascontiguousarray(raw)
            if name == "token_embd.weight":
                if lib().po_model_set_embedding(self.h, ty, P(raw), raw.nbytes) != 0:
                    raise ValueError("oracle: bad embedding")
            elif name == "output.weight":
                m = Mat.from_ggml(ty, dims[1], dims[0], raw)
                lib().po_model_set_wcls(self.h, m.release())
            elif name == "output_norm.weight":
                f = raw.view(np.float32)
                lib().po_model_set_rms_final(self.h, P(f), f.size)
            else:
                assert name.startswith("blk.")
                _, li, rest = name.split(".", 2)
                li = int(li)
                key = rest[: -len(".weight")] if rest.endswith(".weight") else rest
                if key in SLOTS:
                    m = Mat.from_ggml(ty, dims[1], dims[0], raw)
                    lib().po_model_set_linear(self.h, li, SLOTS[key], m.release())
                else:
                    f = np.ascontiguousarray(raw).view(np.float32)
                    lib().po_model_set_vec(self.h, li, VSLOTS[key], P(f), f.size)

    def cache(self, positions):
        return Cache(self, positions)

    def generate(self, prompt, steps, stops=()):
        prompt = np.asarray(prompt, np.uint32)
        stops = np.asarray(stops, np.uint32)
        out = np.zeros(max(steps, 1), np.uint32)
        st = PoStats()
        n = lib().po_generate(self.h, P(prompt), len(prompt), steps, P(stops) if len(stops) else None, len(stops),
                              P(out), C.byref(st))
        return out[:n].copy(), st

    def __del__(self):
        try:
            lib().po_model_free(self.h)
        except Exception:
            pass


def generate_speculative(target, draft, prompt, steps, k, stops=()):
    prompt = np.asarray(prompt, np.uint32)
    stops = np.asarray(stops, np.uint32)
    out = np.zeros(max(steps, 1), np.uint32)
    st = PoStats()
    n = lib().po_generate_speculative(target.h, draft.h, P(prompt), len(prompt), steps, k,
                                      P(stops) if len(stops) else None, len(stops), P(out), C.byref(st))
    return out[:n].copy(), st


class Cache:
    def __init__(self, model, positions):
        self.model = model
        self.h = lib().po_cache_new(model.h, positions)
        self.len = lib().po_cache_len(self.h)
        self.kv = model.config["n_kv_heads"] * model.config["head_dim"]

    def forward(self, token, pos, need_logits=True):
        logits = np.zeros(self.model.config["vocab_size"], np.float32)
        lib().po_forward(self.model.h, self.h, int(token), pos, 1 if need_logits else 0, P(logits))
        return logits if need_logits else None

    def prefill(self, tokens):
        t = np.asarray(tokens, np.uint32)
        lib().po_prefill(self.model.h, self.h, P(t), len(t))

    def forward_batch(self, tokens, pos0):
        t = np.asarray(tokens, np.uint32)
        out = np.zeros((len(t), self.model.config["vocab_size"]), np.float32)
        lib().po_forward_batch(self.model.h, self.h, P(t), len(t), pos0, P(out))
        return out

    def read(self, layer, which, rows):
        ptr = (lib().po_cache_v if which else lib().po_cache_k)(self.h, layer)
        buf = (C.c_uint16 * (rows * self.kv)).from_address(ptr)
        return np.frombuffer(buf, np.uint16).reshape(rows, self.kv).copy()

    def __del__(self):
        try:
            lib().po_cache_free(self.h)
        except Exception:
            pass


class Sampler:
    """Sampler (sampler.rs:6-71): greedy for temp <= 0, else temperature
    sampling with the xorshift64* stream of `seed`."""

    def __init__(self, temp, seed):
        self.temp = float(temp)
        self.state = C.c_uint64(lib().po_xorshift_seed(seed))

    def next_f32(self):
        return lib().po_xorshift_next_f32(C.byref(self.state))

    def sample(self, logits):
        x = np.ascontiguousarray(logits, np.float32)
        return int(lib().po_sampler_sample(self.temp, C.byref(self.state), P(x), x.size))


def sample_pick(probs, r):
    x = np.ascontiguousarray(probs, np.float32)
    return int(lib().po_sample_pick(P(x), x.size, r))


def generate_sampled(model, prompt, steps, sampler, stops=()):
    prompt = np.asarray(prompt, np.uint32)
    stops = np.asarray(stops, np.uint32)
    out = np.zeros(max(steps, 1), np.uint32)
    n = lib().po_generate_sampled(model.h, P(prompt), len(prompt), steps, P(stops) if len(stops) else None, len(stops),
                                  sampler.temp, C.byref(sampler.state), P(out))
    return out[:n].copy()


def set_tier(tier, threads=0):
    """1: the reference's timed SIMD tier on its persistent pool (bench.py's
    cpu_baseline); 0: the scalar tier, the parity oracle. Returns the pool size."""
    return lib().po_set_tier(int(tier), int(threads))


def tier_name():
    return lib().po_tier_name().decode()
