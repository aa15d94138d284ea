"""GGUF byte writer for the loader's fixtures (test infrastructure).

Writes the container exactly as the reference reads it (gguf.rs:157-196):
magic "GGUF", version, tensor count, metadata count, typed key/value pairs
(value types 0..12, gguf.rs:102-130), the tensor directory (name, n_dims,
dims in ggml order, ggml type, offset relative to the data section), padding
to the alignment (general.alignment or 32), then each tensor's bytes at its
aligned offset.

`reference_synthetic_model` restates the reference's own test fixture
generator `synthetic_model_gguf` (gguf.rs:566-666): the same xorshift stream,
tensor order, metadata and tokenizer entries, so the bytes are the ones the
reference's loader tests run on.

Run as a script to (re)write the small committed known-answer files under
tests/golden/gguf/.
"""
import os
import struct

import numpy as np

MAGIC = 0x46554747
U8, I8, U16, I16, U32, I32, F32V, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32V: "<f", BOOL: "<B", U64: "<Q",
        I64: "<q", F64: "<d"}
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K = 0, 1, 2, 8, 12, 14


def gstr(b):
    if isinstance(b, str):
        b = b.encode()
    return struct.pack("<Q", len(b)) + b


def value(ty, v, elem=None):
    if ty == STR:
        return gstr(v)
    if ty == ARR:
        out = struct.pack("<IQ", elem, len(v))
        return out + b"".join(value(elem, x) for x in v)
    return struct.pack(_FMT[ty], v)


class Writer:
    def __init__(self, version=3, alignment=32):
        self.version = version
        self.alignment = alignment
        self.kvs = []
        self.tensors = []

    def kv(self, key, ty, v, elem=None):
        self.kvs.append(gstr(key) + struct.pack("<I", ty) + value(ty, v, elem))
        return self

    def kv_raw(self, raw):
        """A hand-assembled entry (for malformed-input cases)."""
        self.kvs.append(raw)
        return self

    def tensor(self, name, dims, ggml_type, data):
        self.tensors.append((name, list(dims), ggml_type, bytes(data)))
        return self

    def to_bytes(self, n_tensors=None, n_kv=None):
        a = self.alignment
        out = bytearray(struct.pack("<IIQQ", MAGIC, self.version,
                                    len(self.tensors) if n_tensors is None else n_tensors,
                                    len(self.kvs) if n_kv is None else n_kv))
        for e in self.kvs:
            out += e
        off = 0
        offsets = []
        for name, dims, ty, data in self.tensors:
            offsets.append(off)
            out += gstr(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
            out += struct.pack("<IQ", ty, off)
            off = (off + len(data) + a - 1) // a * a
        while len(out) % a:
            out.append(0)
        base = len(out)
        for (name, dims, ty, data), o in zip(self.tensors, offsets):
            while len(out) < base + o:
                out.append(0)
            out += data
        return bytes(out)


# ---------------------------------------------------------------- the reference's synthetic model
class XorShift:
    """The fixture stream of gguf.rs:572-583: xorshift64 (12, 25, 27), then
    ((s >> 40) / 2^24 - 0.5) * scale in f32."""

    def __init__(self, state=0xABCDEF12345):
        self.s = state

    def f32s(self, n, scale):
        out = np.empty(n, np.float32)
        s, m = self.s, (1 << 64) - 1
        for i in range(n):
            s ^= s >> 12
            s = (s ^ (s << 25)) & m
            s ^= s >> 27
            out[i] = np.float32(s >> 40) / np.float32(1 << 24) - np.float32(0.5)
        self.s = s
        return (out * np.float32(scale)).astype(np.float32)


def reference_synthetic_model(arch, with_biases, head_dim):
    """synthetic_model_gguf (gguf.rs:566-666). Returns (bytes, tensors) with
    tensors = {name: (dims, f32 array)} in file order."""
    dim, hidden, n_layers, n_heads, vocab, ctx = 32, 64, 2, 2, 48, 16
    q_dim = n_heads * head_dim
    kv_dim = q_dim
    rng = XorShift()
    t = {}
    t["token_embd.weight"] = ([dim, vocab], rng.f32s(vocab * dim, 0.1))
    for i in range(n_layers):
        p = f"blk.{i}."
        t[p + "attn_norm.weight"] = ([dim], rng.f32s(dim, 0.5))
        t[p + "attn_q.weight"] = ([dim, q_dim], rng.f32s(q_dim * dim, 0.1))
        t[p + "attn_k.weight"] = ([dim, kv_dim], rng.f32s(kv_dim * dim, 0.1))
        t[p + "attn_v.weight"] = ([dim, kv_dim], rng.f32s(kv_dim * dim, 0.1))
        t[p + "attn_output.weight"] = ([q_dim, dim], rng.f32s(dim * q_dim, 0.1))
        if with_biases:
            t[p + "attn_q.bias"] = ([q_dim], rng.f32s(q_dim, 0.05))
            t[p + "attn_k.bias"] = ([kv_dim], rng.f32s(kv_dim, 0.05))
            t[p + "attn_v.bias"] = ([kv_dim], rng.f32s(kv_dim, 0.05))
        t[p + "ffn_norm.weight"] = ([dim], rng.f32s(dim, 0.5))
        t[p + "ffn_gate.weight"] = ([dim, hidden], rng.f32s(hidden * dim, 0.1))
        t[p + "ffn_down.weight"] = ([hidden, dim], rng.f32s(dim * hidden, 0.1))
        t[p + "ffn_up.weight"] = ([dim, hidden], rng.f32s(hidden * dim, 0.1))
    t["output_norm.weight"] = ([dim], rng.f32s(dim, 0.5))

    w = Writer(version=3)
    w.kv("general.architecture", STR, arch)
    for k, v in [("embedding_length", dim), ("block_count", n_layers), ("attention.head_count", n_heads),
                 ("attention.head_count_kv", n_heads), ("feed_forward_length", hidden), ("context_length", ctx),
                 ("attention.key_length", head_dim)]:
        w.kv(f"{arch}.{k}", U32, v)
    w.kv("tokenizer.ggml.model", STR, "llama")
    w.kv("tokenizer.ggml.tokens", ARR, [spm_piece(i) for i in range(vocab)], STR)
    w.kv("tokenizer.ggml.scores", ARR, [-1.0] * vocab, F32V)
    for name, (dims, data) in t.items():
        w.tensor(name, dims, GGML_F32, data.tobytes())
    return w.to_bytes(), t


def spm_piece(i):
    """Token i of the synthetic vocabulary (gguf.rs:623-632)."""
    return {0: b"<unk>", 1: b"<s>", 2: b"</s>", 3: b" "}.get(i, bytes([ord("a") + (i - 4) % 26]))


# ---------------------------------------------------------------- the reference's known-answer files
def kat_metadata_f32():
    """parses_metadata_and_f32_tensor (gguf.rs:899-925): two kv, a [2 x 3] f32 tensor 0..5."""
    w = Writer().kv("general.architecture", STR, "llama").kv("llama.block_count", U32, 6)
    return w.tensor("t", [2, 3], GGML_F32, np.arange(6, dtype=np.float32).tobytes()).to_bytes()


def kat_q4_0():
    """q4_0_tensor_loads_natively_packed (gguf.rs:989-1036): one row of 64 as
    two Q4_0 blocks, d = 1.0 with nibbles (j, 15 - j), then d = 0.5, all 0xC."""
    b0 = struct.pack("<H", 0x3C00) + bytes(j | ((15 - j) << 4) for j in range(16))
    b1 = struct.pack("<H", 0x3800) + bytes([0xCC] * 16)
    return Writer().tensor("w", [64, 1], GGML_Q4_0, b0 + b1).to_bytes()


def kat_q8_0():
    """q8_0_tensor_loads_natively_as_quantmatrix (gguf.rs:1038-1071): one
    block, scale 1.0, q[i] = i - 16."""
    blk = struct.pack("<H", 0x3C00) + bytes(((i - 16) & 0xFF) for i in range(32))
    return Writer().tensor("w", [32, 1], GGML_Q8_0, blk).to_bytes()


def q4k_block_known():
    """q4k_block_dequantizes_known_values (gguf.rs:927-953): d = 1, dmin = 0,
    group scales 2 and 3, qs[i] = (i % 16) | ((15 - i % 16) << 4)."""
    b = bytearray(144)
    b[0:2] = struct.pack("<H", 0x3C00)
    b[4], b[5] = 2, 3
    for i in range(32):
        b[16 + i] = (i % 16) | ((15 - i % 16) << 4)
    return bytes(b)


def q4k_block_high_groups():
    """q4k_packed_scale_min_high_groups_unpack (gguf.rs:955-968): group 4 with
    sc = 53, m = 43 packed across bytes; d = dmin = 1, all nibbles 1 in the
    third 32-byte run (groups 4 and 5)."""
    b = bytearray(144)
    b[0:2] = struct.pack("<H", 0x3C00)
    b[2:4] = struct.pack("<H", 0x3C00)
    s = bytearray(12)
    s[8] = (53 & 0xF) | ((43 & 0xF) << 4)
    s[0] = (53 >> 4) << 6
    s[4] = (43 >> 4) << 6
    b[4:16] = s
    for i in range(32):
        b[16 + 64 + i] = 0x01  # low nibble 1 (group 4), high nibble 0 (group 5)
    return bytes(b)


def q6k_block_known():
    """q6k_block_dequantizes_known_values (gguf.rs:970-987): d = 1, all 16
    sub-block scales 1, ql[0] = 5, qh[0] = 2."""
    b = bytearray(210)
    b[192:208] = bytes([1] * 16)
    b[208:210] = struct.pack("<H", 0x3C00)
    b[0] = 5
    b[128] = 2
    return bytes(b)


def kat_kquants():
    w = Writer()
    w.tensor("q4k", [256], GGML_Q4_K, q4k_block_known())
    w.tensor("q4k_hi", [256], GGML_Q4_K, q4k_block_high_groups())
    w.tensor("q6k", [256], GGML_Q6_K, q6k_block_known())
    return w.to_bytes()


def kat_f16():
    """f16_conversion_covers_the_cases (gguf.rs:888-897) as an F16 tensor."""
    halves = [0x0000, 0x3C00, 0xC000, 0x7C00, 0x7E00, 0x0001, 0x3555, 0x8000]
    return Writer().tensor("h", [len(halves)], GGML_F16, struct.pack(f"<{len(halves)}H", *halves)).to_bytes()


KATS = {
    "metadata_f32.gguf": kat_metadata_f32,
    "q4_0.gguf": kat_q4_0,
    "q8_0.gguf": kat_q8_0,
    "kquants.gguf": kat_kquants,
    "f16.gguf": kat_f16,
}

GOLDEN_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gguf")


def main():
    os.makedirs(GOLDEN_DIR, exist_ok=True)
    for name, fn in KATS.items():
        with open(os.path.join(GOLDEN_DIR, name), "wb") as f:
            f.write(fn())
        print("wrote", name)


if __name__ == "__main__":
    main()
