"""Test fixtures restating the reference tests' own synthetic inputs."""
import numpy as np

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 8, 12, 14
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}


def xorshift_bytes(n, seed):
    """kquant.rs:385-395 `pseudo_bytes`: xorshift64* top bytes."""
    s = max(seed, 1)
    out = np.empty(n, np.uint8)
    M = 0xFFFFFFFFFFFFFFFF
    for i in range(n):
        s ^= s >> 12
        s ^= (s << 25) & M
        s ^= s >> 27
        out[i] = ((s * 0x2545F4914F6CDD1D) & M) >> 56
    return out


def pseudo_blocks(ty, rows, cols, seed):
    """Random valid blocks with finite f16 scale fields (kquant.rs:401-417)."""
    bv, bb = BLOCK[ty]
    raw = xorshift_bytes(rows * cols // bv * bb, seed).reshape(-1, bb)
    if ty in (Q4_0, Q8_0):
        raw[:, 0:2] = np.frombuffer(np.uint16(0x2E66).tobytes(), np.uint8)
    elif ty == Q4_K:
        raw[:, 0:2] = np.frombuffer(np.uint16(0x2E66).tobytes(), np.uint8)
        raw[:, 2:4] = np.frombuffer(np.uint16(0x2A66).tobytes(), np.uint8)
    elif ty == Q6_K:
        raw[:, 208:210] = np.frombuffer(np.uint16(0x2E66).tobytes(), np.uint8)
    return raw.reshape(-1).copy()


def sin_row(n, step, phase=0.0):
    i = np.arange(n, dtype=np.float32)
    return np.sin(i * np.float32(step) + np.float32(phase)).astype(np.float32)


def f16(bits):
    return np.array([bits], np.uint16).view(np.float16)[0].astype(np.float32)


# ------------------------------------------------------------ dequant in numpy (independent of the oracle)
def np_dequant(ty, raw, rows, cols):
    bv, bb = BLOCK[ty]
    b = np.asarray(raw, np.uint8).reshape(-1, bb)
    if ty == Q8_0:
        d = b[:, 0:2].copy().view(np.float16).astype(np.float32)
        q = b[:, 2:].view(np.int8).astype(np.float32)
        return (q * d).reshape(rows, cols)
    if ty == Q4_0:
        d = b[:, 0:2].copy().view(np.float16).astype(np.float32)
        qs = b[:, 2:]
        q = np.concatenate([qs & 0xF, qs >> 4], axis=1).astype(np.float32) - 8.0
        return (d * q).reshape(rows, cols)
    if ty == Q4_K:
        d = b[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
        dmin = b[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
        s = b[:, 4:16].astype(np.int32)
        out = np.zeros((len(b), 256), np.float32)
        for j in range(8):
            if j < 4:
                sc, m = s[:, j] & 63, s[:, j + 4] & 63
            else:
                sc = (s[:, j + 4] & 0xF) | ((s[:, j - 4] >> 6) << 4)
                m = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
            pair, hi = j // 2, j % 2
            qb = b[:, 16 + pair * 32:16 + pair * 32 + 32]
            nib = (qb >> 4) if hi else (qb & 0xF)
            out[:, j * 32:(j + 1) * 32] = (d * sc)[:, None] * nib - (dmin * m)[:, None]
        return out.reshape(rows, cols)
    if ty == Q6_K:
        ql, qh = b[:, 0:128].astype(np.int32), b[:, 128:192].astype(np.int32)
        sc = b[:, 192:208].view(np.int8).astype(np.float32)
        d = b[:, 208:210].copy().view(np.float16).astype(np.float32)[:, 0]
        out = np.zeros((len(b), 256), np.float32)
        for half in range(2):
            for l in range(32):
                for g in range(4):
                    qlb = ql[:, half * 64 + l + (g & 1) * 32]
                    nib = (qlb & 0xF) if g < 2 else (qlb >> 4)
                    hb = (qh[:, half * 32 + l] >> (2 * g)) & 3
                    q = (nib | (hb << 4)) - 32
                    s = half * 8 + l // 16 + 2 * g
                    out[:, half * 128 + g * 32 + l] = d * sc[:, s] * q
        return out.reshape(rows, cols)
    raise ValueError(ty)


def np_int_weights(ty, raw, rows, cols):
    """Integer weight per element as the i8 dots see it (Q4_0: nibble - 8,
    Q4_K: raw nibble, Q6_K: q - 32, Q8: q)."""
    bv, bb = BLOCK[ty]
    b = np.asarray(raw, np.uint8).reshape(-1, bb)
    if ty == Q8_0:
        return b[:, 2:].view(np.int8).astype(np.int64).reshape(rows, cols)
    if ty == Q4_0:
        qs = b[:, 2:]
        return (np.concatenate([qs & 0xF, qs >> 4], axis=1).astype(np.int64) - 8).reshape(rows, cols)
    if ty == Q4_K:
        out = np.zeros((len(b), 256), np.int64)
        for j in range(8):
            qb = b[:, 16 + (j // 2) * 32:16 + (j // 2) * 32 + 32]
            out[:, j * 32:(j + 1) * 32] = (qb >> 4) if j % 2 else (qb & 0xF)
        return out.reshape(rows, cols)
    if ty == Q6_K:
        ql, qh = b[:, 0:128].astype(np.int64), b[:, 128:192].astype(np.int64)
        out = np.zeros((len(b), 256), np.int64)
        for half in range(2):
            for l in range(32):
                for g in range(4):
                    qlb = ql[:, half * 64 + l + (g & 1) * 32]
                    nib = (qlb & 0xF) if g < 2 else (qlb >> 4)
                    hb = (qh[:, half * 32 + l] >> (2 * g)) & 3
                    out[:, half * 128 + g * 32 + l] = (nib | (hb << 4)) - 32
        return out.reshape(rows, cols)
    raise ValueError(ty)


def np_block_isums(ty, raw, rows, cols, q):
    """Brute-force exact block integer dots: [rows, terms]."""
    w = np_int_weights(ty, raw, rows, cols)
    width = 16 if ty == Q6_K else 32
    prod = w * q.astype(np.int64)[None, :]
    return prod.reshape(rows, cols // width, width).sum(-1)


# ------------------------------------------------------------ tiny GGUF models (gguf.rs:567-666)
def synthetic_model(arch, with_biases, head_dim=16):
    """The reference's synthetic_model_gguf tensors: dim 32, hidden 64, 2
    layers, 2 heads (MHA), vocab 48, ctx 16, F32 tensors drawn from one
    xorshift stream (state 0xABCDEF12345) in file order."""
    dim, hidden, n_layers, n_heads, vocab, ctx = 32, 64, 2, 2, 48, 16
    q_dim = n_heads * head_dim
    kv_dim = q_dim
    state = [0xABCDEF12345]
    M = 0xFFFFFFFFFFFFFFFF

    def f32s(n, scale):
        out = np.empty(n, np.float32)
        s = state[0]
        for i in range(n):
            s ^= s >> 12
            s ^= (s << 25) & M
            s ^= s >> 27
            r = np.float32(np.float32(s >> 40) / np.float32(1 << 24)) - np.float32(0.5)
            out[i] = np.float32(r) * np.float32(scale)
        state[0] = s
        return out

    t = {}

    def put(name, dims, arr):
        t[name] = (F32, tuple(dims), arr.view(np.uint8))

    put("token_embd.weight", (dim, vocab), f32s(vocab * dim, 0.1))
    for i in range(n_layers):
        put(f"blk.{i}.attn_norm.weight", (dim,), f32s(dim, 0.5))
        put(f"blk.{i}.attn_q.weight", (dim, q_dim), f32s(q_dim * dim, 0.1))
        put(f"blk.{i}.attn_k.weight", (dim, kv_dim), f32s(kv_dim * dim, 0.1))
        put(f"blk.{i}.attn_v.weight", (dim, kv_dim), f32s(kv_dim * dim, 0.1))
        put(f"blk.{i}.attn_output.weight", (q_dim, dim), f32s(dim * q_dim, 0.1))
        if with_biases:
            put(f"blk.{i}.attn_q.bias", (q_dim,), f32s(q_dim, 0.05))
            put(f"blk.{i}.attn_k.bias", (kv_dim,), f32s(kv_dim, 0.05))
            put(f"blk.{i}.attn_v.bias", (kv_dim,), f32s(kv_dim, 0.05))
        put(f"blk.{i}.ffn_norm.weight", (dim,), f32s(dim, 0.5))
        put(f"blk.{i}.ffn_gate.weight", (dim, hidden), f32s(hidden * dim, 0.1))
        put(f"blk.{i}.ffn_down.weight", (hidden, dim), f32s(dim * hidden, 0.1))
        put(f"blk.{i}.ffn_up.weight", (dim, hidden), f32s(hidden * dim, 0.1))
    put("output_norm.weight", (dim,), f32s(dim, 0.5))
    cfg = dict(dim=dim, hidden_dim=hidden, n_layers=n_layers, n_heads=n_heads, n_kv_heads=n_heads, vocab_size=vocab,
               seq_len=ctx, head_dim=head_dim, rope_theta=10000.0, norm_eps=1e-5, emb_scale=1.0,
               rope_neox=0 if arch == "llama" else 1, act=0)
    return cfg, t
