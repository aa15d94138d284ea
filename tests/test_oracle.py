"""Pins the CPU oracle (oracle/prana_oracle.c) before it is trusted as the
checker: the reference's own known-answer tests (restated, each citing its
reference file:line), closed forms, brute-force integer dots in numpy, and
independent library conversions (numpy's IEEE float16)."""
import math

import numpy as np
import pytest

from oracle import oracle as O
from tests import fixtures as fx


def bits32(x):
    return np.array([x], np.float32).view(np.uint32)[0]


# ------------------------------------------------------------------ f16 (lib.rs:115-155, gguf.rs:887-897)
def test_f16_exact_round_trip():  # lib.rs:120-125
    for v in [0.0, -0.0, 1.0, -1.0, 0.5, 2.0, -2.0, 0.25, 65504.0, -65504.0]:
        assert bits32(O.f16_to_f32(O.f32_to_f16(v))) == bits32(v)


def test_f16_near():  # lib.rs:128-137
    for i in range(-2000, 2000):
        v = np.float32(i) * np.float32(0.0017)
        r = O.f16_to_f32(O.f32_to_f16(v))
        assert abs(r - v) <= abs(v) * 1e-3 + 1e-6


def test_f16_specials():  # lib.rs:140-146
    assert O.f32_to_f16(math.inf) == 0x7C00
    assert O.f32_to_f16(-math.inf) == 0xFC00
    assert math.isnan(O.f16_to_f32(O.f32_to_f16(math.nan)))
    assert O.f32_to_f16(1e30) == 0x7C00
    assert O.f32_to_f16(1e-30) == 0x0000


def test_f16_tie_to_even():  # lib.rs:149-154
    assert O.f32_to_f16(1.0 + 2.0 ** -11) == 0x3C00


def test_f16_decode_kats():  # gguf.rs:888-897
    assert O.f16_to_f32(0x0000) == 0.0
    assert O.f16_to_f32(0x3C00) == 1.0
    assert O.f16_to_f32(0xC000) == -2.0
    assert O.f16_to_f32(0x7C00) == math.inf
    assert math.isnan(O.f16_to_f32(0x7E00))
    assert abs(O.f16_to_f32(0x0001) - 2.0 ** -24) < 1e-12
    assert abs(O.f16_to_f32(0x3555) - 0.33325) < 1e-4


def test_f16_decode_all_against_numpy():
    # Every half value: the oracle must agree with IEEE float16 (numpy).
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([O.f16_to_f32(int(x)) for x in h], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f16_encode_boundaries_against_numpy():
    # RNE on every tie point between adjacent halves and one f32 ulp either side,
    # plus random finite floats: must equal numpy's IEEE float16 conversion.
    h = np.arange(0, 0x7BFF, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)
    cand = np.concatenate([mid, np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(0))])
    rng = np.random.default_rng(7)
    cand = np.concatenate([cand, rng.standard_normal(20000).astype(np.float32) * 1000,
                           rng.standard_normal(20000).astype(np.float32) * 1e-5])
    cand = np.concatenate([cand, -cand])
    ref = cand.astype(np.float16).view(np.uint16)
    got = np.array([O.f32_to_f16(float(x)) for x in cand], np.uint16)
    assert np.array_equal(got, ref)


# ------------------------------------------------------------------ quantize_acts (matmul.rs:105-127)
def test_quantize_acts_invariants():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(32 * 64).astype(np.float32) * 3
    x[32:64] = 0.0  # zero block -> scale 1.0, q = 0
    q, s, m = O.quantize_acts(x)
    q, s, m = q[0].astype(np.int64), s[0], m[0]
    assert np.all(np.abs(q) <= 127)
    assert np.array_equal(m, q.reshape(-1, 32).sum(1))
    assert s[1] == 1.0 and np.all(q[32:64] == 0)
    xb = x.reshape(-1, 32)
    for g in range(64):
        if g == 1:
            continue
        amax = np.abs(xb[g]).max()
        assert s[g] == np.float32(amax) / np.float32(127.0)
        i = np.abs(xb[g]).argmax()
        assert abs(q[g * 32 + i]) == 127
        # every element within half a step of its dequantized value
        err = np.abs(xb[g] - q[g * 32:(g + 1) * 32] * s[g])
        assert np.all(err <= s[g] * 0.5 * (1 + 1e-5))


def test_quantize_acts_round_half_away():
    # 0.5 and 1.5 steps: Rust f32::round rounds half away from zero.
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1] = 0.5
    x[2] = -0.5
    x[3] = 1.5
    x[4] = -2.5
    q, s, _ = O.quantize_acts(x)
    assert s[0, 0] == 1.0
    assert list(q[0, :5]) == [127, 1, -1, 2, -3]


# ------------------------------------------------------------------ block KATs (gguf.rs:929-1070)
def test_q4k_block_kat():  # gguf.rs:930-951
    b = np.zeros(144, np.uint8)
    b[0:2] = [0x00, 0x3C]
    b[4], b[5] = 2, 3
    for i in range(32):
        b[16 + i] = (i % 16) | ((15 - i % 16) << 4)
    m = O.Mat.from_ggml(fx.Q4_K, 1, 256, b)
    out = m.row_f32(0)
    for i in range(32):
        assert out[i] == 2.0 * (i % 16)
        assert out[32 + i] == 3.0 * (15 - i % 16)
    assert np.all(out[64:] == 0.0)


def test_q4k_scale_min_high_groups():  # gguf.rs:954-965
    s = np.zeros(12, np.uint8)
    s[8] = (53 & 0xF) | ((43 & 0xF) << 4)
    s[0] = (53 >> 4) << 6
    s[4] = (43 >> 4) << 6
    sc, mn = np.float32(0), np.float32(0)
    import ctypes as C
    a, b = C.c_float(), C.c_float()
    O.lib().po_q4k_scale_min(4, O.P(s), C.byref(a), C.byref(b))
    assert (a.value, b.value) == (53.0, 43.0)


def test_q6k_block_kat():  # gguf.rs:968-985
    b = np.zeros(210, np.uint8)
    b[192:208] = 1
    b[208:210] = [0x00, 0x3C]
    b[0] = 5
    b[128] = 2
    out = O.Mat.from_ggml(fx.Q6_K, 1, 256, b).row_f32(0)
    assert out[0] == 5.0
    assert out[1] == -32.0
    assert out[64] == -32.0


def test_q4_0_tensor_native():  # gguf.rs:988-1036
    raw = bytearray()
    raw += (0x3C00).to_bytes(2, "little")
    raw += bytes(j | ((15 - j) << 4) for j in range(16))
    raw += (0x3800).to_bytes(2, "little")
    raw += bytes([0xCC] * 16)
    raw = np.frombuffer(bytes(raw), np.uint8)
    m = O.Mat.from_ggml(fx.Q4_0, 1, 64, raw)
    f = m.row_f32(0)
    for j in range(16):
        assert f[j] == j - 8.0
        assert f[16 + j] == (15 - j) - 8.0
    assert np.all(f[32:] == 0.5 * (12.0 - 8.0))
    x = np.sin(np.arange(64, dtype=np.float32) * np.float32(0.37)).astype(np.float32)
    want = float(np.dot(x.astype(np.float64), f.astype(np.float64)))
    got = m.apply(x)[0, 0]
    assert abs(got - want) < 2e-2 * max(abs(want), 1.0)


def test_q8_0_tensor_native():  # gguf.rs:1039-1070
    raw = np.frombuffer((0x3C00).to_bytes(2, "little") + bytes(((i - 16) & 0xFF) for i in range(32)), np.uint8)
    m = O.Mat.from_ggml(fx.Q8_0, 1, 32, raw)
    assert abs(m.apply(np.ones(32, np.float32))[0, 0] + 16.0) < 1e-4


# ------------------------------------------------------------------ native dots == dense reference (kquant.rs:397-477)
@pytest.mark.parametrize("ty,seeds", [(fx.Q4_0, [3, 77, 2024]), (fx.Q4_K, [1, 42, 12345]), (fx.Q6_K, [7, 99, 54321]),
                                      (fx.Q8_0, [5, 6, 8])])
def test_native_matches_dequant_reference(ty, seeds):
    rows, cols, n_tok = 5, 512, 2
    for seed in seeds:
        raw = fx.pseudo_blocks(ty, rows, cols, seed)
        m = O.Mat.from_ggml(ty, rows, cols, raw)
        a = fx.sin_row(n_tok * cols, 0.013).reshape(n_tok, cols)
        native = m.apply(a)
        q, s, _ = O.quantize_acts(a)
        a_dq = (q.astype(np.float32).reshape(n_tok, -1, 32) * s[:, :, None]).reshape(n_tok, cols)
        w = fx.np_dequant(ty, raw, rows, cols)
        dense = a_dq.astype(np.float64) @ w.astype(np.float64).T
        tol = 1e-3 * np.maximum(np.abs(dense), 1.0)
        assert np.all(np.abs(native - dense) < tol), (ty, seed)


@pytest.mark.parametrize("ty", [fx.Q4_0, fx.Q4_K, fx.Q6_K, fx.Q8_0])
def test_block_isums_brute_force(ty):
    # The exact integer part of every term vs a numpy int64 brute force on
    # independently unpacked weights.
    rows, cols = 3, 512
    raw = fx.pseudo_blocks(ty, rows, cols, 11)
    m = O.Mat.from_ggml(ty, rows, cols, raw)
    a = fx.sin_row(cols, 0.021, 0.3)
    q, s, sums = O.quantize_acts(a)
    want = fx.np_block_isums(ty, raw, rows, cols, q[0])
    terms = want.shape[1]
    for r in range(rows):
        assert np.array_equal(m.row_isums(q[0], sums[0], r, terms), want[r])


def test_q40_row_dequant_matches_full():  # kquant.rs:450-463
    raw = fx.pseudo_blocks(fx.Q4_0, 3, 64, 9)
    m = O.Mat.from_ggml(fx.Q4_0, 3, 64, raw)
    full = fx.np_dequant(fx.Q4_0, raw, 3, 64)
    for r in range(3):
        assert np.array_equal(m.row_f32(r), full[r])


# ------------------------------------------------------------------ matmul.rs tests (563-626)
def test_f32_matmul_kat():  # matmul.rs:568-580
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    w = np.array([[1, 0, 0], [0, 1, 0], [0, 0, 1], [1, 1, 1]], np.float32)
    assert np.array_equal(O.Mat.f32(w).apply(a), np.array([[1, 2, 3, 6], [4, 5, 6, 15]], np.float32))


def test_q8_roundtrip_and_tracking():  # matmul.rs:583-611
    w = np.sin(np.arange(8 * 64, dtype=np.float32) * np.float32(0.013)).reshape(8, 64).astype(np.float32)
    q, s = O.quantize_q8(w)
    dq = (q.astype(np.float32).reshape(8, 2, 32) * s[:, :, None]).reshape(8, 64)
    assert np.abs(w - dq).max() < 0.01
    a = np.cos(np.arange(96, dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    w2 = np.sin(np.arange(6 * 96, dtype=np.float32) * np.float32(0.017)).reshape(6, 96).astype(np.float32)
    dense = O.Mat.f32(w2).apply(a)
    q2, s2 = O.quantize_q8(w2)
    quant = O.Mat.q8_parts(q2, s2).apply(a)
    assert np.abs(dense - quant).max() < 0.05


def test_prefill_and_decode_agree_bitwise():  # matmul.rs:614-626
    w = np.sin(np.arange(5 * 32, dtype=np.float32) * np.float32(0.03)).reshape(5, 32).astype(np.float32)
    batch = np.cos(np.arange(3 * 32, dtype=np.float32) * np.float32(0.011)).reshape(3, 32).astype(np.float32)
    m = O.Mat.f32(w)
    allr = m.apply(batch)
    for t in range(3):
        assert np.array_equal(allr[t], m.apply(batch[t])[0])


def test_dot_f32_scalar_order_closed_form():
    # dot_f32_scalar (matmul.rs:377-391): four strided partial sums combined
    # ((a0+a1)+a2)+a3, then the tail. Chosen so any other association differs.
    a = np.array([1e8, 1.0, -1e8, 1.0, 3.0], np.float32)
    b = np.ones(5, np.float32)
    # acc = [1e8, 1, -1e8, 1]; (1e8 + 1) = 1e8 in f32; + (-1e8) = 0; + 1 = 1; tail + 3 = 4
    assert O.Mat.f32(a[None, :]).apply(b)[0, 0] == 4.0


# ------------------------------------------------------------------ norms (norms.rs:59-107)
def test_rmsnorm_constant_row():  # norms.rs:66-74
    y = O.rmsnorm(np.full(4, 2.0, np.float32), np.ones(4, np.float32), 0.0)
    assert np.all(np.abs(y - 1.0) < 1e-5)


def order_cases():
    """Inputs whose left-to-right f32 fold has a closed form that any other
    summation order misses (half-ulp ties against the running sum)."""
    n = 37
    # rmsnorm: squares 1, 2^-24, ... -> every add ties to the even 1.0
    x_rms = np.full(n, 2.0 ** -12, np.float32)
    x_rms[0] = 1.0
    ss = np.float32(1.0)
    y0 = np.float32(1.0) * (np.float32(1.0) / np.sqrt(ss / np.float32(n) + np.float32(0.0)))
    # softmax: exps 1, ~1.5*2^-24, ... -> every add rounds up by exactly one ulp of [1, 2)
    a = np.float32(math.log(1.5) - 24 * math.log(2.0))
    x_sm = np.full(n, a, np.float32)
    x_sm[0] = 0.0
    p0 = np.float32(1.0) * (np.float32(1.0) / np.float32(1.0 + (n - 1) * 2.0 ** -23))
    return x_rms, y0, x_sm, p0


def pv_order_case():
    """q = 0 gives p = 1/4 for 4 cache rows; v[dim 0] = 1, 2^-24, 2^-24, 2^-24
    makes every later product a half-ulp tie against 0.25, so the sequential
    fold stays exactly 0.25 (any regrouping gives 0.25 + 2^-24)."""
    nh = nkv = 1
    hd, pos = 16, 3
    q = np.zeros(hd, np.float32)
    kc = np.zeros((pos + 1) * hd, np.uint16)
    vc = np.zeros((pos + 1) * hd, np.uint16)
    vc[0] = 0x3C00  # 1.0
    vc[hd::hd] = 0x0001  # 2^-24
    return q, kc, vc, pos, nh, nkv, hd


def test_sequential_order_closed_forms():
    x_rms, y0, x_sm, p0 = order_cases()
    assert O.rmsnorm(x_rms, np.ones(x_rms.size, np.float32), 0.0)[0, 0] == y0
    assert O.softmax(x_sm)[0] == p0
    q, kc, vc, pos, nh, nkv, hd = pv_order_case()
    assert O.attention_decode(q, kc, vc, pos, nh, nkv, hd)[0] == np.float32(0.25)


def test_softmax_props():  # norms.rs:77-106
    p = O.softmax(np.array([1.0, 2.0, 3.0], np.float32))
    assert abs(p.sum() - 1.0) < 1e-6 and p[0] < p[1] < p[2]
    p = O.softmax(np.array([1000.0, 1001.0], np.float32))
    assert np.all(np.isfinite(p)) and abs(p.sum() - 1.0) < 1e-6


def test_silu_gelu_points():  # norms.rs:85-103
    y = O.silu(np.array([0.0, 1.0, -1.0, 4.0], np.float32))
    assert y[0] == 0.0 and abs(y[1] - 0.7310586) < 1e-5 and abs(y[2] + 0.2689414) < 1e-5 and 3.9 < y[3] < 4.0
    g = O.gelu_tanh(np.array([0.0, 1.0, -1.0, 3.0], np.float32))
    assert g[0] == 0.0 and abs(g[1] - 0.841192) < 1e-4 and abs(g[2] + 0.158808) < 1e-4 and abs(g[3] - 2.9959) < 1e-3


def test_softmax_uses_glibc_expf_exactly():
    # exp(0) = 1 exactly and p = e * (1/sum) exactly for a 2-element row.
    x = np.array([0.0, 0.0], np.float32)
    assert list(O.softmax(x)) == [0.5, 0.5]


# ------------------------------------------------------------------ RoPE (attention.rs:339-455)
def test_rope_batch_preserves_pair_norm_and_pos0():  # attention.rs:340-373
    seq, nh, hd = 3, 2, 4
    x = (np.sin(np.arange(seq * nh * hd, dtype=np.float32) * np.float32(0.1)) + np.float32(0.3)).astype(np.float32)
    y = O.rope_batch(x, seq, nh, hd, 10000.0)
    xb, yb = x.reshape(seq, nh, hd), y.reshape(seq, nh, hd)
    n0 = xb[..., :2] ** 2 + xb[..., 2:] ** 2
    n1 = yb[..., :2] ** 2 + yb[..., 2:] ** 2
    assert np.all(np.abs(n0 - n1) < 1e-5)
    z = np.arange(8, dtype=np.float32)
    assert np.all(np.abs(O.rope_batch(z, 1, 1, 8, 10000.0) - z) < 1e-6)


def test_rope_interleaved_pos0_and_norm():  # attention.rs:421-434
    x = (np.sin(np.arange(16, dtype=np.float32) * np.float32(0.3)) + np.float32(0.1)).astype(np.float32)
    assert np.array_equal(O.rope_interleaved(x, 0, 8, 10000.0), x)
    y = O.rope_interleaved(x, 7, 8, 10000.0)
    n0 = x[0::2] ** 2 + x[1::2] ** 2
    n1 = y[0::2] ** 2 + y[1::2] ** 2
    assert np.all(np.abs(n0 - n1) < 1e-4)


def test_rope_neox_matches_batch_rope():  # attention.rs:437-455
    nh, hd = 2, 8
    w = nh * hd
    row = (np.sin(np.arange(w, dtype=np.float32) * np.float32(0.17)) + np.float32(0.2)).astype(np.float32)
    batch = np.zeros(4 * w, np.float32)
    batch[3 * w:4 * w] = row
    b = O.rope_batch(batch, 4, nh, hd, 10000.0)
    assert np.all(np.abs(O.rope_neox(row, 3, hd, 10000.0) - b[3 * w:4 * w]) < 1e-5)


def test_rope_rotation_closed_form():
    # One pair at pos 1, hd 2: freq = theta^0 = 1, angle = 1 rad.
    y = O.rope_interleaved(np.array([1.0, 0.0], np.float32), 1, 2, 10000.0)
    assert abs(y[0] - math.cos(1.0)) < 1e-6 and abs(y[1] - math.sin(1.0)) < 1e-6


# ------------------------------------------------------------------ attention (attention.rs:375-502)
def _qkv(seq, nh, nkv, hd, a, b, c):
    q = np.cos(np.arange(seq * nh * hd, dtype=np.float32) * np.float32(a)).astype(np.float32)
    k = np.sin(np.arange(seq * nkv * hd, dtype=np.float32) * np.float32(b)).astype(np.float32)
    v = np.cos(np.arange(seq * nkv * hd, dtype=np.float32) * np.float32(c)).astype(np.float32)
    return q, k, v


def test_attention_pos0_is_v0():  # attention.rs:376-394
    q, k, v = _qkv(4, 2, 2, 3, 0.05, 0.03, 0.02)
    out = O.attention(q, k, v, 4, 2, 2, 3)
    assert np.all(np.abs(out[0] - v[:6]) < 1e-5)


def test_attention_bounded_by_v():  # attention.rs:397-418
    seq, hd = 5, 4
    q = np.sin(np.arange(seq * hd, dtype=np.float32) * np.float32(0.2)).astype(np.float32)
    k = np.cos(np.arange(seq * hd, dtype=np.float32) * np.float32(0.15)).astype(np.float32)
    v = np.sin(np.arange(seq * hd, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    out = O.attention(q, k, v, seq, 1, 1, hd)
    for i in range(seq):
        vis = v[: (i + 1) * hd]
        assert np.all(out[i] >= vis.min() - 1e-5) and np.all(out[i] <= vis.max() + 1e-5)


def test_decode_over_f16_cache_matches_full():  # attention.rs:458-488
    seq, nh, hd = 5, 2, 4
    w = nh * hd
    q = np.sin(np.arange(seq * w, dtype=np.float32) * np.float32(0.07)).astype(np.float32)
    k = np.cos(np.arange(seq * w, dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    v = np.sin(np.arange(seq * w, dtype=np.float32) * np.float32(0.03)).astype(np.float32)
    full = O.attention(q, k, v, seq, nh, nh, hd)
    kh = np.array([O.f32_to_f16(x) for x in k], np.uint16)
    vh = np.array([O.f32_to_f16(x) for x in v], np.uint16)
    for pos in range(seq):
        step = O.attention_decode(q[pos * w:(pos + 1) * w], kh, vh, pos, nh, nh, hd)
        assert np.all(np.abs(full[pos] - step) < 3e-3)


def test_gqa_shapes_and_group_mapping():  # attention.rs:491-502 + h/group mapping
    seq, nh, nkv, hd = 3, 4, 2, 2
    q = np.arange(seq * nh * hd, dtype=np.float32) * np.float32(0.01)
    k = np.arange(seq * nkv * hd, dtype=np.float32) * np.float32(0.02)
    v = np.arange(seq * nkv * hd, dtype=np.float32) * np.float32(0.03)
    out = O.attention(q, k, v, seq, nh, nkv, hd)
    assert out.shape == (seq, nh * hd)
    # position 0: each query head h returns v0 of kv head h // 2
    v0 = v[: nkv * hd].reshape(nkv, hd)
    for h in range(nh):
        assert np.all(np.abs(out[0, h * hd:(h + 1) * hd] - v0[h // 2]) < 1e-6)


def test_verify_equals_decode_rows():
    seq, nh, nkv, hd, pos0 = 3, 4, 2, 8, 5
    n = pos0 + seq
    rng = np.random.default_rng(3)
    kc = rng.standard_normal(n * nkv * hd).astype(np.float32).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal(n * nkv * hd).astype(np.float32).astype(np.float16).view(np.uint16)
    q = rng.standard_normal(seq * nh * hd).astype(np.float32)
    ver = O.attention_verify(q, kc, vc, pos0, seq, nh, nkv, hd)
    for i in range(seq):
        d = O.attention_decode(q[i * nh * hd:(i + 1) * nh * hd], kc, vc, pos0 + i, nh, nkv, hd)
        assert np.array_equal(ver[i], d)


# ------------------------------------------------------------------ model (prana-model lib.rs:65-144, gguf.rs:679-858)
@pytest.fixture(scope="module")
def qwen2():
    return fx.synthetic_model("qwen2", True)


@pytest.fixture(scope="module")
def llama():
    return fx.synthetic_model("llama", False)


def test_forward_deterministic_and_position_dependent(llama):  # lib.rs:73-92
    cfg, t = llama
    m = O.Model(cfg, t)
    a = m.cache(16).forward(7, 0)
    b = m.cache(16).forward(7, 0)
    assert np.array_equal(a, b)
    c1 = m.cache(16)
    c1.forward(7, 0)
    c = c1.forward(7, 1)
    assert not np.array_equal(a, c)
    assert np.all(np.isfinite(a))


def test_qwen2_biases_change_output():  # gguf.rs:849-857
    cfg, tb = fx.synthetic_model("qwen2", True)
    _, tn = fx.synthetic_model("qwen2", False)
    a = O.Model(cfg, tb).cache(16).forward(7, 0)
    b = O.Model(cfg, tn).cache(16).forward(7, 0)
    assert not np.array_equal(a, b)


@pytest.mark.parametrize("arch", ["llama", "qwen2"])
def test_batched_prefill_matches_sequential(arch):  # gguf.rs:715-743
    cfg, t = fx.synthetic_model(arch, arch == "qwen2")
    m = O.Model(cfg, t)
    toks = [3, 9, 14, 7, 21]
    c1 = m.cache(16)
    for pos, tok in enumerate(toks):
        c1.forward(tok, pos)
    seq = c1.forward(5, len(toks))
    c2 = m.cache(16)
    c2.prefill(toks)
    bat = c2.forward(5, len(toks))
    assert np.abs(seq - bat).max() < 1e-2


def test_forward_batch_rows_equal_sequential_decode_bitwise(qwen2):
    # attention_verify runs decode_one_head per row and the batched dots are
    # the decode dots, so verify logits are bit-identical to sequential decode
    # over the same cache contents (the invariant spec == greedy rests on).
    cfg, t = qwen2
    m = O.Model(cfg, t)
    c1, c2 = m.cache(16), m.cache(16)
    pre = [3, 9, 14]
    c1.prefill(pre)
    c2.prefill(pre)
    toks = [7, 21, 4]
    seq = [c1.forward(tk, 3 + i) for i, tk in enumerate(toks)]
    bat = c2.forward_batch(toks, 3)
    for i in range(3):
        assert np.array_equal(bat[i], seq[i])


def _plain_greedy(m, prompt, steps, stops):
    # gguf.rs:804-836
    cache = m.cache(16)
    nxt = None
    for pos, t in enumerate(prompt):
        logits = cache.forward(t, pos)
        if pos + 1 == len(prompt):
            nxt = O.argmax(logits)
    out, pos = [], len(prompt)
    while len(out) < steps:
        if nxt in stops:
            break
        out.append(nxt)
        if len(out) >= steps:
            break
        nxt = O.argmax(cache.forward(out[-1], pos))
        pos += 1
    return out


@pytest.mark.parametrize("draft_arch", ["qwen2", "llama"])
def test_speculative_equals_plain_greedy(draft_arch):  # gguf.rs:746-799
    cfg, t = fx.synthetic_model("qwen2", True)
    target = O.Model(cfg, t)
    dcfg, dt = fx.synthetic_model(draft_arch, draft_arch == "qwen2")
    draft = O.Model(dcfg, dt)
    prompt = [5, 7, 9]  # "&(*" under the test's '!'-offset vocab, no BOS
    stops = (46, 47)
    ref = _plain_greedy(target, prompt, 8, stops)
    spec, st = O.generate_speculative(target, draft, prompt, 8, 4, stops)
    assert list(spec) == ref
    assert st.proposed >= st.accepted
    if draft_arch == "qwen2":
        assert st.accepted > 0


def test_generate_equals_teacher_forced_loop(llama):
    # generate (infer.rs:696-771): batched prefill of p-1, then decode; equals
    # a token-by-token loop up to the f16-cache-vs-f32 prefill difference the
    # reference accepts (compare tokens; here exact for this model).
    cfg, t = llama
    m = O.Model(cfg, t)
    out, st = m.generate([1, 2, 3], 10)
    assert st.prompt_tokens == 3 and st.generated_tokens == len(out)
    assert len(out) == min(16, 3 + 10) - 3  # context cap: max_pos - p
