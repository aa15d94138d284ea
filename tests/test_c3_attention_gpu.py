"""GPU: configuration C3 (GQA decode attention, 32 query / 8 KV heads, hd 128,
f16 cache filled N(0,1), f32 query, NeoX RoPE at position = context length)
against the oracle's attention_decode / attention_verify (attention.rs:129-195,
296-333):
  - split-K flash decoding within its documented tolerance, per element:
    |got - want| <= 1e-4 |want| + 1e-6 S_d with S_d = sum_t p_t |v_t[d]| (the
    scale of a reassociated weighted sum's rounding error, which keeps
    outputs that nearly cancel from failing on a relative bound alone), for
    ctx 1k / 4k / 16k / 32k, batch 1 and batch 8 as eight independent caches,
    and for other group sizes (C2's 14/2 heads) and head widths (48-256);
  - the exact kernels bit for bit at ctx 32768 (decode, eight verify rows, an
    odd row count over a group count that is not a multiple of four) and over
    eight independent caches;
  - adversarial decode rows around the one-lane fold limit (n = 33, 511, 512,
    513): wide score spreads with many ties, NaN / inf in q."""
import numpy as np
import pytest

import prana_amd as P
from oracle import oracle as O

pytestmark = pytest.mark.gpu

NH, NKV, HD, THETA = 32, 8, 128, 1e4


def same_bits(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def abs_weighted(q, kc, vc, pos, nh, nkv, hd):
    """S_d = sum_t p_t |v_t[d]| per output element, in float64."""
    kf = kc.view(np.float16).astype(np.float64).reshape(pos + 1, nkv * hd)
    vf = vc.view(np.float16).astype(np.float64).reshape(pos + 1, nkv * hd)
    g = nh // nkv
    out = np.zeros(nh * hd)
    for h in range(nh):
        kv = h // g
        s = kf[:, kv * hd:(kv + 1) * hd] @ np.asarray(q[h * hd:(h + 1) * hd], np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h * hd:(h + 1) * hd] = p @ np.abs(vf[:, kv * hd:(kv + 1) * hd])
    return out


def within_tolerance(got, want, q, kc, vc, pos, nh, nkv, hd):
    """Per element: |got - want| <= 1e-4 |want| + 1e-6 S_d."""
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    bound = 1e-4 * np.abs(want) + 1e-6 * abs_weighted(q, kc, vc, pos, nh, nkv, hd)
    return bool(np.all(np.abs(got - want) <= bound))


def c3_case(ctx, seed, nh=NH, nkv=NKV, hd=HD):
    """Cache of ctx+1 rows: rows 0..ctx-1 N(0,1) as f16, row ctx the new k
    (NeoX RoPE at position ctx); q N(0,1) with the same RoPE."""
    r = np.random.default_rng(seed)
    kv = nkv * hd
    kc = r.standard_normal((ctx + 1, kv)).astype(np.float16).view(np.uint16)
    vc = r.standard_normal((ctx + 1, kv)).astype(np.float16).view(np.uint16)
    q = O.rope_neox(r.standard_normal(nh * hd).astype(np.float32), ctx, hd, THETA)
    k_new = O.rope_neox(r.standard_normal(kv).astype(np.float32), ctx, hd, THETA)
    kc[ctx] = O.f32_to_f16_n(k_new)
    return q, kc, vc


@pytest.mark.parametrize("ctx", [1024, 4096, 16384, 32768])
def test_splitk_batch1_within_1e4(ctx):
    q, kc, vc = c3_case(ctx, ctx)
    got = P.attention_decode_splitk(q[None, :], [kc], [vc], [ctx], NH, NKV, HD)[0]
    want = O.attention_decode(q, kc, vc, ctx, NH, NKV, HD)
    assert within_tolerance(got, want, q, kc, vc, ctx, NH, NKV, HD)


@pytest.mark.parametrize("ctx", [1024, 4096, 16384, 32768])
def test_splitk_batch8_independent_caches_within_1e4(ctx):
    # eight sequences, each with its own cache; ragged positions below ctx
    cases = [c3_case(ctx - 37 * i, 100 * ctx + i) for i in range(8)]
    pos = [ctx - 37 * i for i in range(8)]
    q = np.stack([c[0] for c in cases])
    got = P.attention_decode_splitk(q, [c[1] for c in cases], [c[2] for c in cases], pos, NH, NKV, HD)
    for i, (qi, kc, vc) in enumerate(cases):
        want = O.attention_decode(qi, kc, vc, pos[i], NH, NKV, HD)
        assert within_tolerance(got[i], want, qi, kc, vc, pos[i], NH, NKV, HD), i


@pytest.mark.parametrize("nh,nkv,hd,ctx", [(8, 8, 128, 3000), (16, 8, 64, 5000), (16, 2, 64, 2047), (4, 4, 64, 1),
                                           (32, 8, 128, 0), (8, 1, 128, 700),
                                           (14, 2, 64, 2048), (14, 2, 64, 4096),   # C2's qwen2 shape: group 7
                                           (12, 4, 96, 3000), (6, 2, 48, 900),     # widths 96 and 48
                                           (8, 2, 256, 5000), (4, 4, 200, 333),    # widths 256 and 200
                                           (32, 1, 128, 2000), (24, 8, 128, 700),  # groups 32 and 3
                                           (20, 4, 64, 1500)])                     # group 5
def test_splitk_other_groups_and_widths(nh, nkv, hd, ctx):
    # any group size (blocks of up to 8 query heads per workgroup) and any
    # head width that is a multiple of 8 up to 256 (attention.rs:42, 129-160)
    q, kc, vc = c3_case(ctx, nh * 1000 + ctx + hd, nh, nkv, hd)
    got = P.attention_decode_splitk(q[None, :], [kc], [vc], [ctx], nh, nkv, hd)[0]
    want = O.attention_decode(q, kc, vc, ctx, nh, nkv, hd)
    assert within_tolerance(got, want, q, kc, vc, ctx, nh, nkv, hd)


def test_splitk_rejects_unsupported_shapes():
    # rows of 16-byte pieces: head widths must be multiples of 8, at most 256
    q, kc, vc = c3_case(64, 1, 4, 4, 36)
    with pytest.raises(P.PranaError, match="multiple of 8 up to 256"):
        P.attention_decode_splitk(q[None, :], [kc], [vc], [64], 4, 4, 36)
    q, kc, vc = c3_case(64, 1, 2, 2, 264)
    with pytest.raises(P.PranaError, match="multiple of 8 up to 256"):
        P.attention_decode_splitk(q[None, :], [kc], [vc], [64], 2, 2, 264)


# ------------------------------------------------------------------ the exact kernels at C3's largest window
def test_exact_decode_ctx32768_bitexact():
    q, kc, vc = c3_case(32768, 7)
    assert same_bits(P.attention_decode(q, kc, vc, 32768, NH, NKV, HD), O.attention_decode(q, kc, vc, 32768, NH,
                                                                                           NKV, HD))


@pytest.mark.parametrize("seq,nh,nkv,ctx", [(8, 32, 8, 32760), (3, 24, 8, 16400), (5, 12, 4, 20000)])
def test_exact_verify_long_windows_bitexact(seq, nh, nkv, ctx):
    # 8 verify rows at 32k; odd row counts with groups of 3 (not a multiple
    # of four) at 16k+ (attention_verify, attention.rs:296-333)
    r = np.random.default_rng(ctx + seq)
    kv = nkv * HD
    kc = r.standard_normal((ctx + seq, kv)).astype(np.float16).view(np.uint16)
    vc = r.standard_normal((ctx + seq, kv)).astype(np.float16).view(np.uint16)
    q = r.standard_normal((seq, nh * HD)).astype(np.float32)
    got = P.attention_verify(q, kc, vc, ctx, seq, nh, nkv, HD)
    want = O.attention_verify(q, kc, vc, ctx, seq, nh, nkv, HD)
    assert same_bits(got, want)


def test_exact_decode_eight_independent_caches_bitexact():
    for i in range(8):
        ctx = 4096 + 611 * i
        q, kc, vc = c3_case(ctx, 50 + i)
        assert same_bits(P.attention_decode(q, kc, vc, ctx, NH, NKV, HD),
                         O.attention_decode(q, kc, vc, ctx, NH, NKV, HD)), i


# ------------------------------------------------------------------ adversarial rows around the one-lane fold limit
@pytest.mark.parametrize("n", [33, 511, 512, 513, 896, 897])
@pytest.mark.parametrize("kind", ["ties", "spread", "nan_q", "inf_q"])
def test_exact_decode_adversarial_near_fold_limit(n, kind):
    nh, nkv, hd = 8, 2, 64
    r = np.random.default_rng(n * 7 + len(kind))
    kv = nkv * hd
    if kind == "ties":
        # small-integer keys and a query of powers of two: many equal scores,
        # exponentials that tie at half an ulp in the sequential sum
        kc = r.integers(-2, 3, (n, kv)).astype(np.float16).view(np.uint16)
        q = np.ldexp(1.0, r.integers(-3, 2, nh * hd)).astype(np.float32)
    else:
        kc = (r.standard_normal((n, kv)) * (30.0 if kind == "spread" else 1.0)).astype(np.float16).view(np.uint16)
        q = r.standard_normal(nh * hd).astype(np.float32)
    vc = r.standard_normal((n, kv)).astype(np.float16).view(np.uint16)
    if kind == "nan_q":
        q[5] = np.nan
    if kind == "inf_q":
        q[hd + 3] = np.inf
    got = P.attention_decode(q, kc, vc, n - 1, nh, nkv, hd)
    want = O.attention_decode(q, kc, vc, n - 1, nh, nkv, hd)
    assert same_bits(got, want)
