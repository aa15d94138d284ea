"""GPU: the closed-form quantized-dot cases of test_oracle_pins on the device
path (decode GEMV at one token, batched matrix-core paths at 9 and 65 rows),
and every shape `assert!` of the reference driven through the C ABI, which
must come back as PRANA_ERR_INVALID with a message instead of aborting."""
import ctypes as C

import numpy as np
import pytest

import prana_amd as P
from prana_amd import _lib
from tests import test_oracle_pins as T

pytestmark = pytest.mark.gpu
f32 = np.float32
ERR_INVALID = -1


def dev_rows(ty, raw, cols, q, sa, n_tok):
    """The device matmul of one row over n_tok copies of the given quantized
    acts (n_tok picks the kernel: 1 decode, 9 skinny / K-quant, 65 prefill)."""
    q = np.tile(np.asarray(q, np.int8).reshape(1, cols), (n_tok, 1))
    sa = np.tile(np.asarray(sa, np.float32).reshape(1, cols // 32), (n_tok, 1))
    sums = q.astype(np.int32).reshape(n_tok, cols // 32, 32).sum(-1).astype(np.int32)
    m = P.Matrix(ty, 1, cols, np.concatenate(raw))
    return m.apply_prefill(q, sa, sums)[:, 0]


@pytest.mark.parametrize("n_tok", [1, 9, 65])
def test_closed_form_terms_and_tie_folds_on_device(n_tok):
    one = np.zeros(32, np.int64)
    one[0] = 1
    # Q8_0: [1, t, t, t, t, -1] with t half an ulp of 1 -> exactly 0
    blocks = [T.q8_0_block(1.0, one)] + [T.q8_0_block(2.0 ** -24, one) for _ in range(4)] + [T.q8_0_block(-1.0, one)]
    got = dev_rows(T.Q8_0, blocks, 192, np.tile(one, 6), [1.0] * 6, n_tok)
    assert np.all(T.bits(got) == T.bits(f32(0.0)))
    # Q4_0 ties -> 1.0
    nib = np.full(32, 8)
    nib[0] = 9
    blocks = [T.q4_0_block(1.0, nib)] + [T.q4_0_block(2.0 ** -24, nib) for _ in range(4)]
    got = dev_rows(T.Q4_0, blocks, 160, np.tile(one, 5), [1.0] * 5, n_tok)
    assert np.all(T.bits(got) == T.bits(f32(1.0)))
    # Q4_K group fold -> 0.0 and 1.0
    nib = np.zeros(256, np.int64)
    qa = np.zeros(256, np.int64)
    for g in range(8):
        nib[g * 32] = 1
        qa[g * 32] = 1
    t = 2.0 ** -24
    blk = T.q4_k_block(1.0, 0.0, np.ones(8, np.int64), np.zeros(8, np.int64), nib)
    got = dev_rows(T.Q4_K, [blk], 256, qa, np.array([1, t, t, t, t, 0.5, -0.5, -1], np.float32), n_tok)
    assert np.all(T.bits(got) == T.bits(f32(0.0)))
    # Q6_K sub-block fold -> 2.0
    q = np.zeros(256, np.int64)
    qa = np.zeros(256, np.int64)
    for s in range(16):
        q[s * 16] = 1
        qa[s * 16] = 1
    got = dev_rows(T.Q6_K, [T.q6_k_block(1.0, np.ones(16, np.int64), q)], 256, qa,
                   np.array([1] + [2.0 ** -23] * 7, np.float32), n_tok)
    assert np.all(T.bits(got) == T.bits(f32(2.0)))


@pytest.mark.parametrize("n_tok", [1, 9, 65])
def test_parenthesisation_cases_on_device(n_tok):
    rng = np.random.default_rng(11)
    # Q8_0 (matmul.rs:404)
    ref = lambda d, sa, qw, qa: f32(d * sa) * f32(int(np.dot(qw, qa)))
    alt = lambda d, sa, qw, qa: d * f32(sa * f32(int(np.dot(qw, qa))))
    samp = lambda r: (T.f16_val(r.uniform(0.001, 0.1)), f32(r.uniform(0.001, 0.1)), r.integers(-127, 128, 32),
                      r.integers(-127, 128, 32))
    (d, sa, qw, qa), want = T.find_distinguishing(ref, [alt], samp, rng)
    got = dev_rows(T.Q8_0, [T.q8_0_block(d, qw)], 32, qa, [sa], n_tok)
    assert np.all(T.bits(got) == T.bits(want))
    # Q4_0 (kquant.rs:250)
    ref = lambda d, sa, nb, qa: f32(d * sa) * f32(int(np.dot(nb, qa)) - 8 * int(qa.sum()))
    alt = lambda d, sa, nb, qa: d * f32(sa * f32(int(np.dot(nb, qa)) - 8 * int(qa.sum())))
    samp = lambda r: (T.f16_val(r.uniform(0.001, 0.1)), f32(r.uniform(0.001, 0.1)), r.integers(0, 16, 32),
                      r.integers(-127, 128, 32))
    (d, sa, nb, qa), want = T.find_distinguishing(ref, [alt], samp, rng)
    got = dev_rows(T.Q4_0, [T.q4_0_block(d, nb)], 32, qa, [sa], n_tok)
    assert np.all(T.bits(got) == T.bits(want))
    # Q6_K (kquant.rs:313-314), sub-block 5
    ref = lambda d, sa, sc, q, qa: f32(f32(d * sa) * f32(sc)) * f32(int(np.dot(q, qa)))
    alt = lambda d, sa, sc, q, qa: f32(d * sa) * f32(f32(sc) * f32(int(np.dot(q, qa))))
    samp = lambda r: (T.f16_val(r.uniform(0.001, 0.05)), f32(r.uniform(0.001, 0.1)), int(r.integers(-128, 128)),
                      r.integers(-32, 32, 16), r.integers(-127, 128, 16))
    (d, sa, sc, q, qa), want = T.find_distinguishing(ref, [alt], samp, rng)
    qs, qa256, scs = np.zeros(256, np.int64), np.zeros(256, np.int64), np.zeros(16, np.int64)
    qs[80:96], qa256[80:96], scs[5] = q, qa, sc
    sas = np.full(8, 0.25, np.float32)
    sas[2] = sa
    got = dev_rows(T.Q6_K, [T.q6_k_block(d, scs, qs)], 256, qa256, sas, n_tok)
    assert np.all(T.bits(got) == T.bits(f32(0.0) + want))


def test_argmax_fixed_answers_on_device():
    rows = [[1, 3, 3, 2], [T.NAN, 5, 7, 0], [1, T.NAN, 3, 0], [-0.0, 0.0, -1, -1], [-T.INF, -T.INF, -1, -T.INF]]
    assert list(P.argmax(np.array(rows, np.float32))) == [1, 0, 2, 0, 2]


# ------------------------------------------------------------------ reference assert! sites through the ABI
def expect_invalid(rc, *words):
    assert rc == ERR_INVALID, rc
    msg = P.load().prana_last_error().decode()
    for w in words:
        assert w in msg, msg


def test_quantmatrix_from_parts_asserts():
    # matmul.rs:35: cols must be a multiple of 32
    lib = P.load()
    P.init()
    q = np.zeros(80, np.int8)
    s = np.zeros(4, np.float32)
    h = C.c_void_p()
    expect_invalid(lib.prana_mat_create_q8(2, 40, q.ctypes.data, s.ctypes.data, C.byref(h)), "multiple of 32")


@pytest.mark.parametrize("ty,rows,cols,nbytes,word", [
    (P.Q4_K, 1, 100, 200, "unaligned"),     # kquant.rs:168 (cols % 256, element count not block-aligned)
    (P.Q6_K, 1, 256, 209, "shorter"),       # kquant.rs:169 (byte count)
    (P.Q4_0, 2, 64, 71, "shorter"),
    (P.Q8_0, 1, 32, 33, "shorter"),
    (99, 1, 32, 128, "unsupported"),
])
def test_kquant_from_raw_asserts(ty, rows, cols, nbytes, word):
    lib = P.load()
    P.init()
    raw = np.zeros(max(nbytes, 1), np.uint8)
    h = C.c_void_p()
    expect_invalid(lib.prana_mat_create(ty, rows, cols, raw.ctypes.data, nbytes, C.byref(h)), word)


@pytest.mark.parametrize("verify", [False, True])
@pytest.mark.parametrize("nh,nkv,hd,word", [
    (3, 2, 16, "multiple of n_kv_heads"),   # attention.rs:139 / 307
    (4, 0, 16, "multiple of n_kv_heads"),
    (2, 1, 258, "head_dim"),                # attention.rs:140 / 308
])
def test_attention_asserts(verify, nh, nkv, hd, word):
    lib = P.load()
    q = P.DeviceArray((2, nh * hd), np.float32)
    kc = P.DeviceArray((4, max(nkv, 1) * hd), np.uint16)
    out = P.DeviceArray((2, nh * hd), np.float32)
    if verify:
        rc = lib.prana_attention_verify(q.ptr, kc.ptr, kc.ptr, 1, 2, nh, nkv, hd, out.ptr, None)
    else:
        rc = lib.prana_attention_decode(q.ptr, kc.ptr, kc.ptr, 2, nh, nkv, hd, out.ptr, None)
    expect_invalid(rc, word)


def test_other_shape_asserts():
    lib = P.load()
    x = P.DeviceArray((64,), np.float32)
    q8 = P.DeviceArray((64,), np.int8)
    s = P.DeviceArray((4,), np.float32)
    expect_invalid(lib.prana_quantize_acts(x.ptr, 1, 33, q8.ptr, s.ptr, s.ptr, None), "multiple of 32")
    expect_invalid(lib.prana_rope_neox(x.ptr, 1, 30, 0, 15, f32(1e4), None), "even")       # attention.rs:91
    expect_invalid(lib.prana_rope_interleaved(x.ptr, 1, 30, 0, 8, f32(1e4), None), "whole")  # attention.rs:92
    cfg = P.PranaConfig(dim=64, hidden_dim=128, n_layers=1, n_heads=3, n_kv_heads=2, vocab_size=16, seq_len=8,
                        head_dim=16, rope_theta=1e4, norm_eps=1e-5, emb_scale=1.0, rope_neox=0, act=0)
    h = C.c_void_p()
    expect_invalid(lib.prana_model_create(C.byref(cfg), C.byref(h)), "n_kv_heads")


def test_model_runtime_asserts():
    from tests import fixtures as fx
    cfg, t = fx.synthetic_model("llama", False)
    m = P.Model(cfg, t)
    c = m.cache(8)
    lib = P.load()
    logits = np.zeros(cfg["vocab_size"], np.float32)
    expect_invalid(lib.prana_forward(m.h, c.h, 0, 8, 1, logits.ctypes.data), "beyond the cache")
    expect_invalid(lib.prana_forward(m.h, c.h, cfg["vocab_size"], 0, 1, logits.ctypes.data), "vocabulary")
    out = np.zeros(4, np.uint32)
    expect_invalid(lib.prana_decode(m.h, c.h, 0, 6, 4, out.ctypes.data), "beyond the cache")
