"""Pins for the oracle's elementwise final-rounding expressions.

Each test takes inputs on which the reference's expression (evaluated in
tests/pin_cases.py with numpy float32 and the platform libm) and every
plausible alternative give different bits, asserts that they do, and then
asserts that the oracle equals the reference expression bit for bit. A
mis-parenthesised or reordered oracle therefore fails here, which a tolerance
check would not see. Runs on the CPU only (the oracle is the thing checked).

References: matmul.rs:116-123 (quantize_acts), norms.rs:15-19 (rmsnorm), 29
(silu), 37-39 (gelu_tanh), 49-54 (softmax), attention.rs:174-184 (score
scale), 96 and 115 (RoPE angle)."""
import numpy as np
import pytest

from oracle import oracle as O
from tests import pin_cases as pc

f32 = np.float32


def same_bits(a, b):
    return np.array_equal(pc.bits(a), pc.bits(b))


# ------------------------------------------------------------------ quantize_acts (matmul.rs:116-123)
def test_quantize_x_times_inv_not_x_over_scale():
    blk = pc.quantize_case_div_vs_mul()
    q_ref, s_ref, m_ref = pc.quantize_ref(blk)
    q_alt, _, _ = pc.quantize_ref(blk, q_mode="div")
    assert not np.array_equal(q_ref, q_alt)
    q, s, m = O.quantize_acts(blk[None, :])
    assert np.array_equal(q[0].astype(np.int32), q_ref)
    assert same_bits(s[0, 0], s_ref) and int(m[0, 0]) == m_ref


def test_quantize_scale_is_amax_over_127():
    blk = pc.quantize_case_scale()
    _, s_ref, _ = pc.quantize_ref(blk)
    _, s_alt, _ = pc.quantize_ref(blk, scale_mode="mul_recip")
    assert not same_bits(s_ref, s_alt)
    _, s, _ = O.quantize_acts(blk[None, :])
    assert same_bits(s[0, 0], s_ref)


def test_quantize_rounds_half_away_from_zero():
    blk = pc.quantize_case_half_away()
    q_ref, _, m_ref = pc.quantize_ref(blk)
    q_even, _, _ = pc.quantize_ref(blk, rounding="even")
    assert list(q_ref[:6]) == [127, 3, -1, 1, -4, 127]
    assert not np.array_equal(q_ref, q_even)
    q, _, m = O.quantize_acts(blk[None, :])
    assert np.array_equal(q[0].astype(np.int32), q_ref) and int(m[0, 0]) == m_ref


# ------------------------------------------------------------------ rmsnorm (norms.rs:15-19)
@pytest.mark.parametrize("dim", [96, 288])
def test_rmsnorm_expression_pinned(dim):
    x, w, eps = pc.rmsnorm_case(dim)
    ref = pc.rmsnorm_ref(x, w, eps)
    for alt in pc.RMS_ALTS:
        assert pc.differs(pc.rmsnorm_ref(x, w, eps, alt), ref), alt
    assert same_bits(O.rmsnorm(x[None, :], w, float(eps))[0], ref)


# ------------------------------------------------------------------ silu / gelu_tanh (norms.rs:29, 37-39)
def test_silu_expression_pinned():
    v = pc.silu_case()
    ref = pc.silu_ref(v)
    for alt in pc.SILU_ALTS:
        assert pc.differs(pc.silu_ref(v, alt), ref), alt
    assert same_bits(O.silu(v), ref)


def test_gelu_tanh_term_order_pinned():
    v = pc.gelu_case()
    ref = pc.gelu_ref(v)
    assert np.isfinite(ref[0])  # (0.5*x)*(1+t) stays finite at 3e38
    for alt in pc.GELU_ALTS:
        assert pc.differs(pc.gelu_ref(v, alt), ref), alt
    assert same_bits(O.gelu_tanh(v), ref)


# ------------------------------------------------------------------ softmax (norms.rs:49-54)
def test_softmax_normalisation_pinned():
    v = pc.softmax_case()
    ref = pc.softmax_ref(v)
    for alt in pc.SOFTMAX_ALTS:
        assert pc.differs(pc.softmax_ref(v, alt), ref), alt
    assert same_bits(O.softmax(v), ref)


# ------------------------------------------------------------------ attention score (attention.rs:174-184)
@pytest.mark.parametrize("hd", [48, 128])
def test_attention_score_scale_pinned(hd):
    q, kc, vc, pos, nh, nkv, hd = pc.attention_case(hd)
    ref = pc.attention_ref(q, kc, vc, pos, nh, nkv, hd)
    assert pc.differs(pc.attention_ref(q, kc, vc, pos, nh, nkv, hd, "div_sqrt"), ref)
    assert same_bits(O.attention_decode(q, kc, vc, pos, nh, nkv, hd), ref)


# ------------------------------------------------------------------ RoPE angle (attention.rs:96, 115)
@pytest.mark.parametrize("neox", [False, True])
@pytest.mark.parametrize("pos", pc.ROPE_POSITIONS)
def test_rope_f32_angle_pinned(pos, neox):
    x = pc.rope_case()
    ref = pc.rope_ref(x, pos, 128, 1e4, neox)
    assert pc.differs(pc.rope_ref(x, pos, 128, 1e4, neox, "f64_angle"), ref)
    fn = O.rope_neox if neox else O.rope_interleaved
    assert same_bits(fn(x, pos, 128, 1e4), ref)


def test_pins_have_power():
    """A planted mistake in a copy of the reference expression is caught by
    the same comparison the pins use (the oracle itself is not touched)."""
    x, w, eps = pc.rmsnorm_case(96)
    planted = pc.rmsnorm_ref(x, w, eps, "inv_times_w")
    assert not same_bits(planted, O.rmsnorm(x[None, :], w, float(eps))[0])
    v = pc.softmax_case()
    assert not same_bits(pc.softmax_ref(v, "div"), O.softmax(v))
