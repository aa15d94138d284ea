"""GPU side of the elementwise pins: the inputs on which the reference's
final-rounding expressions and their plausible alternatives give different
bits (tests/pin_cases.py) run through the device kernels, which must equal the
oracle bit for bit. Together with tests/test_oracle_pins_elementwise.py this
ties the device to the reference expression itself, not only to tolerance.

Also RoPE at the long positions of the attention microbenchmark (1k-32k,
hd 128, theta 1e4), both pairings, against the oracle."""
import numpy as np
import pytest

import prana_amd as P
from oracle import oracle as O
from tests import pin_cases as pc

pytestmark = pytest.mark.gpu


def same_bits(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("case", ["div_vs_mul", "scale", "half_away"])
def test_quantize_acts_pins_on_device(case):
    blk = getattr(pc, f"quantize_case_{case}")()
    x = np.stack([blk, -blk, blk * np.float32(0.5)])
    q, s, m = P.quantize_acts(x)
    qo, so, mo = O.quantize_acts(x)
    assert np.array_equal(q, qo) and same_bits(s, so) and np.array_equal(m, mo)


@pytest.mark.parametrize("dim", [96, 288])
def test_rmsnorm_pins_on_device(dim):
    x, w, eps = pc.rmsnorm_case(dim)
    got = P.rmsnorm(x[None, :], w, float(eps))
    assert same_bits(got, O.rmsnorm(x[None, :], w, float(eps)))


def test_silu_and_gelu_pins_on_device():
    v = pc.silu_case()
    assert same_bits(P.silu(v), O.silu(v))
    g = pc.gelu_case()
    assert same_bits(P.gelu_tanh(g), O.gelu_tanh(g))
    # the gate|up epilogue form: act(g) * u with u = 1 keeps act's bits
    one = np.ones_like(v)
    assert same_bits(P.act_mul(v, one), O.silu(v))
    assert same_bits(P.act_mul(g, np.ones_like(g), gelu=True), O.gelu_tanh(g))


def test_softmax_pins_on_device():
    v = pc.softmax_case()
    assert same_bits(P.softmax(v)[0], O.softmax(v))


@pytest.mark.parametrize("hd", [48, 128])
def test_attention_score_scale_pins_on_device(hd):
    q, kc, vc, pos, nh, nkv, hd = pc.attention_case(hd)
    got = P.attention_decode(q, kc, vc, pos, nh, nkv, hd)
    assert same_bits(got, O.attention_decode(q, kc, vc, pos, nh, nkv, hd))


@pytest.mark.parametrize("neox", [False, True])
def test_rope_long_positions_on_device(neox):
    """Device RoPE (host-built (cos, sin) tables) at positions 1k-32k, hd 128,
    theta 1e4, on rows whose f32-angle rotation differs from a double-angle
    one (checked on the CPU by the oracle pins)."""
    x = pc.rope_case(hd=128, n_heads=32)
    fn = O.rope_neox if neox else O.rope_interleaved
    for pos in pc.ROPE_POSITIONS:
        got = P.rope(x[None, :], pos, 128, 1e4, neox)[0]
        assert same_bits(got, fn(x, pos, 128, 1e4)), pos
    # several consecutive rows: positions pos0 + i
    rows = np.stack([x] * 4)
    got = P.rope(rows, 32764, 128, 1e4, neox)
    for i in range(4):
        assert same_bits(got[i], fn(x, 32764 + i, 128, 1e4)), i
