"""CPU checks of the timed tier behind bench.py's cpu_baseline (the
reference's runtime-selected SIMD dots on its persistent pool, cpu_tier.c)
against the scalar tier (the oracle): Q4_K and Q6_K equal bit for bit (exact
integer horizontal sums, scalar Q6_K, as simd_x86.rs:252-299 and
kquant.rs:361 have it), the other formats within 1e-5 relative, model logits
within 1e-4 relative."""
import numpy as np
import pytest

import prana_amd as P
from oracle import oracle as O
from prana_amd import models as M
from tests import fixtures as fx


@pytest.fixture
def tier():
    def use(threads):
        return O.set_tier(1, threads)
    yield use
    O.set_tier(0)


def rel_err(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


@pytest.mark.parametrize("ty,rows,cols", [(P.Q8_0, 300, 4096), (P.Q4_0, 515, 4096), (P.Q4_K, 260, 1024),
                                          (P.Q6_K, 130, 1024), (P.F32, 200, 600)])
@pytest.mark.parametrize("threads,n", [(1, 1), (4, 1), (8, 3)])
def test_tier_matmul_against_scalar(tier, ty, rows, cols, threads, n):
    raw = P.synth_tensor(ty, rows, cols, rows + cols, 0.02)
    x = np.random.default_rng(rows).standard_normal((n, cols)).astype(np.float32)
    m = O.Mat.from_ggml(ty, rows, cols, raw)
    want = m.apply(x)
    tier(threads)
    got = m.apply(x)
    if ty in (P.Q4_K, P.Q6_K):
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    else:
        assert rel_err(got, want) < 1e-5


def test_tier_model_logits_and_pool_reuse(tier):
    cfg, t = fx.synthetic_model("qwen2", True)
    om = O.Model(cfg, t)
    ref = [om.cache(16).forward(tok, 0) for tok in (5, 9)]
    for threads in (8, 2, 16, 8):  # resize the pool between runs
        tier(threads)
        got = [om.cache(16).forward(tok, 0) for tok in (5, 9)]
        for g, w in zip(got, ref):
            assert rel_err(g, w) < 1e-4


def test_tier_c0_greedy_stream_matches_scalar(tier):
    cfg = dict(M.C0)
    t = M.c0_tensors(seed=1)
    om = O.Model(cfg, t)

    def stream():
        c, tok, out = om.cache(40), 3, []
        for pos in range(24):
            tok = int(O.argmax(c.forward(tok, pos)))
            out.append(tok)
        return out

    want = stream()
    tier(8)
    assert stream() == want
    assert "scalar" in O.tier_name()
