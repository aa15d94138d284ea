"""GPU parity of the decode launches that normalise their own input at
4096-wide rows (rmsnorm, norms.rs:9-23, fused into the Q|K|V and gate|up
GEMVs): in the Q|K|V launch every workgroup evaluates the exact left-to-right
sum of squares; in the gate|up launch one workgroup evaluates it and hands
the factor to the tiles, whose unit waves stream the weights meanwhile (or,
with the wait switched off, each tile evaluates it itself). The inputs are embedding
rows chosen to stress that sum (ties against the running sum, powers of two,
subnormal squares, a wide dynamic range, zeros, a sum that overflows to inf
and falls back to the one-lane fold), each decoded as a token of a one-layer
model, so the layer's first norm sees the row itself; logits and cache rows
must equal the oracle's bit for bit."""
import numpy as np
import pytest

import prana_amd as P
from prana_amd import models as M
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def same_bits(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def stress_rows(dim, seed):
    r = np.random.default_rng(seed)
    rows = [
        np.ldexp(1.0, -r.integers(0, 20, dim)),                              # power-of-two squares
        np.where(np.arange(dim) == 0, 1.0, 2.0 ** -12),                      # half-ulp ties against 1.0
        np.exp2(r.uniform(-70, 30, dim)) * r.choice([-1, 1], dim),           # wide range
        r.integers(1, 1 << 10, dim) * 2.0 ** -80,                            # subnormal squares
        np.where(r.random(dim) < 0.5, 0.0, r.standard_normal(dim)),
        np.full(dim, 1e19),                                                  # the sum overflows to inf
        np.zeros(dim),
        r.standard_normal(dim) * 1e-3,
        1.0 + 1e-3 * r.standard_normal(dim),                                 # near-constant
        np.round(r.standard_normal(dim) * 8),                                # small integers (tie-rich)
        r.standard_normal(dim) * np.exp(2.0 * r.standard_normal(dim)),       # heavy-tailed
        r.standard_normal(dim),
    ]
    return np.stack(rows).astype(np.float32)


@pytest.mark.parametrize("ty,wait", [("Q4_0", None), ("Q8_0", None), ("Q4_0", "0")])
def test_split_norm_stress_rows_bitexact(ty, wait, monkeypatch):
    # wait "0": the gate|up tiles do not wait for the launch's norm workgroup
    # and evaluate the sum themselves (the path of a wait that runs out)
    if wait is not None:
        monkeypatch.setenv("PRANA_SPLIT_WAIT_POLLS", wait)
    kind = {"Q4_0": M.Q4_0, "Q8_0": M.Q8_0}[ty]
    dim = 4096
    emb = stress_rows(dim, 4096 + kind)
    vocab = emb.shape[0]
    cfg = M.config(dim, 1024, 1, 32, 8, vocab, 64, head_dim=128)
    t = M.synth_tensors(cfg, lambda name, cols: kind, 77 + kind)
    t["token_embd.weight"] = (M.F32, (dim, vocab), emb.view(np.uint8).reshape(-1))
    w = (1.0 + 0.1 * np.random.default_rng(5).standard_normal(dim)).astype(np.float32)
    t["blk.0.attn_norm.weight"] = (M.F32, (dim,), w.view(np.uint8))
    t["blk.0.ffn_norm.weight"] = (M.F32, (dim,), w[::-1].copy().view(np.uint8))
    g, o = P.Model(cfg, t), O.Model(cfg, t)
    gc, oc = g.cache(32), o.cache(32)
    for pos in range(vocab):
        assert same_bits(gc.forward(pos, pos), oc.forward(pos, pos)), pos
    for which in (0, 1):
        assert np.array_equal(gc.read(0, which, vocab), oc.read(0, which, vocab)), which
