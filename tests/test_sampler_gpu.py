"""GPU: the device Sampler (prana_sampler_*, prana_sample_pick,
prana_generate_sampled; sampler.rs:6-71) against the oracle's:
  - the bucket walk over random, peaked, flat, tie-heavy and subnormal
    distributions up to 200000 entries, r = 0, r on a bucket boundary, steps
    that land just below a binade boundary (where the coarse grid and f32
    disagree), non-finite probabilities;
  - draw streams of Sampler::sample at the configs' vocabularies;
  - sampled generation on the C0 and tiny models (tokens, stop tokens and the
    sampler's state afterwards)."""
import numpy as np
import pytest

import prana_amd as P
from oracle import oracle as O
from prana_amd import models as M

pytestmark = pytest.mark.gpu


def dists(seed):
    r = np.random.default_rng(seed)
    for n in (1, 2, 7, 1000, 8191, 8192, 8193, 32000, 151936, 200000):
        e = r.standard_normal(n) * 3
        p = np.exp(e - e.max())
        yield f"softmax-like n={n}", (p / p.sum()).astype(np.float32)
    n = 50000
    peaked = np.where(r.random(n) < 0.001, r.random(n), r.random(n) * 1e-7)
    yield "peaked", (peaked / peaked.sum()).astype(np.float32)
    yield "flat", np.full(n, 1.0 / n, np.float32)
    yield "powers of two", np.ldexp(1.0, -r.integers(5, 40, n)).astype(np.float32)
    yield "half-ulp ties", (r.integers(0, 3, n) * 2.0 ** -24).astype(np.float32)
    yield "subnormal", np.ldexp(r.integers(0, 64, n).astype(np.float64), -r.integers(120, 160, n)).astype(np.float32)


def test_pick_matches_the_oracle():
    r = np.random.default_rng(1)
    for tag, p in dists(2):
        rs = [np.float32(0.0), np.float32(r.random()), np.float32(r.random()),
              np.float32(np.cumsum(p, dtype=np.float32)[r.integers(0, p.size)])]  # on a boundary
        for x in rs:
            assert P.sample_pick(p, x) == O.sample_pick(p, x), (tag, float(x))


def test_pick_at_binade_boundaries():
    # r = 2^e + (k+7)u, a step of 7u, a step of (k+f)u that lands just below
    # 2^e, then 2^e - u/2, which ends the walk only if the landing was rounded
    # on the finer grid as f32 does
    for e in range(-30, 0):
        u = 2.0 ** (e - 23)
        for k in range(6):
            for f in np.arange(1, 20) / 20.0:
                r = np.float32(2.0 ** e + (k + 7) * u)
                p = np.float32([7 * u, (k + f) * u, 2.0 ** e - 0.5 * u, 2.0 ** (e - 1), 2.0 ** e, 0.5 * u, 1.5 * u])
                assert P.sample_pick(p, r) == O.sample_pick(p, r), (e, k, f)
                q = p.copy()
                q[3:5] = 0
                q = np.concatenate([q, np.float32([2.0 ** (e - 30) * (j % 3) for j in range(100)] + [1.0])])
                assert P.sample_pick(q, r) == O.sample_pick(q, r), (e, k, f)


def test_pick_non_finite():
    p = np.full(20000, 1e-5, np.float32)
    p[9000] = np.nan
    assert P.sample_pick(p, np.float32(0.5)) == O.sample_pick(p, np.float32(0.5))
    p[9000] = np.inf
    assert P.sample_pick(p, np.float32(0.5)) == O.sample_pick(p, np.float32(0.5))


def test_pick_negative_and_infinite_terms_and_r():
    f = np.float32
    # a negative term raises r: 0.75 -> 0.76 -> 0.51 -> 0.01, never <= 0
    p = f([-0.01, 0.25, 0.5])
    assert O.sample_pick(p, f(0.75)) == 2  # the last index, reached by running off the end
    assert P.sample_pick(p, f(0.75)) == O.sample_pick(p, f(0.75))
    q = f([-0.01, 0.25, 0.5, 0.5])
    assert O.sample_pick(q, f(0.75)) == 3
    assert P.sample_pick(q, f(0.75)) == 3
    rng = np.random.default_rng(7)
    for n in (50, 9000, 20000):
        base = (rng.random(n) * 2.0 / n).astype(np.float32)
        for where, val in ((n // 3, -0.25), (n // 2, -np.inf), (n - 1, -1e-3), (0, -0.0)):
            p = base.copy()
            p[where] = val
            for r in (f(0.3), f(0.999), f(np.inf), f(0.0), f(-1.0)):
                assert P.sample_pick(p, r) == O.sample_pick(p, r), (n, where, val, float(r))
    # r = +inf never reaches <= 0 (inf - p stays inf), unless a term is +inf
    p = np.full(20000, 1e-5, np.float32)
    assert P.sample_pick(p, f(np.inf)) == 19999
    p[123] = np.inf
    assert P.sample_pick(p, f(np.inf)) == O.sample_pick(p, f(np.inf))


@pytest.mark.parametrize("vocab,temp", [(32000, 0.8), (151936, 1.0), (48, 0.5), (32000, 0.0)])
def test_sample_stream(vocab, temp):
    logits = (np.random.default_rng(vocab).standard_normal((30, vocab)) * 4).astype(np.float32)
    g, o = P.Sampler(temp, 99), O.Sampler(temp, 99)
    for row in logits:
        assert g.sample(row) == o.sample(row)
    assert g.next_f32() == o.next_f32()


@pytest.mark.parametrize("temp,seed", [(0.8, 3), (1.3, 0), (0.0, 5)])
def test_generate_sampled_c0(temp, seed):
    t = M.c0_tensors(seed=1)
    g, o = P.Model(M.C0, t), O.Model(M.C0, t)
    prompt = np.random.default_rng(7).integers(0, M.C0["vocab_size"], 5).astype(np.uint32)
    gs, os_ = P.Sampler(temp, seed), O.Sampler(temp, seed)
    got, st = gs.generate(g, prompt, 60)
    want = O.generate_sampled(o, prompt, 60, os_)
    assert list(got) == list(want) and st.generated_tokens == len(want)
    assert gs.state == os_.state.value
    # a stop token (the 20th sampled one): the stream ends before it and the
    # state has taken exactly the draws the reference takes
    if len(want) > 20:
        stop = int(want[19])
        gs2, os2 = P.Sampler(temp, seed), O.Sampler(temp, seed)
        got2, _ = gs2.generate(g, prompt, 60, stops=[stop])
        want2 = O.generate_sampled(o, prompt, 60, os2, stops=[stop])
        assert list(got2) == list(want2) and gs2.state == os2.state.value


def test_generate_sampled_from_one_token_and_full_prompt():
    cfg = dict(M.C0)
    cfg["seq_len"] = 32
    t = M.c0_tensors(seed=1)
    g, o = P.Model(cfg, t), O.Model(cfg, t)
    for prompt in ([17], list(range(3, 40))):  # one token; a prompt longer than the window
        gs, os_ = P.Sampler(0.9, 21), O.Sampler(0.9, 21)
        got, _ = gs.generate(g, np.uint32(prompt), 40)
        want = O.generate_sampled(o, np.uint32(prompt), 40, os_)
        assert list(got) == list(want) and gs.state == os_.state.value
