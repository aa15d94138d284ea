"""The oracle's Sampler (sampler.rs:6-71) pinned on the CPU: the reference's
own tests, a closed-form first draw, the bucket walk's f32 semantics at a
rounding tie, and the sampled distribution."""
import numpy as np

from oracle import oracle as O


def test_greedy_picks_the_max():
    # greedy_picks_the_max (sampler.rs:78-82)
    assert O.Sampler(0.0, 42).sample([0.1, 3.0, -1.0, 2.9]) == 1
    # temp <= 0 is greedy (Sampler::new), the first max wins
    assert O.Sampler(-1.0, 42).sample([1.0, 5.0, 5.0]) == 1


def test_temperature_sampling_is_seeded_and_in_range():
    # temperature_sampling_is_seeded_and_in_range (sampler.rs:84-93)
    logits = [1.0, 2.0, 3.0, 4.0]
    a, b = O.Sampler(0.8, 7), O.Sampler(0.8, 7)
    for _ in range(50):
        x, y = a.sample(logits), b.sample(logits)
        assert x == y and 0 <= x < 4


def test_rng_is_roughly_uniform():
    # rng_is_roughly_uniform (sampler.rs:95-101)
    r = O.Sampler(1.0, 123)
    v = np.float32([r.next_f32() for _ in range(10000)])
    assert abs(float(v.mean()) - 0.5) < 0.02
    assert v.min() >= 0.0 and v.max() < 1.0


def test_first_draw_closed_form():
    # seed 1: x ^= x >> 12 -> 1; x ^= x << 25 -> 2^25 + 1; x ^= x >> 27 -> 2^25 + 1;
    # top 24 bits of (2^25 + 1) * 0x2545F4914F6CDD1D mod 2^64 = 4711630
    assert O.Sampler(1.0, 1).next_f32() == np.float32(4711630) / np.float32(1 << 24)
    # XorShift::new(seed.max(1)): seed 0 is seed 1
    a, b = O.Sampler(1.0, 0), O.Sampler(1.0, 1)
    assert [a.next_f32() for _ in range(5)] == [b.next_f32() for _ in range(5)]


def test_bucket_walk_semantics():
    f = np.float32
    # lands exactly on 0 at index 1: r <= 0 stops there
    assert O.sample_pick(f([0.25, 0.25, 0.5]), 0.5) == 1
    assert O.sample_pick(f([0.25, 0.25, 0.5]), 0.0) == 0
    # the mass never reaches r: round-off leaves r > 0 -> the last index
    assert O.sample_pick(f([0.1, 0.1]), 0.9) == 1
    # f32 order: r = 1 - 2^-24, r - 2^-25 = 1 - 1.5 ulp ties to the even
    # 1 - 2^-23, which the next term cancels exactly (index 1); in exact
    # arithmetic r would stay 2^-25 above 0 until index 2
    assert O.sample_pick(f([2.0 ** -25, 1 - 2.0 ** -23, 0.5]), f(1 - 2.0 ** -24)) == 1


def test_tiny_temperature_is_argmax_and_distribution_matches_softmax():
    s = O.Sampler(1e-3, 5)
    assert all(s.sample([1.0, 2.0, 3.0, 4.0]) == 3 for _ in range(20))
    logits = np.float32([1.0, 2.0, 3.0, 4.0])
    p = np.exp((logits / 0.8).astype(np.float64))
    p /= p.sum()
    s = O.Sampler(0.8, 11)
    n = 20000
    counts = np.bincount([s.sample(logits) for _ in range(n)], minlength=4)
    sigma = np.sqrt(n * p * (1 - p))
    assert np.all(np.abs(counts - n * p) < 4 * sigma), (counts, n * p)
