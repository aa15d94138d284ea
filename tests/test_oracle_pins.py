"""Pins for the oracle functions that the golden vectors leave open.

Each check is built so that a plausible mistake fails it:
  - argmax: fixed answers from the strict `>` / first-max rule of
    infer.rs:560-568 (ties, NaN at the front and inside, signed zeros);
  - quantized row dots: one-row matrices whose terms are chosen so that the
    reference's parenthesisation (matmul.rs:404, kquant.rs:250, 278-279,
    313-314; Rust `a * b * c` is `(a * b) * c`) gives different bits from the
    plausible alternatives, which each test evaluates and shows to differ, and
    whose block fold hits half-ulp ties, so that only the left-to-right fold
    gives the closed-form result;
  - layer wiring: an independent float64 forward of the reference's tiny
    llama / qwen2 models written from infer.rs:142-211 (bias placement, RoPE
    target, silu on w1, residual order, f16 K/V cache), checked to 1e-4
    relative; the same forward with a wiring mistake planted misses the oracle
    by far more, so the check has power.
Runs on the CPU only (the oracle is the thing checked)."""
import numpy as np
import pytest

from oracle import oracle as O
from tests import fixtures as fx

f32 = np.float32
Q4_0, Q8_0, Q4_K, Q6_K = fx.Q4_0, fx.Q8_0, fx.Q4_K, fx.Q6_K


def bits(x):
    return np.asarray(x, np.float32).view(np.uint32)


def f16_bits(v):
    return int(np.array([v], np.float16).view(np.uint16)[0])


def f16_val(v):
    """The f32 value of v rounded to f16 (what a block stores)."""
    return f32(np.float16(v))


# ------------------------------------------------------------------ argmax (infer.rs:560-568)
NAN, INF = float("nan"), float("inf")


@pytest.mark.parametrize("row,want", [
    ([1, 3, 3, 2], 1),             # first of two equal maxima
    ([5], 0),
    ([2, 2, 2], 0),
    ([-1, -3, -1], 0),
    ([NAN, 5, 7], 0),              # nothing compares greater than a leading NaN
    ([1, NAN, 3], 2),              # a NaN inside never wins
    ([3, NAN, 3], 0),
    ([-0.0, 0.0], 0),              # 0.0 > -0.0 is false
    ([INF, INF], 0),
    ([-INF, -INF, -1], 2),
    ([-INF, NAN, -INF], 0),
])
def test_argmax_fixed_answers(row, want):
    assert int(O.argmax(np.array(row, np.float32))) == want


# ------------------------------------------------------------------ block builders (ggml layouts)
def q8_0_block(d, q):
    b = np.zeros(34, np.uint8)
    b[0:2] = np.frombuffer(np.uint16(f16_bits(d)).tobytes(), np.uint8)
    b[2:] = np.asarray(q, np.int8).view(np.uint8)
    return b


def q4_0_block(d, nib):
    """nib[0..32] in 0..15: element j<16 low nibble of byte j, 16+j high nibble."""
    nib = np.asarray(nib, np.uint8)
    b = np.zeros(18, np.uint8)
    b[0:2] = np.frombuffer(np.uint16(f16_bits(d)).tobytes(), np.uint8)
    b[2:] = nib[:16] | (nib[16:] << 4)
    return b


def q4_k_block(d, dmin, sc, mn, nib):
    """sc/mn: 8 six-bit values (kquant.rs:52-61 packing); nib[256] in 0..15."""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(np.uint16(f16_bits(d)).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.uint16(f16_bits(dmin)).tobytes(), np.uint8)
    s = np.zeros(12, np.int64)
    for j in range(4):
        s[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = mn[j] | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4)
    b[4:16] = s.astype(np.uint8)
    nib = np.asarray(nib, np.uint8)
    for p in range(4):
        b[16 + p * 32:16 + p * 32 + 32] = nib[p * 64:p * 64 + 32] | (nib[p * 64 + 32:p * 64 + 64] << 4)
    return b


def q6_k_block(d, sc, q):
    """q[256] in -32..31 in element order; sc: 16 int8 sub-block scales."""
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for e in range(256):
        u = int(q[e]) + 32
        h, r = divmod(e, 128)
        g, l = divmod(r, 32)
        idx = h * 64 + l + (g & 1) * 32
        if g < 2:
            ql[idx] |= u & 0xF
        else:
            ql[idx] |= (u & 0xF) << 4
        qh[h * 32 + l] |= ((u >> 4) & 3) << (2 * g)
    b = np.zeros(210, np.uint8)
    b[0:128], b[128:192] = ql, qh
    b[192:208] = np.asarray(sc, np.int8).view(np.uint8)
    b[208:210] = np.frombuffer(np.uint16(f16_bits(d)).tobytes(), np.uint8)
    return b


def test_block_builders_roundtrip_through_numpy_dequant():
    rng = np.random.default_rng(0)
    q = rng.integers(-32, 32, 256)
    sc = rng.integers(-128, 128, 16)
    raw = q6_k_block(0.5, sc, q)
    want = np.repeat(sc.astype(np.float32), 16) * q * f32(0.5)
    assert np.array_equal(fx.np_dequant(Q6_K, raw, 1, 256)[0], want.astype(np.float32))
    nib = rng.integers(0, 16, 256)
    s8, m8 = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
    raw = q4_k_block(0.25, 0.125, s8, m8, nib)
    want = (np.repeat(s8, 32) * 0.25 * nib - np.repeat(m8, 32) * 0.125).astype(np.float32)
    assert np.array_equal(fx.np_dequant(Q4_K, raw, 1, 256)[0], want)


def oracle_row(ty, raw, cols, q, sa):
    """The oracle's batched matmul of one row over given quantized acts."""
    q = np.asarray(q, np.int8).reshape(1, cols)
    sa = np.asarray(sa, np.float32).reshape(1, cols // 32)
    sums = q.astype(np.int32).reshape(1, cols // 32, 32).sum(-1).astype(np.int32)
    m = O.Mat.from_ggml(ty, 1, cols, np.concatenate(raw))
    return m.apply_prefill(q, sa, sums)[0, 0]


def find_distinguishing(fn_ref, alts, sampler, rng, tries=20000):
    """Draw inputs until the reference expression differs from every
    alternative (so a mis-parenthesised oracle would fail the test)."""
    for _ in range(tries):
        args = sampler(rng)
        r = fn_ref(*args)
        if np.isfinite(r) and all(bits(a(*args)) != bits(r) for a in alts):
            return args, r
    raise AssertionError("no distinguishing input found")


# ------------------------------------------------------------------ Q8 (matmul.rs:404): (sw*sa)*float(acc)
def test_q8_term_parenthesisation_pinned():
    rng = np.random.default_rng(1)

    def sample(r):
        d = f16_val(r.uniform(0.001, 0.1))
        sa = f32(r.uniform(0.001, 0.1))
        qw = r.integers(-127, 128, 32)
        qa = r.integers(-127, 128, 32)
        return d, sa, qw, qa

    ref = lambda d, sa, qw, qa: f32(d * sa) * f32(int(np.dot(qw, qa)))
    alts = [lambda d, sa, qw, qa: d * f32(sa * f32(int(np.dot(qw, qa)))),
            lambda d, sa, qw, qa: f32(d * f32(int(np.dot(qw, qa)))) * sa]
    for _ in range(4):
        (d, sa, qw, qa), want = find_distinguishing(ref, alts, sample, rng)
        got = oracle_row(Q8_0, [q8_0_block(d, qw)], 32, qa, [sa])
        assert bits(got) == bits(want)


def tie_fold_rows(make_block, unit_big, unit_tiny):
    """Blocks whose terms are [1, t, t, t, t] with t = 2^-24 (half an ulp of 1):
    the left-to-right fold gives exactly 1.0; any tree or reversed order gives
    1 + 2^-22."""
    return [make_block(unit_big)] + [make_block(unit_tiny) for _ in range(4)]


def test_q8_block_fold_half_ulp_ties():
    one = np.zeros(32, np.int64)
    one[0] = 1
    blocks = [q8_0_block(1.0, one)] + [q8_0_block(2.0 ** -24, one) for _ in range(4)]
    qa = np.tile(one, 5)
    got = oracle_row(Q8_0, blocks, 160, qa, [1.0] * 5)
    assert got == f32(1.0) and bits(got) == bits(f32(1.0))
    assert f32(1.0) + f32(4 * 2.0 ** -24) != f32(1.0)  # what a reordered fold gives
    # cancellation after the ties: [1, t, t, t, t, -1] -> exactly 0
    blocks.append(q8_0_block(-1.0, one))
    got = oracle_row(Q8_0, blocks, 192, np.tile(one, 6), [1.0] * 6)
    assert bits(got) == bits(f32(0.0))


# ------------------------------------------------------------------ Q4_0 (kquant.rs:250): (d*sa)*float(s - 8*sum_a)
def test_q4_0_term_parenthesisation_pinned():
    rng = np.random.default_rng(2)

    def sample(r):
        d = f16_val(r.uniform(0.001, 0.1))
        sa = f32(r.uniform(0.001, 0.1))
        nib = r.integers(0, 16, 32)
        qa = r.integers(-127, 128, 32)
        return d, sa, nib, qa

    def isum(nib, qa):
        return int(np.dot(nib, qa)) - 8 * int(qa.sum())

    ref = lambda d, sa, nib, qa: f32(d * sa) * f32(isum(nib, qa))
    alts = [lambda d, sa, nib, qa: d * f32(sa * f32(isum(nib, qa))),
            # the correction applied in floats instead of integers
            lambda d, sa, nib, qa: f32(f32(d * sa) * f32(int(np.dot(nib, qa))))
            - f32(f32(d * sa) * f32(8 * int(qa.sum())))]
    for _ in range(4):
        (d, sa, nib, qa), want = find_distinguishing(ref, alts, sample, rng)
        got = oracle_row(Q4_0, [q4_0_block(d, nib)], 32, qa, [sa])
        assert bits(got) == bits(want)


def test_q4_0_block_fold_half_ulp_ties():
    nib = np.full(32, 8)
    nib[0] = 9  # s - 8*sum_a = 1 with qa = e0
    qa = np.zeros(32, np.int64)
    qa[0] = 1
    blocks = [q4_0_block(1.0, nib)] + [q4_0_block(2.0 ** -24, nib) for _ in range(4)]
    got = oracle_row(Q4_0, blocks, 160, np.tile(qa, 5), [1.0] * 5)
    assert bits(got) == bits(f32(1.0))


# ------------------------------------------------------------------ Q4_K (kquant.rs:278-279)
# per group: sa*((d*sc)*float(s) - (dmin*m)*float(sum_a)); groups in element
# order (pair p: group 2p then 2p+1).
def test_q4_k_term_parenthesisation_pinned():
    rng = np.random.default_rng(3)

    def sample(r):
        d, dmin = f16_val(r.uniform(0.001, 0.05)), f16_val(r.uniform(0.001, 0.05))
        sc, mn = int(r.integers(1, 64)), int(r.integers(1, 64))
        sa = f32(r.uniform(0.001, 0.1))
        nib = r.integers(0, 16, 32)
        qa = r.integers(-127, 128, 32)
        return d, dmin, sc, mn, sa, nib, qa

    def ref(d, dmin, sc, mn, sa, nib, qa):
        s, sm = int(np.dot(nib, qa)), int(qa.sum())
        return sa * (f32(f32(d * f32(sc)) * f32(s)) - f32(f32(dmin * f32(mn)) * f32(sm)))

    def alt_distributed(d, dmin, sc, mn, sa, nib, qa):
        s, sm = int(np.dot(nib, qa)), int(qa.sum())
        return f32(sa * f32(f32(d * f32(sc)) * f32(s))) - f32(sa * f32(f32(dmin * f32(mn)) * f32(sm)))

    def alt_scale_first(d, dmin, sc, mn, sa, nib, qa):
        # sa folded into the block scales first, as the Q6_K term does.
        # ((d*sc)*s and d*(sc*s) are both the rounded exact product here, so
        # that reordering is not a distinguishable mistake.)
        s, sm = int(np.dot(nib, qa)), int(qa.sum())
        return f32(f32(sa * f32(d * f32(sc))) * f32(s)) - f32(f32(sa * f32(dmin * f32(mn))) * f32(sm))

    for j in (0, 5):  # one unpacked (j < 4) and one packed (j >= 4) scale slot
        (d, dmin, sc, mn, sa, nib, qa), want = find_distinguishing(ref, [alt_distributed, alt_scale_first], sample,
                                                                   rng)
        scs, mns = np.zeros(8, np.int64), np.zeros(8, np.int64)
        scs[j], mns[j] = sc, mn
        nib256 = np.zeros(256, np.int64)
        nib256[j * 32:(j + 1) * 32] = nib
        qa256 = np.zeros(256, np.int64)
        qa256[j * 32:(j + 1) * 32] = qa
        sas = np.full(8, 0.5, np.float32)
        sas[j] = sa
        # every other group's term is sa*((d*0)*0 - (dmin*0)*0) = +0.0
        got = oracle_row(Q4_K, [q4_k_block(d, dmin, scs, mns, nib256)], 256, qa256, sas)
        assert bits(got) == bits(f32(0.0) + want)


def test_q4_k_group_fold_half_ulp_ties():
    # groups 0..7 of one super-block, d = 1, dmin = 0, sc = 1, s = 1:
    # term_g = sa_g; sa = [1, t, t, t, t, 0.5, -0.5, -1] with t = 2^-24
    nib = np.zeros(256, np.int64)
    qa = np.zeros(256, np.int64)
    for g in range(8):
        nib[g * 32] = 1
        qa[g * 32] = 1
    t = 2.0 ** -24
    sas = np.array([1, t, t, t, t, 0.5, -0.5, -1], np.float32)
    got = oracle_row(Q4_K, [q4_k_block(1.0, 0.0, np.ones(8, np.int64), np.zeros(8, np.int64), nib)], 256, qa, sas)
    # left to right: 1 (ties keep 1) +0.5 -> 1.5, -0.5 -> 1.0, -1 -> 0
    assert bits(got) == bits(f32(0.0))
    sas = np.array([1, t, t, t, t, 0, 0, 0], np.float32)
    got = oracle_row(Q4_K, [q4_k_block(1.0, 0.0, np.ones(8, np.int64), np.zeros(8, np.int64), nib)], 256, qa, sas)
    assert bits(got) == bits(f32(1.0))


# ------------------------------------------------------------------ Q6_K (kquant.rs:313-314): ((d*sa)*sc)*float(isum16)
def test_q6_k_term_parenthesisation_pinned():
    rng = np.random.default_rng(4)

    def sample(r):
        d = f16_val(r.uniform(0.001, 0.05))
        sa = f32(r.uniform(0.001, 0.1))
        sc = int(r.integers(-128, 128))
        q = r.integers(-32, 32, 16)
        qa = r.integers(-127, 128, 16)
        return d, sa, sc, q, qa

    ref = lambda d, sa, sc, q, qa: f32(f32(d * sa) * f32(sc)) * f32(int(np.dot(q, qa)))
    alts = [lambda d, sa, sc, q, qa: f32(d * sa) * f32(f32(sc) * f32(int(np.dot(q, qa)))),
            lambda d, sa, sc, q, qa: f32(f32(d * f32(sc)) * sa) * f32(int(np.dot(q, qa)))]
    for sub in (0, 5, 14):  # sub-blocks in both halves and both 16-lane slots
        (d, sa, sc, q, qa), want = find_distinguishing(ref, alts, sample, rng)
        qs = np.zeros(256, np.int64)
        qs[sub * 16:(sub + 1) * 16] = q
        qa256 = np.zeros(256, np.int64)
        qa256[sub * 16:(sub + 1) * 16] = qa
        scs = np.zeros(16, np.int64)
        scs[sub] = sc
        sas = np.full(8, 0.25, np.float32)
        sas[sub // 2] = sa
        got = oracle_row(Q6_K, [q6_k_block(d, scs, qs)], 256, qa256, sas)
        assert bits(got) == bits(f32(0.0) + want)


def test_q6_k_subblock_fold_half_ulp_ties():
    # 16 sub-block terms of one block, d = 1, sc = 1, isum = 1 per sub-block,
    # sa per 32-group: terms [1, 1, t, t, t, t, ...]: 1 + 1 = 2, then ties at
    # 2^-23 (half an ulp of 2) twice per group -> stays 2.0.
    q = np.zeros(256, np.int64)
    qa = np.zeros(256, np.int64)
    for s in range(16):
        q[s * 16] = 1
        qa[s * 16] = 1
    sas = np.array([1] + [2.0 ** -23] * 7, np.float32)
    got = oracle_row(Q6_K, [q6_k_block(1.0, np.ones(16, np.int64), q)], 256, qa, sas)
    assert bits(got) == bits(f32(2.0))
    assert f32(2.0) + f32(14 * 2.0 ** -23) != f32(2.0)


# ------------------------------------------------------------------ layer wiring: independent float64 forward
def _rope64(x, pos, hd, theta, neox):
    """attention.rs:90-121 restated in float64 on one [heads*hd] row."""
    x = x.copy()
    for h0 in range(0, len(x), hd):
        if neox:
            half = hd // 2
            for j in range(half):
                ang = pos * theta ** (-(2.0 * j) / hd)
                a, b = x[h0 + j], x[h0 + j + half]
                x[h0 + j], x[h0 + j + half] = a * np.cos(ang) - b * np.sin(ang), a * np.sin(ang) + b * np.cos(ang)
        else:
            for j in range(0, hd, 2):
                ang = pos * theta ** (-float(j) / hd)
                a, b = x[h0 + j], x[h0 + j + 1]
                x[h0 + j], x[h0 + j + 1] = a * np.cos(ang) - b * np.sin(ang), a * np.sin(ang) + b * np.cos(ang)
    return x


class Forward64:
    """prana-model forward_impl (infer.rs:142-211) in float64 numpy, with the
    K/V cache rounded to f16 as the reference stores it. `mistake` plants one
    wiring error for the power check."""

    def __init__(self, cfg, tensors, mistake=None):
        self.c, self.m = cfg, mistake
        self.w = {k: np.frombuffer(v[2].tobytes(), np.float32).astype(np.float64).reshape(tuple(reversed(v[1])))
                  for k, v in tensors.items()}
        self.k = [[] for _ in range(cfg["n_layers"])]
        self.v = [[] for _ in range(cfg["n_layers"])]

    def rms(self, x, w):
        return x / np.sqrt(np.mean(x * x) + self.c["norm_eps"]) * w

    def step(self, tok, pos):
        c, w = self.c, self.w
        hd, H, KV = c["head_dim"], c["n_heads"], c["n_kv_heads"]
        x = w["token_embd.weight"][tok].copy()
        for l in range(c["n_layers"]):
            b = f"blk.{l}."
            xb = self.rms(x, w[b + "attn_norm.weight"])
            q, k, v = (w[b + "attn_q.weight"] @ xb, w[b + "attn_k.weight"] @ xb, w[b + "attn_v.weight"] @ xb)
            biased = b + "attn_q.bias" in w
            if biased and self.m != "bias_after_rope":
                q, k = q + w[b + "attn_q.bias"], k + w[b + "attn_k.bias"]
                v = v + (w[b + "attn_q.bias"][: len(v)] if self.m == "v_bias_from_q" else w[b + "attn_v.bias"])
            neox = c["rope_neox"] if self.m != "other_rope_form" else 1 - c["rope_neox"]
            q = _rope64(q, pos, hd, c["rope_theta"], neox)
            if self.m != "no_rope_on_k":
                k = _rope64(k, pos, hd, c["rope_theta"], neox)
            if biased and self.m == "bias_after_rope":
                q, k, v = q + w[b + "attn_q.bias"], k + w[b + "attn_k.bias"], v + w[b + "attn_v.bias"]
            self.k[l].append(k.astype(np.float16).astype(np.float64))
            self.v[l].append(v.astype(np.float16).astype(np.float64))
            K, V = np.array(self.k[l]), np.array(self.v[l])
            att = np.zeros(H * hd)
            for h in range(H):
                kh = h // (H // KV)
                sc = K[:, kh * hd:(kh + 1) * hd] @ q[h * hd:(h + 1) * hd] / np.sqrt(hd)
                p = np.exp(sc - sc.max())
                p /= p.sum()
                att[h * hd:(h + 1) * hd] = p @ V[:, kh * hd:(kh + 1) * hd]
            x = x + w[b + "attn_output.weight"] @ att
            xb = self.rms(x, w[b + "ffn_norm.weight"])
            g, u = w[b + "ffn_gate.weight"] @ xb, w[b + "ffn_up.weight"] @ xb
            if self.m == "silu_on_up":
                g, u = u, g
            h = g / (1.0 + np.exp(-g)) * u
            x = x + w[b + "ffn_down.weight"] @ h
        xf = self.rms(x, w["output_norm.weight"])
        head = w["output.weight"] if "output.weight" in w else w["token_embd.weight"]
        return head @ xf


def rel_err(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - b)) / np.max(np.abs(b)))


def tiny_model(arch, scale):
    """The reference's tiny test model (gguf.rs:567-666); scale > 1 multiplies
    the projections (and the embedding by 10) so every sub-layer moves the
    logits by a visible amount."""
    cfg, t = fx.synthetic_model(arch, arch == "qwen2")
    if scale == 1:
        return cfg, t
    out = {}
    for k, (ty, dims, raw) in t.items():
        a = np.frombuffer(raw.tobytes(), np.float32).copy()
        if k == "token_embd.weight":
            a = (a * f32(10)).astype(np.float32)
        elif k.endswith(".weight") and "norm" not in k:
            a = (a * f32(scale)).astype(np.float32)
        out[k] = (ty, dims, a.view(np.uint8))
    return cfg, out


TOKS = [5, 3, 9, 44, 0, 17, 30]


@pytest.mark.parametrize("arch", ["llama", "qwen2"])
@pytest.mark.parametrize("scale", [1, 8])
def test_oracle_forward_matches_independent_float64_forward(arch, scale):
    cfg, t = tiny_model(arch, scale)
    oc = O.Model(cfg, t).cache(16)
    ref = Forward64(cfg, t)
    for pos, tok in enumerate(TOKS):
        err = rel_err(oc.forward(tok, pos), ref.step(tok, pos))
        assert err < 1e-4, (pos, err)


@pytest.mark.parametrize("arch,mistake", [("llama", "silu_on_up"), ("llama", "no_rope_on_k"),
                                          ("llama", "other_rope_form"), ("qwen2", "silu_on_up"),
                                          ("qwen2", "no_rope_on_k"), ("qwen2", "other_rope_form"),
                                          ("qwen2", "v_bias_from_q"), ("qwen2", "bias_after_rope")])
def test_float64_forward_has_power_against_wiring_mistakes(arch, mistake):
    cfg, t = tiny_model(arch, 8)
    oc = O.Model(cfg, t).cache(16)
    bad = Forward64(cfg, t, mistake)
    worst = max(rel_err(oc.forward(tok, pos), bad.step(tok, pos)) for pos, tok in enumerate(TOKS))
    assert worst > 1e-3, worst  # ten times the tolerance the oracle meets
