"""Distinguishing inputs for the elementwise final-rounding expressions.

For each expression of the reference's scalar path this module evaluates the
reference's own expression independently (numpy float32 operations, each one
IEEE-rounded, and the platform libm that Rust's `f32::exp` / `tanh` / `powf` /
`sin_cos` resolve to on x86_64-linux-gnu) next to the plausible alternatives a
restatement could get wrong, and searches for inputs on which every
alternative gives other bits. The CPU pins check the oracle against the
reference expression on those inputs; the GPU pins run the same inputs through
the device kernels and compare with the oracle bit for bit.

Expressions (reference file:line, Rust `a * b * c` is `(a * b) * c`):
  quantize_acts  scale = amax/127; inv = 1/scale; q = round(x*inv)  matmul.rs:116-123
  rmsnorm        ms = (fold x*x)/dim; inv = 1/sqrt(ms+eps); (x*inv)*w norms.rs:15-19
  silu           v * (1/(1+exp(-v)))                                norms.rs:29
  gelu_tanh      (0.5*v) * (1 + tanh(S*(v + 0.044715*((v*v)*v))))   norms.rs:37-39
  softmax        e_t = exp(v_t - max); p_t = e_t * (1/fold e)       norms.rs:49-54
  attention      score = (fold q*k) * (1/sqrt(hd))                  attention.rs:174-184
  RoPE           angle = (pos as f32) * freq, f32 product           attention.rs:96, 115
"""
import ctypes
import ctypes.util

import numpy as np

f32 = np.float32
_libm = ctypes.CDLL(ctypes.util.find_library("m"))
for _n in ("expf", "tanhf", "sinf", "cosf", "sqrtf"):
    getattr(_libm, _n).restype = ctypes.c_float
    getattr(_libm, _n).argtypes = [ctypes.c_float]
_libm.powf.restype = ctypes.c_float
_libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]
_libm.sin.restype = ctypes.c_double
_libm.sin.argtypes = [ctypes.c_double]
_libm.cos.restype = ctypes.c_double
_libm.cos.argtypes = [ctypes.c_double]


def expf(x):
    return f32(_libm.expf(float(x)))


def tanhf(x):
    return f32(_libm.tanhf(float(x)))


def powf(a, b):
    return f32(_libm.powf(float(a), float(b)))


def bits(x):
    return np.asarray(x, np.float32).view(np.uint32)


def differs(a, b):
    """True when the two float32 arrays differ in any bit pattern."""
    return bool(np.any(bits(a) != bits(b)))


def round_half_away(v):
    """Rust f32::round: halfway cases away from zero."""
    v = np.asarray(v, np.float32)
    return (np.sign(v) * np.floor(np.abs(v).astype(np.float64) + 0.5)).astype(np.float32)


# ------------------------------------------------------------------ quantize_acts
def quantize_ref(x, scale_mode="div", q_mode="mul_inv", rounding="away"):
    """One 32-block in the reference's steps; the keyword arguments select the
    alternatives: scale amax*(1/127), q from x/scale, round-half-even."""
    x = np.asarray(x, np.float32)
    amax = f32(0.0)
    for v in x:
        amax = max(amax, abs(v))
    if amax > 0:
        scale = f32(amax / f32(127.0)) if scale_mode == "div" else f32(amax * f32(f32(1.0) / f32(127.0)))
    else:
        scale = f32(1.0)
    inv = f32(f32(1.0) / scale)
    y = (x * inv).astype(np.float32) if q_mode == "mul_inv" else (x / scale).astype(np.float32)
    r = round_half_away(y) if rounding == "away" else np.rint(y).astype(np.float32)
    q = np.clip(r, -127, 127).astype(np.int32)
    return q, scale, int(q.sum())


def quantize_case_div_vs_mul():
    """A block whose q differs between round(x*inv) and round(x/scale): x is
    walked ulp by ulp across a half-integer boundary of x/scale."""
    for amax in (f32(1.7), f32(3.1), f32(0.37), f32(12.9), f32(5.3)):
        scale = f32(amax / f32(127.0))
        inv = f32(f32(1.0) / scale)
        for k in range(40, 127):
            x0 = f32((k + 0.5) * float(scale))
            x = x0
            for _ in range(64):
                a = round_half_away(f32(x * inv))
                b = round_half_away(f32(x / scale))
                if a != b and abs(x) <= amax:
                    blk = np.zeros(32, np.float32)
                    blk[0], blk[7] = amax, x
                    blk[8:] = np.linspace(-0.3, 0.2, 24, dtype=np.float32) * amax
                    return blk
                x = np.nextafter(x, f32(np.inf), dtype=np.float32)
    raise AssertionError("no block separates x*inv from x/scale")


def quantize_case_scale():
    """A block whose scale differs between amax/127 and amax*(1/127)."""
    rng = np.random.default_rng(7)
    for _ in range(10000):
        amax = f32(rng.uniform(0.01, 10.0))
        if f32(amax / f32(127.0)) != f32(amax * f32(f32(1.0) / f32(127.0))):
            blk = rng.standard_normal(32).astype(np.float32)
            blk *= amax / np.max(np.abs(blk))
            blk[np.argmax(np.abs(blk))] = amax
            return blk.astype(np.float32)
    raise AssertionError("no amax separates the two scales")


def quantize_case_half_away():
    """amax = 127 gives scale = inv = 1 exactly, so x*inv = x: the halves
    2.5, -0.5, 126.5 round away from zero (3, -1, 127), not to even."""
    blk = np.zeros(32, np.float32)
    blk[:6] = [127.0, 2.5, -0.5, 0.5, -3.5, 126.5]
    return blk


# ------------------------------------------------------------------ rmsnorm
def rmsnorm_ref(x, w, eps, variant="ref"):
    x = np.asarray(x, np.float32)
    w = np.asarray(w, np.float32)
    dim = x.size
    if variant == "pairwise_sum":
        ss = f32(np.sum((x * x).astype(np.float32), dtype=np.float32))
    else:
        ss = f32(-0.0)
        for v in x:
            ss = f32(ss + f32(v * v))
    if variant == "mul_recip_dim":
        ms = f32(ss * f32(f32(1.0) / f32(dim)))
    else:
        ms = f32(ss / f32(dim))
    if variant == "sqrt_of_recip":
        inv = f32(np.sqrt(f32(f32(1.0) / f32(ms + f32(eps)))))
    else:
        inv = f32(f32(1.0) / f32(np.sqrt(f32(ms + f32(eps)))))
    if variant == "inv_times_w":
        return (x * (inv * w).astype(np.float32)).astype(np.float32)
    if variant == "x_times_w_first":
        return ((x * w).astype(np.float32) * inv).astype(np.float32)
    return ((x * inv).astype(np.float32) * w).astype(np.float32)


RMS_ALTS = ("pairwise_sum", "mul_recip_dim", "sqrt_of_recip", "inv_times_w", "x_times_w_first")


def rmsnorm_case(dim=96, eps=1e-5):
    """A row and non-unit weights on which every alternative differs."""
    rng = np.random.default_rng(11)
    for _ in range(2000):
        x = (rng.standard_normal(dim) * rng.uniform(0.1, 30.0)).astype(np.float32)
        w = rng.uniform(0.5, 1.5, dim).astype(np.float32)
        ref = rmsnorm_ref(x, w, eps)
        if all(differs(rmsnorm_ref(x, w, eps, a), ref) for a in RMS_ALTS):
            return x, w, f32(eps)
    raise AssertionError("no row separates every rmsnorm alternative")


# ------------------------------------------------------------------ silu, gelu_tanh
def silu_ref(v, variant="ref"):
    out = np.empty_like(np.asarray(v, np.float32))
    for i, x in enumerate(np.asarray(v, np.float32)):
        if variant == "div":
            out[i] = f32(x / f32(f32(1.0) + expf(-x)))
        elif variant == "recip_exp":
            out[i] = f32(x * f32(f32(1.0) / f32(f32(1.0) + f32(f32(1.0) / expf(x)))))
        else:
            out[i] = f32(x * f32(f32(1.0) / f32(f32(1.0) + expf(-x))))
    return out


SILU_ALTS = ("div", "recip_exp")


def silu_case(n=512):
    rng = np.random.default_rng(3)
    v = rng.uniform(-12.0, 12.0, n).astype(np.float32)
    return v


S_GELU = f32(0.7978846)
C_GELU = f32(0.044715)


def gelu_ref(v, variant="ref"):
    out = np.empty_like(np.asarray(v, np.float32))
    for i, x in enumerate(np.asarray(v, np.float32)):
        x3 = f32(f32(x * x) * x)
        if variant == "distributed":
            inner = f32(f32(S_GELU * x) + f32(f32(S_GELU * C_GELU) * x3))
        elif variant == "c_first":
            inner = f32(S_GELU * f32(x + f32(f32(f32(C_GELU * x) * x) * x)))
        else:
            inner = f32(S_GELU * f32(x + f32(C_GELU * x3)))
        t = tanhf(inner)
        if variant == "half_last":
            out[i] = f32(f32(0.5) * f32(x * f32(f32(1.0) + t)))
        else:
            out[i] = f32(f32(f32(0.5) * x) * f32(f32(1.0) + t))
    return out


GELU_ALTS = ("c_first", "distributed", "half_last")


def gelu_case(n=512):
    """Random values, one value per alternative on which that alternative
    changes the output bits (found by search), and one large enough that
    x*(1+t) overflows while (0.5*x)*(1+t) does not: the only place where the
    0.5's position shows."""
    rng = np.random.default_rng(5)
    v = rng.uniform(-6.0, 6.0, n).astype(np.float32)
    v[0] = f32(3.0e38)
    # tanh's argument is formed in numpy for a large pool (vectorized, each
    # operation rounded to f32); libm's tanhf only runs where the argument
    # differs, and a candidate counts once the whole expression differs
    pool = rng.uniform(-3.5, 3.5, 400000).astype(np.float32)
    x3_ref = (pool * pool).astype(np.float32) * pool
    inner_ref = S_GELU * (pool + C_GELU * x3_ref)
    alts = {"c_first": S_GELU * (pool + ((C_GELU * pool) * pool) * pool),
            "distributed": (S_GELU * pool) + (S_GELU * C_GELU) * x3_ref}
    for slot, alt in enumerate(("c_first", "distributed"), start=1):
        cand = np.nonzero(bits(alts[alt]) != bits(inner_ref))[0]
        for i in cand:
            if bits(gelu_ref(pool[i:i + 1], alt)) != bits(gelu_ref(pool[i:i + 1])):
                v[slot] = pool[i]
                break
        else:
            raise AssertionError(f"no value separates gelu alternative {alt}")
    return v


# ------------------------------------------------------------------ softmax
def softmax_ref(v, variant="ref"):
    v = np.asarray(v, np.float32)
    mx = f32(-np.inf)
    for x in v:
        mx = max(mx, x)
    e = np.array([expf(f32(x - mx)) for x in v], np.float32)
    if variant == "pairwise_sum":
        s = f32(np.sum(e, dtype=np.float32))
    else:
        s = f32(-0.0)
        for x in e:
            s = f32(s + x)
    if variant == "div":
        return (e / s).astype(np.float32)
    inv = f32(f32(1.0) / s) if s > 0 else f32(0.0)
    return (e * inv).astype(np.float32)


SOFTMAX_ALTS = ("div", "pairwise_sum")


def softmax_case(n=300):
    rng = np.random.default_rng(13)
    for _ in range(200):
        v = (rng.standard_normal(n) * 3.0).astype(np.float32)
        ref = softmax_ref(v)
        if all(differs(softmax_ref(v, a), ref) for a in SOFTMAX_ALTS):
            return v
    raise AssertionError("no row separates the softmax alternatives")


# ------------------------------------------------------------------ attention score scale
def attention_ref(q, kc, vc, pos, nh, nkv, hd, variant="ref"):
    """decode_one_head for every head (attention.rs:165-195) over an f16
    cache; variant "div_sqrt" scores dot/sqrt(hd) instead of dot*(1/sqrt(hd))."""
    q = np.asarray(q, np.float32)
    kf = np.asarray(kc, np.uint16).view(np.float16).astype(np.float32)
    vf = np.asarray(vc, np.uint16).view(np.float16).astype(np.float32)
    kv_stride, group = nkv * hd, nh // nkv
    sq = f32(np.sqrt(f32(hd)))
    scale = f32(f32(1.0) / sq)
    out = np.zeros(nh * hd, np.float32)
    for h in range(nh):
        kvh = h // group
        qh = q[h * hd:(h + 1) * hd]
        scores = np.empty(pos + 1, np.float32)
        for t in range(pos + 1):
            kr = kf[t * kv_stride + kvh * hd:t * kv_stride + (kvh + 1) * hd]
            dot = f32(-0.0)
            for d in range(hd):
                dot = f32(dot + f32(qh[d] * kr[d]))
            scores[t] = f32(dot / sq) if variant == "div_sqrt" else f32(dot * scale)
        p = softmax_ref(scores)
        acc = np.zeros(hd, np.float32)
        for t in range(pos + 1):
            vr = vf[t * kv_stride + kvh * hd:t * kv_stride + (kvh + 1) * hd]
            acc = (acc + (p[t] * vr).astype(np.float32)).astype(np.float32)
        out[h * hd:(h + 1) * hd] = acc
    return out


def attention_case(hd, nh=2, nkv=1, pos=5):
    """Seeded q and cache on which dot/sqrt(hd) changes the output bits."""
    for seed in range(200):
        rng = np.random.default_rng(1000 * hd + seed)
        q = (rng.standard_normal(nh * hd) * 0.6).astype(np.float32)
        rows = pos + 1
        kc = (rng.standard_normal(rows * nkv * hd)).astype(np.float16).view(np.uint16)
        vc = (rng.standard_normal(rows * nkv * hd)).astype(np.float16).view(np.uint16)
        ref = attention_ref(q, kc, vc, pos, nh, nkv, hd)
        if differs(attention_ref(q, kc, vc, pos, nh, nkv, hd, "div_sqrt"), ref):
            return q, kc, vc, pos, nh, nkv, hd
    raise AssertionError("no case separates dot*(1/sqrt(hd)) from dot/sqrt(hd)")


# ------------------------------------------------------------------ RoPE angle
def rope_ref(x, pos, hd, theta, neox, variant="ref"):
    """rope_neox / rope_interleaved (attention.rs:90-121) on one row; variant
    "f64_angle" forms the angle and its sine / cosine in double precision."""
    x = np.array(x, np.float32, copy=True)
    theta = f32(theta)

    def sc(freq):
        if variant == "f64_angle":
            a = float(pos) * float(freq)
            return f32(_libm.sin(a)), f32(_libm.cos(a))
        a = f32(f32(pos) * freq)
        return f32(_libm.sinf(float(a))), f32(_libm.cosf(float(a)))

    def rot(x0, x1, s, c):
        return f32(f32(x0 * c) - f32(x1 * s)), f32(f32(x0 * s) + f32(x1 * c))

    if neox:
        half = hd // 2
        for h in range(x.size // hd):
            b = h * hd
            for j in range(half):
                freq = powf(theta, f32(f32(-f32(f32(2.0) * f32(j))) / f32(hd)))
                s, c = sc(freq)
                x[b + j], x[b + j + half] = rot(x[b + j], x[b + j + half], s, c)
    else:
        for i in range(0, x.size, 2):
            j = i % hd
            freq = powf(theta, f32(f32(-f32(j)) / f32(hd)))
            s, c = sc(freq)
            x[i], x[i + 1] = rot(x[i], x[i + 1], s, c)
    return x


ROPE_POSITIONS = (1024, 4095, 16384, 32767)


def rope_case(hd=128, n_heads=2, seed=17):
    rng = np.random.default_rng(seed)
    return rng.standard_normal(n_heads * hd).astype(np.float32)
