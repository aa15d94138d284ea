"""GPU parity: every kernel entry point of libprana_hip against the CPU oracle
on the same seeded inputs. Integer and f32 results must be bit-identical
(compared as raw bits)."""
import numpy as np
import pytest

import prana_amd as P
from oracle import oracle as O
from tests import fixtures as fx

pytestmark = pytest.mark.gpu


def same_bits(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def rng(seed):
    return np.random.default_rng(seed)


# ------------------------------------------------------------------ quantize_acts
@pytest.mark.parametrize("rows,k", [(1, 32), (3, 288), (2, 4096), (5, 14336)])
def test_quantize_acts(rows, k):
    x = rng(k).standard_normal((rows, k)).astype(np.float32) * 2
    x[0, :32] = 0.0            # zero block
    x[-1, -32:] *= 1e-30       # tiny block
    q, s, m = P.quantize_acts(x)
    qo, so, mo = O.quantize_acts(x)
    assert np.array_equal(q, qo) and same_bits(s, so) and np.array_equal(m, mo)


# ------------------------------------------------------------------ matmul per format
def _mat_pair(ty, rows, cols, seed, real=False):
    if real:
        raw = P.synth_tensor(ty, rows, cols, seed, 0.02)
    else:
        raw = fx.pseudo_blocks(ty, rows, cols, seed)
    return raw, P.Matrix(ty, rows, cols, raw), O.Mat.from_ggml(ty, rows, cols, raw)


@pytest.mark.parametrize("ty", [fx.Q8_0, fx.Q4_0, fx.Q4_K, fx.Q6_K])
@pytest.mark.parametrize("n_tok", [1, 3])
def test_matmul_formats_small(ty, n_tok):
    rows, cols = 37, 512
    raw, g, o = _mat_pair(ty, rows, cols, 21 + n_tok)
    a = fx.sin_row(n_tok * cols, 0.013).reshape(n_tok, cols)
    assert same_bits(g.apply(a), o.apply(a))


@pytest.mark.parametrize("ty", [fx.Q8_0, fx.Q4_0, fx.Q4_K, fx.Q6_K])
def test_block_sums_exact(ty):
    rows, cols = 19, 1024
    raw, g, o = _mat_pair(ty, rows, cols, 5)
    a = rng(9).standard_normal((2, cols)).astype(np.float32)
    q, s, m = O.quantize_acts(a)
    got = g.block_sums(q, m)
    for t in range(2):
        assert np.array_equal(got[t], fx.np_block_isums(ty, raw, rows, cols, q[t]))


@pytest.mark.parametrize("shape", [(4096, 4096), (14336, 4096), (4096, 14336), (32000, 4096)])
@pytest.mark.parametrize("n_tok", [1, 4])
def test_q8_0_config1_shapes(shape, n_tok):
    rows, cols = shape
    raw, g, o = _mat_pair(fx.Q8_0, rows, cols, 100 + rows + cols, real=True)
    a = rng(rows).standard_normal((n_tok, cols)).astype(np.float32)
    assert same_bits(g.apply(a), o.apply(a))


@pytest.mark.parametrize("shape", [(6144, 4096), (4096, 14336)])
def test_q4_0_7b_shapes(shape):
    rows, cols = shape
    raw, g, o = _mat_pair(fx.Q4_0, rows, cols, 7, real=True)
    a = rng(3).standard_normal((1, cols)).astype(np.float32)
    assert same_bits(g.apply(a), o.apply(a))


def test_matmul_prefill_rows_equal_decode():
    rows, cols, n = 300, 896, 6
    raw, g, o = _mat_pair(fx.Q4_0, rows, cols, 31, real=True)
    a = rng(4).standard_normal((n, cols)).astype(np.float32)
    q, s, m = O.quantize_acts(a)
    pre = g.apply_prefill(q, s, m)
    assert same_bits(pre, o.apply_prefill(q, s, m))
    for t in range(n):
        assert same_bits(pre[t], g.apply(a[t])[0])


@pytest.mark.parametrize("ty", [fx.Q8_0, fx.Q4_0, fx.Q4_K, fx.Q6_K])
@pytest.mark.parametrize("rows,cols,n_tok", [(37, 512, 17), (300, 1024, 33), (129, 256, 70), (37, 512, 5),
                                             (300, 1024, 9), (129, 768, 16), (1000, 512, 48), (64, 1280, 64),
                                             (70, 256, 31)])
def test_matmul_batched(ty, rows, cols, n_tok):
    # Batches of up to 8 tokens: the decode kernel (one launch); 9..64 tokens:
    # the skinny int8 matrix-core kernel for block-32 kinds (ragged row and
    # token tiles, block counts that are not whole fetch groups); more than 64:
    # the LDS-staged 32x32 matrix-core kernel; K-quants above 16 tokens: the
    # K-quant matrix-core kernel
    raw, g, o = _mat_pair(ty, rows, cols, 41 + n_tok, real=True)
    a = rng(n_tok).standard_normal((n_tok, cols)).astype(np.float32)
    assert same_bits(g.apply(a), o.apply(a))


@pytest.mark.parametrize("ty", [fx.Q8_0, fx.Q4_0])
@pytest.mark.parametrize("rows,cols,n_tok", [(300, 1312, 13), (16, 4128, 16), (4100, 256, 9)])
def test_matmul_skinny_block_split_ragged(ty, rows, cols, n_tok):
    # 9..16 tokens over fewer than 8192 rows: four waves take consecutive
    # chunks of 8 blocks and one lane per output folds their terms; 41 and 129
    # blocks leave a partial chunk and a partial group of four chunks, 8 blocks
    # leave three waves with nothing live
    raw, g, o = _mat_pair(ty, rows, cols, 7 + n_tok, real=True)
    a = rng(n_tok).standard_normal((n_tok, cols)).astype(np.float32)
    assert same_bits(g.apply(a), o.apply(a))


@pytest.mark.parametrize("ty", [fx.Q8_0, fx.Q4_0])
@pytest.mark.parametrize("rows,cols,n_tok", [(37, 2048, 10), (300, 4096, 12), (129, 7168, 8), (70, 14336, 3),
                                             (70, 14336, 6), (4097, 4096, 9), (515, 14336, 16), (4100, 14336, 2),
                                             (4100, 14336, 3), (4100, 14336, 5), (12300, 4096, 7)])
def test_matmul_verify_batch_chunked(ty, rows, cols, n_tok):
    # Widths of 2, 4, 7 or 14 chunks of 32 or 64 blocks: the chunk-major
    # multi-token kernel (activations and term rows staged one chunk at a
    # time) takes rows of more than 128 blocks at 2..8 tokens; from 9 tokens,
    # and from 3 tokens for matrices of at least 1.5M blocks, the skinny
    # matrix-core kernel takes the batch. Ragged last tiles.
    raw, g, o = _mat_pair(ty, rows, cols, 60 + n_tok + cols, real=True)
    a = rng(n_tok + 3).standard_normal((n_tok, cols)).astype(np.float32)
    assert same_bits(g.apply(a), o.apply(a))


def test_matmul_verify_batch_chunked_q8_f32_scales():
    w = rng(13).standard_normal((70, 14336)).astype(np.float32)
    q, s = O.quantize_q8(w)
    g, o = P.Matrix.q8_parts(q, s), O.Mat.q8_parts(q, s)
    for n_tok in (3, 6):
        a = rng(19 + n_tok).standard_normal((n_tok, 14336)).astype(np.float32)
        assert same_bits(g.apply(a), o.apply(a))


@pytest.mark.parametrize("ty", [fx.Q8_0, fx.Q4_0])
@pytest.mark.parametrize("rows,cols,n_tok", [(150, 288, 100), (33, 1312, 97), (129, 96, 65)])
def test_matmul_prefill_partial_chunks(ty, rows, cols, n_tok):
    # The staged prefill kernel takes blocks in chunks of four: 9, 41 and 3
    # blocks per row leave a partial last chunk; rows and tokens are ragged
    # against its 128-row x 32-token tiles.
    raw, g, o = _mat_pair(ty, rows, cols, 77 + n_tok, real=True)
    a = rng(n_tok + 1).standard_normal((n_tok, cols)).astype(np.float32)
    assert same_bits(g.apply(a), o.apply(a))


@pytest.mark.parametrize("n_tok", [16, 64])
@pytest.mark.parametrize("shape", [(4096, 4096), (4096, 14336)])
def test_matmul_batched_config1(shape, n_tok):
    rows, cols = shape
    raw, g, o = _mat_pair(fx.Q8_0, rows, cols, 200 + cols, real=True)
    a = rng(n_tok).standard_normal((n_tok, cols)).astype(np.float32)
    assert same_bits(g.apply(a), o.apply(a))


@pytest.mark.parametrize("n_tok", [40, 7, 100])
def test_q8_f32_scales_parts_batched(n_tok):
    w = rng(12).standard_normal((96, 256)).astype(np.float32)
    q, s = O.quantize_q8(w)
    g, o = P.Matrix.q8_parts(q, s), O.Mat.q8_parts(q, s)
    a = rng(18).standard_normal((n_tok, 256)).astype(np.float32)
    assert same_bits(g.apply(a), o.apply(a))


def test_q8_f32_scales_parts():
    w = rng(2).standard_normal((64, 256)).astype(np.float32)
    q, s = O.quantize_q8(w)
    g, o = P.Matrix.q8_parts(q, s), O.Mat.q8_parts(q, s)
    a = rng(8).standard_normal((2, 256)).astype(np.float32)
    assert same_bits(g.apply(a), o.apply(a))


@pytest.mark.parametrize("cols", [32, 288, 301])
def test_dense_f32(cols):
    w = rng(cols).standard_normal((70, cols)).astype(np.float32)
    a = rng(cols + 1).standard_normal((3, cols)).astype(np.float32)
    g = P.Matrix(fx.F32, 70, cols, w.view(np.uint8).reshape(-1))
    assert same_bits(g.apply(a), O.Mat.f32(w).apply(a))


@pytest.mark.parametrize("ty", [fx.F32, fx.Q8_0, fx.Q4_0, fx.Q4_K, fx.Q6_K])
def test_embed_rows(ty):
    rows, cols = 50, 512
    if ty == fx.F32:
        w = rng(1).standard_normal((rows, cols)).astype(np.float32)
        raw = w.view(np.uint8).reshape(-1)
    else:
        raw = fx.pseudo_blocks(ty, rows, cols, 17)
    g = P.Matrix(ty, rows, cols, raw)
    toks = [0, 7, 49, 7]
    got = g.embed_rows(toks)
    ref = fx.np_dequant(ty, raw, rows, cols) if ty != fx.F32 else w
    om = O.Mat.from_ggml(ty, rows, cols, raw)
    for i, t in enumerate(toks):
        assert same_bits(got[i], om.row_f32(t))
    assert np.allclose(got, ref[toks], rtol=0, atol=1e-6)
    assert same_bits(g.embed_rows([3], scale=2.5)[0], om.row_f32(3) * np.float32(2.5))


# ------------------------------------------------------------------ norms / activations
@pytest.mark.parametrize("rows,dim", [(1, 288), (4, 896), (2, 4096)])
def test_rmsnorm(rows, dim):
    x = rng(dim).standard_normal((rows, dim)).astype(np.float32)
    w = (1 + 0.1 * rng(dim + 1).standard_normal(dim)).astype(np.float32)
    assert same_bits(P.rmsnorm(x, w, 1e-5), O.rmsnorm(x, w, 1e-5))


def _adversarial_rows(dim, seed):
    """Rows whose squares stress the exact sequential sum: ties against the
    running sum, powers of two, subnormal squares, zeros, overflow to inf,
    a wide dynamic range and non-finite inputs."""
    r = rng(seed)
    rows = [
        np.ldexp(1.0, -r.integers(0, 20, dim)).astype(np.float32),            # exact power-of-two squares
        np.where(np.arange(dim) == 0, 1.0, 2.0 ** -12).astype(np.float32),      # half-ulp ties against 1.0
        (np.exp2(r.uniform(-70, 30, dim)) * r.choice([-1, 1], dim)).astype(np.float32),  # wide range
        (r.integers(1, 1 << 10, dim) * 2.0 ** -80).astype(np.float32),          # subnormal squares
        np.where(r.random(dim) < 0.5, 0.0, r.standard_normal(dim)).astype(np.float32),
        np.full(dim, 1e19, np.float32),                                         # sum overflows to inf
        np.zeros(dim, np.float32),
        r.standard_normal(dim).astype(np.float32) * 1e-3,
    ]
    bad = r.standard_normal(dim).astype(np.float32)
    bad[dim // 2] = np.nan
    rows.append(bad)
    inf = r.standard_normal(dim).astype(np.float32)
    inf[-1] = np.inf
    rows.append(inf)
    return np.stack(rows)


@pytest.mark.parametrize("dim", [32, 288, 512, 544, 1000, 2080, 3072, 4096, 4128, 14336, 16320, 16384, 20000])
def test_rmsnorm_adversarial(dim):
    x = _adversarial_rows(dim, dim)
    w = np.ones(dim, np.float32)
    got, want = P.rmsnorm(x, w, 1e-6), O.rmsnorm(x, w, 1e-6)
    for i in range(x.shape[0]):
        assert same_bits(got[i], want[i]), i


@pytest.mark.parametrize("dim", [64, 288, 896, 2048, 4096, 5120, 8192])
def test_rmsnorm_register_runs_many_rows(dim):
    # The register-run exact sum (dims % 32 == 0 up to 8192): typical rows
    # (normal, scaled, heavy-tailed, near-constant) and tie-rich rows (small
    # integers, powers of two) that take its fallback, all bit-exact.
    r = rng(dim + 7)
    rows = []
    for k in range(48):
        v = r.standard_normal(dim)
        kind = k % 6
        if kind == 1:
            v = v * 1e-3
        elif kind == 2:
            v = v * np.exp(2.0 * r.standard_normal(dim))
        elif kind == 3:
            v = 1.0 + 1e-3 * v
        elif kind == 4:
            v = np.round(v * 8)
        elif kind == 5:
            v = np.ldexp(1.0, r.integers(-8, 8, dim))
        rows.append(v)
    x = np.stack(rows).astype(np.float32)
    w = (1 + 0.1 * r.standard_normal(dim)).astype(np.float32)
    got, want = P.rmsnorm(x, w, 1e-5), O.rmsnorm(x, w, 1e-5)
    for i in range(x.shape[0]):
        assert same_bits(got[i], want[i]), i


@pytest.mark.parametrize("dim", [2080, 3072, 4096])
def test_rmsnorm_batches_beyond_256_rows(dim):
    # batches of more than 256 rows of 2049..4096 values take 256-lane
    # workgroups (sixteen squares per lane in the exact sum): typical rows and
    # the adversarial ones (ties, powers of two, subnormal squares, overflow,
    # NaN, inf) spread through the batch, all bit-exact
    r = rng(dim + 11)
    adv = _adversarial_rows(dim, dim + 3)
    x = (r.standard_normal((300, dim)) * np.exp(r.standard_normal((300, 1)))).astype(np.float32)
    x[::30][:adv.shape[0]] = adv[: len(x[::30])]
    w = (1 + 0.1 * r.standard_normal(dim)).astype(np.float32)
    got, want = P.rmsnorm(x, w, 1e-5), O.rmsnorm(x, w, 1e-5)
    for i in range(x.shape[0]):
        assert same_bits(got[i], want[i]), i


@pytest.mark.parametrize("dim", [16352, 16384, 49152, 70000])
def test_rmsnorm_rows_wider_than_lds(dim):
    # rows past 16320 values are read from global memory: the exact sum by
    # the predicted-binade scan up to 32 + 1024 * 64 terms, one lane's chain
    # beyond (70000); dense and scaled rows, bit-exact
    r = rng(dim + 5)
    x = np.stack([r.standard_normal(dim), r.standard_normal(dim) * np.exp(r.standard_normal(dim)),
                  np.round(r.standard_normal(dim) * 8)]).astype(np.float32)
    w = (1 + 0.1 * r.standard_normal(dim)).astype(np.float32)
    got, want = P.rmsnorm(x, w, 1e-5), O.rmsnorm(x, w, 1e-5)
    for i in range(x.shape[0]):
        assert same_bits(got[i], want[i]), i


def test_quantize_q8_matches_the_oracle():
    # quantize_q8 (matmul.rs:61-84): a zero block (scale 1), a tiny block, ties
    # at .5 after the scaling, NaN (quantized to 0) and inf in a block
    r = rng(61)
    w = (r.standard_normal((37, 512)) * 3).astype(np.float32)
    w[0, :32] = 0.0
    w[1, 32:64] *= 1e-30
    w[2, 64:96] = (np.arange(32) - 15.5).astype(np.float32) * (127.0 / 15.5)
    w[3, 5] = np.nan
    w[4, 40] = np.inf
    q, s = P.quantize_q8(w)
    qo, so = O.quantize_q8(w)
    assert np.array_equal(q, qo) and same_bits(s, so)


def test_sequential_order_closed_forms_on_device():
    from tests.test_oracle import order_cases, pv_order_case
    x_rms, y0, x_sm, p0 = order_cases()
    assert P.rmsnorm(x_rms[None, :], np.ones(x_rms.size, np.float32), 0.0)[0, 0] == y0
    assert P.softmax(x_sm[None, :])[0, 0] == p0
    q, kc, vc, pos, nh, nkv, hd = pv_order_case()
    assert P.attention_decode(q, kc, vc, pos, nh, nkv, hd)[0] == np.float32(0.25)


def test_silu_and_expf():
    x = np.concatenate([rng(1).standard_normal(100000).astype(np.float32) * 10,
                        np.array([0.0, -0.0, 88.0, -88.0, 100.0, -104.0, -110.0, np.inf, -np.inf], np.float32)])
    assert same_bits(P.silu(x), O.silu(x))
    # device expf against the host glibc expf on the same points
    import ctypes
    libm = ctypes.CDLL("libm.so.6")
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    pts = np.concatenate([x[:3000], x[-9:]])
    want = np.array([libm.expf(float(v)) for v in pts], np.float32)
    assert same_bits(P.expf(pts), want)


def test_expf_exhaustive():
    # Device expf vs the host glibc expf over every f32 bit pattern (16 chunks).
    import ctypes
    lib = P.load()
    n = 1 << 28
    d = P.DeviceArray((n,), np.float32)
    for c in range(16):
        base = c * n
        x = np.arange(base, base + n, dtype=np.uint32).view(np.float32)
        dx = P.DeviceArray.from_host(x)
        P.check(lib.prana_expf(dx.ptr, n, d.ptr, None))
        got = d.to_host()
        want = O.expf_bits(base, n, 16)
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan), c
        assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32)), c
        dx.free()


def test_tanhf_exhaustive():
    # Device tanhf (gelu_tanh's f32::tanh) vs the host glibc tanhf over every
    # f32 bit pattern (16 chunks).
    lib = P.load()
    n = 1 << 28
    d = P.DeviceArray((n,), np.float32)
    for c in range(16):
        base = c * n
        x = np.arange(base, base + n, dtype=np.uint32).view(np.float32)
        dx = P.DeviceArray.from_host(x)
        P.check(lib.prana_tanhf(dx.ptr, n, d.ptr, None))
        got = d.to_host()
        want = O.tanhf_bits(base, n, 16)
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan), c
        assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32)), c
        dx.free()


def test_act_mul_and_add_bias():
    # g = silu(g) * u and x += bias: the oracle's silu, then one IEEE f32
    # multiply / add per element (numpy float32 arithmetic rounds the same way)
    g = rng(31).standard_normal(14336 + 7).astype(np.float32) * 4
    u = rng(32).standard_normal(g.size).astype(np.float32)
    assert same_bits(P.act_mul(g, u), O.silu(g) * u)
    x = rng(33).standard_normal((5, 896)).astype(np.float32)
    b = rng(34).standard_normal(896).astype(np.float32)
    assert same_bits(P.add_bias(x, b), x + b[None, :])


def test_gelu_tanh_bitexact():
    # gelu_tanh (norms.rs:35-41) over normal draws, the tanh saturation range,
    # tiny and special values, alone and fused with the up product
    x = np.concatenate([rng(5).standard_normal(50000).astype(np.float32) * 4,
                        np.linspace(-30, 30, 4001, dtype=np.float32),
                        np.float32([0.0, -0.0, 1e-30, -1e-30, 1e-20, np.inf, -np.inf, 9.5, -9.5])])
    assert same_bits(P.gelu_tanh(x), O.gelu_tanh(x))
    u = rng(6).standard_normal(x.size).astype(np.float32)
    assert same_bits(P.act_mul(x, u, gelu=True), O.gelu_tanh(x) * u)


@pytest.mark.parametrize("n", [1, 2, 7, 256, 512, 513, 2049])
def test_softmax(n):
    x = rng(n).standard_normal((3, n)).astype(np.float32) * 5
    got = P.softmax(x)
    for r in range(3):
        assert same_bits(got[r], O.softmax(x[r]))


@pytest.mark.parametrize("n", [1, 33, 512, 513, 4096, 4097, 20000])
def test_softmax_adversarial(n):
    r = rng(n + 7)
    rows = [
        r.standard_normal(n).astype(np.float32) * 60,          # many exps underflow / subnormal
        np.zeros(n, np.float32),                               # all equal: sum == n
        np.log(np.arange(1, n + 1, dtype=np.float64)).astype(np.float32),
        -np.ldexp(1.0, r.integers(-3, 6, n)).astype(np.float32),
    ]
    for x in rows:
        assert same_bits(P.softmax(x[None, :])[0], O.softmax(x))


# ------------------------------------------------------------------ RoPE / KV
@pytest.mark.parametrize("neox", [0, 1])
@pytest.mark.parametrize("hd,theta", [(48, 1e4), (64, 1e6), (128, 1e4)])
def test_rope(neox, hd, theta):
    nh, rows, pos0 = 4, 5, 250
    x = rng(hd).standard_normal((rows, nh * hd)).astype(np.float32)
    got = P.rope(x, pos0, hd, theta, neox)
    f = O.rope_neox if neox else O.rope_interleaved
    for t in range(rows):
        assert same_bits(got[t], f(x[t], pos0 + t, hd, theta))


def test_kv_write_f16_all_patterns():
    # f32 -> f16 on tie points, specials and randoms, against the oracle.
    h = np.arange(0, 0x7BFF, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)
    x = np.concatenate([mid, np.nextafter(mid, np.float32(1e9)), rng(1).standard_normal(50000).astype(np.float32),
                        np.array([np.inf, -np.inf, np.nan, 1e30, -1e-30, 65520.0], np.float32)])
    x = np.concatenate([x, -x])
    got = P.f32_to_f16(x)
    assert np.array_equal(got, O.f32_to_f16_n(x))
    # every half, NaN payloads included, compared as raw bits
    allh = np.arange(65536, dtype=np.uint16)
    assert np.array_equal(P.f16_to_f32(allh).view(np.uint32), O.f16_to_f32_n(allh).view(np.uint32))


def test_kv_write_rows():
    kv_stride, rows = 64, 6
    cache = np.zeros(rows * kv_stride, np.uint16)
    src = rng(2).standard_normal(2 * kv_stride).astype(np.float32)
    dc = P.DeviceArray.from_host(cache)
    ds = P.DeviceArray.from_host(src)
    P.check(P.load().prana_kv_write_f16(dc.ptr, 3, kv_stride, ds.ptr, src.size, None))
    assert np.array_equal(dc.to_host(), O.f16_kv_write(cache, 3, kv_stride, src))


# ------------------------------------------------------------------ attention
def _cache(n, nkv, hd, seed):
    r = rng(seed)
    kc = r.standard_normal(n * nkv * hd).astype(np.float32).astype(np.float16).view(np.uint16)
    vc = r.standard_normal(n * nkv * hd).astype(np.float32).astype(np.float16).view(np.uint16)
    return kc, vc


# Windows of 2048+ rows with 64/128-wide heads take the three-launch split
# path (scores, softmax, PV); the rest the one-launch kernel (verify batches
# of 256..2047 rows: the wide kernel, see test_attention_verify).
@pytest.mark.parametrize("nh,nkv,hd,pos", [(6, 6, 48, 0), (6, 6, 48, 255), (14, 2, 64, 700), (32, 8, 128, 1030),
                                            (32, 8, 128, 5000), (4, 2, 80, 300), (4, 4, 36, 130), (2, 1, 256, 64),
                                            (32, 8, 128, 2046), (32, 8, 128, 2047), (14, 2, 64, 2600),
                                            (8, 8, 64, 2048), (32, 8, 128, 16500), (4, 2, 80, 4500),
                                            (32, 8, 128, 254), (32, 8, 128, 255), (8, 8, 64, 1023),
                                            (8, 8, 64, 1024), (32, 8, 128, 2045),
                                            # the softmax sum folds on one lane up to 512 rows, by scan beyond
                                            (32, 8, 128, 511), (32, 8, 128, 512), (14, 2, 64, 512)])
def test_attention_decode(nh, nkv, hd, pos):
    kc, vc = _cache(pos + 1, nkv, hd, pos)
    q = rng(pos + 3).standard_normal(nh * hd).astype(np.float32)
    assert same_bits(P.attention_decode(q, kc, vc, pos, nh, nkv, hd), O.attention_decode(q, kc, vc, pos, nh, nkv, hd))


@pytest.mark.parametrize("pos", [32, 510, 511, 512])
def test_attention_decode_adversarial_softmax(pos):
    # Around the softmax sum's one-lane / scan boundary (33 and 511-513 rows):
    # a wide score spread (q scaled by 8: most exponentials underflow or are
    # tiny beside a few large ones), a third of the K rows repeating row 0
    # (equal terms meeting the running sum again and again: the tie-prone
    # case of the exact sum) and zero K rows (scores of exactly 0); then an
    # infinite q entry, whose head turns NaN: NaN in the same places, every
    # other bit equal.
    nh, nkv, hd = 32, 8, 128
    kv = nkv * hd
    kc, vc = _cache(pos + 1, nkv, hd, pos + 40)
    r = rng(pos + 41)
    krows = kc.reshape(pos + 1, kv)
    krows[r.choice(pos + 1, (pos + 1) // 3, replace=False)] = krows[0].copy()
    krows[r.choice(pos + 1, 4, replace=False)] = 0
    q = (rng(pos + 42).standard_normal(nh * hd) * 8).astype(np.float32)
    assert same_bits(P.attention_decode(q, kc, vc, pos, nh, nkv, hd), O.attention_decode(q, kc, vc, pos, nh, nkv, hd))
    q[5] = np.inf
    got, want = P.attention_decode(q, kc, vc, pos, nh, nkv, hd), O.attention_decode(q, kc, vc, pos, nh, nkv, hd)
    nan_g, nan_w = np.isnan(got), np.isnan(want)
    assert np.array_equal(nan_g, nan_w) and nan_g[:hd].all()
    assert same_bits(got[~nan_g], want[~nan_w])


@pytest.mark.parametrize("pos", [300, 2500])
def test_attention_decode_special_values(pos):
    # f16 K/V holding NaNs (quiet and signalling payloads), infinities, the
    # largest finite f16 and subnormals: results must match bit for bit,
    # NaN payloads included (one-launch and split paths). At most one NaN or
    # infinity per (KV head, dim) column of V: which payload an add of two
    # NaNs keeps follows the operand order a compiler picked (IEEE 754 leaves
    # it open), and inf + -inf yields the target's default NaN, whose sign
    # differs between x86 and AMD; neither is part of the reference's
    # contract, so such columns are checked for NaN only (below).
    nh, nkv, hd = 8, 2, 128
    kv = nkv * hd
    kc, vc = _cache(pos + 1, nkv, hd, 11)
    r = rng(12)
    cols = r.choice(kv, 30, replace=False)
    idx_v = r.integers(0, pos + 1, 30) * kv + cols
    vc[idx_v[:10]] = 0x7E00          # quiet NaN
    vc[idx_v[10:20]] = 0x7C01        # signalling NaN payload
    vc[idx_v[20:25]] = 0xFC00        # -inf
    vc[idx_v[25:30]] = 0x7C00        # +inf
    vc[r.choice(vc.size, 10, replace=False)] = r.integers(1, 0x400, 10)  # subnormals
    idx_k = r.choice(kc.size, 20, replace=False)
    kc[idx_k[:10]] = 0x7BFF          # 65504
    kc[idx_k[10:]] = r.integers(1, 0x400, 10)
    q = rng(13).standard_normal(nh * hd).astype(np.float32)
    assert same_bits(P.attention_decode(q, kc, vc, pos, nh, nkv, hd), O.attention_decode(q, kc, vc, pos, nh, nkv, hd))
    # two NaNs and an inf/-inf pair in free columns: NaN there, bit-exact elsewhere
    free = np.setdiff1d(np.arange(kv), cols)[:2]
    vc[[1 * kv + free[0], pos * kv + free[0]]] = [0x7E00, 0x7C01]
    vc[[0 * kv + free[1], (pos // 2) * kv + free[1]]] = [0x7C00, 0xFC00]
    got, want = P.attention_decode(q, kc, vc, pos, nh, nkv, hd), O.attention_decode(q, kc, vc, pos, nh, nkv, hd)
    group = nh // nkv
    mask = np.zeros(nh * hd, bool)
    for c in free:
        kvh, d = divmod(int(c), hd)
        for h in range(kvh * group, (kvh + 1) * group):
            mask[h * hd + d] = True
    assert np.isnan(got[mask]).all() and np.isnan(want[mask]).all()
    assert same_bits(got[~mask], want[~mask])


@pytest.mark.parametrize("nh,nkv,hd,pos0,seq", [(32, 8, 128, 512, 9), (32, 8, 128, 3000, 8), (32, 8, 128, 2040, 9),
                                                 (14, 2, 64, 2046, 3), (32, 8, 128, 2040, 7), (32, 8, 128, 250, 9),
                                                 (14, 2, 64, 700, 5), (14, 2, 64, 1500, 5), (32, 8, 128, 892, 5)])
def test_attention_verify(nh, nkv, hd, pos0, seq):
    # Verify rows over windows of 256..2047 rows take the wide kernel: its
    # softmax sum is one lane's chain over a padded row up to 896 rows and the
    # exact scan beyond (892 + 5: rows 893..897 straddle the switch).
    kc, vc = _cache(pos0 + seq, nkv, hd, 4)
    q = rng(5).standard_normal(seq * nh * hd).astype(np.float32)
    assert same_bits(P.attention_verify(q, kc, vc, pos0, seq, nh, nkv, hd),
                     O.attention_verify(q, kc, vc, pos0, seq, nh, nkv, hd))


# 64/128-wide heads over windows of 16..2048 rows: the block kernel (8 query
# rows per workgroup); the rest the one-launch kernel
@pytest.mark.parametrize("seq,nh,nkv,hd", [(1, 2, 2, 16), (37, 14, 2, 64), (64, 6, 6, 48), (300, 4, 2, 128),
                                            (4200, 2, 1, 16), (50, 3, 3, 20), (17, 4, 2, 64), (16, 2, 2, 128),
                                            (511, 32, 8, 128), (2048, 14, 2, 64), (2049, 2, 1, 64)])
def test_attention_prefill(seq, nh, nkv, hd):
    r = rng(seq)
    q = r.standard_normal(seq * nh * hd).astype(np.float32)
    k = r.standard_normal(seq * nkv * hd).astype(np.float32)
    v = r.standard_normal(seq * nkv * hd).astype(np.float32)
    assert same_bits(P.attention_prefill(q, k, v, seq, nh, nkv, hd), O.attention(q, k, v, seq, nh, nkv, hd))


# ------------------------------------------------------------------ argmax
def test_argmax_semantics():
    rows = [
        rng(1).standard_normal(32000).astype(np.float32),
        np.array([1.0, 3.0, 3.0, 2.0], np.float32),             # first max wins
        np.array([np.nan, 5.0, 7.0], np.float32),               # NaN at 0 pins 0
        np.array([5.0, np.nan, 7.0, 7.0], np.float32),          # later NaN ignored
        np.full(10, -np.inf, np.float32),                       # all -inf -> 0
        np.array([-np.inf, np.nan, -1.0], np.float32),
    ]
    for r in rows:
        assert P.argmax(r)[0] == O.argmax(r), r
    big = rng(2).standard_normal((5, 151936)).astype(np.float32)
    big[3, 1000] = big[3, 2000] = 100.0
    big[4, 10] = big[4, 10 + 1024] = 100.0                      # tie inside one lane's stride
    big[2, 5 + 32768] = big[2, 5 + 2 * 32768] = 100.0           # tie across passes of one lane
    big[1, 70000] = big[1, 3 + 64] = 100.0                      # tie across waves and passes
    big[0, 900] = big[0, 1023] = 100.0                          # tie across the merged waves
    got = P.argmax(big)
    assert [int(v) for v in got] == [O.argmax(b) for b in big]
