"""GPU parity at the benchmark configurations' own sizes, bit for bit against
the oracle built from the same bytes:
  - C1: the Q8_0 sweep's large shapes at N = 16 and 64 (matmul.rs:162-232);
  - C2 / C4 prefill GEMMs at the configurations' batch sizes (N = 2047 and
    511) and single-layer shapes, over the same quantized activations
    (matmul_q8_prefill / matmul_kquant_prefill, matmul.rs:185-232,
    kquant.rs:368-370);
  - C2: the full qwen2-0.5B-shape model, a 64-token prompt and 32 greedy steps
    (stream, logits and KV cache rows), and the stated 2048-token prefill with
    512 greedy steps, 128 of them followed by the oracle;
  - C4: the 7B-shape layer (full width, two layers) after a 511-token prefill."""
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


@pytest.mark.parametrize("rows,cols", [(14336, 4096), (32000, 4096), (4096, 14336), (4096, 4096)])
@pytest.mark.parametrize("n", [16, 64])
def test_c1_large_shapes_batched(rows, cols, n):
    raw = P.synth_tensor(P.Q8_0, rows, cols, rows + n, 0.02)
    x = np.random.default_rng(rows + n).standard_normal((n, cols)).astype(np.float32)
    got = P.Matrix(P.Q8_0, rows, cols, raw).apply(x)
    want = O.Mat.from_ggml(P.Q8_0, rows, cols, raw).apply(x)
    assert same_bits(got, want)


PREFILL_CASES = [
    # (tag, ggml type, rows, cols, N)
    ("C2 ffn_down Q6_K", P.Q6_K, 896, 4864, 2047),
    ("C2 ffn_gate Q4_0", P.Q4_0, 4864, 896, 2047),
    ("C2 attn_q Q4_0", P.Q4_0, 896, 896, 2047),
    ("C2 attn_v Q8_0", P.Q8_0, 128, 896, 2047),
    ("C2-width Q4_K", P.Q4_K, 512, 4096, 2047),
    ("C4 ffn_down Q4_0", P.Q4_0, 4096, 14336, 511),
    ("C4 ffn_gate Q4_0", P.Q4_0, 14336, 4096, 511),
    ("C4 attn_q|k|v Q4_0", P.Q4_0, 6144, 4096, 511),
]


@pytest.mark.parametrize("tag,ty,rows,cols,n", PREFILL_CASES, ids=[c[0] for c in PREFILL_CASES])
def test_prefill_gemm_at_config_batch(tag, ty, rows, cols, n):
    raw = P.synth_tensor(ty, rows, cols, rows * 3 + cols, 0.02)
    x = np.random.default_rng(rows + cols).standard_normal((n, cols)).astype(np.float32)
    q, sa, sums = O.quantize_acts(x)
    got = P.Matrix(ty, rows, cols, raw).apply_prefill(q, sa, sums)
    want = O.Mat.from_ggml(ty, rows, cols, raw).apply_prefill(q, sa, sums)
    assert same_bits(got, want)


def test_c2_full_model_longer_stream():
    cfg = dict(M.C2)
    cfg["seq_len"] = 128
    t = M.c2_tensors(seed=2)
    g, o = P.Model(cfg, t), O.Model(cfg, t)
    prompt = np.random.default_rng(22).integers(0, cfg["vocab_size"], 64).astype(np.uint32)
    gc, oc = g.cache(100), o.cache(100)
    gc.prefill(prompt[:-1])
    oc.prefill(prompt[:-1])
    for layer in (0, 11, 23):
        for which in (0, 1):
            assert np.array_equal(gc.read(layer, which, 63), oc.read(layer, which, 63)), (layer, which)
    got = gc.decode(int(prompt[-1]), 63, 32)
    tok, want = int(prompt[-1]), []
    for i in range(32):
        tok = int(O.argmax(oc.forward(tok, 63 + i)))
        want.append(tok)
    assert list(got) == want
    # the logits of the next step, bit for bit
    assert same_bits(gc.forward(want[-1], 95), oc.forward(want[-1], 95))


def test_c4_width_prefill_511_then_decode():
    cfg = dict(M.C4)
    cfg["n_layers"] = 2
    cfg["seq_len"] = 520
    t = M.c4_tensors(seed=4, n_layers=2)
    g, o = P.Model(cfg, t), O.Model(cfg, t)
    prompt = np.random.default_rng(44).integers(0, cfg["vocab_size"], 512).astype(np.uint32)
    gc, oc = g.cache(520), o.cache(520)
    gc.prefill(prompt[:-1])
    oc.prefill(prompt[:-1])
    for layer in (0, 1):
        for which in (0, 1):
            assert np.array_equal(gc.read(layer, which, 511), oc.read(layer, which, 511)), (layer, which)
    tok = int(prompt[-1])
    for pos in range(511, 514):
        lg, lo = gc.forward(tok, pos), oc.forward(tok, pos)
        assert same_bits(lg, lo), pos
        tok = int(O.argmax(lo))


def test_c2_stated_2048_prefill_then_greedy():
    # C2 as stated: 2048-token random prefill, then 512 greedy steps on the
    # device; the oracle follows the first 128 of them token for token, and
    # the cache rows those steps wrote and the logits after them are compared
    # bit for bit
    cfg = dict(M.C2)
    cfg["seq_len"] = 2600
    t = M.c2_tensors(seed=2)
    g, o = P.Model(cfg, t), O.Model(cfg, t)
    prompt = np.random.default_rng(2048).integers(0, cfg["vocab_size"], 2048).astype(np.uint32)
    gc, oc = g.cache(2600), o.cache(2600)
    gc.prefill(prompt[:-1])
    oc.prefill(prompt[:-1])
    for layer in (0, 23):
        for which in (0, 1):
            assert np.array_equal(gc.read(layer, which, 2047), oc.read(layer, which, 2047)), (layer, which)
    got = gc.decode(int(prompt[-1]), 2047, 512)
    assert len(got) == 512
    tok, want = int(prompt[-1]), []
    for i in range(128):
        tok = int(O.argmax(oc.forward(tok, 2047 + i)))
        want.append(tok)
    assert list(got[:128]) == want
    for layer in (0, 11, 23):
        for which in (0, 1):
            assert np.array_equal(gc.read(layer, which, 2175), oc.read(layer, which, 2175)), (layer, which)
    # step 129 again on both sides (the device rewrites row 2175 with the same
    # token it decoded there): its logits, bit for bit
    assert same_bits(gc.forward(want[-1], 2175), oc.forward(want[-1], 2175))
