"""GPU parity of the model layer: logits, KV caches and greedy token streams
of the device Model against the CPU oracle built from the same tensor bytes,
from the reference's tiny test models up to the 7B benchmark shape."""
import numpy as np
import pytest

import prana_amd as P
from prana_amd import models as M
from oracle import oracle as O
from tests import fixtures as fx

pytestmark = pytest.mark.gpu


def same_bits(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def pair(cfg, t):
    return P.Model(cfg, t), O.Model(cfg, t)


# ------------------------------------------------------------------ the reference's tiny GGUF models (F32 weights)
@pytest.mark.parametrize("arch", ["llama", "qwen2"])
def test_tiny_forward_logits_and_cache_bitexact(arch):
    cfg, t = fx.synthetic_model(arch, arch == "qwen2")
    g, o = pair(cfg, t)
    gc, oc = g.cache(16), o.cache(16)
    toks = [5, 3, 9, 44, 0, 17]
    for pos, tok in enumerate(toks):
        assert same_bits(gc.forward(tok, pos), oc.forward(tok, pos)), pos
    for layer in range(cfg["n_layers"]):
        for which in (0, 1):
            assert np.array_equal(gc.read(layer, which, len(toks)), oc.read(layer, which, len(toks)))


@pytest.mark.parametrize("arch", ["llama", "qwen2"])
def test_tiny_prefill_then_decode_bitexact(arch):
    cfg, t = fx.synthetic_model(arch, arch == "qwen2")
    g, o = pair(cfg, t)
    gc, oc = g.cache(16), o.cache(16)
    toks = [3, 9, 14, 7, 21]
    gc.prefill(toks)
    oc.prefill(toks)
    for layer in range(cfg["n_layers"]):
        assert np.array_equal(gc.read(layer, 0, 5), oc.read(layer, 0, 5))
    assert same_bits(gc.forward(5, 5), oc.forward(5, 5))


def test_tiny_forward_batch_bitexact():
    cfg, t = fx.synthetic_model("qwen2", True)
    g, o = pair(cfg, t)
    gc, oc = g.cache(16), o.cache(16)
    gc.prefill([3, 9, 14])
    oc.prefill([3, 9, 14])
    assert same_bits(gc.forward_batch([7, 21, 4, 40], 3), oc.forward_batch([7, 21, 4, 40], 3))


@pytest.mark.parametrize("draft_arch", ["qwen2", "llama"])
def test_tiny_speculative_equals_greedy_and_oracle(draft_arch):
    cfg, t = fx.synthetic_model("qwen2", True)
    dcfg, dt = fx.synthetic_model(draft_arch, draft_arch == "qwen2")
    g, o = pair(cfg, t)
    gd, od = pair(dcfg, dt)
    prompt, stops = [5, 7, 9], (46, 47)
    plain, _ = g.generate(prompt, 8, stops)
    plain_o, _ = o.generate(prompt, 8, stops)
    spec, st = P.generate_speculative(g, gd, prompt, 8, 4, stops)
    spec_o, st_o = O.generate_speculative(o, od, prompt, 8, 4, stops)
    assert list(plain) == list(plain_o)
    assert list(spec) == list(spec_o)
    assert (st.proposed, st.accepted) == (st_o.proposed, st_o.accepted)
    # The guarantee of gguf.rs:746-799, on the device path.
    assert list(spec)[: len(plain)] == list(plain)[: len(spec)]


def test_tiny_speculative_limits_and_stops():
    # The device accept walk against the oracle's host loop (infer.rs:648-681):
    # step limits inside and at the end of a round, the 16-position window
    # cutting a round's budget, and a stop token at each place in the stream.
    cfg, t = fx.synthetic_model("qwen2", True)
    dcfg, dt = fx.synthetic_model("llama", False)
    g, o = pair(cfg, t)
    gd, od = pair(dcfg, dt)
    prompt = [5, 7, 9]
    plain, _ = o.generate(prompt, 20)
    for k in (1, 2, 3, 5, 16):
        for steps in (1, 2, 5, 13, 20):
            spec, st = P.generate_speculative(g, gd, prompt, steps, k)
            spec_o, st_o = O.generate_speculative(o, od, prompt, steps, k)
            assert list(spec) == list(spec_o), (k, steps)
            assert (st.proposed, st.accepted, st.generated_tokens) == (st_o.proposed, st_o.accepted,
                                                                       st_o.generated_tokens), (k, steps)
        for i in range(0, len(plain), 3):
            stops = (int(plain[i]),)
            spec, st = P.generate_speculative(g, gd, prompt, 20, k, stops)
            spec_o, st_o = O.generate_speculative(o, od, prompt, 20, k, stops)
            assert list(spec) == list(spec_o), (k, stops)
            assert (st.proposed, st.accepted) == (st_o.proposed, st_o.accepted), (k, stops)


def test_long_window_split_attention_bitexact():
    # Decode and verify steps past 2048 cached rows run the split attention
    # path, whose PV launch also quantizes the output for the wo projection.
    cfg = M.config(256, 512, 2, 4, 1, 512, 2200, head_dim=64, rope_neox=1)
    t = M.synth_tensors(cfg, M.types_c0, 7)
    g, o = pair(cfg, t)
    gc, oc = g.cache(2200), o.cache(2200)
    prompt = np.random.default_rng(7).integers(0, cfg["vocab_size"], 2050).astype(np.uint32)
    gc.prefill(prompt[:2045])
    oc.prefill(prompt[:2045])
    tok = int(prompt[2045])
    for pos in range(2045, 2049):  # windows of 2046..2049 rows: both paths
        lg, lo = gc.forward(tok, pos), oc.forward(tok, pos)
        assert same_bits(lg, lo), pos
        tok = int(np.argmax(lo))
    batch = [int(x) for x in prompt[:5]]
    assert same_bits(gc.forward_batch(batch, 2049), oc.forward_batch(batch, 2049))
    for layer in range(cfg["n_layers"]):
        assert np.array_equal(gc.read(layer, 1, 2054), oc.read(layer, 1, 2054))


def oracle_chain(oc, tok, pos, n):
    """The oracle's greedy stream: feed tok at pos, take the argmax, repeat."""
    out = []
    for i in range(n):
        tok = int(O.argmax(oc.forward(tok, pos + i)))
        out.append(tok)
    return out


def test_decode_replay_across_split_window_bitexact():
    # decode() replays one captured step while the window stays below the
    # split attention path (device-side position), then launches kernel by
    # kernel: windows 2040..2051 cover both.
    cfg = M.config(256, 512, 2, 4, 1, 512, 2200, head_dim=64, rope_neox=1)
    t = M.synth_tensors(cfg, M.types_c0, 8)
    g, o = pair(cfg, t)
    gc, oc = g.cache(2200), o.cache(2200)
    prompt = np.random.default_rng(8).integers(0, cfg["vocab_size"], 2040).astype(np.uint32)
    gc.prefill(prompt[:2039])
    oc.prefill(prompt[:2039])
    got = gc.decode(int(prompt[2039]), 2039, 12)
    assert list(got) == oracle_chain(oc, int(prompt[2039]), 2039, 12)
    for layer in range(cfg["n_layers"]):
        for which in (0, 1):
            assert np.array_equal(gc.read(layer, which, 2051), oc.read(layer, which, 2051)), (layer, which)


@pytest.mark.parametrize("heads,kv_heads,neox", [(4, 2, 0), (2, 1, 1)])
def test_decode_replay_reuse_and_recapture_bitexact(heads, kv_heads, neox):
    # Consecutive decode() calls reuse the captured step; a forward_batch in
    # between grows the workspace, so the next call captures again. The
    # one-token Q|K|V launch applies RoPE and writes the cache rows itself:
    # adjacent pairs, and (2 heads of 64, NeoX) pairs half a head apart in
    # tiles of whole heads.
    cfg = M.config(128, 384, 2, heads, kv_heads, 300, 96, rope_neox=neox)
    t = M.synth_tensors(cfg, M.types_c0, 9)
    g, o = pair(cfg, t)
    gc, oc = g.cache(96), o.cache(96)
    prompt = np.random.default_rng(9).integers(0, cfg["vocab_size"], 6).astype(np.uint32)
    gc.prefill(prompt[:5])
    oc.prefill(prompt[:5])
    a = gc.decode(int(prompt[5]), 5, 7)
    ra = oracle_chain(oc, int(prompt[5]), 5, 7)
    assert list(a) == ra
    b = gc.decode(int(a[-1]), 12, 9)
    rb = oracle_chain(oc, ra[-1], 12, 9)
    assert list(b) == rb
    batch = [int(x) for x in prompt[:6]]
    assert same_bits(gc.forward_batch(batch, 21), oc.forward_batch(batch, 21))
    c = gc.decode(int(rb[-1]), 27, 10)
    assert list(c) == oracle_chain(oc, rb[-1], 27, 10)
    for layer in range(cfg["n_layers"]):
        for which in (0, 1):
            assert np.array_equal(gc.read(layer, which, 37), oc.read(layer, which, 37)), (layer, which)


# ------------------------------------------------------------------ config 0: 15M shape, Q8_0, 256-step greedy decode
@pytest.fixture(scope="module")
def c0():
    t = M.c0_tensors(seed=1)
    return M.C0, t


def test_c0_greedy_256_token_identical(c0):
    cfg, t = c0
    g, o = pair(cfg, t)
    prompt = np.random.default_rng(20260712).integers(0, cfg["vocab_size"], 5).astype(np.uint32)
    go, gst = g.generate(prompt, 256)
    oo, ost = o.generate(prompt, 256)
    # max_pos = min(256, 5 + 256): positions 4..254 sample, 251 tokens.
    assert len(oo) == 251
    assert list(go) == list(oo)
    assert gst.generated_tokens == ost.generated_tokens == 251


def test_c0_logits_bitexact_along_the_stream(c0):
    cfg, t = c0
    g, o = pair(cfg, t)
    gc, oc = g.cache(64), o.cache(64)
    prompt = [11, 2200, 31999, 0, 17]
    gc.prefill(prompt[:4])
    oc.prefill(prompt[:4])
    tok = prompt[4]
    for pos in range(4, 40):
        lg, lo = gc.forward(tok, pos), oc.forward(tok, pos)
        assert same_bits(lg, lo), pos
        tok = int(np.argmax(lo))


# ------------------------------------------------------------------ config 2: qwen2-0.5B shape, K-quant mixture
def test_c2_qwen2_05b_short_decode_token_identical():
    cfg = M.C2
    t = M.c2_tensors(seed=2)
    g, o = pair(cfg, t)
    prompt = np.random.default_rng(2).integers(0, cfg["vocab_size"], 12).astype(np.uint32)
    go, _ = g.generate(prompt, 6)
    oo, _ = o.generate(prompt, 6)
    assert list(go) == list(oo)
    gc, oc = g.cache(32), o.cache(32)
    gc.prefill(prompt[:8])
    oc.prefill(prompt[:8])
    assert same_bits(gc.forward(int(prompt[8]), 8), oc.forward(int(prompt[8]), 8))


def test_kquant_prefill_and_verify_batches_bitexact():
    # Q4_K / Q6_K weights (every width a multiple of 256) with prompt and
    # verify batches of more than 16 tokens: the K-quant matrix-core kernel
    cfg = M.config(512, 1536, 2, 8, 2, 1000, 128, head_dim=64, rope_theta=1e6, norm_eps=1e-6, rope_neox=1)
    t = M.synth_tensors(cfg, M.types_c2, 5, biases=True)
    assert {t[k][0] for k in t if k.endswith("ffn_down.weight")} == {P.Q6_K}
    g, o = pair(cfg, t)
    gc, oc = g.cache(128), o.cache(128)
    prompt = np.random.default_rng(5).integers(0, cfg["vocab_size"], 70).astype(np.uint32)
    gc.prefill(prompt[:40])
    oc.prefill(prompt[:40])
    for layer in range(cfg["n_layers"]):
        assert np.array_equal(gc.read(layer, 1, 40), oc.read(layer, 1, 40))
    batch = [int(x) for x in prompt[40:70]]
    assert same_bits(gc.forward_batch(batch, 40), oc.forward_batch(batch, 40))


@pytest.mark.parametrize("ty", [P.Q4_0, P.Q8_0])
def test_block32_verify_batches_bitexact(ty):
    # Verify batches of 2..10 tokens over block-32 weights whose widths take
    # the chunk-major multi-token kernel: Q|K|V (3 matrices, 2048 wide: 32-block
    # chunks), gate|up with the activation (2048 wide) and down (4096 wide:
    # four chunks), and the head; then a model whose down projection is 14336
    # wide: seven 64-block chunks at five tokens, fourteen 32-block chunks at
    # seven.
    cfg = M.config(2048, 4096, 1, 16, 4, 700, 64, head_dim=128)
    t = M.synth_tensors(cfg, lambda name, cols: ty, 11)
    g, o = pair(cfg, t)
    gc, oc = g.cache(64), o.cache(64)
    prompt = np.random.default_rng(11).integers(0, cfg["vocab_size"], 60).astype(np.uint32)
    gc.prefill(prompt[:20])
    oc.prefill(prompt[:20])
    pos = 20
    for n in (2, 5, 8, 10):
        batch = [int(x) for x in prompt[pos:pos + n]]
        assert same_bits(gc.forward_batch(batch, pos), oc.forward_batch(batch, pos)), n
        pos += n
    cfg = M.config(512, 14336, 1, 4, 2, 300, 32, head_dim=128)
    t = M.synth_tensors(cfg, lambda name, cols: ty, 12)
    g, o = pair(cfg, t)
    gc, oc = g.cache(32), o.cache(32)
    prompt = prompt % cfg["vocab_size"]
    gc.prefill(prompt[:4])
    oc.prefill(prompt[:4])
    for n, pos in ((5, 4), (7, 9)):
        batch = [int(x) for x in prompt[pos:pos + n]]
        assert same_bits(gc.forward_batch(batch, pos), oc.forward_batch(batch, pos)), n


@pytest.mark.parametrize("ty,act,dense_down", [(P.Q4_0, 0, False), (P.Q8_0, 0, False), (P.Q4_0, 1, True)])
def test_large_verify_batches_on_matrix_cores_bitexact(ty, act, dense_down):
    # Verify batches of 3..8 tokens over matrices of at least 1.5M blocks take
    # the skinny matrix-core kernel: here down (4096 x 12288) and gate|up (one
    # launch that also forms h = act(g) * u, silu or gelu_tanh, quantizes it
    # and, for a dense f32 down, writes the f32 h); the smaller Q|K|V and wo
    # stay on the decode tiles. At 9 tokens every projection takes it (Q|K|V
    # and wo on the block-split form, too few row tiles for the one-launch form).
    cfg = M.config(4096, 12288, 1, 32, 8, 300, 48, head_dim=128, act=act)
    t = M.synth_tensors(cfg, lambda name, cols: M.F32 if dense_down and "ffn_down" in name else ty, 13 + act)
    g, o = pair(cfg, t)
    gc, oc = g.cache(48), o.cache(48)
    prompt = np.random.default_rng(13).integers(0, cfg["vocab_size"], 40).astype(np.uint32)
    gc.prefill(prompt[:4])
    oc.prefill(prompt[:4])
    pos = 4
    for n in (3, 5, 8, 9):
        batch = [int(x) for x in prompt[pos:pos + n]]
        assert same_bits(gc.forward_batch(batch, pos), oc.forward_batch(batch, pos)), n
        pos += n


@pytest.mark.parametrize("ty", [P.Q4_0, P.Q8_0])
def test_verify_qkv_one_skinny_launch_bitexact(ty):
    # Three matrices in one skinny launch: Q|K|V of 3 x 6144 rows (as many KV
    # heads as query heads) fill the chip with 64-row tiles, so the launch
    # deals workgroups 0..95 to Q, 96..191 to K and 192..287 to V. Batches of
    # 9 and 16 tokens (one 16-token tile, a ragged and a full one).
    cfg = M.config(6144, 1024, 1, 48, 48, 300, 40, head_dim=128)
    t = M.synth_tensors(cfg, lambda name, cols: ty, 29)
    g, o = pair(cfg, t)
    gc, oc = g.cache(40), o.cache(40)
    prompt = np.random.default_rng(29).integers(0, cfg["vocab_size"], 30).astype(np.uint32)
    gc.prefill(prompt[:4])
    oc.prefill(prompt[:4])
    pos = 4
    for n in (9, 16):
        batch = [int(x) for x in prompt[pos:pos + n]]
        assert same_bits(gc.forward_batch(batch, pos), oc.forward_batch(batch, pos)), n
        for layer in range(cfg["n_layers"]):
            assert np.array_equal(gc.read(layer, 0, pos + n), oc.read(layer, 0, pos + n)), (n, layer)
            assert np.array_equal(gc.read(layer, 1, pos + n), oc.read(layer, 1, pos + n)), (n, layer)
        pos += n


@pytest.mark.parametrize("ty,act,dense_down", [(P.Q4_0, 0, False), (P.Q8_0, 1, False), (P.Q4_0, 0, True)])
def test_prefill_gate_up_act_one_launch_bitexact(ty, act, dense_down):
    # Prompts beyond the skinny kernel's batches (more than 64 tokens) run
    # gate|up on the matrix cores in one launch that also forms h = act(g) * u
    # (silu, or gelu_tanh) and quantizes it for down; with a dense f32 down
    # projection it also writes the f32 h that down reads. Ragged token tiles
    # (100 = 3 x 32 + 4), two 64-row tile rows per 32-row quantization block.
    cfg = M.config(512, 1536, 2, 8, 2, 300, 160, head_dim=64, act=act)
    t = M.synth_tensors(cfg, lambda name, cols: M.F32 if dense_down and "ffn_down" in name else ty, 17 + act)
    g, o = pair(cfg, t)
    gc, oc = g.cache(160), o.cache(160)
    prompt = np.random.default_rng(17).integers(0, cfg["vocab_size"], 101).astype(np.uint32)
    gc.prefill(prompt[:100])
    oc.prefill(prompt[:100])
    for layer in range(cfg["n_layers"]):
        assert np.array_equal(gc.read(layer, 0, 100), oc.read(layer, 0, 100)), layer
        assert np.array_equal(gc.read(layer, 1, 100), oc.read(layer, 1, 100)), layer
    assert same_bits(gc.forward(int(prompt[100]), 100), oc.forward(int(prompt[100]), 100))


@pytest.mark.parametrize("dim", [512, 896])
def test_mixed_format_qkv_one_launch_bitexact(dim):
    # The K-quant mixture stores v in another format than q and k: Q4_K with
    # Q6_K (512 wide), and their block-32 fallbacks Q4_0 with Q8_0 (896 wide,
    # C2's widths); Q|K|V then runs as one launch with RoPE and the cache rows
    # in its epilogue (decode) or over a verify batch.
    cfg = M.config(dim, 1024, 2, dim // 64, 2, 500, 64, head_dim=64, rope_theta=1e6, norm_eps=1e-6, rope_neox=1)
    t = M.synth_tensors(cfg, M.types_c2, 6 + dim, biases=True)
    kinds = {t[f"blk.0.attn_{x}.weight"][0] for x in "qkv"}
    assert len(kinds) == 2, kinds
    g, o = pair(cfg, t)
    gc, oc = g.cache(64), o.cache(64)
    prompt = np.random.default_rng(dim).integers(0, cfg["vocab_size"], 30).astype(np.uint32)
    gc.prefill(prompt[:8])
    oc.prefill(prompt[:8])
    tok = int(prompt[8])
    for pos in range(8, 12):
        lg, lo = gc.forward(tok, pos), oc.forward(tok, pos)
        assert same_bits(lg, lo), pos
        tok = int(np.argmax(lo))
    batch = [int(x) for x in prompt[12:17]]
    assert same_bits(gc.forward_batch(batch, 12), oc.forward_batch(batch, 12))
    for layer in range(cfg["n_layers"]):
        for which in (0, 1):
            assert np.array_equal(gc.read(layer, which, 17), oc.read(layer, which, 17)), (layer, which)


@pytest.mark.parametrize("ty,dim,hd,neox", [("Q4_0", 2048, 64, 1), ("Q8_0", 4096, 128, 1), ("Q8_0", 4096, 128, 0),
                                             ("Q4_0", 896, 64, 1), ("Q8_0", 1024, 64, 0)])
def test_fused_norm_decode_bitexact(ty, dim, hd, neox):
    # Decode rows of 1024 < dim <= 4096 let the Q|K|V and gate|up launches
    # normalise x themselves (one 1024-lane workgroup per tile; Q|K|V tiles of
    # 64 rows at 2048 and 32 rows at 4096, gate|up tiles of 64 rows of each
    # matrix, h quantized in the epilogue). NeoX pairs span whole heads, so at
    # hd 128 the 32-row tiles leave RoPE to its own launch; at hd 64, and for
    # adjacent pairs, it rides in the same launch. Rows of 513-1024 values take
    # 256-lane workgroups (Q|K|V tiles of 64 rows at 896 and 32 at 1024,
    # gate|up tiles of 64 rows with 14 or 16 units per lane).
    kind = {"Q4_0": M.Q4_0, "Q8_0": M.Q8_0}[ty]
    n_kv = 4 if (dim // hd) % 4 == 0 else 2
    cfg = M.config(dim, 1024, 2, dim // hd, n_kv, 500, 64, head_dim=hd, rope_neox=neox)
    t = M.synth_tensors(cfg, lambda name, cols: kind, 90 + dim + neox, biases=True)
    g, o = pair(cfg, t)
    gc, oc = g.cache(64), o.cache(64)
    prompt = np.random.default_rng(dim + hd).integers(0, cfg["vocab_size"], 16).astype(np.uint32)
    gc.prefill(prompt[:6])
    oc.prefill(prompt[:6])
    tok = int(prompt[6])
    for pos in range(6, 10):
        lg, lo = gc.forward(tok, pos), oc.forward(tok, pos)
        assert same_bits(lg, lo), pos
        tok = int(np.argmax(lo))
    for layer in range(cfg["n_layers"]):
        for which in (0, 1):
            assert np.array_equal(gc.read(layer, which, 10), oc.read(layer, which, 10)), (layer, which)
    go, _ = g.generate(prompt[:5], 6)
    oo, _ = o.generate(prompt[:5], 6)
    assert list(go) == list(oo)


# ------------------------------------------------------------------ config 4: 7B shape, Q4_0
@pytest.fixture(scope="module")
def c4():
    return M.C4, M.c4_tensors(seed=4)


def test_c4_7b_decode_token_identical(c4):
    cfg, t = c4
    g, o = pair(cfg, t)
    prompt = np.random.default_rng(4).integers(0, cfg["vocab_size"], 4).astype(np.uint32)
    go, _ = g.generate(prompt, 5)
    oo, _ = o.generate(prompt, 5)
    assert len(oo) == 5
    assert list(go) == list(oo)


@pytest.mark.parametrize("k", [4, 8])
def test_c4_speculative_equals_plain_greedy(c4, k):
    cfg, t = c4
    g = P.Model(cfg, t)
    draft = P.Model(M.c4_draft_config(), M.synth_tensors(M.c4_draft_config(), M.types_c0, 1))
    # the stated workload: a 512-token prompt, i.e. a 511-token prefill
    # before the first speculative round
    prompt = np.random.default_rng(44).integers(0, cfg["vocab_size"], 512).astype(np.uint32)
    plain, _ = g.generate(prompt, 24)
    spec, st = P.generate_speculative(g, draft, prompt, 24, k)
    assert list(spec) == list(plain)
    # Self-draft. The reference's loop advances past the last accepted draft
    # token without feeding it to the draft (infer.rs:629-681), so the draft
    # cache keeps a stale row and acceptance is high but not total; the
    # reference test asserts accepted > 0 (gguf.rs:795-797).
    spec2, st2 = P.generate_speculative(g, g, prompt, 12, k)
    assert list(spec2) == list(plain[:12])
    assert 0 < st2.accepted <= st2.proposed


def test_gemv_profile_shapes_add_up():
    # prana_gemv_profile_shapes splits the sampled decode GEMV launches by the
    # weight bytes they stream; the split adds up to prana_gemv_profile_read's
    # totals, and a reset clears it. Entry 1 holds the decode attention
    # launches (one per layer and step at this context), outside the totals.
    cfg = M.config(2048, 1024, 2, 32, 4, 500, 64, head_dim=64, rope_neox=1)
    g = P.Model(cfg, M.synth_tensors(cfg, lambda name, cols: M.Q4_0, 77))
    c = g.cache(32)
    prompt = np.random.default_rng(77).integers(0, cfg["vocab_size"], 8).astype(np.uint32)
    c.prefill(prompt[:4])
    P.gemv_profile(True, period=1)
    P.gemv_profile_read(reset=True)
    tok = int(prompt[4])
    for pos in range(4, 8):
        tok = int(np.argmax(c.forward(tok, pos)))
    shapes = P.gemv_profile_shapes()
    n, sec, total_bytes = P.gemv_profile_read(reset=True)
    P.gemv_profile(False)
    attn = [(k, t) for b, k, t in shapes if b == 1]
    assert len(attn) == 1 and attn[0][0] == 4 * cfg["n_layers"] and attn[0][1] > 0
    shapes = [r for r in shapes if r[0] != 1]
    assert n > 0 and sum(k for _, k, _ in shapes) == n
    assert sum(b * k for b, k, _ in shapes) == total_bytes
    assert abs(sum(t for _, _, t in shapes) - sec) <= 1e-9 * max(sec, 1.0)
    assert len({b for b, _, _ in shapes}) == len(shapes) >= 4
    assert all(k > 0 and t > 0 for _, k, t in shapes)
    assert P.gemv_profile_shapes() == []
