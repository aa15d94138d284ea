"""GPU: models loaded from GGUF bytes by the library (prana_model_load_gguf,
gguf.rs:338-437) against the oracle model built from the same tensors, bit
for bit:
  - the reference's synthetic llama / qwen2 (biases) / gemma files
    (gguf.rs:566-666): NeoX RoPE, gelu_tanh, sqrt(dim) embedding scale, the
    (1 + w) norm fold, a per-head width that is not a multiple of 32;
  - Precision::Q8 (quantize_q8 on every dense matrix and the tied head);
  - a mixed file (Q4_0 / Q8_0 / Q4_K / Q6_K / F16 / F32 tensors, packed
    table, untied head) and K-quant tensors whose rows are not whole
    super-blocks (decoded to dense rows, gguf.rs:295-305);
  - load from a path, missing tensors, and greedy generation."""
import numpy as np
import pytest

import prana_amd as P
from oracle import oracle as O
from tests.golden import gguf_writer as W

pytestmark = pytest.mark.gpu


def same_bits(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def synthetic_config(arch, hd):
    return dict(dim=32, hidden_dim=64, n_layers=2, n_heads=2, n_kv_heads=2, vocab_size=48, seq_len=16,
                head_dim=hd, rope_theta=1e4, norm_eps=float(np.float32(1e-5)),
                emb_scale=float(np.sqrt(np.float32(32))) if arch == "gemma" else 1.0,
                rope_neox=int(arch != "llama"), act=int(arch == "gemma"))


def oracle_tensors(tensors, gemma, q8=False):
    """{name: (type, dims, bytes)} for the oracle from the file's f32 arrays,
    with gemma's +1 fold in f32 and, at Q8, quantize_q8 on every matrix."""
    out = {}
    for name, (dims, a) in tensors.items():
        if gemma and name.endswith("norm.weight"):
            a = (a + np.float32(1.0)).astype(np.float32)
        if q8 and len(dims) == 2 and name != "token_embd.weight" and dims[0] % 32 == 0:
            out[name] = O.Mat.q8_parts(*O.quantize_q8(a.reshape(dims[1], dims[0])))
        else:
            out[name] = (0, dims, a)
    return out


def compare_stream(g, o, tokens, positions):
    gc, oc = g.cache(positions), o.cache(positions)
    for pos, tok in enumerate(tokens):
        lg, lo = gc.forward(int(tok), pos), oc.forward(int(tok), pos)
        assert same_bits(lg, lo), pos
    return gc, oc


@pytest.mark.parametrize("arch,biases,hd", [("llama", False, 16), ("qwen2", True, 16), ("gemma", False, 16),
                                            ("gemma", False, 8), ("llama", True, 8)])
def test_reference_synthetic_models_bitexact(arch, biases, hd):
    b, tensors = W.reference_synthetic_model(arch, biases, hd)
    g = P.load_gguf(b)
    cfg = synthetic_config(arch, hd)
    assert g.config == {**cfg, "norm_eps": g.config["norm_eps"]} and g.config["norm_eps"] == np.float32(1e-5)
    o = O.Model(cfg, oracle_tensors(tensors, arch == "gemma"))
    # qwen2_arch_loads_with_biases_and_runs (gguf.rs:676-695): logits differ by position
    gc = g.cache(16)
    a, c = gc.forward(5, 0), gc.forward(5, 1)
    assert a.shape == (48,) and np.isfinite(a).all() and np.isfinite(c).all() and not np.array_equal(a, c)
    compare_stream(g, o, [3, 17, 40, 2, 9, 9, 31, 0], 16)


def test_gemma_fold_is_what_the_logits_see():
    # gemma_norm_weights_are_folded_plus_one (gguf.rs:874-886): the gemma load
    # equals the oracle with (1 + w) norms and differs from the unfolded one
    b, tensors = W.reference_synthetic_model("gemma", False, 16)
    g = P.load_gguf(b)
    cfg = synthetic_config("gemma", 16)
    folded = O.Model(cfg, oracle_tensors(tensors, True)).cache(4).forward(7, 0)
    unfolded = O.Model(cfg, oracle_tensors(tensors, False)).cache(4).forward(7, 0)
    got = g.cache(4).forward(7, 0)
    assert same_bits(got, folded) and not same_bits(got, unfolded)


@pytest.mark.parametrize("arch", ["llama", "qwen2", "gemma"])
def test_q8_precision_bitexact(arch):
    b, tensors = W.reference_synthetic_model(arch, arch == "qwen2", 16)
    g = P.load_gguf(b, precision="q8")
    ot = oracle_tensors(tensors, arch == "gemma", q8=True)
    # tied head: a quantized copy of the dense table (gguf.rs:426-437)
    emb = tensors["token_embd.weight"][1].reshape(48, 32)
    ot["output.weight"] = O.Mat.q8_parts(*O.quantize_q8(emb))
    o = O.Model(synthetic_config(arch, 16), ot)
    compare_stream(g, o, [1, 4, 44, 12, 30], 16)
    # and it is not the F32 model
    f = P.load_gguf(b).cache(4).forward(1, 0)
    assert not same_bits(f, g.cache(4).forward(1, 0))


MIX_CFG = dict(dim=256, hidden_dim=512, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=300, seq_len=40, head_dim=64,
               rope_theta=1e6, norm_eps=float(np.float32(1e-6)), emb_scale=1.0, rope_neox=1, act=0)
MIX_TYPES = {"attn_q.weight": P.Q4_K, "attn_k.weight": P.Q8_0, "attn_v.weight": P.Q4_0, "attn_output.weight": P.F16,
             "ffn_gate.weight": P.Q4_K, "ffn_down.weight": P.Q6_K, "ffn_up.weight": P.F32}


def mixed_file(emb_type, head_type, seed=0):
    """A qwen2 file mixing every stored type; returns (bytes, oracle tensors)."""
    c = MIX_CFG
    rng = np.random.default_rng(seed)
    w = W.Writer()
    w.kv("general.architecture", W.STR, "qwen2")
    for k, v in [("embedding_length", c["dim"]), ("block_count", c["n_layers"]), ("attention.head_count", 4),
                 ("attention.head_count_kv", 2), ("feed_forward_length", c["hidden_dim"]),
                 ("context_length", c["seq_len"])]:
        w.kv(f"qwen2.{k}", W.U32, v)
    w.kv("qwen2.rope.freq_base", W.F32V, 1e6)
    w.kv("qwen2.attention.layer_norm_rms_epsilon", W.F32V, 1e-6)
    w.kv("tokenizer.ggml.tokens", W.ARR, [b"t%d" % i for i in range(c["vocab_size"])], W.STR)
    ot = {}

    def add(name, ty, rows, cols, s):
        if ty == P.F32:
            raw = (rng.standard_normal(rows * cols) * 0.05).astype(np.float32).view(np.uint8)
        elif ty == P.F16:
            raw = (rng.standard_normal(rows * cols) * 0.05).astype(np.float16).view(np.uint8)
        else:
            raw = P.synth_tensor(ty, rows, cols, s, 0.05)
        dims = [cols, rows]
        w.tensor(name, dims, ty, raw.tobytes())
        if ty == P.F16:  # the oracle takes the decoded rows (gguf.rs:217-221)
            ot[name] = (0, dims, raw.view(np.float16).astype(np.float32))
        else:
            ot[name] = (ty, dims, raw)

    d, h, kvd = c["dim"], c["hidden_dim"], 2 * 64
    add("token_embd.weight", emb_type, c["vocab_size"], d, 1)
    shapes = {"attn_q.weight": (d, d), "attn_k.weight": (kvd, d), "attn_v.weight": (kvd, d),
              "attn_output.weight": (d, d), "ffn_gate.weight": (h, d), "ffn_down.weight": (d, h),
              "ffn_up.weight": (h, d)}
    for layer in range(c["n_layers"]):
        p = f"blk.{layer}."
        for key, ty in MIX_TYPES.items():
            rows, cols = shapes[key]
            add(p + key, ty, rows, cols, 100 * layer + ty)
        for key, n in [("attn_norm.weight", d), ("ffn_norm.weight", d), ("attn_q.bias", d), ("attn_k.bias", kvd),
                       ("attn_v.bias", kvd)]:
            v = (1.0 + rng.standard_normal(n) * 0.1).astype(np.float32)
            w.tensor(p + key, [n], P.F32, v.tobytes())
            ot[p + key] = (0, [n], v)
    v = (1.0 + rng.standard_normal(d) * 0.1).astype(np.float32)
    w.tensor("output_norm.weight", [d], P.F32, v.tobytes())
    ot["output_norm.weight"] = (0, [d], v)
    if head_type is not None:
        add("output.weight", head_type, c["vocab_size"], d, 9)
    return w.to_bytes(), ot


@pytest.mark.parametrize("emb_type,head_type", [(P.Q6_K, None), (P.Q4_0, P.Q8_0), (P.Q8_0, P.Q4_K),
                                                (P.F16, None), (P.Q4_K, P.Q6_K)])
def test_mixed_types_bitexact(emb_type, head_type):
    b, ot = mixed_file(emb_type, head_type, seed=emb_type)
    g = P.load_gguf(b)
    assert g.config == {**MIX_CFG, "norm_eps": g.config["norm_eps"]}
    o = O.Model(MIX_CFG, ot)
    prompt = np.random.default_rng(5).integers(0, 300, 12).astype(np.uint32)
    gc, oc = g.cache(40), o.cache(40)
    gc.prefill(prompt[:-1])
    oc.prefill(prompt[:-1])
    for layer in (0, 1):
        for which in (0, 1):
            assert np.array_equal(gc.read(layer, which, 11), oc.read(layer, which, 11))
    tok = int(prompt[-1])
    for pos in range(11, 16):
        lg, lo = gc.forward(tok, pos), oc.forward(tok, pos)
        assert same_bits(lg, lo), pos
        tok = int(O.argmax(lo))
    got, _ = g.generate(prompt[:5], 20)
    want, _ = o.generate(prompt[:5], 20)
    assert list(got) == list(want)


def test_kquant_rows_not_whole_superblocks_are_decoded(tmp_path):
    # dim 288: a Q4_K / Q6_K matrix of 288 columns is not packed by the
    # reference (cols % 256 != 0) but decoded to dense rows; the element count
    # stays a multiple of 256. Loaded from a path (memory-mapped).
    c = dict(dim=288, hidden_dim=512, n_layers=1, n_heads=4, n_kv_heads=4, vocab_size=64, seq_len=16, head_dim=72,
             rope_theta=1e4, norm_eps=float(np.float32(1e-5)), emb_scale=1.0, rope_neox=0, act=0)
    rng = np.random.default_rng(11)
    w = W.Writer().kv("general.architecture", W.STR, "llama")
    for k, v in [("embedding_length", 288), ("block_count", 1), ("attention.head_count", 4),
                 ("feed_forward_length", 512), ("context_length", 16)]:
        w.kv(f"llama.{k}", W.U32, v)
    w.kv("tokenizer.ggml.tokens", W.ARR, [b"x"] * 64, W.STR)
    ot = {}

    def add(name, ty, rows, cols):
        raw = P.synth_tensor(ty, 1, rows * cols, rows + cols + ty, 0.05)
        w.tensor(name, [cols, rows], ty, raw.tobytes())
        packed = (ty in (P.Q8_0, P.Q4_0) and cols % 32 == 0) or (ty in (P.Q4_K, P.Q6_K) and cols % 256 == 0)
        if packed:
            ot[name] = (ty, [cols, rows], raw)
        else:  # the oracle gets the decoded rows (Linear::new(tensor_f32(..)))
            ot[name] = (0, [cols, rows], O.Mat.from_ggml(ty, 1, rows * cols, raw).row_f32(0))

    add("token_embd.weight", P.Q4_K, 64, 288)  # dense table (288 % 256 != 0)
    add("blk.0.attn_q.weight", P.Q4_K, 288, 288)
    add("blk.0.attn_k.weight", P.Q6_K, 288, 288)
    add("blk.0.attn_v.weight", P.Q8_0, 288, 288)
    add("blk.0.attn_output.weight", P.Q6_K, 288, 288)
    add("blk.0.ffn_gate.weight", P.Q4_K, 512, 288)
    add("blk.0.ffn_down.weight", P.Q6_K, 288, 512)  # 512 columns: packed
    add("blk.0.ffn_up.weight", P.Q4_0, 512, 288)
    for name, n in [("blk.0.attn_norm.weight", 288), ("blk.0.ffn_norm.weight", 288), ("output_norm.weight", 288)]:
        v = (1.0 + rng.standard_normal(n) * 0.1).astype(np.float32)
        w.tensor(name, [n], P.F32, v.tobytes())
        ot[name] = (0, [n], v)
    path = tmp_path / "m.gguf"
    path.write_bytes(w.to_bytes())
    g = P.load_gguf(str(path))
    o = O.Model(c, ot)
    compare_stream(g, o, [5, 63, 0, 17, 17, 40], 16)


def test_missing_tensor_and_bad_precision():
    b, tensors = W.reference_synthetic_model("llama", False, 16)
    w = W.Writer()
    g = P.Gguf(data=b)
    with pytest.raises(KeyError):
        P.load_gguf(g, precision="q4")
    # drop one projection: rewrite the file without it
    src = P.Gguf(data=b)
    w.kv("general.architecture", W.STR, "llama")
    for k in ["embedding_length", "block_count", "attention.head_count", "attention.head_count_kv",
              "feed_forward_length", "context_length", "attention.key_length"]:
        w.kv(f"llama.{k}", W.U32, src.meta_usize(f"llama.{k}"))
    w.kv("tokenizer.ggml.tokens", W.ARR, src.meta_array_str("tokenizer.ggml.tokens"), W.STR)
    for name, (dims, data) in tensors.items():
        if name != "blk.1.ffn_up.weight":
            w.tensor(name, dims, 0, data.tobytes())
    with pytest.raises(P.PranaError, match="missing tensor 'blk.1.ffn_up.weight'"):
        P.load_gguf(w.to_bytes())


@pytest.mark.parametrize("temp", [0.0, 0.9])
def test_text_in_text_out(temp):
    # model and tokenizer from one file (gguf.rs:338-460), then generate from
    # text (infer.rs:696-771): the token stream equals the oracle's for the
    # same encoded prompt, stops are the tokenizer's, pieces decode it
    b, tensors = W.reference_synthetic_model("qwen2", True, 16)
    g = P.Gguf(data=b)
    model, tok = P.load_gguf(g), P.Tokenizer.from_gguf(g)
    prompt = "ab cab"
    ids = tok.encode_prompt(prompt)
    o = O.Model(synthetic_config("qwen2", 16), oracle_tensors(tensors, False))
    sampler = P.Sampler(temp, 17) if temp > 0 else None
    pieces, st = P.generate_text(model, tok, prompt, 8, sampler)
    if temp > 0:
        want = O.generate_sampled(o, ids, 8, O.Sampler(temp, 17), stops=tok.stop_ids())
    else:
        want, _ = o.generate(ids, 8, stops=tok.stop_ids())
    gen = [p for p, in_prompt in pieces if not in_prompt]
    assert len(gen) == st.generated_tokens == len(want)
    prev = ids[-1]
    for piece, t in zip(gen, want):
        assert piece == tok.decode(prev, int(t))
        prev = int(t)
    assert b"".join(p for p, in_prompt in pieces if in_prompt) == b"".join(
        tok.decode(a, c) for a, c in zip(ids[:-1], ids[1:]))
