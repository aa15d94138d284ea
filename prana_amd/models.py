"""Seeded random-init model shapes for the benchmark configurations.

Weights are N(0, sigma) drawn by prana_synth_tensor and encoded straight into
ggml block bytes; norm weights are 1.0; biases (qwen2) are N(0, sigma). Each
tensor's seed is derived from the model seed and the tensor's GGUF name, so a
model is a pure function of (shape, types, seed): the GPU model and the CPU
oracle are built from the very same bytes.
"""
import numpy as np

from . import F32, Q4_0, Q4_K, Q6_K, Q8_0, synth_tensor


def _name_seed(seed, name):
    h = 0xCBF29CE484222325
    for b in name.encode():
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return (h ^ (seed * 0x9E3779B97F4A7C15)) & 0xFFFFFFFFFFFFFFFF


def config(dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len, head_dim=None, rope_theta=10000.0,
           norm_eps=1e-5, rope_neox=0, act=0, emb_scale=1.0):
    return dict(dim=dim, hidden_dim=hidden_dim, n_layers=n_layers, n_heads=n_heads, n_kv_heads=n_kv_heads,
                vocab_size=vocab_size, seq_len=seq_len, head_dim=head_dim or dim // n_heads,
                rope_theta=float(rope_theta), norm_eps=float(norm_eps), emb_scale=float(emb_scale),
                rope_neox=int(rope_neox), act=int(act))


# Config 0: stories15M shape (llama), Q8_0, untied Q8_0 head.
C0 = config(288, 768, 6, 6, 6, 32000, 256)
# Config 2: qwen2-0.5B shape, NeoX theta 1e6, eps 1e-6, QKV biases.
C2 = config(896, 4864, 24, 14, 2, 151936, 4096, head_dim=64, rope_theta=1e6, norm_eps=1e-6, rope_neox=1)
# Config 4: llama-7B shape, Q4_0 everywhere, untied head.
C4 = config(4096, 14336, 32, 32, 8, 32000, 4096, head_dim=128)


def types_c0(name, cols):
    return Q8_0


def types_c2(name, cols):
    """Q4_K_M-style mixture: attn_v and ffn_down Q6_K, the rest Q4_K; tensors
    whose cols are not a multiple of 256 (every K=896 tensor) fall back to the
    nearest native block type (Q4_K -> Q4_0, Q6_K -> Q8_0), since the reference
    loads K-quants only when cols % 256 == 0 (gguf.rs:295-296)."""
    k6 = name.endswith("attn_v.weight") or name.endswith("ffn_down.weight")
    if cols % 256 == 0:
        return Q6_K if k6 else Q4_K
    return Q8_0 if k6 else Q4_0


def types_c4(name, cols):
    return Q4_0


def tensor_specs(cfg, untied_head=True, biases=False):
    """[(name, dims(ggml order), kind)] with kind in {'mat', 'norm', 'bias'}."""
    d, hid, hd = cfg["dim"], cfg["hidden_dim"], cfg["head_dim"]
    q_dim, kv_dim = cfg["n_heads"] * hd, cfg["n_kv_heads"] * hd
    specs = [("token_embd.weight", (d, cfg["vocab_size"]), "mat")]
    for i in range(cfg["n_layers"]):
        b = f"blk.{i}."
        specs += [
            (b + "attn_norm.weight", (d,), "norm"),
            (b + "attn_q.weight", (d, q_dim), "mat"),
            (b + "attn_k.weight", (d, kv_dim), "mat"),
            (b + "attn_v.weight", (d, kv_dim), "mat"),
            (b + "attn_output.weight", (q_dim, d), "mat"),
            (b + "ffn_norm.weight", (d,), "norm"),
            (b + "ffn_gate.weight", (d, hid), "mat"),
            (b + "ffn_down.weight", (hid, d), "mat"),
            (b + "ffn_up.weight", (d, hid), "mat"),
        ]
        if biases:
            specs += [(b + "attn_q.bias", (q_dim,), "bias"), (b + "attn_k.bias", (kv_dim,), "bias"),
                      (b + "attn_v.bias", (kv_dim,), "bias")]
    specs.append(("output_norm.weight", (d,), "norm"))
    if untied_head:
        specs.append(("output.weight", (d, cfg["vocab_size"]), "mat"))
    return specs


def synth_tensors(cfg, types, seed, sigma=0.02, untied_head=True, biases=False, only=None):
    """{name: (ggml_type, dims, bytes)} for a random-init model."""
    out = {}
    for name, dims, kind in tensor_specs(cfg, untied_head, biases):
        if only is not None and name not in only:
            continue
        if kind == "norm":
            out[name] = (F32, dims, np.ones(dims[0], np.float32).view(np.uint8))
        elif kind == "bias":
            out[name] = (F32, dims, synth_tensor(F32, 1, dims[0], _name_seed(seed, name), sigma))
        else:
            cols, rows = dims
            ty = types(name, cols)
            out[name] = (ty, dims, synth_tensor(ty, rows, cols, _name_seed(seed, name), sigma))
    return out


def c0_tensors(seed=1):
    return synth_tensors(C0, types_c0, seed)


def c2_tensors(seed=2):
    return synth_tensors(C2, types_c2, seed, untied_head=False, biases=True)


def c4_tensors(seed=4, n_layers=None):
    cfg = dict(C4)
    if n_layers is not None:
        cfg["n_layers"] = n_layers
    return synth_tensors(cfg, types_c4, seed)


def c4_draft_config():
    """Config-0 shape as the speculative draft; its context is widened to the
    target's so both caches cover the same positions (KvCache::with_len would
    otherwise cap the draft at 256)."""
    cfg = dict(C0)
    cfg["seq_len"] = C4["seq_len"]
    return cfg
