"""GGUF container parsing on the host (no GPU): the library's reader against
the reference's own known-answer tests (gguf.rs:888-1071), its synthetic model
files (gguf.rs:566-666, restated in tests/golden/gguf_writer.py), the oracle's
block decoders for random blocks, and malformed input.

Known-answer files: tests/golden/gguf/*.gguf (written by gguf_writer.py)."""
import math
import os
import struct

import numpy as np
import pytest

import prana_amd as P
from oracle import oracle as O
from tests.golden import gguf_writer as W

GOLD = W.GOLDEN_DIR


def gold(name):
    return os.path.join(GOLD, name)


def test_committed_kat_files_match_the_writer():
    for name, fn in W.KATS.items():
        with open(gold(name), "rb") as f:
            assert f.read() == fn(), name


# ------------------------------------------------------------------ the reference's known answers
def test_metadata_and_f32_tensor():
    # parses_metadata_and_f32_tensor (gguf.rs:899-925)
    g = P.Gguf(path=gold("metadata_f32.gguf"))
    assert g.counts() == (3, 1, 2)
    assert g.meta_usize("llama.block_count") == 6
    assert g.meta_str("general.architecture") == b"llama"
    assert g.meta_type("llama.block_count") == (W.U32, -1)
    assert g.tensor_f32("t").tolist() == [0.0, 1.0, 2.0, 3.0, 4.0, 5.0]
    assert g.tensor_info("t") == (0, [2, 3], 24)
    with pytest.raises(P.PranaError, match="missing tensor 'nope'"):
        g.tensor_f32("nope")
    with pytest.raises(P.PranaError, match="missing metadata"):
        g.meta_usize("general.architecture")  # a string is not an integer (Value::as_usize)


def test_q4_0_tensor_known_values():
    # q4_0_tensor_loads_natively_packed (gguf.rs:989-1036)
    g = P.Gguf(path=gold("q4_0.gguf"))
    f = g.tensor_f32("w")
    assert [f[j] for j in range(16)] == [j - 8.0 for j in range(16)]
    assert [f[16 + j] for j in range(16)] == [(15 - j) - 8.0 for j in range(16)]
    assert np.all(f[32:] == 0.5 * (12.0 - 8.0))
    assert g.tensor_info("w") == (P.Q4_0, [64, 1], 2 * 18)
    # the packed bytes come back as stored
    assert g.tensor_bytes("w") == W.kat_q4_0()[-36:]


def test_q8_0_tensor_known_values():
    # q8_0_tensor_loads_natively_as_quantmatrix (gguf.rs:1038-1071)
    g = P.Gguf(path=gold("q8_0.gguf"))
    f = g.tensor_f32("w")
    assert f.tolist() == [float(i - 16) for i in range(32)]
    assert float(f.sum()) == -16.0


def test_kquant_blocks_known_values():
    g = P.Gguf(path=gold("kquants.gguf"))
    # q4k_block_dequantizes_known_values (gguf.rs:927-953)
    y = g.tensor_f32("q4k")
    assert y.size == 256
    for i in range(32):
        assert y[i] == 2.0 * (i % 16)
        assert y[32 + i] == 3.0 * (15 - i % 16)
    assert np.all(y[64:] == 0.0)
    # q4k_packed_scale_min_high_groups_unpack (gguf.rs:955-968): group 4 has
    # (sc, m) = (53, 43), so a nibble of 1 decodes to 53 - 43
    y = g.tensor_f32("q4k_hi")
    assert np.all(y[128:160] == 10.0)
    assert np.all(y[:128] == 0.0) and np.all(y[160:] == 0.0)
    # q6k_block_dequantizes_known_values (gguf.rs:970-987)
    y = g.tensor_f32("q6k")
    assert y[0] == 5.0 and y[1] == -32.0 and y[64] == -32.0


def test_f16_tensor_known_values():
    # f16_conversion_covers_the_cases (gguf.rs:888-897)
    f = P.Gguf(path=gold("f16.gguf")).tensor_f32("h")
    assert f[0] == 0.0 and f[1] == 1.0 and f[2] == -2.0 and f[3] == math.inf
    assert math.isnan(f[4])
    assert f[5] == 2.0 ** -24
    assert abs(f[6] - 0.33325) < 1e-4
    assert f[7] == 0.0 and math.copysign(1.0, f[7]) == -1.0


@pytest.mark.parametrize("ty", [P.Q4_0, P.Q8_0, P.Q4_K, P.Q6_K, P.F16])
def test_tensor_f32_matches_the_oracle_decoders(ty):
    # random blocks of every stored type: the host decoders against the
    # oracle's (kquant.rs:39-112, gguf.rs:234-245), bit for bit
    rows, cols = 5, 512
    if ty == P.F16:
        raw = np.random.default_rng(3).standard_normal(rows * cols).astype(np.float16).view(np.uint8)
        want = raw.view(np.float16).astype(np.float32)
    else:
        raw = P.synth_tensor(ty, rows, cols, 77 + ty, 0.05)
        m = O.Mat.from_ggml(ty, rows, cols, raw)
        want = np.concatenate([m.row_f32(r) for r in range(rows)])
    b = W.Writer().tensor("w", [cols, rows], ty, raw.tobytes()).to_bytes()
    got = P.Gguf(data=b).tensor_f32("w")
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ------------------------------------------------------------------ the reference's synthetic model files
@pytest.mark.parametrize("arch,biases,hd", [("llama", False, 16), ("qwen2", True, 16), ("gemma", False, 16),
                                            ("gemma", False, 8)])
def test_synthetic_model_parses(arch, biases, hd):
    b, tensors = W.reference_synthetic_model(arch, biases, hd)
    g = P.Gguf(data=b)
    assert g.counts() == (3, len(tensors), 11)
    assert g.tensor_names() == list(tensors)
    for name, (dims, data) in tensors.items():
        ty, d, nb = g.tensor_info(name)
        assert (ty, d, nb) == (0, dims, data.nbytes)
        assert np.array_equal(g.tensor_f32(name), data)
    toks = g.meta_array_str("tokenizer.ggml.tokens")
    assert toks == [W.spm_piece(i) for i in range(48)]
    assert g.meta_array_f32("tokenizer.ggml.scores").tolist() == [-1.0] * 48
    assert g.meta_str("tokenizer.ggml.model") == b"llama"
    c = g.model_config()
    # the knobs of gguf.rs:340-378,410-425
    assert (c["dim"], c["hidden_dim"], c["n_layers"], c["n_heads"], c["n_kv_heads"]) == (32, 64, 2, 2, 2)
    assert (c["vocab_size"], c["seq_len"], c["head_dim"]) == (48, 16, hd)
    assert c["rope_theta"] == 10000.0 and c["norm_eps"] == np.float32(1e-5)
    assert c["rope_neox"] == (arch != "llama")
    assert c["act"] == (1 if arch == "gemma" else 0)
    assert c["emb_scale"] == (np.float32(np.sqrt(np.float32(32))) if arch == "gemma" else 1.0)


def _cfg_file(arch="llama", kv=(), drop=()):
    w = W.Writer().kv("general.architecture", W.STR, arch)
    base = {"embedding_length": (W.U32, 64), "block_count": (W.U32, 1), "attention.head_count": (W.U32, 4),
            "feed_forward_length": (W.U32, 128), "context_length": (W.U32, 32)}
    for k, (ty, v) in base.items():
        if k not in drop:
            w.kv(f"{arch}.{k}", ty, v)
    for k, ty, v in kv:
        w.kv(k, ty, v)
    if "tokens" not in drop:
        w.kv("tokenizer.ggml.tokens", W.ARR, [b"a", b"b", b"c"], W.STR)
    return P.Gguf(data=w.to_bytes())


def test_config_defaults_and_value_types():
    c = _cfg_file().model_config()
    # head_count_kv = head_count, key_length = dim / heads, freq_base 1e4, eps 1e-5
    assert (c["n_kv_heads"], c["head_dim"], c["rope_theta"]) == (4, 16, 10000.0)
    assert c["norm_eps"] == np.float32(1e-5) and c["vocab_size"] == 3
    c = _cfg_file(kv=[("llama.attention.head_count_kv", W.I32, 2), ("llama.rope.freq_base", W.F64, 5e5),
                      ("llama.attention.layer_norm_rms_epsilon", W.F32V, 1e-6),
                      ("llama.attention.key_length", W.U64, 32)]).model_config()
    assert (c["n_kv_heads"], c["head_dim"], c["rope_theta"]) == (2, 32, 5e5)
    assert c["norm_eps"] == np.float32(1e-6)
    # a negative head_count_kv is not an integer for as_usize: the default holds
    assert _cfg_file(kv=[("llama.attention.head_count_kv", W.I32, -2)]).model_config()["n_kv_heads"] == 4
    # an integer freq_base is not a float for as_f32: the default holds
    assert _cfg_file(kv=[("llama.rope.freq_base", W.U32, 7)]).model_config()["rope_theta"] == 10000.0


def test_config_errors():
    with pytest.raises(P.PranaError, match="unsupported architecture 'mistral'"):
        _cfg_file("mistral").model_config()
    with pytest.raises(P.PranaError, match="missing metadata 'llama.block_count'"):
        _cfg_file(drop=("block_count",)).model_config()
    with pytest.raises(P.PranaError, match="missing tokenizer.ggml.tokens"):
        _cfg_file(drop=("tokens",)).model_config()
    with pytest.raises(P.PranaError, match="missing general.architecture"):
        P.Gguf(data=W.Writer().to_bytes()).model_config()


# ------------------------------------------------------------------ layout and malformed input
def test_alignment_key_and_version_2():
    data = np.arange(40, dtype=np.float32)
    for align, used in [(64, 64), (128, 128), (48, 32), (0, 32)]:
        w = W.Writer(version=2, alignment=used).kv("general.alignment", W.U32, align)
        w.tensor("a", [8], 0, data[:8].tobytes()).tensor("b", [32], 0, data[8:].tobytes())
        g = P.Gguf(data=w.to_bytes())
        assert g.counts()[0] == 2
        assert np.array_equal(g.tensor_f32("a"), data[:8]) and np.array_equal(g.tensor_f32("b"), data[8:])


def test_bad_magic_and_versions():
    good = W.kat_metadata_f32()
    with pytest.raises(P.PranaError, match="bad magic"):
        P.Gguf(data=b"GGUG" + good[4:])
    for v in (1, 4):
        with pytest.raises(P.PranaError, match=f"unsupported GGUF version {v}"):
            P.Gguf(data=good[:4] + struct.pack("<I", v) + good[8:])


def test_every_truncation_fails_cleanly():
    full = W.kat_metadata_f32()
    for n in range(len(full)):
        try:
            g = P.Gguf(data=full[:n])
        except P.PranaError as e:
            assert "truncated" in str(e)
            continue
        # the header parsed: the tensor's bytes are what is missing
        with pytest.raises(P.PranaError, match="out of range"):
            g.tensor_f32("t")
    assert P.Gguf(data=full).tensor_f32("t").size == 6


def test_unknown_value_type_and_huge_array():
    w = W.Writer().kv_raw(W.gstr("x") + struct.pack("<I", 13) + b"\0" * 8)
    with pytest.raises(P.PranaError, match="unsupported gguf value type 13"):
        P.Gguf(data=w.to_bytes())
    # an array claiming 2^62 elements in a short file is truncated, not allocated
    w = W.Writer().kv_raw(W.gstr("a") + struct.pack("<IIQ", W.ARR, W.U8, 1 << 62))
    with pytest.raises(P.PranaError, match="truncated"):
        P.Gguf(data=w.to_bytes())


def nested(depth, leaf=b""):
    """An array value nested `depth` levels deep: each level one array of one
    array, the innermost an empty array of u8 (or `leaf` after its header)."""
    raw = struct.pack("<IQ", W.U8, 0) + leaf
    for _ in range(depth - 1):
        raw = struct.pack("<IQ", W.ARR, 1) + raw
    return raw


def test_nested_arrays_parse_like_the_reference():
    # Reader::value (gguf.rs:118-125) reads arrays of arrays; the entries after
    # them still parse, and the array reports its element type
    inner = struct.pack("<IQ", W.U32, 2) + struct.pack("<II", 7, 8)
    empty = struct.pack("<IQ", W.ARR, 0)
    w = W.Writer().kv_raw(W.gstr("arrs") + struct.pack("<IIQ", W.ARR, W.ARR, 2) + inner + inner)
    w.kv_raw(W.gstr("none") + struct.pack("<I", W.ARR) + empty)
    w.kv_raw(W.gstr("deep") + struct.pack("<I", W.ARR) + nested(16))
    w.kv("after", W.U32, 5)
    g = P.Gguf(data=w.to_bytes())
    assert g.meta_type("arrs") == (W.ARR, W.ARR)
    assert g.meta_type("none") == (W.ARR, W.ARR)
    assert g.meta_usize("after") == 5
    # an unknown element type inside a nested array is named
    bad = struct.pack("<IQ", W.ARR, 1) + struct.pack("<IQ", 13, 1) + b"\0" * 8
    with pytest.raises(P.PranaError, match="unsupported gguf value type 13"):
        P.Gguf(data=W.Writer().kv_raw(W.gstr("x") + struct.pack("<I", W.ARR) + bad).to_bytes())
    # deeper than 16 levels is refused (the reference would recurse), and a
    # nested count beyond the file's bytes is a truncation
    with pytest.raises(P.PranaError, match="nested deeper than 16"):
        P.Gguf(data=W.Writer().kv_raw(W.gstr("x") + struct.pack("<I", W.ARR) + nested(17)).to_bytes())
    huge = struct.pack("<IQ", W.ARR, 1) + struct.pack("<IQ", W.ARR, 1 << 40)
    with pytest.raises(P.PranaError, match="truncated"):
        P.Gguf(data=W.Writer().kv_raw(W.gstr("x") + struct.pack("<I", W.ARR) + huge).to_bytes())


def test_tensor_with_many_dimensions():
    # TensorInfo keeps any number of dims (gguf.rs:179-186); the library opens
    # the file and reads the data; only the fixed 8-entry dims buffer of
    # prana_gguf_tensor_info refuses more
    dims = [1, 2, 1, 1, 3, 1, 1, 1, 1, 2]
    vals = np.arange(12, dtype=np.float32)
    w = W.Writer().tensor("t10", dims, 0, vals.tobytes()).tensor("t2", [3, 2], 0, vals[:6].tobytes())
    g = P.Gguf(data=w.to_bytes())
    assert g.tensor_f32("t10").tolist() == vals.tolist()
    assert g.tensor_bytes("t10") == vals.tobytes()
    assert g.tensor_info("t2")[1] == [3, 2]
    with pytest.raises(P.PranaError, match="has 10 dimensions"):
        g.tensor_info("t10")
    import ctypes as C
    nd = C.c_int()
    assert P.load().prana_gguf_tensor_info(g.h, b"t10", None, None, C.byref(nd), None) == 0 and nd.value == 10
    # a dims count beyond the file's bytes is a truncation, not an allocation
    raw = bytearray(w.to_bytes())
    at = raw.index(b"t10") + 3
    raw[at:at + 4] = struct.pack("<I", 1 << 30)
    with pytest.raises(P.PranaError, match="truncated"):
        P.Gguf(data=bytes(raw))


def test_tensor_type_and_alignment_errors():
    w = W.Writer().tensor("q41", [32], 3, b"\0" * 20).tensor("odd", [48], P.Q4_0, b"\0" * 27)
    w.tensor("kq", [128], P.Q4_K, b"\0" * 144)
    g = P.Gguf(data=w.to_bytes())
    with pytest.raises(P.PranaError, match="unsupported ggml type 3"):
        g.tensor_f32("q41")
    with pytest.raises(P.PranaError, match="Q4_0 tensor 'odd' not block-aligned"):
        g.tensor_f32("odd")
    with pytest.raises(P.PranaError, match="K-quant tensor 'kq' not block-aligned"):
        g.tensor_f32("kq")


def test_duplicate_names_last_wins_and_short_buffers():
    w = W.Writer().tensor("t", [2], 0, np.float32([1, 2]).tobytes()).tensor("t", [3], 0,
                                                                           np.float32([3, 4, 5]).tobytes())
    g = P.Gguf(data=w.to_bytes())
    assert g.counts()[1] == 1 and g.tensor_f32("t").tolist() == [3.0, 4.0, 5.0]
    # the caller-sized buffer protocol: a short buffer reports the size needed
    import ctypes as C
    n = C.c_size_t()
    rc = P.load().prana_gguf_tensor_f32(g.h, b"t", None, 0, C.byref(n))
    assert rc == P._lib.ERR_SHORT_BUFFER and n.value == 3


def test_open_missing_file(tmp_path):
    with pytest.raises(P.PranaError, match="cannot open"):
        P.Gguf(path=str(tmp_path / "absent.gguf"))
    p = tmp_path / "m.gguf"
    p.write_bytes(W.kat_q8_0())
    assert P.Gguf(path=str(p)).tensor_f32("w")[0] == -16.0
