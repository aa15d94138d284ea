"""The library's tokenizers (host code, no GPU) against the reference's own
tokenizer tests (tokenizer.rs:212-270, bpe.rs:215-275) and load_tokenizer's
rules (gguf.rs:466-537), plus round trips and malformed input."""
import struct

import pytest

import prana_amd as P
from tests.golden import gguf_writer as W


def llama2c(entries):
    """A tokenizer.bin image from (score, piece) entries (tokenizer.rs:217-226)."""
    data = struct.pack("<I", 8)
    for score, piece in entries:
        data += struct.pack("<fI", score, len(piece)) + piece
    return P.Tokenizer.from_llama2c(data, len(entries))


def tiny_spm():
    return llama2c([(0.0, b"<unk>"), (0.0, b"<s>"), (0.0, b"</s>"), (-1.0, b" "), (-2.0, b"h"), (-2.0, b"i"),
                    (-1.5, b"hi"), (-1.2, b" hi")])


# ------------------------------------------------------------------ SentencePiece
def test_spm_greedy_merges_and_dummy_prefix():
    # encodes_with_greedy_merges_and_dummy_prefix (tokenizer.rs:242-247)
    assert tiny_spm().encode("hi", True, False) == [1, 7]


def test_spm_byte_fallback():
    # byte_fallback_for_unknown_chars (tokenizer.rs:249-254)
    assert tiny_spm().encode("z", False, False) == [3, ord("z") + 3]
    # a multi-byte character without a piece falls back byte by byte
    assert tiny_spm().encode("é", False, True) == [3, 0xC3 + 3, 0xA9 + 3, 2]
    assert tiny_spm().encode("", True, True) == [1, 2]  # no dummy prefix for empty text


def test_spm_decode():
    # decode_strips_space_after_bos_and_parses_byte_tokens (tokenizer.rs:256-262)
    t = llama2c([(0.0, b"<unk>"), (0.0, b"<s>"), (0.0, b"</s>"), (-1.0, b" word"), (0.0, b"<0x0A>"),
                 (0.0, b"<0x+A>"), (0.0, b"<0xZZ>")])
    assert t.decode(1, 3) == b"word"
    assert t.decode(9, 3) == b" word"
    assert t.decode(3, 4) == b"\n"
    assert t.decode(3, 5) == b"\n"  # u8::from_str_radix takes a leading '+'
    assert t.decode(3, 6) == b"<0xZZ>"  # not hex: the piece itself
    assert t.decode(3, 99) == b""  # past the vocabulary
    assert t.is_stop(1) and t.is_stop(2) and not t.is_stop(3)


def test_spm_merge_order_is_best_score_then_leftmost():
    # "aaa": pairs (a,a) at 0 and 1 both merge to "aa"; the leftmost is taken
    # first, leaving "aa"+"a"; "aaa" itself then outranks nothing else
    t = llama2c([(0.0, b"<unk>"), (0.0, b"<s>"), (0.0, b"</s>"), (-1.0, b"a"), (-0.5, b"aa"), (-0.7, b"aaa"),
                 (-3.0, b" ")])
    assert t.encode("aaa", False, False) == [6, 5]  # " " stays: " a" is no piece
    assert t.encode("aaaa", False, False) == [6, 4, 4]


def test_llama2c_truncated():
    with pytest.raises(P.PranaError, match="truncated"):
        P.Tokenizer.from_llama2c(struct.pack("<IfI", 8, 0.0, 5) + b"ab", 1)


# ------------------------------------------------------------------ byte-level BPE
def byte_unicode():
    """bytes_to_unicode (bpe.rs:23-36), independently: the printable bytes keep
    their code point, the rest take 256.. in byte order."""
    out, n = {}, 0
    for b in range(256):
        if 33 <= b <= 126 or 161 <= b <= 172 or 174 <= b <= 255:
            out[b] = chr(b)
        else:
            out[b] = chr(256 + n)
            n += 1
    return out


def bpe_file(vocab, merges, eos=None, bos=None, types=None, add_bos=None):
    w = W.Writer().kv("tokenizer.ggml.model", W.STR, "gpt2")
    w.kv("tokenizer.ggml.tokens", W.ARR, [v.encode() for v in vocab], W.STR)
    w.kv("tokenizer.ggml.merges", W.ARR, [m.encode() for m in merges], W.STR)
    if eos is not None:
        w.kv("tokenizer.ggml.eos_token_id", W.U32, eos)
    if bos is not None:
        w.kv("tokenizer.ggml.bos_token_id", W.U32, bos)
    if add_bos is not None:
        w.kv("tokenizer.ggml.add_bos_token", W.BOOL, int(add_bos))
    if types is not None:
        w.kv("tokenizer.ggml.token_type", W.ARR, types, W.I32)
    return P.Tokenizer.from_gguf(P.Gguf(data=w.to_bytes()))


def tiny_bpe(types=None):
    # tiny (bpe.rs:220-233)
    sp = byte_unicode()[ord(" ")]
    vocab = ["h", "i", sp, "hi", f"{sp}hi", "<|endoftext|>"]
    return bpe_file(vocab, ["h i", f"{sp} hi"], eos=5, types=types)


def test_bpe_merges_apply_in_rank_order():
    t = tiny_bpe()
    assert t.kind == "bpe" and t.vocab_size == 6
    assert t.encode_prompt("hi") == [3]
    assert t.encode_prompt(" hi") == [4]


def test_bpe_decode_roundtrips_bytes_and_stops():
    t = tiny_bpe()
    assert b"".join(t.decode(0, i) for i in t.encode_prompt(" hi")) == b" hi"
    assert t.is_stop(5) and not t.is_stop(3)
    assert t.stop_ids() == [5]


def test_bpe_pre_tokenizer():
    # pre_tokenizer_keeps_leading_spaces_on_words (bpe.rs:252-256)
    assert P.bpe_pre_tokenize("hello world 42!") == ["hello", " world", " 42", "!"]
    assert P.bpe_pre_tokenize("a  b") == ["a", "  ", "b"]
    assert P.bpe_pre_tokenize(" x\ty") == [" x", "\t", "y"]
    # Unicode letters (Rust's char::is_alphabetic); a non-ASCII digit is
    # "other" and takes the pending space like a word
    assert P.bpe_pre_tokenize("naïve café ١٢") == ["naïve", " café", " ١٢"]
    # U+0345 is Alphabetic (Other_Alphabetic), U+0301 is not; U+2160 (Nl) is
    assert P.bpe_pre_tokenize("a\u0345b") == ["a\u0345b"]
    assert P.bpe_pre_tokenize("e\u0301x") == ["e", "\u0301", "x"]
    assert P.bpe_pre_tokenize("x\u2160") == ["x\u2160"]
    assert P.bpe_pre_tokenize("") == []


def test_bpe_special_tokens_verbatim():
    # special_tokens_encode_verbatim_not_split (bpe.rs:258-267); type 3 = CONTROL
    t = tiny_bpe(types=[1, 1, 1, 1, 1, 3])
    assert t.encode_prompt("hi<|endoftext|> hi") == [3, 5, 4]
    assert t.encode_prompt("<|endoftext|>") == [5]
    assert tiny_bpe().encode_prompt("hi<|endoftext|> hi") != [3, 5, 4]


def test_bpe_full_byte_vocab_roundtrip():
    # a vocab holding every mapped byte encodes and decodes any UTF-8 text
    bu = byte_unicode()
    vocab = [bu[b] for b in range(256)] + ["<s>"]
    t = bpe_file(vocab, [], bos=256, add_bos=True)
    text = "Grüße, 世界! 123 \n\t x"
    ids = t.encode_prompt(text)
    assert ids[0] == 256
    assert b"".join(t.decode(0, i) for i in ids[1:]) == text.encode()


# ------------------------------------------------------------------ load_tokenizer (gguf.rs:466-537)
def test_gguf_spm_defaults_and_word_marker():
    w = W.Writer()  # no tokenizer.ggml.model: llama
    w.kv("tokenizer.ggml.tokens", W.ARR, [b"<unk>", b"<s>", b"</s>", "▁hi".encode(), b"h", b"i", "▁".encode(), b"hi"],
         W.STR)
    t = P.Tokenizer.from_gguf(P.Gguf(data=w.to_bytes()))
    assert t.kind == "spm" and t.vocab_size == 8
    # scores default to 0: the first mergeable pair wins ("h"+"i", as " "+"h"
    # is no piece), then " "+"hi"; U+2581 reads as a space; BOS by default
    assert t.encode_prompt("hi") == [1, 3]
    assert t.decode(1, 3) == b"hi" and t.decode(4, 3) == b" hi"
    assert t.stop_ids() == [2, 1]


def test_gguf_spm_special_ids_and_add_bos():
    w = W.Writer().kv("tokenizer.ggml.model", W.STR, "llama")
    w.kv("tokenizer.ggml.tokens", W.ARR, [b"<pad>", b"</s>", b"<s>", b"a"], W.STR)
    w.kv("tokenizer.ggml.scores", W.ARR, [0.0, 0.0, 0.0, -1.0], W.F32V)
    w.kv("tokenizer.ggml.bos_token_id", W.U32, 2).kv("tokenizer.ggml.eos_token_id", W.U32, 1)
    w.kv("tokenizer.ggml.add_bos_token", W.BOOL, 0)
    t = P.Tokenizer.from_gguf(P.Gguf(data=w.to_bytes()))
    assert t.encode_prompt("a") == [3] and t.is_stop(1) and t.is_stop(2) and not t.is_stop(0)


def test_gguf_tokenizer_errors():
    with pytest.raises(P.PranaError, match="missing tokenizer.ggml.tokens"):
        P.Tokenizer.from_gguf(P.Gguf(data=W.Writer().to_bytes()))
    w = W.Writer().kv("tokenizer.ggml.model", W.STR, "gpt2").kv("tokenizer.ggml.tokens", W.ARR, [b"a"], W.STR)
    with pytest.raises(P.PranaError, match="requires tokenizer.ggml.merges"):
        P.Tokenizer.from_gguf(P.Gguf(data=w.to_bytes()))
    w = W.Writer().kv("tokenizer.ggml.model", W.STR, "bert").kv("tokenizer.ggml.tokens", W.ARR, [b"a"], W.STR)
    with pytest.raises(P.PranaError, match="unsupported tokenizer.ggml.model 'bert'"):
        P.Tokenizer.from_gguf(P.Gguf(data=w.to_bytes()))
    w = W.Writer().kv("tokenizer.ggml.tokens", W.ARR, [b"a", b"b"], W.STR)
    w.kv("tokenizer.ggml.scores", W.ARR, [0.0], W.F32V)
    with pytest.raises(P.PranaError, match="differ in length"):
        P.Tokenizer.from_gguf(P.Gguf(data=w.to_bytes()))
    with pytest.raises(P.PranaError, match="not valid UTF-8"):
        tiny_spm().encode_prompt(b"\xff")


def test_reference_synthetic_model_tokenizer():
    # the tokenizer of the reference's synthetic model files (gguf.rs:616-641)
    b, _ = W.reference_synthetic_model("llama", False, 16)
    t = P.Tokenizer.from_gguf(P.Gguf(data=b))
    assert t.vocab_size == 48 and t.kind == "spm"
    ids = t.encode_prompt("ab ba")
    assert ids[0] == 1 and ids[1] == 3
    # the dummy space right after BOS is dropped when decoding
    assert b"".join(t.decode(p, i) for p, i in zip(ids[:-1], ids[1:])) == b"ab ba"
