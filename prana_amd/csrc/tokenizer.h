// Tokenizers of prana-model (tokenizer.rs, bpe.rs, gguf.rs load_tokenizer),
// host code: SentencePiece-style greedy score merges with byte fallback, and
// GPT-2 byte-level BPE with ranked merges and verbatim special tokens.
#pragma once

#include <cstdint>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace prana {

struct Gguf;

// Tokenizer (tokenizer.rs:28-176).
struct SpmTokenizer {
  std::vector<std::string> vocab;  // piece bytes by id
  std::vector<float> scores;
  std::unordered_map<std::string, uint32_t> lookup;  // first occurrence wins
  uint32_t bos_id = 1, eos_id = 2;
  bool add_bos = true;

  void build_lookup();
  std::vector<uint32_t> encode(const std::string& text, bool bos, bool eos) const;
  std::string decode(uint32_t prev, uint32_t token) const;
  bool is_stop(uint32_t t) const { return t == eos_id || t == bos_id; }
};

// BpeTokenizer (bpe.rs:38-241).
struct BpeTokenizer {
  std::vector<std::string> vocab;  // strings over the byte-unicode alphabet
  std::unordered_map<std::string, uint32_t> lookup;
  std::unordered_map<std::string, uint32_t> ranks;  // "left\xffright" -> rank; a later duplicate wins
  std::string byte_enc[256];                         // byte -> UTF-8 of its mapped char
  std::unordered_map<uint32_t, uint8_t> byte_dec;    // mapped code point -> byte
  bool has_bos = false, has_eos = false;
  uint32_t bos_id = 0, eos_id = 0;
  bool add_bos = false;
  std::vector<std::pair<std::string, uint32_t>> specials;  // longest first

  void build(const std::vector<std::string>& merges);
  std::vector<uint32_t> bpe_piece(const std::string& piece) const;
  std::vector<uint32_t> encode_prompt(const std::string& text) const;
  std::string decode(uint32_t token) const;
  bool is_stop(uint32_t t) const { return (has_eos && t == eos_id) || (has_bos && t == bos_id); }
};

// Byte offsets [begin, end) of the pieces of the approximate GPT-2
// pre-tokenization (bpe.rs:96-139) of valid UTF-8 text.
std::vector<std::pair<size_t, size_t>> bpe_pre_tokenize(const std::string& text);
bool utf8_valid(const std::string& s);

struct Tokenizer {
  int kind = 0;  // 0 SentencePiece, 1 byte-level BPE
  SpmTokenizer spm;
  BpeTokenizer bpe;
  size_t vocab_size() const { return kind == 0 ? spm.vocab.size() : bpe.vocab.size(); }
  std::vector<uint32_t> encode_prompt(const std::string& text) const {
    return kind == 0 ? spm.encode(text, spm.add_bos, false) : bpe.encode_prompt(text);
  }
  std::string decode(uint32_t prev, uint32_t token) const {
    return kind == 0 ? spm.decode(prev, token) : bpe.decode(token);
  }
  bool is_stop(uint32_t t) const { return kind == 0 ? spm.is_stop(t) : bpe.is_stop(t); }
};

// load_tokenizer (gguf.rs:466-537).
int tokenizer_from_gguf(const Gguf& g, Tokenizer& out);
// Tokenizer::from_bytes (tokenizer.rs:65-82): llama2.c's tokenizer.bin.
int tokenizer_from_llama2c(const uint8_t* data, size_t n, size_t vocab_size, Tokenizer& out);

}  // namespace prana

struct prana_tokenizer {
  prana::Tokenizer t;
};
