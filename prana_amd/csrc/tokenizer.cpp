// Tokenizers (prana-model tokenizer.rs, bpe.rs; load_tokenizer in gguf.rs),
// host code. Text is UTF-8 bytes; strings read from GGUF metadata are decoded
// the way Rust's String::from_utf8_lossy does (each maximal invalid subpart
// becomes U+FFFD).
#include "tokenizer.h"

#include <algorithm>
#include <cstring>

#include "common.h"
#include "gguf.h"
#include "unicode_alpha.h"

namespace prana {

namespace {

void put_utf8(std::string& out, uint32_t cp) {
  if (cp < 0x80) {
    out += static_cast<char>(cp);
  } else if (cp < 0x800) {
    out += static_cast<char>(0xC0 | (cp >> 6));
    out += static_cast<char>(0x80 | (cp & 0x3F));
  } else if (cp < 0x10000) {
    out += static_cast<char>(0xE0 | (cp >> 12));
    out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
    out += static_cast<char>(0x80 | (cp & 0x3F));
  } else {
    out += static_cast<char>(0xF0 | (cp >> 18));
    out += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
    out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
    out += static_cast<char>(0x80 | (cp & 0x3F));
  }
}

// Length of the well-formed UTF-8 sequence at s[i], or 0 with *bad = the
// length of its maximal invalid subpart (at least 1).
size_t utf8_seq(const unsigned char* s, size_t n, size_t i, size_t* bad) {
  const unsigned b = s[i];
  if (b < 0x80) return 1;
  size_t need;
  unsigned lo = 0x80, hi = 0xBF;
  if (b >= 0xC2 && b <= 0xDF) {
    need = 1;
  } else if (b >= 0xE0 && b <= 0xEF) {
    need = 2;
    if (b == 0xE0) lo = 0xA0;
    if (b == 0xED) hi = 0x9F;
  } else if (b >= 0xF0 && b <= 0xF4) {
    need = 3;
    if (b == 0xF0) lo = 0x90;
    if (b == 0xF4) hi = 0x8F;
  } else {
    *bad = 1;
    return 0;
  }
  size_t j = i + 1;
  for (size_t k = 0; k < need; k++, j++) {
    const unsigned c = j < n ? s[j] : 0x100;
    const unsigned l = k == 0 ? lo : 0x80, h = k == 0 ? hi : 0xBF;
    if (c < l || c > h) {
      *bad = j - i;
      return 0;
    }
  }
  return need + 1;
}

uint32_t cp_at(const unsigned char* s, size_t i, size_t len) {
  if (len == 1) return s[i];
  if (len == 2) return ((s[i] & 0x1Fu) << 6) | (s[i + 1] & 0x3Fu);
  if (len == 3) return ((s[i] & 0x0Fu) << 12) | ((s[i + 1] & 0x3Fu) << 6) | (s[i + 2] & 0x3Fu);
  return ((s[i] & 0x07u) << 18) | ((s[i + 1] & 0x3Fu) << 12) | ((s[i + 2] & 0x3Fu) << 6) | (s[i + 3] & 0x3Fu);
}

// String::from_utf8_lossy.
std::string lossy(const std::string& in) {
  const auto* s = reinterpret_cast<const unsigned char*>(in.data());
  std::string out;
  out.reserve(in.size());
  for (size_t i = 0; i < in.size();) {
    size_t bad = 0;
    const size_t len = utf8_seq(s, in.size(), i, &bad);
    if (len) {
      out.append(in, i, len);
      i += len;
    } else {
      out += "\xEF\xBF\xBD";  // U+FFFD
      i += bad;
    }
  }
  return out;
}

bool is_alphabetic(uint32_t cp) {
  size_t lo = 0, hi = sizeof(kAlphaRanges) / sizeof(kAlphaRanges[0]);
  while (lo < hi) {
    const size_t mid = (lo + hi) / 2;
    if (cp < kAlphaRanges[mid][0]) {
      hi = mid;
    } else if (cp > kAlphaRanges[mid][1]) {
      lo = mid + 1;
    } else {
      return true;
    }
  }
  return false;
}

std::string replace_all(std::string s, const std::string& from, const std::string& to) {
  for (size_t p = s.find(from); p != std::string::npos; p = s.find(from, p + to.size())) s.replace(p, from.size(), to);
  return s;
}

const GValue* meta(const Gguf& g, const char* key) { return g.find(key); }

}  // namespace

bool utf8_valid(const std::string& in) {
  const auto* s = reinterpret_cast<const unsigned char*>(in.data());
  for (size_t i = 0; i < in.size();) {
    size_t bad = 0;
    const size_t len = utf8_seq(s, in.size(), i, &bad);
    if (!len) return false;
    i += len;
  }
  return true;
}

// ------------------------------------------------------------------ SentencePiece (tokenizer.rs)
void SpmTokenizer::build_lookup() {
  lookup.clear();
  lookup.reserve(vocab.size());
  for (size_t id = 0; id < vocab.size(); id++) lookup.emplace(vocab[id], static_cast<uint32_t>(id));
}

// Tokenizer::encode (tokenizer.rs:89-143): BOS, the dummy " " prefix, one
// token per code point (byte fallback <0xNN> = byte + 3), then repeatedly the
// best-scoring adjacent merge (strictly greater score; the leftmost wins).
std::vector<uint32_t> SpmTokenizer::encode(const std::string& text, bool bos, bool eos) const {
  std::vector<uint32_t> t;
  if (bos) t.push_back(bos_id);
  if (!text.empty()) {
    auto sp = lookup.find(" ");
    if (sp != lookup.end()) t.push_back(sp->second);
  }
  const auto* s = reinterpret_cast<const unsigned char*>(text.data());
  for (size_t i = 0; i < text.size();) {
    size_t bad = 0;
    const size_t len = std::max<size_t>(utf8_seq(s, text.size(), i, &bad), 1);  // text is valid UTF-8
    auto it = lookup.find(text.substr(i, len));
    if (it != lookup.end()) {
      t.push_back(it->second);
    } else {
      for (size_t k = 0; k < len; k++) t.push_back(static_cast<uint32_t>(s[i + k]) + 3);
    }
    i += len;
  }
  std::string merged;
  while (t.size() >= 2) {
    bool found = false;
    float best = 0.0f;
    size_t bi = 0;
    uint32_t bid = 0;
    for (size_t i = 0; i + 1 < t.size(); i++) {
      if (t[i] >= vocab.size() || t[i + 1] >= vocab.size()) continue;  // fallback id past the vocab
      merged.assign(vocab[t[i]]);
      merged += vocab[t[i + 1]];
      auto it = lookup.find(merged);
      if (it == lookup.end()) continue;
      const float sc = scores[it->second];
      if (!found || sc > best) {
        found = true;
        best = sc;
        bi = i;
        bid = it->second;
      }
    }
    if (!found) break;
    t[bi] = bid;
    t.erase(t.begin() + static_cast<std::ptrdiff_t>(bi) + 1);
  }
  if (eos) t.push_back(eos_id);
  return t;
}

// Tokenizer::decode (tokenizer.rs:147-162): <0xNN> pieces are raw bytes (the
// two characters parsed as u8 in base 16, which takes a leading '+'); the
// space of a piece right after BOS is dropped.
std::string SpmTokenizer::decode(uint32_t prev, uint32_t token) const {
  if (token >= vocab.size()) return std::string();
  const std::string& p = vocab[token];
  if (p.size() == 6 && p.compare(0, 3, "<0x") == 0 && p[5] == '>') {
    auto hex = [](char c) -> int {
      if (c >= '0' && c <= '9') return c - '0';
      if (c >= 'a' && c <= 'f') return c - 'a' + 10;
      if (c >= 'A' && c <= 'F') return c - 'A' + 10;
      return -1;
    };
    int v = -1;
    if (p[3] == '+') {
      v = hex(p[4]);
    } else if (hex(p[3]) >= 0 && hex(p[4]) >= 0) {
      v = hex(p[3]) * 16 + hex(p[4]);
    }
    if (v >= 0) return std::string(1, static_cast<char>(v));
  }
  if (prev == bos_id && !p.empty() && p[0] == ' ') return p.substr(1);
  return p;
}

// ------------------------------------------------------------------ byte-level BPE (bpe.rs)
void BpeTokenizer::build(const std::vector<std::string>& merges) {
  lookup.clear();
  for (size_t id = 0; id < vocab.size(); id++) lookup.emplace(vocab[id], static_cast<uint32_t>(id));
  ranks.clear();
  for (size_t r = 0; r < merges.size(); r++) {
    const size_t sp = merges[r].find(' ');
    if (sp == std::string::npos) continue;
    ranks[merges[r].substr(0, sp) + '\xff' + merges[r].substr(sp + 1)] = static_cast<uint32_t>(r);
  }
  // bytes_to_unicode (bpe.rs:23-36): printable bytes map to themselves, the
  // others to 256, 257, ... in byte order
  uint32_t n = 0;
  byte_dec.clear();
  for (uint32_t b = 0; b < 256; b++) {
    const bool printable = (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || (b >= 174 && b <= 255);
    const uint32_t cp = printable ? b : 256 + n++;
    byte_enc[b].clear();
    put_utf8(byte_enc[b], cp);
    byte_dec[cp] = static_cast<uint8_t>(b);
  }
}

// bpe_piece (bpe.rs:142-170): one symbol per mapped byte, then repeatedly the
// lowest-ranked adjacent merge (the leftmost on a tie); unknown symbols drop.
std::vector<uint32_t> BpeTokenizer::bpe_piece(const std::string& piece) const {
  std::vector<std::string> sym;
  sym.reserve(piece.size());
  for (unsigned char b : piece) sym.push_back(byte_enc[b]);
  std::string key;
  while (sym.size() >= 2) {
    bool found = false;
    uint32_t best = 0;
    size_t bi = 0;
    for (size_t i = 0; i + 1 < sym.size(); i++) {
      key.assign(sym[i]);
      key += '\xff';
      key += sym[i + 1];
      auto it = ranks.find(key);
      if (it != ranks.end() && (!found || it->second < best)) {
        found = true;
        best = it->second;
        bi = i;
      }
    }
    if (!found) break;
    sym[bi] += sym[bi + 1];
    sym.erase(sym.begin() + static_cast<std::ptrdiff_t>(bi) + 1);
  }
  std::vector<uint32_t> ids;
  for (const auto& s : sym) {
    auto it = lookup.find(s);
    if (it != lookup.end()) ids.push_back(it->second);
  }
  return ids;
}

// encode_prompt (bpe.rs:173-206): BOS if configured; special tokens matched
// verbatim first (the earliest occurrence; at one position the longest, as
// the list is sorted longest first), BPE over the text between them.
std::vector<uint32_t> BpeTokenizer::encode_prompt(const std::string& text) const {
  std::vector<uint32_t> out;
  if (add_bos && has_bos) out.push_back(bos_id);
  size_t at0 = 0;
  while (at0 < text.size()) {
    size_t hit = std::string::npos, hit_len = 0;
    uint32_t hit_id = 0;
    for (const auto& sp : specials) {
      const size_t p = text.find(sp.first, at0);
      if (p != std::string::npos && (hit == std::string::npos || p < hit)) {
        hit = p;
        hit_len = sp.first.size();
        hit_id = sp.second;
      }
    }
    const size_t plain_end = hit == std::string::npos ? text.size() : hit;
    const std::string plain = text.substr(at0, plain_end - at0);
    for (const auto& pr : bpe_pre_tokenize(plain)) {
      const auto ids = bpe_piece(plain.substr(pr.first, pr.second - pr.first));
      out.insert(out.end(), ids.begin(), ids.end());
    }
    if (hit == std::string::npos) break;
    out.push_back(hit_id);
    at0 = hit + hit_len;
  }
  return out;
}

std::string BpeTokenizer::decode(uint32_t token) const {
  if (token >= vocab.size()) return std::string();
  const std::string& s = vocab[token];
  const auto* u = reinterpret_cast<const unsigned char*>(s.data());
  std::string out;
  for (size_t i = 0; i < s.size();) {
    size_t bad = 0;
    const size_t len = std::max<size_t>(utf8_seq(u, s.size(), i, &bad), 1);
    auto it = byte_dec.find(cp_at(u, i, len));
    if (it != byte_dec.end()) out += static_cast<char>(it->second);
    i += len;
  }
  return out;
}

// pre_tokenize (bpe.rs:96-139): runs of one class (alphabetic, ASCII digit,
// space, other) with a single pending space attached to the word after it.
std::vector<std::pair<size_t, size_t>> bpe_pre_tokenize(const std::string& text) {
  enum Class { kLetter, kDigit, kOther, kSpace };
  std::vector<std::pair<size_t, size_t>> out;
  const auto* s = reinterpret_cast<const unsigned char*>(text.data());
  size_t cb = 0, ce = 0;  // current piece [cb, ce)
  Class cur_class = kSpace;
  for (size_t i = 0; i < text.size();) {
    size_t bad = 0;
    const size_t len = std::max<size_t>(utf8_seq(s, text.size(), i, &bad), 1);
    const uint32_t cp = cp_at(s, i, len);
    const Class cl = is_alphabetic(cp) ? kLetter : (cp >= '0' && cp <= '9') ? kDigit : cp == ' ' ? kSpace : kOther;
    const bool empty = ce == cb;
    const bool single_space = ce - cb == 1 && s[cb] == ' ';
    bool starts_new;
    if (empty) {
      starts_new = false;
    } else if (single_space && cl != kSpace) {
      starts_new = false;
    } else {
      starts_new = cl != cur_class;
    }
    if (starts_new || (cl == kSpace && !empty && s[ce - 1] != ' ')) {
      out.emplace_back(cb, ce);
      cb = ce;
    }
    ce = i + len;
    cur_class = cl;
    i += len;
  }
  if (ce > cb) out.emplace_back(cb, ce);
  return out;
}

// ------------------------------------------------------------------ loaders
int tokenizer_from_gguf(const Gguf& g, Tokenizer& out) {
  const GValue* toks = meta(g, "tokenizer.ggml.tokens");
  if (!toks || toks->type != 9) return fail(kErrInvalid, "missing tokenizer.ggml.tokens");
  const GValue* mv = meta(g, "tokenizer.ggml.model");
  const std::string model = mv && mv->type == 8 ? lossy(mv->s) : std::string("llama");
  uint64_t v;
  const GValue* e;
  const bool has_bos = (e = meta(g, "tokenizer.ggml.bos_token_id")) && gvalue_as_u64(*e, &v);
  const uint32_t bos = has_bos ? static_cast<uint32_t>(v) : 0;
  const bool has_eos = (e = meta(g, "tokenizer.ggml.eos_token_id")) && gvalue_as_u64(*e, &v);
  const uint32_t eos = has_eos ? static_cast<uint32_t>(v) : 0;
  const GValue* ab = meta(g, "tokenizer.ggml.add_bos_token");
  const bool add_bos = ab && ab->type == 7 ? ab->u != 0 : model == "llama";
  auto piece = [](const GValue& x) { return x.type == 8 ? x.s : std::string(); };
  if (model == "llama") {
    Tokenizer t;
    t.kind = 0;
    for (const GValue& x : toks->arr) t.spm.vocab.push_back(replace_all(lossy(piece(x)), "\xE2\x96\x81", " "));
    const GValue* sc = meta(g, "tokenizer.ggml.scores");
    if (sc && sc->type == 9) {
      for (const GValue& x : sc->arr) {
        float f = 0.0f;
        t.spm.scores.push_back(gvalue_as_f32(x, &f) ? f : 0.0f);
      }
    } else {
      t.spm.scores.assign(t.spm.vocab.size(), 0.0f);
    }
    if (t.spm.scores.size() != t.spm.vocab.size())
      return fail(kErrInvalid, "tokenizer.ggml.scores and tokenizer.ggml.tokens differ in length");
    t.spm.build_lookup();
    t.spm.bos_id = has_bos ? bos : 1;
    t.spm.eos_id = has_eos ? eos : 2;
    t.spm.add_bos = add_bos;
    out = std::move(t);
    return kOk;
  }
  if (model == "gpt2") {
    Tokenizer t;
    t.kind = 1;
    for (const GValue& x : toks->arr) t.bpe.vocab.push_back(lossy(piece(x)));
    const GValue* mg = meta(g, "tokenizer.ggml.merges");
    if (!mg || mg->type != 9) return fail(kErrInvalid, "gpt2 tokenizer requires tokenizer.ggml.merges");
    std::vector<std::string> merges;
    for (const GValue& x : mg->arr) merges.push_back(lossy(piece(x)));
    t.bpe.build(merges);
    t.bpe.has_bos = has_bos;
    t.bpe.bos_id = bos;
    t.bpe.has_eos = has_eos;
    t.bpe.eos_id = eos;
    t.bpe.add_bos = add_bos;
    // token_type 3 (CONTROL) / 4 (USER_DEFINED): verbatim specials
    const GValue* tt = meta(g, "tokenizer.ggml.token_type");
    if (tt && tt->type == 9) {
      for (size_t id = 0; id < tt->arr.size(); id++) {
        if (!gvalue_as_u64(tt->arr[id], &v) || (v != 3 && v != 4)) continue;
        if (id >= t.bpe.vocab.size())
          return fail(kErrInvalid, "tokenizer.ggml.token_type is longer than tokenizer.ggml.tokens");
        // an empty special would match everywhere without consuming text
        if (!t.bpe.vocab[id].empty()) t.bpe.specials.emplace_back(t.bpe.vocab[id], static_cast<uint32_t>(id));
      }
      std::stable_sort(t.bpe.specials.begin(), t.bpe.specials.end(),
                       [](const auto& a, const auto& b) { return a.first.size() > b.first.size(); });
    }
    out = std::move(t);
    return kOk;
  }
  return fail(kErrUnsupported, "unsupported tokenizer.ggml.model '" + model + "'");
}

int tokenizer_from_llama2c(const uint8_t* data, size_t n, size_t vocab_size, Tokenizer& out) {
  Tokenizer t;
  t.kind = 0;
  size_t off = 4;  // max_token_length, unused
  for (size_t i = 0; i < vocab_size; i++) {
    if (off > n || n - off < 8) return fail(kErrInvalid, "tokenizer.bin truncated");
    float sc;
    uint32_t len;
    std::memcpy(&sc, data + off, 4);
    std::memcpy(&len, data + off + 4, 4);
    if (n - off - 8 < len) return fail(kErrInvalid, "tokenizer.bin truncated");
    t.spm.scores.push_back(sc);
    t.spm.vocab.emplace_back(reinterpret_cast<const char*>(data + off + 8), len);
    off += 8 + static_cast<size_t>(len);
  }
  t.spm.build_lookup();
  out = std::move(t);
  return kOk;
}

}  // namespace prana
