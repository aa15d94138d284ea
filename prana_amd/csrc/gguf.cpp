// GGUF container -> device model: the reference's loader (prana-model
// gguf.rs) on the host side of the boundary. The file is mapped read-only,
// its header, metadata and tensor directory are parsed (gguf.rs:157-196),
// tensors are read in place (gguf.rs:202-264) and the model is assembled with
// the architecture knobs of gguf.rs:338-437 (llama / qwen2 / gemma). Packed
// formats go to the device unchanged through Model::set_tensor.
#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstring>

#include "model.h"

namespace prana {

namespace {

constexpr uint32_t kGgufMagic = 0x46554747u;  // "GGUF" little-endian
// Arrays of arrays are read to this depth; a deeper file is refused rather
// than recursed into without bound.
constexpr int kMaxNesting = 16;

struct Cursor {
  const uint8_t* p;
  size_t n, off = 0;
  bool take(uint64_t k, const uint8_t** out) {
    if (k > n - off) return false;
    *out = p + off;
    off += static_cast<size_t>(k);
    return true;
  }
  template <class T>
  bool pod(T* v) {
    const uint8_t* b;
    if (!take(sizeof(T), &b)) return false;
    std::memcpy(v, b, sizeof(T));
    return true;
  }
  bool str(std::string* s) {
    uint64_t len;
    const uint8_t* b;
    if (!pod(&len) || !take(len, &b)) return false;
    s->assign(reinterpret_cast<const char*>(b), static_cast<size_t>(len));
    return true;
  }
};

// Reader::value (gguf.rs:102-130): value types 0..12, arrays of any element
// type including arrays. Returns 0, or 1 for a truncated file, 2 for an
// unknown value type (stored in *bad), 3 for arrays nested deeper than
// kMaxNesting.
int read_value(Cursor& c, uint32_t ty, GValue* v, uint32_t* bad, int depth = 0) {
  v->type = ty;
  switch (ty) {
    case 0: { uint8_t x; if (!c.pod(&x)) return 1; v->u = x; return 0; }
    case 1: { int8_t x; if (!c.pod(&x)) return 1; v->i = x; return 0; }
    case 2: { uint16_t x; if (!c.pod(&x)) return 1; v->u = x; return 0; }
    case 3: { int16_t x; if (!c.pod(&x)) return 1; v->i = x; return 0; }
    case 4: { uint32_t x; if (!c.pod(&x)) return 1; v->u = x; return 0; }
    case 5: { int32_t x; if (!c.pod(&x)) return 1; v->i = x; return 0; }
    case 6: { float x; if (!c.pod(&x)) return 1; v->f = x; return 0; }
    case 7: { uint8_t x; if (!c.pod(&x)) return 1; v->u = x != 0; return 0; }
    case 8: return c.str(&v->s) ? 0 : 1;
    case 9: {
      uint64_t count;
      if (!c.pod(&v->elem_type) || !c.pod(&count)) return 1;
      if (v->elem_type == 9 && count > 0 && depth + 1 >= kMaxNesting) return 3;
      // every element takes at least one byte (a nested array's header 12),
      // so a count beyond the bytes left is a truncated file
      if (count > c.n - c.off) return 1;
      v->arr.resize(static_cast<size_t>(count));
      for (auto& e : v->arr)
        if (int rc = read_value(c, v->elem_type, &e, bad, depth + 1)) return rc;
      return 0;
    }
    case 10: { uint64_t x; if (!c.pod(&x)) return 1; v->u = x; return 0; }
    case 11: { int64_t x; if (!c.pod(&x)) return 1; v->i = x; return 0; }
    case 12: { double x; if (!c.pod(&x)) return 1; v->f = x; return 0; }
  }
  *bad = ty;
  return 2;
}

float f16_le(const uint8_t* b) { return host_f16_to_f32(static_cast<uint16_t>(b[0] | (b[1] << 8))); }

// Host block decoders (kquant.rs:39-112).
void dq_q40(const uint8_t* b, float* y) {
  const float d = f16_le(b);
  for (int j = 0; j < 16; j++) {
    y[j] = d * (static_cast<float>(b[2 + j] & 0xF) - 8.0f);
    y[16 + j] = d * (static_cast<float>(b[2 + j] >> 4) - 8.0f);
  }
}
void q4k_scale_min(int j, const uint8_t* s, float* sc, float* m) {
  if (j < 4) {
    *sc = static_cast<float>(s[j] & 63);
    *m = static_cast<float>(s[j + 4] & 63);
  } else {
    *sc = static_cast<float>((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
    *m = static_cast<float>((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
  }
}
void dq_q4k(const uint8_t* b, float* y) {
  const float d = f16_le(b), dmin = f16_le(b + 2);
  for (int p = 0; p < 4; p++) {
    float sc1, m1, sc2, m2;
    q4k_scale_min(2 * p, b + 4, &sc1, &m1);
    q4k_scale_min(2 * p + 1, b + 4, &sc2, &m2);
    const float d1 = d * sc1, mn1 = dmin * m1, d2 = d * sc2, mn2 = dmin * m2;
    const uint8_t* q = b + 16 + 32 * p;
    for (int l = 0; l < 32; l++) {
      y[64 * p + l] = d1 * static_cast<float>(q[l] & 0xF) - mn1;
      y[64 * p + 32 + l] = d2 * static_cast<float>(q[l] >> 4) - mn2;
    }
  }
}
void dq_q6k(const uint8_t* b, float* y) {
  const int8_t* sc = reinterpret_cast<const int8_t*>(b + 192);
  const float d = f16_le(b + 208);
  for (int h = 0; h < 2; h++) {
    const uint8_t *ql = b + 64 * h, *qh = b + 128 + 32 * h;
    float* yo = y + 128 * h;
    for (int l = 0; l < 32; l++) {
      const int is = 8 * h + l / 16;
      const float q1 = static_cast<float>(((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32);
      const float q2 = static_cast<float>(((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32);
      const float q3 = static_cast<float>(((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
      const float q4 = static_cast<float>(((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
      yo[l] = (d * static_cast<float>(sc[is])) * q1;
      yo[l + 32] = (d * static_cast<float>(sc[is + 2])) * q2;
      yo[l + 64] = (d * static_cast<float>(sc[is + 4])) * q3;
      yo[l + 96] = (d * static_cast<float>(sc[is + 6])) * q4;
    }
  }
}

// quantize_q8 (matmul.rs:61-84): per 32-block scale = amax/127 (1.0 for a
// zero block; NaN elements do not count toward amax), q = clamp(round(x *
// (1/scale)), -127, 127), rounding half away from zero, NaN to 0.
void quantize_q8_host(size_t rows, size_t cols, const float* w, std::vector<int8_t>& q, std::vector<float>& sc) {
  const size_t G = cols / 32;
  q.resize(rows * cols);
  sc.resize(rows * G);
  for (size_t r = 0; r < rows; r++)
    for (size_t g = 0; g < G; g++) {
      const float* x = w + r * cols + g * 32;
      float amax = 0.0f;
      for (int i = 0; i < 32; i++) amax = std::fmax(amax, std::fabs(x[i]));
      const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
      const float inv = 1.0f / scale;
      for (int i = 0; i < 32; i++) {
        const float v = std::round(x[i] * inv);  // a NaN casts to 0 (Rust's saturating `as i8`)
        q[r * cols + g * 32 + i] = v != v ? 0 : static_cast<int8_t>(v < -127.0f ? -127.0f : v > 127.0f ? 127.0f : v);
      }
      sc[r * G + g] = scale;
    }
}

bool checked_elems(const std::vector<uint64_t>& dims, uint64_t* n) {
  uint64_t p = 1;
  for (uint64_t d : dims) {
    if (d != 0 && p > UINT64_MAX / d) return false;
    p *= d;
  }
  *n = p;
  return true;
}

}  // namespace

bool gvalue_as_u64(const GValue& v, uint64_t* out) {
  switch (v.type) {
    case 0: case 2: case 4: case 10: *out = v.u; return true;
    case 1: case 3: case 5: case 11:
      if (v.i < 0) return false;
      *out = static_cast<uint64_t>(v.i);
      return true;
  }
  return false;
}

bool gvalue_as_f32(const GValue& v, float* out) {
  if (v.type != 6 && v.type != 12) return false;
  *out = static_cast<float>(v.f);
  return true;
}

Gguf::~Gguf() {
  if (map) munmap(map, size);
}

int Gguf::parse() {  // Gguf::from_bytes (gguf.rs:162-196)
  Cursor c{base, size};
  uint32_t magic = 0;
  uint64_t n_tensors = 0, n_kv = 0;
  if (!c.pod(&magic)) return fail(kErrInvalid, "gguf truncated");
  if (magic != kGgufMagic) return fail(kErrInvalid, "not a GGUF file (bad magic)");
  if (!c.pod(&version)) return fail(kErrInvalid, "gguf truncated");
  if (version < 2 || version > 3) return fail(kErrUnsupported, "unsupported GGUF version " + std::to_string(version));
  if (!c.pod(&n_tensors) || !c.pod(&n_kv)) return fail(kErrInvalid, "gguf truncated");
  for (uint64_t i = 0; i < n_kv; i++) {
    std::string key;
    uint32_t ty;
    GValue v;
    if (!c.str(&key) || !c.pod(&ty)) return fail(kErrInvalid, "gguf truncated");
    uint32_t bad = 0;
    if (int rc = read_value(c, ty, &v, &bad)) {
      if (rc == 1) return fail(kErrInvalid, "gguf truncated");
      if (rc == 3)
        return fail(kErrUnsupported, "gguf arrays nested deeper than " + std::to_string(kMaxNesting) + " ('" + key +
                                         "')");
      return fail(kErrUnsupported, "unsupported gguf value type " + std::to_string(bad) + " ('" +
                                       key + "')");
    }
    meta[key] = std::move(v);
  }
  for (uint64_t i = 0; i < n_tensors; i++) {
    std::string name;
    uint32_t nd;
    GTensor t;
    if (!c.str(&name) || !c.pod(&nd)) return fail(kErrInvalid, "gguf truncated");
    if (nd > (c.n - c.off) / 8) return fail(kErrInvalid, "gguf truncated");  // 8 bytes per dim
    t.dims.resize(nd);
    for (auto& d : t.dims)
      if (!c.pod(&d)) return fail(kErrInvalid, "gguf truncated");
    if (!c.pod(&t.type) || !c.pod(&t.offset)) return fail(kErrInvalid, "gguf truncated");
    if (!tensors.count(name)) names.push_back(name);
    tensors[name] = std::move(t);
  }
  uint64_t align = 32, a;
  const GValue* al = find("general.alignment");
  if (al && gvalue_as_u64(*al, &a) && a > 0 && (a & (a - 1)) == 0) align = a;
  const uint64_t off = c.off;
  data_start = static_cast<size_t>((off + align - 1) / align * align);
  return kOk;
}

const GValue* Gguf::find(const std::string& key) const {
  auto it = meta.find(key);
  return it == meta.end() ? nullptr : &it->second;
}

int Gguf::raw(const std::string& name, const GTensor** t, const uint8_t** bytes, size_t* nbytes) const {
  auto it = tensors.find(name);
  if (it == tensors.end()) return fail(kErrInvalid, "missing tensor '" + name + "'");
  *t = &it->second;
  uint64_t n;
  if (!checked_elems(it->second.dims, &n) || n > (uint64_t{1} << 40))
    return fail(kErrInvalid, "tensor '" + name + "': element count out of range");
  const int ty = static_cast<int>(it->second.type);
  if (ty != 0 && ty != 1 && ty != 2 && ty != 8 && ty != 12 && ty != 14)
    return fail(kErrUnsupported, "tensor '" + name + "': unsupported ggml type " + std::to_string(ty));
  const size_t need = ggml_nbytes(ty, static_cast<size_t>(n));
  if (need == 0 && n != 0)
    return fail(kErrInvalid, std::string(ty == 2 ? "Q4_0" : ty == 8 ? "Q8_0" : "K-quant") + " tensor '" + name +
                                 "' not block-aligned");
  const uint64_t start = static_cast<uint64_t>(data_start) + it->second.offset;
  if (start < it->second.offset || start > size || need > size - start)
    return fail(kErrInvalid, "tensor data out of range ('" + name + "')");
  *bytes = base + start;
  *nbytes = need;
  return kOk;
}

int Gguf::tensor_f32(const std::string& name, std::vector<float>& out) const {
  const GTensor* t;
  const uint8_t* b;
  size_t nb;
  if (int rc = raw(name, &t, &b, &nb)) return rc;
  uint64_t n;
  checked_elems(t->dims, &n);
  out.resize(static_cast<size_t>(n));
  switch (t->type) {
    case 0: if (n) std::memcpy(out.data(), b, static_cast<size_t>(n) * 4); break;
    case 1: for (size_t i = 0; i < n; i++) out[i] = f16_le(b + 2 * i); break;
    case 2: for (size_t k = 0; k < n / 32; k++) dq_q40(b + 18 * k, out.data() + 32 * k); break;
    case 8:
      for (size_t k = 0; k < n / 32; k++) {
        const float s = f16_le(b + 34 * k);
        for (int j = 0; j < 32; j++) out[32 * k + j] = static_cast<float>(static_cast<int8_t>(b[34 * k + 2 + j])) * s;
      }
      break;
    case 12: for (size_t k = 0; k < n / 256; k++) dq_q4k(b + 144 * k, out.data() + 256 * k); break;
    case 14: for (size_t k = 0; k < n / 256; k++) dq_q6k(b + 210 * k, out.data() + 256 * k); break;
  }
  return kOk;
}

int gguf_open_file(const char* path, std::unique_ptr<Gguf>& out) {
  const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return fail(kErrInvalid, std::string("cannot open '") + path + "': " + std::strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0) {
    ::close(fd);
    return fail(kErrInvalid, std::string("cannot stat '") + path + "'");
  }
  auto g = std::make_unique<Gguf>();
  if (st.st_size > 0) {
    void* m = mmap(nullptr, static_cast<size_t>(st.st_size), PROT_READ, MAP_PRIVATE, fd, 0);
    if (m == MAP_FAILED) {
      ::close(fd);
      return fail(kErrInvalid, std::string("cannot map '") + path + "'");
    }
    g->map = m;
    g->base = static_cast<const uint8_t*>(m);
    g->size = static_cast<size_t>(st.st_size);
  }
  ::close(fd);
  if (int rc = g->parse()) return rc;
  out = std::move(g);
  return kOk;
}

int gguf_open_bytes(const void* data, size_t n, std::unique_ptr<Gguf>& out) {
  auto g = std::make_unique<Gguf>();
  if (n) g->owned.assign(static_cast<const uint8_t*>(data), static_cast<const uint8_t*>(data) + n);
  g->base = g->owned.data();
  g->size = n;
  if (int rc = g->parse()) return rc;
  out = std::move(g);
  return kOk;
}

// The configuration load (gguf.rs:338-378, 410-425) derives from the file:
// required {arch}.* keys, the optional ones with the reference's defaults,
// the vocabulary from the tokenizer's token list, and the architecture knobs
// (NeoX RoPE for qwen2 / gemma, gelu_tanh and a sqrt(dim) embedding scale for
// gemma).
int gguf_model_config(const Gguf& g, prana_config* out) {
  const GValue* av = g.find("general.architecture");
  if (!av || av->type != 8) return fail(kErrInvalid, "missing general.architecture");
  const std::string& arch = av->s;
  if (arch != "llama" && arch != "qwen2" && arch != "gemma")
    return fail(kErrUnsupported, "unsupported architecture '" + arch + "' (llama, qwen2, gemma)");
  const bool gemma = arch == "gemma";
  auto get = [&](const char* suffix, size_t* v) -> bool {
    const GValue* e = g.find(arch + "." + suffix);
    uint64_t u;
    if (!e || !gvalue_as_u64(*e, &u)) return false;
    *v = static_cast<size_t>(u);
    return true;
  };
  auto req = [&](const char* suffix, size_t* v) -> int {
    return get(suffix, v) ? kOk : fail(kErrInvalid, "missing metadata '" + arch + "." + suffix + "'");
  };
  prana_config c{};
  if (int rc = req("embedding_length", &c.dim)) return rc;
  if (int rc = req("block_count", &c.n_layers)) return rc;
  if (int rc = req("attention.head_count", &c.n_heads)) return rc;
  if (!get("attention.head_count_kv", &c.n_kv_heads)) c.n_kv_heads = c.n_heads;
  if (int rc = req("feed_forward_length", &c.hidden_dim)) return rc;
  if (int rc = req("context_length", &c.seq_len)) return rc;
  float f;
  const GValue* e;
  c.rope_theta = (e = g.find(arch + ".rope.freq_base")) && gvalue_as_f32(*e, &f) ? f : 10000.0f;
  PRANA_CHECK(c.n_heads > 0, "metadata: attention.head_count is 0");
  if (!get("attention.key_length", &c.head_dim)) c.head_dim = c.dim / c.n_heads;
  c.norm_eps = (e = g.find(arch + ".attention.layer_norm_rms_epsilon")) && gvalue_as_f32(*e, &f) ? f : 1e-5f;
  const GValue* tok = g.find("tokenizer.ggml.tokens");
  if (!tok || tok->type != 9) return fail(kErrInvalid, "missing tokenizer.ggml.tokens");
  c.vocab_size = tok->arr.size();
  c.rope_neox = arch != "llama";
  c.act = gemma ? 1 : 0;
  c.emb_scale = gemma ? std::sqrt(static_cast<float>(c.dim)) : 1.0f;
  *out = c;
  return kOk;
}

namespace {

// Gguf::linear (gguf.rs:271-305): Q8_0 / Q4_0 (cols % 32 == 0) and Q4_K /
// Q6_K (cols % 256 == 0) stay packed; anything else is decoded to f32 and
// becomes a Q8 QuantMatrix at precision Q8 when cols % 32 == 0 (Linear::new,
// checkpoint.rs:85-91), else dense rows.
int load_linear(const Gguf& g, Model& m, const std::string& name, int precision) {
  const GTensor* t;
  const uint8_t* b;
  size_t nb;
  if (int rc = g.raw(name, &t, &b, &nb)) return rc;
  if (t->dims.size() != 2) return fail(kErrInvalid, "tensor '" + name + "' is not 2-D");
  const uint64_t cols = t->dims[0], rows = t->dims[1];
  const bool packed =
      ((t->type == 8 || t->type == 2) && cols % 32 == 0) || ((t->type == 12 || t->type == 14) && cols % 256 == 0);
  if (packed) return m.set_tensor(name, static_cast<int>(t->type), t->dims.data(), 2, b, nb);
  std::vector<float> f;
  if (int rc = g.tensor_f32(name, f)) return rc;
  if (precision == 1 && cols % 32 == 0) {
    size_t want_c = 0, want_r = 0;
    if (!m.mat_slot(name, &want_c, &want_r)) return fail(kErrInvalid, "unknown tensor '" + name + "'");
    if (want_c != cols || want_r != rows)
      return fail(kErrInvalid, "tensor '" + name + "': expected shape [" + std::to_string(want_c) + ", " +
                                   std::to_string(want_r) + "]");
    std::vector<int8_t> q;
    std::vector<float> sc;
    quantize_q8_host(rows, cols, f.data(), q, sc);
    return m.set_q8(name, rows, cols, q.data(), sc.data());
  }
  return m.set_tensor(name, 0, t->dims.data(), 2, f.data(), f.size() * 4);
}

}  // namespace

// load (gguf.rs:338-437) onto a model created with gguf_model_config's
// configuration. Norm weights and biases are read as f32 (tensor_f32);
// gemma stores norm weights as (w - 1) and computes rmsnorm(x) * (1 + w), so
// the +1 is folded in here (gguf.rs:383-396).
int gguf_load_model(const Gguf& g, int precision, Model& m) {
  PRANA_CHECK(precision == 0 || precision == 1, "precision must be 0 (F32) or 1 (Q8)");
  const prana_config& c = m.c;
  const GValue* av = g.find("general.architecture");
  const bool gemma = av && av->type == 8 && av->s == "gemma";

  // Gguf::embedding (gguf.rs:309-326): Q4_0 / Q4_K / Q6_K tables with
  // block-aligned rows stay packed, anything else becomes a dense f32 table.
  const GTensor* et;
  const uint8_t* eb;
  size_t enb;
  if (int rc = g.raw("token_embd.weight", &et, &eb, &enb)) return rc;
  uint64_t en;
  checked_elems(et->dims, &en);
  if (en != static_cast<uint64_t>(c.vocab_size) * c.dim)
    return fail(kErrInvalid, "token_embd.weight size mismatch with vocab");
  const bool two_d = et->dims.size() == 2;
  const uint64_t cols = two_d ? et->dims[0] : 0;
  const bool emb_packed = two_d && ((et->type == 2 && cols % 32 == 0) || ((et->type == 12 || et->type == 14) && cols % 256 == 0));
  PRANA_CHECK(!emb_packed || cols == c.dim, "token_embd.weight: packed rows must be dim wide");
  // A dense table is read as vocab rows of dim values whatever its stated shape.
  const uint64_t dims[2] = {c.dim, c.vocab_size};
  std::vector<float> table;
  if (emb_packed) {
    if (int rc = m.set_tensor("token_embd.weight", static_cast<int>(et->type), dims, 2, eb, enb)) return rc;
  } else {
    if (int rc = g.tensor_f32("token_embd.weight", table)) return rc;
    if (int rc = m.set_tensor("token_embd.weight", 0, dims, 2, table.data(), table.size() * 4)) return rc;
  }

  auto put_vec = [&](const std::string& name, bool fold_one) -> int {
    std::vector<float> x;
    if (int rc = g.tensor_f32(name, x)) return rc;
    if (fold_one)
      for (float& v : x) v += 1.0f;
    const uint64_t d = x.size();
    return m.set_tensor(name, 0, &d, 1, x.data(), x.size() * 4);
  };
  for (size_t l = 0; l < c.n_layers; l++) {
    const std::string p = "blk." + std::to_string(l) + ".";
    if (int rc = put_vec(p + "attn_norm.weight", gemma)) return rc;
    for (const char* w : {"attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_output.weight"})
      if (int rc = load_linear(g, m, p + w, precision)) return rc;
    for (const char* b : {"attn_q.bias", "attn_k.bias", "attn_v.bias"})
      if (g.tensors.count(p + b))
        if (int rc = put_vec(p + b, false)) return rc;
    if (int rc = put_vec(p + "ffn_norm.weight", gemma)) return rc;
    for (const char* w : {"ffn_gate.weight", "ffn_down.weight", "ffn_up.weight"})
      if (int rc = load_linear(g, m, p + w, precision)) return rc;
  }
  if (int rc = put_vec("output_norm.weight", gemma)) return rc;

  // Tied classifier (gguf.rs:426-437): a dense table at precision Q8 gets a
  // quantized copy; otherwise the head reads the table itself.
  if (g.tensors.count("output.weight")) {
    if (int rc = load_linear(g, m, "output.weight", precision)) return rc;
  } else if (!emb_packed && precision == 1 && c.dim % 32 == 0) {
    std::vector<int8_t> q;
    std::vector<float> sc;
    quantize_q8_host(c.vocab_size, c.dim, table.data(), q, sc);
    if (int rc = m.set_q8("output.weight", c.vocab_size, c.dim, q.data(), sc.data())) return rc;
  }
  return m.finalize();
}

}  // namespace prana
