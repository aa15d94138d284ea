// extern "C" entry points of libprana_hip (declared in include/prana_hip.h).
// Nothing throws across this boundary: every entry point catches and turns
// failures into status codes with a thread-local message.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <vector>
#include <new>
#include <string>

#include "gguf.h"
#include "graph.h"
#include "model.h"
#include "tokenizer.h"

namespace prana {
const char* last_error_cstr();
}

using namespace prana;

namespace {

// Library-owned scratch for the kernel-level entry points that need
// intermediate buffers (quantized activations, attention scores).
struct Scratch {
  std::mutex mu;
  DevBuf qa, sa, sums, att, flash;
};
Scratch& scratch() {
  static Scratch s;
  return s;
}

template <class F>
int guard(F&& f) {
  try {
    return f();
  } catch (const std::bad_alloc&) {
    return fail(kErrNoMem, "host allocation failed");
  } catch (const std::exception& e) {
    return fail(kErrInvalid, std::string("internal error: ") + e.what());
  } catch (...) {
    return fail(kErrInvalid, "internal error");
  }
}

// Caller-sized string output: *len = bytes needed (no NUL); the copy, NUL
// terminated, happens when buf holds len + 1 bytes, else PRANA_ERR_SHORT_BUFFER
// and the caller grows buf and calls again.
int copy_out(const std::string& s, char* buf, size_t cap, size_t* len) {
  *len = s.size();
  if (!buf || cap < s.size() + 1)
    return fail(kErrShortBuffer, "buffer of " + std::to_string(cap) + " bytes; " + std::to_string(s.size() + 1) +
                                     " needed");
  std::memcpy(buf, s.data(), s.size());
  buf[s.size()] = '\0';
  return kOk;
}

#define INIT_OR_RETURN()          \
  do {                            \
    int rc_ = ensure_init();      \
    if (rc_) return rc_;          \
  } while (0)

}  // namespace

extern "C" {

const char* prana_last_error(void) { return last_error_cstr(); }

int prana_init(int device) {
  return guard([&] {
    INIT_OR_RETURN();
    if (device != 0) return fail(kErrUnsupported, "only device 0 is driven by this build (one GPU per process)");
    return static_cast<int>(kOk);
  });
}

int prana_device_alloc(size_t bytes, void** out) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(out, "null out pointer");
    *out = nullptr;
    if (bytes == 0) return static_cast<int>(kOk);
    PRANA_HIP(hipMalloc(out, bytes));
    return static_cast<int>(kOk);
  });
}

int prana_device_free(void* p) {
  return guard([&] {
    if (p) PRANA_HIP(hipFree(p));
    return static_cast<int>(kOk);
  });
}

int prana_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  return guard([&] {
    INIT_OR_RETURN();
    if (bytes) PRANA_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return static_cast<int>(kOk);
  });
}

int prana_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_HIP(hipStreamSynchronize(ctx().stream));
    if (bytes) PRANA_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return static_cast<int>(kOk);
  });
}

int prana_memcpy_d2d(void* dst, const void* src, size_t bytes) {
  return guard([&] {
    INIT_OR_RETURN();
    if (bytes) PRANA_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx().stream));
    PRANA_HIP(hipStreamSynchronize(ctx().stream));
    return static_cast<int>(kOk);
  });
}

int prana_memset_d(void* dst, int value, size_t bytes) {
  return guard([&] {
    INIT_OR_RETURN();
    if (bytes) PRANA_HIP(hipMemsetAsync(dst, value, bytes, ctx().stream));
    return static_cast<int>(kOk);
  });
}

int prana_synchronize(void) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_HIP(hipStreamSynchronize(ctx().stream));
    PRANA_HIP(hipDeviceSynchronize());
    return static_cast<int>(kOk);
  });
}

// ------------------------------------------------------------------ matrices
int prana_mat_create(int ggml_type, size_t rows, size_t cols, const void* host_bytes, size_t nbytes,
                     prana_mat_t* out) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(out && (host_bytes || rows * cols == 0), "null argument");
    auto* m = new prana_mat();
    int rc = mat_from_ggml(ggml_type, rows, cols, host_bytes, nbytes, m->m);
    if (rc) {
      delete m;
      return rc;
    }
    *out = m;
    return static_cast<int>(kOk);
  });
}

int prana_mat_create_q8(size_t rows, size_t cols, const int8_t* q, const float* scales, prana_mat_t* out) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(out && q && scales, "null argument");
    auto* m = new prana_mat();
    int rc = mat_from_q8_parts(rows, cols, q, scales, m->m);
    if (rc) {
      delete m;
      return rc;
    }
    *out = m;
    return static_cast<int>(kOk);
  });
}

int prana_mat_destroy(prana_mat_t m) {
  return guard([&] {
    delete m;
    return static_cast<int>(kOk);
  });
}

int prana_mat_info(prana_mat_t m, size_t* rows, size_t* cols, int* kind, size_t* stream_bytes) {
  return guard([&] {
    PRANA_CHECK(m, "null matrix");
    if (rows) *rows = m->m.d.rows;
    if (cols) *cols = m->m.d.cols;
    if (kind) *kind = m->m.d.kind;
    if (stream_bytes) *stream_bytes = m->m.stream_bytes;
    return static_cast<int>(kOk);
  });
}

// ------------------------------------------------------------------ kernels
int prana_quantize_acts(const float* x, size_t n_rows, size_t k, int8_t* q, float* scales, int32_t* sums,
                        prana_stream_t stream) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(k % 32 == 0, "quantize_acts: k must be a multiple of 32 (matmul.rs:106)");
    return launch_quantize_acts(x, n_rows, k, q, scales, sums, pick_stream(stream));
  });
}

int prana_quantize_q8(const float* w, size_t rows, size_t cols, int8_t* q, float* scales, prana_stream_t stream) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(w && q && scales, "quantize_q8: null argument");
    PRANA_CHECK(cols % 32 == 0, "quantize_q8: cols must be a multiple of 32 (matmul.rs:63)");
    // the same per-block arithmetic as quantize_acts (matmul.rs:67-80 and 108-121), without the sums
    return launch_quantize_acts(w, rows, cols, q, scales, nullptr, pick_stream(stream));
  });
}

int prana_matmul(prana_mat_t w, const float* x, size_t n_tokens, float* out, prana_stream_t stream) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(w, "null matrix");
    const DevMat& d = w->m.d;
    hipStream_t s = pick_stream(stream);
    GemvOut o{out, d.rows, nullptr, 0};
    if (d.kind == kKindF32) return launch_gemv(d, x, nullptr, nullptr, nullptr, n_tokens, o, s);
    Scratch& sc = scratch();
    std::lock_guard<std::mutex> lk(sc.mu);
    size_t n = n_tokens * d.cols;
    int rc;
    if ((rc = sc.qa.ensure(n)) || (rc = sc.sa.ensure(n / 32 * 4)) || (rc = sc.sums.ensure(n / 32 * 4))) return rc;
    if ((rc = launch_quantize_acts(x, n_tokens, d.cols, sc.qa.as<int8_t>(), sc.sa.as<float>(), sc.sums.as<int>(),
                                   s)))
      return rc;
    rc = launch_gemv(d, x, sc.qa.as<int8_t>(), sc.sa.as<float>(), sc.sums.as<int>(), n_tokens, o, s);
    if (rc) return rc;
    // The scratch is shared: finish before another call may reuse it.
    PRANA_HIP(hipStreamSynchronize(s));
    return static_cast<int>(kOk);
  });
}

int prana_matmul_prefill(prana_mat_t w, const float* x, const int8_t* q, const float* scales, const int32_t* sums,
                         size_t n_tokens, float* out, prana_stream_t stream) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(w, "null matrix");
    const DevMat& d = w->m.d;
    GemvOut o{out, d.rows, nullptr, 0};
    return launch_gemv(d, x, q, scales, sums, n_tokens, o, pick_stream(stream));
  });
}

int prana_matmul_block_sums(prana_mat_t w, const int8_t* q, const int32_t* sums, size_t n_tokens, int32_t* isums,
                            prana_stream_t stream) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(w, "null matrix");
    return launch_block_isums(w->m.d, q, sums, n_tokens, isums, pick_stream(stream));
  });
}

int prana_embed_rows(prana_mat_t table, const uint32_t* tokens, size_t n, float scale, float* out,
                     prana_stream_t stream) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(table, "null table");
    return launch_embed(table->m.d, tokens, n, scale, out, pick_stream(stream));
  });
}

int prana_rmsnorm(const float* x, const float* w, size_t rows, size_t dim, float eps, float* out,
                  prana_stream_t stream) {
  return guard([&] {
    INIT_OR_RETURN();
    return launch_rmsnorm(x, w, rows, dim, eps, out, nullptr, nullptr, nullptr, pick_stream(stream));
  });
}

int prana_silu(float* x, size_t n, prana_stream_t stream) {
  return guard([&] {
    INIT_OR_RETURN();
    return launch_act_mul(x, nullptr, n, 0, nullptr, nullptr, nullptr, pick_stream(stream));
  });
}

int prana_gelu_tanh(float* x, size_t n, prana_stream_t stream) {
  return guard([&] {
    INIT_OR_RETURN();
    return launch_act_mul(x, nullptr, n, 1, nullptr, nullptr, nullptr, pick_stream(stream));
  });
}

int prana_silu_mul(float* g, const float* u, size_t n, prana_stream_t stream) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(g && u, "silu_mul: null buffer");
    return launch_act_mul(g, u, n, 0, nullptr, nullptr, nullptr, pick_stream(stream));
  });
}

int prana_gelu_tanh_mul(float* g, const float* u, size_t n, prana_stream_t stream) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(g && u, "gelu_tanh_mul: null buffer");
    return launch_act_mul(g, u, n, 1, nullptr, nullptr, nullptr, pick_stream(stream));
  });
}

int prana_add_bias(float* x, const float* bias, size_t rows, size_t n, prana_stream_t stream) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(x && bias && n > 0, "add_bias: null buffer or empty row");
    return launch_add(x, bias, rows * n, n, pick_stream(stream));
  });
}

int prana_softmax(const float* in, size_t rows, size_t n, float* out, prana_stream_t stream) {
  return guard([&] {
    INIT_OR_RETURN();
    return launch_softmax(in, rows, n, out, pick_stream(stream));
  });
}

namespace {
int rope_entry(float* x, size_t n_rows, size_t row_len, size_t pos0, size_t hd, float theta, int neox, void* stream) {
  INIT_OR_RETURN();
  PRANA_CHECK(hd % 2 == 0 && hd > 0, "RoPE: head_dim must be even (attention.rs:91)");
  PRANA_CHECK(row_len % hd == 0, "RoPE: row must be a whole number of heads (attention.rs:92)");
  size_t half = hd / 2, npos = pos0 + n_rows;
  std::vector<float> tab(npos * half * 2);
  for (size_t m = 0; m < half; m++) {
    float freq = std::pow(theta, -(2.0f * static_cast<float>(m)) / static_cast<float>(hd));
    for (size_t p = pos0; p < npos; p++) {
      float ang = static_cast<float>(p) * freq;
      tab[(p * half + m) * 2] = std::cos(ang);
      tab[(p * half + m) * 2 + 1] = std::sin(ang);
    }
  }
  hipStream_t s = pick_stream(stream);
  DevBuf t;
  int rc = t.alloc(tab.size() * 4);
  if (rc) return rc;
  PRANA_HIP(hipMemcpyAsync(t.p, tab.data(), tab.size() * 4, hipMemcpyHostToDevice, s));
  rc = launch_rope(x, n_rows, row_len, row_len, hd, t.as<float2>(), pos0, neox, s);
  if (rc) return rc;
  PRANA_HIP(hipStreamSynchronize(s));  // the table dies with this scope
  return static_cast<int>(kOk);
}
}  // namespace

int prana_rope_interleaved(float* x, size_t n_rows, size_t row_len, size_t pos0, size_t head_dim, float theta,
                           prana_stream_t stream) {
  return guard([&] { return rope_entry(x, n_rows, row_len, pos0, head_dim, theta, 0, stream); });
}

int prana_rope_neox(float* x, size_t n_rows, size_t row_len, size_t pos0, size_t head_dim, float theta,
                    prana_stream_t stream) {
  return guard([&] { return rope_entry(x, n_rows, row_len, pos0, head_dim, theta, 1, stream); });
}

int prana_kv_write_f16(uint16_t* cache, size_t first_row, size_t kv_stride, const float* src, size_t n,
                       prana_stream_t stream) {
  return guard([&] {
    INIT_OR_RETURN();
    return launch_kv_write(cache, first_row, kv_stride, src, n, pick_stream(stream));
  });
}

namespace {
int attn_entry(const float* q, const uint16_t* kc, const uint16_t* vc, size_t pos0, size_t seq, size_t nh, size_t nkv,
               size_t hd, float* out, void* stream) {
  INIT_OR_RETURN();
  Scratch& sc = scratch();
  std::lock_guard<std::mutex> lk(sc.mu);
  size_t cap = pos0 + seq;
  const size_t need = attention_scratch_floats(seq, nh, cap);
  int rc = sc.att.ensure(need * 4);
  if (rc) return rc;
  hipStream_t s = pick_stream(stream);
  rc = launch_attention_cache(q, kc, vc, pos0, seq, nh, nkv, hd, out, need ? sc.att.as<float>() : nullptr, cap,
                              nullptr, s);
  if (rc) return rc;
  PRANA_HIP(hipStreamSynchronize(s));
  return static_cast<int>(kOk);
}
}  // namespace

int prana_attention_decode(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, size_t pos,
                           size_t n_heads, size_t n_kv_heads, size_t head_dim, float* out, prana_stream_t stream) {
  return guard([&] { return attn_entry(q, k_cache, v_cache, pos, 1, n_heads, n_kv_heads, head_dim, out, stream); });
}

int prana_attention_verify(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, size_t pos0,
                           size_t seq, size_t n_heads, size_t n_kv_heads, size_t head_dim, float* out,
                           prana_stream_t stream) {
  return guard(
      [&] { return attn_entry(q, k_cache, v_cache, pos0, seq, n_heads, n_kv_heads, head_dim, out, stream); });
}

int prana_attention_decode_splitk(const float* q, const uint16_t* const* k_caches, const uint16_t* const* v_caches,
                                  const size_t* pos, size_t n_seq, size_t n_heads, size_t n_kv_heads, size_t head_dim,
                                  float* out, prana_stream_t stream) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(pos && n_seq >= 1 && n_seq <= 16, "attention_decode_splitk: 1..16 sequences");
    PRANA_CHECK(n_kv_heads > 0 && n_heads % n_kv_heads == 0,
                "attention_decode_splitk: n_heads must be a multiple of n_kv_heads");
    Scratch& sc = scratch();
    std::lock_guard<std::mutex> lk(sc.mu);
    const FlashPlan plan = flash_decode_plan(pos, n_seq, n_heads, n_kv_heads, head_dim);
    int rc = sc.flash.ensure(std::max<size_t>(plan.scratch_floats, 1) * 4);
    if (rc) return rc;
    hipStream_t s = pick_stream(stream);
    rc = launch_flash_decode(q, k_caches, v_caches, pos, n_seq, n_heads, n_kv_heads, head_dim, out,
                             sc.flash.as<float>(), sc.flash.bytes / 4, s);
    if (rc) return rc;
    PRANA_HIP(hipStreamSynchronize(s));
    return static_cast<int>(kOk);
  });
}

int prana_attention_decode_splitk_noalloc(const float* q, const uint16_t* const* k_caches,
                                          const uint16_t* const* v_caches, const size_t* pos, size_t n_seq,
                                          size_t n_heads, size_t n_kv_heads, size_t head_dim, float* out,
                                          prana_stream_t stream) {
  return guard([&] {
    if (int rc = require_init()) return rc;
    PRANA_CHECK(pos && n_seq >= 1 && n_seq <= 16, "attention_decode_splitk_noalloc: 1..16 sequences");
    PRANA_CHECK(n_kv_heads > 0 && n_heads % n_kv_heads == 0,
                "attention_decode_splitk_noalloc: n_heads must be a multiple of n_kv_heads");
    float* sc = flash_noalloc_scratch(ctx().device);
    PRANA_CHECK(sc, "attention_decode_splitk_noalloc: scratch array address unknown");
    const FlashPlan plan = flash_decode_plan(pos, n_seq, n_heads, n_kv_heads, head_dim);
    if (plan.scratch_floats > kFlashNoAllocFloats)
      return fail(kErrInvalid, "attention_decode_splitk_noalloc: the call needs " +
                                   std::to_string(plan.scratch_floats) + " scratch floats, above the fixed " +
                                   std::to_string(kFlashNoAllocFloats) +
                                   " (fewer sequences or shorter windows, or prana_attention_decode_splitk)");
    return launch_flash_decode(q, k_caches, v_caches, pos, n_seq, n_heads, n_kv_heads, head_dim, out, sc,
                               kFlashNoAllocFloats, pick_stream(stream));
  });
}

int prana_attention_prefill(const float* q, const float* k, const float* v, size_t seq, size_t n_heads,
                            size_t n_kv_heads, size_t head_dim, float* out, prana_stream_t stream) {
  return guard([&] {
    INIT_OR_RETURN();
    Scratch& sc = scratch();
    std::lock_guard<std::mutex> lk(sc.mu);
    const size_t need = attention_scratch_floats(seq, n_heads, seq, false);
    int rc = sc.att.ensure(need * 4);
    if (rc) return rc;
    hipStream_t s = pick_stream(stream);
    rc = launch_attention_prefill(q, k, v, seq, n_heads, n_kv_heads, head_dim, out,
                                  need ? sc.att.as<float>() : nullptr, s);
    if (rc) return rc;
    PRANA_HIP(hipStreamSynchronize(s));
    return static_cast<int>(kOk);
  });
}

int prana_argmax(const float* logits, size_t rows, size_t n, uint32_t* out_idx, prana_stream_t stream) {
  return guard([&] {
    INIT_OR_RETURN();
    return launch_argmax(logits, rows, n, out_idx, pick_stream(stream));
  });
}

int prana_f32_to_f16(const float* in, size_t n, uint16_t* out, prana_stream_t stream) {
  return guard([&] {
    INIT_OR_RETURN();
    return launch_f32_to_f16(in, n, out, pick_stream(stream));
  });
}

int prana_f16_to_f32(const uint16_t* in, size_t n, float* out, prana_stream_t stream) {
  return guard([&] {
    INIT_OR_RETURN();
    return launch_f16_to_f32(in, n, out, pick_stream(stream));
  });
}

int prana_expf(const float* in, size_t n, float* out, prana_stream_t stream) {
  return guard([&] {
    INIT_OR_RETURN();
    return launch_expf(in, n, out, pick_stream(stream));
  });
}

int prana_tanhf(const float* in, size_t n, float* out, prana_stream_t stream) {
  return guard([&] {
    INIT_OR_RETURN();
    return launch_tanhf(in, n, out, pick_stream(stream));
  });
}

// ------------------------------------------------------------------ model
int prana_model_create(const prana_config* cfg, prana_model_t* out) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(cfg && out, "null argument");
    const prana_config& c = *cfg;
    if (int rc = check_config(c)) return rc;
    auto* m = new prana_model();
    m->m.c = c;
    m->m.layers.resize(c.n_layers);
    *out = m;
    return static_cast<int>(kOk);
  });
}

int prana_model_destroy(prana_model_t m) {
  return guard([&] {
    delete m;
    return static_cast<int>(kOk);
  });
}

int prana_model_set_tensor(prana_model_t m, const char* name, int ggml_type, const uint64_t* dims, int n_dims,
                           const void* bytes, size_t nbytes) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(m && name && dims && bytes, "null argument");
    PRANA_CHECK(n_dims == 1 || n_dims == 2, "tensor must be 1-D or 2-D");
    m->m.finalized = false;
    return m->m.set_tensor(name, ggml_type, dims, n_dims, bytes, nbytes);
  });
}

int prana_model_finalize(prana_model_t m) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(m, "null model");
    return m->m.finalize();
  });
}

int prana_model_stream_bytes(prana_model_t m, size_t* bytes) {
  return guard([&] {
    PRANA_CHECK(m && bytes && m->m.finalized, "model not finalized");
    *bytes = m->m.stream_bytes();
    return static_cast<int>(kOk);
  });
}

int prana_cache_create(prana_model_t m, size_t positions, prana_cache_t* out) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(m && out, "null argument");
    auto* c = new prana_cache();
    c->owner = m;
    int rc = c->c.create(m->m, positions);
    if (rc) {
      delete c;
      return rc;
    }
    *out = c;
    return static_cast<int>(kOk);
  });
}

int prana_cache_destroy(prana_cache_t c) {
  return guard([&] {
    delete c;
    return static_cast<int>(kOk);
  });
}

int prana_cache_read(prana_cache_t c, size_t layer, int which, size_t rows, uint16_t* host_out) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(c && host_out, "null argument");
    PRANA_CHECK(layer < c->c.n_layers && rows <= c->c.len, "cache_read: out of range");
    PRANA_HIP(hipStreamSynchronize(ctx().stream));
    const uint16_t* src = which ? c->c.v(layer) : c->c.k(layer);
    const size_t kv_dim = c->c.kv_dim, kcap = c->c.kcap;
    if (which || kcap == 0 || rows == 0) {
      PRANA_HIP(hipMemcpy(host_out, src, rows * kv_dim * 2, hipMemcpyDeviceToHost));
    } else {  // K in 8-dim pieces (kcache_index): back to rows, one column of pieces at a time
      for (size_t g = 0; g < kv_dim / 8; g++)
        PRANA_HIP(hipMemcpy2D(host_out + g * 8, kv_dim * 2, src + g * kcap * 8, 16, 16, rows, hipMemcpyDeviceToHost));
    }
    return static_cast<int>(kOk);
  });
}

int prana_forward(prana_model_t m, prana_cache_t c, uint32_t token, size_t pos, int need_logits, float* logits_host) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(m && c && c->owner == m, "cache does not belong to this model");
    return m->m.forward(c->c, token, pos, need_logits != 0, logits_host);
  });
}

int prana_prefill(prana_model_t m, prana_cache_t c, const uint32_t* tokens, size_t n) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(m && c && c->owner == m && (tokens || n == 0), "bad argument");
    return m->m.prefill(c->c, tokens, n);
  });
}

int prana_forward_batch(prana_model_t m, prana_cache_t c, const uint32_t* tokens, size_t n, size_t pos0,
                        float* logits_host) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(m && c && c->owner == m && tokens, "bad argument");
    return m->m.forward_batch(c->c, tokens, n, pos0, logits_host);
  });
}

int prana_decode(prana_model_t m, prana_cache_t c, uint32_t token, size_t pos, size_t n_steps, uint32_t* out) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(m && c && c->owner == m, "cache does not belong to this model");
    PRANA_CHECK(token < m->m.c.vocab_size, "token id out of vocabulary");
    return m->m.decode(c->c, token, pos, n_steps, out);
  });
}

int prana_decode_replay_enabled(void) { return prana::decode_graphs_enabled() ? 1 : 0; }

int prana_gemv_profile(int on) {
  return guard([&] {
    INIT_OR_RETURN();
    GemvProfile& gp = gemv_profile();
    int rc = gp.collect();
    gp.on = on > 0;
    gp.period = on > 0 ? static_cast<size_t>(on) : 1;
    gp.calls = 0;
    return rc;
  });
}

int prana_gemv_profile_read(size_t* launches, double* seconds, double* bytes, int reset) {
  return guard([&] {
    INIT_OR_RETURN();
    GemvProfile& gp = gemv_profile();
    int rc = gp.collect();
    if (rc) return rc;
    if (launches) *launches = gp.launches;
    if (seconds) *seconds = gp.seconds;
    if (bytes) *bytes = gp.bytes;
    if (reset) {
      gp.launches = 0;
      gp.seconds = gp.bytes = 0.0;
      gp.shapes.clear();
    }
    return static_cast<int>(kOk);
  });
}

int prana_gemv_profile_shapes(size_t cap, size_t* bytes, size_t* launches, double* seconds, size_t* n_out) {
  return guard([&] {
    INIT_OR_RETURN();
    GemvProfile& gp = gemv_profile();
    int rc = gp.collect();
    if (rc) return rc;
    PRANA_CHECK(n_out && (cap == 0 || (bytes && launches && seconds)), "gemv_profile_shapes: null output");
    size_t i = 0;
    for (const auto& kv : gp.shapes) {
      if (i < cap) {
        bytes[i] = kv.first;
        launches[i] = kv.second.launches;
        seconds[i] = kv.second.seconds;
      }
      i++;
    }
    *n_out = gp.shapes.size();
    return static_cast<int>(kOk);
  });
}

int prana_generate(prana_model_t m, const uint32_t* prompt, size_t p, size_t steps, const uint32_t* stops,
                   size_t n_stops, uint32_t* out, size_t* n_out, prana_gen_stats* stats) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(m && prompt && (out || steps == 0), "bad argument");
    PRANA_CHECK(m->m.finalized, "model not finalized");
    return m->m.generate(prompt, p, steps, stops, n_stops, out, n_out, stats);
  });
}

int prana_generate_speculative(prana_model_t target, prana_model_t draft, const uint32_t* prompt, size_t p,
                               size_t steps, size_t k, const uint32_t* stops, size_t n_stops, uint32_t* out,
                               size_t* n_out, prana_gen_stats* stats) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(target && draft && prompt && (out || steps == 0), "bad argument");
    PRANA_CHECK(target->m.finalized && draft->m.finalized, "model not finalized");
    return generate_speculative(target->m, draft->m, prompt, p, steps, k, stops, n_stops, out, n_out, stats);
  });
}

size_t prana_ggml_nbytes(int ggml_type, size_t n_elems) { return ggml_nbytes(ggml_type, n_elems); }

// ------------------------------------------------------------------ GGUF (host only; no device work)
int prana_gguf_open(const char* path, prana_gguf_t* out) {
  return guard([&] {
    PRANA_CHECK(path && out, "null argument");
    *out = nullptr;
    auto h = std::make_unique<prana_gguf>();
    if (int rc = gguf_open_file(path, h->g)) return rc;
    *out = h.release();
    return static_cast<int>(kOk);
  });
}

int prana_gguf_open_bytes(const void* data, size_t nbytes, prana_gguf_t* out) {
  return guard([&] {
    PRANA_CHECK((data || nbytes == 0) && out, "null argument");
    *out = nullptr;
    auto h = std::make_unique<prana_gguf>();
    if (int rc = gguf_open_bytes(data, nbytes, h->g)) return rc;
    *out = h.release();
    return static_cast<int>(kOk);
  });
}

int prana_gguf_close(prana_gguf_t g) {
  return guard([&] {
    delete g;
    return static_cast<int>(kOk);
  });
}

int prana_gguf_counts(prana_gguf_t g, uint32_t* version, size_t* n_tensors, size_t* n_meta) {
  return guard([&] {
    PRANA_CHECK(g, "null handle");
    if (version) *version = g->g->version;
    if (n_tensors) *n_tensors = g->g->names.size();
    if (n_meta) *n_meta = g->g->meta.size();
    return static_cast<int>(kOk);
  });
}

int prana_gguf_tensor_name(prana_gguf_t g, size_t index, char* buf, size_t cap, size_t* len) {
  return guard([&] {
    PRANA_CHECK(g && len, "null argument");
    PRANA_CHECK(index < g->g->names.size(), "tensor index out of range");
    return copy_out(g->g->names[index], buf, cap, len);
  });
}

int prana_gguf_tensor_info(prana_gguf_t g, const char* name, int* ggml_type, uint64_t* dims, int* n_dims,
                           size_t* nbytes) {
  return guard([&] {
    PRANA_CHECK(g && name, "null argument");
    const GTensor* t;
    const uint8_t* b;
    size_t nb;
    if (int rc = g->g->raw(name, &t, &b, &nb)) return rc;
    if (dims && t->dims.size() > 8)
      return fail(kErrShortBuffer, "tensor '" + std::string(name) + "' has " + std::to_string(t->dims.size()) +
                                       " dimensions; dims holds 8");
    if (ggml_type) *ggml_type = static_cast<int>(t->type);
    if (n_dims) *n_dims = static_cast<int>(t->dims.size());
    if (dims)
      for (size_t i = 0; i < t->dims.size(); i++) dims[i] = t->dims[i];
    if (nbytes) *nbytes = nb;
    return static_cast<int>(kOk);
  });
}

int prana_gguf_tensor_data(prana_gguf_t g, const char* name, const void** bytes, size_t* nbytes) {
  return guard([&] {
    PRANA_CHECK(g && name && bytes && nbytes, "null argument");
    const GTensor* t;
    const uint8_t* b;
    if (int rc = g->g->raw(name, &t, &b, nbytes)) return rc;
    *bytes = b;
    return static_cast<int>(kOk);
  });
}

int prana_gguf_tensor_f32(prana_gguf_t g, const char* name, float* out, size_t cap, size_t* n) {
  return guard([&] {
    PRANA_CHECK(g && name && n, "null argument");
    std::vector<float> v;
    if (int rc = g->g->tensor_f32(name, v)) return rc;
    *n = v.size();
    if (!out || cap < v.size())
      return fail(kErrShortBuffer, "buffer holds " + std::to_string(cap) + " values, tensor has " +
                                       std::to_string(v.size()));
    if (!v.empty()) std::memcpy(out, v.data(), v.size() * 4);
    return static_cast<int>(kOk);
  });
}

int prana_gguf_meta_type(prana_gguf_t g, const char* key, int* type, int* elem_type) {
  return guard([&] {
    PRANA_CHECK(g && key && type, "null argument");
    const GValue* v = g->g->find(key);
    if (!v) return fail(kErrInvalid, std::string("missing metadata '") + key + "'");
    *type = static_cast<int>(v->type);
    if (elem_type) *elem_type = v->type == 9 ? static_cast<int>(v->elem_type) : -1;
    return static_cast<int>(kOk);
  });
}

int prana_gguf_meta_u64(prana_gguf_t g, const char* key, uint64_t* out) {
  return guard([&] {
    PRANA_CHECK(g && key && out, "null argument");
    const GValue* v = g->g->find(key);
    if (!v || !gvalue_as_u64(*v, out)) return fail(kErrInvalid, std::string("missing metadata '") + key + "'");
    return static_cast<int>(kOk);
  });
}

int prana_gguf_meta_f32(prana_gguf_t g, const char* key, float* out) {
  return guard([&] {
    PRANA_CHECK(g && key && out, "null argument");
    const GValue* v = g->g->find(key);
    if (!v || !gvalue_as_f32(*v, out)) return fail(kErrInvalid, std::string("missing metadata '") + key + "'");
    return static_cast<int>(kOk);
  });
}

int prana_gguf_meta_str(prana_gguf_t g, const char* key, char* buf, size_t cap, size_t* len) {
  return guard([&] {
    PRANA_CHECK(g && key && len, "null argument");
    const GValue* v = g->g->find(key);
    if (!v || v->type != 8) return fail(kErrInvalid, std::string("missing metadata '") + key + "'");
    return copy_out(v->s, buf, cap, len);
  });
}

int prana_gguf_meta_array_len(prana_gguf_t g, const char* key, size_t* n) {
  return guard([&] {
    PRANA_CHECK(g && key && n, "null argument");
    const GValue* v = g->g->find(key);
    if (!v || v->type != 9) return fail(kErrInvalid, std::string("missing metadata '") + key + "'");
    *n = v->arr.size();
    return static_cast<int>(kOk);
  });
}

int prana_gguf_meta_array_str(prana_gguf_t g, const char* key, size_t index, char* buf, size_t cap, size_t* len) {
  return guard([&] {
    PRANA_CHECK(g && key && len, "null argument");
    const GValue* v = g->g->find(key);
    if (!v || v->type != 9 || v->elem_type != 8)
      return fail(kErrInvalid, std::string("missing string array '") + key + "'");
    PRANA_CHECK(index < v->arr.size(), "array index out of range");
    return copy_out(v->arr[index].s, buf, cap, len);
  });
}

int prana_gguf_meta_array_f32(prana_gguf_t g, const char* key, float* out, size_t cap, size_t* n) {
  return guard([&] {
    PRANA_CHECK(g && key && n, "null argument");
    const GValue* v = g->g->find(key);
    if (!v || v->type != 9 || (v->elem_type != 6 && v->elem_type != 12))
      return fail(kErrInvalid, std::string("missing float array '") + key + "'");
    *n = v->arr.size();
    if (!out || cap < v->arr.size()) return fail(kErrShortBuffer, "buffer shorter than the array");
    for (size_t i = 0; i < v->arr.size(); i++) gvalue_as_f32(v->arr[i], &out[i]);
    return static_cast<int>(kOk);
  });
}

int prana_gguf_meta_array_i64(prana_gguf_t g, const char* key, int64_t* out, size_t cap, size_t* n) {
  return guard([&] {
    PRANA_CHECK(g && key && n, "null argument");
    const GValue* v = g->g->find(key);
    const uint32_t et = v ? v->elem_type : 0;
    const bool ints = et <= 5 || et == 7 || et == 10 || et == 11;
    if (!v || v->type != 9 || et == 6 || !ints)
      return fail(kErrInvalid, std::string("missing integer array '") + key + "'");
    *n = v->arr.size();
    if (!out || cap < v->arr.size()) return fail(kErrShortBuffer, "buffer shorter than the array");
    for (size_t i = 0; i < v->arr.size(); i++) {
      const GValue& e = v->arr[i];
      out[i] = (et == 1 || et == 3 || et == 5 || et == 11) ? e.i : static_cast<int64_t>(e.u);
    }
    return static_cast<int>(kOk);
  });
}

int prana_gguf_model_config(prana_gguf_t g, prana_config* cfg) {
  return guard([&] {
    PRANA_CHECK(g && cfg, "null argument");
    return gguf_model_config(*g->g, cfg);
  });
}

int prana_model_load_gguf(prana_gguf_t g, int precision, prana_model_t* out) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(g && out, "null argument");
    *out = nullptr;
    prana_config c{};
    if (int rc = gguf_model_config(*g->g, &c)) return rc;
    if (int rc = check_config(c)) return rc;
    auto m = std::make_unique<prana_model>();
    m->m.c = c;
    m->m.layers.resize(c.n_layers);
    if (int rc = gguf_load_model(*g->g, precision, m->m)) return rc;
    *out = m.release();
    return static_cast<int>(kOk);
  });
}

// ------------------------------------------------------------------ sampler
}  // extern "C"

struct prana_sampler {
  float temp = 0.0f;
  uint64_t state = 1;
  DevBuf work;  // scaled logits, probabilities, the token
};

extern "C" {

int prana_sampler_create(float temp, uint64_t seed, prana_sampler_t* out) {
  return guard([&] {
    PRANA_CHECK(out, "null argument");
    auto* h = new prana_sampler();
    h->temp = temp;
    h->state = xorshift_seed(seed);
    *out = h;
    return static_cast<int>(kOk);
  });
}

int prana_sampler_destroy(prana_sampler_t h) {
  return guard([&] {
    delete h;
    return static_cast<int>(kOk);
  });
}

int prana_sampler_state(prana_sampler_t h, uint64_t* state) {
  return guard([&] {
    PRANA_CHECK(h && state, "null argument");
    *state = h->state;
    return static_cast<int>(kOk);
  });
}

int prana_sampler_next_f32(prana_sampler_t h, float* out) {
  return guard([&] {
    PRANA_CHECK(h && out, "null argument");
    *out = xorshift_next_f32(&h->state);
    return static_cast<int>(kOk);
  });
}

int prana_sampler_sample(prana_sampler_t h, const float* logits, size_t n, uint32_t* token, prana_stream_t stream) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(h && logits && token && n > 0, "bad argument");
    hipStream_t s = pick_stream(stream);
    if (int rc = h->work.ensure((2 * n + 1) * 4)) return rc;
    float* scaled = h->work.as<float>();
    uint32_t* dtok = reinterpret_cast<uint32_t*>(scaled + 2 * n);
    const float r = h->temp <= 0.0f ? 0.0f : xorshift_next_f32(&h->state);
    if (int rc = launch_sample(logits, n, h->temp, nullptr, 0, r, scaled, scaled + n, dtok, s)) return rc;
    PRANA_HIP(hipMemcpyAsync(token, dtok, 4, hipMemcpyDeviceToHost, s));
    PRANA_HIP(hipStreamSynchronize(s));
    return static_cast<int>(kOk);
  });
}

int prana_sample_pick(const float* probs, size_t n, float r, uint32_t* out, prana_stream_t stream) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(probs && out, "null argument");
    return launch_sample_pick(probs, n, nullptr, 0, r, out, pick_stream(stream));
  });
}

int prana_generate_sampled(prana_model_t m, const uint32_t* prompt, size_t p, size_t steps, const uint32_t* stops,
                           size_t n_stops, prana_sampler_t sampler, uint32_t* out, size_t* n_out,
                           prana_gen_stats* stats) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(m && prompt && sampler && (out || steps == 0), "bad argument");
    PRANA_CHECK(m->m.finalized, "model not finalized");
    return m->m.generate_sampled(prompt, p, steps, stops, n_stops, sampler->temp, &sampler->state, out, n_out, stats);
  });
}

// ------------------------------------------------------------------ tokenizers (host only)
int prana_tokenizer_from_gguf(prana_gguf_t g, prana_tokenizer_t* out) {
  return guard([&] {
    PRANA_CHECK(g && out, "null argument");
    *out = nullptr;
    auto h = std::make_unique<prana_tokenizer>();
    if (int rc = tokenizer_from_gguf(*g->g, h->t)) return rc;
    *out = h.release();
    return static_cast<int>(kOk);
  });
}

int prana_tokenizer_from_llama2c(const void* data, size_t nbytes, size_t vocab_size, prana_tokenizer_t* out) {
  return guard([&] {
    PRANA_CHECK((data || nbytes == 0) && out, "null argument");
    *out = nullptr;
    auto h = std::make_unique<prana_tokenizer>();
    if (int rc = tokenizer_from_llama2c(static_cast<const uint8_t*>(data), nbytes, vocab_size, h->t)) return rc;
    *out = h.release();
    return static_cast<int>(kOk);
  });
}

int prana_tokenizer_destroy(prana_tokenizer_t t) {
  return guard([&] {
    delete t;
    return static_cast<int>(kOk);
  });
}

int prana_tokenizer_info(prana_tokenizer_t t, int* kind, size_t* vocab_size) {
  return guard([&] {
    PRANA_CHECK(t, "null tokenizer");
    if (kind) *kind = t->t.kind;
    if (vocab_size) *vocab_size = t->t.vocab_size();
    return static_cast<int>(kOk);
  });
}

static int ids_out(const std::vector<uint32_t>& ids, uint32_t* out, size_t cap, size_t* n) {
  *n = ids.size();
  if (!out || cap < ids.size())
    return fail(kErrShortBuffer, "id buffer of " + std::to_string(cap) + "; " + std::to_string(ids.size()) + " needed");
  std::copy(ids.begin(), ids.end(), out);
  return kOk;
}

int prana_tokenizer_encode(prana_tokenizer_t t, const char* text, size_t len, int bos, int eos, uint32_t* ids,
                           size_t cap, size_t* n) {
  return guard([&] {
    PRANA_CHECK(t && (text || len == 0) && n, "null argument");
    PRANA_CHECK(t->t.kind == 0, "encode with BOS/EOS flags is the SentencePiece tokenizer's (use encode_prompt)");
    const std::string s(text ? text : "", len);
    PRANA_CHECK(utf8_valid(s), "text is not valid UTF-8");
    return ids_out(t->t.spm.encode(s, bos != 0, eos != 0), ids, cap, n);
  });
}

int prana_tokenizer_encode_prompt(prana_tokenizer_t t, const char* text, size_t len, uint32_t* ids, size_t cap,
                                  size_t* n) {
  return guard([&] {
    PRANA_CHECK(t && (text || len == 0) && n, "null argument");
    const std::string s(text ? text : "", len);
    PRANA_CHECK(utf8_valid(s), "text is not valid UTF-8");
    return ids_out(t->t.encode_prompt(s), ids, cap, n);
  });
}

int prana_tokenizer_decode(prana_tokenizer_t t, uint32_t prev, uint32_t token, char* buf, size_t cap, size_t* len) {
  return guard([&] {
    PRANA_CHECK(t && len, "null argument");
    const std::string b = t->t.decode(prev, token);
    *len = b.size();
    if (!buf || cap < b.size())
      return fail(kErrShortBuffer, "byte buffer of " + std::to_string(cap) + "; " + std::to_string(b.size()) + " needed");
    if (!b.empty()) std::memcpy(buf, b.data(), b.size());
    return static_cast<int>(kOk);
  });
}

int prana_tokenizer_is_stop(prana_tokenizer_t t, uint32_t token, int* stop) {
  return guard([&] {
    PRANA_CHECK(t && stop, "null argument");
    *stop = t->t.is_stop(token) ? 1 : 0;
    return static_cast<int>(kOk);
  });
}

int prana_tokenizer_stop_ids(prana_tokenizer_t t, uint32_t* ids, size_t cap, size_t* n) {
  return guard([&] {
    PRANA_CHECK(t && n, "null argument");
    std::vector<uint32_t> v;
    if (t->t.kind == 0) {
      v = {t->t.spm.eos_id, t->t.spm.bos_id};
    } else {
      if (t->t.bpe.has_eos) v.push_back(t->t.bpe.eos_id);
      if (t->t.bpe.has_bos) v.push_back(t->t.bpe.bos_id);
    }
    return ids_out(v, ids, cap, n);
  });
}

int prana_bpe_pre_tokenize(const char* text, size_t len, size_t* bounds, size_t cap, size_t* n) {
  return guard([&] {
    PRANA_CHECK((text || len == 0) && n, "null argument");
    const std::string s(text ? text : "", len);
    PRANA_CHECK(utf8_valid(s), "text is not valid UTF-8");
    const auto pieces = bpe_pre_tokenize(s);
    *n = pieces.size();
    if (!bounds || cap < 2 * pieces.size()) return fail(kErrShortBuffer, "bounds buffer too short");
    for (size_t i = 0; i < pieces.size(); i++) {
      bounds[2 * i] = pieces[i].first;
      bounds[2 * i + 1] = pieces[i].second;
    }
    return static_cast<int>(kOk);
  });
}

// ------------------------------------------------------------------ graph (prana-graph over device buffers)
int prana_graph_create(prana_graph_t* out) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(out, "null argument");
    *out = new prana_graph();
    return static_cast<int>(kOk);
  });
}

int prana_graph_destroy(prana_graph_t g) {
  return guard([&] {
    if (g) (void)hipStreamSynchronize(pick_stream(nullptr));
    delete g;
    return static_cast<int>(kOk);
  });
}

int prana_graph_input(prana_graph_t g, size_t n_tokens, size_t* id) {
  return guard([&] {
    PRANA_CHECK(g && id, "null argument");
    g->g.n_tokens = std::max(g->g.n_tokens, n_tokens);
    *id = g->g.push(GraphNode{});
    return static_cast<int>(kOk);
  });
}

int prana_graph_matmul_f32(prana_graph_t g, size_t x, const float* weight, size_t k, size_t n_rows, size_t* id) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(g && weight && id, "null argument");
    PRANA_CHECK(k > 0 && n_rows > 0, "graph: matmul_f32 needs k > 0 and n_rows > 0");
    if (int rc = g->g.check_id(x, "matmul_f32")) return rc;
    GraphNode n;
    n.op = GraphNode::kMatmulF32;
    n.a = x;
    n.w = std::make_unique<Mat>();
    if (int rc = mat_from_ggml(0, n_rows, k, weight, n_rows * k * 4, *n.w)) return rc;
    *id = g->g.push(std::move(n));
    return static_cast<int>(kOk);
  });
}

int prana_graph_matmul_q8(prana_graph_t g, size_t x, size_t rows, size_t cols, const int8_t* q, const float* scales,
                          size_t* id) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(g && q && scales && id, "null argument");
    PRANA_CHECK(rows > 0 && cols > 0, "graph: matmul_q8 needs a non-empty matrix");
    if (int rc = g->g.check_id(x, "matmul_q8")) return rc;
    GraphNode n;
    n.op = GraphNode::kMatmulQ8;
    n.a = x;
    n.w = std::make_unique<Mat>();
    if (int rc = mat_from_q8_parts(rows, cols, q, scales, *n.w)) return rc;
    *id = g->g.push(std::move(n));
    return static_cast<int>(kOk);
  });
}

int prana_graph_rmsnorm(prana_graph_t g, size_t x, const float* weight, size_t dim, float eps, size_t* id) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(g && weight && id, "null argument");
    PRANA_CHECK(dim > 0, "graph: rmsnorm needs dim > 0");
    if (int rc = g->g.check_id(x, "rmsnorm")) return rc;
    GraphNode n;
    n.op = GraphNode::kRmsNorm;
    n.a = x;
    n.dim = dim;
    n.eps = eps;
    if (int rc = n.vec.alloc(dim * 4)) return rc;
    PRANA_HIP(hipMemcpy(n.vec.p, weight, dim * 4, hipMemcpyHostToDevice));
    *id = g->g.push(std::move(n));
    return static_cast<int>(kOk);
  });
}

int prana_graph_add(prana_graph_t g, size_t a, size_t b, size_t* id) {
  return guard([&] {
    PRANA_CHECK(g && id, "null argument");
    if (int rc = g->g.check_id(a, "add")) return rc;
    if (int rc = g->g.check_id(b, "add")) return rc;
    GraphNode n;
    n.op = GraphNode::kAdd;
    n.a = a;
    n.b = b;
    *id = g->g.push(std::move(n));
    return static_cast<int>(kOk);
  });
}

int prana_graph_softmax(prana_graph_t g, size_t x, size_t* id) {
  return guard([&] {
    PRANA_CHECK(g && id, "null argument");
    if (int rc = g->g.check_id(x, "softmax")) return rc;
    GraphNode n;
    n.op = GraphNode::kSoftmax;
    n.a = x;
    *id = g->g.push(std::move(n));
    return static_cast<int>(kOk);
  });
}

int prana_graph_rope(prana_graph_t g, size_t x, size_t n_heads, size_t head_dim, float theta_base, size_t* id) {
  return guard([&] {
    PRANA_CHECK(g && id, "null argument");
    PRANA_CHECK(head_dim > 0 && head_dim % 2 == 0, "graph: head_dim must be even for RoPE");
    PRANA_CHECK(n_heads > 0, "graph: rope needs n_heads > 0");
    if (int rc = g->g.check_id(x, "rope")) return rc;
    GraphNode n;
    n.op = GraphNode::kRope;
    n.a = x;
    n.n_heads = n_heads;
    n.head_dim = head_dim;
    n.theta = theta_base;
    *id = g->g.push(std::move(n));
    return static_cast<int>(kOk);
  });
}

int prana_graph_attention(prana_graph_t g, size_t q, size_t k, size_t v, size_t n_heads, size_t n_kv_heads,
                          size_t head_dim, size_t* id) {
  return guard([&] {
    PRANA_CHECK(g && id, "null argument");
    PRANA_CHECK(n_kv_heads > 0 && n_heads % n_kv_heads == 0, "graph: n_heads must be a multiple of n_kv_heads");
    PRANA_CHECK(n_heads > 0 && head_dim > 0 && head_dim <= 256, "graph: attention needs head_dim in 1..=256");
    for (size_t in : {q, k, v})
      if (int rc = g->g.check_id(in, "attention")) return rc;
    GraphNode n;
    n.op = GraphNode::kAttention;
    n.a = q;
    n.b = k;
    n.c = v;
    n.n_heads = n_heads;
    n.n_kv_heads = n_kv_heads;
    n.head_dim = head_dim;
    *id = g->g.push(std::move(n));
    return static_cast<int>(kOk);
  });
}

int prana_graph_set_input(prana_graph_t g, size_t id, const float* values, const size_t* shape, int n_dims) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(g, "null graph");
    return g->g.set_value(id, values, false, shape, n_dims, pick_stream(nullptr));
  });
}

int prana_graph_set_input_device(prana_graph_t g, size_t id, const float* values, const size_t* shape, int n_dims) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(g, "null graph");
    return g->g.set_value(id, values, true, shape, n_dims, pick_stream(nullptr));
  });
}

int prana_graph_execute(prana_graph_t g, int* error_kind, size_t* error_node) {
  return guard([&] {
    INIT_OR_RETURN();
    PRANA_CHECK(g, "null graph");
    int kind = 0;
    size_t node = 0;
    const int rc = g->g.execute(pick_stream(nullptr), &kind, &node);
    if (error_kind) *error_kind = kind;
    if (error_node) *error_node = node;
    return rc;
  });
}

int prana_graph_reset(prana_graph_t g) {
  return guard([&] {
    PRANA_CHECK(g, "null graph");
    for (GraphNode& n : g->g.nodes)
      if (n.op != GraphNode::kInput) n.has_value = false;
    return static_cast<int>(kOk);
  });
}

int prana_graph_shape(prana_graph_t g, size_t id, size_t* shape, int* n_dims) {
  return guard([&] {
    PRANA_CHECK(g && shape && n_dims, "null argument");
    if (int rc = g->g.check_id(id, "shape")) return rc;
    const GraphNode& n = g->g.nodes[id];
    if (!n.has_value) return fail(kErrInvalid, "graph: node " + std::to_string(id) + " has no value");
    *n_dims = static_cast<int>(n.shape.size());
    for (size_t i = 0; i < n.shape.size(); i++) shape[i] = n.shape[i];
    return static_cast<int>(kOk);
  });
}

int prana_graph_output_f32(prana_graph_t g, size_t id, float* out, size_t cap, size_t* n) {
  return guard([&] {
    PRANA_CHECK(g && n, "null argument");
    if (int rc = g->g.check_id(id, "output_f32")) return rc;
    const GraphNode& node = g->g.nodes[id];
    if (!node.has_value) return fail(kErrInvalid, "graph: input node " + std::to_string(id) + " is unset");
    *n = node.numel();
    if (!out || cap < *n) return fail(kErrShortBuffer, "graph: output buffer shorter than the node's value");
    if (*n) PRANA_HIP(hipMemcpy(out, node.value.p, *n * 4, hipMemcpyDeviceToHost));
    return static_cast<int>(kOk);
  });
}

int prana_graph_output_device(prana_graph_t g, size_t id, const float** ptr, size_t* n) {
  return guard([&] {
    PRANA_CHECK(g && ptr && n, "null argument");
    if (int rc = g->g.check_id(id, "output_device")) return rc;
    const GraphNode& node = g->g.nodes[id];
    if (!node.has_value) return fail(kErrInvalid, "graph: input node " + std::to_string(id) + " is unset");
    *ptr = node.value.as<float>();
    *n = node.numel();
    return static_cast<int>(kOk);
  });
}

int prana_model_config(prana_model_t m, prana_config* cfg) {
  return guard([&] {
    PRANA_CHECK(m && cfg, "null argument");
    *cfg = m->m.c;
    return static_cast<int>(kOk);
  });
}

}  // extern "C"
