// Device-resident model, KV cache and the forward passes (prana-model
// checkpoint.rs / infer.rs), driving the kernels of kernels.h in the order the
// reference runs its scalar kernels, so logits and token streams are
// bit-identical to the CPU path.
#include "model.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include <unistd.h>

namespace prana {

namespace {

double now_s() {
  return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

bool parse_layer(const std::string& name, size_t& layer, std::string& rest) {
  if (name.rfind("blk.", 0) != 0) return false;
  size_t dot = name.find('.', 4);
  if (dot == std::string::npos) return false;
  layer = std::strtoull(name.substr(4, dot - 4).c_str(), nullptr, 10);
  rest = name.substr(dot + 1);
  return true;
}

}  // namespace

// ------------------------------------------------------------------ tensors
int Model::set_tensor(const std::string& name, int t, const uint64_t* dims, int n_dims, const void* bytes,
                      size_t nbytes) {
  const prana_config& k = c;
  size_t q_dim = k.n_heads * k.head_dim, kv_dim = k.n_kv_heads * k.head_dim;
  size_t n = 1;
  for (int i = 0; i < n_dims; i++) n *= dims[i];
  auto want2 = [&](size_t cols, size_t rows) -> int {
    if (n_dims != 2 || dims[0] != cols || dims[1] != rows)
      return fail(kErrInvalid, "tensor '" + name + "': expected shape [" + std::to_string(cols) + ", " +
                                   std::to_string(rows) + "]");
    return kOk;
  };
  auto vec_of = [&](size_t len, DevBuf& dst, bool& flag) -> int {
    if (n_dims != 1 || dims[0] != len)
      return fail(kErrInvalid, "tensor '" + name + "': expected length " + std::to_string(len));
    std::vector<float> f(len);
    if (t == 0) {
      PRANA_CHECK(nbytes >= len * 4, "vector tensor: short buffer");
      std::memcpy(f.data(), bytes, len * 4);
    } else if (t == 1) {
      PRANA_CHECK(nbytes >= len * 2, "vector tensor: short buffer");
      const uint8_t* b = static_cast<const uint8_t*>(bytes);
      for (size_t i = 0; i < len; i++) f[i] = host_f16_to_f32(static_cast<uint16_t>(b[2 * i] | (b[2 * i + 1] << 8)));
    } else {
      return fail(kErrUnsupported, "tensor '" + name + "': norm/bias vectors must be F32 or F16");
    }
    int rc = dst.alloc(len * 4);
    if (rc) return rc;
    PRANA_HIP(hipMemcpy(dst.p, f.data(), len * 4, hipMemcpyHostToDevice));
    flag = true;
    return kOk;
  };

  if (name == "token_embd.weight") {
    int rc = want2(k.dim, k.vocab_size);
    if (rc) return rc;
    // gguf.rs:309-326: Q4_0/Q4_K/Q6_K tables stay packed; anything else
    // becomes a dense f32 table (also what a tied classifier then reads).
    bool packed = (t == 2 && k.dim % 32 == 0) || ((t == 12 || t == 14) && k.dim % 256 == 0);
    auto m = std::make_unique<Mat>();
    if (packed) {
      rc = mat_from_ggml(t, k.vocab_size, k.dim, bytes, nbytes, *m);
    } else {
      PRANA_CHECK(t == 0 || t == 1 || t == 2 || t == 8, "token_embd.weight: unsupported type for a dense table");
      // force a dense table: F32/F16 already are; Q8_0/Q4_0 with odd dims are densified.
      if (t == 8 || t == 2) {
        // dequantize on the host through a dense upload path
        Mat tmp;
        std::vector<float> f(k.vocab_size * k.dim);
        const uint8_t* raw = static_cast<const uint8_t*>(bytes);
        auto f16 = [&](const uint8_t* p) { return host_f16_to_f32(static_cast<uint16_t>(p[0] | (p[1] << 8))); };
        size_t nn = f.size();
        if (t == 8) {
          for (size_t b = 0; b < nn / 32; b++) {
            float s = f16(raw + b * 34);
            for (int j = 0; j < 32; j++) f[b * 32 + j] = static_cast<float>(static_cast<int8_t>(raw[b * 34 + 2 + j])) * s;
          }
        } else {
          for (size_t b = 0; b < nn / 32; b++) {
            const uint8_t* p = raw + b * 18;
            float d = f16(p);
            for (int j = 0; j < 16; j++) f[b * 32 + j] = d * (static_cast<float>(p[2 + j] & 0xF) - 8.0f);
            for (int j = 0; j < 16; j++) f[b * 32 + 16 + j] = d * (static_cast<float>(p[2 + j] >> 4) - 8.0f);
          }
        }
        rc = mat_from_ggml(0, k.vocab_size, k.dim, f.data(), f.size() * 4, *m);
      } else {
        rc = mat_from_ggml(t, k.vocab_size, k.dim, bytes, nbytes, *m);
      }
    }
    if (rc) return rc;
    emb = std::move(m);
    return kOk;
  }
  if (name == "output_norm.weight") return vec_of(k.dim, rms_final, has_rms_final);
  size_t cols = 0, rows = 0;
  if (std::unique_ptr<Mat>* slot = mat_slot(name, &cols, &rows)) {
    int rc = want2(cols, rows);
    if (rc) return rc;
    auto m = std::make_unique<Mat>();
    if ((rc = mat_from_ggml(t, rows, cols, bytes, nbytes, *m))) return rc;
    *slot = std::move(m);
    return kOk;
  }

  size_t l;
  std::string rest;
  if (!parse_layer(name, l, rest) || l >= layers.size()) return fail(kErrInvalid, "unknown tensor '" + name + "'");
  Layer& L = layers[l];
  if (rest == "attn_norm.weight") return vec_of(k.dim, L.vec[kRmsAtt], L.has[kRmsAtt]);
  if (rest == "ffn_norm.weight") return vec_of(k.dim, L.vec[kRmsFfn], L.has[kRmsFfn]);
  if (rest == "attn_q.bias") return vec_of(q_dim, L.vec[kBq], L.has[kBq]);
  if (rest == "attn_k.bias") return vec_of(kv_dim, L.vec[kBk], L.has[kBk]);
  if (rest == "attn_v.bias") return vec_of(kv_dim, L.vec[kBv], L.has[kBv]);
  return fail(kErrInvalid, "unknown tensor '" + name + "'");
}

// The projection / classifier slot a GGUF name addresses, with its expected
// [cols, rows]; null for any other name.
std::unique_ptr<Mat>* Model::mat_slot(const std::string& name, size_t* cols, size_t* rows) {
  const size_t q_dim = c.n_heads * c.head_dim, kv_dim = c.n_kv_heads * c.head_dim;
  if (name == "output.weight") {
    *cols = c.dim;
    *rows = c.vocab_size;
    return &wcls;
  }
  size_t l;
  std::string rest;
  if (!parse_layer(name, l, rest) || l >= layers.size()) return nullptr;
  static const struct {
    const char* name;
    LayerMat slot;
  } kMats[] = {{"attn_q.weight", kWq},      {"attn_k.weight", kWk},   {"attn_v.weight", kWv},
               {"attn_output.weight", kWo}, {"ffn_gate.weight", kW1}, {"ffn_down.weight", kW2},
               {"ffn_up.weight", kW3}};
  for (const auto& e : kMats) {
    if (rest != e.name) continue;
    const size_t in[7] = {c.dim, c.dim, c.dim, q_dim, c.dim, c.hidden_dim, c.dim};
    const size_t out[7] = {q_dim, kv_dim, kv_dim, c.dim, c.hidden_dim, c.dim, c.hidden_dim};
    *cols = in[e.slot];
    *rows = out[e.slot];
    return &layers[l].w[e.slot];
  }
  return nullptr;
}

// A QuantMatrix with f32 scales (quantize_q8's output, matmul.rs:61-84) into
// a projection or classifier slot.
int Model::set_q8(const std::string& name, size_t rows, size_t cols, const int8_t* q, const float* scales) {
  size_t want_c = 0, want_r = 0;
  std::unique_ptr<Mat>* slot = mat_slot(name, &want_c, &want_r);
  if (!slot) return fail(kErrInvalid, "unknown matrix '" + name + "'");
  PRANA_CHECK(rows == want_r && cols == want_c, "tensor '" + name + "': shape does not match the config");
  auto m = std::make_unique<Mat>();
  if (int rc = mat_from_q8_parts(rows, cols, q, scales, *m)) return rc;
  *slot = std::move(m);
  finalized = false;
  return kOk;
}

// Config checks shared by prana_model_create and the GGUF loader: what the
// kernels of this backend need (the activation quantizer and the fused
// norm/MLP epilogues work in whole 32-blocks of dim and hidden_dim).
int check_config(const prana_config& c) {
  PRANA_CHECK(c.dim > 0 && c.n_layers > 0 && c.n_heads > 0 && c.vocab_size > 0 && c.seq_len > 0,
              "config: zero-sized dimension");
  PRANA_CHECK(c.n_kv_heads > 0 && c.n_heads % c.n_kv_heads == 0, "config: n_heads % n_kv_heads != 0");
  PRANA_CHECK(c.head_dim > 0 && c.head_dim % 2 == 0 && c.head_dim <= 256, "config: head_dim must be even and <= 256");
  PRANA_CHECK(c.dim % 32 == 0 && c.hidden_dim % 32 == 0, "config: dim and hidden_dim must be multiples of 32");
  PRANA_CHECK(c.act == 0 || c.act == 1, "config: act must be 0 (silu) or 1 (gelu_tanh)");
  return kOk;
}

int Model::finalize() {
  PRANA_CHECK(emb != nullptr, "model: token_embd.weight missing");
  PRANA_CHECK(has_rms_final, "model: output_norm.weight missing");
  for (size_t l = 0; l < layers.size(); l++) {
    for (int i = 0; i < 7; i++)
      if (!layers[l].w[i]) return fail(kErrInvalid, "model: layer " + std::to_string(l) + " is missing a projection");
    if (!layers[l].has[kRmsAtt] || !layers[l].has[kRmsFfn])
      return fail(kErrInvalid, "model: layer " + std::to_string(l) + " is missing a norm weight");
  }
  // RoPE table: (cosf, sinf) of (pos as f32) * powf(theta, -(2m)/hd), the
  // values attention.rs:95-96 / 114-115 compute for every pair.
  size_t half = c.head_dim / 2;
  std::vector<float> tab(c.seq_len * half * 2);
  for (size_t m = 0; m < half; m++) {
    float freq = std::pow(c.rope_theta, -(2.0f * static_cast<float>(m)) / static_cast<float>(c.head_dim));
    for (size_t p = 0; p < c.seq_len; p++) {
      float ang = static_cast<float>(p) * freq;
      tab[(p * half + m) * 2] = std::cos(ang);
      tab[(p * half + m) * 2 + 1] = std::sin(ang);
    }
  }
  int rc = rope.alloc(tab.size() * 4);
  if (rc) return rc;
  PRANA_HIP(hipMemcpy(rope.p, tab.data(), tab.size() * 4, hipMemcpyHostToDevice));
  finalized = true;
  return kOk;
}

size_t Model::stream_bytes() const {
  size_t b = 0;
  for (auto& L : layers)
    for (auto& w : L.w)
      if (w) b += w->stream_bytes;
  b += head().stream_bytes;
  return b;
}

const Mat& Model::head() const { return wcls ? *wcls : *emb; }

// ------------------------------------------------------------------ workspace
int Model::ensure_ws(size_t n_tok, size_t ctx_cap, bool prefill_attn) {
  size_t q_dim = c.n_heads * c.head_dim, kv_dim = c.n_kv_heads * c.head_dim;
  size_t kmax = std::max(c.dim, std::max(q_dim, c.hidden_dim));
  int rc;
  if (n_tok > ws.cap_tok) {
    size_t n = n_tok;
    ws.gen++;
    if ((rc = ws.x.alloc(n * c.dim * 4)) || (rc = ws.xb.alloc(n * c.dim * 4)) || (rc = ws.q.alloc(n * q_dim * 4)) ||
        (rc = ws.k.alloc(n * kv_dim * 4)) || (rc = ws.v.alloc(n * kv_dim * 4)) ||
        (rc = ws.attn.alloc(n * q_dim * 4)) || (rc = ws.gate.alloc(n * c.hidden_dim * 4)) ||
        (rc = ws.up.alloc(n * c.hidden_dim * 4)) || (rc = ws.logits.alloc(n * c.vocab_size * 4)) ||
        (rc = ws.qa.alloc(n * kmax)) || (rc = ws.sa.alloc(n * (kmax / 32 + 1) * 4)) ||
        (rc = ws.sums.alloc(n * (kmax / 32 + 1) * 4)) || (rc = ws.hq.alloc(n * c.hidden_dim)) ||
        (rc = ws.hsa.alloc(n * (c.hidden_dim / 32) * 4)) || (rc = ws.hsum.alloc(n * (c.hidden_dim / 32) * 4)) ||
        (rc = ws.tokens.alloc(n * 4)) ||
        (rc = ws.argmax.alloc(n * 4)))
      return rc;
    ws.cap_tok = n;
  }
  if (!ws.xch.p) {  // zeroed once; each launch that uses it leaves it zeroed
    if ((rc = ws.xch.alloc(kNormXchBytes))) return rc;
    PRANA_HIP(hipMemset(ws.xch.p, 0, ws.xch.bytes));
    ws.gen++;
  }
  size_t need = (prefill_attn ? attention_scratch_floats(n_tok, c.n_heads, n_tok, false)
                              : attention_scratch_floats(n_tok, c.n_heads, ctx_cap)) * 4;
  const void* before = ws.scratch.p;
  if ((rc = ws.scratch.ensure(std::max<size_t>(need, 4)))) return rc;
  if (ws.scratch.p != before) ws.gen++;
  return kOk;
}

// ------------------------------------------------------------------ cache
int Cache::create(const Model& m, size_t positions) {
  len = std::min(positions, m.c.seq_len);
  kv_dim = m.c.n_kv_heads * m.c.head_dim;
  n_layers = m.c.n_layers;
  kcap = m.c.head_dim == 64 || m.c.head_dim == 128 ? len : 0;
  size_t per = len * kv_dim * 2;
  int rc = buf.alloc(std::max<size_t>(per * 2 * n_layers, 2));
  if (rc) return rc;
  PRANA_HIP(hipMemset(buf.p, 0, buf.bytes));
  return kOk;
}

uint16_t* Cache::k(size_t l) const { return buf.as<uint16_t>() + (2 * l) * len * kv_dim; }
uint16_t* Cache::v(size_t l) const { return buf.as<uint16_t>() + (2 * l + 1) * len * kv_dim; }

// ------------------------------------------------------------------ forward pieces
template <class F>
int Model::timed(size_t bytes, size_t n, hipStream_t s, F&& launch) {
  GemvProfile& gp = gemv_profile();
  size_t ev = 0;
  const bool sample = gp.on && (gp.calls++ % gp.period == 0);
  if (sample) {
    if (int rc = gp.next_pair(&ev)) return rc;
    launch_events() = LaunchEvents{gp.pool[ev], gp.pool[ev + 1]};
  }
  int rc = launch();
  if (sample) {
    if (launch_events().start) {  // not a single timestamped decode launch: bracket on the stream
      launch_events() = LaunchEvents{};
      gp.skipped += 1;
    } else {
      gp.pending.push_back({ev, bytes, n});
    }
  }
  return rc;
}

int Model::apply(const Mat& w, size_t n, const float* xf, const GemvOut& o, hipStream_t s, bool hset) {
  return timed(w.stream_bytes, n, s, [&] {
    if (hset) return launch_gemv(w.d, xf, ws.hq.as<int8_t>(), ws.hsa.as<float>(), ws.hsum.as<int>(), n, o, s);
    return launch_gemv(w.d, xf, ws.qa.as<int8_t>(), ws.sa.as<float>(), ws.sums.as<int>(), n, o, s);
  });
}

int Model::apply_multi(const Mat* const* w, const GemvOut* o, int n_mats, size_t n, const float* xf, hipStream_t s,
                       const RopeKv* rk, bool* fused, const NormIn* norm) {
  if (fused) *fused = false;
  if (norm) {  // one launch over all matrices, which normalises its own input
    PRANA_CHECK(n == 1 && n_mats >= 1 && n_mats <= 3, "apply_multi: a fused rmsnorm takes one token");
    DevMat d[3];
    size_t bytes = 0;
    for (int k = 0; k < n_mats; k++) {
      d[k] = w[k]->d;
      bytes += w[k]->stream_bytes;
    }
    return timed(bytes, n, s, [&] {
      return launch_gemv_multi(d, o, n_mats, nullptr, nullptr, nullptr, n, s, rk, fused, norm);
    });
  }
  // three quantized matrices that one launch takes (one format, or a fusable
  // pair of formats) go together; otherwise runs of one format
  bool fuse3 = n_mats == 3;
  for (int k = 0; fuse3 && k < 3; k++) fuse3 = w[k]->d.kind != kKindF32;
  if (fuse3) {
    const DevMat d3[3] = {w[0]->d, w[1]->d, w[2]->d};
    fuse3 = gemv_multi_fusable(d3, 3);
  }
  int i = 0;
  while (i < n_mats) {
    int j = i + 1;
    if (fuse3) j = 3;
    else
      while (j < n_mats && j - i < 3 && w[j]->d.kind == w[i]->d.kind && w[j]->d.cols == w[i]->d.cols) j++;
    if (j - i == 1 || w[i]->d.kind == kKindF32) {
      for (int k = i; k < j; k++)
        if (int rc = apply(*w[k], n, xf, o[k], s)) return rc;
    } else {
      DevMat d[3];
      size_t bytes = 0;
      for (int k = i; k < j; k++) {
        d[k - i] = w[k]->d;
        bytes += w[k]->stream_bytes;
      }
      const bool all3 = i == 0 && j - i == 3;
      int rc = timed(bytes, n, s, [&] {
        return launch_gemv_multi(d, o + i, j - i, ws.qa.as<int8_t>(), ws.sa.as<float>(), ws.sums.as<int>(), n, s,
                                 all3 ? rk : nullptr, all3 ? fused : nullptr);
      });
      if (rc) return rc;
    }
    i = j;
  }
  return kOk;
}

int Model::apply_gate_up(const Mat& gate, const Mat& up, size_t n, hipStream_t s, const NormIn* norm, bool dense_h) {
  const size_t H = c.hidden_dim;
  // where the skinny matrix-core kernel takes the batch (from 9 tokens, and
  // from 3 for matrices as large as the 7B gate|up): one skinny launch that
  // also forms and quantizes h (at 5 tokens on the 7B gate|up the fused
  // decode-tile launch and the quantization of h take 40.1 + 5.1 us)
  const bool fuse = gate.d.kind != kKindF32 && gate.d.kind == up.d.kind && n <= kGemvDecodeMaxTokens &&
                    !gemv_batch_skinny(gate.d, n);
  PRANA_CHECK(!norm || (fuse && n == 1), "apply_gate_up: a fused rmsnorm takes one token of fusable matrices");
  if (fuse) {
    return timed(gate.stream_bytes + up.stream_bytes, n, s, [&] {
      return launch_gemv_act(gate.d, up.d, c.act, ws.qa.as<int8_t>(), ws.sa.as<float>(), ws.sums.as<int>(), n,
                             ws.gate.as<float>(), ws.hq.as<int8_t>(), ws.hsa.as<float>(), ws.hsum.as<int>(), s,
                             norm);
    });
  }
  if (gemm_skinny_act_fusable(gate.d, up.d, n)) {  // verify batches: the same, on the skinny kernel
    float* h = dense_h ? ws.gate.as<float>() : nullptr;
    return timed(gate.stream_bytes + up.stream_bytes, n, s, [&] {
      return launch_gemm_skinny_act(gate.d, up.d, ws.qa.as<int8_t>(), ws.sa.as<float>(), ws.sums.as<int>(), n, c.act,
                                    h, ws.hq.as<int8_t>(), ws.hsa.as<float>(), ws.hsum.as<int>(), s);
    });
  }
  if (gemm_act_fusable(gate.d, up.d, n)) {  // prefill: gate|up, the activation and h's quantization in one launch
    float* h = dense_h ? ws.gate.as<float>() : nullptr;
    return timed(gate.stream_bytes + up.stream_bytes, n, s, [&] {
      return launch_gemm_act(gate.d, up.d, ws.qa.as<int8_t>(), ws.sa.as<float>(), n, c.act, h, ws.hq.as<int8_t>(),
                             ws.hsa.as<float>(), ws.hsum.as<int>(), s);
    });
  }
  GemvOut og{ws.gate.as<float>(), H, nullptr, 0};
  GemvOut ou{ws.up.as<float>(), H, nullptr, 0};
  const Mat* w[2] = {&gate, &up};
  const GemvOut o[2] = {og, ou};
  if (int rc = apply_multi(w, o, 2, n, ws.xb.as<float>(), s)) return rc;
  return launch_act_mul(ws.gate.as<float>(), ws.up.as<float>(), n * H, c.act, ws.hq.as<int8_t>(), ws.hsa.as<float>(),
                        ws.hsum.as<int>(), s);
}

GemvProfile& gemv_profile() {
  static GemvProfile p;
  return p;
}

int GemvProfile::next_pair(size_t* ev) {
  while (used + 2 > pool.size()) {
    hipEvent_t e;
    PRANA_HIP(hipEventCreate(&e));
    pool.push_back(e);
  }
  *ev = used;
  used += 2;
  return kOk;
}

int GemvProfile::collect() {
  for (auto& r : pending) {
    PRANA_HIP(hipEventSynchronize(pool[r.ev + 1]));
    float ms = 0.0f;
    PRANA_HIP(hipEventElapsedTime(&ms, pool[r.ev], pool[r.ev + 1]));
    if (r.bytes != kProfileAttentionKey) {  // the GEMV totals
      launches += 1;
      seconds += ms * 1e-3;
      bytes += static_cast<double>(r.bytes);
    }
    Shape& sh = shapes[r.bytes];
    sh.launches += 1;
    sh.seconds += ms * 1e-3;
  }
  pending.clear();
  used = 0;
  return kOk;
}

// Greedy decode of n_steps tokens over an existing cache: feed `token` at
// `pos`, take the argmax, feed it at pos+1, ... (the sampled part of the
// generate loop, infer.rs:729-763, without prompt handling or stop ids).
void StepGraph::reset() {
  if (exec) (void)hipGraphExecDestroy(exec);
  if (graph) (void)hipGraphDestroy(graph);
  exec = nullptr;
  graph = nullptr;
  cache_buf = ids = nullptr;
}

constexpr size_t kStreamFloorIds = 4096;

// A profiling tool loaded into this process: rocprofv3 preloads
// librocprofiler-sdk-tool and exports ROCPROF_* settings (older tools load
// librocprofiler64 / libroctracer64 through ROCP_TOOL_LIBRARIES / HSA_TOOLS_LIB).
// librocprofiler-register, which every HIP process maps, does not count.
bool profiler_tool_present() {
  for (char** e = environ; e && *e; ++e)
    if (std::strncmp(*e, "ROCPROF_", 8) == 0 || std::strncmp(*e, "ROCP_TOOL_LIBRARIES=", 20) == 0 ||
        std::strncmp(*e, "HSA_TOOLS_LIB=", 14) == 0)
      return true;
  std::FILE* f = std::fopen("/proc/self/maps", "r");
  if (!f) return false;
  char line[4096];
  bool hit = false;
  while (!hit && std::fgets(line, sizeof line, f))
    hit = std::strstr(line, "librocprofiler-sdk") || std::strstr(line, "librocprofiler64") ||
          std::strstr(line, "libroctracer64") || std::strstr(line, "librocprofv3");
  std::fclose(f);
  return hit;
}

// Replay of the captured decode step. Off with PRANA_DECODE_GRAPH=0, and off
// whenever a profiling tool is present: under rocprofv3's kernel tracing a
// process replaying the step crashed in host code inside hipGraphLaunch, so
// the same kernels are then launched one by one (decided once per process).
bool decode_graphs_enabled() {
  static const bool on = [] {
    const char* e = std::getenv("PRANA_DECODE_GRAPH");
    if (e && e[0] == '0') return false;
    return !profiler_tool_present();
  }();
  return on;
}

int Model::step_graph_ready(Cache& cache, size_t pos, uint32_t* ids, hipStream_t s, hipGraphExec_t* exec) {
  StepGraph& g = step_graph[attention_split_window(pos + 1, c.head_dim) ? 1 : 0];
  *exec = nullptr;
  if (g.exec && g.cache_buf == cache.buf.p && g.cache_len == cache.len && g.ws_gen == ws.gen && g.ids == ids) {
    *exec = g.exec;
    return kOk;
  }
  g.reset();
  pos_dev = ws.step_state.as<int>();
  PRANA_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
  int rc = forward_dev(cache, nullptr, ws.tokens.as<uint32_t>(), pos, true, s);
  if (!rc) rc = launch_argmax(ws.logits.as<float>(), 1, c.vocab_size, ws.tokens.as<uint32_t>(), s);
  if (!rc) rc = launch_decode_advance(ws.step_state.as<int>(), ws.tokens.as<uint32_t>(), ids, s);
  pos_dev = nullptr;
  hipGraph_t graph = nullptr;
  const hipError_t e = hipStreamEndCapture(s, &graph);
  if (!rc && e == hipSuccess) {
    const hipError_t ei = hipGraphInstantiate(&g.exec, graph, nullptr, nullptr, 0);
    if (ei != hipSuccess) {
      g.exec = nullptr;
      rc = fail(kErrHip, std::string("decode step graph: ") + hipGetErrorString(ei));
    }
  } else if (!rc) {
    rc = fail(kErrHip, std::string("decode step capture: ") + hipGetErrorString(e));
  }
  if (rc) {
    if (graph) (void)hipGraphDestroy(graph);
    return rc;
  }
  g.graph = graph;
  g.cache_buf = cache.buf.p;
  g.cache_len = cache.len;
  g.ws_gen = ws.gen;
  g.ids = ids;
  *exec = g.exec;
  return kOk;
}

int Model::decode(Cache& cache, uint32_t token, size_t pos, size_t n_steps, uint32_t* out) {
  hipStream_t s = ctx().stream;
  uint32_t* ids = nullptr;
  if (int rc = decode_stream(cache, token, pos, n_steps, s, &ids)) return rc;
  if (out && n_steps) PRANA_HIP(hipMemcpyAsync(out, ids + 1, n_steps * 4, hipMemcpyDeviceToHost, s));
  PRANA_HIP(hipStreamSynchronize(s));
  return kOk;
}

int Model::decode_stream(Cache& cache, uint32_t token, size_t pos, size_t n_steps, hipStream_t s, uint32_t** out_ids) {
  PRANA_CHECK(pos + n_steps <= cache.len, "decode: positions beyond the cache length");
  PRANA_CHECK(cache.len <= 0x7fffffff, "decode: cache length out of range");
  int rc = ensure_ws(1, cache.len, false);
  if (rc) return rc;
  // The token stream keeps a floor capacity and grows geometrically: its
  // address is part of the captured step's key, so a reallocation would force
  // a fresh capture and instantiation of the step for the next decode call.
  if ((n_steps + 1) * 4 > ws.stream_out.bytes) {
    const size_t want = std::max<size_t>({(n_steps + 1) * 4, 2 * ws.stream_out.bytes, kStreamFloorIds * 4});
    if ((rc = ws.stream_out.ensure(want))) return rc;
  }
  if ((rc = ws.step_state.ensure(8))) return rc;
  uint32_t* ids = ws.stream_out.as<uint32_t>();
  // ids[i] feeds step i; step i's argmax lands in ids[i+1].
  if ((rc = launch_decode_seed(nullptr, 0, token, ids, nullptr, s))) return rc;
  // Steps replay a captured step (the position and the step index live in
  // device memory), one captured step per run of steps on the same attention
  // path; while GEMV dispatches are being timed, steps launch kernel by
  // kernel. Both run the same kernels on the same data.
  size_t i = 0;
  if (decode_graphs_enabled() && !gemv_profile().on && n_steps > 0) {
    if ((rc = launch_decode_seed(ws.step_state.as<int>(), static_cast<int>(pos), token, nullptr,
                                 ws.tokens.as<uint32_t>(), s)))
      return rc;
    auto regime = [&](size_t k) { return attention_split_window(pos + k + 1, c.head_dim); };
    while (i < n_steps) {
      size_t j = i;
      while (j < n_steps && regime(j) == regime(i)) j++;
      hipGraphExec_t exec;
      if ((rc = step_graph_ready(cache, pos + i, ids, s, &exec))) return rc;
      for (; i < j; i++) PRANA_HIP(hipGraphLaunch(exec, s));
    }
  }
  for (; i < n_steps; i++) {
    if ((rc = forward_dev(cache, nullptr, ids + i, pos + i, true, s))) return rc;
    if ((rc = launch_argmax(ws.logits.as<float>(), 1, c.vocab_size, ids + i + 1, s))) return rc;
  }
  *out_ids = ids;
  return kOk;
}

int Model::norm_quant(const float* x, const DevBuf& w, size_t n, hipStream_t s) {
  return launch_rmsnorm(x, w.as<float>(), n, c.dim, c.norm_eps, ws.xb.as<float>(), ws.qa.as<int8_t>(),
                        ws.sa.as<float>(), ws.sums.as<int>(), s);
}

// The layer stack shared by forward (n = 1), prefill and forward_batch.
// mode: 0 decode (pos0 = pos), 1 prefill (f32-K/V attention over the window,
// positions 0..n), 2 verify (cache attention at pos0..pos0+n).
int Model::layers_pass(Cache& cache, size_t n, size_t pos0, int mode, hipStream_t s) {
  size_t hd = c.head_dim, q_dim = c.n_heads * hd, kv_dim = c.n_kv_heads * hd;
  float* x = ws.x.as<float>();
  const float2* tab = rope.as<float2>();
  int rc;
  for (size_t l = 0; l < layers.size(); l++) {
    Layer& L = layers[l];
    uint16_t* kc = cache.k(l);
    uint16_t* vc = cache.v(l);
    // --- attention block (infer.rs:163-188)
    // decode: the Q|K|V launch normalises x itself when its matrices allow it
    const Mat* wqkv[3] = {L.w[kWq].get(), L.w[kWk].get(), L.w[kWv].get()};
    const NormIn nin{x, L.vec[kRmsAtt].as<float>(), c.norm_eps};
    bool norm_fused = false;
    if (mode == 0 && n == 1) {
      const DevMat d3[3] = {wqkv[0]->d, wqkv[1]->d, wqkv[2]->d};
      norm_fused = gemv_norm_fusable(d3, 3);
    }
    if (!norm_fused && (rc = norm_quant(x, L.vec[kRmsAtt], n, s))) return rc;
    GemvOut oq{ws.q.as<float>(), q_dim, L.has[kBq] ? L.vec[kBq].as<float>() : nullptr, 0};
    GemvOut ok{ws.k.as<float>(), kv_dim, L.has[kBk] ? L.vec[kBk].as<float>() : nullptr, 0};
    GemvOut ov{ws.v.as<float>(), kv_dim, L.has[kBv] ? L.vec[kBv].as<float>() : nullptr, 0};
    bool roped = false;  // the Q|K|V launch also did RoPE and the cache rows
    {
      const GemvOut o[3] = {oq, ok, ov};
      // decode reads its position from device memory; a batch's positions
      // pos0..pos0+n-1 are known here
      const RopeKv rk{tab, static_cast<int>(hd), c.rope_neox, static_cast<int>(pos0), mode == 0 ? pos_dev : nullptr,
                      kc, vc, static_cast<int>(cache.kcap)};
      if ((rc = apply_multi(wqkv, o, 3, n, ws.xb.as<float>(), s, &rk, &roped, norm_fused ? &nin : nullptr)))
        return rc;
    }
    const ActQuant aq{ws.qa.as<int8_t>(), ws.sa.as<float>(), ws.sums.as<int>()};
    bool quantized = false;
    if (mode == 0) {
      if (!roped && (rc = launch_rope_kv(ws.q.as<float>(), ws.k.as<float>(), ws.v.as<float>(), q_dim, kv_dim, hd,
                                         tab, c.rope_neox, kc, vc, cache.kcap, pos_dev, pos0, s)))
        return rc;
      if ((rc = timed(kProfileAttentionKey, 1, s, [&] {
             return launch_attention_cache(ws.q.as<float>(), kc, vc, pos0, 1, c.n_heads, c.n_kv_heads, hd,
                                           ws.attn.as<float>(), ws.scratch.as<float>(), cache.len, pos_dev, s, &aq,
                                           &quantized, cache.kcap);
           })))
        return rc;
    } else {
      if (!roped && (rc = launch_rope_kv_rows(ws.q.as<float>(), ws.k.as<float>(), ws.v.as<float>(), n, q_dim, kv_dim,
                                              hd, tab, c.rope_neox, kc, vc, cache.kcap, pos0, s)))
        return rc;
      if (mode == 1)
        rc = launch_attention_prefill(ws.q.as<float>(), ws.k.as<float>(), ws.v.as<float>(), n, c.n_heads,
                                      c.n_kv_heads, hd, ws.attn.as<float>(), ws.scratch.as<float>(), s, &aq,
                                      &quantized);
      else
        rc = launch_attention_cache(ws.q.as<float>(), kc, vc, pos0, n, c.n_heads, c.n_kv_heads, hd,
                                    ws.attn.as<float>(), ws.scratch.as<float>(), cache.len, nullptr, s, &aq,
                                    &quantized, cache.kcap);
      if (rc) return rc;
    }
    // A q_dim that is not a whole number of 32-blocks only occurs with a dense
    // f32 wo (quantized formats need cols % 32 == 0), which reads ws.attn.
    if (!quantized && q_dim % 32 == 0 &&
        (rc = launch_quantize_acts(ws.attn.as<float>(), n, q_dim, ws.qa.as<int8_t>(), ws.sa.as<float>(),
                                   ws.sums.as<int>(), s)))
      return rc;
    GemvOut ores{x, c.dim, nullptr, 1};
    if ((rc = apply(*L.w[kWo], n, ws.attn.as<float>(), ores, s))) return rc;
    // --- gated MLP block (infer.rs:191-203)
    // decode: the gate|up launch normalises x itself when its matrices allow it
    const NormIn nin_ffn{x, L.vec[kRmsFfn].as<float>(), c.norm_eps, ws.xch.as<unsigned>()};
    const bool ffn_fused = mode == 0 && n == 1 && gemv_norm_act_fusable(L.w[kW1]->d, L.w[kW3]->d);
    if (!ffn_fused && (rc = norm_quant(x, L.vec[kRmsFfn], n, s))) return rc;
    if ((rc = apply_gate_up(*L.w[kW1], *L.w[kW3], n, s, ffn_fused ? &nin_ffn : nullptr,
                            L.w[kW2]->d.kind == kKindF32)))
      return rc;
    if ((rc = apply(*L.w[kW2], n, ws.gate.as<float>(), ores, s, true))) return rc;
  }
  return kOk;
}

// Model::logits / logits_batch (checkpoint.rs:239-265): final norm, then the
// head over n rows into ws.logits.
int Model::logits_pass(size_t n, hipStream_t s) {
  int rc = norm_quant(ws.x.as<float>(), rms_final, n, s);
  if (rc) return rc;
  GemvOut o{ws.logits.as<float>(), c.vocab_size, nullptr, 0};
  return apply(head(), n, ws.xb.as<float>(), o, s);
}

int Model::embed_tokens(const uint32_t* dev_ids, size_t n, hipStream_t s) {
  return launch_embed(emb->d, dev_ids, n, c.emb_scale, ws.x.as<float>(), s);
}

int Model::check_tokens(const uint32_t* t, size_t n) {
  for (size_t i = 0; i < n; i++)
    if (t[i] >= c.vocab_size) return fail(kErrInvalid, "token id " + std::to_string(t[i]) + " out of vocabulary");
  return kOk;
}

int Model::forward_dev(Cache& cache, const uint32_t* host_token, const uint32_t* dev_token, size_t pos,
                       bool need_logits, hipStream_t s) {
  PRANA_CHECK(finalized, "model not finalized");
  PRANA_CHECK(pos < cache.len, "forward: position beyond the cache length");
  int rc = ensure_ws(1, cache.len, false);
  if (rc) return rc;
  if (host_token) {
    if ((rc = check_tokens(host_token, 1))) return rc;
    PRANA_HIP(hipMemcpyAsync(ws.tokens.p, host_token, 4, hipMemcpyHostToDevice, s));
  }
  if ((rc = embed_tokens(dev_token ? dev_token : ws.tokens.as<uint32_t>(), 1, s))) return rc;
  if ((rc = layers_pass(cache, 1, pos, 0, s))) return rc;
  if (need_logits && (rc = logits_pass(1, s))) return rc;
  return kOk;
}

int Model::forward(Cache& cache, uint32_t token, size_t pos, bool need_logits, float* logits_host) {
  hipStream_t s = ctx().stream;
  int rc = forward_dev(cache, &token, nullptr, pos, need_logits, s);
  if (rc) return rc;
  if (need_logits && logits_host)
    PRANA_HIP(hipMemcpyAsync(logits_host, ws.logits.p, c.vocab_size * 4, hipMemcpyDeviceToHost, s));
  PRANA_HIP(hipStreamSynchronize(s));
  return kOk;
}

int Model::batch_dev(Cache& cache, const uint32_t* tokens, size_t n, size_t pos0, int mode, hipStream_t s) {
  PRANA_CHECK(finalized, "model not finalized");
  PRANA_CHECK(n > 0, "empty token batch");
  PRANA_CHECK(pos0 + n <= cache.len, "batch: positions beyond the cache length");
  int rc = check_tokens(tokens, n);
  if (rc) return rc;
  if ((rc = ensure_ws(n, cache.len, mode == 1))) return rc;
  PRANA_HIP(hipMemcpyAsync(ws.tokens.p, tokens, n * 4, hipMemcpyHostToDevice, s));
  if ((rc = embed_tokens(ws.tokens.as<uint32_t>(), n, s))) return rc;
  return layers_pass(cache, n, pos0, mode, s);
}

int Model::batch_dev_ids(Cache& cache, const uint32_t* dev_tokens, size_t n, size_t pos0, int mode, hipStream_t s) {
  PRANA_CHECK(finalized, "model not finalized");
  PRANA_CHECK(n > 0, "empty token batch");
  PRANA_CHECK(pos0 + n <= cache.len, "batch: positions beyond the cache length");
  int rc = ensure_ws(n, cache.len, mode == 1);
  if (rc) return rc;
  if ((rc = embed_tokens(dev_tokens, n, s))) return rc;
  return layers_pass(cache, n, pos0, mode, s);
}

int Model::prefill(Cache& cache, const uint32_t* tokens, size_t n) {
  hipStream_t s = ctx().stream;
  if (n == 0) return kOk;
  int rc = batch_dev(cache, tokens, n, 0, 1, s);
  if (rc) return rc;
  PRANA_HIP(hipStreamSynchronize(s));
  return kOk;
}

int Model::forward_batch(Cache& cache, const uint32_t* tokens, size_t n, size_t pos0, float* logits_host) {
  hipStream_t s = ctx().stream;
  int rc = batch_dev(cache, tokens, n, pos0, 2, s);
  if (!rc) rc = logits_pass(n, s);
  if (rc) return rc;
  if (logits_host)
    PRANA_HIP(hipMemcpyAsync(logits_host, ws.logits.p, n * c.vocab_size * 4, hipMemcpyDeviceToHost, s));
  PRANA_HIP(hipStreamSynchronize(s));
  return kOk;
}

// ------------------------------------------------------------------ generation
namespace {
bool is_stop(uint32_t t, const uint32_t* stops, size_t n) {
  for (size_t i = 0; i < n; i++)
    if (stops[i] == t) return true;
  return false;
}
}  // namespace

// generate (infer.rs:696-771), greedy. The sampled id goes from the device
// argmax straight into the next step's embedding input; the host reads the
// ids back a chunk of steps at a time to emit them and test the stop set.
int Model::generate(const uint32_t* prompt, size_t p, size_t steps, const uint32_t* stops, size_t n_stops,
                    uint32_t* out, size_t* n_out, prana_gen_stats* st) {
  PRANA_CHECK(p > 0, "prompt encoded to zero tokens");
  hipStream_t s = ctx().stream;
  size_t max_pos = std::min(c.seq_len, p + steps);
  Cache cache;
  int rc = cache.create(*this, max_pos);
  if (rc) return rc;
  if ((rc = check_tokens(prompt, p))) return rc;
  double t0 = now_s();
  uint32_t token = prompt[0];
  size_t start_pos = 0, generated = 0;
  if (p > 1 && p <= max_pos) {
    if ((rc = prefill(cache, prompt, p - 1))) return rc;
    start_pos = p - 1;
    token = prompt[p - 1];
  }
  double t1 = now_s();
  if (start_pos == p - 1) {
    // The prompt is in the cache: steps at positions p-1 .. max_pos-2 each
    // produce one token. They run as decode() chunks (one host round trip
    // per chunk); the chunk is scanned for stop ids, and tokens after a stop
    // are discarded (greedy steps do not depend on later ones).
    const size_t total = max_pos - p;
    constexpr size_t kChunk = 16;
    size_t pos = start_pos;
    bool stopped = false;
    while (generated < total && !stopped) {
      const size_t n = std::min(kChunk, total - generated);
      if ((rc = decode(cache, token, pos, n, out + generated))) return rc;
      size_t keep = n;
      for (size_t j = 0; j < n; j++)
        if (is_stop(out[generated + j], stops, n_stops)) {
          keep = j;
          stopped = true;
          break;
        }
      token = out[generated + n - 1];
      generated += keep;
      pos += n;
    }
  }
  bool token_on_device = false;
  for (size_t pos = start_pos; start_pos != p - 1 && pos < max_pos; pos++) {
    bool need = pos + 1 >= p && pos + 1 < max_pos;
    if ((rc = forward_dev(cache, token_on_device ? nullptr : &token, nullptr, pos, need, s))) return rc;
    if (pos + 1 >= max_pos) break;
    uint32_t next;
    if (pos + 1 < p) {
      next = prompt[pos + 1];
      token_on_device = false;
    } else {
      if ((rc = launch_argmax(ws.logits.as<float>(), 1, c.vocab_size, ws.tokens.as<uint32_t>(), s))) return rc;
      PRANA_HIP(hipMemcpyAsync(&next, ws.tokens.p, 4, hipMemcpyDeviceToHost, s));
      PRANA_HIP(hipStreamSynchronize(s));
      token_on_device = true;
    }
    if (pos + 1 >= p) {
      if (is_stop(next, stops, n_stops)) break;
      out[generated++] = next;
    }
    token = next;
  }
  PRANA_HIP(hipStreamSynchronize(s));
  double t2 = now_s();
  if (n_out) *n_out = generated;
  if (st) {
    st->prompt_tokens = p;
    st->generated_tokens = generated;
    st->proposed = st->accepted = 0;
    st->seconds = t2 - t0;
    st->prefill_seconds = t1 - t0;
    st->decode_seconds = t2 - t1;
  }
  return kOk;
}

// generate (infer.rs:696-771) with Sampler::sample for the sampled
// positions. The steps at positions p-1 .. max_pos-2 run in chunks: the
// chunk's uniform draws are taken on the host (in the reference's order, one
// per step) and uploaded, every step samples on the device into the token
// stream the next step embeds, and the chunk comes back once. Draws of steps
// after a stop token are given back, so *rng ends where the reference's does.
int Model::generate_sampled(const uint32_t* prompt, size_t p, size_t steps, const uint32_t* stops, size_t n_stops,
                            float temp, uint64_t* rng, uint32_t* out, size_t* n_out, prana_gen_stats* st) {
  if (temp <= 0.0f) return generate(prompt, p, steps, stops, n_stops, out, n_out, st);  // greedy: no draws
  PRANA_CHECK(p > 0, "prompt encoded to zero tokens");
  PRANA_CHECK(rng, "sampler state missing");
  hipStream_t s = ctx().stream;
  const size_t max_pos = std::min(c.seq_len, p + steps);
  Cache cache;
  int rc = cache.create(*this, max_pos);
  if (rc) return rc;
  if ((rc = check_tokens(prompt, p))) return rc;
  const double t0 = now_s();
  if (p > 1 && p <= max_pos && (rc = prefill(cache, prompt, p - 1))) return rc;
  const double t1 = now_s();
  size_t generated = 0;
  // with p > max_pos every position is teacher-forced and nothing is sampled
  if (p <= max_pos && max_pos > p) {
    constexpr size_t kChunk = 16;
    const size_t V = c.vocab_size;
    if ((rc = ensure_ws(1, cache.len, false))) return rc;
    if ((rc = ws.sampling.ensure((2 * V + kChunk) * 4))) return rc;
    if ((rc = ws.stream_out.ensure(std::max<size_t>((kChunk + 1) * 4, kStreamFloorIds * 4)))) return rc;
    float* scaled = ws.sampling.as<float>();
    float* probs = scaled + V;
    float* draws_dev = probs + V;
    uint32_t* ids = ws.stream_out.as<uint32_t>();
    const size_t total = max_pos - p;
    size_t pos = p - 1, done = 0;
    uint32_t token = prompt[p - 1];
    float draws[kChunk];
    uint32_t got[kChunk];
    while (done < total) {
      const size_t n = std::min(kChunk, total - done);
      const uint64_t state0 = *rng;
      for (size_t j = 0; j < n; j++) draws[j] = xorshift_next_f32(rng);
      PRANA_HIP(hipMemcpyAsync(draws_dev, draws, n * 4, hipMemcpyHostToDevice, s));
      if ((rc = launch_decode_seed(nullptr, 0, token, ids, nullptr, s))) return rc;
      for (size_t j = 0; j < n; j++) {
        if ((rc = forward_dev(cache, nullptr, ids + j, pos + j, true, s))) return rc;
        if ((rc = launch_sample(ws.logits.as<float>(), V, temp, draws_dev, static_cast<int>(j), 0.0f, scaled, probs,
                                ids + j + 1, s)))
          return rc;
      }
      PRANA_HIP(hipMemcpyAsync(got, ids + 1, n * 4, hipMemcpyDeviceToHost, s));
      PRANA_HIP(hipStreamSynchronize(s));
      size_t keep = n;
      for (size_t j = 0; j < n; j++)
        if (is_stop(got[j], stops, n_stops)) {
          keep = j;
          break;
        }
      for (size_t j = 0; j < keep; j++) out[generated + j] = got[j];
      generated += keep;
      if (keep < n) {  // the stop token's draw was the last one the reference takes
        *rng = state0;
        for (size_t j = 0; j <= keep; j++) (void)xorshift_next_f32(rng);
        break;
      }
      token = got[n - 1];
      pos += n;
      done += n;
    }
  }
  PRANA_HIP(hipStreamSynchronize(s));
  const double t2 = now_s();
  if (n_out) *n_out = generated;
  if (st) {
    st->prompt_tokens = p;
    st->generated_tokens = generated;
    st->proposed = st->accepted = 0;
    st->seconds = t2 - t0;
    st->prefill_seconds = t1 - t0;
    st->decode_seconds = t2 - t1;
  }
  return kOk;
}

// generate_speculative (infer.rs:581-690), greedy.
int generate_speculative(Model& target, Model& draft, const uint32_t* prompt, size_t p, size_t steps, size_t k,
                         const uint32_t* stops, size_t n_stops, uint32_t* out, size_t* n_out, prana_gen_stats* st) {
  PRANA_CHECK(k >= 1, "draft length must be >= 1");
  PRANA_CHECK(target.c.vocab_size == draft.c.vocab_size, "draft and target must share a vocabulary");
  PRANA_CHECK(p > 0, "prompt encoded to zero tokens");
  hipStream_t s = ctx().stream;
  size_t V = target.c.vocab_size;
  size_t max_pos = std::min(target.c.seq_len, p + steps);
  Cache tc, dc;
  int rc = tc.create(target, max_pos);
  if (!rc) rc = dc.create(draft, max_pos);
  if (rc) return rc;
  if ((rc = target.check_tokens(prompt, p))) return rc;
  double t0 = now_s();
  if (p > 1) {
    if ((rc = target.prefill(tc, prompt, p - 1))) return rc;
    if ((rc = draft.prefill(dc, prompt, p - 1))) return rc;
  }
  double t1 = now_s();
  size_t pos = p - 1, generated = 0, proposed = 0, accepted = 0;
  uint32_t last = prompt[p - 1];
  // Rounds stay on the device: the draft's greedy steps write [last, drafts]
  // to its token stream, the target verifies that stream in place, and the
  // accept walk runs on the device; the host reads back once per round the
  // emitted tokens and the counts, which set the next round's positions.
  DevBuf stops_dev, round;
  if ((rc = stops_dev.alloc(std::max<size_t>(n_stops, 1) * 4))) return rc;
  if (n_stops) PRANA_HIP(hipMemcpy(stops_dev.p, stops, n_stops * 4, hipMemcpyHostToDevice));
  if ((rc = round.alloc((k + 4) * 4))) return rc;
  std::vector<int> res(k + 4);
  bool done = false;
  while (!done && pos + 1 < max_pos) {
    const size_t budget = std::min(max_pos - 1 - pos, k);
    uint32_t* ids = nullptr;
    if ((rc = draft.decode_stream(dc, last, pos, budget, s, &ids))) return rc;
    proposed += budget;
    if ((rc = target.batch_dev_ids(tc, ids, budget + 1, pos, 2, s))) return rc;
    if ((rc = target.logits_pass(budget + 1, s))) return rc;
    uint32_t* tnext = target.ws.argmax.as<uint32_t>();
    if ((rc = launch_argmax(target.ws.logits.as<float>(), budget + 1, V, tnext, s))) return rc;
    if ((rc = launch_spec_accept(ids + 1, tnext, static_cast<int>(budget), stops_dev.as<uint32_t>(),
                                 static_cast<int>(n_stops), generated, steps, pos, max_pos, round.as<int>(), s)))
      return rc;
    PRANA_HIP(hipMemcpyAsync(res.data(), round.p, (budget + 4) * 4, hipMemcpyDeviceToHost, s));
    PRANA_HIP(hipStreamSynchronize(s));
    const size_t n_emit = static_cast<size_t>(res[0]);
    const uint32_t* toks = reinterpret_cast<const uint32_t*>(res.data() + 3);
    for (size_t i = 0; i < n_emit; i++) out[generated + i] = toks[i];
    generated += n_emit;
    pos += n_emit;
    accepted += static_cast<size_t>(res[1]);
    if (n_emit) last = toks[n_emit - 1];
    done = res[2] != 0;
  }
  double t2 = now_s();
  if (n_out) *n_out = generated;
  if (st) {
    st->prompt_tokens = p;
    st->generated_tokens = generated;
    st->proposed = proposed;
    st->accepted = accepted;
    st->seconds = t2 - t0;
    st->prefill_seconds = t1 - t0;
    st->decode_seconds = t2 - t1;
  }
  return kOk;
}

}  // namespace prana
