// Device-resident Model / KvCache (prana-model checkpoint.rs:32-265,
// infer.rs:25-45) and the forward passes.
#pragma once

#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/prana_hip.h"
#include "runtime.h"

namespace prana {

struct Model;

enum LayerMat { kWq = 0, kWk, kWv, kWo, kW1, kW2, kW3 };
enum LayerVec { kRmsAtt = 0, kRmsFfn, kBq, kBk, kBv };

struct Layer {
  std::unique_ptr<Mat> w[7];
  DevBuf vec[5];
  bool has[5] = {false, false, false, false, false};
};

// KvCache::with_len: per layer K then V, each [len][kv_dim] f16, one allocation.
struct Cache {
  size_t len = 0, kv_dim = 0, n_layers = 0;
  size_t kcap = 0;  // K layout (kcache_index): len for 64- or 128-wide heads (8-dim pieces), else 0 (rows)
  DevBuf buf;
  int create(const Model& m, size_t positions);
  uint16_t* k(size_t l) const;
  uint16_t* v(size_t l) const;
};

// Per-model scratch for the passes (single stream; grown on demand).
struct Workspace {
  size_t cap_tok = 0;
  DevBuf x, xb, q, k, v, attn, gate, up, logits;
  DevBuf qa, sa, sums;  // quantized activations of the current GEMV input
  DevBuf hq, hsa, hsum;  // quantized MLP hidden state (input of the down projection)
  DevBuf scratch;       // attention scores
  DevBuf tokens, argmax;
  DevBuf stream_out;  // device-side token stream of decode()
  DevBuf step_state;  // {position, step} of a replayed decode step
  DevBuf sampling;    // scaled logits, probabilities and uniform draws of sampled steps
  DevBuf xch;         // norm handoff words of the split gate|up launch (NormIn::xch)
  size_t gen = 0;     // bumped whenever a buffer above moves
};

// decode()'s captured step: embed, layers, head, argmax and the state
// advance, replayed once per token (one per attention path: the kernels read
// the position from device memory, the host position at capture chooses the
// path). Valid while the buffers it was captured with stay where they are.
struct StepGraph {
  hipGraph_t graph = nullptr;  // kept alive as long as its executable form
  hipGraphExec_t exec = nullptr;
  const void* cache_buf = nullptr;
  size_t cache_len = 0, ws_gen = 0;
  const void* ids = nullptr;
  void reset();
  ~StepGraph() { reset(); }
};

// Optional per-launch timing of the model's GEMVs (HIP events on the stream
// the GEMV runs on), for roofline accounting.
// Each timed GEMV launch carries its own dispatch timestamps (no extra
// markers on the stream); events come from a pool that grows on demand and
// is reused across collections. Launches that are not a single decode-GEMV
// dispatch are counted in `skipped` and not timed. With period P only every
// P-th launch is timed (129 GEMV launches per 7B token, so the sampled
// positions rotate over all shapes).
struct GemvProfile {
  struct Rec {
    size_t ev;  // index of the first of two pool events
    size_t bytes, n_tok;
  };
  bool on = false;
  size_t period = 1;  // time every period-th GEMV launch
  size_t calls = 0;
  std::vector<hipEvent_t> pool;
  size_t used = 0;
  std::vector<Rec> pending;
  double seconds = 0.0, bytes = 0.0;
  size_t launches = 0, skipped = 0;
  struct Shape {
    size_t launches = 0;
    double seconds = 0.0;
  };
  std::map<size_t, Shape> shapes;  // by weight bytes per launch
  int next_pair(size_t* ev);
  int collect();
};
GemvProfile& gemv_profile();

struct Model {
  prana_config c{};
  std::vector<Layer> layers;
  DevBuf rms_final;
  bool has_rms_final = false;
  std::unique_ptr<Mat> emb;   // packed (Q4_0/Q4_K/Q6_K) or dense f32 table
  std::unique_ptr<Mat> wcls;  // null => classifier tied to emb
  DevBuf rope;                // float2 [seq_len][head_dim/2] (cos, sin)
  bool finalized = false;
  Workspace ws;
  StepGraph step_graph[2];  // windows below / on the split attention path
  // While a decode step is captured: the position the step's RoPE and
  // attention read (device memory) instead of the host-side one.
  const int* pos_dev = nullptr;

  int set_tensor(const std::string& name, int ggml_type, const uint64_t* dims, int n_dims, const void* bytes,
                 size_t nbytes);
  int set_q8(const std::string& name, size_t rows, size_t cols, const int8_t* q, const float* scales);
  std::unique_ptr<Mat>* mat_slot(const std::string& name, size_t* cols, size_t* rows);
  int finalize();
  size_t stream_bytes() const;
  const Mat& head() const;

  int ensure_ws(size_t n_tok, size_t ctx_cap, bool prefill_attn);
  int check_tokens(const uint32_t* t, size_t n);
  // hset: read the quantized MLP hidden state (ws.hq) instead of ws.qa.
  int apply(const Mat& w, size_t n, const float* xf, const GemvOut& o, hipStream_t s, bool hset = false);
  // Several matrices over the same input (Q|K|V); runs of equal kind share a launch.
  // rk: one-token Q|K|V glue (rope, cache rows) the launch may fold in;
  // *fused tells whether it did.
  // norm: one token whose rmsnorm the single launch computes itself (the
  // caller has checked gemv_norm_fusable on all n_mats matrices).
  int apply_multi(const Mat* const* w, const GemvOut* o, int n_mats, size_t n, const float* xf, hipStream_t s,
                  const RopeKv* rk = nullptr, bool* fused = nullptr, const NormIn* norm = nullptr);
  // gate/up projections with the activation and the down projection's
  // quantization fused when both share a kind; h lands in ws.gate (f32) and
  // ws.hq/hsa/hsum (quantized).
  // norm: one token whose rmsnorm the launch computes (gemv_norm_act_fusable).
  // dense_h: the down projection reads the f32 h (a dense matrix), not only its quantized form
  int apply_gate_up(const Mat& gate, const Mat& up, size_t n, hipStream_t s, const NormIn* norm = nullptr,
                    bool dense_h = true);
  template <class F>
  int timed(size_t bytes, size_t n, hipStream_t s, F&& launch);
  int norm_quant(const float* x, const DevBuf& w, size_t n, hipStream_t s);
  int embed_tokens(const uint32_t* dev_ids, size_t n, hipStream_t s);
  int layers_pass(Cache& cache, size_t n, size_t pos0, int mode, hipStream_t s);
  int logits_pass(size_t n, hipStream_t s);

  // The token comes from host_token when given, else from dev_token (a
  // device id), else from ws.tokens[0].
  int forward_dev(Cache& cache, const uint32_t* host_token, const uint32_t* dev_token, size_t pos,
                  bool need_logits, hipStream_t s);
  int batch_dev(Cache& cache, const uint32_t* tokens, size_t n, size_t pos0, int mode, hipStream_t s);

  int forward(Cache& cache, uint32_t token, size_t pos, bool need_logits, float* logits_host);
  int decode(Cache& cache, uint32_t token, size_t pos, size_t n_steps, uint32_t* out);
  // decode's steps, queued on s: ids[0] = token, ids[1..n_steps] the greedy
  // stream (device memory, *ids); nothing is copied back or awaited.
  int decode_stream(Cache& cache, uint32_t token, size_t pos, size_t n_steps, hipStream_t s, uint32_t** ids);
  // batch_dev over token ids already in device memory (argmax outputs).
  int batch_dev_ids(Cache& cache, const uint32_t* dev_tokens, size_t n, size_t pos0, int mode, hipStream_t s);
  // Capture (or reuse) the replayable decode step for the attention path of
  // position pos, writing its tokens to ids.
  int step_graph_ready(Cache& cache, size_t pos, uint32_t* ids, hipStream_t s, hipGraphExec_t* exec);
  int prefill(Cache& cache, const uint32_t* tokens, size_t n);
  int forward_batch(Cache& cache, const uint32_t* tokens, size_t n, size_t pos0, float* logits_host);
  int generate(const uint32_t* prompt, size_t p, size_t steps, const uint32_t* stops, size_t n_stops,
               uint32_t* out, size_t* n_out, prana_gen_stats* st);
  // generate with a temperature Sampler (sampler.rs): *rng is its xorshift
  // state and advances by one draw per sampled position, as the reference's.
  int generate_sampled(const uint32_t* prompt, size_t p, size_t steps, const uint32_t* stops, size_t n_stops,
                       float temp, uint64_t* rng, uint32_t* out, size_t* n_out, prana_gen_stats* st);
};

int check_config(const prana_config& c);

// Whether a profiling tool is loaded into the process, and whether decode
// replays its captured step (not with PRANA_DECODE_GRAPH=0 or a tool present).
bool profiler_tool_present();
bool decode_graphs_enabled();

int generate_speculative(Model& target, Model& draft, const uint32_t* prompt, size_t p, size_t steps, size_t k,
                         const uint32_t* stops, size_t n_stops, uint32_t* out, size_t* n_out, prana_gen_stats* st);

}  // namespace prana

struct prana_model {
  prana::Model m;
};
struct prana_cache {
  prana::Cache c;
  prana_model* owner;
};
struct prana_mat {
  prana::Mat m;
};
