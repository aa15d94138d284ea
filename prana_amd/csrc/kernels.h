// Device-side matrix descriptor and the host launch functions of every kernel.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace prana {

// Device storage kinds. Byte layouts (all rows contiguous, row-major):
//   F32  : float [rows][cols]
//   Q8F  : int8 [rows][cols] + float scale [rows][cols/32]      (QuantMatrix, f32 scales)
//   Q8_0 : int8 [rows][cols] + f16 d [rows][cols/32]            (GGUF Q8_0, 34 B / 32)
//   Q4_0 : u8 [rows][cols/32][16] + f16 d [rows][cols/32]       (GGUF Q4_0, 18 B / 32)
//   Q4_K : u8 [rows][cols/256][144]                            (GGUF block, unchanged)
//   Q6_K : u8 [rows][cols/256][208] (ql|qh|scales) + f16 d [rows][cols/256]  (210 B / 256)
// The split keeps every quant run 16-byte aligned for 128-bit loads; the
// byte count per block is the GGUF one, so roofline bytes are unchanged.
enum Kind : int { kKindF32 = 0, kKindQ8F = 1, kKindQ8_0 = 2, kKindQ4_0 = 3, kKindQ4_K = 4, kKindQ6_K = 5 };

// f16 K cache layouts. kcap == 0: rows [pos][kv_dim] (the reference's, and
// the C entry points' caller-owned caches). kcap > 0 (a model's own cache,
// 64- or 128-wide heads): pieces of 8 consecutive dims, position-major,
// [kv_dim/8][kcap][8], so the attention kernels' lanes (one position each)
// read a piece of a head with one coalesced wave load. Index of element
// (position t, kv dim d):
__host__ __device__ inline size_t kcache_index(size_t t, size_t d, size_t kv_dim, size_t kcap) {
  return kcap ? ((d >> 3) * kcap + t) * 8 + (d & 7) : t * kv_dim + d;
}

struct DevMat {
  int kind;
  size_t rows, cols;
  const uint8_t* qs;  // quants (or f32 weights)
  const void* sc;     // per-block scales (nullptr for Q4_K)
};

// Algorithmic bytes of a weight matrix (what a GEMV must stream).
size_t devmat_bytes(const DevMat& m);

// ---- elementwise.hip
int launch_quantize_acts(const float* x, size_t n_rows, size_t k, int8_t* q, float* sa, int* sums, hipStream_t s);
int launch_rmsnorm(const float* x, const float* w, size_t rows, size_t dim, float eps, float* out, int8_t* q,
                   float* sa, int* sums, hipStream_t s);
int launch_act_mul(float* g, const float* u, size_t n, int gelu, int8_t* q, float* sa, int* sums, hipStream_t s);
int launch_softmax(const float* in, size_t rows, size_t n, float* out, hipStream_t s);
int launch_add(float* x, const float* y, size_t n, size_t period, hipStream_t s);
int launch_rope(float* x, size_t n_rows, size_t row_len, size_t row_stride, size_t hd, const float2* table,
                size_t pos0, int neox, hipStream_t s);
int launch_kv_write(uint16_t* cache, size_t first_row, size_t kv_stride, const float* src, size_t n, hipStream_t s);
// n token rows at positions pos0..pos0+n-1: RoPE of q and k in place, and
// the f16 cache rows of k and v.
int launch_rope_kv_rows(float* q, float* k, const float* v, size_t n, size_t q_dim, size_t kv_dim, size_t hd,
                        const float2* table, int neox, uint16_t* kc, uint16_t* vc, size_t kcap, size_t pos0,
                        hipStream_t s);
int launch_rope_kv(float* q, float* k, const float* v, size_t q_dim, size_t kv_dim, size_t hd, const float2* table,
                   int neox, uint16_t* kc, uint16_t* vc, size_t kcap, const int* pos_dev, size_t pos_host,
                   hipStream_t s);
int launch_f32_to_f16(const float* in, size_t n, uint16_t* out, hipStream_t s);
int launch_f16_to_f32(const uint16_t* in, size_t n, float* out, hipStream_t s);
int launch_expf(const float* in, size_t n, float* out, hipStream_t s);
int launch_tanhf(const float* in, size_t n, float* out, hipStream_t s);
int launch_expf_bits(uint32_t base, uint32_t n, float* out, hipStream_t s);
int launch_argmax(const float* v, size_t rows, size_t n, uint32_t* out, hipStream_t s);
int launch_embed(const DevMat& m, const uint32_t* tokens, size_t n, float scale, float* out, hipStream_t s);
// state = {position, step} in device memory: ids[step + 1] = tok[0], then
// position and step advance by one (the tail of a replayed decode step).
int launch_decode_advance(int* state, const uint32_t* tok, uint32_t* ids, hipStream_t s);
// state = {pos, 0}, ids[0] = token, tok0[0] = token (each pointer optional).
int launch_decode_seed(int* state, int pos, uint32_t token, uint32_t* ids, uint32_t* tok0, hipStream_t s);

// One speculative round's accept walk (infer.rs:648-681): drafts[0..budget),
// target argmaxes tnext[0..budget]; res = {emitted, accepted, done, tokens...}.
int launch_spec_accept(const uint32_t* drafts, const uint32_t* tnext, int budget, const uint32_t* stops, int n_stops,
                       size_t generated, size_t steps, size_t pos, size_t max_pos, int* res, hipStream_t s);

// ---- sampler.hip
// Sampler::sample's bucket walk (sampler.rs:29-36) over device probabilities:
// the first i with (r -= p[i]) <= 0, else n - 1; r from rs[r_index] when rs
// is non-null, else r_host. One 1024-lane workgroup, exact f32 order.
int launch_sample_pick(const float* probs, size_t n, const float* rs, int r_index, float r_host, uint32_t* out,
                       hipStream_t s);
// Sampler::sample (sampler.rs:22-39): argmax for temp <= 0, else logits /
// temp -> scaled, softmax -> probs (n floats each), the walk -> out[0].
int launch_sample(const float* logits, size_t n, float temp, const float* rs, int r_index, float r_host,
                  float* scaled, float* probs, uint32_t* out, hipStream_t s);

// XorShift (sampler.rs:51-71): xorshift64* (12, 25, 27, 0x2545F4914F6CDD1D),
// next_f32 = top 24 bits / 2^24; a seed of 0 becomes 1.
inline uint64_t xorshift_seed(uint64_t seed) { return seed ? seed : 1; }
inline float xorshift_next_f32(uint64_t* state) {
  uint64_t x = *state;
  x ^= x >> 12;
  x ^= x << 25;
  x ^= x >> 27;
  *state = x;
  return static_cast<float>((x * 0x2545F4914F6CDD1DULL) >> 40) / static_cast<float>(1ULL << 24);
}

// ---- gemv.hip
// Optional dispatch timestamps for the next decode GEMV launch on this
// thread: when set, the launch records start/stop into these events as part
// of the kernel dispatch itself (hipExtLaunchKernelGGL), then clears them.
struct LaunchEvents {
  hipEvent_t start = nullptr, stop = nullptr;
};
LaunchEvents& launch_events();
// The sampled launch profile's key of the one-launch decode attention kernel
// (the GEMV launches are keyed by the weight bytes they stream).
constexpr size_t kProfileAttentionKey = 1;

// out[t*ldo + r] (mode): 0 = store, 1 = store + bias[r], 2 = out += result
// (the residual add x += o of infer.rs:186-188, 201-203).
struct GemvOut {
  float* out;
  size_t ldo;
  const float* bias;
  int residual;
};
// Token counts up to this use the weight-streaming decode kernel (and
// launch_gemv_act; up to 8 tokens per launch); larger batches use the
// matrix-core kernels.
constexpr size_t kGemvDecodeMaxTokens = 16;
// launch_gemv over block-32 kinds (Q8F, Q8_0, Q4_0) takes batches of
// kGemvSkinnyMinTokens..kGemvSkinnyMaxTokens tokens to the skinny
// matrix-core kernel, except widths of 2, 4, 7 or 14 chunks of 32/64 blocks,
// which keep batches of up to kGemvDecodeMaxTokens on the decode path's
// chunk-major multi-token kernel; smaller batches stay on the decode kernels,
// which also keep the fused Q|K|V and gate|up launches up to
// kGemvDecodeMaxTokens.
constexpr size_t kGemvSkinnyMinTokens = 9;
constexpr size_t kGemvSkinnyMaxTokens = 64;
inline bool gemv_skinny(int kind, size_t n_tok) {
  return (kind == kKindQ8F || kind == kKindQ8_0 || kind == kKindQ4_0) && n_tok >= kGemvSkinnyMinTokens &&
         n_tok <= kGemvSkinnyMaxTokens;
}
// Whether a batch of n_tok tokens over m runs on the skinny matrix-core
// kernel (block-32 kinds; see launch_gemv).
bool gemv_batch_skinny(const DevMat& m, size_t n_tok);
// Batches beyond the skinny kernel's (prefill): gate and up (block-32 kind,
// H = rows % 64 == 0) on the matrix cores in one launch whose epilogue forms
// h = act(g) * u (gelu: gelu_tanh, else silu) and quantizes it into
// (hq, hsa, hsum), as launch_act_mul; h (optional) gets the f32 values.
bool gemm_act_fusable(const DevMat& gate, const DevMat& up, size_t n_tok);
// Verify batches (1..16 tokens) that the skinny matrix-core kernel takes:
// gate|up, h = act(g) * u and h's quantization in one launch (equal
// block-32 matrices, rows % 32 == 0); h (f32, [n_tok][rows]) is optional.
bool gemm_skinny_act_fusable(const DevMat& gate, const DevMat& up, size_t n_tok);
int launch_gemm_skinny_act(const DevMat& gate, const DevMat& up, const int8_t* q, const float* sa, const int* sums,
                           size_t n_tok, int gelu, float* h, int8_t* hq, float* hsa, int* hsum, hipStream_t s);
int launch_gemm_act(const DevMat& gate, const DevMat& up, const int8_t* q, const float* sa, size_t n_tok, int gelu,
                    float* h, int8_t* hq, float* hsa, int* hsum, hipStream_t s);
// Quantized kinds read (q, sa, sums) for n_tok rows; F32 reads x.
int launch_gemv(const DevMat& m, const float* x, const int8_t* q, const float* sa, const int* sums, size_t n_tok,
                const GemvOut& o, hipStream_t s);
// Up to three quantized matrices of one kind sharing the input (fused
// Q|K|V), one launch.
// Decode glue a one-token Q|K|V launch (n = 3: q, k, v rows) can fold into
// its epilogue (infer.rs:169-178): rope q and k at the position, then write k
// and v as the f16 cache row at that position, exactly as launch_rope_kv. The
// launcher sets *fused when it did (kinds, widths and the tile layout allow
// it); otherwise the caller runs launch_rope_kv.
struct RopeKv {
  const float2* table;  // [pos][hd/2] (cos, sin)
  int hd, neox;
  int pos;              // used when pos_dev is null
  const int* pos_dev;
  uint16_t* kc;         // layout kcache_index(.., kcap)
  uint16_t* vc;         // rows
  int kcap;
};
// rmsnorm (norms.rs:9-23) folded into a one-token GEMV launch: every
// workgroup normalises the row x with the weights w itself (the exact
// left-to-right sum of squares, then (x*inv)*w) and quantizes the result into
// its own activation buffer, as launch_rmsnorm followed by the GEMV would.
struct NormIn {
  const float* x;
  const float* w;
  float eps;
  // optional: kNormXchBytes of zeroed, 8-byte-aligned device memory through
  // which the split gate|up launch hands its norm workgroup's factor to the
  // tiles (a 64-bit flag|value word, then one flag word per tile; left zeroed
  // again at the end of each launch; one launch at a time)
  unsigned* xch = nullptr;
  int xch_polls = 0;  // (set by the launch)
};
constexpr size_t kNormXchBytes = 4096;
// Whether launch_gemv_multi can take these matrices with a NormIn (one token):
// block-32 formats, 512 < cols <= 4096, every tile's workgroup resident at once.
bool gemv_norm_fusable(const DevMat* ms, int n);
int launch_gemv_multi(const DevMat* ms, const GemvOut* os, int n, const int8_t* q, const float* sa, const int* sums,
                      size_t n_tok, hipStream_t s, const RopeKv* rk = nullptr, bool* fused = nullptr,
                      const NormIn* norm = nullptr);
// Whether launch_gemv_multi takes these matrices in one launch: same cols and
// either one kind, or two kinds of the same unit width and tile geometry
// (Q4_0 with Q8_0, Q4_K with Q6_K: a Q|K|V whose v is stored in another
// format).
bool gemv_multi_fusable(const DevMat* ms, int n);
// gate|up in one launch with the activation fused: h = act(gate) * up
// (norms.rs:27-41, infer.rs:193-199), quantized for the down projection;
// act 0 = silu, 1 = gelu_tanh. h (f32) is optional when tiles hold whole
// 32-row blocks; otherwise h is required and a quantize_acts launch follows.
// norm: one token whose rmsnorm the launch computes itself (the caller has
// checked gemv_norm_act_fusable); h is then always quantized in the kernel.
bool gemv_norm_act_fusable(const DevMat& gate, const DevMat& up);
int launch_gemv_act(const DevMat& gate, const DevMat& up, int act, const int8_t* q, const float* sa, const int* sums,
                    size_t n_tok, float* h, int8_t* hq, float* hsa, int* hsum, hipStream_t s,
                    const NormIn* norm = nullptr);
// The exact i32 part of every term (debug / bit-exactness entry point):
// isums[t][r][term] with T terms per row (cols/32, or cols/16 for Q6_K).
int launch_block_isums(const DevMat& m, const int8_t* q, const int* sums, size_t n_tok, int* isums, hipStream_t s);
size_t terms_per_row(const DevMat& m);

// ---- attention.hip
// attention_decode / attention_verify (attention.rs:129-160, 296-333) over the
// f16 cache: n_q query rows at positions pos0 + i (pos0 read from pos_dev when
// non-null). scratch >= attention_scratch_floats(n_q, n_heads, ctx_cap)
// floats, ctx_cap >= pos0+n_q (0 = exactly pos0+n_q). Windows of at least
// 2048 rows with 64- or 128-wide heads take the three-launch split path;
// with pos_dev the host-side pos0 still chooses the path, and the launches
// cover any device position up to ctx_cap - n_q.
// Optional quantized copy of an attention output (quantize_acts layout, one
// row of n_heads*hd per query). The launchers fill it in the same pass when
// every workgroup's output dims are whole 32-element blocks and report that
// through *quantized; otherwise the caller quantizes.
struct ActQuant {
  int8_t* q;
  float* sa;
  int* sums;
};
int launch_attention_cache(const float* q, const uint16_t* kc, const uint16_t* vc, size_t pos0, size_t n_q,
                           size_t n_heads, size_t n_kv_heads, size_t hd, float* out, float* scratch, size_t ctx_cap,
                           const int* pos_dev, hipStream_t s, const ActQuant* aq = nullptr,
                           bool* quantized = nullptr, size_t kcap = 0);
// attention (prefill, attention.rs:236-284) over f32 K/V of the window.
// scratch >= attention_scratch_floats(seq, n_heads, seq, false) floats.
// Score scratch a launch needs: cache windows (cache = true) keep the scores
// of every (query row, head) there on the split path; probabilities beyond
// 4096 positions spill from LDS to it on the one-launch path. Also the dim
// slices per head a launch uses.
size_t attention_scratch_floats(size_t n_q, size_t n_heads, size_t ctx_cap, bool cache = true);
// Whether a one-row cache window of `rows` rows takes the split path.
bool attention_split_window(size_t rows, size_t hd);
int attention_dim_slices(size_t n_q, size_t n_heads, size_t hd, size_t elem, bool aligned);
int launch_attention_prefill(const float* q, const float* k, const float* v, size_t seq, size_t n_heads,
                             size_t n_kv_heads, size_t hd, float* out, float* scratch, hipStream_t s,
                             const ActQuant* aq = nullptr, bool* quantized = nullptr);

// ---- flash_decode.hip
// Split-K flash decoding (attention_decode, attention.rs:129-195, for up to 16
// independent sequences; f32 within 1e-4 relative, not bit-exact). The plan
// fixes the tile size and the partial-state scratch a call needs.
struct FlashPlan {
  int iter, rows_per_split, max_splits;
  size_t scratch_floats;
};
FlashPlan flash_decode_plan(const size_t* pos, size_t n_seq, size_t n_heads, size_t n_kv_heads, size_t hd);
// k_caches / v_caches: host arrays of n_seq device pointers ([rows][n_kv_heads*hd]
// f16 each); pos: host array, sequence i attends to rows 0..=pos[i]; q / out:
// device [n_seq][n_heads*hd] f32.
int launch_flash_decode(const float* q, const uint16_t* const* k_caches, const uint16_t* const* v_caches,
                        const size_t* pos, size_t n_seq, size_t n_heads, size_t n_kv_heads, size_t hd, float* out,
                        float* part_buf, size_t part_floats, hipStream_t s);
// The library's fixed partial-state array for the allocation-free entry point
// (kFlashNoAllocFloats floats per GPU): setup looks its device address up
// once per device (that device current); scratch() returns it (null before).
constexpr size_t kFlashNoAllocFloats = size_t{1} << 23;  // 32 MiB
int flash_noalloc_setup(int device);
float* flash_noalloc_scratch(int device);

}  // namespace prana
