/*
 * prana_oracle.h — CPU restatement of the reference's *scalar tier* and model
 * loop, used ONLY as the checker (tests/, __graft_entry__.smoke(), and the
 * cpu_baseline leg of bench.py). Nothing in the shipped library links it.
 *
 * Every function restates, in C, the arithmetic order of a reference
 * function (Rust, pariharshyamu/Prana); each definition in prana_oracle.c cites
 * the file:line it follows. Compiled with -O2 -ffp-contract=off and no
 * fast-math so f32 expressions evaluate exactly as Rust evaluates them
 * (no FMA contraction, IEEE div/sqrt, round-half-away-from-zero).
 *
 * Transcendentals come from the host libm (glibc), exactly as the Rust
 * reference reaches them through f32::{exp, powf, sin, cos, tanh}.
 */
#ifndef PRANA_ORACLE_H
#define PRANA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------- f16 (prana-kernels/src/lib.rs:57-113) ---------------- */
float po_f16_to_f32(uint16_t h);
uint16_t po_f32_to_f16(float x);
/* Bulk forms (results written as raw bits: no float->double hop that would
 * quiet signalling NaNs on the way to a caller). */
void po_f16_to_f32_n(const uint16_t *h, size_t n, float *out);
void po_f32_to_f16_n(const float *x, size_t n, uint16_t *out);

/* Bulk host-libm expf over [base, base+n) f32 bit patterns (the reference's
 * f32::exp is glibc expf), threaded; for exhaustive device comparisons. */
void po_expf_bits(uint32_t base, size_t n, float *out, int threads);
/* tanhf (norms.rs:40, f32::tanh -> glibc) over the same kind of range. */
void po_tanhf_bits(uint32_t base, size_t n, float *out, int threads);

/* ---------------- timed tier (cpu_tier.c; bench.py's cpu_baseline only) ---------------- */
/* tier 1: the reference's runtime-selected SIMD dots (simd_x86.rs) on its
 * persistent pool (pool.rs) with threads workers (<= 0: min(nproc, 8));
 * tier 0: the scalar tier, the parity oracle (default). Returns the pool size. */
int po_set_tier(int tier, int threads);
const char *po_tier_name(void);

/* ---------------- activations (matmul.rs:105-127) ---------------- */
/* a[k] -> q[k] (i8), scales[k/32] (f32), sums[k/32] (i32). k % 32 == 0. */
void po_quantize_acts(const float *a, size_t k, int8_t *q, float *scales, int32_t *sums);

/* quantize_q8 (matmul.rs:61-84): f32 weights -> i8 + per-32 f32 scale. */
void po_quantize_q8(size_t rows, size_t cols, const float *w, int8_t *q, float *scales);

/* ---------------- row dots (scalar tier) ---------------- */
float po_dot_f32(const float *a, const float *b, size_t n);                       /* matmul.rs:377-391 */
float po_dot_q8_q8(const int8_t *qa, const float *sa, const int8_t *qw,
                   const float *sw, size_t groups);                              /* matmul.rs:395-406 */
float po_dot_q40_q8(const int8_t *qa, const float *sa, const int32_t *suma,
                    const uint8_t *row, const float *ds, size_t nblocks);        /* kquant.rs:240-252 */
float po_dot_q4k_q8(const int8_t *qa, const float *sa, const int32_t *suma,
                    const uint8_t *row, const float *ds, size_t nblocks);        /* kquant.rs:257-282 */
float po_dot_q6k_q8(const int8_t *qa, const float *sa, const int32_t *suma,
                    const uint8_t *row, const float *ds, size_t nblocks);        /* kquant.rs:287-318 */

/* ---------------- block decoders (kquant.rs:39-112) ---------------- */
void po_dequant_q40_block(const uint8_t *b, float *out32);
void po_q4k_scale_min(int j, const uint8_t *s, float *sc, float *m);
void po_dequant_q4k_block(const uint8_t *b, float *out256);
void po_dequant_q6k_block(const uint8_t *b, float *out256);

/* ---------------- matrices (Linear / QuantMatrix / KQuantMatrix) ---------------- */
enum po_kind {
  PO_F32 = 0,   /* Linear::F32 (checkpoint.rs:77) */
  PO_Q8 = 1,    /* Linear::Q8 / QuantMatrix (matmul.rs:21-28): i8 + f32 scale */
  PO_Q4_0 = 2,  /* KQuantMatrix Q40 */
  PO_Q4_K = 3,  /* KQuantMatrix Q4K */
  PO_Q6_K = 4,  /* KQuantMatrix Q6K */
};
/* ggml tensor type ids (gguf.rs:33-38) */
enum po_ggml { PO_GGML_F32 = 0, PO_GGML_F16 = 1, PO_GGML_Q4_0 = 2, PO_GGML_Q8_0 = 8,
               PO_GGML_Q4_K = 12, PO_GGML_Q6_K = 14 };

typedef struct po_mat po_mat;

po_mat *po_mat_f32(size_t rows, size_t cols, const float *w);
po_mat *po_mat_q8_parts(size_t rows, size_t cols, const int8_t *q, const float *scales); /* from_parts */
/* Build from raw ggml bytes exactly as gguf.rs:271-305 `Gguf::linear` does
 * (Q8_0 -> QuantMatrix with f16 scales decoded; Q4_0/Q4_K/Q6_K -> packed
 * KQuantMatrix with hoisted f32 scales; F32/F16 -> dense). Returns NULL if the
 * shape is not block-aligned. */
po_mat *po_mat_from_ggml(int ggml_type, size_t rows, size_t cols, const void *raw, size_t nbytes);
void po_mat_free(po_mat *m);
size_t po_mat_rows(const po_mat *m);
size_t po_mat_cols(const po_mat *m);
int po_mat_kind(const po_mat *m);

/* Linear::apply for n tokens (matmul_f32 / matmul_q8_f32 / matmul_kquant_f32): out[n][rows]. */
void po_matmul(const po_mat *m, const float *a, size_t n_tokens, float *out);
/* Linear::apply_prefill: quantized rows given (one QuantActs per token), out[n][rows]. */
void po_matmul_prefill(const po_mat *m, const float *xs, const int8_t *q, const float *sa,
                       const int32_t *sums, size_t n_tokens, float *out);
/* One element: weight row r against one quantized (or dense) activation row. */
float po_mat_row_dot(const po_mat *m, const float *x, const int8_t *q, const float *sa,
                     const int32_t *sums, size_t r);
/* Per-block integer sums of row r (the exact i32 part of each term), G values
 * (Q6_K: 16 per super-block, one per 16-element sub-block). Returns count. */
size_t po_mat_row_block_isums(const po_mat *m, const int8_t *q, const int32_t *sums, size_t r,
                              int32_t *isums);
/* Dequantize row r (Embedding::row / KQuantMatrix::dequantize_row, or the
 * dense copy). out[cols]. */
void po_mat_row_f32(const po_mat *m, size_t r, float *out);

/* Threads used by the row-parallel drivers (results are order-independent
 * per row, so this never changes a bit). 0 = serial. */
void po_set_threads(int n);

/* ---------------- norms (norms.rs:9-56) ---------------- */
void po_rmsnorm(const float *x, const float *w, size_t rows, size_t dim, float eps, float *out);
void po_silu(float *x, size_t n);
void po_gelu_tanh(float *x, size_t n);
void po_softmax(const float *in, size_t n, float *out);

/* ---------------- RoPE (attention.rs:59-121) ---------------- */
void po_rope(float *x, size_t seq, size_t n_heads, size_t head_dim, float theta);
void po_rope_interleaved(float *x, size_t len, size_t pos, size_t head_dim, float theta);
void po_rope_neox(float *x, size_t len, size_t pos, size_t head_dim, float theta);

/* ---------------- attention (attention.rs:47-333) ---------------- */
void po_f16_kv_write(uint16_t *cache, size_t first_row, size_t kv_stride, const float *src, size_t n);
void po_attention_decode(const float *q, const uint16_t *kc, const uint16_t *vc, size_t pos,
                         size_t n_heads, size_t n_kv_heads, size_t head_dim, float *out);
void po_attention_verify(const float *q, const uint16_t *kc, const uint16_t *vc, size_t pos0,
                         size_t seq, size_t n_heads, size_t n_kv_heads, size_t head_dim, float *out);
void po_attention(const float *q, const float *k, const float *v, size_t seq, size_t n_heads,
                  size_t n_kv_heads, size_t head_dim, float *out);

/* ---------------- model (checkpoint.rs / infer.rs) ---------------- */
typedef struct po_config {
  size_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len, head_dim;
  float rope_theta, norm_eps, emb_scale;
  int rope_neox;  /* 0 interleaved, 1 NeoX */
  int act;        /* 0 silu, 1 gelu_tanh */
} po_config;

/* Which layer tensor (Layer fields, checkpoint.rs:192-206). */
enum po_slot { PO_WQ = 0, PO_WK, PO_WV, PO_WO, PO_W1, PO_W2, PO_W3,
               PO_RMS_ATT, PO_RMS_FFN, PO_BQ, PO_BK, PO_BV };

typedef struct po_model po_model;
typedef struct po_cache po_cache;

po_model *po_model_new(const po_config *cfg);
void po_model_free(po_model *m);
/* Ownership of `mat` passes to the model. */
void po_model_set_linear(po_model *m, size_t layer, int slot, po_mat *mat);
void po_model_set_vec(po_model *m, size_t layer, int slot, const float *v, size_t n);
void po_model_set_rms_final(po_model *m, const float *v, size_t n);
/* Token embedding from raw ggml bytes (gguf.rs:309-326: Q4_0/Q4_K/Q6_K stay
 * packed, anything else is dequantized to an f32 table). */
int po_model_set_embedding(po_model *m, int ggml_type, const void *raw, size_t nbytes);
/* Untied classifier (wcls). Without it the classifier is tied to tok_emb. */
void po_model_set_wcls(po_model *m, po_mat *mat);

po_cache *po_cache_new(const po_model *m, size_t positions);   /* KvCache::with_len */
void po_cache_free(po_cache *c);
const uint16_t *po_cache_k(const po_cache *c, size_t layer);
const uint16_t *po_cache_v(const po_cache *c, size_t layer);
size_t po_cache_len(const po_cache *c);

/* forward_impl (infer.rs:142-211). logits may be NULL when need_logits = 0. */
void po_forward(const po_model *m, po_cache *c, uint32_t token, size_t pos, int need_logits, float *logits);
void po_prefill(const po_model *m, po_cache *c, const uint32_t *tokens, size_t n);          /* infer.rs:220-286 */
void po_forward_batch(const po_model *m, po_cache *c, const uint32_t *tokens, size_t n,
                      size_t pos0, float *logits);                                          /* infer.rs:296-374 */
uint32_t po_argmax(const float *v, size_t n);                                               /* infer.rs:560-568 */

typedef struct po_gen_stats {
  size_t prompt_tokens, generated_tokens, proposed, accepted;
} po_gen_stats;
/* Greedy `generate` (infer.rs:696-771). `stops` = ids for which is_stop holds
 * (tokenizer.rs:174-176); generated ids are written to out (capacity steps). */
size_t po_generate(const po_model *m, const uint32_t *prompt, size_t p, size_t steps,
                   const uint32_t *stops, size_t n_stops, uint32_t *out, po_gen_stats *st);
/* Greedy speculative decode (infer.rs:581-690). */
/* Sampler (sampler.rs:6-71): xorshift64* RNG, bucket walk, sample, and
 * generate driven by a sampler. */
uint64_t po_xorshift_seed(uint64_t seed);
float po_xorshift_next_f32(uint64_t *state);
uint32_t po_sample_pick(const float *probs, size_t n, float r);
uint32_t po_sampler_sample(float temp, uint64_t *state, const float *logits, size_t n);
size_t po_generate_sampled(const po_model *m, const uint32_t *prompt, size_t p, size_t steps, const uint32_t *stops,
                           size_t n_stops, float temp, uint64_t *state, uint32_t *out);
size_t po_generate_speculative(const po_model *target, const po_model *draft, const uint32_t *prompt,
                               size_t p, size_t steps, size_t k, const uint32_t *stops, size_t n_stops,
                               uint32_t *out, po_gen_stats *st);

#ifdef __cplusplus
}
#endif
#endif
