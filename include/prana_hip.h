/*
 * prana_hip.h — C ABI of libprana_hip, the MI355X (gfx950) backend for the
 * inference hot path of pariharshyamu/Prana.
 *
 * The reference exposes this path as a Rust crate API (prana-kernels
 * src/lib.rs:35-54, re-exported by prana-model). Each entry point below
 * replaces one of those functions (cited per declaration) on device-resident
 * buffers; the model-level entry points replace prana-model's Model / KvCache /
 * forward / prefill / forward_batch / generate / generate_speculative.
 *
 * Conventions (the reference's own C-ABI idiom, prana-cactus sys.rs:5-9):
 *   - every function returns int: 0 = success, negative = failure;
 *   - prana_last_error() returns a thread-local message for the last failure;
 *   - shape/layout violations (assert! panics in the reference, e.g.
 *     matmul.rs:31-39, kquant.rs:166-169, attention.rs:138-143) come back as
 *     PRANA_ERR_INVALID instead of aborting; nothing throws across the ABI;
 *   - kernel entry points take DEVICE pointers and a stream (NULL = the
 *     library's stream) and are asynchronous; model entry points take host
 *     buffers and synchronise before returning.
 *
 * Numerics: results are bit-identical to the reference's scalar tier
 * (integer block dots exact, f32 folds in the reference's order).
 */
#ifndef PRANA_HIP_H
#define PRANA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PRANA_OK 0
#define PRANA_ERR_INVALID (-1)
#define PRANA_ERR_HIP (-2)
#define PRANA_ERR_NOMEM (-3)
#define PRANA_ERR_UNSUPPORTED (-4)
/* A caller-sized output buffer was too small; the out-length argument holds
 * the size needed (prana-cactus lib.rs:337-354 grow-and-retry idiom). */
#define PRANA_ERR_SHORT_BUFFER (-5)

typedef void *prana_stream_t; /* hipStream_t */

/* ---------------------------------------------------------------- runtime */
/* Thread-local message of the last failure (prana-cactus sys.rs:210
 * cactus_get_last_error idiom). Never NULL. */
const char *prana_last_error(void);
/* Select the device and initialise tables (idempotent). */
int prana_init(int device);
/* Minimal device-memory helpers so any FFI (ctypes, cgo, JNI) can drive the
 * kernel entry points without a HIP binding of its own. */
int prana_device_alloc(size_t bytes, void **out);
int prana_device_free(void *p);
int prana_memcpy_h2d(void *dst, const void *src, size_t bytes);
int prana_memcpy_d2h(void *dst, const void *src, size_t bytes);
/* Device-to-device copy on the library stream (synchronous). No reference
 * counterpart: a plain copy of known size, used to calibrate HBM traffic
 * counters against the GEMVs. */
int prana_memcpy_d2d(void *dst, const void *src, size_t bytes);
int prana_memset_d(void *dst, int value, size_t bytes);
int prana_synchronize(void);

/* ---------------------------------------------------------------- matrices */
/* ggml tensor type ids, as the reference's GGUF loader uses them
 * (gguf.rs:33-38). PRANA_Q8_F32 is QuantMatrix with f32 block scales
 * (matmul.rs:21-28, produced by quantize_q8 / QuantMatrix::from_parts). */
enum prana_ggml_type {
  PRANA_F32 = 0,
  PRANA_F16 = 1,
  PRANA_Q4_0 = 2,
  PRANA_Q8_0 = 8,
  PRANA_Q4_K = 12,
  PRANA_Q6_K = 14,
};

typedef struct prana_mat *prana_mat_t;

/* Upload a rows x cols matrix from GGUF tensor bytes (ggml block layout).
 * Replaces Gguf::linear (gguf.rs:271-305) -> QuantMatrix::from_parts
 * (matmul.rs:34-39) / KQuantMatrix::from_raw (kquant.rs:166-183) / Linear::F32.
 * Q8_0/Q4_0 need cols % 32 == 0, Q4_K/Q6_K cols % 256 == 0. F16 tensors become
 * dense f32 (the reference dequantizes them, gguf.rs:217-221). */
int prana_mat_create(int ggml_type, size_t rows, size_t cols, const void *host_bytes, size_t nbytes,
                     prana_mat_t *out);
/* QuantMatrix::from_parts with f32 scales (matmul.rs:34-39). */
int prana_mat_create_q8(size_t rows, size_t cols, const int8_t *q, const float *scales, prana_mat_t *out);
int prana_mat_destroy(prana_mat_t m);
/* rows, cols, device storage kind and the bytes a GEMV streams. */
int prana_mat_info(prana_mat_t m, size_t *rows, size_t *cols, int *kind, size_t *stream_bytes);

/* ---------------------------------------------------------------- kernels */
/* quantize_acts (matmul.rs:105-127) for n_rows rows of k (k % 32 == 0):
 * q[n_rows*k] i8, scales/sums[n_rows*k/32]. */
int prana_quantize_acts(const float *x, size_t n_rows, size_t k, int8_t *q, float *scales, int32_t *sums,
                        prana_stream_t stream);
/* quantize_q8 (matmul.rs:61-84): a dense f32 weight matrix w[rows*cols]
 * (cols % 32 == 0) to Q8, q[rows*cols] i8 and scales[rows*cols/32] f32 (the
 * parts prana_mat_create_q8 takes, host copies). */
int prana_quantize_q8(const float *w, size_t rows, size_t cols, int8_t *q, float *scales, prana_stream_t stream);
/* Linear::apply for n_tokens rows (checkpoint.rs:94-100): matmul_f32
 * (matmul.rs:150-157) / matmul_q8_f32 (162-178) / matmul_kquant_f32
 * (kquant.rs:323-333). x[n_tokens*cols] -> out[n_tokens*rows]. Quantizes the
 * activations itself; scratch comes from the library. */
int prana_matmul(prana_mat_t w, const float *x, size_t n_tokens, float *out, prana_stream_t stream);
/* Linear::apply_prefill (checkpoint.rs:140-146): matmul_q8_prefill
 * (matmul.rs:185-187) / matmul_kquant_prefill (kquant.rs:368-370) over
 * already-quantized rows; x is read only for F32 matrices. */
int prana_matmul_prefill(prana_mat_t w, const float *x, const int8_t *q, const float *scales, const int32_t *sums,
                         size_t n_tokens, float *out, prana_stream_t stream);
/* The exact i32 block dots behind every term (Q4_0: s - 8*sum_a; Q4_K: the
 * nibble dot per 32-group; Q6_K: per 16-element sub-block). isums is
 * [n_tokens][rows][terms], terms = cols/32 (cols/16 for Q6_K). */
int prana_matmul_block_sums(prana_mat_t w, const int8_t *q, const int32_t *sums, size_t n_tokens, int32_t *isums,
                            prana_stream_t stream);
/* Embedding::row (checkpoint.rs:169-174) for n tokens (device ids), times
 * scale when scale != 1 (infer.rs:155-159). out[n*cols]. */
int prana_embed_rows(prana_mat_t table, const uint32_t *tokens, size_t n, float scale, float *out,
                     prana_stream_t stream);
/* rmsnorm (norms.rs:9-23), rows x dim (rows wider than 16320 values read from
 * global memory instead of LDS, slower; dim < 2^31 - 4096). */
int prana_rmsnorm(const float *x, const float *w, size_t rows, size_t dim, float eps, float *out,
                  prana_stream_t stream);
/* silu in place (norms.rs:27-31); gelu_tanh in place (norms.rs:35-41). */
int prana_silu(float *x, size_t n, prana_stream_t stream);
int prana_gelu_tanh(float *x, size_t n, prana_stream_t stream);
/* The gated-MLP step of forward_impl (infer.rs:193-199): g = act(g) * u
 * elementwise over n values, act = silu / gelu_tanh. */
int prana_silu_mul(float *g, const float *u, size_t n, prana_stream_t stream);
int prana_gelu_tanh_mul(float *g, const float *u, size_t n, prana_stream_t stream);
/* add_bias (infer.rs:73-79) on each of `rows` rows of n: x[r*n + i] += bias[i]. */
int prana_add_bias(float *x, const float *bias, size_t rows, size_t n, prana_stream_t stream);
/* softmax (norms.rs:44-56) over each of `rows` rows of n. */
int prana_softmax(const float *in, size_t rows, size_t n, float *out, prana_stream_t stream);
/* rope_interleaved (attention.rs:90-101) / rope_neox (107-121) in place on
 * n_rows rows of row_len at positions pos0 + i; rope (attention.rs:59-80) is
 * rope_neox with pos0 = 0 over [seq, n_heads*head_dim]. */
int prana_rope_interleaved(float *x, size_t n_rows, size_t row_len, size_t pos0, size_t head_dim, float theta,
                           prana_stream_t stream);
int prana_rope_neox(float *x, size_t n_rows, size_t row_len, size_t pos0, size_t head_dim, float theta,
                    prana_stream_t stream);
/* f16_kv_write (attention.rs:47-52). */
int prana_kv_write_f16(uint16_t *cache, size_t first_row, size_t kv_stride, const float *src, size_t n,
                       prana_stream_t stream);
/* attention_decode (attention.rs:129-160) over the f16 cache rows 0..=pos. */
int prana_attention_decode(const float *q, const uint16_t *k_cache, const uint16_t *v_cache, size_t pos,
                           size_t n_heads, size_t n_kv_heads, size_t head_dim, float *out, prana_stream_t stream);
/* attention_verify (attention.rs:296-333): seq rows at pos0.. over the cache. */
int prana_attention_verify(const float *q, const uint16_t *k_cache, const uint16_t *v_cache, size_t pos0,
                           size_t seq, size_t n_heads, size_t n_kv_heads, size_t head_dim, float *out,
                           prana_stream_t stream);
/* Split-K flash decoding: attention_decode (attention.rs:129-160) for n_seq
 * (1..16) independent sequences, each over its own f16 cache, in tiles of
 * cache rows whose partial softmax states (max, sum, P.V) are merged by a
 * second launch. Each output element is within 1e-4 relative of the
 * reference's sequential order plus 1e-6 of sum_t p_t |v_t[d]| (the error scale
 * of the reassociated weighted sum), not bit-identical (the exact path is
 * prana_attention_decode). q, out: device [n_seq][n_heads*head_dim] f32, RoPE
 * already applied to q; k_caches / v_caches: host arrays of n_seq device
 * pointers to [rows][n_kv_heads*head_dim] f16, 16-byte aligned; pos: host
 * array, sequence i attends to rows 0..=pos[i]. Any n_heads / n_kv_heads; a
 * head_dim that is a multiple of 8 up to 256 (MAX_HEAD_DIM, attention.rs:42;
 * others return PRANA_ERR_INVALID). Synchronous; scratch comes from the
 * library. */
int prana_attention_decode_splitk(const float *q, const uint16_t *const *k_caches, const uint16_t *const *v_caches,
                                  const size_t *pos, size_t n_seq, size_t n_heads, size_t n_kv_heads,
                                  size_t head_dim, float *out, prana_stream_t stream);
/* prana_attention_decode_splitk without any allocation: no counterpart in the
 * reference; for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops). The partial softmax states go to a
 * fixed array of the library, 2^23 floats (32 MiB) per GPU, held until the
 * process ends; a call whose plan needs more (n_seq * n_heads *
 * ceil(rows/tile) * (head_dim + 2) floats) fails with PRANA_ERR_INVALID.
 * Asynchronous on `stream` (NULL = the library's); prana_init must have run.
 * Every call on one GPU shares that GPU's array, so calls that overlap on one
 * GPU race; the array keeps the last call's contents. */
int prana_attention_decode_splitk_noalloc(const float *q, const uint16_t *const *k_caches,
                                          const uint16_t *const *v_caches, const size_t *pos, size_t n_seq,
                                          size_t n_heads, size_t n_kv_heads, size_t head_dim, float *out,
                                          prana_stream_t stream);
/* attention (prefill, attention.rs:236-284): causal over f32 K/V. */
int prana_attention_prefill(const float *q, const float *k, const float *v, size_t seq, size_t n_heads,
                            size_t n_kv_heads, size_t head_dim, float *out, prana_stream_t stream);
/* Greedy argmax (infer.rs:560-568 / sampler.rs:40-48) of each row. */
int prana_argmax(const float *logits, size_t rows, size_t n, uint32_t *out_idx, prana_stream_t stream);
/* f32_to_f16 / f16_to_f32 (lib.rs:57-113) elementwise. */
int prana_f32_to_f16(const float *in, size_t n, uint16_t *out, prana_stream_t stream);
int prana_f16_to_f32(const uint16_t *in, size_t n, float *out, prana_stream_t stream);
/* The device expf behind silu/softmax (f32::exp, norms.rs:29,49). */
int prana_expf(const float *in, size_t n, float *out, prana_stream_t stream);
/* The device tanhf behind gelu_tanh (f32::tanh, norms.rs:35-41): glibc's
 * fdlibm tanhf / expm1f, bit for bit. */
int prana_tanhf(const float *in, size_t n, float *out, prana_stream_t stream);

/* ---------------------------------------------------------------- model */
/* Config (checkpoint.rs:32-56). rope_neox: 0 interleaved / 1 NeoX;
 * act: 0 silu / 1 gelu_tanh. */
typedef struct prana_config {
  size_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len, head_dim;
  float rope_theta, norm_eps, emb_scale;
  int rope_neox;
  int act;
} prana_config;

typedef struct prana_model *prana_model_t;
typedef struct prana_cache *prana_cache_t;

int prana_model_create(const prana_config *cfg, prana_model_t *out);
int prana_model_destroy(prana_model_t m);
/* Attach one tensor by its GGUF name (gguf.rs:381-437): token_embd.weight,
 * output_norm.weight, output.weight, blk.N.{attn_norm,attn_q,attn_k,attn_v,
 * attn_output,ffn_norm,ffn_gate,ffn_down,ffn_up}.weight, blk.N.attn_{q,k,v}.bias.
 * dims follow ggml order (dims[0] = cols). */
int prana_model_set_tensor(prana_model_t m, const char *name, int ggml_type, const uint64_t *dims, int n_dims,
                           const void *bytes, size_t nbytes);
/* Validate that every required tensor is present and shapes agree. */
int prana_model_finalize(prana_model_t m);
/* Total bytes of projection + head weights streamed per decoded token. */
int prana_model_stream_bytes(prana_model_t m, size_t *bytes);

/* KvCache::with_len (infer.rs:37-44): f16 K/V per layer, min(positions, seq_len) rows. */
int prana_cache_create(prana_model_t m, size_t positions, prana_cache_t *out);
int prana_cache_destroy(prana_cache_t c);
/* Copy layer `layer`'s K or V (which = 0/1) rows [0, rows) to the host. */
int prana_cache_read(prana_cache_t c, size_t layer, int which, size_t rows, uint16_t *host_out);

/* forward / forward_impl (infer.rs:134-211): one token at pos; logits
 * (host, vocab floats) written when need_logits. */
int prana_forward(prana_model_t m, prana_cache_t c, uint32_t token, size_t pos, int need_logits,
                  float *logits_host);
/* prefill (infer.rs:220-286): tokens at positions 0..n. */
int prana_prefill(prana_model_t m, prana_cache_t c, const uint32_t *tokens, size_t n);
/* forward_batch (infer.rs:296-374): n tokens at pos0..; logits [n][vocab]. */
int prana_forward_batch(prana_model_t m, prana_cache_t c, const uint32_t *tokens, size_t n, size_t pos0,
                        float *logits_host);

/* Greedy decode of n_steps tokens over an existing cache: feed `token` at pos,
 * then each argmax at the next position — the sampled part of generate's loop
 * (infer.rs:729-763) with the ids kept on the device; out[n_steps] gets the
 * sampled ids at the end. No stop ids. */
int prana_decode(prana_model_t m, prana_cache_t c, uint32_t token, size_t pos, size_t n_steps, uint32_t *out);

/* 1 when prana_decode / prana_generate replay a captured decode step (a HIP
 * graph per attention regime), 0 when they launch the same kernels one by one:
 * with PRANA_DECODE_GRAPH=0, or when a profiling tool (rocprofv3's
 * librocprofiler-sdk-tool, ROCPROF_* settings, librocprofiler64,
 * libroctracer64) is loaded into the process, under whose kernel tracing graph
 * replays crashed the host. Host-only; needs no GPU. Decided once per process.
 * No counterpart in the reference (its decode loop has no graphs). */
int prana_decode_replay_enabled(void);

/* GEMV launch profiling for roofline accounting: with on = P > 0, every P-th
 * model decode-GEMV dispatch records start/stop HIP events as part of the
 * dispatch itself (on its stream); on = 0 turns it off. read returns the timed
 * launches, their summed kernel seconds and summed algorithmic weight bytes
 * since the last reset.
 * No counterpart in the reference (its timing is PRANA_TIMING, infer.rs:81-130). */
int prana_gemv_profile(int on);
int prana_gemv_profile_read(size_t *launches, double *seconds, double *bytes, int reset);
/* The same timed launches split by shape: one entry per distinct weight-byte
 * count streamed by a launch (which tells the projections apart), in
 * ascending byte order; up to cap entries are written and *n_out gets the
 * number of shapes. Entry 1 (bytes = 1) is the decode attention launch (the
 * one-launch kernel, which also quantizes its output for wo), sampled in the
 * same rotation and left out of prana_gemv_profile_read's GEMV totals; the
 * norms of a decode step run inside the Q|K|V and gate|up launches. Cleared
 * by prana_gemv_profile_read with reset set.
 * No counterpart in the reference (a measurement hook for the benchmark; its
 * PRANA_TIMING buckets, infer.rs:81-130, are these entries by projection). */
int prana_gemv_profile_shapes(size_t cap, size_t *bytes, size_t *launches, double *seconds, size_t *n_out);

typedef struct prana_gen_stats {
  size_t prompt_tokens, generated_tokens, proposed, accepted;
  double seconds, prefill_seconds, decode_seconds;
} prana_gen_stats;

/* generate (infer.rs:696-771) with the greedy sampler; stops = ids for which
 * Tokenize::is_stop holds (tokenizer.rs:174-176). out has room for `steps`. */
int prana_generate(prana_model_t m, const uint32_t *prompt, size_t p, size_t steps, const uint32_t *stops,
                   size_t n_stops, uint32_t *out, size_t *n_out, prana_gen_stats *stats);
/* generate_speculative (infer.rs:581-690), greedy, draft length k. */
int prana_generate_speculative(prana_model_t target, prana_model_t draft, const uint32_t *prompt, size_t p,
                               size_t steps, size_t k, const uint32_t *stops, size_t n_stops, uint32_t *out,
                               size_t *n_out, prana_gen_stats *stats);

/* Bytes of a ggml tensor of the given type and element count. */
size_t prana_ggml_nbytes(int ggml_type, size_t n_elems);

/* ---------------------------------------------------------------- GGUF
 * The reference's container reader and model loader (prana-model gguf.rs).
 * These entry points run on the host and make no device call, except
 * prana_model_load_gguf, which uploads the model. Strings and arrays come
 * back through caller-sized buffers: the out-length is always set, and a
 * buffer that is too small gives PRANA_ERR_SHORT_BUFFER (grow and retry). */
typedef struct prana_gguf *prana_gguf_t;

/* Gguf::read (gguf.rs:157-160): the file is memory-mapped read-only, not
 * copied. GGUF v2/v3; bad magic, other versions, truncation and unknown
 * value types fail with the reference's messages (gguf.rs:97-130,162-172). */
int prana_gguf_open(const char *path, prana_gguf_t *out);
/* Gguf::from_bytes (gguf.rs:162-196) over a copy of the caller's bytes. */
int prana_gguf_open_bytes(const void *data, size_t nbytes, prana_gguf_t *out);
int prana_gguf_close(prana_gguf_t g);
/* Header fields: format version, tensor count (distinct names, file order),
 * metadata entry count. */
int prana_gguf_counts(prana_gguf_t g, uint32_t *version, size_t *n_tensors, size_t *n_meta);
/* Name of the index-th tensor of the directory (file order). */
int prana_gguf_tensor_name(prana_gguf_t g, size_t index, char *buf, size_t cap, size_t *len);
/* TensorInfo (gguf.rs:133-138): ggml type, dims in ggml order (dims[0] =
 * contiguous), and the byte size of its data, checked against the data
 * section (Gguf::raw, gguf.rs:202-205). dims holds up to 8: a tensor with more
 * gives PRANA_ERR_SHORT_BUFFER unless dims is NULL (then *n_dims says how many
 * it has; its data and f32 readers take any count). */
int prana_gguf_tensor_info(prana_gguf_t g, const char *name, int *ggml_type, uint64_t *dims, int *n_dims,
                           size_t *nbytes);
/* The tensor's bytes in place (valid until prana_gguf_close). */
int prana_gguf_tensor_data(prana_gguf_t g, const char *name, const void **bytes, size_t *nbytes);
/* Gguf::tensor_f32 (gguf.rs:208-264): F32, F16, Q4_0, Q8_0, Q4_K, Q6_K
 * decoded to f32 on the host (kquant.rs:39-112 block decoders). cap counts
 * floats; *n = the tensor's element count. */
int prana_gguf_tensor_f32(prana_gguf_t g, const char *name, float *out, size_t cap, size_t *n);
/* Value type (0..12, gguf.rs:102-130) of a metadata entry; elem_type is the
 * element type of an array (type 9), else -1. */
int prana_gguf_meta_type(prana_gguf_t g, const char *key, int *type, int *elem_type);
/* Value::as_usize (gguf.rs:63-75): unsigned, or signed >= 0, integers. */
int prana_gguf_meta_u64(prana_gguf_t g, const char *key, uint64_t *out);
/* Value::as_f32 (gguf.rs:77-83): f32, or f64 narrowed. */
int prana_gguf_meta_f32(prana_gguf_t g, const char *key, float *out);
/* A string value's bytes, NUL terminated (GGUF strings may hold NULs: use *len). */
int prana_gguf_meta_str(prana_gguf_t g, const char *key, char *buf, size_t cap, size_t *len);
int prana_gguf_meta_array_len(prana_gguf_t g, const char *key, size_t *n);
/* Element index of a string array (tokenizer.ggml.tokens / merges). */
int prana_gguf_meta_array_str(prana_gguf_t g, const char *key, size_t index, char *buf, size_t cap, size_t *len);
/* A float array (tokenizer.ggml.scores) as f32; cap counts elements. */
int prana_gguf_meta_array_f32(prana_gguf_t g, const char *key, float *out, size_t cap, size_t *n);
/* An integer or bool array (tokenizer.ggml.token_type) as int64. */
int prana_gguf_meta_array_i64(prana_gguf_t g, const char *key, int64_t *out, size_t cap, size_t *n);
/* The Config load derives (gguf.rs:340-378,410-425): llama / qwen2 / gemma
 * keys with the reference's defaults (head_count_kv = head_count, freq_base
 * 1e4, key_length = dim / heads, rms epsilon 1e-5), vocab = the length of
 * tokenizer.ggml.tokens, rope_neox for qwen2 and gemma, gemma's gelu_tanh and
 * sqrt(dim) embedding scale. */
int prana_gguf_model_config(prana_gguf_t g, prana_config *cfg);
/* load (gguf.rs:338-437) without the tokenizer: every tensor by name onto a
 * new finalized device model. precision 0 = Precision::F32, 1 =
 * Precision::Q8 (checkpoint.rs:85-91). Q8_0 / Q4_0 rows with cols % 32 == 0
 * and Q4_K / Q6_K rows with cols % 256 == 0 stay packed (gguf.rs:271-305);
 * other matrices are decoded to f32 and, at Q8 with cols % 32 == 0,
 * quantized by quantize_q8 (matmul.rs:61-84), else kept dense. The
 * embedding stays packed for Q4_0 / Q4_K / Q6_K (gguf.rs:309-326). Gemma
 * norm weights get the +1 fold (gguf.rs:383-396). Without output.weight the
 * head reads the table; a dense table at Q8 gets a quantized copy
 * (gguf.rs:426-437). Backend limits: dim and hidden_dim multiples of 32,
 * head_dim even and <= 256. */
int prana_model_load_gguf(prana_gguf_t g, int precision, prana_model_t *out);
/* The configuration a model was created or loaded with. */
int prana_model_config(prana_model_t m, prana_config *cfg);

/* ---------------------------------------------------------------- tokenizers
 * prana-model's tokenizers (tokenizer.rs, bpe.rs), host only: SentencePiece
 * (greedy highest-score merges over per-code-point seeds with <0xNN> byte
 * fallback) and GPT-2 byte-level BPE (ranked merges over the byte-unicode
 * alphabet, the reference's approximate pre-tokenizer, verbatim special
 * tokens). Text is UTF-8 bytes (invalid UTF-8 is PRANA_ERR_INVALID); id and
 * byte outputs are caller-sized (PRANA_ERR_SHORT_BUFFER gives the size). */
typedef struct prana_tokenizer *prana_tokenizer_t;

/* load_tokenizer (gguf.rs:466-537): tokenizer.ggml.model "llama" (default)
 * or "gpt2", tokens (U+2581 read as a space for llama), scores / merges /
 * token_type, bos_token_id / eos_token_id (llama defaults 1 / 2), and
 * add_bos_token (default: llama yes, gpt2 no). */
int prana_tokenizer_from_gguf(prana_gguf_t g, prana_tokenizer_t *out);
/* Tokenizer::from_bytes (tokenizer.rs:65-82): llama2.c's tokenizer.bin. */
int prana_tokenizer_from_llama2c(const void *data, size_t nbytes, size_t vocab_size, prana_tokenizer_t *out);
int prana_tokenizer_destroy(prana_tokenizer_t t);
/* kind: 0 SentencePiece, 1 byte-level BPE. */
int prana_tokenizer_info(prana_tokenizer_t t, int *kind, size_t *vocab_size);
/* Tokenizer::encode (tokenizer.rs:89-143), SentencePiece only. */
int prana_tokenizer_encode(prana_tokenizer_t t, const char *text, size_t len, int bos, int eos, uint32_t *ids,
                           size_t cap, size_t *n);
/* Tokenize::encode_prompt (tokenizer.rs:19-26; bpe.rs:173-206). */
int prana_tokenizer_encode_prompt(prana_tokenizer_t t, const char *text, size_t len, uint32_t *ids, size_t cap,
                                  size_t *n);
/* Tokenize::decode (tokenizer.rs:147-162; bpe.rs:208-213): the bytes of one
 * token given the previous one. */
int prana_tokenizer_decode(prana_tokenizer_t t, uint32_t prev, uint32_t token, char *buf, size_t cap, size_t *len);
/* Tokenize::is_stop: EOS or BOS. */
int prana_tokenizer_is_stop(prana_tokenizer_t t, uint32_t token, int *stop);
/* The ids is_stop accepts, for the stops argument of prana_generate*. */
int prana_tokenizer_stop_ids(prana_tokenizer_t t, uint32_t *ids, size_t cap, size_t *n);
/* BpeTokenizer::pre_tokenize (bpe.rs:96-139): piece i is bytes
 * [bounds[2i], bounds[2i+1]) of text; cap counts size_t slots. */
int prana_bpe_pre_tokenize(const char *text, size_t len, size_t *bounds, size_t cap, size_t *n);

/* ---------------------------------------------------------------- sampler
 * Sampler (prana-model sampler.rs:6-71): greedy for temp <= 0, else
 * temperature sampling driven by a seeded xorshift64* stream. Sampling runs
 * on the device: logits / temp, the exact softmax, and the bucket walk
 * (r -= p[i] until r <= 0) in the reference's f32 order, so the same seed
 * gives the reference's tokens. */
typedef struct prana_sampler *prana_sampler_t;

/* Sampler::new (sampler.rs:13-19); XorShift::new maps seed 0 to 1. */
int prana_sampler_create(float temp, uint64_t seed, prana_sampler_t *out);
int prana_sampler_destroy(prana_sampler_t s);
/* The RNG state (advances by one per temperature draw). */
int prana_sampler_state(prana_sampler_t s, uint64_t *state);
/* XorShift::next_f32 (sampler.rs:66-70): uniform in [0, 1). */
int prana_sampler_next_f32(prana_sampler_t s, float *out);
/* Sampler::sample (sampler.rs:22-39) over device logits [n]; one draw;
 * *token is host memory; returns when the token is known. */
int prana_sampler_sample(prana_sampler_t s, const float *logits, size_t n, uint32_t *token, prana_stream_t stream);
/* The bucket walk alone (sampler.rs:29-36) over device probabilities for a
 * given r: *out (device) = the first i with (r -= probs[i]) <= 0, else n-1. */
int prana_sample_pick(const float *probs, size_t n, float r, uint32_t *out, prana_stream_t stream);
/* generate (infer.rs:696-771) with a sampler: teacher-forced prompt, then one
 * draw per sampled position (none for temp <= 0, which is prana_generate);
 * stops on a token of stops; the sampler's state ends where the reference's
 * would. */
int prana_generate_sampled(prana_model_t m, const uint32_t *prompt, size_t p, size_t steps, const uint32_t *stops,
                           size_t n_stops, prana_sampler_t sampler, uint32_t *out, size_t *n_out,
                           prana_gen_stats *stats);

/* ---------------------------------------------------------------- graph
 * prana-graph (prana-graph/src/lib.rs:25-220) over device buffers: a
 * define-then-run graph whose node values are f32 buffers in device memory
 * and whose ops are this library's kernels (the same ones the model runs, so
 * each value equals the reference op's output bit for bit). Node ids are
 * indices handed out by the builders; every builder checks the ids it is
 * given. Weights are copied to the device when the node is built. */
typedef struct prana_graph *prana_graph_t;

/* GraphError (lib.rs:55-63), reported by prana_graph_execute. */
#define PRANA_GRAPH_UNSET_INPUT 1
#define PRANA_GRAPH_SHAPE_MISMATCH 2
#define PRANA_GRAPH_NOT_F32 3

/* Graph::new (lib.rs:66-68). */
int prana_graph_create(prana_graph_t *out);
int prana_graph_destroy(prana_graph_t g);
/* Graph::input (lib.rs:82-87): the graph's row count becomes
 * max(previous, n_tokens). */
int prana_graph_input(prana_graph_t g, size_t n_tokens, size_t *id);
/* Graph::matmul_f32 (lib.rs:89-91): weight host [n_rows][k] f32; the value
 * is [n_tokens, n_rows] (matmul_f32, matmul.rs:150-157). */
int prana_graph_matmul_f32(prana_graph_t g, size_t x, const float *weight, size_t k, size_t n_rows, size_t *id);
/* Graph::matmul_q8 (lib.rs:93-95): a QuantMatrix by its parts, host q
 * [rows][cols] i8 and scales [rows][cols/32] f32 (cols % 32 == 0); the value
 * is [n_tokens, rows] (matmul_q8_f32, matmul.rs:162-178). */
int prana_graph_matmul_q8(prana_graph_t g, size_t x, size_t rows, size_t cols, const int8_t *q, const float *scales,
                          size_t *id);
/* Graph::rmsnorm (lib.rs:97-99): weight host [dim]; value [rows, dim]. */
int prana_graph_rmsnorm(prana_graph_t g, size_t x, const float *weight, size_t dim, float eps, size_t *id);
/* Graph::add (lib.rs:101-103): elementwise, the shape of a. */
int prana_graph_add(prana_graph_t g, size_t a, size_t b, size_t *id);
/* Graph::softmax (lib.rs:105-107): one softmax over all values; value [n]. */
int prana_graph_softmax(prana_graph_t g, size_t x, size_t *id);
/* Graph::rope (lib.rs:109-113): NeoX RoPE (attention.rs:59-80) on
 * [n_tokens, n_heads*head_dim], row p at position p. */
int prana_graph_rope(prana_graph_t g, size_t x, size_t n_heads, size_t head_dim, float theta_base, size_t *id);
/* Graph::attention (lib.rs:115-124): causal attention over f32 Q/K/V of the
 * n_tokens rows (attention.rs:236-284); head_dim <= 256 on this backend. */
int prana_graph_attention(prana_graph_t g, size_t q, size_t k, size_t v, size_t n_heads, size_t n_kv_heads,
                          size_t head_dim, size_t *id);
/* Graph::set_input (lib.rs:126-129) with Tensor::from_f32(shape, values):
 * host values, or (_device) a device pointer, copied into the graph. Any node
 * may be given a value; execute then keeps it. */
int prana_graph_set_input(prana_graph_t g, size_t id, const float *values, const size_t *shape, int n_dims);
int prana_graph_set_input_device(prana_graph_t g, size_t id, const float *values, const size_t *shape, int n_dims);
/* Graph::execute (lib.rs:132-141): evaluates every node without a value in
 * definition order and returns when the device is done. Values are kept, as
 * in the reference: a later set_input does not recompute nodes already
 * evaluated (see prana_graph_reset). On a GraphError it returns
 * PRANA_ERR_INVALID with *error_kind = PRANA_GRAPH_* and *error_node = the
 * unset input or the mismatching node; both are 0 on success. */
int prana_graph_execute(prana_graph_t g, int *error_kind, size_t *error_node);
/* No counterpart in the reference: drops every computed (non-input) value so
 * the next execute recomputes the graph over new inputs, weights kept. */
int prana_graph_reset(prana_graph_t g);
/* Shape of a node's value (up to 8 dims). */
int prana_graph_shape(prana_graph_t g, size_t id, size_t *shape, int *n_dims);
/* Graph::output_f32 (lib.rs:216-219): copy to host; cap counts floats,
 * *n = the value's element count (PRANA_ERR_SHORT_BUFFER when cap < *n). */
int prana_graph_output_f32(prana_graph_t g, size_t id, float *out, size_t cap, size_t *n);
/* The value in place: a device pointer valid until the node is recomputed
 * or the graph destroyed. */
int prana_graph_output_device(prana_graph_t g, size_t id, const float **ptr, size_t *n);

#ifdef __cplusplus
}
#endif
#endif /* PRANA_HIP_H */
