/*
 * prana_oracle.c — TEST INFRASTRUCTURE ONLY. The CPU oracle: a plain-C
 * restatement of pariharshyamu/Prana's scalar tier (crates/prana-kernels) and
 * model loop (crates/prana-model). Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it, and only as the checker.
 *
 * Build: -O2 -ffp-contract=off, no fast-math (see oracle/Makefile). Rust never
 * contracts a*b+c into an FMA and rounds f32::round half away from zero; the
 * flags and roundf() reproduce both.
 *
 * Row sums written as Rust `iter().sum::<f32>()` are folds that start from
 * -0.0 (the neutral element of f32 Sum since Rust 1.83; the reference needs
 * >= 1.87 for `is_multiple_of`). `seq_sum` below is that fold.
 */
#define _GNU_SOURCE
#include "prana_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* f16 <-> f32 (prana-kernels/src/lib.rs:57-113)                        */
/* ------------------------------------------------------------------ */
static float f_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t bits_f(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* lib.rs:57-73 */
float po_f16_to_f32(uint16_t h) {
  uint32_t sign = (h >> 15) & 1u, exp = (h >> 10) & 0x1fu, frac = h & 0x3ffu;
  if (exp == 0 && frac == 0) return f_bits(sign << 31);
  if (exp == 0) { /* subnormal: frac * 2^-24, sign applied numerically */
    float v = (float)frac * ldexpf(1.0f, -24);
    return sign ? -v : v;
  }
  if (exp == 0x1f && frac == 0) return f_bits((sign << 31) | 0x7f800000u);
  if (exp == 0x1f) return f_bits((sign << 31) | 0x7f800000u | (frac << 13));
  return f_bits((sign << 31) | ((exp + 127 - 15) << 23) | (frac << 13));
}

/* lib.rs:78-113: RNE, subnormals exact, overflow -> inf, NaN keeps bit 9. */
uint16_t po_f32_to_f16(float x) {
  uint32_t bits = bits_f(x);
  uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
  int32_t exp = (int32_t)((bits >> 23) & 0xffu);
  uint32_t frac = bits & 0x007fffffu;
  if (exp == 0xff) return sign | 0x7c00u | (frac ? 0x0200u : 0u);
  int32_t e = exp - 127 + 15;
  if (e >= 0x1f) return sign | 0x7c00u;
  if (e <= 0) {
    if (e < -10) return sign;
    uint32_t m = frac | 0x00800000u;
    uint32_t shift = (uint32_t)(14 - e);
    uint16_t half = (uint16_t)(m >> shift);
    uint32_t round_bit = 1u << (shift - 1);
    uint32_t rem = m & (round_bit * 2 - 1);
    int round = rem > round_bit || (rem == round_bit && (half & 1));
    return sign | (uint16_t)(half + round);
  }
  uint16_t half = (uint16_t)(((uint32_t)e << 10) | (frac >> 13));
  uint32_t rem = frac & 0x1fffu;
  int round = rem > 0x1000u || (rem == 0x1000u && (half & 1));
  return sign | (uint16_t)(half + round);
}

void po_f16_to_f32_n(const uint16_t *h, size_t n, float *out) {
  for (size_t i = 0; i < n; i++) out[i] = po_f16_to_f32(h[i]);
}
void po_f32_to_f16_n(const float *x, size_t n, uint16_t *out) {
  for (size_t i = 0; i < n; i++) out[i] = po_f32_to_f16(x[i]);
}

/* The platform libm over a contiguous range of f32 bit patterns: the values
 * Rust's f32::exp / f32::tanh return on the reference's host (glibc). */
typedef struct { uint32_t base; size_t i0, i1; float *out; float (*fn)(float); } bits_job;
static void *bits_run(void *p) {
  bits_job *j = p;
  for (size_t i = j->i0; i < j->i1; i++) j->out[i] = j->fn(f_bits(j->base + (uint32_t)i));
  return NULL;
}
static void libm_bits(float (*fn)(float), uint32_t base, size_t n, float *out, int threads) {
  if (threads < 1) threads = 1;
  if (threads > 64) threads = 64;
  pthread_t th[64];
  bits_job jobs[64];
  size_t chunk = (n + threads - 1) / threads;
  int k = 0;
  for (int t = 0; t < threads; t++) {
    size_t i0 = t * chunk, i1 = i0 + chunk > n ? n : i0 + chunk;
    if (i0 >= i1) break;
    jobs[t] = (bits_job){base, i0, i1, out, fn};
    pthread_create(&th[t], NULL, bits_run, &jobs[t]);
    k++;
  }
  for (int t = 0; t < k; t++) pthread_join(th[t], NULL);
}
static float libm_expf(float x) { return expf(x); }
static float libm_tanhf(float x) { return tanhf(x); }
void po_expf_bits(uint32_t base, size_t n, float *out, int threads) { libm_bits(libm_expf, base, n, out, threads); }
void po_tanhf_bits(uint32_t base, size_t n, float *out, int threads) { libm_bits(libm_tanhf, base, n, out, threads); }

/* Rust `v.round().clamp(-127.0, 127.0) as i32` (matmul.rs:123): NaN -> 0. */
static int32_t round_clamp127(float v) {
  float r = roundf(v);
  if (isnan(r)) return 0;
  if (r < -127.0f) r = -127.0f;
  if (r > 127.0f) r = 127.0f;
  return (int32_t)r;
}

/* fold(-0.0, +) — Rust f32 Sum */
static float seq_sum(const float *v, size_t n) {
  float s = -0.0f;
  for (size_t i = 0; i < n; i++) s += v[i];
  return s;
}

/* ------------------------------------------------------------------ */
/* quantize_acts (matmul.rs:105-127), quantize_q8 (matmul.rs:61-84)    */
/* ------------------------------------------------------------------ */
void po_quantize_acts(const float *a, size_t k, int8_t *q, float *scales, int32_t *sums) {
  size_t groups = k / 32;
  for (size_t g = 0; g < groups; g++) {
    const float *blk = a + g * 32;
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(blk[i])); /* fold(0, max(|x|)) */
    float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    float inv = 1.0f / scale;
    int32_t sum = 0;
    for (int i = 0; i < 32; i++) {
      int32_t v = round_clamp127(blk[i] * inv);
      q[g * 32 + i] = (int8_t)v;
      sum += v;
    }
    scales[g] = scale;
    sums[g] = sum;
  }
}

void po_quantize_q8(size_t rows, size_t cols, const float *w, int8_t *q, float *scales) {
  size_t gpr = cols / 32;
  for (size_t r = 0; r < rows; r++)
    for (size_t g = 0; g < gpr; g++) {
      size_t base = r * cols + g * 32;
      float amax = 0.0f;
      for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(w[base + i]));
      float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
      float inv = 1.0f / scale;
      for (int i = 0; i < 32; i++) q[base + i] = (int8_t)round_clamp127(w[base + i] * inv);
      scales[r * gpr + g] = scale;
    }
}

/* ------------------------------------------------------------------ */
/* scalar dots                                                          */
/* ------------------------------------------------------------------ */
/* matmul.rs:377-391: four strided partial sums, then the tail. */
float po_dot_f32(const float *a, const float *b, size_t n) {
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  size_t chunks = n / 4;
  for (size_t i = 0; i < chunks; i++)
    for (int l = 0; l < 4; l++) acc[l] += a[i * 4 + l] * b[i * 4 + l];
  float sum = acc[0] + acc[1] + acc[2] + acc[3];
  for (size_t i = chunks * 4; i < n; i++) sum += a[i] * b[i];
  return sum;
}

/* matmul.rs:395-406: sum += (sw*sa)*float(acc), acc = exact i32 block dot. */
float po_dot_q8_q8(const int8_t *qa, const float *sa, const int8_t *qw, const float *sw, size_t groups) {
  float sum = 0.0f;
  for (size_t g = 0; g < groups; g++) {
    int32_t acc = 0;
    for (int l = 0; l < 32; l++) acc += (int32_t)qa[g * 32 + l] * (int32_t)qw[g * 32 + l];
    sum += sw[g] * sa[g] * (float)acc;
  }
  return sum;
}

/* kquant.rs:240-252: total += (d*sa)*float(s - 8*sum_a). */
float po_dot_q40_q8(const int8_t *qa, const float *sa, const int32_t *suma, const uint8_t *row,
                    const float *ds, size_t nblocks) {
  float total = 0.0f;
  for (size_t i = 0; i < nblocks; i++) {
    const uint8_t *b = row + i * 18;
    const int8_t *a = qa + i * 32;
    int32_t s = 0;
    for (int l = 0; l < 16; l++)
      s += (int32_t)a[l] * (int32_t)(b[2 + l] & 0xF) + (int32_t)a[16 + l] * (int32_t)(b[2 + l] >> 4);
    total += ds[i] * sa[i] * (float)(s - 8 * suma[i]);
  }
  return total;
}

/* kquant.rs:52-61 (llama.cpp get_scale_min_k4) */
void po_q4k_scale_min(int j, const uint8_t *s, float *sc, float *m) {
  if (j < 4) {
    *sc = (float)(s[j] & 63);
    *m = (float)(s[j + 4] & 63);
  } else {
    *sc = (float)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
    *m = (float)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
  }
}

/* kquant.rs:257-282: per pair p, lo then hi group:
 * total += sa*((d*sc)*float(s) - (dmin*m)*float(sum_a)). */
float po_dot_q4k_q8(const int8_t *qa, const float *sa, const int32_t *suma, const uint8_t *row,
                    const float *ds, size_t nblocks) {
  float total = 0.0f;
  for (size_t bi = 0; bi < nblocks; bi++) {
    const uint8_t *b = row + bi * 144;
    float d = ds[bi * 2], dmin = ds[bi * 2 + 1];
    const uint8_t *scales = b + 4, *qs = b + 16;
    for (int pair = 0; pair < 4; pair++) {
      const uint8_t *q = qs + pair * 32;
      size_t g_lo = bi * 8 + pair * 2, g_hi = g_lo + 1;
      const int8_t *a_lo = qa + g_lo * 32, *a_hi = qa + g_hi * 32;
      float sc1, m1, sc2, m2;
      po_q4k_scale_min(pair * 2, scales, &sc1, &m1);
      po_q4k_scale_min(pair * 2 + 1, scales, &sc2, &m2);
      int32_t s1 = 0, s2 = 0;
      for (int l = 0; l < 32; l++) {
        s1 += (int32_t)a_lo[l] * (int32_t)(q[l] & 0xF);
        s2 += (int32_t)a_hi[l] * (int32_t)(q[l] >> 4);
      }
      total += sa[g_lo] * (d * sc1 * (float)s1 - dmin * m1 * (float)suma[g_lo]);
      total += sa[g_hi] * (d * sc2 * (float)s2 - dmin * m2 * (float)suma[g_hi]);
    }
  }
  return total;
}

/* kquant.rs:287-318: per half, per 32-group g, sub-block 0 then 1:
 * total += ((d*sa)*float(i8 sc))*float(isum16). */
float po_dot_q6k_q8(const int8_t *qa, const float *sa, const int32_t *suma, const uint8_t *row,
                    const float *ds, size_t nblocks) {
  (void)suma;
  float total = 0.0f;
  for (size_t bi = 0; bi < nblocks; bi++) {
    const uint8_t *b = row + bi * 210;
    const uint8_t *ql0 = b, *qh0 = b + 128, *sc = b + 192;
    float d = ds[bi];
    const int8_t *ablk = qa + bi * 256;
    for (int half = 0; half < 2; half++) {
      const uint8_t *ql = ql0 + half * 64, *qh = qh0 + half * 32;
      int s0 = half * 8, ao = half * 128;
      int32_t sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      for (int l = 0; l < 32; l++) {
        int sub = l / 16;
        int32_t q1 = (int32_t)(int8_t)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
        int32_t q2 = (int32_t)(int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
        int32_t q3 = (int32_t)(int8_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
        int32_t q4 = (int32_t)(int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
        sums[sub] += (int32_t)ablk[ao + l] * q1;
        sums[2 + sub] += (int32_t)ablk[ao + l + 32] * q2;
        sums[4 + sub] += (int32_t)ablk[ao + l + 64] * q3;
        sums[6 + sub] += (int32_t)ablk[ao + l + 96] * q4;
      }
      for (int g = 0; g < 4; g++) {
        float s_a = sa[bi * 8 + half * 4 + g];
        total += d * s_a * (float)(int8_t)sc[s0 + g * 2] * (float)sums[g * 2];
        total += d * s_a * (float)(int8_t)sc[s0 + g * 2 + 1] * (float)sums[g * 2 + 1];
      }
    }
  }
  return total;
}

/* ------------------------------------------------------------------ */
/* block decoders (kquant.rs:39-112)                                    */
/* ------------------------------------------------------------------ */
static float f16_at(const uint8_t *b) { return po_f16_to_f32((uint16_t)(b[0] | (b[1] << 8))); }

void po_dequant_q40_block(const uint8_t *b, float *out) { /* kquant.rs:39-47 */
  float d = f16_at(b);
  for (int j = 0; j < 16; j++) out[j] = d * ((float)(b[2 + j] & 0xF) - 8.0f);
  for (int j = 0; j < 16; j++) out[16 + j] = d * ((float)(b[2 + j] >> 4) - 8.0f);
}

void po_dequant_q4k_block(const uint8_t *b, float *out) { /* kquant.rs:66-84 */
  float d = f16_at(b), dmin = f16_at(b + 2);
  const uint8_t *scales = b + 4, *qs = b + 16;
  for (int pair = 0; pair < 4; pair++) {
    const uint8_t *q = qs + pair * 32;
    float sc1, m1, sc2, m2;
    po_q4k_scale_min(pair * 2, scales, &sc1, &m1);
    po_q4k_scale_min(pair * 2 + 1, scales, &sc2, &m2);
    float d1 = d * sc1, min1 = dmin * m1, d2 = d * sc2, min2 = dmin * m2;
    for (int l = 0; l < 32; l++) *out++ = d1 * (float)(q[l] & 0xF) - min1;
    for (int l = 0; l < 32; l++) *out++ = d2 * (float)(q[l] >> 4) - min2;
  }
}

void po_dequant_q6k_block(const uint8_t *b, float *y) { /* kquant.rs:89-112 */
  const uint8_t *ql0 = b, *qh0 = b + 128, *sc = b + 192;
  float d = f16_at(b + 208);
  for (int half = 0; half < 2; half++) {
    const uint8_t *ql = ql0 + half * 64, *qh = qh0 + half * 32;
    int s0 = half * 8, yo = half * 128;
    for (int l = 0; l < 32; l++) {
      int is = s0 + l / 16;
      float q1 = (float)((int8_t)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32);
      float q2 = (float)((int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32);
      float q3 = (float)((int8_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
      float q4 = (float)((int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
      y[yo + l] = d * (float)(int8_t)sc[is] * q1;
      y[yo + l + 32] = d * (float)(int8_t)sc[is + 2] * q2;
      y[yo + l + 64] = d * (float)(int8_t)sc[is + 4] * q3;
      y[yo + l + 96] = d * (float)(int8_t)sc[is + 6] * q4;
    }
  }
}

/* ------------------------------------------------------------------ */
/* matrices                                                             */
/* ------------------------------------------------------------------ */
struct po_mat {
  int kind;
  size_t rows, cols;
  float *w;        /* F32 */
  int8_t *q;       /* Q8 */
  float *scales;   /* Q8: rows*cols/32; KQuant: hoisted dscales (kquant.rs:122-127) */
  uint8_t *blocks; /* KQuant raw rows */
  size_t row_bytes, scales_per_row;
};

static size_t kq_block_values(int kind) { return kind == PO_Q4_0 ? 32 : 256; }
static size_t kq_block_bytes(int kind) { return kind == PO_Q4_0 ? 18 : kind == PO_Q4_K ? 144 : 210; }
static size_t kq_spb(int kind) { return kind == PO_Q4_K ? 2 : 1; }

po_mat *po_mat_f32(size_t rows, size_t cols, const float *w) {
  po_mat *m = calloc(1, sizeof *m);
  m->kind = PO_F32; m->rows = rows; m->cols = cols;
  m->w = malloc(rows * cols * sizeof(float));
  memcpy(m->w, w, rows * cols * sizeof(float));
  return m;
}

/* QuantMatrix::from_parts (matmul.rs:34-39) */
po_mat *po_mat_q8_parts(size_t rows, size_t cols, const int8_t *q, const float *scales) {
  if (cols % 32) return NULL;
  po_mat *m = calloc(1, sizeof *m);
  m->kind = PO_Q8; m->rows = rows; m->cols = cols;
  m->q = malloc(rows * cols);
  memcpy(m->q, q, rows * cols);
  m->scales = malloc(rows * (cols / 32) * sizeof(float));
  memcpy(m->scales, scales, rows * (cols / 32) * sizeof(float));
  return m;
}

/* KQuantMatrix::from_raw (kquant.rs:166-183): keep bytes, hoist f16 scales. */
static po_mat *kq_from_raw(int kind, size_t rows, size_t cols, const uint8_t *raw) {
  size_t bv = kq_block_values(kind), bb = kq_block_bytes(kind);
  if (cols % bv) return NULL;
  po_mat *m = calloc(1, sizeof *m);
  m->kind = kind; m->rows = rows; m->cols = cols;
  size_t nblk = rows * cols / bv;
  m->blocks = malloc(nblk * bb);
  memcpy(m->blocks, raw, nblk * bb);
  m->row_bytes = cols / bv * bb;
  m->scales_per_row = cols / bv * kq_spb(kind);
  m->scales = malloc(nblk * kq_spb(kind) * sizeof(float));
  for (size_t i = 0; i < nblk; i++) {
    const uint8_t *b = raw + i * bb;
    if (kind == PO_Q4_0) m->scales[i] = f16_at(b);
    else if (kind == PO_Q4_K) { m->scales[2 * i] = f16_at(b); m->scales[2 * i + 1] = f16_at(b + 2); }
    else m->scales[i] = f16_at(b + 208);
  }
  return m;
}

/* Full-tensor dequant of ggml bytes, gguf.rs:208-267 (tensor_f32). */
static float *ggml_to_f32(int ty, size_t n, const uint8_t *raw) {
  float *out = malloc(n * sizeof(float));
  if (ty == PO_GGML_F32) memcpy(out, raw, n * 4);
  else if (ty == PO_GGML_F16) for (size_t i = 0; i < n; i++) out[i] = f16_at(raw + 2 * i);
  else if (ty == PO_GGML_Q4_0) for (size_t b = 0; b < n / 32; b++) po_dequant_q40_block(raw + b * 18, out + b * 32);
  else if (ty == PO_GGML_Q8_0)
    for (size_t b = 0; b < n / 32; b++) {
      float s = f16_at(raw + b * 34);
      for (int j = 0; j < 32; j++) out[b * 32 + j] = (float)(int8_t)raw[b * 34 + 2 + j] * s;
    }
  else if (ty == PO_GGML_Q4_K) for (size_t b = 0; b < n / 256; b++) po_dequant_q4k_block(raw + b * 144, out + b * 256);
  else if (ty == PO_GGML_Q6_K) for (size_t b = 0; b < n / 256; b++) po_dequant_q6k_block(raw + b * 210, out + b * 256);
  else { free(out); return NULL; }
  return out;
}

/* gguf.rs:271-305 (Gguf::linear at Precision::F32). */
po_mat *po_mat_from_ggml(int ty, size_t rows, size_t cols, const void *rawv, size_t nbytes) {
  const uint8_t *raw = rawv;
  (void)nbytes;
  if (ty == PO_GGML_Q8_0 && cols % 32 == 0) {
    size_t blocks = rows * cols / 32;
    int8_t *q = malloc(rows * cols);
    float *sc = malloc(blocks * sizeof(float));
    for (size_t b = 0; b < blocks; b++) {
      sc[b] = f16_at(raw + b * 34);
      memcpy(q + b * 32, raw + b * 34 + 2, 32);
    }
    po_mat *m = po_mat_q8_parts(rows, cols, q, sc);
    free(q); free(sc);
    return m;
  }
  if (ty == PO_GGML_Q4_0 && cols % 32 == 0) return kq_from_raw(PO_Q4_0, rows, cols, raw);
  if (ty == PO_GGML_Q4_K && cols % 256 == 0) return kq_from_raw(PO_Q4_K, rows, cols, raw);
  if (ty == PO_GGML_Q6_K && cols % 256 == 0) return kq_from_raw(PO_Q6_K, rows, cols, raw);
  /* Linear::new(tensor_f32, .., Precision::F32) -> dense */
  if ((ty == PO_GGML_Q4_K || ty == PO_GGML_Q6_K) && (rows * cols) % 256) return NULL;
  if ((ty == PO_GGML_Q4_0 || ty == PO_GGML_Q8_0) && (rows * cols) % 32) return NULL;
  float *f = ggml_to_f32(ty, rows * cols, raw);
  if (!f) return NULL;
  po_mat *m = po_mat_f32(rows, cols, f);
  free(f);
  return m;
}

void po_mat_free(po_mat *m) {
  if (!m) return;
  free(m->w); free(m->q); free(m->scales); free(m->blocks);
  free(m);
}
size_t po_mat_rows(const po_mat *m) { return m->rows; }
size_t po_mat_cols(const po_mat *m) { return m->cols; }
int po_mat_kind(const po_mat *m) { return m->kind; }

/* The timed tier (cpu_tier.c): 0 = the scalar tier (the oracle), 1 = the
 * reference's runtime-selected SIMD dots on its persistent pool. */
static int g_tier = 0;
float pt_row_dot(int kind, const float *x, const float *w, const int8_t *qa, const float *sa, const int32_t *suma,
                 const int8_t *qw, const float *sw, const uint8_t *row, const float *ds, size_t k);
const char *pt_simd_tier(void);
int pt_pool_start(int threads);
void pt_pool_run(size_t n_chunks, void (*fn)(void *, size_t), void *ctx);
int pt_pool_threads(void);

int po_set_tier(int tier, int threads) {
  g_tier = tier ? 1 : 0;
  return g_tier ? pt_pool_start(threads) : 0;
}
const char *po_tier_name(void) { return g_tier ? pt_simd_tier() : "scalar"; }

/* Linear::row_dot (checkpoint.rs:129-135) -> the scalar dot of the format. */
float po_mat_row_dot(const po_mat *m, const float *x, const int8_t *q, const float *sa,
                     const int32_t *sums, size_t r) {
  size_t k = m->cols;
  if (g_tier) {
    const int kind = m->kind == PO_F32 ? 0 : m->kind == PO_Q8 ? 1 : m->kind == PO_Q4_0 ? 2 : m->kind == PO_Q4_K ? 3 : 4;
    return pt_row_dot(kind, x, m->w ? m->w + r * k : NULL, q, sa, sums, m->q ? m->q + r * k : NULL,
                      m->kind == PO_Q8 ? m->scales + r * (k / 32) : NULL,
                      m->blocks ? m->blocks + r * m->row_bytes : NULL,
                      m->kind >= PO_Q4_0 ? m->scales + r * m->scales_per_row : NULL, k);
  }
  switch (m->kind) {
    case PO_F32: return po_dot_f32(x, m->w + r * k, k);
    case PO_Q8: return po_dot_q8_q8(q, sa, m->q + r * k, m->scales + r * (k / 32), k / 32);
    case PO_Q4_0:
      return po_dot_q40_q8(q, sa, sums, m->blocks + r * m->row_bytes, m->scales + r * m->scales_per_row, k / 32);
    case PO_Q4_K:
      return po_dot_q4k_q8(q, sa, sums, m->blocks + r * m->row_bytes, m->scales + r * m->scales_per_row, k / 256);
    default:
      return po_dot_q6k_q8(q, sa, sums, m->blocks + r * m->row_bytes, m->scales + r * m->scales_per_row, k / 256);
  }
}

size_t po_mat_row_block_isums(const po_mat *m, const int8_t *qa, const int32_t *suma, size_t r, int32_t *out) {
  size_t k = m->cols, n = 0;
  if (m->kind == PO_Q8) {
    const int8_t *qw = m->q + r * k;
    for (size_t g = 0; g < k / 32; g++) {
      int32_t acc = 0;
      for (int l = 0; l < 32; l++) acc += (int32_t)qa[g * 32 + l] * qw[g * 32 + l];
      out[n++] = acc;
    }
  } else if (m->kind == PO_Q4_0) {
    const uint8_t *row = m->blocks + r * m->row_bytes;
    for (size_t i = 0; i < k / 32; i++) {
      const uint8_t *b = row + i * 18;
      int32_t s = 0;
      for (int l = 0; l < 16; l++)
        s += (int32_t)qa[i * 32 + l] * (b[2 + l] & 0xF) + (int32_t)qa[i * 32 + 16 + l] * (b[2 + l] >> 4);
      out[n++] = s - 8 * suma[i];
    }
  } else if (m->kind == PO_Q4_K) {
    const uint8_t *row = m->blocks + r * m->row_bytes;
    for (size_t bi = 0; bi < k / 256; bi++)
      for (int g = 0; g < 8; g++) {
        const uint8_t *q = row + bi * 144 + 16 + (g / 2) * 32;
        int32_t s = 0;
        for (int l = 0; l < 32; l++) s += (int32_t)qa[(bi * 8 + g) * 32 + l] * ((g & 1) ? (q[l] >> 4) : (q[l] & 0xF));
        out[n++] = s;
      }
  } else if (m->kind == PO_Q6_K) {
    float tmp[256];
    const uint8_t *row = m->blocks + r * m->row_bytes;
    for (size_t bi = 0; bi < k / 256; bi++) {
      /* integer weights q-32 via the decoder with d = 1 and unit scales */
      uint8_t b[210];
      memcpy(b, row + bi * 210, 210);
      memset(b + 192, 1, 16);
      b[208] = 0x00; b[209] = 0x3c;
      po_dequant_q6k_block(b, tmp);
      for (int s = 0; s < 16; s++) {
        int32_t acc = 0;
        for (int l = 0; l < 16; l++) acc += (int32_t)qa[bi * 256 + s * 16 + l] * (int32_t)tmp[s * 16 + l];
        out[n++] = acc;
      }
    }
  }
  return n;
}

void po_mat_row_f32(const po_mat *m, size_t r, float *out) {
  size_t k = m->cols;
  switch (m->kind) {
    case PO_F32: memcpy(out, m->w + r * k, k * 4); break;
    case PO_Q8:
      for (size_t i = 0; i < k; i++) out[i] = (float)m->q[r * k + i] * m->scales[r * (k / 32) + i / 32];
      break;
    case PO_Q4_0:
      for (size_t b = 0; b < k / 32; b++) po_dequant_q40_block(m->blocks + r * m->row_bytes + b * 18, out + b * 32);
      break;
    case PO_Q4_K:
      for (size_t b = 0; b < k / 256; b++) po_dequant_q4k_block(m->blocks + r * m->row_bytes + b * 144, out + b * 256);
      break;
    default:
      for (size_t b = 0; b < k / 256; b++) po_dequant_q6k_block(m->blocks + r * m->row_bytes + b * 210, out + b * 256);
  }
}

/* ---------------- row-parallel driver (order-free per output) ---------------- */
static int g_threads = 0;
void po_set_threads(int n) { g_threads = n < 0 ? 0 : n; }

typedef struct {
  const po_mat *m;
  const float *x;        /* dense rows [n][cols] (F32) */
  const int8_t *q;       /* quantized rows [n][cols] */
  const float *sa;       /* [n][cols/32] */
  const int32_t *sums;   /* [n][cols/32] */
  size_t n, r0, r1;
  float *out;            /* [n][rows] */
} job_t;

static void *job_run(void *p) {
  job_t *j = p;
  size_t k = j->m->cols, g = k / 32, R = j->m->rows;
  for (size_t r = j->r0; r < j->r1; r++)
    for (size_t t = 0; t < j->n; t++)
      j->out[t * R + r] = po_mat_row_dot(j->m, j->x ? j->x + t * k : NULL, j->q ? j->q + t * k : NULL,
                                         j->sa ? j->sa + t * g : NULL, j->sums ? j->sums + t * g : NULL, r);
  return NULL;
}

/* run_rows / run_rows_multi chunking (matmul.rs:192-232, 318-350) on the
 * timed tier's pool. */
typedef struct { job_t base; size_t chunk; } tier_rows;
static void tier_chunk(void *ctx, size_t c) {
  tier_rows *t = ctx;
  job_t j = t->base;
  j.r0 = c * t->chunk;
  j.r1 = j.r0 + t->chunk > j.m->rows ? j.m->rows : j.r0 + t->chunk;
  job_run(&j);
}
static void tier_run_rows(job_t base) {
  const size_t R = base.m->rows, T = (size_t)pt_pool_threads();
  const size_t macs = R * base.m->cols * base.n;
  const int multi = base.n > 1;
  if (macs < (multi ? (1u << 20) : 256u * 1024u) || T <= 1) {
    base.r0 = 0;
    base.r1 = R;
    job_run(&base);
    return;
  }
  size_t chunk = (R + 4 * T - 1) / (4 * T);
  if (chunk < (multi ? 4u : 16u)) chunk = multi ? 4 : 16;
  tier_rows t = {base, chunk};
  pt_pool_run((R + chunk - 1) / chunk, tier_chunk, &t);
}

static void run_rows(job_t base) {
  if (g_tier) {
    tier_run_rows(base);
    return;
  }
  size_t R = base.m->rows;
  int nt = g_threads;
  if (nt <= 1 || R * base.m->cols * base.n < (1u << 16)) {
    base.r0 = 0; base.r1 = R;
    job_run(&base);
    return;
  }
  if (nt > 256) nt = 256;
  pthread_t th[256];
  job_t jobs[256];
  size_t chunk = (R + nt - 1) / nt;
  int launched = 0;
  for (int i = 0; i < nt; i++) {
    jobs[i] = base;
    jobs[i].r0 = i * chunk;
    jobs[i].r1 = jobs[i].r0 + chunk > R ? R : jobs[i].r0 + chunk;
    if (jobs[i].r0 >= jobs[i].r1) break;
    pthread_create(&th[i], NULL, job_run, &jobs[i]);
    launched++;
  }
  for (int i = 0; i < launched; i++) pthread_join(th[i], NULL);
}

/* matmul_f32 (matmul.rs:150-157), matmul_q8_f32 (162-178),
 * matmul_kquant_f32 (kquant.rs:323-333): quantize each token's row, then dot. */
void po_matmul(const po_mat *m, const float *a, size_t n_tokens, float *out) {
  size_t k = m->cols, g = k / 32;
  job_t j = {0};
  j.m = m; j.n = n_tokens; j.out = out;
  if (m->kind == PO_F32) {
    j.x = a;
    run_rows(j);
    return;
  }
  int8_t *q = malloc(n_tokens * k);
  float *sa = malloc(n_tokens * g * sizeof(float));
  int32_t *sums = malloc(n_tokens * g * sizeof(int32_t));
  for (size_t t = 0; t < n_tokens; t++) po_quantize_acts(a + t * k, k, q + t * k, sa + t * g, sums + t * g);
  j.q = q; j.sa = sa; j.sums = sums;
  run_rows(j);
  free(q); free(sa); free(sums);
}

/* Linear::apply_prefill (checkpoint.rs:140-146) -> matmul_f32 / run_rows_multi
 * (matmul.rs:192-232): each element is the same row dot as decode. */
void po_matmul_prefill(const po_mat *m, const float *xs, const int8_t *q, const float *sa,
                       const int32_t *sums, size_t n_tokens, float *out) {
  job_t j = {0};
  j.m = m; j.n = n_tokens; j.out = out;
  if (m->kind == PO_F32) j.x = xs;
  else { j.q = q; j.sa = sa; j.sums = sums; }
  run_rows(j);
}

/* ------------------------------------------------------------------ */
/* norms (norms.rs:9-56)                                                */
/* ------------------------------------------------------------------ */
void po_rmsnorm(const float *x, const float *w, size_t rows, size_t dim, float eps, float *out) {
  for (size_t r = 0; r < rows; r++) {
    const float *row = x + r * dim;
    float ss = -0.0f;
    for (size_t i = 0; i < dim; i++) ss += row[i] * row[i];
    float mean_sq = ss / (float)dim;
    float inv = 1.0f / sqrtf(mean_sq + eps);
    for (size_t i = 0; i < dim; i++) out[r * dim + i] = row[i] * inv * w[i];
  }
}

void po_silu(float *x, size_t n) { /* norms.rs:27-31 */
  for (size_t i = 0; i < n; i++) x[i] *= 1.0f / (1.0f + expf(-x[i]));
}

void po_gelu_tanh(float *x, size_t n) { /* norms.rs:35-41 */
  const float SQRT_2_OVER_PI = 0.7978846f;
  for (size_t i = 0; i < n; i++) {
    float v = x[i];
    float x3 = v * v * v;
    x[i] = 0.5f * v * (1.0f + tanhf(SQRT_2_OVER_PI * (v + 0.044715f * x3)));
  }
}

void po_softmax(const float *in, size_t n, float *out) { /* norms.rs:44-56 */
  if (n == 0) return;
  float mx = -INFINITY;
  for (size_t i = 0; i < n; i++) mx = fmaxf(mx, in[i]);
  for (size_t i = 0; i < n; i++) out[i] = expf(in[i] - mx);
  float sum = seq_sum(out, n);
  float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
  for (size_t i = 0; i < n; i++) out[i] *= inv;
}

/* ------------------------------------------------------------------ */
/* RoPE (attention.rs:59-121)                                           */
/* ------------------------------------------------------------------ */
void po_rope(float *x, size_t seq, size_t n_heads, size_t hd, float theta) { /* 59-80 */
  size_t half = hd / 2, stride = n_heads * hd;
  for (size_t p = 0; p < seq; p++)
    for (size_t h = 0; h < n_heads; h++) {
      size_t base = p * stride + h * hd;
      for (size_t j = 0; j < half; j++) {
        float freq = powf(theta, -(2.0f * (float)j) / (float)hd);
        float angle = (float)p * freq;
        float s = sinf(angle), c = cosf(angle);
        float x1 = x[base + j], x2 = x[base + j + half];
        x[base + j] = x1 * c - x2 * s;
        x[base + j + half] = x1 * s + x2 * c;
      }
    }
}

void po_rope_interleaved(float *x, size_t len, size_t pos, size_t hd, float theta) { /* 90-101 */
  for (size_t i = 0; i < len; i += 2) {
    size_t j = i % hd;
    float freq = powf(theta, -((float)j) / (float)hd);
    float angle = (float)pos * freq;
    float s = sinf(angle), c = cosf(angle);
    float x0 = x[i], x1 = x[i + 1];
    x[i] = x0 * c - x1 * s;
    x[i + 1] = x0 * s + x1 * c;
  }
}

void po_rope_neox(float *x, size_t len, size_t pos, size_t hd, float theta) { /* 107-121 */
  size_t half = hd / 2;
  for (size_t h = 0; h < len / hd; h++) {
    size_t base = h * hd;
    for (size_t j = 0; j < half; j++) {
      float freq = powf(theta, -(2.0f * (float)j) / (float)hd);
      float angle = (float)pos * freq;
      float s = sinf(angle), c = cosf(angle);
      float x1 = x[base + j], x2 = x[base + j + half];
      x[base + j] = x1 * c - x2 * s;
      x[base + j + half] = x1 * s + x2 * c;
    }
  }
}

/* ------------------------------------------------------------------ */
/* attention (attention.rs:47-333)                                      */
/* ------------------------------------------------------------------ */
void po_f16_kv_write(uint16_t *cache, size_t first_row, size_t kv_stride, const float *src, size_t n) {
  for (size_t i = 0; i < n; i++) cache[first_row * kv_stride + i] = po_f32_to_f16(src[i]);
}

/* decode_one_head (attention.rs:165-195). kf/vf: f32 K/V rows when the f16
 * cache is not used (prefill `attention`, 256-284, same order). */
static void one_head(const float *qv, const uint16_t *kc, const uint16_t *vc, const float *kf,
                     const float *vf, size_t pos, size_t kv_h, size_t kv_stride, size_t hd, float *dst,
                     float *scores, float *probs) {
  float scale = 1.0f / sqrtf((float)hd);
  for (size_t t = 0; t <= pos; t++) {
    size_t base = t * kv_stride + kv_h * hd;
    float dot = -0.0f;
    for (size_t d = 0; d < hd; d++) {
      float kk = kc ? po_f16_to_f32(kc[base + d]) : kf[base + d];
      dot += qv[d] * kk;
    }
    scores[t] = dot * scale;
  }
  po_softmax(scores, pos + 1, probs);
  for (size_t d = 0; d < hd; d++) dst[d] = 0.0f;
  for (size_t t = 0; t <= pos; t++) {
    size_t base = t * kv_stride + kv_h * hd;
    float p = probs[t];
    for (size_t d = 0; d < hd; d++) {
      float vv = vc ? po_f16_to_f32(vc[base + d]) : vf[base + d];
      dst[d] += p * vv;
    }
  }
}

/* Heads are independent outputs; long windows deal them to threads. */
typedef struct {
  const float *q;
  const uint16_t *kc, *vc;
  size_t pos, n_heads, group, kv_stride, hd, first, step;
  float *out;
} head_job;

static void *head_rows(void *p) {
  head_job *j = p;
  float *scores = malloc((j->pos + 1) * sizeof(float)), *probs = malloc((j->pos + 1) * sizeof(float));
  for (size_t h = j->first; h < j->n_heads; h += j->step)
    one_head(j->q + h * j->hd, j->kc, j->vc, NULL, NULL, j->pos, h / j->group, j->kv_stride, j->hd,
             j->out + h * j->hd, scores, probs);
  free(scores); free(probs);
  return NULL;
}

void po_attention_decode(const float *q, const uint16_t *kc, const uint16_t *vc, size_t pos,
                         size_t n_heads, size_t n_kv_heads, size_t hd, float *out) {
  head_job base = {q, kc, vc, pos, n_heads, n_heads / n_kv_heads, n_kv_heads * hd, hd, 0, 1, out};
  int nt = g_threads;
  if (nt > 64) nt = 64;
  if ((size_t)nt > n_heads) nt = (int)n_heads;
  if (nt <= 1 || (pos + 1) * n_heads * hd < (1u << 18)) {
    head_rows(&base);
    return;
  }
  pthread_t th[64];
  head_job jobs[64];
  for (int t = 0; t < nt; t++) {
    jobs[t] = base;
    jobs[t].first = (size_t)t;
    jobs[t].step = (size_t)nt;
    pthread_create(&th[t], NULL, head_rows, &jobs[t]);
  }
  for (int t = 0; t < nt; t++) pthread_join(th[t], NULL);
}

void po_attention_verify(const float *q, const uint16_t *kc, const uint16_t *vc, size_t pos0, size_t seq,
                         size_t n_heads, size_t n_kv_heads, size_t hd, float *out) {
  size_t q_stride = n_heads * hd;
  for (size_t i = 0; i < seq; i++)
    po_attention_decode(q + i * q_stride, kc, vc, pos0 + i, n_heads, n_kv_heads, hd, out + i * q_stride);
}

/* Each (query row, head) output is computed by one_head alone, so the rows are
 * dealt round-robin to threads (row i costs i + 1 dots); the bits do not depend
 * on the split. */
typedef struct {
  const float *q, *k, *v;
  size_t seq, n_heads, group, kv_stride, hd, first, step;
  float *out;
} attn_job;

static void *attn_rows(void *p) {
  attn_job *j = p;
  size_t q_stride = j->n_heads * j->hd;
  float *scores = malloc(j->seq * sizeof(float)), *probs = malloc(j->seq * sizeof(float));
  for (size_t i = j->first; i < j->seq; i += j->step)
    for (size_t h = 0; h < j->n_heads; h++)
      one_head(j->q + i * q_stride + h * j->hd, NULL, NULL, j->k, j->v, i, h / j->group, j->kv_stride, j->hd,
               j->out + i * q_stride + h * j->hd, scores, probs);
  free(scores); free(probs);
  return NULL;
}

void po_attention(const float *q, const float *k, const float *v, size_t seq, size_t n_heads,
                  size_t n_kv_heads, size_t hd, float *out) {
  attn_job base = {q, k, v, seq, n_heads, n_heads / n_kv_heads, n_kv_heads * hd, hd, 0, 1, out};
  int nt = g_threads;
  if (nt > 64) nt = 64;
  if ((size_t)nt > seq) nt = (int)seq;
  if (nt <= 1 || seq < 64) {
    attn_rows(&base);
    return;
  }
  pthread_t th[64];
  attn_job jobs[64];
  for (int t = 0; t < nt; t++) {
    jobs[t] = base;
    jobs[t].first = (size_t)t;
    jobs[t].step = (size_t)nt;
    pthread_create(&th[t], NULL, attn_rows, &jobs[t]);
  }
  for (int t = 0; t < nt; t++) pthread_join(th[t], NULL);
}

/* ------------------------------------------------------------------ */
/* model                                                                */
/* ------------------------------------------------------------------ */
typedef struct {
  po_mat *w[7];      /* wq wk wv wo w1 w2 w3 */
  float *vec[5];     /* rms_att rms_ffn bq bk bv (NULL = absent) */
} po_layer;

struct po_model {
  po_config c;
  po_layer *layers;
  float *rms_final;
  float *emb_f32;    /* Embedding::F32 */
  po_mat *emb_kq;    /* Embedding::KQuant */
  po_mat *wcls;      /* None => tied */
};

struct po_cache {
  size_t len, kv_dim, n_layers;
  uint16_t **k, **v;
};

po_model *po_model_new(const po_config *cfg) {
  po_model *m = calloc(1, sizeof *m);
  m->c = *cfg;
  m->layers = calloc(cfg->n_layers, sizeof(po_layer));
  return m;
}

void po_model_free(po_model *m) {
  if (!m) return;
  for (size_t l = 0; l < m->c.n_layers; l++) {
    for (int i = 0; i < 7; i++) po_mat_free(m->layers[l].w[i]);
    for (int i = 0; i < 5; i++) free(m->layers[l].vec[i]);
  }
  free(m->layers); free(m->rms_final); free(m->emb_f32);
  po_mat_free(m->emb_kq); po_mat_free(m->wcls);
  free(m);
}

void po_model_set_linear(po_model *m, size_t layer, int slot, po_mat *mat) {
  po_mat_free(m->layers[layer].w[slot]);
  m->layers[layer].w[slot] = mat;
}

void po_model_set_vec(po_model *m, size_t layer, int slot, const float *v, size_t n) {
  int i = slot - PO_RMS_ATT;
  free(m->layers[layer].vec[i]);
  m->layers[layer].vec[i] = malloc(n * sizeof(float));
  memcpy(m->layers[layer].vec[i], v, n * sizeof(float));
}

void po_model_set_rms_final(po_model *m, const float *v, size_t n) {
  free(m->rms_final);
  m->rms_final = malloc(n * sizeof(float));
  memcpy(m->rms_final, v, n * sizeof(float));
}

int po_model_set_embedding(po_model *m, int ty, const void *raw, size_t nbytes) {
  size_t rows = m->c.vocab_size, cols = m->c.dim;
  (void)nbytes;
  po_mat_free(m->emb_kq); m->emb_kq = NULL;
  free(m->emb_f32); m->emb_f32 = NULL;
  if ((ty == PO_GGML_Q4_0 && cols % 32 == 0) || (ty == PO_GGML_Q4_K && cols % 256 == 0) ||
      (ty == PO_GGML_Q6_K && cols % 256 == 0)) {
    int kind = ty == PO_GGML_Q4_0 ? PO_Q4_0 : ty == PO_GGML_Q4_K ? PO_Q4_K : PO_Q6_K;
    m->emb_kq = kq_from_raw(kind, rows, cols, raw);
    return m->emb_kq ? 0 : -1;
  }
  m->emb_f32 = ggml_to_f32(ty, rows * cols, raw);
  return m->emb_f32 ? 0 : -1;
}

void po_model_set_wcls(po_model *m, po_mat *mat) { po_mat_free(m->wcls); m->wcls = mat; }

po_cache *po_cache_new(const po_model *m, size_t positions) { /* infer.rs:37-44 */
  po_cache *c = calloc(1, sizeof *c);
  c->len = positions < m->c.seq_len ? positions : m->c.seq_len;
  c->kv_dim = m->c.n_kv_heads * m->c.head_dim;
  c->n_layers = m->c.n_layers;
  c->k = calloc(c->n_layers, sizeof(uint16_t *));
  c->v = calloc(c->n_layers, sizeof(uint16_t *));
  for (size_t l = 0; l < c->n_layers; l++) {
    c->k[l] = calloc(c->len * c->kv_dim, 2);
    c->v[l] = calloc(c->len * c->kv_dim, 2);
  }
  return c;
}
void po_cache_free(po_cache *c) {
  if (!c) return;
  for (size_t l = 0; l < c->n_layers; l++) { free(c->k[l]); free(c->v[l]); }
  free(c->k); free(c->v); free(c);
}
const uint16_t *po_cache_k(const po_cache *c, size_t l) { return c->k[l]; }
const uint16_t *po_cache_v(const po_cache *c, size_t l) { return c->v[l]; }
size_t po_cache_len(const po_cache *c) { return c->len; }

static void add_into(float *x, const float *y, size_t n) { for (size_t i = 0; i < n; i++) x[i] += y[i]; }
static void add_bias(float *x, const float *b, size_t n) { if (b) add_into(x, b, n); } /* infer.rs:73-79 */

/* Embedding::row (checkpoint.rs:169-174) then the emb_scale multiply. */
static void embed(const po_model *m, uint32_t tok, float *x) {
  size_t dim = m->c.dim;
  if (m->emb_kq) po_mat_row_f32(m->emb_kq, tok, x);
  else memcpy(x, m->emb_f32 + (size_t)tok * dim, dim * sizeof(float));
  if (m->c.emb_scale != 1.0f)
    for (size_t i = 0; i < dim; i++) x[i] *= m->c.emb_scale;
}

static void rope_row(const po_config *c, float *x, size_t len, size_t pos) {
  if (c->rope_neox) po_rope_neox(x, len, pos, c->head_dim, c->rope_theta);
  else po_rope_interleaved(x, len, pos, c->head_dim, c->rope_theta);
}

static void act(const po_config *c, float *g, size_t n) {
  if (c->act == 0) po_silu(g, n); else po_gelu_tanh(g, n);
}

/* Model::logits (checkpoint.rs:239-248) */
static void model_logits(const po_model *m, const float *x, float *logits) {
  if (m->wcls) po_matmul(m->wcls, x, 1, logits);
  else if (m->emb_f32) {
    po_mat tmp = {0};
    tmp.kind = PO_F32; tmp.rows = m->c.vocab_size; tmp.cols = m->c.dim; tmp.w = m->emb_f32;
    po_matmul(&tmp, x, 1, logits);
  } else po_matmul(m->emb_kq, x, 1, logits);
}

/* forward_impl (infer.rs:142-211) */
void po_forward(const po_model *m, po_cache *cache, uint32_t token, size_t pos, int need_logits, float *logits) {
  const po_config *c = &m->c;
  size_t dim = c->dim, hd = c->head_dim, kv_dim = c->n_kv_heads * hd, q_dim = c->n_heads * hd, hid = c->hidden_dim;
  float *x = malloc(dim * 4), *xb = malloc(dim * 4), *q = malloc(q_dim * 4), *k = malloc(kv_dim * 4),
        *v = malloc(kv_dim * 4), *attn = malloc(q_dim * 4), *o = malloc(dim * 4), *gate = malloc(hid * 4),
        *up = malloc(hid * 4);
  embed(m, token, x);
  for (size_t l = 0; l < c->n_layers; l++) {
    const po_layer *L = &m->layers[l];
    po_rmsnorm(x, L->vec[0], 1, dim, c->norm_eps, xb);
    po_matmul(L->w[PO_WQ], xb, 1, q);
    po_matmul(L->w[PO_WK], xb, 1, k);
    po_matmul(L->w[PO_WV], xb, 1, v);
    add_bias(q, L->vec[2], q_dim);
    add_bias(k, L->vec[3], kv_dim);
    add_bias(v, L->vec[4], kv_dim);
    rope_row(c, q, q_dim, pos);
    rope_row(c, k, kv_dim, pos);
    po_f16_kv_write(cache->k[l], pos, kv_dim, k, kv_dim);
    po_f16_kv_write(cache->v[l], pos, kv_dim, v, kv_dim);
    po_attention_decode(q, cache->k[l], cache->v[l], pos, c->n_heads, c->n_kv_heads, hd, attn);
    po_matmul(L->w[PO_WO], attn, 1, o);
    add_into(x, o, dim);
    po_rmsnorm(x, L->vec[1], 1, dim, c->norm_eps, xb);
    po_matmul(L->w[PO_W1], xb, 1, gate);
    po_matmul(L->w[PO_W3], xb, 1, up);
    act(c, gate, hid);
    for (size_t i = 0; i < hid; i++) gate[i] *= up[i];
    po_matmul(L->w[PO_W2], gate, 1, o);
    add_into(x, o, dim);
  }
  if (need_logits) {
    po_rmsnorm(x, m->rms_final, 1, dim, c->norm_eps, xb);
    model_logits(m, xb, logits);
  }
  free(x); free(xb); free(q); free(k); free(v); free(attn); free(o); free(gate); free(up);
}

typedef struct { int8_t *q; float *s; int32_t *sum; } acts_t;
static acts_t row_acts(const float *xs, size_t n, size_t width) { /* infer.rs:235-237 */
  acts_t a;
  size_t g = width / 32;
  a.q = malloc(n * width); a.s = malloc(n * g * 4); a.sum = malloc(n * g * 4);
  for (size_t t = 0; t < n; t++) po_quantize_acts(xs + t * width, width, a.q + t * width, a.s + t * g, a.sum + t * g);
  return a;
}
static void acts_free(acts_t a) { free(a.q); free(a.s); free(a.sum); }
static void apply_prefill(const po_mat *w, const float *xs, acts_t a, size_t n, float *out) {
  po_matmul_prefill(w, xs, a.q, a.s, a.sum, n, out);
}

/* Shared body of prefill (infer.rs:220-286) and forward_batch (296-374);
 * `verify` selects attention over the f16 cache at pos0+t (attention_verify)
 * instead of prefill attention over the window's f32 K/V. */
static void batch_body(const po_model *m, po_cache *cache, const uint32_t *tokens, size_t n, size_t pos0,
                       int verify, float *x) {
  const po_config *c = &m->c;
  size_t dim = c->dim, hd = c->head_dim, kv_dim = c->n_kv_heads * hd, q_dim = c->n_heads * hd, hid = c->hidden_dim;
  for (size_t t = 0; t < n; t++) embed(m, tokens[t], x + t * dim);
  float *xb = malloc(n * dim * 4), *q = malloc(n * q_dim * 4), *k = malloc(n * kv_dim * 4),
        *v = malloc(n * kv_dim * 4), *attn = malloc(n * q_dim * 4), *o = malloc(n * dim * 4),
        *gate = malloc(n * hid * 4), *up = malloc(n * hid * 4);
  for (size_t l = 0; l < c->n_layers; l++) {
    const po_layer *L = &m->layers[l];
    po_rmsnorm(x, L->vec[0], n, dim, c->norm_eps, xb);
    acts_t a = row_acts(xb, n, dim);
    apply_prefill(L->w[PO_WQ], xb, a, n, q);
    apply_prefill(L->w[PO_WK], xb, a, n, k);
    apply_prefill(L->w[PO_WV], xb, a, n, v);
    acts_free(a);
    for (size_t t = 0; t < n; t++) {
      add_bias(q + t * q_dim, L->vec[2], q_dim);
      add_bias(k + t * kv_dim, L->vec[3], kv_dim);
      add_bias(v + t * kv_dim, L->vec[4], kv_dim);
      rope_row(c, q + t * q_dim, q_dim, pos0 + t);
      rope_row(c, k + t * kv_dim, kv_dim, pos0 + t);
    }
    po_f16_kv_write(cache->k[l], pos0, kv_dim, k, n * kv_dim);
    po_f16_kv_write(cache->v[l], pos0, kv_dim, v, n * kv_dim);
    if (verify)
      po_attention_verify(q, cache->k[l], cache->v[l], pos0, n, c->n_heads, c->n_kv_heads, hd, attn);
    else
      po_attention(q, k, v, n, c->n_heads, c->n_kv_heads, hd, attn);
    acts_t aa = row_acts(attn, n, q_dim);
    apply_prefill(L->w[PO_WO], attn, aa, n, o);
    acts_free(aa);
    add_into(x, o, n * dim);
    po_rmsnorm(x, L->vec[1], n, dim, c->norm_eps, xb);
    acts_t a2 = row_acts(xb, n, dim);
    apply_prefill(L->w[PO_W1], xb, a2, n, gate);
    apply_prefill(L->w[PO_W3], xb, a2, n, up);
    acts_free(a2);
    act(c, gate, n * hid);
    for (size_t i = 0; i < n * hid; i++) gate[i] *= up[i];
    acts_t ah = row_acts(gate, n, hid);
    apply_prefill(L->w[PO_W2], gate, ah, n, o);
    acts_free(ah);
    add_into(x, o, n * dim);
  }
  free(xb); free(q); free(k); free(v); free(attn); free(o); free(gate); free(up);
}

void po_prefill(const po_model *m, po_cache *cache, const uint32_t *tokens, size_t n) {
  float *x = malloc(n * m->c.dim * 4);
  batch_body(m, cache, tokens, n, 0, 0, x);
  free(x);
}

/* Model::logits_batch (checkpoint.rs:256-265) */
static void model_logits_batch(const po_model *m, const float *xs, size_t n, float *logits) {
  size_t dim = m->c.dim;
  if (m->emb_f32 && !m->wcls) {
    po_mat tmp = {0};
    tmp.kind = PO_F32; tmp.rows = m->c.vocab_size; tmp.cols = dim; tmp.w = m->emb_f32;
    po_matmul(&tmp, xs, n, logits);
    return;
  }
  acts_t a = row_acts(xs, n, dim);
  apply_prefill(m->wcls ? m->wcls : m->emb_kq, xs, a, n, logits);
  acts_free(a);
}

void po_forward_batch(const po_model *m, po_cache *cache, const uint32_t *tokens, size_t n, size_t pos0,
                      float *logits) {
  size_t dim = m->c.dim;
  float *x = malloc(n * dim * 4), *xb = malloc(n * dim * 4);
  batch_body(m, cache, tokens, n, pos0, 1, x);
  po_rmsnorm(x, m->rms_final, n, dim, m->c.norm_eps, xb);
  model_logits_batch(m, xb, n, logits);
  free(x); free(xb);
}

uint32_t po_argmax(const float *v, size_t n) { /* infer.rs:560-568: strict >, first max wins */
  size_t best = 0;
  for (size_t i = 0; i < n; i++)
    if (v[i] > v[best]) best = i;
  return (uint32_t)best;
}

static int is_stop(uint32_t t, const uint32_t *stops, size_t n) {
  for (size_t i = 0; i < n; i++)
    if (stops[i] == t) return 1;
  return 0;
}

/* generate (infer.rs:696-771) with the greedy sampler (sampler.rs:40-48). */
size_t po_generate(const po_model *m, const uint32_t *prompt, size_t p, size_t steps, const uint32_t *stops,
                   size_t n_stops, uint32_t *out, po_gen_stats *st) {
  size_t max_pos = m->c.seq_len < p + steps ? m->c.seq_len : p + steps;
  po_cache *cache = po_cache_new(m, max_pos);
  float *logits = malloc(m->c.vocab_size * 4);
  uint32_t token = prompt[0];
  size_t generated = 0, start_pos = 0;
  if (p > 1 && p <= max_pos) {
    po_prefill(m, cache, prompt, p - 1);
    start_pos = p - 1;
    token = prompt[p - 1];
  }
  for (size_t pos = start_pos; pos < max_pos; pos++) {
    int need = pos + 1 >= p && pos + 1 < max_pos;
    po_forward(m, cache, token, pos, need, logits);
    if (pos + 1 >= max_pos) break;
    uint32_t next = pos + 1 < p ? prompt[pos + 1] : po_argmax(logits, m->c.vocab_size);
    if (pos + 1 >= p) {
      if (is_stop(next, stops, n_stops)) break;
      out[generated++] = next;
    }
    token = next;
  }
  if (st) { st->prompt_tokens = p; st->generated_tokens = generated; st->proposed = st->accepted = 0; }
  free(logits);
  po_cache_free(cache);
  return generated;
}

/* ---- Sampler (sampler.rs:6-71) ---------------------------------------- */
/* XorShift::new / next_u64 / next_f32 (sampler.rs:55-71): xorshift64* with
 * shifts 12, 25, 27 and multiplier 0x2545F4914F6CDD1D; next_f32 takes the
 * top 24 bits / 2^24. */
uint64_t po_xorshift_seed(uint64_t seed) { return seed ? seed : 1; }
float po_xorshift_next_f32(uint64_t *state) {
  uint64_t x = *state;
  x ^= x >> 12;
  x ^= x << 25;
  x ^= x >> 27;
  *state = x;
  const uint64_t out = x * 0x2545F4914F6CDD1DULL;
  return (float)(out >> 40) / (float)(1ULL << 24);
}

/* The bucket walk of Sampler::sample (sampler.rs:29-36): r -= p[i] until
 * r <= 0; the last index when round-off leaves r above 0. */
uint32_t po_sample_pick(const float *probs, size_t n, float r) {
  for (size_t i = 0; i < n; i++) {
    r -= probs[i];
    if (r <= 0.0f) return (uint32_t)i;
  }
  return (uint32_t)(n - 1);
}

/* Sampler::sample (sampler.rs:22-39): greedy for temp <= 0, else logits /
 * temp, softmax, one uniform draw, the bucket walk. */
uint32_t po_sampler_sample(float temp, uint64_t *state, const float *logits, size_t n) {
  if (temp <= 0.0f) return po_argmax(logits, n);  /* Sampler::new: greedy iff temp <= 0 */
  float *scaled = malloc(n * 4), *probs = malloc(n * 4);
  for (size_t i = 0; i < n; i++) scaled[i] = logits[i] / temp;
  po_softmax(scaled, n, probs);
  const float r = po_xorshift_next_f32(state);
  const uint32_t t = po_sample_pick(probs, n, r);
  free(scaled);
  free(probs);
  return t;
}

/* generate (infer.rs:696-771) with a Sampler: teacher-forced prompt, then
 * sampled tokens; *state is the sampler's RNG and advances. */
size_t po_generate_sampled(const po_model *m, const uint32_t *prompt, size_t p, size_t steps, const uint32_t *stops,
                           size_t n_stops, float temp, uint64_t *state, uint32_t *out) {
  size_t max_pos = m->c.seq_len < p + steps ? m->c.seq_len : p + steps;
  po_cache *cache = po_cache_new(m, max_pos);
  float *logits = malloc(m->c.vocab_size * 4);
  uint32_t token = prompt[0];
  size_t generated = 0, start_pos = 0;
  if (p > 1 && p <= max_pos) {
    po_prefill(m, cache, prompt, p - 1);
    start_pos = p - 1;
    token = prompt[p - 1];
  }
  for (size_t pos = start_pos; pos < max_pos; pos++) {
    int need = pos + 1 >= p && pos + 1 < max_pos;
    po_forward(m, cache, token, pos, need, logits);
    if (pos + 1 >= max_pos) break;
    uint32_t next = pos + 1 < p ? prompt[pos + 1] : po_sampler_sample(temp, state, logits, m->c.vocab_size);
    if (pos + 1 >= p) {
      if (is_stop(next, stops, n_stops)) break;
      out[generated++] = next;
    }
    token = next;
  }
  free(logits);
  po_cache_free(cache);
  return generated;
}

/* generate_speculative (infer.rs:581-690) */
size_t po_generate_speculative(const po_model *target, const po_model *draft, const uint32_t *prompt, size_t p,
                               size_t steps, size_t k, const uint32_t *stops, size_t n_stops, uint32_t *out,
                               po_gen_stats *st) {
  size_t V = target->c.vocab_size;
  size_t max_pos = target->c.seq_len < p + steps ? target->c.seq_len : p + steps;
  po_cache *tc = po_cache_new(target, max_pos), *dc = po_cache_new(draft, max_pos);
  if (p > 1) {
    po_prefill(target, tc, prompt, p - 1);
    po_prefill(draft, dc, prompt, p - 1);
  }
  size_t pos = p - 1, generated = 0, proposed = 0, accepted = 0;
  uint32_t last = prompt[p - 1];
  float *dlog = malloc(draft->c.vocab_size * 4);
  uint32_t *drafts = malloc((k + 1) * 4), *inputs = malloc((k + 1) * 4);
  float *logits = malloc((k + 1) * V * 4);
  int done = 0;
  while (!done && pos + 1 < max_pos) {
    size_t budget = max_pos - 1 - pos < k ? max_pos - 1 - pos : k;
    uint32_t d_tok = last;
    for (size_t j = 0; j < budget; j++) {
      po_forward(draft, dc, d_tok, pos + j, 1, dlog);
      d_tok = po_argmax(dlog, draft->c.vocab_size);
      drafts[j] = d_tok;
    }
    proposed += budget;
    inputs[0] = last;
    for (size_t j = 0; j < budget; j++) inputs[j + 1] = drafts[j];
    po_forward_batch(target, tc, inputs, budget + 1, pos, logits);
    for (size_t i = 0; i <= budget; i++) {
      uint32_t tn = po_argmax(logits + i * V, V);
      if (i < budget && tn == drafts[i]) accepted++;
      if (is_stop(tn, stops, n_stops)) { done = 1; break; }
      out[generated++] = tn;
      pos += 1;
      last = tn;
      if (generated >= steps || pos + 1 >= max_pos) { done = 1; break; }
      if (i == budget || tn != drafts[i]) break;
    }
  }
  if (st) { st->prompt_tokens = p; st->generated_tokens = generated; st->proposed = proposed; st->accepted = accepted; }
  free(dlog); free(drafts); free(inputs); free(logits);
  po_cache_free(tc); po_cache_free(dc);
  return generated;
}
