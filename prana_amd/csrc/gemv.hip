// Packed-weight matrix x quantized-activation products (decode GEMV and the
// row-outer batched form).
//
// Exactness contract (the scalar tier, matmul.rs:395-406, kquant.rs:240-318):
// every output is a fold `acc = 0; for each term in element order: acc += term`
// where a term is a few f32 products of per-block scales and one exact i32
// block dot. The i32 dots are order-free and run 4-wide on v_dot4_i32_i8; the
// f32 terms are computed in parallel; only the fold is sequential, one lane per
// output, reading the terms back from LDS in block order.
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace prana {

size_t devmat_bytes(const DevMat& m) {
  size_t n = m.rows * m.cols;
  switch (m.kind) {
    case kKindF32: return n * 4;
    case kKindQ8F: return n + n / 32 * 4;
    case kKindQ8_0: return n / 32 * 34;
    case kKindQ4_0: return n / 32 * 18;
    case kKindQ4_K: return n / 256 * 144;
    case kKindQ6_K: return n / 256 * 210;
  }
  return 0;
}

size_t terms_per_row(const DevMat& m) { return m.kind == kKindQ6_K ? m.cols / 16 : m.cols / 32; }

namespace {

constexpr int kMask = 0x0F0F0F0F;

__device__ __forceinline__ float ld_f16(const void* p, size_t i) {
  return f16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
}

// Activation block view in LDS: words w[cols/4] (i8x4), scales sa[G], sums sm[G].
struct Acts {
  const int* w;
  const float* sa;
  const int* sm;
};

template <int KIND>
struct Fmt;

// Q8 (f32 or f16 block scale): term = (sw*sa)*float(acc)   (matmul.rs:404)
template <int KIND>
struct Q8Fmt {
  static constexpr int kUnit = 32, kTpu = 1;
  __device__ static int isum(const DevMat& m, size_t r, int b, const Acts& a) {
    const int4* wp = reinterpret_cast<const int4*>(m.qs + r * m.cols + (size_t)b * 32);
    int4 w0 = wp[0], w1 = wp[1];
    const int* aw = a.w + b * 8;
    int s = 0;
    s = sdot4(w0.x, aw[0], s);
    s = sdot4(w0.y, aw[1], s);
    s = sdot4(w0.z, aw[2], s);
    s = sdot4(w0.w, aw[3], s);
    s = sdot4(w1.x, aw[4], s);
    s = sdot4(w1.y, aw[5], s);
    s = sdot4(w1.z, aw[6], s);
    s = sdot4(w1.w, aw[7], s);
    return s;
  }
  __device__ static void terms(const DevMat& m, size_t r, int b, const Acts& a, float* t) {
    size_t G = m.cols / 32;
    float d = KIND == kKindQ8F ? reinterpret_cast<const float*>(m.sc)[r * G + b] : ld_f16(m.sc, r * G + b);
    t[0] = d * a.sa[b] * static_cast<float>(isum(m, r, b, a));
  }
  __device__ static void isums(const DevMat& m, size_t r, int b, const Acts& a, int* o) { o[0] = isum(m, r, b, a); }
};
template <>
struct Fmt<kKindQ8F> : Q8Fmt<kKindQ8F> {};
template <>
struct Fmt<kKindQ8_0> : Q8Fmt<kKindQ8_0> {};

// Q4_0: term = (d*sa)*float(s - 8*sum_a); element j<16 = low nibble of byte j,
// element 16+j = high nibble (kquant.rs:240-252).
template <>
struct Fmt<kKindQ4_0> {
  static constexpr int kUnit = 32, kTpu = 1;
  __device__ static int isum(const DevMat& m, size_t r, int b, const Acts& a) {
    size_t G = m.cols / 32;
    int4 w = *reinterpret_cast<const int4*>(m.qs + (r * G + b) * 16);
    const int* aw = a.w + b * 8;
    int s = 0;
    s = sdot4(w.x & kMask, aw[0], s);
    s = sdot4(w.y & kMask, aw[1], s);
    s = sdot4(w.z & kMask, aw[2], s);
    s = sdot4(w.w & kMask, aw[3], s);
    s = sdot4((w.x >> 4) & kMask, aw[4], s);
    s = sdot4((w.y >> 4) & kMask, aw[5], s);
    s = sdot4((w.z >> 4) & kMask, aw[6], s);
    s = sdot4((w.w >> 4) & kMask, aw[7], s);
    return s - 8 * a.sm[b];
  }
  __device__ static void terms(const DevMat& m, size_t r, int b, const Acts& a, float* t) {
    size_t G = m.cols / 32;
    float d = ld_f16(m.sc, r * G + b);
    t[0] = d * a.sa[b] * static_cast<float>(isum(m, r, b, a));
  }
  __device__ static void isums(const DevMat& m, size_t r, int b, const Acts& a, int* o) { o[0] = isum(m, r, b, a); }
};

// Q4_K super-block (144 B): 8 groups of 32; pair p's 32 bytes hold group 2p
// in the low nibbles and 2p+1 in the high nibbles. Per group:
// term = sa*((d*sc)*float(s) - (dmin*m)*float(sum_a))   (kquant.rs:257-282)
template <>
struct Fmt<kKindQ4_K> {
  static constexpr int kUnit = 256, kTpu = 8;
  __device__ static void scale_min(int j, const uint8_t* s, int& sc, int& mn) {
    if (j < 4) {
      sc = s[j] & 63;
      mn = s[j + 4] & 63;
    } else {
      sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
      mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
  }
  __device__ static int gsum(const int* qw, int g, const int* aw) {
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      int w = qw[(g >> 1) * 8 + i];
      int nib = (g & 1) ? ((w >> 4) & kMask) : (w & kMask);
      s = sdot4(nib, aw[i], s);
    }
    return s;
  }
  __device__ static void terms(const DevMat& m, size_t r, int b, const Acts& a, float* t) {
    size_t nb = m.cols / 256;
    const uint8_t* blk = m.qs + (r * nb + b) * 144;
    float d = f16_to_f32(static_cast<uint16_t>(blk[0] | (blk[1] << 8)));
    float dmin = f16_to_f32(static_cast<uint16_t>(blk[2] | (blk[3] << 8)));
    const int* qw = reinterpret_cast<const int*>(blk + 16);
#pragma unroll
    for (int g = 0; g < 8; g++) {
      int gi = b * 8 + g;
      int s = gsum(qw, g, a.w + gi * 8);
      int sc, mn;
      scale_min(g, blk + 4, sc, mn);
      t[g] = a.sa[gi] * (d * static_cast<float>(sc) * static_cast<float>(s) -
                         dmin * static_cast<float>(mn) * static_cast<float>(a.sm[gi]));
    }
  }
  __device__ static void isums(const DevMat& m, size_t r, int b, const Acts& a, int* o) {
    size_t nb = m.cols / 256;
    const int* qw = reinterpret_cast<const int*>(m.qs + (r * nb + b) * 144 + 16);
    for (int g = 0; g < 8; g++) o[g] = gsum(qw, g, a.w + (b * 8 + g) * 8);
  }
};

// Q6_K super-block (208 B here + f16 d): 16 sub-blocks of 16 in element
// order; q = (ql nibble | qh 2 bits << 4) - 32;
// term = ((d*sa)*float(i8 scale))*float(isum16)   (kquant.rs:287-318)
template <>
struct Fmt<kKindQ6_K> {
  static constexpr int kUnit = 256, kTpu = 16;
  __device__ static int ssum(const uint8_t* blk, int half, int g, int sub, const int* aw) {
    int s = 0, ones = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      int l = sub * 16 + 4 * i;
      int qlw = *reinterpret_cast<const int*>(blk + half * 64 + (g & 1) * 32 + l);
      int nib = g < 2 ? (qlw & kMask) : ((qlw >> 4) & kMask);
      int qhw = *reinterpret_cast<const int*>(blk + 128 + half * 32 + l);
      int hb = (qhw >> (2 * g)) & 0x03030303;
      int qv = nib | (hb << 4);  // 0..63 per byte
      s = sdot4(qv, aw[i], s);
      ones = sdot4(0x01010101, aw[i], ones);
    }
    return s - 32 * ones;
  }
  __device__ static void terms(const DevMat& m, size_t r, int b, const Acts& a, float* t) {
    size_t nb = m.cols / 256;
    const uint8_t* blk = m.qs + (r * nb + b) * 208;
    float d = ld_f16(m.sc, r * nb + b);
    const int8_t* sc = reinterpret_cast<const int8_t*>(blk + 192);
#pragma unroll
    for (int half = 0; half < 2; half++)
#pragma unroll
      for (int g = 0; g < 4; g++) {
        float s_a = a.sa[b * 8 + half * 4 + g];
#pragma unroll
        for (int sub = 0; sub < 2; sub++) {
          const int* aw = a.w + (b * 256 + half * 128 + g * 32 + sub * 16) / 4;
          int is = half * 8 + g * 2 + sub;
          t[is] = d * s_a * static_cast<float>(sc[is]) * static_cast<float>(ssum(blk, half, g, sub, aw));
        }
      }
  }
  __device__ static void isums(const DevMat& m, size_t r, int b, const Acts& a, int* o) {
    size_t nb = m.cols / 256;
    const uint8_t* blk = m.qs + (r * nb + b) * 208;
    for (int half = 0; half < 2; half++)
      for (int g = 0; g < 4; g++)
        for (int sub = 0; sub < 2; sub++)
          o[half * 8 + g * 2 + sub] = ssum(blk, half, g, sub, a.w + (b * 256 + half * 128 + g * 32 + sub * 16) / 4);
  }
};

// Stage one token's quantized activations in LDS.
__device__ __forceinline__ Acts stage_acts(int* smem, const int8_t* q, const float* sa, const int* sums, int K,
                                           int tok) {
  int W = K / 4, G = K / 32;
  int* aw = smem;
  float* as = reinterpret_cast<float*>(aw + W);
  int* am = reinterpret_cast<int*>(as + G);
  const int* qw = reinterpret_cast<const int*>(q + (size_t)tok * K);
  for (int i = threadIdx.x; i < W; i += blockDim.x) aw[i] = qw[i];
  for (int i = threadIdx.x; i < G; i += blockDim.x) {
    as[i] = sa[(size_t)tok * G + i];
    am[i] = sums[(size_t)tok * G + i];
  }
  return Acts{aw, as, am};
}

__device__ __forceinline__ void store_out(const GemvOut& o, int tok, size_t r, float acc) {
  float* dst = o.out + (size_t)tok * o.ldo + r;
  if (o.residual)
    *dst = *dst + acc;
  else if (o.bias)
    *dst = acc + o.bias[r];
  else
    *dst = acc;
}

// grid: (ceil(rows/rt), n_tok). LDS: acts + rt x (T+1) terms.
template <int KIND>
__global__ __launch_bounds__(256) void gemv_kernel(DevMat m, const int8_t* __restrict__ q,
                                                   const float* __restrict__ sa, const int* __restrict__ sums,
                                                   GemvOut o, int rt) {
  extern __shared__ int smem[];
  using F = Fmt<KIND>;
  const int K = static_cast<int>(m.cols);
  const int tok = blockIdx.y;
  Acts a = stage_acts(smem, q, sa, sums, K, tok);
  const int T = K / F::kUnit * F::kTpu;
  const int TS = T + 1;
  const int U = K / F::kUnit;
  float* terms = reinterpret_cast<float*>(smem + K / 4 + 2 * (K / 32));
  __syncthreads();
  const size_t r0 = (size_t)blockIdx.x * rt;
  for (int u = threadIdx.x; u < rt * U; u += blockDim.x) {
    int rr = u / U, b = u % U;
    size_t r = r0 + rr;
    if (r < m.rows) F::terms(m, r, b, a, terms + rr * TS + b * F::kTpu);
  }
  __syncthreads();
  if ((int)threadIdx.x < rt) {
    size_t r = r0 + threadIdx.x;
    if (r < m.rows) {
      const float* t = terms + threadIdx.x * TS;
      float acc = 0.0f;
      for (int i = 0; i < T; i++) acc += t[i];
      store_out(o, tok, r, acc);
    }
  }
}

// ===================================================================
// Decode GEMV (v2): few tokens, weights streamed once, loads issued a stage
// ahead, exact per-row fold in block order.
//
// A workgroup (256 lanes) owns RT rows of up to three matrices that share one
// input (fused Q|K|V, gate|up). The K dimension is walked in stages: in each
// stage every lane holds U storage units of weights in registers (loaded one
// stage ahead), computes their f32 terms against the LDS-staged activations
// and writes them to LDS; then one lane per (token, row) folds the stage's
// terms in block order. The fold lanes carry their accumulators across
// stages, so each output is exactly the reference's left-to-right sum.
// ===================================================================

// Raw storage units held in registers.
template <int KIND>
struct RegUnit;

template <>
struct RegUnit<kKindQ4_0> {
  static constexpr int kUnits = 8;  // units per lane per stage
  int4 q;
  uint32_t d;
  __device__ void load(const DevMat& m, size_t r, int b) {
    size_t G = m.cols / 32;
    q = *reinterpret_cast<const int4*>(m.qs + (r * G + b) * 16);
    d = reinterpret_cast<const uint16_t*>(m.sc)[r * G + b];
  }
  __device__ void terms(const Acts& a, int b, float* t) const {
    const int* aw = a.w + b * 8;
    int s = 0;
    s = sdot4(q.x & kMask, aw[0], s);
    s = sdot4(q.y & kMask, aw[1], s);
    s = sdot4(q.z & kMask, aw[2], s);
    s = sdot4(q.w & kMask, aw[3], s);
    s = sdot4((q.x >> 4) & kMask, aw[4], s);
    s = sdot4((q.y >> 4) & kMask, aw[5], s);
    s = sdot4((q.z >> 4) & kMask, aw[6], s);
    s = sdot4((q.w >> 4) & kMask, aw[7], s);
    s -= 8 * a.sm[b];
    t[0] = f16_to_f32(static_cast<uint16_t>(d)) * a.sa[b] * static_cast<float>(s);
  }
};

template <int KIND>
struct RegUnitQ8 {
  static constexpr int kUnits = 4;
  int4 q0, q1;
  uint32_t d;  // f16 bits or f32 bits
  __device__ void load(const DevMat& m, size_t r, int b) {
    size_t G = m.cols / 32;
    const int4* p = reinterpret_cast<const int4*>(m.qs + r * m.cols + (size_t)b * 32);
    q0 = p[0];
    q1 = p[1];
    d = KIND == kKindQ8F ? reinterpret_cast<const uint32_t*>(m.sc)[r * G + b]
                         : reinterpret_cast<const uint16_t*>(m.sc)[r * G + b];
  }
  __device__ void terms(const Acts& a, int b, float* t) const {
    const int* aw = a.w + b * 8;
    int s = 0;
    s = sdot4(q0.x, aw[0], s);
    s = sdot4(q0.y, aw[1], s);
    s = sdot4(q0.z, aw[2], s);
    s = sdot4(q0.w, aw[3], s);
    s = sdot4(q1.x, aw[4], s);
    s = sdot4(q1.y, aw[5], s);
    s = sdot4(q1.z, aw[6], s);
    s = sdot4(q1.w, aw[7], s);
    float dv = KIND == kKindQ8F ? __uint_as_float(d) : f16_to_f32(static_cast<uint16_t>(d));
    t[0] = dv * a.sa[b] * static_cast<float>(s);
  }
};
template <>
struct RegUnit<kKindQ8_0> : RegUnitQ8<kKindQ8_0> {};
template <>
struct RegUnit<kKindQ8F> : RegUnitQ8<kKindQ8F> {};

template <>
struct RegUnit<kKindQ4_K> {
  static constexpr int kUnits = 1;
  int4 v[9];
  __device__ void load(const DevMat& m, size_t r, int b) {
    size_t nb = m.cols / 256;
    const int4* p = reinterpret_cast<const int4*>(m.qs + (r * nb + b) * 144);
#pragma unroll
    for (int i = 0; i < 9; i++) v[i] = p[i];
  }
  __device__ void terms(const Acts& a, int b, float* t) const {
    const uint8_t* blk = reinterpret_cast<const uint8_t*>(v);
    float d = f16_to_f32(static_cast<uint16_t>(blk[0] | (blk[1] << 8)));
    float dmin = f16_to_f32(static_cast<uint16_t>(blk[2] | (blk[3] << 8)));
    const int* qw = reinterpret_cast<const int*>(blk + 16);
#pragma unroll
    for (int g = 0; g < 8; g++) {
      int gi = b * 8 + g;
      int s = Fmt<kKindQ4_K>::gsum(qw, g, a.w + gi * 8);
      int sc, mn;
      Fmt<kKindQ4_K>::scale_min(g, blk + 4, sc, mn);
      t[g] = a.sa[gi] * (d * static_cast<float>(sc) * static_cast<float>(s) -
                         dmin * static_cast<float>(mn) * static_cast<float>(a.sm[gi]));
    }
  }
};

template <>
struct RegUnit<kKindQ6_K> {
  static constexpr int kUnits = 1;
  int4 v[13];
  uint32_t d;
  __device__ void load(const DevMat& m, size_t r, int b) {
    size_t nb = m.cols / 256;
    const int4* p = reinterpret_cast<const int4*>(m.qs + (r * nb + b) * 208);
#pragma unroll
    for (int i = 0; i < 13; i++) v[i] = p[i];
    d = reinterpret_cast<const uint16_t*>(m.sc)[r * nb + b];
  }
  __device__ void terms(const Acts& a, int b, float* t) const {
    const uint8_t* blk = reinterpret_cast<const uint8_t*>(v);
    float dv = f16_to_f32(static_cast<uint16_t>(d));
    const int8_t* sc = reinterpret_cast<const int8_t*>(blk + 192);
#pragma unroll
    for (int half = 0; half < 2; half++)
#pragma unroll
      for (int g = 0; g < 4; g++) {
        float s_a = a.sa[b * 8 + half * 4 + g];
#pragma unroll
        for (int sub = 0; sub < 2; sub++) {
          const int* aw = a.w + (b * 256 + half * 128 + g * 32 + sub * 16) / 4;
          int is = half * 8 + g * 2 + sub;
          t[is] = dv * s_a * static_cast<float>(sc[is]) *
                  static_cast<float>(Fmt<kKindQ6_K>::ssum(blk, half, g, sub, aw));
        }
      }
  }
};

struct DecodeJob {
  DevMat m[3];
  GemvOut o[3];
  int n_mats;
  int tiles[3];  // row tiles per matrix (prefix-summed at launch)
  // act mode: m[0] = gate, m[1] = up (equal shapes); each workgroup owns the
  // same rt rows of both, and writes h = silu(g)*u (or gelu) quantized.
  int act;       // 0 none, 1 silu*up, 2 gelu*up
  float* h;      // optional f32 h [n][rows]
  int8_t* hq;
  float* hsa;
  int* hsum;
};

constexpr int kDecRT = 16;    // rows per matrix per workgroup (act mode: 32)
constexpr int kDecMaxTok = 4;

// LDS layout: acts [n][K bytes + 8*G] | terms [n][ROWS][S*TPU + 1].
// Lane mapping per stage: unit u of lane t covers (slot = u*(256/S) + t/S,
// unit t%S of the stage), so a wave reads contiguous runs of one row.
template <int KIND, bool ACT>
__global__ __launch_bounds__(256) void gemv_decode_kernel(DecodeJob job, const int8_t* __restrict__ q,
                                                          const float* __restrict__ sa,
                                                          const int* __restrict__ sums, int n_tok) {
  extern __shared__ int smem[];
  using R = RegUnit<KIND>;
  using F = Fmt<KIND>;
  constexpr int U = R::kUnits;
  constexpr int UNIT = F::kUnit, TPU = F::kTpu;
  constexpr int RT = ACT ? 32 : kDecRT;      // rows per matrix
  constexpr int ROWS = ACT ? 2 * RT : RT;    // rows held by the workgroup
  constexpr int S = 256 * U / ROWS;          // units per row per stage
  constexpr int LPS = 256 / S;               // slots covered per unit index
  constexpr int TS = S * TPU + 1;            // padded term row
  static_assert(S * LPS == 256 && U * LPS == ROWS, "tile shape");
  const int tid = threadIdx.x;

  int mi = 0, tile = blockIdx.x;
  if (!ACT) {
    while (mi < job.n_mats - 1 && tile >= job.tiles[mi]) tile -= job.tiles[mi++];
  }
  const int K = static_cast<int>(job.m[0].cols);
  const int G = K / 32, W = K / 4;
  const int upr = K / UNIT;
  const int n_stages = (upr + S - 1) / S;
  const size_t r0 = (size_t)tile * RT;

  const int act_words = (K + 8 * G) / 4;
  for (int t = 0; t < n_tok; t++) {
    int* aw = smem + t * act_words;
    float* as = reinterpret_cast<float*>(aw + W);
    int* am = reinterpret_cast<int*>(as + G);
    const int* qw = reinterpret_cast<const int*>(q + (size_t)t * K);
    for (int i = tid; i < W; i += 256) aw[i] = qw[i];
    for (int i = tid; i < G; i += 256) {
      as[i] = sa[(size_t)t * G + i];
      am[i] = sums[(size_t)t * G + i];
    }
  }
  float* terms = reinterpret_cast<float*>(smem + n_tok * act_words);

  const int bb = tid % S;       // unit within the stage (same for every u)
  const int slot0 = tid / S;
  // Per unit index: matrix and row (compile-time matrix choice in act mode).
  bool live[U];
  size_t rowi[U];
#pragma unroll
  for (int u = 0; u < U; u++) {
    int slot = u * LPS + slot0;
    int which = ACT ? slot / RT : mi;
    int rr = ACT ? slot % RT : slot;
    rowi[u] = r0 + rr;
    live[u] = rowi[u] < job.m[which].rows;
  }

  R buf0[U], buf1[U];
  __syncthreads();  // activations staged

#define PRANA_LOAD_STAGE(BUF, STG)                                          \
  do {                                                                     \
    int b_ = (STG) * S + bb;                                               \
    if (b_ < upr) {                                                        \
      _Pragma("unroll") for (int u = 0; u < U; u++) {                      \
        int which_ = ACT ? (u * LPS + slot0) / RT : mi;                    \
        if (live[u]) BUF[u].load(job.m[which_], rowi[u], b_);              \
      }                                                                    \
    }                                                                      \
  } while (0)

  const int fl_tok = tid / ROWS, fl_slot = tid % ROWS;
  const bool folder = tid < n_tok * ROWS;
  float acc = 0.0f;

  auto process = [&](const R* buf, int stg) {
    const int b = stg * S + bb;
    const int s_units = min(S, upr - stg * S);
    if (b < upr) {
      for (int t = 0; t < n_tok; t++) {
        int* aw = smem + t * act_words;
        float* as = reinterpret_cast<float*>(aw + W);
        int* am = reinterpret_cast<int*>(as + G);
        Acts a{aw, as, am};
        float* tt = terms + t * ROWS * TS;
#pragma unroll
        for (int u = 0; u < U; u++)
          if (live[u]) buf[u].terms(a, b, tt + (u * LPS + slot0) * TS + bb * TPU);
      }
    }
    __syncthreads();
    if (folder) {
      const float* tr = terms + fl_tok * ROWS * TS + fl_slot * TS;
      const int nt = s_units * TPU;
      int i = 0;
      for (; i + 4 <= nt; i += 4) {
        float t0 = tr[i], t1 = tr[i + 1], t2 = tr[i + 2], t3 = tr[i + 3];
        acc += t0;
        acc += t1;
        acc += t2;
        acc += t3;
      }
      for (; i < nt; i++) acc += tr[i];
    }
    __syncthreads();
  };

  PRANA_LOAD_STAGE(buf0, 0);
  for (int stg = 0; stg < n_stages; stg += 2) {
    if (stg + 1 < n_stages) PRANA_LOAD_STAGE(buf1, stg + 1);
    process(buf0, stg);
    if (stg + 1 >= n_stages) break;
    if (stg + 2 < n_stages) PRANA_LOAD_STAGE(buf0, stg + 2);
    process(buf1, stg + 1);
  }
#undef PRANA_LOAD_STAGE

  if (!ACT) {
    if (folder) {
      size_t r = r0 + fl_slot;
      if (r < job.m[mi].rows) store_out(job.o[mi], fl_tok, r, acc);
    }
    return;
  }
  // act epilogue: gate lanes (slot < RT) pair with up lanes (slot + RT);
  // h = act(g) * u, then quantize each 32-row block (one 32-lane group).
  float* hx = terms;
  if (folder) hx[fl_tok * ROWS + fl_slot] = acc;
  __syncthreads();
  const size_t H = job.m[0].rows;
  if (tid < n_tok * ROWS) {
    const bool gate_lane = fl_slot < RT;
    size_t r = r0 + fl_slot;
    bool lv = gate_lane && r < H;
    float v = 0.0f;
    if (gate_lane) {
      float g = acc, u = hx[fl_tok * ROWS + RT + fl_slot];
      if (job.act == 2) {
        const float kS = 0.7978846f;
        float x3 = g * g * g;
        g = 0.5f * g * (1.0f + tanhf(kS * (g + 0.044715f * x3)));
      } else {
        g = g * (1.0f / (1.0f + dev_expf(-g)));
      }
      v = g * u;
      if (lv && job.h) job.h[fl_tok * H + r] = v;
    }
    float scale;
    int sum;
    int qi = quantize_lane(lv ? v : 0.0f, &scale, &sum);
    if (lv) {
      size_t gi = fl_tok * H + r;
      job.hq[gi] = static_cast<int8_t>(qi);
      if ((gi & 31) == 0) {
        job.hsa[gi >> 5] = scale;
        job.hsum[gi >> 5] = sum;
      }
    }
  }
}

template <int KIND>
int launch_decode_t(DecodeJob job, const int8_t* q, const float* sa, const int* sums, size_t n_tok, hipStream_t s) {
  using R = RegUnit<KIND>;
  using F = Fmt<KIND>;
  const bool act = job.act != 0;
  const int rt = act ? 32 : kDecRT;
  const int rows_wg = act ? 2 * rt : rt;
  const size_t K = job.m[0].cols;
  const int S = 256 * R::kUnits / rows_wg;
  const size_t act_bytes = K + 8 * (K / 32);
  const size_t term_bytes = (size_t)rows_wg * (S * F::kTpu + 1) * 4;
  int total = 0;
  if (act) {
    total = static_cast<int>((job.m[0].rows + rt - 1) / rt);
  } else {
    for (int i = 0; i < job.n_mats; i++) {
      job.tiles[i] = static_cast<int>((job.m[i].rows + rt - 1) / rt);
      total += job.tiles[i];
    }
  }
  const size_t per_tok = act_bytes + term_bytes;
  const size_t group = std::min<size_t>(kDecMaxTok, (64 * 1024) / per_tok);
  PRANA_CHECK(group >= 1, "gemv: decode tile exceeds LDS");
  for (size_t t0 = 0; t0 < n_tok; t0 += group) {
    size_t nt = std::min<size_t>(group, n_tok - t0);
    size_t lds = nt * per_tok;
    DecodeJob j = job;
    for (int i = 0; i < 3; i++)
      if (j.o[i].out) j.o[i].out += t0 * j.o[i].ldo;
    if (act) {
      size_t H = j.m[0].rows;
      if (j.h) j.h += t0 * H;
      j.hq += t0 * H;
      j.hsa += t0 * H / 32;
      j.hsum += t0 * H / 32;
    }
    size_t G = K / 32;
    if (act)
      hipLaunchKernelGGL((gemv_decode_kernel<KIND, true>), dim3(total), dim3(256), lds, s, j, q + t0 * K,
                         sa + t0 * G, sums + t0 * G, (int)nt);
    else
      hipLaunchKernelGGL((gemv_decode_kernel<KIND, false>), dim3(total), dim3(256), lds, s, j, q + t0 * K,
                         sa + t0 * G, sums + t0 * G, (int)nt);
    PRANA_LAUNCH_CHECK();
  }
  return kOk;
}

template <int KIND>
__global__ __launch_bounds__(256) void isums_kernel(DevMat m, const int8_t* __restrict__ q,
                                                    const int* __restrict__ sums, int* __restrict__ out) {
  extern __shared__ int smem[];
  using F = Fmt<KIND>;
  const int K = static_cast<int>(m.cols);
  const int tok = blockIdx.y;
  // sa is unused by the integer parts; stage zeros in its place.
  int W = K / 4, G = K / 32;
  int* aw = smem;
  float* as = reinterpret_cast<float*>(aw + W);
  int* am = reinterpret_cast<int*>(as + G);
  const int* qw = reinterpret_cast<const int*>(q + (size_t)tok * K);
  for (int i = threadIdx.x; i < W; i += blockDim.x) aw[i] = qw[i];
  for (int i = threadIdx.x; i < G; i += blockDim.x) {
    as[i] = 0.0f;
    am[i] = sums[(size_t)tok * G + i];
  }
  __syncthreads();
  Acts a{aw, as, am};
  const int U = K / F::kUnit;
  const int T = U * F::kTpu;
  size_t r = blockIdx.x;
  for (int b = threadIdx.x; b < U; b += blockDim.x)
    F::isums(m, r, b, a, out + ((size_t)tok * m.rows + r) * T + b * F::kTpu);
}

// Dense f32 rows: dot_f32_scalar (matmul.rs:377-391) — four strided partial
// sums, combined ((a0+a1)+a2)+a3, then the tail. One lane per partial sum.
__global__ __launch_bounds__(256) void gemv_f32_kernel(DevMat m, const float* __restrict__ x, GemvOut o) {
  __shared__ float part[256];
  const int K = static_cast<int>(m.cols);
  const int tok = blockIdx.y;
  const int rr = threadIdx.x >> 2, l = threadIdx.x & 3;
  const size_t r = (size_t)blockIdx.x * 64 + rr;
  const float* xr = x + (size_t)tok * K;
  float acc = 0.0f;
  if (r < m.rows) {
    const float* w = reinterpret_cast<const float*>(m.qs) + r * K;
    const int chunks = K / 4;
    for (int i = 0; i < chunks; i++) acc += xr[i * 4 + l] * w[i * 4 + l];
  }
  part[threadIdx.x] = acc;
  __syncthreads();
  if (l == 0 && r < m.rows) {
    const float* w = reinterpret_cast<const float*>(m.qs) + r * K;
    float sum = part[threadIdx.x] + part[threadIdx.x + 1] + part[threadIdx.x + 2] + part[threadIdx.x + 3];
    for (int i = (K / 4) * 4; i < K; i++) sum += xr[i] * w[i];
    store_out(o, tok, r, sum);
  }
}

template <int KIND>
int launch_q(const DevMat& m, const int8_t* q, const float* sa, const int* sums, size_t n_tok, const GemvOut& o,
             hipStream_t s) {
  using F = Fmt<KIND>;
  const size_t K = m.cols;
  const size_t T = K / F::kUnit * F::kTpu;
  const size_t act_bytes = K + 8 * (K / 32);
  const size_t budget = 64 * 1024;
  PRANA_CHECK(act_bytes + (T + 1) * 4 <= budget, "gemv: cols too large for the LDS tile");
  int rt = 16;
  while (rt > 1 && act_bytes + (size_t)rt * (T + 1) * 4 > budget) rt >>= 1;
  size_t lds = act_bytes + (size_t)rt * (T + 1) * 4;
  dim3 grid((m.rows + rt - 1) / rt, n_tok);
  hipLaunchKernelGGL(gemv_kernel<KIND>, grid, dim3(256), lds, s, m, q, sa, sums, o, rt);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

template <int KIND>
int launch_isums_t(const DevMat& m, const int8_t* q, const int* sums, size_t n_tok, int* out, hipStream_t s) {
  size_t lds = m.cols + 8 * (m.cols / 32);
  PRANA_CHECK(lds <= 64 * 1024, "isums: cols too large");
  hipLaunchKernelGGL(isums_kernel<KIND>, dim3(m.rows, n_tok), dim3(256), lds, s, m, q, sums, out);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

}  // namespace

namespace {
template <class F>
int dispatch_kind(int kind, F&& f) {
  switch (kind) {
    case kKindQ8F: return f(std::integral_constant<int, kKindQ8F>());
    case kKindQ8_0: return f(std::integral_constant<int, kKindQ8_0>());
    case kKindQ4_0: return f(std::integral_constant<int, kKindQ4_0>());
    case kKindQ4_K: return f(std::integral_constant<int, kKindQ4_K>());
    case kKindQ6_K: return f(std::integral_constant<int, kKindQ6_K>());
  }
  return fail(kErrUnsupported, "gemv: no decode kernel for this matrix kind");
}
}  // namespace

constexpr size_t kDecodeMaxTokens = kGemvDecodeMaxTokens;

int launch_gemv_multi(const DevMat* ms, const GemvOut* os, int n, const int8_t* q, const float* sa, const int* sums,
                      size_t n_tok, hipStream_t s) {
  PRANA_CHECK(n >= 1 && n <= 3, "gemv_multi: 1..3 matrices");
  if (n_tok == 0) return kOk;
  for (int i = 1; i < n; i++)
    PRANA_CHECK(ms[i].kind == ms[0].kind && ms[i].cols == ms[0].cols, "gemv_multi: matrices must share kind and cols");
  if (ms[0].kind == kKindF32 || n_tok > kDecodeMaxTokens) {
    for (int i = 0; i < n; i++) {
      int rc = launch_gemv(ms[i], nullptr, q, sa, sums, n_tok, os[i], s);
      if (rc) return rc;
    }
    return kOk;
  }
  DecodeJob job{};
  for (int i = 0; i < n; i++) {
    job.m[i] = ms[i];
    job.o[i] = os[i];
  }
  job.n_mats = n;
  return dispatch_kind(ms[0].kind, [&](auto k) { return launch_decode_t<decltype(k)::value>(job, q, sa, sums, n_tok, s); });
}

int launch_gemv_act(const DevMat& gate, const DevMat& up, int act, const int8_t* q, const float* sa, const int* sums,
                    size_t n_tok, float* h, int8_t* hq, float* hsa, int* hsum, hipStream_t s) {
  PRANA_CHECK(gate.kind == up.kind && gate.rows == up.rows && gate.cols == up.cols, "gemv_act: gate/up mismatch");
  PRANA_CHECK(gate.rows % 32 == 0 && hq && hsa && hsum, "gemv_act: rows must be a multiple of 32");
  PRANA_CHECK(gate.kind != kKindF32 && n_tok <= kDecodeMaxTokens, "gemv_act: decode-sized quantized inputs only");
  if (n_tok == 0) return kOk;
  DecodeJob job{};
  job.m[0] = gate;
  job.m[1] = up;
  job.n_mats = 2;
  job.act = act == 1 ? 2 : 1;
  job.h = h;
  job.hq = hq;
  job.hsa = hsa;
  job.hsum = hsum;
  return dispatch_kind(gate.kind, [&](auto k) { return launch_decode_t<decltype(k)::value>(job, q, sa, sums, n_tok, s); });
}

int launch_gemv(const DevMat& m, const float* x, const int8_t* q, const float* sa, const int* sums, size_t n_tok,
                const GemvOut& o, hipStream_t s) {
  if (n_tok == 0 || m.rows == 0) return kOk;
  if (m.kind != kKindF32 && n_tok <= kDecodeMaxTokens) {
    DecodeJob job{};
    job.m[0] = m;
    job.o[0] = o;
    job.n_mats = 1;
    return dispatch_kind(m.kind, [&](auto k) { return launch_decode_t<decltype(k)::value>(job, q, sa, sums, n_tok, s); });
  }
  switch (m.kind) {
    case kKindF32: {
      PRANA_CHECK(x != nullptr, "gemv f32: dense activations required");
      dim3 grid((m.rows + 63) / 64, n_tok);
      hipLaunchKernelGGL(gemv_f32_kernel, grid, dim3(256), 0, s, m, x, o);
      PRANA_LAUNCH_CHECK();
      return kOk;
    }
    case kKindQ8F: return launch_q<kKindQ8F>(m, q, sa, sums, n_tok, o, s);
    case kKindQ8_0: return launch_q<kKindQ8_0>(m, q, sa, sums, n_tok, o, s);
    case kKindQ4_0: return launch_q<kKindQ4_0>(m, q, sa, sums, n_tok, o, s);
    case kKindQ4_K: return launch_q<kKindQ4_K>(m, q, sa, sums, n_tok, o, s);
    case kKindQ6_K: return launch_q<kKindQ6_K>(m, q, sa, sums, n_tok, o, s);
  }
  return fail(kErrUnsupported, "gemv: unknown matrix kind");
}

int launch_block_isums(const DevMat& m, const int8_t* q, const int* sums, size_t n_tok, int* out, hipStream_t s) {
  if (n_tok == 0 || m.rows == 0) return kOk;
  switch (m.kind) {
    case kKindQ8F: return launch_isums_t<kKindQ8F>(m, q, sums, n_tok, out, s);
    case kKindQ8_0: return launch_isums_t<kKindQ8_0>(m, q, sums, n_tok, out, s);
    case kKindQ4_0: return launch_isums_t<kKindQ4_0>(m, q, sums, n_tok, out, s);
    case kKindQ4_K: return launch_isums_t<kKindQ4_K>(m, q, sums, n_tok, out, s);
    case kKindQ6_K: return launch_isums_t<kKindQ6_K>(m, q, sums, n_tok, out, s);
  }
  return fail(kErrUnsupported, "block sums: dense matrices have no integer part");
}

}  // namespace prana
