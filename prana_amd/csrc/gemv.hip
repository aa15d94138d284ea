// Packed-weight matrix x quantized-activation products: the decode GEMV (up
// to 8 tokens per launch), the row-outer fallback, and the int8 matrix-core
// batched forms (skinny 16x16 tiles, LDS-staged 32x32 prefill tiles, K-quant
// super-block tiles).
//
// Exactness contract (the scalar tier, matmul.rs:395-406, kquant.rs:240-318):
// every output is a fold `acc = 0; for each term in element order: acc += term`
// where a term is a few f32 products of per-block scales and one exact i32
// block dot. The i32 dots are order-free and run 4-wide on v_dot4_i32_i8; the
// f32 terms are computed in parallel; only the fold is sequential, one lane per
// output, reading the terms back from LDS in block order.
#include <hip/hip_ext.h>

#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "common.h"
#include "exact_sum.h"
#include "kernels.h"

namespace prana {

LaunchEvents& launch_events() {
  thread_local LaunchEvents ev;
  return ev;
}

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

// One 32-element block of the activations out of LDS (its 32 int8 values, scale
// and sum), read once and shared by every unit of a lane that sits on the
// same block.
struct ActBlk {
  int4 a0, a1;
  float sa;
  int sm;
  __device__ static ActBlk at(const Acts& a, int b) {
    const int4* aw = reinterpret_cast<const int4*>(a.w) + b * 2;
    return ActBlk{aw[0], aw[1], a.sa[b], a.sm[b]};
  }
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
// Decode GEMV: few tokens, every weight byte read once.
//
// A workgroup (256 lanes) owns a tile of rows of one matrix (for the fused
// gate|up form, the same 32 rows of both) and walks the row blocks in stages
// of SB units. In each stage every lane holds U storage units in registers
// (the next stage's units are already in flight), computes their f32 terms
// for each token against the LDS-staged activations and writes them to LDS;
// one lane per (token, row) then folds the stage's terms in block order,
// carrying its accumulator across stages, so each output is exactly the
// reference's left-to-right sum. A lane's units sit at the same (row, block
// offset) in every stage, so their addresses are fixed 32-bit unit indices
// plus a per-stage step; partial tiles and stages clamp addresses instead of
// branching and skip the writes.
// ===================================================================

// Raw storage units held in registers: load(quant bytes, scale bytes) of one
// unit; terms() gives its kTpu f32 terms against the LDS activations.
template <int KIND>
struct RegUnit;

template <>
struct RegUnit<kKindQ4_0> {
  static constexpr int kQB = 16, kSB = 2, kTpu = 1, kElems = 32;
  int4 q;
  uint32_t d;
  __device__ void load(const uint8_t* qp, const uint8_t* sp) {
    q = *reinterpret_cast<const int4*>(qp);
    d = *reinterpret_cast<const uint16_t*>(sp);
  }
  // sum_j (nibble_j - 8) * qa_j over the block, from the stored nibbles
  // (unsigned, one dot per half) and the activations' sum
  __device__ int isum(const int4& a0, const int4& a1, int sm) const {
    int s = 0;
    s = sdot4(q.x & kMask, a0.x, s);
    s = sdot4(q.y & kMask, a0.y, s);
    s = sdot4(q.z & kMask, a0.z, s);
    s = sdot4(q.w & kMask, a0.w, s);
    s = sdot4((q.x >> 4) & kMask, a1.x, s);
    s = sdot4((q.y >> 4) & kMask, a1.y, s);
    s = sdot4((q.z >> 4) & kMask, a1.z, s);
    s = sdot4((q.w >> 4) & kMask, a1.w, s);
    return s - 8 * sm;
  }
  __device__ void terms_blk(const ActBlk& ab, float* t) const {
    t[0] = f16_to_f32(static_cast<uint16_t>(d)) * ab.sa * static_cast<float>(isum(ab.a0, ab.a1, ab.sm));
  }
  __device__ void terms(const Acts& a, int b, float* t) const { terms_blk(ActBlk::at(a, b), t); }
  // The block's integer dot s = sum_j (nibble_j - 8) * qa_j (|s| <= 32*8*127,
  // so 16 bits) packed above the block's f16 scale bits; term() of the word
  // and the activation scale gives terms()' value.
  __device__ int slot_blk(const ActBlk& ab) const {
    return static_cast<int>((d & 0xffffu) | (static_cast<uint32_t>(isum(ab.a0, ab.a1, ab.sm)) << 16));
  }
  __device__ int slot(const Acts& a, int b) const { return slot_blk(ActBlk::at(a, b)); }
  // (the scale only feeds this product, so f16_operand's conversion gives
  // f16_to_f32's result; see common.h)
  __device__ static float term(int w, float sa) {
    return f16_operand(static_cast<uint16_t>(w & 0xffff)) * sa * static_cast<float>(w >> 16);
  }
};

template <int KIND>
struct RegUnitQ8 {
  static constexpr int kQB = 32, kSB = KIND == kKindQ8F ? 4 : 2, kTpu = 1, kElems = 32;
  int4 q0, q1;
  uint32_t d;  // f16 bits or f32 bits
  __device__ void load(const uint8_t* qp, const uint8_t* sp) {
    const int4* p = reinterpret_cast<const int4*>(qp);
    q0 = p[0];
    q1 = p[1];
    d = KIND == kKindQ8F ? *reinterpret_cast<const uint32_t*>(sp) : *reinterpret_cast<const uint16_t*>(sp);
  }
  __device__ void terms_blk(const ActBlk& ab, float* t) const {
    int s = 0;
    s = sdot4(q0.x, ab.a0.x, s);
    s = sdot4(q0.y, ab.a0.y, s);
    s = sdot4(q0.z, ab.a0.z, s);
    s = sdot4(q0.w, ab.a0.w, s);
    s = sdot4(q1.x, ab.a1.x, s);
    s = sdot4(q1.y, ab.a1.y, s);
    s = sdot4(q1.z, ab.a1.z, s);
    s = sdot4(q1.w, ab.a1.w, s);
    float dv = KIND == kKindQ8F ? __uint_as_float(d) : f16_to_f32(static_cast<uint16_t>(d));
    t[0] = dv * ab.sa * static_cast<float>(s);
  }
  __device__ void terms(const Acts& a, int b, float* t) const { terms_blk(ActBlk::at(a, b), t); }
};
template <>
struct RegUnit<kKindQ8_0> : RegUnitQ8<kKindQ8_0> {};
template <>
struct RegUnit<kKindQ8F> : RegUnitQ8<kKindQ8F> {};

template <>
struct RegUnit<kKindQ4_K> {
  static constexpr int kQB = 144, kSB = 0, kTpu = 8, kElems = 256;
  int4 v[9];
  __device__ void load(const uint8_t* qp, const uint8_t*) {
    const int4* p = reinterpret_cast<const int4*>(qp);
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
  static constexpr int kQB = 208, kSB = 2, kTpu = 16, kElems = 256;
  int4 v[13];
  uint32_t d;
  __device__ void load(const uint8_t* qp, const uint8_t* sp) {
    const int4* p = reinterpret_cast<const int4*>(qp);
#pragma unroll
    for (int i = 0; i < 13; i++) v[i] = p[i];
    d = *reinterpret_cast<const uint16_t*>(sp);
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
  int tiles[3];  // row tiles per matrix
  int rt;        // rows per matrix per tile
  int sb;        // units per row per stage
  // act mode: m[0] = gate, m[1] = up (equal shapes, rt = 32); each tile owns
  // the same rows of both and writes h = silu(g)*u (or gelu) quantized.
  int act;       // 0 none, 1 silu*up, 2 gelu*up
  float* h;      // optional f32 h [n][rows]
  int8_t* hq;
  float* hsa;
  int* hsum;
  // one-token Q|K|V (m = q, k, v): rope and the cache rows in the epilogue
  // when rk.table is set (tiles then hold whole rotation pairs)
  RopeKv rk;
  // one token: the activations are rmsnorm(nin.x) quantized, computed by
  // every workgroup (NORM kernels) instead of read from q / sa / sums
  NormIn nin;
};

constexpr int kDecMaxTok = 8;   // tokens per launch (LDS and folder lanes permitting)
constexpr int kActRows = 32;    // act-mode rows per matrix of a staged tile: one quantization block
constexpr int kNormNT = 1024;    // lanes of a NORM workgroup for rows of 1025..4096 values (one per CU)
constexpr int kNormNTSmall = 256;  // ... for rows of 513..1024 values
constexpr int kNormMaxK = 4096;  // NORM rows: four values per lane
constexpr int kSplitUAct = 4;    // units per unit lane per stage of a split gate|up launch (two stages in registers)
constexpr int kSplitMaxStages = 16;
constexpr int kSplitStage0 = 5;    // first stage counter in the split launch's LDS words
constexpr int kSplitSB = kNormNT / 2 * kSplitUAct / 128;  // blocks per row per stage of a split launch
constexpr int kXchPolls = 1 << 16; // bound on a split launch's wait for workgroup 0's norm

// A tile's bound on its wait for the norm workgroup: kXchPolls unless
// PRANA_SPLIT_WAIT_POLLS sets it (0 sends every tile to its own evaluation of
// the sum, the path a wait that runs out takes; the tests use it).
int split_wait_polls() {
  const char* e = std::getenv("PRANA_SPLIT_WAIT_POLLS");  // (read per launch; a replayed graph keeps its value)
  return e ? std::max(0, std::atoi(e)) : kXchPolls;
}

// Handoff words of a split launch, xch = {64-bit word, ..., one flag word per
// tile}: the norm workgroup publishes the word, each tile sets its flag once
// it is done with the word, and the norm workgroup, once every flag is set (or
// its wait runs out), sets the word and the flags back to zero for the next
// launch in the stream. A tile that finds the word zero for longer than its
// own wait evaluates the sum itself, so a late reader costs time, never bits.
constexpr int kXchIn = 64;  // words: the tiles' count-in flags
constexpr int kXchMaxTiles = 512;
static_assert((kXchIn + kXchMaxTiles) * 4 <= static_cast<int>(kNormXchBytes), "handoff words fit the buffer");

// Each tile sets its own flag word with a device-scope store (many workgroups
// adding to one counter serialise at its address); one wave of the norm
// workgroup waits for all of them, lanes reading 64 apart. Bounded.
__device__ __forceinline__ void split_count_in(unsigned* xch, int tile) {
  __hip_atomic_store(xch + kXchIn + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void split_wait_counted(const unsigned* xch, int n) {
  const int lane = threadIdx.x & 63;
  for (int polls = 0; polls < kXchPolls; polls++) {
    bool all = true;
    for (int i = lane; i < n; i += 64)
      all &= __hip_atomic_load(const_cast<unsigned*>(xch) + kXchIn + i, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT) != 0u;
    if (__builtin_amdgcn_ballot_w64(!all) == 0) return;
    __builtin_amdgcn_s_sleep(8);
  }
}

// Orders this wave's LDS accesses before the ones that follow (a wait for
// its outstanding LDS operations plus a compiler barrier) without waiting for
// its global loads, which a workgroup-scope fence would also do.
__device__ __forceinline__ void lds_order() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt and expcnt left at their maximum
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// LDS: acts [n_tok][astride bytes] | terms [nbuf][n_tok][ROWS][SB*TPU + 1].
// STAGED: more than one stage (double-buffered registers and terms);
// otherwise the whole row tile is one stage. NT lanes per workgroup.
// The workgroup's tile: matrix mi (tiles are numbered matrix after matrix)
// and its row tile.
__device__ __forceinline__ void job_tile(const DecodeJob& job, int* mi, int* tile) {
  *mi = 0;
  *tile = blockIdx.x;
  while (*mi < job.n_mats - 1 && *tile >= job.tiles[*mi]) *tile -= job.tiles[(*mi)++];
}

// NORM (one token, K <= 4 * NT): the activations are rmsnorm(job.nin.x)
// quantized, as launch_rmsnorm would produce them, computed in the prologue
// while this workgroup's first weight loads are in flight; the row and the
// sum's terms use the term region of LDS, which the fold reuses afterwards.
// SPLIT (NORM at kNormNT lanes): waves 0..7 compute the norm, eight values
// per lane, and later fold the terms; waves 8..15 hold the weight units and
// keep up to two stages of them in flight from the start (see the prologue).
template <int KIND, int U, bool ACT, bool STAGED, int NT, bool NORM = false, bool SPLIT = false>
__device__ __forceinline__ void gemv_tile_body(const DecodeJob& job, const int8_t* __restrict__ q,
                                               const float* __restrict__ sa, const int* __restrict__ sums,
                                               int n_tok, int mi, int tile) {
  static_assert(!NORM || NT == kNormNT || NT == kNormNTSmall, "NORM workgroups of 256 or 1024 lanes");
  static_assert(!SPLIT || (NORM && NT == kNormNT), "split norm launches are 1024-lane NORM launches");
  if constexpr (NORM) n_tok = 1;  // a constant the token loops fold away
  extern __shared__ int4 smem4[];
  using R = RegUnit<KIND>;
  constexpr int TPU = R::kTpu;
  const int tid = threadIdx.x;
  constexpr int NTL = SPLIT ? NT / 2 : NT;          // lanes holding weight units
  // SPLIT: norm-wave barrier, flag, marked blocks, the handoff's inv bits and
  // outcome, then one completion count per stage (unit waves that have stored
  // the stage's dots)
  __shared__ int s_dfr[SPLIT ? kSplitStage0 + kSplitMaxStages : 1];
  const int lt = SPLIT ? tid - NT / 2 : tid;        // this lane's index among them
  const bool loader = !SPLIT || tid >= NT / 2;      // (uniform per wave)
  const int rt = job.rt, SB = job.sb;
  const int ROWS = ACT ? 2 * rt : rt;
  const int K = static_cast<int>(job.m[0].cols);
  const int nb = K / R::kElems, G = K / 32;
  const int n_stages = (nb + SB - 1) / SB;
  const size_t rows_m = job.m[mi].rows;
  const size_t r0 = (size_t)tile * rt;
  const int rows_here = static_cast<int>(min((size_t)rt, rows_m - r0));

  // ---- this lane's units: (matrix, row, block offset), fixed for all stages
  const uint8_t* qbase[ACT ? 2 : 1];
  const uint8_t* sbase[ACT ? 2 : 1];
#pragma unroll
  for (int j = 0; j < (ACT ? 2 : 1); j++) {
    qbase[j] = job.m[ACT ? j : mi].qs;
    sbase[j] = static_cast<const uint8_t*>(job.m[ACT ? j : mi].sc);
  }
  // unit i of this lane: v = tid + NT*i -> (row, block offset) = divmod(v, SB),
  // recomputed where needed (cheaper in registers than keeping U pairs),
  // except in NORM launches, which work out the pairs before the norm so
  // that the divisions stay off the path from the norm to the terms.
  constexpr bool kPairs = NORM;
  int urow[kPairs ? U : 1], uoff[kPairs ? U : 1];
  if constexpr (kPairs) {
#pragma unroll
    for (int i = 0; i < U; i++) {
      urow[i] = (lt + NTL * i) / SB;
      uoff[i] = (lt + NTL * i) % SB;
    }
  }
  auto unit_row = [&](int i) {
    if constexpr (kPairs) return urow[i];
    else return (lt + NTL * i) / SB;
  };
  auto unit_off = [&](int i) {
    if constexpr (kPairs) return uoff[i];
    else return (lt + NTL * i) % SB;
  };
  auto unit_up = [&](int i) { return ACT && unit_row(i) >= rt; };
  auto unit_lr = [&](int i) { return unit_up(i) ? unit_row(i) - rt : unit_row(i); };
  auto load_stage = [&](R* buf, int s) {
    if (!loader) return;
#pragma unroll
    for (int i = 0; i < U; i++) {
      int row = unit_row(i), off = unit_off(i);
      if constexpr (NORM) {
        // rebuild each stage's addresses from the 32-bit unit indices: kept
        // across the norm, the hoisted 64-bit pointers would spill
        asm volatile("" : "+v"(row), "+v"(off));
      }
      const bool up = ACT && row >= rt;
      const int lr = up ? row - rt : row;
      const int blk = min(s * SB + off, nb - 1);
      const size_t rr = r0 + min(lr, rows_here - 1);
      const size_t ui = rr * nb + blk;
      const int j = up ? 1 : 0;
      buf[i].load(qbase[ACT ? j : 0] + ui * R::kQB, sbase[ACT ? j : 0] + ui * R::kSB);
    }
  };

  // token 0's activations go into registers first (the oldest loads), then
  // the weights; the rest of the tokens are staged after the weights.
  const int astride = ((K + 8 * G) + 15) & ~15;
  constexpr int kAw4 = (16384 / 16 + NT - 1) / NT;  // int4 words per lane, K <= 16384
  constexpr int kAg = (512 + NT - 1) / NT;          // block scales per lane
  int4 a0w[NORM ? 1 : kAw4];
  float a0s[NORM ? 1 : kAg];
  int a0m[NORM ? 1 : kAg];
  // NORM: elements 4*tid .. 4*tid+3 of the row (K <= 4 * NT, K % 32 == 0)
  const bool nlive = NORM && 4 * tid < K;
  float4 nx4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), nw4 = nx4;
  if constexpr (NORM) {
    if (nlive) {
      nx4 = reinterpret_cast<const float4*>(job.nin.x)[tid];
      nw4 = reinterpret_cast<const float4*>(job.nin.w)[tid];
    }
  } else {
    const int4* qw = reinterpret_cast<const int4*>(q);
#pragma unroll
    for (int i = 0; i < kAw4; i++) {
      const int w = tid + NT * i;
      a0w[i] = w < K / 16 ? qw[w] : make_int4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < kAg; i++) {
      const int g = tid + NT * i;
      a0s[i] = g < G ? sa[g] : 0.0f;
      a0m[i] = g < G ? sums[g] : 0;
    }
  }
  R buf0[U];
  R buf1[STAGED ? U : 1];
  uint8_t* sm8 = reinterpret_cast<uint8_t*>(smem4);
  if (!NORM) {
    load_stage(buf0, 0);
    if (STAGED && n_stages > 1) load_stage(buf1, 1);
  }
  float pacc = 0.0f;  // SPLIT: a row lane's fold, when the norm waves fold during the stream
  if constexpr (NORM && SPLIT) {
    // Deferred block scales (one token, Q4_0, K <= 4096). A block's term is
    // (d*sa)*float(s) with s an exact integer dot of the weights and the
    // quantized activations q; sa depends on the norm's exact sum of squares
    // (norms.rs:15), which takes microseconds, but q hardly does: q_i =
    // round(y_i * 127/amax) is a ratio of values that all scale with the
    // norm's factor. So:
    //   waves 0..7  load the row, quantize y = x*w (the norm's factor left
    //               out: q is a ratio within each block, so it hardly
    //               depends on it), publish that q through LDS, each wave
    //               counting itself in a flag; then evaluate the exact sum
    //               (eight values per lane, synchronising through an LDS
    //               counter), the exact y, scales and q, and mark every
    //               32-block whose q differs from the published one;
    //   waves 8..15 stream the weight units (two stages in flight from the
    //               start) and, once the flag is up, store each (row, block)
    //               dot with its f16 scale in LDS as the bytes arrive.
    // After one workgroup barrier the marked blocks' dots are recomputed
    // from the exact q (their units re-read), and one lane per row folds
    // (d*sa)*float(s) in block order with the exact scales: the reference's
    // terms in the reference's order, whatever the approximation gave.
    static_assert(KIND == kKindQ4_0, "deferred block scales: Q4_0 units");
    const int SR = nb + 1;                                     // padded slot row
    int* slots = reinterpret_cast<int*>(sm8 + astride);        // [ROWS][SR]
    float* xs = reinterpret_cast<float*>(sm8 + astride + (size_t)ROWS * SR * 4);  // row (one-lane fallback)
    int8_t* qx = reinterpret_cast<int8_t*>(xs + exact::run_pad(K - 1) + 1);       // exact q
    float* sx = reinterpret_cast<float*>(qx + K);              // exact block scales
    int* smx = reinterpret_cast<int*>(sx + G);                 // exact block sums
    int* mism = smx + G;                                       // 1: the block's q changed
    int& s_nbar = s_dfr[0];
    int& s_flag = s_dfr[1];
    int& s_nmis = s_dfr[2];
    const bool nl = !loader && 8 * tid < K;
    float nx[8], nw[8];
    if (nl) {
      const float4* x4 = reinterpret_cast<const float4*>(job.nin.x) + 2 * tid;
      const float4* w4 = reinterpret_cast<const float4*>(job.nin.w) + 2 * tid;
      const float4 a = x4[0], b = x4[1], c = w4[0], d = w4[1];
      nx[0] = a.x, nx[1] = a.y, nx[2] = a.z, nx[3] = a.w, nx[4] = b.x, nx[5] = b.y, nx[6] = b.z, nx[7] = b.w;
      nw[0] = c.x, nw[1] = c.y, nw[2] = c.z, nw[3] = c.w, nw[4] = d.x, nw[5] = d.y, nw[6] = d.z, nw[7] = d.w;
    } else {
#pragma unroll
      for (int j = 0; j < 8; j++) nx[j] = nw[j] = 0.0f;
    }
    if (tid < kSplitStage0 + kSplitMaxStages) s_dfr[tid] = 0;
    // the row loads are issued before this barrier, the weight loads after it
    __syncthreads();
    float* as_a = reinterpret_cast<float*>(sm8 + K);
    int* am_a = reinterpret_cast<int*>(as_a + G);
    if (loader) {
      load_stage(buf0, 0);
      if (STAGED && n_stages > 1) load_stage(buf1, 1);
      for (int polls = 0; polls < (1 << 22); polls++) {  // bounded: the norm waves count in early
        if (__hip_atomic_load(&s_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= NT / 2 / 64) break;
        __builtin_amdgcn_s_sleep(1);
      }
      lds_order();  // (not a workgroup fence: that would also wait for this wave's weight loads)
      const Acts a{reinterpret_cast<const int*>(sm8), as_a, am_a};
      auto stage_done = [&](int st) {  // this wave's dots of stage st are in LDS
        lds_order();
        if ((tid & 63) == 0) __hip_atomic_fetch_add(&s_dfr[kSplitStage0 + st], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      };
      // (the split geometry has NTL % SB == 0: all of a lane's units sit on
      // block offset lt % SB and share one read of its activations)
      auto slot_stage = [&](const R* buf, int st) {
        const int off = unit_off(0);
        const int blk = st * SB + off;
        if (blk < nb) {
          const ActBlk av = ActBlk::at(a, blk);
#pragma unroll
          for (int i = 0; i < U; i++) {
            const int row = unit_row(i);
            const int lr = ACT && row >= rt ? row - rt : row;
            if (lr < rows_here) slots[row * SR + blk] = buf[i].slot_blk(av);
          }
        }
      };
      if (!STAGED) {
        slot_stage(buf0, 0);
        stage_done(0);
      } else {
        for (int st = 0; st < n_stages; st += 2) {
          slot_stage(buf0, st);
          stage_done(st);
          if (st + 2 < n_stages) load_stage(buf0, st + 2);
          if (st + 1 >= n_stages) break;
          slot_stage(buf1, st + 1);
          stage_done(st + 1);
          if (st + 3 < n_stages) load_stage(buf1, st + 3);
        }
      }
    } else {
      exact::LdsGroupBarrier bar{&s_nbar, NT / 2 / 64, 0};
      // the staged row serves the exact sum's one-lane fallback only
      if (nl) {
#pragma unroll
        for (int j = 0; j < 8; j++) xs[exact::run_pad(8 * tid + j)] = nx[j];
      }
      float t8[8];
#pragma unroll
      for (int j = 0; j < 8; j++) t8[j] = nx[j] * nx[j];  // zero on lanes past K
      float y[8], sc;
      int qa[8], qe[8], sm;
#pragma unroll
      for (int j = 0; j < 8; j++) y[j] = nx[j] * nw[j];
      quantize_oct4(y, qa, &sc, &sm);  // K % 32 == 0: 4-lane groups are all live or all past K
      auto pack4 = [](const int* v) {
        return (v[0] & 0xff) | ((v[1] & 0xff) << 8) | ((v[2] & 0xff) << 16) | (static_cast<int>(v[3]) << 24);
      };
      if (nl) {
        int* qw = reinterpret_cast<int*>(sm8) + 2 * tid;
        qw[0] = pack4(qa);
        qw[1] = pack4(qa + 4);
        if ((tid & 3) == 0) am_a[tid >> 2] = sm;
      }
      lds_order();  // this wave's q is in LDS
      if ((tid & 63) == 0) __hip_atomic_fetch_add(&s_flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      // exact: norms.rs:9-23 in the reference's order, then quantize_acts.
      // Every workgroup normalises the same row, so with a handoff buffer
      // the launch's extra workgroup 0 (dispatched first) evaluates the sum
      // and the tiles wait for its inv = 1/sqrt(ss/K + eps), their norm
      // waves idle instead of competing with the unit waves for issue slots.
      // A wait that runs out evaluates the sum here instead (same bits).
      auto exact_inv = [&]() {
        const float ss = exact::lanes_seq_sum<NT / 2, 8>(t8, K, tid, bar, [xs](int i) {
          const float v = xs[exact::run_pad(i)];
          return v * v;
        });
        const float mean_sq = ss / static_cast<float>(K);
        return 1.0f / sqrtf(mean_sq + job.nin.eps);
      };
      // The handoff word holds (1 << 32) | bits(inv) once published, so one
      // single-copy-atomic 64-bit load gives the flag and the value together;
      // relaxed device-scope accesses throughout (an acquire would invalidate
      // the caches that the weight stream runs through on every poll).
      unsigned long long* const xch = reinterpret_cast<unsigned long long*>(job.nin.xch);
      float inv;
      {
        if (tid == 0) {
          unsigned long long w = 0;
          for (int polls = 0; polls < job.nin.xch_polls; polls++) {
            w = __hip_atomic_load(&xch[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (w >> 32) break;
            __builtin_amdgcn_s_sleep(2);
          }
          s_dfr[3] = static_cast<int>(w & 0xffffffffu);
          s_dfr[4] = static_cast<int>(w >> 32);
        }
        bar();  // the handoff's outcome is in LDS
        inv = s_dfr[4] ? __int_as_float(s_dfr[3]) : exact_inv();  // (uniform)
      }
      if (tid == 0) split_count_in(job.nin.xch, static_cast<int>(blockIdx.x) - 1);
#pragma unroll
      for (int j = 0; j < 8; j++) y[j] = nl ? nx[j] * inv * nw[j] : 0.0f;
      quantize_oct4(y, qe, &sc, &sm);
      int diff = 0;
#pragma unroll
      for (int j = 0; j < 8; j++) diff |= qe[j] != qa[j];
      diff |= dpp_lane_mov<0xB1>(diff);  // the block's four lanes
      diff |= dpp_lane_mov<0x4E>(diff);
      if (nl) {
        int* qw = reinterpret_cast<int*>(qx) + 2 * tid;
        qw[0] = pack4(qe);
        qw[1] = pack4(qe + 4);
        if ((tid & 3) == 0) {
          sx[tid >> 2] = sc;
          smx[tid >> 2] = sm;
          mism[tid >> 2] = diff;
          if (diff) __hip_atomic_fetch_add(&s_nmis, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
      }
      bar();  // every block's exact scale and mark is in LDS
      const int unit_waves = NT / 2 / 64;
      auto stage_wait = [&](int st) {  // until the unit waves have stored stage st
        for (int polls = 0; polls < (1 << 22); polls++) {
          if (__hip_atomic_load(&s_dfr[kSplitStage0 + st], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= unit_waves)
            break;
          __builtin_amdgcn_s_sleep(1);
        }
        lds_order();
      };
      if (s_nmis == 0) {
        // no block changed q: the row lanes fold each stage's terms
        // (d*sa)*float(s) in block order as soon as it is stored, so that
        // only the last stage's adds remain once the weights are in
        if (tid < ROWS) {
          const int lr = ACT && tid >= rt ? tid - rt : tid;
          const int* sr = slots + tid * SR;
          for (int st = 0; st < n_stages; st++) {
            stage_wait(st);
            const int b0 = st * SB;
            if (lr >= rows_here) continue;
            if (b0 + kSplitSB <= nb && SB == kSplitSB) {
              int w[kSplitSB];
              float sc16[kSplitSB];
#pragma unroll
              for (int j = 0; j < kSplitSB; j++) {
                w[j] = sr[b0 + j];
                sc16[j] = sx[b0 + j];
              }
#pragma unroll
              for (int j = 0; j < kSplitSB; j++) pacc += R::term(w[j], sc16[j]);
            } else {
              for (int b = b0; b < min(b0 + SB, nb); b++) pacc += R::term(sr[b], sx[b]);
            }
          }
        }
      } else {
        // the norm waves turn each stage's (row, block) words into f32 terms
        // as soon as the unit waves have stored the stage; the marked blocks
        // are recomputed after the workgroup barrier, then folded with the
        // rest. Lane l takes block column l % SB of the stage and every
        // (NT/2)/SB-th row.
        float* tf = reinterpret_cast<float*>(slots);
        for (int st = 0; st < n_stages; st++) {
          stage_wait(st);
          const int b = st * SB + tid % SB;
          if (b < nb) {
            const float scale = sx[b];
            for (int row = tid / SB; row < ROWS; row += NT / 2 / SB) {
              const int i = row * SR + b;
              tf[i] = R::term(slots[i], scale);
            }
          }
        }
      }
    }
  } else if constexpr (NORM) {
    // norms.rs:9-23 on this workgroup: the sum of squares in the reference's
    // left-to-right order (evaluated exactly), ms = ss/dim, inv =
    // 1/sqrt(ms+eps), y = (x*inv)*w, then quantize_acts' 32-blocks. The
    // weight loads go out once the row is here: issued with it, they would
    // queue ahead of it, and the norm outlasts them either way.
    float* xs = reinterpret_cast<float*>(sm8 + astride);
    const float nx[4] = {nx4.x, nx4.y, nx4.z, nx4.w}, nw[4] = {nw4.x, nw4.y, nw4.z, nw4.w};
    if (nlive) {
#pragma unroll
      for (int j = 0; j < 4; j++) xs[exact::run_pad(4 * tid + j)] = nx[j];
    }
    __builtin_amdgcn_sched_barrier(0);
    load_stage(buf0, 0);
    // the squares from registers; the staged row serves the sum's one-lane
    // fallback only (its first barrier publishes it)
    float t4[4];
#pragma unroll
    for (int j = 0; j < 4; j++) t4[j] = nlive && 4 * tid + j < K ? nx[j] * nx[j] : 0.0f;
    const float ss = exact::quad_seq_sum<NT>(t4, K, [xs](int i) {
      const float v = xs[exact::run_pad(i)];
      return v * v;
    });
    const float mean_sq = ss / static_cast<float>(K);
    const float inv = 1.0f / sqrtf(mean_sq + job.nin.eps);
    // The second stage goes out once the sum is done: its registers are
    // needed by the sum, and a second stage of loads issued before the norm
    // stalls the waves at issue (the CU's outstanding loads are full), which
    // delays the norm by more than the earlier loads save; issued by the idle
    // waves during the sum's final one-wave walk it was slower too (measured
    // on the 7B gate|up).
    if (STAGED && n_stages > 1) load_stage(buf1, 1);
    float y[4], sc;
    int qi[4], sm;
#pragma unroll
    for (int j = 0; j < 4; j++) y[j] = nlive ? nx[j] * inv * nw[j] : 0.0f;
    quantize_quad8(y, qi, &sc, &sm);  // K % 32 == 0: 8-lane groups are all live or all past K
    float* as = reinterpret_cast<float*>(sm8 + K);
    int* am = reinterpret_cast<int*>(as + G);
    if (nlive) {
      reinterpret_cast<int*>(sm8)[tid] =
          (qi[0] & 0xff) | ((qi[1] & 0xff) << 8) | ((qi[2] & 0xff) << 16) | (static_cast<int>(qi[3]) << 24);
      if ((tid & 7) == 0) {
        as[tid >> 3] = sc;
        am[tid >> 3] = sm;
      }
    }
  } else {
    int4* aw = reinterpret_cast<int4*>(sm8);
    float* as = reinterpret_cast<float*>(sm8 + K);
    int* am = reinterpret_cast<int*>(as + G);
#pragma unroll
    for (int i = 0; i < kAw4; i++) {
      const int w = tid + NT * i;
      if (w < K / 16) aw[w] = a0w[i];
    }
#pragma unroll
    for (int i = 0; i < kAg; i++) {
      const int g = tid + NT * i;
      if (g < G) {
        as[g] = a0s[i];
        am[g] = a0m[i];
      }
    }
  }
  for (int t = 1; t < n_tok; t++) {
    int4* aw = reinterpret_cast<int4*>(sm8 + t * astride);
    float* as = reinterpret_cast<float*>(sm8 + t * astride + K);
    int* am = reinterpret_cast<int*>(as + G);
    const int4* qw = reinterpret_cast<const int4*>(q + (size_t)t * K);
    for (int i = tid; i < K / 16; i += NT) aw[i] = qw[i];
    for (int i = tid; i < G; i += NT) {
      as[i] = sa[(size_t)t * G + i];
      am[i] = sums[(size_t)t * G + i];
    }
  }
  const int TS = SB * TPU + 1;  // padded term row
  float* terms = reinterpret_cast<float*>(sm8 + n_tok * astride);
  const int buf_floats = n_tok * ROWS * TS;
  __syncthreads();

  const int fl_tok = tid / ROWS, fl_row = tid % ROWS;
  const int fl_lr = ACT ? (fl_row >= rt ? fl_row - rt : fl_row) : fl_row;
  const bool folder = tid < n_tok * ROWS && fl_lr < rows_here;
  float acc = 0.0f;

  auto process = [&](const R* buf, int s) {
    float* tb = terms + (s & 1) * buf_floats;
    bool shared = false;
    if constexpr (R::kElems == 32) shared = NTL % SB == 0;
    if (shared) {
      // every unit of this lane sits on block offset lt % SB: one read of
      // that activation block per token serves all U of them
      int off = unit_off(0);
      if constexpr (NORM) asm volatile("" : "+v"(off));  // as in load_stage
      const int blk = s * SB + off;
      if (loader && blk < nb) {
        for (int t = 0; t < n_tok; t++) {
          const uint8_t* ab = sm8 + t * astride;
          const ActBlk av = ActBlk::at(Acts{reinterpret_cast<const int*>(ab), reinterpret_cast<const float*>(ab + K),
                                            reinterpret_cast<const int*>(ab + K) + G},
                                       blk);
#pragma unroll
          for (int i = 0; i < U; i++) {
            int row = unit_row(i);
            if constexpr (NORM) asm volatile("" : "+v"(row));
            const int lr = ACT && row >= rt ? row - rt : row;
            if constexpr (R::kElems == 32)
              if (lr < rows_here) buf[i].terms_blk(av, tb + (t * ROWS + row) * TS + off * TPU);
          }
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < U; i++) {
        int row = unit_row(i), off = unit_off(i);
        if constexpr (NORM) asm volatile("" : "+v"(row), "+v"(off));  // as in load_stage
        const int lr = ACT && row >= rt ? row - rt : row;
        const int blk = s * SB + off;
        if (loader && blk < nb && lr < rows_here) {
          for (int t = 0; t < n_tok; t++) {
            const uint8_t* ab = sm8 + t * astride;
            Acts a{reinterpret_cast<const int*>(ab), reinterpret_cast<const float*>(ab + K),
                   reinterpret_cast<const int*>(ab + K) + G};
            buf[i].terms(a, blk, tb + (t * ROWS + row) * TS + off * TPU);
          }
        }
      }
    }
    __syncthreads();
    if (folder) {
      const float* tr = tb + (fl_tok * ROWS + fl_row) * TS;
      const int cnt = min(SB, nb - s * SB) * TPU;
      int i = 0;
      for (; i + 8 <= cnt; i += 8) {
        float x0 = tr[i], x1 = tr[i + 1], x2 = tr[i + 2], x3 = tr[i + 3];
        float x4 = tr[i + 4], x5 = tr[i + 5], x6 = tr[i + 6], x7 = tr[i + 7];
        acc += x0;
        acc += x1;
        acc += x2;
        acc += x3;
        acc += x4;
        acc += x5;
        acc += x6;
        acc += x7;
      }
      for (; i < cnt; i++) acc += tr[i];
    }
  };

  if constexpr (SPLIT) {
    // the deferred terms: every (row, block) dot is in LDS (see the prologue)
    const int SR = nb + 1;
    int* slots = reinterpret_cast<int*>(sm8 + astride);
    const float* xs = reinterpret_cast<const float*>(sm8 + astride + (size_t)ROWS * SR * 4);
    const int8_t* qx = reinterpret_cast<const int8_t*>(xs + exact::run_pad(K - 1) + 1);
    const float* sx = reinterpret_cast<const float*>(qx + K);
    const int* smx = reinterpret_cast<const int*>(sx + G);
    const int* mism = smx + G;
    if (s_dfr[2] == 0) {  // (uniform) the row lanes folded every stage already
      if (folder) acc = pacc;
    } else {  // blocks the norm waves marked before the barrier above
      // a block whose exact q differs from the published one: its dots are
      // recomputed from the exact activations (units re-read from memory)
      const Acts ax{reinterpret_cast<const int*>(qx), sx, smx};
      for (int idx = tid; idx < ROWS * nb; idx += NT) {
        const int row = idx / nb, b = idx - row * nb;
        if (!mism[b]) continue;
        const bool up = ACT && row >= rt;
        const int lr = up ? row - rt : row;
        if (lr >= rows_here) continue;
        const size_t ui = (r0 + lr) * nb + b;
        const int j = up ? 1 : 0;
        R u;
        u.load(qbase[ACT ? j : 0] + ui * R::kQB, sbase[ACT ? j : 0] + ui * R::kSB);
        reinterpret_cast<float*>(slots)[row * SR + b] = R::term(u.slot(ax, b), sx[b]);
      }
      __syncthreads();
      // one lane per row folds the terms (formed by the norm waves) in block order
      const float* tf = reinterpret_cast<const float*>(slots);
      if (folder) {
        const float* tr = tf + fl_row * SR;
        int i = 0;
        for (; i + 8 <= nb; i += 8) {
          float x0 = tr[i], x1 = tr[i + 1], x2 = tr[i + 2], x3 = tr[i + 3];
          float x4 = tr[i + 4], x5 = tr[i + 5], x6 = tr[i + 6], x7 = tr[i + 7];
          acc += x0;
          acc += x1;
          acc += x2;
          acc += x3;
          acc += x4;
          acc += x5;
          acc += x6;
          acc += x7;
        }
        for (; i < nb; i++) acc += tr[i];
      }
    }
  } else if (!STAGED) {
    process(buf0, 0);
  } else {
    for (int s = 0; s < n_stages; s += 2) {
      process(buf0, s);
      if (s + 1 >= n_stages) break;
      if (s + 2 < n_stages) load_stage(buf0, s + 2);
      process(buf1, s + 1);
      if (s + 3 < n_stages) load_stage(buf1, s + 3);
    }
  }

  if (!ACT) {
    if (!job.rk.table) {
      if (folder) store_out(job.o[mi], fl_tok, r0 + fl_lr, acc);
      return;
    }
    // q/k/v + bias, exchanged through LDS for the rotation pairs; token t of
    // the batch sits at position pos + t
    __syncthreads();  // every fold read of the term buffers is done
    float* xv = reinterpret_cast<float*>(sm8) + fl_tok * ROWS;
    const GemvOut& o = job.o[mi];
    const size_t r = r0 + fl_lr;
    float val = 0.0f;
    if (folder) {
      val = o.bias ? acc + o.bias[r] : acc;
      xv[fl_lr] = val;
    }
    __syncthreads();
    if (folder) {
      const RopeKv& rk = job.rk;
      const int pos = (rk.pos_dev ? *rk.pos_dev : rk.pos) + fl_tok;
      const size_t crow = (size_t)pos * rows_m + r;  // k and v have kv_dim = rows_m rows
      float* out = o.out + (size_t)fl_tok * o.ldo;
      if (mi == 2) {
        out[r] = val;
        rk.vc[crow] = f32_to_f16(val);
      } else {
        const int half = rk.hd / 2;
        bool first;
        int lp, m;
        if (rk.neox) {  // pairs (j, j + hd/2) of a head; tiles start on head boundaries
          const int j = fl_lr % rk.hd;
          first = j < half;
          lp = first ? fl_lr + half : fl_lr - half;
          m = first ? j : j - half;
        } else {  // adjacent pairs; tiles start on even rows
          first = (fl_lr & 1) == 0;
          lp = fl_lr ^ 1;
          m = static_cast<int>((r & ~static_cast<size_t>(1)) % rk.hd) / 2;
        }
        float a = first ? val : xv[lp], b = first ? xv[lp] : val;
        rotate(a, b, rk.table[(size_t)pos * half + m]);
        const float y = first ? a : b;
        out[r] = y;
        if (mi == 1) rk.kc[kcache_index(pos, r, rows_m, rk.kcap)] = f32_to_f16(y);
      }
    }
    return;
  }
  // act epilogue: gate lanes (row < rt) pair with up lanes (row + rt);
  // h = act(g) * u. When the tile holds whole 32-row blocks (rt % 32 == 0),
  // each block is quantized here by one 32-lane group; otherwise the caller
  // quantizes h afterwards.
  __syncthreads();  // every fold read of the term buffers is done
  float* hx = terms;
  if (tid < n_tok * ROWS) hx[tid] = acc;
  __syncthreads();
  const size_t H = rows_m;
  if (tid < n_tok * ROWS) {
    const bool gate_lane = fl_row < rt;
    const size_t r = r0 + fl_row;
    const bool lv = gate_lane && fl_row < rows_here;
    float v = 0.0f;
    if (gate_lane) {
      float g = acc, u = hx[fl_tok * ROWS + rt + fl_row];
      if (job.act == 2) {
        const float kS = 0.7978846f;  // norms.rs:36
        float x3 = g * g * g;
        g = 0.5f * g * (1.0f + dev_tanhf(kS * (g + 0.044715f * x3)));
      } else {
        g = g * (1.0f / (1.0f + dev_expf(-g)));
      }
      v = g * u;
      if (lv && job.h) job.h[fl_tok * H + r] = v;
    }
    if (rt % 32 == 0) {  // whole waves take part (ROWS = 2*rt is a multiple of 64)
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
}

// The norm workgroup of a split gate|up launch with a handoff buffer: the
// exact left-to-right sum of squares of the row (norms.rs:15) over all NT
// lanes, four values each, then inv = 1/sqrt(ss/K + eps) (norms.rs:16-17)
// published as (1 << 32) | bits(inv) in the buffer's 64-bit word, where the
// tile workgroups wait for it. It streams no weights, so nothing competes
// with the sum for issue slots; it re-arms the words once the tiles have read
// them (split_count_in).
template <int NT>
__device__ __forceinline__ void split_norm_producer(const NormIn& nin, int K) {
  extern __shared__ int4 smem4[];
  float* xs = reinterpret_cast<float*>(smem4);  // the row (the sum's one-lane fallback)
  const int tid = threadIdx.x;
  const bool live = 4 * tid < K;
  float4 x4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (live) x4 = reinterpret_cast<const float4*>(nin.x)[tid];
  const float nx[4] = {x4.x, x4.y, x4.z, x4.w};
  if (live) {
#pragma unroll
    for (int j = 0; j < 4; j++) xs[exact::run_pad(4 * tid + j)] = nx[j];
  }
  float t4[4];
#pragma unroll
  for (int j = 0; j < 4; j++) t4[j] = nx[j] * nx[j];  // zero past K
  const float ss = exact::quad_seq_sum<NT>(t4, K, [xs](int i) {
    const float v = xs[exact::run_pad(i)];
    return v * v;
  });
  if (tid < 64) {  // publish inv; once every tile has read it, re-arm the words for the next launch
    unsigned long long* const word = reinterpret_cast<unsigned long long*>(nin.xch);
    if (tid == 0) {
      const float inv = 1.0f / sqrtf(ss / static_cast<float>(K) + nin.eps);
      __hip_atomic_store(word, (1ull << 32) | __float_as_uint(inv), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const int n = static_cast<int>(gridDim.x) - 1;
    split_wait_counted(nin.xch, n);
    for (int i = tid; i < n; i += 64)
      __hip_atomic_store(nin.xch + kXchIn + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid == 0) __hip_atomic_store(word, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <int KIND, int U, bool ACT, bool STAGED, int NT, bool NORM = false, bool SPLIT = false>
__global__ __launch_bounds__(NT) void gemv_tile_kernel(DecodeJob job, const int8_t* __restrict__ q,
                                                        const float* __restrict__ sa,
                                                        const int* __restrict__ sums, int n_tok) {
  int mi = 0, tile = blockIdx.x;
  if (!ACT) job_tile(job, &mi, &tile);
  if constexpr (SPLIT) {  // workgroup 0 evaluates the norm for the tiles, which start at 1
    if (blockIdx.x == 0) {
      split_norm_producer<NT>(job.nin, static_cast<int>(job.m[0].cols));
      return;
    }
    // Consecutive workgroups land on different XCDs (round robin); tile
    // numbers are dealt so that each XCD streams one contiguous run of rows
    // (every XCD then reads every memory channel alike).
    const int b = blockIdx.x - 1, nt = gridDim.x - 1;
    tile = nt % 8 == 0 ? (b % 8) * (nt / 8) + b / 8 : b;
  }
  // decode's one-token launches get a copy of the body in which the token
  // loops fold away (the branch is uniform)
  if (n_tok == 1) gemv_tile_body<KIND, U, ACT, STAGED, NT, NORM, SPLIT>(job, q, sa, sums, 1, mi, tile);
  else gemv_tile_body<KIND, U, ACT, STAGED, NT, NORM, SPLIT>(job, q, sa, sums, n_tok, mi, tile);
}

// Matrices of two formats with the same unit width and tile geometry in one
// launch (a fused Q|K|V whose v projection is stored in another format, as
// K-quant-mixture GGUF files store it): each workgroup runs the body of its
// matrix's format.
template <int KA, int KB, int U, bool STAGED, int NT, bool NORM = false>
__global__ __launch_bounds__(NT) void gemv_tile_mixed_kernel(DecodeJob job, const int8_t* __restrict__ q,
                                                              const float* __restrict__ sa,
                                                              const int* __restrict__ sums, int n_tok) {
  int mi, tile;
  job_tile(job, &mi, &tile);
  if (job.m[mi].kind == KA)
    gemv_tile_body<KA, U, false, STAGED, NT, NORM>(job, q, sa, sums, n_tok, mi, tile);
  else
    gemv_tile_body<KB, U, false, STAGED, NT, NORM>(job, q, sa, sums, n_tok, mi, tile);
}

// ---- verify batches: 2..8 tokens, 32-element formats
// Chunk-major units: with W = nb / U blocks per chunk and ROWS = 256 / W rows
// per tile (gate and up rows together in act mode), lane t's unit i is row
// t / W, block i*W + t % W, so chunk i of every row of the tile is one unit
// index. All weights are loaded at once, as in gemv_tile_kernel. The
// activations of every token are staged in LDS one chunk at a time (two
// chunk buffers; chunk c+2's loads are issued before chunk c's terms and
// stored once chunk c's buffer is free) and so are the term rows, so a
// workgroup holds two chunks of every token instead of whole rows per token
// and several workgroups fit per CU. The folder lane of (token, row) adds
// chunk c's W terms after chunk c-1's: the left-to-right block order of the
// one-token kernel, so both give the same bits.
constexpr int kKmNT = 256;
constexpr int kKmQ4 = 4;  // int4 words of one chunk's activations per lane (8 tokens x 64 blocks x 2 / 256)
constexpr int kKmSc = 2;  // (scale, sum) pairs of one chunk per lane (8 tokens x 64 blocks / 256)

struct KmActs {
  int4 q[kKmQ4];
  float s[kKmSc];
  int m[kKmSc];
};

template <int KIND, int U, bool ACT>
__global__ __launch_bounds__(kKmNT) void gemv_km_kernel(DecodeJob job, const int8_t* __restrict__ q,
                                                        const float* __restrict__ sa,
                                                        const int* __restrict__ sums, int n_tok) {
  using R = RegUnit<KIND>;
  static_assert(R::kElems == 32 && R::kTpu == 1, "32-element formats");
  extern __shared__ int4 smem4[];
  const int tid = threadIdx.x;
  int mi = 0, tile = blockIdx.x;
  if (!ACT) {
    while (mi < job.n_mats - 1 && tile >= job.tiles[mi]) tile -= job.tiles[mi++];
  }
  const int rt = job.rt;
  const int ROWS = ACT ? 2 * rt : rt;
  const int K = static_cast<int>(job.m[0].cols), nb = K / 32;
  const int W = job.sb;  // blocks per chunk: nb == U * W, ROWS * W == kKmNT
  const size_t rows_m = job.m[mi].rows;
  const size_t r0 = (size_t)tile * rt;
  const int rows_here = static_cast<int>(min((size_t)rt, rows_m - r0));
  const int lrow = tid / W, loff = tid % W;  // this lane's row in the tile and block in a chunk
  const bool lup = ACT && lrow >= rt;
  const int llr = lup ? lrow - rt : lrow;    // its row within its matrix
  const bool lane_live = llr < rows_here;

  const int CS = W * 40;  // bytes of one token's chunk: W*32 q, W*4 scales, W*4 sums
  const int TW = W + 1;   // padded term row
  uint8_t* sm8 = reinterpret_cast<uint8_t*>(smem4);
  float* tbase = reinterpret_cast<float*>(sm8 + 2 * n_tok * CS);
  const int G = nb;
  auto load_acts = [&](KmActs& ar, int c) {
    const int nq = n_tok * W * 2;
#pragma unroll
    for (int i = 0; i < kKmQ4; i++) {
      const int w = tid + kKmNT * i;
      if (w < nq) {
        const int t = w / (2 * W), r = w % (2 * W);
        ar.q[i] = reinterpret_cast<const int4*>(q + (size_t)t * K)[c * W * 2 + r];
      }
    }
    const int ns = n_tok * W;
#pragma unroll
    for (int i = 0; i < kKmSc; i++) {
      const int e = tid + kKmNT * i;
      if (e < ns) {
        const size_t gi = (size_t)(e / W) * G + c * W + e % W;
        ar.s[i] = sa[gi];
        ar.m[i] = sums[gi];
      }
    }
  };
  auto store_acts = [&](const KmActs& ar, int c) {
    uint8_t* base = sm8 + (c & 1) * n_tok * CS;
    const int nq = n_tok * W * 2;
#pragma unroll
    for (int i = 0; i < kKmQ4; i++) {
      const int w = tid + kKmNT * i;
      if (w < nq) reinterpret_cast<int4*>(base + (w / (2 * W)) * CS)[w % (2 * W)] = ar.q[i];
    }
    const int ns = n_tok * W;
#pragma unroll
    for (int i = 0; i < kKmSc; i++) {
      const int e = tid + kKmNT * i;
      if (e < ns) {
        uint8_t* tb = base + (e / W) * CS;
        reinterpret_cast<float*>(tb + W * 32)[e % W] = ar.s[i];
        reinterpret_cast<int*>(tb + W * 36)[e % W] = ar.m[i];
      }
    }
  };

  // chunks 0 and 1 of the activations first (the oldest loads), then every
  // weight unit of this lane
  KmActs ar[2];
  load_acts(ar[0], 0);
  if (U > 1) load_acts(ar[1], 1);
  R buf[U];
  {
    const uint8_t* qb = ACT ? (lup ? job.m[1].qs : job.m[0].qs) : job.m[mi].qs;
    const uint8_t* sb = static_cast<const uint8_t*>(ACT ? (lup ? job.m[1].sc : job.m[0].sc) : job.m[mi].sc);
    const size_t rr = r0 + min(llr, rows_here - 1);
#pragma unroll
    for (int i = 0; i < U; i++) {
      const size_t ui = rr * nb + i * W + loff;
      buf[i].load(qb + ui * R::kQB, sb + ui * R::kSB);
    }
  }
  store_acts(ar[0], 0);
  if (U > 1) store_acts(ar[1], 1);
  __syncthreads();

  const int fl_tok = tid / ROWS, fl_row = tid % ROWS;
  const int fl_lr = ACT ? (fl_row >= rt ? fl_row - rt : fl_row) : fl_row;
  const bool folder = tid < n_tok * ROWS && fl_lr < rows_here;
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < U; c++) {
    if (c + 2 < U) load_acts(ar[c & 1], c + 2);
    float* tb = tbase + (c & 1) * n_tok * ROWS * TW;
    if (lane_live) {
      const uint8_t* abuf = sm8 + (c & 1) * n_tok * CS;
      for (int t = 0; t < n_tok; t++) {
        const uint8_t* ab = abuf + t * CS;
        Acts a{reinterpret_cast<const int*>(ab), reinterpret_cast<const float*>(ab + W * 32),
               reinterpret_cast<const int*>(ab + W * 36)};
        buf[c].terms(a, loff, tb + (t * ROWS + lrow) * TW + loff);
      }
    }
    __syncthreads();  // chunk c's terms are in LDS; its activation buffer is free
    if (folder) {
      const float* tr = tb + (fl_tok * ROWS + fl_row) * TW;
      for (int i = 0; i < W; i++) acc += tr[i];
    }
    if (c + 2 < U) store_acts(ar[c & 1], c + 2);  // read by chunk c+2, after the next barrier
  }

  if (!ACT) {
    if (folder) store_out(job.o[mi], fl_tok, r0 + fl_lr, acc);
    return;
  }
  // act epilogue: gate lanes (row < rt) pair with up lanes (row + rt) through
  // LDS; h = act(g) * u goes out in f32 (tiles here hold fewer than 32 rows,
  // so the caller quantizes h)
  __syncthreads();  // every fold read of the term buffers is done
  float* hx = tbase;
  if (tid < n_tok * ROWS) hx[tid] = acc;
  __syncthreads();
  if (tid < n_tok * ROWS && fl_row < rt && fl_row < rows_here) {
    float g = acc, u = hx[fl_tok * ROWS + rt + fl_row];
    if (job.act == 2) {
      const float kS = 0.7978846f;  // norms.rs:36
      float x3 = g * g * g;
      g = 0.5f * g * (1.0f + dev_tanhf(kS * (g + 0.044715f * x3)));
    } else {
      g = g * (1.0f / (1.0f + dev_expf(-g)));
    }
    job.h[fl_tok * rows_m + r0 + fl_row] = g * u;
  }
}

// Tile geometry: units per lane per stage U, rows per matrix per tile rt,
// units per row per stage sb and lanes nt, with rows(tile) * sb == nt * U.
struct TileGeom {
  int u, rt, sb, nt;
};

template <int KIND>
TileGeom choose_geom(size_t K, bool act) {
  using R = RegUnit<KIND>;
  const int nb = static_cast<int>(K / R::kElems);
  const bool small_unit = R::kElems == 32;
  if (act) {  // rt rows of gate and of up: 2*rt rows x sb units = 256 * u
    const int cand_act[] = {4, 2, 8, 7, 1};
    for (int c = 0; small_unit && c < 5; c++) {  // one stage: whole rows per tile
      const int u = cand_act[c];
      if ((128 * u) % nb == 0 && 128 * u / nb <= kActRows) return TileGeom{u, 128 * u / nb, nb, 256};
    }
    if (small_unit) return TileGeom{8, kActRows, 32, 256};
    return TileGeom{1, kActRows, 4, 256};
  }
  const int cand_small[] = {4, 2, 1, 7, 8};
  const int cand_k[] = {1, 2};
  const int* cand = small_unit ? cand_small : cand_k;
  const int nc = small_unit ? 5 : 2;
  for (int c = 0; c < nc; c++) {  // one stage: whole rows per tile
    const int u = cand[c];
    if ((256 * u) % nb == 0 && 256 * u / nb <= 64) return TileGeom{u, 256 * u / nb, nb, 256};
  }
  if (small_unit) return TileGeom{2, 8, 64, 256};
  // K-quant rows of up to 64 super-blocks that no whole-row stage divides
  // (e.g. 19 for 4864-wide rows): one stage padded to the next power of two
  // (the spare slots clamp their loads and write nothing), so short matrices
  // still spread over many workgroups; at most 64 rows per tile keeps a
  // folder lane for every (token, row).
  int sb = 4;
  while (sb < nb) sb *= 2;
  if (sb <= 64) return TileGeom{1, 256 / sb, sb, 256};
  return TileGeom{1, 32, 8, 256};
}

// Tile geometry of a NORM launch (kNormNT lanes for rows of more than 1024
// values, kNormNTSmall up to 1024; whole rows per tile, 8..64 rows), or u == 0
// when none fits. Block-32 kinds only.
template <int KIND>
TileGeom norm_geom(size_t K) {
  const int nb = static_cast<int>(K / RegUnit<KIND>::kElems);
  if (RegUnit<KIND>::kElems != 32 || nb < 1 || K <= 512 || K > static_cast<size_t>(kNormMaxK))
    return TileGeom{0, 0, 0, 0};
  const int nt = K > 1024 ? kNormNT : kNormNTSmall;
  for (int u : {4, 2, 7}) {
    if (nt == kNormNT && u == 7) continue;  // not instantiated at 1024 lanes
    const int units = nt * u;
    if (units % nb == 0 && units / nb >= 8 && units / nb <= 64) return TileGeom{u, units / nb, nb, nt};
  }
  return TileGeom{0, 0, 0, 0};
}

// Act-mode (gate|up) geometry of a NORM launch: 64 rows of each matrix per
// tile (whole 32-row blocks, so h is quantized in the epilogue); beyond 1024
// values kNormNT lanes in stages of 32 blocks, four units per lane, up to
// 1024 values kNormNTSmall lanes in one stage (rows of 28 or 32 blocks); u == 0
// when the rows do not split so.
template <int KIND>
TileGeom norm_act_geom(size_t K) {
  const int nb = static_cast<int>(K / RegUnit<KIND>::kElems);
  if (RegUnit<KIND>::kElems != 32 || K <= 512 || K > static_cast<size_t>(kNormMaxK)) return TileGeom{0, 0, 0, 0};
  if (K > 1024) return nb % 32 == 0 ? TileGeom{4, 64, 32, kNormNT} : TileGeom{0, 0, 0, 0};
  // 256 lanes, one stage of whole 64-row tiles: nb/2 units per lane
  return nb == 28 || nb == 32 ? TileGeom{nb / 2, 64, nb, kNormNTSmall} : TileGeom{0, 0, 0, 0};
}

// Geometry of a split gate|up NORM launch (deferred block scales: Q4_0 rows
// of 2049..4096 values; kNormNT lanes, the second half holding kSplitUAct
// units per lane per stage): tiles of 64 rows of each matrix in stages of
// 4 * kSplitUAct blocks, or u == 0 when off. (The Q|K|V launch keeps the
// plain NORM form, which measured faster: there the exact sum, not the
// weight stream, sets the launch's length.) On unless PRANA_NORM_SPLIT=0
// (decided once per process).
template <int KIND>
TileGeom norm_split_act_geom(size_t K) {
  static const bool on = [] {
    const char* e = std::getenv("PRANA_NORM_SPLIT");
    return !(e && e[0] == '0');
  }();
  const int nb = static_cast<int>(K / RegUnit<KIND>::kElems);
  if (!on || KIND != kKindQ4_0 || K <= 2048 || K > static_cast<size_t>(kNormMaxK) || K % 32 != 0)
    return TileGeom{0, 0, 0, 0};
  // (the norm waves convert a stage as columns of (kNormNT/2) % sb == 0
  // lanes, and the stage counters cover every stage)
  constexpr int sb = kSplitSB;
  static_assert((kNormNT / 2) % sb == 0, "stage columns tile the norm lanes; a unit lane's units share a block");
  return (nb + sb - 1) / sb <= kSplitMaxStages ? TileGeom{kSplitUAct, 64, sb, kNormNT} : TileGeom{0, 0, 0, 0};
}

// KB >= 0: the matrices come in two formats, KIND and KB, with the same tile
// geometry (gemv_tile_mixed_kernel; not in act mode).
template <int KIND, int U, bool ACT, bool STAGED, int NT, int KB = -1, bool NORM = false, bool SPLIT = false>
int launch_tile_u(const DecodeJob& job0, const TileGeom& g, const int8_t* q, const float* sa, const int* sums,
                  size_t n_tok, hipStream_t s) {
  using R = RegUnit<KIND>;
  static_assert(KB < 0 || !ACT, "two formats only outside act mode");
  static_assert(KB < 0 || !SPLIT, "split norm launches take one format");
  constexpr int kTpuMax = KB < 0 ? R::kTpu : std::max(R::kTpu, RegUnit<(KB < 0 ? KIND : KB)>::kTpu);
  const void* const fn = [] {
    if constexpr (KB < 0) return reinterpret_cast<const void*>(gemv_tile_kernel<KIND, U, ACT, STAGED, NT, NORM, SPLIT>);
    else return reinterpret_cast<const void*>(gemv_tile_mixed_kernel<KIND, KB, U, STAGED, NT, NORM>);
  }();
  DecodeJob job = job0;
  job.rt = g.rt;
  job.sb = g.sb;
  const size_t K = job.m[0].cols;
  const int nb = static_cast<int>(K / R::kElems);
  const int rows_wg = ACT ? 2 * g.rt : g.rt;
  const int n_stages = (nb + g.sb - 1) / g.sb;
  PRANA_CHECK(STAGED || n_stages == 1, "gemv: single-stage tile with several stages");
  const size_t astride = ((K + 8 * (K / 32)) + 15) & ~static_cast<size_t>(15);
  const size_t term_bytes = (size_t)(n_stages > 1 ? 2 : 1) * rows_wg * (g.sb * kTpuMax + 1) * 4;
  int total = 0;
  for (int i = 0; i < (ACT ? 1 : job.n_mats); i++) {
    job.tiles[i] = static_cast<int>((job.m[i].rows + g.rt - 1) / g.rt);
    total += job.tiles[i];
  }
  // NORM: the row staged for the sum of squares shares the term region
  const size_t norm_bytes = NORM ? (static_cast<size_t>(exact::run_pad(static_cast<int>(K) - 1)) + 1) * 4 : 0;
  // SPLIT (deferred block scales): the (row, block) dots of the whole tile,
  // the staged row, the exact q, block scales, sums and change marks
  const size_t split_bytes = static_cast<size_t>(rows_wg) * (nb + 1) * 4 + norm_bytes + K + 3 * (K / 32) * 4;
  const size_t per_tok = astride + (SPLIT ? split_bytes : std::max(term_bytes, norm_bytes));
  PRANA_CHECK(!NORM || (n_tok == 1 && K <= static_cast<size_t>(4 * NT) && K % 32 == 0 && job.nin.x &&
                        job.nin.w && reinterpret_cast<uintptr_t>(job.nin.x) % 16 == 0 &&
                        reinterpret_cast<uintptr_t>(job.nin.w) % 16 == 0),
              "gemv: a fused rmsnorm takes one 16-byte-aligned token of at most 4096 values (a multiple of 32)");
  // verify batches of up to kDecMaxTok tokens stream the weights once; the
  // activations and term rows of every token sit in LDS, beyond 64 KB when
  // the device grants it
  static const size_t lds_cap = [fn] {
    int dev = 0, b = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&b, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || b <= 65536)
      return size_t{65536};
    const int dyn = b - static_cast<int>(static_lds_bytes(fn));
    return dyn > 65536 && set_max_dynamic_lds(fn, dyn) ? static_cast<size_t>(dyn) : size_t{65536};
  }();
  size_t group = std::min<size_t>(kDecMaxTok, lds_cap / per_tok);
  group = std::min<size_t>(group, NT / rows_wg);  // one folder lane per (token, row)
  PRANA_CHECK(K <= 16384, "gemv: decode kernel supports cols <= 16384");
  PRANA_CHECK(rows_wg * g.sb == (SPLIT ? NT / 2 : NT) * U, "gemv: tile geometry mismatch");
  PRANA_CHECK(group >= 1, "gemv: decode tile exceeds LDS");
  // a split launch leads with its norm workgroup, which hands inv over
  if (SPLIT) {
    PRANA_CHECK(job.nin.xch && reinterpret_cast<uintptr_t>(job.nin.xch) % 8 == 0,
                "gemv: a split norm launch needs 8-byte-aligned handoff words");
    job.nin.xch_polls = split_wait_polls();
    PRANA_CHECK(total <= kXchMaxTiles, "gemv: more split tiles than handoff flags");
    PRANA_CHECK((static_cast<size_t>(exact::run_pad(static_cast<int>(K) - 1)) + 1) * 4 <= per_tok,
                "gemv: split norm row exceeds the launch's LDS");
    total += 1;
  }
  for (size_t t0 = 0; t0 < n_tok; t0 += group) {
    const size_t nt = std::min<size_t>(group, n_tok - t0);
    DecodeJob j = job;
    for (int i = 0; i < 3; i++)
      if (j.o[i].out) j.o[i].out += t0 * j.o[i].ldo;
    j.rk.pos += static_cast<int>(t0);  // the group's first token (a batch's positions are on the host)
    if (ACT) {
      const size_t H = j.m[0].rows;
      if (j.h) j.h += t0 * H;
      j.hq += t0 * H;
      j.hsa += t0 * H / 32;
      j.hsum += t0 * H / 32;
    }
    const size_t G = K / 32;
    LaunchEvents& le = launch_events();
    if constexpr (KB >= 0) {
      hipLaunchKernelGGL((gemv_tile_mixed_kernel<KIND, KB, U, STAGED, NT, NORM>), dim3(total),
                         dim3(NT), nt * per_tok, s, j, q + t0 * K, sa + t0 * G, sums + t0 * G, (int)nt);
    } else if (le.start && t0 + nt >= n_tok && t0 == 0) {  // one launch: timestamp it
      hipExtLaunchKernelGGL((gemv_tile_kernel<KIND, U, ACT, STAGED, NT, NORM, SPLIT>), dim3(total), dim3(NT),
                            nt * per_tok, s, le.start, le.stop, 0, j, q + t0 * K, sa + t0 * G, sums + t0 * G,
                            (int)nt);
      le = LaunchEvents{};
    } else {
      hipLaunchKernelGGL((gemv_tile_kernel<KIND, U, ACT, STAGED, NT, NORM, SPLIT>), dim3(total), dim3(NT),
                         nt * per_tok, s, j, q + t0 * K, sa + t0 * G, sums + t0 * G, (int)nt);
    }
    PRANA_LAUNCH_CHECK();
  }
  return kOk;
}

// Chunk width W (blocks) of the verify-batch kernel for nb blocks per row and
// a batch of n_tok tokens, or 0 when it does not apply. W is 32 or 64 with
// nb / W in {2, 4, 7, 14}; rows of up to 128 blocks take W = 32 (eight rows
// per tile: half the workgroups of W = 64), longer rows W = 64 while two
// chunks of every token (activations and term rows) stay within 40 KB of LDS.
// Launches take as many tokens as kKmLdsBudget allows.
inline size_t km_per_tok(int w) { return 2 * static_cast<size_t>(w) * 40 + 2 * (kKmNT / w) * (w + 1) * 4; }
constexpr size_t kKmLdsBudget = 49152;  // per launch: three workgroups per CU
inline int km_chunk(int nb, size_t n_tok) {
  auto ok = [&](int w) {
    const int u = nb / w;
    return nb % w == 0 && (u == 2 || u == 4 || u == 7 || u == 14);
  };
  if (nb <= 128 && ok(32)) return 32;
  if (ok(64) && n_tok * 64 <= 512 && n_tok * km_per_tok(64) <= 40960) return 64;
  if (ok(32)) return 32;
  return 0;
}

template <int KIND, int U, bool ACT>
int launch_km_u(const DecodeJob& job0, int w, const int8_t* q, const float* sa, const int* sums, size_t n_tok,
                hipStream_t s) {
  DecodeJob job = job0;
  const int rows_wg = kKmNT / w;
  job.rt = ACT ? rows_wg / 2 : rows_wg;
  job.sb = w;
  const size_t K = job.m[0].cols;
  PRANA_CHECK(static_cast<int>(K / 32) == U * w, "gemv: verify-batch chunk geometry mismatch");
  int total = 0;
  for (int i = 0; i < (ACT ? 1 : job.n_mats); i++) {
    job.tiles[i] = static_cast<int>((job.m[i].rows + job.rt - 1) / job.rt);
    total += job.tiles[i];
  }
  const size_t per_tok = km_per_tok(w);
  // one chunk's activations fit the lanes' registers (kKmQ4, kKmSc) for up to
  // 512 / w tokens; one folder lane per (token, row)
  const size_t group = std::min<size_t>({static_cast<size_t>(512 / w), static_cast<size_t>(kKmNT / rows_wg),
                                         std::max<size_t>(1, kKmLdsBudget / per_tok)});
  const size_t G = K / 32;
  for (size_t t0 = 0; t0 < n_tok; t0 += group) {
    const size_t nt = std::min<size_t>(group, n_tok - t0);
    DecodeJob j = job;
    for (int i = 0; i < 3; i++)
      if (j.o[i].out) j.o[i].out += t0 * j.o[i].ldo;
    if (ACT) j.h += t0 * j.m[0].rows;
    hipLaunchKernelGGL((gemv_km_kernel<KIND, U, ACT>), dim3(total), dim3(kKmNT), nt * per_tok, s, j, q + t0 * K,
                       sa + t0 * G, sums + t0 * G, (int)nt);
    PRANA_LAUNCH_CHECK();
  }
  return kOk;
}

template <int KIND, bool ACT>
int launch_km(const DecodeJob& job, int w, const int8_t* q, const float* sa, const int* sums, size_t n_tok,
              hipStream_t s) {
  switch (static_cast<int>(job.m[0].cols / 32) / w) {
    case 2: return launch_km_u<KIND, 2, ACT>(job, w, q, sa, sums, n_tok, s);
    case 4: return launch_km_u<KIND, 4, ACT>(job, w, q, sa, sums, n_tok, s);
    case 7: return launch_km_u<KIND, 7, ACT>(job, w, q, sa, sums, n_tok, s);
    case 14: return launch_km_u<KIND, 14, ACT>(job, w, q, sa, sums, n_tok, s);
  }
  return fail(kErrInvalid, "gemv: no verify-batch chunk geometry");
}

template <int KIND>
int launch_decode_t(const DecodeJob& job, const int8_t* q, const float* sa, const int* sums, size_t n_tok,
                    hipStream_t s) {
  constexpr bool kSmall = RegUnit<KIND>::kElems == 32;
  const bool act = job.act != 0;
  if constexpr (kSmall) {
    // verify batches: the chunk-major kernel for long rows (more than 128
    // blocks: whole-row staging of several tokens limits the tile kernel to
    // one workgroup per CU), for the act tiles, and for batches of more than
    // kDecMaxTok tokens (one launch instead of two); the tile kernel keeps
    // the other batches of up to kDecMaxTok tokens, where it is faster
    // (measured on the 7B shapes). Act tiles here have fewer than 32 rows per
    // matrix, so the caller quantizes h, as it does after the tile kernel.
    const int nb_k = static_cast<int>(job.m[0].cols / 32);
    const bool km_pref = nb_k > 128 || act || n_tok > static_cast<size_t>(kDecMaxTok);
    const int w = n_tok >= 2 && km_pref && !job.rk.table ? km_chunk(nb_k, n_tok) : 0;
    if (w > 0 && (!act || choose_geom<KIND>(job.m[0].cols, true).rt % 32 != 0) && (!act || job.h)) {
      if (act) return launch_km<KIND, true>(job, w, q, sa, sums, n_tok, s);
      return launch_km<KIND, false>(job, w, q, sa, sums, n_tok, s);
    }
  }
  const TileGeom g = choose_geom<KIND>(job.m[0].cols, act);
  const int nb = static_cast<int>(job.m[0].cols / RegUnit<KIND>::kElems);
  const bool staged = g.sb < nb;
  if (act) {
    if constexpr (kSmall) {
      if (staged) return launch_tile_u<KIND, 8, true, true, 256>(job, g, q, sa, sums, n_tok, s);
      switch (g.u) {
        case 1: return launch_tile_u<KIND, 1, true, false, 256>(job, g, q, sa, sums, n_tok, s);
        case 2: return launch_tile_u<KIND, 2, true, false, 256>(job, g, q, sa, sums, n_tok, s);
        case 4: return launch_tile_u<KIND, 4, true, false, 256>(job, g, q, sa, sums, n_tok, s);
        case 7: return launch_tile_u<KIND, 7, true, false, 256>(job, g, q, sa, sums, n_tok, s);
        case 8: return launch_tile_u<KIND, 8, true, false, 256>(job, g, q, sa, sums, n_tok, s);
      }
      return fail(kErrInvalid, "gemv: no act tile geometry");
    } else {
      if (!staged) return launch_tile_u<KIND, 1, true, false, 256>(job, g, q, sa, sums, n_tok, s);
      return launch_tile_u<KIND, 1, true, true, 256>(job, g, q, sa, sums, n_tok, s);
    }
  }
  if (staged) {
    if constexpr (kSmall) return launch_tile_u<KIND, 2, false, true, 256>(job, g, q, sa, sums, n_tok, s);
    else return launch_tile_u<KIND, 1, false, true, 256>(job, g, q, sa, sums, n_tok, s);
  }
  switch (g.u) {
    case 1: return launch_tile_u<KIND, 1, false, false, 256>(job, g, q, sa, sums, n_tok, s);
    case 2: return launch_tile_u<KIND, 2, false, false, 256>(job, g, q, sa, sums, n_tok, s);
  }
  if constexpr (kSmall) {
    switch (g.u) {
      case 4: return launch_tile_u<KIND, 4, false, false, 256>(job, g, q, sa, sums, n_tok, s);
      case 7: return launch_tile_u<KIND, 7, false, false, 256>(job, g, q, sa, sums, n_tok, s);
      case 8: return launch_tile_u<KIND, 8, false, false, 256>(job, g, q, sa, sums, n_tok, s);
    }
  }
  return fail(kErrInvalid, "gemv: no tile geometry");
}

// Two formats in one decode launch (non-act): the tile geometry of KA, which
// the caller has checked KB shares.
template <int KA, int KB>
int launch_decode_mixed(const DecodeJob& job, const int8_t* q, const float* sa, const int* sums, size_t n_tok,
                        hipStream_t s) {
  constexpr bool kSmall = RegUnit<KA>::kElems == 32;
  static_assert(RegUnit<KA>::kElems == RegUnit<KB>::kElems, "one unit width");
  const TileGeom g = choose_geom<KA>(job.m[0].cols, false);
  const int nb = static_cast<int>(job.m[0].cols / RegUnit<KA>::kElems);
  if (g.sb < nb) {
    if constexpr (kSmall) return launch_tile_u<KA, 2, false, true, 256, KB>(job, g, q, sa, sums, n_tok, s);
    else return launch_tile_u<KA, 1, false, true, 256, KB>(job, g, q, sa, sums, n_tok, s);
  }
  switch (g.u) {
    case 1: return launch_tile_u<KA, 1, false, false, 256, KB>(job, g, q, sa, sums, n_tok, s);
    case 2: return launch_tile_u<KA, 2, false, false, 256, KB>(job, g, q, sa, sums, n_tok, s);
  }
  if constexpr (kSmall) {
    switch (g.u) {
      case 4: return launch_tile_u<KA, 4, false, false, 256, KB>(job, g, q, sa, sums, n_tok, s);
      case 7: return launch_tile_u<KA, 7, false, false, 256, KB>(job, g, q, sa, sums, n_tok, s);
      case 8: return launch_tile_u<KA, 8, false, false, 256, KB>(job, g, q, sa, sums, n_tok, s);
    }
  }
  return fail(kErrInvalid, "gemv: no tile geometry");
}

// The supported pair of two formats among ms[0..n) (same cols), as (KA, KB)
// in canonical order, or {-1, -1}: Q4_0 with Q8_0 (block-32), Q4_K with Q6_K.
std::pair<int, int> mixed_pair(const DevMat* ms, int n) {
  int a = ms[0].kind, b = -1;
  for (int i = 1; i < n; i++) {
    if (ms[i].kind == a || ms[i].kind == b) continue;
    if (b >= 0) return {-1, -1};
    b = ms[i].kind;
  }
  if (b < 0) return {-1, -1};
  if (a > b) std::swap(a, b);
  const bool ok = (a == kKindQ4_0 && b == kKindQ8_0) || (a == kKindQ8_0 && b == kKindQ4_0) ||
                  (a == kKindQ4_K && b == kKindQ6_K) || (a == kKindQ6_K && b == kKindQ4_K);
  if (!ok) return {-1, -1};
  // canonical: the 4-bit format first
  return a == kKindQ4_0 || a == kKindQ4_K ? std::make_pair(a, b) : std::make_pair(b, a);
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

// ===================================================================
// Batched matmul on the int8 matrix cores (prefill / verify, N > 16 tokens).
// Q4_0 needs no activation sums here: its nibbles enter the matrix cores as
// the signed values n - 8.
//
// One v_mfma_i32_32x32x32_i8 gives the exact i32 block dots of one
// 32-element block for a 32-token x 32-row tile; the f32 term of each
// (token, row) is then formed with the decode kernels' expression and added
// to that output's accumulator, block after block, so every output is the
// same left-to-right fold as in the decode path (bitwise equal per element,
// as matmul_q8_prefill / matmul_kquant_prefill are to their decode forms).
// Lane layout (checked on the device): A[i][k] i = lane%32, B[k][j]
// j = lane%32, with the same k for byte b of an A lane and of a B lane in
// the same lane half; D[i][j] j = lane%32, i = 8*(v/4) + 4*(lane/32) + v%4
// for the 16 values v of a lane.
// A = activations (i = token), B = weights (j = row): each lane owns one
// weight row and sixteen tokens of its wave's tile.
typedef int v16i_t __attribute__((ext_vector_type(16)));
typedef int v4i_t __attribute__((ext_vector_type(4)));  // also the skinny kernels' result type

constexpr int kMmaRows = 128;  // weight rows per workgroup (32 per wave)
constexpr int kMmaToks = 32;   // tokens per workgroup

// Operands stream through LDS in chunks of L::CB blocks: every lane loads
// its share of chunk c+3 (16-byte pieces) into registers while chunk c is
// multiplied, so two chunks of loads are in flight behind the one in use.
// LDS rows are padded by 8 bytes (8-byte accesses of neighbouring rows fall
// in different banks).
constexpr int kMmaCB = 4;  // blocks per staged chunk (small chunks: several workgroups per CU)
typedef int sk_i4 __attribute__((ext_vector_type(4)));  // plain vector: stays in registers

template <int KIND>
struct MmaLayout {
  static constexpr int QB = KIND == kKindQ4_0 ? 16 : 32;  // quant bytes per block
  static constexpr int CB = kMmaCB;  // blocks per chunk
  static constexpr int WSTR = CB * QB + 8;             // bytes per staged weight row
  static constexpr int ASTR = CB * 32 + 8;             // bytes per staged activation row
  static constexpr int DSTR = CB + 1;                  // words per staged weight-scale row
  // one buffer: W [kMmaRows][WSTR] | A [kMmaToks][ASTR] | D [kMmaRows][DSTR] | SA [CB][kMmaToks]
  static constexpr int A_OFF = kMmaRows * WSTR;
  static constexpr int D_OFF = A_OFF + kMmaToks * ASTR;
  static constexpr int SA_OFF = D_OFF + kMmaRows * DSTR * 4;
  static constexpr int BYTES = SA_OFF + CB * kMmaToks * 4;
  // 16-byte pieces per chunk and per lane (256 lanes)
  static constexpr int WPR = CB * QB / 16;  // pieces per weight row
  static constexpr int WP = kMmaRows * WPR, AP = kMmaToks * CB * 2;
  static constexpr int WPL = WP / 256, APL = AP / 256;
  static constexpr int SP = kMmaToks * CB;  // activation scales per chunk
  static constexpr int DPL = kMmaRows * CB / 256, SPL = (SP + 255) / 256;
  static_assert(WP % 256 == 0 && AP % 256 == 0 && DPL * 256 == kMmaRows * CB, "whole pieces per lane");
};

// A block scale as loaded into a staging register: f32 bits for Q8F, else
// the f16 bits. Held at their loaded width, so nothing touches the loaded
// value before the register set is stored to LDS (a widening of a 16-bit
// load there makes the compiler wait for every load in flight).
template <int KIND>
using ScaleReg = typename std::conditional<KIND == kKindQ8F, uint32_t, uint16_t>::type;

template <int KIND>
struct MmaRegs {
  using L = MmaLayout<KIND>;
  sk_i4 w[L::WPL], a[L::APL];
  ScaleReg<KIND> d[L::DPL];
  float sa[L::SPL];
};

// Up to three matrices of one kind and width over the same activations
// (Q|K|V, gate|up) in one launch: x-blocks [t0[i], t0[i+1]) are matrix i's
// row tiles, so a small matrix (a GQA K or V) does not leave most of the
// chip idle in a launch of its own.
struct MmaJob {
  DevMat m[3];
  GemvOut o[3];
  int t0[3];  // first x-block of each matrix (t0[0] = 0)
  int n_mats;
  // ACT launches (m[0] = gate, m[1] = up, H = rows % 64 == 0): x-block b
  // holds rows 64b..64b+63 of both, and the epilogue forms h = act(g) * u
  // (infer.rs:197-199) and its 32-row blocks quantized for the down
  // projection (matmul.rs:105-127), as launch_act_mul does
  int gelu;  // 0 silu, 1 gelu_tanh
  float* h;  // optional f32 h [n_tok][H]
  int8_t* hq;
  float* hsa;
  int* hsum;
};

template <int KIND, bool ACT = false>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(MmaJob job, const int8_t* __restrict__ q,
                                                        const float* __restrict__ sa, int n_tok) {
  static_assert(KIND == kKindQ4_0 || KIND == kKindQ8_0 || KIND == kKindQ8F, "block-32 kinds");
  using L = MmaLayout<KIND>;
  extern __shared__ int4 mma_smem[];
  uint8_t* lds = reinterpret_cast<uint8_t*>(mma_smem);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, h = lane >> 5;
  const int bx = blockIdx.x;
  const int mi = ACT ? 0 : job.n_mats > 2 && bx >= job.t0[2] ? 2 : job.n_mats > 1 && bx >= job.t0[1] ? 1 : 0;
  const DevMat m = mi == 0 ? job.m[0] : mi == 1 ? job.m[1] : job.m[2];
  const GemvOut o = mi == 0 ? job.o[0] : mi == 1 ? job.o[1] : job.o[2];
  const int K = static_cast<int>(m.cols), G = K / 32;
  const int R = static_cast<int>(m.rows);
  const int row0 = ACT ? bx * (kMmaRows / 2) : (bx - (mi == 0 ? 0 : mi == 1 ? job.t0[1] : job.t0[2])) * kMmaRows;
  const int m0 = blockIdx.y * kMmaToks;
  const int n_chunks = (G + L::CB - 1) / L::CB;
  // tile row lr (0..127): its matrix row, and (ACT) gate rows 0..63 / up rows 64..127
  auto tile_row = [&](int lr) { return min(row0 + (ACT ? (lr & 63) : lr), R - 1); };
  const uint8_t* const qs_up = ACT ? job.m[1].qs : m.qs;
  const void* const sc_up = ACT ? job.m[1].sc : m.sc;
  auto tile_qs = [&](int lr) { return ACT && lr >= 64 ? qs_up : m.qs; };
  auto tile_sc = [&](int lr) { return ACT && lr >= 64 ? sc_up : m.sc; };

  auto load = [&](int c) __attribute__((always_inline)) {  // this lane's share of chunk c (clamped addresses)
    MmaRegs<KIND> r;
    const int cb0 = c * L::CB;
#pragma unroll
    for (int i = 0; i < L::WPL; i++) {
      const int p = tid + 256 * i;
      const int rr = tile_row(p / L::WPR), pr = p % L::WPR;
      const int blk = min(cb0 + pr / (L::QB / 16), G - 1);
      r.w[i] = *reinterpret_cast<const sk_i4*>(tile_qs(p / L::WPR) + (size_t)rr * G * L::QB + (size_t)blk * L::QB +
                                               (pr % (L::QB / 16)) * 16);
    }
#pragma unroll
    for (int i = 0; i < L::APL; i++) {
      const int p = tid + 256 * i;
      const int t = min(m0 + p / (2 * L::CB), n_tok - 1), pr = p % (2 * L::CB);
      const int blk = min(cb0 + pr / 2, G - 1);
      r.a[i] = *reinterpret_cast<const sk_i4*>(q + (size_t)t * K + (size_t)blk * 32 + (pr & 1) * 16);
    }
#pragma unroll
    for (int i = 0; i < L::DPL; i++) {
      const int p = tid + 256 * i;
      const size_t gi = (size_t)tile_row(p / L::CB) * G + min(cb0 + p % L::CB, G - 1);
      if constexpr (KIND == kKindQ8F) r.d[i] = reinterpret_cast<const uint32_t*>(tile_sc(p / L::CB))[gi];
      else r.d[i] = reinterpret_cast<const uint16_t*>(tile_sc(p / L::CB))[gi];
    }
#pragma unroll
    for (int i = 0; i < L::SPL; i++) {
      const int p = min(tid + 256 * i, L::SP - 1);  // consecutive lanes: consecutive blocks of one token
      const size_t gi = (size_t)min(m0 + p / L::CB, n_tok - 1) * G + min(cb0 + p % L::CB, G - 1);
      r.sa[i] = sa[gi];
    }
    return r;
  };
  auto store = [&](const MmaRegs<KIND>& r, int buf) __attribute__((always_inline)) {
    uint8_t* b = lds + buf * L::BYTES;
#pragma unroll
    for (int i = 0; i < L::WPL; i++) {  // two 8-byte halves (padded rows are 8-byte aligned)
      const int p = tid + 256 * i;
      long* dst = reinterpret_cast<long*>(b + (p / L::WPR) * L::WSTR + (p % L::WPR) * 16);
      dst[0] = static_cast<long>(static_cast<uint32_t>(r.w[i].x)) | (static_cast<long>(r.w[i].y) << 32);
      dst[1] = static_cast<long>(static_cast<uint32_t>(r.w[i].z)) | (static_cast<long>(r.w[i].w) << 32);
    }
#pragma unroll
    for (int i = 0; i < L::APL; i++) {
      const int p = tid + 256 * i;
      long* dst = reinterpret_cast<long*>(b + L::A_OFF + (p / (2 * L::CB)) * L::ASTR + (p % (2 * L::CB)) * 16);
      dst[0] = static_cast<long>(static_cast<uint32_t>(r.a[i].x)) | (static_cast<long>(r.a[i].y) << 32);
      dst[1] = static_cast<long>(static_cast<uint32_t>(r.a[i].z)) | (static_cast<long>(r.a[i].w) << 32);
    }
#pragma unroll
    for (int i = 0; i < L::DPL; i++) {
      const int p = tid + 256 * i;
      reinterpret_cast<uint32_t*>(b + L::D_OFF)[(p / L::CB) * L::DSTR + p % L::CB] = r.d[i];
    }
#pragma unroll
    for (int i = 0; i < L::SPL; i++) {
      const int p = tid + 256 * i;
      if (p < L::SP) {
        reinterpret_cast<float*>(b + L::SA_OFF)[(p % L::CB) * kMmaToks + p / L::CB] = r.sa[i];
      }
    }
  };
  float acc[16];
#pragma unroll
  for (int v = 0; v < 16; v++) acc[v] = 0.0f;
  const int wr_row = wave * 32 + (lane & 31);  // this lane's weight row in the tile (B column)
  auto compute = [&](int buf, int c) __attribute__((always_inline)) {
    const uint8_t* b = lds + buf * L::BYTES;
    const uint8_t* arow = b + L::A_OFF + (lane & 31) * L::ASTR + 8 * h;  // this lane's A row (token)
    const uint8_t* wrow = b + wr_row * L::WSTR + 8 * h;
    const uint32_t* drow = reinterpret_cast<const uint32_t*>(b + L::D_OFF) + wr_row * L::DSTR;
    const float* sab = reinterpret_cast<const float*>(b + L::SA_OFF) + 4 * h;
    const int nlive = min(L::CB, G - c * L::CB);  // uniform
    // block bb's integer dots (tokens 8g + 4h + e of the tile in values v = 4g + e)
    auto dots = [&](int bb) __attribute__((always_inline)) {
      const long a1 = *reinterpret_cast<const long*>(arow + bb * 32);
      const long a2 = *reinterpret_cast<const long*>(arow + bb * 32 + 16);
      long b1, b2;
      if constexpr (KIND == kKindQ4_0) {
        // nibbles n -> signed bytes n - 8, so the matrix cores give
        // isum - 8*sum_a itself: ((n | 0x80) - 8) ^ 0x80 per byte, with no
        // borrow between bytes (every byte is >= 0x80 before the subtract)
        constexpr long kLo = 0x0F0F0F0F0F0F0F0FL, kHi = static_cast<long>(0x8080808080808080UL),
                       k8 = 0x0808080808080808L;
        const long w = *reinterpret_cast<const long*>(wrow + bb * 16);
        b1 = (((w & kLo) | kHi) - k8) ^ kHi;
        b2 = ((((w >> 4) & kLo) | kHi) - k8) ^ kHi;
      } else {
        b1 = *reinterpret_cast<const long*>(wrow + bb * 32);
        b2 = *reinterpret_cast<const long*>(wrow + bb * 32 + 16);
      }
      // one 32-deep product: byte j of either operand is element 8h + j
      // (j < 8) or 16 + 8h + (j - 8), the same pairing for A and B, so the
      // sum over the instruction's k is the block's dot whatever order the
      // matrix core gives k
      const v4i_t av = {static_cast<int>(a1), static_cast<int>(a1 >> 32), static_cast<int>(a2),
                        static_cast<int>(a2 >> 32)};
      const v4i_t bv = {static_cast<int>(b1), static_cast<int>(b1 >> 32), static_cast<int>(b2),
                        static_cast<int>(b2 >> 32)};
      const v16i_t zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
      return __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, zero, 0, 0, 0);
    };
    // block bb's f32 terms, added to each output's running total
    auto terms = [&](const v16i_t& cc, int bb) __attribute__((always_inline)) {
      const float d = KIND == kKindQ8F ? __uint_as_float(drow[bb]) : f16_operand(static_cast<uint16_t>(drow[bb]));
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const float4 s4 = *reinterpret_cast<const float4*>(sab + bb * kMmaToks + 8 * g);
        const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
        for (int e = 0; e < 4; e++)  // (d*sa)*float(isum), as the decode terms
          acc[4 * g + e] += d * sv[e] * static_cast<float>(cc[4 * g + e]);
      }
    };
    if (nlive == L::CB) {  // uniform: a whole chunk, each block's dots issued one block ahead of its terms
      static_assert(L::CB % 2 == 0, "blocks in pairs");
      v16i_t c0 = dots(0), c1;
#pragma unroll
      for (int bb = 0; bb < L::CB; bb += 2) {
        c1 = dots(bb + 1);
        terms(c0, bb);
        if (bb + 2 < L::CB) c0 = dots(bb + 2);
        terms(c1, bb + 1);
      }
    } else {
      for (int bb = 0; bb < nlive; bb++) terms(dots(bb), bb);  // the row's last, partial chunk
    }
  };

  MmaRegs<KIND> r0 = load(0), r1;
  store(r0, 0);
  if (n_chunks > 1) r0 = load(1);
  if (n_chunks > 2) r1 = load(2);
  __syncthreads();
  // chunk c+1 sits in r0 when c is even, in r1 when c is odd
  for (int c = 0; c < n_chunks; c += 2) {
    compute(0, c);
    if (c + 1 < n_chunks) store(r0, 1);
    if (c + 3 < n_chunks) r0 = load(c + 3);
    __syncthreads();
    if (c + 1 >= n_chunks) break;
    compute(1, c + 1);
    if (c + 2 < n_chunks) store(r1, 0);
    if (c + 4 < n_chunks) r1 = load(c + 4);
    __syncthreads();
  }
  if constexpr (ACT) {
    // waves 2 and 3 hold the up rows of waves 0 and 1's gate rows: the pair
    // swaps half of its values through LDS (free: the last chunk's barrier is
    // behind), so that wave w < 2 forms h for its values 0..7 and wave w + 2
    // for values 8..15 (tokens 8g + 4h + e for value 4g + e); the 32 lanes of
    // a half hold one 32-row block of h for each of those tokens
    float* s_x = reinterpret_cast<float*>(lds);  // [4 waves][64 lanes][9]
    const int pw = wave & 1, up_wave = wave >> 1;
#pragma unroll
    for (int v = 0; v < 8; v++) s_x[(wave * 64 + lane) * 9 + v] = acc[up_wave ? v : v + 8];
    __syncthreads();
    const int r = row0 + pw * 32 + (lane & 31);  // < H (H % 64 == 0)
    const int H = R;
    const float* other = s_x + (((up_wave ? pw : pw + 2) * 64) + lane) * 9;  // the partner wave's values
    float hv[8];
#pragma unroll
    for (int v = 0; v < 8; v++) {
      float g = up_wave ? other[v] : acc[v];
      const float u = up_wave ? acc[v + 8] : other[v];
      if (job.gelu) {
        const float kS = 0.7978846f;  // norms.rs:36
        const float x3 = g * g * g;
        g = 0.5f * g * (1.0f + dev_tanhf(kS * (g + 0.044715f * x3)));
      } else {
        g = g * (1.0f / (1.0f + dev_expf(-g)));
      }
      hv[v] = g * u;
    }
    int qv[8], sm[8];
    float sc[8];
    quantize_lanes<8>(hv, qv, sc, sm);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int v = up_wave ? j + 8 : j;
      const int t = m0 + 8 * (v / 4) + 4 * h + (v % 4);
      if (t < n_tok) {
        const size_t gi = (size_t)t * H + r;
        job.hq[gi] = static_cast<int8_t>(qv[j]);
        if (job.h) job.h[gi] = hv[j];
        if ((lane & 31) == 0) {
          job.hsa[gi >> 5] = sc[j];
          job.hsum[gi >> 5] = sm[j];
        }
      }
    }
    return;
  }
  const int n_row = row0 + wr_row;
  if (n_row < R) {
#pragma unroll
    for (int v = 0; v < 16; v++) {
      const int t = m0 + 8 * (v / 4) + 4 * h + (v % 4);
      if (t < n_tok) store_out(o, t, n_row, acc[v]);
    }
  }
}

template <int KIND>
int launch_gemm_mfma(const DevMat* ms, const GemvOut* os, int n_mats, const int8_t* q, const float* sa, size_t n_tok,
                     hipStream_t s) {
  PRANA_CHECK(n_mats >= 1 && n_mats <= 3, "gemm: 1..3 matrices");
  using L = MmaLayout<KIND>;
  static const bool attr_ok = [] {
    return L::BYTES * 2 <= 65536 ||
           set_max_dynamic_lds(reinterpret_cast<const void*>(gemm_mfma_kernel<KIND>), L::BYTES * 2);
  }();
  PRANA_CHECK(attr_ok, "gemm: LDS size not granted");
  MmaJob job{};
  size_t tiles = 0;
  for (int i = 0; i < n_mats; i++) {
    const DevMat& m = ms[i];
    PRANA_CHECK(m.kind == KIND && m.cols == ms[0].cols, "gemm: matrices must share kind and cols");
    PRANA_CHECK(m.cols % 32 == 0 && m.cols <= (1u << 30) && m.rows <= (1u << 30), "gemm: shape out of range");
    job.m[i] = m;
    job.o[i] = os[i];
    job.t0[i] = static_cast<int>(tiles);
    tiles += (m.rows + kMmaRows - 1) / kMmaRows;
  }
  job.n_mats = n_mats;
  PRANA_CHECK(tiles >= 1 && tiles < (1u << 31), "gemm: row tiles out of range");
  dim3 grid(static_cast<unsigned>(tiles), (n_tok + kMmaToks - 1) / kMmaToks);
  hipLaunchKernelGGL(gemm_mfma_kernel<KIND>, grid, dim3(256), L::BYTES * 2, s, job, q, sa, (int)n_tok);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

// gate|up, the activation and the quantization of h in one launch (batches
// beyond the skinny kernel's, block-32 kinds, H % 64 == 0).
template <int KIND>
int launch_gemm_mfma_act(const DevMat& gate, const DevMat& up, const int8_t* q, const float* sa, size_t n_tok,
                         int gelu, float* h, int8_t* hq, float* hsa, int* hsum, hipStream_t s) {
  using L = MmaLayout<KIND>;
  static const bool attr_ok = [] {
    return L::BYTES * 2 <= 65536 ||
           set_max_dynamic_lds(reinterpret_cast<const void*>(gemm_mfma_kernel<KIND, true>), L::BYTES * 2);
  }();
  PRANA_CHECK(attr_ok, "gemm: LDS size not granted");
  static_assert(4 * 64 * 9 * 4 <= L::BYTES * 2, "the gate/up exchange fits the staging LDS");
  PRANA_CHECK(gate.kind == KIND && up.kind == KIND && gate.rows == up.rows && gate.cols == up.cols &&
                  gate.rows % 64 == 0 && gate.cols % 32 == 0 && gate.cols <= (1u << 30) && gate.rows <= (1u << 30),
              "gemm act: gate and up must share kind and shape, rows a multiple of 64");
  PRANA_CHECK(hq && hsa && hsum, "gemm act: quantized h outputs required");
  MmaJob job{};
  job.m[0] = gate;
  job.m[1] = up;
  job.n_mats = 2;
  job.gelu = gelu;
  job.h = h;
  job.hq = hq;
  job.hsa = hsa;
  job.hsum = hsum;
  dim3 grid(static_cast<unsigned>(gate.rows / 64), (n_tok + kMmaToks - 1) / kMmaToks);
  hipLaunchKernelGGL((gemm_mfma_kernel<KIND, true>), grid, dim3(256), L::BYTES * 2, s, job, q, sa, (int)n_tok);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

// ---- skinny batches (a few tokens) on the 16x16x32 int8 matrix cores
// v_mfma_i32_16x16x32_i8 takes one whole 32-element block per instruction:
// A[i][k] = activation k of token i, B[k][j] = quant k of weight row j; lane
// (j = lane%16, kg = lane/16) supplies elements 8kg..8kg+7 of token / row j
// and receives D for tokens 4kg+v, row j (v = 0..3). A wave owns 16 rows x
// 16 tokens; a workgroup's RW*TT waves cover 16*RW rows x 16*TT tokens.
// Weights, activations and both scale sets stream through LDS in chunks of
// kSkCB blocks: every lane fetches its share of chunk c+3 into registers
// while chunk c is multiplied, so two chunks of loads are in flight behind
// the one being used. Every output folds its block terms (d*sa)*float(isum)
// in block order, as the decode kernels do.
constexpr int kSkCB = 8;  // blocks per staged chunk

template <int KIND, int RW, int TT>
struct SkLayout {
  static constexpr int NT = 64 * RW * TT;
  static constexpr int QB = KIND == kKindQ4_0 ? 16 : 32;  // quant bytes per block
  static constexpr int ROWS = 16 * RW, TOKS = 16 * TT;
  // padded rows: 16 consecutive rows / tokens start 4 banks apart
  static constexpr int WSTR = kSkCB * QB + 16;  // bytes per staged weight row
  static constexpr int ASTR = kSkCB * 32 + 16;  // bytes per staged activation row
  static constexpr int DSTR = kSkCB + 1;        // words per staged weight-scale row
  // one buffer: W [ROWS][WSTR] | A [TOKS][ASTR] | D [ROWS][DSTR] | SA [kSkCB][TOKS] | SM [kSkCB][TOKS]
  static constexpr int A_OFF = ROWS * WSTR;
  static constexpr int D_OFF = A_OFF + TOKS * ASTR;
  static constexpr int SA_OFF = D_OFF + ROWS * DSTR * 4;
  static constexpr int SM_OFF = SA_OFF + kSkCB * TOKS * 4;
  static constexpr int BYTES = SM_OFF + kSkCB * TOKS * 4;
  // pieces of a chunk and their share per lane
  static constexpr int WPR = kSkCB * QB / 16;  // 16-byte weight pieces per row
  static constexpr int WP = ROWS * WPR, AP = TOKS * kSkCB * 2, DP = ROWS * kSkCB, SP = TOKS * kSkCB;
  static constexpr int WPL = (WP + NT - 1) / NT, APL = (AP + NT - 1) / NT;
  static constexpr int DPL = (DP + NT - 1) / NT, SPL = (SP + NT - 1) / NT;
};

template <int KIND, int RW, int TT>
struct SkRegs {
  using L = SkLayout<KIND, RW, TT>;
  sk_i4 w[L::WPL], a[L::APL];
  ScaleReg<KIND> d[L::DPL];
  float sa[L::SPL];
  int sm[L::SPL];
};

// Up to three matrices of one block-32 kind and width over the same
// activations (gate|up, Q|K|V) in one launch: workgroups t0[i].. take the row
// tiles of matrix i, so two 14336-row matrices fill the chip with 64-row tiles
// where each alone would leave CUs idle or need 32-row tiles.
// Act form (gate|up): m[0] = gate, m[1] = up, equal shapes, rows % 32 == 0.
// A workgroup stages 32 rows of each (its staged rows 0..31 are gate rows,
// 32..63 the same up rows), so waves 0-1 fold gate and waves 2-3 up; the
// epilogue forms h = act(g) * u (silu, or gelu_tanh) and quantizes each
// token's 32-row block of h for down, as launch_act_mul does.
struct SkJob {
  DevMat m[3];
  GemvOut o[3];
  int t0[3];  // first workgroup of matrix i (t0[0] = 0; unused entries INT32_MAX)
  int gelu;   // act form: gelu_tanh instead of silu
  float* h;   // act form: optional f32 h [n_tok][rows]
  int8_t* hq;
  float* hsa;
  int* hsum;
};

template <int KIND, int RW, int TT, bool ACT = false>
__global__ __launch_bounds__(64 * RW * TT) void gemm_skinny_kernel(SkJob job, const int8_t* __restrict__ q,
                                                                   const float* __restrict__ sa,
                                                                   const int* __restrict__ sums, int n_tok) {
  static_assert(KIND == kKindQ4_0 || KIND == kKindQ8_0 || KIND == kKindQ8F, "block-32 kinds");
  static_assert(!ACT || (RW == 4 && TT == 1), "the act form stages 32 rows of each matrix for one token tile");
  using L = SkLayout<KIND, RW, TT>;
  extern __shared__ int4 sk_smem[];
  uint8_t* lds = reinterpret_cast<uint8_t*>(sk_smem);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rtile = wave % RW, ttile = wave / RW;
  const int j = lane & 15, kg = lane >> 4;
  const int bx = static_cast<int>(blockIdx.x);
  const int mi = ACT ? 0 : (bx >= job.t0[1]) + (bx >= job.t0[2]);  // uniform
  const DevMat m = mi == 0 ? job.m[0] : mi == 1 ? job.m[1] : job.m[2];
  const GemvOut o = mi == 0 ? job.o[0] : mi == 1 ? job.o[1] : job.o[2];
  const int K = static_cast<int>(m.cols), G = K / 32, R = static_cast<int>(m.rows);
  const int row0 = ACT ? bx * 32 : (bx - (mi == 0 ? 0 : mi == 1 ? job.t0[1] : job.t0[2])) * L::ROWS;
  // staged row lr: its matrix row, and which matrix (the act form's rows 32..63 are up rows)
  auto src_row = [&](int lr) { return min(row0 + (ACT ? (lr & 31) : lr), R - 1); };
  auto src_qs = [&](int lr) { return ACT && lr >= 32 ? job.m[1].qs : m.qs; };
  auto src_sc = [&](int lr) { return ACT && lr >= 32 ? job.m[1].sc : m.sc; };
  const int n_chunks = (G + kSkCB - 1) / kSkCB;

  auto load = [&](int c) __attribute__((always_inline)) {  // this lane's share of chunk c (clamped addresses)
    SkRegs<KIND, RW, TT> r;
    const int cb0 = c * kSkCB;
#pragma unroll
    for (int i = 0; i < L::WPL; i++) {
      const int p = min(tid + L::NT * i, L::WP - 1);
      const int lr = p / L::WPR, rr = src_row(lr), pr = p % L::WPR;
      const int blk = min(cb0 + pr / (L::QB / 16), G - 1);
      const uint8_t* src = src_qs(lr) + (size_t)rr * G * L::QB + (size_t)blk * L::QB + (pr % (L::QB / 16)) * 16;
      r.w[i] = *reinterpret_cast<const sk_i4*>(src);
    }
#pragma unroll
    for (int i = 0; i < L::APL; i++) {
      const int p = min(tid + L::NT * i, L::AP - 1);
      const int t = min(p / (2 * kSkCB), n_tok - 1), pr = p % (2 * kSkCB);
      const int blk = min(cb0 + pr / 2, G - 1);
      r.a[i] = *reinterpret_cast<const sk_i4*>(q + (size_t)t * K + (size_t)blk * 32 + (pr & 1) * 16);
    }
#pragma unroll
    for (int i = 0; i < L::DPL; i++) {
      const int p = min(tid + L::NT * i, L::DP - 1);
      const int lr = p / kSkCB;
      const size_t gi = (size_t)src_row(lr) * G + min(cb0 + p % kSkCB, G - 1);
      if constexpr (KIND == kKindQ8F) r.d[i] = reinterpret_cast<const uint32_t*>(src_sc(lr))[gi];
      else r.d[i] = reinterpret_cast<const uint16_t*>(src_sc(lr))[gi];
    }
#pragma unroll
    for (int i = 0; i < L::SPL; i++) {
      const int p = min(tid + L::NT * i, L::SP - 1);
      const size_t gi = (size_t)min(p / kSkCB, n_tok - 1) * G + min(cb0 + p % kSkCB, G - 1);
      r.sa[i] = sa[gi];
      r.sm[i] = sums[gi];
    }
    return r;
  };
  auto store = [&](const SkRegs<KIND, RW, TT>& r, int buf) __attribute__((always_inline)) {
    uint8_t* b = lds + buf * L::BYTES;
#pragma unroll
    for (int i = 0; i < L::WPL; i++) {
      const int p = tid + L::NT * i;
      if (p < L::WP) *reinterpret_cast<sk_i4*>(b + (p / L::WPR) * L::WSTR + (p % L::WPR) * 16) = r.w[i];
    }
#pragma unroll
    for (int i = 0; i < L::APL; i++) {
      const int p = tid + L::NT * i;
      if (p < L::AP)
        *reinterpret_cast<sk_i4*>(b + L::A_OFF + (p / (2 * kSkCB)) * L::ASTR + (p % (2 * kSkCB)) * 16) = r.a[i];
    }
#pragma unroll
    for (int i = 0; i < L::DPL; i++) {
      const int p = tid + L::NT * i;
      if (p < L::DP) reinterpret_cast<uint32_t*>(b + L::D_OFF)[(p / kSkCB) * L::DSTR + p % kSkCB] = r.d[i];
    }
#pragma unroll
    for (int i = 0; i < L::SPL; i++) {
      const int p = tid + L::NT * i;
      if (p < L::SP) {
        reinterpret_cast<float*>(b + L::SA_OFF)[(p % kSkCB) * L::TOKS + p / kSkCB] = r.sa[i];
        reinterpret_cast<int*>(b + L::SM_OFF)[(p % kSkCB) * L::TOKS + p / kSkCB] = r.sm[i];
      }
    }
  };
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  auto compute_t = [&](int buf, int c, auto full) __attribute__((always_inline)) {
    const uint8_t* b = lds + buf * L::BYTES;
    const uint8_t* arow = b + L::A_OFF + (ttile * 16 + j) * L::ASTR + 8 * kg;
    const uint8_t* wrow = b + (rtile * 16 + j) * L::WSTR + (KIND == kKindQ4_0 ? 8 * (kg & 1) : 8 * kg);
    const uint32_t* drow = reinterpret_cast<const uint32_t*>(b + L::D_OFF) + (rtile * 16 + j) * L::DSTR;
    const float* sab = reinterpret_cast<const float*>(b + L::SA_OFF) + ttile * 16 + 4 * kg;
    const int nlive = min(kSkCB, G - c * kSkCB);  // uniform
#pragma unroll
    for (int bb = 0; bb < kSkCB; bb++) {
      const long av = *reinterpret_cast<const long*>(arow + bb * 32);
      long wb = *reinterpret_cast<const long*>(wrow + bb * L::QB);
      if constexpr (KIND == kKindQ4_0) {
        // signed nibbles n - 8 (as gemm_mfma_kernel): the product is isum - 8*sum_a
        constexpr long kLo = 0x0F0F0F0F0F0F0F0FL, kHi = static_cast<long>(0x8080808080808080UL),
                       k8 = 0x0808080808080808L;
        wb = kg < 2 ? (wb & kLo) : ((wb >> 4) & kLo);
        wb = ((wb | kHi) - k8) ^ kHi;
      }
      const v4i_t z = {0, 0, 0, 0};
      const v4i_t cc = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, wb, z, 0, 0, 0);
      const float d = KIND == kKindQ8F ? __uint_as_float(drow[bb]) : f16_operand(static_cast<uint16_t>(drow[bb]));
      const float4 s4 = *reinterpret_cast<const float4*>(sab + bb * L::TOKS);
      const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
      const bool live = decltype(full)::value || bb < nlive;
#pragma unroll
      for (int v = 0; v < 4; v++) {
        const int isum = cc[v];
        const float t = acc[v] + d * sv[v] * static_cast<float>(isum);  // (d*sa)*float(isum), as the decode terms
        acc[v] = live ? t : acc[v];
      }
      // every fourth block: the LDS reads of later blocks may not be hoisted
      // above this point (registers)
      if (bb % 4 == 3) asm volatile("" ::"v"(acc[0]), "v"(acc[1]), "v"(acc[2]), "v"(acc[3]) : "memory");
    }
  };
  // a whole chunk needs no select of live blocks in its epilogue
  auto compute = [&](int buf, int c) __attribute__((always_inline)) {
    if (G - c * kSkCB >= kSkCB) compute_t(buf, c, std::true_type{});
    else compute_t(buf, c, std::false_type{});
  };

  SkRegs<KIND, RW, TT> r0 = load(0), r1;
  store(r0, 0);
  if (n_chunks > 1) r0 = load(1);
  if (n_chunks > 2) r1 = load(2);
  __syncthreads();
  // chunk c+1 sits in r0 when c is even, in r1 when c is odd
  for (int c = 0; c < n_chunks; c += 2) {
    compute(0, c);
    if (c + 1 < n_chunks) store(r0, 1);
    if (c + 3 < n_chunks) r0 = load(c + 3);
    __syncthreads();
    if (c + 1 >= n_chunks) break;
    compute(1, c + 1);
    if (c + 2 < n_chunks) store(r1, 0);
    if (c + 4 < n_chunks) r1 = load(c + 4);
    __syncthreads();
  }
  if constexpr (ACT) {
    // the last chunk's barrier is behind: the staging buffers are free.
    // s_x[t][row] holds the gate values, then h, of this workgroup's 32 rows.
    constexpr int kXs = 33;  // padded row of 32 values per token
    float* s_x = reinterpret_cast<float*>(lds);
    const int lr = (rtile & 1) * 16 + j;  // row within the 32
    if (rtile < 2) {
#pragma unroll
      for (int v = 0; v < 4; v++) s_x[(4 * kg + v) * kXs + lr] = acc[v];
    }
    __syncthreads();
    if (rtile >= 2) {
#pragma unroll
      for (int v = 0; v < 4; v++) {
        float g = s_x[(4 * kg + v) * kXs + lr];
        if (job.gelu) {
          const float kS = 0.7978846f;  // norms.rs:36
          const float x3 = g * g * g;
          g = 0.5f * g * (1.0f + dev_tanhf(kS * (g + 0.044715f * x3)));
        } else {
          g = g * (1.0f / (1.0f + dev_expf(-g)));
        }
        s_x[(4 * kg + v) * kXs + lr] = g * acc[v];
      }
    }
    __syncthreads();
    // half-wave g (tid / 32) takes tokens g and g + 8, one row per lane: one
    // 32-row block of h per token for quantize_lanes
    const int hr = tid & 31, tg = tid >> 5;
    float hv[2] = {s_x[tg * kXs + hr], s_x[(tg + 8) * kXs + hr]};
    int qv[2], sm[2];
    float sc[2];
    quantize_lanes<2>(hv, qv, sc, sm);
#pragma unroll
    for (int b = 0; b < 2; b++) {
      const int t = tg + 8 * b;
      if (t < n_tok) {
        const size_t gi = (size_t)t * R + row0 + hr;
        job.hq[gi] = static_cast<int8_t>(qv[b]);
        if (job.h) job.h[gi] = hv[b];
        if (hr == 0) {
          job.hsa[gi >> 5] = sc[b];
          job.hsum[gi >> 5] = sm[b];
        }
      }
    }
    return;
  }
  const int n_row = row0 + rtile * 16 + j;
  if (n_row < R) {
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const int t = 16 * ttile + 4 * kg + v;
      if (t < n_tok) store_out(o, t, n_row, acc[v]);
    }
  }
}

// ---- one 16-row x 16-token tile per workgroup, blocks split over 8 waves
// Below 8192 rows, 16-row workgroups of one wave per token tile leave most
// SIMDs idle, and each wave walks its row tile's blocks alone. Here a
// workgroup takes one 16-row x 16-token tile (grid: row tiles x token tiles;
// a row tile's weights are read once per token tile, mostly from the caches
// for matrices this small), and its 8 waves take
// consecutive chunks of kSkCB blocks (wave w: chunk 8i + w), each staged in
// the wave's own LDS region and multiplied on the matrix cores as in
// gemm_skinny_kernel; each block's term (d*sa)*float(isum) goes to LDS, and
// lane (row, token) of the first four waves then adds the 8*kSkCB terms of
// its output in block order: the same left-to-right fold as every other
// kernel. With one such workgroup per CU, the weight bytes in flight are
// what bounds the stream (4 waves: 8 KB per CU, ~1.3 TB/s over the chip),
// so the workgroup is as wide as the LDS allows. Tokens past n_tok load
// nothing: their columns of the products are never stored.
// A batch of more than one token tile has a workgroup per (row tile, token
// tile): there two four-wave workgroups per CU (70 KB each) beat one of
// eight (4096 x 14336 at 64 tokens: 73.0 against 82.7 us).
template <int KIND, int kKsWaves>
__global__ __launch_bounds__(64 * kKsWaves) void gemm_skinny_ks_kernel(DevMat m, const int8_t* __restrict__ q,
                                                                      const float* __restrict__ sa,
                                                                      const int* __restrict__ sums, int n_tok,
                                                                      GemvOut o) {
  static_assert(KIND == kKindQ4_0 || KIND == kKindQ8_0 || KIND == kKindQ8F, "block-32 kinds");
  using L = SkLayout<KIND, 1, 1>;  // one wave's staging: 16 rows x 16 tokens x kSkCB blocks
  static_assert(L::NT == 64, "one wave per staged chunk");
  // terms of one block: token t, row r at (t + t/4)*16 + r (the 4 tokens of a
  // lane's MFMA result land 16 banks apart from the next lane group's)
  constexpr int kTermStride = 20 * 16;
  extern __shared__ int4 sk_smem[];
  uint8_t* lds = reinterpret_cast<uint8_t*>(sk_smem);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 15, kg = lane >> 4;
  const int K = static_cast<int>(m.cols), G = K / 32, R = static_cast<int>(m.rows);
  const int row0 = static_cast<int>(blockIdx.x) * 16;
  const int tok0 = static_cast<int>(blockIdx.y) * 16;  // this workgroup's token tile
  const int n_chunks = (G + kSkCB - 1) / kSkCB;
  // each wave's staging region ends before the layout's activation sums,
  // which this kernel does not use
  uint8_t* stage = lds + wave * L::SM_OFF;
  float* terms = reinterpret_cast<float*>(lds + kKsWaves * L::SM_OFF);

  auto load = [&](int c) __attribute__((always_inline)) {  // this lane's share of chunk c (clamped addresses)
    SkRegs<KIND, 1, 1> r;
    const int cb0 = c * kSkCB;
#pragma unroll
    for (int i = 0; i < L::WPL; i++) {
      const int p = min(lane + 64 * i, L::WP - 1);
      const int rr = min(row0 + p / L::WPR, R - 1), pr = p % L::WPR;
      const int blk = min(cb0 + pr / (L::QB / 16), G - 1);
      const uint8_t* src = m.qs + (size_t)rr * G * L::QB + (size_t)blk * L::QB + (pr % (L::QB / 16)) * 16;
      r.w[i] = *reinterpret_cast<const sk_i4*>(src);
    }
#pragma unroll
    for (int i = 0; i < L::APL; i++) {
      const int p = min(lane + 64 * i, L::AP - 1);
      const int t = tok0 + p / (2 * kSkCB), pr = p % (2 * kSkCB);
      const int blk = min(cb0 + pr / 2, G - 1);
      r.a[i] = sk_i4{};
      if (t < n_tok) r.a[i] = *reinterpret_cast<const sk_i4*>(q + (size_t)t * K + (size_t)blk * 32 + (pr & 1) * 16);
    }
#pragma unroll
    for (int i = 0; i < L::DPL; i++) {
      const int p = min(lane + 64 * i, L::DP - 1);
      const size_t gi = (size_t)min(row0 + p / kSkCB, R - 1) * G + min(cb0 + p % kSkCB, G - 1);
      if constexpr (KIND == kKindQ8F) r.d[i] = reinterpret_cast<const uint32_t*>(m.sc)[gi];
      else r.d[i] = reinterpret_cast<const uint16_t*>(m.sc)[gi];
    }
#pragma unroll
    for (int i = 0; i < L::SPL; i++) {
      const int p = min(lane + 64 * i, L::SP - 1);
      const int t = tok0 + p / kSkCB;
      r.sa[i] = 0.0f;
      if (t < n_tok) r.sa[i] = sa[(size_t)t * G + min(cb0 + p % kSkCB, G - 1)];
    }
    return r;
  };
  auto store = [&](const SkRegs<KIND, 1, 1>& r) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < L::WPL; i++) {
      const int p = lane + 64 * i;
      if (p < L::WP) *reinterpret_cast<sk_i4*>(stage + (p / L::WPR) * L::WSTR + (p % L::WPR) * 16) = r.w[i];
    }
#pragma unroll
    for (int i = 0; i < L::APL; i++) {
      const int p = lane + 64 * i;
      if (p < L::AP)
        *reinterpret_cast<sk_i4*>(stage + L::A_OFF + (p / (2 * kSkCB)) * L::ASTR + (p % (2 * kSkCB)) * 16) = r.a[i];
    }
#pragma unroll
    for (int i = 0; i < L::DPL; i++) {
      const int p = lane + 64 * i;
      if (p < L::DP) reinterpret_cast<uint32_t*>(stage + L::D_OFF)[(p / kSkCB) * L::DSTR + p % kSkCB] = r.d[i];
    }
#pragma unroll
    for (int i = 0; i < L::SPL; i++) {
      const int p = lane + 64 * i;
      if (p < L::SP) reinterpret_cast<float*>(stage + L::SA_OFF)[(p % kSkCB) * L::TOKS + p / kSkCB] = r.sa[i];
    }
  };
  // block terms of this wave's staged chunk -> terms[wave][bb]
  auto products = [&]() __attribute__((always_inline)) {
    const uint8_t* arow = stage + L::A_OFF + j * L::ASTR + 8 * kg;
    const uint8_t* wrow = stage + j * L::WSTR + (KIND == kKindQ4_0 ? 8 * (kg & 1) : 8 * kg);
    const uint32_t* drow = reinterpret_cast<const uint32_t*>(stage + L::D_OFF) + j * L::DSTR;
    const float* sab = reinterpret_cast<const float*>(stage + L::SA_OFF) + 4 * kg;
    float* tw = terms + wave * kSkCB * kTermStride + 5 * kg * 16 + j;
#pragma unroll
    for (int bb = 0; bb < kSkCB; bb++) {
      const long av = *reinterpret_cast<const long*>(arow + bb * 32);
      long wb = *reinterpret_cast<const long*>(wrow + bb * L::QB);
      if constexpr (KIND == kKindQ4_0) {
        // signed nibbles n - 8: the product is isum - 8*sum_a
        constexpr long kLo = 0x0F0F0F0F0F0F0F0FL, kHi = static_cast<long>(0x8080808080808080UL),
                       k8 = 0x0808080808080808L;
        wb = kg < 2 ? (wb & kLo) : ((wb >> 4) & kLo);
        wb = ((wb | kHi) - k8) ^ kHi;
      }
      const v4i_t z = {0, 0, 0, 0};
      const v4i_t cc = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, wb, z, 0, 0, 0);
      const float d = KIND == kKindQ8F ? __uint_as_float(drow[bb]) : f16_operand(static_cast<uint16_t>(drow[bb]));
      const float4 s4 = *reinterpret_cast<const float4*>(sab + bb * L::TOKS);
      const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
      for (int v = 0; v < 4; v++) tw[bb * kTermStride + v * 16] = d * sv[v] * static_cast<float>(cc[v]);
    }
  };

  const int fr = tid & 15, ft = (tid >> 4) & 15;  // the output this lane folds: row fr, token ft
  const bool folder = tid < 256;                  // (uniform per wave)
  const float* tf = terms + (ft + (ft >> 2)) * 16 + fr;
  float acc = 0.0f;
  // a chunk at or past n_chunks holds clamped (repeated) blocks, never folded
  SkRegs<KIND, 1, 1> r = load(wave);
  for (int c0 = 0; c0 < n_chunks; c0 += kKsWaves) {
    store(r);
    if (c0 + kKsWaves + wave < n_chunks) r = load(c0 + kKsWaves + wave);
    __syncthreads();  // staged chunks visible; the previous group's terms all folded
    products();
    __syncthreads();  // terms visible
    const int nb = min(kKsWaves * kSkCB, G - c0 * kSkCB);  // uniform: live blocks of this group
    if (!folder) {
    } else if (nb == kKsWaves * kSkCB) {
      // whole group: every read issued before the adds
      float t[kKsWaves * kSkCB];
#pragma unroll
      for (int b = 0; b < kKsWaves * kSkCB; b++) t[b] = tf[b * kTermStride];
#pragma unroll
      for (int b = 0; b < kKsWaves * kSkCB; b++) acc = acc + t[b];
    } else {
      for (int b = 0; b < nb; b++) acc = acc + tf[b * kTermStride];
    }
  }
  const int n_row = row0 + fr;
  if (folder && n_row < R && tok0 + ft < n_tok) store_out(o, tok0 + ft, n_row, acc);
}

template <int KIND, int W>
int launch_skinny_ks_w(const DevMat& m, const int8_t* q, const float* sa, const int* sums, size_t n_tok,
                       const GemvOut& o, hipStream_t s) {
  using L = SkLayout<KIND, 1, 1>;
  constexpr int kBytes = W * L::SM_OFF + W * kSkCB * 20 * 16 * 4;
  static_assert(kBytes <= 160 * 1024, "one workgroup's staging and terms fit a CU's LDS");
  static const bool attr_ok = [] {
    return kBytes <= 65536 ||
           set_max_dynamic_lds(reinterpret_cast<const void*>(gemm_skinny_ks_kernel<KIND, W>), kBytes);
  }();
  PRANA_CHECK(attr_ok, "gemm_skinny: LDS size not granted");
  hipLaunchKernelGGL((gemm_skinny_ks_kernel<KIND, W>), dim3((m.rows + 15) / 16, (n_tok + 15) / 16), dim3(64 * W),
                     kBytes, s, m, q, sa, sums, (int)n_tok, o);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

template <int KIND>
int launch_skinny_ks(const DevMat& m, const int8_t* q, const float* sa, const int* sums, size_t n_tok,
                     const GemvOut& o, hipStream_t s) {
  if (n_tok <= 16) return launch_skinny_ks_w<KIND, 8>(m, q, sa, sums, n_tok, o, s);
  return launch_skinny_ks_w<KIND, 4>(m, q, sa, sums, n_tok, o, s);
}

template <int KIND, int RW, int TT>
int launch_skinny_t(const DevMat* ms, const GemvOut* os, int n_mats, const int8_t* q, const float* sa,
                    const int* sums, size_t n_tok, hipStream_t s) {
  using L = SkLayout<KIND, RW, TT>;
  static const bool attr_ok = [] {
    return L::BYTES * 2 <= 65536 ||
           set_max_dynamic_lds(reinterpret_cast<const void*>(gemm_skinny_kernel<KIND, RW, TT>), L::BYTES * 2);
  }();
  PRANA_CHECK(attr_ok, "gemm_skinny: LDS size not granted");
  SkJob job{};
  size_t tiles = 0;
  for (int i = 0; i < 3; i++) {
    job.t0[i] = i < n_mats ? static_cast<int>(tiles) : INT32_MAX;
    job.m[i] = ms[i < n_mats ? i : 0];
    job.o[i] = os[i < n_mats ? i : 0];
    if (i < n_mats) tiles += (ms[i].rows + L::ROWS - 1) / L::ROWS;
  }
  PRANA_CHECK(tiles <= static_cast<size_t>(INT32_MAX), "gemm_skinny: too many row tiles");
  hipLaunchKernelGGL((gemm_skinny_kernel<KIND, RW, TT>), dim3(tiles), dim3(L::NT), L::BYTES * 2, s, job, q, sa,
                     sums, (int)n_tok);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

template <int KIND, int TT>
int launch_skinny_tt(const DevMat* ms, const GemvOut* os, int n_mats, const int8_t* q, const float* sa,
                     const int* sums, size_t n_tok, hipStream_t s) {
  // rows per workgroup: grow while at least 256 workgroups remain over all
  // the matrices (bigger tiles share each staged activation chunk among more
  // rows); where even 32-row tiles leave fewer, each matrix goes to the
  // block-split kernel instead
  auto tiles = [&](size_t rows_per_tile) {
    size_t t = 0;
    for (int i = 0; i < n_mats; i++) t += (ms[i].rows + rows_per_tile - 1) / rows_per_tile;
    return t;
  };
  int rw = 1;
  while (rw < 4 && tiles(32 * rw) >= 256) rw *= 2;
  if (rw == 1) {
    for (int i = 0; i < n_mats; i++)
      if (int rc = launch_skinny_ks<KIND>(ms[i], q, sa, sums, n_tok, os[i], s)) return rc;
    return kOk;
  }
  if (rw == 2) return launch_skinny_t<KIND, 2, TT>(ms, os, n_mats, q, sa, sums, n_tok, s);
  return launch_skinny_t<KIND, 4, TT>(ms, os, n_mats, q, sa, sums, n_tok, s);
}

template <int KIND>
int launch_gemm_skinny(const DevMat* ms, const GemvOut* os, int n_mats, const int8_t* q, const float* sa,
                       const int* sums, size_t n_tok, hipStream_t s) {
  PRANA_CHECK(n_mats >= 1 && n_mats <= 3 && n_tok >= 1 && n_tok <= 64, "gemm_skinny: job out of range");
  for (int i = 0; i < n_mats; i++)
    PRANA_CHECK(ms[i].kind == KIND && ms[i].cols == ms[0].cols && ms[i].cols % 32 == 0 &&
                    ms[i].cols <= (1u << 30) && ms[i].rows <= (1u << 30),
                "gemm_skinny: shape out of range");
  if (n_tok <= 16) return launch_skinny_tt<KIND, 1>(ms, os, n_mats, q, sa, sums, n_tok, s);
  if (n_tok <= 32) return launch_skinny_tt<KIND, 2>(ms, os, n_mats, q, sa, sums, n_tok, s);
  return launch_skinny_tt<KIND, 4>(ms, os, n_mats, q, sa, sums, n_tok, s);
}

template <int KIND>
int launch_skinny_act(const DevMat& gate, const DevMat& up, const int8_t* q, const float* sa, const int* sums,
                      size_t n_tok, int gelu, float* h, int8_t* hq, float* hsa, int* hsum, hipStream_t s) {
  using L = SkLayout<KIND, 4, 1>;
  static const bool attr_ok = [] {
    return L::BYTES * 2 <= 65536 ||
           set_max_dynamic_lds(reinterpret_cast<const void*>(gemm_skinny_kernel<KIND, 4, 1, true>), L::BYTES * 2);
  }();
  PRANA_CHECK(attr_ok, "gemm_skinny: LDS size not granted");
  static_assert(16 * 33 * 4 <= 2 * L::BYTES, "the act epilogue's h rows fit the staging buffers");
  SkJob job{};
  job.m[0] = job.m[2] = gate;
  job.m[1] = up;
  job.t0[0] = 0;
  job.t0[1] = job.t0[2] = INT32_MAX;
  job.gelu = gelu;
  job.h = h;
  job.hq = hq;
  job.hsa = hsa;
  job.hsum = hsum;
  hipLaunchKernelGGL((gemm_skinny_kernel<KIND, 4, 1, true>), dim3(gate.rows / 32), dim3(L::NT), L::BYTES * 2, s, job,
                     q, sa, sums, (int)n_tok);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

int launch_gemm_skinny_any(const DevMat* ms, const GemvOut* os, int n_mats, const int8_t* q, const float* sa,
                           const int* sums, size_t n_tok, hipStream_t s) {
  switch (ms[0].kind) {
    case kKindQ8F: return launch_gemm_skinny<kKindQ8F>(ms, os, n_mats, q, sa, sums, n_tok, s);
    case kKindQ8_0: return launch_gemm_skinny<kKindQ8_0>(ms, os, n_mats, q, sa, sums, n_tok, s);
    case kKindQ4_0: return launch_gemm_skinny<kKindQ4_0>(ms, os, n_mats, q, sa, sums, n_tok, s);
    default: return fail(kErrInvalid, "gemm_skinny: block-32 kinds only");
  }
}

// ---- K-quant batches (Q4_K, Q6_K) on the 16x16x32 int8 matrix cores
// The same tiling and LDS staging as the skinny kernel, with chunks of two
// 256-element super-blocks. One MFMA step is one 32-element group:
//   Q4_K: s = sum a*q over the group's nibbles (unsigned, one MFMA), then
//         term = sa*((d*sc)*float(s) - (dmin*m)*float(sum_a))   (kquant.rs:257-282)
//   Q6_K: q - 32 as signed bytes; the group's two 16-element sub-blocks are
//         two MFMAs whose activation operands zero the other half, then
//         term = ((d*sa)*float(sc))*float(isum16), sub-block 0 first   (kquant.rs:287-318)
// Every output folds its terms in element order.
constexpr int kKqCS = 1;  // super-blocks per staged chunk

template <int KIND, int RW, int TT>
struct KqLayout {
  static constexpr int NT = 64 * RW * TT;
  static constexpr int ROWS = 16 * RW, TOKS = 16 * TT;
  static constexpr int UB = KIND == kKindQ4_K ? 144 : 208;  // quant-array bytes per super-block
  static constexpr int WSTR = kKqCS * UB + 16;               // padded staged weight row
  static constexpr int ASTR = kKqCS * 256 + 16;              // padded staged activation row
  static constexpr int DSTR = kKqCS + 1;                     // Q6_K d words per staged row
  static constexpr int NG = kKqCS * 8;                       // 32-element groups per chunk
  static constexpr int A_OFF = ROWS * WSTR;
  static constexpr int D_OFF = A_OFF + TOKS * ASTR;
  static constexpr int SA_OFF = D_OFF + ROWS * DSTR * 4;
  static constexpr int SM_OFF = SA_OFF + NG * TOKS * 4;
  static constexpr int BYTES = SM_OFF + NG * TOKS * 4;
  static constexpr int WPR = kKqCS * UB / 16;  // 16-byte pieces per row
  static constexpr int WP = ROWS * WPR, AP = TOKS * kKqCS * 16, DP = ROWS * kKqCS, SP = TOKS * NG;
  static constexpr int WPL = (WP + NT - 1) / NT, APL = (AP + NT - 1) / NT;
  static constexpr int DPL = (DP + NT - 1) / NT, SPL = (SP + NT - 1) / NT;
};

template <int KIND, int RW, int TT>
struct KqRegs {
  using L = KqLayout<KIND, RW, TT>;
  sk_i4 w[L::WPL], a[L::APL];
  uint16_t d[L::DPL];  // Q6_K's f16 scale (0 for the other kinds)
  float sa[L::SPL];
  int sm[L::SPL];
};

template <int KIND, int RW, int TT>
__global__ __launch_bounds__(64 * RW * TT) void gemm_kq_kernel(DevMat m, const int8_t* __restrict__ q,
                                                               const float* __restrict__ sa,
                                                               const int* __restrict__ sums, int n_tok, GemvOut o) {
  static_assert(KIND == kKindQ4_K || KIND == kKindQ6_K, "K-quant kinds");
  using L = KqLayout<KIND, RW, TT>;
  {  // blockIdx.y: this workgroup's group of TOKS tokens
    const size_t t0 = (size_t)blockIdx.y * L::TOKS;
    q += t0 * m.cols;
    sa += t0 * (m.cols / 32);
    sums += t0 * (m.cols / 32);
    o.out += t0 * o.ldo;
    n_tok = min(n_tok - static_cast<int>(t0), L::TOKS);
  }
  extern __shared__ int4 kq_smem[];
  uint8_t* lds = reinterpret_cast<uint8_t*>(kq_smem);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rtile = wave % RW, ttile = wave / RW;
  const int j = lane & 15, kg = lane >> 4;
  const int K = static_cast<int>(m.cols), G = K / 32, NB = K / 256, R = static_cast<int>(m.rows);
  const int row0 = static_cast<int>(blockIdx.x) * L::ROWS;
  const int n_chunks = (NB + kKqCS - 1) / kKqCS;

  auto load = [&](int c) __attribute__((always_inline)) {
    KqRegs<KIND, RW, TT> r;
    const int sb0 = c * kKqCS;
#pragma unroll
    for (int i = 0; i < L::WPL; i++) {
      const int p = min(tid + L::NT * i, L::WP - 1);
      const int rr = min(row0 + p / L::WPR, R - 1), pr = p % L::WPR;
      const int sb = min(sb0 + pr / (L::UB / 16), NB - 1);
      r.w[i] = *reinterpret_cast<const sk_i4*>(m.qs + ((size_t)rr * NB + sb) * L::UB + (pr % (L::UB / 16)) * 16);
    }
#pragma unroll
    for (int i = 0; i < L::APL; i++) {
      const int p = min(tid + L::NT * i, L::AP - 1);
      const int t = min(p / (kKqCS * 16), n_tok - 1), pr = p % (kKqCS * 16);
      const int sb = min(sb0 + pr / 16, NB - 1);
      r.a[i] = *reinterpret_cast<const sk_i4*>(q + (size_t)t * K + (size_t)sb * 256 + (pr % 16) * 16);
    }
#pragma unroll
    for (int i = 0; i < L::DPL; i++) {
      const int p = min(tid + L::NT * i, L::DP - 1);
      const size_t gi = (size_t)min(row0 + p / kKqCS, R - 1) * NB + min(sb0 + p % kKqCS, NB - 1);
      r.d[i] = KIND == kKindQ6_K ? reinterpret_cast<const uint16_t*>(m.sc)[gi] : uint16_t{0};
    }
#pragma unroll
    for (int i = 0; i < L::SPL; i++) {
      const int p = min(tid + L::NT * i, L::SP - 1);
      const size_t gi = (size_t)min(p / L::NG, n_tok - 1) * G + min(sb0 * 8 + p % L::NG, G - 1);
      r.sa[i] = sa[gi];
      r.sm[i] = sums[gi];
    }
    return r;
  };
  auto store = [&](const KqRegs<KIND, RW, TT>& r, int buf) __attribute__((always_inline)) {
    uint8_t* b = lds + buf * L::BYTES;
#pragma unroll
    for (int i = 0; i < L::WPL; i++) {
      const int p = tid + L::NT * i;
      if (p < L::WP) *reinterpret_cast<sk_i4*>(b + (p / L::WPR) * L::WSTR + (p % L::WPR) * 16) = r.w[i];
    }
#pragma unroll
    for (int i = 0; i < L::APL; i++) {
      const int p = tid + L::NT * i;
      if (p < L::AP)
        *reinterpret_cast<sk_i4*>(b + L::A_OFF + (p / (kKqCS * 16)) * L::ASTR + (p % (kKqCS * 16)) * 16) = r.a[i];
    }
#pragma unroll
    for (int i = 0; i < L::DPL; i++) {
      const int p = tid + L::NT * i;
      if (p < L::DP) reinterpret_cast<uint32_t*>(b + L::D_OFF)[(p / kKqCS) * L::DSTR + p % kKqCS] = r.d[i];
    }
#pragma unroll
    for (int i = 0; i < L::SPL; i++) {
      const int p = tid + L::NT * i;
      if (p < L::SP) {
        reinterpret_cast<float*>(b + L::SA_OFF)[(p % L::NG) * L::TOKS + p / L::NG] = r.sa[i];
        reinterpret_cast<int*>(b + L::SM_OFF)[(p % L::NG) * L::TOKS + p / L::NG] = r.sm[i];
      }
    }
  };
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  auto compute = [&](int buf, int c) __attribute__((always_inline)) {
    const uint8_t* b = lds + buf * L::BYTES;
    const uint8_t* arow = b + L::A_OFF + (ttile * 16 + j) * L::ASTR + 8 * kg;
    const uint8_t* wrow = b + (rtile * 16 + j) * L::WSTR;
    const uint32_t* drow = reinterpret_cast<const uint32_t*>(b + L::D_OFF) + (rtile * 16 + j) * L::DSTR;
    const float* sab = reinterpret_cast<const float*>(b + L::SA_OFF) + ttile * 16 + 4 * kg;
    const int* smb = reinterpret_cast<const int*>(b + L::SM_OFF) + ttile * 16 + 4 * kg;
    const int nlive = min(kKqCS, NB - c * kKqCS);  // uniform
#pragma unroll
    for (int sbl = 0; sbl < kKqCS; sbl++) {
      const uint8_t* blk = wrow + sbl * L::UB;
      const bool live = sbl < nlive;
#pragma unroll
      for (int g32 = 0; g32 < 8; g32++) {
        const int gl = sbl * 8 + g32;  // group within the chunk
        const long av = *reinterpret_cast<const long*>(arow + sbl * 256 + g32 * 32);
        const float4 s4 = *reinterpret_cast<const float4*>(sab + gl * L::TOKS);
        const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
        const v4i_t z = {0, 0, 0, 0};
        if constexpr (KIND == kKindQ4_K) {
          const int4 m4 = *reinterpret_cast<const int4*>(smb + gl * L::TOKS);
          const int mv[4] = {m4.x, m4.y, m4.z, m4.w};
          const long raw = *reinterpret_cast<const long*>(blk + 16 + (g32 >> 1) * 32 + 8 * kg);
          const long nib = (g32 & 1) ? ((raw >> 4) & 0x0F0F0F0F0F0F0F0FL) : (raw & 0x0F0F0F0F0F0F0F0FL);
          const v4i_t cc = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, nib, z, 0, 0, 0);
          const uint32_t dd = *reinterpret_cast<const uint32_t*>(blk);
          const float d = f16_to_f32(static_cast<uint16_t>(dd & 0xffffu));
          const float dmin = f16_to_f32(static_cast<uint16_t>(dd >> 16));
          int sc, mn;
          Fmt<kKindQ4_K>::scale_min(g32, blk + 4, sc, mn);
          const float dsc = d * static_cast<float>(sc), dmn = dmin * static_cast<float>(mn);
#pragma unroll
          for (int v = 0; v < 4; v++) {
            const float t = acc[v] + sv[v] * (dsc * static_cast<float>(cc[v]) - dmn * static_cast<float>(mv[v]));
            acc[v] = live ? t : acc[v];
          }
        } else {
          const int half = g32 >> 2, g = g32 & 3;
          const long ql = *reinterpret_cast<const long*>(blk + half * 64 + (g & 1) * 32 + 8 * kg);
          const long qh = *reinterpret_cast<const long*>(blk + 128 + half * 32 + 8 * kg);
          const long nib = g < 2 ? (ql & 0x0F0F0F0F0F0F0F0FL) : ((ql >> 4) & 0x0F0F0F0F0F0F0F0FL);
          const long q6 = nib | (((qh >> (2 * g)) & 0x0303030303030303L) << 4);  // 0..63 per byte
          // q - 32 per byte: add 0x80, subtract 0x20 (no borrow leaves a byte), flip the top bit
          const long qs = ((q6 | static_cast<long>(0x8080808080808080ULL)) - 0x2020202020202020L) ^
                          static_cast<long>(0x8080808080808080ULL);
          const v4i_t c0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(kg < 2 ? av : 0L, qs, z, 0, 0, 0);
          const v4i_t c1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(kg < 2 ? 0L : av, qs, z, 0, 0, 0);
          const float d = f16_operand(static_cast<uint16_t>(drow[sbl]));
          const int8_t* scp = reinterpret_cast<const int8_t*>(blk + 192 + half * 8 + g * 2);
          const float sc0 = static_cast<float>(scp[0]), sc1 = static_cast<float>(scp[1]);
#pragma unroll
          for (int v = 0; v < 4; v++) {
            const float ds = d * sv[v];
            float t = acc[v] + ds * sc0 * static_cast<float>(c0[v]);
            t = t + ds * sc1 * static_cast<float>(c1[v]);
            acc[v] = live ? t : acc[v];
          }
        }
        if (g32 % 4 == 3) asm volatile("" ::"v"(acc[0]), "v"(acc[1]), "v"(acc[2]), "v"(acc[3]) : "memory");
      }
    }
  };

  KqRegs<KIND, RW, TT> r0 = load(0), r1;
  store(r0, 0);
  if (n_chunks > 1) r0 = load(1);
  if (n_chunks > 2) r1 = load(2);
  __syncthreads();
  for (int c = 0; c < n_chunks; c += 2) {
    compute(0, c);
    if (c + 1 < n_chunks) store(r0, 1);
    if (c + 3 < n_chunks) r0 = load(c + 3);
    __syncthreads();
    if (c + 1 >= n_chunks) break;
    compute(1, c + 1);
    if (c + 2 < n_chunks) store(r1, 0);
    if (c + 4 < n_chunks) r1 = load(c + 4);
    __syncthreads();
  }
  const int n_row = row0 + rtile * 16 + j;
  if (n_row < R) {
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const int t = 16 * ttile + 4 * kg + v;
      if (t < n_tok) store_out(o, t, n_row, acc[v]);
    }
  }
}

template <int KIND, int RW, int TT>
int launch_kq_t(const DevMat& m, const int8_t* q, const float* sa, const int* sums, size_t n_tok, const GemvOut& o,
                hipStream_t s) {
  using L = KqLayout<KIND, RW, TT>;
  static const bool attr_ok = [] {
    return L::BYTES * 2 <= 65536 ||
           set_max_dynamic_lds(reinterpret_cast<const void*>(gemm_kq_kernel<KIND, RW, TT>), L::BYTES * 2);
  }();
  PRANA_CHECK(attr_ok, "gemm_kq: LDS size not granted");
  hipLaunchKernelGGL((gemm_kq_kernel<KIND, RW, TT>),
                     dim3((m.rows + L::ROWS - 1) / L::ROWS, (n_tok + L::TOKS - 1) / L::TOKS), dim3(L::NT),
                     L::BYTES * 2, s, m, q, sa, sums, (int)n_tok, o);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

// Batches of any size: grid (row tiles, groups of 64 tokens).
template <int KIND>
int launch_gemm_kq(const DevMat& m, const int8_t* q, const float* sa, const int* sums, size_t n_tok,
                   const GemvOut& o, hipStream_t s) {
  PRANA_CHECK(m.cols % 256 == 0 && m.cols <= (1u << 30) && m.rows <= (1u << 30) && n_tok <= (1u << 24),
              "gemm_kq: shape out of range");
  const bool two = (m.rows + 31) / 32 * ((n_tok + 63) / 64) >= 256;  // 32-row tiles still fill the GPU
  if (two) return launch_kq_t<KIND, 2, 4>(m, q, sa, sums, n_tok, o, s);
  return launch_kq_t<KIND, 1, 4>(m, q, sa, sums, n_tok, o, s);
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

bool gemm_skinny_act_fusable(const DevMat& gate, const DevMat& up, size_t n_tok) {
  const int k = gate.kind;
  return (k == kKindQ8F || k == kKindQ8_0 || k == kKindQ4_0) && up.kind == k && gate.rows == up.rows &&
         gate.cols == up.cols && gate.rows % 32 == 0 && gate.rows <= (1u << 30) && gate.cols % 32 == 0 &&
         gate.cols <= (1u << 30) && n_tok >= 1 && n_tok <= 16 && gemv_batch_skinny(gate, n_tok);
}

int launch_gemm_skinny_act(const DevMat& gate, const DevMat& up, const int8_t* q, const float* sa, const int* sums,
                           size_t n_tok, int gelu, float* h, int8_t* hq, float* hsa, int* hsum, hipStream_t s) {
  PRANA_CHECK(gemm_skinny_act_fusable(gate, up, n_tok) && hq && hsa && hsum,
              "gemm_skinny_act: gate and up must be equal block-32 matrices of rows % 32 == 0, 1..16 tokens");
  switch (gate.kind) {
    case kKindQ8F: return launch_skinny_act<kKindQ8F>(gate, up, q, sa, sums, n_tok, gelu, h, hq, hsa, hsum, s);
    case kKindQ8_0: return launch_skinny_act<kKindQ8_0>(gate, up, q, sa, sums, n_tok, gelu, h, hq, hsa, hsum, s);
    default: return launch_skinny_act<kKindQ4_0>(gate, up, q, sa, sums, n_tok, gelu, h, hq, hsa, hsum, s);
  }
}

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

// Compute units of the current device (cached per device).
static int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cus[dev] == 0) {
    int c = 0;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cus[dev] = c;
  }
  return cus[dev];
}

// A fused rmsnorm pays the norm once per workgroup, so it is taken when one
// workgroup per compute unit covers every tile: block-32 units of one format
// (or the Q4_0 / Q8_0 pair for rows of at most 1024 values), rows of
// 512 < cols <= kNormMaxK (a multiple of 32) that norm_geom tiles, with 256
// lanes up to 1024 values and kNormNT lanes beyond.
bool gemv_norm_fusable(const DevMat* ms, int n) {
  if (n < 1 || n > 3) return false;
  const size_t K = ms[0].cols;
  bool one_kind = true;
  for (int i = 0; i < n; i++) {
    if (ms[i].cols != K) return false;
    one_kind = one_kind && ms[i].kind == ms[0].kind;
  }
  if (K <= 512 || K > static_cast<size_t>(kNormMaxK) || K % 32 != 0) return false;
  // two formats: the block-32 pair, at 256 lanes (rows of at most 1024 values)
  if (!one_kind && (K > 1024 || mixed_pair(ms, n) != std::make_pair(static_cast<int>(kKindQ4_0),
                                                                     static_cast<int>(kKindQ8_0))))
    return false;
  const int kind = ms[0].kind;
  if (kind != kKindQ8F && kind != kKindQ8_0 && kind != kKindQ4_0) return false;
  size_t tiles = 0;
  int rt = 0;
  dispatch_kind(kind, [&](auto k) {
    rt = norm_geom<decltype(k)::value>(K).rt;
    return 0;
  });
  if (rt == 0) return false;
  for (int i = 0; i < n; i++) tiles += (ms[i].rows + rt - 1) / rt;
  const int cus = device_cus();
  return cus > 0 && tiles <= static_cast<size_t>(cus);
}

int launch_gemv_multi(const DevMat* ms, const GemvOut* os, int n, const int8_t* q, const float* sa, const int* sums,
                      size_t n_tok, hipStream_t s, const RopeKv* rk, bool* fused, const NormIn* norm) {
  PRANA_CHECK(n >= 1 && n <= 3, "gemv_multi: 1..3 matrices");
  if (fused) *fused = false;
  if (n_tok == 0) return kOk;
  if (norm) {
    PRANA_CHECK(n_tok == 1 && norm->x && norm->w && gemv_norm_fusable(ms, n),
                "gemv_multi: these matrices cannot take a fused rmsnorm");
    DecodeJob job{};
    for (int i = 0; i < n; i++) {
      job.m[i] = ms[i];
      job.o[i] = os[i];
    }
    job.n_mats = n;
    job.nin = *norm;
    bool mixed = false;
    for (int i = 1; i < n; i++) mixed = mixed || ms[i].kind != ms[0].kind;
    return dispatch_kind(ms[0].kind, [&](auto k) {
      constexpr int KIND = decltype(k)::value;
      if constexpr (RegUnit<KIND>::kElems == 32) {
        const TileGeom g = norm_geom<KIND>(ms[0].cols);
        // RoPE and the cache rows ride along when the tiles hold whole pairs
        if (rk && n == 3 && ms[1].rows == ms[2].rows && rk->hd > 0 && rk->hd % 2 == 0 &&
            ms[0].rows % rk->hd == 0 && ms[1].rows % rk->hd == 0 && !os[0].residual && !os[1].residual &&
            !os[2].residual && (rk->neox ? g.rt % rk->hd == 0 : g.rt % 2 == 0)) {
          job.rk = *rk;
          if (fused) *fused = true;
        }
        constexpr int B = kNormNT, S = kNormNTSmall;
        if (mixed) {  // Q4_0 with Q8_0 (gemv_norm_fusable), 256 lanes
          constexpr int KA = kKindQ4_0, KB = kKindQ8_0;
          if (g.nt == S && g.u == 7)
            return launch_tile_u<KA, 7, false, false, S, KB, true>(job, g, q, sa, sums, 1, s);
          if (g.nt == S && g.u == 4)
            return launch_tile_u<KA, 4, false, false, S, KB, true>(job, g, q, sa, sums, 1, s);
          if (g.nt == S && g.u == 2)
            return launch_tile_u<KA, 2, false, false, S, KB, true>(job, g, q, sa, sums, 1, s);
        } else {
          if (g.nt == B && g.u == 4)
            return launch_tile_u<KIND, 4, false, false, B, -1, true>(job, g, q, sa, sums, 1, s);
          if (g.nt == B && g.u == 2)
            return launch_tile_u<KIND, 2, false, false, B, -1, true>(job, g, q, sa, sums, 1, s);
          if (g.nt == S && g.u == 7)
            return launch_tile_u<KIND, 7, false, false, S, -1, true>(job, g, q, sa, sums, 1, s);
          if (g.nt == S && g.u == 4)
            return launch_tile_u<KIND, 4, false, false, S, -1, true>(job, g, q, sa, sums, 1, s);
          if (g.nt == S && g.u == 2)
            return launch_tile_u<KIND, 2, false, false, S, -1, true>(job, g, q, sa, sums, 1, s);
        }
      }
      return fail(kErrInvalid, "gemv_multi: no fused-rmsnorm tile geometry");
    });
  }
  for (int i = 1; i < n; i++) PRANA_CHECK(ms[i].cols == ms[0].cols, "gemv_multi: matrices must share cols");
  bool one_kind = true;
  for (int i = 1; i < n; i++) one_kind = one_kind && ms[i].kind == ms[0].kind;
  const std::pair<int, int> pair = one_kind ? std::make_pair(-1, -1) : mixed_pair(ms, n);
  PRANA_CHECK(one_kind || gemv_multi_fusable(ms, n), "gemv_multi: matrices must share a kind or form a fusable pair");
  const int k0 = ms[0].kind;
  if (one_kind && n > 1 && (k0 == kKindQ8F || k0 == kKindQ8_0 || k0 == kKindQ4_0) && n_tok > kDecodeMaxTokens &&
      !gemv_skinny(k0, n_tok)) {  // one matrix-core launch over all the matrices' row tiles
    switch (k0) {
      case kKindQ8F: return launch_gemm_mfma<kKindQ8F>(ms, os, n, q, sa, n_tok, s);
      case kKindQ8_0: return launch_gemm_mfma<kKindQ8_0>(ms, os, n, q, sa, n_tok, s);
      default: return launch_gemm_mfma<kKindQ4_0>(ms, os, n, q, sa, n_tok, s);
    }
  }
  bool per_matrix = ms[0].kind == kKindF32 || n_tok > kDecodeMaxTokens;
  bool skinny_all = one_kind, skinny_any = false;
  for (int i = 0; i < n; i++) {
    const bool sk = gemv_batch_skinny(ms[i], n_tok);
    skinny_any = skinny_any || sk;
    skinny_all = skinny_all && sk && ms[i].cols == ms[0].cols;
  }
  if (skinny_all && n_tok <= kDecodeMaxTokens)  // the matrices' row tiles in one skinny launch
    return launch_gemm_skinny_any(ms, os, n, q, sa, sums, n_tok, s);
  per_matrix = per_matrix || skinny_any;
  if (per_matrix) {
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
  // (a batch's tokens go to positions pos..pos+n_tok-1, given on the host)
  if (rk && n == 3 && (n_tok == 1 || (!rk->pos_dev && (rk->kcap == 0 || rk->pos + n_tok <= (size_t)rk->kcap))) &&
      ms[1].rows == ms[2].rows && rk->hd > 0 && rk->hd % 2 == 0 && ms[0].rows % rk->hd == 0 &&
      ms[1].rows % rk->hd == 0 && (rk->kcap == 0 || ms[1].rows % 8 == 0) && !os[0].residual && !os[1].residual && !os[2].residual) {
    // the tile must hold whole rotation pairs: even row counts (adjacent
    // pairs) or whole heads (NeoX pairs), in a single stage
    // (batches that launch_decode_t gives the chunk-major kernel keep it and
    // the separate RoPE launch)
    const bool ok = dispatch_kind(ms[0].kind, [&](auto k) {
      constexpr int KIND = decltype(k)::value;
      const TileGeom g = choose_geom<KIND>(ms[0].cols, false);
      const int nb = static_cast<int>(ms[0].cols / RegUnit<KIND>::kElems);
      const bool km = RegUnit<KIND>::kElems == 32 && n_tok >= 2 &&
                      (nb > 128 || n_tok > static_cast<size_t>(kDecMaxTok));
      return static_cast<int>(!km && g.sb >= nb && (rk->neox ? g.rt % rk->hd == 0 : g.rt % 2 == 0));
    });
    if (ok) {
      job.rk = *rk;
      if (fused) *fused = true;
    }
  }
  if (!one_kind) {
    if (pair.first == kKindQ4_0) return launch_decode_mixed<kKindQ4_0, kKindQ8_0>(job, q, sa, sums, n_tok, s);
    return launch_decode_mixed<kKindQ4_K, kKindQ6_K>(job, q, sa, sums, n_tok, s);
  }
  return dispatch_kind(ms[0].kind, [&](auto k) { return launch_decode_t<decltype(k)::value>(job, q, sa, sums, n_tok, s); });
}

bool gemv_multi_fusable(const DevMat* ms, int n) {
  if (n < 2 || n > 3) return n == 1;
  for (int i = 1; i < n; i++)
    if (ms[i].cols != ms[0].cols) return false;
  bool one_kind = true;
  for (int i = 1; i < n; i++) one_kind = one_kind && ms[i].kind == ms[0].kind;
  if (one_kind) return true;
  const std::pair<int, int> p = mixed_pair(ms, n);
  if (p.first < 0) return false;
  // the two formats must give the same tile geometry
  auto geom = [&](int kind) {
    return dispatch_kind(kind, [&](auto k) {
      const TileGeom g = choose_geom<decltype(k)::value>(ms[0].cols, false);
      return g.u * 1000000 + g.rt * 1000 + g.sb;
    });
  };
  return geom(p.first) == geom(p.second);
}

bool gemv_norm_act_fusable(const DevMat& gate, const DevMat& up) {
  if (gate.kind != up.kind || gate.rows != up.rows || gate.cols != up.cols) return false;
  const size_t K = gate.cols;
  if (K <= 512 || K > static_cast<size_t>(kNormMaxK) || K % 32 != 0) return false;
  if (gate.kind != kKindQ8F && gate.kind != kKindQ8_0 && gate.kind != kKindQ4_0) return false;
  int rt = 0;
  dispatch_kind(gate.kind, [&](auto k) {
    rt = norm_act_geom<decltype(k)::value>(K).rt;
    return 0;
  });
  const int cus = device_cus();
  return rt > 0 && gate.rows % rt == 0 && cus > 0 && gate.rows / rt <= static_cast<size_t>(cus);
}

int launch_gemv_act(const DevMat& gate, const DevMat& up, int act, const int8_t* q, const float* sa, const int* sums,
                    size_t n_tok, float* h, int8_t* hq, float* hsa, int* hsum, hipStream_t s, const NormIn* norm) {
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
  if (norm) {
    PRANA_CHECK(n_tok == 1 && norm->x && norm->w && gemv_norm_act_fusable(gate, up),
                "gemv_act: these matrices cannot take a fused rmsnorm");
    job.nin = *norm;
    return dispatch_kind(gate.kind, [&](auto k) {
      constexpr int KIND = decltype(k)::value;
      if constexpr (RegUnit<KIND>::kElems == 32) {
        // (the split launch needs the handoff words for its norm workgroup)
        const TileGeom gs = norm->xch ? norm_split_act_geom<KIND>(gate.cols) : TileGeom{0, 0, 0, 0};
        if constexpr (KIND == kKindQ4_0)
          if (gs.u == kSplitUAct)
            return launch_tile_u<KIND, kSplitUAct, true, true, kNormNT, -1, true, true>(job, gs, q, sa, sums, 1, s);
        const TileGeom g = norm_act_geom<KIND>(gate.cols);
        if (g.nt == kNormNT) return launch_tile_u<KIND, 4, true, true, kNormNT, -1, true>(job, g, q, sa, sums, 1, s);
        if (g.u == 14) return launch_tile_u<KIND, 14, true, false, kNormNTSmall, -1, true>(job, g, q, sa, sums, 1, s);
        if (g.u == 16) return launch_tile_u<KIND, 16, true, false, kNormNTSmall, -1, true>(job, g, q, sa, sums, 1, s);
      }
      return fail(kErrInvalid, "gemv_act: no fused-rmsnorm tile geometry");
    });
  }
  bool in_kernel = false;
  int rc = dispatch_kind(gate.kind, [&](auto k) {
    constexpr int KIND = decltype(k)::value;
    in_kernel = choose_geom<KIND>(gate.cols, true).rt % 32 == 0;
    if (!in_kernel && h == nullptr) return fail(kErrInvalid, "gemv_act: this shape needs the f32 h output");
    return launch_decode_t<KIND>(job, q, sa, sums, n_tok, s);
  });
  if (rc || in_kernel) return rc;
  return launch_quantize_acts(h, n_tok, gate.rows, hq, hsa, hsum, s);  // matmul.rs:105-127 on h
}

bool gemm_act_fusable(const DevMat& gate, const DevMat& up, size_t n_tok) {
  const int k = gate.kind;
  return (k == kKindQ8F || k == kKindQ8_0 || k == kKindQ4_0) && up.kind == k && gate.rows == up.rows &&
         gate.cols == up.cols && gate.rows % 64 == 0 && gate.cols % 32 == 0 && n_tok > kGemvSkinnyMaxTokens;
}

int launch_gemm_act(const DevMat& gate, const DevMat& up, const int8_t* q, const float* sa, size_t n_tok, int gelu,
                    float* h, int8_t* hq, float* hsa, int* hsum, hipStream_t s) {
  PRANA_CHECK(gemm_act_fusable(gate, up, n_tok), "gemm act: these matrices and batch do not take the fused launch");
  switch (gate.kind) {
    case kKindQ8F: return launch_gemm_mfma_act<kKindQ8F>(gate, up, q, sa, n_tok, gelu, h, hq, hsa, hsum, s);
    case kKindQ8_0: return launch_gemm_mfma_act<kKindQ8_0>(gate, up, q, sa, n_tok, gelu, h, hq, hsa, hsum, s);
    default: return launch_gemm_mfma_act<kKindQ4_0>(gate, up, q, sa, n_tok, gelu, h, hq, hsa, hsum, s);
  }
}

// Batches of block-32 kinds on the skinny matrix-core kernel: from 9 tokens
// always, from 3 tokens for matrices of at least kSkinnyMinBlocks blocks.
// Its cost hardly grows with the batch up to 16 tokens (one 16-token tile),
// while the decode tiles and the chunk-major verify kernel pay per token:
// on the 7B Q4_0 shapes at 5 tokens, down 17.7 against 33.8 us, the head
// 26.3 against 39.6 us, gate|up in one launch 25.7 against 40.1 us; at 9
// tokens wo 6.6 against 14.6 us; at 2 tokens and for Q|K|V or wo up to 8
// tokens the decode tiles stay ahead.
constexpr size_t kSkinnyMinBlocks = 1536 * 1024;
bool gemv_batch_skinny(const DevMat& m, size_t n_tok) {
  if (m.kind != kKindQ8F && m.kind != kKindQ8_0 && m.kind != kKindQ4_0) return false;
  if (n_tok >= kGemvSkinnyMinTokens && n_tok <= kGemvSkinnyMaxTokens) return true;
  return n_tok >= 3 && n_tok < kGemvSkinnyMinTokens && m.rows * (m.cols / 32) >= kSkinnyMinBlocks;
}

// A single matrix of 512K+ blocks below 8192 rows (the block-split form of
// the skinny kernel) also takes it at 3..8 tokens: the 7B wo at 5 tokens 6.7
// against 7.7 us on the decode tiles. (Q|K|V, a multi-matrix launch with its
// RoPE epilogue, stays on the tiles: as one matrix its 6144 rows took 12.6
// against 9.7 us.)
bool gemv_verify_block_split(const DevMat& m, size_t n_tok) {
  return (m.kind == kKindQ8F || m.kind == kKindQ8_0 || m.kind == kKindQ4_0) && n_tok >= 3 && n_tok <= 8 &&
         m.rows < 8192 && m.rows * (m.cols / 32) >= 512 * 1024;
}

int launch_gemv(const DevMat& m, const float* x, const int8_t* q, const float* sa, const int* sums, size_t n_tok,
                const GemvOut& o, hipStream_t s) {
  if (n_tok == 0 || m.rows == 0) return kOk;
  if (gemv_batch_skinny(m, n_tok) || gemv_verify_block_split(m, n_tok)) {
    switch (m.kind) {
      case kKindQ8F: return launch_gemm_skinny<kKindQ8F>(&m, &o, 1, q, sa, sums, n_tok, s);
      case kKindQ8_0: return launch_gemm_skinny<kKindQ8_0>(&m, &o, 1, q, sa, sums, n_tok, s);
      case kKindQ4_0: return launch_gemm_skinny<kKindQ4_0>(&m, &o, 1, q, sa, sums, n_tok, s);
    }
  }
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
    case kKindQ8F: return launch_gemm_mfma<kKindQ8F>(&m, &o, 1, q, sa, n_tok, s);
    case kKindQ8_0: return launch_gemm_mfma<kKindQ8_0>(&m, &o, 1, q, sa, n_tok, s);
    case kKindQ4_0: return launch_gemm_mfma<kKindQ4_0>(&m, &o, 1, q, sa, n_tok, s);
    case kKindQ4_K: return launch_gemm_kq<kKindQ4_K>(m, q, sa, sums, n_tok, o, s);
    case kKindQ6_K: return launch_gemm_kq<kKindQ6_K>(m, q, sa, sums, n_tok, o, s);
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
