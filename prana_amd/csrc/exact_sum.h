// Bit-exact parallel evaluation of the sequential f32 fold
//   s = (((-0.0 + a0) + a1) + ...) + a_{n-1}        (round-to-nearest-even)
// for non-negative terms, the sums behind rmsnorm (norms.rs:15) and softmax
// (norms.rs:53), which the reference evaluates strictly left to right.
//
// While the running sum s stays inside one binade [2^e, 2^(e+1)) (e >= -126;
// e = -126 also covers the subnormals), every partial sum is an integer
// multiple m of the grid u = 2^(e-23) and one step is m' = rne(m + a/u). For
// a/u = I + f the increment is I (f < 1/2), I+1 (f > 1/2), or on a tie the
// choice that makes m' even — which depends only on the parity of m. So each
// term is a pair of increments (for even / odd incoming m); pairs compose
// associatively, and a workgroup scan gives every partial sum of the binade
// exactly. The first step whose exact result reaches 2^24 ulps leaves the
// binade: that one step is evaluated with an ordinary f32 add and the scan
// restarts in the new binade. A sum of n comparable terms crosses about
// log2(n) binades, so the whole fold costs a few dozen workgroup steps
// instead of n dependent adds (used for long sums; short ones are cheaper as
// one lane's chain). Non-finite terms fall back to a single-lane loop; a sum
// that overflows to +inf stays +inf.
//
// Terms are decoded from their bits with integer arithmetic only. The sign
// bit is ignored (the callers' terms are squares and exponentials, never
// -0.0).
#pragma once

#include <cstdint>

namespace prana {
namespace exact {

constexpr int32_t kCap = 1 << 28;  // saturation: anything >= 2^24 crosses

struct Pair {
  int32_t e, o;  // increment of m when the incoming m is even / odd
};

__host__ __device__ inline int32_t sat_add(int32_t a, int32_t b) {
  int32_t s = a + b;  // a, b <= 2^28: no overflow
  return s > kCap ? kCap : s;
}

// f then g.
__host__ __device__ inline Pair compose(Pair f, Pair g) {
  Pair r;
  r.e = sat_add(f.e, (f.e & 1) ? g.o : g.e);
  r.o = sat_add(f.o, ((f.o + 1) & 1) ? g.o : g.e);
  return r;
}

__host__ __device__ inline int32_t apply(Pair p, int32_t m) { return sat_add(m, (m & 1) ? p.o : p.e); }

// Increment pair of the term with bit pattern `bits` (finite) on the grid
// 2^(e-23), e >= -126.
__host__ __device__ inline Pair term_pair_bits(uint32_t bits, int e) {
  const uint32_t b = bits & 0x7fffffffu;
  const int E = static_cast<int>(b >> 23);
  const uint32_t M = E ? ((b & 0x7fffffu) | 0x800000u) : (b & 0x7fffffu);
  // term = M * 2^(Eeff-150); a/u = M * 2^(Eeff-127-e); right shift by sh
  const int sh = 127 + e - (E ? E : 1);
  if (sh <= 0) {
    if (sh <= -5) return Pair{kCap, kCap};
    uint32_t A = M << (-sh);
    int32_t i = A >= static_cast<uint32_t>(kCap) ? kCap : static_cast<int32_t>(A);
    return Pair{i, i};
  }
  if (sh >= 25) return Pair{0, 0};  // M < 2^24 <= half an ulp
  const int32_t I = static_cast<int32_t>(M >> sh);
  const uint32_t r = M & ((1u << sh) - 1u), half = 1u << (sh - 1);
  if (r < half) return Pair{I, I};
  if (r > half) return Pair{I + 1, I + 1};
  return Pair{I + (I & 1), I + 1 - (I & 1)};
}

// Same, from the value (host checks).
__host__ __device__ inline Pair term_pair(float a, int e) {
  union {
    float f;
    uint32_t u;
  } c{a};
  return term_pair_bits(c.u, e);
}

// Binade of finite s >= 0: exponent e (>= -126) and s = m * 2^(e-23).
__host__ __device__ inline void decompose(float s, int* e, int32_t* m) {
  union {
    float f;
    uint32_t u;
  } c{s};
  const uint32_t b = c.u & 0x7fffffffu;
  const int E = static_cast<int>(b >> 23);
  *e = E ? E - 127 : -126;
  if (*e < -126) *e = -126;
  *m = static_cast<int32_t>(E ? ((b & 0x7fffffu) | 0x800000u) : (b & 0x7fffffu));
}

__host__ __device__ inline int binade(float s) {
  int e;
  int32_t m;
  decompose(s, &e, &m);
  return e;
}

#if defined(__HIPCC__)
// Workgroup-wide exclusive scan of Pair over NT lanes (NT/64 waves).
// s_wave: LDS scratch of 2*NT/64 ints. *total gets the workgroup-wide
// composition (valid in every lane). Contains one barrier.
template <int NT>
__device__ inline Pair block_exclusive_scan(Pair v, int* s_wave, Pair* total) {
  constexpr int W = NT / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  Pair inc = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    Pair o;
    o.e = __shfl_up(inc.e, d, 64);
    o.o = __shfl_up(inc.o, d, 64);
    if (lane >= d) inc = compose(o, inc);
  }
  if (lane == 63) {
    s_wave[2 * wave] = inc.e;
    s_wave[2 * wave + 1] = inc.o;
  }
  __syncthreads();
  Pair pre{0, 0}, all{0, 0};
#pragma unroll
  for (int w = 0; w < W; w++) {
    Pair wt{s_wave[2 * w], s_wave[2 * w + 1]};
    if (w < wave) pre = compose(pre, wt);
    all = compose(all, wt);
  }
  Pair ex_lane;
  ex_lane.e = __shfl_up(inc.e, 1, 64);
  ex_lane.o = __shfl_up(inc.o, 1, 64);
  if (lane == 0) ex_lane = Pair{0, 0};
  *total = all;
  return compose(pre, ex_lane);
}

// The same fold by one lane over an LDS buffer that is 16-byte aligned and
// zero-filled from n up to lane_pad(n) terms (a multiple of 64, plus one
// 32-term batch that is fetched ahead but never added). Batches of 32 terms
// are fetched with 16-byte loads one batch ahead of the dependent adds (two
// register sets, straight-line loop body), so the chain runs at the add
// latency. Terms are >= +0 and n >= 1, so the zero padding leaves the sum
// unchanged.
__host__ __device__ constexpr int lane_pad(int n) { return (n + 63) / 64 * 64 + 32; }

__device__ __forceinline__ float lane_seq_sum_padded(const float* a, int n) {
  const float4* p = reinterpret_cast<const float4*>(a);
  const int nb = (n + 63) / 64 * 2;  // even number of 32-term batches
  float s = -0.0f;
  float4 x[8], y[8];
#pragma unroll
  for (int j = 0; j < 8; j++) x[j] = p[j];
  for (int b = 0; b < nb; b += 2) {
    const float4* q = p + 8 * b;
#pragma unroll
    for (int j = 0; j < 8; j++) y[j] = q[8 + j];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      s += x[j].x;
      s += x[j].y;
      s += x[j].z;
      s += x[j].w;
    }
#pragma unroll
    for (int j = 0; j < 8; j++) x[j] = q[16 + j];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      s += y[j].x;
      s += y[j].y;
      s += y[j].z;
      s += y[j].w;
    }
  }
  return s;
}

// Up to this length a padded sum is one lane's chain (about five cycles per
// term); longer sums use the binade scan, whose steps cost a few thousand
// cycles each but whose step count grows only with log2(n).
constexpr int kSerialMax = 8192;

// The sequential fold of a[0..n), a[i] >= 0, evaluated by an NT-lane
// workgroup (blockDim.x == NT); every lane returns the same value. Must be
// called by all lanes. a may live in LDS or global memory (read-only here,
// visible to the whole workgroup). PADDED: a is an LDS buffer, 16-byte
// aligned and zero-filled up to lane_pad(n) terms; sums of up to kSerialMax
// terms are then folded by one lane. Other sums use the binade scan,
// holding up to NT*CMAX terms in
// registers (thread t owns the contiguous run [t*C, t*C + C),
// C = ceil(n/NT)) and streaming longer sums from `a`. Sums with non-finite
// terms run on one lane.
template <int NT, bool PADDED, int CMAX = 16>
__device__ __forceinline__ float block_seq_sum_nonneg(const float* a, int n) {
  static_assert(NT % 64 == 0 && NT <= 1024, "whole waves");
  __shared__ int s_wave[2 * (NT / 64)];
  __shared__ float s_sum;
  __shared__ int s_k, s_first;
  const int tid = threadIdx.x;
  if (n <= 0) return -0.0f;
  if (PADDED && n <= kSerialMax) {
    bool bad = false;
    for (int j = tid; j < n; j += NT) bad |= !(a[j] <= 3.4028234663852886e38f);
    if (__syncthreads_or(bad)) {
      if (tid == 0) {
        float s = -0.0f;
        for (int i = 0; i < n; i++) s += a[i];
        s_sum = s;
      }
      __syncthreads();
      return s_sum;
    }
    if (tid == 0) s_sum = lane_seq_sum_padded(a, n);
    __syncthreads();
    return s_sum;
  }

  const bool in_regs = n <= NT * CMAX;
  const int C = (n + NT - 1) / NT;
  const int j0 = tid * C, j1 = min(n, j0 + C);
  uint32_t v[CMAX];
  bool bad = false;
  if (in_regs) {
#pragma unroll
    for (int i = 0; i < CMAX; i++) {
      const float x = (i < C && j0 + i < n) ? a[j0 + i] : 0.0f;
      bad |= !(x <= 3.4028234663852886e38f);  // NaN or +inf
      v[i] = __float_as_uint(x);
    }
  } else {
    for (int j = j0; j < j1; j++) bad |= !(a[j] <= 3.4028234663852886e38f);
  }
  if (__syncthreads_or(bad)) {
    if (tid == 0) {
      float s = -0.0f;
      for (int i = 0; i < n; i++) s += a[i];
      s_sum = s;
    }
    __syncthreads();
    return s_sum;
  }
  constexpr int kHead = 32;  // the fast-growing prefix is cheaper serially
  if (tid == 0) {
    float h[kHead];
#pragma unroll
    for (int i = 0; i < kHead; i++) h[i] = i < n ? a[i] : 0.0f;
    float s = -0.0f;
#pragma unroll
    for (int i = 0; i < kHead; i++)
      if (i < n) s += h[i];
    s_sum = s;
    s_k = min(n, kHead);
  }
  __syncthreads();
  while (true) {
    const int k = s_k;
    const float s = s_sum;
    if (k >= n || !(s <= 3.4028234663852886e38f)) return s;  // done, or overflowed to +inf
    int e;
    int32_t m;
    decompose(s, &e, &m);
    const float u = ldexpf(1.0f, e - 23);
    // local composition of this thread's terms at indices >= k
    Pair loc{0, 0};
    if (in_regs) {
#pragma unroll
      for (int i = 0; i < CMAX; i++)
        if (i < C && j0 + i >= k && j0 + i < n) loc = compose(loc, term_pair_bits(v[i], e));
    } else {
      for (int j = max(j0, k); j < j1; j++) loc = compose(loc, term_pair_bits(__float_as_uint(a[j]), e));
    }
    if (tid == 0) s_first = n;
    Pair total;
    const Pair pre = block_exclusive_scan<NT>(loc, s_wave, &total);  // barrier
    // walk this run from its prefix to find the first step leaving the binade
    int32_t mm = apply(pre, m);
    int first = n;
    int32_t mprev = 0;
    float fval = 0.0f;
    if (in_regs) {
#pragma unroll
      for (int i = 0; i < CMAX; i++) {
        if (first == n && i < C && j0 + i >= k && j0 + i < n) {
          const int32_t m2 = apply(term_pair_bits(v[i], e), mm);
          if (m2 >= (1 << 24)) {
            first = j0 + i;
            mprev = mm;
            fval = __uint_as_float(v[i]);
          }
          mm = m2;
        }
      }
    } else {
      for (int j = max(j0, k); j < j1; j++) {
        const float x = a[j];
        const int32_t m2 = apply(term_pair_bits(__float_as_uint(x), e), mm);
        if (m2 >= (1 << 24)) {
          first = j;
          mprev = mm;
          fval = x;
          break;
        }
        mm = m2;
      }
    }
    if (first < n) atomicMin(&s_first, first);
    __syncthreads();
    const int f = s_first;
    if (f < n && first == f) {  // the owner of the crossing step
      s_sum = static_cast<float>(mprev) * u + fval;
      s_k = f + 1;
    } else if (f == n && tid == 0) {
      s_sum = static_cast<float>(apply(total, m)) * u;
      s_k = n;
    }
    __syncthreads();
  }
}
#endif

}  // namespace exact
}  // namespace prana
