// Bit-exact parallel evaluation of the sequential f32 fold
//   s = (((-0.0 + a0) + a1) + ...) + a_{n-1}        (round-to-nearest-even)
// for non-negative terms, the sums behind rmsnorm (norms.rs:15) and softmax
// (norms.rs:53), which the reference evaluates strictly left to right.
//
// While the running sum s stays inside one binade [2^e, 2^(e+1)) (e >= -126),
// every partial sum is an integer multiple m of the grid u = 2^(e-23) and one
// step is m' = rne(m + a/u). For a/u = I + f the increment is I (f < 1/2),
// I+1 (f > 1/2), or on a tie the choice that makes m' even — which depends
// only on the parity of m and always leaves m' even. So each term is a pair of
// increments (for even / odd incoming m); pairs compose associatively, and a
// block scan gives every partial sum of the binade exactly. The first step
// whose exact result reaches 2^24 ulps leaves the binade: that one step is
// evaluated with an ordinary f32 add and the scan restarts in the new binade.
// Non-finite terms fall back to a single-lane loop.
#pragma once

#include <cstdint>

namespace prana {
namespace exact {

constexpr int32_t kCap = 1 << 28;  // saturation: anything >= 2^24 crosses

struct Pair {
  int32_t e, o;  // increment of m when the incoming m is even / odd
};

__host__ __device__ inline int32_t sat_add(int32_t a, int32_t b) {
  int64_t s = static_cast<int64_t>(a) + b;
  return s > kCap ? kCap : static_cast<int32_t>(s);
}

// f then g.
__host__ __device__ inline Pair compose(Pair f, Pair g) {
  Pair r;
  r.e = sat_add(f.e, (f.e & 1) ? g.o : g.e);
  r.o = sat_add(f.o, ((f.o + 1) & 1) ? g.o : g.e);
  return r;
}

// Increment pair of term a (>= 0, finite) on the grid 2^(e-23).
__host__ __device__ inline Pair term_pair_scaled(float a, double scale) {
  double A = static_cast<double>(a) * scale;  // exact: scale is a power of two
  if (A >= static_cast<double>(kCap)) return Pair{kCap, kCap};
  double I = floor(A);
  double f = A - I;
  int32_t i = static_cast<int32_t>(I);
  if (f < 0.5) return Pair{i, i};
  if (f > 0.5) return Pair{i + 1, i + 1};
  return Pair{i + (i & 1), i + 1 - (i & 1)};
}

__host__ __device__ inline Pair term_pair(float a, int e) {
  double A = static_cast<double>(a) * ldexp(1.0, 23 - e);  // exact
  if (A >= static_cast<double>(kCap)) return Pair{kCap, kCap};
  double I = floor(A);
  double f = A - I;
  int32_t i = static_cast<int32_t>(I);
  if (f < 0.5) return Pair{i, i};
  if (f > 0.5) return Pair{i + 1, i + 1};
  return Pair{i + (i & 1), i + 1 - (i & 1)};
}

__host__ __device__ inline int32_t apply(Pair p, int32_t m) { return sat_add(m, (m & 1) ? p.o : p.e); }

// Binade exponent of s >= 0 (s < 2^-125 uses the subnormal grid 2^-149).
__host__ __device__ inline int binade(float s) {
  int e;
  (void)frexpf(s, &e);  // s = f * 2^e, f in [0.5, 1)
  e -= 1;
  return s < 0x1p-125f ? -126 : e;
}

// Workgroup-wide exclusive scan of Pair over a 256-lane block (4 waves).
// s_wave: LDS scratch of 8 ints. Returns the exclusive prefix; *total gets the
// block-wide composition (valid in every lane).
__device__ inline Pair block_exclusive_scan(Pair v, int* s_wave, Pair* total) {
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
  for (int w = 0; w < 4; w++) {
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

// The sequential fold of a[0..n), a[i] >= +0, evaluated by a 256-lane
// workgroup; every lane returns the same value. Must be called by all lanes.
// a may live in LDS or global memory (read-only here).
__device__ inline float block_seq_sum_nonneg(const float* a, int n) {
  __shared__ int s_wave[8];
  __shared__ float s_sum;
  __shared__ int s_k, s_first;
  __shared__ int32_t s_mprev;
  const int tid = threadIdx.x;
  if (n <= 0) return -0.0f;
  bool bad = false;
  for (int i = tid; i < n; i += 256) bad |= !(a[i] <= 3.4028234663852886e38f);  // NaN or inf
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
    float s = -0.0f;
    int k = 0;
    for (; k < n && k < kHead; k++) s += a[k];
    s_sum = s;
    s_k = k;
  }
  __syncthreads();
  while (true) {
    const int k = s_k;
    const float s = s_sum;
    if (k >= n) return s;
    const int e = binade(s);
    const float u = ldexpf(1.0f, e - 23);
    const double scale = ldexp(1.0, 23 - e);
    const int32_t m = static_cast<int32_t>(s * ldexpf(1.0f, 23 - e));
    const int R = n - k, C = (R + 255) / 256;
    const int j0 = k + tid * C, j1 = min(n, j0 + C);
    Pair loc{0, 0};
    for (int j = j0; j < j1; j++) loc = compose(loc, term_pair_scaled(a[j], scale));
    if (tid == 0) s_first = n;
    Pair total;
    Pair pre = block_exclusive_scan(loc, s_wave, &total);  // contains a barrier
    int32_t mm = apply(pre, m);
    int first = n;
    int32_t mprev = 0;
    for (int j = j0; j < j1; j++) {
      int32_t m2 = apply(term_pair_scaled(a[j], scale), mm);
      if (m2 >= (1 << 24)) {
        first = j;
        mprev = mm;
        break;
      }
      mm = m2;
    }
    if (first < n) atomicMin(&s_first, first);
    __syncthreads();
    const int f = s_first;
    if (f < n && first == f) {  // the owner of the crossing step
      s_sum = static_cast<float>(mprev) * u + a[f];
      s_k = f + 1;
    } else if (f == n && tid == 0) {
      s_sum = static_cast<float>(apply(total, m)) * u;
      s_k = n;
    }
    __syncthreads();
  }
}

}  // namespace exact
}  // namespace prana
