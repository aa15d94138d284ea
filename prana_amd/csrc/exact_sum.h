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
// exactly. A step that leaves the binade is evaluated with an ordinary f32
// add. Two drivers place those steps: the predicted-binade scan guesses all
// of them at once from approximate prefix sums and verifies the guess while
// it walks the segments (one workgroup scan in total), and the adaptive scan
// finds them one at a time (one workgroup scan per binade, for sums too long
// for the first). Either replaces n dependent adds, each costing several
// cycles of latency. Non-finite terms fall back to a single-lane loop; a sum
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

// ---- predicted binades: one scan for the whole sum
// The binade of every partial sum is predicted from approximate prefix sums
// (ordinary f32 adds in any order, only used to choose grids). A step whose
// predicted result binade differs from the predicted binade of its input is a
// crossing; the steps between two crossings form a segment that stays on one
// grid, so a single segmented workgroup scan of increment pairs gives every
// segment's composed map. One lane then walks the K+1 segments: each crossing
// step is an ordinary f32 add of the exact value before it, and each segment
// applies its map to the exact value at its start. The walk also verifies the
// prediction, which makes the result exact whenever it reports success:
//   - a segment's start value must lie in the binade whose grid its pairs use;
//   - its end value must still lie in that binade (< 2^24 grid units).
// Increments are non-negative, so the sum never leaves a binade in the middle
// of a segment without the end check seeing it, and inside the binade every
// step's grid rounding is the f32 rounding. When a check fails (or there are
// more than kPredMaxCross crossings) the caller folds serially instead.
// The exact partial sums drift from the approximate ones by their rounding
// errors (random-walk-like, ~sqrt(n) units at most in practice). A step whose
// approximate result lies within pred_margin(n) units of a binade boundary is
// "ambiguous": it is made a crossing (a plain add in the walk) and so is the
// step after it, so no segment starts or ends on a guessed binade. Such
// crossings carry the binade code kPredAmb; the walk skips the (empty)
// segment that follows them.
constexpr int kPredHead = 32;       // folded serially first (the sum grows fastest here)
constexpr int kPredAmb = 1000;      // binade code of an ambiguous step
constexpr int kPredMaxCross = 63;   // crossings the walk accepts (one per lane of a wave)
constexpr int kPredMaxPerLane = 64; // terms per lane of the predicted scan

struct SegAcc {
  Pair p;  // composed increments since the last crossing
  int c;   // crossings so far (a crossing resets p to the identity)
};

__host__ __device__ inline SegAcc seg_combine(SegAcc a, SegAcc b) {
  return SegAcc{b.c > 0 ? b.p : compose(a.p, b.p), a.c + b.c};
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
    __builtin_amdgcn_sched_barrier(0);  // keep the next batch's loads ahead of these adds
#pragma unroll
    for (int j = 0; j < 8; j++) {
      s += x[j].x;
      s += x[j].y;
      s += x[j].z;
      s += x[j].w;
    }
#pragma unroll
    for (int j = 0; j < 8; j++) x[j] = q[16 + j];
    __builtin_amdgcn_sched_barrier(0);
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

// LDS index of term i for buffers read as per-lane runs: one spare word per
// 16 terms staggers the runs of neighbouring lanes across banks (a run length
// of C words would otherwise put lanes C apart on the same bank). A buffer of
// n terms needs run_pad(n - 1) + 1 words.
__host__ __device__ constexpr int run_pad(int i) { return i + (i >> 4); }

// Visit term(i0 + j), j = 0..nv-1, in order: f(j, value), in blocks of four
// whose fetches are issued one block ahead. The last block is padded with
// zero terms, which leave every pass below unchanged, so the body needs no
// guards; fetches stay inside term(0..n).
template <class Term, class F>
__device__ __forceinline__ void for_each_run(Term a, int i0, int nv, int n, F&& f) {
  if (nv <= 0) return;
  float t[4], u[4];
#pragma unroll
  for (int k = 0; k < 4; k++) t[k] = a(min(i0 + k, n - 1));
  for (int jb = 0; jb < nv; jb += 4) {
#pragma unroll
    for (int k = 0; k < 4; k++) u[k] = a(min(i0 + jb + 4 + k, n - 1));
#pragma unroll
    for (int k = 0; k < 4; k++) f(jb + k, jb + k < nv ? t[k] : 0.0f);
#pragma unroll
    for (int k = 0; k < 4; k++) t[k] = u[k];
  }
}

// Binade of a finite p >= 0 (the exponent field, subnormals and zero -> -126).
__device__ __forceinline__ int binade_fast(float p) {
  const int E = static_cast<int>((__float_as_uint(p) >> 23) & 0xffu);
  return (E > 1 ? E : 1) - 127;
}

// Margin, in units of the last place, around binade boundaries inside which
// an approximate partial sum of an n-term fold does not decide the binade.
__host__ __device__ inline int pred_margin(int n) { return 8 * static_cast<int>(sqrtf(static_cast<float>(n))) + 16; }

// The binade code of an approximate partial sum p >= 0: its binade, or
// kPredAmb when p > 0 lies within r units of either boundary of its binade.
// (Bitwise logic throughout: short-circuit forms compile to a branch per
// call, and these run once per term.)
__device__ __forceinline__ int binade_code(float p, int r) {
  const uint32_t u = __float_as_uint(p);
  const uint32_t f = u & 0x7fffffu;
  const bool amb = ((u & 0x7fffffffu) != 0) & ((f < static_cast<uint32_t>(r)) | (f > 0x7fffffu - static_cast<uint32_t>(r)));
  return amb ? kPredAmb : binade_fast(p);
}

// A step with binade code ec after a step with code ein starts a new segment.
__device__ __forceinline__ bool seg_break(int ec, int ein) { return (ec != ein) | (ec == kPredAmb); }

// term_pair_bits(bits(t), e) for finite t >= 0, from exact float operations
// (scaling by a power of two, floor and the difference are exact here; a
// scaled value small enough to lose bits is far below one half), without
// branches.
__device__ __forceinline__ Pair term_pair_fast(float t, int e) {
  const float A = ldexpf(t, 23 - e);
  const bool big = !(A < 268435456.0f);  // >= 2^28 (or +inf): leaves the binade
  const float I = floorf(fminf(A, 268435456.0f));
  const float f = A - I;
  const int i = static_cast<int>(I);
  const int v = i + (f > 0.5f ? 1 : 0);
  const bool tie = f == 0.5f;
  const int odd = i & 1;
  return Pair{big ? kCap : (tie ? i + odd : v), big ? kCap : (tie ? i + 1 - odd : v)};
}

// One DPP step of a wave scan (bound_ctrl: lanes without a source read 0,
// the identity of every operator scanned here).
template <int CTRL, int ROWS>
__device__ __forceinline__ int dpp_src(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, ROWS, 0xf, true);
}
// Inclusive wave-wide scan with an associative operator whose identity is
// all-zero bits: shifts of 1, 2, 4, 8 inside 16-lane rows, then the row
// broadcasts of lanes 15 and 31.
template <class T, class Get, class Op>
__device__ __forceinline__ T wave_scan_incl(T x, Get get, Op op) {
  x = op(get([](int v) { return dpp_src<0x111, 0xf>(v); }, x), x);
  x = op(get([](int v) { return dpp_src<0x112, 0xf>(v); }, x), x);
  x = op(get([](int v) { return dpp_src<0x114, 0xf>(v); }, x), x);
  x = op(get([](int v) { return dpp_src<0x118, 0xf>(v); }, x), x);
  x = op(get([](int v) { return dpp_src<0x142, 0xa>(v); }, x), x);
  x = op(get([](int v) { return dpp_src<0x143, 0xc>(v); }, x), x);
  return x;
}
// The same inside each 16-lane row only (enough for the per-wave totals of
// a workgroup of up to 16 waves).
template <class T, class Get, class Op>
__device__ __forceinline__ T row_scan_incl(T x, Get get, Op op) {
  x = op(get([](int v) { return dpp_src<0x111, 0xf>(v); }, x), x);
  x = op(get([](int v) { return dpp_src<0x112, 0xf>(v); }, x), x);
  x = op(get([](int v) { return dpp_src<0x114, 0xf>(v); }, x), x);
  x = op(get([](int v) { return dpp_src<0x118, 0xf>(v); }, x), x);
  return x;
}
// The value of the previous lane (lane 0: all-zero bits).
__device__ __forceinline__ int wave_shr1(int v) { return dpp_src<0x138, 0xf>(v); }

__device__ __forceinline__ float scan_add_f32(float x) {
  return wave_scan_incl(
      x, [](auto mv, float v) { return __int_as_float(mv(__float_as_int(v))); },
      [](float a, float b) { return a + b; });
}
__device__ __forceinline__ SegAcc scan_seg(SegAcc x) {
  return wave_scan_incl(
      x, [](auto mv, SegAcc v) { return SegAcc{Pair{mv(v.p.e), mv(v.p.o)}, mv(v.c)}; },
      [](SegAcc a, SegAcc b) { return seg_combine(a, b); });
}
__device__ __forceinline__ float row_scan_add_f32(float x) {
  return row_scan_incl(
      x, [](auto mv, float v) { return __int_as_float(mv(__float_as_int(v))); },
      [](float a, float b) { return a + b; });
}
__device__ __forceinline__ SegAcc row_scan_seg(SegAcc x) {
  return row_scan_incl(
      x, [](auto mv, SegAcc v) { return SegAcc{Pair{mv(v.p.e), mv(v.p.o)}, mv(v.c)}; },
      [](SegAcc a, SegAcc b) { return seg_combine(a, b); });
}

// Running composition of a lane's steps (a crossing resets it).
__device__ __forceinline__ void seg_push(SegAcc& acc, bool cross, Pair pr) {
  const Pair c = compose(acc.p, pr);
  acc.p.e = cross ? 0 : c.e;
  acc.p.o = cross ? 0 : c.o;
  acc.c += cross ? 1 : 0;
}

// The walk of the predicted-binade scan (one wave): segment j's composed map
// (te, to), the crossing term ct that starts it and the binade code ce of
// that step sit in lane j. From the head's exact value sH it adds each
// crossing as an f32 add and applies each segment's map to the exact value at
// its start, checking that the start lies in the binade the map assumed and
// that the end stays inside it. A value lies in binade E (e >= -126) exactly
// when its count of E's ulps, val * 2^(23-E) (an exact scaling here), is in
// [2^23, 2^24) ([0, 2^24) for E = -126), and that count is the m of
// decompose(); the loop carries no early exit, only the check result (when a
// check fails, the caller folds serially and drops this value).
__device__ __forceinline__ float walk_segments(float sH, int K, int te, int to, float ct, int ce, bool* good_out) {
  bool good = K <= kPredMaxCross;
  const int Kc = min(K, kPredMaxCross);
  float val = sH;
  int E = binade_fast(sH);
  for (int j = 0; j <= Kc; j++) {
    if (j > 0) {
      val = val + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ct), j));
      E = __builtin_amdgcn_readlane(ce, j);
    }
    if (E == kPredAmb) continue;  // an ambiguous crossing: its segment is empty
    const float mf = ldexpf(val, 23 - E);
    good &= (mf < 16777216.0f) & ((E == -126) | (mf >= 8388608.0f));  // false for inf and NaN too
    const int32_t m = static_cast<int32_t>(fminf(mf, 16777216.0f));
    const int32_t me = apply(Pair{__builtin_amdgcn_readlane(te, j), __builtin_amdgcn_readlane(to, j)}, m);
    good &= me < (1 << 24);
    val = ldexpf(static_cast<float>(me), E - 23);
  }
  *good_out = good;
  return val;
}

// Barrier and OR-vote of a lane group (see group_seq_sum_pred): the
// workgroup for NG == 1, else the calling wave.
template <int NG>
__device__ __forceinline__ void group_sync() {
  if constexpr (NG == 1) {
    __syncthreads();
  } else {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}
template <int NG>
__device__ __forceinline__ bool group_or(bool p) {
  if constexpr (NG == 1) {
    return __syncthreads_or(p) != 0;
  } else {
    group_sync<NG>();
    return __builtin_amdgcn_ballot_w64(p) != 0;
  }
}

// The fold of term(0..n) with n > kPredHead and n - kPredHead <= NT *
// kPredMaxPerLane, terms >= 0; term(i) must return the same value in every
// lane and every call (an LDS or global read, or a pure function of one).
// Lane t owns positions [H + t*C, H + t*C + C): for LDS-backed terms, lay
// them out so that runs of C consecutive positions in different lanes fall
// in different banks. Returns the value in every lane and *ok; *ok is false
// (value meaningless) when a term is not finite or the prediction failed.
// Must be called by all NT lanes; contains five group barriers.
// NG lane groups of NT lanes each evaluate their own sum at once (group g is
// lanes [g*NT, g*NT + NT) of the workgroup, with its own LDS records): NG ==
// 1 is the whole workgroup; NG > 1 needs NT == 64, one sum per wave, and
// then the barriers are wave-level (a wave's LDS accesses complete in issue
// order, so compiler fences suffice).
template <int NT, int NG, class Term>
__device__ inline float group_seq_sum_pred(Term a, int n, bool* ok) {
  static_assert(NG == 1 || NT == 64, "groups are the workgroup or single waves");
  constexpr int W = NT / 64;
  static_assert(kPredMaxCross < 64, "the walk keeps one segment per lane of wave 0");
  __shared__ float s_fw_[NG][W];
  __shared__ int s_epl_[NG][W], s_sw_[NG][3 * W];
  __shared__ int s_tot_[NG][2 * (kPredMaxCross + 1)];
  __shared__ float s_ct_[NG][kPredMaxCross + 1];
  __shared__ int s_ce_[NG][kPredMaxCross + 1];
  __shared__ float s_head_[NG], s_res_[NG];
  __shared__ int s_ok_[NG];
  const int g = NG > 1 ? static_cast<int>(threadIdx.x) / NT : 0;
  float* s_fw = s_fw_[g];
  int* s_epl = s_epl_[g];
  int* s_sw = s_sw_[g];
  int* s_tot = s_tot_[g];
  float* s_ct = s_ct_[g];
  int* s_ce = s_ce_[g];
  float& s_head = s_head_[g];
  float& s_res = s_res_[g];
  int& s_ok = s_ok_[g];
  const int tid = NG > 1 ? static_cast<int>(threadIdx.x) % NT : static_cast<int>(threadIdx.x);
  const int lane = tid & 63, wave = tid >> 6;
  const int C = (n - kPredHead + NT - 1) / NT;
  const int i0 = kPredHead + tid * C;
  const int nv = max(0, min(C, n - i0));
  const int R = pred_margin(n);
  bool bad = false;
  if (tid == 0) {
    float h[kPredHead];
#pragma unroll
    for (int i = 0; i < kPredHead; i++) h[i] = a(i);
    float s = -0.0f;
#pragma unroll
    for (int i = 0; i < kPredHead; i++) s += h[i];
    s_head = s;
    bad = !(s <= 3.4028234663852886e38f);  // a head term is NaN or +inf
  }
  // pass 1: approximate prefix sums (any rounding; only the grids depend on
  // them) and the finiteness check
  float ls = 0.0f;
  for_each_run(a, i0, nv, n, [&](int, float x) {
    ls += x;
    bad |= !(x <= 3.4028234663852886e38f);
  });
  const float inc = scan_add_f32(ls);
  if (lane == 63) s_fw[wave] = inc;
  if (group_or<NG>(bad)) {
    *ok = false;
    return 0.0f;
  }
  static_assert(W <= 16, "wave totals are scanned inside one 16-lane row");
  // every wave scans the wave totals in its first row and picks its prefix
  const float tw = row_scan_add_f32(lane < W ? s_fw[lane] : 0.0f);
  const float pre = wave > 0 ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tw), wave - 1)) : 0.0f;
  const float sH = s_head;
  const float P0 = sH + (pre + __int_as_float(wave_shr1(__float_as_int(inc))));
  // pass 2: the predicted result binade of every owned step (P is recomputed
  // identically in the fallback pass), the composition of steps 1..nv-1
  // (their crossing flags are local; step 0's needs the previous lane's
  // binade), and the first two local crossings: position, term, binade and
  // the composition since the previous crossing (or since step 1).
  int ep_first = 0, ep_last = 0, ncross = 0, e1 = 0, e2 = 0;
  float x0 = 0.0f, x1 = 0.0f, x2 = 0.0f;
  SegAcc rest{Pair{0, 0}, 0};
  Pair pre1{0, 0}, pre2{0, 0};
  {
    // Blocks of four steps. The common block has no crossing and no tie:
    // four symmetric increments, added at once (the increments are >= 0, so
    // one saturating add equals four). Other blocks take the steps one by one.
    float P = P0;
    int elast = 0;
    float t[4], u[4];
#pragma unroll
    for (int k = 0; k < 4; k++) t[k] = a(min(i0 + k, n - 1));
    for (int jb = 0; jb < nv; jb += 4) {
#pragma unroll
      for (int k = 0; k < 4; k++) u[k] = a(min(i0 + jb + 4 + k, n - 1));
      float x[4], fr[4];
      int e[4], ec[4], v[4], ii[4];
      bool slow = false;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        x[k] = jb + k < nv ? t[k] : 0.0f;  // zero padding: no change to any state
        P += x[k];
        e[k] = binade_fast(P);
        ec[k] = binade_code(P, R);
      }
      if (jb == 0) {
        ep_first = ec[0];
        x0 = x[0];
        elast = ec[0];
      }
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const float A = ldexpf(x[k], 23 - e[k]);
        const float I = floorf(fminf(A, 268435456.0f));
        fr[k] = A - I;
        ii[k] = static_cast<int>(I);
        const bool step = !(jb == 0 && k == 0);  // step 0 is combined after the exchange
        const int ein = k == 0 ? elast : ec[k - 1];
        slow |= step && (seg_break(ec[k], ein) || fr[k] == 0.5f);
        v[k] = step ? min(ii[k] + (fr[k] > 0.5f ? 1 : 0), kCap) : 0;
      }
      if (slow) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
          if (jb == 0 && k == 0) continue;
          const int ein = k == 0 ? elast : ec[k - 1];
          if (seg_break(ec[k], ein)) {
            // plain selects keep the records in registers
            const bool r1 = ncross == 0, r2 = ncross == 1;
            x1 = r1 ? x[k] : x1;
            e1 = r1 ? ec[k] : e1;
            pre1.e = r1 ? rest.p.e : pre1.e;
            pre1.o = r1 ? rest.p.o : pre1.o;
            x2 = r2 ? x[k] : x2;
            e2 = r2 ? ec[k] : e2;
            pre2.e = r2 ? rest.p.e : pre2.e;
            pre2.o = r2 ? rest.p.o : pre2.o;
            ncross++;
            rest.p = Pair{0, 0};
            rest.c++;
          } else if (fr[k] == 0.5f) {
            const int i = ii[k];
            rest.p = compose(rest.p, Pair{i + (i & 1), i + 1 - (i & 1)});
          } else {
            rest.p.e = min(rest.p.e + v[k], kCap);
            rest.p.o = min(rest.p.o + v[k], kCap);
          }
        }
      } else {
        const int s4 = (v[0] + v[1]) + (v[2] + v[3]);  // each <= 2^28: no overflow
        rest.p.e = min(rest.p.e + s4, kCap);
        rest.p.o = min(rest.p.o + s4, kCap);
      }
      elast = ec[3];
#pragma unroll
      for (int k = 0; k < 4; k++) t[k] = u[k];
    }
    ep_last = elast;
  }
  int prev_last = wave_shr1(ep_last);
  if (lane == 63) s_epl[wave] = ep_last;
  group_sync<NG>();
  if (lane == 0) prev_last = wave > 0 ? s_epl[wave - 1] : binade_code(sH, R);
  int next_first = __shfl_down(ep_first, 1, 64);
  const bool cross0 = seg_break(ep_first, prev_last);
  const SegAcc el0 = cross0 ? SegAcc{Pair{0, 0}, 1} : SegAcc{term_pair_fast(x0, ep_first), 0};
  const SegAcc loc = nv > 0 ? seg_combine(el0, rest) : SegAcc{Pair{0, 0}, 0};
  // workgroup exclusive segmented scan of the lanes' compositions
  const SegAcc incs = scan_seg(loc);
  if (lane == 63) {
    s_sw[3 * wave] = incs.p.e;
    s_sw[3 * wave + 1] = incs.p.o;
    s_sw[3 * wave + 2] = incs.c;
  }
  // the first lane of each wave needs the next wave's first binade
  __shared__ int s_epf_[NG][W];
  int* s_epf = s_epf_[g];
  if (lane == 0) s_epf[wave] = ep_first;
  group_sync<NG>();
  if (lane == 63) next_first = wave + 1 < W ? s_epf[wave + 1] : 0;
  SegAcc run{Pair{0, 0}, 0}, all;
  {
    const SegAcc tw = row_scan_seg(lane < W ? SegAcc{Pair{s_sw[3 * lane], s_sw[3 * lane + 1]}, s_sw[3 * lane + 2]}
                                            : SegAcc{Pair{0, 0}, 0});
    auto pick = [&](int w) {
      return SegAcc{Pair{__builtin_amdgcn_readlane(tw.p.e, w), __builtin_amdgcn_readlane(tw.p.o, w)},
                    __builtin_amdgcn_readlane(tw.c, w)};
    };
    if (wave > 0) run = pick(wave - 1);
    all = pick(W - 1);
  }
  run = seg_combine(run, SegAcc{Pair{wave_shr1(incs.p.e), wave_shr1(incs.p.o)}, wave_shr1(incs.c)});
  // pass 3: segment totals and crossing terms, indexed by segment, from the
  // records of pass 2 (a lane with more crossings walks its run again)
  if (all.c <= kPredMaxCross && nv > 0) {
    const SegAcc r0 = seg_combine(run, el0);  // after step 0
    if (cross0) {
      s_ct[r0.c] = x0;
      s_ce[r0.c] = ep_first;
      if (r0.c == 1 && i0 == kPredHead) {  // segment 0 is empty
        s_tot[0] = 0;
        s_tot[1] = 0;
      }
    }
    if (ncross <= 2) {
      if (ncross >= 1) {
        const Pair t1 = compose(r0.p, pre1);  // the segment ending at step j1-1
        s_tot[2 * r0.c] = t1.e;
        s_tot[2 * r0.c + 1] = t1.o;
        s_ct[r0.c + 1] = x1;
        s_ce[r0.c + 1] = e1;
      }
      if (ncross == 2) {
        s_tot[2 * (r0.c + 1)] = pre2.e;
        s_tot[2 * (r0.c + 1) + 1] = pre2.o;
        s_ct[r0.c + 2] = x2;
        s_ce[r0.c + 2] = e2;
      }
    } else {
      SegAcc r = r0;
      float P = P0;
      int ein = prev_last;
      for_each_run(a, i0, nv, n, [&](int j, float x) {
        P += x;
        const int e = binade_code(P, R);
        if (j > 0) {
          const bool cross = seg_break(e, ein);
          if (cross) {  // step j-1 ends its segment
            s_tot[2 * r.c] = r.p.e;
            s_tot[2 * r.c + 1] = r.p.o;
          }
          seg_push(r, cross, term_pair_fast(x, e));
          if (cross) {
            s_ct[r.c] = x;
            s_ce[r.c] = e;
          }
        }
        ein = e;
      });
    }
    if (i0 + nv == n || seg_break(next_first, ep_last)) {  // the lane's last step ends its segment
      const SegAcc fin = seg_combine(run, loc);
      s_tot[2 * fin.c] = fin.p.e;
      s_tot[2 * fin.c + 1] = fin.p.o;
    }
  }
  group_sync<NG>();
  // the walk: wave 0 holds segment j in lane j and carries the exact value
  // from segment to segment
  if (wave == 0) {
    const int K = all.c;
    const int jl = min(lane, kPredMaxCross);
    bool good;
    const float val = walk_segments(sH, K, s_tot[2 * jl], s_tot[2 * jl + 1], s_ct[jl], s_ce[jl], &good);
    if (lane == 0) {
      s_res = val;
      s_ok = good;
    }
  }
  group_sync<NG>();
  *ok = s_ok != 0;
  return s_res;
}


template <int NT, class Term>
__device__ __forceinline__ float block_seq_sum_pred(Term a, int n, bool* ok) {
  return group_seq_sum_pred<NT, 1>(a, n, ok);
}

// The sequential fold of a[0..n), a[i] >= 0, evaluated by an NT-lane
// workgroup (blockDim.x == NT); every lane returns the same value. Must be
// called by all lanes. a may live in LDS or global memory (read-only here,
// visible to the whole workgroup). Sums of up to kPredHead + NT *
// kPredMaxPerLane terms use the predicted-binade scan, falling back to one
// lane's chain for non-finite terms, very short sums and failed predictions
// (PADDED: a is an LDS buffer, 16-byte aligned and zero-filled up to
// lane_pad(n) terms, so the chain runs on 16-byte loads; such rows of up to
// kPadSerialMax terms take that chain directly). Longer sums use the
// adaptive binade scan, holding up to NT*CMAX terms in registers (thread t
// owns the contiguous run [t*C, t*C + C), C = ceil(n/NT)) and streaming
// longer sums from `a`; non-finite terms again run on one lane.
// The same fold for sums of at most kPredHead + NT * kPredMaxPerLane terms
// given by a term function (see group_seq_sum_pred): the predicted-binade
// scan with a one-lane fallback, evaluated by NG lane groups at once, each
// with its own term function and n (uniform within the group); every lane of
// a group gets its group's sum.
template <int NT, int NG, class Term>
__device__ __forceinline__ float group_seq_sum_short(Term term, int n) {
  __shared__ float s_short[NG];
  const int g = NG > 1 ? static_cast<int>(threadIdx.x) / NT : 0;
  if (n > kPredHead) {
    bool ok;
    const float v = group_seq_sum_pred<NT, NG>(term, n, &ok);
    if (ok) return v;
  }
  if (threadIdx.x % NT == 0) {
    float s = -0.0f;
    for (int i = 0; i < n; i++) s += term(i);
    s_short[g] = s;
  }
  group_sync<NG>();
  return s_short[g];
}
template <int NT, class Term>
__device__ __forceinline__ float block_seq_sum_short(Term term, int n) {
  return group_seq_sum_short<NT, 1>(term, n);
}

// The predicted-binade fold for terms held in registers, TPL consecutive
// terms per lane, evaluated by a group of NL lanes (NL a multiple of 64, at
// most 16 waves): group lane r (0 <= r < NL, r = 0 on the group's first lane,
// waves whole) holds t[k] = term(TPL*r + k), zero past n, with n <= TPL * NL.
// The lanes holding the kPredHead = 32 head terms (r < 32 / TPL) are folded
// serially by the group's wave 0 (read lane by lane); lane r beyond them owns
// steps TPL*r .. TPL*r + TPL-1. Differences from group_seq_sum_pred: no term
// is read from memory; the binade code of the partial sum between two lanes
// is taken from one value both of them compute with the same operations (the
// later lane's approximate entry sum), so the lanes need not exchange their
// last codes (one barrier fewer); and the lane that owns a crossing records
// the segment ending before it. The walk and its verification are the same,
// and so is the fallback: non-finite terms, more than kPredMaxCross crossings
// or a failed check fold term(0..n) on one lane (term reads memory the whole
// group sees). Every lane of the group returns the fold.
//
// sync() is a barrier of the group's waves that also orders their LDS
// accesses: __syncthreads() when the group is the workgroup, an LDS-counter
// barrier for a group of waves inside a larger workgroup. Four group
// barriers (six on the fallback).
template <int NL, int TPL, class Sync, class Term>
__device__ __forceinline__ float lanes_seq_sum(const float (&t)[TPL], int n, int r, Sync&& sync, Term term) {
  static_assert(NL % 64 == 0 && NL / 64 <= 16, "whole waves, at most 16");
  static_assert(TPL >= 1 && kPredHead % TPL == 0, "the head is whole lanes");
  constexpr int W = NL / 64;
  constexpr int kHeadLanes = kPredHead / TPL;
  static_assert(kHeadLanes <= 64, "the head sits in wave 0");
  __shared__ float s_fw[W];
  __shared__ int s_bad[W];
  __shared__ int s_sw[3 * W];
  __shared__ int s_tot[2 * (kPredMaxCross + 1)];
  __shared__ float s_ct[kPredMaxCross + 1];
  __shared__ int s_ce[kPredMaxCross + 1];
  __shared__ float s_head, s_res;
  __shared__ int s_ok;
  const int lane = r & 63, wave = r >> 6;
  bool bad = false;
#pragma unroll
  for (int k = 0; k < TPL; k++) bad |= !(t[k] <= 3.4028234663852886e38f);  // zero past n: finite
  // the head: term(0 .. min(n, 32)) left to right, read from lanes 0..kHeadLanes-1
  if (wave == 0) {
    float h = -0.0f;
    if (n >= kPredHead) {  // (uniform) every head term is live: no select between the adds
#pragma unroll
      for (int j = 0; j < kHeadLanes; j++)
#pragma unroll
        for (int k = 0; k < TPL; k++) h += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t[k]), j));
    } else {
#pragma unroll
      for (int j = 0; j < kHeadLanes; j++)
#pragma unroll
        for (int k = 0; k < TPL; k++) {
          const float v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t[k]), j));
          if (TPL * j + k < n) h += v;
        }
    }
    if (lane == 0) s_head = h;
  }
  const int nv = r < kHeadLanes ? 0 : max(0, min(TPL, n - TPL * r));
  // pass 1: approximate prefix sums (only the grids depend on them)
  float ls = 0.0f;
  if (nv > 0) {
    if constexpr (TPL == 4) {
      ls = (t[0] + t[1]) + (t[2] + t[3]);
    } else {
#pragma unroll
      for (int k = 0; k < TPL; k++) ls += t[k];
    }
  }
  const float inc = scan_add_f32(ls);
  if (lane == 63) s_fw[wave] = inc;
  if (lane == 0) s_bad[wave] = __builtin_amdgcn_ballot_w64(bad) != 0;
  sync();  // barrier 1: also publishes s_head
  bool any_bad = false;
#pragma unroll
  for (int w = 0; w < W; w++) any_bad |= s_bad[w] != 0;
  const float sH = s_head;
  float result = sH;
  bool ok = !any_bad;
  if (ok && n > kPredHead) {
    const int R = pred_margin(n);
    const float tw = row_scan_add_f32(lane < W ? s_fw[lane] : 0.0f);
    const float pre = wave > 0 ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tw), wave - 1)) : 0.0f;
    const float P0 = sH + (pre + __int_as_float(wave_shr1(__float_as_int(inc))));
    // the next lane's entry, by the same operations as that lane computes it
    const float pre_n = wave + 1 < W ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tw), wave)) : 0.0f;
    const float P0n = lane < 63 ? sH + (pre + inc) : sH + (pre_n + 0.0f);
    const bool next_steps = TPL * (r + 1) < n;  // the next lane owns steps (it is past the head when nv > 0)
    // pass 2: codes, crossings and increment pairs of this lane's steps. The
    // approximate partial sums come first (one dependent add per step); the
    // codes, flags and pairs of the steps are then independent of each
    // other, and the lane's segment accumulator is a balanced tree of
    // seg_combine over the steps (each step a crossing {identity, 1} or
    // {pair, 0}; steps past nv the identity), no branches.
    int ec[TPL];
    bool cross[TPL];
    Pair pr[TPL];
    SegAcc el[TPL];
    {
      float Pk[TPL];
      float P = P0;
#pragma unroll
      for (int k = 0; k < TPL; k++) {
        P += t[k];
        Pk[k] = P;
      }
      const int e0 = binade_code(P0, R);
      const int en = binade_code(P0n, R);
#pragma unroll
      for (int k = 0; k < TPL; k++) {
        const bool last = (k == nv - 1) & next_steps;
        const int ek = binade_code(Pk[k], R);
        ec[k] = last ? en : ek;
      }
#pragma unroll
      for (int k = 0; k < TPL; k++) {
        const bool live = k < nv;
        cross[k] = live & seg_break(ec[k], k == 0 ? e0 : ec[k - 1]);
        const Pair q = term_pair_fast(t[k], ec[k]);
        const bool use = live & !cross[k];
        pr[k] = Pair{use ? q.e : 0, use ? q.o : 0};
        el[k] = SegAcc{pr[k], cross[k] ? 1 : 0};
      }
    }
    SegAcc loc;
    {
      SegAcc tr[TPL];
#pragma unroll
      for (int k = 0; k < TPL; k++) tr[k] = el[k];
#pragma unroll
      for (int w = 1; w < TPL; w *= 2)
#pragma unroll
        for (int k = 0; k + w < TPL; k += 2 * w) tr[k] = seg_combine(tr[k], tr[k + w]);
      loc = tr[0];
    }
    const SegAcc incs = scan_seg(loc);
    if (lane == 63) {
      s_sw[3 * wave] = incs.p.e;
      s_sw[3 * wave + 1] = incs.p.o;
      s_sw[3 * wave + 2] = incs.c;
    }
    sync();  // barrier 2
    SegAcc run{Pair{0, 0}, 0}, all;
    {
      const SegAcc tws = row_scan_seg(lane < W ? SegAcc{Pair{s_sw[3 * lane], s_sw[3 * lane + 1]}, s_sw[3 * lane + 2]}
                                              : SegAcc{Pair{0, 0}, 0});
      auto pick = [&](int w) {
        return SegAcc{Pair{__builtin_amdgcn_readlane(tws.p.e, w), __builtin_amdgcn_readlane(tws.p.o, w)},
                      __builtin_amdgcn_readlane(tws.c, w)};
      };
      if (wave > 0) run = pick(wave - 1);
      all = pick(W - 1);
    }
    run = seg_combine(run, SegAcc{Pair{wave_shr1(incs.p.e), wave_shr1(incs.p.o)}, wave_shr1(incs.c)});
    // records: a crossing closes the segment before it; the lane of the last
    // step closes the last segment
    if (all.c <= kPredMaxCross && nv > 0) {
      SegAcc rr = run;
#pragma unroll
      for (int k = 0; k < TPL; k++) {
        if (cross[k]) {  // rare: the segment before this step closes here
          s_tot[2 * rr.c] = rr.p.e;
          s_tot[2 * rr.c + 1] = rr.p.o;
          s_ct[rr.c + 1] = t[k];
          s_ce[rr.c + 1] = ec[k];
        }
        rr = seg_combine(rr, el[k]);
      }
      if (TPL * r + nv == n) {
        s_tot[2 * rr.c] = rr.p.e;
        s_tot[2 * rr.c + 1] = rr.p.o;
      }
    }
    sync();  // barrier 3
    // the walk (group_seq_sum_pred's): wave 0 holds segment j in lane j
    if (wave == 0) {
      const int K = all.c;
      const int jl = min(lane, kPredMaxCross);
      bool good;
      const float val = walk_segments(sH, K, s_tot[2 * jl], s_tot[2 * jl + 1], s_ct[jl], s_ce[jl], &good);
      if (lane == 0) {
        s_res = val;
        s_ok = good;
      }
    }
    sync();  // barrier 4
    ok = s_ok != 0;
    result = s_res;
  }
  if (!ok) {  // non-finite terms or a failed prediction: one lane's chain
    sync();  // every read of s_res above is done
    if (r == 0) {
      float s = -0.0f;
      for (int i = 0; i < n; i++) s += term(i);
      s_res = s;
    }
    sync();
    result = s_res;
  }
  return result;
}

// lanes_seq_sum over the whole workgroup (blockDim.x == NT), four terms per
// lane: lane t holds t4[k] = term(4t + k).
template <int NT, class Term>
__device__ __forceinline__ float quad_seq_sum(const float (&t4)[4], int n, Term term) {
  return lanes_seq_sum<NT, 4>(t4, n, static_cast<int>(threadIdx.x), [] { __syncthreads(); }, term);
}

// A barrier among `waves` consecutive waves of a workgroup whose other waves
// do not take part: each wave adds one to an LDS counter once its earlier LDS
// accesses are done, then waits until the counter reaches waves times the
// number of barriers passed so far. The counter must be zero before the
// group's first barrier (and it is never reset in between). The waiting waves
// issue no global memory operations, so the wait ends once every wave of the
// group has arrived; a bound on the polls keeps a wave from waiting forever
// should one never arrive (the caller's result is then wrong, not hung).
struct LdsGroupBarrier {
  int* ctr;
  int waves;
  int passed;
  __device__ void operator()() {
    passed += 1;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    const int target = waves * passed;
    for (int polls = 0; polls < (1 << 22); polls++) {
      if (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) break;
      __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  }
};

constexpr int kPadSerialMax = 896;
template <int NT, bool PADDED, int CMAX = 16>
__device__ __forceinline__ float block_seq_sum_nonneg(const float* a, int n) {
  static_assert(NT % 64 == 0 && NT <= 1024, "whole waves");
  __shared__ int s_wave[2 * (NT / 64)];
  __shared__ float s_sum;
  __shared__ int s_k, s_first;
  const int tid = threadIdx.x;
  if (n <= 0) return -0.0f;
  if (n <= kPredHead + NT * kPredMaxPerLane) {
    // a padded LDS row folds on one lane at the add latency (~4 ns a term, its
    // 16-byte loads a batch ahead), which beats the scan's fixed cost (five
    // barriers, ~3.5 us) for rows of up to kPadSerialMax terms
    if (n > (PADDED ? kPadSerialMax : kPredHead)) {
      bool ok;
      const float v = block_seq_sum_pred<NT>([a](int i) { return a[i]; }, n, &ok);
      if (ok) return v;
    }
    // non-finite terms, short sums and failed predictions: one lane's chain
    if (tid == 0) {
      if (PADDED) {
        s_sum = lane_seq_sum_padded(a, n);
      } else {
        float s = -0.0f;
        for (int i = 0; i < n; i++) s += a[i];
        s_sum = s;
      }
    }
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
