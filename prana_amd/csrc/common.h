// Shared device helpers and host error plumbing for libprana_hip.
//
// Numerics contract: every f32 expression that feeds an output is evaluated
// in the same order as the reference scalar tier (no FMA contraction — the
// library is built with -ffp-contract=off — IEEE division and square root,
// round-half-away-from-zero), so results are bit-identical to the CPU path.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

namespace prana {

// ---------------------------------------------------------------- errors
// Status codes of the C ABI (see include/prana_hip.h).
enum Status : int {
  kOk = 0,
  kErrInvalid = -1,
  kErrHip = -2,
  kErrNoMem = -3,
  kErrUnsupported = -4,
  kErrShortBuffer = -5,
};

void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int hip_fail(hipError_t e, const char* what);

#define PRANA_HIP(expr)                                   \
  do {                                                    \
    hipError_t e_ = (expr);                               \
    if (e_ != hipSuccess) return ::prana::hip_fail(e_, #expr); \
  } while (0)

#define PRANA_CHECK(cond, msg)                                 \
  do {                                                         \
    if (!(cond)) return ::prana::fail(::prana::kErrInvalid, msg); \
  } while (0)

#define PRANA_LAUNCH_CHECK()                                   \
  do {                                                         \
    hipError_t e_ = hipGetLastError();                         \
    if (e_ != hipSuccess) return ::prana::hip_fail(e_, "kernel launch"); \
  } while (0)

// ---------------------------------------------------------------- f16
// f16 bits -> f32 exactly as prana-kernels lib.rs:57-73. The hardware
// conversion agrees with the reference on every non-NaN input (checked
// exhaustively on gfx950); NaNs keep their payload unquieted, as the
// reference does.
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  float hw = __half2float(__ushort_as_half(h));
  bool nan = ((h & 0x7c00u) == 0x7c00u) && (h & 0x03ffu);
  uint32_t nb = (static_cast<uint32_t>(h & 0x8000u) << 16) | 0x7f800000u |
                (static_cast<uint32_t>(h & 0x03ffu) << 13);
  return nan ? __uint_as_float(nb) : hw;
}

// f16 bits -> f32 for a value that only feeds arithmetic (a dot product
// operand). Identical to f16_to_f32 except that a signalling NaN comes out
// quiet with the same sign and payload — which is what the first arithmetic
// operation does to f16_to_f32's signalling result anyway, so every result
// computed from it is unchanged. One instruction instead of five.
__device__ __forceinline__ float f16_operand(uint16_t h) { return __half2float(__ushort_as_half(h)); }

// f32 -> f16 bits, round-to-nearest-even, exactly as lib.rs:78-113 (NaN ->
// sign | 0x7e00; hardware RNE matches every other input exhaustively).
__device__ __forceinline__ uint16_t f32_to_f16(float x) {
  uint32_t u = __float_as_uint(x);
  bool nan = (u & 0x7fffffffu) > 0x7f800000u;
  uint16_t hw = __half_as_ushort(__float2half_rn(x));
  return nan ? static_cast<uint16_t>(((u >> 16) & 0x8000u) | 0x7e00u) : hw;
}

// RoPE pair rotation with host-computed (cos, sin) = glibc (cosf, sinf) of
// (pos as f32) * powf(theta, -(2m)/hd), the exact values the reference
// computes inline (attention.rs:93-100, 111-119).
__device__ __forceinline__ void rotate(float& a, float& b, float2 cs) {
  float x0 = a, x1 = b;
  a = x0 * cs.x - x1 * cs.y;
  b = x0 * cs.y + x1 * cs.x;
}

// ---------------------------------------------------------------- launch attributes
// hipFuncSetAttribute(MaxDynamicSharedMemorySize). A refusal returns false and
// is cleared from HIP's last-error state, so that a later launch check does not
// report it as a failed launch.
inline bool set_max_dynamic_lds(const void* fn, int bytes) {
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) == hipSuccess) return true;
  (void)hipGetLastError();
  return false;
}

// Static LDS bytes of a kernel (0 when the query fails).
inline size_t static_lds_bytes(const void* fn) {
  hipFuncAttributes a{};
  if (hipFuncGetAttributes(&a, fn) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return a.sharedSizeBytes;
}

// ---------------------------------------------------------------- expf
// The reference reaches expf through Rust's f32::exp -> glibc expf. glibc
// (2.28+) computes it with the ARM optimized-routines algorithm: a 32-entry
// table of 2^(i/32) and a cubic in double precision; on x86_64 hosts with FMA
// the multiarch build contracts four products into FMAs. This restatement
// reproduces that evaluation exactly; it equals the host glibc expf on all
// 2^32 inputs (exhaustive check in the GPU test suite).
// Upstream: ARM optimized-routines math/expf.c and math/exp2f_data.c (MIT OR
// Apache-2.0 WITH LLVM-exception), shipped in glibc as
// sysdeps/ieee754/flt-32/e_expf.c and e_exp2f_data.c (LGPL-2.1+).
// kExp2Tab[i] = asuint64(double(2^(i/32))) - (i << 47); the CPU test
// tests/test_device_tables.py regenerates it from that definition. The three
// polynomial coefficients below are upstream's minimax fit for N = 32 (with
// the 1/N scalings folded in), kept unchanged because bit-identical results
// need exactly upstream's constants.
static __constant__ const uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

__device__ __forceinline__ float dev_expf(float x) {
  uint32_t ux = __float_as_uint(x);
  uint32_t abstop = (ux >> 20) & 0x7ffu;
  if (abstop >= 0x42bu) {                       // |x| >= 88 or x is NaN/inf
    if (ux == 0xff800000u) return 0.0f;         // exp(-inf)
    if (abstop >= 0x7f8u) return x + x;         // +inf or NaN
    if (x > 0x1.62e42ep6f) return __uint_as_float(0x7f800000u);  // overflow
    if (x < -0x1.9fe368p6f) return 0.0f;                          // underflow
  }
  const double kInvLn2N = 0x1.71547652b82fep+0 * 32.0;
  const double kShift = 0x1.8p+52;
  const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
  const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
  const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
  double xd = static_cast<double>(x);
  double kd = __fma_rn(kInvLn2N, xd, kShift);
  uint64_t ki = static_cast<uint64_t>(__double_as_longlong(kd));
  kd -= kShift;
  double r = __fma_rn(kInvLn2N, xd, -kd);
  uint64_t t = kExp2Tab[ki % 32] + (ki << 47);
  double s = __longlong_as_double(static_cast<long long>(t));
  double z = __fma_rn(c0, r, c1);
  double r2 = r * r;
  double y = __fma_rn(c2, r, 1.0);
  y = __fma_rn(z, r2, y);
  y = y * s;
  return static_cast<float>(y);
}

// ---------------------------------------------------------------- tanhf
// gelu_tanh (norms.rs:35-41) reaches tanhf through Rust's f32::tanh ->
// glibc tanhf, which (through glibc 2.40) is the fdlibm single-precision
// tanhf over fdlibm's expm1f: tanh|x| = 1 - 2/(expm1(2|x|) + 2) for |x| >= 1,
// -t/(t + 2) with t = expm1(-2|x|) below, x(1 + x) under 2^-55, 1 past 22.
// expm1f reduces x = k ln2 + r (ln2 split hi/lo, correction c) and evaluates
// fdlibm's rational form with a degree-5 polynomial R1 in x^2/2. The
// constants are fdlibm's (Sun Microsystems, freely distributable), needed
// unchanged for bit-identical results. This restatement equals glibc 2.35's
// tanhf on all 2^32 inputs (exhaustive check in the GPU test suite).
// Upstream: fdlibm s_tanh.c / s_expm1.c, float versions in glibc
// sysdeps/ieee754/flt-32/s_tanhf.c and s_expm1f.c.
__device__ __forceinline__ float dev_expm1f(float x) {
  const float kHuge = 1.0e+30f, kTiny = 1.0e-30f;
  const float kOThreshold = 8.8721679688e+01f, kLn2Hi = 6.9313812256e-01f, kLn2Lo = 9.0580006145e-06f;
  const float kInvLn2 = 1.4426950216e+00f;
  const float Q1 = -3.3333335072e-02f, Q2 = 1.5873016091e-03f, Q3 = -7.9365076090e-05f, Q4 = 4.0082177293e-06f,
              Q5 = -2.0109921195e-07f;
  const uint32_t bits = __float_as_uint(x);
  const bool neg = (bits >> 31) != 0;
  const uint32_t hx = bits & 0x7fffffffu;
  if (hx >= 0x4195b844u) {  // |x| >= 27 ln2
    if (hx >= 0x42b17218u) {
      if (hx > 0x7f800000u) return x + x;  // NaN
      if (hx == 0x7f800000u) return neg ? -1.0f : x;
      if (x > kOThreshold) return kHuge * kHuge;  // overflow
    }
    if (neg) return kTiny - 1.0f;  // expm1 -> -1
  }
  float hi, lo, c = 0.0f;
  int k;
  if (hx > 0x3eb17218u) {    // |x| > ln2 / 2
    if (hx < 0x3f851592u) {  // and |x| < 1.5 ln2
      if (!neg) {
        hi = x - kLn2Hi;
        lo = kLn2Lo;
        k = 1;
      } else {
        hi = x + kLn2Hi;
        lo = -kLn2Lo;
        k = -1;
      }
    } else {
      k = static_cast<int>(kInvLn2 * x + (neg ? -0.5f : 0.5f));
      const float t = static_cast<float>(k);
      hi = x - t * kLn2Hi;
      lo = t * kLn2Lo;
    }
    x = hi - lo;
    c = (hi - x) - lo;
  } else if (hx < 0x33000000u) {  // |x| < 2^-25
    const float t = kHuge + x;
    return x - (t - (kHuge + x));
  } else {
    k = 0;
  }
  const float hfx = 0.5f * x;
  const float hxs = x * hfx;
  const float r1 = 1.0f + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
  float t = 3.0f - r1 * hfx;
  float e = hxs * ((r1 - t) / (6.0f - x * t));
  if (k == 0) return x - (x * e - hxs);
  e = (x * (e - c) - c);
  e -= hxs;
  if (k == -1) return 0.5f * (x - e) - 0.5f;
  if (k == 1) {
    if (x < -0.25f) return -2.0f * (e - (x + 0.5f));
    return 1.0f + 2.0f * (x - e);
  }
  const uint32_t kexp = static_cast<uint32_t>(k) << 23;  // adds k to the exponent
  float y;
  if (k <= -2 || k > 56) {
    y = 1.0f - (e - x);
    return __uint_as_float(__float_as_uint(y) + kexp) - 1.0f;
  }
  if (k < 23) {
    t = __uint_as_float(0x3f800000u - (0x1000000u >> k));  // 1 - 2^-k
    y = t - (e - x);
  } else {
    t = __uint_as_float(static_cast<uint32_t>(0x7f - k) << 23);  // 2^-k
    y = x - (e + t);
    y += 1.0f;
  }
  return __uint_as_float(__float_as_uint(y) + kexp);
}

__device__ __forceinline__ float dev_tanhf(float x) {
  const uint32_t jx = __float_as_uint(x), ix = jx & 0x7fffffffu;
  const bool neg = (jx >> 31) != 0;
  if (ix >= 0x7f800000u) return neg ? 1.0f / x - 1.0f : 1.0f / x + 1.0f;  // +-inf -> +-1, NaN -> NaN
  float z;
  if (ix < 0x41b00000u) {  // |x| < 22
    if (ix == 0) return x;
    if (ix < 0x24000000u) return x * (1.0f + x);  // |x| < 2^-55
    if (ix >= 0x3f800000u) {                      // |x| >= 1
      const float t = dev_expm1f(2.0f * fabsf(x));
      z = 1.0f - 2.0f / (t + 2.0f);
    } else {
      const float t = dev_expm1f(-2.0f * fabsf(x));
      z = -t / (t + 2.0f);
    }
  } else {
    z = 1.0f - 1.0e-30f;
  }
  return neg ? -z : z;
}

// ---------------------------------------------------------------- rounding
// Rust `(x).round().clamp(-127.0, 127.0) as i32` (matmul.rs:123): half away
// from zero, saturate, NaN -> 0.
__device__ __forceinline__ int round_clamp127(float v) {
  float r = roundf(v);
  if (r != r) return 0;
  r = r < -127.0f ? -127.0f : r;
  r = r > 127.0f ? 127.0f : r;
  return static_cast<int>(r);
}

// ---------------------------------------------------------------- wave ops
__device__ __forceinline__ float wave_max_f32(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ int wave_sum_i32(int v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
// Reductions over aligned groups of 32 lanes (one quantization block), every
// lane getting the result: within quads (DPP quad_perm), then with the
// mirrored half-row and row partners (DPP, so each lane meets the other
// quad / half-row), then across the two 16-lane rows. Max and integer sums
// do not depend on the combination order.
template <int CTRL>
__device__ __forceinline__ int dpp_lane_mov(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ float half_wave_max_f32(float v) {
  v = fmaxf(v, __int_as_float(dpp_lane_mov<0xB1>(__float_as_int(v))));   // quad_perm [1,0,3,2]
  v = fmaxf(v, __int_as_float(dpp_lane_mov<0x4E>(__float_as_int(v))));   // quad_perm [2,3,0,1]
  v = fmaxf(v, __int_as_float(dpp_lane_mov<0x141>(__float_as_int(v))));  // row_half_mirror
  v = fmaxf(v, __int_as_float(dpp_lane_mov<0x140>(__float_as_int(v))));  // row_mirror
  return fmaxf(v, __shfl_xor(v, 16, 64));
}
__device__ __forceinline__ int half_wave_sum_i32(int v) {
  v += dpp_lane_mov<0xB1>(v);
  v += dpp_lane_mov<0x4E>(v);
  v += dpp_lane_mov<0x141>(v);
  v += dpp_lane_mov<0x140>(v);
  return v + __shfl_xor(v, 16, 64);
}

// Quantize one 32-element activation block held one value per lane of an
// aligned 32-lane group (quantize_acts, matmul.rs:111-125). Returns the i8
// value of this lane; the group's scale and integer sum come back by pointer
// (valid in every lane of the group).
__device__ __forceinline__ int quantize_lane(float x, float* scale_out, int* sum_out) {
  float amax = half_wave_max_f32(fabsf(x));   // max is exact in any order
  float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
  float inv = 1.0f / scale;
  int v = round_clamp127(x * inv);
  *scale_out = scale;
  *sum_out = half_wave_sum_i32(v);            // integer sum: order-free
  return v;
}

// quantize_lane for B independent blocks at once (value b of this lane in
// y[b]); the B cross-lane reductions are interleaved so that their latencies
// overlap.
template <int B>
__device__ __forceinline__ void quantize_lanes(const float* y, int* q, float* scale, int* sum) {
  float amax[B];
#pragma unroll
  for (int b = 0; b < B; b++) amax[b] = half_wave_max_f32(fabsf(y[b]));
#pragma unroll
  for (int b = 0; b < B; b++) {
    scale[b] = amax[b] > 0.0f ? amax[b] / 127.0f : 1.0f;
    q[b] = round_clamp127(y[b] * (1.0f / scale[b]));
    sum[b] = q[b];
  }
#pragma unroll
  for (int b = 0; b < B; b++) sum[b] = half_wave_sum_i32(sum[b]);
}

// quantize_lane for a block held as four consecutive values per lane of an
// aligned 8-lane group (y[j] = element 4*(lane%8)+j of the block): one scale
// per lane and three DPP steps per reduction. Same scale, values and sum.
__device__ __forceinline__ void quantize_quad8(const float* y, int* q, float* scale_out, int* sum_out) {
  float amax = fmaxf(fmaxf(fabsf(y[0]), fabsf(y[1])), fmaxf(fabsf(y[2]), fabsf(y[3])));
  amax = fmaxf(amax, __int_as_float(dpp_lane_mov<0xB1>(__float_as_int(amax))));   // quad_perm [1,0,3,2]
  amax = fmaxf(amax, __int_as_float(dpp_lane_mov<0x4E>(__float_as_int(amax))));   // quad_perm [2,3,0,1]
  amax = fmaxf(amax, __int_as_float(dpp_lane_mov<0x141>(__float_as_int(amax))));  // row_half_mirror
  const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
  const float inv = 1.0f / scale;
  int s = 0;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    q[j] = round_clamp127(y[j] * inv);
    s += q[j];
  }
  s += dpp_lane_mov<0xB1>(s);
  s += dpp_lane_mov<0x4E>(s);
  s += dpp_lane_mov<0x141>(s);
  *scale_out = scale;
  *sum_out = s;
}

// quantize_lane for a block held as eight consecutive values per lane of an
// aligned 4-lane group (y[j] = element 8*(lane%4)+j of the block): one scale
// per lane and two DPP steps per reduction. Same scale, values and sum.
__device__ __forceinline__ void quantize_oct4(const float* y, int* q, float* scale_out, int* sum_out) {
  float amax = fmaxf(fmaxf(fmaxf(fabsf(y[0]), fabsf(y[1])), fmaxf(fabsf(y[2]), fabsf(y[3]))),
                     fmaxf(fmaxf(fabsf(y[4]), fabsf(y[5])), fmaxf(fabsf(y[6]), fabsf(y[7]))));
  amax = fmaxf(amax, __int_as_float(dpp_lane_mov<0xB1>(__float_as_int(amax))));  // quad_perm [1,0,3,2]
  amax = fmaxf(amax, __int_as_float(dpp_lane_mov<0x4E>(__float_as_int(amax))));  // quad_perm [2,3,0,1]
  const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
  const float inv = 1.0f / scale;
  int s = 0;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    q[j] = round_clamp127(y[j] * inv);
    s += q[j];
  }
  s += dpp_lane_mov<0xB1>(s);
  s += dpp_lane_mov<0x4E>(s);
  *scale_out = scale;
  *sum_out = s;
}

__device__ __forceinline__ int sdot4(int a, int b, int c) {
  return __builtin_amdgcn_sdot4(a, b, c, false);
}

}  // namespace prana
