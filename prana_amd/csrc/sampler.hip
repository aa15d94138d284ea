// Temperature sampling (Sampler::sample, sampler.rs:22-39) on the device:
// logits / temp, the exact softmax (softmax_kernel), then the bucket walk
//   r = u01; for i: r -= p[i]; if r <= 0 return i;   (last index otherwise)
// in the reference's left-to-right f32 order.
//
// The walk is a sequential f32 fold with a data-dependent stop. While r
// stays inside one binade [2^e, 2^(e+1)) it is m * 2^(e-23) with an integer
// m, and one step is m' = rne(m - p/u): the decrement is I or I+1 for p/u = I
// + f, and on a tie the one that leaves m' even, which depends only on the
// parity of m. That is the increment pair of exact_sum.h with the sign
// flipped (rounding to nearest even is symmetric), and pairs compose
// associatively, so a workgroup scan over 8192 terms gives every r of the
// span exactly as long as no step leaves the binade. The first step that
// could leave it (grid result <= 2^23, where the finer grid below could round
// differently) is evaluated as the plain f32 subtraction from the exact value
// before it; it either ends the walk (r <= 0) or starts the next scan. In the
// lowest binade (e = -126, grid 2^-149 down to 0) only r <= 0 ends a segment.
// Spans holding a negative or non-finite probability, and an r that is not a
// positive finite number, walk on one lane.
#include <climits>

#include "common.h"
#include "exact_sum.h"
#include "kernels.h"

namespace prana {

namespace {

constexpr int kPickNT = 1024;
constexpr int kPickCT = 8;  // terms per lane per scan
constexpr int kPickSpan = kPickNT * kPickCT;

__device__ __forceinline__ int32_t apply_dec(exact::Pair p, int32_t m) { return m - ((m & 1) ? p.o : p.e); }

__global__ void scale_kernel(const float* __restrict__ x, size_t n, float temp, float* __restrict__ out) {
  const size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i < n) out[i] = x[i] / temp;  // sampler.rs:27
}

// r comes from rs[r_index] when rs is non-null, else from r_host.
__global__ __launch_bounds__(kPickNT) void sample_pick_kernel(const float* __restrict__ p, int n,
                                                              const float* __restrict__ rs, int r_index, float r_host,
                                                              uint32_t* __restrict__ out) {
  __shared__ int s_wave[2 * (kPickNT / 64)];
  __shared__ float s_r;
  __shared__ int s_b, s_first, s_ans;
  const int tid = threadIdx.x;
  if (tid == 0) {
    s_r = rs ? rs[r_index] : r_host;
    s_b = 0;
    s_ans = -1;
  }
  __syncthreads();
  while (true) {
    const float r = s_r;
    const int b = s_b;
    if (s_ans >= 0 || b >= n) break;  // uniform: read after the barrier that ends each pass
    const int j0 = b + tid * kPickCT;
    float v[kPickCT];
    bool bad = false;
#pragma unroll
    for (int i = 0; i < kPickCT; i++) {
      v[i] = j0 + i < n ? p[j0 + i] : 0.0f;
      // the scan's pairs are decrements: negative, NaN and infinite terms
      // (-0.0 included in neither) take the one-lane walk
      bad |= !(v[i] >= 0.0f && v[i] <= 3.4028234663852886e38f);
    }
    if (__syncthreads_or(bad) || !(r > 0.0f && r <= 3.4028234663852886e38f)) {
      if (tid == 0) {  // this span, one term at a time
        const int end = min(n, b + kPickSpan);
        float rr = r;
        int ans = -1;
        for (int i = b; i < end; i++) {
          rr -= p[i];
          if (rr <= 0.0f) {
            ans = i;
            break;
          }
        }
        s_r = rr;
        s_b = end;
        s_ans = ans;
      }
      __syncthreads();
      continue;
    }
    int e;
    int32_t m;
    exact::decompose(r, &e, &m);
    const float u = ldexpf(1.0f, e - 23);
    const int32_t lo = e > -126 ? (1 << 23) + 1 : 1;  // grid values below this may leave the binade
    exact::Pair pr[kPickCT];
    exact::Pair loc{0, 0};
#pragma unroll
    for (int i = 0; i < kPickCT; i++) {
      pr[i] = exact::term_pair_bits(__float_as_uint(v[i]), e);
      loc = exact::compose(loc, pr[i]);
    }
    if (tid == 0) s_first = INT_MAX;
    exact::Pair total;
    const exact::Pair pre = exact::block_exclusive_scan<kPickNT>(loc, s_wave, &total);  // barrier
    int32_t mm = apply_dec(pre, m), mprev = 0;
    int first = INT_MAX;
    float pv = 0.0f;
#pragma unroll
    for (int i = 0; i < kPickCT; i++) {
      if (first == INT_MAX && j0 + i < n) {
        const int32_t m2 = apply_dec(pr[i], mm);
        if (m2 < lo) {
          first = j0 + i;
          mprev = mm;
          pv = v[i];
        }
        mm = m2;
      }
    }
    if (first != INT_MAX) atomicMin(&s_first, first);
    __syncthreads();
    const int f = s_first;
    if (f == INT_MAX) {
      if (tid == 0) {  // the whole span stayed in the binade
        s_r = static_cast<float>(apply_dec(total, m)) * u;
        s_b = b + kPickSpan;
      }
    } else if (first == f) {  // the step that may leave the binade, as an f32 subtraction
      const float rn = static_cast<float>(mprev) * u - pv;
      if (rn <= 0.0f) {
        s_ans = f;
      } else {
        s_r = rn;
        s_b = f + 1;
      }
    }
    __syncthreads();
  }
  if (tid == 0) out[0] = s_ans >= 0 ? static_cast<uint32_t>(s_ans) : static_cast<uint32_t>(n - 1);
}

}  // namespace

int launch_sample_pick(const float* probs, size_t n, const float* rs, int r_index, float r_host, uint32_t* out,
                       hipStream_t s) {
  PRANA_CHECK(n >= 1 && n <= static_cast<size_t>(INT_MAX) - kPickSpan, "sample: vocabulary size out of range");
  hipLaunchKernelGGL(sample_pick_kernel, dim3(1), dim3(kPickNT), 0, s, probs, static_cast<int>(n), rs, r_index,
                     r_host, out);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

int launch_sample(const float* logits, size_t n, float temp, const float* rs, int r_index, float r_host,
                  float* scaled, float* probs, uint32_t* out, hipStream_t s) {
  if (temp <= 0.0f) return launch_argmax(logits, 1, n, out, s);  // Sampler::new: greedy iff temp <= 0
  hipLaunchKernelGGL(scale_kernel, dim3((n + 255) / 256), dim3(256), 0, s, logits, n, temp, scaled);
  PRANA_LAUNCH_CHECK();
  if (int rc = launch_softmax(scaled, 1, n, probs, s)) return rc;
  return launch_sample_pick(probs, n, rs, r_index, r_host, out, s);
}

}  // namespace prana
