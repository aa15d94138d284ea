// Elementwise, normalisation, RoPE, KV-cache, embedding and argmax kernels.
//
// Every reduction that the reference performs as a sequential f32 fold
// (rmsnorm's sum of squares, softmax's sum) gives exactly that fold's result
// (exact_sum.h); order-free parts (max, integer sums, elementwise products)
// run in parallel.
#include "common.h"
#include "exact_sum.h"
#include "kernels.h"

namespace prana {

// ---------------------------------------------------------------- quantize_acts
// matmul.rs:105-127. One 32-lane group per 32-element block.
__global__ __launch_bounds__(256) void quantize_acts_kernel(const float* __restrict__ x, size_t n_blocks,
                                                            int8_t* __restrict__ q, float* __restrict__ sa,
                                                            int* __restrict__ sums) {
  size_t gid = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  size_t blk = gid >> 5;
  bool live = blk < n_blocks;
  float v = live ? x[gid] : 0.0f;
  float scale;
  int sum;
  int qi = quantize_lane(v, &scale, &sum);
  if (live) {
    q[gid] = static_cast<int8_t>(qi);
    if ((threadIdx.x & 31) == 0) {
      sa[blk] = scale;
      if (sums) sums[blk] = sum;  // (quantize_q8 has none)
    }
  }
}

int launch_quantize_acts(const float* x, size_t n_rows, size_t k, int8_t* q, float* sa, int* sums,
                         hipStream_t s) {
  size_t n = n_rows * k;
  if (n == 0) return kOk;
  size_t grid = (n + 255) / 256;
  hipLaunchKernelGGL(quantize_acts_kernel, dim3(grid), dim3(256), 0, s, x, n / 32, q, sa, sums);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

// ---------------------------------------------------------------- rmsnorm
// norms.rs:9-23: ms = (sum_seq x*x)/dim; inv = 1/sqrt(ms+eps); y = (x*inv)*w.
// One workgroup per row: 1024 lanes for long rows, 256 for rows up to
// kNormSmallDim (the exact scan's fixed costs grow with the wave count, its
// per-term work shrinks with it). The sum of squares is the reference's
// left-to-right fold from -0.0, evaluated exactly by the whole workgroup; the
// normalise + optional quantize is parallel.
constexpr int kNormMaxDim = 16320;  // row and weights staged in LDS (about 132 KB)
constexpr int kNormSmallDim = 2048;
constexpr int kNormSerialMax = 512;  // rows up to this fold their squares on one lane
// Batches of more rows than this (two 1024-lane workgroups per CU and more)
// take 256-lane workgroups for rows of up to 4096 values: slower per row
// (about 11 us against 8), faster per batch (a 511-row prefill batch:
// 13.6 us against 17.6).
constexpr size_t kNormBatchRows = 256;
template <int kNormNT>
__global__ __launch_bounds__(kNormNT) void rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                          int dim, float eps, float* __restrict__ out,
                                                          int8_t* __restrict__ q, float* __restrict__ sa,
                                                          int* __restrict__ sums) {
  // (256 lanes: rows of up to kNormSmallDim, or 16 * 256 in batches)
  constexpr int kPer = ((kNormNT == 1024 ? kNormMaxDim : 16 * 256) + kNormNT - 1) / kNormNT;
  extern __shared__ float4 smem_n4[];
  float* xs = reinterpret_cast<float*>(smem_n4);  // the row, at exact::run_pad(i)
  float* wl = xs + exact::run_pad(dim);           // the weights
  const float* row = x + (size_t)blockIdx.x * dim;
  const int tid = threadIdx.x;
  {  // every load in flight at once
    float xv[kPer], wv[kPer];
#pragma unroll
    for (int k = 0; k < kPer; k++) {
      if (k * kNormNT >= dim) break;                  // uniform
      const int i = min(tid + k * kNormNT, dim - 1);  // in bounds; stored only below dim
      xv[k] = row[i];
      wv[k] = w[i];
    }
#pragma unroll
    for (int k = 0; k < kPer; k++) {
      if (k * kNormNT >= dim) break;
      const int i = tid + k * kNormNT;
      if (i < dim) {
        xs[exact::run_pad(i)] = xv[k];
        wl[i] = wv[k];
      }
    }
  }
  __syncthreads();
  // sum of squares in the reference's left-to-right order (norms.rs:15)
  float ss;
  if (dim <= kNormSerialMax) {
    // short rows: one lane folds the squares from a zero-padded LDS row at
    // the add latency, which beats the parallel scan's fixed cost
    __shared__ __align__(16) float sq[exact::lane_pad(kNormSerialMax)];
    __shared__ float s_ss;
    for (int i = tid; i < exact::lane_pad(dim); i += kNormNT) {
      const float v = i < dim ? xs[exact::run_pad(i)] : 0.0f;
      sq[i] = v * v;
    }
    __syncthreads();
    if (tid == 0) s_ss = exact::lane_seq_sum_padded(sq, dim);
    __syncthreads();
    ss = s_ss;
  } else if (dim <= 4 * kNormNT) {
    // four consecutive squares per lane, folded from registers
    float t4[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int i = 4 * tid + j;
      const float v = i < dim ? xs[exact::run_pad(i)] : 0.0f;
      t4[j] = v * v;
    }
    ss = exact::quad_seq_sum<kNormNT>(t4, dim, [xs](int i) {
      const float v = xs[exact::run_pad(i)];
      return v * v;
    });
  } else if (kNormNT == 256 && dim <= 16 * kNormNT) {
    // batches of rows (a workgroup per row, several per CU): sixteen
    // consecutive squares per lane, four waves in the scan
    float t16[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const int i = 16 * tid + j;
      const float v = i < dim ? xs[exact::run_pad(i)] : 0.0f;
      t16[j] = v * v;
    }
    ss = exact::lanes_seq_sum<kNormNT, 16>(t16, dim, tid, [] { __syncthreads(); }, [xs](int i) {
      const float v = xs[exact::run_pad(i)];
      return v * v;
    });
  } else {
    ss = exact::block_seq_sum_short<kNormNT>(
        [xs](int i) {
          const float v = xs[exact::run_pad(i)];
          return v * v;
        },
        dim);
  }
  const float mean_sq = ss / static_cast<float>(dim);
  const float inv = 1.0f / sqrtf(mean_sq + eps);
  if (dim <= 4 * kNormNT) {
    // rows of up to four values per lane: lane t takes elements 4t..4t+3, so
    // a 32-block of the quantization is eight lanes (quantize_quad8: one
    // scale per lane, three DPP steps per reduction); dim is a multiple of
    // 32 whenever q != nullptr, so 8-lane groups are all live or all past it
    const int i0 = 4 * tid;
    float y[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int i = i0 + j;
      y[j] = i < dim ? xs[exact::run_pad(i)] * inv * wl[i] : 0.0f;
      if (i < dim && out) out[(size_t)blockIdx.x * dim + i] = y[j];
    }
    if (q) {
      float scale;
      int qi[4], sum;
      quantize_quad8(y, qi, &scale, &sum);
      if (i0 < dim) {
        const size_t gi = (size_t)blockIdx.x * dim + i0;
#pragma unroll
        for (int j = 0; j < 4; j++) q[gi + j] = static_cast<int8_t>(qi[j]);
        if ((tid & 7) == 0) {
          sa[gi >> 5] = scale;
          sums[gi >> 5] = sum;
        }
      }
    }
    return;
  }
  // four elements per lane at a time; dim is a multiple of 32 whenever
  // q != nullptr, so every 32-lane group is then all live or all past the end
  // and reduces together.
  for (int base = 0; base < dim; base += 4 * kNormNT) {
    float y[4];
#pragma unroll
    for (int b = 0; b < 4; b++) {
      const int i = base + b * kNormNT + tid;
      y[b] = i < dim ? xs[exact::run_pad(i)] * inv * wl[i] : 0.0f;
      if (i < dim && out) out[(size_t)blockIdx.x * dim + i] = y[b];
    }
    if (q) {
      float scale[4];
      int qi[4], sum[4];
      quantize_lanes<4>(y, qi, scale, sum);
#pragma unroll
      for (int b = 0; b < 4; b++) {
        const int i = base + b * kNormNT + tid;
        if (i < dim) {
          const size_t gi = (size_t)blockIdx.x * dim + i;
          q[gi] = static_cast<int8_t>(qi[b]);
          if ((i & 31) == 0) {
            sa[gi >> 5] = scale[b];
            sums[gi >> 5] = sum[b];
          }
        }
      }
    }
  }
}

// Rows wider than kNormMaxDim (no limit in norms.rs:9-23): the same
// arithmetic with the row read from global memory instead of LDS. The sum of
// squares is the exact left-to-right fold (the predicted-binade scan up to
// kPredHead + 1024 * kPredMaxPerLane terms, one lane's chain beyond that);
// each lane reads an element before it writes it, so out may be x.
__global__ __launch_bounds__(1024) void rmsnorm_wide_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                            int dim, float eps, float* __restrict__ out,
                                                            int8_t* __restrict__ q, float* __restrict__ sa,
                                                            int* __restrict__ sums) {
  constexpr int NT = 1024;
  const float* row = x + (size_t)blockIdx.x * dim;
  const int tid = threadIdx.x;
  auto sq = [row](int i) {
    const float v = row[i];
    return v * v;
  };
  float ss;
  if (dim <= exact::kPredHead + NT * exact::kPredMaxPerLane) {
    ss = exact::block_seq_sum_short<NT>(sq, dim);
  } else {
    __shared__ float s_ss;
    if (tid == 0) {
      float a = -0.0f;
      for (int i = 0; i < dim; i++) a += sq(i);
      s_ss = a;
    }
    __syncthreads();
    ss = s_ss;
  }
  const float mean_sq = ss / static_cast<float>(dim);
  const float inv = 1.0f / sqrtf(mean_sq + eps);
  // four elements per lane at a time; with q, dim % 32 == 0, so every 32-lane
  // group is all live or all past the end and reduces together
  for (int base = 0; base < dim; base += 4 * NT) {
    float y[4];
#pragma unroll
    for (int b = 0; b < 4; b++) {
      const int i = base + b * NT + tid;
      y[b] = i < dim ? row[i] * inv * w[i] : 0.0f;
      if (i < dim && out) out[(size_t)blockIdx.x * dim + i] = y[b];
    }
    if (q) {
      float scale[4];
      int qi[4], sum[4];
      quantize_lanes<4>(y, qi, scale, sum);
#pragma unroll
      for (int b = 0; b < 4; b++) {
        const int i = base + b * NT + tid;
        if (i < dim) {
          const size_t gi = (size_t)blockIdx.x * dim + i;
          q[gi] = static_cast<int8_t>(qi[b]);
          if ((i & 31) == 0) {
            sa[gi >> 5] = scale[b];
            sums[gi >> 5] = sum[b];
          }
        }
      }
    }
  }
}

int launch_rmsnorm(const float* x, const float* w, size_t rows, size_t dim, float eps, float* out, int8_t* q,
                   float* sa, int* sums, hipStream_t s) {
  if (rows == 0) return kOk;
  PRANA_CHECK(!q || dim % 32 == 0, "rmsnorm: fused quantize needs dim % 32 == 0");
  PRANA_CHECK(dim >= 1 && dim <= static_cast<size_t>(INT32_MAX) - 4096, "rmsnorm: dim must be in 1..2^31-4097");
  if (dim > static_cast<size_t>(kNormMaxDim)) {  // the row does not fit LDS: read it from global memory
    hipLaunchKernelGGL(rmsnorm_wide_kernel, dim3(rows), dim3(1024), 0, s, x, w, (int)dim, eps, out, q, sa, sums);
    PRANA_LAUNCH_CHECK();
    return kOk;
  }
  const size_t lds = (exact::run_pad(static_cast<int>(dim)) + dim) * 4;
  if (dim <= static_cast<size_t>(kNormSmallDim) || (rows > kNormBatchRows && dim <= 16 * 256))
    hipLaunchKernelGGL(rmsnorm_kernel<256>, dim3(rows), dim3(256), lds, s, x, w, (int)dim, eps, out, q, sa, sums);
  else
    hipLaunchKernelGGL(rmsnorm_kernel<1024>, dim3(rows), dim3(1024), lds, s, x, w, (int)dim, eps, out, q, sa, sums);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

// ---------------------------------------------------------------- activations
// silu (norms.rs:27-31) then `g *= u` (infer.rs:197-199), optionally
// quantizing the product for the down projection.
__global__ __launch_bounds__(256) void silu_mul_kernel(float* __restrict__ g, const float* __restrict__ u,
                                                       size_t n, int8_t* __restrict__ q, float* __restrict__ sa,
                                                       int* __restrict__ sums, int gelu) {
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  bool live = i < n;
  float v = live ? g[i] : 0.0f;
  if (gelu) {
    const float kS = 0.7978846f;  // norms.rs:36
    float x3 = v * v * v;
    v = 0.5f * v * (1.0f + dev_tanhf(kS * (v + 0.044715f * x3)));
  } else {
    v = v * (1.0f / (1.0f + dev_expf(-v)));
  }
  if (u) v = v * (live ? u[i] : 0.0f);
  if (live) g[i] = v;
  if (q) {
    float scale;
    int sum;
    int qi = quantize_lane(v, &scale, &sum);
    if (live) {
      q[i] = static_cast<int8_t>(qi);
      if ((i & 31) == 0) {
        sa[i >> 5] = scale;
        sums[i >> 5] = sum;
      }
    }
  }
}

int launch_act_mul(float* g, const float* u, size_t n, int gelu, int8_t* q, float* sa, int* sums, hipStream_t s) {
  if (n == 0) return kOk;
  PRANA_CHECK(!q || n % 32 == 0, "act: fused quantize needs n % 32 == 0");
  hipLaunchKernelGGL(silu_mul_kernel, dim3((n + 255) / 256), dim3(256), 0, s, g, u, n, q, sa, sums, gelu);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

// ---------------------------------------------------------------- softmax
// norms.rs:44-56, one workgroup per row; the sum is the sequential fold,
// evaluated exactly by the workgroup.
__global__ __launch_bounds__(256) void softmax_kernel(const float* __restrict__ in, int n, float* __restrict__ out) {
  __shared__ float s_red[4];
  const float* row = in + (size_t)blockIdx.x * n;
  float* dst = out + (size_t)blockIdx.x * n;
  float mx = -INFINITY;
  for (int i = threadIdx.x; i < n; i += 256) mx = fmaxf(mx, row[i]);
  mx = wave_max_f32(mx);
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
  for (int i = threadIdx.x; i < n; i += 256) dst[i] = dev_expf(row[i] - mx);
  __syncthreads();
  const float sum = exact::block_seq_sum_nonneg<256, false>(dst, n);  // norms.rs:53 order
  const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
  for (int i = threadIdx.x; i < n; i += 256) dst[i] = dst[i] * inv;
}

int launch_softmax(const float* in, size_t rows, size_t n, float* out, hipStream_t s) {
  if (rows == 0 || n == 0) return kOk;
  hipLaunchKernelGGL(softmax_kernel, dim3(rows), dim3(256), 0, s, in, (int)n, out);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

// ---------------------------------------------------------------- add
__global__ void add_kernel(float* __restrict__ x, const float* __restrict__ y, size_t n, size_t period) {
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i < n) x[i] = x[i] + y[period ? i % period : i];
}

int launch_add(float* x, const float* y, size_t n, size_t period, hipStream_t s) {
  if (n == 0) return kOk;
  hipLaunchKernelGGL(add_kernel, dim3((n + 255) / 256), dim3(256), 0, s, x, y, n, period);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

// ---------------------------------------------------------------- RoPE
// Pair rotation: see rotate() in common.h. table: [pos][hd/2] float2.

// x: n_rows rows of row_len floats (row_stride apart); row t is at position
// pos0 + t. neox: pairs (j, j + hd/2) per head; else adjacent pairs.
__global__ void rope_kernel(float* __restrict__ x, int n_rows, int row_len, size_t row_stride, int hd,
                            const float2* __restrict__ table, int pos0, int neox) {
  int pairs = row_len / 2;
  size_t gid = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (gid >= (size_t)n_rows * pairs) return;
  int t = static_cast<int>(gid / pairs);
  int p = static_cast<int>(gid % pairs);
  int half = hd / 2;
  float* row = x + t * row_stride;
  const float2* tab = table + (size_t)(pos0 + t) * half;
  int i0, i1, m;
  if (neox) {
    int h = p / half, j = p % half;
    i0 = h * hd + j;
    i1 = i0 + half;
    m = j;
  } else {
    i0 = 2 * p;
    i1 = i0 + 1;
    m = (i0 % hd) / 2;
  }
  rotate(row[i0], row[i1], tab[m]);
}

int launch_rope(float* x, size_t n_rows, size_t row_len, size_t row_stride, size_t hd, const float2* table,
                size_t pos0, int neox, hipStream_t s) {
  size_t n = n_rows * (row_len / 2);
  if (n == 0) return kOk;
  hipLaunchKernelGGL(rope_kernel, dim3((n + 255) / 256), dim3(256), 0, s, x, (int)n_rows, (int)row_len, row_stride,
                     (int)hd, table, (int)pos0, neox);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

// f16_kv_write (attention.rs:47-52): cache[first_row*kv_stride + i] = f16(src[i]).
__global__ void kv_write_kernel(uint16_t* __restrict__ cache, const float* __restrict__ src, size_t n) {
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i < n) cache[i] = f32_to_f16(src[i]);
}

int launch_kv_write(uint16_t* cache, size_t first_row, size_t kv_stride, const float* src, size_t n,
                    hipStream_t s) {
  if (n == 0) return kOk;
  hipLaunchKernelGGL(kv_write_kernel, dim3((n + 255) / 256), dim3(256), 0, s, cache + first_row * kv_stride, src,
                     n);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

// Decode glue after the Q/K/V projections (infer.rs:169-178): rope q and k
// in place at `pos`, then write k and v to the f16 cache row `pos` (K in the
// kcache_index layout of kcap).
__global__ void rope_kv_kernel(float* __restrict__ q, float* __restrict__ k, const float* __restrict__ v,
                               int q_dim, int kv_dim, int hd, const float2* __restrict__ table, int neox,
                               uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int kcap,
                               const int* __restrict__ pos_dev, int pos_host) {
  int pos = pos_dev ? *pos_dev : pos_host;
  int half = hd / 2;
  const float2* tab = table + (size_t)pos * half;
  int qp = q_dim / 2, kp = kv_dim / 2;
  int gid = blockIdx.x * blockDim.x + threadIdx.x;
  if (gid < qp + kp) {
    float* row = gid < qp ? q : k;
    int p = gid < qp ? gid : gid - qp;
    int i0, i1, m;
    if (neox) {
      int h = p / half, j = p % half;
      i0 = h * hd + j;
      i1 = i0 + half;
      m = j;
    } else {
      i0 = 2 * p;
      i1 = i0 + 1;
      m = (i0 % hd) / 2;
    }
    float a = row[i0], b = row[i1];
    rotate(a, b, tab[m]);
    row[i0] = a;
    row[i1] = b;
    if (gid >= qp) {
      kc[kcache_index(pos, i0, kv_dim, kcap)] = f32_to_f16(a);
      kc[kcache_index(pos, i1, kv_dim, kcap)] = f32_to_f16(b);
    }
  } else if (gid < qp + kp + kv_dim) {
    int i = gid - qp - kp;
    vc[(size_t)pos * kv_dim + i] = f32_to_f16(v[i]);
  }
}

// The same for n consecutive token rows (q [n][q_dim], k and v [n][kv_dim])
// at positions pos0..pos0+n-1: the batched passes' RoPE of q and k and their
// f16 cache rows (infer.rs:247-262, 322-338) in one launch.
__global__ void rope_kv_rows_kernel(float* __restrict__ q, float* __restrict__ k, const float* __restrict__ v,
                                    int n, int q_dim, int kv_dim, int hd, const float2* __restrict__ table, int neox,
                                    uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int kcap, int pos0) {
  const int half = hd / 2;
  const int qp = q_dim / 2, kp = kv_dim / 2, per = qp + kp + kv_dim;
  const size_t gid = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (gid >= (size_t)n * per) return;
  const int t = static_cast<int>(gid / per), e = static_cast<int>(gid % per);
  const int pos = pos0 + t;
  if (e < qp + kp) {
    float* row = e < qp ? q + (size_t)t * q_dim : k + (size_t)t * kv_dim;
    const int p = e < qp ? e : e - qp;
    int i0, i1, m;
    if (neox) {
      const int h = p / half, j = p % half;
      i0 = h * hd + j;
      i1 = i0 + half;
      m = j;
    } else {
      i0 = 2 * p;
      i1 = i0 + 1;
      m = (i0 % hd) / 2;
    }
    float a = row[i0], b = row[i1];
    rotate(a, b, table[(size_t)pos * half + m]);
    row[i0] = a;
    row[i1] = b;
    if (e >= qp) {
      kc[kcache_index(pos, i0, kv_dim, kcap)] = f32_to_f16(a);
      kc[kcache_index(pos, i1, kv_dim, kcap)] = f32_to_f16(b);
    }
  } else {
    const int i = e - qp - kp;
    vc[(size_t)pos * kv_dim + i] = f32_to_f16(v[(size_t)t * kv_dim + i]);
  }
}

int launch_rope_kv_rows(float* q, float* k, const float* v, size_t n, size_t q_dim, size_t kv_dim, size_t hd,
                        const float2* table, int neox, uint16_t* kc, uint16_t* vc, size_t kcap, size_t pos0,
                        hipStream_t s) {
  const size_t total = n * (q_dim / 2 + kv_dim / 2 + kv_dim);
  if (total == 0) return kOk;
  PRANA_CHECK(kcap == 0 || (kv_dim % 8 == 0 && pos0 + n <= kcap), "rope_kv_rows: rows beyond the K cache");
  hipLaunchKernelGGL(rope_kv_rows_kernel, dim3((total + 255) / 256), dim3(256), 0, s, q, k, v, (int)n, (int)q_dim,
                     (int)kv_dim, (int)hd, table, neox, kc, vc, (int)kcap, (int)pos0);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

int launch_rope_kv(float* q, float* k, const float* v, size_t q_dim, size_t kv_dim, size_t hd, const float2* table,
                   int neox, uint16_t* kc, uint16_t* vc, size_t kcap, const int* pos_dev, size_t pos_host,
                   hipStream_t s) {
  size_t n = q_dim / 2 + kv_dim / 2 + kv_dim;
  PRANA_CHECK(kcap == 0 || kv_dim % 8 == 0, "rope_kv: a piecewise K cache needs kv_dim % 8 == 0");
  hipLaunchKernelGGL(rope_kv_kernel, dim3((n + 255) / 256), dim3(256), 0, s, q, k, v, (int)q_dim, (int)kv_dim,
                     (int)hd, table, neox, kc, vc, (int)kcap, pos_dev, (int)pos_host);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

// ---------------------------------------------------------------- f16 conversions
__global__ void f32_to_f16_kernel(const float* __restrict__ in, size_t n, uint16_t* __restrict__ out) {
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i < n) out[i] = f32_to_f16(in[i]);
}
__global__ void f16_to_f32_kernel(const uint16_t* __restrict__ in, size_t n, float* __restrict__ out) {
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i < n) out[i] = f16_to_f32(in[i]);
}
__global__ void expf_kernel(const float* __restrict__ in, size_t n, float* __restrict__ out) {
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i < n) out[i] = dev_expf(in[i]);
}
__global__ void tanhf_kernel(const float* __restrict__ in, size_t n, float* __restrict__ out) {
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i < n) out[i] = dev_tanhf(in[i]);
}
// exp over a contiguous range of f32 bit patterns [base, base + n).
__global__ void expf_bits_kernel(uint32_t base, uint32_t n, float* __restrict__ out) {
  uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = dev_expf(__uint_as_float(base + i));
}

int launch_f32_to_f16(const float* in, size_t n, uint16_t* out, hipStream_t s) {
  if (!n) return kOk;
  hipLaunchKernelGGL(f32_to_f16_kernel, dim3((n + 255) / 256), dim3(256), 0, s, in, n, out);
  PRANA_LAUNCH_CHECK();
  return kOk;
}
int launch_f16_to_f32(const uint16_t* in, size_t n, float* out, hipStream_t s) {
  if (!n) return kOk;
  hipLaunchKernelGGL(f16_to_f32_kernel, dim3((n + 255) / 256), dim3(256), 0, s, in, n, out);
  PRANA_LAUNCH_CHECK();
  return kOk;
}
int launch_expf(const float* in, size_t n, float* out, hipStream_t s) {
  if (!n) return kOk;
  hipLaunchKernelGGL(expf_kernel, dim3((n + 255) / 256), dim3(256), 0, s, in, n, out);
  PRANA_LAUNCH_CHECK();
  return kOk;
}
int launch_tanhf(const float* in, size_t n, float* out, hipStream_t s) {
  if (!n) return kOk;
  hipLaunchKernelGGL(tanhf_kernel, dim3((n + 255) / 256), dim3(256), 0, s, in, n, out);
  PRANA_LAUNCH_CHECK();
  return kOk;
}
int launch_expf_bits(uint32_t base, uint32_t n, float* out, hipStream_t s) {
  if (!n) return kOk;
  hipLaunchKernelGGL(expf_bits_kernel, dim3((n + 255) / 256), dim3(256), 0, s, base, n, out);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

// ---------------------------------------------------------------- argmax
// infer.rs:560-568: strict `>` scan, first max wins. A NaN at index 0 pins the
// result to 0; later NaNs never win. Parallel form: per-lane strided scans
// (increasing index, strict >, 32 loads in flight per lane: one pass covers
// 32768 values), then a (value, lowest index) reduction across the workgroup.
constexpr int kArgNT = 1024;
constexpr int kArgPer = 32;  // loads per lane per pass

__device__ __forceinline__ void argmax_merge(float& av, int& aj, float bv, int bj, int n) {
  if (bj < n && (aj >= n || bv > av || (bv == av && bj < aj))) {
    av = bv;
    aj = bj;
  }
}

__global__ __launch_bounds__(kArgNT) void argmax_kernel(const float* __restrict__ v, int n, uint32_t* __restrict__ out) {
  __shared__ float s_v[kArgNT / 64];
  __shared__ int s_i[kArgNT / 64];
  const float* row = v + (size_t)blockIdx.x * n;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float best = -INFINITY;
  int bi = n;  // none
  bool nan0 = false;  // row[0] is NaN (lane 0's first value)
  for (int base = 0; base < n; base += kArgPer * kArgNT) {
    float x[kArgPer];
#pragma unroll
    for (int u = 0; u < kArgPer; u++) x[u] = row[min(base + u * kArgNT + tid, n - 1)];
    if (base == 0 && tid == 0) nan0 = x[0] != x[0];
#pragma unroll
    for (int u = 0; u < kArgPer; u++) {
      const int i = base + u * kArgNT + tid;
      if (i < n && x[u] > best) {
        best = x[u];
        bi = i;
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) argmax_merge(best, bi, __shfl_xor(best, o, 64), __shfl_xor(bi, o, 64), n);
  if (lane == 0) {
    s_v[wave] = best;
    s_i[wave] = bi;
  }
  __syncthreads();
  if (wave == 0) {
    // the 16 waves' results in lanes 0..15, merged by the same rule
    best = lane < kArgNT / 64 ? s_v[lane] : -INFINITY;
    bi = lane < kArgNT / 64 ? s_i[lane] : n;
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) argmax_merge(best, bi, __shfl_xor(best, o, 64), __shfl_xor(bi, o, 64), n);
    if (tid == 0) {
      if (bi >= n || nan0) bi = 0;  // all -inf / NaN, or a NaN at index 0
      out[blockIdx.x] = static_cast<uint32_t>(bi);
    }
  }
}

int launch_argmax(const float* v, size_t rows, size_t n, uint32_t* out, hipStream_t s) {
  if (rows == 0) return kOk;
  PRANA_CHECK(n > 0 && n <= 0x7fffffff, "argmax: row length out of range");
  hipLaunchKernelGGL(argmax_kernel, dim3(rows), dim3(kArgNT), 0, s, v, (int)n, out);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

// One replayed decode step's bookkeeping: state = {position, step}; the
// step's argmax (tok) becomes ids[step + 1], then both counters advance.
__global__ void decode_advance_kernel(int* __restrict__ state, const uint32_t* __restrict__ tok,
                                      uint32_t* __restrict__ ids) {
  if (threadIdx.x == 0) {
    const int step = state[1];
    ids[step + 1] = tok[0];
    state[0] += 1;
    state[1] = step + 1;
  }
}

int launch_decode_advance(int* state, const uint32_t* tok, uint32_t* ids, hipStream_t s) {
  hipLaunchKernelGGL(decode_advance_kernel, dim3(1), dim3(64), 0, s, state, tok, ids);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

// Seeds a decode run: state = {pos, 0}; the first step's token goes to
// ids[0] and to tok0 (the embedding input of a replayed step). Values are
// kernel arguments, so no host buffer has to outlive the call.
__global__ void decode_seed_kernel(int* __restrict__ state, int pos, uint32_t token, uint32_t* __restrict__ ids,
                                   uint32_t* __restrict__ tok0) {
  if (threadIdx.x == 0) {
    if (state) {
      state[0] = pos;
      state[1] = 0;
    }
    if (ids) ids[0] = token;
    if (tok0) tok0[0] = token;
  }
}

int launch_decode_seed(int* state, int pos, uint32_t token, uint32_t* ids, uint32_t* tok0, hipStream_t s) {
  hipLaunchKernelGGL(decode_seed_kernel, dim3(1), dim3(64), 0, s, state, pos, token, ids, tok0);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

// The accept walk of one speculative round (infer.rs:648-681) on the device:
// the target's tokens tnext[0..budget] are emitted while each agrees with the
// draft's; a stop token ends the run unemitted, the step and position limits
// end it after the token that reaches them. res = {emitted, accepted, done},
// then the emitted tokens.
__global__ void spec_accept_kernel(const uint32_t* __restrict__ drafts, const uint32_t* __restrict__ tnext,
                                   int budget, const uint32_t* __restrict__ stops, int n_stops, long long generated,
                                   long long steps, long long pos, long long max_pos, int* __restrict__ res) {
  if (threadIdx.x != 0) return;
  int n = 0, acc = 0, done = 0;
  uint32_t* out = reinterpret_cast<uint32_t*>(res + 3);
  for (int i = 0; i <= budget; i++) {
    const uint32_t tn = tnext[i];
    if (i < budget && tn == drafts[i]) acc++;
    bool stop = false;
    for (int j = 0; j < n_stops; j++) stop |= stops[j] == tn;
    if (stop) {
      done = 1;
      break;
    }
    out[n++] = tn;
    generated++;
    pos++;
    if (generated >= steps || pos + 1 >= max_pos) {
      done = 1;
      break;
    }
    if (i == budget || tn != drafts[i]) break;
  }
  res[0] = n;
  res[1] = acc;
  res[2] = done;
}

int launch_spec_accept(const uint32_t* drafts, const uint32_t* tnext, int budget, const uint32_t* stops, int n_stops,
                       size_t generated, size_t steps, size_t pos, size_t max_pos, int* res, hipStream_t s) {
  hipLaunchKernelGGL(spec_accept_kernel, dim3(1), dim3(64), 0, s, drafts, tnext, budget, stops, n_stops,
                     static_cast<long long>(generated), static_cast<long long>(steps), static_cast<long long>(pos),
                     static_cast<long long>(max_pos), res);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

// ---------------------------------------------------------------- embedding
// Embedding::row (checkpoint.rs:169-174): dense copy, or one row of a packed
// table dequantized (kquant.rs:39-112; Q8_0 tables are f32 rows q*d as
// gguf.rs:234-245 produces), then `x *= emb_scale` when it is not 1
// (infer.rs:155-159).
__device__ float dequant_elem(const DevMat& m, size_t r, int c) {
  switch (m.kind) {
    case kKindF32:
      return reinterpret_cast<const float*>(m.qs)[r * m.cols + c];
    case kKindQ8F: {
      const int8_t* q = reinterpret_cast<const int8_t*>(m.qs);
      const float* sc = reinterpret_cast<const float*>(m.sc);
      return static_cast<float>(q[r * m.cols + c]) * sc[r * (m.cols / 32) + c / 32];
    }
    case kKindQ8_0: {
      const int8_t* q = reinterpret_cast<const int8_t*>(m.qs);
      const uint16_t* sc = reinterpret_cast<const uint16_t*>(m.sc);
      return static_cast<float>(q[r * m.cols + c]) * f16_to_f32(sc[r * (m.cols / 32) + c / 32]);
    }
    case kKindQ4_0: {
      size_t G = m.cols / 32;
      size_t b = c / 32;
      int j = c % 32;
      const uint8_t* blk = m.qs + (r * G + b) * 16;
      float d = f16_to_f32(reinterpret_cast<const uint16_t*>(m.sc)[r * G + b]);
      int nib = j < 16 ? (blk[j] & 0xF) : (blk[j - 16] >> 4);
      return d * (static_cast<float>(nib) - 8.0f);
    }
    case kKindQ4_K: {
      size_t nb = m.cols / 256;
      const uint8_t* b = m.qs + (r * nb + c / 256) * 144;
      int e = c % 256;
      int pair = e / 64, hi = (e % 64) / 32, l = e % 32;
      float d = f16_to_f32(static_cast<uint16_t>(b[0] | (b[1] << 8)));
      float dmin = f16_to_f32(static_cast<uint16_t>(b[2] | (b[3] << 8)));
      const uint8_t* s = b + 4;
      int j = pair * 2 + hi;
      float sc, mn;
      if (j < 4) {
        sc = static_cast<float>(s[j] & 63);
        mn = static_cast<float>(s[j + 4] & 63);
      } else {
        sc = static_cast<float>((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
        mn = static_cast<float>((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
      }
      uint8_t byte = b[16 + pair * 32 + l];
      int nib = hi ? (byte >> 4) : (byte & 0xF);
      float d1 = d * sc, m1 = dmin * mn;
      return d1 * static_cast<float>(nib) - m1;
    }
    case kKindQ6_K: {
      size_t nb = m.cols / 256;
      const uint8_t* b = m.qs + (r * nb + c / 256) * 208;
      float d = f16_to_f32(reinterpret_cast<const uint16_t*>(m.sc)[r * nb + c / 256]);
      int e = c % 256;
      int half = e / 128, rem = e % 128, g = rem / 32, l = rem % 32;
      const uint8_t* ql = b + half * 64;
      const uint8_t* qh = b + 128 + half * 32;
      const int8_t* sc = reinterpret_cast<const int8_t*>(b + 192);
      int qlb = ql[l + (g & 1) * 32];
      int nib = g < 2 ? (qlb & 0xF) : (qlb >> 4);
      int hb = (qh[l] >> (2 * g)) & 3;
      int qv = static_cast<int>(static_cast<int8_t>(nib | (hb << 4))) - 32;
      int is = half * 8 + l / 16 + 2 * g;
      return d * static_cast<float>(sc[is]) * static_cast<float>(qv);
    }
  }
  return 0.0f;
}

__global__ void embed_kernel(DevMat m, const uint32_t* __restrict__ tokens, float scale, float* __restrict__ out) {
  int c = blockIdx.x * blockDim.x + threadIdx.x;
  int t = blockIdx.y;
  if (c >= (int)m.cols) return;
  size_t r = tokens[t];
  if (r >= m.rows) r = 0;  // out-of-vocabulary ids are rejected on the host
  float v = dequant_elem(m, r, c);
  if (scale != 1.0f) v = v * scale;
  out[(size_t)t * m.cols + c] = v;
}

int launch_embed(const DevMat& m, const uint32_t* tokens, size_t n, float scale, float* out, hipStream_t s) {
  if (n == 0) return kOk;
  hipLaunchKernelGGL(embed_kernel, dim3((m.cols + 255) / 256, n), dim3(256), 0, s, m, tokens, scale, out);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

}  // namespace prana
