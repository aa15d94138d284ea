// Causal grouped-query attention in the reference's exact evaluation order
// (decode_one_head, attention.rs:165-195; prefill `attention`, 236-284):
//   score_t = (fold_d q[d]*k_t[d] from -0.0) * (1/sqrt(hd))      parallel over t
//   softmax: max (order-free), e_t = expf(score_t - max),
//            sum = fold_t e_t (one lane), p_t = e_t * (1/sum)
//   out[d]  = fold_t p_t * v_t[d] from 0.0                     parallel over d
// One workgroup per (query row, head).
#include "common.h"
#include "kernels.h"

namespace prana {

namespace {

template <bool F16>
struct KvSrc;
template <>
struct KvSrc<true> {
  const uint16_t* k;
  const uint16_t* v;
  __device__ float kval(size_t i) const { return f16_to_f32(k[i]); }
  __device__ float vval(size_t i) const { return f16_to_f32(v[i]); }
};
template <>
struct KvSrc<false> {
  const float* k;
  const float* v;
  __device__ float kval(size_t i) const { return k[i]; }
  __device__ float vval(size_t i) const { return v[i]; }
};

// q_row: this query row (n_heads*hd); pos: its absolute position; scores:
// scratch of pos+1 floats owned by this workgroup.
template <bool F16>
__device__ void one_head(const float* __restrict__ q_row, KvSrc<F16> kv, int pos, int h, int group, int kv_stride,
                         int hd, float* __restrict__ dst, float* __restrict__ scores) {
  __shared__ float s_q[256];
  __shared__ float s_red[4];
  __shared__ float s_inv;
  const int kvh = h / group;
  const float scale = 1.0f / sqrtf(static_cast<float>(hd));
  for (int d = threadIdx.x; d < hd; d += blockDim.x) s_q[d] = q_row[h * hd + d];
  __syncthreads();
  float mx = -INFINITY;
  for (int t = threadIdx.x; t <= pos; t += blockDim.x) {
    size_t base = (size_t)t * kv_stride + (size_t)kvh * hd;
    float dot = -0.0f;
    for (int d = 0; d < hd; d++) dot += s_q[d] * kv.kval(base + d);
    float sc = dot * scale;
    scores[t] = sc;
    mx = fmaxf(mx, sc);
  }
  mx = wave_max_f32(mx);
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
  for (int t = threadIdx.x; t <= pos; t += blockDim.x) scores[t] = dev_expf(scores[t] - mx);
  __syncthreads();
  if (threadIdx.x == 0) {
    float sum = -0.0f;
    for (int t = 0; t <= pos; t++) sum += scores[t];
    s_inv = sum > 0.0f ? 1.0f / sum : 0.0f;
  }
  __syncthreads();
  const float inv = s_inv;
  for (int t = threadIdx.x; t <= pos; t += blockDim.x) scores[t] = scores[t] * inv;
  __syncthreads();
  for (int d = threadIdx.x; d < hd; d += blockDim.x) {
    float acc = 0.0f;
    size_t base = (size_t)kvh * hd + d;
    for (int t = 0; t <= pos; t++) acc += scores[t] * kv.vval(base + (size_t)t * kv_stride);
    dst[h * hd + d] = acc;
  }
}

// grid: (n_heads, n_q). Row i attends to cache rows 0..=pos0+i.
__global__ __launch_bounds__(256) void attn_cache_kernel(const float* __restrict__ q, const uint16_t* __restrict__ kc,
                                                         const uint16_t* __restrict__ vc, int pos0, int n_heads,
                                                         int group, int hd, float* __restrict__ out,
                                                         float* __restrict__ scratch, int ctx_cap,
                                                         const int* __restrict__ pos_dev) {
  const int h = blockIdx.x, i = blockIdx.y;
  const int p0 = pos_dev ? *pos_dev : pos0;
  const int q_stride = n_heads * hd;
  const int kv_stride = (n_heads / group) * hd;
  KvSrc<true> kv{kc, vc};
  one_head<true>(q + (size_t)i * q_stride, kv, p0 + i, h, group, kv_stride, hd, out + (size_t)i * q_stride,
                 scratch + ((size_t)i * n_heads + h) * ctx_cap);
}

__global__ __launch_bounds__(256) void attn_prefill_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                           const float* __restrict__ v, int seq, int n_heads,
                                                           int group, int hd, float* __restrict__ out,
                                                           float* __restrict__ scratch) {
  const int h = blockIdx.x, i = blockIdx.y;
  const int q_stride = n_heads * hd;
  const int kv_stride = (n_heads / group) * hd;
  KvSrc<false> kv{k, v};
  one_head<false>(q + (size_t)i * q_stride, kv, i, h, group, kv_stride, hd, out + (size_t)i * q_stride,
                  scratch + ((size_t)i * n_heads + h) * seq);
}

}  // namespace

int launch_attention_cache(const float* q, const uint16_t* kc, const uint16_t* vc, size_t pos0, size_t n_q,
                           size_t n_heads, size_t n_kv_heads, size_t hd, float* out, float* scratch, size_t ctx_cap,
                           const int* pos_dev, hipStream_t s) {
  if (n_q == 0) return kOk;
  PRANA_CHECK(n_kv_heads > 0 && n_heads % n_kv_heads == 0, "attention: n_heads must be a multiple of n_kv_heads");
  PRANA_CHECK(hd > 0 && hd <= 256, "attention: head_dim must be in 1..=256");
  if (ctx_cap == 0) ctx_cap = pos0 + n_q;
  PRANA_CHECK(pos_dev || pos0 + n_q <= ctx_cap, "attention: scratch capacity below pos0 + n_q");
  hipLaunchKernelGGL(attn_cache_kernel, dim3(n_heads, n_q), dim3(256), 0, s, q, kc, vc, (int)pos0, (int)n_heads,
                     (int)(n_heads / n_kv_heads), (int)hd, out, scratch, (int)ctx_cap, pos_dev);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

int launch_attention_prefill(const float* q, const float* k, const float* v, size_t seq, size_t n_heads,
                             size_t n_kv_heads, size_t hd, float* out, float* scratch, hipStream_t s) {
  if (seq == 0) return kOk;
  PRANA_CHECK(n_kv_heads > 0 && n_heads % n_kv_heads == 0, "attention: n_heads must be a multiple of n_kv_heads");
  PRANA_CHECK(hd > 0 && hd <= 256, "attention: head_dim must be in 1..=256");
  hipLaunchKernelGGL(attn_prefill_kernel, dim3(n_heads, seq), dim3(256), 0, s, q, k, v, (int)seq, (int)n_heads,
                     (int)(n_heads / n_kv_heads), (int)hd, out, scratch);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

}  // namespace prana
