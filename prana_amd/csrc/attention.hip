// Causal grouped-query attention in the reference's exact evaluation order
// (decode_one_head, attention.rs:165-195; prefill `attention`, 236-284):
//   score_t = (fold_d q[d]*k_t[d] from -0.0) * (1/sqrt(hd))      parallel over t
//   softmax: max (order-free), e_t = expf(score_t - max),
//            sum = fold_t e_t (the sequential fold, evaluated exactly by
//            the whole workgroup), p_t = e_t * (1/sum)
//   out[d]  = fold_t p_t * v_t[d] from 0.0                     parallel over d
// One workgroup per (query row, head).
#include "common.h"
#include "exact_sum.h"
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

// Dot of q (LDS) with one K row, folded left to right from -0.0. HD > 0: the
// head width is a compile-time constant, the row start is 16-byte aligned and
// the row is fetched with 16-byte loads (f16: whole row in flight, HD/2 VGPRs;
// f32: 32-wide chunks) before the chain; HD == 0: runtime width.
template <int HD, bool F16>
__device__ __forceinline__ float row_dot(const float* s_q, KvSrc<F16> kv, size_t base, int hd) {
  float dot = -0.0f;
  if constexpr (HD > 0 && F16) {
    static_assert(HD % 8 == 0, "f16 rows load 8 halves at a time");
    uint4 raw[HD / 8];
    const uint4* p = reinterpret_cast<const uint4*>(kv.k + base);
#pragma unroll
    for (int i = 0; i < HD / 8; i++) raw[i] = p[i];
#pragma unroll
    for (int i = 0; i < HD / 8; i++) {
      const uint32_t w[4] = {raw[i].x, raw[i].y, raw[i].z, raw[i].w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        dot += s_q[8 * i + 2 * j] * f16_to_f32(static_cast<uint16_t>(w[j] & 0xffffu));
        dot += s_q[8 * i + 2 * j + 1] * f16_to_f32(static_cast<uint16_t>(w[j] >> 16));
      }
    }
  } else if constexpr (HD > 0) {
    static_assert(HD % 16 == 0, "f32 rows load in chunks of 16");
    const float4* p = reinterpret_cast<const float4*>(kv.k + base);
#pragma unroll
    for (int c = 0; c < HD / 16; c++) {
      float4 raw[4];
#pragma unroll
      for (int i = 0; i < 4; i++) raw[i] = p[4 * c + i];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int d = 16 * c + 4 * i;
        dot += s_q[d] * raw[i].x;
        dot += s_q[d + 1] * raw[i].y;
        dot += s_q[d + 2] * raw[i].z;
        dot += s_q[d + 3] * raw[i].w;
      }
    }
  } else {
    for (int d = 0; d < hd; d++) dot += s_q[d] * kv.kval(base + d);
  }
  return dot;
}

// q_row: this query row (n_heads*hd); pos: its absolute position; scores:
// scratch of pos+1 floats owned by this workgroup.
template <int HD, bool F16>
__device__ void one_head(const float* __restrict__ q_row, KvSrc<F16> kv, int pos, int h, int group, int kv_stride,
                         int hd, float* __restrict__ dst, float* __restrict__ scores) {
  __shared__ float s_q[256];
  __shared__ float s_red[4];
  const int kvh = h / group;
  const float scale = 1.0f / sqrtf(static_cast<float>(hd));
  for (int d = threadIdx.x; d < hd; d += blockDim.x) s_q[d] = q_row[h * hd + d];
  __syncthreads();
  float mx = -INFINITY;
  for (int t = threadIdx.x; t <= pos; t += blockDim.x) {
    float sc = row_dot<HD, F16>(s_q, kv, (size_t)t * kv_stride + (size_t)kvh * hd, hd) * scale;
    scores[t] = sc;
    mx = fmaxf(mx, sc);
  }
  mx = wave_max_f32(mx);
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
  for (int t = threadIdx.x; t <= pos; t += blockDim.x) scores[t] = dev_expf(scores[t] - mx);
  __syncthreads();
  // softmax sum in the reference's left-to-right order (norms.rs:53)
  const float sum = exact::block_seq_sum_nonneg(scores, pos + 1);
  const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
  for (int t = threadIdx.x; t <= pos; t += blockDim.x) scores[t] = scores[t] * inv;
  __syncthreads();
  for (int d = threadIdx.x; d < hd; d += blockDim.x) {
    float acc = 0.0f;
    const size_t base = (size_t)kvh * hd + d;
    int t = 0;
    for (; t + 8 <= pos + 1; t += 8) {  // 8 loads in flight ahead of the chain
      float v[8], p[8];
#pragma unroll
      for (int j = 0; j < 8; j++) {
        v[j] = kv.vval(base + (size_t)(t + j) * kv_stride);
        p[j] = scores[t + j];
      }
#pragma unroll
      for (int j = 0; j < 8; j++) acc += p[j] * v[j];
    }
    for (; t <= pos; t++) acc += scores[t] * kv.vval(base + (size_t)t * kv_stride);
    dst[h * hd + d] = acc;
  }
}

// vec_hd: the compiled head width when K is 16-byte aligned at every row
// start (checked on the host), else 0 for the generic path.
template <bool F16, class KV>
__device__ void one_head_dispatch(const float* q_row, KV kv, int pos, int h, int group, int kv_stride, int hd,
                                  int vec_hd, float* dst, float* scores) {
  switch (vec_hd) {
    case 48: one_head<48, F16>(q_row, kv, pos, h, group, kv_stride, hd, dst, scores); break;
    case 64: one_head<64, F16>(q_row, kv, pos, h, group, kv_stride, hd, dst, scores); break;
    case 128: one_head<128, F16>(q_row, kv, pos, h, group, kv_stride, hd, dst, scores); break;
    default: one_head<0, F16>(q_row, kv, pos, h, group, kv_stride, hd, dst, scores); break;
  }
}

// Head widths with a compiled row loader, used when every K row start is
// 16-byte aligned (base pointer aligned and hd a multiple of the vector).
int pick_vec_hd(const void* k, size_t hd, size_t elem) {
  if (reinterpret_cast<uintptr_t>(k) % 16 != 0) return 0;
  if ((hd * elem) % 16 != 0 || (elem == 4 && hd % 16 != 0)) return 0;
  return (hd == 48 || hd == 64 || hd == 128) ? static_cast<int>(hd) : 0;
}

// grid: (n_heads, n_q). Row i attends to cache rows 0..=pos0+i.
__global__ __launch_bounds__(256) void attn_cache_kernel(const float* __restrict__ q, const uint16_t* __restrict__ kc,
                                                         const uint16_t* __restrict__ vc, int pos0, int n_heads,
                                                         int group, int hd, float* __restrict__ out,
                                                         float* __restrict__ scratch, int ctx_cap,
                                                         const int* __restrict__ pos_dev, int vec_hd) {
  const int h = blockIdx.x, i = blockIdx.y;
  const int p0 = pos_dev ? *pos_dev : pos0;
  const int q_stride = n_heads * hd;
  const int kv_stride = (n_heads / group) * hd;
  KvSrc<true> kv{kc, vc};
  one_head_dispatch<true>(q + (size_t)i * q_stride, kv, p0 + i, h, group, kv_stride, hd, vec_hd,
                          out + (size_t)i * q_stride, scratch + ((size_t)i * n_heads + h) * ctx_cap);
}

__global__ __launch_bounds__(256) void attn_prefill_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                           const float* __restrict__ v, int seq, int n_heads,
                                                           int group, int hd, float* __restrict__ out,
                                                           float* __restrict__ scratch, int vec_hd) {
  const int h = blockIdx.x, i = blockIdx.y;
  const int q_stride = n_heads * hd;
  const int kv_stride = (n_heads / group) * hd;
  KvSrc<false> kv{k, v};
  one_head_dispatch<false>(q + (size_t)i * q_stride, kv, i, h, group, kv_stride, hd, vec_hd, out + (size_t)i * q_stride,
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
                     (int)(n_heads / n_kv_heads), (int)hd, out, scratch, (int)ctx_cap, pos_dev,
                     pick_vec_hd(kc, hd, 2));
  PRANA_LAUNCH_CHECK();
  return kOk;
}

int launch_attention_prefill(const float* q, const float* k, const float* v, size_t seq, size_t n_heads,
                             size_t n_kv_heads, size_t hd, float* out, float* scratch, hipStream_t s) {
  if (seq == 0) return kOk;
  PRANA_CHECK(n_kv_heads > 0 && n_heads % n_kv_heads == 0, "attention: n_heads must be a multiple of n_kv_heads");
  PRANA_CHECK(hd > 0 && hd <= 256, "attention: head_dim must be in 1..=256");
  hipLaunchKernelGGL(attn_prefill_kernel, dim3(n_heads, seq), dim3(256), 0, s, q, k, v, (int)seq, (int)n_heads,
                     (int)(n_heads / n_kv_heads), (int)hd, out, scratch, pick_vec_hd(k, hd, 4));
  PRANA_LAUNCH_CHECK();
  return kOk;
}

}  // namespace prana
