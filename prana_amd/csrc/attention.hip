// Causal grouped-query attention in the reference's exact evaluation order
// (decode_one_head, attention.rs:165-195; prefill `attention`, 236-284):
//   score_t = (fold_d q[d]*k_t[d] from -0.0) * (1/sqrt(hd))      parallel over t
//   softmax: max (order-free), e_t = expf(score_t - max),
//            sum = fold_t e_t (the sequential fold, evaluated exactly by
//            the whole workgroup), p_t = e_t * (1/sum)
//   out[d]  = fold_t p_t * v_t[d] from 0.0                     parallel over d
//
// One workgroup per (query row, head, slice of head dims). Every slice
// recomputes the head's probabilities (K rows are shared through L2: the
// slices and the heads of one KV group are placed on the same XCD) and then
// folds its own dims; V rows of the slice stream through LDS in chunks that
// are fetched with 16-byte loads one chunk ahead of the fold.
#include "common.h"
#include "exact_sum.h"
#include "kernels.h"

namespace prana {

namespace {

constexpr int kNT = 256;             // lanes per workgroup
constexpr int kScoreLds = 4096;      // probabilities kept in LDS up to this length
constexpr int kVChunkBytes = 16384;  // V slice bytes per LDS chunk
constexpr int kVLoads = kVChunkBytes / 16 / kNT;  // 16-byte loads per lane per chunk

template <bool F16>
struct Elem;
template <>
struct Elem<true> {
  using T = uint16_t;
  static __device__ float get(T v) { return f16_to_f32(v); }
};
template <>
struct Elem<false> {
  using T = float;
  static __device__ float get(T v) { return v; }
};

// Dot of q (LDS) with one K row, folded left to right from -0.0. HD > 0: the
// head width is a compile-time constant, the row start is 16-byte aligned and
// the row is fetched with 16-byte loads before the chain; HD == 0: runtime
// width, scalar loads.
template <int HD, bool F16>
__device__ __forceinline__ float row_dot(const float* s_q, const typename Elem<F16>::T* krow, int hd) {
  float dot = -0.0f;
  if constexpr (HD > 0 && F16) {
    static_assert(HD % 8 == 0, "f16 rows load 8 halves at a time");
    uint4 raw[HD / 8];
    const uint4* p = reinterpret_cast<const uint4*>(krow);
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
    const float4* p = reinterpret_cast<const float4*>(krow);
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
    for (int d = 0; d < hd; d++) dot += s_q[d] * Elem<F16>::get(krow[d]);
  }
  return dot;
}

struct HeadJob {
  const float* q_row;  // this query row (n_heads*hd)
  const void* k;       // K rows (kv_stride elements apart)
  const void* v;
  int pos;  // absolute position: attends to rows 0..=pos
  int h, kvh, kv_stride, hd;
  int d0, dw;        // dims folded by this workgroup
  float* dst;        // output row (n_heads*hd)
  float* gscores;    // global scratch of >= pos+1 floats (used beyond kScoreLds)
  bool vec;          // 16-byte aligned rows: V streams through LDS chunks
};

struct Lds {
  float* q;       // hd floats
  float* red;     // kNT/64 floats
  float* scores;  // kScoreLds floats
  uint4* v;       // kVChunkBytes
};

// V chunk: rows [t0, t0+nr) of dims [d0, d0+dw), packed row-major in LDS.
// Lane i fetches 16-byte piece p = i + kNT*j of the chunk; pieces past the
// chunk re-read its first row (in bounds) and are not stored.
struct VRegs {
  uint4 r0, r1, r2, r3;
};
static_assert(kVLoads == 4, "VRegs holds four pieces per lane");

template <bool F16>
__device__ __forceinline__ VRegs fetch_v(const HeadJob& J, int t0, int nr) {
  using T = typename Elem<F16>::T;
  constexpr int EPV = 16 / sizeof(T);  // elements per 16-byte piece
  const int ppr = J.dw / EPV;          // pieces per row
  const T* base = static_cast<const T*>(J.v) + (size_t)J.kvh * J.hd + J.d0 + (size_t)t0 * J.kv_stride;
  auto piece = [&](int j) {
    const int p = threadIdx.x + kNT * j;
    int row = p / ppr, col = p % ppr;
    if (row >= nr) row = 0;
    return *reinterpret_cast<const uint4*>(base + (size_t)row * J.kv_stride + col * EPV);
  };
  VRegs r;
  r.r0 = piece(0);
  r.r1 = piece(1);
  r.r2 = piece(2);
  r.r3 = piece(3);
  return r;
}

template <bool F16>
__device__ __forceinline__ void store_v(uint4* s_v, int nr, int dw, const VRegs& r) {
  using T = typename Elem<F16>::T;
  const int lim = nr * (dw / (16 / static_cast<int>(sizeof(T))));  // pieces in the chunk
  const int p = threadIdx.x;
  if (p < lim) s_v[p] = r.r0;
  if (p + kNT < lim) s_v[p + kNT] = r.r1;
  if (p + 2 * kNT < lim) s_v[p + 2 * kNT] = r.r2;
  if (p + 3 * kNT < lim) s_v[p + 3 * kNT] = r.r3;
}

// Scores of rows 0..n into sc; returns the workgroup-wide max (every lane).
template <int HD, bool F16>
__device__ __forceinline__ float head_scores(const HeadJob& J, const Lds& L, float* sc) {
  using T = typename Elem<F16>::T;
  const int tid = threadIdx.x;
  const int n = J.pos + 1;
  const int hd = HD > 0 ? HD : J.hd;
  const float scale = 1.0f / sqrtf(static_cast<float>(hd));
  const T* kb = static_cast<const T*>(J.k) + (size_t)J.kvh * hd;
  float mx = -INFINITY;
  for (int t = tid; t < n; t += kNT) {
    float s = row_dot<HD, F16>(L.q, kb + (size_t)t * J.kv_stride, hd) * scale;
    sc[t] = s;
    mx = fmaxf(mx, s);
  }
  return mx;
}

template <bool F16>
__device__ __forceinline__ void one_head(const HeadJob& J, int vec_hd, const Lds& L) {
  using T = typename Elem<F16>::T;
  const int tid = threadIdx.x;
  const int n = J.pos + 1;
  float* sc = n <= kScoreLds ? L.scores : J.gscores;
  for (int d = tid; d < J.hd; d += kNT) L.q[d] = J.q_row[J.h * J.hd + d];
  __syncthreads();
  float mx;
  switch (vec_hd) {
    case 48: mx = head_scores<48, F16>(J, L, sc); break;
    case 64: mx = head_scores<64, F16>(J, L, sc); break;
    case 128: mx = head_scores<128, F16>(J, L, sc); break;
    default: mx = head_scores<0, F16>(J, L, sc); break;
  }
  mx = wave_max_f32(mx);
  if ((tid & 63) == 0) L.red[tid >> 6] = mx;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kNT / 64; w++) mx = fmaxf(mx, L.red[w]);
  for (int t = tid; t < n; t += kNT) sc[t] = dev_expf(sc[t] - mx);
  const bool in_lds = n <= kScoreLds;
  if (in_lds)  // zero fill for the single-lane fold
    for (int t = n + tid; t < exact::lane_pad(n); t += kNT) sc[t] = 0.0f;
  __syncthreads();
  // softmax sum in the reference's left-to-right order (norms.rs:53)
  const float sum = in_lds ? exact::block_seq_sum_nonneg<kNT, true>(sc, n)
                           : exact::block_seq_sum_nonneg<kNT, false>(sc, n);
  const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
  for (int t = tid; t < n; t += kNT) sc[t] = sc[t] * inv;
  __syncthreads();

  // ---- PV over dims [d0, d0+dw): lane d folds dim d0 + d
  const int d = tid;
  const bool folder = d < J.dw;
  float acc = 0.0f;
  if (J.vec) {
    const int rows_per_chunk = kVChunkBytes / (J.dw * static_cast<int>(sizeof(T)));
    const T* s_vt = reinterpret_cast<const T*>(L.v);
    int t0 = 0;
    VRegs r = fetch_v<F16>(J, t0, min(rows_per_chunk, n - t0));
    while (t0 < n) {
      const int nr = min(rows_per_chunk, n - t0);
      store_v<F16>(L.v, nr, J.dw, r);
      __syncthreads();
      const int t1 = t0 + nr;
      if (t1 < n) r = fetch_v<F16>(J, t1, min(rows_per_chunk, n - t1));  // in flight during the fold
      if (folder) {
        int i = 0;
        for (; i + 8 <= nr; i += 8) {
          float vv[8], pp[8];
#pragma unroll
          for (int j = 0; j < 8; j++) {
            vv[j] = Elem<F16>::get(s_vt[(i + j) * J.dw + d]);
            pp[j] = sc[t0 + i + j];
          }
#pragma unroll
          for (int j = 0; j < 8; j++) acc += pp[j] * vv[j];
        }
        for (; i < nr; i++) acc += sc[t0 + i] * Elem<F16>::get(s_vt[i * J.dw + d]);
      }
      __syncthreads();
      t0 = t1;
    }
  } else if (folder) {
    const T* vb = static_cast<const T*>(J.v) + (size_t)J.kvh * J.hd + J.d0 + d;
    for (int t = 0; t < n; t++) acc += sc[t] * Elem<F16>::get(vb[(size_t)t * J.kv_stride]);
  }
  if (folder) J.dst[J.h * J.hd + J.d0 + d] = acc;
}

// blockIdx.x -> (head, dim slice). When the count divides by the 8 XCDs,
// consecutive logical blocks (the slices of one head, then the heads of one
// KV group) land on one XCD, so they share its L2 for K and V.
__device__ __forceinline__ int logical_block(int nb) {
  const int b = blockIdx.x;
  if (nb % 8 != 0) return b;
  return (b % 8) * (nb / 8) + b / 8;
}

// grid: (n_heads*dsplit, n_q). Query row i sits at position p0 + i.
// mode: 0 scalar rows; -1 vector V chunks with a runtime head width;
// 48/64/128 vector K and V loads with that compiled head width.
template <bool F16>
__global__ __launch_bounds__(kNT) void attn_kernel(const float* __restrict__ q, const void* __restrict__ k,
                                                   const void* __restrict__ v, int pos0,
                                                   const int* __restrict__ pos_dev, int n_heads, int group, int hd,
                                                   int dsplit, float* __restrict__ out, float* __restrict__ scratch,
                                                   int scratch_stride, int mode) {
  __shared__ float s_q[256];
  __shared__ float s_red[kNT / 64];
  __shared__ __align__(16) float s_scores[exact::lane_pad(kScoreLds)];
  __shared__ uint4 s_v[kVChunkBytes / 16];
  const int lb = logical_block(n_heads * dsplit);
  const int h = lb / dsplit, ds = lb % dsplit, i = blockIdx.y;
  const int p0 = pos_dev ? *pos_dev : pos0;
  HeadJob J;
  J.q_row = q + (size_t)i * n_heads * hd;
  J.k = k;
  J.v = v;
  J.pos = p0 + i;
  J.h = h;
  J.kvh = h / group;
  J.kv_stride = (n_heads / group) * hd;
  J.hd = hd;
  J.dw = hd / dsplit;
  J.d0 = ds * J.dw;
  J.dst = out + (size_t)i * n_heads * hd;
  J.gscores = scratch ? scratch + ((size_t)i * n_heads * dsplit + lb) * scratch_stride : nullptr;
  J.vec = mode != 0;
  Lds L{s_q, s_red, s_scores, s_v};
  one_head<F16>(J, mode, L);
}

template <bool F16>
int launch_attn(const float* q, const void* k, const void* v, size_t pos0, const int* pos_dev, size_t n_q,
                size_t n_heads, size_t n_kv_heads, size_t hd, float* out, float* scratch, size_t ctx_cap,
                hipStream_t s) {
  const size_t elem = F16 ? 2 : 4;
  const bool aligned = reinterpret_cast<uintptr_t>(k) % 16 == 0 && reinterpret_cast<uintptr_t>(v) % 16 == 0 &&
                       (hd * elem) % 16 == 0;
  int mode = 0;
  if (aligned) {
    const bool compiled = (hd == 48 || hd == 64 || hd == 128) && (F16 || hd % 16 == 0);
    mode = compiled ? static_cast<int>(hd) : -1;
  }
  const int ds = attention_dim_slices(n_q, n_heads, hd, elem, aligned);
  PRANA_CHECK(ctx_cap <= static_cast<size_t>(kScoreLds) || scratch != nullptr,
              "attention: contexts beyond 4096 positions need score scratch");
  hipLaunchKernelGGL(attn_kernel<F16>, dim3(n_heads * ds, n_q), dim3(kNT), 0, s, q, k, v, (int)pos0, pos_dev,
                     (int)n_heads, (int)(n_heads / n_kv_heads), (int)hd, ds, out, scratch, (int)ctx_cap, mode);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

}  // namespace

// Dim slices per head: enough workgroups to keep the V stream parallel when
// there are few (query row, head) pairs; each slice stays a whole number of
// 16-byte pieces wide.
int attention_dim_slices(size_t n_q, size_t n_heads, size_t hd, size_t elem, bool aligned) {
  if (!aligned) return 1;
  int ds = 1;
  while (n_q * n_heads * ds < 128 && ds < 4 && hd % (2 * ds) == 0 && (hd / (2 * ds)) * elem % 16 == 0) ds *= 2;
  return ds;
}

size_t attention_scratch_floats(size_t n_q, size_t n_heads, size_t ctx_cap) {
  if (ctx_cap <= static_cast<size_t>(kScoreLds)) return 0;
  size_t ds = 1;  // upper bound of attention_dim_slices
  while (n_q * n_heads * ds < 128 && ds < 4) ds *= 2;
  return n_q * n_heads * ds * ctx_cap;
}

int launch_attention_cache(const float* q, const uint16_t* kc, const uint16_t* vc, size_t pos0, size_t n_q,
                           size_t n_heads, size_t n_kv_heads, size_t hd, float* out, float* scratch, size_t ctx_cap,
                           const int* pos_dev, hipStream_t s) {
  if (n_q == 0) return kOk;
  PRANA_CHECK(n_kv_heads > 0 && n_heads % n_kv_heads == 0, "attention: n_heads must be a multiple of n_kv_heads");
  PRANA_CHECK(hd > 0 && hd <= 256, "attention: head_dim must be in 1..=256");
  if (ctx_cap == 0) ctx_cap = pos0 + n_q;
  PRANA_CHECK(pos_dev || pos0 + n_q <= ctx_cap, "attention: scratch capacity below pos0 + n_q");
  return launch_attn<true>(q, kc, vc, pos0, pos_dev, n_q, n_heads, n_kv_heads, hd, out, scratch, ctx_cap, s);
}

int launch_attention_prefill(const float* q, const float* k, const float* v, size_t seq, size_t n_heads,
                             size_t n_kv_heads, size_t hd, float* out, float* scratch, hipStream_t s) {
  if (seq == 0) return kOk;
  PRANA_CHECK(n_kv_heads > 0 && n_heads % n_kv_heads == 0, "attention: n_heads must be a multiple of n_kv_heads");
  PRANA_CHECK(hd > 0 && hd <= 256, "attention: head_dim must be in 1..=256");
  return launch_attn<false>(q, k, v, 0, nullptr, seq, n_heads, n_kv_heads, hd, out, scratch, seq, s);
}

}  // namespace prana
