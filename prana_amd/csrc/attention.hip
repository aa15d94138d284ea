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
constexpr int kPieces = 2 * kNT;     // 16-byte V pieces per PV chunk (two per lane)
constexpr int kProdFloats = 512 * 8 + 4 * 256;  // one product buffer: dw*(rows+4) <= this

template <bool F16>
struct Elem;
template <>
struct Elem<true> {
  using T = uint16_t;
  static __device__ float get(T v) { return f16_operand(v); }  // K/V only feed products
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
        dot += s_q[8 * i + 2 * j] * f16_operand(static_cast<uint16_t>(w[j] & 0xffffu));
        dot += s_q[8 * i + 2 * j + 1] * f16_operand(static_cast<uint16_t>(w[j] >> 16));
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
  // optional: the output row quantized in 32-element blocks (quantize_acts,
  // matmul.rs:105-127) for the next projection; set only when dw % 32 == 0
  int8_t* qd;
  float* qsa;
  int* qsum;
};

struct Lds {
  float* q;       // hd floats
  float* red;     // kNT/64 floats
  float* scores;  // lane_pad(kScoreLds) floats
  float* prod;    // 2 x kProdFloats: products p_t*v_t[d] of a PV chunk, [d][row]
};

// PV in chunks of `ch` rows: every lane turns up to two 16-byte V pieces (EPV
// consecutive dims of one row) into products p_t * v_t[d] written to LDS as
// [d][row]; then the fold lanes (one per dim) add their chunk's products in
// row order. Products of the next chunk are written to the other buffer while
// the current one is folded; V pieces are fetched one chunk ahead.
struct VPieces {
  uint4 a, b;
};

template <bool F16>
__device__ __forceinline__ VPieces fetch_v(const HeadJob& J, int t0, int nr, int ppr) {
  using T = typename Elem<F16>::T;
  constexpr int EPV = 16 / sizeof(T);
  const T* base = static_cast<const T*>(J.v) + (size_t)J.kvh * J.hd + J.d0 + (size_t)t0 * J.kv_stride;
  auto piece = [&](int p) {
    int row = p / ppr, col = p - (p / ppr) * ppr;
    if (row >= nr) row = 0;  // in bounds; not used
    return *reinterpret_cast<const uint4*>(base + (size_t)row * J.kv_stride + col * EPV);
  };
  return VPieces{piece(threadIdx.x), piece(threadIdx.x + kNT)};
}

template <bool F16>
__device__ __forceinline__ void make_products(const VPieces& v, const float* sc, int t0, int nr, int ppr, int ch,
                                              float* prod) {
  using T = typename Elem<F16>::T;
  constexpr int EPV = 16 / sizeof(T);
  const int stride = ch + 4;
  auto one = [&](const uint4& w, int p) {
    const int row = p / ppr, col = p - (p / ppr) * ppr;
    if (row >= nr) return;
    const float pt = sc[t0 + row];
    float x[EPV];
    if constexpr (F16) {
      const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int k = 0; k < 4; k++) {
        x[2 * k] = f16_operand(static_cast<uint16_t>(u[k] & 0xffffu));
        x[2 * k + 1] = f16_operand(static_cast<uint16_t>(u[k] >> 16));
      }
    } else {
      x[0] = __uint_as_float(w.x);
      x[1] = __uint_as_float(w.y);
      x[2] = __uint_as_float(w.z);
      x[3] = __uint_as_float(w.w);
    }
#pragma unroll
    for (int k = 0; k < EPV; k++) prod[(col * EPV + k) * stride + row] = pt * x[k];
  };
  one(v.a, threadIdx.x);
  one(v.b, threadIdx.x + kNT);
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

// SC_LDS: the probabilities live in LDS (sc is the LDS array), else in the
// global scratch; the two bodies are separate so every access to sc compiles
// to one address space.
template <bool F16, bool SC_LDS>
__device__ __forceinline__ void one_head_body(const HeadJob& J, int vec_hd, const Lds& L, float* __restrict__ sc) {
  using T = typename Elem<F16>::T;
  const int tid = threadIdx.x;
  const int n = J.pos + 1;
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
  if (SC_LDS)  // zero fill for the single-lane fold
    for (int t = n + tid; t < exact::lane_pad(n); t += kNT) sc[t] = 0.0f;
  __syncthreads();
  // softmax sum in the reference's left-to-right order (norms.rs:53)
  const float sum = exact::block_seq_sum_nonneg<kNT, SC_LDS>(sc, n);
  const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
  for (int t = tid; t < n; t += kNT) sc[t] = sc[t] * inv;
  __syncthreads();

  // ---- PV over dims [d0, d0+dw): lane d folds dim d0 + d
  const int d = tid;
  const bool folder = d < J.dw;
  float acc = 0.0f;
  if (J.vec) {
    constexpr int EPV = 16 / sizeof(T);
    const int ppr = J.dw / EPV;                 // pieces per row
    const int ch = (kPieces / ppr) / 4 * 4;     // rows per chunk, a multiple of 4
    const int stride = ch + 4;
    const int n_chunks = (n + ch - 1) / ch;
    VPieces v = fetch_v<F16>(J, 0, min(ch, n), ppr);
    make_products<F16>(v, sc, 0, min(ch, n), ppr, ch, L.prod);
    if (n_chunks > 1) v = fetch_v<F16>(J, ch, min(ch, n - ch), ppr);
    __syncthreads();
    for (int c = 0; c < n_chunks; c++) {
      const int t0 = c * ch, nr = min(ch, n - t0);
      if (folder) {
        const float* pr = L.prod + (c & 1) * kProdFloats + d * stride;
        int i = 0;
        for (; i + 4 <= nr; i += 4) {
          const float4 x = *reinterpret_cast<const float4*>(pr + i);
          acc += x.x;
          acc += x.y;
          acc += x.z;
          acc += x.w;
        }
        for (; i < nr; i++) acc += pr[i];
      }
      if (c + 1 < n_chunks) {
        const int t1 = t0 + ch;
        make_products<F16>(v, sc, t1, min(ch, n - t1), ppr, ch, L.prod + ((c + 1) & 1) * kProdFloats);
        if (c + 2 < n_chunks) v = fetch_v<F16>(J, t1 + ch, min(ch, n - t1 - ch), ppr);
      }
      __syncthreads();
    }
  } else if (folder) {
    const T* vb = static_cast<const T*>(J.v) + (size_t)J.kvh * J.hd + J.d0 + d;
    for (int t = 0; t < n; t++) acc += sc[t] * Elem<F16>::get(vb[(size_t)t * J.kv_stride]);
  }
  if (folder) J.dst[J.h * J.hd + J.d0 + d] = acc;
  if (J.qd && folder) {  // the folders are whole 32-lane groups here
    float scale;
    int sum;
    const int qi = quantize_lane(acc, &scale, &sum);
    const int gi = J.h * J.hd + J.d0 + d;
    J.qd[gi] = static_cast<int8_t>(qi);
    if ((gi & 31) == 0) {
      J.qsa[gi >> 5] = scale;
      J.qsum[gi >> 5] = sum;
    }
  }
}

template <bool F16>
__device__ __forceinline__ void one_head(const HeadJob& J, int vec_hd, const Lds& L) {
  if (J.pos + 1 <= kScoreLds)
    one_head_body<F16, true>(J, vec_hd, L, L.scores);
  else
    one_head_body<F16, false>(J, vec_hd, L, J.gscores);
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
                                                   int scratch_stride, int mode, int8_t* __restrict__ qd,
                                                   float* __restrict__ qsa, int* __restrict__ qsum) {
  __shared__ float s_q[256];
  __shared__ float s_red[kNT / 64];
  __shared__ __align__(16) float s_scores[exact::lane_pad(kScoreLds)];
  __shared__ __align__(16) float s_prod[2 * kProdFloats];
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
  const size_t row_len = (size_t)n_heads * hd;
  J.qd = qd ? qd + i * row_len : nullptr;
  J.qsa = qd ? qsa + i * row_len / 32 : nullptr;
  J.qsum = qd ? qsum + i * row_len / 32 : nullptr;
  Lds L{s_q, s_red, s_scores, s_prod};
  one_head<F16>(J, mode, L);
}

template <bool F16>
int launch_attn(const float* q, const void* k, const void* v, size_t pos0, const int* pos_dev, size_t n_q,
                size_t n_heads, size_t n_kv_heads, size_t hd, float* out, float* scratch, size_t ctx_cap,
                const ActQuant* aq, bool* quantized, hipStream_t s) {
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
  // fused quantization needs every workgroup's dims to be whole 32-blocks
  const bool fuse_q = aq && aq->q && (hd / ds) % 32 == 0;
  if (quantized) *quantized = fuse_q;
  hipLaunchKernelGGL(attn_kernel<F16>, dim3(n_heads * ds, n_q), dim3(kNT), 0, s, q, k, v, (int)pos0, pos_dev,
                     (int)n_heads, (int)(n_heads / n_kv_heads), (int)hd, ds, out, scratch, (int)ctx_cap, mode,
                     fuse_q ? aq->q : nullptr, fuse_q ? aq->sa : nullptr, fuse_q ? aq->sums : nullptr);
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
                           const int* pos_dev, hipStream_t s, const ActQuant* aq, bool* quantized) {
  if (n_q == 0) return kOk;
  PRANA_CHECK(n_kv_heads > 0 && n_heads % n_kv_heads == 0, "attention: n_heads must be a multiple of n_kv_heads");
  PRANA_CHECK(hd > 0 && hd <= 256, "attention: head_dim must be in 1..=256");
  if (ctx_cap == 0) ctx_cap = pos0 + n_q;
  PRANA_CHECK(pos_dev || pos0 + n_q <= ctx_cap, "attention: scratch capacity below pos0 + n_q");
  return launch_attn<true>(q, kc, vc, pos0, pos_dev, n_q, n_heads, n_kv_heads, hd, out, scratch, ctx_cap, aq, quantized,
                           s);
}

int launch_attention_prefill(const float* q, const float* k, const float* v, size_t seq, size_t n_heads,
                             size_t n_kv_heads, size_t hd, float* out, float* scratch, hipStream_t s,
                             const ActQuant* aq, bool* quantized) {
  if (seq == 0) return kOk;
  PRANA_CHECK(n_kv_heads > 0 && n_heads % n_kv_heads == 0, "attention: n_heads must be a multiple of n_kv_heads");
  PRANA_CHECK(hd > 0 && hd <= 256, "attention: head_dim must be in 1..=256");
  return launch_attn<false>(q, k, v, 0, nullptr, seq, n_heads, n_kv_heads, hd, out, scratch, seq, aq, quantized, s);
}

}  // namespace prana
