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
#include <hip/hip_ext.h>

#include <algorithm>

#include "common.h"
#include "exact_sum.h"
#include "kernels.h"

namespace prana {

namespace {

constexpr int kNT = 512;             // lanes per workgroup
constexpr int kScoreLds = 4096;      // probabilities kept in LDS up to this length
constexpr int kPieces = 2 * kNT;     // 16-byte V pieces per PV chunk (two per lane)
constexpr int kProdFloats = kPieces * 8 + 4 * 256;  // one product buffer: dw*(rows+4) <= this

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
__device__ __forceinline__ float row_dot(const float* s_q, const typename Elem<F16>::T* krow, int hd, int ps = 1) {
  float dot = -0.0f;
  if constexpr (HD > 0 && F16) {
    static_assert(HD % 8 == 0, "f16 rows load 8 halves at a time");
    uint4 raw[HD / 8];
    const uint4* p = reinterpret_cast<const uint4*>(krow);
#pragma unroll
    for (int i = 0; i < HD / 8; i++) raw[i] = p[(size_t)i * ps];  // piece i: ps 16-byte words on
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
  const void* k;       // K rows (kv_stride elements apart), or pieces (kcache_index, kcap > 0)
  const void* v;
  int pos;  // absolute position: attends to rows 0..=pos
  int h, kvh, kv_stride, hd;
  int kcap;
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
__device__ __forceinline__ void make_products(const VPieces& v, const float* sc, float inv, int t0, int nr, int ppr,
                                              int ch, float* prod) {
  using T = typename Elem<F16>::T;
  constexpr int EPV = 16 / sizeof(T);
  const int stride = ch + 4;
  auto one = [&](const uint4& w, int p) {
    const int row = p / ppr, col = p - (p / ppr) * ppr;
    if (row >= nr) return;
    const float pt = sc[t0 + row] * inv;  // the softmax's p_t = e_t * (1/sum)
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

// Dots of q with two f16 K rows of a compiled head width, as two
// side-by-side chains (each folded left to right from -0.0, as row_dot): the
// second chain fills the first's dependent-add latency.
template <int HD>
__device__ __forceinline__ void row_dot2_f16(const float* s_q, const uint16_t* ka, const uint16_t* kb, float* da,
                                             float* db, int ps) {
  static_assert(HD % 8 == 0, "f16 rows load 8 halves at a time");
  uint4 ra[HD / 8], rb[HD / 8];
  const uint4* pa = reinterpret_cast<const uint4*>(ka);
  const uint4* pb = reinterpret_cast<const uint4*>(kb);
#pragma unroll
  for (int i = 0; i < HD / 8; i++) ra[i] = pa[(size_t)i * ps];  // piece i: ps 16-byte words on
#pragma unroll
  for (int i = 0; i < HD / 8; i++) rb[i] = pb[(size_t)i * ps];
  float a = -0.0f, b = -0.0f;
#pragma unroll
  for (int i = 0; i < HD / 8; i++) {
    const uint32_t wa[4] = {ra[i].x, ra[i].y, ra[i].z, ra[i].w};
    const uint32_t wb[4] = {rb[i].x, rb[i].y, rb[i].z, rb[i].w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float q0 = s_q[8 * i + 2 * j], q1 = s_q[8 * i + 2 * j + 1];
      a += q0 * f16_operand(static_cast<uint16_t>(wa[j] & 0xffffu));
      b += q0 * f16_operand(static_cast<uint16_t>(wb[j] & 0xffffu));
      a += q1 * f16_operand(static_cast<uint16_t>(wa[j] >> 16));
      b += q1 * f16_operand(static_cast<uint16_t>(wb[j] >> 16));
    }
  }
  *da = a;
  *db = b;
}

// Scores of rows 0..n into sc; returns the workgroup-wide max (every lane).
// Compiled f16 widths take a lane's rows two at a time.
template <int HD, bool F16>
__device__ __forceinline__ float head_scores(const HeadJob& J, const Lds& L, float* sc) {
  using T = typename Elem<F16>::T;
  const int tid = threadIdx.x;
  const int n = J.pos + 1;
  const int hd = HD > 0 ? HD : J.hd;
  const float scale = 1.0f / sqrtf(static_cast<float>(hd));
  float mx = -INFINITY;
  if constexpr (HD > 0 && F16) {
    // row t at kb + t * rs, its 8-dim pieces ps 16-byte words apart
    const bool pcs = J.kcap > 0;
    const T* kb = static_cast<const T*>(J.k) + (size_t)J.kvh * hd * (pcs ? J.kcap : 1);
    const size_t rs = pcs ? 8 : J.kv_stride;
    const int ps = pcs ? J.kcap : 1;
    for (int t = tid; t < n; t += 2 * kNT) {
      const int t2 = t + kNT;
      float da, db;
      row_dot2_f16<HD>(L.q, kb + (size_t)t * rs, kb + (size_t)min(t2, n - 1) * rs, &da, &db, ps);
      const float s = da * scale;
      sc[t] = s;
      mx = fmaxf(mx, s);
      if (t2 < n) {
        const float s2 = db * scale;
        sc[t2] = s2;
        mx = fmaxf(mx, s2);
      }
    }
    return mx;
  }
  const T* kb = static_cast<const T*>(J.k) + (size_t)J.kvh * hd;  // rows (kcap == 0 here)
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
  // the first V chunk does not depend on the probabilities: its loads are
  // issued here and land during the sum
  constexpr int EPV = 16 / sizeof(T);
  const int ppr = J.vec ? J.dw / EPV : 1;  // pieces per row (vector rows are whole pieces)
  const int ch = (kPieces / ppr) / 4 * 4;  // rows per chunk, a multiple of 4
  VPieces v{};
  if (J.vec) v = fetch_v<F16>(J, 0, min(ch, n), ppr);
  // softmax sum in the reference's left-to-right order (norms.rs:53)
  const float sum = exact::block_seq_sum_nonneg<kNT, SC_LDS>(sc, n);
  const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
  // p_t = e_t * inv is formed where the P.V products use it (no pass of its own)

  // ---- PV over dims [d0, d0+dw): lane d folds dim d0 + d
  const int d = tid;
  const bool folder = d < J.dw;
  float acc = 0.0f;
  if (J.vec) {
    const int stride = ch + 4;
    const int n_chunks = (n + ch - 1) / ch;
    make_products<F16>(v, sc, inv, 0, min(ch, n), ppr, ch, L.prod);
    if (n_chunks > 1) v = fetch_v<F16>(J, ch, min(ch, n - ch), ppr);
    __syncthreads();
    for (int c = 0; c < n_chunks; c++) {
      const int t0 = c * ch, nr = min(ch, n - t0);
      if (folder) {
        // groups of 32 rows in two register sets: the next group's reads are
        // issued before this group's adds (the empty asm, consuming acc and
        // ordering memory, keeps later reads from being hoisted further)
        const float* pr = L.prod + (c & 1) * kProdFloats + d * stride;
        const float4* p4 = reinterpret_cast<const float4*>(pr);
        const int ng = nr / 32;
        float4 x[8], y[8];
        auto add8 = [&acc](const float4* z) {
#pragma unroll
          for (int j = 0; j < 8; j++) {
            acc += z[j].x;
            acc += z[j].y;
            acc += z[j].z;
            acc += z[j].w;
          }
        };
        if (ng > 0) {
#pragma unroll
          for (int j = 0; j < 8; j++) x[j] = p4[j];
        }
        int g = 0;
        for (; g + 1 < ng; g += 2) {
#pragma unroll
          for (int j = 0; j < 8; j++) y[j] = p4[(g + 1) * 8 + j];
          add8(x);
          asm volatile("" ::"v"(acc) : "memory");
          if (g + 2 < ng) {
#pragma unroll
            for (int j = 0; j < 8; j++) x[j] = p4[(g + 2) * 8 + j];
          }
          add8(y);
          asm volatile("" ::"v"(acc) : "memory");
        }
        if (g < ng) {
          add8(x);
          g++;
        }
        int i = 32 * g;
        for (; i + 4 <= nr; i += 4) {
          const float4 z = p4[i / 4];
          acc += z.x;
          acc += z.y;
          acc += z.z;
          acc += z.w;
        }
        for (; i < nr; i++) acc += pr[i];
      }
      if (c + 1 < n_chunks) {
        const int t1 = t0 + ch;
        make_products<F16>(v, sc, inv, t1, min(ch, n - t1), ppr, ch, L.prod + ((c + 1) & 1) * kProdFloats);
        if (c + 2 < n_chunks) v = fetch_v<F16>(J, t1 + ch, min(ch, n - t1 - ch), ppr);
      }
      __syncthreads();
    }
  } else if (folder) {
    const T* vb = static_cast<const T*>(J.v) + (size_t)J.kvh * J.hd + J.d0 + d;
    for (int t = 0; t < n; t++) acc += (sc[t] * inv) * Elem<F16>::get(vb[(size_t)t * J.kv_stride]);
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

// ---------------------------------------------------------------- split path
// The same arithmetic in three launches, for the f16 cache with 64- or
// 128-wide heads: every phase then gets the parallelism it can use instead of
// the one fixed by a workgroup per head.
//   scores : one lane per (K row, KV head); the group's query heads are folded
//            side by side (independent chains), scores -> scratch
//   softmax: one 1024-lane workgroup per (query row, head): max, expf, the
//            exact left-to-right sum, probabilities -> scratch (in place)
//   PV     : one workgroup per (query row, head, 64-dim slice): one folder
//            wave adds the products of its dims in row order while eight
//            producer waves stream V and form the products of the next chunk
// Scratch rows are (query row, head) major with a stride of
// split_stride(ctx_cap) floats.
constexpr int kSplitRows = 256;     // K rows per scores workgroup
constexpr int kSmNT = 1024;         // softmax lanes
constexpr int kPvProd = 512;        // producer lanes (their V loads, not the fold, set the pace)
constexpr int kPvNT = 64 + kPvProd; // one folder wave + producers
// cache windows from this many rows on take the split path
constexpr size_t kSplitMinRows = 2048;

__host__ __device__ constexpr size_t split_stride(size_t ctx_cap) {
  return (ctx_cap + kSplitRows - 1) / kSplitRows * kSplitRows;
}

// grid: (ceil(rows / kSplitRows), n_q * n_kv * ceil(group / 4)). Lane t of
// block x scores K row x*kSplitRows + t against a block of up to four query
// heads of one KV group (side-by-side chains) for query row i; rows past that
// row's position are skipped. A short head block repeats its first head in
// the spare chains (computed, not stored) so the body has no branches.
template <int HD>
__global__ __launch_bounds__(kSplitRows) void attn_split_scores(const float* __restrict__ q,
                                                                const uint16_t* __restrict__ k, int pos0,
                                                                const int* __restrict__ pos_dev, int n_heads,
                                                                int group, int n_kv, float* __restrict__ sc,
                                                                int sc_stride, int kcap) {
  __shared__ __align__(16) float s_q[4 * HD];
  const int nhb = (group + 3) / 4;
  const int hb = blockIdx.y % nhb, ik = blockIdx.y / nhb;
  const int i = ik / n_kv, kvh = ik % n_kv;
  const int n = (pos_dev ? *pos_dev : pos0) + i + 1;
  const int row0 = blockIdx.x * kSplitRows;
  if (row0 >= n) return;  // uniform, before the barrier
  const int h0 = kvh * group + 4 * hb;  // first head of the block
  const int nh = min(4, group - 4 * hb);
  const float* qh = q + (size_t)i * n_heads * HD + (size_t)h0 * HD;
  for (int e = threadIdx.x; e < 4 * HD; e += kSplitRows) s_q[e] = qh[e / HD < nh ? e : e % HD];
  __syncthreads();
  const int t = row0 + threadIdx.x;
  if (t >= n) return;
  const int kv_stride = n_kv * HD;
  const uint4* kp = reinterpret_cast<const uint4*>(
      kcap ? k + (size_t)kvh * HD * kcap + (size_t)t * 8 : k + (size_t)t * kv_stride + (size_t)kvh * HD);
  const int ps = kcap ? kcap : 1;  // 16-byte words between a row's 8-dim pieces
  uint4 raw[HD / 8];
#pragma unroll
  for (int e = 0; e < HD / 8; e++) raw[e] = kp[(size_t)e * ps];
  const float4* qv = reinterpret_cast<const float4*>(s_q);
  float dot[4] = {-0.0f, -0.0f, -0.0f, -0.0f};
  // q of step e+1 is read while step e computes. The empty asm after each
  // step consumes that step's partial dots and orders memory, so the reads
  // of later steps cannot be hoisted above it (all of them at once would
  // need 4*HD registers).
  float4 qa[4][2], qn[4][2];
#pragma unroll
  for (int hh = 0; hh < 4; hh++) qa[hh][0] = qv[hh * (HD / 4)], qa[hh][1] = qv[hh * (HD / 4) + 1];
#pragma unroll
  for (int e = 0; e < HD / 8; e++) {
    if (e + 1 < HD / 8) {
#pragma unroll
      for (int hh = 0; hh < 4; hh++)
        qn[hh][0] = qv[hh * (HD / 4) + 2 * e + 2], qn[hh][1] = qv[hh * (HD / 4) + 2 * e + 3];
    }
    const uint32_t w[4] = {raw[e].x, raw[e].y, raw[e].z, raw[e].w};
    float kf[8];
#pragma unroll
    for (int j = 0; j < 8; j++)
      kf[j] = f16_operand(static_cast<uint16_t>(j & 1 ? w[j >> 1] >> 16 : w[j >> 1] & 0xffffu));
#pragma unroll
    for (int hh = 0; hh < 4; hh++) {
      const float4 a = qa[hh][0], b = qa[hh][1];
      dot[hh] += a.x * kf[0];
      dot[hh] += a.y * kf[1];
      dot[hh] += a.z * kf[2];
      dot[hh] += a.w * kf[3];
      dot[hh] += b.x * kf[4];
      dot[hh] += b.y * kf[5];
      dot[hh] += b.z * kf[6];
      dot[hh] += b.w * kf[7];
    }
    asm volatile("" ::"v"(dot[0]), "v"(dot[1]), "v"(dot[2]), "v"(dot[3]) : "memory");
#pragma unroll
    for (int hh = 0; hh < 4; hh++) qa[hh][0] = qn[hh][0], qa[hh][1] = qn[hh][1];
  }
  const float scale = 1.0f / sqrtf(static_cast<float>(HD));
  float* dst = sc + ((size_t)i * n_heads + h0) * sc_stride + t;
#pragma unroll
  for (int hh = 0; hh < 4; hh++)
    if (hh < nh) dst[(size_t)hh * sc_stride] = dot[hh] * scale;
}

// grid: (ceil(rows / kSplitRows), ceil(n_q / 2) * n_kv * ceil(group / 4)).
// The verify form of the scores launch: two query rows per workgroup share
// each K row's load (eight side-by-side chains: four heads x two rows, each
// folded over d in order as above); a row's keys past its own position are
// not stored, and a dead second row repeats the first (computed, not stored).
template <int HD>
__global__ __launch_bounds__(kSplitRows) void attn_split_scores_rows(const float* __restrict__ q,
                                                                     const uint16_t* __restrict__ k, int pos0,
                                                                     const int* __restrict__ pos_dev, int n_q,
                                                                     int n_heads, int group, int n_kv,
                                                                     float* __restrict__ sc, int sc_stride,
                                                                     int kcap) {
  constexpr int QR = 2;
  __shared__ __align__(16) float s_q[QR][4 * HD];
  const int nhb = (group + 3) / 4;
  const int hb = blockIdx.y % nhb, ik = blockIdx.y / nhb;
  const int ig = ik / n_kv, kvh = ik % n_kv;
  const int i0 = ig * QR, nr = min(QR, n_q - i0);
  const int p0 = pos_dev ? *pos_dev : pos0;
  const int n_max = p0 + i0 + nr;  // keys of the block's last live row
  const int row0 = blockIdx.x * kSplitRows;
  if (row0 >= n_max) return;  // uniform, before the barrier
  const int h0 = kvh * group + 4 * hb;
  const int nh = min(4, group - 4 * hb);
  for (int e = threadIdx.x; e < QR * 4 * HD; e += kSplitRows) {
    const int r = e / (4 * HD), ee = e % (4 * HD);
    const float* qh = q + (size_t)(i0 + min(r, nr - 1)) * n_heads * HD + (size_t)h0 * HD;
    s_q[r][ee] = qh[ee / HD < nh ? ee : ee % HD];
  }
  __syncthreads();
  const int t = row0 + threadIdx.x;
  if (t >= n_max) return;
  const int kv_stride = n_kv * HD;
  const uint4* kp = reinterpret_cast<const uint4*>(
      kcap ? k + (size_t)kvh * HD * kcap + (size_t)t * 8 : k + (size_t)t * kv_stride + (size_t)kvh * HD);
  const int ps = kcap ? kcap : 1;  // 16-byte words between a row's 8-dim pieces
  uint4 raw[HD / 8];
#pragma unroll
  for (int e = 0; e < HD / 8; e++) raw[e] = kp[(size_t)e * ps];
  float dot[QR][4];
#pragma unroll
  for (int r = 0; r < QR; r++)
#pragma unroll
    for (int hh = 0; hh < 4; hh++) dot[r][hh] = -0.0f;
#pragma unroll
  for (int e = 0; e < HD / 8; e++) {
    const uint32_t w[4] = {raw[e].x, raw[e].y, raw[e].z, raw[e].w};
    float kf[8];
#pragma unroll
    for (int j = 0; j < 8; j++)
      kf[j] = f16_operand(static_cast<uint16_t>(j & 1 ? w[j >> 1] >> 16 : w[j >> 1] & 0xffffu));
#pragma unroll
    for (int r = 0; r < QR; r++)
#pragma unroll
      for (int hh = 0; hh < 4; hh++) {
        const float4 a = reinterpret_cast<const float4*>(s_q[r])[hh * (HD / 4) + 2 * e];
        const float4 b = reinterpret_cast<const float4*>(s_q[r])[hh * (HD / 4) + 2 * e + 1];
        dot[r][hh] += a.x * kf[0];
        dot[r][hh] += a.y * kf[1];
        dot[r][hh] += a.z * kf[2];
        dot[r][hh] += a.w * kf[3];
        dot[r][hh] += b.x * kf[4];
        dot[r][hh] += b.y * kf[5];
        dot[r][hh] += b.z * kf[6];
        dot[r][hh] += b.w * kf[7];
      }
    // keep later steps' q reads from being hoisted above this one (registers)
    asm volatile("" ::"v"(dot[0][0]), "v"(dot[0][1]), "v"(dot[0][2]), "v"(dot[0][3]), "v"(dot[1][0]),
                 "v"(dot[1][1]), "v"(dot[1][2]), "v"(dot[1][3])
                 : "memory");
  }
  const float scale = 1.0f / sqrtf(static_cast<float>(HD));
#pragma unroll
  for (int r = 0; r < QR; r++) {
    if (r < nr && t < p0 + i0 + r + 1) {
      float* dst = sc + ((size_t)(i0 + r) * n_heads + h0) * sc_stride + t;
#pragma unroll
      for (int hh = 0; hh < 4; hh++)
        if (hh < nh) dst[(size_t)hh * sc_stride] = dot[r][hh] * scale;
    }
  }
}

// grid: (n_heads, n_q). Softmax of the row's scores in place. Rows of up to
// kSmNT*kSmPer scores are held in registers (every load in flight at once);
// longer rows stream. IN_LDS: the exponentials are staged in LDS
// (exact::run_pad layout) for the exact sum; otherwise the sum reads them
// back from the scratch row.
constexpr int kSmPer = 36;
template <bool IN_LDS>
__global__ __launch_bounds__(kSmNT) void attn_split_softmax(float* __restrict__ sc, int sc_stride, int pos0,
                                                            const int* __restrict__ pos_dev, int n_heads) {
  extern __shared__ float4 smem_e4[];
  float* e = reinterpret_cast<float*>(smem_e4);
  __shared__ float s_red[kSmNT / 64];
  const int h = blockIdx.x, i = blockIdx.y, tid = threadIdx.x;
  const int n = (pos_dev ? *pos_dev : pos0) + i + 1;
  float* row = sc + ((size_t)i * n_heads + h) * sc_stride;
  const bool in_regs = n <= kSmNT * kSmPer;
  float vals[kSmPer];
  float mx = -INFINITY;
  if (in_regs) {
#pragma unroll
    for (int k = 0; k < kSmPer; k++) {
      if (k * kSmNT >= n) break;  // uniform
      vals[k] = row[min(tid + k * kSmNT, n - 1)];
    }
#pragma unroll
    for (int k = 0; k < kSmPer; k++) {
      if (k * kSmNT >= n) break;
      if (tid + k * kSmNT < n) mx = fmaxf(mx, vals[k]);
    }
  } else {
    for (int t = tid; t < n; t += kSmNT) mx = fmaxf(mx, row[t]);
  }
  mx = wave_max_f32(mx);
  if ((tid & 63) == 0) s_red[tid >> 6] = mx;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kSmNT / 64; w++) mx = fmaxf(mx, s_red[w]);
  auto put = [&](int t, float v) {
    if constexpr (IN_LDS)
      e[exact::run_pad(t)] = v;
    else
      row[t] = v;
  };
  if (in_regs) {
#pragma unroll
    for (int k = 0; k < kSmPer; k++) {
      if (k * kSmNT >= n) break;
      const int t = tid + k * kSmNT;
      vals[k] = dev_expf(vals[k] - mx);
      if (t < n) put(t, vals[k]);
    }
  } else {
    for (int t = tid; t < n; t += kSmNT) put(t, dev_expf(row[t] - mx));
  }
  __syncthreads();
  // softmax sum in the reference's left-to-right order (norms.rs:53)
  float sum;
  if constexpr (IN_LDS)
    sum = exact::block_seq_sum_short<kSmNT>([e](int t) { return e[exact::run_pad(t)]; }, n);
  else if (n <= exact::kPredHead + kSmNT * exact::kPredMaxPerLane)
    sum = exact::block_seq_sum_short<kSmNT>([row](int t) { return row[t]; }, n);
  else
    sum = exact::block_seq_sum_nonneg<kSmNT, false>(row, n);
  const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
  if (in_regs) {
#pragma unroll
    for (int k = 0; k < kSmPer; k++) {
      if (k * kSmNT >= n) break;
      const int t = tid + k * kSmNT;
      if (t < n) row[t] = vals[k] * inv;
    }
  } else {
    for (int t = tid; t < n; t += kSmNT) {
      if constexpr (IN_LDS)
        row[t] = e[exact::run_pad(t)] * inv;
      else
        row[t] = row[t] * inv;
    }
  }
}

// grid: (n_heads * HD/64, n_q). Folder lane d (wave 0) owns dim 64*slice + d;
// a producer task (waves 1..8) is one row quad of one 8-dim piece: four
// 16-byte V loads (with one 4-byte word per load, the producers' loads set
// the pace: ~4x the load instructions). Products of a chunk of CH rows sit in
// LDS as [row/4][dim][row%4], a pad word after every 8 dims so that
// neighbouring pieces' 16-byte stores fall on different banks; the folder
// reads four rows of its dim with one 16-byte load. Rows past n are zero
// products, which leave the fold (started from +0.0) unchanged.
template <int HD, int CH>
__global__ __launch_bounds__(kPvNT) void attn_split_pv(const float* __restrict__ prob, int sc_stride,
                                                       const uint16_t* __restrict__ v, int pos0,
                                                       const int* __restrict__ pos_dev, int n_heads,
                                                       int group, float* __restrict__ out,
                                                       int8_t* __restrict__ qd, float* __restrict__ qsa,
                                                       int* __restrict__ qsum) {
  constexpr int NS = HD / 64;
  constexpr int kTasks = CH / 4 * 8;  // (row quad, 8-dim piece) per chunk
  constexpr int kPer = (kTasks + kPvProd - 1) / kPvProd;
  constexpr int QS = 64 + 8;          // float4 words per row quad: a pad word after every 8 dims
  static_assert(kSplitRows % CH == 0, "probability reads of the last chunk stay inside the scratch row");
  __shared__ __align__(16) float s_prod[2][CH / 4 * QS * 4];
  const int lb = logical_block(n_heads * NS);
  const int h = lb / NS, slice = lb % NS, i = blockIdx.y;
  const int n = (pos_dev ? *pos_dev : pos0) + i + 1;
  const int kvh = h / group;
  const int kv_words = (n_heads / group) * HD / 2;  // a cache row in 32-bit words
  const int tid = threadIdx.x;
  const int n_chunks = (n + CH - 1) / CH;
  const bool folder = tid < 64;
  const int pl = tid - 64;
  // this head's 64-dim slice of V, and its probability row
  const uint16_t* vs = v + (size_t)kvh * HD + slice * 64;
  const size_t kv_stride = 2 * (size_t)kv_words;  // a cache row in f16 values
  const float* prow = prob + ((size_t)i * n_heads + h) * sc_stride;

  uint4 vr[kPer][4];
  float4 pr[kPer];
  auto fetch = [&](int c) {
#pragma unroll
    for (int k = 0; k < kPer; k++) {
      const int task = min(pl + kPvProd * k, kTasks - 1);
      const int pc = task % 8, t = c * CH + 4 * (task / 8);
      pr[k] = *reinterpret_cast<const float4*>(prow + t);  // t + 3 < sc_stride
#pragma unroll
      for (int r = 0; r < 4; r++)  // rows past n: clamped, unused
        vr[k][r] = *reinterpret_cast<const uint4*>(vs + (size_t)min(t + r, n - 1) * kv_stride + 8 * pc);
    }
  };
  auto produce = [&](int c, float* buf) {
#pragma unroll
    for (int k = 0; k < kPer; k++) {
      const int task = pl + kPvProd * k;
      if (task >= kTasks) break;
      const int pc = task % 8, rq = task / 8, t = c * CH + 4 * rq;
      const float pv[4] = {pr[k].x, pr[k].y, pr[k].z, pr[k].w};
      float4* dst = reinterpret_cast<float4*>(buf) + rq * QS + 9 * pc;
#pragma unroll
      for (int w = 0; w < 4; w++) {  // dims 8pc + 2w, 8pc + 2w + 1
        float a[4], b[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const uint32_t word = w == 0 ? vr[k][r].x : w == 1 ? vr[k][r].y : w == 2 ? vr[k][r].z : vr[k][r].w;
          const bool live = t + r < n;
          a[r] = live ? pv[r] * f16_operand(static_cast<uint16_t>(word & 0xffffu)) : 0.0f;
          b[r] = live ? pv[r] * f16_operand(static_cast<uint16_t>(word >> 16)) : 0.0f;
        }
        dst[2 * w] = make_float4(a[0], a[1], a[2], a[3]);
        dst[2 * w + 1] = make_float4(b[0], b[1], b[2], b[3]);
      }
    }
  };

  float acc = 0.0f;
  if (!folder) {
    fetch(0);
    produce(0, s_prod[0]);
    if (n_chunks > 1) fetch(1);
  }
  __syncthreads();
  for (int c = 0; c < n_chunks; c++) {
    if (folder) {
      // groups of 8 row quads; the next group's reads are issued before this
      // group's adds, and the empty asm (consuming acc, ordering memory)
      // keeps later reads from being hoisted further
      const float4* src = reinterpret_cast<const float4*>(s_prod[c & 1]) + tid + tid / 8;
      float4 x[8], y[8];
#pragma unroll
      for (int j = 0; j < 8; j++) x[j] = src[j * QS];
#pragma unroll
      for (int g = 0; g < CH / 32; g++) {
        if (g + 1 < CH / 32) {
#pragma unroll
          for (int j = 0; j < 8; j++) y[j] = src[((g + 1) * 8 + j) * QS];
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
          acc += x[j].x;
          acc += x[j].y;
          acc += x[j].z;
          acc += x[j].w;
        }
        asm volatile("" ::"v"(acc) : "memory");
#pragma unroll
        for (int j = 0; j < 8; j++) x[j] = y[j];
      }
    } else if (c + 1 < n_chunks) {
      produce(c + 1, s_prod[(c + 1) & 1]);
      if (c + 2 < n_chunks) fetch(c + 2);
    }
    __syncthreads();
  }
  if (folder) {
    const size_t gi = (size_t)i * n_heads * HD + (size_t)h * HD + slice * 64 + tid;
    out[gi] = acc;
    if (qd) {
      float scale;
      int sum;
      const int qi = quantize_lane(acc, &scale, &sum);
      qd[gi] = static_cast<int8_t>(qi);
      if ((gi & 31) == 0) {
        qsa[gi >> 5] = scale;
        qsum[gi >> 5] = sum;
      }
    }
  }
}

// grid: (n_heads * HD/64, ceil(n_q / QR)). The verify form of the PV launch:
// QR query rows of one (head, 64-dim slice) per workgroup share each V chunk;
// eight producer waves keep the VALU load on each fold wave's SIMD light (a
// busy neighbour delays the fold's dependent adds).
// Fold wave q (q < QR) owns dim 64*slice + lane of query row i0 + q; the
// producer lanes take (row quad, dim pair) tasks, load the four V rows' dim
// pair once and form the products of all QR query rows (a row's keys past
// its own window are zero products, which leave its fold from +0.0
// unchanged). LDS: [2][QR][CH/4][64] float4, dynamic.
constexpr int kPvrQR = 2;      // query rows per workgroup
constexpr int kPvrCH = 128;    // cache rows per chunk
constexpr int kPvrProd = 512;  // producer lanes: light VALU load beside each fold wave
template <int HD>
__global__ __launch_bounds__(64 * kPvrQR + kPvrProd) void attn_split_pv_rows(
    const float* __restrict__ prob, int sc_stride, const uint16_t* __restrict__ v, int pos0,
    const int* __restrict__ pos_dev, int n_q, int n_heads, int group, float* __restrict__ out,
    int8_t* __restrict__ qd, float* __restrict__ qsa, int* __restrict__ qsum) {
  constexpr int QR = kPvrQR, CH = kPvrCH;
  constexpr int NS = HD / 64;
  constexpr int kTasks = CH / 4 * 32;
  constexpr int kPer = kTasks / kPvrProd;
  constexpr int kQuadStep = kPvrProd / 32;
  static_assert(kTasks % kPvrProd == 0, "whole tasks per producer lane");
  static_assert(kSplitRows % CH == 0, "probability reads of the last chunk stay inside the scratch row");
  extern __shared__ float4 pvr_smem[];
  float* s_prod = reinterpret_cast<float*>(pvr_smem);
  const int lb = logical_block(n_heads * NS);
  const int h = lb / NS, slice = lb % NS;
  const int i0 = blockIdx.y * QR;
  const int nr = min(QR, n_q - i0);  // live query rows of this block
  const int p0 = pos_dev ? *pos_dev : pos0;
  const int n_max = p0 + i0 + nr;  // keys of the block's last live row
  const int kvh = h / group;
  const int kv_words = (n_heads / group) * HD / 2;
  const int tid = threadIdx.x;
  const int n_chunks = (n_max + CH - 1) / CH;
  const bool folder = tid < 64 * QR;
  const int pl = tid - 64 * QR;
  const int dp = pl & 31, rq0 = pl >> 5;
  const uint32_t* vlane = reinterpret_cast<const uint32_t*>(v + (size_t)kvh * HD + slice * 64) + dp;
  const float* plane[QR];
#pragma unroll
  for (int q = 0; q < QR; q++)  // dead rows read the last live row's (valid) scratch
    plane[q] = prob + ((size_t)(i0 + min(q, nr - 1)) * n_heads + h) * sc_stride + 4 * rq0;

  uint32_t vr[kPer][4];
  float4 pr[kPer][QR];
  auto fetch = [&](int c) {
#pragma unroll
    for (int k = 0; k < kPer; k++) {
      const int t = c * CH + 4 * rq0 + 4 * kQuadStep * k;
#pragma unroll
      for (int q = 0; q < QR; q++)
        pr[k][q] = *reinterpret_cast<const float4*>(plane[q] + c * CH + 4 * kQuadStep * k);  // t + 3 < sc_stride
#pragma unroll
      for (int r = 0; r < 4; r++) vr[k][r] = vlane[(size_t)min(t + r, n_max - 1) * kv_words];  // past n_max: unused
    }
  };
  auto produce = [&](int c, float* buf) {
#pragma unroll
    for (int k = 0; k < kPer; k++) {
      const int t = c * CH + 4 * rq0 + 4 * kQuadStep * k;
      float va[4], vb[4];
#pragma unroll
      for (int r = 0; r < 4; r++) {
        va[r] = f16_operand(static_cast<uint16_t>(vr[k][r] & 0xffffu));
        vb[r] = f16_operand(static_cast<uint16_t>(vr[k][r] >> 16));
      }
#pragma unroll
      for (int q = 0; q < QR; q++) {
        const int n = p0 + i0 + q + 1;  // keys of query row i0 + q
        const float pv[4] = {pr[k][q].x, pr[k][q].y, pr[k][q].z, pr[k][q].w};
        float a[4], b[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const bool live = t + r < n;
          a[r] = live ? pv[r] * va[r] : 0.0f;
          b[r] = live ? pv[r] * vb[r] : 0.0f;
        }
        float4* dst = reinterpret_cast<float4*>(buf + q * CH * 64) + (rq0 + kQuadStep * k) * 64 + 2 * dp;
        dst[0] = make_float4(a[0], a[1], a[2], a[3]);
        dst[1] = make_float4(b[0], b[1], b[2], b[3]);
      }
    }
  };

  float acc = 0.0f;
  if (!folder) {
    fetch(0);
    produce(0, s_prod);
    if (n_chunks > 1) fetch(1);
  }
  __syncthreads();
  const int fq = tid >> 6, lane = tid & 63;
  for (int c = 0; c < n_chunks; c++) {
    if (folder) {
      const float4* src = reinterpret_cast<const float4*>(s_prod + ((c & 1) * QR + fq) * CH * 64) + lane;
      float4 x[8], y[8];
#pragma unroll
      for (int j = 0; j < 8; j++) x[j] = src[j * 64];
#pragma unroll
      for (int g = 0; g < CH / 32; g++) {
        if (g + 1 < CH / 32) {
#pragma unroll
          for (int j = 0; j < 8; j++) y[j] = src[((g + 1) * 8 + j) * 64];
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
          acc += x[j].x;
          acc += x[j].y;
          acc += x[j].z;
          acc += x[j].w;
        }
        asm volatile("" ::"v"(acc) : "memory");
#pragma unroll
        for (int j = 0; j < 8; j++) x[j] = y[j];
      }
    } else if (c + 1 < n_chunks) {
      produce(c + 1, s_prod + ((c + 1) & 1) * QR * CH * 64);
      if (c + 2 < n_chunks) fetch(c + 2);
    }
    __syncthreads();
  }
  if (folder && fq < nr) {
    const size_t gi = (size_t)(i0 + fq) * n_heads * HD + (size_t)h * HD + slice * 64 + lane;
    out[gi] = acc;
    if (qd) {  // one wave: two whole 32-blocks
      float scale;
      int sum;
      const int qi = quantize_lane(acc, &scale, &sum);
      qd[gi] = static_cast<int8_t>(qi);
      if ((gi & 31) == 0) {
        qsa[gi >> 5] = scale;
        qsum[gi >> 5] = sum;
      }
    }
  }
}

// ---------------------------------------------------------------- wide path
// Verify batches (two or more query rows) over cache windows below
// kSplitMinRows with 64/128-wide heads: one 1024-lane workgroup per (query
// row, head) does the whole head. Scores: one lane per cache row (a second
// row past 1024), into LDS at exact::run_pad positions; softmax with the
// exact sum over that LDS row; P·V like the split path's PV launch (fold
// waves for the head's dims, the other waves form the products of the next
// chunk from the LDS probabilities and V). A single decode row stays on the
// one-launch kernel: with one workgroup per head the row-per-lane K gathers
// of 32 workgroups are slower than its 128 (23.0 against 18.7 us at 512
// rows), while 8 verify rows gain (24.4 against 31.8 us).
constexpr int kWideNT = 1024;
constexpr int kWideMax = kSplitMinRows - 1;  // rows a wide workgroup takes at most
constexpr size_t kWideMinRows = 256;          // shorter windows stay on the one-launch kernel

template <int HD>
struct WideCfg {
  static constexpr int F = HD / 64;                 // fold waves
  static constexpr int CH = HD == 128 ? 128 : 256;  // rows per PV chunk
  static constexpr int PL = kWideNT - 64 * F;       // producer lanes
  static constexpr int TASKS = CH / 4 * (HD / 8);   // (row quad, 8-dim piece) per chunk
  static constexpr int PER = (TASKS + PL - 1) / PL;
  static constexpr int QS = HD + HD / 8;            // float4 words per row quad: a pad word after every 8 dims
  static constexpr int SC = exact::run_pad(kWideMax - 1) + 1;  // probability words
};

template <int HD>
__global__ __launch_bounds__(kWideNT) void attn_wide_kernel(const float* __restrict__ q,
                                                            const uint16_t* __restrict__ k,
                                                            const uint16_t* __restrict__ v, int pos0, int n_heads,
                                                            int group, float* __restrict__ out,
                                                            int8_t* __restrict__ qd, float* __restrict__ qsa,
                                                            int* __restrict__ qsum, int kcap) {
  using C = WideCfg<HD>;
  __shared__ __align__(16) float s_q[HD];
  __shared__ float s_red[kWideNT / 64];
  __shared__ __align__(16) float s_p[C::SC];
  // windows of up to kPadSerialMax rows: the exponentials again, contiguous
  // and zero-padded, for the one-lane fold on 16-byte loads
  __shared__ __align__(16) float s_e[exact::lane_pad(exact::kPadSerialMax)];
  __shared__ __align__(16) float s_prod[2][C::CH / 4 * C::QS * 4];
  const int h = blockIdx.x, i = blockIdx.y, tid = threadIdx.x;
  const int n = pos0 + i + 1;  // <= kWideMax rows
  const int kvh = h / group;
  const int kv_stride = (n_heads / group) * HD;
  for (int d = tid; d < HD; d += kWideNT) s_q[d] = q[((size_t)i * n_heads + h) * HD + d];
  __syncthreads();
  // ---- scores (attention.rs:165-185): (fold_d q[d]*k_t[d] from -0.0) * (1/sqrt(hd))
  const float scale = 1.0f / sqrtf(static_cast<float>(HD));
  // row t at kb + t * rs, its 8-dim pieces ps 16-byte words apart
  const uint16_t* kb = k + (size_t)kvh * HD * (kcap ? kcap : 1);
  const size_t rs = kcap ? 8 : kv_stride;
  const int ps = kcap ? kcap : 1;
  const int t1 = tid, t2 = tid + kWideNT;
  float mx = -INFINITY;
  if (t1 < n) {
    const float s1 = row_dot<HD, true>(s_q, kb + (size_t)t1 * rs, HD, ps) * scale;
    s_p[exact::run_pad(t1)] = s1;
    mx = s1;
  }
  if (t2 < n) {
    const float s2 = row_dot<HD, true>(s_q, kb + (size_t)t2 * rs, HD, ps) * scale;
    s_p[exact::run_pad(t2)] = s2;
    mx = fmaxf(mx, s2);
  }
  mx = wave_max_f32(mx);
  if ((tid & 63) == 0) s_red[tid >> 6] = mx;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kWideNT / 64; w++) mx = fmaxf(mx, s_red[w]);
  float e1 = 0.0f, e2 = 0.0f;
  if (t1 < n) s_p[exact::run_pad(t1)] = e1 = dev_expf(s_p[exact::run_pad(t1)] - mx);
  if (t2 < n) s_p[exact::run_pad(t2)] = e2 = dev_expf(s_p[exact::run_pad(t2)] - mx);
  const bool short_row = n <= exact::kPadSerialMax;  // uniform
  if (short_row && t1 < exact::lane_pad(n)) s_e[t1] = t1 < n ? e1 : 0.0f;  // lane_pad(896) < kWideNT
  __syncthreads();
  // softmax sum in the reference's left-to-right order (norms.rs:53): one
  // lane's chain over the padded row when it is short (~4 ns a term, against
  // the scan's fixed ~4.5 us), the exact scan otherwise
  const float sum = short_row ? exact::block_seq_sum_nonneg<kWideNT, true>(s_e, n)
                              : exact::block_seq_sum_short<kWideNT>([](int t) { return s_p[exact::run_pad(t)]; }, n);
  const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
  if (t1 < n) s_p[exact::run_pad(t1)] = e1 * inv;
  if (t2 < n) s_p[exact::run_pad(t2)] = e2 * inv;
  __syncthreads();

  // ---- P·V: fold lanes (waves 0..F-1) own the head's dims; the others form
  // the products of the next chunk as [row/4][dim][row%4] (a pad word after
  // every 8 dims, so that the producers' 16-byte stores of neighbouring
  // pieces fall on different banks). A producer task is one row quad of one
  // 8-dim piece: four 16-byte V loads (4-byte loads made the texture
  // address unit the bound). Rows past n are zero products, which leave the
  // fold (started from +0.0) unchanged.
  const bool folder = tid < 64 * C::F;
  const int pl = tid - 64 * C::F;
  const uint16_t* vh = v + (size_t)kvh * HD;
  const int n_chunks = (n + C::CH - 1) / C::CH;
  uint4 vr[C::PER][4];
  auto fetch = [&](int c) {
#pragma unroll
    for (int kk = 0; kk < C::PER; kk++) {
      const int task = min(pl + C::PL * kk, C::TASKS - 1);
      const int pc = task % (HD / 8), rq = task / (HD / 8);
      const int t = c * C::CH + 4 * rq;
#pragma unroll
      for (int r = 0; r < 4; r++)
        vr[kk][r] = *reinterpret_cast<const uint4*>(vh + (size_t)min(t + r, n - 1) * kv_stride + 8 * pc);
    }
  };
  auto produce = [&](int c, float* buf) {
#pragma unroll
    for (int kk = 0; kk < C::PER; kk++) {
      const int task = pl + C::PL * kk;
      if (task >= C::TASKS) break;
      const int pc = task % (HD / 8), rq = task / (HD / 8);
      const int t = c * C::CH + 4 * rq;
      float p[4];
      bool live[4];
#pragma unroll
      for (int r = 0; r < 4; r++) {
        live[r] = t + r < n;
        p[r] = s_p[exact::run_pad(min(t + r, n - 1))];
      }
      float4* dst = reinterpret_cast<float4*>(buf) + rq * C::QS + 9 * pc;
#pragma unroll
      for (int w = 0; w < 4; w++) {  // dims 8pc + 2w, 8pc + 2w + 1
        float a[4], b[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const uint32_t word = w == 0 ? vr[kk][r].x : w == 1 ? vr[kk][r].y : w == 2 ? vr[kk][r].z : vr[kk][r].w;
          a[r] = live[r] ? p[r] * f16_operand(static_cast<uint16_t>(word & 0xffffu)) : 0.0f;
          b[r] = live[r] ? p[r] * f16_operand(static_cast<uint16_t>(word >> 16)) : 0.0f;
        }
        dst[2 * w] = make_float4(a[0], a[1], a[2], a[3]);
        dst[2 * w + 1] = make_float4(b[0], b[1], b[2], b[3]);
      }
    }
  };
  float acc = 0.0f;
  if (!folder) {
    fetch(0);
    produce(0, s_prod[0]);
    if (n_chunks > 1) fetch(1);
  }
  __syncthreads();
  for (int c = 0; c < n_chunks; c++) {
    if (folder) {
      const float4* src = reinterpret_cast<const float4*>(s_prod[c & 1]) + tid + tid / 8;
#pragma unroll
      for (int g = 0; g < C::CH / 32; g++) {
        float4 x[8];
#pragma unroll
        for (int jj = 0; jj < 8; jj++) x[jj] = src[(g * 8 + jj) * C::QS];
#pragma unroll
        for (int jj = 0; jj < 8; jj++) {
          acc += x[jj].x;
          acc += x[jj].y;
          acc += x[jj].z;
          acc += x[jj].w;
        }
      }
    } else if (c + 1 < n_chunks) {
      produce(c + 1, s_prod[(c + 1) & 1]);
      if (c + 2 < n_chunks) fetch(c + 2);
    }
    __syncthreads();
  }
  if (folder) {
    const size_t gi = ((size_t)i * n_heads + h) * HD + tid;
    out[gi] = acc;
    if (qd) {
      float qscale;
      int qs;
      const int qi = quantize_lane(acc, &qscale, &qs);
      qd[gi] = static_cast<int8_t>(qi);
      if ((gi & 31) == 0) {
        qsa[gi >> 5] = qscale;
        qsum[gi >> 5] = qs;
      }
    }
  }
}

template <int HD>
int launch_wide(const float* q, const uint16_t* k, const uint16_t* v, size_t pos0, size_t n_q, size_t n_heads,
                size_t n_kv_heads, float* out, const ActQuant* aq, bool* quantized, size_t kcap, hipStream_t s) {
  const bool fuse_q = aq && aq->q;  // whole heads are whole 32-blocks
  if (quantized) *quantized = fuse_q;
  hipLaunchKernelGGL(attn_wide_kernel<HD>, dim3(n_heads, n_q), dim3(kWideNT), 0, s, q, k, v, (int)pos0,
                     (int)n_heads, (int)(n_heads / n_kv_heads), out, fuse_q ? aq->q : nullptr,
                     fuse_q ? aq->sa : nullptr, fuse_q ? aq->sums : nullptr, (int)kcap);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

// ---------------------------------------------------------------- prefill blocks
// Prefill attention over the f32 K/V of the window (attention.rs:236-284)
// with one 256-lane workgroup per (head, pair of blocks of kPbQ consecutive
// query rows, one from each end of the causal window, taken one after the
// other): each K row a lane fetches serves the block's kPbQ score chains (side
// by side), and each V element a lane fetches serves kPbQ*hd/256 P·V chains.
// Row qq of the block attends keys 0..i0+qq; its softmax sum is the exact
// left-to-right fold, one row after another.
constexpr int kPbQ = 8;
constexpr int kPbNT = 256;
constexpr int kPbMax = 2048;  // window rows a block workgroup takes
constexpr int kPbW = exact::run_pad(kPbMax - 1) + 1;

// DYN: the probability rows are dynamic LDS of scw words each (windows up to
// kPbDynMax: several workgroups per CU); otherwise a static array sized for
// kPbMax positions (the compiler then keeps more of the score loop in
// registers, which long windows need more than occupancy).
constexpr size_t kPbDynMax = 1024;
template <int HD, bool DYN>
__global__ __launch_bounds__(kPbNT) void attn_prefill_blk(const float* __restrict__ q, const float* __restrict__ k,
                                                          const float* __restrict__ v, int seq, int n_heads,
                                                          int group, float* __restrict__ out,
                                                          int8_t* __restrict__ qd, float* __restrict__ qsa,
                                                          int* __restrict__ qsum, int scw_arg) {
  static_assert(HD % 4 == 0 && (kPbQ * HD) % kPbNT == 0, "whole chains per lane");
  constexpr int QPL = kPbQ * HD / kPbNT;  // P·V chains per lane
  constexpr int QSTEP = kPbNT / HD;       // query rows between a lane's chains
  __shared__ __align__(16) float s_q[kPbQ][HD];
  // the block's probability rows, scw words each (run_pad layout)
  __shared__ __align__(16) float s_sc_st[DYN ? 4 : kPbQ * kPbW];
  extern __shared__ float4 pb_smem[];
  float* s_scd = DYN ? reinterpret_cast<float*>(pb_smem) : s_sc_st;
  const int scw = DYN ? scw_arg : kPbW;
  __shared__ float s_red[kPbQ][kPbNT / 64];
  const int h = blockIdx.x, tid = threadIdx.x;
  // Workgroup y takes query blocks y and nqb-1-y (the causal window's short
  // and long ends), so every workgroup has about the same keys to cover
  const int nqb = (seq + kPbQ - 1) / kPbQ;
  for (int pass = 0; pass < 2; pass++) {
    const int qb = pass == 0 ? static_cast<int>(blockIdx.y) : nqb - 1 - static_cast<int>(blockIdx.y);
    if (pass == 1) {
      if (qb <= static_cast<int>(blockIdx.y)) break;  // uniform: an odd count's middle block, done once
      __syncthreads();  // the first block's reads of the LDS rows are done
    }
    const int i0 = qb * kPbQ;
    const int nk = min(i0 + kPbQ, seq);  // keys any row of the block attends
    const int kvh = h / group;
    const int kv_dim = (n_heads / group) * HD;
    for (int e = tid; e < kPbQ * HD; e += kPbNT) {
      const int qq = e / HD, d = e % HD;
      s_q[qq][d] = i0 + qq < seq ? q[((size_t)(i0 + qq) * n_heads + h) * HD + d] : 0.0f;
    }
    __syncthreads();
    // ---- scores: (fold_d q[d]*k_t[d] from -0.0) * (1/sqrt(hd)), lane per key row
    const float scale = 1.0f / sqrtf(static_cast<float>(HD));
    float mxl[kPbQ];
  #pragma unroll
    for (int qq = 0; qq < kPbQ; qq++) mxl[qq] = -INFINITY;
    for (int t = tid; t < nk; t += kPbNT) {
      const float4* kp = reinterpret_cast<const float4*>(k + (size_t)t * kv_dim + (size_t)kvh * HD);
      float dot[kPbQ];
  #pragma unroll
      for (int qq = 0; qq < kPbQ; qq++) dot[qq] = -0.0f;
  #pragma unroll 4
      for (int c = 0; c < HD / 4; c++) {
        const float4 kv = kp[c];
  #pragma unroll
        for (int qq = 0; qq < kPbQ; qq++) {
          const float4 qv = reinterpret_cast<const float4*>(s_q[qq])[c];
          dot[qq] += qv.x * kv.x;
          dot[qq] += qv.y * kv.y;
          dot[qq] += qv.z * kv.z;
          dot[qq] += qv.w * kv.w;
        }
      }
  #pragma unroll
      for (int qq = 0; qq < kPbQ; qq++) {
        if (t <= i0 + qq) {  // causal: row i0+qq attends keys 0..i0+qq
          const float sv = dot[qq] * scale;
          s_scd[(qq) * scw + exact::run_pad(t)] = sv;
          mxl[qq] = fmaxf(mxl[qq], sv);
        }
      }
    }
  #pragma unroll
    for (int qq = 0; qq < kPbQ; qq++) {
      const float m = wave_max_f32(mxl[qq]);
      if ((tid & 63) == 0) s_red[qq][tid >> 6] = m;
    }
    __syncthreads();
    float mx[kPbQ];
  #pragma unroll
    for (int qq = 0; qq < kPbQ; qq++) {
      mx[qq] = -INFINITY;
  #pragma unroll
      for (int w = 0; w < kPbNT / 64; w++) mx[qq] = fmaxf(mx[qq], s_red[qq][w]);
    }
  #pragma unroll
    for (int qq = 0; qq < kPbQ; qq++) {
      const int n = i0 + qq + 1;
      if (i0 + qq < seq)
        for (int t = tid; t < n; t += kPbNT) s_scd[(qq) * scw + exact::run_pad(t)] = dev_expf(s_scd[(qq) * scw + exact::run_pad(t)] - mx[qq]);
    }
    __syncthreads();
    // softmax sums in the reference's left-to-right order (norms.rs:53): each
    // wave folds one row at a time, the waves' rows at once
    __shared__ float s_inv[kPbQ];
    static_assert(kPbQ % (kPbNT / 64) == 0, "whole rounds of rows");
  #pragma unroll
    for (int r = 0; r < kPbQ / (kPbNT / 64); r++) {
      const int qq = r * (kPbNT / 64) + (tid >> 6);
      if (i0 + qq < seq) {  // wave-uniform; the group barriers are the wave's own
        const float sum =
            exact::group_seq_sum_short<64, kPbNT / 64>([s_scd, scw, qq](int t) { return s_scd[(qq) * scw + exact::run_pad(t)]; }, i0 + qq + 1);
        if ((tid & 63) == 0) s_inv[qq] = sum > 0.0f ? 1.0f / sum : 0.0f;
      } else if ((tid & 63) == 0) {
        s_inv[qq] = 0.0f;
      }
    }
    __syncthreads();
    float inv[kPbQ];
  #pragma unroll
    for (int qq = 0; qq < kPbQ; qq++) inv[qq] = s_inv[qq];
  #pragma unroll
    for (int qq = 0; qq < kPbQ; qq++) {
      const int n = i0 + qq + 1;
      if (i0 + qq < seq)
        for (int t = tid; t < n; t += kPbNT) s_scd[(qq) * scw + exact::run_pad(t)] = s_scd[(qq) * scw + exact::run_pad(t)] * inv[qq];
    }
    __syncthreads();
    // ---- P·V: lane (d, qg) folds rows qg, qg+QSTEP, ... of dim d over t from +0.0
    const int d = tid % HD, qg = tid / HD;
    const float* vcol = v + (size_t)kvh * HD + d;
    float acc[QPL];
  #pragma unroll
    for (int c = 0; c < QPL; c++) acc[c] = 0.0f;
    // rows 0..i0 are attended by every query row of the block: no causal test
    // there, so the probability and V reads of a batch issue together; only
    // the last kPbQ - 1 keys need the per-row select
    int t = 0;
    for (; t + 8 <= i0 + 1; t += 8) {
      float vt[8], pt[8][QPL];
  #pragma unroll
      for (int u = 0; u < 8; u++) vt[u] = vcol[(size_t)(t + u) * kv_dim];
  #pragma unroll
      for (int u = 0; u < 8; u++)
  #pragma unroll
        for (int c = 0; c < QPL; c++) pt[u][c] = s_scd[(qg + c * QSTEP) * scw + exact::run_pad(t + u)];
  #pragma unroll
      for (int u = 0; u < 8; u++)
  #pragma unroll
        for (int c = 0; c < QPL; c++) acc[c] = acc[c] + pt[u][c] * vt[u];
    }
    for (; t <= i0; t++) {
      const float vt = vcol[(size_t)t * kv_dim];
  #pragma unroll
      for (int c = 0; c < QPL; c++) acc[c] = acc[c] + s_scd[(qg + c * QSTEP) * scw + exact::run_pad(t)] * vt;
    }
    for (; t < nk; t++) {
      const float vt = vcol[(size_t)t * kv_dim];
  #pragma unroll
      for (int c = 0; c < QPL; c++) {
        const int qq = qg + c * QSTEP;
        const float nv = acc[c] + s_scd[(qq) * scw + exact::run_pad(t)] * vt;
        acc[c] = t <= i0 + qq ? nv : acc[c];
      }
    }
  #pragma unroll
    for (int c = 0; c < QPL; c++) {
      const int qq = qg + c * QSTEP, i = i0 + qq;
      const bool live = i < seq;
      const size_t gi = ((size_t)min(i, seq - 1) * n_heads + h) * HD + d;
      if (live) out[gi] = acc[c];
      if (qd) {  // 32-lane groups share qq (HD is a multiple of 32 here)
        float qscale;
        int qs;
        const int qi = quantize_lane(live ? acc[c] : 0.0f, &qscale, &qs);
        if (live) {
          qd[gi] = static_cast<int8_t>(qi);
          if ((gi & 31) == 0) {
            qsa[gi >> 5] = qscale;
            qsum[gi >> 5] = qs;
          }
        }
      }
    }
  }
}

template <int HD>
int launch_prefill_blk(const float* q, const float* k, const float* v, size_t seq, size_t n_heads,
                       size_t n_kv_heads, float* out, const ActQuant* aq, bool* quantized, hipStream_t s) {
  const bool fuse_q = aq && aq->q;
  if (quantized) *quantized = fuse_q;
  const size_t nqb = (seq + kPbQ - 1) / kPbQ;
  const dim3 grid(n_heads, (nqb + 1) / 2);  // a pair of query blocks per workgroup
  int8_t* qd = fuse_q ? aq->q : nullptr;
  float* qsa = fuse_q ? aq->sa : nullptr;
  int* qsum = fuse_q ? aq->sums : nullptr;
  const int group = static_cast<int>(n_heads / n_kv_heads);
  if (seq <= kPbDynMax) {
    const int scw = (exact::run_pad(static_cast<int>(seq) - 1) + 1 + 3) & ~3;  // 16-byte aligned rows
    hipLaunchKernelGGL((attn_prefill_blk<HD, true>), grid, dim3(kPbNT), (size_t)kPbQ * scw * sizeof(float), s, q, k,
                       v, (int)seq, (int)n_heads, group, out, qd, qsa, qsum, scw);
  } else {
    hipLaunchKernelGGL((attn_prefill_blk<HD, false>), grid, dim3(kPbNT), 0, s, q, k, v, (int)seq, (int)n_heads,
                       group, out, qd, qsa, qsum, 0);
  }
  PRANA_LAUNCH_CHECK();
  return kOk;
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
                                                   float* __restrict__ qsa, int* __restrict__ qsum, int kcap) {
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
  J.kcap = kcap;
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

// Largest dynamic LDS a launch may request on this device (queried once).
size_t max_dyn_lds() {
  static const size_t v = [] {
    int dev = 0, b = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&b, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
      return size_t{65536};
    return static_cast<size_t>(b);
  }();
  return v;
}

template <int HD>
int launch_split(const float* q, const uint16_t* k, const uint16_t* v, size_t pos0, const int* pos_dev, size_t n_q,
                 size_t n_heads, size_t n_kv_heads, float* out, float* scratch, size_t ctx_cap, const ActQuant* aq,
                 bool* quantized, size_t kcap, hipStream_t s) {
  const int group = static_cast<int>(n_heads / n_kv_heads);
  const int stride = static_cast<int>(split_stride(ctx_cap));
  // a position read from device memory can be anything up to the capacity:
  // the grid and the staging cover the whole window then (blocks past the
  // window return at once)
  const size_t rows = pos_dev ? ctx_cap : pos0 + n_q;
  if (n_q >= 2)  // verify: two query rows per workgroup share each K row
    hipLaunchKernelGGL(attn_split_scores_rows<HD>,
                       dim3((rows + kSplitRows - 1) / kSplitRows, (n_q + 1) / 2 * n_kv_heads * ((group + 3) / 4)),
                       dim3(kSplitRows), 0, s, q, k, (int)pos0, pos_dev, (int)n_q, (int)n_heads, group,
                       (int)n_kv_heads, scratch, stride, (int)kcap);
  else
    hipLaunchKernelGGL(attn_split_scores<HD>,
                       dim3((rows + kSplitRows - 1) / kSplitRows, n_q * n_kv_heads * ((group + 3) / 4)),
                       dim3(kSplitRows), 0, s, q, k, (int)pos0, pos_dev, (int)n_heads, group,
                       (int)n_kv_heads, scratch, stride, (int)kcap);
  PRANA_LAUNCH_CHECK();
  // the softmax stages the longest row's exponentials in LDS when they fit
  const size_t lds = (exact::run_pad(static_cast<int>(rows) - 1) + 1) * sizeof(float);
  static const size_t lds_cap = [] {
    const size_t cap = max_dyn_lds() > 16384 ? max_dyn_lds() - 16384 : 0;  // static LDS of the sum
    if (cap > 65536)
      (void)set_max_dynamic_lds(reinterpret_cast<const void*>(attn_split_softmax<true>), static_cast<int>(cap));
    return cap;
  }();
  if (lds <= lds_cap)
    hipLaunchKernelGGL(attn_split_softmax<true>, dim3(n_heads, n_q), dim3(kSmNT), lds, s, scratch, stride,
                       (int)pos0, pos_dev, (int)n_heads);
  else
    hipLaunchKernelGGL(attn_split_softmax<false>, dim3(n_heads, n_q), dim3(kSmNT), 0, s, scratch, stride,
                       (int)pos0, pos_dev, (int)n_heads);
  PRANA_LAUNCH_CHECK();
  const bool fuse_q = aq && aq->q;  // 64-dim slices are whole 32-blocks
  if (quantized) *quantized = fuse_q;
  // long chunks amortize the per-chunk barrier; short ones keep two
  // workgroups per CU when there are many
  int8_t* qd = fuse_q ? aq->q : nullptr;
  float* qsa = fuse_q ? aq->sa : nullptr;
  int* qsum = fuse_q ? aq->sums : nullptr;
  // several query rows (verify): rows of one head slice share each V chunk,
  // one 128 KB workgroup per CU, when the device grants that much LDS
  constexpr size_t kPvrLds = 2 * kPvrQR * kPvrCH * 64 * sizeof(float);
  static const bool pvr_ok =
      max_dyn_lds() >= kPvrLds &&
      set_max_dynamic_lds(reinterpret_cast<const void*>(attn_split_pv_rows<HD>), static_cast<int>(kPvrLds));
  if (n_q >= 2 && pvr_ok)
    hipLaunchKernelGGL(attn_split_pv_rows<HD>, dim3(n_heads * (HD / 64), (n_q + kPvrQR - 1) / kPvrQR),
                       dim3(64 * kPvrQR + kPvrProd), kPvrLds, s, scratch, stride, v, (int)pos0, pos_dev, (int)n_q,
                       (int)n_heads, group, out, qd, qsa, qsum);
  else if (n_heads * (HD / 64) * n_q <= 256)
    hipLaunchKernelGGL((attn_split_pv<HD, 256>), dim3(n_heads * (HD / 64), n_q), dim3(kPvNT), 0, s, scratch, stride,
                       v, (int)pos0, pos_dev, (int)n_heads, group, out, qd, qsa, qsum);
  else
    hipLaunchKernelGGL((attn_split_pv<HD, 128>), dim3(n_heads * (HD / 64), n_q), dim3(kPvNT), 0, s, scratch, stride,
                       v, (int)pos0, pos_dev, (int)n_heads, group, out, qd, qsa, qsum);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

template <bool F16>
int launch_attn(const float* q, const void* k, const void* v, size_t pos0, const int* pos_dev, size_t n_q,
                size_t n_heads, size_t n_kv_heads, size_t hd, float* out, float* scratch, size_t ctx_cap,
                const ActQuant* aq, bool* quantized, size_t kcap, hipStream_t s) {
  const size_t elem = F16 ? 2 : 4;
  const bool aligned = reinterpret_cast<uintptr_t>(k) % 16 == 0 && reinterpret_cast<uintptr_t>(v) % 16 == 0 &&
                       (hd * elem) % 16 == 0;
  // a piecewise K cache: every path below reads it through a compiled head width
  PRANA_CHECK(kcap == 0 || (F16 && aligned && (hd == 64 || hd == 128) && kcap >= pos0 + n_q &&
                            kcap <= static_cast<size_t>(INT32_MAX / 8)),
              "attention: a piecewise K cache needs aligned f16 rows of 64 or 128 dims");
  if (F16 && aligned && !pos_dev && n_q >= 2 && pos0 + n_q >= kWideMinRows && pos0 + n_q <= (size_t)kWideMax &&
      (hd == 64 || hd == 128)) {
    const uint16_t* kc = static_cast<const uint16_t*>(k);
    const uint16_t* vc = static_cast<const uint16_t*>(v);
    return hd == 64 ? launch_wide<64>(q, kc, vc, pos0, n_q, n_heads, n_kv_heads, out, aq, quantized, kcap, s)
                    : launch_wide<128>(q, kc, vc, pos0, n_q, n_heads, n_kv_heads, out, aq, quantized, kcap, s);
  }
  // with pos_dev, pos0 still picks the path (the kernels read the position)
  if (F16 && aligned && scratch && pos0 + n_q >= kSplitMinRows && (hd == 64 || hd == 128)) {
    const uint16_t* kc = static_cast<const uint16_t*>(k);
    const uint16_t* vc = static_cast<const uint16_t*>(v);
    return hd == 64 ? launch_split<64>(q, kc, vc, pos0, pos_dev, n_q, n_heads, n_kv_heads, out, scratch, ctx_cap,
                                       aq, quantized, kcap, s)
                    : launch_split<128>(q, kc, vc, pos0, pos_dev, n_q, n_heads, n_kv_heads, out, scratch, ctx_cap,
                                        aq, quantized, kcap, s);
  }
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
  LaunchEvents& le = launch_events();
  if (le.start) {  // a sampled decode launch: timestamps as part of the dispatch
    hipExtLaunchKernelGGL(attn_kernel<F16>, dim3(n_heads * ds, n_q), dim3(kNT), 0, s, le.start, le.stop, 0, q, k, v,
                          (int)pos0, pos_dev, (int)n_heads, (int)(n_heads / n_kv_heads), (int)hd, ds, out, scratch,
                          (int)ctx_cap, mode, fuse_q ? aq->q : nullptr, fuse_q ? aq->sa : nullptr,
                          fuse_q ? aq->sums : nullptr, (int)kcap);
    le = LaunchEvents{};
  } else {
    hipLaunchKernelGGL(attn_kernel<F16>, dim3(n_heads * ds, n_q), dim3(kNT), 0, s, q, k, v, (int)pos0, pos_dev,
                       (int)n_heads, (int)(n_heads / n_kv_heads), (int)hd, ds, out, scratch, (int)ctx_cap, mode,
                       fuse_q ? aq->q : nullptr, fuse_q ? aq->sa : nullptr, fuse_q ? aq->sums : nullptr, (int)kcap);
  }
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

bool attention_split_window(size_t rows, size_t hd) { return rows >= kSplitMinRows && (hd == 64 || hd == 128); }

size_t attention_scratch_floats(size_t n_q, size_t n_heads, size_t ctx_cap, bool cache) {
  // split path (cache windows): scores / probabilities of every (query row, head)
  size_t need = cache ? n_q * n_heads * split_stride(ctx_cap) : 0;
  if (ctx_cap > static_cast<size_t>(kScoreLds)) {
    size_t ds = 1;  // upper bound of attention_dim_slices
    while (n_q * n_heads * ds < 128 && ds < 4) ds *= 2;
    need = std::max(need, n_q * n_heads * ds * ctx_cap);
  }
  return need;
}

int launch_attention_cache(const float* q, const uint16_t* kc, const uint16_t* vc, size_t pos0, size_t n_q,
                           size_t n_heads, size_t n_kv_heads, size_t hd, float* out, float* scratch, size_t ctx_cap,
                           const int* pos_dev, hipStream_t s, const ActQuant* aq, bool* quantized, size_t kcap) {
  if (n_q == 0) return kOk;
  PRANA_CHECK(n_kv_heads > 0 && n_heads % n_kv_heads == 0, "attention: n_heads must be a multiple of n_kv_heads");
  PRANA_CHECK(hd > 0 && hd <= 256, "attention: head_dim must be in 1..=256");
  if (ctx_cap == 0) ctx_cap = pos0 + n_q;
  PRANA_CHECK(pos_dev || pos0 + n_q <= ctx_cap, "attention: scratch capacity below pos0 + n_q");
  return launch_attn<true>(q, kc, vc, pos0, pos_dev, n_q, n_heads, n_kv_heads, hd, out, scratch, ctx_cap, aq, quantized,
                           kcap, s);
}

int launch_attention_prefill(const float* q, const float* k, const float* v, size_t seq, size_t n_heads,
                             size_t n_kv_heads, size_t hd, float* out, float* scratch, hipStream_t s,
                             const ActQuant* aq, bool* quantized) {
  if (seq == 0) return kOk;
  PRANA_CHECK(n_kv_heads > 0 && n_heads % n_kv_heads == 0, "attention: n_heads must be a multiple of n_kv_heads");
  PRANA_CHECK(hd > 0 && hd <= 256, "attention: head_dim must be in 1..=256");
  const bool aligned = reinterpret_cast<uintptr_t>(q) % 16 == 0 && reinterpret_cast<uintptr_t>(k) % 16 == 0;
  if (aligned && seq <= (size_t)kPbMax && seq >= 2 * kPbQ && (hd == 64 || hd == 128)) {
    return hd == 64 ? launch_prefill_blk<64>(q, k, v, seq, n_heads, n_kv_heads, out, aq, quantized, s)
                    : launch_prefill_blk<128>(q, k, v, seq, n_heads, n_kv_heads, out, aq, quantized, s);
  }
  return launch_attn<false>(q, k, v, 0, nullptr, seq, n_heads, n_kv_heads, hd, out, scratch, seq, aq, quantized, 0, s);
}

}  // namespace prana
