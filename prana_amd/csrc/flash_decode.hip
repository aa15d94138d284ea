// Split-K flash decoding over the f16 KV cache: the attention of
// attention_decode (attention.rs:129-195) for independent sequences with long
// windows, evaluated in tiles of cache rows whose partial softmax states are
// merged afterwards. The f32 result is within 1e-4 relative of the
// reference's sequential order (it is not bit-identical: the score dots, the
// softmax sum and the P.V fold are reassociated); the exact one-query kernels
// in attention.hip remain the path of the model's decode.
//
//   split  : one workgroup per (tile of T cache rows, KV head and block of
//            up to GB of its query heads, sequence). A K or V row of one KV
//            head is read once per head block, coalesced (HDP/8 lanes x 16
//            bytes, HDP = the head width rounded up to 64, 128 or 256; lanes
//            past the width load nothing), and serves the block's query
//            heads: every lane holds 8 dims of q for each of them, the
//            partial dots of a row are reduced over its lanes with DPP; each
//            wave keeps its own max, sum of exp(s - max) and P.V per head in
//            registers, and the four waves are merged once at the end of the
//            tile. Any group size (heads per KV head) and any head width that
//            is a multiple of 8, up to 256.
//   combine: one workgroup per (query head, sequence, 32 dims):
//            M = max m_s, L = sum l_s exp(m_s - M),
//            out = sum acc_s exp(m_s - M) / L, in parallel over splits.
// Every K/V byte is read once, with all of a tile's loads in flight at once,
// so the split kernel is bound by HBM bandwidth. Products are fused
// (explicit fmaf): this path is not held to the reference's rounding.
#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace prana {

// Partial-state scratch of prana_attention_decode_splitk_noalloc: a fixed
// array in device memory (one copy per GPU, held until the process ends).
// Host code never uses the array's name as an address: the device address
// comes from hipGetSymbolAddress, looked up once per device at set-up
// (flash_noalloc_setup, called by the library's init with the device
// current) and kept in g_scratch_dev.
static __device__ __align__(256) float scratch[kFlashNoAllocFloats];

namespace {
constexpr int kMaxDevices = 16;
float* g_scratch_dev[kMaxDevices] = {};
}  // namespace

int flash_noalloc_setup(int device) {
  if (device < 0 || device >= kMaxDevices) return fail(kErrUnsupported, "flash scratch: device index out of range");
  if (g_scratch_dev[device]) return kOk;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
  if (!p) return fail(kErrHip, "hipGetSymbolAddress(scratch) returned a null address");
  g_scratch_dev[device] = static_cast<float*>(p);
  return kOk;
}

float* flash_noalloc_scratch(int device) {
  return device >= 0 && device < kMaxDevices ? g_scratch_dev[device] : nullptr;
}

namespace {

constexpr int kFdNT = 256;  // lanes per split workgroup (4 waves)
constexpr int kFdMaxSeq = 16;

struct FlashArgs {
  const float* q;  // [n_seq][n_heads * hd], RoPE applied
  const uint16_t* kc[kFdMaxSeq];
  const uint16_t* vc[kFdMaxSeq];
  int pos[kFdMaxSeq];  // attends to rows 0..=pos of sequence s
  int n_heads, n_kv_heads, max_splits, rows_per_split;
  int hd, group, head_blocks;  // head width, query heads per KV head, blocks of GB of them
  float scale;  // 1 / sqrt(hd), as attention.rs:172 computes it
  float* part;  // [n_seq][n_heads][max_splits][hd + 2]: acc[hd], m, l
};

// 16 bytes of the cache, loaded non-temporally: every K/V byte is read once,
// so the lines are not kept for reuse.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream(const uint16_t* p) {
  const u32x4_t t = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(t.x, t.y, t.z, t.w);
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over aligned groups of LPR lanes (8, 16 or 32), every lane getting it.
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
  v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);  // row_half_mirror: the other quad of the 8-lane half
  if constexpr (LPR >= 16) v += dpp_f<0x140>(v);  // row_mirror: the other half of the row
  if constexpr (LPR == 32) v += __shfl_xor(v, 16, 64);  // the other row of the 32-lane group
  return v;
}

__device__ __forceinline__ void halves8(const uint4& w, float* x) {
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int k = 0; k < 4; k++) {
    x[2 * k] = f16_operand(static_cast<uint16_t>(u[k] & 0xffffu));
    x[2 * k + 1] = f16_operand(static_cast<uint16_t>(u[k] >> 16));
  }
}

// HD: the padded head width (64, 128 or 256; a.hd <= HD is the real one, a
// multiple of 8); G: query heads per workgroup (the block of a KV head's
// group, a.group of them in all: block b takes heads b*G .. b*G+G-1 of the
// group, those past a.group are computed on a valid head and not stored);
// ITER: rows each lane group takes per tile (T = 4 waves * ITER * 512/HD rows).
template <int HD, int G, int ITER>
__global__ __launch_bounds__(kFdNT) void flash_split_kernel(FlashArgs a) {
  constexpr int LPR = HD / 8;      // lanes per cache row
  constexpr int RPI = 64 / LPR;    // rows per wave per iteration
  constexpr int T = 4 * ITER * RPI;
  __shared__ float s_m[4][G], s_l[4][G];
  __shared__ float s_acc[4][G][HD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rg = lane / LPR, sub = lane % LPR;
  const int split = blockIdx.x, seq = blockIdx.z;
  const int kvh = blockIdx.y / a.head_blocks, hblk = blockIdx.y % a.head_blocks;
  const int n = a.pos[seq] + 1;
  const int r0 = split * T;
  if (r0 >= n) return;  // uniform: past this sequence's window
  const int hd = a.hd;
  const bool live = sub * 8 < hd;  // this lane's 8 dims lie inside the head
  const int kv_stride = a.n_kv_heads * hd;
  const uint16_t* kb = a.kc[seq] + (size_t)kvh * hd + sub * 8;
  const uint16_t* vb = a.vc[seq] + (size_t)kvh * hd + sub * 8;
  const int wrow0 = r0 + wave * ITER * RPI + rg;  // this lane group's first row
  // every K and V load of the tile in flight at once (rows past the window
  // read row n-1 and are masked below; lanes past the width read nothing)
  uint4 kr[ITER], vr[ITER];
#pragma unroll
  for (int it = 0; it < ITER; it++) {
    const int row = min(wrow0 + it * RPI, n - 1);
    kr[it] = live ? ld_stream(kb + (size_t)row * kv_stride) : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int it = 0; it < ITER; it++) {
    const int row = min(wrow0 + it * RPI, n - 1);
    vr[it] = live ? ld_stream(vb + (size_t)row * kv_stride) : make_uint4(0, 0, 0, 0);
  }
  float qv[G][8];
  const int gb0 = hblk * G;                       // first head of the block within the group
  const int h0 = kvh * a.group + gb0;             // its query head index
  const int nh_here = min(G, a.group - gb0);      // heads of the block inside the group
#pragma unroll
  for (int g = 0; g < G; g++) {
    const int h = h0 + min(g, nh_here - 1);
    if (live) {
      const float4* qp = reinterpret_cast<const float4*>(a.q + ((size_t)seq * a.n_heads + h) * hd + sub * 8);
      const float4 x0 = qp[0], x1 = qp[1];
      qv[g][0] = x0.x; qv[g][1] = x0.y; qv[g][2] = x0.z; qv[g][3] = x0.w;
      qv[g][4] = x1.x; qv[g][5] = x1.y; qv[g][6] = x1.z; qv[g][7] = x1.w;
    } else {
#pragma unroll
      for (int k = 0; k < 8; k++) qv[g][k] = 0.0f;
    }
#pragma unroll
    for (int k = 0; k < 8; k++) qv[g][k] *= a.scale;  // (q/sqrt(hd)).k
  }
  const bool full = r0 + T <= n;  // uniform: no row of the tile lies past the window
  // scores: after the group sum every lane of a row's group holds its G dots
  float sc[G][ITER], mx[G];
#pragma unroll
  for (int g = 0; g < G; g++) mx[g] = -INFINITY;
#pragma unroll
  for (int it = 0; it < ITER; it++) {
    float k8[8];
    halves8(kr[it], k8);
    const bool valid = full || wrow0 + it * RPI < n;
#pragma unroll
    for (int g = 0; g < G; g++) {
      float d = 0.0f;
#pragma unroll
      for (int k = 0; k < 8; k++) d = fmaf(qv[g][k], k8[k], d);
      d = group_sum<LPR>(d);
      sc[g][it] = valid ? d : -INFINITY;
      mx[g] = fmaxf(mx[g], sc[g][it]);
    }
  }
  // each wave keeps its own softmax state (max, sum of exp(s - max), P.V);
  // the four are merged once at the end
  float ls[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; g++) {
#pragma unroll
    for (int o = LPR; o < 64; o <<= 1) mx[g] = fmaxf(mx[g], __shfl_xor(mx[g], o, 64));
    // a wave whose rows all lie past the window has max -inf: its
    // probabilities are exp(-inf) = 0 against a reference of 0
    const float mref = mx[g] == -INFINITY ? 0.0f : mx[g];
    ls[g] = 0.0f;
#pragma unroll
    for (int it = 0; it < ITER; it++) {
      sc[g][it] = __expf(sc[g][it] - mref);
      ls[g] += sc[g][it];
    }
#pragma unroll
    for (int k = 0; k < 8; k++) acc[g][k] = 0.0f;
  }
#pragma unroll
  for (int it = 0; it < ITER; it++) {
    if (full || wrow0 + it * RPI < n) {
      float v8[8];
      halves8(vr[it], v8);
#pragma unroll
      for (int g = 0; g < G; g++)
#pragma unroll
        for (int k = 0; k < 8; k++) acc[g][k] = fmaf(sc[g][it], v8[k], acc[g][k]);
    }
  }
  // sum the wave's lane groups (lanes LPR apart)
#pragma unroll
  for (int o = LPR; o < 64; o <<= 1)
#pragma unroll
    for (int g = 0; g < G; g++) {
      ls[g] += __shfl_xor(ls[g], o, 64);
#pragma unroll
      for (int k = 0; k < 8; k++) acc[g][k] += __shfl_xor(acc[g][k], o, 64);
    }
  if (rg == 0)
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
      for (int k = 0; k < 8; k++) s_acc[wave][g][sub * 8 + k] = acc[g][k];  // (zeros past the width)
  if (lane == 0)
#pragma unroll
    for (int g = 0; g < G; g++) {
      s_m[wave][g] = mx[g];
      s_l[wave][g] = ls[g];
    }
  __syncthreads();
  // merge the waves: M = max m_w, each state scaled by exp(m_w - M) (0 for a
  // wave past the window; wave 0 holds row r0 < n, so M is finite)
  float* base = a.part + (((size_t)seq * a.n_heads + h0) * a.max_splits + split) * (hd + 2);
  const size_t hstride = (size_t)a.max_splits * (hd + 2);
  for (int e = tid; e < G * HD; e += kFdNT) {
    const int g = e / HD, d = e % HD;
    if (g >= nh_here || d >= hd) continue;
    const float M = fmaxf(fmaxf(s_m[0][g], s_m[1][g]), fmaxf(s_m[2][g], s_m[3][g]));
    float o = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; w++)
      if (s_m[w][g] != -INFINITY) o = fmaf(s_acc[w][g][d], __expf(s_m[w][g] - M), o);
    base[g * hstride + d] = o;
  }
  if (tid < nh_here) {
    const float M = fmaxf(fmaxf(s_m[0][tid], s_m[1][tid]), fmaxf(s_m[2][tid], s_m[3][tid]));
    float l = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; w++)
      if (s_m[w][tid] != -INFINITY) l = fmaf(s_l[w][tid], __expf(s_m[w][tid] - M), l);
    base[tid * hstride + hd] = M;
    base[tid * hstride + hd + 1] = l;
  }
}

struct CombineArgs {
  const float* part;
  int n_splits[kFdMaxSeq];
  int n_heads, max_splits;
  float* out;
};

constexpr int kFcNT = 256;
constexpr int kFcDims = 32;             // output dims per combine workgroup
constexpr int kFcPG = kFcNT / kFcDims;  // split groups per dim
constexpr int kFcBatch = 16;            // splits per lane whose loads are in flight together

// One workgroup per (query head, sequence, 32 output dims). Lane (g, d) takes
// splits g, g+8, ...: a batch of their acc[d] and m values is loaded before
// the maxima are known, so the kernel waits on memory about twice, not once
// per split. M = max m_s; L = sum l_s exp(m_s - M);
// out[d] = (sum_s acc_s[d] exp(m_s - M)) / L.
__global__ __launch_bounds__(kFcNT) void flash_combine_kernel(CombineArgs c, int hd) {
  __shared__ float s_r[kFcNT / 64];
  __shared__ float s_o[kFcPG][kFcDims];
  const int h = blockIdx.x, seq = blockIdx.y, d0 = blockIdx.z * kFcDims;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int dl = tid % kFcDims, pg = tid / kFcDims;
  const int rec = hd + 2;
  const float* p = c.part + ((size_t)seq * c.n_heads + h) * c.max_splits * rec;
  const int ns = c.n_splits[seq];
  float av[kFcBatch], mv[kFcBatch];
  auto load_batch = [&](int sp0) {
#pragma unroll
    for (int k = 0; k < kFcBatch; k++) {
      const int sp = min(sp0 + k * kFcPG, ns - 1);
      av[k] = p[(size_t)sp * rec + min(d0 + dl, hd - 1)];
      mv[k] = p[(size_t)sp * rec + hd];
    }
  };
  load_batch(pg);
  float M = -INFINITY, lm[4], ll[4];
  for (int sp0 = tid; sp0 < ns; sp0 += 4 * kFcNT) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int sp = min(sp0 + k * kFcNT, ns - 1);
      lm[k] = p[(size_t)sp * rec + hd];
      ll[k] = p[(size_t)sp * rec + hd + 1];
    }
#pragma unroll
    for (int k = 0; k < 4; k++) M = fmaxf(M, lm[k]);
  }
  for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
  if (lane == 0) s_r[wave] = M;
  __syncthreads();
  M = s_r[0];
#pragma unroll
  for (int w = 1; w < kFcNT / 64; w++) M = fmaxf(M, s_r[w]);
  __syncthreads();  // s_r is reused for L
  float L = 0.0f;
  for (int sp0 = tid; sp0 < ns; sp0 += 4 * kFcNT) {
    if (sp0 != tid || ns > 4 * kFcNT) {  // the first pass's values are still in registers otherwise
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int sp = min(sp0 + k * kFcNT, ns - 1);
        lm[k] = p[(size_t)sp * rec + hd];
        ll[k] = p[(size_t)sp * rec + hd + 1];
      }
    }
#pragma unroll
    for (int k = 0; k < 4; k++)
      if (sp0 + k * kFcNT < ns) L = fmaf(ll[k], __expf(lm[k] - M), L);
  }
  for (int o = 32; o > 0; o >>= 1) L += __shfl_xor(L, o, 64);
  if (lane == 0) s_r[wave] = L;
  __syncthreads();
  L = 0.0f;
#pragma unroll
  for (int w = 0; w < kFcNT / 64; w++) L += s_r[w];
  float o = 0.0f;
  for (int sp0 = pg; sp0 < ns; sp0 += kFcBatch * kFcPG) {
    if (sp0 != pg) load_batch(sp0);
#pragma unroll
    for (int k = 0; k < kFcBatch; k++)
      if (sp0 + k * kFcPG < ns) o = fmaf(av[k], __expf(mv[k] - M), o);
  }
  s_o[pg][dl] = o;
  __syncthreads();
  if (tid < kFcDims && d0 + tid < hd) {
    float t = 0.0f;
#pragma unroll
    for (int g = 0; g < kFcPG; g++) t += s_o[g][tid];
    c.out[((size_t)seq * c.n_heads + h) * hd + d0 + tid] = t / L;
  }
}

template <int HD, int G, int ITER>
int launch_flash_t(FlashArgs a, const CombineArgs& c, int n_seq, hipStream_t s) {
  a.head_blocks = (a.group + G - 1) / G;
  hipLaunchKernelGGL((flash_split_kernel<HD, G, ITER>), dim3(a.max_splits, a.n_kv_heads * a.head_blocks, n_seq),
                     dim3(kFdNT), 0, s, a);
  PRANA_LAUNCH_CHECK();
  hipLaunchKernelGGL(flash_combine_kernel, dim3(a.n_heads, n_seq, (a.hd + kFcDims - 1) / kFcDims), dim3(kFcNT), 0, s,
                     c, a.hd);
  PRANA_LAUNCH_CHECK();
  return kOk;
}

template <int HD, int G>
int launch_flash_g(const FlashArgs& a, const CombineArgs& c, int iter, int n_seq, hipStream_t s) {
  if (iter == 16) return launch_flash_t<HD, G, 8>(a, c, n_seq, s);
  return launch_flash_t<HD, G, 4>(a, c, n_seq, s);
}

// Heads per workgroup: the group itself when it is 1, 2 or 4, else blocks of
// 8 (a group of 3 takes one block of 4; 5-7 one of 8, the spare heads
// computed and not stored; larger groups several blocks of 8).
template <int HD>
int launch_flash_hd(const FlashArgs& a, const CombineArgs& c, int g, int iter, int n_seq, hipStream_t s) {
  if (g == 1) return launch_flash_g<HD, 1>(a, c, iter, n_seq, s);
  if (g == 2) return launch_flash_g<HD, 2>(a, c, iter, n_seq, s);
  if (g <= 4) return launch_flash_g<HD, 4>(a, c, iter, n_seq, s);
  return launch_flash_g<HD, 8>(a, c, iter, n_seq, s);
}

}  // namespace

// The head width the split kernel's lanes cover: 64, 128 or 256.
static size_t flash_padded_hd(size_t hd) { return hd <= 64 ? 64 : hd <= 128 ? 128 : 256; }

// Tile size: long windows take T = 4 waves * 8 rows per lane group (small
// enough in registers for several workgroups per CU, whose load and compute
// phases then overlap); shorter ones half that, so the grid still spreads
// over the CUs.
FlashPlan flash_decode_plan(const size_t* pos, size_t n_seq, size_t n_heads, size_t n_kv_heads, size_t hd) {
  FlashPlan p{};
  const int rpi = static_cast<int>(512 / flash_padded_hd(hd));
  size_t max_rows = 0;
  for (size_t i = 0; i < n_seq; i++) max_rows = std::max(max_rows, pos[i] + 1);
  const int big_iter = 8;
  const size_t t_big = static_cast<size_t>(4 * big_iter * rpi);
  const size_t wgs_big = (max_rows + t_big - 1) / t_big * n_kv_heads * n_seq;
  p.iter = wgs_big >= 512 ? 16 : 4;
  p.rows_per_split = p.iter == 16 ? static_cast<int>(t_big) : 4 * 4 * rpi;
  p.max_splits = static_cast<int>((max_rows + p.rows_per_split - 1) / p.rows_per_split);
  p.scratch_floats = n_seq * n_heads * static_cast<size_t>(p.max_splits) * (hd + 2);
  return p;
}

int launch_flash_decode(const float* q, const uint16_t* const* k_caches, const uint16_t* const* v_caches,
                        const size_t* pos, size_t n_seq, size_t n_heads, size_t n_kv_heads, size_t hd, float* out,
                        float* part_buf, size_t part_floats, hipStream_t s) {
  PRANA_CHECK(n_seq >= 1 && n_seq <= static_cast<size_t>(kFdMaxSeq), "flash decode: 1..16 sequences per call");
  PRANA_CHECK(n_kv_heads > 0 && n_heads % n_kv_heads == 0, "flash decode: n_heads must be a multiple of n_kv_heads");
  PRANA_CHECK(hd > 0 && hd <= 256 && hd % 8 == 0, "flash decode: head_dim must be a multiple of 8 up to 256");
  PRANA_CHECK(q && out && k_caches && v_caches && pos && part_buf, "flash decode: null argument");
  const FlashPlan plan = flash_decode_plan(pos, n_seq, n_heads, n_kv_heads, hd);
  PRANA_CHECK(part_floats >= plan.scratch_floats, "flash decode: partial-state buffer below the plan's size");
  FlashArgs a{};
  CombineArgs c{};
  a.q = q;
  for (size_t i = 0; i < n_seq; i++) {
    PRANA_CHECK(k_caches[i] && v_caches[i], "flash decode: null cache pointer");
    PRANA_CHECK(reinterpret_cast<uintptr_t>(k_caches[i]) % 16 == 0 && reinterpret_cast<uintptr_t>(v_caches[i]) % 16 == 0,
                "flash decode: caches must be 16-byte aligned");
    PRANA_CHECK(pos[i] < 0x7fffffffu, "flash decode: position out of range");
    a.kc[i] = k_caches[i];
    a.vc[i] = v_caches[i];
    a.pos[i] = static_cast<int>(pos[i]);
    c.n_splits[i] = static_cast<int>((pos[i] + plan.rows_per_split) / plan.rows_per_split);
  }
  a.n_heads = static_cast<int>(n_heads);
  a.n_kv_heads = static_cast<int>(n_kv_heads);
  a.max_splits = plan.max_splits;
  a.rows_per_split = plan.rows_per_split;
  a.hd = static_cast<int>(hd);
  a.group = static_cast<int>(n_heads / n_kv_heads);
  a.scale = 1.0f / sqrtf(static_cast<float>(hd));
  a.part = part_buf;
  c.part = part_buf;
  c.n_heads = a.n_heads;
  c.max_splits = a.max_splits;
  c.out = out;
  const int g = a.group;
  const size_t hdp = flash_padded_hd(hd);
  if (hdp == 256) return launch_flash_hd<256>(a, c, g, plan.iter, static_cast<int>(n_seq), s);
  if (hdp == 128) return launch_flash_hd<128>(a, c, g, plan.iter, static_cast<int>(n_seq), s);
  return launch_flash_hd<64>(a, c, g, plan.iter, static_cast<int>(n_seq), s);
}

}  // namespace prana
