// Block encoders and seeded synthetic weights for random-init models: the
// fixture side of the tests and the benchmark, built as its own host-only
// library (libprana_synth.so) so the product library carries no encoders.
//
// The reference ships no Q8_0 / Q4_0 encoder (its quantize_q8 stores f32
// scales, matmul.rs:61-84, and Q4_0 is decode-only), so Q8_0 / Q4_0 follow the
// usual ggml reference encoders (amax/127 with f16 d and round-half-away q;
// d = max/-8 with q = min(15, trunc(x/d + 8.5))). Q4_K / Q6_K follow the
// reference's own converter (scripts/convert-to-gguf.py:29-89), which computes
// in Python floats (f64) with round-half-even and packs f16 from f64.
#include "prana_synth.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

namespace prana_synth {

namespace {

constexpr int kOk = 0, kErrInvalid = -1, kErrUnsupported = -4;

std::string& last_error() {
  thread_local std::string e;
  return e;
}

int fail(int code, const char* msg) {
  last_error() = msg;
  return code;
}

#define SYNTH_CHECK(cond, msg)                 \
  do {                                         \
    if (!(cond)) return fail(kErrInvalid, msg); \
  } while (0)

uint16_t f32_to_f16_host(float x) {  // lib.rs:78-113
  uint32_t bits;
  std::memcpy(&bits, &x, 4);
  uint16_t sign = static_cast<uint16_t>((bits >> 16) & 0x8000u);
  int exp = static_cast<int>((bits >> 23) & 0xffu);
  uint32_t frac = bits & 0x7fffffu;
  if (exp == 0xff) return sign | 0x7c00u | (frac ? 0x0200u : 0u);
  int e = exp - 127 + 15;
  if (e >= 0x1f) return sign | 0x7c00u;
  if (e <= 0) {
    if (e < -10) return sign;
    uint32_t m = frac | 0x800000u;
    uint32_t shift = static_cast<uint32_t>(14 - e);
    uint16_t half = static_cast<uint16_t>(m >> shift);
    uint32_t rb = 1u << (shift - 1);
    uint32_t rem = m & (rb * 2 - 1);
    int round = rem > rb || (rem == rb && (half & 1));
    return sign | static_cast<uint16_t>(half + round);
  }
  uint16_t half = static_cast<uint16_t>((static_cast<uint32_t>(e) << 10) | (frac >> 13));
  uint32_t rem = frac & 0x1fffu;
  int round = rem > 0x1000u || (rem == 0x1000u && (half & 1));
  return sign | static_cast<uint16_t>(half + round);
}

// f64 -> f16 bits, round-half-even directly from f64 (Python struct 'e').
uint16_t f64_to_f16_host(double x) {
  uint16_t sign = std::signbit(x) ? 0x8000u : 0u;
  double a = std::fabs(x);
  if (std::isnan(x)) return sign | 0x7e00u;
  if (a < 0x1p-14) return sign | static_cast<uint16_t>(std::nearbyint(a * 0x1p24));
  int e;
  (void)std::frexp(a, &e);  // a = f * 2^e, f in [0.5, 1)  => unbiased exponent e-1
  int E = e - 1;
  double m = std::nearbyint(std::ldexp(a, 10 - E));  // in [1024, 2048]
  if (m >= 2048.0) {
    m = 1024.0;
    E += 1;
  }
  if (E + 15 >= 31) return sign | 0x7c00u;
  return sign | static_cast<uint16_t>(((E + 15) << 10) | (static_cast<int>(m) - 1024));
}

void put16(uint8_t* p, uint16_t v) {
  p[0] = static_cast<uint8_t>(v & 0xff);
  p[1] = static_cast<uint8_t>(v >> 8);
}

void enc_q8_0(const float* x, uint8_t* out) {
  float amax = 0.0f;
  for (int j = 0; j < 32; j++) amax = std::max(amax, std::fabs(x[j]));
  float d = amax / 127.0f;
  float id = d != 0.0f ? 1.0f / d : 0.0f;
  put16(out, f32_to_f16_host(d));
  for (int j = 0; j < 32; j++) out[2 + j] = static_cast<uint8_t>(static_cast<int8_t>(std::roundf(x[j] * id)));
}

void enc_q4_0(const float* x, uint8_t* out) {
  float amax = 0.0f, mx = 0.0f;
  for (int j = 0; j < 32; j++) {
    float v = x[j];
    if (amax < std::fabs(v)) {
      amax = std::fabs(v);
      mx = v;
    }
  }
  float d = mx / -8.0f;
  float id = d != 0.0f ? 1.0f / d : 0.0f;
  put16(out, f32_to_f16_host(d));
  for (int j = 0; j < 16; j++) {
    float x0 = x[j] * id, x1 = x[16 + j] * id;
    int xi0 = std::min(15, static_cast<int>(static_cast<int8_t>(x0 + 8.5f)));
    int xi1 = std::min(15, static_cast<int>(static_cast<int8_t>(x1 + 8.5f)));
    out[2 + j] = static_cast<uint8_t>(xi0 | (xi1 << 4));
  }
}

// convert-to-gguf.py:29-60 (q4k_encode_block), Python-float semantics.
void enc_q4_k(const float* xf, uint8_t* out) {
  double v[256];
  for (int i = 0; i < 256; i++) v[i] = xf[i];
  double scs[8], ms[8];
  for (int g = 0; g < 8; g++) {
    double vmin = v[g * 32], vmax = v[g * 32];
    for (int l = 1; l < 32; l++) {  // Python min()/max(): first extreme wins
      if (v[g * 32 + l] < vmin) vmin = v[g * 32 + l];
      if (v[g * 32 + l] > vmax) vmax = v[g * 32 + l];
    }
    double nv = -vmin;
    double m = nv > 0.0 ? nv : 0.0;  // max(0.0, -vmin)
    double t = (vmax + m) / 15;
    scs[g] = t > 0.0 ? t : 0.0;
    ms[g] = m;
  }
  double mxs = scs[0], mxm = ms[0];
  for (int g = 1; g < 8; g++) {
    if (scs[g] > mxs) mxs = scs[g];
    if (ms[g] > mxm) mxm = ms[g];
  }
  double d = mxs / 63;
  if (d == 0.0) d = 1e-12;
  double dmin = mxm / 63;
  if (dmin == 0.0) dmin = 1e-12;
  int ls[8], lm[8];
  for (int g = 0; g < 8; g++) {
    ls[g] = static_cast<int>(std::min(63.0, std::max(0.0, std::nearbyint(scs[g] / d))));
    lm[g] = static_cast<int>(std::min(63.0, std::max(0.0, std::nearbyint(ms[g] / dmin))));
  }
  put16(out, f64_to_f16_host(d));
  put16(out + 2, f64_to_f16_host(dmin));
  uint8_t* sc = out + 4;
  for (int j = 0; j < 4; j++) {
    sc[j] = static_cast<uint8_t>((ls[j] & 63) | ((ls[j + 4] >> 4) << 6));
    sc[j + 4] = static_cast<uint8_t>((lm[j] & 63) | ((lm[j + 4] >> 4) << 6));
    sc[j + 8] = static_cast<uint8_t>((ls[j + 4] & 0xF) | ((lm[j + 4] & 0xF) << 4));
  }
  uint8_t* qs = out + 16;
  std::memset(qs, 0, 128);
  for (int pair = 0; pair < 4; pair++)
    for (int kind = 0; kind < 2; kind++) {
      int g = pair * 2 + kind;
      double d1 = d * ls[g], m1 = dmin * lm[g];
      for (int l = 0; l < 32; l++) {
        int q = 0;
        if (d1 > 0.0) q = static_cast<int>(std::min(15.0, std::max(0.0, std::nearbyint((v[g * 32 + l] + m1) / d1))));
        qs[pair * 32 + l] |= static_cast<uint8_t>(q << (4 * kind));
      }
    }
}

// convert-to-gguf.py:63-89 (q6k_encode_block).
void enc_q6_k(const float* xf, uint8_t* out) {
  double v[256];
  for (int i = 0; i < 256; i++) v[i] = xf[i];
  double s16[16];
  for (int s = 0; s < 16; s++) {
    int half = s / 8, w = s % 8;
    int base = half * 128 + (w / 2) * 32 + (w % 2) * 16;
    double mx = std::fabs(v[base]);
    for (int i = 1; i < 16; i++)
      if (std::fabs(v[base + i]) > mx) mx = std::fabs(v[base + i]);
    s16[s] = mx / 31;
  }
  double mxs = s16[0];
  for (int s = 1; s < 16; s++)
    if (s16[s] > mxs) mxs = s16[s];
  double d = mxs / 127;
  if (d == 0.0) d = 1e-12;
  int ls[16];
  for (int s = 0; s < 16; s++) ls[s] = static_cast<int>(std::min(127.0, std::max(1.0, std::nearbyint(s16[s] / d))));
  auto q6 = [&](double x, int s) -> int {
    double eff = d * ls[s];
    if (!(eff > 0.0)) return 32;
    double r = std::nearbyint(x / eff) + 32;
    return static_cast<int>(std::min(63.0, std::max(0.0, r)));
  };
  uint8_t* ql = out;
  uint8_t* qh = out + 128;
  for (int half = 0; half < 2; half++)
    for (int l = 0; l < 32; l++) {
      int sub = half * 8 + l / 16;
      int qs[4];
      for (int g = 0; g < 4; g++) qs[g] = q6(v[half * 128 + g * 32 + l], sub + g * 2);
      ql[half * 64 + l] = static_cast<uint8_t>((qs[0] & 0xF) | ((qs[2] & 0xF) << 4));
      ql[half * 64 + l + 32] = static_cast<uint8_t>((qs[1] & 0xF) | ((qs[3] & 0xF) << 4));
      qh[half * 32 + l] =
          static_cast<uint8_t>((qs[0] >> 4) | ((qs[1] >> 4) << 2) | ((qs[2] >> 4) << 4) | ((qs[3] >> 4) << 6));
    }
  for (int s = 0; s < 16; s++) out[192 + s] = static_cast<uint8_t>(static_cast<int8_t>(ls[s]));
  put16(out + 208, f64_to_f16_host(d));
}

int block_shape(int t, size_t& bv, size_t& bb) {
  switch (t) {
    case 0: bv = 1; bb = 4; return kOk;
    case 1: bv = 1; bb = 2; return kOk;
    case 2: bv = 32; bb = 18; return kOk;
    case 8: bv = 32; bb = 34; return kOk;
    case 12: bv = 256; bb = 144; return kOk;
    case 14: bv = 256; bb = 210; return kOk;
  }
  return fail(kErrUnsupported, "unsupported ggml type");
}

void encode_blocks(int t, const float* src, size_t n_blocks, uint8_t* out) {
  for (size_t b = 0; b < n_blocks; b++) {
    switch (t) {
      case 0: std::memcpy(out + b * 4, src + b, 4); break;
      case 1: put16(out + b * 2, f32_to_f16_host(src[b])); break;
      case 2: enc_q4_0(src + b * 32, out + b * 18); break;
      case 8: enc_q8_0(src + b * 32, out + b * 34); break;
      case 12: enc_q4_k(src + b * 256, out + b * 144); break;
      case 14: enc_q6_k(src + b * 256, out + b * 210); break;
    }
  }
}

unsigned n_workers() {
  unsigned n = std::thread::hardware_concurrency();
  return std::max(1u, std::min(n ? n : 1u, 16u));
}

template <class F>
void parallel_chunks(size_t n_chunks, F&& f) {
  unsigned nw = std::min<size_t>(n_workers(), n_chunks ? n_chunks : 1);
  if (nw <= 1) {
    for (size_t c = 0; c < n_chunks; c++) f(c);
    return;
  }
  std::vector<std::thread> th;
  for (unsigned w = 0; w < nw; w++)
    th.emplace_back([&, w] {
      for (size_t c = w; c < n_chunks; c += nw) f(c);
    });
  for (auto& t : th) t.join();
}

// splitmix64 (seed mixing) and xorshift64* (sampler.rs:51-71 XorShift).
uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}
struct XorShift {
  uint64_t s;
  explicit XorShift(uint64_t seed) : s(seed ? seed : 1) {}
  uint64_t next() {
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    return s * 0x2545F4914F6CDD1Dull;
  }
  uint32_t u24() { return static_cast<uint32_t>(next() >> 40); }
};

constexpr size_t kChunk = 65536;  // values per independently seeded stream

void fill_chunk(uint64_t seed, size_t c, float sigma, float* out, size_t n) {
  XorShift rng(splitmix64(seed ^ splitmix64(c + 1)));
  for (size_t i = 0; i < n; i += 2) {
    float u1 = static_cast<float>(rng.u24() + 1) * 5.9604644775390625e-08f;  // (0, 1]
    float u2 = static_cast<float>(rng.u24()) * 5.9604644775390625e-08f;      // [0, 1)
    float r = std::sqrt(-2.0f * std::log(u1));
    float th = 6.2831855f * u2;
    out[i] = r * std::cos(th) * sigma;
    if (i + 1 < n) out[i + 1] = r * std::sin(th) * sigma;
  }
}

}  // namespace

int quantize_tensor(int t, const float* src, size_t rows, size_t cols, uint8_t* out, size_t nbytes) {
  size_t bv, bb;
  int rc = block_shape(t, bv, bb);
  if (rc) return rc;
  SYNTH_CHECK(cols % bv == 0, "quantize_tensor: cols not a multiple of the block width");
  size_t n = rows * cols;
  SYNTH_CHECK(nbytes >= n / bv * bb, "quantize_tensor: output buffer too small");
  size_t blocks = n / bv;
  size_t per = std::max<size_t>(1, kChunk / bv);
  parallel_chunks((blocks + per - 1) / per, [&](size_t c) {
    size_t b0 = c * per, b1 = std::min(blocks, b0 + per);
    encode_blocks(t, src + b0 * bv, b1 - b0, out + b0 * bb);
  });
  return kOk;
}

void synth_normal(uint64_t seed, float sigma, float* out, size_t n) {
  parallel_chunks((n + kChunk - 1) / kChunk, [&](size_t c) {
    size_t i0 = c * kChunk;
    fill_chunk(seed, c, sigma, out + i0, std::min(kChunk, n - i0));
  });
}

int synth_tensor(int t, size_t rows, size_t cols, uint64_t seed, float sigma, uint8_t* out, size_t nbytes) {
  size_t bv, bb;
  int rc = block_shape(t, bv, bb);
  if (rc) return rc;
  SYNTH_CHECK(cols % bv == 0, "synth_tensor: cols not a multiple of the block width");
  size_t n = rows * cols;
  SYNTH_CHECK(nbytes >= n / bv * bb, "synth_tensor: output buffer too small");
  parallel_chunks((n + kChunk - 1) / kChunk, [&](size_t c) {
    std::vector<float> buf(kChunk);
    size_t i0 = c * kChunk, m = std::min(kChunk, n - i0);
    fill_chunk(seed, c, sigma, buf.data(), m);
    encode_blocks(t, buf.data(), m / bv, out + i0 / bv * bb);
  });
  return kOk;
}

}  // namespace prana_synth

extern "C" {

const char* prana_synth_last_error(void) { return prana_synth::last_error().c_str(); }

int prana_quantize_tensor(int ggml_type, const float* src, size_t rows, size_t cols, void* out, size_t nbytes) {
  if (!src || !out) return prana_synth::fail(prana_synth::kErrInvalid, "null argument");
  return prana_synth::quantize_tensor(ggml_type, src, rows, cols, static_cast<uint8_t*>(out), nbytes);
}

int prana_synth_normal(uint64_t seed, float sigma, float* out, size_t n) {
  if (!out && n) return prana_synth::fail(prana_synth::kErrInvalid, "null argument");
  prana_synth::synth_normal(seed, sigma, out, n);
  return prana_synth::kOk;
}

int prana_synth_tensor(int ggml_type, size_t rows, size_t cols, uint64_t seed, float sigma, void* out,
                       size_t nbytes) {
  if (!out) return prana_synth::fail(prana_synth::kErrInvalid, "null argument");
  return prana_synth::synth_tensor(ggml_type, rows, cols, seed, sigma, static_cast<uint8_t*>(out), nbytes);
}

}  // extern "C"
