// Context, errors, device buffers and weight upload (GGUF bytes -> device layout).
#include "runtime.h"

#include <cstring>
#include <mutex>
#include <string>

namespace prana {

namespace {
thread_local std::string g_last_error = "no error";
std::mutex g_init_mu;
}  // namespace

void set_error(const std::string& msg) { g_last_error = msg; }
const char* last_error_cstr() { return g_last_error.c_str(); }

int fail(int code, const std::string& msg) {
  set_error(msg);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  set_error(std::string("HIP error in ") + what + ": " + hipGetErrorString(e));
  return e == hipErrorOutOfMemory ? kErrNoMem : kErrHip;
}

Context& ctx() {
  static Context c;
  return c;
}

int ensure_init() {
  std::lock_guard<std::mutex> lk(g_init_mu);
  Context& c = ctx();
  if (c.device >= 0) {
    PRANA_HIP(hipSetDevice(c.device));
    return kOk;
  }
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0) return fail(kErrHip, "no HIP device visible (libprana_hip needs an MI355X / gfx950 GPU)");
  PRANA_HIP(hipSetDevice(0));
  PRANA_HIP(hipStreamCreateWithFlags(&c.stream, hipStreamNonBlocking));
  if (int rc = flash_noalloc_setup(0)) return rc;
  c.device = 0;
  return kOk;
}

int require_init() {
  std::lock_guard<std::mutex> lk(g_init_mu);
  const Context& c = ctx();
  if (c.device < 0) return fail(kErrInvalid, "library not initialised: call prana_init first");
  PRANA_HIP(hipSetDevice(c.device));
  return kOk;
}

hipStream_t pick_stream(void* s) { return s ? static_cast<hipStream_t>(s) : ctx().stream; }

DevBuf::~DevBuf() {
  if (p) (void)hipFree(p);
}

int DevBuf::alloc(size_t n) {
  if (p) {
    (void)hipFree(p);
    p = nullptr;
    bytes = 0;
  }
  if (n == 0) return kOk;
  PRANA_HIP(hipMalloc(&p, n));
  bytes = n;
  return kOk;
}

int DevBuf::ensure(size_t n) { return n <= bytes ? kOk : alloc(n); }

float host_f16_to_f32(uint16_t h) {
  uint32_t sign = (h >> 15) & 1u, exp = (h >> 10) & 0x1fu, frac = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0 && frac == 0) {
    bits = sign << 31;
  } else if (exp == 0) {
    float v = static_cast<float>(frac) * 5.9604644775390625e-08f;  // 2^-24
    return sign ? -v : v;
  } else if (exp == 0x1f) {
    bits = (sign << 31) | 0x7f800000u | (frac << 13);
  } else {
    bits = (sign << 31) | ((exp + 127 - 15) << 23) | (frac << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

size_t ggml_nbytes(int t, size_t n) {
  switch (t) {
    case 0: return n * 4;                               // F32
    case 1: return n * 2;                               // F16
    case 2: return n % 32 ? 0 : n / 32 * 18;            // Q4_0
    case 8: return n % 32 ? 0 : n / 32 * 34;            // Q8_0
    case 12: return n % 256 ? 0 : n / 256 * 144;        // Q4_K
    case 14: return n % 256 ? 0 : n / 256 * 210;        // Q6_K
  }
  return 0;
}

namespace {

int upload(DevBuf& b, const void* host, size_t n) {
  int rc = b.alloc(n);
  if (rc) return rc;
  if (n) PRANA_HIP(hipMemcpy(b.p, host, n, hipMemcpyHostToDevice));
  return kOk;
}

// Dense f32 table of any ggml tensor (gguf.rs:208-267 tensor_f32).
std::vector<float> to_f32(int t, size_t n, const uint8_t* raw) {
  std::vector<float> out(n);
  auto f16 = [&](const uint8_t* p) { return host_f16_to_f32(static_cast<uint16_t>(p[0] | (p[1] << 8))); };
  if (t == 0) {
    std::memcpy(out.data(), raw, n * 4);
  } else if (t == 1) {
    for (size_t i = 0; i < n; i++) out[i] = f16(raw + 2 * i);
  } else if (t == 8) {
    for (size_t b = 0; b < n / 32; b++) {
      float s = f16(raw + b * 34);
      for (int j = 0; j < 32; j++) out[b * 32 + j] = static_cast<float>(static_cast<int8_t>(raw[b * 34 + 2 + j])) * s;
    }
  } else if (t == 2) {
    for (size_t b = 0; b < n / 32; b++) {
      const uint8_t* p = raw + b * 18;
      float d = f16(p);
      for (int j = 0; j < 16; j++) out[b * 32 + j] = d * (static_cast<float>(p[2 + j] & 0xF) - 8.0f);
      for (int j = 0; j < 16; j++) out[b * 32 + 16 + j] = d * (static_cast<float>(p[2 + j] >> 4) - 8.0f);
    }
  } else {
    out.clear();  // K-quant tensors are never densified by the loader paths used here
  }
  return out;
}

}  // namespace

int mat_from_q8_parts(size_t rows, size_t cols, const int8_t* q, const float* scales, Mat& out) {
  PRANA_CHECK(cols % 32 == 0, "QuantMatrix: cols must be a multiple of 32 (matmul.rs:35)");
  int rc = upload(out.qs, q, rows * cols);
  if (!rc) rc = upload(out.sc, scales, rows * (cols / 32) * 4);
  if (rc) return rc;
  out.d = DevMat{kKindQ8F, rows, cols, out.qs.as<uint8_t>(), out.sc.p};
  out.stream_bytes = devmat_bytes(out.d);
  return kOk;
}

// Gguf::linear (gguf.rs:271-305) onto the device layouts of kernels.h.
int mat_from_ggml(int t, size_t rows, size_t cols, const void* bytes, size_t nbytes, Mat& out) {
  const uint8_t* raw = static_cast<const uint8_t*>(bytes);
  size_t n = rows * cols;
  size_t need = ggml_nbytes(t, n);
  PRANA_CHECK(need != 0 || n == 0, "matrix: unsupported ggml type or unaligned element count");
  PRANA_CHECK(nbytes >= need, "matrix: byte buffer shorter than the tensor");
  int rc = kOk;
  if (t == 8 && cols % 32 == 0) {  // Q8_0 -> QuantMatrix (f16 scale kept as f16)
    size_t G = n / 32;
    std::vector<uint8_t> q(n);
    std::vector<uint16_t> d(G);
    for (size_t b = 0; b < G; b++) {
      d[b] = static_cast<uint16_t>(raw[b * 34] | (raw[b * 34 + 1] << 8));
      std::memcpy(&q[b * 32], raw + b * 34 + 2, 32);
    }
    if (!(rc = upload(out.qs, q.data(), n))) rc = upload(out.sc, d.data(), G * 2);
    if (rc) return rc;
    out.d = DevMat{kKindQ8_0, rows, cols, out.qs.as<uint8_t>(), out.sc.p};
  } else if (t == 2 && cols % 32 == 0) {  // Q4_0 -> KQuantMatrix
    size_t G = n / 32;
    std::vector<uint8_t> q(G * 16);
    std::vector<uint16_t> d(G);
    for (size_t b = 0; b < G; b++) {
      d[b] = static_cast<uint16_t>(raw[b * 18] | (raw[b * 18 + 1] << 8));
      std::memcpy(&q[b * 16], raw + b * 18 + 2, 16);
    }
    if (!(rc = upload(out.qs, q.data(), q.size()))) rc = upload(out.sc, d.data(), G * 2);
    if (rc) return rc;
    out.d = DevMat{kKindQ4_0, rows, cols, out.qs.as<uint8_t>(), out.sc.p};
  } else if (t == 12 && cols % 256 == 0) {  // Q4_K: block layout kept
    if ((rc = upload(out.qs, raw, need))) return rc;
    out.d = DevMat{kKindQ4_K, rows, cols, out.qs.as<uint8_t>(), nullptr};
  } else if (t == 14 && cols % 256 == 0) {  // Q6_K: 208 B body + f16 d split
    size_t nb = n / 256;
    std::vector<uint8_t> body(nb * 208);
    std::vector<uint16_t> d(nb);
    for (size_t b = 0; b < nb; b++) {
      std::memcpy(&body[b * 208], raw + b * 210, 208);
      d[b] = static_cast<uint16_t>(raw[b * 210 + 208] | (raw[b * 210 + 209] << 8));
    }
    if (!(rc = upload(out.qs, body.data(), body.size()))) rc = upload(out.sc, d.data(), nb * 2);
    if (rc) return rc;
    out.d = DevMat{kKindQ6_K, rows, cols, out.qs.as<uint8_t>(), out.sc.p};
  } else {
    // Linear::new(tensor_f32(..), Precision::F32) -> dense rows.
    PRANA_CHECK(t == 0 || t == 1 || t == 2 || t == 8, "matrix: K-quant tensor with cols not a multiple of 256");
    std::vector<float> f = to_f32(t, n, raw);
    if ((rc = upload(out.qs, f.data(), n * 4))) return rc;
    out.d = DevMat{kKindF32, rows, cols, out.qs.as<uint8_t>(), nullptr};
  }
  out.stream_bytes = devmat_bytes(out.d);
  return kOk;
}

}  // namespace prana
