// Host-side runtime objects shared by the C ABI and the model layer.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <vector>

#include "common.h"
#include "kernels.h"

namespace prana {

// Process-wide context: selected device and the library's default stream
// (default priority — no stream-priority games).
struct Context {
  int device = -1;
  hipStream_t stream = nullptr;
};
Context& ctx();
int ensure_init();
// Selects the library's device when prana_init has run; fails (creating
// nothing) otherwise.
int require_init();
hipStream_t pick_stream(void* s);

// RAII device buffer.
struct DevBuf {
  void* p = nullptr;
  size_t bytes = 0;
  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  DevBuf(DevBuf&& o) noexcept : p(o.p), bytes(o.bytes) {
    o.p = nullptr;
    o.bytes = 0;
  }
  DevBuf& operator=(DevBuf&& o) noexcept {
    if (this != &o) {
      if (p) (void)hipFree(p);
      p = o.p;
      bytes = o.bytes;
      o.p = nullptr;
      o.bytes = 0;
    }
    return *this;
  }
  ~DevBuf();
  int alloc(size_t n);  // frees the previous allocation
  int ensure(size_t n);  // grow-only
  template <class T>
  T* as() const {
    return static_cast<T*>(p);
  }
};

// A device-resident weight matrix (Linear / QuantMatrix / KQuantMatrix).
struct Mat {
  DevMat d{};
  DevBuf qs, sc;
  size_t stream_bytes = 0;  // algorithmic bytes (GGUF block bytes)
};

// Build from ggml bytes (host). Returns status; `out` owns device memory.
int mat_from_ggml(int ggml_type, size_t rows, size_t cols, const void* bytes, size_t nbytes, Mat& out);
int mat_from_q8_parts(size_t rows, size_t cols, const int8_t* q, const float* scales, Mat& out);
size_t ggml_nbytes(int ggml_type, size_t n_elems);

// Host f16 conversion, same semantics as the device helpers (lib.rs:57-113).
float host_f16_to_f32(uint16_t h);

}  // namespace prana
