// GGUF container parsing and the model loader (prana-model gguf.rs).
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/prana_hip.h"

namespace prana {

// A parsed metadata value (gguf.rs:44-58): the file's value type, integers
// widened, floats as double, strings as bytes, arrays as their elements.
struct GValue {
  uint32_t type = 0;  // GGUF value type 0..12
  uint64_t u = 0;     // unsigned integers and bool
  int64_t i = 0;      // signed integers
  double f = 0.0;     // f32 / f64
  std::string s;      // string bytes
  uint32_t elem_type = 0;
  std::vector<GValue> arr;
};

struct GTensor {
  std::vector<uint64_t> dims;  // ggml order: dims[0] is the contiguous one
  uint32_t type = 0;
  uint64_t offset = 0;
};

// The parsed file (gguf.rs:140-145): metadata, tensor directory (names in
// file order) and the data section, a read-only mapping of the file or an
// owned copy of caller bytes.
struct Gguf {
  uint32_t version = 0;
  std::map<std::string, GValue> meta;
  std::map<std::string, GTensor> tensors;
  std::vector<std::string> names;
  const uint8_t* base = nullptr;
  size_t size = 0, data_start = 0;
  void* map = nullptr;
  std::vector<uint8_t> owned;

  Gguf() = default;
  Gguf(const Gguf&) = delete;
  Gguf& operator=(const Gguf&) = delete;
  ~Gguf();

  int parse();
  const GValue* find(const std::string& key) const;
  // The tensor's bytes inside the data section (Gguf::raw, gguf.rs:202-205).
  int raw(const std::string& name, const GTensor** t, const uint8_t** bytes, size_t* nbytes) const;
  // Gguf::tensor_f32 (gguf.rs:208-264): any supported type decoded on the host.
  int tensor_f32(const std::string& name, std::vector<float>& out) const;
};

int gguf_open_file(const char* path, std::unique_ptr<Gguf>& out);
int gguf_open_bytes(const void* data, size_t n, std::unique_ptr<Gguf>& out);

bool gvalue_as_u64(const GValue& v, uint64_t* out);  // Value::as_usize (gguf.rs:63-75)
bool gvalue_as_f32(const GValue& v, float* out);     // Value::as_f32 (gguf.rs:77-83)

// load (gguf.rs:338-437) without the tokenizer, onto a new device model.
// precision: 0 = F32, 1 = Q8 (Precision, checkpoint.rs).
struct Model;
int gguf_load_model(const Gguf& g, int precision, Model& m);
int gguf_model_config(const Gguf& g, prana_config* c);

}  // namespace prana

struct prana_gguf {
  std::unique_ptr<prana::Gguf> g;
};
