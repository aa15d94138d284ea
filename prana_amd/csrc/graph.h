// prana-graph (prana-graph/src/lib.rs) over device buffers: a define-then-run
// list of nodes whose values live in HBM, each op one of the library's
// kernels on the library stream.
#pragma once

#include <memory>
#include <string>
#include <vector>

#include "runtime.h"

namespace prana {

// GraphError (lib.rs:55-63).
enum GraphErrorKind : int { kGraphOk = 0, kGraphUnsetInput = 1, kGraphShapeMismatch = 2, kGraphNotF32 = 3 };

struct GraphNode {
  // Op (lib.rs:25-42).
  enum Op { kInput, kMatmulF32, kMatmulQ8, kRmsNorm, kAdd, kSoftmax, kRope, kAttention } op = kInput;
  size_t a = 0, b = 0, c = 0;  // input node ids (x / a, b / q, k, v)
  std::unique_ptr<Mat> w;      // matmul weights on the device
  DevBuf vec;                  // rmsnorm weight
  size_t dim = 0, n_heads = 0, n_kv_heads = 0, head_dim = 0;
  float eps = 0.0f, theta = 0.0f;
  // the node's value (lib.rs:45-48): f32 on the device, with its shape
  bool has_value = false;
  DevBuf value;
  std::vector<size_t> shape;
  size_t numel() const;
};

struct Graph {
  std::vector<GraphNode> nodes;
  size_t n_tokens = 0;  // set by the inputs (lib.rs:51-53, 84-87)
  DevBuf qa, sa, sums, scratch, table;

  int check_id(size_t id, const char* what) const;
  size_t push(GraphNode&& n);
  int set_value(size_t id, const float* src, bool src_on_device, const size_t* shape, int n_dims, hipStream_t s);
  // execute (lib.rs:132-141): every node without a value, in definition
  // order; on a GraphError *kind / *node name it.
  int execute(hipStream_t s, int* kind, size_t* node);
  int eval(size_t i, hipStream_t s, int* kind, size_t* node);
};

}  // namespace prana

struct prana_graph {
  prana::Graph g;
};
