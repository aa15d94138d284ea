// prana-graph over device buffers (prana-graph/src/lib.rs:25-220): nodes are
// appended and reference only earlier ids, so execute evaluates in definition
// order; every value is an f32 buffer in HBM and every op is one of the
// library's kernels, so each node's value equals the reference op's output
// bit for bit (the same kernels as the model path).
#include "graph.h"

#include <climits>
#include <cmath>

#include "kernels.h"

namespace prana {

size_t GraphNode::numel() const {
  size_t n = 1;
  for (size_t d : shape) n *= d;
  return n;
}

int Graph::check_id(size_t id, const char* what) const {
  if (id >= nodes.size())
    return fail(kErrInvalid, std::string("graph: ") + what + ": node " + std::to_string(id) + " does not exist");
  return kOk;
}

size_t Graph::push(GraphNode&& n) {
  nodes.push_back(std::move(n));
  return nodes.size() - 1;
}

// set_input (lib.rs:126-129): any node may be given a value; execute then
// skips it.
int Graph::set_value(size_t id, const float* src, bool on_device, const size_t* shape, int n_dims, hipStream_t s) {
  if (int rc = check_id(id, "set_input")) return rc;
  PRANA_CHECK(n_dims >= 0 && n_dims <= 8 && (shape || n_dims == 0), "graph: set_input: bad shape");
  GraphNode& n = nodes[id];
  std::vector<size_t> sh(shape, shape + n_dims);
  size_t count = 1;
  for (size_t d : sh) count *= d;
  PRANA_CHECK(src || count == 0, "graph: set_input: null data");
  if (int rc = n.value.alloc(std::max<size_t>(count, 1) * 4)) return rc;
  if (count)
    PRANA_HIP(hipMemcpyAsync(n.value.p, src, count * 4, on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
                             s));
  PRANA_HIP(hipStreamSynchronize(s));
  n.shape = std::move(sh);
  n.has_value = true;
  return kOk;
}

int Graph::eval(size_t i, hipStream_t s, int* kind, size_t* node) {
  GraphNode& n = nodes[i];
  auto unset = [&](size_t id) {
    *kind = kGraphUnsetInput;
    *node = id;
    return fail(kErrInvalid, "graph: input node " + std::to_string(id) + " is unset");
  };
  auto mismatch = [&](const char* what) {
    *kind = kGraphShapeMismatch;
    *node = i;
    return fail(kErrInvalid, std::string("graph: shape mismatch (") + what + ") at node " + std::to_string(i));
  };
  auto out = [&](std::vector<size_t> shape) -> int {
    n.shape = std::move(shape);
    return n.value.alloc(std::max<size_t>(n.numel(), 1) * 4);
  };
  const size_t T = n_tokens;
  switch (n.op) {
    case GraphNode::kInput:
      return unset(i);
    case GraphNode::kMatmulF32:
    case GraphNode::kMatmulQ8: {  // lib.rs:152-169
      const GraphNode& x = nodes[n.a];
      if (!x.has_value) return unset(n.a);
      const DevMat& d = n.w->d;
      if (x.numel() != T * d.cols) return mismatch(n.op == GraphNode::kMatmulF32 ? "matmul_f32 input" : "matmul_q8 input");
      if (int rc = out({T, d.rows})) return rc;
      const GemvOut o{n.value.as<float>(), d.rows, nullptr, 0};
      if (n.op == GraphNode::kMatmulF32) return launch_gemv(d, x.value.as<float>(), nullptr, nullptr, nullptr, T, o, s);
      if (int rc = launch_quantize_acts(x.value.as<float>(), T, d.cols, qa.as<int8_t>(), sa.as<float>(),
                                        sums.as<int>(), s))
        return rc;
      return launch_gemv(d, x.value.as<float>(), qa.as<int8_t>(), sa.as<float>(), sums.as<int>(), T, o, s);
    }
    case GraphNode::kRmsNorm: {  // lib.rs:170-178
      const GraphNode& x = nodes[n.a];
      if (!x.has_value) return unset(n.a);
      if (x.numel() % n.dim != 0) return mismatch("rmsnorm dim");
      const size_t rows = x.numel() / n.dim;
      if (int rc = out({rows, n.dim})) return rc;
      return launch_rmsnorm(x.value.as<float>(), n.vec.as<float>(), rows, n.dim, n.eps, n.value.as<float>(), nullptr,
                            nullptr, nullptr, s);
    }
    case GraphNode::kAdd: {  // lib.rs:179-188: the shape of a
      const GraphNode &a = nodes[n.a], &b = nodes[n.b];
      if (!a.has_value) return unset(n.a);
      if (!b.has_value) return unset(n.b);
      if (a.numel() != b.numel()) return mismatch("add");
      if (int rc = out(a.shape)) return rc;
      if (a.numel())
        PRANA_HIP(hipMemcpyAsync(n.value.p, a.value.p, a.numel() * 4, hipMemcpyDeviceToDevice, s));
      return launch_add(n.value.as<float>(), b.value.as<float>(), a.numel(), 0, s);
    }
    case GraphNode::kSoftmax: {  // lib.rs:189-193: one row over every value
      const GraphNode& x = nodes[n.a];
      if (!x.has_value) return unset(n.a);
      PRANA_CHECK(x.numel() <= static_cast<size_t>(INT_MAX), "graph: softmax over more than 2^31 values");
      if (int rc = out({x.numel()})) return rc;
      return launch_softmax(x.value.as<float>(), 1, x.numel(), n.value.as<float>(), s);
    }
    case GraphNode::kRope: {  // lib.rs:194-201; rope (attention.rs:59-80), positions = rows
      const GraphNode& x = nodes[n.a];
      if (!x.has_value) return unset(n.a);
      const size_t width = n.n_heads * n.head_dim;
      if (x.numel() != T * width) return mismatch("rope input");
      if (int rc = out({T, width})) return rc;
      // (cos, sin) of p * theta^(-(2j)/head_dim) for the rows of this pass,
      // the values attention.rs:70-72 computes per element
      const size_t half = n.head_dim / 2;
      std::vector<float> tab(std::max<size_t>(T * half * 2, 2));
      for (size_t j = 0; j < half; j++) {
        const float freq = std::pow(n.theta, -(2.0f * static_cast<float>(j)) / static_cast<float>(n.head_dim));
        for (size_t p = 0; p < T; p++) {
          const float ang = static_cast<float>(p) * freq;
          tab[(p * half + j) * 2] = std::cos(ang);
          tab[(p * half + j) * 2 + 1] = std::sin(ang);
        }
      }
      // each rope node keeps its own table: a shared one could be rewritten
      // while an earlier launch on the stream still reads it
      if (int rc = n.vec.alloc(tab.size() * 4)) return rc;
      PRANA_HIP(hipMemcpy(n.vec.p, tab.data(), tab.size() * 4, hipMemcpyHostToDevice));
      if (x.numel())
        PRANA_HIP(hipMemcpyAsync(n.value.p, x.value.p, x.numel() * 4, hipMemcpyDeviceToDevice, s));
      return launch_rope(n.value.as<float>(), T, width, width, n.head_dim, n.vec.as<float2>(), 0, 1, s);
    }
    case GraphNode::kAttention: {  // lib.rs:202-214; attention (attention.rs:236-284)
      const GraphNode &q = nodes[n.a], &k = nodes[n.b], &v = nodes[n.c];
      if (!q.has_value) return unset(n.a);
      if (!k.has_value) return unset(n.b);
      if (!v.has_value) return unset(n.c);
      const size_t qw = n.n_heads * n.head_dim, kw = n.n_kv_heads * n.head_dim;
      if (q.numel() != T * qw || k.numel() != T * kw || v.numel() != T * kw) return mismatch("attention qkv");
      if (int rc = out({T, qw})) return rc;
      return launch_attention_prefill(q.value.as<float>(), k.value.as<float>(), v.value.as<float>(), T, n.n_heads,
                                      n.n_kv_heads, n.head_dim, n.value.as<float>(), scratch.as<float>(), s);
    }
  }
  return fail(kErrInvalid, "graph: unknown op");
}

int Graph::execute(hipStream_t s, int* kind, size_t* node) {
  *kind = kGraphOk;
  *node = 0;
  // Shared scratch sized up front for every node still to run, so no buffer
  // is reallocated while a launch on the stream may read it.
  size_t q_elems = 0, att_floats = 0;
  for (const GraphNode& n : nodes) {
    if (n.has_value) continue;
    if (n.op == GraphNode::kMatmulQ8) q_elems = std::max(q_elems, n_tokens * n.w->d.cols);
    if (n.op == GraphNode::kAttention)
      att_floats = std::max(att_floats, attention_scratch_floats(n_tokens, n.n_heads, n_tokens, false));
  }
  int rc;
  if (q_elems && ((rc = qa.ensure(q_elems)) || (rc = sa.ensure(q_elems / 32 * 4)) || (rc = sums.ensure(q_elems / 32 * 4))))
    return rc;
  if (att_floats && (rc = scratch.ensure(att_floats * 4))) return rc;
  for (size_t i = 0; i < nodes.size(); i++) {
    if (nodes[i].has_value) continue;
    if ((rc = eval(i, s, kind, node))) {
      (void)hipStreamSynchronize(s);  // drain what was launched before reporting
      return rc;
    }
    nodes[i].has_value = true;
  }
  PRANA_HIP(hipStreamSynchronize(s));
  return kOk;
}

}  // namespace prana
