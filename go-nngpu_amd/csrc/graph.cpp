// graph.cpp — the reference bridge's MPSGraph calls (metal_bridge.h:1800-1826; in
// metal_bridge_phase9b.m:82-97 and :298-410 compile and execute are placeholders) as a
// working graph of GEMM and activation nodes compiled into a HIP graph.
//
// A graph holds placeholders (2-D, fp32 or fp16) and nodes: MatMul (op(A) * op(B), fp32
// result) and element-wise activations. Compiling a subgraph (given inputs and outputs)
// orders the nodes the outputs need, fuses a MatMul whose only use is an activation into
// one GEMM with that activation in its epilogue (the LinearActivation pattern of
// gpu/matrix/mps-graph-integration.go:103-115), allocates a device buffer per live
// tensor, and captures the launches once on a private stream into a HIP graph.
// Executing copies the caller's input buffers into the placeholders' buffers, replays
// the graph and copies the outputs back, all on one stream, then synchronises.
#include <algorithm>
#include <map>
#include <memory>
#include <mutex>
#include <vector>

#include "common.h"

namespace gn {
namespace {

constexpr uint64_t kGraphMagic = 0x6E6E67706867726FULL;     // graph
constexpr uint64_t kCompiledMagic = 0x6E6E6770657865FULL;   // compiled
constexpr uint64_t kTensorMagic = 0x6E6E677074656E73ULL;    // tensor

struct Graph;

struct GraphTensor {
  uint64_t magic = kTensorMagic;
  Graph *graph = nullptr;
  int id = 0;
  long rows = 0, cols = 0;
  int dtype = GN_F32;
  int op = -1;  // producing node, -1 for a placeholder
};

struct GraphOp {
  bool matmul = true;
  int a = -1, b = -1;  // operand tensor ids (b unused by activations)
  bool ta = false, tb = false;
  int act = GN_ACT_NONE;
  float alpha = 0.0f;
  int out = -1;
};

struct Graph {
  uint64_t magic = kGraphMagic;
  std::mutex mu;
  std::vector<std::unique_ptr<GraphTensor>> tensors;
  std::vector<GraphOp> ops;
};

struct Compiled {
  uint64_t magic = kCompiledMagic;
  std::mutex mu;  // one execution at a time: the buffers are shared
  hipStream_t stream = nullptr;
  hipGraphExec_t exec = nullptr;
  std::vector<void *> owned;  // device buffers
  std::vector<void *> in_buf, out_buf;
  std::vector<size_t> in_bytes, out_bytes;
};

Graph *as_graph(void *p) {
  auto *g = static_cast<Graph *>(p);
  return g && g->magic == kGraphMagic ? g : nullptr;
}
GraphTensor *as_tensor(Graph *g, void *p) {
  auto *t = static_cast<GraphTensor *>(p);
  return t && t->magic == kTensorMagic && t->graph == g ? t : nullptr;
}
Compiled *as_compiled(void *p) {
  auto *c = static_cast<Compiled *>(p);
  return c && c->magic == kCompiledMagic ? c : nullptr;
}

size_t tensor_bytes(const GraphTensor &t) { return (size_t)t.rows * (size_t)t.cols * (t.dtype == GN_F16 ? 2 : 4); }

GraphTensor *add_tensor(Graph *g, long rows, long cols, int dtype, int op) {
  auto t = std::make_unique<GraphTensor>();
  t->graph = g;
  t->id = (int)g->tensors.size();
  t->rows = rows;
  t->cols = cols;
  t->dtype = dtype;
  t->op = op;
  g->tensors.push_back(std::move(t));
  return g->tensors.back().get();
}

void release_compiled(Compiled *c) {
  if (c->exec) (void)hipGraphExecDestroy(c->exec);
  if (c->stream) (void)hipStreamDestroy(c->stream);
  for (void *p : c->owned) dev_free(p);
  c->magic = 0;
  delete c;
}

}  // namespace
}  // namespace gn

using gn::Compiled;
using gn::Graph;
using gn::GraphOp;
using gn::GraphTensor;

extern "C" {

void *createMPSGraph(void) {
  if (!gn::context(nullptr)) return nullptr;
  return new Graph();
}

void *gn_graph_placeholder(void *graph, long rows, long cols, int dtype) {
  Graph *g = gn::as_graph(graph);
  size_t bytes;
  if (!g || !gn::matrix_bytes(rows, cols, 4, &bytes) || (dtype != GN_F32 && dtype != GN_F16)) return nullptr;
  std::lock_guard<std::mutex> lk(g->mu);
  return gn::add_tensor(g, rows, cols, dtype, -1);
}

void *gn_graph_matmul(void *graph, void *inputA, void *inputB, int transA, int transB) {
  Graph *g = gn::as_graph(graph);
  if (!g) return nullptr;
  std::lock_guard<std::mutex> lk(g->mu);
  GraphTensor *a = gn::as_tensor(g, inputA), *b = gn::as_tensor(g, inputB);
  if (!a || !b || a->dtype != b->dtype) return nullptr;
  const long M = transA ? a->cols : a->rows, K = transA ? a->rows : a->cols;
  const long K2 = transB ? b->cols : b->rows, N = transB ? b->rows : b->cols;
  size_t out_bytes;
  if (K != K2 || !gn::matrix_bytes(M, N, 4, &out_bytes)) return nullptr;
  GraphOp op;
  op.matmul = true;
  op.a = a->id;
  op.b = b->id;
  op.ta = transA != 0;
  op.tb = transB != 0;
  op.out = (int)g->tensors.size();
  g->ops.push_back(op);
  return gn::add_tensor(g, M, N, GN_F32, (int)g->ops.size() - 1);
}

void *createMatMulNode(void *graph, void *inputA, void *inputB) { return gn_graph_matmul(graph, inputA, inputB, 0, 0); }

void *gn_graph_activation(void *graph, void *input, int act, float alpha) {
  Graph *g = gn::as_graph(graph);
  if (!g || !gn::act_forward_supported(act) || act == GN_ACT_NONE) return nullptr;
  std::lock_guard<std::mutex> lk(g->mu);
  GraphTensor *x = gn::as_tensor(g, input);
  if (!x || x->dtype != GN_F32) return nullptr;
  GraphOp op;
  op.matmul = false;
  op.a = x->id;
  op.act = act;
  op.alpha = alpha;
  op.out = (int)g->tensors.size();
  g->ops.push_back(op);
  return gn::add_tensor(g, x->rows, x->cols, GN_F32, (int)g->ops.size() - 1);
}

void *createReLUNode(void *graph, void *input) { return gn_graph_activation(graph, input, 0, 0.0f); }

int gn_graph_compile(void *graph, void *const *inputs, long numInputs, void *const *outputs, long numOutputs,
                     void **compiled, CError *err) {
  if (compiled) *compiled = nullptr;
  gn::Context *ctx = gn::context(err);
  if (!ctx) return -1;
  Graph *g = gn::as_graph(graph);
  if (!g || !compiled || numInputs < 0 || numOutputs < 1 || (numInputs > 0 && !inputs) || !outputs)
    return gn::set_error(err, -1, "graph compile: invalid arguments");
  std::lock_guard<std::mutex> lk(g->mu);
  const int nt = (int)g->tensors.size();
  std::vector<int> in_ids, out_ids;
  for (long i = 0; i < numInputs; ++i) {
    GraphTensor *t = gn::as_tensor(g, inputs[i]);
    if (!t || t->op >= 0) return gn::set_error(err, -1, "graph compile: input %ld is not a placeholder of this graph", i);
    in_ids.push_back(t->id);
  }
  for (long i = 0; i < numOutputs; ++i) {
    GraphTensor *t = gn::as_tensor(g, outputs[i]);
    if (!t) return gn::set_error(err, -1, "graph compile: output %ld is not a tensor of this graph", i);
    out_ids.push_back(t->id);
  }
  // Live nodes: everything the outputs depend on; every placeholder reached must be fed.
  std::vector<char> live_t(nt, 0), live_op(g->ops.size(), 0), fed(nt, 0);
  for (int id : in_ids) fed[id] = 1;
  std::vector<int> stack(out_ids.begin(), out_ids.end());
  while (!stack.empty()) {
    const int id = stack.back();
    stack.pop_back();
    if (live_t[id]) continue;
    live_t[id] = 1;
    const GraphTensor &t = *g->tensors[id];
    if (t.op < 0) {
      if (!fed[id]) return gn::set_error(err, -1, "graph compile: placeholder %d is needed but not an input", id);
      continue;
    }
    live_op[t.op] = 1;
    const GraphOp &op = g->ops[t.op];
    stack.push_back(op.a);
    if (op.matmul) stack.push_back(op.b);
  }
  for (int id : in_ids) live_t[id] = 1;  // an input the outputs do not need still gets its buffer
  // Uses of each tensor by live nodes, and whether it is an output.
  std::vector<int> uses(nt, 0);
  std::vector<char> is_out(nt, 0);
  for (int id : out_ids) is_out[id] = 1;
  for (size_t i = 0; i < g->ops.size(); ++i)
    if (live_op[i]) {
      ++uses[g->ops[i].a];
      if (g->ops[i].matmul) ++uses[g->ops[i].b];
    }
  // Fusion: activation over a MatMul result that nothing else reads.
  std::vector<GraphOp> plan;
  std::vector<char> fused_away(g->ops.size(), 0);
  for (size_t i = 0; i < g->ops.size(); ++i) {
    if (!live_op[i] || g->ops[i].matmul) continue;
    const GraphOp &act = g->ops[i];
    const GraphTensor &src = *g->tensors[act.a];
    if (src.op >= 0 && g->ops[src.op].matmul && uses[src.id] == 1 && !is_out[src.id]) fused_away[src.op] = 1;
  }
  for (size_t i = 0; i < g->ops.size(); ++i) {  // nodes are created after their operands: creation order is topological
    if (!live_op[i] || fused_away[i]) continue;
    GraphOp op = g->ops[i];
    if (!op.matmul) {
      const GraphTensor &src = *g->tensors[op.a];
      if (src.op >= 0 && fused_away[src.op]) {
        GraphOp mm = g->ops[src.op];
        mm.act = op.act;
        mm.alpha = op.alpha;
        mm.out = op.out;
        live_t[src.id] = 0;  // the MatMul result itself is never stored
        plan.push_back(mm);
        continue;
      }
    }
    plan.push_back(op);
  }
  auto c = std::make_unique<Compiled>();
  std::vector<void *> buf(nt, nullptr);
  auto fail = [&](int code) {
    for (void *p : c->owned) gn::dev_free(p);
    c->owned.clear();
    if (c->stream) (void)hipStreamDestroy(c->stream);
    c->stream = nullptr;
    return code;
  };
  for (int id = 0; id < nt; ++id) {
    if (!live_t[id]) continue;
    const size_t bytes = gn::tensor_bytes(*g->tensors[id]);
    if (bytes == 0) continue;
    buf[id] = gn::dev_alloc(bytes, err);
    if (!buf[id]) return fail(-1);
    c->owned.push_back(buf[id]);
  }
  for (int id : in_ids) {
    c->in_buf.push_back(buf[id]);
    c->in_bytes.push_back(gn::tensor_bytes(*g->tensors[id]));
  }
  for (int id : out_ids) {
    c->out_buf.push_back(buf[id]);
    c->out_bytes.push_back(gn::tensor_bytes(*g->tensors[id]));
  }
  hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e != hipSuccess) return fail(gn::hip_error(err, -1, "graph compile: stream", e));
  e = hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) return fail(gn::hip_error(err, -1, "graph compile: begin capture", e));
  int rc = 0;
  for (const GraphOp &op : plan) {
    const GraphTensor &o = *g->tensors[op.out];
    if (op.matmul) {
      const GraphTensor &a = *g->tensors[op.a], &b = *g->tensors[op.b];
      const long K = op.ta ? a.rows : a.cols;
      gn::GemmDesc d{a.dtype, op.ta, op.tb, o.rows, o.cols, K, 1.0f, 0.0f, buf[a.id], a.cols, 0, buf[b.id], b.cols,
                     0, static_cast<float *>(buf[o.id]), o.cols, 0, 1, nullptr, op.act, op.alpha};
      rc = gn::launch_gemm(d, c->stream, err);
    } else {
      rc = gn::launch_act_forward(static_cast<const float *>(buf[op.a]), static_cast<float *>(buf[o.id]),
                                  o.rows * o.cols, op.act, op.alpha, c->stream, err);
    }
    if (rc) break;
  }
  hipGraph_t hg = nullptr;
  e = hipStreamEndCapture(c->stream, &hg);
  if (rc) {
    if (hg) (void)hipGraphDestroy(hg);
    return fail(-1);
  }
  if (e != hipSuccess) return fail(gn::hip_error(err, -1, "graph compile: end capture", e));
  e = hipGraphInstantiate(&c->exec, hg, nullptr, nullptr, 0);
  (void)hipGraphDestroy(hg);
  if (e != hipSuccess) return fail(gn::hip_error(err, -1, "graph compile: instantiate", e));
  *compiled = c.release();
  return 0;
}

void *compileGraph(void *graph, void *device) {
  (void)device;
  Graph *g = gn::as_graph(graph);
  if (!g) return nullptr;
  std::vector<void *> ins, outs;
  {
    std::lock_guard<std::mutex> lk(g->mu);
    std::vector<char> consumed(g->tensors.size(), 0);
    for (const GraphOp &op : g->ops) {
      consumed[op.a] = 1;
      if (op.matmul) consumed[op.b] = 1;
    }
    for (auto &t : g->tensors) {
      if (t->op < 0) ins.push_back(t.get());
      else if (!consumed[t->id]) outs.push_back(t.get());
    }
  }
  if (outs.empty()) return nullptr;
  void *c = nullptr;
  CError e{nullptr};
  if (gn_graph_compile(graph, ins.data(), (long)ins.size(), outs.data(), (long)outs.size(), &c, &e) != 0) {
    free_c_error_message(e.message);
    return nullptr;
  }
  return c;
}

int gn_graph_execute(void *compiledGraph, void *stream, GPUPtr const *inputs, long numInputs, GPUPtr const *outputs,
                     long numOutputs, CError *err) {
  gn::Context *ctx = gn::context(err);
  if (!ctx) return -1;
  Compiled *c = gn::as_compiled(compiledGraph);
  if (!c) return gn::set_error(err, -1, "graph execute: not a compiled graph");
  if (numInputs != (long)c->in_buf.size() || numOutputs != (long)c->out_buf.size())
    return gn::set_error(err, -1, "graph execute: expected %zu inputs and %zu outputs, got %ld and %ld",
                         c->in_buf.size(), c->out_buf.size(), numInputs, numOutputs);
  std::lock_guard<std::mutex> lk(c->mu);
  hipStream_t s = gn::resolve_stream(stream);
  for (long i = 0; i < numInputs; ++i) {
    gn::Buffer *b = gn::as_buffer(inputs[i]);
    if (!b || b->bytes < c->in_bytes[i]) return gn::set_error(err, -1, "graph execute: input %ld is not a buffer of %zu bytes", i, c->in_bytes[i]);
  }
  for (long i = 0; i < numOutputs; ++i) {
    gn::Buffer *b = gn::as_buffer(outputs[i]);
    if (!b || b->bytes < c->out_bytes[i]) return gn::set_error(err, -1, "graph execute: output %ld is not a buffer of %zu bytes", i, c->out_bytes[i]);
  }
  for (long i = 0; i < numInputs; ++i) {
    if (!c->in_bytes[i]) continue;
    hipError_t e = hipMemcpyAsync(c->in_buf[i], gn::as_buffer(inputs[i])->dptr, c->in_bytes[i], hipMemcpyDeviceToDevice, s);
    if (e != hipSuccess) return gn::hip_error(err, -1, "graph execute: input copy", e);
  }
  hipError_t e = hipGraphLaunch(c->exec, s);
  if (e != hipSuccess) return gn::hip_error(err, -1, "graph execute: launch", e);
  for (long i = 0; i < numOutputs; ++i) {
    if (!c->out_bytes[i]) continue;
    e = hipMemcpyAsync(gn::as_buffer(outputs[i])->dptr, c->out_buf[i], c->out_bytes[i], hipMemcpyDeviceToDevice, s);
    if (e != hipSuccess) return gn::hip_error(err, -1, "graph execute: output copy", e);
  }
  e = hipStreamSynchronize(s);
  return e == hipSuccess ? 0 : gn::hip_error(err, -1, "graph execute", e);
}

void executeCompiledGraph(void *compiledGraph, void *commandBuffer, void **inputs, long numInputs, void **outputs,
                          long numOutputs) {
  CError e{nullptr};
  gn_graph_execute(compiledGraph, commandBuffer, inputs, numInputs, outputs, numOutputs, &e);
  free_c_error_message(e.message);
}

void gn_graph_release(void *graphOrCompiled) {
  if (Compiled *c = gn::as_compiled(graphOrCompiled)) {
    (void)hipStreamSynchronize(c->stream);
    gn::release_compiled(c);
    return;
  }
  if (Graph *g = gn::as_graph(graphOrCompiled)) {
    for (auto &t : g->tensors) t->magic = 0;
    g->magic = 0;
    delete g;
  }
}

}  // extern "C"
