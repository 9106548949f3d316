// MPSGraphManager (gpu/matrix/mps-graph-integration.go:15-296) over the graph calls of
// the C ABI (include/gonngpu.h: createMPSGraph, gn_graph_*).
#include <cstdio>

#include "../../include/gonngpu.h"
#include "gometal.hpp"

namespace gometal {
namespace matrix {

namespace {
std::string error_text(CError &e) {
  std::string m = e.message ? e.message : "";
  if (e.message) free_c_error_message(e.message);
  e.message = nullptr;
  return m;
}

// Element-wise codes of the activation types ActivationOp accepts (:200-210).
int activation_code(const std::string &t) {
  if (t == "ReLU") return ReLU;
  if (t == "Sigmoid") return Sigmoid;
  if (t == "Tanh") return Tanh;
  return -2;
}
}  // namespace

MPSGraphManager::MPSGraphManager(void *device) {
  (void)device;  // one GPU per process
  graph_ = createMPSGraph();
  if (!graph_) throw Panic("MPSGraphManager: cannot create a graph (no HIP device?)");
}

MPSGraphManager::~MPSGraphManager() {
  for (auto &kv : compiled_) gn_graph_release(kv.second->Executable);
  gn_graph_release(graph_);
}

const MPSGraphManager::Node &MPSGraphManager::node(const std::string &name) const {
  auto it = tensors_.find(name);
  if (it == tensors_.end()) throw Panic("MPSGraphManager: unknown tensor " + name);
  return it->second;
}

void *MPSGraphManager::CreateTensor(const std::string &name, const std::vector<int> &shape,
                                    const std::string &dataType) {
  std::lock_guard<std::mutex> lk(mu_);
  auto it = tensors_.find(name);
  if (it != tensors_.end()) return it->second.handle;
  if (shape.size() != 2) throw Panic("MPSGraphManager: graph tensors are 2-D, got " + std::to_string(shape.size()));
  const bool half = dataType == "float16" || dataType == "half";
  void *h = gn_graph_placeholder(graph_, shape[0], shape[1], half ? GN_F16 : GN_F32);
  if (!h) throw Panic("MPSGraphManager: invalid placeholder " + name);
  tensors_[name] = Node{h, shape, half};
  return h;
}

std::string MPSGraphManager::MatMulOp(const std::string &a, const std::string &b, bool transposeA, bool transposeB) {
  const std::string out = "matmul_" + a + "_" + b;
  std::lock_guard<std::mutex> lk(mu_);
  const Node &na = node(a), &nb = node(b);
  void *h = gn_graph_matmul(graph_, na.handle, nb.handle, transposeA, transposeB);
  if (!h) throw Panic("MPSGraphManager: MatMul of " + a + " and " + b + " has mismatched shapes or data types");
  const int M = transposeA ? na.shape[1] : na.shape[0], N = transposeB ? nb.shape[0] : nb.shape[1];
  tensors_[out] = Node{h, {M, N}, false};
  return out;
}

std::string MPSGraphManager::ActivationOp(const std::string &input, const std::string &activationType) {
  const std::string out = activationType + "_" + input;
  const int code = activation_code(activationType);
  if (code < -1) throw Panic("Unknown activation type: " + activationType);  // :209
  std::lock_guard<std::mutex> lk(mu_);
  const Node &x = node(input);
  void *h = gn_graph_activation(graph_, x.handle, code, 0.0f);
  if (!h) throw Panic("MPSGraphManager: activation of " + input + " (an fp32 tensor is needed)");
  tensors_[out] = Node{h, x.shape, false};
  return out;
}

Result<std::shared_ptr<CompiledOperation>> MPSGraphManager::CompileGraph(const std::vector<std::string> &inputs,
                                                                         const std::vector<std::string> &outputs) {
  std::string key = "[";
  for (size_t i = 0; i < inputs.size(); ++i) key += (i ? " " : "") + inputs[i];
  key += "]->[";
  for (size_t i = 0; i < outputs.size(); ++i) key += (i ? " " : "") + outputs[i];
  key += "]";
  std::lock_guard<std::mutex> lk(mu_);
  auto it = compiled_.find(key);
  if (it != compiled_.end()) return {it->second, {}};
  auto op = std::make_shared<CompiledOperation>();
  std::vector<void *> ins, outs;
  for (const std::string &n : inputs) {
    auto t = tensors_.find(n);
    if (t == tensors_.end()) return {nullptr, Errorf("compile: unknown input tensor %s", n.c_str())};
    ins.push_back(t->second.handle);
    op->InputShapes.push_back(t->second.shape);
  }
  for (const std::string &n : outputs) {
    auto t = tensors_.find(n);
    if (t == tensors_.end()) return {nullptr, Errorf("compile: unknown output tensor %s", n.c_str())};
    outs.push_back(t->second.handle);
    op->OutputShapes.push_back(t->second.shape);
  }
  CError ce{nullptr};
  if (gn_graph_compile(graph_, ins.data(), (long)ins.size(), outs.data(), (long)outs.size(), &op->Executable, &ce))
    return {nullptr, Errorf("graph compilation failed: %s", error_text(ce).c_str())};
  op->Inputs = inputs;
  op->Outputs = outputs;
  op->CacheKey = key;
  compiled_[key] = op;
  return {op, {}};
}

Result<std::map<std::string, TensorPtr>> MPSGraphManager::Execute(const CompiledOperation &compiled,
                                                                  const std::map<std::string, Tensor *> &inputs) {
  std::vector<GPUPtr> in_bufs, temps;
  auto release_temps = [&]() {
    for (GPUPtr t : temps) release_gpu_buffer(t);
  };
  for (size_t i = 0; i < compiled.Inputs.size(); ++i) {
    const std::string &name = compiled.Inputs[i];
    auto it = inputs.find(name);
    if (it == inputs.end() || !it->second) {
      release_temps();
      return {{}, Errorf("execute: missing input %s", name.c_str())};
    }
    Tensor &t = *it->second;
    const std::vector<int> &shape = compiled.InputShapes[i];
    const long n = (long)shape[0] * shape[1];
    if (t.Size() != n) {
      release_temps();
      return {{}, Errorf("execute: input %s has %ld values, the graph expects %dx%d", name.c_str(), t.Size(), shape[0],
                         shape[1])};
    }
    if (Error e = t.EnsureGPU()) {
      release_temps();
      return {{}, Errorf("execute: failed to move %s to GPU: %s", name.c_str(), e.message.c_str())};
    }
    bool half;
    {
      std::lock_guard<std::mutex> lk(mu_);
      half = node(name).half;
    }
    if (!half) {
      in_bufs.push_back(t.GPUPtr());
      continue;
    }
    // fp16 placeholder: round the fp32 values to fp16 (RNE) into a temporary buffer, on
    // the library stream that gn_graph_execute also uses
    GPUPtr h16 = nullptr;
    DevicePtr dev = nullptr;
    CError ce{nullptr};
    if (create_gpu_buffer(nullptr, n * 2, &h16, &dev, &ce) ||
        gn_cast_f32_f16(static_cast<const float *>(gn_buffer_device_ptr(t.GPUPtr())),
                        static_cast<uint16_t *>(gn_buffer_device_ptr(h16)), (size_t)n, GN_ROUND_NEAREST_EVEN,
                        nullptr, &ce)) {
      if (h16) release_gpu_buffer(h16);
      release_temps();
      return {{}, Errorf("execute: fp16 cast of %s failed: %s", name.c_str(), error_text(ce).c_str())};
    }
    temps.push_back(h16);
    in_bufs.push_back(h16);
  }
  std::map<std::string, TensorPtr> result;
  std::vector<GPUPtr> out_bufs;
  for (size_t i = 0; i < compiled.Outputs.size(); ++i) {
    auto [t, err] = Tensor::NewDeviceResult(compiled.OutputShapes[i]);
    if (err) {
      release_temps();
      return {{}, Errorf("execute: output allocation: %s", err.message.c_str())};
    }
    out_bufs.push_back(t->GPUPtr());
    result[compiled.Outputs[i]] = t;
  }
  CError ce{nullptr};
  const int rc = gn_graph_execute(compiled.Executable, nullptr, in_bufs.data(), (long)in_bufs.size(), out_bufs.data(),
                                  (long)out_bufs.size(), &ce);
  release_temps();
  if (rc) return {{}, Errorf("graph execution failed (code %d): %s", rc, error_text(ce).c_str())};
  return {result, {}};
}

}  // namespace matrix
}  // namespace gometal
