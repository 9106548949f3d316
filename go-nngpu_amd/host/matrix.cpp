// matrix.cpp — gometal::matrix tensor-level operations over the C ABI: MatMul,
// Transpose, OptimizedGEMM / OptimizedBatchMatMul, SparseMatMul / SparseMatVec /
// SparseTranspose, FusedLinearActivation, the fp16 MixedPrecisionTrainer path and
// LinearLayer. Error messages follow the Go functions they mirror.
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>

#include "../../include/gonngpu.h"
#include "gometal.hpp"

namespace gometal {
namespace matrix {

namespace {

// "<what> failed (code N): <message>", freeing the C message (gpu/matrix/matrix.go:95-102).
Error op_error(const char *what, int code, CError &e) {
  std::string msg;
  if (e.message) {
    msg = e.message;
    free_c_error_message(e.message);
    e.message = nullptr;
  }
  return Errorf("%s failed (code %d): %s", what, code, msg.c_str());
}

Error wrap(const char *prefix, const Error &e) { return Errorf("%s: %s", prefix, e.message.c_str()); }

// Device pointer behind a tensor's GPUPtr handle (for the gn_* device-pointer API).
float *dptr(const Tensor &t) { return static_cast<float *>(gn_buffer_device_ptr(t.GPUPtr())); }

// Scoped device scratch from the library pool.
struct DeviceScratch {
  void *p = nullptr;
  ~DeviceScratch() {
    if (p) gn_free(p);
  }
  Error alloc(size_t bytes) {
    CError e{nullptr};
    int rc = gn_malloc(&p, bytes, &e);
    return rc == 0 ? Error{} : op_error("device allocation", rc, e);
  }
};

}  // namespace

// ------------------------------------------------------------------ dense
Result<TensorPtr> MatMul(Tensor &A, Tensor &B) {
  if (A.Shape.size() != 2 || B.Shape.size() != 2) return {nullptr, Errorf("MatMul requires 2D tensors (matrices)")};
  if (A.Shape[1] != B.Shape[0])
    return {nullptr, Errorf("incompatible matrix dimensions for multiplication: A columns (%d) != B rows (%d)",
                            A.Shape[1], B.Shape[0])};
  auto [result, rerr] = Tensor::NewDeviceResult({A.Shape[0], B.Shape[1]});
  if (rerr) return {nullptr, wrap("failed to create result tensor", rerr)};
  if (Error e = A.EnsureGPU()) return {nullptr, wrap("failed to move tensor A to GPU", e)};
  if (Error e = B.EnsureGPU()) return {nullptr, wrap("failed to move tensor B to GPU", e)};
  CError ce{nullptr};
  int rc = perform_mps_matrix_multiplication(A.GPUPtr(), A.Shape[0], A.Shape[1], B.GPUPtr(), B.Shape[0], B.Shape[1],
                                             result->GPUPtr(), result->Shape[0], result->Shape[1], A.DevicePtr(), &ce);
  if (rc != 0) return {nullptr, op_error("GPU matrix multiplication", rc, ce)};
  return {result, {}};
}

Result<TensorPtr> MatMulTransposed(Tensor &A, bool transA, Tensor &B, bool transB) {
  if (!transA && !transB) return MatMul(A, B);
  if (A.Shape.size() != 2 || B.Shape.size() != 2) return {nullptr, Errorf("MatMul requires 2D tensors (matrices)")};
  const int M = transA ? A.Shape[1] : A.Shape[0], K = transA ? A.Shape[0] : A.Shape[1];
  const int KB = transB ? B.Shape[1] : B.Shape[0], N = transB ? B.Shape[0] : B.Shape[1];
  if (K != KB)
    return {nullptr, Errorf("incompatible matrix dimensions for multiplication: A columns (%d) != B rows (%d)", K, KB)};
  auto [result, rerr] = Tensor::NewDeviceResult({M, N});
  if (rerr) return {nullptr, wrap("failed to create result tensor", rerr)};
  if (Error e = A.EnsureGPU()) return {nullptr, wrap("failed to move tensor A to GPU", e)};
  if (Error e = B.EnsureGPU()) return {nullptr, wrap("failed to move tensor B to GPU", e)};
  if ((long)M * N == 0) return {result, {}};
  CError ce{nullptr};
  // The GEMM reads op(A) and op(B) in place: A stored [K, M] with transA, B [N, K] with transB.
  int rc = gn_gemm(GN_F32, transA, transB, M, N, K, 1.0f, dptr(A), A.Shape[1], 0, dptr(B), B.Shape[1], 0, 0.0f,
                   dptr(*result), N, 0, 1, nullptr, GN_ACT_NONE, 0.0f, nullptr, &ce);
  if (rc == 0) rc = gn_synchronize(nullptr, &ce);
  if (rc != 0) return {nullptr, op_error("GPU matrix multiplication", rc, ce)};
  return {result, {}};
}

Result<TensorPtr> Transpose(Tensor &A) {
  if (A.Shape.size() != 2) return {nullptr, Errorf("Transpose requires 2D tensor (matrix)")};
  auto [result, rerr] = Tensor::NewDeviceResult({A.Shape[1], A.Shape[0]});
  if (rerr) return {nullptr, wrap("failed to create result tensor for transpose", rerr)};
  if (Error e = A.EnsureGPU()) return {nullptr, wrap("failed to move input tensor to GPU", e)};
  CError ce{nullptr};
  int rc = perform_mps_matrix_transpose(A.GPUPtr(), A.Shape[0], A.Shape[1], result->GPUPtr(), result->Shape[0],
                                        result->Shape[1], A.DevicePtr(), &ce);
  if (rc != 0) return {nullptr, op_error("GPU matrix transpose", rc, ce)};
  return {result, {}};
}

namespace {
void *g_matrix_device = nullptr;
}
void SetGlobalMatrixDevice(void *device) { g_matrix_device = device; }

std::string String(ActivationType t) {
  switch (t) {
    case ReLU: return "ReLU";
    case Sigmoid: return "Sigmoid";
    case Tanh: return "Tanh";
    case Softmax: return "Softmax";
    case LeakyReLU: return "LeakyReLU";
    case ELU: return "ELU";
    case Swish: return "Swish";
    case GELU: return "GELU";
  }
  return "Unknown";
}

Result<TensorPtr> ActivationForward(Tensor &input, ActivationType activationType, float alpha) {
  if (input.Shape.empty()) return {nullptr, Errorf("cannot apply activation to empty tensor")};
  // The rank and type errors of the reference's switch (:146-160), checked before any
  // device work rather than after the result allocation.
  if (activationType == Softmax && input.Shape.size() > 2)
    return {nullptr, Errorf("softmax currently supports only 1D and 2D tensors")};
  if (String(activationType) == "Unknown")
    return {nullptr, Errorf("unsupported activation type: %s", String(activationType).c_str())};
  long size = 1;
  for (int d : input.Shape) size *= d;
  auto [result, rerr] = Tensor::NewDeviceResult(input.Shape);
  if (rerr) return {nullptr, wrap("failed to create result tensor", rerr)};
  if (Error e = input.EnsureGPU()) return {nullptr, wrap("failed to move input tensor to GPU", e)};
  GPUPtr in = input.GPUPtr(), out = result->GPUPtr();
  DevicePtr dev = input.DevicePtr();
  CError ce{nullptr};
  int rc = 0;
  switch (activationType) {
    case ReLU: rc = perform_activation_relu_forward(in, size, out, dev, &ce); break;
    case Sigmoid: rc = perform_activation_sigmoid_forward(in, size, out, dev, &ce); break;
    case Tanh: rc = perform_activation_tanh_forward(in, size, out, dev, &ce); break;
    case LeakyReLU: rc = perform_activation_leaky_relu_forward(in, size, alpha, out, dev, &ce); break;
    case ELU: rc = perform_activation_elu_forward(in, size, alpha, out, dev, &ce); break;
    case Swish: rc = perform_activation_swish_forward(in, size, out, dev, &ce); break;
    case GELU: rc = perform_activation_gelu_forward(in, size, out, dev, &ce); break;
    case Softmax:
      if (input.Shape.size() == 1)
        rc = perform_activation_softmax_1d_forward(in, input.Shape[0], out, dev, &ce);
      else
        rc = perform_activation_softmax_2d_forward(in, input.Shape[0], input.Shape[1], out, dev, &ce);
      break;
  }
  if (rc != 0) return {nullptr, op_error("GPU activation forward", rc, ce)};
  return {result, {}};
}

Result<TensorPtr> OptimizedGEMM(Tensor &A, Tensor &B, float alpha, float beta) {
  if (A.Shape.size() != 2 || B.Shape.size() != 2) return {nullptr, Errorf("optimized GEMM requires 2D tensors")};
  const int M = A.Shape[0], K = A.Shape[1], K2 = B.Shape[0], N = B.Shape[1];
  if (K != K2) return {nullptr, Errorf("matrix dimensions don't match: A(%dx%d) x B(%dx%d)", M, K, K2, N)};
  auto [out, rerr] = Tensor::NewDeviceResult({M, N});  // fresh zeros: beta scales zeros, as in the reference
  if (rerr) return {nullptr, wrap("failed to create output tensor", rerr)};
  if (Error e = A.EnsureGPU()) return {nullptr, wrap("failed to move A to GPU", e)};
  if (Error e = B.EnsureGPU()) return {nullptr, wrap("failed to move B to GPU", e)};
  CError ce{nullptr};
  int rc = perform_optimized_gemm(A.GPUPtr(), B.GPUPtr(), out->GPUPtr(), M, N, K, alpha, beta, A.DevicePtr(), &ce);
  if (rc != 0) return {nullptr, op_error("optimized GEMM", rc, ce)};
  return {out, {}};
}

Result<TensorPtr> OptimizedBatchMatMul(Tensor &A, Tensor &B) {
  if (A.Shape.size() != 3 || B.Shape.size() != 3)
    return {nullptr, Errorf("batch matrix multiplication requires 3D tensors")};
  const int batch = A.Shape[0], M = A.Shape[1], K = A.Shape[2], K2 = B.Shape[1], N = B.Shape[2];
  if (A.Shape[0] != B.Shape[0]) return {nullptr, Errorf("batch sizes don't match: %d vs %d", A.Shape[0], B.Shape[0])};
  if (K != K2) return {nullptr, Errorf("matrix dimensions don't match: K=%d vs K2=%d", K, K2)};
  auto [out, rerr] = Tensor::NewDeviceResult({batch, M, N});
  if (rerr) return {nullptr, wrap("failed to create output tensor", rerr)};
  if (Error e = A.EnsureGPU()) return {nullptr, wrap("failed to move A to GPU", e)};
  if (Error e = B.EnsureGPU()) return {nullptr, wrap("failed to move B to GPU", e)};
  CError ce{nullptr};
  int rc = perform_batch_matmul_optimized(A.GPUPtr(), B.GPUPtr(), out->GPUPtr(), batch, M, N, K, A.DevicePtr(), &ce);
  if (rc != 0) return {nullptr, op_error("optimized batch matrix multiplication", rc, ce)};
  return {out, {}};
}

// ------------------------------------------------------------------ sparse
namespace {
Error check_matmul_shapes(const std::vector<int> &a, const std::vector<int> &b) {  // sparse-matrix.go:46-52
  if (a.size() != 2 || b.size() != 2) return Errorf("sparse matrix multiplication requires 2D tensors");
  if (a[1] != b[0])
    return Errorf("incompatible matrix dimensions for multiplication: A columns (%d) != B rows (%d)", a[1], b[0]);
  return {};
}
}  // namespace

Result<TensorPtr> SparseMatMul(SparseTensor &A, Tensor &B) {  // sparseDenseMatMul, sparse-matrix.go:134-190
  if (Error e = check_matmul_shapes(A.Shape, B.Shape)) return {nullptr, e};
  if (Error e = A.ConvertToCSR()) return {nullptr, wrap("failed to convert A to CSR", e)};
  if (Error e = A.EnsureGPU()) return {nullptr, wrap("failed to move sparse tensor A to GPU", e)};
  if (Error e = B.EnsureGPU()) return {nullptr, wrap("failed to move tensor B to GPU", e)};
  auto [result, rerr] = Tensor::NewDeviceResult({A.Shape[0], B.Shape[1]});
  if (rerr) return {nullptr, wrap("failed to create result tensor", rerr)};
  CError ce{nullptr};
  int rc = perform_sparse_dense_matmul(
      A.GPUPtr(), A.RowPtr.data(), (long)A.RowPtr.size(), A.Indices.empty() ? nullptr : A.Indices.data(),
      (long)A.Indices.size(), A.Shape[0], A.Shape[1], A.NNZ, B.GPUPtr(), B.Shape[0], B.Shape[1], result->GPUPtr(),
      result->Shape[0], result->Shape[1], A.DevicePtr(), &ce);
  if (rc != 0) return {nullptr, op_error("GPU sparse-dense matrix multiplication", rc, ce)};
  return {result, {}};
}

Result<TensorPtr> SparseMatMul(Tensor &A, Tensor &B) {  // both dense: MatMul (sparse-matrix.go:62-65)
  if (Error e = check_matmul_shapes(A.Shape, B.Shape)) return {nullptr, e};
  return MatMul(A, B);
}

namespace {
template <typename T>
T *data_or_null(std::vector<T> &v) {
  return v.empty() ? nullptr : v.data();
}
}  // namespace

Result<TensorPtr> SparseMatMul(SparseTensor &A, SparseTensor &B) {  // sparseSparseMatMul, sparse-matrix.go:69-131
  if (Error e = check_matmul_shapes(A.Shape, B.Shape)) return {nullptr, e};
  if (Error e = A.ConvertToCSR()) return {nullptr, wrap("failed to convert A to CSR", e)};
  if (Error e = B.ConvertToCSC()) return {nullptr, wrap("failed to convert B to CSC", e)};
  if (Error e = A.EnsureGPU()) return {nullptr, wrap("failed to move sparse tensor A to GPU", e)};
  if (Error e = B.EnsureGPU()) return {nullptr, wrap("failed to move sparse tensor B to GPU", e)};
  auto [result, rerr] = Tensor::NewDeviceResult({A.Shape[0], B.Shape[1]});
  if (rerr) return {nullptr, wrap("failed to create result tensor", rerr)};
  CError ce{nullptr};
  int rc = perform_sparse_sparse_matmul(A.GPUPtr(), A.RowPtr.data(), (long)A.RowPtr.size(), data_or_null(A.Indices),
                                        (long)A.Indices.size(), A.Shape[0], A.Shape[1], A.NNZ, B.GPUPtr(),
                                        B.ColPtr.data(), (long)B.ColPtr.size(), data_or_null(B.Indices),
                                        (long)B.Indices.size(), B.Shape[0], B.Shape[1], B.NNZ, result->GPUPtr(),
                                        result->Shape[0], result->Shape[1], A.DevicePtr(), &ce);
  if (rc != 0) return {nullptr, op_error("GPU sparse-sparse matrix multiplication", rc, ce)};
  return {result, {}};
}

Result<TensorPtr> SparseMatMul(Tensor &A, SparseTensor &B) {  // denseSparseMatMul, sparse-matrix.go:193-250
  if (Error e = check_matmul_shapes(A.Shape, B.Shape)) return {nullptr, e};
  if (Error e = B.ConvertToCSC()) return {nullptr, wrap("failed to convert B to CSC", e)};
  if (Error e = A.EnsureGPU()) return {nullptr, wrap("failed to move tensor A to GPU", e)};
  if (Error e = B.EnsureGPU()) return {nullptr, wrap("failed to move sparse tensor B to GPU", e)};
  auto [result, rerr] = Tensor::NewDeviceResult({A.Shape[0], B.Shape[1]});
  if (rerr) return {nullptr, wrap("failed to create result tensor", rerr)};
  CError ce{nullptr};
  int rc = perform_dense_sparse_matmul(A.GPUPtr(), A.Shape[0], A.Shape[1], B.GPUPtr(), B.ColPtr.data(),
                                       (long)B.ColPtr.size(), data_or_null(B.Indices), (long)B.Indices.size(),
                                       B.Shape[0], B.Shape[1], B.NNZ, result->GPUPtr(), result->Shape[0],
                                       result->Shape[1], A.DevicePtr(), &ce);
  if (rc != 0) return {nullptr, op_error("GPU dense-sparse matrix multiplication", rc, ce)};
  return {result, {}};
}

Result<SparseTensorPtr> SparseAdd(SparseTensor &A, SparseTensor &B) {  // sparse-matrix.go:252-320
  if (Error e = A.IsCompatibleWith(B)) return {nullptr, wrap("incompatible tensors for addition", e)};
  if (Error e = A.ConvertToCSR()) return {nullptr, wrap("failed to convert A to CSR", e)};
  if (Error e = B.ConvertToCSR()) return {nullptr, wrap("failed to convert B to CSR", e)};
  if (Error e = A.EnsureGPU()) return {nullptr, wrap("failed to move sparse tensor A to GPU", e)};
  if (Error e = B.EnsureGPU()) return {nullptr, wrap("failed to move sparse tensor B to GPU", e)};
  const long maxResultNNZ = (long)A.NNZ + (long)B.NNZ;
  std::vector<int32_t> ri((size_t)maxResultNNZ), ci((size_t)maxResultNNZ);
  std::vector<float> vv((size_t)maxResultNNZ);
  long actual = 0;
  CError ce{nullptr};
  int rc = perform_sparse_add(A.GPUPtr(), A.RowPtr.data(), (long)A.RowPtr.size(), data_or_null(A.Indices),
                              (long)A.Indices.size(), A.Shape[0], A.Shape[1], A.NNZ, B.GPUPtr(), B.RowPtr.data(),
                              (long)B.RowPtr.size(), data_or_null(B.Indices), (long)B.Indices.size(), B.Shape[0],
                              B.Shape[1], B.NNZ, data_or_null(ri), data_or_null(ci), data_or_null(vv), &actual,
                              maxResultNNZ, A.DevicePtr(), &ce);
  if (rc != 0) return {nullptr, op_error("GPU sparse addition", rc, ce)};
  ri.resize((size_t)actual);
  ci.resize((size_t)actual);
  vv.resize((size_t)actual);
  return tensor::NewSparseTensorCOO(A.Shape, ri, ci, vv);
}

Result<SparseTensorPtr> SparseScalarMul(SparseTensor &A, float scalar) {  // sparse-matrix.go:322-364
  if (Error e = A.ConvertToCSR()) return {nullptr, wrap("failed to convert A to CSR", e)};
  auto [result, cerr] = A.Clone();
  if (cerr) return {nullptr, wrap("failed to clone sparse tensor", cerr)};
  if (Error e = result->EnsureGPU()) return {nullptr, wrap("failed to move sparse tensor to GPU", e)};
  CError ce{nullptr};
  int rc = perform_sparse_scalar_multiply(result->GPUPtr(), result->RowPtr.data(), (long)result->RowPtr.size(),
                                          data_or_null(result->Indices), (long)result->Indices.size(),
                                          result->Shape[0], result->Shape[1], result->NNZ, scalar,
                                          result->DevicePtr(), &ce);
  if (rc != 0) return {nullptr, op_error("GPU sparse scalar multiplication", rc, ce)};
  return {result, {}};
}

Result<TensorPtr> SparseToDense(SparseTensor &A) {  // sparse-matrix.go:425-473
  if (Error e = A.ConvertToCSR()) return {nullptr, wrap("failed to convert to CSR", e)};
  auto [result, rerr] = Tensor::NewDeviceResult(A.Shape);
  if (rerr) return {nullptr, wrap("failed to create dense result tensor", rerr)};
  if (Error e = A.EnsureGPU()) return {nullptr, wrap("failed to move sparse tensor to GPU", e)};
  CError ce{nullptr};
  int rc = perform_sparse_to_dense(A.GPUPtr(), A.RowPtr.data(), (long)A.RowPtr.size(), data_or_null(A.Indices),
                                   (long)A.Indices.size(), A.Shape[0], A.Shape[1], A.NNZ, result->GPUPtr(),
                                   result->Shape[0], result->Shape[1], A.DevicePtr(), &ce);
  if (rc != 0) return {nullptr, op_error("GPU sparse to dense conversion", rc, ce)};
  return {result, {}};
}

Result<SparseTensorPtr> DenseToSparse(Tensor &A, float threshold) {  // sparse-matrix.go:475-525
  if (A.Shape.size() != 2) return {nullptr, Errorf("dense to sparse conversion requires 2D tensor")};
  const long maxNNZ = (long)A.Shape[0] * A.Shape[1];
  std::vector<int32_t> ri((size_t)maxNNZ), ci((size_t)maxNNZ);
  std::vector<float> vv((size_t)maxNNZ);
  if (Error e = A.EnsureGPU()) return {nullptr, wrap("failed to move tensor to GPU", e)};
  long actual = 0;
  CError ce{nullptr};
  int rc = perform_dense_to_sparse(A.GPUPtr(), A.Shape[0], A.Shape[1], threshold, data_or_null(ri),
                                   data_or_null(ci), data_or_null(vv), &actual, maxNNZ, A.DevicePtr(), &ce);
  if (rc != 0) return {nullptr, op_error("GPU dense to sparse conversion", rc, ce)};
  ri.resize((size_t)actual);
  ci.resize((size_t)actual);
  vv.resize((size_t)actual);
  return tensor::NewSparseTensorCOO(A.Shape, ri, ci, vv);
}

Result<TensorPtr> SparseMatVec(SparseTensor &A, Tensor &x) {  // sparse-matrix.go:527-583
  if (A.Shape.size() != 2 || x.Shape.size() != 1)
    return {nullptr, Errorf("sparse matrix-vector multiplication requires 2D matrix and 1D vector")};
  if (A.Shape[1] != x.Shape[0])
    return {nullptr, Errorf("incompatible dimensions: matrix cols (%d) != vector size (%d)", A.Shape[1], x.Shape[0])};
  if (Error e = A.ConvertToCSR()) return {nullptr, wrap("failed to convert to CSR", e)};
  auto [result, rerr] = Tensor::NewDeviceResult({A.Shape[0]});
  if (rerr) return {nullptr, wrap("failed to create result vector", rerr)};
  if (Error e = A.EnsureGPU()) return {nullptr, wrap("failed to move sparse matrix to GPU", e)};
  if (Error e = x.EnsureGPU()) return {nullptr, wrap("failed to move vector to GPU", e)};
  CError ce{nullptr};
  int rc = perform_sparse_matvec(A.GPUPtr(), A.RowPtr.data(), (long)A.RowPtr.size(),
                                 A.Indices.empty() ? nullptr : A.Indices.data(), (long)A.Indices.size(), A.Shape[0],
                                 A.Shape[1], A.NNZ, x.GPUPtr(), x.Shape[0], result->GPUPtr(), result->Shape[0],
                                 A.DevicePtr(), &ce);
  if (rc != 0) return {nullptr, op_error("GPU sparse matrix-vector multiplication", rc, ce)};
  return {result, {}};
}

Result<SparseTensorPtr> SparseTranspose(const SparseTensor &A) {  // sparse-matrix.go:366-420
  switch (A.Format) {
    case tensor::SparseFormat::COO:
      return tensor::NewSparseTensorCOO({A.Shape[1], A.Shape[0]}, A.ColIndices, A.RowIndices, A.Values);
    case tensor::SparseFormat::CSR:
    case tensor::SparseFormat::CSC: {
      const bool csr = A.Format == tensor::SparseFormat::CSR;
      auto r = std::make_shared<SparseTensor>();
      r->Shape = {A.Shape[1], A.Shape[0]};
      r->Format = csr ? tensor::SparseFormat::CSC : tensor::SparseFormat::CSR;
      r->NNZ = A.NNZ;
      (csr ? r->ColPtr : r->RowPtr) = csr ? A.RowPtr : A.ColPtr;
      r->Indices = A.Indices;
      r->Data = A.Data;
      r->density_ = A.density_;
      return {r, {}};
    }
  }
  return {nullptr, Errorf("unsupported sparse format for transpose: %d", (int)A.Format)};
}

// ------------------------------------------------------------------ fused linear
namespace {
const FusedLinearConfig *linear_config(const std::any &config, bool &ok) {
  ok = true;
  if (auto p = std::any_cast<FusedLinearConfig *>(&config)) return *p;
  if (auto q = std::any_cast<const FusedLinearConfig *>(&config)) return *q;
  ok = false;
  return nullptr;
}

struct FusionRegistry {
  std::mutex mu;
  std::map<std::string, std::shared_ptr<FusedOperation>> ops;
  FusionRegistry() { ops["linear_activation"] = std::make_shared<FusedLinearActivation>(); }
};
FusionRegistry &registry() {
  static FusionRegistry r;
  return r;
}
}  // namespace

void RegisterFusedOperation(const std::string &name, std::shared_ptr<FusedOperation> operation) {
  FusionRegistry &r = registry();
  std::lock_guard<std::mutex> lk(r.mu);
  r.ops[name] = std::move(operation);
}

std::pair<std::shared_ptr<FusedOperation>, bool> GetFusedOperation(const std::string &name) {
  FusionRegistry &r = registry();
  std::lock_guard<std::mutex> lk(r.mu);
  auto it = r.ops.find(name);
  if (it == r.ops.end()) return {nullptr, false};
  return {it->second, true};
}

Result<TensorPtr> FusedLinearActivation::Forward(const std::vector<Tensor *> &inputs, const std::any &config) {
  bool ok;
  const FusedLinearConfig *c = linear_config(config, ok);
  if (!ok) return {nullptr, Errorf("invalid config type for FusedLinearActivation")};
  return Forward(inputs, c);
}

Result<std::vector<TensorPtr>> FusedLinearActivation::Backward(Tensor &gradOutput,
                                                               const std::vector<Tensor *> &savedTensors,
                                                               const std::any &config) {
  bool ok;
  const FusedLinearConfig *c = linear_config(config, ok);
  if (!ok) return {{}, Errorf("invalid config type for FusedLinearActivation backward")};
  return Backward(gradOutput, savedTensors, c);
}

Result<TensorPtr> FusedLinearActivation::Forward(const std::vector<Tensor *> &inputs,
                                                  const FusedLinearConfig *config) {
  if (!config) return {nullptr, Errorf("invalid config type for FusedLinearActivation")};
  if (inputs.size() < 2 || !inputs[0] || !inputs[1])
    return {nullptr, Errorf("FusedLinearActivation requires at least input and weight tensors")};
  Tensor &input = *inputs[0];
  Tensor &weight = *inputs[1];
  Tensor *bias = (inputs.size() >= 3 && config->Bias) ? inputs[2] : nullptr;
  if (input.Shape.size() != 2 || weight.Shape.size() != 2 || input.Shape[1] != weight.Shape[0])
    return {nullptr, Errorf("FusedLinearActivation needs input [batch, in] and weight [in, out]")};
  if (Error e = input.EnsureGPU()) return {nullptr, wrap("failed to move input to GPU", e)};
  if (Error e = weight.EnsureGPU()) return {nullptr, wrap("failed to move weight to GPU", e)};
  if (bias)
    if (Error e = bias->EnsureGPU()) return {nullptr, wrap("failed to move bias to GPU", e)};
  const int batchSize = input.Shape[0], inputSize = input.Shape[1], outputSize = weight.Shape[1];
  auto [output, rerr] = Tensor::NewDeviceResult({batchSize, outputSize});
  if (rerr) return {nullptr, wrap("failed to create output tensor", rerr)};
  // Activation defaults to ReLU (the documented intent of fused-operations.go:432-433).
  int act = ReLU;
  float alpha = 0.0f;
  if (config->Activation) {
    act = config->Activation->ActivationType;
    alpha = config->Activation->Alpha;
  }
  CError ce{nullptr};
  int rc = perform_fused_linear_activation(input.GPUPtr(), batchSize, inputSize, weight.GPUPtr(), outputSize,
                                           bias ? bias->GPUPtr() : nullptr, act, alpha, output->GPUPtr(),
                                           input.DevicePtr(), &ce);
  if (rc != 0) return {nullptr, op_error("fused linear+activation", rc, ce)};
  return {output, {}};
}

namespace {

// C[M,N] = op(A) * op(B) in fp32 on device pointers (row-major, packed), synchronised.
Error gemm_f32(bool ta, bool tb, long M, long N, long K, const float *A, const float *B, float *C, const char *what) {
  CError ce{nullptr};
  int rc = gn_gemm(GN_F32, ta ? 1 : 0, tb ? 1 : 0, M, N, K, 1.0f, A, ta ? M : K, 0, B, tb ? K : N, 0, 0.0f, C, N, 0,
                   1, nullptr, GN_ACT_NONE, 0.0f, nullptr, &ce);
  if (rc == 0) rc = gn_synchronize(nullptr, &ce);
  return rc == 0 ? Error{} : op_error(what, rc, ce);
}

}  // namespace

Result<std::vector<TensorPtr>> FusedLinearActivation::Backward(Tensor &gradOutput,
                                                               const std::vector<Tensor *> &savedTensors,
                                                               const FusedLinearConfig *config) {
  if (!config) return {{}, Errorf("invalid config type for FusedLinearActivation backward")};
  if (savedTensors.size() < 2 || !savedTensors[0] || !savedTensors[1])
    return {{}, Errorf("insufficient saved tensors for FusedLinearActivation backward")};
  Tensor &input = *savedTensors[0];
  Tensor &weight = *savedTensors[1];
  Tensor *pre = savedTensors.size() > 2 ? savedTensors[2] : nullptr;
  if (input.Shape.size() != 2 || weight.Shape.size() != 2 || gradOutput.Shape.size() != 2 ||
      input.Shape[1] != weight.Shape[0] || gradOutput.Shape[0] != input.Shape[0] ||
      gradOutput.Shape[1] != weight.Shape[1])
    return {{}, Errorf("FusedLinearActivation backward needs input [batch,in], weight [in,out], grad [batch,out]")};
  const long batch = input.Shape[0], in = input.Shape[1], out = weight.Shape[1];
  // Step 1: activation backward at the pre-activation (the reference switch, :489-523).
  int act = GN_ACT_NONE;
  float alpha = 0.0f;
  if (config->Activation) {
    switch (config->Activation->ActivationType) {
      case ReLU: case LeakyReLU: case Sigmoid: case Tanh: case GELU:
        act = config->Activation->ActivationType;
        alpha = config->Activation->Alpha;
        break;
      default: break;  // the reference's default branch: gradient passes through
    }
  }
  if (act != GN_ACT_NONE && (!pre || pre->Shape != gradOutput.Shape))
    return {{}, Errorf("failed to apply activation backward: pre-activation tensor [batch,out] required")};
  // Step 2: dropout scaling (:528-537).
  const float scale = config->Dropout > 0.0f ? (float)(1.0 / (1.0 - (double)config->Dropout)) : 1.0f;
  const bool want_bias = config->Bias && savedTensors.size() >= 3;
  if (Error e = gradOutput.EnsureGPU()) return {{}, wrap("failed to move gradient to GPU", e)};
  if (Error e = input.EnsureGPU()) return {{}, wrap("failed to move input to GPU", e)};
  if (Error e = weight.EnsureGPU()) return {{}, wrap("failed to move weight to GPU", e)};
  if (pre && act != GN_ACT_NONE)
    if (Error e = pre->EnsureGPU()) return {{}, wrap("failed to move pre-activation to GPU", e)};
  DeviceScratch g;
  if (Error e = g.alloc((size_t)(batch * out) * 4)) return {{}, e};
  TensorPtr gradBias;
  if (want_bias) {
    auto [gb, berr] = Tensor::NewDeviceResult({1, (int)out});
    if (berr) return {{}, wrap("failed to create bias gradient", berr)};
    gradBias = gb;
  }
  CError ce{nullptr};
  int rc = gn_activation_backward(dptr(gradOutput), act != GN_ACT_NONE ? dptr(*pre) : dptr(gradOutput), batch, out,
                                  act, alpha, scale, (float *)g.p, gradBias ? dptr(*gradBias) : nullptr, nullptr, &ce);
  if (rc != 0) return {{}, op_error("activation backward", rc, ce)};
  // Step 3: grad_input = G W^T, grad_weight = X^T G (:540-563).
  auto [gradInput, ierr] = Tensor::NewDeviceResult({(int)batch, (int)in});
  if (ierr) return {{}, wrap("failed to compute input gradient", ierr)};
  auto [gradWeight, werr] = Tensor::NewDeviceResult({(int)in, (int)out});
  if (werr) return {{}, wrap("failed to compute weight gradient", werr)};
  if (Error e = gemm_f32(false, true, batch, in, out, (const float *)g.p, dptr(weight), dptr(*gradInput),
                         "input gradient"))
    return {{}, e};
  if (Error e = gemm_f32(true, false, in, out, batch, dptr(input), (const float *)g.p, dptr(*gradWeight),
                         "weight gradient"))
    return {{}, e};
  std::vector<TensorPtr> results{gradInput, gradWeight};
  if (gradBias) results.push_back(gradBias);
  return {results, {}};
}

Result<std::vector<TensorPtr>> MatMulBackward(Tensor &gradOutput, Tensor &A, Tensor &B) {
  if (A.Shape.size() != 2 || B.Shape.size() != 2 || gradOutput.Shape.size() != 2 || A.Shape[1] != B.Shape[0] ||
      gradOutput.Shape[0] != A.Shape[0] || gradOutput.Shape[1] != B.Shape[1])
    return {{}, Errorf("insufficient or mismatched tensors for matmul backward")};
  const long M = A.Shape[0], K = A.Shape[1], N = B.Shape[1];
  if (Error e = gradOutput.EnsureGPU()) return {{}, e};
  if (Error e = A.EnsureGPU()) return {{}, e};
  if (Error e = B.EnsureGPU()) return {{}, e};
  auto [gradA, aerr] = Tensor::NewDeviceResult({(int)M, (int)K});
  if (aerr) return {{}, wrap("failed to compute gradient for first input", aerr)};
  auto [gradB, berr] = Tensor::NewDeviceResult({(int)K, (int)N});
  if (berr) return {{}, wrap("failed to compute gradient for second input", berr)};
  if (Error e = gemm_f32(false, true, M, K, N, dptr(gradOutput), dptr(B), dptr(*gradA),
                         "gradient for first input"))
    return {{}, e};
  if (Error e = gemm_f32(true, false, K, N, M, dptr(A), dptr(gradOutput), dptr(*gradB), "gradient for second input"))
    return {{}, e};
  return {{gradA, gradB}, {}};
}

// ------------------------------------------------------------------ mixed precision
// Float32ToFloatMP16 (mixed-precision.go:106-151): truncation toward zero, fp32
// subnormals to signed zero, overflow to infinity, NaN keeps the top mantissa bits.
FloatMP16 Float32ToFloatMP16(float f) {
  uint32_t bits;
  std::memcpy(&bits, &f, 4);
  const uint32_t sign = (bits >> 31) & 1u, exp = (bits >> 23) & 0xFFu;
  uint32_t mant = bits & 0x7FFFFFu;
  if (exp == 0) return (FloatMP16)(sign << 15);
  if (exp == 0xFF) return (FloatMP16)((sign << 15) | 0x7C00u | (mant >> 13));
  const int e = (int)exp - 127 + 15;
  if (e >= 31) return (FloatMP16)((sign << 15) | 0x7C00u);
  if (e <= 0) {
    if (e < -10) return (FloatMP16)(sign << 15);
    mant = (mant | 0x800000u) >> (uint32_t)(1 - e);
    return (FloatMP16)((sign << 15) | (mant >> 13));
  }
  return (FloatMP16)((sign << 15) | ((uint32_t)e << 10) | (mant >> 13));
}

// FloatMP16ToFloat32 (mixed-precision.go:154-189): exact widening.
float FloatMP16ToFloat32(FloatMP16 h) {
  const uint32_t sign = (h >> 15) & 1u;
  uint32_t exp = (h >> 10) & 0x1Fu, mant = h & 0x3FFu, r;
  if (exp == 0) {
    if (mant == 0) {
      r = sign << 31;
    } else {
      while ((mant & 0x400u) == 0) {
        mant <<= 1;
        exp--;
      }
      mant &= 0x3FFu;
      exp = exp - 15 + 127 + 1;
      r = (sign << 31) | (exp << 23) | (mant << 13);
    }
  } else if (exp == 31) {
    r = (sign << 31) | 0x7F800000u | (mant << 13);
  } else {
    r = (sign << 31) | ((exp - 15 + 127) << 23) | (mant << 13);
  }
  float f;
  std::memcpy(&f, &r, 4);
  return f;
}

std::shared_ptr<MixedPrecisionConfig> DefaultMixedPrecisionConfig() { return std::make_shared<MixedPrecisionConfig>(); }

MixedPrecisionTrainer::MixedPrecisionTrainer(std::shared_ptr<MixedPrecisionConfig> cfg)
    : config_(cfg ? cfg : DefaultMixedPrecisionConfig()), currentLossScale_(config_->LossScale) {}

Result<std::shared_ptr<MixedPrecisionTrainer>> NewMixedPrecisionTrainer(std::shared_ptr<MixedPrecisionConfig> cfg) {
  return {std::make_shared<MixedPrecisionTrainer>(std::move(cfg)), {}};
}

Result<TensorPtr> MixedPrecisionTrainer::ConvertTensorToFloat16(const Tensor &input) const {
  std::vector<float> d(input.Data.size());
  for (size_t i = 0; i < d.size(); ++i)
    d[i] = config_->Enabled ? FloatMP16ToFloat32(Float32ToFloatMP16(input.Data[i])) : input.Data[i];
  auto [t, err] = tensor::NewTensor(input.Shape, std::move(d));
  if (err) return {nullptr, wrap("failed to create float16 tensor", err)};
  return {t, {}};
}

namespace {
// input (rounded to fp16 by truncation on the device) x w16 [K, N] (device fp16), plus
// the fp16-rounded bias in the GEMM epilogue; device-resident fp32 result.
// The bias is added as the reference's loop does, result[i] += bias[i % len] over the flat
// output (mixed-precision.go:352-354): by the GEMM epilogue when len is the output width
// (the same sum, one rounding), else by a cyclic add after the product.
Result<TensorPtr> forward_f16(Tensor &input, const void *w16, long K, long N, Tensor *bias) {
  const long M = input.Shape[0];
  const long L = bias ? bias->Size() : 0;
  if (bias && L == 0 && M * N > 0)
    return {nullptr, Errorf("bias is empty: the reference's bias loop would divide by zero")};
  if (Error e = input.EnsureGPU()) return {nullptr, wrap("failed to convert input to float16", e)};
  if (bias && L > 0)
    if (Error e = bias->EnsureGPU()) return {nullptr, wrap("failed to convert bias to float16", e)};
  auto [result, rerr] = Tensor::NewDeviceResult({(int)M, (int)N});
  if (rerr) return {nullptr, wrap("failed to perform float16 matrix multiplication", rerr)};
  DeviceScratch a16, b16, bf;
  if (Error e = a16.alloc((size_t)(M * K) * 2)) return {nullptr, e};
  if (L > 0) {
    if (Error e = b16.alloc((size_t)L * 2)) return {nullptr, e};
    if (Error e = bf.alloc((size_t)L * 4)) return {nullptr, e};
  }
  CError ce{nullptr};
  int rc = gn_cast_f32_f16(dptr(input), (uint16_t *)a16.p, (size_t)(M * K), GN_ROUND_TOWARD_ZERO, nullptr, &ce);
  if (rc == 0 && L > 0) {
    rc = gn_cast_f32_f16(dptr(*bias), (uint16_t *)b16.p, (size_t)L, GN_ROUND_TOWARD_ZERO, nullptr, &ce);
    if (rc == 0) rc = gn_cast_f16_f32((const uint16_t *)b16.p, (float *)bf.p, (size_t)L, nullptr, &ce);
  }
  const bool epilogue = L > 0 && L == N;
  if (rc == 0)
    rc = gn_gemm(GN_F16, 0, 0, M, N, K, 1.0f, a16.p, K, 0, w16, N, 0, 0.0f, dptr(*result), N, 0, 1,
                 epilogue ? (const float *)bf.p : nullptr, GN_ACT_NONE, 0.0f, nullptr, &ce);
  if (rc == 0 && L > 0 && !epilogue)
    rc = gn_add_bias_cyclic_f32((float *)dptr(*result), M * N, (const float *)bf.p, L, nullptr, &ce);
  if (rc == 0) rc = gn_synchronize(nullptr, &ce);
  if (rc != 0) return {nullptr, op_error("float16 matrix multiplication", rc, ce)};
  return {result, {}};
}
}  // namespace

Result<TensorPtr> MixedPrecisionTrainer::ForwardFloat16(Tensor &input, Tensor &weights, Tensor *bias) {
  if (!config_->Enabled) return MatMul(input, weights);
  if (input.Shape.size() != 2 || weights.Shape.size() != 2) return {nullptr, Errorf("MatMul requires 2D tensors (matrices)")};
  const long K = input.Shape[1], N = weights.Shape[1];
  if (weights.Shape[0] != K)
    return {nullptr, Errorf("incompatible matrix dimensions for multiplication: A columns (%ld) != B rows (%d)", K,
                            weights.Shape[0])};
  if (Error e = weights.EnsureGPU()) return {nullptr, wrap("failed to convert weights to float16", e)};
  DeviceScratch w16;
  if (Error e = w16.alloc((size_t)(K * N) * 2)) return {nullptr, e};
  CError ce{nullptr};
  if (int rc = gn_cast_f32_f16(dptr(weights), (uint16_t *)w16.p, (size_t)(K * N), GN_ROUND_TOWARD_ZERO, nullptr, &ce))
    return {nullptr, op_error("float16 matrix multiplication", rc, ce)};
  return forward_f16(input, w16.p, K, N, bias);
}

Result<TensorPtr> MixedPrecisionTrainer::ForwardFloat16(Tensor &input, const tensor::Float16Tensor &weights,
                                                        Tensor *bias) {
  if (input.Shape.size() != 2 || weights.Shape.size() != 2) return {nullptr, Errorf("MatMul requires 2D tensors (matrices)")};
  const long K = input.Shape[1], N = weights.Shape[1];
  if (weights.Shape[0] != K)
    return {nullptr, Errorf("incompatible matrix dimensions for multiplication: A columns (%ld) != B rows (%d)", K,
                            weights.Shape[0])};
  if (!config_->Enabled) {  // fp32 MatMul of the (already rounded) weights, as the reference's disabled path
    auto [w32, err] = weights.ToFloat32();
    if (err) return {nullptr, err};
    return MatMul(input, *w32);
  }
  return forward_f16(input, weights.DeviceData(), K, N, bias);
}

Result<TensorPtr> MatMulFloat16(const tensor::Float16Tensor &A, const tensor::Float16Tensor &B) {
  if (A.Shape.size() != 2 || B.Shape.size() != 2) return {nullptr, Errorf("MatMul requires 2D tensors (matrices)")};
  const long M = A.Shape[0], K = A.Shape[1], N = B.Shape[1];
  if (B.Shape[0] != K)
    return {nullptr, Errorf("incompatible matrix dimensions for multiplication: A columns (%ld) != B rows (%d)", K,
                            B.Shape[0])};
  auto [C, err] = Tensor::NewDeviceResult({(int)M, (int)N});
  if (err) return {nullptr, wrap("failed to create result tensor", err)};
  CError ce{nullptr};
  int rc = gn_gemm(GN_F16, 0, 0, M, N, K, 1.0f, A.DeviceData(), K, 0, B.DeviceData(), N, 0, 0.0f, dptr(*C), N, 0, 1,
                   nullptr, GN_ACT_NONE, 0.0f, nullptr, &ce);
  if (rc == 0) rc = gn_synchronize(nullptr, &ce);
  if (rc != 0) return {nullptr, op_error("float16 matrix multiplication", rc, ce)};
  return {C, {}};
}

// ------------------------------------------------------------------ LinearLayer
namespace {
uint64_t splitmix(uint64_t &s) {
  uint64_t z = (s += 0x9E3779B97F4A7C15ULL);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}
}  // namespace

// layers.go:30-52: Xavier-uniform weights (rand.Float32()*2-1)*sqrt(2/(in+out)); Go's
// global generator is replaced by a seeded SplitMix64 stream.
std::shared_ptr<LinearLayer> NewLinearLayer(int inputSize, int outputSize, bool useBias, uint64_t seed) {
  auto l = std::make_shared<LinearLayer>();
  std::vector<float> w((size_t)inputSize * (size_t)outputSize);
  const float scale = (float)std::sqrt(2.0 / (double)(inputSize + outputSize));
  uint64_t s = seed;
  for (float &x : w) x = ((float)(splitmix(s) >> 40) * (1.0f / 16777216.0f) * 2.0f - 1.0f) * scale;
  l->Weight = tensor::NewTensor({inputSize, outputSize}, std::move(w)).value;
  if (useBias) l->Bias = tensor::NewTensor({outputSize}, std::vector<float>((size_t)outputSize, 0.0f)).value;
  l->InputSize = inputSize;
  l->OutputSize = outputSize;
  l->UseBias = useBias;
  return l;
}

// layers.go:55-74: output = input @ Weight (+ Bias). The bias is added by the GEMM
// epilogue on the device instead of the reference's host loop (layers.go:271-279).
TensorPtr LinearLayer::Forward(TensorPtr input) {
  input_ = input;
  auto zero = [&]() {
    const int rows = input && !input->Shape.empty() ? input->Shape[0] : 0;
    return tensor::NewTensor({rows, OutputSize}, std::vector<float>((size_t)rows * OutputSize, 0.0f)).value;
  };
  if (!input || input->Shape.size() != 2 || input->Shape[1] != Weight->Shape[0]) return zero();
  const bool bias = UseBias && Bias;
  if (input->EnsureGPU() || Weight->EnsureGPU() || (bias && Bias->EnsureGPU())) return zero();
  auto [out, err] = Tensor::NewDeviceResult({input->Shape[0], OutputSize});
  if (err) return zero();
  const long M = input->Shape[0], K = input->Shape[1], N = OutputSize;
  CError ce{nullptr};
  int rc = gn_gemm(GN_F32, 0, 0, M, N, K, 1.0f, dptr(*input), K, 0, dptr(*Weight), N, 0, 0.0f, dptr(*out), N, 0, 1,
                   bias ? dptr(*Bias) : nullptr, GN_ACT_NONE, 0.0f, nullptr, &ce);
  if (rc == 0) rc = gn_synchronize(nullptr, &ce);
  if (rc != 0) {
    if (ce.message) free_c_error_message(ce.message);
    return zero();
  }
  return out;
}

}  // namespace matrix
}  // namespace gometal
