// gometal.hpp — C++ host API of the MI355X GEMM/SpMM backend, mirroring the Go
// packages of go-nngpu (module github.com/tsawler/gometal) for the matmul path:
//
//   gometal::tensor   tensor/tensor.go, tensor/sparse-tensor.go
//   gometal::matrix   gpu/matrix/matrix.go (MatMul, Transpose), sparse-matrix.go
//                     (SparseMatMul, SparseMatVec, SparseTranspose), optimized-kernels.go
//                     (OptimizedGEMM, OptimizedBatchMatMul), fused-operations.go
//                     (FusedLinearActivation), mixed-precision.go (FloatMP16,
//                     MixedPrecisionTrainer), layers.go (LinearLayer), activation.go
//                     (ActivationType), gonum-compat.go (GPUDense, GPUMatMul),
//                     sparse-gonum-compat.go (GPUSparse, GPUSparseMatMul)
//   gometal::mat      the part of gonum's mat package those files use: the Matrix
//                     interface and a row-major float64 Dense
//
// Names, argument meaning and error behaviour follow the Go code. Go's (T, error)
// returns become Result<T> (usable as `auto [t, err] = ...`); a nil error is an empty
// Error. Go panics (the gonum-compatible wrappers panic on failure) become a thrown
// gometal::Panic. Every device operation goes through the C ABI in include/gonngpu.h,
// exactly as the Go code goes through cgo.
//
// Residency: a Tensor's device copy is a GPUPtr from create_gpu_buffer. Unlike the
// reference's Metal buffers it does not alias Data: EnsureGPU copies Data to the
// device, RetrieveCPU copies the device copy back into Data and marks the tensor as
// host-resident (isOnGPU = false, as tensor/tensor.go:182 does), and the next
// EnsureGPU uploads Data again, so host writes between the two are seen. The device
// allocation is released when it is replaced or when the tensor is destroyed.
#pragma once

#include <any>
#include <cstdint>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

namespace gometal {

// ---------------------------------------------------------------- errors
struct Error {
  std::string message;
  explicit operator bool() const { return !message.empty(); }  // true = an error
};
Error Errorf(const char *fmt, ...) __attribute__((format(printf, 1, 2)));

template <typename T>
struct Result {
  T value;
  Error err;
};

// A Go panic raised by the gonum-compatible wrappers.
struct Panic : std::runtime_error {
  using std::runtime_error::runtime_error;
};

namespace tensor {

class Tensor;
class SparseTensor;
using TensorPtr = std::shared_ptr<Tensor>;
using SparseTensorPtr = std::shared_ptr<SparseTensor>;
class Float16Tensor;
using Float16TensorPtr = std::shared_ptr<Float16Tensor>;

// GetGlobalMemoryStats (tensor/tensor.go:74-77): bytes held by tensors' device
// copies, the peak of that, and the number of live allocations.
struct MemoryStats {
  int64_t currentUsage, peakUsage;
  int numAllocations;
};
MemoryStats GetGlobalMemoryStats();

// tensor.Tensor (tensor/tensor.go:80-87): fp32 data with shape, plus a device copy.
class Tensor {
 public:
  std::vector<int> Shape;
  std::vector<float> Data;

  Tensor() = default;
  Tensor(const Tensor &) = delete;
  Tensor &operator=(const Tensor &) = delete;
  ~Tensor();

  Error EnsureGPU();   // tensor.go:113-150
  Error RetrieveCPU();  // tensor.go:154-184
  // tensor.go:189-202. The reference's buffer aliases Data, so after the release Data
  // holds what the device computed; here a device copy newer than Data (a GPU result not
  // yet retrieved) is copied back first, then the allocation is returned.
  void ReleaseGPU();
  void *GPUPtr() const { return gpuPtr_; }        // tensor.go:206
  void *DevicePtr() const { return devicePtr_; }  // tensor.go:211
  bool IsOnGPU() const { return isOnGPU_; }
  long Size() const;  // product of Shape

  // Result tensors of GPU operations: Data sized but left zero, a device buffer
  // allocated without an upload, marked device-resident.
  static Result<TensorPtr> NewDeviceResult(std::vector<int> shape);

 private:
  void *gpuPtr_ = nullptr;
  void *devicePtr_ = nullptr;
  bool isOnGPU_ = false;
  bool isOwner_ = true;
  bool hostStale_ = false;  // the device copy is newer than Data (NewDeviceResult)
  long gpuBytes_ = 0;
  void dropDeviceCopy();
};

// A device-resident fp16 matrix with no host copy: the fp16 data type of the chaining
// path. Operands converted once (weights, typically) are reused by every fp16 GEMM
// (MixedPrecisionTrainer::ForwardFloat16, matrix::MatMulFloat16) without another upload
// or cast. FromTensor converts an fp32 tensor on the device, with the reference's
// truncation (Float32ToFloatMP16, gpu/matrix/mixed-precision.go:106-151) by default or
// with IEEE round-to-nearest-even.
class Float16Tensor {
 public:
  std::vector<int> Shape;

  Float16Tensor(const Float16Tensor &) = delete;
  Float16Tensor &operator=(const Float16Tensor &) = delete;
  ~Float16Tensor();
  static Result<Float16TensorPtr> FromTensor(Tensor &t, bool truncate = true);
  const void *DeviceData() const { return data_; }
  long Size() const;
  Result<TensorPtr> ToFloat32() const;  // exact fp16 -> fp32 widening, device-resident

 private:
  Float16Tensor() = default;
  void *data_ = nullptr;
};


// NewTensor (tensor.go:90-109): len(data) must equal the product of shape.
Result<TensorPtr> NewTensor(std::vector<int> shape, std::vector<float> data);

// tensor.SparseFormat (sparse-tensor.go:18-24).
enum class SparseFormat { COO = 0, CSR = 1, CSC = 2 };
std::string String(SparseFormat f);  // sparse-tensor.go:423-434

// tensor.SparseTensor (sparse-tensor.go:27-51): 2-D, int32 indices, fp32 values;
// explicit zeros and duplicate coordinates are kept.
class SparseTensor {
 public:
  std::vector<int> Shape;
  SparseFormat Format = SparseFormat::COO;
  int NNZ = 0;
  std::vector<int32_t> RowIndices, ColIndices;  // COO
  std::vector<float> Values;
  std::vector<int32_t> RowPtr, ColPtr, Indices;  // CSR (RowPtr) / CSC (ColPtr)
  std::vector<float> Data;
  bool IsOwner = true;

  SparseTensor() = default;
  SparseTensor(const SparseTensor &) = delete;
  SparseTensor &operator=(const SparseTensor &) = delete;
  ~SparseTensor();

  Error ConvertToCSR();                  // sparse-tensor.go:127-181
  Error ConvertToCSC();                  // sparse-tensor.go:184-238
  Result<TensorPtr> ToDense() const;     // sparse-tensor.go:241-272
  Error EnsureGPU();                     // sparse-tensor.go:275-337 (uploads Data only)
  Error RetrieveCPU();                   // sparse-tensor.go:340-384
  void ReleaseGPU();                     // sparse-tensor.go:387-395
  void *GPUPtr() const { return gpuPtr_; }
  void *DevicePtr() const { return devicePtr_; }
  bool IsOnGPU() const { return isOnGPU_; }
  double GetDensity() const { return density_; }  // :408
  int GetNNZ() const { return NNZ; }              // :413
  SparseFormat GetFormat() const { return Format; }
  Error IsCompatibleWith(const SparseTensor &other) const;  // :437-449
  Result<SparseTensorPtr> Clone() const;                   // :452-489

  double density_ = 0.0;

 private:
  void *gpuPtr_ = nullptr;
  void *devicePtr_ = nullptr;
  bool isOnGPU_ = false;
};

// NewSparseTensorCOO (sparse-tensor.go:54-99) and NewSparseTensorFromDense (:102-124,
// keeps |v| > threshold).
Result<SparseTensorPtr> NewSparseTensorCOO(std::vector<int> shape, const std::vector<int32_t> &rowIndices,
                                           const std::vector<int32_t> &colIndices, const std::vector<float> &values);
Result<SparseTensorPtr> NewSparseTensorFromDense(const Tensor &dense, float threshold);

}  // namespace tensor

namespace mat {

// gonum's mat.Matrix interface (the subset the reference's wrappers implement).
class Matrix {
 public:
  virtual ~Matrix() = default;
  virtual void Dims(int &r, int &c) const = 0;
  virtual double At(int i, int j) const = 0;
  virtual std::shared_ptr<Matrix> T() const = 0;
};
using MatrixPtr = std::shared_ptr<Matrix>;

// gonum's mat.Dense: row-major float64; NewDense panics if len(data) != r*c.
class Dense : public Matrix, public std::enable_shared_from_this<Dense> {
 public:
  Dense(int r, int c, std::vector<double> data);
  void Dims(int &r, int &c) const override { r = rows_; c = cols_; }
  double At(int i, int j) const override;
  std::shared_ptr<Matrix> T() const override;  // a transposed view, as gonum's mat.Transpose
  void Set(int i, int j, double v);
  const std::vector<double> &RawData() const { return data_; }

 private:
  int rows_, cols_;
  std::vector<double> data_;
};
std::shared_ptr<Dense> NewDense(int r, int c, std::vector<double> data);

}  // namespace mat

namespace matrix {

using tensor::Tensor;
using tensor::TensorPtr;
using tensor::SparseTensor;
using tensor::SparseTensorPtr;

// ActivationType (gpu/matrix/activation.go:18-29).
enum ActivationType { ReLU = 0, Sigmoid = 1, Tanh = 2, Softmax = 3, LeakyReLU = 4, ELU = 5, Swish = 6, GELU = 7 };
std::string String(ActivationType t);  // activation.go:32-53 ("Unknown" otherwise)

// ActivationForward (activation.go:56-175): a new tensor of input's shape holding
// act(input), computed on the device by the perform_activation_*_forward entries. Softmax
// is row-wise over the last dimension of a 1-D or 2-D tensor; other ranks are an error,
// as are an empty shape and an unknown type. alpha is used by LeakyReLU and ELU.
Result<TensorPtr> ActivationForward(Tensor &input, ActivationType activationType, float alpha);

// SetGlobalMatrixDevice (matrix.go:22-24). The reference routes MatMul through a
// unified-memory adapter once a device is set (:27-50), which loses the result (defect
// D2). Here the device is implicit (one GPU per process), so the pointer is only kept.
void SetGlobalMatrixDevice(void *device);

// Dense ops (gpu/matrix/matrix.go:53-105, :357-404).
Result<TensorPtr> MatMul(Tensor &A, Tensor &B);
Result<TensorPtr> Transpose(Tensor &A);

// C = A * B of two device fp16 matrices (fp16 MFMA, fp32 accumulation), device-resident
// fp32 result: chained fp16 GEMMs without host round trips or casts of their operands.
Result<TensorPtr> MatMulFloat16(const tensor::Float16Tensor &A, const tensor::Float16Tensor &B);

// Custom-kernel GEMMs (gpu/matrix/optimized-kernels.go:21-75, :78-135).
Result<TensorPtr> OptimizedGEMM(Tensor &A, Tensor &B, float alpha, float beta);
Result<TensorPtr> OptimizedBatchMatMul(Tensor &A, Tensor &B);

// Sparse ops (gpu/matrix/sparse-matrix.go). SparseMatMul dispatches on operand kinds
// like the Go type switch (:20-66): sparse x dense is the CSR SpMM kernel (:134-190),
// sparse x sparse converts A to CSR and B to CSC (:69-131), dense x sparse converts B
// to CSC (:193-250), dense x dense is MatMul. Conversions follow the reference: only
// COO converts, so a CSR operand where CSC is needed is an error.
Result<TensorPtr> SparseMatMul(SparseTensor &A, Tensor &B);
Result<TensorPtr> SparseMatMul(Tensor &A, Tensor &B);
Result<TensorPtr> SparseMatMul(SparseTensor &A, SparseTensor &B);
Result<TensorPtr> SparseMatMul(Tensor &A, SparseTensor &B);
Result<TensorPtr> SparseMatVec(SparseTensor &A, Tensor &x);
Result<SparseTensorPtr> SparseTranspose(const SparseTensor &A);
// SparseAdd (:252-320): A + B as a new COO tensor (coinciding entries summed, zero
// sums dropped).
Result<SparseTensorPtr> SparseAdd(SparseTensor &A, SparseTensor &B);
// SparseScalarMul (:322-364): a CSR clone with its values scaled on the GPU (the
// clone's host Data is refreshed by RetrieveCPU, as in the reference).
Result<SparseTensorPtr> SparseScalarMul(SparseTensor &A, float scalar);
// SparseToDense (:425-473) and DenseToSparse (:475-525; keeps |v| > threshold, COO).
Result<TensorPtr> SparseToDense(SparseTensor &A);
Result<SparseTensorPtr> DenseToSparse(Tensor &A, float threshold);

// Fused linear + activation (gpu/matrix/fused-operations.go:24-54, :380-465).
struct FusedActivationConfig {
  gometal::matrix::ActivationType ActivationType = ReLU;
  float Alpha = 0.0f;
  bool InPlace = false;
};
struct FusedLinearConfig {
  bool Bias = false;
  std::shared_ptr<FusedActivationConfig> Activation;  // nil -> ReLU
  float Dropout = 0.0f;
};
// FusedOperation (fused-operations.go:67-73). config stands for Go's interface{}: a
// std::any holding a pointer to the operation's config type (FusedLinearConfig * or
// const FusedLinearConfig * for linear_activation); anything else is "invalid config
// type", as a failed Go type assertion.
class FusedOperation {
 public:
  virtual ~FusedOperation() = default;
  virtual Result<TensorPtr> Forward(const std::vector<Tensor *> &inputs, const std::any &config) = 0;
  virtual Result<std::vector<TensorPtr>> Backward(Tensor &gradOutput, const std::vector<Tensor *> &savedTensors,
                                                  const std::any &config) = 0;
  virtual std::string GetName() const = 0;
  virtual int64_t GetMemorySavings() const = 0;
  virtual float GetSpeedup() const = 0;
};

class FusedLinearActivation : public FusedOperation {
 public:
  std::string GetName() const override { return "linear_activation"; }
  int64_t GetMemorySavings() const override { return 512 * 1024; }  // fused-operations.go:372-374
  float GetSpeedup() const override { return 1.4f; }                 // :376-378
  Result<TensorPtr> Forward(const std::vector<Tensor *> &inputs, const std::any &config) override;
  Result<std::vector<TensorPtr>> Backward(Tensor &gradOutput, const std::vector<Tensor *> &savedTensors,
                                          const std::any &config) override;
  // inputs = {input [batch,in], weight [in,out], optional bias [out]}.
  Result<TensorPtr> Forward(const std::vector<Tensor *> &inputs, const FusedLinearConfig *config);
  // FusedLinearActivation.Backward (fused-operations.go:467-578). savedTensors =
  // {input [batch,in], weight [in,out], pre-activation [batch,out] (needed by ReLU,
  // LeakyReLU, Sigmoid, Tanh and GELU)}. Returns {grad_input [batch,in],
  // grad_weight [in,out]} plus grad_bias [1,out] when config->Bias and three tensors
  // were saved. A nil activation, and Softmax / ELU / Swish, pass the gradient through
  // unchanged, as the reference's switch does.
  Result<std::vector<TensorPtr>> Backward(Tensor &gradOutput, const std::vector<Tensor *> &savedTensors,
                                          const FusedLinearConfig *config);
};

// The fusion registry (fused-operations.go:75-121). It starts with linear_activation,
// the one fused operation on this library's path; the reference's other entries
// (conv_bn_relu, attention, gelu_dropout, layer_norm_linear, residual_block) are not
// provided, so looking them up reports false. Safe for concurrent use.
void RegisterFusedOperation(const std::string &name, std::shared_ptr<FusedOperation> operation);
std::pair<std::shared_ptr<FusedOperation>, bool> GetFusedOperation(const std::string &name);

// matmulBackward of gpu/matrix/gradient.go:601-637 for C = A * B:
// {grad_A = grad_output * B^T, grad_B = A^T * grad_output} (device-resident).
Result<std::vector<TensorPtr>> MatMulBackward(Tensor &gradOutput, Tensor &A, Tensor &B);

// MPSGraphManager (gpu/matrix/mps-graph-integration.go:15-296): named graph tensors,
// MatMul and activation nodes, compiled subgraphs and their execution, over the graph
// calls of the C ABI (a compiled subgraph is a HIP graph; a MatMul read only by one
// activation runs as one GEMM with the activation in its epilogue, the LinearActivation
// fusion of :103-115). Names follow the Go code: MatMulOp returns "matmul_<a>_<b>",
// ActivationOp "<type>_<input>". Unknown names, mismatched shapes and unknown activation
// types panic, where the Go code would dereference a nil tensor or panic itself (:209).
// CompileGraph and Execute report errors instead of returning nil / empty maps.
struct CompiledOperation {
  void *Executable = nullptr;  // the compiled HIP graph (owned by the manager)
  std::vector<std::string> Inputs, Outputs;
  std::vector<std::vector<int>> InputShapes, OutputShapes;
  std::string CacheKey;
};
class MPSGraphManager {
 public:
  explicit MPSGraphManager(void *device = nullptr);
  ~MPSGraphManager();
  MPSGraphManager(const MPSGraphManager &) = delete;
  MPSGraphManager &operator=(const MPSGraphManager &) = delete;
  // A 2-D placeholder ("float16" / "half": fp16 on the device, cast from the fp32 input
  // tensors at execution; anything else fp32). Cached by name, as :136-148.
  void *CreateTensor(const std::string &name, const std::vector<int> &shape, const std::string &dataType);
  std::string MatMulOp(const std::string &a, const std::string &b, bool transposeA, bool transposeB);
  std::string ActivationOp(const std::string &input, const std::string &activationType);  // ReLU, Sigmoid, Tanh
  // Cached by "inputs->outputs" (:227-268).
  Result<std::shared_ptr<CompiledOperation>> CompileGraph(const std::vector<std::string> &inputs,
                                                          const std::vector<std::string> &outputs);
  // Runs a compiled subgraph: inputs by name (fp32 host tensors, uploaded as needed);
  // the outputs come back as device-resident tensors by name.
  Result<std::map<std::string, TensorPtr>> Execute(const CompiledOperation &compiled,
                                                   const std::map<std::string, Tensor *> &inputs);

 private:
  struct Node {
    void *handle;
    std::vector<int> shape;
    bool half;
  };
  void *graph_ = nullptr;
  std::mutex mu_;
  std::map<std::string, Node> tensors_;
  std::map<std::string, std::shared_ptr<CompiledOperation>> compiled_;
  const Node &node(const std::string &name) const;
};

// Mixed precision (gpu/matrix/mixed-precision.go).
using FloatMP16 = uint16_t;
FloatMP16 Float32ToFloatMP16(float f);   // :106-151 (truncation, reference bit semantics)
float FloatMP16ToFloat32(FloatMP16 h);   // :154-189
struct MixedPrecisionConfig {
  bool Enabled = true;
  float LossScale = 65536.0f;
  float LossScaleGrowthRate = 2.0f;
  float LossScaleBackoffRate = 0.5f;
  int GrowthInterval = 2000;
  float MaxLossScale = 1048576.0f;
  float MinLossScale = 1.0f;
  bool SkipOverflowSteps = true;
};
std::shared_ptr<MixedPrecisionConfig> DefaultMixedPrecisionConfig();  // :38-49
class MixedPrecisionTrainer {
 public:
  explicit MixedPrecisionTrainer(std::shared_ptr<MixedPrecisionConfig> cfg);
  // :192-210: fp32 values rounded through FloatMP16 (stored as fp32).
  Result<TensorPtr> ConvertTensorToFloat16(const Tensor &input) const;
  // :315-358: input x weights on fp16-rounded operands, plus the fp16-rounded bias added as
  // the reference's loop does, result[i] += bias[i % len(bias)] over the flat output (in the
  // GEMM epilogue when len is the output width). Runs the cast and an fp16 MFMA GEMM (exact
  // fp16 products, fp32 accumulation) on the device; an empty bias is an error.
  Result<TensorPtr> ForwardFloat16(Tensor &input, Tensor &weights, Tensor *bias);
  // The same product with weights already converted (Float16Tensor::FromTensor with the
  // default truncation): bit-identical to the call above, without the weights' cast.
  Result<TensorPtr> ForwardFloat16(Tensor &input, const tensor::Float16Tensor &weights, Tensor *bias);
  float GetCurrentLossScale() const { return currentLossScale_; }

 private:
  std::shared_ptr<MixedPrecisionConfig> config_;
  float currentLossScale_;
};
Result<std::shared_ptr<MixedPrecisionTrainer>> NewMixedPrecisionTrainer(std::shared_ptr<MixedPrecisionConfig> cfg);

// LinearLayer (gpu/matrix/layers.go:11-74): Y = X W + b with W [in, out].
class LinearLayer {
 public:
  TensorPtr Weight, Bias;
  int InputSize = 0, OutputSize = 0;
  bool UseBias = false;
  // Returns a zero output on failure, as the reference does (layers.go:61-67).
  TensorPtr Forward(TensorPtr input);

 private:
  TensorPtr input_;
};
std::shared_ptr<LinearLayer> NewLinearLayer(int inputSize, int outputSize, bool useBias, uint64_t seed = 1);

// gonum-compatible dense wrapper (gpu/matrix/gonum-compat.go:9-110, :321-367, :744-827).
//
// T() returns a transposed view, as gonum's mat.Transpose does, instead of the reference's
// materialised GPU transpose (gonum-compat.go:61-68): the view shares the tensor, and Dims,
// At, Set and ToGonum read it transposed. Mul and GPUMatMul hand a view's tensor to the
// GEMM with its transpose flag (the kernels read op(A) = A^T in place), so Mul(a.T(), b)
// is one GEMM launch with no transpose kernel and no copy. GetTensor() of a view returns a
// materialised transpose (a tensor of the view's shape); ReleaseGPU() of a view does
// nothing (the view owns no device memory).
class GPUDense : public mat::Matrix {
 public:
  explicit GPUDense(TensorPtr t, bool transposed = false) : tensor_(std::move(t)), trans_(transposed) {}
  void Dims(int &r, int &c) const override;
  double At(int i, int j) const override;         // panics on out-of-range indices
  // The transpose. As in the reference (gonum-compat.go:61-68, a materialised Transpose) it
  // behaves as an independent matrix; it starts as a view of the same tensor (so that Mul
  // and GPUMatMul read it in place, with a transposed GEMM operand) and the two share the
  // tensor copy-on-write: Set on either first gives it a private copy, and Mul replaces
  // only the receiver's tensor.
  std::shared_ptr<mat::Matrix> T() const override;
  void Set(int i, int j, double v);
  void Mul(const mat::Matrix &a, const mat::Matrix &b);  // receiver := a*b (device-resident)
  std::shared_ptr<mat::Dense> ToGonum() const;
  void ReleaseGPU();
  TensorPtr GetTensor() const;
  bool IsTransposedView() const { return trans_; }
  // The stored tensor and whether this matrix is its transpose (what the GEMM consumes).
  const TensorPtr &Storage() const { return tensor_; }

 private:
  TensorPtr tensor_;
  bool trans_ = false;
  void detach();  // gives this matrix a private copy of a tensor it shares
};
// C = op(A) * op(B) on the device, with op(X) = X^T when the flag is set: the GEMM reads
// the stored operands in place (device-resident fp32 result).
Result<TensorPtr> MatMulTransposed(Tensor &A, bool transA, Tensor &B, bool transB);
std::shared_ptr<GPUDense> NewGPUDense(int rows, int cols, const std::vector<double> &data);
std::shared_ptr<GPUDense> FromGonum(const mat::Matrix &m);
std::shared_ptr<GPUDense> NewGPUDenseFromTensor(TensorPtr t);
std::shared_ptr<mat::Dense> GPUMatMul(const mat::Matrix &a, const mat::Matrix &b);
struct MatMulOp {
  std::shared_ptr<mat::Matrix> A, B;
};
std::vector<std::shared_ptr<mat::Dense>> BatchGPUMatMul(const std::vector<MatMulOp> &operations);

// gonum-compatible sparse wrapper (gpu/matrix/sparse-gonum-compat.go:12-382).
class GPUSparse : public mat::Matrix {
 public:
  explicit GPUSparse(SparseTensorPtr s) : sparse_(std::move(s)) {}
  void Dims(int &r, int &c) const override;
  double At(int i, int j) const override;  // first stored entry at (i, j), else 0
  std::shared_ptr<mat::Matrix> T() const override;
  int GetNNZ() const { return sparse_->GetNNZ(); }
  double GetDensity() const { return sparse_->GetDensity(); }
  tensor::SparseFormat GetFormat() const { return sparse_->GetFormat(); }
  Error ConvertToCSR() { return sparse_->ConvertToCSR(); }
  Error ConvertToCSC() { return sparse_->ConvertToCSC(); }
  // (*GPUSparse).SparseMul(a, b) (sparse-gonum-compat.go:147-166): SparseMatMul(a, b)
  // returned as a mat::Dense; the receiver itself is not an operand.
  std::shared_ptr<mat::Dense> SparseMul(SparseTensor &a, Tensor &b);
  std::shared_ptr<mat::Dense> SparseMul(Tensor &a, Tensor &b);
  std::vector<double> SparseMatVec(const std::vector<double> &x);
  void ReleaseGPU() { sparse_->ReleaseGPU(); }
  SparseTensorPtr GetSparseTensor() const { return sparse_; }

 private:
  SparseTensorPtr sparse_;
};
std::shared_ptr<GPUSparse> NewGPUSparse(int rows, int cols, const std::vector<int32_t> &rowIndices,
                                        const std::vector<int32_t> &colIndices, const std::vector<float> &values);
std::shared_ptr<GPUSparse> NewGPUSparseFromDense(const mat::Matrix &m, double threshold);
std::shared_ptr<GPUSparse> FromGonumSparse(int rows, int cols, const std::vector<double> &data, double threshold);
// GPUSparseMatMul (sparse-gonum-compat.go:253-337): a *GPUSparse operand stays sparse,
// any other mat::Matrix is densified.
std::shared_ptr<mat::Dense> GPUSparseMatMul(const mat::Matrix &a, const mat::Matrix &b);
struct SparseMatMulOp {
  std::shared_ptr<mat::Matrix> A, B;
};
std::vector<std::shared_ptr<mat::Dense>> BatchGPUSparseMatMul(const std::vector<SparseMatMulOp> &operations);
std::vector<std::vector<double>> BatchGPUSparseMatVec(const std::vector<std::shared_ptr<GPUSparse>> &matrices,
                                                      const std::vector<std::vector<double>> &vectors);

}  // namespace matrix
}  // namespace gometal
