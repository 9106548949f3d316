// tensor.cpp — gometal::tensor: Tensor residency over the C ABI, the global device
// memory statistics, and SparseTensor (COO / CSR / CSC) construction and conversion.
#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <numeric>
#include <unordered_map>

#include "../../include/gonngpu.h"
#include "gometal.hpp"

namespace gometal {

Error Errorf(const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  return Error{buf};
}

namespace {
// Converts a failed C-ABI call into an Error, freeing the message as the Go code does
// (tensor/tensor.go:135-142).
Error abi_error(const char *what, int code, CError &e) {
  std::string msg;
  if (e.message) {
    msg = e.message;
    free_c_error_message(e.message);
    e.message = nullptr;
  }
  return Errorf("%s (code %d): %s", what, code, msg.c_str());
}
}  // namespace

namespace tensor {

// ------------------------------------------------------------------ memory statistics
// GlobalMemoryPool (tensor/tensor.go:22-77): allocations made by Tensor.EnsureGPU.
namespace {
struct Pool {
  std::mutex mu;
  std::unordered_map<void *, int64_t> allocations;
  int64_t total = 0, peak = 0;
};
Pool &pool() {
  static Pool *p = new Pool();
  return *p;
}
void track(void *ptr, int64_t bytes) {
  Pool &p = pool();
  std::lock_guard<std::mutex> lk(p.mu);
  p.allocations[ptr] = bytes;
  p.total += bytes;
  p.peak = std::max(p.peak, p.total);
}
void untrack(void *ptr) {
  Pool &p = pool();
  std::lock_guard<std::mutex> lk(p.mu);
  auto it = p.allocations.find(ptr);
  if (it != p.allocations.end()) {
    p.total -= it->second;
    p.allocations.erase(it);
  }
}
}  // namespace

MemoryStats GetGlobalMemoryStats() {
  Pool &p = pool();
  std::lock_guard<std::mutex> lk(p.mu);
  return MemoryStats{p.total, p.peak, (int)p.allocations.size()};
}

// ------------------------------------------------------------------ Tensor
long Tensor::Size() const {
  long n = 1;
  for (int d : Shape) n *= d;
  return n;
}

Result<TensorPtr> NewTensor(std::vector<int> shape, std::vector<float> data) {
  long size = 1;
  for (int d : shape) size *= d;
  if ((long)data.size() != size)
    return {nullptr, Errorf("data length (%zu) does not match shape dimensions (%ld)", data.size(), size)};
  auto t = std::make_shared<Tensor>();
  t->Shape = std::move(shape);
  t->Data = std::move(data);
  return {t, {}};
}

Tensor::~Tensor() { dropDeviceCopy(); }

void Tensor::dropDeviceCopy() {
  if (gpuPtr_ && isOwner_) {
    untrack(gpuPtr_);
    release_gpu_buffer(gpuPtr_);
  }
  gpuPtr_ = nullptr;
  gpuBytes_ = 0;
  isOnGPU_ = false;
}

Error Tensor::EnsureGPU() {
  if (isOnGPU_) return {};
  // A device copy left behind by RetrieveCPU may be stale (host writes); replace it.
  dropDeviceCopy();
  const long bytes = (long)Data.size() * (long)sizeof(float);
  ::GPUPtr buf = nullptr;
  ::DevicePtr dev = nullptr;
  CError e{nullptr};
  int rc = create_gpu_buffer(Data.empty() ? nullptr : Data.data(), bytes, &buf, &dev, &e);
  if (rc != 0) return abi_error("failed to create GPU buffer", rc, e);
  gpuPtr_ = buf;
  devicePtr_ = dev;
  gpuBytes_ = bytes;
  isOnGPU_ = true;
  isOwner_ = true;
  track(gpuPtr_, bytes);
  return {};
}

Result<TensorPtr> Tensor::NewDeviceResult(std::vector<int> shape) {
  long size = 1;
  for (int d : shape) size *= d;
  auto t = std::make_shared<Tensor>();
  t->Shape = std::move(shape);
  t->Data.assign((size_t)size, 0.0f);
  const long bytes = size * (long)sizeof(float);
  ::GPUPtr buf = nullptr;
  ::DevicePtr dev = nullptr;
  CError e{nullptr};
  int rc = create_gpu_buffer(nullptr, bytes, &buf, &dev, &e);  // zero-filled on the device
  if (rc != 0) return {nullptr, abi_error("failed to create result GPU buffer", rc, e)};
  t->gpuPtr_ = buf;
  t->devicePtr_ = dev;
  t->gpuBytes_ = bytes;
  t->isOnGPU_ = true;
  t->hostStale_ = true;
  track(buf, bytes);
  return {t, {}};
}

Error Tensor::RetrieveCPU() {
  if (!isOnGPU_) return {};
  if (!gpuPtr_) return Errorf("tensor is marked as on GPU but has no GPU pointer");
  CError e{nullptr};
  const long bytes = (long)Data.size() * (long)sizeof(float);
  int rc = retrieve_gpu_buffer_data(gpuPtr_, Data.empty() ? nullptr : Data.data(), bytes, &e);
  if (rc != 0) return abi_error("failed to retrieve GPU buffer data", rc, e);
  isOnGPU_ = false;  // tensor.go:182; the allocation is kept until replaced or freed
  hostStale_ = false;
  return {};
}

void Tensor::ReleaseGPU() {
  if (!(isOnGPU_ && gpuPtr_ && isOwner_)) return;
  // Data must hold the device's results afterwards, as the reference's aliased slice does.
  if (hostStale_ && RetrieveCPU()) return;  // keep the only valid copy if the read-back fails
  dropDeviceCopy();
}

// ------------------------------------------------------------------ Float16Tensor
Float16Tensor::~Float16Tensor() {
  if (data_) gn_free(data_);
}

long Float16Tensor::Size() const {
  long n = 1;
  for (int d : Shape) n *= d;
  return n;
}

Result<Float16TensorPtr> Float16Tensor::FromTensor(Tensor &t, bool truncate) {
  Float16TensorPtr h(new Float16Tensor());
  h->Shape = t.Shape;
  const long n = t.Size();
  if (Error e = t.EnsureGPU()) return {nullptr, e};
  CError ce{nullptr};
  int rc = n > 0 ? gn_malloc(&h->data_, (size_t)n * 2, &ce) : 0;
  if (rc == 0 && n > 0)
    rc = gn_cast_f32_f16(static_cast<const float *>(gn_buffer_device_ptr(t.GPUPtr())),
                         static_cast<uint16_t *>(h->data_), (size_t)n,
                         truncate ? GN_ROUND_TOWARD_ZERO : GN_ROUND_NEAREST_EVEN, nullptr, &ce);
  if (rc == 0) rc = gn_synchronize(nullptr, &ce);
  if (rc != 0) return {nullptr, abi_error("float16 conversion", rc, ce)};
  return {h, {}};
}

Result<TensorPtr> Float16Tensor::ToFloat32() const {
  auto [t, err] = Tensor::NewDeviceResult(Shape);
  if (err) return {nullptr, err};
  CError ce{nullptr};
  int rc = Size() > 0 ? gn_cast_f16_f32(static_cast<const uint16_t *>(data_),
                                        static_cast<float *>(gn_buffer_device_ptr(t->GPUPtr())), (size_t)Size(),
                                        nullptr, &ce)
                      : 0;
  if (rc == 0) rc = gn_synchronize(nullptr, &ce);
  if (rc != 0) return {nullptr, abi_error("float16 widening", rc, ce)};
  return {t, {}};
}

// ------------------------------------------------------------------ SparseTensor
std::string String(SparseFormat f) {
  switch (f) {
    case SparseFormat::COO: return "COO";
    case SparseFormat::CSR: return "CSR";
    case SparseFormat::CSC: return "CSC";
  }
  return "Unknown";
}

Result<SparseTensorPtr> NewSparseTensorCOO(std::vector<int> shape, const std::vector<int32_t> &rowIndices,
                                           const std::vector<int32_t> &colIndices, const std::vector<float> &values) {
  if (rowIndices.size() != colIndices.size() || rowIndices.size() != values.size())
    return {nullptr, Errorf("length mismatch: rowIndices=%zu, colIndices=%zu, values=%zu", rowIndices.size(),
                            colIndices.size(), values.size())};
  if (shape.size() != 2)
    return {nullptr, Errorf("sparse tensors currently support only 2D matrices, got %zu dimensions", shape.size())};
  const int rows = shape[0], cols = shape[1];
  for (size_t i = 0; i < rowIndices.size(); ++i) {
    if (rowIndices[i] < 0 || rowIndices[i] >= rows)
      return {nullptr, Errorf("row index %d out of bounds [0, %d)", rowIndices[i], rows)};
    if (colIndices[i] < 0 || colIndices[i] >= cols)
      return {nullptr, Errorf("column index %d out of bounds [0, %d)", colIndices[i], cols)};
  }
  auto st = std::make_shared<SparseTensor>();
  st->Shape = std::move(shape);
  st->Format = SparseFormat::COO;
  st->NNZ = (int)values.size();
  st->RowIndices = rowIndices;
  st->ColIndices = colIndices;
  st->Values = values;
  st->density_ = (double)values.size() / ((double)rows * (double)cols);
  return {st, {}};
}

Result<SparseTensorPtr> NewSparseTensorFromDense(const Tensor &dense, float threshold) {
  if (dense.Shape.size() != 2) return {nullptr, Errorf("sparse tensors currently support only 2D matrices")};
  const int rows = dense.Shape[0], cols = dense.Shape[1];
  std::vector<int32_t> ri, ci;
  std::vector<float> v;
  for (int i = 0; i < rows; ++i)
    for (int j = 0; j < cols; ++j) {
      const float x = dense.Data[(size_t)i * cols + j];
      if (x > threshold || x < -threshold) {  // sparse-tensor.go:113
        ri.push_back(i);
        ci.push_back(j);
        v.push_back(x);
      }
    }
  return NewSparseTensorCOO(dense.Shape, ri, ci, v);
}

namespace {
// Sorts COO triplets by (major, minor) and fills ptr/idx/data, as ConvertToCSR /
// ConvertToCSC do (sparse-tensor.go:143-177). The sort is stable, so duplicates keep
// their COO order (Go's sort.Slice leaves their order unspecified).
void compress(int nmajor, const std::vector<int32_t> &major, const std::vector<int32_t> &minor,
              const std::vector<float> &vals, std::vector<int32_t> &ptr, std::vector<int32_t> &idx,
              std::vector<float> &data) {
  const size_t nnz = vals.size();
  std::vector<size_t> order(nnz);
  std::iota(order.begin(), order.end(), 0);
  std::stable_sort(order.begin(), order.end(), [&](size_t a, size_t b) {
    return major[a] != major[b] ? major[a] < major[b] : minor[a] < minor[b];
  });
  ptr.assign((size_t)nmajor + 1, 0);
  idx.resize(nnz);
  data.resize(nnz);
  for (size_t k = 0; k < nnz; ++k) {
    ptr[(size_t)major[order[k]] + 1]++;
    idx[k] = minor[order[k]];
    data[k] = vals[order[k]];
  }
  for (int r = 0; r < nmajor; ++r) ptr[(size_t)r + 1] += ptr[(size_t)r];
}
}  // namespace

Error SparseTensor::ConvertToCSR() {
  if (Format == SparseFormat::CSR) return {};
  if (Format != SparseFormat::COO) return Errorf("can only convert from COO to CSR format");
  compress(Shape[0], RowIndices, ColIndices, Values, RowPtr, Indices, Data);
  Format = SparseFormat::CSR;
  return {};
}

Error SparseTensor::ConvertToCSC() {
  if (Format == SparseFormat::CSC) return {};
  if (Format != SparseFormat::COO) return Errorf("can only convert from COO to CSC format");
  compress(Shape[1], ColIndices, RowIndices, Values, ColPtr, Indices, Data);
  Format = SparseFormat::CSC;
  return {};
}

Result<TensorPtr> SparseTensor::ToDense() const {
  const int rows = Shape[0], cols = Shape[1];
  std::vector<float> d((size_t)rows * (size_t)cols, 0.0f);
  switch (Format) {  // later duplicates overwrite earlier ones (sparse-tensor.go:246-266)
    case SparseFormat::COO:
      for (int k = 0; k < NNZ; ++k) d[(size_t)RowIndices[k] * cols + ColIndices[k]] = Values[k];
      break;
    case SparseFormat::CSR:
      for (int r = 0; r < rows; ++r)
        for (int k = RowPtr[r]; k < RowPtr[r + 1]; ++k) d[(size_t)r * cols + Indices[k]] = Data[k];
      break;
    case SparseFormat::CSC:
      for (int c = 0; c < cols; ++c)
        for (int k = ColPtr[c]; k < ColPtr[c + 1]; ++k) d[(size_t)Indices[k] * cols + c] = Data[k];
      break;
  }
  return NewTensor(Shape, std::move(d));
}

SparseTensor::~SparseTensor() {
  if (gpuPtr_ && IsOwner) release_gpu_buffer(gpuPtr_);
}

Error SparseTensor::EnsureGPU() {
  if (isOnGPU_) return {};
  if (Format == SparseFormat::COO)
    if (Error e = ConvertToCSR()) return Errorf("failed to convert to CSR format: %s", e.message.c_str());
  if (Format != SparseFormat::CSR && Format != SparseFormat::CSC)
    return Errorf("GPU operations require CSR or CSC format");
  if (gpuPtr_ && IsOwner) release_gpu_buffer(gpuPtr_);
  gpuPtr_ = nullptr;
  if (Data.empty()) {  // empty sparse matrix: no buffer (sparse-tensor.go:311-315)
    isOnGPU_ = true;
    return {};
  }
  ::GPUPtr buf = nullptr;
  ::DevicePtr dev = nullptr;
  CError e{nullptr};
  int rc = create_gpu_buffer(Data.data(), (long)(Data.size() * sizeof(float)), &buf, &dev, &e);
  if (rc != 0) return abi_error("failed to create sparse GPU buffer", rc, e);
  gpuPtr_ = buf;
  devicePtr_ = dev;
  isOnGPU_ = true;
  return {};
}

Error SparseTensor::RetrieveCPU() {
  if (!isOnGPU_) return {};
  if (Data.empty()) {
    isOnGPU_ = false;
    return {};
  }
  if (!gpuPtr_) return Errorf("sparse tensor is marked as on GPU but has no GPU pointer");
  CError e{nullptr};
  int rc = retrieve_gpu_buffer_data(gpuPtr_, Data.data(), (long)(Data.size() * sizeof(float)), &e);
  if (rc != 0) return abi_error("failed to retrieve sparse GPU buffer data", rc, e);
  isOnGPU_ = false;
  return {};
}

void SparseTensor::ReleaseGPU() {
  if (isOnGPU_ && gpuPtr_ && IsOwner) {
    release_gpu_buffer(gpuPtr_);
    gpuPtr_ = nullptr;
    isOnGPU_ = false;
  }
}

Error SparseTensor::IsCompatibleWith(const SparseTensor &other) const {
  if (Shape.size() != other.Shape.size())
    return Errorf("dimension mismatch: %zu vs %zu", Shape.size(), other.Shape.size());
  for (size_t i = 0; i < Shape.size(); ++i)
    if (Shape[i] != other.Shape[i])
      return Errorf("shape mismatch at dimension %zu: %d vs %d", i, Shape[i], other.Shape[i]);
  return {};
}

Result<SparseTensorPtr> SparseTensor::Clone() const {
  auto c = std::make_shared<SparseTensor>();
  c->Shape = Shape;
  c->Format = Format;
  c->NNZ = NNZ;
  c->density_ = density_;
  switch (Format) {
    case SparseFormat::COO:
      c->RowIndices = RowIndices;
      c->ColIndices = ColIndices;
      c->Values = Values;
      break;
    case SparseFormat::CSR:
      c->RowPtr = RowPtr;
      c->Indices = Indices;
      c->Data = Data;
      break;
    case SparseFormat::CSC:
      c->ColPtr = ColPtr;
      c->Indices = Indices;
      c->Data = Data;
      break;
  }
  return {c, {}};
}

}  // namespace tensor
}  // namespace gometal
