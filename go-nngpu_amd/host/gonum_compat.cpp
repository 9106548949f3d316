// gonum_compat.cpp — gometal::mat (gonum's Matrix interface and Dense) and the
// gonum-compatible wrappers of gometal::matrix: GPUDense / GPUMatMul
// (gpu/matrix/gonum-compat.go) and GPUSparse / GPUSparseMatMul
// (gpu/matrix/sparse-gonum-compat.go). Failures panic, as the Go wrappers do.
#include <cmath>
#include <utility>

#include "gometal.hpp"

namespace gometal {

namespace mat {

Dense::Dense(int r, int c, std::vector<double> data) : rows_(r), cols_(c), data_(std::move(data)) {
  if (r < 0 || c < 0) throw Panic("mat: negative dimension");
  if (data_.empty()) data_.assign((size_t)r * (size_t)c, 0.0);
  if (data_.size() != (size_t)r * (size_t)c) throw Panic("mat: dimension mismatch");
}

double Dense::At(int i, int j) const {
  if (i < 0 || i >= rows_) throw Panic("mat: row index out of range");
  if (j < 0 || j >= cols_) throw Panic("mat: column index out of range");
  return data_[(size_t)i * cols_ + j];
}

void Dense::Set(int i, int j, double v) {
  if (i < 0 || i >= rows_) throw Panic("mat: row index out of range");
  if (j < 0 || j >= cols_) throw Panic("mat: column index out of range");
  data_[(size_t)i * cols_ + j] = v;
}

namespace {
// gonum's mat.Transpose: a view whose At(i, j) is the parent's At(j, i).
class TransposeView : public Matrix {
 public:
  explicit TransposeView(std::shared_ptr<const Matrix> m) : m_(std::move(m)) {}
  void Dims(int &r, int &c) const override { m_->Dims(c, r); }
  double At(int i, int j) const override { return m_->At(j, i); }
  std::shared_ptr<Matrix> T() const override { return std::const_pointer_cast<Matrix>(m_); }

 private:
  std::shared_ptr<const Matrix> m_;
};
}  // namespace

std::shared_ptr<Matrix> Dense::T() const { return std::make_shared<TransposeView>(shared_from_this()); }

std::shared_ptr<Dense> NewDense(int r, int c, std::vector<double> data) {
  return std::make_shared<Dense>(r, c, std::move(data));
}

}  // namespace mat

namespace matrix {

namespace {
[[noreturn]] void panic(const Error &e) { throw Panic(e.message); }

std::shared_ptr<mat::Dense> to_dense(Tensor &t) {  // RetrieveCPU + float64 copy
  if (Error e = t.RetrieveCPU()) panic(e);
  std::vector<double> d(t.Data.begin(), t.Data.end());
  const int r = t.Shape[0], c = t.Shape.size() > 1 ? t.Shape[1] : 1;
  return mat::NewDense(r, c, std::move(d));
}
}  // namespace

// ------------------------------------------------------------------ GPUDense
std::shared_ptr<GPUDense> NewGPUDense(int rows, int cols, const std::vector<double> &data) {
  std::vector<float> f(data.begin(), data.end());  // float64 -> float32 (round to nearest)
  auto [t, err] = tensor::NewTensor({rows, cols}, std::move(f));
  if (err) panic(err);
  return std::make_shared<GPUDense>(t);
}

std::shared_ptr<GPUDense> FromGonum(const mat::Matrix &m) {
  int rows, cols;
  m.Dims(rows, cols);
  std::vector<double> data((size_t)rows * (size_t)cols);
  for (int i = 0; i < rows; ++i)
    for (int j = 0; j < cols; ++j) data[(size_t)i * cols + j] = m.At(i, j);
  return NewGPUDense(rows, cols, data);
}

std::shared_ptr<GPUDense> NewGPUDenseFromTensor(TensorPtr t) { return std::make_shared<GPUDense>(std::move(t)); }

void GPUDense::Dims(int &r, int &c) const {
  r = tensor_->Shape[0];
  c = tensor_->Shape[1];
  if (trans_) std::swap(r, c);
}

double GPUDense::At(int i, int j) const {
  if (Error e = tensor_->RetrieveCPU()) panic(e);
  int rows, cols;
  Dims(rows, cols);
  if (i < 0 || i >= rows || j < 0 || j >= cols) throw Panic("matrix index out of range");
  const int ld = tensor_->Shape[1];
  return trans_ ? tensor_->Data[(size_t)j * ld + i] : tensor_->Data[(size_t)i * ld + j];
}

std::shared_ptr<mat::Matrix> GPUDense::T() const { return std::make_shared<GPUDense>(tensor_, !trans_); }

void GPUDense::detach() {
  if (tensor_.use_count() <= 1) return;
  if (Error e = tensor_->RetrieveCPU()) panic(e);
  auto [t, err] = tensor::NewTensor(tensor_->Shape, tensor_->Data);
  if (err) panic(err);
  tensor_ = t;
}

void GPUDense::Set(int i, int j, double v) {
  detach();  // a T() view and its parent are separate matrices (copy-on-write)
  if (Error e = tensor_->RetrieveCPU()) panic(e);
  int rows, cols;
  Dims(rows, cols);
  if (i < 0 || i >= rows || j < 0 || j >= cols) throw Panic("matrix index out of range");
  const int ld = tensor_->Shape[1];
  (trans_ ? tensor_->Data[(size_t)j * ld + i] : tensor_->Data[(size_t)i * ld + j]) = (float)v;
}

TensorPtr GPUDense::GetTensor() const {
  if (!trans_) return tensor_;
  auto [t, err] = Transpose(*tensor_);
  if (err) panic(err);
  return t;
}

namespace {
// The stored tensor and transpose flag of a matrix operand: a GPUDense (or a view of one)
// as it is, anything else converted by FromGonum (held in `keep`).
Tensor &operand(const mat::Matrix &m, std::shared_ptr<GPUDense> &keep, bool &trans) {
  if (const GPUDense *g = dynamic_cast<const GPUDense *>(&m)) {
    trans = g->IsTransposedView();
    return *g->Storage();
  }
  keep = FromGonum(m);
  trans = false;
  return *keep->Storage();
}
}  // namespace

void GPUDense::Mul(const mat::Matrix &a, const mat::Matrix &b) {
  // GPUDense operands (and their T() views) are used as they are; anything else goes
  // through FromGonum.
  std::shared_ptr<GPUDense> ka, kb;
  bool ta, tb;
  Tensor &A = operand(a, ka, ta);
  Tensor &B = operand(b, kb, tb);
  auto [result, err] = MatMulTransposed(A, ta, B, tb);
  if (err) panic(err);
  // The old tensor goes with its last owner: a T() view taken earlier keeps it, with its data.
  tensor_ = result;  // device-resident until read
  trans_ = false;
}

std::shared_ptr<mat::Dense> GPUDense::ToGonum() const {
  auto d = to_dense(*tensor_);
  if (!trans_) return d;
  int r, c;
  Dims(r, c);
  std::vector<double> t((size_t)r * (size_t)c);
  for (int i = 0; i < r; ++i)
    for (int j = 0; j < c; ++j) t[(size_t)i * c + j] = d->At(j, i);
  return mat::NewDense(r, c, std::move(t));
}

void GPUDense::ReleaseGPU() { tensor_->ReleaseGPU(); }  // Data keeps the values (Tensor::ReleaseGPU)

std::shared_ptr<mat::Dense> GPUMatMul(const mat::Matrix &a, const mat::Matrix &b) {
  // gonum-compat.go:342-367 converts both operands with FromGonum; GPUDense operands and
  // their views are used in place instead (same values: FromGonum would copy them).
  std::shared_ptr<GPUDense> ka, kb;
  bool ta, tb;
  Tensor &A = operand(a, ka, ta);
  Tensor &B = operand(b, kb, tb);
  auto [result, err] = MatMulTransposed(A, ta, B, tb);
  if (err) panic(err);
  auto out = to_dense(*result);
  result->ReleaseGPU();
  return out;
}

std::vector<std::shared_ptr<mat::Dense>> BatchGPUMatMul(const std::vector<MatMulOp> &operations) {
  std::vector<std::shared_ptr<mat::Dense>> results;
  results.reserve(operations.size());
  for (const auto &op : operations) results.push_back(GPUMatMul(*op.A, *op.B));
  return results;
}

// ------------------------------------------------------------------ GPUSparse
std::shared_ptr<GPUSparse> NewGPUSparse(int rows, int cols, const std::vector<int32_t> &rowIndices,
                                        const std::vector<int32_t> &colIndices, const std::vector<float> &values) {
  auto [s, err] = tensor::NewSparseTensorCOO({rows, cols}, rowIndices, colIndices, values);
  if (err) panic(err);
  return std::make_shared<GPUSparse>(s);
}

std::shared_ptr<GPUSparse> NewGPUSparseFromDense(const mat::Matrix &m, double threshold) {
  int rows, cols;
  m.Dims(rows, cols);
  std::vector<int32_t> ri, ci;
  std::vector<float> v;
  for (int i = 0; i < rows; ++i)
    for (int j = 0; j < cols; ++j) {
      const double x = m.At(i, j);
      if (std::fabs(x) > threshold) {  // sparse-gonum-compat.go:36
        ri.push_back(i);
        ci.push_back(j);
        v.push_back((float)x);
      }
    }
  return NewGPUSparse(rows, cols, ri, ci, v);
}

std::shared_ptr<GPUSparse> FromGonumSparse(int rows, int cols, const std::vector<double> &data, double threshold) {
  std::vector<int32_t> ri, ci;
  std::vector<float> v;
  for (int i = 0; i < rows; ++i)
    for (int j = 0; j < cols; ++j) {
      const double x = data[(size_t)i * cols + j];
      if (std::fabs(x) > threshold) {
        ri.push_back(i);
        ci.push_back(j);
        v.push_back((float)x);
      }
    }
  return NewGPUSparse(rows, cols, ri, ci, v);
}

void GPUSparse::Dims(int &r, int &c) const {
  r = sparse_->Shape[0];
  c = sparse_->Shape[1];
}

double GPUSparse::At(int i, int j) const {  // sparse-gonum-compat.go:74-107
  int rows, cols;
  Dims(rows, cols);
  if (i < 0 || i >= rows || j < 0 || j >= cols) throw Panic("matrix index out of range");
  const SparseTensor &s = *sparse_;
  switch (s.Format) {
    case tensor::SparseFormat::COO:
      for (int k = 0; k < s.NNZ; ++k)
        if (s.RowIndices[k] == i && s.ColIndices[k] == j) return s.Values[k];
      break;
    case tensor::SparseFormat::CSR:
      for (int k = s.RowPtr[i]; k < s.RowPtr[i + 1]; ++k)
        if (s.Indices[k] == j) return s.Data[k];
      break;
    case tensor::SparseFormat::CSC:
      for (int k = s.ColPtr[j]; k < s.ColPtr[j + 1]; ++k)
        if (s.Indices[k] == i) return s.Data[k];
      break;
  }
  return 0.0;
}

std::shared_ptr<mat::Matrix> GPUSparse::T() const {
  auto [t, err] = SparseTranspose(*sparse_);
  if (err) panic(err);
  return std::make_shared<GPUSparse>(t);
}

std::shared_ptr<mat::Dense> GPUSparse::SparseMul(SparseTensor &a, Tensor &b) {
  auto [result, err] = SparseMatMul(a, b);
  if (err) panic(err);
  auto out = to_dense(*result);
  result->ReleaseGPU();
  return out;
}

std::shared_ptr<mat::Dense> GPUSparse::SparseMul(Tensor &a, Tensor &b) {
  auto [result, err] = SparseMatMul(a, b);
  if (err) panic(err);
  auto out = to_dense(*result);
  result->ReleaseGPU();
  return out;
}

std::vector<double> GPUSparse::SparseMatVec(const std::vector<double> &x) {  // sparse-gonum-compat.go:187-217
  auto [xt, xerr] = tensor::NewTensor({(int)x.size()}, std::vector<float>(x.begin(), x.end()));
  if (xerr) panic(xerr);
  auto [result, err] = matrix::SparseMatVec(*sparse_, *xt);
  if (err) panic(err);
  if (Error e = result->RetrieveCPU()) panic(e);
  std::vector<double> out(result->Data.begin(), result->Data.end());
  result->ReleaseGPU();
  xt->ReleaseGPU();
  return out;
}

std::shared_ptr<mat::Dense> GPUSparseMatMul(const mat::Matrix &a, const mat::Matrix &b) {
  // sparse-gonum-compat.go:253-337: a *GPUSparse operand stays sparse, any other
  // mat.Matrix becomes a dense fp32 tensor.
  auto densify = [](const mat::Matrix &m) { return FromGonum(m)->GetTensor(); };
  const GPUSparse *sa = dynamic_cast<const GPUSparse *>(&a);
  const GPUSparse *sb = dynamic_cast<const GPUSparse *>(&b);
  TensorPtr da = sa ? nullptr : densify(a);
  TensorPtr db = sb ? nullptr : densify(b);
  Result<TensorPtr> r;
  if (sa && !sb) r = SparseMatMul(*sa->GetSparseTensor(), *db);
  else if (!sa && !sb) r = SparseMatMul(*da, *db);
  else if (sa && sb) r = SparseMatMul(*sa->GetSparseTensor(), *sb->GetSparseTensor());
  else r = SparseMatMul(*da, *sb->GetSparseTensor());
  if (r.err) panic(r.err);
  auto out = to_dense(*r.value);
  r.value->ReleaseGPU();
  return out;
}

std::vector<std::shared_ptr<mat::Dense>> BatchGPUSparseMatMul(const std::vector<SparseMatMulOp> &operations) {
  std::vector<std::shared_ptr<mat::Dense>> results;
  results.reserve(operations.size());
  for (const auto &op : operations) results.push_back(GPUSparseMatMul(*op.A, *op.B));
  return results;
}

std::vector<std::vector<double>> BatchGPUSparseMatVec(const std::vector<std::shared_ptr<GPUSparse>> &matrices,
                                                      const std::vector<std::vector<double>> &vectors) {
  if (matrices.size() != vectors.size()) throw Panic("number of matrices must equal number of vectors");
  std::vector<std::vector<double>> results;
  results.reserve(matrices.size());
  for (size_t i = 0; i < matrices.size(); ++i) results.push_back(matrices[i]->SparseMatVec(vectors[i]));
  return results;
}

}  // namespace matrix
}  // namespace gometal
