// Tests of the C++ host API (go-nngpu_amd/host/gometal.hpp), written in the shape of
// the reference's Go tests: one function per behaviour, checked against the CPU
// checker in oracle/ (linked as test infrastructure) or against closed forms.
//
//   test_host --cpu   host-only behaviour (no device calls)
//   test_host --gpu   everything, including the device paths through the C ABI
#include <algorithm>
#include <any>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "../../go-nngpu_amd/host/gometal.hpp"
#include "../../include/gonngpu.h"
#include "../../oracle/oracle.h"

using namespace gometal;
using gometal::tensor::NewSparseTensorCOO;
using gometal::tensor::NewTensor;
using gometal::tensor::SparseFormat;

namespace {

int g_failures = 0;
std::string g_current;

void fail(const char *file, int line, const std::string &what) {
  ++g_failures;
  std::printf("  FAIL %s (%s:%d): %s\n", g_current.c_str(), file, line, what.c_str());
  std::fflush(stdout);
}
#define CHECK(cond)                                    \
  do {                                                 \
    if (!(cond)) fail(__FILE__, __LINE__, #cond);      \
  } while (0)
#define CHECK_NOERR(err)                                                        \
  do {                                                                          \
    const gometal::Error &e_ = (err);                                           \
    if (e_) fail(__FILE__, __LINE__, std::string("unexpected error: ") + e_.message); \
  } while (0)
#define CHECK_ERR_HAS(err, sub)                                                                     \
  do {                                                                                              \
    const gometal::Error &e_ = (err);                                                               \
    if (!e_) fail(__FILE__, __LINE__, std::string("expected error containing: ") + (sub));          \
    else if (e_.message.find(sub) == std::string::npos)                                             \
      fail(__FILE__, __LINE__, std::string("error '") + e_.message + "' lacks '" + (sub) + "'");    \
  } while (0)
#define CHECK_PANICS(stmt)                              \
  do {                                                  \
    bool p_ = false;                                    \
    try {                                               \
      stmt;                                             \
    } catch (const gometal::Panic &) {                  \
      p_ = true;                                        \
    }                                                   \
    if (!p_) fail(__FILE__, __LINE__, "expected a panic: " #stmt); \
  } while (0)

std::vector<float> uniform(size_t n, uint64_t stream, float lo = -1.0f, float hi = 1.0f) {
  std::vector<float> v(n);
  orc_fill_uniform_f32(v.data(), n, 42, stream, lo, hi);
  return v;
}

// relFrob of fp32 data against a float64 reference.
double rel(const std::vector<float> &x, const std::vector<double> &r) { return orc_rel_frob(x.data(), r.data(), x.size()); }

std::vector<double> gemm64(const std::vector<float> &A, const std::vector<float> &B, long M, long N, long K) {
  std::vector<double> C((size_t)(M * N));
  orc_gemm_f64(0, 0, M, N, K, 1.0, A.data(), K, B.data(), N, 0.0, C.data(), N, 8);
  return C;
}

// ============================================================== host-only tests
void TestNewTensorValidates() {
  auto [t, err] = NewTensor({2, 3}, std::vector<float>(6, 1.0f));
  CHECK_NOERR(err);
  CHECK(t && t->Size() == 6 && !t->IsOnGPU());
  auto [bad, err2] = NewTensor({2, 3}, std::vector<float>(5));
  CHECK(!bad);
  CHECK_ERR_HAS(err2, "does not match shape dimensions");
}

void TestSparseCOOValidation() {
  CHECK_ERR_HAS(NewSparseTensorCOO({4, 4}, {0, 1}, {0}, {1.f, 2.f}).err, "length mismatch");
  CHECK_ERR_HAS(NewSparseTensorCOO({4, 4, 4}, {0}, {0}, {1.f}).err, "only 2D");
  CHECK_ERR_HAS(NewSparseTensorCOO({4, 4}, {4}, {0}, {1.f}).err, "row index 4 out of bounds");
  CHECK_ERR_HAS(NewSparseTensorCOO({4, 4}, {0}, {-1}, {1.f}).err, "column index -1 out of bounds");
  auto [s, err] = NewSparseTensorCOO({4, 5}, {0, 3}, {1, 4}, {1.f, 0.f});  // explicit zero is kept
  CHECK_NOERR(err);
  CHECK(s->GetNNZ() == 2 && s->GetFormat() == SparseFormat::COO);
  CHECK(std::fabs(s->GetDensity() - 2.0 / 20.0) < 1e-12);
  CHECK(tensor::String(SparseFormat::CSR) == "CSR" && tensor::String(SparseFormat::CSC) == "CSC");
}

void TestConvertToCSRMatchesOracle() {
  // COO with duplicates, explicit zeros, empty rows and arbitrary order.
  const int rows = 50, cols = 40;
  std::vector<int32_t> ri, ci;
  std::vector<float> v;
  uint64_t x = 7;
  for (int k = 0; k < 400; ++k) {
    x = x * 6364136223846793005ULL + 1442695040888963407ULL;
    int r = (int)((x >> 33) % rows);
    if (r % 7 == 3) continue;  // empty rows
    ri.push_back(r);
    ci.push_back((int)((x >> 13) % cols));
    v.push_back((k % 11 == 0) ? 0.0f : (float)((int)((x >> 40) % 200) - 100) / 8.0f);
  }
  ri.push_back(5); ci.push_back(6); v.push_back(1.5f);  // duplicate coordinates
  ri.push_back(5); ci.push_back(6); v.push_back(-0.25f);
  auto [s, err] = NewSparseTensorCOO({rows, cols}, ri, ci, v);
  CHECK_NOERR(err);
  CHECK_NOERR(s->ConvertToCSR());
  std::vector<int32_t> rp(rows + 1), idx(v.size());
  std::vector<float> data(v.size());
  CHECK(orc_coo_to_csr(rows, cols, (long)v.size(), ri.data(), ci.data(), v.data(), rp.data(), idx.data(),
                       data.data()) == 0);
  CHECK(s->Format == SparseFormat::CSR && s->RowPtr == rp && s->Indices == idx && s->Data == data);
  CHECK_NOERR(s->ConvertToCSR());                          // no-op
  CHECK_ERR_HAS(s->ConvertToCSC(), "can only convert from COO to CSC");
  // ToDense: last duplicate wins (sparse-tensor.go:251-258)
  auto [d, derr] = s->ToDense();
  CHECK_NOERR(derr);
  std::vector<float> ref((size_t)rows * cols);
  orc_csr_to_dense(rows, cols, rp.data(), idx.data(), data.data(), ref.data());
  CHECK(d->Data == ref);
  // CSC of the same COO densifies to the same matrix
  auto [s2, e2] = NewSparseTensorCOO({rows, cols}, ri, ci, v);
  CHECK_NOERR(e2);
  CHECK_NOERR(s2->ConvertToCSC());
  CHECK(s2->ColPtr.size() == (size_t)cols + 1 && s2->ColPtr.back() == (int)v.size());
  for (int c = 0; c < cols; ++c)
    for (int k = s2->ColPtr[c] + 1; k < s2->ColPtr[c + 1]; ++k) CHECK(s2->Indices[k - 1] <= s2->Indices[k]);
  CHECK(s2->ToDense().value->Data == ref);
  // Clone copies the compressed arrays
  auto [c, cerr] = s->Clone();
  CHECK_NOERR(cerr);
  CHECK(c->RowPtr == s->RowPtr && c->Data == s->Data && c->Format == SparseFormat::CSR);
  CHECK_NOERR(s->IsCompatibleWith(*c));
  CHECK_ERR_HAS(s->IsCompatibleWith(*NewSparseTensorCOO({rows, cols + 1}, {}, {}, {}).value), "shape mismatch");
}

void TestSparseTranspose() {
  auto [s, err] = NewSparseTensorCOO({3, 5}, {0, 2, 2}, {4, 0, 1}, {1.f, 2.f, 3.f});
  CHECK_NOERR(err);
  auto [t, terr] = matrix::SparseTranspose(*s);
  CHECK_NOERR(terr);
  CHECK(t->Shape == std::vector<int>({5, 3}) && t->RowIndices == s->ColIndices);
  CHECK_NOERR(s->ConvertToCSR());
  auto [tc, tcerr] = matrix::SparseTranspose(*s);
  CHECK_NOERR(tcerr);
  CHECK(tc->Format == SparseFormat::CSC && tc->ColPtr == s->RowPtr);
  matrix::GPUSparse gs(tc);
  for (int i = 0; i < 5; ++i)
    for (int j = 0; j < 3; ++j) CHECK(gs.At(i, j) == matrix::GPUSparse(s).At(j, i));
}

void TestFloatMP16MatchesReferenceBits() {
  // Float32ToFloatMP16 against the oracle's restatement over a spread of values.
  uint64_t x = 1;
  for (int k = 0; k < 200000; ++k) {
    x = x * 6364136223846793005ULL + 1442695040888963407ULL;
    uint32_t bits = (uint32_t)(x >> 32);
    float f;
    std::memcpy(&f, &bits, 4);
    CHECK(matrix::Float32ToFloatMP16(f) == orc_f32_to_f16_rtz(f));
    if (g_failures) return;
  }
  for (uint32_t h = 0; h < 65536; ++h) {
    const float a = matrix::FloatMP16ToFloat32((uint16_t)h), b = orc_f16_to_f32((uint16_t)h);
    CHECK(std::memcmp(&a, &b, 4) == 0 || (std::isnan(a) && std::isnan(b)));
  }
  CHECK(matrix::Float32ToFloatMP16(1.0f) == 0x3C00 && matrix::Float32ToFloatMP16(65520.0f) == 0x7BFF);
}

void TestMixedPrecisionConfigDefaults() {
  auto c = matrix::DefaultMixedPrecisionConfig();
  CHECK(c->Enabled && c->LossScale == 65536.0f && c->MaxLossScale == 1048576.0f && c->GrowthInterval == 2000);
  auto [mp, err] = matrix::NewMixedPrecisionTrainer(nullptr);
  CHECK_NOERR(err);
  CHECK(mp->GetCurrentLossScale() == 65536.0f);
  auto [t, e2] = NewTensor({4}, {1.0f, 1.0009765625f, 1.00048828125f, 0.1f});
  CHECK_NOERR(e2);
  auto [h, e3] = mp->ConvertTensorToFloat16(*t);
  CHECK_NOERR(e3);
  CHECK(h->Data[0] == 1.0f && h->Data[1] == 1.0009765625f && h->Data[2] == 1.0f);  // truncation
  CHECK(h->Data[3] == orc_f16_to_f32(orc_f32_to_f16_rtz(0.1f)));
}

void TestGonumDense() {
  auto d = mat::NewDense(2, 3, {1, 2, 3, 4, 5, 6});
  int r, c;
  d->Dims(r, c);
  CHECK(r == 2 && c == 3 && d->At(1, 2) == 6);
  auto t = d->T();
  t->Dims(r, c);
  CHECK(r == 3 && c == 2 && t->At(2, 1) == 6 && t->At(0, 1) == 4);
  CHECK_PANICS(d->At(2, 0));
  CHECK_PANICS(mat::NewDense(2, 2, {1, 2, 3}));
}

void TestGPUSparseAtAndErrors() {
  auto gs = matrix::NewGPUSparse(3, 3, {0, 1, 1}, {0, 2, 2}, {5.f, 7.f, 9.f});
  CHECK(gs->At(0, 0) == 5 && gs->At(1, 2) == 7 && gs->At(2, 2) == 0);  // first duplicate wins
  CHECK_PANICS(gs->At(3, 0));
  CHECK_PANICS(matrix::NewGPUSparse(3, 3, {0}, {3}, {1.f}));
  CHECK_NOERR(gs->ConvertToCSR());
  CHECK(gs->At(1, 2) == 7 && gs->GetNNZ() == 3);
  auto dense = mat::NewDense(2, 2, {0.5, -0.05, 0, 2});
  auto fs = matrix::NewGPUSparseFromDense(*dense, 0.1);  // strict |v| > threshold
  CHECK(fs->GetNNZ() == 2 && fs->At(0, 1) == 0);
  CHECK_PANICS(matrix::BatchGPUSparseMatVec({fs}, {}));
}

void TestShapeErrorsBeforeDevice() {
  auto a = NewTensor({2, 3}, std::vector<float>(6)).value;
  auto b = NewTensor({2, 3}, std::vector<float>(6)).value;
  auto v = NewTensor({6}, std::vector<float>(6)).value;
  CHECK_ERR_HAS(matrix::MatMul(*a, *b).err, "A columns (3) != B rows (2)");
  CHECK_ERR_HAS(matrix::MatMul(*a, *v).err, "requires 2D tensors");
  CHECK_ERR_HAS(matrix::Transpose(*v).err, "requires 2D tensor");
  CHECK_ERR_HAS(matrix::OptimizedGEMM(*a, *b, 1, 0).err, "don't match");
  CHECK_ERR_HAS(matrix::OptimizedBatchMatMul(*a, *b).err, "requires 3D tensors");
  auto s = NewSparseTensorCOO({3, 4}, {0}, {0}, {1.f}).value;
  CHECK_ERR_HAS(matrix::SparseMatMul(*s, *a).err, "A columns (4) != B rows (2)");
  CHECK_ERR_HAS(matrix::SparseMatVec(*s, *v).err, "matrix cols (4) != vector size (6)");
  CHECK_ERR_HAS(matrix::SparseMatMul(*s, *s).err, "incompatible matrix dimensions");
  auto sq = NewSparseTensorCOO({3, 3}, {0}, {0}, {1.f}).value;
  // the same tensor as both operands: A goes to CSR, then B (already CSR) cannot become
  // CSC, as in sparseSparseMatMul (sparse-matrix.go:71-76, sparse-tensor.go:189-191)
  CHECK_ERR_HAS(matrix::SparseMatMul(*sq, *sq).err, "can only convert from COO to CSC format");
  // ActivationForward (activation.go:56-175): errors before any device call
  tensor::Tensor empty;
  CHECK_ERR_HAS(matrix::ActivationForward(empty, matrix::ReLU, 0).err, "cannot apply activation to empty tensor");
  auto t3 = NewTensor({2, 1, 3}, std::vector<float>(6)).value;
  CHECK_ERR_HAS(matrix::ActivationForward(*t3, matrix::Softmax, 0).err, "softmax currently supports only 1D and 2D");
  CHECK(matrix::String(matrix::GELU) == "GELU" && matrix::String((matrix::ActivationType)42) == "Unknown");
  CHECK_ERR_HAS(matrix::ActivationForward(*t3, (matrix::ActivationType)42, 0).err, "unsupported activation type: Unknown");
  matrix::FusedLinearActivation f;
  CHECK_ERR_HAS(f.Forward({a.get(), b.get()}, nullptr).err, "invalid config");
  matrix::FusedLinearConfig cfg;
  CHECK_ERR_HAS(f.Forward({a.get()}, &cfg).err, "requires at least input and weight");
}

void TestFusionRegistry() {
  auto [op, ok] = matrix::GetFusedOperation("linear_activation");
  CHECK(ok && op && op->GetName() == "linear_activation");
  CHECK(op->GetMemorySavings() == 512 * 1024 && op->GetSpeedup() == 1.4f);
  CHECK(!matrix::GetFusedOperation("attention").second);  // not on this library's path
  auto x = NewTensor({2, 3}, std::vector<float>(6)).value;
  auto w = NewTensor({3, 4}, std::vector<float>(12)).value;
  CHECK_ERR_HAS(op->Forward({x.get(), w.get()}, std::any(42)).err, "invalid config type for FusedLinearActivation");
  CHECK_ERR_HAS(op->Backward(*x, {x.get(), w.get()}, std::any()).err, "invalid config type for FusedLinearActivation backward");
  matrix::RegisterFusedOperation("my_linear", std::make_shared<matrix::FusedLinearActivation>());
  CHECK(matrix::GetFusedOperation("my_linear").second);
}

// ============================================================== device tests
void TestActivationForward() {
  // activation_test.go:32-51: ReLU of [-2,-1,0,1,2,3]
  auto x = NewTensor({2, 3}, {-2, -1, 0, 1, 2, 3}).value;
  auto [r, err] = matrix::ActivationForward(*x, matrix::ReLU, 0);
  CHECK_NOERR(err);
  CHECK_NOERR(r->RetrieveCPU());
  CHECK((r->Data == std::vector<float>{0, 0, 0, 1, 2, 3}));
  auto in = NewTensor({64, 129}, uniform(64 * 129, 9, -6.0f, 6.0f)).value;
  const matrix::ActivationType types[] = {matrix::ReLU, matrix::Sigmoid, matrix::Tanh, matrix::LeakyReLU,
                                          matrix::ELU, matrix::Swish, matrix::GELU};
  for (matrix::ActivationType t : types) {
    const float alpha = t == matrix::LeakyReLU ? 0.1f : 1.0f;
    auto y = matrix::ActivationForward(*in, t, alpha).value;
    CHECK(y && y->Shape == in->Shape);
    if (!y) continue;
    CHECK_NOERR(y->RetrieveCPU());
    std::vector<double> ref(in->Data.size());
    for (size_t i = 0; i < ref.size(); ++i) ref[i] = orc_act_f64((int)t, alpha, in->Data[i]);
    CHECK(rel(y->Data, ref) <= 1e-5);
  }
  std::vector<double> sm(in->Data.size());
  orc_softmax_rows_f64(64, 129, in->Data.data(), sm.data());
  auto s2 = matrix::ActivationForward(*in, matrix::Softmax, 0).value;
  CHECK_NOERR(s2->RetrieveCPU());
  CHECK(rel(s2->Data, sm) <= 1e-5);
  auto v = NewTensor({129}, std::vector<float>(in->Data.begin(), in->Data.begin() + 129)).value;
  auto s1 = matrix::ActivationForward(*v, matrix::Softmax, 0).value;
  CHECK_NOERR(s1->RetrieveCPU());
  CHECK(rel(s1->Data, std::vector<double>(sm.begin(), sm.begin() + 129)) <= 1e-5);
}

void TestMPSGraphManager() {
  const int B = 64, IN = 96, HID = 80, OUT = 48;
  auto x = NewTensor({B, IN}, uniform((size_t)B * IN, 31)).value;
  auto w1 = NewTensor({IN, HID}, uniform((size_t)IN * HID, 32)).value;
  auto w2 = NewTensor({OUT, HID}, uniform((size_t)OUT * HID, 33)).value;  // used transposed
  matrix::MPSGraphManager g;
  g.CreateTensor("x", {B, IN}, "float32");
  g.CreateTensor("w1", {IN, HID}, "float32");
  g.CreateTensor("w2", {OUT, HID}, "float32");
  const std::string h = g.MatMulOp("x", "w1", false, false);
  CHECK(h == "matmul_x_w1");
  const std::string r = g.ActivationOp(h, "ReLU");  // fused into the first GEMM
  CHECK(r == "ReLU_matmul_x_w1");
  const std::string y = g.MatMulOp(r, "w2", false, true);
  auto [c, err] = g.CompileGraph({"x", "w1", "w2"}, {y});
  CHECK_NOERR(err);
  if (!c) return;
  CHECK(g.CompileGraph({"x", "w1", "w2"}, {y}).value == c);  // cached by key
  // float64 reference: relu(x w1) w2^T
  std::vector<double> H = gemm64(x->Data, w1->Data, B, HID, IN);
  std::vector<float> Hf(H.size());
  for (size_t i = 0; i < H.size(); ++i) Hf[i] = (float)std::max(0.0, H[i]);
  std::vector<float> w2t((size_t)HID * OUT);
  for (int o = 0; o < OUT; ++o)
    for (int k = 0; k < HID; ++k) w2t[(size_t)k * OUT + o] = w2->Data[(size_t)o * HID + k];
  for (int rep = 0; rep < 2; ++rep) {  // the second run replays the same HIP graph
    auto [out, e2] = g.Execute(*c, {{"x", x.get()}, {"w1", w1.get()}, {"w2", w2.get()}});
    CHECK_NOERR(e2);
    if (e2) return;
    tensor::TensorPtr Y = out[y];
    CHECK(Y && Y->IsOnGPU() && Y->Shape == (std::vector<int>{B, OUT}));
    CHECK_NOERR(Y->RetrieveCPU());
    CHECK(rel(Y->Data, gemm64(Hf, w2t, B, OUT, HID)) <= 1e-5);
  }
  // fp16 placeholders: sigmoid(f16(a) f16(b)), fp32 accumulation
  matrix::MPSGraphManager g16;
  g16.CreateTensor("a", {B, IN}, "float16");
  g16.CreateTensor("b", {IN, HID}, "float16");
  const std::string s16 = g16.ActivationOp(g16.MatMulOp("a", "b", false, false), "Sigmoid");
  auto c16 = g16.CompileGraph({"a", "b"}, {s16}).value;
  CHECK(c16);
  if (c16) {
    auto o16 = g16.Execute(*c16, {{"a", x.get()}, {"b", w1.get()}}).value;
    tensor::TensorPtr S = o16[s16];
    CHECK(S);
    if (S) {
      CHECK_NOERR(S->RetrieveCPU());
      auto r16 = [](const std::vector<float> &v) {
        std::vector<float> o(v.size());
        for (size_t i = 0; i < v.size(); ++i) o[i] = orc_f16_to_f32(orc_f32_to_f16_rne(v[i]));
        return o;
      };
      std::vector<double> P = gemm64(r16(x->Data), r16(w1->Data), B, HID, IN);
      for (double &v : P) v = orc_act_f64(matrix::Sigmoid, 0.0, v);
      CHECK(rel(S->Data, P) <= 1e-5);
    }
  }
  CHECK_PANICS(g.ActivationOp(h, "Softplus"));
  CHECK_PANICS(g.MatMulOp("x", "x", false, false));
  CHECK_PANICS(g.MatMulOp("x", "nope", false, false));
  CHECK_ERR_HAS(g.CompileGraph({"x"}, {y}).err, "is needed but not an input");
  CHECK_ERR_HAS(g.Execute(*c, {{"x", x.get()}}).err, "missing input w1");
}

void TestMatMul() {
  const int M = 96, K = 130, N = 70;
  auto A = NewTensor({M, K}, uniform((size_t)M * K, 1)).value;
  auto B = NewTensor({K, N}, uniform((size_t)K * N, 2)).value;
  auto [C, err] = matrix::MatMul(*A, *B);
  CHECK_NOERR(err);
  CHECK(C->IsOnGPU());
  CHECK_NOERR(C->RetrieveCPU());
  CHECK(!C->IsOnGPU());
  CHECK(rel(C->Data, gemm64(A->Data, B->Data, M, N, K)) <= 1e-5);
  // 256^3 (config C1)
  auto A2 = NewTensor({256, 256}, uniform(65536, 3)).value;
  auto B2 = NewTensor({256, 256}, uniform(65536, 4)).value;
  auto C2 = matrix::MatMul(*A2, *B2).value;
  CHECK_NOERR(C2->RetrieveCPU());
  CHECK(rel(C2->Data, gemm64(A2->Data, B2->Data, 256, 256, 256)) <= 1e-5);
}

void TestResidencyReuploadsHostWrites() {
  auto A = NewTensor({2, 2}, {1, 2, 3, 4}).value;
  auto I = NewTensor({2, 2}, {1, 0, 0, 1}).value;
  auto C = matrix::MatMul(*A, *I).value;
  CHECK_NOERR(C->RetrieveCPU());
  CHECK(C->Data == std::vector<float>({1, 2, 3, 4}));
  CHECK_NOERR(A->RetrieveCPU());     // host-resident again
  A->Data[0] = 10.0f;                // host write
  auto C2 = matrix::MatMul(*A, *I).value;  // EnsureGPU re-uploads
  CHECK_NOERR(C2->RetrieveCPU());
  CHECK(C2->Data[0] == 10.0f);
}

void TestMemoryStatsTrackTensors() {
  auto before = tensor::GetGlobalMemoryStats();
  {
    auto t = NewTensor({1024}, std::vector<float>(1024, 1.0f)).value;
    CHECK_NOERR(t->EnsureGPU());
    auto mid = tensor::GetGlobalMemoryStats();
    CHECK(mid.numAllocations == before.numAllocations + 1 && mid.currentUsage == before.currentUsage + 4096);
    CHECK(mid.peakUsage >= mid.currentUsage);
  }
  auto after = tensor::GetGlobalMemoryStats();
  CHECK(after.numAllocations == before.numAllocations && after.currentUsage == before.currentUsage);
}

void TestTranspose() {
  auto A = NewTensor({3, 70}, uniform(210, 5)).value;
  auto [T, err] = matrix::Transpose(*A);
  CHECK_NOERR(err);
  CHECK(T->Shape == std::vector<int>({70, 3}));
  CHECK_NOERR(T->RetrieveCPU());
  std::vector<float> ref(210);
  orc_transpose_f32(3, 70, A->Data.data(), ref.data());
  CHECK(T->Data == ref);
}

void TestOptimizedGEMMAndBatch() {
  const int M = 33, K = 17, N = 20, bs = 3;
  auto A = NewTensor({M, K}, uniform((size_t)M * K, 6)).value;
  auto B = NewTensor({K, N}, uniform((size_t)K * N, 7)).value;
  auto [C, err] = matrix::OptimizedGEMM(*A, *B, 2.0f, 0.5f);  // beta scales a fresh zero output
  CHECK_NOERR(err);
  CHECK_NOERR(C->RetrieveCPU());
  auto ref = gemm64(A->Data, B->Data, M, N, K);
  for (double &r : ref) r *= 2.0;
  CHECK(rel(C->Data, ref) <= 1e-5);
  auto A3 = NewTensor({bs, M, K}, uniform((size_t)bs * M * K, 8)).value;
  auto B3 = NewTensor({bs, K, N}, uniform((size_t)bs * K * N, 9)).value;
  auto [C3, e3] = matrix::OptimizedBatchMatMul(*A3, *B3);
  CHECK_NOERR(e3);
  CHECK_NOERR(C3->RetrieveCPU());
  for (int z = 0; z < bs; ++z) {
    std::vector<float> a(A3->Data.begin() + (long)z * M * K, A3->Data.begin() + (long)(z + 1) * M * K);
    std::vector<float> b(B3->Data.begin() + (long)z * K * N, B3->Data.begin() + (long)(z + 1) * K * N);
    std::vector<float> c(C3->Data.begin() + (long)z * M * N, C3->Data.begin() + (long)(z + 1) * M * N);
    CHECK(rel(c, gemm64(a, b, M, N, K)) <= 1e-5);
  }
}

void TestSparseMatMulAndMatVec() {
  const int rows = 300, cols = 200, N = 64;
  std::vector<int32_t> ri, ci;
  std::vector<float> v;
  uint64_t x = 99;
  for (int k = 0; k < 2500; ++k) {
    x = x * 6364136223846793005ULL + 1442695040888963407ULL;
    ri.push_back((int)((x >> 33) % rows));
    ci.push_back((int)((x >> 11) % cols));
    v.push_back((float)((int)((x >> 45) % 1000) - 500) / 256.0f);
  }
  auto S = NewSparseTensorCOO({rows, cols}, ri, ci, v).value;
  auto D = NewTensor({cols, N}, uniform((size_t)cols * N, 10)).value;
  auto [C, err] = matrix::SparseMatMul(*S, *D);  // COO converted to CSR on the way
  CHECK_NOERR(err);
  CHECK(S->GetFormat() == SparseFormat::CSR);
  CHECK_NOERR(C->RetrieveCPU());
  std::vector<float> ref((size_t)rows * N);
  orc_spmm_csr_f32(rows, N, S->RowPtr.data(), S->Indices.data(), S->Data.data(), D->Data.data(), N, ref.data(), N, 1);
  CHECK(C->Data == ref);  // CSR-order fma accumulation, bit for bit
  auto xv = NewTensor({cols}, uniform(cols, 11)).value;
  auto [y, yerr] = matrix::SparseMatVec(*S, *xv);
  CHECK_NOERR(yerr);
  CHECK_NOERR(y->RetrieveCPU());
  std::vector<double> y64(rows);
  orc_spmv_csr_f64(rows, S->RowPtr.data(), S->Indices.data(), S->Data.data(), xv->Data.data(), y64.data());
  CHECK(rel(y->Data, y64) <= 1e-5);
  // dense x dense through SparseMatMul is MatMul
  auto A = NewTensor({4, cols}, uniform((size_t)4 * cols, 12)).value;
  auto [C2, e2] = matrix::SparseMatMul(*A, *D);
  CHECK_NOERR(e2);
  CHECK_NOERR(C2->RetrieveCPU());
  CHECK(rel(C2->Data, gemm64(A->Data, D->Data, 4, N, cols)) <= 1e-5);
  // nnz = 0 gives zeros (the reference panics on &A.Indices[0])
  auto E = NewSparseTensorCOO({5, cols}, {}, {}, {}).value;
  auto [Z, zerr] = matrix::SparseMatMul(*E, *D);
  CHECK_NOERR(zerr);
  CHECK_NOERR(Z->RetrieveCPU());
  for (float z : Z->Data) CHECK(z == 0.0f);
  // a CSC operand is rejected as in the reference (ConvertToCSR from CSC)
  auto Cs = NewSparseTensorCOO({rows, cols}, ri, ci, v).value;
  CHECK_NOERR(Cs->ConvertToCSC());
  CHECK_ERR_HAS(matrix::SparseMatMul(*Cs, *D).err, "failed to convert A to CSR");
}

void TestFusedLinearActivation() {
  const int batch = 40, in = 96, out = 70;
  auto X = NewTensor({batch, in}, uniform((size_t)batch * in, 13)).value;
  auto W = NewTensor({in, out}, uniform((size_t)in * out, 14)).value;
  auto b = NewTensor({out}, uniform(out, 15)).value;
  matrix::FusedLinearActivation f;
  matrix::FusedLinearConfig cfg;
  cfg.Bias = true;  // Activation nil -> ReLU
  auto [Y, err] = f.Forward({X.get(), W.get(), b.get()}, &cfg);
  CHECK_NOERR(err);
  CHECK_NOERR(Y->RetrieveCPU());
  std::vector<double> ref((size_t)batch * out);
  orc_linear_f64(batch, in, out, X->Data.data(), W->Data.data(), 0, b->Data.data(), 0, 0.0, ref.data(), 8);
  CHECK(rel(Y->Data, ref) <= 1e-5);
  cfg.Activation = std::make_shared<matrix::FusedActivationConfig>();
  cfg.Activation->ActivationType = matrix::GELU;
  cfg.Bias = false;  // bias tensor passed but config.Bias false: ignored (fused-operations.go:394-397)
  auto [Y2, e2] = f.Forward({X.get(), W.get(), b.get()}, &cfg);
  CHECK_NOERR(e2);
  CHECK_NOERR(Y2->RetrieveCPU());
  orc_linear_f64(batch, in, out, X->Data.data(), W->Data.data(), 0, nullptr, 7, 0.0, ref.data(), 8);
  CHECK(rel(Y2->Data, ref) <= 1e-5);
  cfg.Activation->ActivationType = matrix::Softmax;  // not an element-wise epilogue
  CHECK_ERR_HAS(f.Forward({X.get(), W.get()}, &cfg).err, "fused linear+activation failed (code -1)");
}

// FusedLinearActivation.Backward (fused-operations.go:467-578) against the float64
// restatement: G = dY * act'(pre) * scale, grad_input = G W^T, grad_weight = X^T G,
// grad_bias = column sums of G (shape [1, out]).
void TestFusedOperationInterface() {
  const int B = 33, IN = 70, OUT = 50;
  auto x = NewTensor({B, IN}, uniform((size_t)B * IN, 21)).value;
  auto w = NewTensor({IN, OUT}, uniform((size_t)IN * OUT, 22)).value;
  auto b = NewTensor({OUT}, uniform(OUT, 23)).value;
  matrix::FusedLinearConfig cfg;
  cfg.Bias = true;
  cfg.Activation = std::make_shared<matrix::FusedActivationConfig>();
  cfg.Activation->ActivationType = matrix::GELU;
  auto op = matrix::GetFusedOperation("linear_activation").first;
  auto y1 = op->Forward({x.get(), w.get(), b.get()}, std::any(&cfg)).value;
  matrix::FusedLinearActivation direct;
  auto y2 = direct.Forward({x.get(), w.get(), b.get()}, &cfg).value;
  CHECK(y1 && y2);
  if (!y1 || !y2) return;
  CHECK_NOERR(y1->RetrieveCPU());
  CHECK_NOERR(y2->RetrieveCPU());
  CHECK(y1->Data == y2->Data);
}

void TestFusedLinearBackward() {
  const int batch = 33, in = 50, out = 70;
  auto X = NewTensor({batch, in}, uniform((size_t)batch * in, 21)).value;
  auto W = NewTensor({in, out}, uniform((size_t)in * out, 22)).value;
  auto pre = NewTensor({batch, out}, uniform((size_t)batch * out, 23, -2.0f, 2.0f)).value;
  auto dY = NewTensor({batch, out}, uniform((size_t)batch * out, 24)).value;
  matrix::FusedLinearActivation f;
  for (int act : {(int)matrix::ReLU, (int)matrix::GELU, (int)matrix::Sigmoid}) {
    matrix::FusedLinearConfig cfg;
    cfg.Bias = true;
    cfg.Dropout = 0.25f;
    cfg.Activation = std::make_shared<matrix::FusedActivationConfig>();
    cfg.Activation->ActivationType = (matrix::ActivationType)act;
    auto [grads, err] = f.Backward(*dY, {X.get(), W.get(), pre.get()}, &cfg);
    CHECK_NOERR(err);
    CHECK(grads.size() == 3);
    if (grads.size() != 3) return;
    std::vector<double> G((size_t)batch * out), dX((size_t)batch * in), dW((size_t)in * out), db(out, 0.0);
    orc_act_backward_f64(act, 0.0, 1.0 / 0.75, dY->Data.data(), pre->Data.data(), (long)G.size(), G.data());
    for (int i = 0; i < batch; ++i)
      for (int k = 0; k < in; ++k) {
        double s = 0;
        for (int o = 0; o < out; ++o) s += G[(size_t)i * out + o] * (double)W->Data[(size_t)k * out + o];
        dX[(size_t)i * in + k] = s;
      }
    for (int k = 0; k < in; ++k)
      for (int o = 0; o < out; ++o) {
        double s = 0;
        for (int i = 0; i < batch; ++i) s += (double)X->Data[(size_t)i * in + k] * G[(size_t)i * out + o];
        dW[(size_t)k * out + o] = s;
      }
    for (int i = 0; i < batch; ++i)
      for (int o = 0; o < out; ++o) db[o] += G[(size_t)i * out + o];
    for (auto &t : grads) CHECK_NOERR(t->RetrieveCPU());
    CHECK(grads[0]->Shape == std::vector<int>({batch, in}));
    CHECK(grads[1]->Shape == std::vector<int>({in, out}));
    CHECK(grads[2]->Shape == std::vector<int>({1, out}));
    CHECK(rel(grads[0]->Data, dX) <= 1e-5);
    CHECK(rel(grads[1]->Data, dW) <= 1e-5);
    CHECK(rel(grads[2]->Data, db) <= 1e-5);
  }
  // nil activation: the gradient passes through; no bias gradient with two saved tensors
  matrix::FusedLinearConfig plain;
  plain.Bias = true;
  auto [g2, e2] = f.Backward(*dY, {X.get(), W.get()}, &plain);
  CHECK_NOERR(e2);
  CHECK(g2.size() == 2);
  // ReLU without the pre-activation is an error
  matrix::FusedLinearConfig relu;
  relu.Activation = std::make_shared<matrix::FusedActivationConfig>();
  CHECK_ERR_HAS(f.Backward(*dY, {X.get(), W.get()}, &relu).err, "pre-activation tensor");
  CHECK_ERR_HAS(f.Backward(*dY, {X.get()}, &relu).err, "insufficient saved tensors");
}

// matmulBackward (gradient.go:601-637): grad_A = dC B^T, grad_B = A^T dC.
void TestMatMulBackward() {
  const int M = 37, K = 45, N = 29;
  auto A = NewTensor({M, K}, uniform((size_t)M * K, 31)).value;
  auto B = NewTensor({K, N}, uniform((size_t)K * N, 32)).value;
  auto dC = NewTensor({M, N}, uniform((size_t)M * N, 33)).value;
  auto [g, err] = matrix::MatMulBackward(*dC, *A, *B);
  CHECK_NOERR(err);
  CHECK(g.size() == 2);
  if (g.size() != 2) return;
  std::vector<double> gA((size_t)M * K), gB((size_t)K * N);
  orc_gemm_f64(0, 1, M, K, N, 1.0, dC->Data.data(), N, B->Data.data(), N, 0.0, gA.data(), K, 8);
  orc_gemm_f64(1, 0, K, N, M, 1.0, A->Data.data(), K, dC->Data.data(), N, 0.0, gB.data(), N, 8);
  for (auto &t : g) CHECK_NOERR(t->RetrieveCPU());
  CHECK(rel(g[0]->Data, gA) <= 1e-5);
  CHECK(rel(g[1]->Data, gB) <= 1e-5);
  CHECK_ERR_HAS(matrix::MatMulBackward(*dC, *B, *A).err, "matmul backward");
}

void TestForwardFloat16() {
  const int M = 64, K = 200, N = 48;
  auto X = NewTensor({M, K}, uniform((size_t)M * K, 16)).value;
  auto W = NewTensor({K, N}, uniform((size_t)K * N, 17, -0.05f, 0.05f)).value;
  auto b = NewTensor({N}, uniform(N, 18, -0.01f, 0.01f)).value;
  auto [mp, merr] = matrix::NewMixedPrecisionTrainer(nullptr);
  CHECK_NOERR(merr);
  auto [Y, err] = mp->ForwardFloat16(*X, *W, b.get());
  CHECK_NOERR(err);
  CHECK_NOERR(Y->RetrieveCPU());
  // reference: host RTZ rounding of X, W and b (mixed-precision.go:192-210), float64 GEMM
  auto Xh = mp->ConvertTensorToFloat16(*X).value, Wh = mp->ConvertTensorToFloat16(*W).value;
  auto bh = mp->ConvertTensorToFloat16(*b).value;
  auto ref = gemm64(Xh->Data, Wh->Data, M, N, K);
  for (int i = 0; i < M; ++i)
    for (int j = 0; j < N; ++j) ref[(size_t)i * N + j] += bh->Data[j];
  CHECK(rel(Y->Data, ref) <= 1e-5);
  auto ref_unrounded = gemm64(X->Data, W->Data, M, N, K);  // unrounded inputs, same bias
  for (int i = 0; i < M; ++i)
    for (int j = 0; j < N; ++j) ref_unrounded[(size_t)i * N + j] += b->Data[j];
  CHECK(rel(Y->Data, ref_unrounded) <= 2e-2);
  // A bias of any other length is added cyclically over the flat output, result[i] +=
  // bias[i % len] (mixed-precision.go:352-354): the same fp32 sums as the product without a
  // bias plus the rounded bias element, bit for bit.
  auto [Y0, err0] = mp->ForwardFloat16(*X, *W, nullptr);
  CHECK_NOERR(err0);
  if (!Y0) return;
  CHECK_NOERR(Y0->RetrieveCPU());
  for (int L : {1, 7, N + 1, 2 * N, M * N}) {
    auto bl = NewTensor({L}, uniform((size_t)L, 19 + L, -0.5f, 0.5f)).value;
    auto blh = mp->ConvertTensorToFloat16(*bl).value;
    auto [Yl, errl] = mp->ForwardFloat16(*X, *W, bl.get());
    CHECK_NOERR(errl);
    if (!Yl) continue;
    CHECK_NOERR(Yl->RetrieveCPU());
    bool same = true;
    for (size_t i = 0; i < Yl->Data.size(); ++i) same = same && Yl->Data[i] == Y0->Data[i] + blh->Data[i % (size_t)L];
    CHECK(same);
  }
  auto empty = NewTensor({0}, std::vector<float>()).value;
  if (empty) CHECK_ERR_HAS(mp->ForwardFloat16(*X, *W, empty.get()).err, "bias is empty");
}

void TestFloat16Chaining() {
  const int M = 70, K = 136, N = 90;
  auto X = NewTensor({M, K}, uniform((size_t)M * K, 41)).value;
  auto W = NewTensor({K, N}, uniform((size_t)K * N, 42, -0.05f, 0.05f)).value;
  auto b = NewTensor({N}, uniform(N, 43, -0.01f, 0.01f)).value;
  auto mp = matrix::NewMixedPrecisionTrainer(nullptr).value;
  auto [W16, werr] = tensor::Float16Tensor::FromTensor(*W);  // the reference's truncation
  CHECK_NOERR(werr);
  if (!W16) return;
  // reusing the converted weights gives the same bits as converting them per call
  auto Y1 = mp->ForwardFloat16(*X, *W, b.get()).value;
  auto Y2 = mp->ForwardFloat16(*X, *W16, b.get()).value;
  CHECK(Y1 && Y2);
  if (!Y1 || !Y2) return;
  CHECK_NOERR(Y1->RetrieveCPU());
  CHECK_NOERR(Y2->RetrieveCPU());
  CHECK(Y1->Data == Y2->Data);
  // widening is exact: the truncated values of Float32ToFloatMP16
  auto W32 = W16->ToFloat32().value;
  CHECK_NOERR(W32->RetrieveCPU());
  bool same = true;
  for (size_t i = 0; i < W->Data.size(); ++i)
    same &= W32->Data[i] == matrix::FloatMP16ToFloat32(matrix::Float32ToFloatMP16(W->Data[i]));
  CHECK(same);
  // a chained fp16 product from round-to-nearest conversions
  auto X16 = tensor::Float16Tensor::FromTensor(*X, false).value;
  auto Wn16 = tensor::Float16Tensor::FromTensor(*W, false).value;
  auto C = matrix::MatMulFloat16(*X16, *Wn16).value;
  CHECK(C && C->IsOnGPU());
  if (!C) return;
  CHECK_NOERR(C->RetrieveCPU());
  auto rne = [](const std::vector<float> &v) {
    std::vector<float> o(v.size());
    for (size_t i = 0; i < v.size(); ++i) o[i] = orc_f16_to_f32(orc_f32_to_f16_rne(v[i]));
    return o;
  };
  CHECK(rel(C->Data, gemm64(rne(X->Data), rne(W->Data), M, N, K)) <= 1e-5);
  CHECK_ERR_HAS(matrix::MatMulFloat16(*W16, *W16).err, "incompatible matrix dimensions");
}

void TestLinearLayer() {
  auto layer = matrix::NewLinearLayer(50, 30, true, 5);
  for (int j = 0; j < 30; ++j) layer->Bias->Data[j] = 0.01f * (float)j;
  auto X = NewTensor({8, 50}, uniform(400, 19)).value;
  auto Y = layer->Forward(X);
  CHECK(Y->Shape == std::vector<int>({8, 30}));
  CHECK_NOERR(Y->RetrieveCPU());
  auto ref = gemm64(X->Data, layer->Weight->Data, 8, 30, 50);
  for (int i = 0; i < 8; ++i)
    for (int j = 0; j < 30; ++j) ref[(size_t)i * 30 + j] += layer->Bias->Data[j];
  CHECK(rel(Y->Data, ref) <= 1e-5);
  auto bad = NewTensor({8, 49}, std::vector<float>(392)).value;
  auto Z = layer->Forward(bad);  // zero output on failure (layers.go:61-67)
  CHECK(Z->Shape == std::vector<int>({8, 30}));
  for (float z : Z->Data) CHECK(z == 0.0f);
}

void TestGPUDenseAndGPUMatMul() {
  const int M = 20, K = 30, N = 10;
  std::vector<double> a((size_t)M * K), b((size_t)K * N);
  for (size_t i = 0; i < a.size(); ++i) a[i] = std::sin(0.37 * (double)i);
  for (size_t i = 0; i < b.size(); ++i) b[i] = std::cos(0.11 * (double)i);
  auto da = mat::NewDense(M, K, a), db = mat::NewDense(K, N, b);
  std::vector<float> af(a.begin(), a.end()), bf(b.begin(), b.end());
  auto ref = gemm64(af, bf, M, N, K);
  auto C = matrix::GPUMatMul(*da, *db);
  std::vector<float> cf(C->RawData().begin(), C->RawData().end());
  CHECK(rel(cf, ref) <= 1e-5);
  // GPUDense.Mul: receiver becomes the device-resident product; At reads it back
  auto g = matrix::NewGPUDense(M, N, std::vector<double>((size_t)M * N, 0.0));
  auto ga = matrix::FromGonum(*da);
  g->Mul(*ga, *db);
  CHECK(g->GetTensor()->IsOnGPU());
  CHECK(std::fabs(g->At(3, 4) - ref[3 * N + 4]) <= 1e-4 * (1.0 + std::fabs(ref[3 * N + 4])));
  CHECK_PANICS(g->At(M, 0));
  g->Set(0, 0, 42.0);
  CHECK(g->At(0, 0) == 42.0);
  // T() is the transpose (a copy-on-write view of the same tensor)
  auto t = ga->T();
  int r, c;
  t->Dims(r, c);
  CHECK(r == K && c == M && t->At(5, 7) == (double)(float)a[7 * K + 5]);
  // Batch
  auto res = matrix::BatchGPUMatMul({{da, db}, {db->T(), da->T()}});
  CHECK(res.size() == 2);
  res[1]->Dims(r, c);
  CHECK(r == N && c == M && std::fabs(res[1]->At(2, 3) - ref[3 * N + 2]) <= 1e-4);
  auto back = g->ToGonum();
  CHECK(back->At(0, 0) == 42.0);
}

// T() views: Mul / GPUMatMul of transposed views run one GEMM with in-place transposes
// (gonum's mat.Transpose semantics; the reference materialises, gonum-compat.go:61-68).
void TestGPUDenseTransposeViews() {
  // Ragged shapes in all four layouts against float64 of the stored operands.
  {
    const int M = 37, K = 53, N = 29;
    for (int ta = 0; ta < 2; ++ta)
      for (int tb = 0; tb < 2; ++tb) {
        const int ar = ta ? K : M, ac = ta ? M : K, br = tb ? N : K, bc = tb ? K : N;
        std::vector<float> af = uniform((size_t)ar * ac, 300 + 2 * ta + tb), bf = uniform((size_t)br * bc, 310 + 2 * ta + tb);
        auto ga = matrix::NewGPUDense(ar, ac, std::vector<double>(af.begin(), af.end()));
        auto gb = matrix::NewGPUDense(br, bc, std::vector<double>(bf.begin(), bf.end()));
        std::shared_ptr<mat::Matrix> opA = ta ? ga->T() : std::shared_ptr<mat::Matrix>(ga);
        std::shared_ptr<mat::Matrix> opB = tb ? gb->T() : std::shared_ptr<mat::Matrix>(gb);
        int r, c;
        opA->Dims(r, c);
        CHECK(r == M && c == K);
        std::vector<double> ref((size_t)M * N);
        orc_gemm_f64(ta, tb, M, N, K, 1.0, af.data(), ac, bf.data(), bc, 0.0, ref.data(), N, 8);
        auto g = matrix::NewGPUDense(M, N, std::vector<double>((size_t)M * N, 0.0));
        g->Mul(*opA, *opB);
        auto got = g->ToGonum();
        std::vector<float> gf(got->RawData().begin(), got->RawData().end());
        CHECK(rel(gf, ref) <= 1e-5);
        auto viaGPUMatMul = matrix::GPUMatMul(*opA, *opB);
        std::vector<float> mf(viaGPUMatMul->RawData().begin(), viaGPUMatMul->RawData().end());
        CHECK(mf == gf);  // same kernel, same operands
        // view semantics: At reads the parent transposed; T() of a view is the parent again
        if (ta) {
          CHECK(opA->At(3, 5) == (double)af[(size_t)5 * ac + 3]);
          auto back = opA->T();
          CHECK(back->At(5, 3) == (double)af[(size_t)5 * ac + 3]);
        }
      }
  }
  // C2 size: 4096^3 with the three transposed layouts, sampled rows against float64 and
  // whole-output column sums against (1^T op(A)) op(B) in float64.
  const int n = 4096;
  std::vector<float> af = uniform((size_t)n * n, 320), bf = uniform((size_t)n * n, 321);
  auto ga = matrix::NewGPUDense(n, n, std::vector<double>(af.begin(), af.end()));
  auto gb = matrix::NewGPUDense(n, n, std::vector<double>(bf.begin(), bf.end()));
  const long rows[6] = {0, 1, 777, 2048, 4000, 4095};
  for (int v = 1; v < 4; ++v) {
    const int ta = v >> 1, tb = v & 1;
    auto g = matrix::NewGPUDense(n, n, std::vector<double>((size_t)n * n, 0.0));
    g->Mul(ta ? *ga->T() : *ga, tb ? *gb->T() : *gb);
    auto C = g->GetTensor();
    CHECK_NOERR(C->RetrieveCPU());
    std::vector<double> ref((size_t)6 * n);
    orc_gemm_f64_rows(ta, tb, n, n, n, af.data(), n, bf.data(), n, rows, 6, ref.data(), n, 8);
    std::vector<float> got((size_t)6 * n);
    for (int i = 0; i < 6; ++i)
      std::copy(C->Data.begin() + rows[i] * n, C->Data.begin() + (rows[i] + 1) * n, got.begin() + (size_t)i * n);
    CHECK(rel(got, ref) <= 1e-5);
    // column sums: s_j = sum_k (sum_i opA[i,k]) opB[k,j]
    std::vector<double> colA(n, 0.0), colref(n, 0.0), colgot(n, 0.0);
    for (int i = 0; i < n; ++i)
      for (int k = 0; k < n; ++k) colA[k] += ta ? af[(size_t)k * n + i] : af[(size_t)i * n + k];
    for (int k = 0; k < n; ++k)
      for (int j = 0; j < n; ++j) colref[j] += colA[k] * (tb ? bf[(size_t)j * n + k] : bf[(size_t)k * n + j]);
    for (int i = 0; i < n; ++i)
      for (int j = 0; j < n; ++j) colgot[j] += C->Data[(size_t)i * n + j];
    double num = 0, den = 0;
    for (int j = 0; j < n; ++j) num += (colgot[j] - colref[j]) * (colgot[j] - colref[j]), den += colref[j] * colref[j];
    CHECK(std::sqrt(num / den) <= 1e-5);
  }
}

// The reference's T() is a separate, materialised matrix (gonum-compat.go:61-68). Here it
// starts as a view of the same tensor, shared copy-on-write: a later Mul into the parent,
// Set on either side, and ReleaseGPU of a device-resident parent leave the other unchanged.
void TestGPUDenseTransposeIsIndependent() {
  const int M = 33, K = 21, N = 17;
  std::vector<float> af = uniform((size_t)M * K, 400), bf = uniform((size_t)K * N, 401);
  std::vector<float> xf = uniform((size_t)M * K, 402), yf = uniform((size_t)K * N, 403);
  auto ga = matrix::NewGPUDense(M, K, std::vector<double>(af.begin(), af.end()));
  auto gb = matrix::NewGPUDense(K, N, std::vector<double>(bf.begin(), bf.end()));
  auto gx = matrix::NewGPUDense(M, K, std::vector<double>(xf.begin(), xf.end()));
  auto gy = matrix::NewGPUDense(K, N, std::vector<double>(yf.begin(), yf.end()));
  std::vector<double> ab((size_t)M * N), xy((size_t)M * N);
  orc_gemm_f64(0, 0, M, N, K, 1.0, af.data(), K, bf.data(), N, 0.0, ab.data(), N, 1);
  orc_gemm_f64(0, 0, M, N, K, 1.0, xf.data(), K, yf.data(), N, 0.0, xy.data(), N, 1);
  auto close = [](double a, double b) { return std::fabs(a - b) <= 1e-5 * (1.0 + std::fabs(b)); };
  auto c = matrix::NewGPUDense(M, N, std::vector<double>((size_t)M * N, 0.0));
  c->Mul(*ga, *gb);  // c holds a device-resident product
  auto t = c->T();   // transpose of the first product
  c->Mul(*gx, *gy);  // the parent gets a new product; t keeps the first one
  bool ok = true;
  for (int i = 0; i < M; ++i)
    for (int j = 0; j < N; ++j) ok = ok && close(t->At(j, i), ab[(size_t)i * N + j]) && close(c->At(i, j), xy[(size_t)i * N + j]);
  CHECK(ok);
  // Set on the view changes only the view, Set on the parent only the parent.
  auto tv = std::dynamic_pointer_cast<matrix::GPUDense>(t);
  CHECK(tv != nullptr);
  auto u = c->T();
  std::dynamic_pointer_cast<matrix::GPUDense>(u)->Set(2, 3, 7.0);
  CHECK(u->At(2, 3) == 7.0 && close(c->At(3, 2), xy[(size_t)3 * N + 2]));
  auto w = c->T();
  c->Set(4, 1, -9.0);
  CHECK(c->At(4, 1) == -9.0 && close(w->At(1, 4), xy[(size_t)4 * N + 1]));
  // ReleaseGPU of a device-resident result keeps its values (the reference's buffer
  // aliases the tensor's data), for the matrix and for a view taken before.
  auto d = matrix::NewGPUDense(M, N, std::vector<double>((size_t)M * N, 0.0));
  d->Mul(*ga, *gb);
  auto dv = d->T();
  CHECK(d->GetTensor()->IsOnGPU());
  d->ReleaseGPU();
  CHECK(!d->GetTensor()->IsOnGPU());
  CHECK(close(d->At(5, 6), ab[(size_t)5 * N + 6]) && close(dv->At(6, 5), ab[(size_t)5 * N + 6]));
  // the same at the tensor level: a GPU result released without RetrieveCPU
  auto [r, err] = matrix::MatMul(*ga->GetTensor(), *gb->GetTensor());
  CHECK_NOERR(err);
  if (r) {
    r->ReleaseGPU();
    CHECK(!r->IsOnGPU() && close(r->Data[(size_t)7 * N + 8], ab[(size_t)7 * N + 8]));
  }
}

// Config C1 (256^3, U[-1,1]) through the gonum-compatible facade on the committed fixture
// (tests/golden/gemm_256.npz, float64 product), unpacked by the Python runner into the
// raw file named by GONNGPU_C1_FIXTURE: A, B (256^2 fp32 each), C (256^2 fp64).
void TestGPUMatMulC1Golden() {
  const char *path = std::getenv("GONNGPU_C1_FIXTURE");
  CHECK(path != nullptr);
  if (!path) return;
  const int n = 256;
  std::vector<float> af((size_t)n * n), bf((size_t)n * n);
  std::vector<double> c64((size_t)n * n);
  FILE *f = std::fopen(path, "rb");
  CHECK(f != nullptr);
  if (!f) return;
  const bool ok = std::fread(af.data(), 4, af.size(), f) == af.size() && std::fread(bf.data(), 4, bf.size(), f) == bf.size() &&
                  std::fread(c64.data(), 8, c64.size(), f) == c64.size();
  std::fclose(f);
  CHECK(ok);
  auto da = mat::NewDense(n, n, std::vector<double>(af.begin(), af.end()));
  auto db = mat::NewDense(n, n, std::vector<double>(bf.begin(), bf.end()));
  auto C = matrix::GPUMatMul(*da, *db);
  std::vector<float> cf(C->RawData().begin(), C->RawData().end());
  CHECK(rel(cf, c64) <= 1e-5);
  auto g = matrix::NewGPUDense(n, n, std::vector<double>((size_t)n * n, 0.0));
  g->Mul(*da, *db);
  auto back = g->ToGonum();
  std::vector<float> gf(back->RawData().begin(), back->RawData().end());
  CHECK(gf == cf);
}

void TestGPUSparseMatMulAndMatVec() {
  auto gs = matrix::NewGPUSparse(4, 3, {0, 1, 3, 3}, {2, 0, 1, 1}, {1.f, 2.f, 3.f, 4.f});  // (3,1) duplicated
  auto d = mat::NewDense(3, 2, {1, 2, 3, 4, 5, 6});
  auto C = matrix::GPUSparseMatMul(*gs, *d);
  // rows: [0,0,1]x -> (5,6); [2,0,0] -> (2,4); 0; [0,7,0] -> (21,28)
  const double ref[8] = {5, 6, 2, 4, 0, 0, 21, 28};
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 2; ++j) CHECK(C->At(i, j) == ref[i * 2 + j]);
  auto y = gs->SparseMatVec({1.0, 10.0, 100.0});
  CHECK(y.size() == 4 && y[0] == 100 && y[1] == 2 && y[2] == 0 && y[3] == 70);
  auto ys = matrix::BatchGPUSparseMatVec({gs, gs}, {{1, 0, 0}, {0, 1, 0}});
  CHECK(ys[0][1] == 2 && ys[1][3] == 7);
  // dense x dense through GPUSparseMatMul, and SparseMul on tensors
  auto dd = matrix::GPUSparseMatMul(*mat::NewDense(1, 3, {1, 1, 1}), *d);
  CHECK(dd->At(0, 0) == 9 && dd->At(0, 1) == 12);
  auto S = gs->GetSparseTensor();
  auto Dt = NewTensor({3, 2}, {1, 2, 3, 4, 5, 6}).value;
  auto C2 = gs->SparseMul(*S, *Dt);
  CHECK(C2->At(3, 1) == 28);
  // sparse x sparse: CSR x CSC merge, duplicates pair up in order ((3,1): 3*3 + 4*4)
  auto G2 = matrix::GPUSparseMatMul(*gs, *gs->T());
  CHECK(G2->At(0, 0) == 1 && G2->At(1, 1) == 4 && G2->At(0, 1) == 0 && G2->At(3, 3) == 25);
}

// A random COO tensor (distinct or duplicate coordinates) from the splitmix generator.
tensor::SparseTensorPtr random_coo(int rows, int cols, int n, uint64_t seed) {
  std::vector<int32_t> ri, ci;
  std::vector<float> v;
  uint64_t x = seed;
  for (int k = 0; k < n; ++k) {
    x = x * 6364136223846793005ULL + 1442695040888963407ULL;
    ri.push_back((int)((x >> 33) % rows));
    ci.push_back((int)((x >> 13) % cols));
    v.push_back((float)((int)((x >> 45) % 1000) - 500) / 128.0f);
  }
  return NewSparseTensorCOO({rows, cols}, ri, ci, v).value;
}

// The remaining sparse-matrix.go entry points against the oracle restatements.
void TestSparseOps() {
  // sparse x sparse (sparse-matrix.go:69-131): A to CSR, B to CSC, bit-exact merge
  auto A = random_coo(60, 80, 500, 7), B = random_coo(80, 50, 400, 8);
  auto [C, err] = matrix::SparseMatMul(*A, *B);
  CHECK_NOERR(err);
  CHECK(A->GetFormat() == SparseFormat::CSR && B->GetFormat() == SparseFormat::CSC);
  CHECK_NOERR(C->RetrieveCPU());
  std::vector<float> ref(60 * 50);
  orc_spgemm_csr_csc_f32(60, 50, A->RowPtr.data(), A->Indices.data(), A->Data.data(), B->ColPtr.data(),
                         B->Indices.data(), B->Data.data(), ref.data(), 50, 1);
  CHECK(C->Data == ref);
  // dense x sparse (:193-250): B to CSC, accumulated over B's column entries in order
  auto X = NewTensor({30, 60}, uniform(30 * 60, 40)).value;
  auto S = random_coo(60, 80, 700, 9);
  auto [D, derr] = matrix::SparseMatMul(*X, *S);
  CHECK_NOERR(derr);
  CHECK_NOERR(D->RetrieveCPU());
  std::vector<float> ref2(30 * 80);
  orc_dense_csc_f32(30, 60, 80, X->Data.data(), 60, S->ColPtr.data(), S->Indices.data(), S->Data.data(), ref2.data(),
                    80, 1);
  CHECK(D->Data == ref2);
  // a CSR operand where CSC is needed is rejected, as ConvertToCSC does (:184-191)
  CHECK_ERR_HAS(matrix::SparseMatMul(*X, *A).err, "can only convert from COO to CSC format");
  // SparseAdd (:252-320)
  auto P = random_coo(40, 50, 300, 10), Q = random_coo(40, 50, 300, 11);
  auto [Sum, aerr] = matrix::SparseAdd(*P, *Q);
  CHECK_NOERR(aerr);
  std::vector<int32_t> ri(600), ci(600);
  std::vector<float> vv(600);
  long n = 0;
  CHECK(orc_sparse_add(40, P->RowPtr.data(), P->Indices.data(), P->Data.data(), Q->RowPtr.data(), Q->Indices.data(),
                       Q->Data.data(), ri.data(), ci.data(), vv.data(), 600, &n) == 0);
  ri.resize(n), ci.resize(n), vv.resize(n);
  CHECK(Sum->GetFormat() == SparseFormat::COO && Sum->NNZ == n);
  CHECK(Sum->RowIndices == ri && Sum->ColIndices == ci && Sum->Values == vv);
  CHECK_ERR_HAS(matrix::SparseAdd(*P, *A).err, "incompatible tensors for addition");
  // SparseScalarMul (:322-364): a scaled clone, the original untouched
  auto [Sc, serr] = matrix::SparseScalarMul(*P, -2.5f);
  CHECK_NOERR(serr);
  CHECK_NOERR(Sc->RetrieveCPU());
  CHECK(Sc->Data.size() == P->Data.size());
  for (size_t k = 0; k < P->Data.size(); ++k) CHECK(Sc->Data[k] == P->Data[k] * -2.5f);
  // SparseToDense (:425-473): later duplicates win
  auto [Pd, pderr] = matrix::SparseToDense(*P);
  CHECK_NOERR(pderr);
  CHECK_NOERR(Pd->RetrieveCPU());
  std::vector<float> dref(40 * 50);
  orc_csr_to_dense(40, 50, P->RowPtr.data(), P->Indices.data(), P->Data.data(), dref.data());
  CHECK(Pd->Data == dref);
  // DenseToSparse (:475-525)
  auto [Xs, xerr] = matrix::DenseToSparse(*X, 0.5f);
  CHECK_NOERR(xerr);
  std::vector<int32_t> r2(1800), c2(1800);
  std::vector<float> v2(1800);
  long n2 = 0;
  CHECK(orc_dense_to_coo(30, 60, X->Data.data(), 0.5f, r2.data(), c2.data(), v2.data(), 1800, &n2) == 0);
  r2.resize(n2), c2.resize(n2), v2.resize(n2);
  CHECK(Xs->RowIndices == r2 && Xs->ColIndices == c2 && Xs->Values == v2);
}

struct Case {
  const char *name;
  std::function<void()> fn;
  bool device;
};

}  // namespace

int main(int argc, char **argv) {
  const bool gpu = argc > 1 && std::strcmp(argv[1], "--gpu") == 0;
  const std::vector<Case> cases = {
      {"TestNewTensorValidates", TestNewTensorValidates, false},
      {"TestSparseCOOValidation", TestSparseCOOValidation, false},
      {"TestConvertToCSRMatchesOracle", TestConvertToCSRMatchesOracle, false},
      {"TestSparseTranspose", TestSparseTranspose, false},
      {"TestFloatMP16MatchesReferenceBits", TestFloatMP16MatchesReferenceBits, false},
      {"TestMixedPrecisionConfigDefaults", TestMixedPrecisionConfigDefaults, false},
      {"TestGonumDense", TestGonumDense, false},
      {"TestGPUSparseAtAndErrors", TestGPUSparseAtAndErrors, false},
      {"TestShapeErrorsBeforeDevice", TestShapeErrorsBeforeDevice, false},
      {"TestFusionRegistry", TestFusionRegistry, false},
      {"TestActivationForward", TestActivationForward, true},
      {"TestMPSGraphManager", TestMPSGraphManager, true},
      {"TestMatMul", TestMatMul, true},
      {"TestResidencyReuploadsHostWrites", TestResidencyReuploadsHostWrites, true},
      {"TestMemoryStatsTrackTensors", TestMemoryStatsTrackTensors, true},
      {"TestTranspose", TestTranspose, true},
      {"TestOptimizedGEMMAndBatch", TestOptimizedGEMMAndBatch, true},
      {"TestSparseMatMulAndMatVec", TestSparseMatMulAndMatVec, true},
      {"TestFusedLinearActivation", TestFusedLinearActivation, true},
      {"TestFusedOperationInterface", TestFusedOperationInterface, true},
      {"TestFusedLinearBackward", TestFusedLinearBackward, true},
      {"TestMatMulBackward", TestMatMulBackward, true},
      {"TestForwardFloat16", TestForwardFloat16, true},
      {"TestFloat16Chaining", TestFloat16Chaining, true},
      {"TestLinearLayer", TestLinearLayer, true},
      {"TestGPUDenseAndGPUMatMul", TestGPUDenseAndGPUMatMul, true},
      {"TestGPUDenseTransposeViews", TestGPUDenseTransposeViews, true},
      {"TestGPUDenseTransposeIsIndependent", TestGPUDenseTransposeIsIndependent, true},
      {"TestGPUMatMulC1Golden", TestGPUMatMulC1Golden, true},
      {"TestGPUSparseMatMulAndMatVec", TestGPUSparseMatMulAndMatVec, true},
      {"TestSparseOps", TestSparseOps, true},
  };
  // Optional test names after the mode select a subset (e.g. for a profiler run).
  auto selected = [&](const char *name) {
    if (argc <= 2) return true;
    for (int i = 2; i < argc; ++i)
      if (std::strcmp(argv[i], name) == 0) return true;
    return false;
  };
  int run = 0;
  for (const Case &c : cases) {
    if ((c.device && !gpu) || !selected(c.name)) continue;
    g_current = c.name;
    const int before = g_failures;
    std::printf("=== RUN %s\n", c.name);
    std::fflush(stdout);
    try {
      c.fn();
    } catch (const std::exception &e) {
      fail(__FILE__, __LINE__, std::string("uncaught exception: ") + e.what());
    }
    std::printf("--- %s %s\n", g_failures == before ? "PASS" : "FAIL", c.name);
    std::fflush(stdout);
    ++run;
  }
  std::printf("%s: %d tests, %d failures\n", g_failures ? "FAIL" : "ok", run, g_failures);
  return g_failures ? 1 : 0;
}
