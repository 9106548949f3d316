// bridge_compat.cpp — Part 3 of include/gonngpu.h: the entry points of the reference's bridge
// header (internal/cgo/metal_bridge.h) that the Go packages gpu/matrix, gpu/optimizer and
// tensor call besides the matmul path, so that those packages compile and link against this
// library unchanged. The element-wise matrix operations and the activation backwards run on
// the device (compat_ops.hip); every other entry reports that this backend does not provide
// it.
#include <cstring>

#include "common.h"

using gn::Buffer;
using gn::set_error;

namespace {

int not_provided(CError *err, const char *name) {
  return set_error(err, -1, "%s: not provided by the go-nngpu MI355X GEMM/SpMM backend", name);
}

const float *fptr(const Buffer *b) { return static_cast<const float *>(b->dptr); }
float *fptr_mut(const Buffer *b) { return static_cast<float *>(b->dptr); }

// The element-wise a (op) b entries (metal_bridge_matrix.m:172-479): shapes first (-2, the
// reference checks them before the buffers), then the buffers (-3).
int binary_entry(int op, GPUPtr aPtr, long aRows, long aCols, GPUPtr bPtr, long bRows, long bCols, GPUPtr cPtr,
                 long cRows, long cCols, const char *what, CError *err) {
  if (aRows != bRows || aCols != bCols || aRows != cRows || aCols != cCols)
    return set_error(err, -2, "Matrices must have the same dimensions for element-wise %s.", what);
  const Buffer *a = gn::as_buffer(aPtr), *b = gn::as_buffer(bPtr), *c = gn::as_buffer(cPtr);
  if (!a || !b || !c) return set_error(err, -3, "Invalid input or output buffer pointers.");
  if (!gn::buffer_fits(a, aRows, aCols, 4) || !gn::buffer_fits(b, aRows, aCols, 4) ||
      !gn::buffer_fits(c, aRows, aCols, 4))
    return set_error(err, -3, "Buffer smaller than the %ld x %ld matrix of element-wise %s.", aRows, aCols, what);
  gn::Context *ctx = gn::context(err);
  if (!ctx) return -1;
  long zero_at = -1;
  if (gn::launch_binary_f32(op, fptr(a), fptr(b), fptr_mut(c), aRows * aCols, op == 3 ? &zero_at : nullptr,
                            ctx->stream, err))
    return -1;
  if (zero_at >= 0) return set_error(err, -4, "Division by zero encountered at element %ld.", zero_at);
  return gn::sync_stream(ctx->stream, err, -1);
}

int scalar_entry(bool mul, GPUPtr inPtr, long rows, long cols, float scalar, GPUPtr outPtr, CError *err) {
  gn::Context *ctx = gn::context(err);
  if (!ctx) return -1;
  const Buffer *in = gn::as_buffer(inPtr), *out = gn::as_buffer(outPtr);
  if (!in || !out) return set_error(err, -1, "Invalid input or output buffer pointers.");
  if (!gn::buffer_fits(in, rows, cols, 4) || !gn::buffer_fits(out, rows, cols, 4))
    return set_error(err, -1, "Buffer smaller than the %ld x %ld matrix of the scalar operation.", rows, cols);
  if (gn::launch_scalar_f32(mul, fptr(in), scalar, fptr_mut(out), rows * cols, ctx->stream, err)) return -1;
  return gn::sync_stream(ctx->stream, err, -1);
}

// The activation backwards (metal_bridge_activation.m): gradIn from the gradient and the
// activation output, over rows x cols floats (rows = 1 except 2-D softmax).
int act_backward_entry(int act, GPUPtr gPtr, GPUPtr yPtr, long rows, long cols, float alpha, GPUPtr ginPtr,
                       const char *name, CError *err) {
  gn::Context *ctx = gn::context(err);
  if (!ctx) return -1;
  const Buffer *g = gn::as_buffer(gPtr), *y = gn::as_buffer(yPtr), *gin = gn::as_buffer(ginPtr);
  if (!g || !y || !gin) return set_error(err, -1, "Invalid buffer pointers for %s backward.", name);
  if (rows < 0 || cols < 0) return set_error(err, -1, "Invalid size for %s backward.", name);
  if (!gn::buffer_fits(g, rows, cols, 4) || !gn::buffer_fits(y, rows, cols, 4) || !gn::buffer_fits(gin, rows, cols, 4))
    return set_error(err, -1, "Buffer smaller than the %ld values of %s backward.", rows * cols, name);
  const int rc = act == 3 ? gn::launch_softmax_backward(fptr(g), fptr(y), fptr_mut(gin), rows, cols, ctx->stream, err)
                          : gn::launch_act_backward_from_output(fptr(g), fptr(y), fptr_mut(gin), rows * cols, act,
                                                                alpha, ctx->stream, err);
  if (rc) return -1;
  return gn::sync_stream(ctx->stream, err, -1);
}

}  // namespace

extern "C" {

// ---------------------------------------------------------------- element-wise matrix ops
int perform_mps_matrix_add(GPUPtr aMatrixPtr, long aRows, long aCols, GPUPtr bMatrixPtr, long bRows, long bCols,
                           GPUPtr resultMatrixPtr, long resultRows, long resultCols, DevicePtr, CError *err) {
  return binary_entry(0, aMatrixPtr, aRows, aCols, bMatrixPtr, bRows, bCols, resultMatrixPtr, resultRows, resultCols,
                      "addition", err);
}
int perform_mps_matrix_subtract(GPUPtr aMatrixPtr, long aRows, long aCols, GPUPtr bMatrixPtr, long bRows, long bCols,
                                GPUPtr resultMatrixPtr, long resultRows, long resultCols, DevicePtr, CError *err) {
  return binary_entry(1, aMatrixPtr, aRows, aCols, bMatrixPtr, bRows, bCols, resultMatrixPtr, resultRows, resultCols,
                      "subtraction", err);
}
int perform_mps_matrix_element_multiply(GPUPtr aMatrixPtr, long aRows, long aCols, GPUPtr bMatrixPtr, long bRows,
                                        long bCols, GPUPtr resultMatrixPtr, long resultRows, long resultCols,
                                        DevicePtr, CError *err) {
  return binary_entry(2, aMatrixPtr, aRows, aCols, bMatrixPtr, bRows, bCols, resultMatrixPtr, resultRows, resultCols,
                      "multiplication", err);
}
int perform_mps_matrix_element_divide(GPUPtr aMatrixPtr, long aRows, long aCols, GPUPtr bMatrixPtr, long bRows,
                                      long bCols, GPUPtr resultMatrixPtr, long resultRows, long resultCols, DevicePtr,
                                      CError *err) {
  return binary_entry(3, aMatrixPtr, aRows, aCols, bMatrixPtr, bRows, bCols, resultMatrixPtr, resultRows, resultCols,
                      "division", err);
}

// The four broadcast patterns of metal_bridge_matrix.m:267-311, tried in the reference's order.
int perform_mps_matrix_add_broadcast(GPUPtr aMatrixPtr, long aRows, long aCols, GPUPtr bMatrixPtr, long bRows,
                                     long bCols, GPUPtr resultMatrixPtr, long resultRows, long resultCols, DevicePtr,
                                     CError *err) {
  const Buffer *a = gn::as_buffer(aMatrixPtr), *b = gn::as_buffer(bMatrixPtr), *c = gn::as_buffer(resultMatrixPtr);
  if (!a || !b || !c) return set_error(err, -3, "Invalid input or output buffer pointers.");
  const long M = resultRows, N = resultCols;
  long sa_r, sa_c, sb_r, sb_c;
  if (aRows == M && aCols == N && bRows == 1 && bCols == N) {  // [M,N] + [1,N]
    sa_r = N, sa_c = 1, sb_r = 0, sb_c = 1;
  } else if (bRows == M && bCols == N && aRows == 1 && aCols == N) {  // [1,N] + [M,N]
    sa_r = 0, sa_c = 1, sb_r = N, sb_c = 1;
  } else if (aRows == M && aCols == N && bRows == M && bCols == 1) {  // [M,N] + [M,1]
    sa_r = N, sa_c = 1, sb_r = 1, sb_c = 0;
  } else if (bRows == M && bCols == N && aRows == M && aCols == 1) {  // [M,1] + [M,N]
    sa_r = 1, sa_c = 0, sb_r = N, sb_c = 1;
  } else {
    return set_error(err, -2, "Unsupported broadcasting pattern: A (%ldx%ld) + B (%ldx%ld) -> Result (%ldx%ld)", aRows,
                     aCols, bRows, bCols, resultRows, resultCols);
  }
  if (!gn::buffer_fits(a, aRows, aCols, 4) || !gn::buffer_fits(b, bRows, bCols, 4) || !gn::buffer_fits(c, M, N, 4))
    return set_error(err, -3, "Buffer smaller than the matrix it describes.");
  gn::Context *ctx = gn::context(err);
  if (!ctx) return -1;
  if (gn::launch_add_broadcast_f32(fptr(a), sa_r, sa_c, fptr(b), sb_r, sb_c, fptr_mut(c), M, N, ctx->stream, err))
    return -1;
  return gn::sync_stream(ctx->stream, err, -1);
}

int perform_mps_matrix_scalar_add(GPUPtr inputMatrixPtr, long rows, long cols, float scalar, GPUPtr resultMatrixPtr,
                                  DevicePtr, CError *err) {
  return scalar_entry(false, inputMatrixPtr, rows, cols, scalar, resultMatrixPtr, err);
}
int perform_mps_matrix_scalar_multiply(GPUPtr inputMatrixPtr, long rows, long cols, float scalar,
                                       GPUPtr resultMatrixPtr, DevicePtr, CError *err) {
  return scalar_entry(true, inputMatrixPtr, rows, cols, scalar, resultMatrixPtr, err);
}

// ---------------------------------------------------------------- activation backward
int perform_activation_relu_backward(GPUPtr gradOutputPtr, GPUPtr activationOutputPtr, long size,
                                     GPUPtr gradInputPtr, DevicePtr, CError *err) {
  return act_backward_entry(0, gradOutputPtr, activationOutputPtr, 1, size, 0.0f, gradInputPtr, "ReLU", err);
}
int perform_activation_sigmoid_backward(GPUPtr gradOutputPtr, GPUPtr activationOutputPtr, long size,
                                        GPUPtr gradInputPtr, DevicePtr, CError *err) {
  return act_backward_entry(1, gradOutputPtr, activationOutputPtr, 1, size, 0.0f, gradInputPtr, "Sigmoid", err);
}
int perform_activation_tanh_backward(GPUPtr gradOutputPtr, GPUPtr activationOutputPtr, long size,
                                     GPUPtr gradInputPtr, DevicePtr, CError *err) {
  return act_backward_entry(2, gradOutputPtr, activationOutputPtr, 1, size, 0.0f, gradInputPtr, "Tanh", err);
}
int perform_activation_softmax_1d_backward(GPUPtr gradOutputPtr, GPUPtr activationOutputPtr, long size,
                                           GPUPtr gradInputPtr, DevicePtr, CError *err) {
  return act_backward_entry(3, gradOutputPtr, activationOutputPtr, 1, size, 0.0f, gradInputPtr, "Softmax 1D", err);
}
int perform_activation_softmax_2d_backward(GPUPtr gradOutputPtr, GPUPtr activationOutputPtr, long batchSize,
                                           long features, GPUPtr gradInputPtr, DevicePtr, CError *err) {
  return act_backward_entry(3, gradOutputPtr, activationOutputPtr, batchSize, features, 0.0f, gradInputPtr,
                            "Softmax 2D", err);
}
int perform_activation_leaky_relu_backward(GPUPtr gradOutputPtr, GPUPtr activationOutputPtr, long size, float alpha,
                                           GPUPtr gradInputPtr, DevicePtr, CError *err) {
  return act_backward_entry(4, gradOutputPtr, activationOutputPtr, 1, size, alpha, gradInputPtr, "Leaky ReLU", err);
}
int perform_activation_elu_backward(GPUPtr gradOutputPtr, GPUPtr activationOutputPtr, long size, float alpha,
                                    GPUPtr gradInputPtr, DevicePtr, CError *err) {
  return act_backward_entry(5, gradOutputPtr, activationOutputPtr, 1, size, alpha, gradInputPtr, "ELU", err);
}
int perform_activation_swish_backward(GPUPtr gradOutputPtr, GPUPtr activationOutputPtr, long size,
                                      GPUPtr gradInputPtr, DevicePtr, CError *err) {
  return act_backward_entry(6, gradOutputPtr, activationOutputPtr, 1, size, 0.0f, gradInputPtr, "Swish", err);
}
int perform_activation_gelu_backward(GPUPtr gradOutputPtr, GPUPtr activationOutputPtr, long size,
                                     GPUPtr gradInputPtr, DevicePtr, CError *err) {
  return act_backward_entry(7, gradOutputPtr, activationOutputPtr, 1, size, 0.0f, gradInputPtr, "GELU", err);
}

// ---------------------------------------------------------------- device memory report
// metal_bridge.h:1817: total and used device memory of the library's device.
void getGPUMemoryUsage(long *totalBytes, long *usedBytes) {
  size_t free_b = 0, total_b = 0;
  if (!gn::context(nullptr) || hipMemGetInfo(&free_b, &total_b) != hipSuccess) free_b = total_b = 0;
  if (totalBytes) *totalBytes = (long)total_b;
  if (usedBytes) *usedBytes = (long)(total_b - free_b);
}

// ---------------------------------------------------------------- not provided
// ---- Dense decompositions (LAPACK in the reference)
int perform_matrix_cholesky_decomposition(GPUPtr, long, long, GPUPtr, DevicePtr, CError *err) {
  return not_provided(err, "perform_matrix_cholesky_decomposition");
}
int perform_matrix_determinant(GPUPtr, long, long, float *, DevicePtr, CError *err) {
  return not_provided(err, "perform_matrix_determinant");
}
int perform_matrix_eigenvalue_decomposition(GPUPtr, long, long, GPUPtr, GPUPtr, DevicePtr, CError *err) {
  return not_provided(err, "perform_matrix_eigenvalue_decomposition");
}
int perform_matrix_inverse(GPUPtr, long, long, GPUPtr, DevicePtr, CError *err) {
  return not_provided(err, "perform_matrix_inverse");
}
int perform_matrix_lu_decomposition(GPUPtr, long, long, GPUPtr, GPUPtr, int *, DevicePtr, CError *err) {
  return not_provided(err, "perform_matrix_lu_decomposition");
}
int perform_matrix_qr_decomposition(GPUPtr, long, long, GPUPtr, GPUPtr, DevicePtr, CError *err) {
  return not_provided(err, "perform_matrix_qr_decomposition");
}
int perform_matrix_svd_decomposition(GPUPtr, long, long, GPUPtr, GPUPtr, GPUPtr, DevicePtr, CError *err) {
  return not_provided(err, "perform_matrix_svd_decomposition");
}

// ---- Losses
int perform_loss_binary_crossentropy_backward(GPUPtr, GPUPtr, long, GPUPtr, DevicePtr, CError *err) {
  return not_provided(err, "perform_loss_binary_crossentropy_backward");
}
int perform_loss_binary_crossentropy_forward(GPUPtr, GPUPtr, long, float *, DevicePtr, CError *err) {
  return not_provided(err, "perform_loss_binary_crossentropy_forward");
}
int perform_loss_categorical_crossentropy_backward(GPUPtr, GPUPtr, long, long, GPUPtr, DevicePtr, CError *err) {
  return not_provided(err, "perform_loss_categorical_crossentropy_backward");
}
int perform_loss_categorical_crossentropy_forward(GPUPtr, GPUPtr, long, long, float *, DevicePtr, CError *err) {
  return not_provided(err, "perform_loss_categorical_crossentropy_forward");
}
int perform_loss_hinge_backward(GPUPtr, GPUPtr, long, GPUPtr, DevicePtr, CError *err) {
  return not_provided(err, "perform_loss_hinge_backward");
}
int perform_loss_hinge_forward(GPUPtr, GPUPtr, long, float *, DevicePtr, CError *err) {
  return not_provided(err, "perform_loss_hinge_forward");
}
int perform_loss_huber_backward(GPUPtr, GPUPtr, long, float, GPUPtr, DevicePtr, CError *err) {
  return not_provided(err, "perform_loss_huber_backward");
}
int perform_loss_huber_forward(GPUPtr, GPUPtr, long, float, float *, DevicePtr, CError *err) {
  return not_provided(err, "perform_loss_huber_forward");
}
int perform_loss_mae_backward(GPUPtr, GPUPtr, long, GPUPtr, DevicePtr, CError *err) {
  return not_provided(err, "perform_loss_mae_backward");
}
int perform_loss_mae_forward(GPUPtr, GPUPtr, long, float *, DevicePtr, CError *err) {
  return not_provided(err, "perform_loss_mae_forward");
}
int perform_loss_mse_backward(GPUPtr, GPUPtr, long, GPUPtr, DevicePtr, CError *err) {
  return not_provided(err, "perform_loss_mse_backward");
}
int perform_loss_mse_forward(GPUPtr, GPUPtr, long, float *, DevicePtr, CError *err) {
  return not_provided(err, "perform_loss_mse_forward");
}
int perform_loss_sparse_categorical_crossentropy_backward(GPUPtr, int *, long, long, GPUPtr, DevicePtr, CError *err) {
  return not_provided(err, "perform_loss_sparse_categorical_crossentropy_backward");
}
int perform_loss_sparse_categorical_crossentropy_forward(GPUPtr, int *, long, long, float *, DevicePtr, CError *err) {
  return not_provided(err, "perform_loss_sparse_categorical_crossentropy_forward");
}

// ---- Apple memory-pool and buffer-placement helpers
int allocate_aligned_gpu_buffer(long, long, GPUPtr *, DevicePtr, CError *err) {
  return not_provided(err, "allocate_aligned_gpu_buffer");
}
int allocate_gpu_memory(long, GPUPtr *, CError *error) { return not_provided(error, "allocate_gpu_memory"); }
int cleanup_memory_pool(CError *error) { return not_provided(error, "cleanup_memory_pool"); }
int coalesced_memory_copy(GPUPtr, GPUPtr, long, long, long, DevicePtr, CError *err) {
  return not_provided(err, "coalesced_memory_copy");
}
int flush_gpu_cache(DevicePtr, CError *err) { return not_provided(err, "flush_gpu_cache"); }
int free_gpu_memory(GPUPtr, CError *error) { return not_provided(error, "free_gpu_memory"); }
int initialize_memory_pool(long, CError *error) { return not_provided(error, "initialize_memory_pool"); }
int prefetch_gpu_data(GPUPtr, long, long, DevicePtr, CError *err) { return not_provided(err, "prefetch_gpu_data"); }
int release_optimized_gpu_buffer(GPUPtr, CError *err) { return not_provided(err, "release_optimized_gpu_buffer"); }

// ---- Convolution, pooling, padding, im2col
int perform_avgpool2d_backward(GPUPtr, long, long, long, long, GPUPtr, long, long, long, long, long, long, long,
                               long, long, long, DevicePtr, CError *err) {
  return not_provided(err, "perform_avgpool2d_backward");
}
int perform_avgpool2d_forward(GPUPtr, long, long, long, long, GPUPtr, long, long, long, long, long, long, long,
                              long, long, long, DevicePtr, CError *err) {
  return not_provided(err, "perform_avgpool2d_forward");
}
int perform_col2im(GPUPtr, GPUPtr, long, long, long, long, long, long, long, long, long, long, long, long,
                   DevicePtr, CError *err) {
  return not_provided(err, "perform_col2im");
}
int perform_conv2d_backward_input(GPUPtr, long, long, long, long, GPUPtr, long, long, long, long, GPUPtr, long,
                                  long, long, long, long, long, long, long, DevicePtr, CError *err) {
  return not_provided(err, "perform_conv2d_backward_input");
}
int perform_conv2d_backward_kernel(GPUPtr, long, long, long, long, GPUPtr, long, long, long, long, GPUPtr, long,
                                   long, long, long, long, long, long, long, DevicePtr, CError *err) {
  return not_provided(err, "perform_conv2d_backward_kernel");
}
int perform_conv2d_forward(GPUPtr, long, long, long, long, GPUPtr, long, long, long, long, GPUPtr, long, long, long,
                           long, long, long, long, long, DevicePtr, CError *err) {
  return not_provided(err, "perform_conv2d_forward");
}
int perform_im2col(GPUPtr, long, long, long, long, GPUPtr, long, long, long, long, long, long, long, long,
                   DevicePtr, CError *err) {
  return not_provided(err, "perform_im2col");
}
int perform_maxpool2d_backward(GPUPtr, long, long, long, long, GPUPtr, GPUPtr, long, long, long, long, long, long,
                               long, long, long, long, DevicePtr, CError *err) {
  return not_provided(err, "perform_maxpool2d_backward");
}
int perform_maxpool2d_forward(GPUPtr, long, long, long, long, GPUPtr, long, long, long, long, GPUPtr, long, long,
                              long, long, long, long, DevicePtr, CError *err) {
  return not_provided(err, "perform_maxpool2d_forward");
}
int perform_pad2d(GPUPtr, long, long, long, long, GPUPtr, long, long, long, long, long, long, long, long, float,
                  DevicePtr, CError *err) {
  return not_provided(err, "perform_pad2d");
}
int perform_unpad2d(GPUPtr, long, long, long, long, GPUPtr, long, long, long, long, long, long, long, long,
                    DevicePtr, CError *err) {
  return not_provided(err, "perform_unpad2d");
}

// ---- Normalisation
int perform_batch_mean(GPUPtr, long, long, GPUPtr, DevicePtr, CError *err) {
  return not_provided(err, "perform_batch_mean");
}
int perform_batch_norm_backward_input(GPUPtr, long, long, GPUPtr, GPUPtr, GPUPtr, GPUPtr, float, GPUPtr, DevicePtr,
                                      CError *err) {
  return not_provided(err, "perform_batch_norm_backward_input");
}
int perform_batch_norm_backward_params(GPUPtr, long, long, GPUPtr, GPUPtr, GPUPtr, float, GPUPtr, GPUPtr, DevicePtr,
                                       CError *err) {
  return not_provided(err, "perform_batch_norm_backward_params");
}
int perform_batch_norm_forward(GPUPtr, long, long, GPUPtr, GPUPtr, GPUPtr, GPUPtr, float, GPUPtr, DevicePtr,
                               CError *err) {
  return not_provided(err, "perform_batch_norm_forward");
}
int perform_batch_variance(GPUPtr, GPUPtr, long, long, GPUPtr, DevicePtr, CError *err) {
  return not_provided(err, "perform_batch_variance");
}
int perform_group_norm_forward(GPUPtr, long, long, long, long, long, GPUPtr, GPUPtr, float, GPUPtr, DevicePtr,
                               CError *err) {
  return not_provided(err, "perform_group_norm_forward");
}
int perform_instance_norm_forward(GPUPtr, long, long, long, long, GPUPtr, GPUPtr, float, GPUPtr, DevicePtr,
                                  CError *err) {
  return not_provided(err, "perform_instance_norm_forward");
}
int perform_layer_norm_backward(GPUPtr, long, long, GPUPtr, GPUPtr, GPUPtr, GPUPtr, float, GPUPtr, GPUPtr, GPUPtr,
                                DevicePtr, CError *err) {
  return not_provided(err, "perform_layer_norm_backward");
}
int perform_layer_norm_forward(GPUPtr, long, long, GPUPtr, GPUPtr, float, GPUPtr, GPUPtr, GPUPtr, DevicePtr,
                               CError *err) {
  return not_provided(err, "perform_layer_norm_forward");
}
int perform_update_running_stats(GPUPtr, GPUPtr, GPUPtr, GPUPtr, float, long, DevicePtr, CError *err) {
  return not_provided(err, "perform_update_running_stats");
}

// ---- Fused operations other than the linear layer
int perform_fused_attention(GPUPtr, GPUPtr, GPUPtr, long, long, long, int, float, float, bool, GPUPtr, DevicePtr,
                            CError *error) {
  return not_provided(error, "perform_fused_attention");
}
int perform_fused_conv_bn_relu(GPUPtr, long, long, long, long, GPUPtr, long, long, long, GPUPtr, GPUPtr, GPUPtr,
                               long, long, long, long, float, bool, GPUPtr, long, long, DevicePtr, CError *error) {
  return not_provided(error, "perform_fused_conv_bn_relu");
}
int perform_fused_gelu_dropout(GPUPtr, long, float, unsigned int, GPUPtr, DevicePtr, CError *error) {
  return not_provided(error, "perform_fused_gelu_dropout");
}
int perform_fused_layer_norm_linear(GPUPtr, long, long, long, GPUPtr, GPUPtr, float, GPUPtr, long, GPUPtr, GPUPtr,
                                    DevicePtr, CError *error) {
  return not_provided(error, "perform_fused_layer_norm_linear");
}
int perform_fused_residual_block(GPUPtr, long, long, long, long, GPUPtr, GPUPtr, GPUPtr, GPUPtr, GPUPtr, GPUPtr,
                                 float, GPUPtr, DevicePtr, CError *error) {
  return not_provided(error, "perform_fused_residual_block");
}

// ---- Embedded-MSL kernels other than the GEMMs
int perform_conv1x1_optimized(GPUPtr, GPUPtr, GPUPtr, long, long, long, long, long, DevicePtr, CError *err) {
  return not_provided(err, "perform_conv1x1_optimized");
}
int perform_depthwise_conv_optimized(GPUPtr, GPUPtr, GPUPtr, long, long, long, long, long, long, long, long, long,
                                     long, DevicePtr, CError *err) {
  return not_provided(err, "perform_depthwise_conv_optimized");
}
int perform_elementwise_binary_op_optimized(GPUPtr, GPUPtr, GPUPtr, int, long, long, long, DevicePtr, CError *err) {
  return not_provided(err, "perform_elementwise_binary_op_optimized");
}
int perform_layer_norm_optimized(GPUPtr, GPUPtr, GPUPtr, GPUPtr, GPUPtr, GPUPtr, long, long, float, DevicePtr,
                                 CError *err) {
  return not_provided(err, "perform_layer_norm_optimized");
}
int perform_reduce_optimized(GPUPtr, GPUPtr, long, int, DevicePtr, CError *err) {
  return not_provided(err, "perform_reduce_optimized");
}
int perform_softmax_optimized(GPUPtr, GPUPtr, long, long, DevicePtr, CError *err) {
  return not_provided(err, "perform_softmax_optimized");
}

// ---- Gradient utilities
int perform_dropout_backward(GPUPtr, GPUPtr, long, float, GPUPtr, DevicePtr, CError *error) {
  return not_provided(error, "perform_dropout_backward");
}
int perform_dropout_forward(GPUPtr, long, float, unsigned int, GPUPtr, GPUPtr, DevicePtr, CError *error) {
  return not_provided(error, "perform_dropout_forward");
}
int perform_gradient_accumulate(GPUPtr, GPUPtr, long, DevicePtr, CError *error) {
  return not_provided(error, "perform_gradient_accumulate");
}
int perform_sum_along_axis(GPUPtr, int, long, long *, GPUPtr, long, long *, DevicePtr, CError *error) {
  return not_provided(error, "perform_sum_along_axis");
}
int perform_tensor_fill(GPUPtr, long, float, DevicePtr, CError *error) {
  return not_provided(error, "perform_tensor_fill");
}
int perform_tensor_sum_squares(GPUPtr, long, float *, DevicePtr, CError *error) {
  return not_provided(error, "perform_tensor_sum_squares");
}

// ---- Optimizer steps, clipping, learning-rate schedules (package gpu/optimizer)
int perform_adam_step(GPUPtr, GPUPtr, long, float, float, float, float, float, GPUPtr, GPUPtr, long, DevicePtr,
                      CError *err) {
  return not_provided(err, "perform_adam_step");
}
int perform_adamw_step(GPUPtr, GPUPtr, long, float, float, float, float, float, GPUPtr, GPUPtr, long, DevicePtr,
                       CError *err) {
  return not_provided(err, "perform_adamw_step");
}
int perform_global_gradient_clip(GPUPtr *, long *, long, float, float *, DevicePtr, CError *err) {
  return not_provided(err, "perform_global_gradient_clip");
}
int perform_global_gradient_norm(GPUPtr *, long *, long, float *, DevicePtr, CError *err) {
  return not_provided(err, "perform_global_gradient_norm");
}
int perform_gradient_clip_by_value(GPUPtr, long, float, float, DevicePtr, CError *err) {
  return not_provided(err, "perform_gradient_clip_by_value");
}
int perform_lr_cosine_annealing(float *, float, float, long, long, CError *err) {
  return not_provided(err, "perform_lr_cosine_annealing");
}
int perform_lr_exponential_decay(float *, float, float, long, long, CError *err) {
  return not_provided(err, "perform_lr_exponential_decay");
}
int perform_lr_polynomial_decay(float *, float, float, long, long, float, CError *err) {
  return not_provided(err, "perform_lr_polynomial_decay");
}
int perform_lr_step_decay(float *, float, float, long, long, CError *err) {
  return not_provided(err, "perform_lr_step_decay");
}
int perform_lr_warmup(float *, float, long, long, int, CError *err) {
  return not_provided(err, "perform_lr_warmup");
}
int perform_rmsprop_step(GPUPtr, GPUPtr, long, float, float, float, float, float, GPUPtr, GPUPtr, DevicePtr,
                         CError *err) {
  return not_provided(err, "perform_rmsprop_step");
}
int perform_sgd_step(GPUPtr, GPUPtr, long, float, float, GPUPtr, float, DevicePtr, CError *err) {
  return not_provided(err, "perform_sgd_step");
}

// ---- Command queues, events, shared / mapped memory, counters, MPSGraph convolution
void *allocateSharedMemory(long) { return nullptr; }
void *createCommandQueue(void *) { return nullptr; }
void *createConv2DNode(void *, void *, void *, long, long, long, long) { return nullptr; }
void *createGPUBufferFromSharedMemory(void *, void *, long) { return nullptr; }
void *createMetalEvent(void *) { return nullptr; }
void getGPUCounters(GPUCounters *counters) {
  if (counters) *counters = GPUCounters{0.0f, 0.0f, 0.0f};
}
float getGPUPowerUsage(void) { return 0.0f; }
float getGPUTemperature(void) { return 0.0f; }
void makeBufferGPUResident(void *) {}
void *memoryMapFile(const char *, long *, CError *error) {
  not_provided(error, "memoryMapFile");
  return nullptr;
}
void synchronizeCommandQueue(void *) {}
void unmapMemory(void *, long) {}
}  // extern "C"
