/*
 * TEST INFRASTRUCTURE — the parity oracle. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library; the product (frame-public_amd/) never links or calls it.
 *
 * A single-threaded C++ restatement of the arithmetic of Frame's reference CPU backend for the compiled-graph
 * forward path. Every function cites the reference file:line it follows. Summation orders, the position of
 * every rounding and the special-value behaviour (NaN, -0.0, padding) are kept identical so that, given the
 * same inputs, the outputs are bit-identical to the reference CPU kernels (pinned by tests/test_oracle_*.py
 * against oracle/_ref, the reference built from its own sources, and against the reference tests' known
 * answers).
 *
 * dtype codes follow frame::DTypeCode: 0 = float32, 2 = float16, 3 = bfloat16. Buffers are host memory,
 * dense row-major. Return value 0 = success, non-zero = invalid arguments.
 */
#ifndef FRAME_ORACLE_CPU_KERNELS_H_
#define FRAME_ORACLE_CPU_KERNELS_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype bridge (reference: include/frame/core/dtype.h:51-131) */
uint16_t oracle_float_to_bf16(float v);
float oracle_bf16_to_float(uint16_t b);
uint16_t oracle_float_to_f16(float v);
float oracle_f16_to_float(uint16_t h);
void oracle_f32_to_bf16_array(const float* in, uint16_t* out, int64_t n);
void oracle_f32_to_f16_array(const float* in, uint16_t* out, int64_t n);

/* matmul (reference: src/backends/cpu/kernels/matmul.cpp:92-129) */
int oracle_matmul(int dtype, const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t k);
/* The same per-element formula evaluated only at (rows[i], cols[i]); out holds `count` values of dtype. */
int oracle_matmul_sample(int dtype, const void* a, const void* b, int64_t m, int64_t n, int64_t k,
                         const int64_t* rows, const int64_t* cols, int64_t count, void* out);

/* conv2d forward (reference: src/backends/cpu/kernels/conv.cpp:174-251).
 * geom = {N, Cin, H, W, Cout, KH, KW, stride_h, stride_w, pad_h, pad_w, groups}; bias may be NULL. */
int oracle_conv2d(int dtype, const void* x, const void* w, const void* bias, void* y, const int64_t* geom);
/* Only the flat output indices idx[i]. */
int oracle_conv2d_sample(int dtype, const void* x, const void* w, const void* bias, const int64_t* geom,
                         const int64_t* idx, int64_t count, void* out);

/* Fused elementwise chain (reference: src/ops/fused_elementwise_utils.cpp:122-206 for segment order and
 * per-segment rounding; sub-op arithmetic: src/backends/cpu/kernels/elementwise.cpp:146-331).
 * op codes: 1 add, 2 mul, 3 relu, 4 square, 5 gelu, 6 relu_grad (binary: x > 0 ? gy : 0), 7 sigmoid, 8 tanh,
 * 9 rsqrt, 10 gelu_grad (binary: gy * gelu'(x)). */
int oracle_ew_program(int dtype, int nseg, const uint8_t* ops, const int8_t* arities, const void* const* ins,
                      int nin, void* out, int64_t numel);

/* softmax over the last axis (reference: src/backends/cpu/kernels/sequence.cpp:114-174) */
int oracle_softmax(int dtype, const void* x, void* y, int64_t rows, int64_t cols);

/* layer_norm over the last axis (reference: src/backends/cpu/kernels/sequence.cpp:182-279) */
int oracle_layer_norm(int dtype, const void* x, const void* gamma, const void* beta, void* y, int64_t rows,
                      int64_t cols, double eps);

/* pooling (reference: src/backends/cpu/kernels/pool.cpp:178-306). mode 0 = max, 1 = avg.
 * geom = {N, C, H, W, KH, KW, stride_h, stride_w, pad_h, pad_w}. Returns 2 when a max window is empty. */
int oracle_pool2d(int dtype, int mode, const void* x, void* y, const int64_t* geom);

/* transpose (reference: src/backends/cpu/kernels/shape.cpp:72-165): out.dims[i] = in.dims[perm[i]] */
int oracle_transpose(int itemsize, const void* x, void* y, int rank, const int64_t* in_dims, const int64_t* perm);
/* slice along axis to [start, stop) (reference: src/backends/cpu/kernels/shape.cpp:275-392) */
int oracle_slice(int itemsize, const void* x, void* y, int rank, const int64_t* in_dims, int64_t axis,
                 int64_t start, int64_t stop);
/* concat of `count` inputs along axis (reference: src/backends/cpu/kernels/shape.cpp:170-270);
 * dims is count x rank, row per input */
int oracle_concat(int itemsize, const void* const* xs, int count, void* y, int rank, const int64_t* dims,
                  int64_t axis);

/* constant materialisation: value[i % nvalues] cast to dtype (reference: src/ops/constant_utils.cpp) */
int oracle_constant(int dtype, const double* values, int64_t nvalues, void* out, int64_t numel);

/* ---- training path ---- */
/* matmul_grad_{lhs,rhs}_internal (reference: src/backends/cpu/kernels/matmul.cpp:187-327).
 * rhs = 0: p = gy [m,n], q = b [k,n], out [m,k]; rhs = 1: p = a [m,k], q = gy [m,n], out [k,n]. */
int oracle_matmul_grad(int dtype, int rhs, const void* p, const void* q, void* out, int64_t m, int64_t n, int64_t k);

/* conv2d_grad_{input,filter}_internal (reference: src/backends/cpu/kernels/conv.cpp:320-452); geom as
 * oracle_conv2d with x's dims. */
int oracle_conv2d_grad_input(int dtype, const void* dy, const void* w, void* dx, const int64_t* geom);
int oracle_conv2d_grad_filter(int dtype, const void* x, const void* dy, void* dw, const int64_t* geom);

/* max (mode 0, x required) / avg (mode 1, x unused) pool gradients (reference: src/backends/cpu/kernels/pool.cpp:
 * 186-206, 358-388, 543-566); geom as oracle_pool2d. Returns 2 when a max window is empty. */
int oracle_pool2d_grad(int dtype, int mode, const void* dy, const void* x, void* dx, const int64_t* geom);

/* sum over the axes flagged in reduced[] and its gradient (reference: src/backends/cpu/kernels/reduction.cpp:
 * 87-116, 215-241, 378-388). */
int oracle_sum(int dtype, const void* x, void* out, int rank, const int64_t* dims, const uint8_t* reduced);
int oracle_sum_grad(int itemsize, const void* gy, void* gx, int rank, const int64_t* dims, const uint8_t* reduced);

/* mse_loss and mse_loss_grad_internal (reference: src/backends/cpu/kernels/loss.cpp:110-147, 230-262). */
int oracle_mse_loss(int dtype, const void* pred, const void* target, void* out, int64_t numel);
int oracle_mse_loss_grad(int dtype, const void* pred, const void* target, const void* gy, void* out, int64_t numel);

#ifdef __cplusplus
}
#endif

#endif
