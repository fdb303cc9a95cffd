/*
 * frame_hip_abi.h — the C ABI of the MI355X (gfx950) kernel library `libframe_hip_kernels.so`.
 *
 * This is the thin boundary between Frame's C++20 host side (the `hip` backend plugin: HipBackend,
 * HipStream, HipEvent, HipAllocator, HipExecutable and its KernelFn wrappers) and hand-written HIP
 * code. No C++ type crosses it: only plain pointers, sizes, enums and POD structs.
 *
 * Conventions
 *  - Every function returns fh_status. On failure a thread-local message is available from
 *    fh_last_error(). Codes equal frame::ErrorCode ordinals (reference: include/frame/core/status.h:18-27).
 *  - Device pointers are caller-owned. Kernel entry points only enqueue work on `stream`
 *    (NULL = the device's null stream); they never allocate, never free and never synchronize.
 *  - Argument validation (shapes, alignment, dtype) happens on the host before any launch and
 *    returns FH_INVALID_ARGUMENT / FH_UNIMPLEMENTED synchronously.
 *  - All floating-point arithmetic is fp32; 16-bit results are rounded once to nearest-even with the
 *    reference's quiet-NaN rule (reference: include/frame/core/dtype.h:51-131).
 *  - Tensors are dense row-major (reference: include/frame/core/tensor.h:64-66).
 */
#ifndef FRAME_HIP_ABI_H_
#define FRAME_HIP_ABI_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FH_ABI_VERSION 1

typedef enum fh_status {
  FH_OK = 0,
  FH_INVALID_ARGUMENT = 1,
  FH_NOT_FOUND = 2,
  FH_UNIMPLEMENTED = 4,
  FH_OUT_OF_MEMORY = 5,
  FH_INTERNAL = 6,
  FH_DEVICE_ERROR = 7
} fh_status;

/* Equal to frame::DTypeCode ordinals (reference: include/frame/core/dtype.h:17-29). */
typedef enum fh_dtype { FH_F32 = 0, FH_F16 = 2, FH_BF16 = 3 } fh_dtype;

/* Elementwise sub-op codes understood by fh_ew_program and the GEMM/conv epilogues.
 * add/mul/relu/square are the reference's fusable ops (reference: src/ops/schemas/elementwise.cpp:667-707);
 * gelu is this build's addition (exact erf form). */
typedef enum fh_ew_op {
  FH_EW_ADD = 1,
  FH_EW_MUL = 2,
  FH_EW_RELU = 3,
  FH_EW_SQUARE = 4,
  FH_EW_GELU = 5,
  /* relu_grad_internal(x, gy): gy where x > 0, else 0 (reference: src/backends/cpu/kernels/elementwise.cpp:407-414);
   * binary, the running value is x and the next input gy */
  FH_EW_RELU_GRAD = 6,
  /* unary, the reference's formulas (src/backends/cpu/kernels/elementwise.cpp:342-405) */
  FH_EW_SIGMOID = 7,
  FH_EW_TANH = 8,
  FH_EW_RSQRT = 9,
  /* gelu_grad_internal(x, gy) = gy * (Phi(x) + x phi(x)): binary like FH_EW_RELU_GRAD; no reference counterpart */
  FH_EW_GELU_GRAD = 10,
  /* relu_grad_internal with its operands the other way round: the running value where the next input is > 0, else
   * 0 (so a program can mask a sum it has just formed: add then mask = relu_grad(x, a + b)); no reference counterpart */
  FH_EW_RELU_MASK = 11
} fh_ew_op;

#define FH_MAX_SEGMENTS 8
#define FH_MAX_EW_INPUTS 9

/* memcpy directions */
typedef enum fh_copy_kind { FH_H2H = 0, FH_H2D = 1, FH_D2H = 2, FH_D2D = 3 } fh_copy_kind;

/* ---------------------------------------------------------------------------------------------
 * Diagnostics
 * ------------------------------------------------------------------------------------------- */
const char* fh_last_error(void);
int32_t fh_abi_version(void);

/* ---------------------------------------------------------------------------------------------
 * Runtime shims behind the HAL objects.
 * Replace: cuda_backend.cpp:42-163 (device count, cudaMalloc/cudaFree, streams, events, cudaMemcpy[Async]),
 *          cuda_allocator.cpp:26-66, cuda_backend.cpp:118-128 (event), cuda_backend.cpp:185-204 (copy).
 * ------------------------------------------------------------------------------------------- */
fh_status fh_device_count(int32_t* count);
fh_status fh_set_device(int32_t device);
fh_status fh_malloc(void** ptr, size_t bytes, int32_t device);
fh_status fh_free(void* ptr);
fh_status fh_host_alloc(void** ptr, size_t bytes); /* pinned host memory */
fh_status fh_host_free(void* ptr);
/* stream == NULL: synchronous copy. Otherwise enqueued on `stream`. */
fh_status fh_memcpy(void* dst, const void* src, size_t bytes, int32_t kind, void* stream);
fh_status fh_stream_create(void** stream, int32_t device);
fh_status fh_stream_destroy(void* stream);
fh_status fh_stream_synchronize(void* stream);
fh_status fh_device_synchronize(void);
/* *capturing = 1 while `stream` is being captured into a graph (hipStreamIsCapturing), else 0. For the allocator,
 * which records no fence event on a capturing stream. No counterpart in the reference. */
fh_status fh_stream_capturing(void* stream, int32_t* capturing);
/* Replay of a captured step sequence (hipStreamBeginCapture / EndCapture / hipGraphInstantiate / hipGraphLaunch).
 * end_capture with keep = 0 discards the capture (after a failure inside it). No counterpart in the reference,
 * whose executables launch every step each run (src/backends/cuda/cuda_executable.cpp:55-95). */
fh_status fh_graph_begin_capture(void* stream);
fh_status fh_graph_end_capture(void* stream, int32_t keep, void** exec);
fh_status fh_graph_launch(void* exec, void* stream);
fh_status fh_graph_destroy(void* exec);
fh_status fh_event_create(void** event, int32_t device);
fh_status fh_event_destroy(void* event);
fh_status fh_event_record(void* event, void* stream);
fh_status fh_stream_wait_event(void* stream, void* event);
fh_status fh_event_query(void* event, int32_t* done);
fh_status fh_event_synchronize(void* event);
fh_status fh_event_elapsed_ms(void* start, void* stop, float* ms);

/* ---------------------------------------------------------------------------------------------
 * Kernels
 * ------------------------------------------------------------------------------------------- */

/* Elementwise epilogue applied to a contraction's rounded output before the single store.
 * Segment i consumes the previous value as its first operand and, for binary ops, the next
 * external operand from `ins` (each a dense tensor of the output's shape and dtype).
 * When round_between != 0 each segment's result is rounded to the output dtype before the next
 * segment reads it, which is what Frame's unfused graph computes (reference:
 * src/ops/fused_elementwise_utils.cpp:122-206). */
typedef struct fh_epilogue {
  int32_t nseg; /* 0 = plain store */
  int32_t round_between;
  uint8_t ops[FH_MAX_SEGMENTS];
  const void* ins[FH_MAX_SEGMENTS];
} fh_epilogue;

/* C[M,N] = A[M,K] · B[K,N] (row-major, dtype in = out, fp32 accumulate), then the epilogue.
 * Replaces the cuBLASLt call in matmul_cuda_kernel (reference: src/backends/cuda/kernels/matmul.cpp:90-276)
 * and the CPU semantics of matmul_compute (reference: src/backends/cpu/kernels/matmul.cpp:92-185). */
fh_status fh_gemm(int32_t dtype, const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                  const fh_epilogue* epilogue, void* stream);

/* fh_gemm with flags. FH_GEMM_ANY_ORDER: the sum over k may be taken in any order (the host passes it at
 * opt_level >= 1, where results are checked within tolerance rather than bit for bit); small problems then run
 * a split-k kernel instead of the sequential-order one. No reference counterpart beyond fh_gemm's. */
#define FH_GEMM_ANY_ORDER 1
/* FH_GEMM_ROW_SOFTMAX (with FH_GEMM_ANY_ORDER, N <= 16): every output row, after the epilogue and its rounding,
 * goes through softmax in the same launch (HipBackend::compile fuses a softmax that reads such a GEMM, e.g. C1's
 * classifier layer; the reference runs softmax as its own op, reference: src/backends/cpu/kernels/sequence.cpp:111-160). */
#define FH_GEMM_ROW_SOFTMAX 2
fh_status fh_gemm_ex(int32_t dtype, const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                     const fh_epilogue* epilogue, int32_t flags, void* stream);

/* `groups` GEMMs sharing A[M,K] and one shape, in one launch: C_g[M,N] = A · B_g[K,N], then epilogues[g]
 * (every group the same program, its own operands). Used where HipBackend::compile merges the Q/K/V
 * projections of an attention block, which read the same normalised input (the reference runs three
 * Linear layers, reference: src/nn/layers.cpp:1014-1080). */
#define FH_GEMM_MAX_GROUPS 4
fh_status fh_gemm_grouped(int32_t dtype, const void* A, int32_t groups, const void* const* B, void* const* C,
                          int64_t M, int64_t N, int64_t K, const fh_epilogue* epilogues, int32_t flags,
                          void* stream);

/* Batched GEMM over `batch` independent problems with element strides between problems.
 * Used by the fused attention lowering of per-(batch, head) matmuls (no reference counterpart in one
 * call: the reference launches one matmul per (batch, head), reference: src/nn/layers.cpp:1014-1080). */
fh_status fh_gemm_batched(int32_t dtype, const void* A, const void* B, void* C, int64_t M, int64_t N,
                          int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int64_t stride_a,
                          int64_t stride_b, int64_t stride_c, int64_t batch, void* stream);

/* Conv2d forward, NCHW, optional [Cout] bias added inside the fp32 accumulator, then the epilogue
 * (e.g. ReLU). geom = {N, Cin, H, W, Cout, KH, KW, stride_h, stride_w, pad_h, pad_w, groups}.
 * Replaces cuDNN conv + cudnnAddTensor (reference: src/backends/cuda/kernels/conv.cpp:385-520) with the
 * CPU semantics of conv2d_forward_compute (reference: src/backends/cpu/kernels/conv.cpp:223-314). */
fh_status fh_conv2d_fwd(int32_t dtype, const void* x, const void* w, const void* bias, void* y,
                        const int64_t geom[12], const fh_epilogue* epilogue, void* stream);

/* Conv2d forward as an implicit GEMM on MFMA over channels-last operands: x_nhwc [N,H,W,Cin],
 * w_khwc [Cout,KH,KW,Cin], bias [Cout] or NULL; y is written NCHW [N,Cout,Ho,Wo]. Same semantics and geom as
 * fh_conv2d_fwd (bias inside the fp32 accumulator, one rounding, then the epilogue). The operands come from
 * fh_transpose_batched; HipBackend::compile inserts those steps. Replaces the same cuDNN call
 * (reference: src/backends/cuda/kernels/conv.cpp:385-520) for the geometries fh_conv2d_nhwc_supported accepts. */
fh_status fh_conv2d_nhwc_fwd(int32_t dtype, const void* x_nhwc, const void* w_khwc, const void* bias, void* y,
                             const int64_t geom[12], const fh_epilogue* epilogue, void* stream);

/* fh_conv2d_nhwc_fwd with flags: FH_CONV_OUT_NHWC writes y channels-last, [N,Ho,Wo,Cout], and reads the
 * epilogue's binary operands in that layout too, so a conv can feed the next one without a layout step.
 * HipBackend::compile uses it for activations whose every consumer takes channels-last data. No counterpart in
 * the reference (NCHW throughout, reference: src/backends/cuda/kernels/conv.cpp:385-520). */
#define FH_CONV_OUT_NHWC 1
/* FH_CONV_IMPLICIT_GEMM selects the implicit-GEMM kernel (one im2col row per pixel and tap per stage) even where the
 * resident-patch kernel for 3x3 stride-1 convolutions would run; both compute the same sums, so tests use it to
 * cover both kernels on one geometry. */
#define FH_CONV_IMPLICIT_GEMM 2
/* FH_CONV_IN_NCHW: x is NCHW [N][Cin][H][W] instead of channels-last (the filter stays [Cout][KH][KW][Cin]); the
 * resident-patch kernel transposes it on the way into LDS, so a graph-input activation needs no channels-last
 * copy. Only where fh_conv2d_nchw_in_supported says so. */
#define FH_CONV_IN_NCHW 4
/* FH_CONV_W_OIHW (with FH_CONV_IN_NCHW and NCHW output): the filter is [Cout][Cin][KH][KW], the layout Frame's
 * conv2d takes it in (reference: src/backends/cpu/kernels/conv.cpp:223-314, filter index ((co*Cin + ci)*KH + kh)*KW
 * + kw), so a graph-input filter needs no transposed copy either: the band kernel transposes it on its way into
 * LDS. Only where fh_conv2d_w_oihw_supported says so. */
#define FH_CONV_W_OIHW 8
fh_status fh_conv2d_nhwc_fwd_ex(int32_t dtype, const void* x_nhwc, const void* w_khwc, const void* bias, void* y,
                                const int64_t geom[12], const fh_epilogue* epilogue, int32_t flags, void* stream);

/* Split-K form of fh_conv2d_nhwc_fwd_ex, for convolutions with few output tiles and a long reduction (ResNet's
 * 7x7x512 layers at batch 64: 100 tiles of 128 x 128 for 256 CUs, K = 4608): each tile's K range is cut into
 * `splits` consecutive ranges of k stages, one workgroup each, whose fp32 sums go to `workspace`
 * ([splits][N*Ho*Wo][Cout] floats); a second launch sums them in split order, adds the bias, rounds once and runs
 * the epilogue (same semantics as fh_conv2d_fwd; the fp32 sum is associated differently, hence not bit-identical
 * to the unsplit kernels). bf16/f16, flags == FH_CONV_OUT_NHWC, Cin % 32 == 0, Cout % 128 == 0; the workspace,
 * bias, y and epilogue operands 16-byte aligned.
 * fh_conv2d_nhwc_split_workspace: with *splits <= 0, the planned count (0 where the unsplit kernels are used:
 * Cout <= 256, fewer than 128 k stages, too many tiles to split in two) is written to *splits; with *splits > 0 that
 * count is used (reduced so no split is empty, written back). Returns the workspace bytes (0: no split, the call
 * runs fh_conv2d_nhwc_fwd_ex), or -1 where split K does not apply. fh_conv2d_nhwc_fwd_split takes the same
 * `splits` argument. No counterpart in the reference (cuDNN picks its own algorithm and workspace:
 * src/backends/cuda/kernels/conv.cpp:385-520). */
int64_t fh_conv2d_nhwc_split_workspace(int32_t dtype, const int64_t geom[12], int32_t flags, int32_t* splits);
fh_status fh_conv2d_nhwc_fwd_split(int32_t dtype, const void* x_nhwc, const void* w_khwc, const void* bias, void* y,
                                   const int64_t geom[12], const fh_epilogue* epilogue, int32_t flags, int32_t splits,
                                   void* workspace, int64_t workspace_bytes, void* stream);

/* 1 if fh_conv2d_nhwc_fwd accepts dtype and geom (bf16/f16, groups 1, Cin % 32 == 0 or Cin == 8, 32-bit
 * offsets), else 0. Host-only query used at graph compile time; no counterpart in the reference.
 * With Cin == 8 the operands are in the C8 layout: x from fh_conv_pack_input_c8 and w from
 * fh_conv_pack_filter_c8 ([Cout][fh_conv_c8_filter_k(KH, KW)]). */
int32_t fh_conv2d_nhwc_supported(int32_t dtype, const int64_t geom[12]);

/* 1 if fh_conv2d_nhwc_fwd_ex takes dtype and geom with FH_CONV_IN_NCHW (bf16/f16, 3x3, stride 1, padding 1,
 * groups 1, Cin % 32 == 0, W % 8 == 0, a resident patch of at most 30 KB), else 0. Host-only query. */
int32_t fh_conv2d_nchw_in_supported(int32_t dtype, const int64_t geom[12]);

/* 1 if fh_conv2d_nhwc_fwd_ex takes dtype, geom and the epilogue program (nseg and ops of `epilogue`; NULL for
 * none) with FH_CONV_IN_NCHW | FH_CONV_W_OIHW, given a 16-byte aligned output and epilogue operands: bf16, 3x3,
 * stride 1, padding 1, Cin 64, Cout <= 64, W % 8 == 0, no epilogue, relu or add;relu, and a geometry whose bands of
 * whole output rows spread over the CUs more evenly than 256-pixel tiles; else 0. Host-only query (it launches
 * nothing, but reads the current device's CU count once per process, 256 when no device is visible, so the answer
 * depends on the device); no counterpart in the reference. */
int32_t fh_conv2d_w_oihw_supported(int32_t dtype, const int64_t geom[12], const fh_epilogue* epilogue);

/* A network stem in one launch: y = max_pool2d(act(conv2d(x, w) + bias)), NCHW x [N][Cin][H][W], w [64][Cin][7][7],
 * bias [64] or NULL, y [N][64][PH][PW]; the convolution 7x7, stride 2, padding 3 (geom as fh_conv2d_fwd; act relu
 * when relu != 0, else identity on the rounded convolution), the pool 3x3, stride 2, padding 1 (pool = {kh, kw,
 * sh, sw, ph, pw}). The convolution output is never stored. Each convolution value is rounded once (bias inside the
 * fp32 sum, MFMA order: within tolerance of the reference's sequential sum); relu and the pool's selection are the
 * reference's bit for bit on those values (reference: src/backends/cpu/kernels/conv.cpp:223-314,
 * elementwise.cpp:329-331, pool.cpp:187-234, first valid element of the window in (kh, kw) order, then a strictly
 * greater one). Replaces the reference's conv2d + relu + max_pool2d chain (cuDNN calls in
 * src/backends/cuda/kernels/conv.cpp:385-520 and pool.cpp:172-244). fh_conv2d_stem_pool_supported: bf16 / f16,
 * Cin <= 3, Cout 64, W % 8 == 0, W <= 224; host-only query. x and y 16-byte aligned. */
int32_t fh_conv2d_stem_pool_supported(int32_t dtype, const int64_t geom[12], const int64_t pool[6]);
fh_status fh_conv2d_stem_pool(int32_t dtype, const void* x, const void* w, const void* bias, void* y,
                              const int64_t geom[12], const int64_t pool[6], int32_t relu, void* stream);

/* C8 layout for convolutions with Cin <= 8 (e.g. an RGB stem): x NCHW [N][C][H*W] (16-bit) ->
 * [N][H*W][8] with channels C..7 zero. No counterpart in the reference (cuDNN consumes NCHW). */
fh_status fh_conv_pack_input_c8(const void* x, void* y, int64_t n, int32_t c, int64_t hw, void* stream);

/* C8 filter: w [Cout][C][KH][KW] (16-bit, C <= 8) -> [Cout][K] with element (kh*KW + kw)*8 + ci, zeros for
 * ci >= C and past KH*KW*8; K = fh_conv_c8_filter_k(KH, KW) = KH*KW*8 rounded up to 32. */
fh_status fh_conv_pack_filter_c8(const void* w, void* y, int32_t cout, int32_t c, int32_t kh, int32_t kw, void* stream);
int64_t fh_conv_c8_filter_k(int64_t kh, int64_t kw);

/* Batched transpose y[b][c][r] = x[b][r][c] (b < batch, r < rows, c < cols), itemsize 2 or 4.
 * Lays out the channels-last conv operands: x NCHW -> NHWC is (batch N, rows Cin, cols H*W); w
 * [Cout][Cin][KH][KW] -> [Cout][KH][KW][Cin] is (batch Cout, rows Cin, cols KH*KW). The reference has no
 * such step (cuDNN consumes NCHW, reference: src/backends/cuda/kernels/conv.cpp:385-520). */
fh_status fh_transpose_batched(int32_t itemsize, const void* x, void* y, int64_t batch, int64_t rows, int64_t cols,
                               void* stream);

/* Several small batched transposes in one launch: for tensor i < n (n <= 32), ys[i][b][c][r] = xs[i][b][r][c] for
 * b < batch[i], r < rows[i], c < cols[i], with rows[i] * cols[i] <= 8192. HipBackend::compile puts all the
 * filters of a graph's channels-last convolutions into one such step. No counterpart in the reference (cuDNN
 * consumes KCRS filters, reference: src/backends/cuda/kernels/conv.cpp:385-520). */
fh_status fh_transpose_planes_multi(int32_t itemsize, int32_t n, const void* const* xs, void* const* ys,
                                    const int64_t* batch, const int64_t* rows, const int64_t* cols, void* stream);

/* One-pass fused elementwise program over `numel` elements.
 * ops/arities follow the fused_elementwise_internal attrs (reference: src/ops/fused_elementwise_utils.cpp:17-120);
 * ins are the node's external inputs in order. Single add/mul/relu nodes are programs with nseg = 1.
 * Replaces elementwise.cu:139-360 and execute_fused_chain (reference: src/ops/fused_elementwise_utils.cpp:122-206). */
fh_status fh_ew_program(int32_t dtype, int32_t nseg, const uint8_t* ops, const int8_t* arities,
                        const void* const* ins, int32_t nin, void* out, int64_t numel,
                        int32_t round_between, void* stream);

/* Row softmax over the last axis of [rows, cols].
 * Replaces cudnnSoftmaxForward (reference: src/backends/cuda/kernels/sequence.cpp:108-178);
 * semantics of softmax_cpu_kernel (reference: src/backends/cpu/kernels/sequence.cpp:114-174). */
fh_status fh_softmax_rows(int32_t dtype, const void* x, void* y, int64_t rows, int64_t cols, void* stream);

/* Row LayerNorm: y = gamma * (x - mean) * (1 / sqrt(var + eps)) + beta.
 * Replaces layer_norm_kernel (reference: src/backends/cuda/kernels/sequence.cu:103-160);
 * semantics of layer_norm_cpu_kernel (reference: src/backends/cpu/kernels/sequence.cpp:182-279). */
fh_status fh_layer_norm_rows(int32_t dtype, const void* x, const void* gamma, const void* beta, void* y,
                             int64_t rows, int64_t cols, float eps, void* stream);

/* Fused scaled dot-product attention over Frame's per-(batch, head) decomposition (reference:
 * src/nn/layers.cpp:1014-1080): q, k, v and out are [batch*seq, heads*dh] row-major; for each (b, h)
 *   out[b*seq.., h*dh..] = round(softmax(round(round(Q_bh K_bh^T) * scale)) V_bh)
 * with every intermediate rounded to the storage dtype where the reference's matmul, mul, softmax and matmul
 * nodes round it. `scale` is the value of the graph's 1/sqrt(dh) constant splat after narrowing to dtype.
 * Replaces, per (b, h), two cuBLASLt matmuls (reference: src/backends/cuda/kernels/matmul.cpp:90-276), a
 * transpose (src/backends/cuda/kernels/shape.cu:65-192), an elementwise mul (elementwise.cu:139-360), a
 * cudnnSoftmaxForward (sequence.cpp:108-178) and the slice/concat copies (shape.cpp:52-355): HipBackend::compile
 * rewrites the whole decomposition into one call. bf16/f16, dh = 64, seq a multiple of 64 up to 512. */
fh_status fh_attention_fwd(int32_t dtype, const void* q, const void* k, const void* v, void* out, int64_t batch,
                           int64_t seq, int64_t heads, int64_t dh, float scale, void* stream);

/* 1 if fh_attention_fwd accepts (dtype, seq, dh), else 0. Host-only query; no counterpart in the reference. */
int32_t fh_attention_supported(int32_t dtype, int64_t seq, int64_t dh);

/* 2-D pooling, NCHW. mode 0 = max (-inf padding, first max wins), 1 = average (include padding).
 * geom = {N, C, H, W, KH, KW, stride_h, stride_w, pad_h, pad_w}.
 * Replaces cudnnPoolingForward (reference: src/backends/cuda/kernels/pool.cpp:172-244);
 * semantics of pool.cpp (reference: src/backends/cpu/kernels/pool.cpp:8-350). */
fh_status fh_pool2d(int32_t dtype, int32_t mode, const void* x, void* y, const int64_t geom[10], void* stream);

/* fh_pool2d over channels-last data: x [N,H,W,C] -> y [N,Ho,Wo,C], same geom (N, C, H, W, ...), semantics and
 * scan order per channel. For activations HipBackend::compile keeps channels-last between convolutions. No
 * counterpart in the reference (NCHW only, reference: src/backends/cpu/kernels/pool.cpp:8-350). */
fh_status fh_pool2d_nhwc(int32_t dtype, int32_t mode, const void* x, void* y, const int64_t geom[10], void* stream);

/* out[i0..] = x[perm-gathered], rank <= 8, itemsize in {1,2,4,8}. out_dims are the output dims;
 * in_strides_permuted[d] is the input element stride of the input axis that output axis d reads.
 * Replaces transpose_kernel (reference: src/backends/cuda/kernels/shape.cu:65-192). */
fh_status fh_permute(int32_t itemsize, const void* x, void* y, int32_t rank, const int64_t* out_dims,
                     const int64_t* in_strides_permuted, void* stream);

/* Strided 2-D byte copy (rows of width_bytes). Backs slice/concat/reshape.
 * Replaces the per-segment cudaMemcpyAsync loops (reference: src/backends/cuda/kernels/shape.cpp:52-355). */
fh_status fh_copy2d(void* dst, int64_t dst_pitch, const void* src, int64_t src_pitch, int64_t width_bytes,
                    int64_t rows, void* stream);

/* Fill `count` elements of `itemsize` bytes with the bit pattern `pattern` (little-endian low bytes).
 * Used for constant materialisation (reference: src/backends/cuda/kernels/constant.cpp:23-73) and to clear
 * memory without hipMemsetAsync. */
fh_status fh_fill(void* dst, int32_t itemsize, uint64_t pattern, int64_t count, void* stream);

/* ---- training path (the gradient-only ops of compiler::build_backward_graph) ---- */

/* matmul_grad_lhs_internal (rhs = 0): out [m,k] = p [m,n] * q[k,n]^T (p = gy, q = b); matmul_grad_rhs_internal
 * (rhs = 1): out [k,n] = p[m,k]^T * q [m,n] (p = a, q = gy). Transposed operands are read in place; every output
 * is one fp32 sum in the reference's order (src/backends/cpu/kernels/matmul.cpp:187-327), so results are
 * bit-identical. HipBackend::compile lowers both ops to a transpose plus the GEMM kernels where those are faster;
 * this entry serves eager launches. The CUDA backend has no kernel for either op (CPU fallback). */
fh_status fh_matmul_grad(int32_t dtype, int32_t rhs, const void* p, const void* q, void* out, int64_t m, int64_t n,
                         int64_t k, void* stream);

/* max_pool2d_grad_internal (mode 0; x = the forward input) / avg_pool2d_grad_internal (mode 1; x unused), NCHW.
 * Mode 2 (no reference counterpart) is mode 0 followed by relu_grad_internal against x, dx = x > 0 ? mode 0's dx
 * : 0, bit for bit the two ops' result: the stem of a training graph, whose pool input is a relu's output.
 * geom as fh_pool2d (the forward input's dims). One thread per input element gathers its covering windows in the
 * reference's order, so results are bit-identical to the CPU reference (src/backends/cpu/kernels/pool.cpp:186-206,
 * 358-388, 543-566). Replaces the recompute-y + cudnnPoolingBackward of max_pool2d_grad_internal
 * (reference: src/backends/cuda/kernels/pool.cpp:245-363) and avg_pool2d_grad_internal's kernel
 * (reference: src/backends/cuda/kernels/pool.cu:250-320). */
fh_status fh_pool2d_grad(int32_t dtype, int32_t mode, const void* dy, const void* x, void* dx, const int64_t geom[10],
                         void* stream);

/* conv2d_grad_input_internal: dx [N,Cin,H,W] from dy [N,Cout,Ho,Wo] and w [Cout,Cin/g,KH,KW];
 * conv2d_grad_filter_internal: dw [Cout,Cin/g,KH,KW] from x and dy. geom as fh_conv2d_fwd (x's dims).
 * Each output is one fp32 sum in the reference's order (src/backends/cpu/kernels/conv.cpp:320-452).
 * Replace cudnnConvolutionBackwardData / cudnnConvolutionBackwardFilter
 * (reference: src/backends/cuda/kernels/conv.cpp:560-789). */
fh_status fh_conv2d_grad_input(int32_t dtype, const void* dy, const void* w, void* dx, const int64_t geom[12],
                               void* stream);
fh_status fh_conv2d_grad_filter(int32_t dtype, const void* x, const void* dy, void* dw, const int64_t geom[12],
                                void* stream);

/* conv2d_grad_filter_internal on MFMA (bf16 / f16, groups 1): x channels-last [N,H,W,cin_pad] (cin_pad % 8 == 0,
 * channels past geom's Cin zero, e.g. the C8 pack of a 3-channel stem), dy channels-last [N,Ho,Wo,Cout]
 * (Cout % 8 == 0), dw [Cout][Cin][KH][KW] as the reference lays it out. geom as fh_conv2d_fwd. The long
 * contraction (N*Ho*Wo) is split across workgroups into fp32 partials in `workspace`, summed in split order;
 * fh_conv2d_wgrad_workspace returns the bytes needed (and the split count), or -1 where this path does not
 * apply (then fh_conv2d_grad_filter). Replaces cudnnConvolutionBackwardFilter
 * (reference: src/backends/cuda/kernels/conv.cpp:700-789). */
int64_t fh_conv2d_wgrad_workspace(int32_t dtype, const int64_t geom[12], int32_t cin_pad, int32_t* splits);
fh_status fh_conv2d_wgrad_nhwc(int32_t dtype, const void* x, const void* dy, void* dw, void* workspace,
                               int64_t workspace_bytes, const int64_t geom[12], int32_t cin_pad, void* stream);
/* fh_conv2d_wgrad_nhwc without a caller workspace and without any allocation: the split-K partials go to a
 * 64 MiB file-scope device array that each device holds until the process ends. No counterpart in the
 * reference; it is for callers that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Geometries whose partials (fh_conv2d_wgrad_workspace) exceed 64 MiB fail with
 * FH_INVALID_ARGUMENT. Every call on a device shares that device's array; calls on one device are ordered by it in
 * the order the host makes them (each call's stream waits for an event the previous call recorded after its
 * kernels, whatever stream that was), except under graph capture, where the graph's own order applies and
 * overlapping replays on one device race. */
fh_status fh_conv2d_wgrad_nhwc_noalloc(int32_t dtype, const void* x, const void* dy, void* dw, const int64_t geom[12],
                                       int32_t cin_pad, void* stream);

/* Operands of conv2d_grad_input as a stride-1 convolution on the implicit-GEMM kernel (dx = conv(dilate(dy),
 * flip(w)), padding KH-1-pad): fh_conv_filter_flip writes out[ci][a][b][co] = w[co][ci][KH-1-a][KW-1-b] (the
 * channels-last filter [Cin][KH][KW][Cout] of that convolution); fh_dilate_nhwc writes the channels-last
 * [N,Hu,Wu,C] tensor holding x's element (n, c, h, w) at (h*sh, w*sw) and zeros elsewhere, x NCHW (in_nhwc 0) or
 * channels-last [N,H,W,C] (in_nhwc 1, C*itemsize % 16 == 0). No counterpart in the reference
 * (cudnnConvolutionBackwardData does this inside the library). */
fh_status fh_conv_filter_flip(int32_t dtype, const void* w, void* out, int64_t cout, int64_t cin, int64_t kh, int64_t kw,
                              void* stream);
fh_status fh_dilate_nhwc(int32_t dtype, int32_t in_nhwc, const void* x, void* out, int64_t n, int64_t c, int64_t h,
                         int64_t w, int64_t sh, int64_t sw, int64_t hu, int64_t wu, void* stream);

/* fh_conv_filter_flip of up to FH_FLIP_MAX same-dtype filters in one launch: out[i] = flip(w[i]) with
 * dims[4i .. 4i+3] = {cout, cin, kh, kw} (kh * kw <= FH_FLIP_MAX_TAPS), each output identical to a separate
 * fh_conv_filter_flip call; the filters must not overlap the outputs. A training graph's filters are all known
 * before its first input gradient, so one launch replaces one per convolution. No counterpart in the reference. */
#define FH_FLIP_MAX 32
#define FH_FLIP_MAX_TAPS 255
fh_status fh_conv_filter_flip_multi(int32_t dtype, int32_t count, const void* const* w, void* const* out,
                                    const int64_t* dims, void* stream);

/* avg_pool2d_grad_internal on channels-last dy [N,Ho,Wo,C] -> dx [N,H,W,C] (C*itemsize % 16 == 0), geom as fh_pool2d;
 * the reference's summation order, bit-identical to fh_pool2d_grad mode 1. For backward graphs whose activations
 * stay channels-last; no counterpart in the reference. */
fh_status fh_avg_pool2d_grad_nhwc(int32_t dtype, const void* dy, void* dx, const int64_t geom[10], void* stream);

/* sum over the axes flagged in reduced[0..rank) (rank <= 8; every axis for the reference's axes = []), output dense
 * with the reduced axes dropped (keepdims only adds size-1 dims, same layout). fp32 tree per output.
 * Replaces sum_cuda_kernel (reference: src/backends/cuda/kernels/reduction.cu:322-460). */
fh_status fh_sum(int32_t dtype, const void* x, void* out, int32_t rank, const int64_t* dims, const uint8_t* reduced,
                 void* stream);

/* sum over every axis but the last of a dense tensor viewed as [rows, cols] (cols*itemsize % 16 == 0): the bias
 * gradient of channels-last activations. Per-workgroup fp32 partials (about 256 workgroups) in `workspace`
 * (fh_sum_rows_workspace bytes, -1 if unsupported), then summed in workgroup order; deterministic. Replaces
 * sum_cuda_kernel for that shape (reference: src/backends/cuda/kernels/reduction.cu:322-460). */
int64_t fh_sum_rows_workspace(int32_t dtype, int64_t rows, int64_t cols);
fh_status fh_sum_rows(int32_t dtype, const void* x, void* out, int64_t rows, int64_t cols, void* workspace,
                      int64_t workspace_bytes, void* stream);

/* out_i = x_i + s_i * y_i over up to FH_AXPY_MAX same-dtype tensors in one launch, with the product rounded to the
 * storage type before the add: the SGD update graph's `add(param, mul(constant(-lr), grad))` pairs, bit-identical to
 * the two elementwise nodes it replaces (reference: src/compiler/autograd.cpp:418-440 builds them; the CPU mul and
 * add are src/backends/cpu/kernels/elementwise.cpp:146-331). numel[i] elements each; s_i is the value the constant
 * holds (already narrowed to the storage type). Any alignment; 16-byte aligned tensors move in 16-byte vectors. */
#define FH_AXPY_MAX 32
fh_status fh_axpy_multi(int32_t dtype, int32_t count, const void* const* x, const void* const* y, void* const* out,
                        const int64_t* numel, const float* scales, void* stream);

/* sum_grad_internal: gx (dims) = gy broadcast along the reduced axes, a copy of the stored bits
 * (reference: src/backends/cpu/kernels/reduction.cpp:378-388; the CUDA backend has no kernel for it and falls
 * back to the CPU). */
fh_status fh_sum_grad(int32_t dtype, const void* gy, void* gx, int32_t rank, const int64_t* dims,
                      const uint8_t* reduced, void* stream);

/* mse_loss: out (one element) = mean((pred - target)^2), fp32 tree; mse_loss_grad_internal: out = 2 * gy / numel *
 * (pred - target), bit-identical to the CPU reference (src/backends/cpu/kernels/loss.cpp:110-262; the CUDA backend
 * has no kernel for either and falls back to the CPU). */
fh_status fh_mse_loss(int32_t dtype, const void* pred, const void* target, void* out, int64_t numel, void* stream);
fh_status fh_mse_loss_grad(int32_t dtype, const void* pred, const void* target, const void* gy, void* out,
                           int64_t numel, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FRAME_HIP_ABI_H_ */
