// Shared definitions of the GEMM kernels: launch arguments, the epilogue program, and the entry points of the
// 16-bit MFMA path (fh_gemm16.hip) used by the dispatcher in fh_gemm.hip.
#pragma once

#include <hip/hip_runtime.h>

#include "fh_common.h"

namespace fh {

struct EpilogueArgs {
  int32_t nseg;
  int32_t round_between;
  uint8_t ops[FH_MAX_SEGMENTS];
  const void* ins[FH_MAX_SEGMENTS];
};

constexpr int kGemmMaxGroups = FH_GEMM_MAX_GROUPS;

struct GemmArgs {
  const void* A;
  const void* B;
  void* C;
  int64_t M, N, K;
  int64_t lda, ldb, ldc;                 // row strides in elements
  int64_t stride_a, stride_b, stride_c;  // batch strides in elements (blockIdx.y)
  int32_t tiles_m, tiles_n;
  EpilogueArgs ep;
  // Transposed operand storage, honoured by the sequential kernel only: A(m, k) = A[k * lda + m],
  // B(k, n) = B[n * ldb + k].
  int32_t trans_a, trans_b;
  // FH_GEMM_ANY_ORDER: the k-sum may be reassociated (small problems then take the split-k kernel).
  int32_t any_order;
  // FH_GEMM_ROW_SOFTMAX: softmax over every output row after the epilogue (split-k kernel, N <= 16).
  int32_t row_softmax;
  // groups > 0 (16-bit MFMA kernel only): blockIdx.y = g selects B, C and the epilogue operands from these
  // arrays instead of the batch strides; A is shared (stride_a = 0).
  int32_t groups;
  const void* group_b[kGemmMaxGroups];
  void* group_c[kGemmMaxGroups];
  const void* group_ins[kGemmMaxGroups][FH_MAX_SEGMENTS];
};

typedef float f32x16_t __attribute__((ext_vector_type(16)));

// bf16 / f16 GEMM on 32x32x16 MFMA with direct-to-LDS operand loads (fh_gemm16.hip).
// Accepts: K % 32 == 0, N % 8 == 0, lda/ldb/ldc % 8 == 0, 16-byte aligned base pointers and batch strides,
// 16-byte aligned epilogue operands. Returns false (and launches nothing) otherwise.
bool gemm16_try_launch(int32_t dtype, const GemmArgs& args, int64_t batch, hipStream_t stream, fh_status* status);

}  // namespace fh
