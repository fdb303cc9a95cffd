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

struct GemmArgs {
  const void* A;
  const void* B;
  void* C;
  int64_t M, N, K;
  int64_t lda, ldb, ldc;                 // row strides in elements
  int64_t stride_a, stride_b, stride_c;  // batch strides in elements (blockIdx.y)
  int32_t tiles_m, tiles_n;
  EpilogueArgs ep;
};

typedef float f32x16_t __attribute__((ext_vector_type(16)));

// Accumulator drain between a GEMM main loop and its epilogue. Measured on MI355X: when several waves share a
// SIMD, a VALU read of an MFMA result placed at the compiler's minimum distance after the MFMA (12 wait states
// for v_mfma_f32_32x32x16_bf16) can return the accumulator's previous value. Each accumulator is tied to an
// AGPR-resident asm statement so no copy or read of it can be scheduled earlier; the first one carries 24 wait
// states. Call acc_to_agpr() once before the main loop (keeps the accumulators in AGPRs for the whole loop,
// so the ties below add no copies) and drain_accumulators() right after it.
template <int TM, int TN>
__device__ __forceinline__ void acc_to_agpr(f32x16_t (&acc)[TM][TN]) {
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) asm volatile("" : "+a"(acc[i][j]));
}

template <int TM, int TN>
__device__ __forceinline__ void drain_accumulators(f32x16_t (&acc)[TM][TN]) {
  asm volatile("s_nop 7\n s_nop 7\n s_nop 7" : "+a"(acc[0][0]));
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) asm volatile("" : "+a"(acc[i][j]));
}

// bf16 / f16 GEMM on 32x32x16 MFMA with direct-to-LDS operand loads (fh_gemm16.hip).
// Accepts: K % 32 == 0, N % 8 == 0, lda/ldb/ldc % 8 == 0, 16-byte aligned base pointers and batch strides,
// 16-byte aligned epilogue operands. Returns false (and launches nothing) otherwise.
bool gemm16_try_launch(int32_t dtype, const GemmArgs& args, int64_t batch, hipStream_t stream, fh_status* status);

}  // namespace fh
