// Device helpers shared by the MFMA kernels (fh_gemm16.hip, fh_conv_igemm.hip, fh_attention.hip): MFMA wrapper, explicit
// wait counts, LDS fragment reads, direct-to-LDS loads, LDS
// swizzles and the in-loop instruction spreading used by the software pipelines.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>
#include <utility>

#include "fh_common.h"
#include "fh_gemm.h"

namespace fh {
namespace mfma16 {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

#define FH_LDS __attribute__((address_space(3)))

constexpr int kBK = 32;      // k per stage
constexpr int kStages = 4;   // LDS ring depth

// One k-slice of the 32x32 MFMA tile from a 16-byte fragment per lane (lane half h holds k-chunk h of the
// slice). 16-bit: the chunk is 8 k-values, one 32x32x16 instruction. fp32: the chunk is 4 k-values; four 32x32x2
// instructions take component j of both halves' chunks, and since both operands use the same k assignment the
// slice's 8 products are all summed.
template <typename T>
__device__ __forceinline__ void mfma32(const u32x4_t& a, const u32x4_t& b, f32x16_t& acc) {
  if constexpr (std::is_same_v<T, float>) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a[j]), __uint_as_float(b[j]), acc, 0, 0, 0);
  } else if constexpr (std::is_same_v<T, bf16_t>) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                  acc, 0, 0, 0);
  } else {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b),
                                                 acc, 0, 0, 0);
  }
}

typedef float f32x4_t __attribute__((ext_vector_type(4)));

// One 16x16 tile, k 32: lane l holds row (A) / column (B) l % 16 and k 8 (l / 16) .. + 7 as one 16-byte fragment;
// the result's lane l holds column l % 16, rows 4 (l / 16) .. + 3. At equal MFMA throughput to the 32x32x16 form
// it moves a quarter of the accumulator bytes per product through the register file.
template <typename T>
__device__ __forceinline__ void mfma16x(const u32x4_t& a, const u32x4_t& b, f32x4_t& acc) {
  static_assert(!std::is_same_v<T, float>, "16-bit operands");
  if constexpr (std::is_same_v<T, bf16_t>) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                  acc, 0, 0, 0);
  } else {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), acc,
                                                 0, 0, 0);
  }
}

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[15:14]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Fragment reads are inline asm without a memory clobber: the compiler's LDS-DMA wait tracking does not follow
// the stage ring across the loop (it either waits for every in-flight prefetch or, on other paths, for
// nothing), so the kernel orders LDS itself: explicit vmcnt waits + s_barrier before a stage is read, and
// fence_fragments() (lgkmcnt(0), tied to the fragment registers) before the MFMAs consume them.
template <int OFF>
__device__ __forceinline__ u32x4_t lds_read_b128(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
  u32x4_t v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF));
  return v;
}

template <int OFF>
__device__ __forceinline__ u32x2_t lds_read_tr16_b64(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
  u32x2_t v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF));
  return v;
}

__device__ __forceinline__ uint32_t lds_addr(const FH_LDS void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}

__device__ __forceinline__ void global_to_lds16(const void* g, FH_LDS void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(g, lds_wave_base, 16, 0, 0);
}

// Runs the epilogue program on 8 rounded outputs (one 16-byte vector) at flat output index idx.
// XOR swizzles of the 16-byte chunks of an LDS row (gfx950 LDS: 64 banks of 4 bytes, 256 B per cycle).
// A rows are 64 B (4 chunks); XOR with (row >> 2) & 3 makes the ds_read_b128 fragment reads (32 consecutive
// rows, one chunk each) conflict-free. B rows are BN*2 B: the 4 consecutive k rows of one transpose-read group
// get disjoint 64-byte windows. Both were chosen by measuring SQ_LDS_BANK_CONFLICT for candidate patterns on
// an MI355X (zero conflict cycles per instruction for both).
__device__ __forceinline__ int a_swizzle(int row) { return (row >> 2) & 3; }
template <int B_CHUNKS>
__device__ __forceinline__ int b_swizzle(int krow) {
  if constexpr (B_CHUNKS >= 16) {
    return (2 * (krow & 3)) ^ (8 * (krow & 1));
  } else {
    return 2 * (krow & 3);
  }
}

// B swizzle for the 16x16x32 fragment reads: the two 16-lane groups served together read the same columns at
// k rows 8 apart, so bit 3 of the row also moves the chunk (by 2, onto the pairs rows 0-3 leave free).
template <int B_CHUNKS>
__device__ __forceinline__ int b_swizzle16(int krow) {
  return b_swizzle<B_CHUNKS>(krow) ^ (2 * ((krow >> 3) & 1));
}

// Number of items issued right after MFMA m when n items are spread over the first r MFMAs of a half, and the
// index of the first of them.
constexpr int share(int m, int n, int r) { return m < r ? (m + 1) * n / r - m * n / r : 0; }
constexpr int first(int m, int n, int r) { return (m < r ? m : r) * n / r; }

}  // namespace mfma16
}  // namespace fh
