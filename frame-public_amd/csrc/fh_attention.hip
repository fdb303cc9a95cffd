// Fused scaled dot-product attention for Frame's per-(batch, head) decomposition (reference:
// src/nn/layers.cpp:1014-1080). For batch b and head h, with Q/K/V the [batch*seq, heads*dh] projections:
//   S  = round(Q_bh · K_bhᵀ)            (matmul, fp32 accumulate, one rounding)
//   S2 = round(S * scale)                (mul by the 1/sqrt(dh) constant splat)
//   P  = softmax rows of S2, rounded     (m = max, e = exp(x - m), s = sum e, y = round(e / s))
//   O  = round(P · V_bh)                 (matmul)
// and O lands at rows [b*seq, (b+1)*seq), columns [h*dh, (h+1)*dh) of the output: the layout of the reference's
// head concat (axis 1) and batch concat (axis 0). Every intermediate is rounded where the reference rounds it;
// only the summation order (MFMA blocks, a tree for the softmax sum) and the exp routine differ.
//
// One workgroup (4 waves) per (64-row block, head, batch). LDS: the Q block [64][64], K_bh then V_bh [seq][64]
// (the same buffer, reused), and the score / probability rows [64][seq], all bf16/f16:
//   1. Q block and K_bh -> LDS (global_load_lds_dwordx4), rows k-contiguous, 16-byte chunks swizzled by row.
//   2. S: waves 2 x 2 (32 rows x seq/2 keys each) on v_mfma_f32_32x32x16; both operands k-contiguous in LDS.
//      Rounded twice (product, scale) into the score rows.
//   3. V_bh -> LDS (overlapping the softmax); softmax per row, one row per wave at a time, wave reductions.
//   4. O: waves 2 x 2 (32 rows x 32 columns), A = probability rows, B = V through ds_read_b64_tr_b16.
#include <hip/hip_runtime.h>

#include <string>

#include "fh_common.h"
#include "fh_gemm.h"
#include "fh_mfma16.h"

namespace fh {
namespace {

using namespace mfma16;

constexpr int kDh = 64;      // head dim
constexpr int kRows = 64;    // query rows per workgroup
constexpr int kMaxSeq = 512;

typedef short s16x4_t __attribute__((ext_vector_type(4)));

// 16-byte chunk swizzles: Q/K rows (8 chunks) by row & 7; score rows (seq/8 chunks) by row & pmask, pmask = 15
// when the chunk count is a multiple of 16 (16 rows of one ds_read_b128 phase hit 16 distinct 16-byte bank
// groups), else 7 (the count is a multiple of 8, so the swizzled chunk stays inside the row); V rows (8 chunks)
// for transpose reads as in the GEMM.
__device__ __forceinline__ int qk_chunk(int row, int c) { return c ^ (row & 7); }
__device__ __forceinline__ int p_chunk(int row, int c, int pmask) { return c ^ (row & pmask); }
__device__ __forceinline__ int v_chunk(int krow, int c) { return c ^ (2 * (krow & 3)); }

template <typename T>
__global__ __launch_bounds__(256) void attention_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                                        const uint16_t* __restrict__ v, uint16_t* __restrict__ out,
                                                        int seq, int heads, float scale) {
  __shared__ __attribute__((aligned(1024))) unsigned char qs[kRows * kDh * 2];
  __shared__ __attribute__((aligned(1024))) unsigned char kv[kMaxSeq * kDh * 2];
  __shared__ __attribute__((aligned(1024))) unsigned char ps[kRows * kMaxSeq * 2];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, hi = lane >> 5;
  const int r0 = blockIdx.x * kRows, h = blockIdx.y, b = blockIdx.z;
  const int64_t ld = static_cast<int64_t>(heads) * kDh;        // row stride of q/k/v/out (elements)
  const int64_t base = (static_cast<int64_t>(b) * seq) * ld + static_cast<int64_t>(h) * kDh;
  const int pchunks = seq / 8;                                  // 16-byte chunks per score row
  const int pmask = (pchunks & 15) == 0 ? 15 : 7;

  // ---- 1. Q block and K_bh into LDS: one wave instruction = 8 rows of 128 B ----
  {
    const int row_in = lane >> 3, pc = lane & 7;  // lane -> (row within the 8, physical chunk)
    for (int i = wave; i < kRows / 8; i += 4) {
      const int row = i * 8 + row_in;
      const uint16_t* src = q + base + static_cast<int64_t>(r0 + row) * ld + qk_chunk(row, pc) * 8;
      __builtin_amdgcn_global_load_lds(src, (FH_LDS void*)(qs + i * 1024), 16, 0, 0);
    }
    for (int i = wave; i < seq / 8; i += 4) {
      const int row = i * 8 + row_in;
      const uint16_t* src = k + base + static_cast<int64_t>(row) * ld + qk_chunk(row, pc) * 8;
      __builtin_amdgcn_global_load_lds(src, (FH_LDS void*)(kv + i * 1024), 16, 0, 0);
    }
  }
  wait_vmcnt<0>();
  __syncthreads();

  // ---- 2. S = Q K^T for rows wm*32.., keys wn*(seq/2).. ; rounded, scaled, rounded, into the score rows ----
  {
    const int keys_per_wave = seq / 2;
    const int tiles = keys_per_wave / 32;  // <= 8
    f32x16_t acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int x = 0; x < 16; ++x) acc[j][x] = 0.0f;
    const int arow = wm * 32 + l32;
#pragma unroll
    for (int s = 0; s < kDh / 16; ++s) {
      const u32x4_t a = *reinterpret_cast<const u32x4_t*>(qs + arow * 128 + qk_chunk(arow, 2 * s + hi) * 16);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (j < tiles) {
          const int key = wn * keys_per_wave + j * 32 + l32;
          const u32x4_t bf = *reinterpret_cast<const u32x4_t*>(kv + key * 128 + qk_chunk(key, 2 * s + hi) * 16);
          mfma32<T>(a, bf, acc[j]);
        }
      }
    }
    uint16_t* prow = reinterpret_cast<uint16_t*>(ps);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (j < tiles) {
        const int col = wn * keys_per_wave + j * 32 + l32;
#pragma unroll
        for (int x = 0; x < 16; ++x) {
          const int row = wm * 32 + 8 * (x >> 2) + 4 * hi + (x & 3);
          const float s1 = Io<T>::round(acc[j][x]);
          prow[row * seq + p_chunk(row, col >> 3, pmask) * 8 + (col & 7)] = Io<T>::store(s1 * scale);
        }
      }
    }
  }
  __syncthreads();  // score rows complete; K no longer read

  // ---- 3. V_bh into LDS (rows = keys, n-contiguous, chunks swizzled for transpose reads), then softmax ----
  {
    const int row_in = lane >> 3, pc = lane & 7;
    for (int i = wave; i < seq / 8; i += 4) {
      const int row = i * 8 + row_in;
      const uint16_t* src = v + base + static_cast<int64_t>(row) * ld + v_chunk(row, pc) * 8;
      __builtin_amdgcn_global_load_lds(src, (FH_LDS void*)(kv + i * 1024), 16, 0, 0);
    }
  }
  {
    uint16_t* prow = reinterpret_cast<uint16_t*>(ps);
    for (int row = wave; row < kRows; row += 4) {
      float e[8];
      const bool mine = lane < pchunks;
      uint4 w = make_uint4(0, 0, 0, 0);
      if (mine) w = *reinterpret_cast<const uint4*>(prow + row * seq + p_chunk(row, lane, pmask) * 8);
      uint16_t raw[8];
      __builtin_memcpy(raw, &w, 16);
      float m = -__builtin_inff();
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        e[i] = Io<T>::load(raw[i]);
        if (mine) m = fmaxf(m, e[i]);
      }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
      float sum = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        e[i] = mine ? expf(e[i] - m) : 0.0f;
        sum += e[i];
      }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off);
      if (mine) {
#pragma unroll
        for (int i = 0; i < 8; ++i) raw[i] = Io<T>::store(e[i] / sum);
        __builtin_memcpy(&w, raw, 16);
        *reinterpret_cast<uint4*>(prow + row * seq + p_chunk(row, lane, pmask) * 8) = w;
      }
    }
  }
  wait_vmcnt<0>();  // this wave's V rows have landed
  __syncthreads();

  // ---- 4. O = P V: rows wm*32.., columns wn*32.. ----
  {
    f32x16_t acc;
#pragma unroll
    for (int x = 0; x < 16; ++x) acc[x] = 0.0f;
    const int arow = wm * 32 + l32;
    // transpose reads: group g = lane/16 covers 16 columns and 4 k; lane r = qd + 4e of the group points at
    // row (kbase + e), columns n + 4 qd .. n + 4 qd + 3
    const int g = lane >> 4, r = lane & 15, qd = r & 3, e = r >> 2;
    const int ncol = wn * 32 + 16 * (g & 1) + 4 * qd;
    for (int t = 0; t < seq / 16; ++t) {
      const u32x4_t a = *reinterpret_cast<const u32x4_t*>(ps + arow * seq * 2 + p_chunk(arow, 2 * t + hi, pmask) * 16);
      u32x4_t bf;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int krow = 16 * t + 8 * (g >> 1) + 4 * half + e;
        const int off = krow * 128 + v_chunk(krow, ncol >> 3) * 16 + (ncol & 7) * 2;
        const s16x4_t tr = __builtin_amdgcn_ds_read_tr16_b64_v4i16((FH_LDS s16x4_t*)(kv + off));
        const u32x2_t t2 = __builtin_bit_cast(u32x2_t, tr);
        bf[2 * half] = t2[0];
        bf[2 * half + 1] = t2[1];
      }
      mfma32<T>(a, bf, acc);
    }
    const int col = h * kDh + wn * 32 + l32;
#pragma unroll
    for (int x = 0; x < 16; ++x) {
      const int row = r0 + wm * 32 + 8 * (x >> 2) + 4 * hi + (x & 3);
      out[(static_cast<int64_t>(b) * seq + row) * ld + col] = Io<T>::store(acc[x]);
    }
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace fh

using namespace fh;

extern "C" int32_t fh_attention_supported(int32_t dtype, int64_t seq, int64_t dh) {
  return (dtype == FH_BF16 || dtype == FH_F16) && dh == kDh && seq >= kRows && seq <= kMaxSeq && seq % kRows == 0 ? 1 : 0;
}

extern "C" fh_status fh_attention_fwd(int32_t dtype, const void* q, const void* k, const void* v, void* out, int64_t batch,
                                      int64_t seq, int64_t heads, int64_t dh, float scale, void* stream) {
  if (!fh_attention_supported(dtype, seq, dh))
    return fail(FH_UNIMPLEMENTED, "fh_attention_fwd: needs bf16/f16, head dim 64, seq a multiple of 64 up to 512");
  if (batch < 0 || heads < 1 || batch > 65535 || heads > 65535) return fail(FH_INVALID_ARGUMENT, "fh_attention_fwd: bad batch/heads");
  if (batch == 0) return FH_OK;
  if (q == nullptr || k == nullptr || v == nullptr || out == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_attention_fwd: null pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v)) return fail(FH_INVALID_ARGUMENT, "fh_attention_fwd: q/k/v must be 16-byte aligned");
  const dim3 grid(static_cast<uint32_t>(seq / kRows), static_cast<uint32_t>(heads), static_cast<uint32_t>(batch));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const auto* qq = static_cast<const uint16_t*>(q);
  const auto* kk = static_cast<const uint16_t*>(k);
  const auto* vv = static_cast<const uint16_t*>(v);
  auto* oo = static_cast<uint16_t*>(out);
  if (dtype == FH_BF16) {
    hipLaunchKernelGGL(attention_kernel<bf16_t>, grid, dim3(256), 0, s, qq, kk, vv, oo, static_cast<int>(seq),
                       static_cast<int>(heads), scale);
  } else {
    hipLaunchKernelGGL(attention_kernel<f16_t>, grid, dim3(256), 0, s, qq, kk, vv, oo, static_cast<int>(seq),
                       static_cast<int>(heads), scale);
  }
  return launch_status("attention_kernel launch");
}
