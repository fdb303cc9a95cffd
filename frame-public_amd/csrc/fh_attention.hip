// Fused scaled dot-product attention for Frame's per-(batch, head) decomposition (reference:
// src/nn/layers.cpp:1014-1080). For batch b and head h, with Q/K/V the [batch*seq, heads*dh] projections:
//   S  = round(Q_bh · K_bhᵀ)            (matmul, fp32 accumulate, one rounding)
//   S2 = round(S * scale)                (mul by the 1/sqrt(dh) constant splat)
//   P  = softmax rows of S2, rounded     (m = max, e = exp(x - m), s = sum e, y = round(e / s))
//   O  = round(P · V_bh)                 (matmul)
// and O lands at rows [b*seq, (b+1)*seq), columns [h*dh, (h+1)*dh) of the output: the layout of the reference's
// head concat (axis 1) and batch concat (axis 0). S and S2 are rounded where the reference rounds them and m is
// the exact row maximum of S2. The normalisation moves behind the second product: the kernel multiplies
// round(e) (not round(e / s)) by V and scales the fp32 sums by 1/s before the one output rounding, so every
// exponential is evaluated once. That, the summation orders (MFMA blocks, per-lane partial sums) and the exp
// routine (v_exp_f32 of x log2(e) - m log2(e)) differ from the decomposition, each well inside one rounding of
// the stored probabilities.
//
// One wave owns 32 queries and all seq keys; a workgroup is W waves (4, or 2 when seq is not a multiple of 128).
// The work is bound by its VALU instruction stream (about 7 VALU instructions per score, one of them the
// quarter-rate exponential, against two MFMA k-steps per 32 x 32 tile), so the per-score code is kept short.
//  1. Scores transposed, Sᵀ = K·Qᵀ on v_mfma_f32_32x32x16, per 64-key block: K blocks stream through a
//     double-buffered 8 KB LDS ring (global_load_lds_dwordx4, 16-byte chunks swizzled by row), the Q fragments
//     stay in registers. Each lane's accumulator then holds one query and 16 keys of a 32-key tile; they are
//     rounded, scaled, rounded and kept as packed bf16/f16 in registers (seq/2 values per lane). The running
//     maximum is taken over the scaled values before their rounding: rounding is monotonic, so the rounded
//     maximum is the maximum of the rounded values.
//  2. m per query: the lane's maximum and its partner lane's (lane ^ 32, same query).
//  3. Oᵀ = Vᵀ·Pᵀ: p = round(exp(S2 - m)) is produced in registers already in the B-operand layout (k = the
//     lane's 8 keys of one query, in the accumulator's key order) while the lane sums the unrounded e; the A
//     operand (Vᵀ) comes from V blocks in LDS through ds_read_b64_tr_b16 in the same key order. V streams like
//     K did. The output is round(acc * (1/s)), s = the lane's sum plus its partner's.
// LDS: 32 KB per workgroup (two K and two V blocks), so two workgroups share a CU.
#include <hip/hip_runtime.h>

#include <cmath>
#include <string>
#include <utility>

#include "fh_common.h"
#include "fh_gemm.h"
#include "fh_mfma16.h"

namespace fh {
namespace {

using namespace mfma16;

constexpr int kDh = 64;      // head dim
constexpr int kMaxSeq = 512;

typedef short s16x4_t __attribute__((ext_vector_type(4)));

// 16-byte chunk swizzles of a 128-byte LDS row: K rows by row & 7 (the 32 rows of one fragment read spread over
// the banks); V rows by 2 * (row & 3) for the transpose reads (4 consecutive rows hit disjoint 32-byte windows).
__device__ __forceinline__ int k_chunk(int row, int c) { return c ^ (row & 7); }
__device__ __forceinline__ int v_chunk(int row, int c) { return c ^ (2 * (row & 3)); }

template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) { return store2<T>(lo, hi); }
template <typename T>
__device__ __forceinline__ float lo16(uint32_t v) { return load_lo<T>(v); }
template <typename T>
__device__ __forceinline__ float hi16(uint32_t v) { return load_hi<T>(v); }

// POW2: scale is a power of two (1/sqrt(dh) for dh = 64, 256, ...). Then round(S) * scale is exact, so
// round(round(S) * scale) = round(S) * scale: pass 1 keeps round(S) and the maximum of the fp32 sums, and the
// scale moves into the exponent's constant, scale log2(e) = scale * round(log2(e)) exactly, which gives the same
// fma arguments bit for bit. (Products that fall into T's denormal range are the exception: they lose bits in
// the reference's rounding; their exponentials are 1 to within an fp32 rounding either way.)
template <typename T, int NB, int W, bool POW2>
__global__ __launch_bounds__(W * 64, 2) void attention_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                                              const uint16_t* __restrict__ v, uint16_t* __restrict__ out,
                                                              int heads, float scale) {
  constexpr int SEQ = NB * 64;
  constexpr int NT = SEQ / 32;  // 32-key tiles
  constexpr int BLK = 64 * 128;  // one 64-key block of K or V, bytes
  constexpr int LOADS = 8 / W;   // 1 KB global->LDS instructions per wave and block
  static_assert(LOADS * NB < 64, "vmcnt range");
  // Slot b holds K block b, then V block b: every K block is requested at the start, and V block b goes into
  // slot b as soon as every wave has read K block b, so V is resident well before pass 3 reads it.
  __shared__ __attribute__((aligned(1024))) unsigned char kv[NB * BLK];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l32 = lane & 31, hi = lane >> 5;
  const int h = blockIdx.y, b = blockIdx.z;
  const int q0 = blockIdx.x * (32 * W) + wave * 32;
  const int64_t ld = static_cast<int64_t>(heads) * kDh;
  const int64_t base = (static_cast<int64_t>(b) * SEQ) * ld + static_cast<int64_t>(h) * kDh;

  // Q fragments (B operand of Sᵀ = K·Qᵀ): lane -> query q0 + l32, d = 16 s + 8 hi .. + 7
  u32x4_t qf[4];
#pragma unroll
  for (int s = 0; s < 4; ++s)
    qf[s] = *reinterpret_cast<const u32x4_t*>(q + base + static_cast<int64_t>(q0 + l32) * ld + 16 * s + 8 * hi);
  // the vmcnt counts below count the K / V loads only: the Q loads stay ahead of them (loads retire in order)
  asm volatile("" ::: "memory");

  // block loaders: instruction i of a block = rows 8i .. 8i + 7, lane -> (row 8i + lane / 8, physical chunk lane % 8)
  auto load_block = [&](const uint16_t* src, int blk, bool is_v) {
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      const int i = wave + W * j;
      const int row = 8 * i + (lane >> 3), pc = lane & 7;
      const int c = is_v ? v_chunk(row, pc) : k_chunk(row, pc);
      const uint16_t* g = src + base + static_cast<int64_t>(blk * 64 + row) * ld + c * 8;
      __builtin_amdgcn_global_load_lds(g, (FH_LDS void*)(kv + blk * BLK + i * 1024), 16, 0, 0);
    }
  };
  // The LDS reads below are inline asm the compiler does not order against the LDS-DMA loads (its own tracking
  // would wait for every load in flight at each read or barrier), so the kernel orders them itself: a block is
  // read after this wave's vmcnt wait for it and an s_barrier (every wave's share landed), and a slot is
  // refilled only after a barrier that every wave reached with its reads of the slot complete (lgkmcnt(0)).
  auto barrier = [] {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  const uint32_t kv_addr = lds_addr((const FH_LDS void*)kv);

#pragma unroll
  for (int blk = 0; blk < NB; ++blk) load_block(k, blk, false);

  // K fragment of (k-slice s, key tile t) for this lane: row 32 t + l32, chunk 2 s + hi; the swizzle uses row & 7
  // = l32 & 7 only, so tile t adds 32 rows = 4096 bytes
  uint32_t k_off[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) k_off[s] = kv_addr + l32 * 128 + k_chunk(l32, 2 * s + hi) * 16;

  // ---- 1. scores, kept as packed 16-bit values: s2[t][j] = keys (x = 2j, 2j + 1) of tile t ----
  uint32_t s2[NT][8];
  float mraw = -__builtin_inff();  // maximum of the scaled scores (POW2: of the sums) before their rounding
  [&]<int... B_>(std::integer_sequence<int, B_...>) {
    (
        [&] {
          constexpr int blk = B_;
          // this wave's loads of K block blk have landed when no more than the ones issued after them are in
          // flight: K blocks blk+1 .. NB-1 and V blocks 0 .. blk-2
          wait_vmcnt<LOADS * ((NB - 1 - blk) + (blk >= 2 ? blk - 1 : 0))>();
          barrier();
          if constexpr (blk >= 1) load_block(v, blk - 1, true);  // every wave has read K block blk - 1
          u32x4_t kf[4][2];
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            kf[s][0] = lds_read_b128<blk * BLK>(k_off[s]);
            kf[s][1] = lds_read_b128<blk * BLK + 4096>(k_off[s]);
          }
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
          for (int s = 0; s < 4; ++s) asm volatile("" : "+v"(kf[s][0]), "+v"(kf[s][1]));
          f32x16_t acc[2];
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int x = 0; x < 16; ++x) acc[t][x] = 0.0f;
#pragma unroll
          for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int t = 0; t < 2; ++t) mfma32<T>(kf[s][t], qf[s], acc[t]);
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
              const uint32_t sr = pack2<T>(acc[t][2 * j], acc[t][2 * j + 1]);  // round(S), two keys
              if constexpr (POW2) {
                // max(mraw, a, b) in one instruction: fmaxf on the raw MFMA results would first canonicalise
                // each of them (the compiler cannot prove an MFMA result is not a signalling NaN; it never is)
                float mx;
                asm("v_max3_f32 %0, %1, %2, %3" : "=v"(mx) : "v"(mraw), "v"(acc[t][2 * j]), "v"(acc[t][2 * j + 1]));
                mraw = mx;
                s2[2 * blk + t][j] = sr;
              } else {
                const float a0 = lo16<T>(sr) * scale, a1 = hi16<T>(sr) * scale;
                mraw = fmaxf(mraw, fmaxf(a0, a1));
                s2[2 * blk + t][j] = pack2<T>(a0, a1);  // round(S * scale)
              }
              asm volatile("" : "+v"(s2[2 * blk + t][j]));  // pass 3 unpacks; nothing of a0, a1 stays live
            }
        }(),
        ...);
  }(std::make_integer_sequence<int, NB>{});
  barrier();  // every wave has read K block NB - 1
  load_block(v, NB - 1, true);

  // ---- 2. row maximum ----
  constexpr float kLog2e = 1.44269504088896340736f;
  const float mr = Io<T>::round(fmaxf(mraw, __shfl_xor(mraw, 32)));
  const float m = POW2 ? mr * scale : mr;
  const float ml = m * kLog2e;                      // exp(x - m) = exp2(x log2(e) - ml)
  const float c = POW2 ? scale * kLog2e : kLog2e;   // x = c-scaled stored value

  // ---- 3. Oᵀ = Vᵀ·Pᵀ, two 32-row d tiles ----
  f32x16_t acc_o[2];
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int x = 0; x < 16; ++x) acc_o[dt][x] = 0.0f;
  // transpose reads: group g = lane / 16 covers d columns 16 (g & 1) .. + 15 of a d tile and the key half
  // g >> 1; source lane qd + 4 e of the group points at key row (kbase + e), columns n0 + 4 qd .. + 3. The key
  // row is 32 tt + 16 hf + 4 (g >> 1) + 8 part + e, so its swizzle (row & 3 = e) is the same for every read and
  // tt, hf, part add whole rows.
  const int g = lane >> 4, rr = lane & 15, qd = rr & 3, e = rr >> 2;
  uint32_t v_off[2];
#pragma unroll
  for (int dt = 0; dt < 2; ++dt) {
    const int n0 = 32 * dt + 16 * (g & 1) + 4 * qd;
    const int krow = 4 * (g >> 1) + e;
    v_off[dt] = kv_addr + krow * 128 + v_chunk(krow, n0 >> 3) * 16 + (n0 & 7) * 2;
  }
  float sum = 0.0f;
  wait_vmcnt<LOADS>();  // this wave's V blocks 0 .. NB-2
  barrier();
  [&]<int... B_>(std::integer_sequence<int, B_...>) {
    (
        [&] {
          constexpr int blk = B_;
          if constexpr (blk == NB - 1) {
            wait_vmcnt<0>();
            barrier();
          }
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) {
            const int t = 2 * blk + tt;
            // this tile's V fragments first, so the exponentials below run while they are in flight
            u32x2_t vf[2][2][2];
            [&]<int... R_>(std::integer_sequence<int, R_...>) {
              (
                  [&] {
                    constexpr int dt = R_ / 4, hf = (R_ / 2) % 2, part = R_ % 2;
                    constexpr int off = blk * BLK + (16 * hf + 8 * part) * 128;
                    vf[dt][hf][part] = lds_read_tr16_b64<off>(v_off[dt] + tt * 32 * 128);
                  }(),
                  ...);
            }(std::make_integer_sequence<int, 8>{});
            u32x4_t pf[2];
            float part[8];
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                uint32_t w = s2[t][4 * hf + j];
                asm volatile("" : "+v"(w));  // keeps the exp of this tile here, after the block's barrier
                const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(lo16<T>(w), c, -ml));
                const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(hi16<T>(w), c, -ml));
                part[4 * hf + j] = e0 + e1;
                pf[hf][j] = pack2<T>(e0, e1);
              }
            // the tile's sum joins the running sum here (tied), so no tile's exponentials outlive the tile
            sum += ((part[0] + part[1]) + (part[2] + part[3])) + ((part[4] + part[5]) + (part[6] + part[7]));
            asm volatile("" : "+v"(sum));
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
            for (int dt = 0; dt < 2; ++dt)
#pragma unroll
              for (int hf = 0; hf < 2; ++hf) {
                asm volatile("" : "+v"(vf[dt][hf][0]), "+v"(vf[dt][hf][1]));
                // keys of this MFMA for k-half g >> 1: 32 tt + 16 hf + 4 (g >> 1) + {0..3, 8..11}
                const u32x4_t a{vf[dt][hf][0][0], vf[dt][hf][0][1], vf[dt][hf][1][0], vf[dt][hf][1][1]};
                mfma32<T>(a, pf[hf], acc_o[dt]);
              }
          }
        }(),
        ...);
  }(std::make_integer_sequence<int, NB>{});

  // ---- output: acc_o[dt][x] = O[query q0 + l32][d = 32 dt + 8 (x / 4) + 4 hi + x % 4] ----
  sum += __shfl_xor(sum, 32);
  const float r = 1.0f / sum;
  uint16_t* orow = out + base + static_cast<int64_t>(q0 + l32) * ld;
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      u32x2_t w;
      w[0] = pack2<T>(acc_o[dt][4 * gq] * r, acc_o[dt][4 * gq + 1] * r);
      w[1] = pack2<T>(acc_o[dt][4 * gq + 2] * r, acc_o[dt][4 * gq + 3] * r);
      *reinterpret_cast<u32x2_t*>(orow + 32 * dt + 8 * gq + 4 * hi) = w;
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace fh

using namespace fh;

extern "C" int32_t fh_attention_supported(int32_t dtype, int64_t seq, int64_t dh) {
  return (dtype == FH_BF16 || dtype == FH_F16) && dh == kDh && seq >= 64 && seq <= kMaxSeq && seq % 64 == 0 ? 1 : 0;
}

extern "C" fh_status fh_attention_fwd(int32_t dtype, const void* q, const void* k, const void* v, void* out, int64_t batch,
                                      int64_t seq, int64_t heads, int64_t dh, float scale, void* stream) {
  if (!fh_attention_supported(dtype, seq, dh))
    return fail(FH_UNIMPLEMENTED, "fh_attention_fwd: needs bf16/f16, head dim 64, seq a multiple of 64 up to 512");
  if (batch < 0 || heads < 1 || batch > 65535 || heads > 65535) return fail(FH_INVALID_ARGUMENT, "fh_attention_fwd: bad batch/heads");
  if (batch == 0) return FH_OK;
  if (q == nullptr || k == nullptr || v == nullptr || out == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_attention_fwd: null pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v)) return fail(FH_INVALID_ARGUMENT, "fh_attention_fwd: q/k/v must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const auto* qq = static_cast<const uint16_t*>(q);
  const auto* kk = static_cast<const uint16_t*>(k);
  const auto* vv = static_cast<const uint16_t*>(v);
  auto* oo = static_cast<uint16_t*>(out);
  const int nb = static_cast<int>(seq / 64);
  const int w = seq % 128 == 0 ? 4 : 2;
  const dim3 grid(static_cast<uint32_t>(seq / (32 * w)), static_cast<uint32_t>(heads), static_cast<uint32_t>(batch));
  const bool bf = dtype == FH_BF16;
  const int hd = static_cast<int>(heads);
  int e2 = 0;
  const bool pow2 = std::isfinite(scale) && scale > 0.0f && std::frexp(scale, &e2) == 0.5f && e2 > -60 && e2 < 60;
  auto go = [&]<int NB>() {
    constexpr int W = (NB * 64) % 128 == 0 ? 4 : 2;
    auto launch = [&]<typename T, bool P>() {
      hipLaunchKernelGGL((attention_kernel<T, NB, W, P>), grid, dim3(W * 64), 0, s, qq, kk, vv, oo, hd, scale);
    };
    if (bf) {
      if (pow2) launch.template operator()<bf16_t, true>(); else launch.template operator()<bf16_t, false>();
    } else {
      if (pow2) launch.template operator()<f16_t, true>(); else launch.template operator()<f16_t, false>();
    }
  };
  switch (nb) {
    case 1: go.template operator()<1>(); break;
    case 2: go.template operator()<2>(); break;
    case 3: go.template operator()<3>(); break;
    case 4: go.template operator()<4>(); break;
    case 5: go.template operator()<5>(); break;
    case 6: go.template operator()<6>(); break;
    case 7: go.template operator()<7>(); break;
    default: go.template operator()<8>(); break;
  }
  (void)w;
  return launch_status("attention_kernel launch");
}
