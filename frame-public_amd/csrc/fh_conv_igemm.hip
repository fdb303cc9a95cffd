// Conv2d as an implicit GEMM on MFMA, over channels-last operands (reference semantics:
// src/backends/cpu/kernels/conv.cpp:223-314 — out = round(sum_{ci,kh,kw} x*w + bias[co]) in fp32, then the
// fused elementwise chain).
//
// The graph keeps Frame's NCHW layout. HipBackend::compile lowers an eligible conv2d to
//   x_nhwc = transpose_batched(x: batch N,    [Cin][H*W]   -> [H*W][Cin])
//   w_khwc = transpose_batched(w: batch Cout, [Cin][KH*KW] -> [KH*KW][Cin])
//   y      = conv2d_nhwc(x_nhwc, w_khwc, bias)   (y written NCHW)
// so the transposed tensors are ordinary arena intermediates of the memory plan.
//
// GEMM view: M = Cout, N = P = batch*Ho*Wo output pixels, K = KH*KW*Cin ordered (kh, kw, ci). Every stage is
// one 64-byte row per operand row: 32 channels (bf16/f16, Cin % 32 == 0) or 16 (fp32, Cin % 16 == 0) of one
// filter position (kh, kw), so both operands are k-contiguous 64-byte rows:
//  * A rows = w_khwc[co] (row-major [Cout][K]), loaded with global_load_lds_dwordx4 like the GEMM's A;
//  * B rows = one output pixel's receptive-field slice x_nhwc[img, oh*sh-ph+kh, ow*sw-pw+kw, ci0..ci0+31],
//    loaded with buffer_load_dwordx4 ... lds. Positions in the zero padding get an offset past the buffer's
//    size, and the buffer bounds check returns zeros, so padding costs nothing.
// Both operands use the A-operand LDS layout ([rows][32 k], 16-byte chunks XOR-swizzled) and ds_read_b128
// fragments. The main loop is the same software pipeline as the bf16 GEMM (fh_gemm16.hip): a 4-stage ring
// refilled three stages ahead, fragment reads of the next k16 half interleaved with the current half's MFMAs,
// one barrier per stage. The filter position (kh, kw, ci0) of the next stage to load advances with scalar
// counters, not divisions.
//
// C8 mode (Cin <= 8, e.g. an RGB stem): x is packed channels-last with the channels zero-padded to 8, so one
// 16-byte chunk is one filter position's 8 channels, and a BK = 32 stage covers four consecutive filter positions
// (K = KH*KW*8 rounded up to 32, the filter packed to match with zeros). Each B-load lane then follows its own
// filter position, advancing by four per stage; positions past KH*KW load zeros like the padding does.
//
// Epilogue: bias is added to the fp32 accumulator, the sum is rounded once, the chain runs on the rounded
// value (rounding after every segment), and the tile is written NCHW — 16-byte stores along the pixel axis
// when Ho*Wo % 8 == 0, element stores otherwise.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>
#include <type_traits>
#include <utility>

#include "fh_common.h"
#include "fh_gemm.h"
#include "fh_mfma16.h"

namespace fh {
namespace {

using namespace mfma16;

struct ConvNhwcArgs {
  const void* x;     // [N][H][W][Cin]
  const void* w;     // [Cout][KH][KW][Cin]
  const void* bias;  // [Cout] or nullptr
  void* y;           // [N][Cout][Ho][Wo]
  int32_t cin, h, w_in, cout, kh, kw, sh, sw, ph, pw, wo, howo;
  int32_t k;         // KH*KW*Cin
  int64_t p;         // N*Ho*Wo
  uint32_t x_bytes;
  int32_t tiles_m, tiles_n;
  int32_t vec_store;  // NCHW: Ho*Wo % V == 0; NHWC: Cout % V == 0; and 16-byte aligned output / epilogue operands
  int32_t out_nhwc;   // 1: y (and the epilogue operands) are [N][Ho][Wo][Cout]
  EpilogueArgs ep;
  float* part;        // split K (kEpiSplitK instances): fp32 partial sums [gridDim.y][P][Cout]
  int32_t kt_split;   // split K: k stages per split
};

// Epilogue "program" of the split-K instances: the workgroup of split s writes its fp32 sums over k stages
// [s * kt_split, (s + 1) * kt_split) to part[s] instead of running an epilogue; conv_split_reduce_kernel sums the
// splits in order and runs the real epilogue. Distinct from every EpiKind.
constexpr int kEpiSplitK = 6;

template <int TM, int TN>
struct KFragments {
  u32x4_t a[TM];
  u32x4_t b[TN];
};

template <int TM, int TN>
__device__ __forceinline__ void fence_kfragments(KFragments<TM, TN>& f) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < TM; ++i) asm volatile("" : "+v"(f.a[i]));
#pragma unroll
  for (int j = 0; j < TN; ++j) asm volatile("" : "+v"(f.b[j]));
}
// Word j (a constant after unrolling) of a 16-byte vector.
__device__ __forceinline__ uint32_t uint4_word(const uint4& v, int j) {
  return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w;
}
// Ties the fragment registers to the preceding wait (no consumer is scheduled above it), as fence_kfragments does
// after its full wait.
template <int TM, int TN>
__device__ __forceinline__ void tie_kfragments(KFragments<TM, TN>& f) {
#pragma unroll
  for (int i = 0; i < TM; ++i) asm volatile("" : "+v"(f.a[i]));
#pragma unroll
  for (int j = 0; j < TN; ++j) asm volatile("" : "+v"(f.b[j]));
}
// s_waitcnt with only lgkmcnt constrained (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[15:14]).
template <int N>
__device__ __forceinline__ void wait_lgkmcnt() {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  __builtin_amdgcn_s_waitcnt(0xc07f | (N << 8));
}

// Writes one wave's accumulator tile (output channels m0w.. m0w+WM-1, output pixels n0w.. n0w+WN-1): bias added to
// the fp32 sum, one rounding, the fused chain on the rounded value, stored NCHW or channels-last (args.out_nhwc),
// staged through `lds` (LDS_BYTES of LDS the caller no longer needs; each wave uses its own slice).
template <typename T, int E, int WM, int WN, int NW, int LDS_BYTES>
__device__ __forceinline__ void conv_store_tile(const ConvNhwcArgs& args, f32x16_t (&acc)[WM / 32][WN / 32],
                                                unsigned char* lds, int wave, int lane, int m0w, int64_t n0w,
                                                const float* bias_lds = nullptr) {
  using S = typename Io<T>::storage;
  constexpr int ES = static_cast<int>(sizeof(S));
  constexpr int V = 16 / ES;
  constexpr int TM = WM / 32, TN = WN / 32;
  const int l32 = lane & 31, hi = lane >> 5;
  S* __restrict__ Y = static_cast<S*>(args.y);
  const S* bias = static_cast<const S*>(args.bias);
  // The bias of every accumulator row of this lane. Lane l loads row l of the wave tile (one coalesced load per
  // wave) and the rows each lane needs are exchanged across lanes. Every workgroup reads the same few bias lines:
  // sixteen 2-byte gathers per lane, as a per-row load would issue, pile up on one L2 channel (measured: 5-15 us of
  // a 30 us C3 conv spent waiting for them).
  static_assert(WM <= 64, "one bias row per lane");
  float bv[TM][16];
  {
    // bias_lds: the kernel staged the whole bias as floats in LDS (no global access in its epilogue)
    const int brow = min(m0w + lane % WM, args.cout - 1);
    const float mine = bias_lds != nullptr ? bias_lds[brow] : bias != nullptr ? Io<T>::load(bias[brow]) : 0.0f;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int x = 0; x < 16; ++x) bv[i][x] = __shfl(mine, i * 32 + 8 * (x >> 2) + 4 * hi + (x & 3));
  }
  if (args.out_nhwc) {
    // Channels-last output. The wave tile is staged pixel-major: pixel pc's WM channels are a row of PITCH
    // elements (padded by one 16-byte chunk so the 32 pixels of one accumulator register spread over the banks),
    // written two channels at a time. Then lane -> (pixel, group g of V channels) with g fastest: each lane reads
    // 16 contiguous bytes and consecutive lanes write consecutive 16-byte chunks of a pixel's channel run.
    constexpr int PITCH = WM + V;
    constexpr int GPW = WM / V;
    static_assert((WN * GPW) % 64 == 0, "whole waves of (pixel, channel group) pairs");
    // configurations whose pixel-major staging would not fit the ring are never launched with out_nhwc
    // (launch_conv refuses them)
    if constexpr (NW * WN * PITCH * ES <= LDS_BYTES) {
    S* wl = reinterpret_cast<S*>(lds + wave * (WN * PITCH * ES));
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int x = 0; x < 16; x += 2) {
        const int rr = i * 32 + 8 * (x >> 2) + 4 * hi + (x & 3);  // even: rows rr, rr + 1 are registers x, x + 1
        const float b0 = bv[i][x], b1 = bv[i][x + 1];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          S* dst = wl + (j * 32 + l32) * PITCH + rr;
          if constexpr (ES == 2) {
            *reinterpret_cast<uint32_t*>(dst) = epi_stage2<E, T>(acc[i][j][x] + b0, acc[i][j][x + 1] + b1);
          } else {
            dst[0] = epi_stage<E, T>(acc[i][j][x] + b0);
            dst[1] = epi_stage<E, T>(acc[i][j][x + 1] + b1);
          }
        }
      }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    constexpr int EA = epi_after_stage<E>();
    constexpr int ITERS = WN * GPW / 64;
    if constexpr (EA != kEpiAny) {
      if (args.vec_store) {
        // every operand load issued before the first is used and no wait between the stores (a wait for one
        // iteration's operand would also wait for the previous iteration's store)
        constexpr int NOP = epi_operands<EA>() > 0 ? epi_operands<EA>() : 1;
        uint4 in[ITERS][NOP];
        if constexpr (epi_operands<EA>() > 0) {
#pragma unroll
          for (int it = 0; it < ITERS; ++it) {
            const int id = it * 64 + lane;
            const int co0 = min(m0w + (id % GPW) * V, args.cout - V);
            const int64_t p = min(n0w + id / GPW, args.p - 1);
            epi_load<EA, T>(args.ep, p * args.cout + co0, in[it]);
          }
        }
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
          const int id = it * 64 + lane;
          const int g = id % GPW, pc = id / GPW;
          const int co0 = m0w + g * V;
          const int64_t p = n0w + pc;
          if (co0 < args.cout && p < args.p) {
            const uint4 packed = *reinterpret_cast<const uint4*>(wl + pc * PITCH + g * V);
            *reinterpret_cast<uint4*>(Y + p * args.cout + co0) = epi_apply<EA, T>(args.ep, packed, in[it]);
          }
        }
        return;
      }
    }
#pragma unroll 2
    for (int it = 0; it < ITERS; ++it) {
      const int id = it * 64 + lane;
      const int g = id % GPW, pc = id / GPW;
      const int co0 = m0w + g * V;
      const int64_t p = n0w + pc;
      if (co0 >= args.cout || p >= args.p) continue;
      uint4 packed = *reinterpret_cast<const uint4*>(wl + pc * PITCH + g * V);
      const int64_t idx = p * args.cout + co0;
      if (args.vec_store && co0 + V <= args.cout) {
        packed = epi_vec<EA, T>(args.ep, packed, idx);
        *reinterpret_cast<uint4*>(Y + idx) = packed;
      } else {
        S vals[V];
        __builtin_memcpy(vals, &packed, 16);
        for (int e = 0; e < V && co0 + e < args.cout; ++e) {
          S v = vals[e];
          if constexpr (EA != kEpiNone) v = Io<T>::store(epi_one<EA, T>(args.ep, Io<T>::load(v), idx + e));
          Y[idx + e] = v;
        }
      }
    }
    }
    return;
  }
  constexpr int WTILE_BYTES = WM * WN * ES;
  static_assert(NW * WTILE_BYTES <= LDS_BYTES, "the wave tiles fit in the LDS space");
  S* wl = reinterpret_cast<S*>(lds + wave * WTILE_BYTES);
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int x = 0; x < 16; ++x) {
      const int rr = i * 32 + 8 * (x >> 2) + 4 * hi + (x & 3);
#pragma unroll
      for (int j = 0; j < TN; ++j) wl[rr * WN + j * 32 + l32] = epi_stage<E, T>(acc[i][j][x] + bv[i][x]);
    }
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();
  constexpr int LPR = WN / V;
  constexpr int RPI = 64 / LPR;
  static_assert(64 % LPR == 0 && WM % RPI == 0, "epilogue access shape");
  const int c = (lane % LPR) * V;
  const int64_t p0 = n0w + c;
  constexpr int EA = epi_after_stage<E>();
  // the lane's 8 pixels lie in one image (vector path: Ho*Wo % 8 == 0): its output offset without the channel term
  const uint32_t img0 = static_cast<uint32_t>(p0) / static_cast<uint32_t>(args.howo);  // P < 2^31
  const int64_t base0 = static_cast<int64_t>(img0) * args.cout * args.howo +
                        (static_cast<uint32_t>(p0) - img0 * static_cast<uint32_t>(args.howo));
  constexpr int ITERS = WM / RPI;
  if constexpr (EA != kEpiAny) {
    if (args.vec_store && p0 + V <= args.p) {
      // operand loads first, then the stores with no wait between them (see the channels-last path)
      constexpr int NOP = epi_operands<EA>() > 0 ? epi_operands<EA>() : 1;
      uint4 in[ITERS][NOP];
      if constexpr (epi_operands<EA>() > 0) {
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
          const int co = min(m0w + it * RPI + lane / LPR, args.cout - 1);
          epi_load<EA, T>(args.ep, base0 + static_cast<int64_t>(co) * args.howo, in[it]);
        }
      }
#pragma unroll
      for (int it = 0; it < ITERS; ++it) {
        const int rr = it * RPI + lane / LPR;
        const int co = m0w + rr;
        if (co < args.cout) {
          const uint4 packed = *reinterpret_cast<const uint4*>(wl + rr * WN + c);
          *reinterpret_cast<uint4*>(Y + base0 + static_cast<int64_t>(co) * args.howo) =
              epi_apply<EA, T>(args.ep, packed, in[it]);
        }
      }
      return;
    }
  }
  for (int it = 0; it < ITERS; ++it) {
    const int rr = it * RPI + lane / LPR;
    const int co = m0w + rr;
    if (co >= args.cout || p0 >= args.p) continue;
    uint4 packed = *reinterpret_cast<const uint4*>(wl + rr * WN + c);
    if (args.vec_store && p0 + V <= args.p) {
      const int64_t idx = base0 + static_cast<int64_t>(co) * args.howo;
      packed = epi_vec<EA, T>(args.ep, packed, idx);
      *reinterpret_cast<uint4*>(Y + idx) = packed;
    } else {
      S vals[V];
      __builtin_memcpy(vals, &packed, 16);
      for (int e = 0; e < V && p0 + e < args.p; ++e) {
        const int64_t p = p0 + e;
        const int64_t img = p / args.howo;
        const int64_t idx = (img * args.cout + co) * args.howo + (p - img * args.howo);
        S v = vals[e];
        if constexpr (EA != kEpiNone) v = Io<T>::store(epi_one<EA, T>(args.ep, Io<T>::load(v), idx));
        Y[idx] = v;
      }
    }
  }
}

// NS: LDS ring depth (stages in flight NS - 1); deeper rings for launches of one workgroup per CU, whose loads have
// no other workgroup to hide behind.
template <typename T, int BM, int BN, int WAVES_M, int WAVES_N, bool C8, int E, int NS = kStages>
__global__ __launch_bounds__(WAVES_M* WAVES_N * 64) void conv_nhwc_kernel(ConvNhwcArgs args) {
  using S = typename Io<T>::storage;
  constexpr int ES = static_cast<int>(sizeof(S));
  constexpr int EPC = 16 / ES;     // elements per 16-byte chunk
  constexpr int KBK = 64 / ES;     // k per stage: one 64-byte row per operand row
  static_assert(!C8 || ES == 2, "the C8 layout is 16-bit");
  constexpr int NW = WAVES_M * WAVES_N;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int A_BYTES = BM * 64;
  constexpr int B_BYTES = BN * 64;
  constexpr int STAGE = A_BYTES + B_BYTES;
  constexpr int A_PER_WAVE = A_BYTES / 1024 / NW;
  constexpr int B_PER_WAVE = B_BYTES / 1024 / NW;
  constexpr int LOADS = A_PER_WAVE + B_PER_WAVE;
  static_assert((A_BYTES / 1024) % NW == 0 && A_PER_WAVE >= 1, "A stage loads split evenly over waves");
  static_assert((B_BYTES / 1024) % NW == 0 && B_PER_WAVE >= 1, "B stage loads split evenly over waves");
  static_assert(TM >= 1 && TN >= 1, "wave tile at least 32x32");
  static_assert((NS - 2) * LOADS <= 63, "vmcnt range");
  static_assert(NS >= 4 && (NS & (NS - 1)) == 0, "ring depth a power of two");

  __shared__ __attribute__((aligned(1024))) unsigned char ring[NS * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;

  const int tiles = args.tiles_m * args.tiles_n;
  int bid = blockIdx.x;
  if ((tiles & 7) == 0) bid = (bid & 7) * (tiles >> 3) + (bid >> 3);
  constexpr int GROUP_M = 8;
  const int group = bid / (GROUP_M * args.tiles_n);
  const int first_m = group * GROUP_M;
  const int gsize = min(args.tiles_m - first_m, GROUP_M);
  const int tm = first_m + (bid % gsize);
  const int tn = (bid % (GROUP_M * args.tiles_n)) / gsize;
  const int m0 = tm * BM;                              // first output channel of the tile
  const int64_t n0 = static_cast<int64_t>(tn) * BN;   // first output pixel of the tile

  const S* __restrict__ W = static_cast<const S*>(args.w);
  const int cin = args.cin, K = args.k;
  // stages [kt0, kt0 + KT) of the K / KBK: all of them, or this workgroup's split (kEpiSplitK)
  const int kt0 = E == kEpiSplitK ? static_cast<int>(blockIdx.y) * args.kt_split : 0;
  const int KT = E == kEpiSplitK ? min(args.kt_split, K / KBK - kt0) : K / KBK;
  static_assert(E != kEpiSplitK || !C8, "split K walks the filter positions of whole-channel stages");

  // ---- A (filter) sources: row co, clamped to the last channel ----
  int64_t a_src[A_PER_WAVE];
#pragma unroll
  for (int j = 0; j < A_PER_WAVE; ++j) {
    const int row = (wave * A_PER_WAVE + j) * 16 + (lane >> 2);
    const int chunk = (lane & 3) ^ a_swizzle(row);
    a_src[j] = static_cast<int64_t>(min(m0 + row, args.cout - 1)) * K + chunk * EPC;
  }
  // ---- B (im2col) sources: per load row, the pixel's window origin (element offset in x_nhwc, possibly
  // outside the image) and its top-left input coordinates ----
  int32_t b_org[B_PER_WAVE], b_ih[B_PER_WAVE], b_iw[B_PER_WAVE];
#pragma unroll
  for (int j = 0; j < B_PER_WAVE; ++j) {
    const int row = (wave * B_PER_WAVE + j) * 16 + (lane >> 2);
    const int chunk = (lane & 3) ^ a_swizzle(row);
    const int64_t p = min(n0 + row, args.p - 1);
    const int img = static_cast<int>(p / args.howo);
    const int rem = static_cast<int>(p - static_cast<int64_t>(img) * args.howo);
    const int oh = rem / args.wo, ow = rem - (rem / args.wo) * args.wo;
    b_ih[j] = oh * args.sh - args.ph;
    b_iw[j] = ow * args.sw - args.pw;
    b_org[j] = ((img * args.h + b_ih[j]) * args.w_in + b_iw[j]) * cin + (C8 ? 0 : chunk * EPC);
  }
  // C8 mode: filter position (kh, kw) of this lane's chunk in each B load, for the next stage to load
  // (stage s, chunk c -> position 4s + c); c8_live is false once the position is past KH*KW.
  int32_t c8_kh[B_PER_WAVE], c8_kw[B_PER_WAVE];
  if constexpr (C8) {
#pragma unroll
    for (int j = 0; j < B_PER_WAVE; ++j) {
      const int row = (wave * B_PER_WAVE + j) * 16 + (lane >> 2);
      const int c = (lane & 3) ^ a_swizzle(row);
      c8_kh[j] = 0;
      c8_kw[j] = c;
      while (c8_kw[j] >= args.kw) {
        c8_kw[j] -= args.kw;
        ++c8_kh[j];
      }
    }
  }
  const __amdgpu_buffer_rsrc_t xr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(args.x), static_cast<short>(0), static_cast<int>(args.x_bytes),
                                        0x00020000);

  // Filter position of the next stage to load; stays on the last stage once every stage has been issued.
  // ld_off = the stage's element offset from a window origin, (kh * W + kw) * Cin + ci0.
  int ld_kh = 0, ld_kw = 0, ld_ci = 0, ld_next = 0, ld_off = 0;
  if constexpr (E == kEpiSplitK) {
    const int k_first = kt0 * KBK, pos = k_first / cin;
    ld_ci = k_first - pos * cin;
    ld_kh = pos / args.kw;
    ld_kw = pos - ld_kh * args.kw;
    ld_off = (ld_kh * args.w_in + ld_kw) * cin + ld_ci;
  }
  auto advance = [&]() {
    if (ld_next + 1 < KT) {
      ++ld_next;
      if constexpr (C8) {
#pragma unroll
        for (int j = 0; j < B_PER_WAVE; ++j) {
          c8_kw[j] += 4;
          while (c8_kw[j] >= args.kw) {
            c8_kw[j] -= args.kw;
            ++c8_kh[j];
          }
        }
        return;
      }
      ld_ci += KBK;
      if (ld_ci == cin) {
        ld_ci = 0;
        if (++ld_kw == args.kw) {
          ld_kw = 0;
          ++ld_kh;
        }
      }
      ld_off = (ld_kh * args.w_in + ld_kw) * cin + ld_ci;
    }
  };

  // Load instruction J of this wave's share of stage kt (filter position = the ld_* counters).
  auto load_one = [&]<int J>(int kt) {
    unsigned char* st = ring + (kt & (NS - 1)) * STAGE;
    if constexpr (J < A_PER_WAVE) {
      const int64_t k0 = static_cast<int64_t>(kt0 + min(kt, KT - 1)) * KBK;
      global_to_lds16(W + a_src[J] + k0, (FH_LDS void*)(st + (wave * A_PER_WAVE + J) * 1024));
    } else {
      constexpr int JB = J - A_PER_WAVE;
      const int kh_ = C8 ? c8_kh[JB] : ld_kh, kw_ = C8 ? c8_kw[JB] : ld_kw;
      const int ih = b_ih[JB] + kh_, iw = b_iw[JB] + kw_;
      const bool inside = static_cast<unsigned>(ih) < static_cast<unsigned>(args.h) &&
                          static_cast<unsigned>(iw) < static_cast<unsigned>(args.w_in) && (!C8 || kh_ < args.kh);
      // computed unconditionally so the padding case is a select, not a branch
      const int off = C8 ? (kh_ * args.w_in + kw_) * cin : ld_off;
      const uint32_t at = static_cast<uint32_t>(b_org[JB] + off) * static_cast<uint32_t>(ES);
      const uint32_t voff = inside ? at : 0x80000000u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (FH_LDS void*)(st + A_BYTES + (wave * B_PER_WAVE + JB) * 1024), 16,
                                               static_cast<int>(voff), 0, 0, 0);
    }
  };
  auto issue_stage = [&](int kt) {
    [&]<int... J>(std::integer_sequence<int, J...>) {
      (load_one.template operator()<J>(kt), ...);
    }(std::make_integer_sequence<int, LOADS>{});
    advance();
  };

  const int l32 = lane & 31, hi = lane >> 5;
  int a_off[2], b_off[2];
  {
    const int arow = wm * WM + l32, brow = wn * WN + l32;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      a_off[s] = arow * 64 + (((2 * s + hi) ^ a_swizzle(arow)) * 16);
      b_off[s] = A_BYTES + brow * 64 + (((2 * s + hi) ^ a_swizzle(brow)) * 16);
    }
  }
  const uint32_t ring_addr = lds_addr((const FH_LDS void*)ring);

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int x = 0; x < 16; ++x) acc[i][j][x] = 0.0f;

  KFragments<TM, TN> f0, f1;
  constexpr int NREAD = TM + TN;
  constexpr int NMFMA = TM * TN;
  auto read_one = [&]<int H, int R>(uint32_t base, KFragments<TM, TN>& f) {
    if constexpr (R < TM) {
      f.a[R] = lds_read_b128<R * 2048>(base + a_off[H]);
    } else {
      f.b[R - TM] = lds_read_b128<(R - TM) * 2048>(base + b_off[H]);
    }
  };
  constexpr int R_SPAN = NMFMA * 3 / 4 > 0 ? NMFMA * 3 / 4 : 1;
  constexpr int L_SPAN = NMFMA / 2 > 0 ? NMFMA / 2 : 1;
  auto multiply_and_read = [&]<int H, bool LOADS_TOO>(KFragments<TM, TN>& cur, uint32_t base,
                                                      KFragments<TM, TN>& nxt, int load_kt) {
    [&]<int... M_>(std::integer_sequence<int, M_...>) {
      (
          [&] {
            constexpr int i = M_ / TN, j = M_ % TN;
            mfma32<T>(cur.a[i], cur.b[j], acc[i][j]);
            constexpr int r0 = first(M_, NREAD, R_SPAN);
            [&]<int... R_>(std::integer_sequence<int, R_...>) {
              (read_one.template operator()<H, r0 + R_>(base, nxt), ...);
            }(std::make_integer_sequence<int, share(M_, NREAD, R_SPAN)>{});
            if constexpr (LOADS_TOO) {
              constexpr int l0 = first(M_, LOADS, L_SPAN);
              [&]<int... L_>(std::integer_sequence<int, L_...>) {
                (load_one.template operator()<l0 + L_>(load_kt), ...);
              }(std::make_integer_sequence<int, share(M_, LOADS, L_SPAN)>{});
            }
            __builtin_amdgcn_sched_barrier(0);
          }(),
          ...);
    }(std::make_integer_sequence<int, NMFMA>{});
  };

#pragma unroll
  for (int st = 0; st < NS - 1; ++st) issue_stage(st);
  wait_vmcnt<(NS - 2) * LOADS>();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  [&]<int... R_>(std::integer_sequence<int, R_...>) {
    (read_one.template operator()<0, R_>(ring_addr, f0), ...);
  }(std::make_integer_sequence<int, NREAD>{});

  for (int kt = 0; kt < KT; ++kt) {
    const uint32_t cur = ring_addr + (kt & (NS - 1)) * STAGE;
    const uint32_t nxt = ring_addr + ((kt + 1) & (NS - 1)) * STAGE;
    fence_kfragments(f0);
    multiply_and_read.template operator()<1, false>(f0, cur, f1, 0);
    wait_vmcnt<(NS - 3) * LOADS>();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    fence_kfragments(f1);
    multiply_and_read.template operator()<0, true>(f1, nxt, f0, kt + NS - 1);
    advance();
  }
  // The last step read the next half's fragments (past the end: unused). Those LDS reads are still in flight
  // and would write their registers after the compiler has reused them in the epilogue, so they are fenced with
  // the registers tied before anything else may use them.
  fence_kfragments(f0);

  // ---- epilogue ----
  wait_vmcnt<0>();
  if constexpr (E == kEpiSplitK) {
    // fp32 partials, channels-last: registers 4q .. 4q + 3 of accumulator (i, j) are channels
    // i * 32 + 8 q + 4 hi .. + 3 of pixel j * 32 + l32, one 16-byte store (Cout % 64 == 0: whole channel tiles)
    float* __restrict__ part = args.part + static_cast<int64_t>(blockIdx.y) * args.p * args.cout;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int64_t p = n0 + wn * WN + j * 32 + l32;
        if (p >= args.p) continue;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int co = m0 + wm * WM + i * 32 + 8 * q + 4 * hi;
          *reinterpret_cast<float4*>(part + p * args.cout + co) =
              make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
        }
      }
    return;
  } else {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __syncthreads();
    conv_store_tile<T, E, WM, WN, NW, NS * STAGE>(args, acc, ring, wave, lane, m0 + wm * WM, n0 + wn * WN);
  }
}

// The second launch of a split-K convolution (16-bit, channels-last output): one thread per 8 channels of one
// pixel sums the splits' fp32 partials in split order, adds the bias, rounds once and runs the epilogue program on
// the rounded values, as conv_store_tile does for an unsplit tile.
template <typename T, int E>
__global__ __launch_bounds__(256) void conv_split_reduce_kernel(ConvNhwcArgs args, int32_t splits) {
  using S = typename Io<T>::storage;
  static_assert(sizeof(S) == 2, "16-bit outputs");
  const int groups = args.cout / 8;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (gid >= args.p * groups) return;
  const int64_t p = gid / groups;
  const int co0 = static_cast<int>(gid - p * groups) * 8;
  const int64_t idx = p * args.cout + co0, stride = args.p * args.cout;
  float v[8];
  {
    const float4* src = reinterpret_cast<const float4*>(args.part + idx);
    const float4 a = src[0], b = src[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
  for (int s = 1; s < splits; ++s) {
    const float4* src = reinterpret_cast<const float4*>(args.part + s * stride + idx);
    const float4 a = src[0], b = src[1];
    v[0] += a.x; v[1] += a.y; v[2] += a.z; v[3] += a.w; v[4] += b.x; v[5] += b.y; v[6] += b.z; v[7] += b.w;
  }
  if (args.bias != nullptr) {
    const uint4 braw = *reinterpret_cast<const uint4*>(static_cast<const S*>(args.bias) + co0);
    float bv[8];
    unpack_vec<T>(braw, bv);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] += bv[e];
  }
  uint4 packed;
  packed.x = epi_stage2<E, T>(v[0], v[1]);
  packed.y = epi_stage2<E, T>(v[2], v[3]);
  packed.z = epi_stage2<E, T>(v[4], v[5]);
  packed.w = epi_stage2<E, T>(v[6], v[7]);
  constexpr int EA = epi_after_stage<E>();
  *reinterpret_cast<uint4*>(static_cast<S*>(args.y) + idx) = epi_vec<EA, T>(args.ep, packed, idx);
}

// Whether a configuration can stage its wave tiles pixel-major (channels-last output) in its LDS ring.
template <typename T, int BM, int BN, int WAVES_M, int WAVES_N>
constexpr bool nhwc_out_fits() {
  constexpr int es = static_cast<int>(sizeof(typename Io<T>::storage));
  constexpr int wm = BM / WAVES_M, wn = BN / WAVES_N;
  return WAVES_M * WAVES_N * wn * (wm + 16 / es) * es <= kStages * (BM + BN) * 64;
}

// Runs f.template operator()<E>() with the fixed epilogue program of `kind` when bit E of MASK allows it, else
// with kEpiAny (the instantiations each kernel family carries are listed by its MASK).
template <unsigned MASK, typename F>
fh_status with_epi(int kind, F&& f) {
  switch (kind) {
    case kEpiNone:
      if constexpr ((MASK >> kEpiNone) & 1) return f.template operator()<kEpiNone>();
      break;
    case kEpiRelu:
      if constexpr ((MASK >> kEpiRelu) & 1) return f.template operator()<kEpiRelu>();
      break;
    case kEpiAddRelu:
      if constexpr ((MASK >> kEpiAddRelu) & 1) return f.template operator()<kEpiAddRelu>();
      break;
    default:
      break;
  }
  return f.template operator()<kEpiAny>();
}

// bf16 (the configurations' type) gets the ResNet programs as their own kernels; other types the interpreter.
template <typename T, bool C8>
constexpr unsigned conv_epi_mask() {
  if constexpr (!std::is_same_v<T, bf16_t>) return 0;
  else if constexpr (C8) return 1u << kEpiRelu;
  else return (1u << kEpiNone) | (1u << kEpiRelu) | (1u << kEpiAddRelu);
}

template <typename T, int BM, int BN, int WAVES_M, int WAVES_N, bool C8>
fh_status launch_conv(ConvNhwcArgs a, hipStream_t stream) {
  if (a.out_nhwc && !nhwc_out_fits<T, BM, BN, WAVES_M, WAVES_N>())
    return fail(FH_INTERNAL, "conv_nhwc_kernel: channels-last output does not fit this tile configuration");
  a.tiles_m = (a.cout + BM - 1) / BM;
  a.tiles_n = static_cast<int32_t>((a.p + BN - 1) / BN);
  const dim3 grid(static_cast<uint32_t>(a.tiles_m) * static_cast<uint32_t>(a.tiles_n));
  return with_epi<conv_epi_mask<T, C8>()>(epi_kind(a.ep), [&]<int E>() {
    hipLaunchKernelGGL((conv_nhwc_kernel<T, BM, BN, WAVES_M, WAVES_N, C8, E>), grid, dim3(WAVES_M * WAVES_N * 64), 0,
                       stream, a);
    return launch_status("conv_nhwc_kernel launch");
  });
}

// Split-K launch (16-bit, channels-last output, Cout % BM == 0): gridDim.y = splits workgroups per tile, each over
// kt_split consecutive k stages, then the reduction with the epilogue. The caller sized a.part for `splits`
// (split_count below gives the count that leaves no split empty).
template <typename T, int BM, int BN, int WAVES_M, int WAVES_N, int NS = kStages>
fh_status launch_conv_split(ConvNhwcArgs a, int32_t splits, hipStream_t stream) {
  a.tiles_m = a.cout / BM;
  a.tiles_n = static_cast<int32_t>((a.p + BN - 1) / BN);
  const int32_t kt = a.k / 32;
  a.kt_split = (kt + splits - 1) / splits;
  hipLaunchKernelGGL((conv_nhwc_kernel<T, BM, BN, WAVES_M, WAVES_N, false, kEpiSplitK, NS>),
                     dim3(static_cast<uint32_t>(a.tiles_m) * static_cast<uint32_t>(a.tiles_n), static_cast<uint32_t>(splits)),
                     dim3(WAVES_M * WAVES_N * 64), 0, stream, a);
  if (const fh_status st = launch_status("conv_nhwc_kernel launch (split K)"); st != FH_OK) return st;
  const int64_t threads = a.p * (a.cout / 8);
  return with_epi<conv_epi_mask<T, false>()>(epi_kind(a.ep), [&]<int E>() {
    hipLaunchKernelGGL((conv_split_reduce_kernel<T, E>), dim3(static_cast<uint32_t>((threads + 255) / 256)), dim3(256), 0,
                       stream, a, splits);
    return launch_status("conv_split_reduce_kernel launch");
  });
}

// Splits that leave none empty: ceil(kt / ceil(kt / want)).
int32_t split_count(int32_t kt, int32_t want) {
  const int32_t per = (kt + want - 1) / want;
  return (kt + per - 1) / per;
}

// ---- 3x3 stride-1 convolutions with the input patch resident in LDS -------------------------------------------
//
// For KH = KW = 3, stride 1, padding 1 (output plane = input plane), 16-bit, Cin % 32 == 0, Cout <= 512. A tile is
// 64 output channels x BN consecutive output pixels (flattened n, oh, ow). Those pixels cover a band of output
// rows; the input they read is that band plus one halo row above and below, addressed by global input row
// gi = n * H + ih, each row W + 2 positions wide (the two padding columns are zeros). For each chunk of 32 input
// channels the workgroup loads the patch [rows][W + 2][32 ch] once and runs all 9 taps out of LDS: the B
// fragment of output pixel (band row r, column c) for tap (kh, kw) is patch position (r + kh) * (W + 2) + c + kw.
// The implicit GEMM streams one 64-byte im2col row per pixel and tap (every input byte crosses L2 -> LDS 9 times,
// as half cache lines); here each crosses about (rows + 2) / rows times, in contiguous runs of whole lines. A tap
// whose input row falls outside the pixel's own image (the first and last rows of every image; the patch holds
// the neighbouring image's row there) reads three zero positions kept after the patch instead. Positions use the
// A layout's 16-byte chunk swizzle.
//
// The kernel is persistent: one workgroup per CU walks tiles blockIdx.x, blockIdx.x + gridDim.x, ..., and its
// (tile, chunk) steps form one double-buffered pipeline, so the next step's loads (the next tile's first patch
// included) are in flight while a step is multiplied and while a finished tile is written out. RES_A (Cout <= 64,
// Cin <= 64): the whole filter, [chunk][tap][64 rows][32 ch], is loaded once and stays in LDS; otherwise each step
// also loads its 64 filter rows for the 9 taps of the chunk. The bias is staged in LDS once, so a tile's epilogue
// reads no global memory and never waits behind the loads in flight.
struct ConvHaloArgs {
  ConvNhwcArgs c;
  int32_t rw;          // W + 2: positions per patch row
  int32_t p_loads;     // 1 KB LDS-DMA loads that fill the patch positions this geometry needs
  int32_t rows_total;  // N * H: global input rows
  int32_t tiles;       // tiles_m * tiles_n
  int32_t patch_rows;  // rows of the patch a BN-pixel tile reads (NCHW input fill)
};

constexpr int kHaloPatchBytes = 30 * 1024;

constexpr int kHaloResidentCin = 64;  // RES_A: the filter of Cout <= 64, Cin <= 64 (72 KB) stays in LDS

template <typename T, int BN, bool RES_A, int E>
__global__ __launch_bounds__(512) void conv_halo_kernel(ConvHaloArgs ha) {
  const ConvNhwcArgs& args = ha.c;
  using S = typename Io<T>::storage;
  static_assert(sizeof(S) == 2, "16-bit operands");
  constexpr int BM = 64, WAVES_M = 2, WAVES_N = 4, NW = 8;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int TAPS = 9;
  constexpr int A_CHUNK = TAPS * BM * 64;                       // one chunk's filter rows
  constexpr int A_RES = RES_A ? (kHaloResidentCin / 32) * A_CHUNK : 0;
  constexpr int A_STEP = RES_A ? 0 : A_CHUNK;                   // filter bytes loaded with every step
  constexpr int A_LOADS = A_CHUNK / 1024;
  constexpr int A_PER_WAVE = (A_LOADS + NW - 1) / NW;
  constexpr int P_MAX = kHaloPatchBytes / 1024;
  constexpr int P_PER_WAVE = (P_MAX + NW - 1) / NW;
  constexpr int STAGE_BYTES = NW * WN * (WM + 8) * 2;  // conv_store_tile's channels-last staging (the larger)
  constexpr int SB_USED = A_STEP + kHaloPatchBytes > STAGE_BYTES ? A_STEP + kHaloPatchBytes : STAGE_BYTES;
  // one step buffer: [filter rows (!RES_A)][patch] (or the epilogue's staging), then three zero positions at its
  // end, which neither the loads nor the staging touch
  constexpr int SB = (SB_USED + 3 * 64 + 1023) / 1024 * 1024;
  constexpr int ZERO_OFF = SB - 256;
  constexpr int ZERO_POS = (ZERO_OFF - A_STEP) / 64;  // patch position index of the zero positions
  static_assert(ZERO_OFF >= SB_USED && (ZERO_OFF - A_STEP) % 64 == 0, "zero positions after loads and staging");
  constexpr int NSTORE = WM * WN / 512;  // 16-byte stores per lane of a full tile (conv_store_tile, vector path)
  constexpr int BIAS_OFF = A_RES + 2 * SB;
  static_assert(A_CHUNK % 1024 == 0 && kHaloPatchBytes % 1024 == 0, "whole 1 KB loads");
  static_assert(BIAS_OFF + 512 * 4 <= 160 * 1024, "LDS budget");

  __shared__ __attribute__((aligned(1024))) unsigned char lds[BIAS_OFF + 512 * 4];
  float* bias_lds = reinterpret_cast<float*>(lds + BIAS_OFF);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int l32 = lane & 31, hi = lane >> 5;
  const int W = args.w_in, H = args.h, cin = args.cin, rw = ha.rw;
  const int nchunks = cin / 32;
  const S* __restrict__ Wt = static_cast<const S*>(args.w);
  const __amdgpu_buffer_rsrc_t xr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(args.x), static_cast<short>(0), static_cast<int>(args.x_bytes),
                                        0x00020000);

  // tile -> (m0, n0): channel tiles fastest, so consecutive tiles of a workgroup share pixels
  auto tile_m0 = [&](int t) { return (t % args.tiles_m) * BM; };
  auto tile_n0 = [&](int t) { return static_cast<int64_t>(t / args.tiles_m) * BN; };

  // ---- load side: sources of this wave's loads for a (tile, chunk) step ----
  // patch position of load i, lane: fixed over tiles; only the band's first global row changes
  int p_r[P_PER_WAVE], p_c[P_PER_WAVE], p_ch[P_PER_WAVE];
#pragma unroll
  for (int i = 0; i < P_PER_WAVE; ++i) {
    const int q = (wave + NW * i) * 16 + (lane >> 2);
    p_ch[i] = ((lane & 3) ^ ((q >> 2) & 3)) * 8;
    p_r[i] = q / rw;
    p_c[i] = q - p_r[i] * rw;
  }
  auto a_row_src = [&](int j, int m0) {  // element offset (without ci0) of filter load j, this lane
    const int tap = j / (BM / 16);
    const int row = (j % (BM / 16)) * 16 + (lane >> 2);
    const int gch = (lane & 3) ^ a_swizzle(row);
    return (min(m0 + row, args.cout - 1) * TAPS + tap) * cin + gch * 8;
  };
  // issue the loads of step (tile t, chunk c) into step buffer b
  auto issue_step = [&](int t, int c, int b) {
    unsigned char* base = lds + A_RES + b * SB;
    const int ci0 = c * 32;
    if constexpr (!RES_A) {
      const int m0 = tile_m0(t);
#pragma unroll
      for (int i = 0; i < A_PER_WAVE; ++i) {
        const int j = wave + NW * i;
        if (j < A_LOADS) global_to_lds16(Wt + a_row_src(j, m0) + ci0, (FH_LDS void*)(base + j * 1024));
      }
    }
    const int gi_lo = static_cast<int>(tile_n0(t) / W) - 1;
#pragma unroll
    for (int i = 0; i < P_PER_WAVE; ++i) {
      const int j = wave + NW * i;
      if (j < ha.p_loads) {
        const int gi = gi_lo + p_r[i];
        const bool ok = gi >= 0 && gi < ha.rows_total && p_c[i] >= 1 && p_c[i] <= W;
        const uint32_t voff = ok ? static_cast<uint32_t>((gi * W + p_c[i] - 1) * cin + p_ch[i] + ci0) * 2u : 0x80000000u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (FH_LDS void*)(base + A_STEP + j * 1024), 16,
                                                 static_cast<int>(voff), 0, 0, 0);
      }
    }
  };

  // ---- compute side: fragment addresses of the tile being multiplied ----
  int a_off[TM][2];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int arow = wm * WM + i * 32 + l32;
#pragma unroll
    for (int h = 0; h < 2; ++h) a_off[i][h] = arow * 64 + (((2 * h + hi) ^ a_swizzle(arow)) * 16);
  }
  int rowpos[TN][3];
  auto set_tile = [&](int t) {  // B: patch position of tap (kh, 0) per n-tile, or ZERO_POS outside the image
    const int64_t n0 = tile_n0(t);
    const int gr_first = static_cast<int>(n0 / W);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t p = min(n0 + wn * WN + j * 32 + l32, args.p - 1);
      const int gr = static_cast<int>(p / W);
      const int ow = static_cast<int>(p - static_cast<int64_t>(gr) * W);
      const int oh = gr % H;
      const int pbase = (gr - gr_first) * rw + ow;
#pragma unroll
      for (int kh = 0; kh < 3; ++kh)
        rowpos[j][kh] = static_cast<unsigned>(oh + kh - 1) < static_cast<unsigned>(H) ? pbase + kh * rw : ZERO_POS;
    }
  };

  f32x16_t acc[TM][TN];
  auto clear_acc = [&]() {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int x = 0; x < 16; ++x) acc[i][j][x] = 0.0f;
  };

  // ---- prologue: zero positions, bias, the resident filter, the first step ----
  const int first = blockIdx.x;
  if (first >= ha.tiles) return;
  if (tid < 2 * 12) {
    const int b = tid / 12, k = tid % 12;
    *reinterpret_cast<uint4*>(lds + A_RES + b * SB + ZERO_OFF + k * 16) = uint4{0, 0, 0, 0};
  }
  if (tid < args.cout)
    bias_lds[tid] = args.bias != nullptr ? Io<T>::load(static_cast<const S*>(args.bias)[tid]) : 0.0f;
  if constexpr (RES_A) {
    for (int c = 0; c < nchunks; ++c)
#pragma unroll
      for (int i = 0; i < A_PER_WAVE; ++i) {
        const int j = wave + NW * i;
        if (j < A_LOADS) global_to_lds16(Wt + a_row_src(j, 0) + c * 32, (FH_LDS void*)(lds + c * A_CHUNK + j * 1024));
      }
  }
  issue_step(first, 0, 0);
  wait_vmcnt<0>();
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  const uint32_t lds_base = lds_addr((const FH_LDS void*)lds);
  KFragments<TM, TN> f0, f1, f2;
  auto read_step = [&]<int STEP>(uint32_t ab, uint32_t pb, KFragments<TM, TN>& f) {
    constexpr int tap = STEP / 2, h = STEP % 2, kh = tap / 3, kw = tap % 3;
#pragma unroll
    for (int i = 0; i < TM; ++i) f.a[i] = lds_read_b128<tap * BM * 64>(ab + a_off[i][h]);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int pos = rowpos[j][kh] + kw;
      f.b[j] = lds_read_b128<0>(pb + pos * 64 + ((((2 * h + hi) ^ ((pos >> 2) & 3))) * 16));
    }
  };
  auto multiply = [&](KFragments<TM, TN>& f) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) mfma32<T>(f.a[i], f.b[j], acc[i][j]);
  };

  clear_acc();
  set_tile(first);
  int t = first, c = 0, buf = 0;
  while (true) {
    // next step: the next chunk of this tile, or the first chunk of the next tile
    int nt = t, nc = c + 1;
    if (nc == nchunks) {
      nc = 0;
      nt = t + static_cast<int>(gridDim.x);
    }
    const bool more = nt < ha.tiles;
    if (more) issue_step(nt, nc, buf ^ 1);
    const uint32_t sb = lds_base + A_RES + buf * SB;
    const uint32_t ab = RES_A ? lds_base + c * A_CHUNK : sb;
    const uint32_t pb = sb + A_STEP;
    // fragments read two steps ahead (three buffers): before step s's MFMAs every LDS operation but step s+1's
    // reads (the last TM + TN issued; LDS operations complete in order) has completed
    read_step.template operator()<0>(ab, pb, f0);
    read_step.template operator()<1>(ab, pb, f1);
    [&]<int... STEP>(std::integer_sequence<int, STEP...>) {
      (
          [&] {
            constexpr int s = STEP;
            KFragments<TM, TN>& cur = (s % 3 == 0) ? f0 : (s % 3 == 1) ? f1 : f2;
            KFragments<TM, TN>& ahead = (s % 3 == 0) ? f2 : (s % 3 == 1) ? f0 : f1;
            if constexpr (s + 1 < 2 * TAPS) {
              wait_lgkmcnt<TM + TN>();
            } else {
              wait_lgkmcnt<0>();
            }
            tie_kfragments(cur);
            if constexpr (s + 2 < 2 * TAPS) read_step.template operator()<s + 2>(ab, pb, ahead);
            multiply(cur);
            __builtin_amdgcn_sched_barrier(0);
          }(),
          ...);
    }(std::make_integer_sequence<int, 2 * TAPS>{});
    fence_kfragments(f0);
    fence_kfragments(f1);
    fence_kfragments(f2);
    bool exact = true;  // the vmcnt wait below may leave this tile's NSTORE stores in flight
    if (c + 1 == nchunks) {
      // tile done: every wave has finished reading this step buffer, which then stages the output
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      const int m0 = tile_m0(t);
      const int64_t n0 = tile_n0(t);
      conv_store_tile<T, E, WM, WN, NW, SB>(args, acc, lds + A_RES + buf * SB, wave, lane, m0 + wm * WM,
                                            n0 + wn * WN, bias_lds);
      exact = args.vec_store && m0 + BM <= args.cout && n0 + BN <= args.p;
      clear_acc();
      if (more) set_tile(nt);
    }
    if (!more) break;
    if (exact) {
      wait_vmcnt<NSTORE>();
    } else {
      wait_vmcnt<0>();
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    t = nt;
    c = nc;
    buf ^= 1;
  }
}

// Channels-last output of a whole workgroup tile (BM = 64 channels x BN pixels): every wave stages its accumulators
// pixel-major into one shared [BN][BM + 8] layout, then eight consecutive lanes write a pixel's 64 channels as one
// 128-byte line. (Per-wave staging writes each pixel's channels in 32-channel halves from two different waves,
// half cache lines that cost the C4 layers a third of their time.) Ends with every wave past a barrier.
template <typename T, int E, int BM, int BN, int WAVES_N, int NW>
__device__ __forceinline__ void conv_store_tile_wg_nhwc(const ConvNhwcArgs& args, f32x16_t (&acc)[BM / (NW / WAVES_N) / 32][BN / WAVES_N / 32],
                                                        unsigned char* lds, int wave, int lane, int m0, int64_t n0) {
  using S = typename Io<T>::storage;
  static_assert(sizeof(S) == 2 && BM == 64, "16-bit, 64-channel tiles");
  constexpr int WAVES_M = NW / WAVES_N;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int PITCH = BM + 8;  // elements per staged pixel (one 16-byte pad chunk)
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int l32 = lane & 31, hi = lane >> 5;
  const S* bias = static_cast<const S*>(args.bias);
  float bv[TM][16];
  {
    const float mine = bias != nullptr ? Io<T>::load(bias[min(m0 + wm * WM + lane % WM, args.cout - 1)]) : 0.0f;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int x = 0; x < 16; ++x) bv[i][x] = __shfl(mine, i * 32 + 8 * (x >> 2) + 4 * hi + (x & 3));
  }
  S* st = reinterpret_cast<S*>(lds);
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int x = 0; x < 16; x += 2) {
      const int ch = wm * WM + i * 32 + 8 * (x >> 2) + 4 * hi + (x & 3);  // even; channels ch, ch + 1
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int pc = wn * WN + j * 32 + l32;
        *reinterpret_cast<uint32_t*>(st + pc * PITCH + ch) = epi_stage2<E, T>(acc[i][j][x] + bv[i][x], acc[i][j][x + 1] + bv[i][x + 1]);
      }
    }
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __syncthreads();
  const int tid = wave * 64 + lane;
  constexpr int ITERS = BN * 8 / (NW * 64);
  if constexpr (epi_after_stage<E>() != kEpiAny) {
    if (args.vec_store) {
      // operand loads first, then the stores with no wait between them (see conv_store_tile)
      constexpr int EA = epi_after_stage<E>();
      constexpr int NOP = epi_operands<EA>() > 0 ? epi_operands<EA>() : 1;
      S* __restrict__ Y = static_cast<S*>(args.y);
      uint4 in[ITERS][NOP];
      if constexpr (epi_operands<EA>() > 0) {
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
          const int id = it * NW * 64 + tid;
          const int co0 = min(m0 + (id & 7) * 8, args.cout - 8);
          const int64_t p = min(n0 + (id >> 3), args.p - 1);
          epi_load<EA, T>(args.ep, p * args.cout + co0, in[it]);
        }
      }
#pragma unroll
      for (int it = 0; it < ITERS; ++it) {
        const int id = it * NW * 64 + tid;
        const int g = id & 7, pc = id >> 3;
        const int co0 = m0 + g * 8;
        const int64_t p = n0 + pc;
        if (co0 < args.cout && p < args.p) {
          const uint4 packed = *reinterpret_cast<const uint4*>(st + pc * PITCH + g * 8);
          *reinterpret_cast<uint4*>(Y + p * args.cout + co0) = epi_apply<EA, T>(args.ep, packed, in[it]);
        }
      }
      return;
    }
  }
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    const int id = it * NW * 64 + tid;
    const int g = id & 7, pc = id >> 3;
    const int co0 = m0 + g * 8;
    const int64_t p = n0 + pc;
    if (co0 >= args.cout || p >= args.p) continue;
    uint4 packed = *reinterpret_cast<const uint4*>(st + pc * PITCH + g * 8);
    const int64_t idx = p * args.cout + co0;
    S* __restrict__ Y = static_cast<S*>(args.y);
    constexpr int EA = epi_after_stage<E>();
    if (args.vec_store && co0 + 8 <= args.cout) {
      packed = epi_vec<EA, T>(args.ep, packed, idx);
      *reinterpret_cast<uint4*>(Y + idx) = packed;
    } else {
      S vals[8];
      __builtin_memcpy(vals, &packed, 16);
      for (int e = 0; e < 8 && co0 + e < args.cout; ++e) {
        S v = vals[e];
        if constexpr (EA != kEpiNone) v = Io<T>::store(epi_one<EA, T>(args.ep, Io<T>::load(v), idx + e));
        Y[idx + e] = v;
      }
    }
  }
}

// Single-buffered variant: one tile per workgroup, each (chunk) step loaded, waited for and multiplied in turn,
// 66 KB of LDS, so two workgroups share a CU and each one's loads, barriers and epilogue overlap the other's
// multiplications (the persistent kernel above keeps one workgroup per CU and has nothing to overlap them with).
//
// NCHW_IN: x is NCHW [N][Cin][H][W] (W % 8 == 0), the layout a graph input arrives in, so no channels-last copy of
// the activations is made first. The patch of a chunk is then filled through registers: a thread takes 8
// channels x 8 consecutive pixels of one patch row (8 loads of 16 bytes, one per channel plane), transposes the
// 8 x 8 block of 16-bit values in registers, and writes 8 positions' 16-byte chunks of the channels-last patch;
// other threads zero the two padding positions of every row. Everything after the patch fill is unchanged.
template <typename T, int BN, int E, bool NCHW_IN>
__global__ __launch_bounds__(512, 4) void conv_halo1_kernel(ConvHaloArgs ha) {
  const ConvNhwcArgs& args = ha.c;
  using S = typename Io<T>::storage;
  static_assert(sizeof(S) == 2, "16-bit operands");
  constexpr int BM = 64, WAVES_M = 2, WAVES_N = 4, NW = 8;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int TAPS = 9;
  constexpr int A_CHUNK = TAPS * BM * 64;
  constexpr int A_LOADS = A_CHUNK / 1024;
  constexpr int A_PER_WAVE = (A_LOADS + NW - 1) / NW;
  constexpr int P_MAX = kHaloPatchBytes / 1024;
  constexpr int P_PER_WAVE = (P_MAX + NW - 1) / NW;
  constexpr int STAGE_BYTES = NW * WN * (WM + 8) * 2;
  constexpr int SB_USED = A_CHUNK + kHaloPatchBytes > STAGE_BYTES ? A_CHUNK + kHaloPatchBytes : STAGE_BYTES;
  constexpr int SB = (SB_USED + 3 * 64 + 255) / 256 * 256;
  constexpr int ZERO_OFF = SB - 256;
  constexpr int ZERO_POS = (ZERO_OFF - A_CHUNK) / 64;
  static_assert(ZERO_OFF >= SB_USED && (ZERO_OFF - A_CHUNK) % 64 == 0, "zero positions after loads and staging");
  static_assert(2 * SB <= 160 * 1024, "two workgroups per CU");

  __shared__ __attribute__((aligned(1024))) unsigned char lds[SB];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int l32 = lane & 31, hi = lane >> 5;
  const int W = args.w_in, H = args.h, cin = args.cin, rw = ha.rw;
  const int nchunks = cin / 32;
  const S* __restrict__ Wt = static_cast<const S*>(args.w);
  const __amdgpu_buffer_rsrc_t xr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(args.x), static_cast<short>(0), static_cast<int>(args.x_bytes),
                                        0x00020000);
  // XCD-aware order: consecutive tiles (sharing halo rows and filter rows) on one XCD's L2
  int t = blockIdx.x;
  if ((ha.tiles & 7) == 0) t = (t & 7) * (ha.tiles >> 3) + (t >> 3);
  const int m0 = (t % args.tiles_m) * BM;
  const int64_t n0 = static_cast<int64_t>(t / args.tiles_m) * BN;
  const int gr_first = static_cast<int>(n0 / W);
  const int gi_lo = gr_first - 1;

  int32_t a_src[A_PER_WAVE];
#pragma unroll
  for (int i = 0; i < A_PER_WAVE; ++i) {
    const int j = wave + NW * i;
    const int tap = j / (BM / 16);
    const int row = (j % (BM / 16)) * 16 + (lane >> 2);
    const int gch = (lane & 3) ^ a_swizzle(row);
    a_src[i] = (min(m0 + row, args.cout - 1) * TAPS + tap) * cin + gch * 8;
  }
  int32_t p_src[P_PER_WAVE];
#pragma unroll
  for (int i = 0; i < P_PER_WAVE; ++i) {
    const int q = (wave + NW * i) * 16 + (lane >> 2);
    const int gch = (lane & 3) ^ ((q >> 2) & 3);
    const int r = q / rw;
    const int c = q - r * rw;
    const int gi = gi_lo + r;
    const bool ok = gi >= 0 && gi < ha.rows_total && c >= 1 && c <= W;
    p_src[i] = ok ? (gi * W + c - 1) * cin + gch * 8 : -1;
  }
  // NCHW_IN: this thread's 8 x 8 block (patch row nr, 8-channel group ncg of the chunk, 8-pixel group npg) or
  // padding position. Recomputed at every chunk from an opaque copy of the thread id, so none of it stays live
  // (in registers) across the multiply loop, which keeps the kernel within 128 VGPRs (two workgroups per CU).
  auto fill_nchw = [&](int ci0) {
    int tq = tid;
    asm volatile("" : "+v"(tq));
    const int pgroups = W / 8;
    const int blocks = ha.patch_rows * 4 * pgroups;
    const int nr = tq / (4 * pgroups), ncg = tq % 4, npg = (tq / 4) % pgroups;
    const int ngi = gi_lo + nr;
    const bool nblock = tq < blocks && ngi >= 0 && ngi < ha.rows_total;
    const S* __restrict__ Xn = static_cast<const S*>(args.x);
    const int64_t plane = static_cast<int64_t>(H) * W;
    const int64_t nsrc =
        nblock ? ((static_cast<int64_t>(ngi / H) * cin + 8 * ncg + ci0) * H + ngi % H) * W + 8 * npg : 0;
    if (tq < blocks) {
      uint4 v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[e] = uint4{0, 0, 0, 0};
        if (nblock) v[e] = *reinterpret_cast<const uint4*>(Xn + nsrc + e * plane);
      }
      // o[i] = the 8 channels of pixel i: dword k holds channels 2k (low half) and 2k + 1 (high half)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint32_t d[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t lo = reinterpret_cast<const uint32_t*>(&v[2 * k])[i / 2];
          const uint32_t hi = reinterpret_cast<const uint32_t*>(&v[2 * k + 1])[i / 2];
          d[k] = (i % 2 == 0) ? ((lo & 0xffffu) | (hi << 16)) : ((lo >> 16) | (hi & 0xffff0000u));
        }
        const int q = nr * rw + 1 + 8 * npg + i;
        *reinterpret_cast<uint4*>(lds + A_CHUNK + q * 64 + ((ncg ^ ((q >> 2) & 3)) * 16)) = uint4{d[0], d[1], d[2], d[3]};
      }
    } else if (tq < blocks + ha.patch_rows * 8) {  // the padding positions (columns 0 and W + 1), 4 chunks each
      const int z = tq - blocks;
      const int q = (z >> 3) * rw + ((z >> 2) & 1) * (W + 1);
      *reinterpret_cast<uint4*>(lds + A_CHUNK + q * 64 + (z & 3) * 16) = uint4{0, 0, 0, 0};
    }
  };
  auto issue_step = [&](int ci0) {
#pragma unroll
    for (int i = 0; i < A_PER_WAVE; ++i) {
      const int j = wave + NW * i;
      if (j < A_LOADS) global_to_lds16(Wt + a_src[i] + ci0, (FH_LDS void*)(lds + j * 1024));
    }
    if constexpr (NCHW_IN) {
      fill_nchw(ci0);
    } else {
#pragma unroll
      for (int i = 0; i < P_PER_WAVE; ++i) {
        const int j = wave + NW * i;
        if (j < ha.p_loads) {
          const uint32_t voff = p_src[i] >= 0 ? static_cast<uint32_t>(p_src[i] + ci0) * 2u : 0x80000000u;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (FH_LDS void*)(lds + A_CHUNK + j * 1024), 16,
                                                   static_cast<int>(voff), 0, 0, 0);
        }
      }
    }
  };
  int a_off[TM][2];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int arow = wm * WM + i * 32 + l32;
#pragma unroll
    for (int h = 0; h < 2; ++h) a_off[i][h] = arow * 64 + (((2 * h + hi) ^ a_swizzle(arow)) * 16);
  }
  int rowpos[TN][3];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t p = min(n0 + wn * WN + j * 32 + l32, args.p - 1);
    const int gr = static_cast<int>(p / W);
    const int ow = static_cast<int>(p - static_cast<int64_t>(gr) * W);
    const int oh = gr % H;
    const int pbase = (gr - gr_first) * rw + ow;
#pragma unroll
    for (int kh = 0; kh < 3; ++kh)
      rowpos[j][kh] = static_cast<unsigned>(oh + kh - 1) < static_cast<unsigned>(H) ? pbase + kh * rw : ZERO_POS;
  }
  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int x = 0; x < 16; ++x) acc[i][j][x] = 0.0f;

  const uint32_t ab = lds_addr((const FH_LDS void*)lds);
  const uint32_t pb = ab + A_CHUNK;
  KFragments<TM, TN> f0, f1;
  auto read_step = [&]<int STEP>(KFragments<TM, TN>& f) {
    constexpr int tap = STEP / 2, h = STEP % 2, kh = tap / 3, kw = tap % 3;
#pragma unroll
    for (int i = 0; i < TM; ++i) f.a[i] = lds_read_b128<tap * BM * 64>(ab + a_off[i][h]);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int pos = rowpos[j][kh] + kw;
      f.b[j] = lds_read_b128<0>(pb + pos * 64 + ((((2 * h + hi) ^ ((pos >> 2) & 3))) * 16));
    }
  };
  auto multiply = [&](KFragments<TM, TN>& f) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) mfma32<T>(f.a[i], f.b[j], acc[i][j]);
  };

  if (tid < 12) *reinterpret_cast<uint4*>(lds + ZERO_OFF + tid * 16) = uint4{0, 0, 0, 0};
  for (int c = 0; c < nchunks; ++c) {
    issue_step(c * 32);
    wait_vmcnt<0>();
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    // one step ahead: at two workgroups per CU this kernel is held to 128 VGPRs, where a third fragment buffer
    // measured 1-2 % slower
    read_step.template operator()<0>(f0);
    [&]<int... STEP>(std::integer_sequence<int, STEP...>) {
      (
          [&] {
            constexpr int s = STEP;
            KFragments<TM, TN>& cur = (s % 2 == 0) ? f0 : f1;
            KFragments<TM, TN>& nxt = (s % 2 == 0) ? f1 : f0;
            fence_kfragments(cur);
            if constexpr (s + 1 < 2 * TAPS) read_step.template operator()<s + 1>(nxt);
            multiply(cur);
            __builtin_amdgcn_sched_barrier(0);
          }(),
          ...);
    }(std::make_integer_sequence<int, 2 * TAPS>{});
    fence_kfragments(f0);
    fence_kfragments(f1);
    // every wave is done with this step's operands before the next step (or the epilogue) overwrites them
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }
  if (args.out_nhwc) {
    static_assert(BN * (BM + 8) * 2 <= SB, "workgroup staging fits");
    conv_store_tile_wg_nhwc<T, E, BM, BN, WAVES_N, NW>(args, acc, lds, wave, lane, m0, n0);
  } else {
    conv_store_tile<T, E, WM, WN, NW, SB>(args, acc, lds, wave, lane, m0 + wm * WM, n0 + wn * WN);
  }
}

// ---- 3x3 stride-1 convolutions over bands of whole output rows, NCHW in and out ---------------------------------
//
// For Cin = 64, Cout <= 64, NCHW input and output (a conv on a graph input whose result is a graph output). One
// workgroup per band of R consecutive output rows of one image, R chosen so the bands spread evenly over the CUs
// (C3, 32 x 56 rows: R = 7 gives 256 bands of 392 pixels, one per CU; the 256-pixel tiles of the kernel above make
// 392 tiles, two on some CUs and one on the others). The whole filter (2 chunks x 9 taps x 64 rows x 64 B = 72 KB)
// and both 32-channel chunks of the band's patch ((R + 2) x (W + 2) positions each) are resident in LDS. Chunk 1's
// input is loaded into registers before chunk 0 is multiplied and written to LDS after it, so its load overlaps
// the first multiplications. Patch rows outside the image and the two padding columns hold zeros.
// The band's pixels (R * W <= 512) go in two phases of 32-pixel tiles, one tile per wave and phase, all 64 output
// channels each: band pixels 0-255, then 256 onwards (waves without a tile skip the phase). A tile's result is
// written from registers as soon as its phase ends, so phase 0's stores drain while phase 1 multiplies (no LDS
// staging, which would need space the resident operands fill). The products and their order per output are
// those of the kernels above (chunk, tap, k16 half), so the result is the same bit for bit.
constexpr int kBandPatchBytes = 34 * 1024;  // one chunk's patch: (R + 2) * (W + 2) positions of 64 B

struct ConvBandArgs {
  ConvNhwcArgs c;
  int32_t rows;           // R: output rows per band, a divisor of H
  int32_t bands_per_img;  // H / R
};

template <typename T, int E, bool W_OIHW>
__global__ __launch_bounds__(512) void conv_band_kernel(ConvBandArgs ba) {
  const ConvNhwcArgs& args = ba.c;
  using S = typename Io<T>::storage;
  static_assert(sizeof(S) == 2, "16-bit operands");
  constexpr int BM = 64, NW = 8, TM = 2, TAPS = 9;
  constexpr int A_CHUNK = TAPS * BM * 64;  // [tap][64 rows][32 channels] of one chunk
  constexpr int A_BYTES = 2 * A_CHUNK;     // Cin = 64: two chunks
  constexpr int A_PER_WAVE = A_BYTES / 1024 / NW;
  constexpr int PB = kBandPatchBytes;
  constexpr int LDS_BYTES = A_BYTES + 2 * PB;
  static_assert((A_BYTES / 1024) % NW == 0, "filter loads split evenly over the waves");
  static_assert(LDS_BYTES <= 160 * 1024, "filter and both patches fit the LDS");
  __shared__ __attribute__((aligned(1024))) unsigned char lds[LDS_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hi = lane >> 5;
  const int W = args.w_in, H = args.h, R = ba.rows, rw = W + 2;
  const int npx = R * W;
  // XCD-aware order: consecutive bands (sharing halo rows) on one XCD's L2
  int b = blockIdx.x;
  if ((gridDim.x & 7) == 0) b = (b & 7) * static_cast<int>(gridDim.x >> 3) + (b >> 3);
  const int img = b / ba.bands_per_img;
  const int r0 = (b - img * ba.bands_per_img) * R;

  // the filter, [chunk][tap][64 rows][32 channels] in LDS (16-byte chunks of a row swizzled)
  const S* __restrict__ Wt = static_cast<const S*>(args.w);
  uint4 wv[TAPS];  // W_OIHW: this thread's 8 input channels x 9 taps of one output channel
  if constexpr (!W_OIHW) {
    // [Cout][3][3][64]: 1 KB load j covers chunk j / 36, tap (j / 4) % 9, rows 16 * (j % 4) .. + 15
#pragma unroll
    for (int i = 0; i < A_PER_WAVE; ++i) {
      const int j = wave + NW * i;
      const int ch = j / (TAPS * 4), tap = (j / 4) % TAPS;
      const int row = (j % 4) * 16 + (lane >> 2);
      const int gch = (lane & 3) ^ a_swizzle(row);
      global_to_lds16(Wt + (min(row, args.cout - 1) * TAPS + tap) * 64 + ch * 32 + gch * 8,
                      (FH_LDS void*)(lds + j * 1024));
    }
  }
  // W_OIHW: thread = (output channel row, input channels 8 cg .. 8 cg + 7) with tid bits [cg & 3 | row & 3 | cg >> 2 |
  // row >> 2], so the 16 lanes of one LDS write cover 4 rows x 4 chunks of one 32-channel half: 16 distinct 16-byte
  // bank slots (row & 3 picks the 64-byte quarter of a 256-byte bank row, the swizzled chunk the slot in it)
  const int f_row = ((tid >> 5) << 2) | ((tid >> 2) & 3), f_cg = (((tid >> 4) & 1) << 2) | (tid & 3);
  if constexpr (W_OIHW) {
    // [Cout][64][3][3] (the graph's own layout): the thread's 72 filter values are 144 contiguous bytes,
    // transposed in registers after they land
    const int co = min(f_row, args.cout - 1);
    const uint4* src = reinterpret_cast<const uint4*>(Wt + (co * 64 + f_cg * 8) * TAPS);
#pragma unroll
    for (int q = 0; q < TAPS; ++q) wv[q] = src[q];
  }
  // W_OIHW: writes the thread's 9 taps x 8 channels as 9 16-byte chunks (channel pairs packed per dword)
  auto store_filter = [&]() {
    if constexpr (W_OIHW) {
      const int row = f_row, cg = f_cg;
      uint16_t e[8 * TAPS];  // e[ci * 9 + tap]
      __builtin_memcpy(e, wv, sizeof(e));
      unsigned char* dst = lds + (cg >> 2) * A_CHUNK + row * 64 + (((cg & 3) ^ a_swizzle(row)) * 16);
#pragma unroll
      for (int tap = 0; tap < TAPS; ++tap) {
        uint32_t d[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
          d[k] = static_cast<uint32_t>(e[(2 * k) * TAPS + tap]) | (static_cast<uint32_t>(e[(2 * k + 1) * TAPS + tap]) << 16);
        *reinterpret_cast<uint4*>(dst + tap * BM * 64) = uint4{d[0], d[1], d[2], d[3]};
      }
    }
  };
  // the padding columns (positions 0 and W + 1 of every patch row) of both patches: 2 (R + 2) 8 16-byte slots,
  // more than the 512 threads when R > 30 (W = 8 allows R up to 62)
  for (int t = tid; t < 2 * (R + 2) * 8; t += 512) {
    const int buf = t / ((R + 2) * 8), z = t % ((R + 2) * 8);
    const int q = (z >> 3) * rw + ((z >> 2) & 1) * (W + 1);
    *reinterpret_cast<uint4*>(lds + A_BYTES + buf * PB + q * 64 + (z & 3) * 16) = uint4{0, 0, 0, 0};
  }
  // NCHW fill: thread -> (8-channel group ncg, patch row nr, 8-pixel group npg), npg fastest, so the lanes of one
  // load instruction read one channel plane's (R + 2) band rows, which are contiguous in memory.
  const int pgroups = W / 8;
  const int per_cg = (R + 2) * pgroups;
  const int ncg = tid / per_cg, nr = (tid % per_cg) / pgroups, npg = tid % pgroups;
  const int ih = r0 - 1 + nr;
  const bool filler = tid < 4 * per_cg;
  const bool inside = filler && ih >= 0 && ih < H;
  const S* __restrict__ Xn = static_cast<const S*>(args.x);
  const int64_t plane = static_cast<int64_t>(H) * W;
  const int64_t src = inside ? ((static_cast<int64_t>(img) * 64 + 8 * ncg) * H + ih) * W + 8 * npg : 0;
  auto load_chunk = [&](int ci0, uint4 (&v)[8]) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[e] = uint4{0, 0, 0, 0};
      if (inside) v[e] = *reinterpret_cast<const uint4*>(Xn + src + (ci0 + e) * plane);
    }
  };
  // transposes the 8 x 8 block in registers and writes 8 positions' 16-byte chunks (zeros outside the image)
  auto store_chunk = [&](const uint4 (&v)[8], unsigned char* patch) {
    if (!filler) return;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint32_t d[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t lo = uint4_word(v[2 * k], i / 2);
        const uint32_t hi2 = uint4_word(v[2 * k + 1], i / 2);
        d[k] = (i % 2 == 0) ? ((lo & 0xffffu) | (hi2 << 16)) : ((lo >> 16) | (hi2 & 0xffff0000u));
      }
      const int q = nr * rw + 1 + 8 * npg + i;
      *reinterpret_cast<uint4*>(patch + q * 64 + ((ncg ^ ((q >> 2) & 3)) * 16)) = uint4{d[0], d[1], d[2], d[3]};
    }
  };

  // filter fragment offsets: channel row 32 i + l32, k-chunk 2 h + hi of the stage
  int a_off[TM][2];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int arow = i * 32 + l32;
#pragma unroll
    for (int h = 0; h < 2; ++h) a_off[i][h] = arow * 64 + (((2 * h + hi) ^ a_swizzle(arow)) * 16);
  }
  // the bias of this lane's output channels (32 i + l32), fetched with the first fill
  const S* bias_g = static_cast<const S*>(args.bias);
  float bias_v[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) bias_v[i] = bias_g != nullptr ? Io<T>::load(bias_g[min(i * 32 + l32, args.cout - 1)]) : 0.0f;

  const uint32_t ab = lds_addr((const FH_LDS void*)lds);
  // One chunk of the pixel tile whose tap-(0, 0) patch position for this lane is pb. The MFMA's A operand is the
  // patch (rows = the tile's 32 pixels) and B the filter (columns = 32 channels), so each lane ends with one
  // channel's values for runs of four consecutive pixels (see store_tile).
  // ONLY: -1 multiplies both 32-channel halves of the tile, 0 or 1 that half alone (one filter fragment and one
  // MFMA per step; acc[ONLY] is the only accumulator written).
  auto chunk = [&]<int ONLY>(f32x16_t (&acc)[TM], int pb, uint32_t a_base, uint32_t p_base) {
    constexpr int I0 = ONLY < 0 ? 0 : ONLY, I1 = ONLY < 0 ? TM : ONLY + 1;
    constexpr int READS = I1 - I0 + 1;  // LDS reads per step
    KFragments<TM, 1> f0, f1, f2;
    auto read_step = [&]<int STEP>(KFragments<TM, 1>& f) {
      constexpr int tap = STEP / 2, h = STEP % 2, kh = tap / 3, kw = tap % 3;
#pragma unroll
      for (int i = I0; i < I1; ++i) f.a[i] = lds_read_b128<tap * BM * 64>(a_base + a_off[i][h]);
      const int pos = pb + kh * rw + kw;
      f.b[0] = lds_read_b128<0>(p_base + pos * 64 + ((((2 * h + hi) ^ ((pos >> 2) & 3))) * 16));
    };
    auto tie = [&](KFragments<TM, 1>& f) {
#pragma unroll
      for (int i = I0; i < I1; ++i) asm volatile("" : "+v"(f.a[i]));
      asm volatile("" : "+v"(f.b[0]));
    };
    // fragments read two steps ahead (three buffers): before step s's MFMAs, every LDS read but step s+1's (the
    // last READS issued; LDS reads complete in order) has landed
    read_step.template operator()<0>(f0);
    read_step.template operator()<1>(f1);
    [&]<int... STEP>(std::integer_sequence<int, STEP...>) {
      (
          [&] {
            constexpr int s = STEP;
            KFragments<TM, 1>& cur = (s % 3 == 0) ? f0 : (s % 3 == 1) ? f1 : f2;
            KFragments<TM, 1>& ahead = (s % 3 == 0) ? f2 : (s % 3 == 1) ? f0 : f1;
            if constexpr (s + 1 < 2 * TAPS) {
              wait_lgkmcnt<READS>();
            } else {
              wait_lgkmcnt<0>();
            }
            tie(cur);
            if constexpr (s + 2 < 2 * TAPS) read_step.template operator()<s + 2>(ahead);
#pragma unroll
            for (int i = I0; i < I1; ++i) mfma32<T>(cur.b[0], cur.a[i], acc[i]);
            __builtin_amdgcn_sched_barrier(0);
          }(),
          ...);
    }(std::make_integer_sequence<int, 2 * TAPS>{});
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    tie(f0);
    tie(f1);
    tie(f2);
  };
  // Writes the pixel tile px0 .. px0 + 31 of the band from registers. Register x of a lane holds pixel
  // px0 + 8 (x >> 2) + 4 hi + (x & 3) of channel 32 i + l32: the lanes l32 and l32 + 32 exchange one 4-pixel
  // run each (hi = 0 keeps pixels 0-3 and takes 4-7, hi = 1 takes 8-11 and keeps 12-15; likewise for 16-31),
  // after which every lane holds two 8-pixel vectors of its channel and writes them with 16-byte stores.
  S* __restrict__ Y = static_cast<S*>(args.y);
  const int64_t ybase = static_cast<int64_t>(img) * args.cout * args.howo + static_cast<int64_t>(r0) * W;
  constexpr int EA = epi_after_stage<E>();
  auto store_tile = [&]<int ONLY>(f32x16_t (&acc)[TM], int px0) {
#pragma unroll
    for (int i = ONLY < 0 ? 0 : ONLY; i < (ONLY < 0 ? TM : ONLY + 1); ++i) {
      const int co = i * 32 + l32;
      const float b = bias_v[i];
      // runs 2 half and 2 half + 1 (registers 8 half .. 8 half + 7): pixels 16 half + 4 hi + 0..3 and
      // 16 half + 8 + 4 hi + 0..3, packed pairwise, exchanged into the 8-pixel vector 16 half + 8 hi + 0..7
      auto vector = [&](int x0) {
        const uint32_t a0 = epi_stage2<E, T>(acc[i][x0] + b, acc[i][x0 + 1] + b);
        const uint32_t a1 = epi_stage2<E, T>(acc[i][x0 + 2] + b, acc[i][x0 + 3] + b);
        const uint32_t c0 = epi_stage2<E, T>(acc[i][x0 + 4] + b, acc[i][x0 + 5] + b);
        const uint32_t c1 = epi_stage2<E, T>(acc[i][x0 + 6] + b, acc[i][x0 + 7] + b);
        const uint32_t r0v = static_cast<uint32_t>(__shfl_xor(static_cast<int>(hi ? a0 : c0), 32));
        const uint32_t r1v = static_cast<uint32_t>(__shfl_xor(static_cast<int>(hi ? a1 : c1), 32));
        return hi ? uint4{r0v, r1v, c0, c1} : uint4{a0, a1, r0v, r1v};
      };
      const uint4 v0 = vector(0), v1 = vector(8);
      if (co < args.cout) {
        const int64_t idx = ybase + static_cast<int64_t>(co) * args.howo + px0 + 8 * hi;
        if (px0 + 8 * hi < npx) *reinterpret_cast<uint4*>(Y + idx) = epi_vec<EA, T>(args.ep, v0, idx);
        if (px0 + 16 + 8 * hi < npx) *reinterpret_cast<uint4*>(Y + idx + 16) = epi_vec<EA, T>(args.ep, v1, idx + 16);
      }
    }
  };
  auto zero = [](f32x16_t (&acc)[TM]) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int x = 0; x < 16; ++x) acc[i][x] = 0.0f;
  };
  auto patch_pos = [&](int px0) {
    const int bp = min(px0 + l32, npx - 1);
    const int r = bp / W;
    return r * rw + (bp - r * W);
  };

  // phase 0: pixels 32 wave .. + 31 (band pixels 0-255), both chunks; chunk 1's fill lands in between
  uint4 v[8];
  load_chunk(0, v);
  wait_vmcnt<0>();  // chunk 0's input, the whole filter and the bias
  store_filter();
  store_chunk(v, lds + A_BYTES);
  load_chunk(32, v);  // chunk 1 stays in flight during chunk 0's multiplications
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  {
    const int px0 = wave * 32;
    const bool active = px0 < npx;  // uniform
    const int pb = patch_pos(px0);
    f32x16_t acc[TM];
    zero(acc);
    if (active) chunk.template operator()<-1>(acc, pb, ab, ab + A_BYTES);
    wait_vmcnt<0>();
    store_chunk(v, lds + A_BYTES + PB);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (active) {
      chunk.template operator()<-1>(acc, pb, ab + A_CHUNK, ab + A_BYTES + PB);
      store_tile.template operator()<-1>(acc, px0);
    }
  }
  // phase 1: tiles 8 .. ntiles - 1 (pixels from 256; the LDS operands are read-only from here, phase 0's stores
  // drain meanwhile). Wave w runs on SIMD w % 4, and phase 0 gave every SIMD two tiles. When the phase holds
  // 4 k + 1 tiles, its last tile goes to waves n1 and n1 + 1 (SIMDs 1 and 2) as two 32-channel halves instead of
  // to wave n1 - 1 (SIMD 0) whole: C3's bands of 13 tiles then hold 3.5 tiles on their busiest SIMD, not 4.
  {
    const int ntiles = (npx + 31) / 32, n1 = ntiles - 8;
    const bool split = n1 > 0 && (n1 & 3) == 1;
    int tile = -1, half = -1;  // uniform per wave
    if (split) {
      if (wave < n1 - 1) {
        tile = 8 + wave;
      } else if (wave == n1 || wave == n1 + 1) {
        tile = 8 + n1 - 1;
        half = wave - n1;
      }
    } else if (wave < n1) {
      tile = 8 + wave;
    }
    if (tile >= 0) {
      const int px0 = tile * 32;
      const int pb = patch_pos(px0);
      f32x16_t acc[TM];
      zero(acc);
      if (half < 0) {
        chunk.template operator()<-1>(acc, pb, ab, ab + A_BYTES);
        chunk.template operator()<-1>(acc, pb, ab + A_CHUNK, ab + A_BYTES + PB);
        store_tile.template operator()<-1>(acc, px0);
      } else if (half == 0) {
        chunk.template operator()<0>(acc, pb, ab, ab + A_BYTES);
        chunk.template operator()<0>(acc, pb, ab + A_CHUNK, ab + A_BYTES + PB);
        store_tile.template operator()<0>(acc, px0);
      } else {
        chunk.template operator()<1>(acc, pb, ab, ab + A_BYTES);
        chunk.template operator()<1>(acc, pb, ab + A_CHUNK, ab + A_BYTES + PB);
        store_tile.template operator()<1>(acc, px0);
      }
    }
  }
}

// Rows per band for the band kernel, or 0 when it does not take this geometry (NCHW input and output, Cin = 64,
// Cout <= 64, W % 8 == 0, 16-byte aligned output and epilogue operands) or would not finish sooner than the 256-pixel tiles: the divisor R of H with the least
// pixels per CU (rounds of one band per CU x R x W), R * W <= 512, both patches within kBandPatchBytes and one
// fill thread per 8 x 8 block.
int conv_band_rows(const ConvNhwcArgs& c, const int64_t* g, int64_t cus) {
  if (c.out_nhwc || !c.vec_store || g[1] != 64 || g[4] > 64 || g[3] % 8 != 0) return 0;
  const int64_t n = g[0], h = g[2], w = g[3];
  int best = 0;
  int64_t best_px = 0;
  for (int64_t r = 1; r <= h && r * w <= 512; ++r) {
    if (h % r != 0 || (r + 2) * (w + 2) * 64 > kBandPatchBytes || 4 * (r + 2) * (w / 8) > 512) continue;
    const int64_t bands = n * h / r;
    const int64_t px = (bands + cus - 1) / cus * r * w;
    if (best == 0 || px <= best_px) {
      best = static_cast<int>(r);
      best_px = px;
    }
  }
  // the single-buffered kernel at two 256-pixel tiles per CU slot pair
  const int64_t tiles = (c.p + 255) / 256;
  const int64_t halo_px = (tiles + 2 * cus - 1) / (2 * cus) * 2 * 256;
  return best != 0 && best_px < halo_px ? best : 0;
}

// bf16 with the fixed programs (none, relu, add;relu) only: other programs and f16 take the single-buffered kernel
// (the interpreted epilogue would need scratch memory here).
bool band_program(int kind) { return kind == kEpiNone || kind == kEpiRelu || kind == kEpiAddRelu; }

bool halo_nchw_supported(int32_t dtype, const int64_t* g);

// Rows per band when the band kernel takes (dtype, geometry, program) with NCHW input and output, else 0.
int band_rows_for(int32_t dtype, const ConvNhwcArgs& c, const int64_t* g) {
  if (dtype != FH_BF16 || !band_program(epi_kind(c.ep)) || !halo_nchw_supported(dtype, g)) return 0;
  return conv_band_rows(c, g, device_cu_count());
}

template <bool W_OIHW>
fh_status launch_band(ConvNhwcArgs c, int rows, hipStream_t stream) {
  ConvBandArgs a{};
  a.c = c;
  a.rows = rows;
  a.bands_per_img = c.h / rows;
  const dim3 grid(static_cast<uint32_t>(c.p / (static_cast<int64_t>(rows) * c.w_in)));
  switch (epi_kind(c.ep)) {
    case kEpiNone:
      hipLaunchKernelGGL((conv_band_kernel<bf16_t, kEpiNone, W_OIHW>), grid, dim3(512), 0, stream, a);
      break;
    case kEpiRelu:
      hipLaunchKernelGGL((conv_band_kernel<bf16_t, kEpiRelu, W_OIHW>), grid, dim3(512), 0, stream, a);
      break;
    case kEpiAddRelu:
      hipLaunchKernelGGL((conv_band_kernel<bf16_t, kEpiAddRelu, W_OIHW>), grid, dim3(512), 0, stream, a);
      break;
    default: return fail(FH_INTERNAL, "conv_band_kernel: epilogue program without a band instance");
  }
  return launch_status("conv_band_kernel launch");
}

// Whether the resident-patch kernel takes this geometry: patch rows of a BN-pixel tile (at most (BN - 1) / W + 2
// output rows plus the two halo rows) must fit kHaloPatchBytes; p_loads = the 1 KB loads that fill them.
bool halo_supported(int32_t dtype, const int64_t* g, int bn, int32_t* p_loads, int32_t* patch_rows = nullptr) {
  if (dtype != FH_BF16 && dtype != FH_F16) return false;
  if (g[11] != 1 || g[5] != 3 || g[6] != 3 || g[7] != 1 || g[8] != 1 || g[9] != 1 || g[10] != 1) return false;
  if (g[1] % 32 != 0 || g[2] < 1 || g[3] < 1 || g[4] < 1 || g[4] > 512) return false;
  const int64_t rows = (bn - 1) / g[3] + 2 + 2;
  const int64_t positions = rows * (g[3] + 2);
  if (positions * 64 > kHaloPatchBytes) return false;
  // 32-bit element offsets: the whole input, the filter
  if (g[0] * g[2] * g[3] * g[1] >= (int64_t{1} << 30) || g[4] * 9 * g[1] >= (int64_t{1} << 30)) return false;
  if (p_loads != nullptr) *p_loads = static_cast<int32_t>((positions + 15) / 16);
  if (patch_rows != nullptr) *patch_rows = static_cast<int32_t>(rows);
  return true;
}

// NCHW input for the single-buffered kernel: whole 8-pixel groups per row, and one thread per 8 x 8 block plus
// the padding positions.
bool halo_nchw_supported(int32_t dtype, const int64_t* g) {
  int32_t loads = 0, rows = 0;
  if (!halo_supported(dtype, g, 128, &loads, &rows) || g[3] % 8 != 0) return false;
  return rows * 4 * (g[3] / 8) + rows * 8 <= 512;
}

template <typename T, int BN, bool NCHW_IN = false>
fh_status launch_halo1(ConvHaloArgs a, hipStream_t stream) {
  a.c.tiles_m = (a.c.cout + 63) / 64;
  a.c.tiles_n = static_cast<int32_t>((a.c.p + BN - 1) / BN);
  a.tiles = a.c.tiles_m * a.c.tiles_n;
  return with_epi<conv_epi_mask<T, false>()>(epi_kind(a.c.ep), [&]<int E>() {
    hipLaunchKernelGGL((conv_halo1_kernel<T, BN, E, NCHW_IN>), dim3(static_cast<uint32_t>(a.tiles)), dim3(512), 0,
                       stream, a);
    return launch_status("conv_halo1_kernel launch");
  });
}

template <typename T, int BN>
fh_status launch_halo(ConvHaloArgs a, hipStream_t stream) {
  a.c.tiles_m = (a.c.cout + 63) / 64;
  a.c.tiles_n = static_cast<int32_t>((a.c.p + BN - 1) / BN);
  a.tiles = a.c.tiles_m * a.c.tiles_n;
  const dim3 grid(static_cast<uint32_t>(std::min<int64_t>(a.tiles, device_cu_count())));
  const bool res_a = a.c.cout <= 64 && a.c.cin <= kHaloResidentCin;
  return with_epi<conv_epi_mask<T, false>()>(epi_kind(a.c.ep), [&]<int E>() {
    if (res_a)
      hipLaunchKernelGGL((conv_halo_kernel<T, BN, true, E>), grid, dim3(512), 0, stream, a);
    else
      hipLaunchKernelGGL((conv_halo_kernel<T, BN, false, E>), grid, dim3(512), 0, stream, a);
    return launch_status("conv_halo_kernel launch");
  });
}

// Which resident-patch kernel, from measurements of C3 and the ResNet-18 3x3 stride-1 layers on an MI355X (bf16,
// relu epilogue, batch 64; us per launch, implicit GEMM in brackets):
//   NCHW input and output, Cin 64, bf16:     the band kernel when its bands spread more evenly (C3 13.5; 16.2
//                                            single-buffered)
//   NCHW output (a graph output, C3):        single-buffered, two per CU    C3 16.3 (20.6)
//   channels-last output, Cout <= 64:        persistent, resident filter    56x56x64 34.2 (41.9)
//   channels-last output, 64 < Cout <= 256:  single-buffered                28x28x128 31.1 (32.8), 14x14x256 32.1 (36.2)
//   Cout > 256 (7x7x512):                    the implicit GEMM (31.6; 43.8 here)
// Single-buffered tiles: 256 pixels when that still makes 1.5 workgroups per CU slot pair, else 128; persistent:
// 256 when the tiles fill the device 1.5 times over, else 128.
template <typename T>
fh_status dispatch_halo(const ConvNhwcArgs& c, const int64_t* geom, hipStream_t stream, bool* launched,
                        bool nchw_in = false) {
  *launched = false;
  if (c.out_nhwc && c.cout > 256 && !nchw_in) return FH_OK;
  const int64_t cus = device_cu_count();
  if (nchw_in && std::is_same_v<T, bf16_t>) {
    const int band_rows = band_rows_for(FH_BF16, c, geom);
    if (band_rows > 0) {
      *launched = true;
      return launch_band<false>(c, band_rows, stream);
    }
  }
  const int64_t tiles_m = (c.cout + 63) / 64;
  const bool persistent = c.out_nhwc && c.cout <= 64 && !nchw_in;
  ConvHaloArgs a{};
  a.c = c;
  a.rw = c.w_in + 2;
  a.rows_total = static_cast<int32_t>(geom[0] * geom[2]);
  int32_t loads = 0, rows = 0;
  if (2 * tiles_m * ((c.p + 255) / 256) >= 3 * cus && halo_supported(FH_BF16, geom, 256, &loads, &rows) &&
      (!nchw_in || rows * 4 * (geom[3] / 8) + rows * 8 <= 512)) {
    a.p_loads = loads;
    a.patch_rows = rows;
    *launched = true;
    if (nchw_in) return launch_halo1<T, 256, true>(a, stream);
    return persistent ? launch_halo<T, 256>(a, stream) : launch_halo1<T, 256>(a, stream);
  }
  if (halo_supported(FH_BF16, geom, 128, &loads, &rows)) {
    a.p_loads = loads;
    a.patch_rows = rows;
    *launched = true;
    if (nchw_in) return launch_halo1<T, 128, true>(a, stream);
    return persistent ? launch_halo<T, 128>(a, stream) : launch_halo1<T, 128>(a, stream);
  }
  return FH_OK;
}

// Tile choice, from measurements of the ResNet layer shapes on an MI355X (bf16, 3x3, batch 64): by output
// channels M and output pixels P, the per-layer best of {64x256, 64x128, 64x64, 128x128, 128x256}:
//   M <= 64: 64x128 when P >= 150K (56x56 at batch 64: 35.4 us vs 37.5 for 64x256), else 64x256 (C3: 20.7 vs 22.2);
//   M == 128: 128x256 (28x28: 22.9 us vs 25.5 for 128x128);  M in (128, 256]: 128x128 (14x14: 31.0 vs 34.9);
//   larger M: 64x64 (7x7 at 512 channels: 40.1 us vs 42.0 for 64x128).
// Every choice keeps at least as many tiles as a quarter of the CUs; otherwise the smallest tile.
template <typename T, bool C8>
fh_status dispatch_conv(const ConvNhwcArgs& a, hipStream_t stream) {
  const int64_t cus = device_cu_count();
  auto tiles = [&](int64_t bm, int64_t bn) { return ((a.cout + bm - 1) / bm) * ((a.p + bn - 1) / bn); };
  auto enough = [&](int64_t bm, int64_t bn) { return tiles(bm, bn) * 4 >= cus; };
  constexpr bool k16 = sizeof(typename Io<T>::storage) == 2;  // fp32 wave tiles of 64x64 do not fit the ring
  if (a.cout <= 64) {
    if (a.p < 150000 && enough(64, 256)) return launch_conv<T, 64, 256, 1, 4, C8>(a, stream);
    if (enough(64, 128)) return launch_conv<T, 64, 128, 2, 2, C8>(a, stream);
  } else if (a.cout <= 128) {
    if constexpr (k16) {
      if (enough(128, 256)) return launch_conv<T, 128, 256, 2, 4, C8>(a, stream);
    }
    if (enough(128, 128) && (k16 || !a.out_nhwc)) return launch_conv<T, 128, 128, 2, 4, C8>(a, stream);
  } else if (a.cout <= 256) {
    if (enough(128, 128) && (k16 || !a.out_nhwc)) return launch_conv<T, 128, 128, 2, 4, C8>(a, stream);
  }
  return launch_conv<T, 64, 64, 2, 2, C8>(a, stream);
}

// Batched transpose through a 64 x 64 LDS tile: y[b][c][r] = x[b][r][c]; reads and writes are coalesced.
template <typename E>
__global__ __launch_bounds__(256) void transpose_batched_kernel(const E* __restrict__ x, E* __restrict__ y,
                                                                int64_t rows, int64_t cols) {
  __shared__ E tile[64][65];
  const int64_t b = blockIdx.z;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 64, c0 = static_cast<int64_t>(blockIdx.x) * 64;
  const E* xb = x + b * rows * cols;
  E* yb = y + b * rows * cols;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4) {
    const int64_t gr = r0 + r, gc = c0 + tx;
    if (gr < rows && gc < cols) tile[r][tx] = xb[gr * cols + gc];
  }
  __syncthreads();
  for (int c = ty; c < 64; c += 4) {
    const int64_t gc = c0 + c, gr = r0 + tx;
    if (gc < cols && gr < rows) yb[gc * rows + gr] = tile[tx][c];
  }
}

// 16-bit batched transpose with 16-byte writes (rows % 8 == 0, 16-byte aligned output) and, when cols % 8 == 0
// and the input is aligned too, 16-byte reads (otherwise one element per lane, still coalesced along a row): a
// 64 x 64 tile goes through LDS (chunk cc of tile row r stored at cc ^ ((r >> 3) & 7), which keeps the column
// reads below free of bank conflicts), and each thread then gathers 8 consecutive rows of one column and writes
// them as one 16-byte chunk of the output row.
template <bool WIDE_READ>
__global__ __launch_bounds__(256) void transpose_wide_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
                                                             int64_t rows, int64_t cols) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[64 * 64];
  const int64_t b = blockIdx.z;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 64, c0 = static_cast<int64_t>(blockIdx.x) * 64;
  const uint16_t* xb = x + b * rows * cols;
  uint16_t* yb = y + b * rows * cols;
  const int t = threadIdx.x;
  if constexpr (WIDE_READ) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int id = t + 256 * j, r = id >> 3, cc = id & 7;
      const int64_t gr = r0 + r, gc = c0 + 8 * cc;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (gr < rows && gc < cols) v = *reinterpret_cast<const uint4*>(xb + gr * cols + gc);
      *reinterpret_cast<uint4*>(tile + r * 64 + ((cc ^ ((r >> 3) & 7)) * 8)) = v;
    }
  } else {
    // lane -> column t % 64 of rows t / 64 + 4 i: reads coalesced along the input row
    const int c = t & 63;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = (t >> 6) + 4 * i;
      const int64_t gr = r0 + r, gc = c0 + c;
      const uint16_t v = (gr < rows && gc < cols) ? xb[gr * cols + gc] : uint16_t{0};
      tile[r * 64 + (((c >> 3) ^ ((r >> 3) & 7)) * 8) + (c & 7)] = v;
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int id = t + 256 * j, c = id >> 3, rc = id & 7;
    const int64_t gc = c0 + c, gr = r0 + 8 * rc;
    uint16_t o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = tile[(8 * rc + i) * 64 + (((c >> 3) ^ rc) * 8) + (c & 7)];
    if (gc < cols && gr < rows) {
      uint4 v;
      __builtin_memcpy(&v, o, 16);
      *reinterpret_cast<uint4*>(yb + gc * rows + gr) = v;
    }
  }
}

// Small planes (rows * cols <= kPlaneMax, e.g. a filter's [Cin][KH*KW]): one workgroup per batch item moves the
// whole plane through LDS, reading and writing it contiguously.
constexpr int kPlaneMax = 8192;
template <typename E>
__global__ __launch_bounds__(256) void transpose_plane_kernel(const E* __restrict__ x, E* __restrict__ y, int32_t rows,
                                                              int32_t cols) {
  __shared__ E plane[kPlaneMax];
  const int n = rows * cols;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * n;
  for (int i = threadIdx.x; i < n; i += 256) plane[i] = x[base + i];
  __syncthreads();
  for (int o = threadIdx.x; o < n; o += 256) {
    const int c = o / rows, r = o - (o / rows) * rows;
    y[base + o] = plane[r * cols + c];
  }
}

// Up to kMultiMax small batched transposes in one launch (a graph's filters, [Cout][Cin][KH*KW] ->
// [Cout][KH*KW][Cin]): blockIdx.y picks the tensor, blockIdx.x the plane, each plane as in
// transpose_plane_kernel. One launch instead of one per layer: each of these is too small to be more than
// launch and memory latency on its own.
constexpr int kMultiMax = 32;
struct PlaneBatch {
  const void* x[kMultiMax];
  void* y[kMultiMax];
  int32_t batch[kMultiMax], rows[kMultiMax], cols[kMultiMax];
};
template <typename E>
__global__ __launch_bounds__(256) void transpose_planes_multi_kernel(PlaneBatch a) {
  __shared__ E plane[kPlaneMax];
  const int ti = blockIdx.y;
  if (static_cast<int32_t>(blockIdx.x) >= a.batch[ti]) return;
  const int rows = a.rows[ti], cols = a.cols[ti], n = rows * cols;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * n;
  const E* x = static_cast<const E*>(a.x[ti]) + base;
  E* y = static_cast<E*>(a.y[ti]) + base;
  for (int i = threadIdx.x; i < n; i += 256) plane[i] = x[i];
  __syncthreads();
  for (int o = threadIdx.x; o < n; o += 256) {
    const int c = o / rows, r = o - (o / rows) * rows;
    y[o] = plane[r * cols + c];
  }
}

// 16-bit filters whose every plane is [Cin][9] or [Cin][1] with Cin % 8 == 0 (a ResNet's 3x3 and 1x1 convs), in
// 16-byte vectors: thread = (tensor blockIdx.y, output channel, 8 input channels); a 3x3 thread loads its 8 x 9
// values (144 contiguous bytes) and writes 9 vectors of 8 channels, one per tap; a 1x1 plane is its own
// transpose (a copy). Lanes of one store write consecutive 16-byte vectors.
__global__ __launch_bounds__(256) void transpose_filters_vec_kernel(PlaneBatch a) {
  __shared__ uint4 stage[256 * 9];
  const int ti = blockIdx.y;
  const int rows = a.rows[ti], cols = a.cols[ti], groups = rows / 8;
  const int64_t total = static_cast<int64_t>(a.batch[ti]) * groups;  // (co, 8-channel group) pairs
  const int64_t i0 = static_cast<int64_t>(blockIdx.x) * 256, i = i0 + threadIdx.x;
  if (i0 >= total) return;  // the whole workgroup
  const int64_t co = i / groups, cg = i - co * groups;
  const uint16_t* x = static_cast<const uint16_t*>(a.x[ti]);
  uint16_t* y = static_cast<uint16_t*>(a.y[ti]);
  if (cols == 1) {
    if (i < total)
      *reinterpret_cast<uint4*>(y + co * rows + cg * 8) = *reinterpret_cast<const uint4*>(x + co * rows + cg * 8);
    return;
  }
  // pair i's 72 values are the nine vectors 9i .. 9i + 8 of x, so the workgroup's pairs read one contiguous run:
  // staged through LDS with consecutive lanes on consecutive vectors, then each thread takes its nine
  const int32_t nvec = static_cast<int32_t>(min<int64_t>(256, total - i0)) * 9;
  const uint4* src = reinterpret_cast<const uint4*>(x) + i0 * 9;
  for (int32_t q = threadIdx.x; q < nvec; q += 256) stage[q] = src[q];
  __syncthreads();
  if (i >= total) return;
  uint4 v[9];
#pragma unroll
  for (int q = 0; q < 9; ++q) v[q] = stage[threadIdx.x * 9 + q];
  // value (channel c, tap t) is element c * 9 + t of the 72 loaded
  auto value = [&](int f) -> uint32_t {
    const uint32_t w = uint4_word(v[f / 8], (f % 8) / 2);
    return (f % 2 == 0) ? (w & 0xffffu) : (w >> 16);
  };
  uint16_t* dst = y + co * 9 * rows + cg * 8;
#pragma unroll
  for (int t = 0; t < 9; ++t) {
    uint32_t d[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) d[k] = value((2 * k) * 9 + t) | (value((2 * k + 1) * 9 + t) << 16);
    *reinterpret_cast<uint4*>(dst + t * rows) = uint4{d[0], d[1], d[2], d[3]};
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// K of a C8 filter: KH*KW positions of 8 channels, rounded up to whole stages.
int64_t conv_c8_filter_k(int64_t kh, int64_t kw) { return (kh * kw * 8 + kBK - 1) / kBK * kBK; }

// x [N][C][HW] (C <= 8) -> y [N][HW][8], channels C..7 zero. One thread per pixel, one 16-byte store.
__global__ __launch_bounds__(256) void pack_input_c8_kernel(const uint16_t* __restrict__ x, uint4* __restrict__ y,
                                                            int64_t n, int32_t c, int64_t hw) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n * hw; i += stride) {
    const int64_t img = i / hw, pix = i - img * hw;
    uint16_t v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int ch = 0; ch < c; ++ch) v[ch] = x[(img * c + ch) * hw + pix];
    uint4 o;
    __builtin_memcpy(&o, v, 16);
    y[i] = o;
  }
}

// The same packing with the image from blockIdx.y: 32-bit, division-free index math; a wave's plane loads
// and its 16-byte stores are each one contiguous run.
__global__ __launch_bounds__(256) void pack_input_c8_2d_kernel(const uint16_t* __restrict__ x, uint4* __restrict__ y,
                                                               int32_t c, int32_t hw) {
  const int32_t pix = static_cast<int32_t>(blockIdx.x) * 256 + static_cast<int32_t>(threadIdx.x);
  if (pix >= hw) return;
  const int64_t img = blockIdx.y;
  const uint16_t* src = x + img * c * hw + pix;
  uint32_t d[4] = {0, 0, 0, 0};
#pragma unroll
  for (int ch = 0; ch < 8; ++ch)
    if (ch < c) d[ch / 2] |= static_cast<uint32_t>(src[static_cast<int64_t>(ch) * hw]) << (16 * (ch % 2));
  y[img * hw + pix] = uint4{d[0], d[1], d[2], d[3]};
}

// w [Cout][C][KH*KW] (C <= 8) -> y [Cout][K] with y[co][pos*8 + ci] = w[co][ci][pos], zeros elsewhere.
__global__ __launch_bounds__(256) void pack_filter_c8_kernel(const uint16_t* __restrict__ w, uint16_t* __restrict__ y,
                                                             int32_t cout, int32_t c, int32_t khw, int32_t k) {
  const int64_t total = static_cast<int64_t>(cout) * k;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total; i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t co = i / k;
    const int q = static_cast<int>(i - co * k), pos = q / 8, ci = q % 8;
    y[i] = (pos < khw && ci < c) ? w[(co * c + ci) * khw + pos] : uint16_t{0};
  }
}

// Geometry accepted by the channels-last MFMA path.
bool nhwc_supported(int32_t dtype, const int64_t* g) {
  if (dtype != FH_BF16 && dtype != FH_F16 && dtype != FH_F32) return false;
  const int64_t n = g[0], cin = g[1], h = g[2], w = g[3], cout = g[4], kh = g[5], kw = g[6], sh = g[7], sw = g[8],
                ph = g[9], pw = g[10], groups = g[11];
  const int64_t es = dtype == FH_F32 ? 4 : 2, stage_k = 64 / es;
  // 16-bit: Cin % 32 == 0, or Cin == 8 (the C8 layout; a conv with fewer channels is packed to 8 first).
  // fp32: Cin % 16 == 0 (one 64-byte row of channels per stage).
  const bool c8 = es == 2 && cin == 8;
  if (groups != 1 || (cin % stage_k != 0 && !c8) || n <= 0 || h <= 0 || w <= 0 || cout <= 0 || kh <= 0 || kw <= 0)
    return false;
  if (sh <= 0 || sw <= 0 || ph < 0 || pw < 0 || h + 2 * ph < kh || w + 2 * pw < kw) return false;
  const int64_t oh = (h + 2 * ph - kh) / sh + 1, ow = (w + 2 * pw - kw) / sw + 1;
  // 32-bit offsets inside the kernel: input bytes, window origins and filter rows
  if (n * h * w * cin * es >= (int64_t{1} << 31)) return false;
  if (kh * kw * cin >= (int64_t{1} << 24) || n * oh * ow >= (int64_t{1} << 31)) return false;
  return true;
}

}  // namespace
}  // namespace fh

using namespace fh;

extern "C" fh_status fh_transpose_batched(int32_t itemsize, const void* x, void* y, int64_t batch, int64_t rows,
                                          int64_t cols, void* stream) {
  if (batch < 0 || rows < 0 || cols < 0) return fail(FH_INVALID_ARGUMENT, "fh_transpose_batched: negative size");
  if (batch == 0 || rows == 0 || cols == 0) return FH_OK;
  if (x == nullptr || y == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_transpose_batched: null pointer");
  if (batch > 65535) return fail(FH_UNIMPLEMENTED, "fh_transpose_batched: batch above 65535");
  if ((rows + 63) / 64 > 65535) return fail(FH_UNIMPLEMENTED, "fh_transpose_batched: too many row tiles");
  const dim3 grid(static_cast<uint32_t>((cols + 63) / 64), static_cast<uint32_t>((rows + 63) / 64),
                  static_cast<uint32_t>(batch));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (rows * cols <= kPlaneMax && batch <= 0x7fffffffLL) {
    if (itemsize == 2) {
      hipLaunchKernelGGL(transpose_plane_kernel<uint16_t>, dim3(static_cast<uint32_t>(batch)), dim3(256), 0, s,
                         static_cast<const uint16_t*>(x), static_cast<uint16_t*>(y), static_cast<int32_t>(rows),
                         static_cast<int32_t>(cols));
    } else if (itemsize == 4) {
      hipLaunchKernelGGL(transpose_plane_kernel<uint32_t>, dim3(static_cast<uint32_t>(batch)), dim3(256), 0, s,
                         static_cast<const uint32_t*>(x), static_cast<uint32_t*>(y), static_cast<int32_t>(rows),
                         static_cast<int32_t>(cols));
    } else {
      return fail(FH_INVALID_ARGUMENT, "fh_transpose_batched: itemsize must be 2 or 4");
    }
    return launch_status("transpose_plane_kernel launch");
  }
  if (itemsize == 2 && rows % 8 == 0 && aligned16(y)) {
    if (cols % 8 == 0 && aligned16(x)) {
      hipLaunchKernelGGL(transpose_wide_kernel<true>, grid, dim3(256), 0, s, static_cast<const uint16_t*>(x),
                         static_cast<uint16_t*>(y), rows, cols);
    } else {
      hipLaunchKernelGGL(transpose_wide_kernel<false>, grid, dim3(256), 0, s, static_cast<const uint16_t*>(x),
                         static_cast<uint16_t*>(y), rows, cols);
    }
    return launch_status("transpose_wide_kernel launch");
  }
  switch (itemsize) {
    case 2:
      hipLaunchKernelGGL(transpose_batched_kernel<uint16_t>, grid, dim3(256), 0, s, static_cast<const uint16_t*>(x),
                         static_cast<uint16_t*>(y), rows, cols);
      break;
    case 4:
      hipLaunchKernelGGL(transpose_batched_kernel<uint32_t>, grid, dim3(256), 0, s, static_cast<const uint32_t*>(x),
                         static_cast<uint32_t*>(y), rows, cols);
      break;
    default:
      return fail(FH_INVALID_ARGUMENT, "fh_transpose_batched: itemsize must be 2 or 4");
  }
  return launch_status("transpose_batched_kernel launch");
}

extern "C" fh_status fh_transpose_planes_multi(int32_t itemsize, int32_t n, const void* const* xs, void* const* ys,
                                               const int64_t* batch, const int64_t* rows, const int64_t* cols,
                                               void* stream) {
  if (n < 0 || n > kMultiMax) return fail(FH_INVALID_ARGUMENT, "fh_transpose_planes_multi: 0 to 32 tensors");
  if (n == 0) return FH_OK;
  if (xs == nullptr || ys == nullptr || batch == nullptr || rows == nullptr || cols == nullptr)
    return fail(FH_INVALID_ARGUMENT, "fh_transpose_planes_multi: null argument");
  if (itemsize != 2 && itemsize != 4) return fail(FH_INVALID_ARGUMENT, "fh_transpose_planes_multi: itemsize must be 2 or 4");
  PlaneBatch a{};
  int64_t max_batch = 0;
  for (int i = 0; i < n; ++i) {
    if (batch[i] < 0 || rows[i] < 0 || cols[i] < 0 || rows[i] * cols[i] > kPlaneMax || batch[i] > 0x7fffffffLL)
      return fail(FH_INVALID_ARGUMENT, "fh_transpose_planes_multi: planes of at most 8192 elements");
    if (batch[i] * rows[i] * cols[i] > 0 && (xs[i] == nullptr || ys[i] == nullptr))
      return fail(FH_INVALID_ARGUMENT, "fh_transpose_planes_multi: null tensor");
    a.x[i] = xs[i];
    a.y[i] = ys[i];
    a.batch[i] = rows[i] * cols[i] == 0 ? 0 : static_cast<int32_t>(batch[i]);
    a.rows[i] = static_cast<int32_t>(rows[i]);
    a.cols[i] = static_cast<int32_t>(cols[i]);
    max_batch = std::max<int64_t>(max_batch, a.batch[i]);
  }
  if (max_batch == 0) return FH_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  bool vec = itemsize == 2;
  int64_t max_threads = 0;
  for (int i = 0; i < n && vec; ++i) {
    if (a.batch[i] == 0) continue;
    vec = a.rows[i] % 8 == 0 && (a.cols[i] == 1 || a.cols[i] == 9) && aligned16(xs[i]) && aligned16(ys[i]);
    max_threads = std::max<int64_t>(max_threads, static_cast<int64_t>(a.batch[i]) * (a.rows[i] / 8));
  }
  if (vec) {
    const dim3 vgrid(static_cast<uint32_t>((max_threads + 255) / 256), static_cast<uint32_t>(n));
    hipLaunchKernelGGL(transpose_filters_vec_kernel, vgrid, dim3(256), 0, s, a);
    return launch_status("transpose_filters_vec_kernel launch");
  }
  const dim3 grid(static_cast<uint32_t>(max_batch), static_cast<uint32_t>(n));
  if (itemsize == 2) {
    hipLaunchKernelGGL(transpose_planes_multi_kernel<uint16_t>, grid, dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL(transpose_planes_multi_kernel<uint32_t>, grid, dim3(256), 0, s, a);
  }
  return launch_status("transpose_planes_multi_kernel launch");
}

extern "C" int32_t fh_conv2d_nhwc_supported(int32_t dtype, const int64_t geom[12]) {
  return geom != nullptr && nhwc_supported(dtype, geom) ? 1 : 0;
}

extern "C" int32_t fh_conv2d_nchw_in_supported(int32_t dtype, const int64_t geom[12]) {
  return geom != nullptr && nhwc_supported(dtype, geom) && halo_nchw_supported(dtype, geom) ? 1 : 0;
}

extern "C" fh_status fh_conv2d_nhwc_fwd_ex(int32_t dtype, const void* x_nhwc, const void* w_khwc, const void* bias,
                                           void* y, const int64_t geom[12], const fh_epilogue* epilogue,
                                           int32_t flags, void* stream);

extern "C" int32_t fh_conv2d_w_oihw_supported(int32_t dtype, const int64_t geom[12], const fh_epilogue* epilogue) {
  if (geom == nullptr || !nhwc_supported(dtype, geom) || !halo_nchw_supported(dtype, geom)) return 0;
  if (epilogue != nullptr && (epilogue->nseg < 0 || epilogue->nseg > FH_MAX_SEGMENTS)) return 0;
  ConvNhwcArgs a{};
  a.cout = static_cast<int32_t>(geom[4]);
  a.p = geom[0] * geom[2] * geom[3];  // 3x3, stride 1, padding 1: the output plane is the input plane
  a.vec_store = 1;
  if (epilogue != nullptr) {
    a.ep.nseg = epilogue->nseg;
    for (int s = 0; s < a.ep.nseg; ++s) {
      if (!epilogue_op_ok(epilogue->ops[s])) return 0;
      a.ep.ops[s] = epilogue->ops[s];
    }
  }
  return band_rows_for(dtype, a, geom) > 0 ? 1 : 0;
}

extern "C" fh_status fh_conv2d_nhwc_fwd(int32_t dtype, const void* x_nhwc, const void* w_khwc, const void* bias, void* y,
                                        const int64_t geom[12], const fh_epilogue* epilogue, void* stream) {
  return fh_conv2d_nhwc_fwd_ex(dtype, x_nhwc, w_khwc, bias, y, geom, epilogue, 0, stream);
}

namespace fh {
namespace {
// Checks the arguments of fh_conv2d_nhwc_fwd_ex and fills the kernel arguments (everything but the tiling).
fh_status nhwc_args(int32_t dtype, const void* x_nhwc, const void* w_khwc, const void* bias, void* y,
                    const int64_t geom[12], const fh_epilogue* epilogue, int32_t flags, ConvNhwcArgs* out) {
  if ((flags & ~(FH_CONV_OUT_NHWC | FH_CONV_IMPLICIT_GEMM | FH_CONV_IN_NCHW | FH_CONV_W_OIHW)) != 0)
    return fail(FH_INVALID_ARGUMENT, "fh_conv2d_nhwc_fwd_ex: unknown flags");
  const bool w_oihw = (flags & FH_CONV_W_OIHW) != 0;
  if (w_oihw && (flags & (FH_CONV_IN_NCHW | FH_CONV_OUT_NHWC | FH_CONV_IMPLICIT_GEMM)) != FH_CONV_IN_NCHW)
    return fail(FH_INVALID_ARGUMENT, "fh_conv2d_nhwc_fwd_ex: FH_CONV_W_OIHW goes with FH_CONV_IN_NCHW and NCHW output only");
  if (geom == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_conv2d_nhwc_fwd: null geometry");
  const bool nchw_in = (flags & FH_CONV_IN_NCHW) != 0;
  if (nchw_in && ((flags & FH_CONV_IMPLICIT_GEMM) != 0 || !halo_nchw_supported(dtype, geom)))
    return fail(FH_UNIMPLEMENTED, "fh_conv2d_nhwc_fwd_ex: FH_CONV_IN_NCHW needs the resident-patch geometry (bf16/f16, "
                                  "3x3, stride 1, padding 1, groups 1, Cin % 32 == 0, W % 8 == 0, a patch of at most "
                                  "30 KB) and excludes FH_CONV_IMPLICIT_GEMM");
  if (!nhwc_supported(dtype, geom))
    return fail(FH_UNIMPLEMENTED, "fh_conv2d_nhwc_fwd: geometry or dtype not supported by the channels-last path "
                                  "(needs groups 1 and bf16/f16 with Cin % 32 == 0 or Cin == 8, or fp32 with "
                                  "Cin % 16 == 0)");
  if (x_nhwc == nullptr || w_khwc == nullptr || y == nullptr)
    return fail(FH_INVALID_ARGUMENT, "fh_conv2d_nhwc_fwd: null pointer");
  if (!aligned16(x_nhwc) || !aligned16(w_khwc)) return fail(FH_INVALID_ARGUMENT, "fh_conv2d_nhwc_fwd: operands must be 16-byte aligned");
  ConvNhwcArgs& a = *out;
  a = ConvNhwcArgs{};
  a.x = x_nhwc;
  a.w = w_khwc;
  a.bias = bias;
  a.y = y;
  a.cin = static_cast<int32_t>(geom[1]);
  a.h = static_cast<int32_t>(geom[2]);
  a.w_in = static_cast<int32_t>(geom[3]);
  a.cout = static_cast<int32_t>(geom[4]);
  a.kh = static_cast<int32_t>(geom[5]);
  a.kw = static_cast<int32_t>(geom[6]);
  a.sh = static_cast<int32_t>(geom[7]);
  a.sw = static_cast<int32_t>(geom[8]);
  a.ph = static_cast<int32_t>(geom[9]);
  a.pw = static_cast<int32_t>(geom[10]);
  const int64_t oh = (geom[2] + 2 * geom[9] - geom[5]) / geom[7] + 1;
  const int64_t ow = (geom[3] + 2 * geom[10] - geom[6]) / geom[8] + 1;
  a.wo = static_cast<int32_t>(ow);
  a.howo = static_cast<int32_t>(oh * ow);
  const bool c8 = geom[1] == 8 && dtype != FH_F32;
  a.k = static_cast<int32_t>(c8 ? conv_c8_filter_k(geom[5], geom[6]) : geom[5] * geom[6] * geom[1]);
  a.p = geom[0] * oh * ow;
  const int64_t es = dtype == FH_F32 ? 4 : 2;
  a.x_bytes = static_cast<uint32_t>(geom[0] * geom[2] * geom[3] * geom[1] * es);
  if (epilogue != nullptr) {
    if (epilogue->nseg < 0 || epilogue->nseg > FH_MAX_SEGMENTS)
      return fail(FH_INVALID_ARGUMENT, "fh_conv2d_nhwc_fwd: epilogue nseg out of range");
    a.ep.nseg = epilogue->nseg;
    a.ep.round_between = epilogue->round_between;
    for (int s = 0; s < a.ep.nseg; ++s) {
      const uint8_t op = epilogue->ops[s];
      if (!epilogue_op_ok(op)) return fail(FH_INVALID_ARGUMENT, "fh_conv2d_nhwc_fwd: unknown epilogue op");
      if (ew_is_binary(op) && epilogue->ins[s] == nullptr)
        return fail(FH_INVALID_ARGUMENT, "fh_conv2d_nhwc_fwd: binary epilogue segment without operand");
      a.ep.ops[s] = op;
      a.ep.ins[s] = epilogue->ins[s];
    }
  }
  a.out_nhwc = (flags & FH_CONV_OUT_NHWC) ? 1 : 0;
  const int64_t vwidth = dtype == FH_F32 ? 4 : 8;  // elements per 16-byte vector
  bool vec = (a.out_nhwc ? a.cout % vwidth == 0 : a.howo % vwidth == 0) && aligned16(y);
  for (int s = 0; s < a.ep.nseg; ++s)
    if (ew_is_binary(a.ep.ops[s]) && !aligned16(a.ep.ins[s])) vec = false;
  a.vec_store = vec ? 1 : 0;
  return FH_OK;
}
}  // namespace
}  // namespace fh

extern "C" fh_status fh_conv2d_nhwc_fwd_ex(int32_t dtype, const void* x_nhwc, const void* w_khwc, const void* bias,
                                           void* y, const int64_t geom[12], const fh_epilogue* epilogue,
                                           int32_t flags, void* stream) {
  ConvNhwcArgs a{};
  if (const fh_status st = nhwc_args(dtype, x_nhwc, w_khwc, bias, y, geom, epilogue, flags, &a); st != FH_OK) return st;
  const bool w_oihw = (flags & FH_CONV_W_OIHW) != 0, nchw_in = (flags & FH_CONV_IN_NCHW) != 0;
  const bool c8 = geom[1] == 8 && dtype != FH_F32;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (w_oihw) {
    const int rows = band_rows_for(dtype, a, geom);
    if (rows == 0)
      return fail(FH_UNIMPLEMENTED, "fh_conv2d_nhwc_fwd_ex: FH_CONV_W_OIHW needs the band kernel (bf16, 3x3 stride 1 "
                                    "padding 1, Cin 64, Cout <= 64, W % 8 == 0, 16-byte aligned output and operands, "
                                    "no epilogue, relu or add;relu); see fh_conv2d_w_oihw_supported");
    if (a.p == 0) return FH_OK;
    return launch_band<true>(a, rows, s);
  }
  if (a.p == 0) return FH_OK;
  if ((dtype == FH_BF16 || dtype == FH_F16) && !c8 && (flags & FH_CONV_IMPLICIT_GEMM) == 0) {
    bool launched = false;
    const fh_status st = dtype == FH_BF16 ? dispatch_halo<bf16_t>(a, geom, s, &launched, nchw_in)
                                          : dispatch_halo<f16_t>(a, geom, s, &launched, nchw_in);
    if (launched || st != FH_OK) return st;
    if (nchw_in) return fail(FH_INTERNAL, "fh_conv2d_nhwc_fwd_ex: NCHW input accepted but no kernel launched");
  }
  if (dtype == FH_F32) return dispatch_conv<float, false>(a, s);
  if (c8) return dtype == FH_BF16 ? dispatch_conv<bf16_t, true>(a, s) : dispatch_conv<f16_t, true>(a, s);
  return dtype == FH_BF16 ? dispatch_conv<bf16_t, false>(a, s) : dispatch_conv<f16_t, false>(a, s);
}

namespace fh {
namespace {
// Split count of fh_conv2d_nhwc_fwd_split's planned form, or 0 where the unsplit kernels run. Measured on an MI355X
// (ResNet-18 layer 4 at batch 64, bf16, 64 x 64 unsplit vs 128 x 128 tiles split in two): 3x3 stride 1, K = 4608:
// 36.6 -> 30.4 us (add;relu), 34.0 -> 30.4 us (relu); 3x3 stride 2, K = 2304: 19.0 -> 21.3 us, so not split; more
// splits than the CUs hold in one round of 128 x 128 tiles were slower (3: 34 us, 8: 43 us). So: 16-bit,
// channels-last output of whole 128-channel tiles, not C8, a channel count the resident-patch kernels do not take
// (Cout > 256), at least 128 k stages, and as many splits as whole rounds of tiles fit the CUs once (at least two).
int32_t split_plan(int32_t dtype, const int64_t* g, int32_t flags) {
  if ((dtype != FH_BF16 && dtype != FH_F16) || flags != FH_CONV_OUT_NHWC || !nhwc_supported(dtype, g)) return 0;
  if (g[1] == 8 || g[4] % 128 != 0 || g[4] <= 256) return 0;
  const int64_t oh = (g[2] + 2 * g[9] - g[5]) / g[7] + 1, ow = (g[3] + 2 * g[10] - g[6]) / g[8] + 1;
  const int64_t tiles = g[4] / 128 * ((g[0] * oh * ow + 127) / 128);
  const int64_t cus = device_cu_count();
  const int32_t kt = static_cast<int32_t>(g[5] * g[6] * g[1] / 32);
  if (kt < 128) return 0;
  const int64_t want = std::min<int64_t>(cus / tiles, kt / 32);
  return want >= 2 ? split_count(kt, static_cast<int32_t>(want)) : 0;
}
}  // namespace
}  // namespace fh

extern "C" int64_t fh_conv2d_nhwc_split_workspace(int32_t dtype, const int64_t geom[12], int32_t flags, int32_t* splits) {
  if (geom == nullptr || splits == nullptr) return -1;
  int32_t n = *splits;
  if (n <= 0) {
    n = split_plan(dtype, geom, flags);
  } else {
    if ((dtype != FH_BF16 && dtype != FH_F16) || flags != FH_CONV_OUT_NHWC || !nhwc_supported(dtype, geom) ||
        geom[1] == 8 || geom[4] % 128 != 0)
      return -1;
    n = split_count(static_cast<int32_t>(geom[5] * geom[6] * geom[1] / 32), n);
  }
  *splits = n;
  if (n <= 1) return 0;
  const int64_t oh = (geom[2] + 2 * geom[9] - geom[5]) / geom[7] + 1, ow = (geom[3] + 2 * geom[10] - geom[6]) / geom[8] + 1;
  return int64_t{n} * geom[0] * oh * ow * geom[4] * 4;
}

extern "C" fh_status fh_conv2d_nhwc_fwd_split(int32_t dtype, const void* x_nhwc, const void* w_khwc, const void* bias,
                                              void* y, const int64_t geom[12], const fh_epilogue* epilogue,
                                              int32_t flags, int32_t splits, void* workspace, int64_t workspace_bytes,
                                              void* stream) {
  if (geom == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_conv2d_nhwc_fwd_split: null geometry");
  int32_t n = splits;
  const int64_t need = fh_conv2d_nhwc_split_workspace(dtype, geom, flags, &n);
  if (need < 0)
    return fail(FH_UNIMPLEMENTED, "fh_conv2d_nhwc_fwd_split: split K needs bf16/f16, FH_CONV_OUT_NHWC only, "
                                  "Cin % 32 == 0 and Cout % 128 == 0");
  if (need == 0) return fh_conv2d_nhwc_fwd_ex(dtype, x_nhwc, w_khwc, bias, y, geom, epilogue, flags, stream);
  ConvNhwcArgs a{};
  if (const fh_status st = nhwc_args(dtype, x_nhwc, w_khwc, bias, y, geom, epilogue, flags, &a); st != FH_OK) return st;
  if (workspace == nullptr || workspace_bytes < need)
    return fail(FH_INVALID_ARGUMENT, "fh_conv2d_nhwc_fwd_split: workspace smaller than fh_conv2d_nhwc_split_workspace");
  if (!aligned16(workspace) || (bias != nullptr && !aligned16(bias)) || !a.vec_store)
    return fail(FH_INVALID_ARGUMENT, "fh_conv2d_nhwc_fwd_split: workspace, bias, y and the epilogue operands must be "
                                     "16-byte aligned");
  if (a.p == 0) return FH_OK;
  a.part = static_cast<float*>(workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dtype == FH_BF16 ? launch_conv_split<bf16_t, 128, 128, 2, 4>(a, n, s) : launch_conv_split<f16_t, 128, 128, 2, 4>(a, n, s);
}

extern "C" fh_status fh_conv_pack_input_c8(const void* x, void* y, int64_t n, int32_t c, int64_t hw, void* stream) {
  if (n < 0 || hw < 0 || c < 1 || c > 8) return fail(FH_INVALID_ARGUMENT, "fh_conv_pack_input_c8: needs 1 <= C <= 8");
  if (n * hw == 0) return FH_OK;
  if (x == nullptr || y == nullptr || !aligned16(y)) return fail(FH_INVALID_ARGUMENT, "fh_conv_pack_input_c8: bad pointer");
  if (n <= 65535 && hw < (int64_t{1} << 31)) {
    const dim3 grid(static_cast<uint32_t>((hw + 255) / 256), static_cast<uint32_t>(n));
    hipLaunchKernelGGL(pack_input_c8_2d_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint16_t*>(x), static_cast<uint4*>(y), c, static_cast<int32_t>(hw));
    return launch_status("pack_input_c8_2d_kernel launch");
  }
  int64_t blocks = (n * hw + 255) / 256;
  blocks = blocks > 256LL * 16 ? 256LL * 16 : blocks;
  hipLaunchKernelGGL(pack_input_c8_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(x), static_cast<uint4*>(y), n, c, hw);
  return launch_status("pack_input_c8_kernel launch");
}

extern "C" int64_t fh_conv_c8_filter_k(int64_t kh, int64_t kw) { return conv_c8_filter_k(kh, kw); }

extern "C" fh_status fh_conv_pack_filter_c8(const void* w, void* y, int32_t cout, int32_t c, int32_t kh, int32_t kw,
                                            void* stream) {
  if (cout < 1 || c < 1 || c > 8 || kh < 1 || kw < 1) return fail(FH_INVALID_ARGUMENT, "fh_conv_pack_filter_c8: bad shape");
  if (w == nullptr || y == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_conv_pack_filter_c8: null pointer");
  const int32_t k = static_cast<int32_t>(conv_c8_filter_k(kh, kw));
  const int64_t total = static_cast<int64_t>(cout) * k;
  hipLaunchKernelGGL(pack_filter_c8_kernel, dim3(static_cast<uint32_t>((total + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(w), static_cast<uint16_t*>(y), cout, c,
                     kh * kw, k);
  return launch_status("pack_filter_c8_kernel launch");
}
