// Fused scaled dot-product attention for Frame's per-(batch, head) decomposition (reference:
// src/nn/layers.cpp:1014-1080). For batch b and head h, with Q/K/V the [batch*seq, heads*dh] projections:
//   S  = round(Q_bh · K_bhᵀ)            (matmul, fp32 accumulate, one rounding)
//   S2 = round(S * scale)                (mul by the 1/sqrt(dh) constant splat)
//   P  = softmax rows of S2, rounded     (m = max, e = exp(x - m), s = sum e, y = round(e / s))
//   O  = round(P · V_bh)                 (matmul)
// and O lands at rows [b*seq, (b+1)*seq), columns [h*dh, (h+1)*dh) of the output: the layout of the reference's
// head concat (axis 1) and batch concat (axis 0). S and S2 are rounded where the reference rounds them, m is the
// exact row maximum of S2, and the stored probabilities are round(e / s) as the reference's softmax stores them,
// so P·V multiplies the same 16-bit P. What differs from the decomposition: the summation orders (MFMA blocks,
// per-lane partial sums of e), the exponential (v_exp_f32 of x log2(e) - m log2(e) instead of expf(x - m), within
// a few fp32 ulps), and e / s evaluated as e * (1 / s) (within one fp32 rounding); each changes a stored
// probability only where the exact value lies that close to a 16-bit rounding boundary, and the tests report the
// fraction of outputs that come out bit-identical (above 99.7 % at 512 keys).
//
// attention_kernel: one wave owns 32 queries and all seq keys; a workgroup is W waves (4, or 2 when seq is not a
// multiple of 128). attention_split_kernel (bf16, seq % 128 == 0) splits each query block's keys over two waves.
// The unsplit kernel is bound by its VALU instruction stream (about 9 VALU instructions and two quarter-rate
// exponentials per score, against two MFMA k-steps per 32 x 32 tile), so the per-score code is kept short; the
// split kernel evaluates one exponential per score.
//  1. Scores transposed, Sᵀ = K·Qᵀ on v_mfma_f32_32x32x16, per 64-key block: K blocks go to LDS
//     (global_load_lds_dwordx4, 16-byte chunks swizzled by row), all requested at the start; the Q fragments
//     stay in registers. Each lane's accumulator then holds one query and 16 keys of a 32-key tile; they are
//     rounded, scaled, rounded and kept as packed bf16/f16 in registers (seq/2 values per lane). The running
//     maximum is taken over the scaled values before their rounding: rounding is monotonic, so the rounded
//     maximum is the maximum of the rounded values.
//  2. m per query: the lane's maximum and its partner lane's (lane ^ 32, same query); then s, the sum of
//     e = exp(S2 - m) over the lane's keys and its partner's.
//  3. Oᵀ = Vᵀ·Pᵀ: p = round(e / s) is produced in registers already in the B-operand layout (k = the lane's 8
//     keys of one query, in the accumulator's key order); the A operand (Vᵀ) comes from V blocks in LDS through
//     ds_read_b64_tr_b16 in the same key order. V block b replaces K block b in LDS once every wave has read it.
//     The output is round(acc).
// LDS: seq x 128 bytes per workgroup (64 KB at seq 512), so two workgroups share a CU.
#include <hip/hip_runtime.h>

#include <cmath>
#include <string>
#include <type_traits>
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
  // the sum of the exponentials first, so that pass 3 stores round(e / s) as the reference's softmax does (every
  // exponential is evaluated here and again in pass 3); e / s as e * (1 / s), see attention_split_kernel
  float esum = 0.0f;
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t w = s2[t][j];
      esum += __builtin_amdgcn_exp2f(__builtin_fmaf(lo16<T>(w), c, -ml)) +
              __builtin_amdgcn_exp2f(__builtin_fmaf(hi16<T>(w), c, -ml));
    }
  const float r = 1.0f / (esum + __shfl_xor(esum, 32));
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
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                uint32_t w = s2[t][4 * hf + j];
                asm volatile("" : "+v"(w));  // keeps the exp of this tile here, after the block's barrier
                const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(lo16<T>(w), c, -ml));
                const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(hi16<T>(w), c, -ml));
                pf[hf][j] = pack2<T>(e0 * r, e1 * r);  // P = round(e / s)
              }
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
  uint16_t* orow = out + base + static_cast<int64_t>(q0 + l32) * ld;
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      u32x2_t w;
      w[0] = pack2<T>(acc_o[dt][4 * gq], acc_o[dt][4 * gq + 1]);
      w[1] = pack2<T>(acc_o[dt][4 * gq + 2], acc_o[dt][4 * gq + 3]);
      *reinterpret_cast<u32x2_t*>(orow + 32 * dt + 8 * gq + 4 * hi) = w;
    }
}

// Key-split form for seq % 128 == 0. A workgroup is 8 waves over 128 queries: waves w and w + 4 own the same 32
// queries, w < 4 the first half of the keys and w >= 4 the second. Each wave keeps the packed scores of seq / 2
// keys (64 registers at seq 512) and, after the row maximum is known, their fp32 exponentials (128 registers), so
// every exponential is evaluated once: the sum pass stores them and the P pass only scales and rounds them (at C5's
// shape 21.1 us against 23.0 us when pass 3 evaluated them again with four waves per SIMD; the registers leave two
// waves per SIMD, one workgroup per CU). With more tasks (128-query blocks) than CUs a workgroup runs two tasks
// from two LDS buffers: the second task's Q fragments and K blocks are requested right after the first task's last
// V blocks, so they arrive while the first task finishes (20.8 us against 21.2-21.4 us with the second task as a
// second round of workgroups). The blocks of K (then V) are loaded by all 8 waves, the halves' blocks in
// pairs (i, NB/2 + i) so both halves start together. Per query the halves combine through LDS: the row maximum
// (exact either way), the sum of the exponentials s = s_first + s_second, and the fp32 products P·V: half h
// writes the output's d tile h (32 columns) as round(O_first + O_second), taking the other half's partial from
// LDS. Everything else (roundings, exponentials, key order inside a half) is attention_kernel's.
template <typename T, int NB, bool POW2>
__global__ __launch_bounds__(512, 1) void attention_split_kernel(const uint16_t* __restrict__ q,
                                                                 const uint16_t* __restrict__ k,
                                                                 const uint16_t* __restrict__ v,
                                                                 uint16_t* __restrict__ out, int heads, float scale,
                                                                 int tasks) {
  constexpr int SEQ = NB * 64;
  constexpr int H = NB / 2;        // 64-key blocks per half
  constexpr int NTH = 2 * H;       // 32-key tiles per half
  constexpr int BLK = 64 * 128;    // one 64-key block of K or V, bytes
  static_assert(NB % 2 == 0 && 2 * NB < 64, "whole block pairs; vmcnt range");
  // K / V blocks, then the halves' fp32 partial products: 8 waves x 64 lanes x 16 floats = 32 KB
  constexpr int KV_BYTES = NB * BLK > 8 * 64 * 16 * 4 ? NB * BLK : 8 * 64 * 16 * 4;
  // two task buffers: the next task's K blocks land in one while the current task runs in the other
  __shared__ __attribute__((aligned(1024))) unsigned char kvs[2][KV_BYTES];
  __shared__ float xmax[8][64], xsum[8][64];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int half = wave >> 2;
  const int l32 = lane & 31, hi = lane >> 5;
  const int nq = SEQ / 128;
  const int64_t ld = static_cast<int64_t>(heads) * kDh;
  // Task -> (query block, head, batch), XCD-aware: workgroup L runs on XCD L % 8 and takes tasks L and
  // L + gridDim.x; the remap gives each XCD consecutive (head, batch) pairs with all their query blocks, so the
  // 4 workgroups that read one pair's K and V share that XCD's L2 (tasks L and L + gridDim.x stay on L's XCD when
  // gridDim.x is a multiple of 8).
  auto geo = [&](int t, int64_t& base, int& q0) {
    int idx = t;
    if ((tasks & 7) == 0) idx = (idx & 7) * (tasks >> 3) + (idx >> 3);
    const int qb = idx % nq, hb = idx / nq;
    const int h = hb % heads, b = hb / heads;
    q0 = qb * 128 + (wave & 3) * 32;
    base = (static_cast<int64_t>(b) * SEQ) * ld + static_cast<int64_t>(h) * kDh;
  };
  auto load_q = [&](int64_t base, int q0, u32x4_t (&qf)[4]) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
      qf[s] = *reinterpret_cast<const u32x4_t*>(q + base + static_cast<int64_t>(q0 + l32) * ld + 16 * s + 8 * hi);
  };
  // one 1 KB instruction per wave and block: rows 8 wave .. 8 wave + 7
  auto load_block_to = [&](unsigned char* buf, int64_t base, const uint16_t* src, int blk, bool is_v) {
    const int row = 8 * wave + (lane >> 3), pc = lane & 7;
    const int c = is_v ? v_chunk(row, pc) : k_chunk(row, pc);
    const uint16_t* g = src + base + static_cast<int64_t>(blk * 64 + row) * ld + c * 8;
    __builtin_amdgcn_global_load_lds(g, (FH_LDS void*)(buf + blk * BLK + wave * 1024), 16, 0, 0);
  };
  auto issue_k = [&](unsigned char* buf, int64_t base) {
#pragma unroll
    for (int i = 0; i < H; ++i) {
      load_block_to(buf, base, k, i, false);
      load_block_to(buf, base, k, H + i, false);
    }
  };
  auto barrier = [] {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  // One task whose Q fragments and K blocks were requested before (their loads are the oldest outstanding ones).
  // NEXT: request the next task's (4 + NB loads per wave) after this task's last V loads. PRIOR: the previous
  // task's 4 output stores were issued after this task's K loads, so they are in flight during pass 1.
  auto run = [&]<bool NEXT, bool PRIOR>(unsigned char* kv, int64_t base, int q0, u32x4_t (&qf)[4],
                                        unsigned char* nbuf, int64_t nbase, int nq0, u32x4_t (&qfn)[4]) {
    constexpr int NEXT_LOADS = NEXT ? 4 + NB : 0;
    auto load_block = [&](const uint16_t* src, int blk, bool is_v) { load_block_to(kv, base, src, blk, is_v); };
    const uint32_t kv_addr = lds_addr((const FH_LDS void*)kv);
    const uint32_t half_addr = kv_addr + half * H * BLK;  // this half's first block
    uint32_t k_off[4];
  #pragma unroll
    for (int s = 0; s < 4; ++s) k_off[s] = half_addr + l32 * 128 + k_chunk(l32, 2 * s + hi) * 16;

    // ---- 1. scores of this half's keys ----
    uint32_t s2[NTH][8];
    float mraw = -__builtin_inff();
    [&]<int... B_>(std::integer_sequence<int, B_...>) {
      (
          [&] {
            constexpr int i = B_;
            // K pair i has landed when no more than the loads issued after it are in flight: K pairs i+1 .. H-1
            // and V pairs 0 .. i-2
            wait_vmcnt<2 * (H - 1 - i) + 2 * (i >= 2 ? i - 1 : 0) + (PRIOR ? 4 : 0)>();
            barrier();
            if constexpr (i >= 1) {  // every wave has read K pair i - 1
              load_block(v, i - 1, true);
              load_block(v, H + i - 1, true);
            }
            // one 32-key tile at a time: 16 fragment and 16 accumulator registers
            auto tile = [&]<int t>() {
              u32x4_t kf[4];
  #pragma unroll
              for (int s = 0; s < 4; ++s) kf[s] = lds_read_b128<i * BLK + t * 4096>(k_off[s]);
              asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  #pragma unroll
              for (int s = 0; s < 4; ++s) asm volatile("" : "+v"(kf[s]));
              f32x16_t acc;
  #pragma unroll
              for (int x = 0; x < 16; ++x) acc[x] = 0.0f;
  #pragma unroll
              for (int s = 0; s < 4; ++s) mfma32<T>(kf[s], qf[s], acc);
  #pragma unroll
              for (int j = 0; j < 8; ++j) {
                const uint32_t sr = pack2<T>(acc[2 * j], acc[2 * j + 1]);
                if constexpr (POW2) {
                  float mx;
                  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(mx) : "v"(mraw), "v"(acc[2 * j]), "v"(acc[2 * j + 1]));
                  mraw = mx;
                  s2[2 * i + t][j] = sr;
                } else {
                  const float a0 = lo16<T>(sr) * scale, a1 = hi16<T>(sr) * scale;
                  mraw = fmaxf(mraw, fmaxf(a0, a1));
                  s2[2 * i + t][j] = pack2<T>(a0, a1);
                }
                asm volatile("" : "+v"(s2[2 * i + t][j]));
              }
            };
            tile.template operator()<0>();
            tile.template operator()<1>();
          }(),
          ...);
    }(std::make_integer_sequence<int, H>{});

    // ---- 2. row maximum over both halves ----
    xmax[wave][lane] = fmaxf(mraw, __shfl_xor(mraw, 32));
    barrier();  // also: every wave has read K pair H - 1
    load_block(v, H - 1, true);
    load_block(v, NB - 1, true);
    if constexpr (NEXT) {  // the next task's Q fragments and K blocks, into the other buffer
      load_q(nbase, nq0, qfn);
      asm volatile("" ::: "memory");
      issue_k(nbuf, nbase);
    }
    const float mh0 = xmax[wave & 3][lane], mh1 = xmax[(wave & 3) + 4][lane];
    constexpr float kLog2e = 1.44269504088896340736f;
    const float mr = Io<T>::round(fmaxf(mh0, mh1));
    const float m = POW2 ? mr * scale : mr;
    const float ml = m * kLog2e;
    const float c = POW2 ? scale * kLog2e : kLog2e;

    // ---- 3. this half's share of Oᵀ = Vᵀ·Pᵀ ----
    f32x16_t acc_o[2];
  #pragma unroll
    for (int dt = 0; dt < 2; ++dt)
  #pragma unroll
      for (int x = 0; x < 16; ++x) acc_o[dt][x] = 0.0f;
    const int g = lane >> 4, rr = lane & 15, qd = rr & 3, e = rr >> 2;
    uint32_t v_off[2];
  #pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      const int n0 = 32 * dt + 16 * (g & 1) + 4 * qd;
      const int krow = 4 * (g >> 1) + e;
      v_off[dt] = half_addr + krow * 128 + v_chunk(krow, n0 >> 3) * 16 + (n0 & 7) * 2;
    }
    // ---- 2b. the exponentials and their sum over both halves, so that pass 3 stores round(e / s) as the reference's
    // softmax does ----
    float esum = 0.0f;
    float ev[NTH][16];  // the exponentials, kept in fp32 for pass 3
  #pragma unroll
    for (int t = 0; t < NTH; ++t)
  #pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t w = s2[t][j];
        ev[t][2 * j] = __builtin_amdgcn_exp2f(__builtin_fmaf(lo16<T>(w), c, -ml));
        ev[t][2 * j + 1] = __builtin_amdgcn_exp2f(__builtin_fmaf(hi16<T>(w), c, -ml));
        esum += ev[t][2 * j] + ev[t][2 * j + 1];
      }
    xsum[wave][lane] = esum + __shfl_xor(esum, 32);
    wait_vmcnt<2 + NEXT_LOADS>();  // this wave's V pairs 0 .. H-2 (V pair H-1 and the next task's loads may be in flight)
    barrier();
    // e / s as e * (1 / s): the two differ by at most one fp32 rounding, which changes the stored 16-bit probability
    // only when e / s lies within that rounding of a 16-bit rounding boundary
    const float r = 1.0f / (xsum[wave & 3][lane] + xsum[(wave & 3) + 4][lane]);
    [&]<int... B_>(std::integer_sequence<int, B_...>) {
      (
          [&] {
            constexpr int i = B_;
            if constexpr (i == H - 1) {
              wait_vmcnt<NEXT_LOADS>();
              barrier();
            }
  #pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
              const int t = 2 * i + tt;
              // V fragments of one d tile at a time (8 registers): d tile 0's are read before the exponentials,
              // d tile 1's while d tile 0's products run
              auto read_v = [&]<int dt>(u32x2_t (&vf)[2][2]) {
                [&]<int... R_>(std::integer_sequence<int, R_...>) {
                  (
                      [&] {
                        constexpr int hf = R_ / 2, part = R_ % 2;
                        constexpr int off = i * BLK + (16 * hf + 8 * part) * 128;
                        vf[hf][part] = lds_read_tr16_b64<off>(v_off[dt] + tt * 32 * 128);
                      }(),
                      ...);
                }(std::make_integer_sequence<int, 4>{});
              };
              u32x2_t vf[2][2];
              read_v.template operator()<0>(vf);
              u32x4_t pf[2];
  #pragma unroll
              for (int hf = 0; hf < 2; ++hf)
  #pragma unroll
                for (int j = 0; j < 4; ++j)
                  pf[hf][j] = pack2<T>(ev[t][8 * hf + 2 * j] * r, ev[t][8 * hf + 2 * j + 1] * r);  // P = round(e / s)
              auto multiply = [&](u32x2_t (&f)[2][2], f32x16_t& acc) {
  #pragma unroll
                for (int hf = 0; hf < 2; ++hf) {
                  asm volatile("" : "+v"(f[hf][0]), "+v"(f[hf][1]));
                  const u32x4_t a{f[hf][0][0], f[hf][0][1], f[hf][1][0], f[hf][1][1]};
                  mfma32<T>(a, pf[hf], acc);
                }
              };
              asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
              multiply(vf, acc_o[0]);
              read_v.template operator()<1>(vf);
              asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
              multiply(vf, acc_o[1]);
            }
          }(),
          ...);
    }(std::make_integer_sequence<int, H>{});

    // ---- output: half h writes d tile h from its partial and its partner's (kv is free: every V read is done) ----
    float* xo = reinterpret_cast<float*>(kv);
    {
      const int other = 1 - half;
      float4* dst = reinterpret_cast<float4*>(xo + (wave * 64 + lane) * 16);
      barrier();  // every wave's V reads are complete before kv is overwritten
  #pragma unroll
      for (int x4 = 0; x4 < 4; ++x4)
        dst[x4] = make_float4(acc_o[other][4 * x4], acc_o[other][4 * x4 + 1], acc_o[other][4 * x4 + 2], acc_o[other][4 * x4 + 3]);
    }
    barrier();
    const float4* src = reinterpret_cast<const float4*>(xo + ((wave ^ 4) * 64 + lane) * 16);
    f32x16_t o = half == 0 ? acc_o[0] : acc_o[1];
  #pragma unroll
    for (int x4 = 0; x4 < 4; ++x4) {
      const float4 p = src[x4];
      o[4 * x4] += p.x;
      o[4 * x4 + 1] += p.y;
      o[4 * x4 + 2] += p.z;
      o[4 * x4 + 3] += p.w;
    }
    uint16_t* orow = out + base + static_cast<int64_t>(q0 + l32) * ld + 32 * half;
  #pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      u32x2_t w;
      w[0] = pack2<T>(o[4 * gq], o[4 * gq + 1]);
      w[1] = pack2<T>(o[4 * gq + 2], o[4 * gq + 3]);
      *reinterpret_cast<u32x2_t*>(orow + 8 * gq + 4 * hi) = w;
    }

  };

  const int t0 = static_cast<int>(blockIdx.x), t1 = t0 + static_cast<int>(gridDim.x);
  int64_t base0, base1 = 0;
  int q00, q01 = 0;
  geo(t0, base0, q00);
  u32x4_t qf0[4], qf1[4];
  load_q(base0, q00, qf0);
  asm volatile("" ::: "memory");
  issue_k(kvs[0], base0);
  if (t1 < tasks) {
    geo(t1, base1, q01);
    run.template operator()<true, false>(kvs[0], base0, q00, qf0, kvs[1], base1, q01, qf1);
    run.template operator()<false, true>(kvs[1], base1, q01, qf1, kvs[0], 0, 0, qf0);
  } else {
    run.template operator()<false, false>(kvs[0], base0, q00, qf0, kvs[1], 0, 0, qf1);
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
      // bf16 takes the key-split form (8 waves over the same 128 queries) where seq % 128 == 0; f16's conversions
      // need more registers than its four waves per SIMD allow, so f16 keeps the unsplit kernel
      // (the split form's workgroups form one flat grid, hence the 2^31 bound)
      const int64_t flat = int64_t{grid.x} * grid.y * grid.z;
      if constexpr (NB % 2 == 0 && std::is_same_v<T, bf16_t>) {
        if (flat <= 0x7fffffff) {
          // more tasks than CUs: each workgroup runs two (one workgroup per CU fits), the second one's loads
          // issued while the first finishes
          const int64_t wgs = flat > device_cu_count() ? (flat + 1) / 2 : flat;
          hipLaunchKernelGGL((attention_split_kernel<T, NB, P>), dim3(static_cast<uint32_t>(wgs)), dim3(512), 0, s, qq,
                             kk, vv, oo, hd, scale, static_cast<int>(flat));
          return;
        }
      }
      (void)flat;
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
