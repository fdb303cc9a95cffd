// bf16 / f16 GEMM for gfx950: C[M,N] = A[M,K] · B[K,N], row-major, fp32 accumulation on
// v_mfma_f32_32x32x16_{bf16,f16}, one round-to-nearest-even per output, then the optional elementwise epilogue
// (semantics of Frame's matmul: reference src/backends/cpu/kernels/matmul.cpp:92-185).
//
// Data path (CDNA4-specific):
//  * Operands go global -> LDS with global_load_lds_dwordx4 (no VGPR staging): every wave instruction writes
//    1 KB of LDS contiguously, lane L at +16*L. The lane -> global address map applies an XOR swizzle of the
//    16-byte chunks inside each LDS row, so the fragment reads below are bank-conflict free.
//  * A tile: [BM rows][32 k] bf16 = 64 B per row, chunk swizzle c ^ ((row >> 1) & 3). A fragments are
//    ds_read_b128 (8 consecutive k of one row per lane), the MFMA's A layout.
//  * B tile: [32 k rows][BN n] bf16 kept n-contiguous as in memory, chunk swizzle c ^ (2 * (k & 3)).
//    B fragments need 8 consecutive k of one column per lane; ds_read_b64_tr_b16 (gfx950 LDS transpose read)
//    delivers them in two reads of 4 k each, with no register transposes.
//  * A ring of 4 LDS stages of BK = 32: loads for stage kt+3 are issued while stage kt is multiplied, so about
//    three stages of MFMA work cover the global-load latency. Waits use explicit vmcnt counts and a bare
//    s_barrier, so prefetched stages are never waited for early.
//  * Workgroups are remapped XCD-aware (consecutive tile ids on one XCD) and grouped along M for L2 reuse.
//  * Epilogue: the rounded tile is staged through LDS per wave and written with 16-byte stores; epilogue
//    operands are read with matching 16-byte loads.
#include <hip/hip_runtime.h>

#include <string>
#include <type_traits>
#include <utility>

#include "fh_common.h"
#include "fh_gemm.h"

namespace fh {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

#define FH_LDS __attribute__((address_space(3)))

constexpr int kBK = 32;      // k per stage
constexpr int kStages = 4;   // LDS ring depth

template <typename T, typename V>
__device__ __forceinline__ void mfma32(const V& a, const V& b, f32x16_t& acc) {
  static_assert(sizeof(V) == 16, "8 x 16-bit fragments");
  if constexpr (std::is_same_v<T, bf16_t>) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                  acc, 0, 0, 0);
  } else {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b),
                                                 acc, 0, 0, 0);
  }
}

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[15:14]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

// Fragment reads are written as inline asm without a memory clobber. The compiler's LDS-DMA wait tracking does
// not follow the stage ring across the loop (it either waits for every in-flight prefetch or, on other paths,
// for nothing), so the main loop orders LDS itself: explicit vmcnt waits + s_barrier before a stage is read,
// and fragment_fence() (lgkmcnt(0), tied to the fragment registers) before the MFMAs consume them.
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

// Keeps an accumulator's MFMA above later fences: VGPR or AGPR constraint, wherever the accumulators live.
template <bool IN_AGPR>
__device__ __forceinline__ void pin(f32x16_t& acc) {
  if constexpr (IN_AGPR) {
    asm volatile("" : "+a"(acc));
  } else {
    asm volatile("" : "+v"(acc));
  }
}

// Waits until at most PENDING LDS reads are outstanding (they complete in order), then ties the fragment
// registers to the wait so no consumer is scheduled above it.
template <int PENDING, int TM, int TN>
__device__ __forceinline__ void fragment_fence(u32x4_t (&a)[TM], u32x4_t (&b)[TN]) {
  static_assert(PENDING >= 0 && PENDING <= 15, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(PENDING) : "memory");
#pragma unroll
  for (int i = 0; i < TM; ++i) asm volatile("" : "+v"(a[i]));
#pragma unroll
  for (int j = 0; j < TN; ++j) asm volatile("" : "+v"(b[j]));
}

__device__ __forceinline__ uint32_t lds_addr(const FH_LDS void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}

__device__ __forceinline__ void global_to_lds16(const void* g, FH_LDS void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(g, lds_wave_base, 16, 0, 0);
}

// Runs the epilogue program on 8 rounded outputs (one 16-byte vector) at flat output index idx.
template <typename T>
__device__ __forceinline__ uint4 apply_epilogue_vec(const EpilogueArgs& ep, uint4 packed, int64_t idx) {
  using S = uint16_t;
  S vals[8];
  __builtin_memcpy(vals, &packed, 16);
  float v[8];
#pragma unroll
  for (int x = 0; x < 8; ++x) v[x] = Io<T>::load(vals[x]);
  for (int sg = 0; sg < ep.nseg; ++sg) {
    const uint8_t op = ep.ops[sg];
    if (ew_is_binary(op)) {
      const uint4 in = *reinterpret_cast<const uint4*>(static_cast<const S*>(ep.ins[sg]) + idx);
      S iv[8];
      __builtin_memcpy(iv, &in, 16);
#pragma unroll
      for (int x = 0; x < 8; ++x) v[x] = ew_binary(op, v[x], Io<T>::load(iv[x]));
    } else {
#pragma unroll
      for (int x = 0; x < 8; ++x) v[x] = ew_unary(op, v[x]);
    }
    if (ep.round_between) {
#pragma unroll
      for (int x = 0; x < 8; ++x) v[x] = Io<T>::round(v[x]);
    }
  }
#pragma unroll
  for (int x = 0; x < 8; ++x) vals[x] = Io<T>::store(v[x]);
  __builtin_memcpy(&packed, vals, 16);
  return packed;
}

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

template <typename T, int BM, int BN, int WAVES_M, int WAVES_N>
__global__ __launch_bounds__(WAVES_M* WAVES_N * 64) void gemm16_kernel(GemmArgs args) {
  using S = uint16_t;
  constexpr int NT = WAVES_M * WAVES_N * 64;
  constexpr int NW = WAVES_M * WAVES_N;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int A_BYTES = BM * kBK * 2;        // one stage of A
  constexpr int B_BYTES = BN * kBK * 2;        // one stage of B
  constexpr int STAGE = A_BYTES + B_BYTES;
  constexpr int A_INSTR = A_BYTES / 1024;      // wave instructions per stage
  constexpr int B_INSTR = B_BYTES / 1024;
  constexpr int A_PER_WAVE = A_INSTR / NW;
  constexpr int B_PER_WAVE = B_INSTR / NW;
  constexpr int LOADS = A_PER_WAVE + B_PER_WAVE;  // vmcnt units per stage per wave
  constexpr int B_CHUNKS = BN / 8;               // 16-byte chunks per B row
  constexpr int B_ROWS_PER_INSTR = 64 / B_CHUNKS;
  static_assert(A_INSTR % NW == 0 && B_INSTR % NW == 0, "stage loads must split evenly over the waves");
  static_assert(B_CHUNKS >= 8 && B_CHUNKS <= 64, "BN in [64, 512]");
  static_assert(TM >= 1 && TN >= 1, "wave tile at least 32x32");

  // One LDS object per stage: the compiler's LDS-DMA wait tracking then distinguishes the stages and waits
  // only for the stage being read, not for the prefetches still in flight.
  __shared__ __attribute__((aligned(1024))) unsigned char st0[STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char st1[STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char st2[STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char st3[STAGE];
  static_assert(kStages == 4, "one LDS object per stage");
  auto stage_mem = [&]<int SI>() -> unsigned char* {
    if constexpr (SI == 0) return st0;
    else if constexpr (SI == 1) return st1;
    else if constexpr (SI == 2) return st2;
    else return st3;
  };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;

  // ---- tile id: XCD-aware remap, then GROUP_M-row groups ----
  const int tiles = args.tiles_m * args.tiles_n;
  int bid = blockIdx.x;
  if ((tiles & 7) == 0) bid = (bid & 7) * (tiles >> 3) + (bid >> 3);
  constexpr int GROUP_M = 8;
  const int group = bid / (GROUP_M * args.tiles_n);
  const int first_m = group * GROUP_M;
  const int gsize = min(args.tiles_m - first_m, GROUP_M);
  const int tm = first_m + (bid % gsize);
  const int tn = (bid % (GROUP_M * args.tiles_n)) / gsize;
  const int64_t m0 = static_cast<int64_t>(tm) * BM;
  const int64_t n0 = static_cast<int64_t>(tn) * BN;

  const S* __restrict__ A = static_cast<const S*>(args.A) + blockIdx.y * args.stride_a;
  const S* __restrict__ B = static_cast<const S*>(args.B) + blockIdx.y * args.stride_b;
  S* __restrict__ C = static_cast<S*>(args.C) + blockIdx.y * args.stride_c;
  const int64_t M = args.M, N = args.N;
  const int64_t lda = args.lda, ldb = args.ldb, ldc = args.ldc;
  const int KT = static_cast<int>(args.K / kBK);

  // ---- per-lane global source offsets (elements), fixed across k; rows / columns past the edge are clamped
  // to the last valid one (their products land in discarded outputs) ----
  int64_t a_src[A_PER_WAVE];
#pragma unroll
  for (int j = 0; j < A_PER_WAVE; ++j) {
    const int row = (wave * A_PER_WAVE + j) * 16 + (lane >> 2);  // 16 rows of 64 B per instruction
    const int chunk = (lane & 3) ^ a_swizzle(row);
    const int64_t grow = min(m0 + row, M - 1);
    a_src[j] = grow * lda + chunk * 8;
  }
  int64_t b_src[B_PER_WAVE];
#pragma unroll
  for (int j = 0; j < B_PER_WAVE; ++j) {
    const int krow = (wave * B_PER_WAVE + j) * B_ROWS_PER_INSTR + lane / B_CHUNKS;
    const int chunk = (lane % B_CHUNKS) ^ b_swizzle<B_CHUNKS>(krow);
    const int64_t gcol = min(n0 + chunk * 8, N - 8);
    b_src[j] = static_cast<int64_t>(krow) * ldb + gcol;
  }

  // Stages past the end re-load the last stage (into a buffer nobody reads again), so every step issues the
  // same number of loads and the vmcnt bookkeeping is identical on every path.
  auto issue_stage = [&]<int SI>(int kt) {
    unsigned char* st = stage_mem.template operator()<SI>();
    const int64_t k0 = static_cast<int64_t>(min(kt, KT - 1)) * kBK;
#pragma unroll
    for (int j = 0; j < A_PER_WAVE; ++j)
      global_to_lds16(A + a_src[j] + k0, (FH_LDS void*)(st + (wave * A_PER_WAVE + j) * 1024));
#pragma unroll
    for (int j = 0; j < B_PER_WAVE; ++j)
      global_to_lds16(B + b_src[j] + k0 * ldb, (FH_LDS void*)(st + A_BYTES + (wave * B_PER_WAVE + j) * 1024));
  };

  // ---- per-lane LDS read offsets (bytes within a stage). Tile i of A adds i*32 rows (the swizzle depends on
  // row bits 2-3 only, so it is a constant 2048 B); k-half s and 4-k group h of B add whole rows. ----
  const int l32 = lane & 31, hi = lane >> 5;
  int a_off[2];
  {
    const int row = wm * WM + l32;
#pragma unroll
    for (int s = 0; s < 2; ++s) a_off[s] = row * 64 + (((2 * s + hi) ^ a_swizzle(row)) * 16);
  }
  // transpose reads: group g = lane/16 covers 16 columns and 4 k; lane r = q + 4e of the group points at
  // row (kbase + e), columns n + 4q .. n + 4q + 3
  const int g = lane >> 4, r = lane & 15, q = r & 3, e = r >> 2;
  int b_off[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int ncol = wn * WN + j * 32 + 16 * (g & 1) + 4 * q;
    const int krow = 8 * (g >> 1) + e;  // + 16 s + 4 h (immediates): krow & 3 and krow & 1 are unchanged
    const int chunk = (ncol >> 3) ^ b_swizzle<B_CHUNKS>(krow);
    b_off[j] = A_BYTES + krow * (BN * 2) + chunk * 16 + (ncol & 7) * 2;
  }
  constexpr int B_S = 16 * BN * 2, B_H = 4 * BN * 2;

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int x = 0; x < 16; ++x) acc[i][j][x] = 0.0f;

  // One k step on stage SI (= kt % kStages): wait for this wave's part of the stage, barrier (every wave's
  // part has landed and the stage refilled next was consumed by all), refill it kStages-1 steps ahead, multiply.
  auto step = [&]<int SI>(int kt) {
    wait_vmcnt<2 * LOADS>();  // this wave's loads of stage kt are done; stages kt+1, kt+2 may be in flight
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    issue_stage.template operator()<(SI + kStages - 1) % kStages>(kt + kStages - 1);
    const uint32_t base = lds_addr((const FH_LDS void*)stage_mem.template operator()<SI>());
    u32x4_t af[2][TM], bfr[2][TN];
    auto read = [&]<int S>() {
      const uint32_t abase = base + a_off[S];
      [&]<int... I>(std::integer_sequence<int, I...>) {
        ((af[S][I] = lds_read_b128<I * 2048>(abase)), ...);
      }(std::make_integer_sequence<int, TM>{});
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const u32x2_t lo = lds_read_tr16_b64<S * B_S>(base + b_off[j]);
        const u32x2_t hi2 = lds_read_tr16_b64<S * B_S + B_H>(base + b_off[j]);
        bfr[S][j] = u32x4_t{lo[0], lo[1], hi2[0], hi2[1]};
      }
    };
    // both k16 halves are requested up front; the second half's reads are in flight (and write registers
    // distinct from the first half's) while the first half is multiplied
    constexpr int READS = TM + 2 * TN;
    constexpr bool ACC_IN_AGPR = TM * TN * 16 > 128;
    read.template operator()<0>();
    read.template operator()<1>();
    fragment_fence<READS, TM, TN>(af[0], bfr[0]);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        mfma32<T>(af[0][i], bfr[0][j], acc[i][j]);
        pin<ACC_IN_AGPR>(acc[i][j]);  // keeps the first half's MFMAs above the second fence
      }
    fragment_fence<0, TM, TN>(af[1], bfr[1]);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) mfma32<T>(af[1][i], bfr[1][j], acc[i][j]);
  };

  // ---- prologue: stages 0..kStages-2 in flight ----
  issue_stage.template operator()<0>(0);
  issue_stage.template operator()<1>(1);
  issue_stage.template operator()<2>(2);

  for (int kt = 0; kt < KT; kt += kStages) {
    step.template operator()<0>(kt);
    if (kt + 1 < KT) step.template operator()<1>(kt + 1);
    if (kt + 2 < KT) step.template operator()<2>(kt + 2);
    if (kt + 3 < KT) step.template operator()<3>(kt + 3);
  }

  // ---- epilogue: round, stage the whole wave tile in LDS, then 16-byte coalesced read-modify-store ----
  wait_vmcnt<0>();  // the trailing re-loads must land before the ring is reused
  __syncthreads();  // all waves are done with the ring; reuse it
  // The whole wave tile is staged (rounded) in LDS, then read back row-wise as 16-byte vectors. Each wave's
  // tile lies inside one stage object.
  constexpr int WTILE_BYTES = WM * WN * 2;
  constexpr int PER_STAGE = STAGE / WTILE_BYTES;
  static_assert(PER_STAGE >= 1 && NW <= kStages * PER_STAGE, "the wave tiles fit in the ring");
  const int slot = wave / PER_STAGE;
  unsigned char* tile_base = slot == 0 ? st0 : slot == 1 ? st1 : slot == 2 ? st2 : st3;
  S* wl = reinterpret_cast<S*>(tile_base + (wave % PER_STAGE) * WTILE_BYTES);
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        const int rr = i * 32 + 8 * (x >> 2) + 4 * hi + (x & 3);
        wl[rr * WN + j * 32 + l32] = Io<T>::store(acc[i][j][x]);
      }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's tile is in LDS (wave-private region)
  __builtin_amdgcn_wave_barrier();
  constexpr int V = 8;           // elements per 16-byte vector
  constexpr int LPR = WN / V;    // lanes per staged row
  constexpr int RPI = 64 / LPR;  // rows per wave-wide access
  static_assert(64 % LPR == 0 && WM % RPI == 0, "epilogue access shape");
  const int c = (lane % LPR) * V;
  const int64_t col = n0 + wn * WN + c;
  for (int it = 0; it < WM / RPI; ++it) {
    const int rr = it * RPI + lane / LPR;
    const int64_t row = m0 + wm * WM + rr;
    if (row < M && col < N) {
      uint4 packed = *reinterpret_cast<const uint4*>(wl + rr * WN + c);
      const int64_t idx = row * ldc + col;
      if (args.ep.nseg > 0) packed = apply_epilogue_vec<T>(args.ep, packed, idx);
      *reinterpret_cast<uint4*>(C + idx) = packed;
    }
  }
}

template <typename T, int BM, int BN, int WAVES_M, int WAVES_N>
fh_status launch(GemmArgs args, int64_t batch, hipStream_t stream) {
  args.tiles_m = static_cast<int32_t>((args.M + BM - 1) / BM);
  args.tiles_n = static_cast<int32_t>((args.N + BN - 1) / BN);
  dim3 grid(static_cast<uint32_t>(args.tiles_m) * static_cast<uint32_t>(args.tiles_n), static_cast<uint32_t>(batch));
  hipLaunchKernelGGL((gemm16_kernel<T, BM, BN, WAVES_M, WAVES_N>), grid, dim3(WAVES_M * WAVES_N * 64), 0, stream, args);
  return launch_status("gemm16_kernel launch");
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <typename T>
fh_status dispatch(const GemmArgs& args, int64_t batch, hipStream_t stream) {
  const int cus = device_cu_count();
  auto tiles = [&](int64_t bm, int64_t bn) { return ((args.M + bm - 1) / bm) * ((args.N + bn - 1) / bn) * batch; };
  if (args.M >= 256 && args.N >= 256 && tiles(256, 256) >= cus) return launch<T, 256, 256, 4, 2>(args, batch, stream);
  if (args.M >= 128 && args.N >= 128 && tiles(128, 128) >= cus / 2) return launch<T, 128, 128, 2, 2>(args, batch, stream);
  if (args.N >= 128 && tiles(64, 128) >= cus / 2) return launch<T, 64, 128, 1, 2>(args, batch, stream);
  return launch<T, 64, 64, 2, 2>(args, batch, stream);
}

}  // namespace

bool gemm16_try_launch(int32_t dtype, const GemmArgs& args, int64_t batch, hipStream_t stream, fh_status* status) {
  if (dtype != FH_BF16 && dtype != FH_F16) return false;
  const size_t esz = 2;
  if (args.K <= 0 || args.K % kBK != 0 || args.N % 8 != 0 || args.N < 64) return false;
  if (args.lda % 8 || args.ldb % 8 || args.ldc % 8) return false;
  if (!aligned16(args.A) || !aligned16(args.B) || !aligned16(args.C)) return false;
  if ((args.stride_a * esz) % 16 || (args.stride_b * esz) % 16 || (args.stride_c * esz) % 16) return false;
  for (int s = 0; s < args.ep.nseg; ++s)
    if (ew_is_binary(args.ep.ops[s]) && !aligned16(args.ep.ins[s])) return false;
  *status = dtype == FH_BF16 ? dispatch<bf16_t>(args, batch, stream) : dispatch<f16_t>(args, batch, stream);
  return true;
}

}  // namespace fh
