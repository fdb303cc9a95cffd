// bf16 / f16 GEMM for gfx950: C[M,N] = A[M,K] · B[K,N], row-major, fp32 accumulation on
// v_mfma_f32_16x16x32_{bf16,f16}, one round-to-nearest-even per output, then the optional elementwise epilogue
// (semantics of Frame's matmul: reference src/backends/cpu/kernels/matmul.cpp:92-185).
//
// Data path (CDNA4-specific):
//  * Operands go global -> LDS with global_load_lds_dwordx4 (no VGPR staging): every wave instruction writes
//    1 KB of LDS contiguously, lane L at +16*L. The lane -> global address map applies an XOR swizzle of the
//    16-byte chunks inside each LDS row, so the fragment reads below are bank-conflict free.
//  * A tile: [BM rows][32 k] bf16 = 64 B per row. A fragments are ds_read_b128 (8 consecutive k of one row
//    per lane), the MFMA's A layout.
//  * B tile: [32 k rows][BN n] bf16 kept n-contiguous as in memory. B fragments need 8 consecutive k of one
//    column per lane; ds_read_b64_tr_b16 (gfx950 LDS transpose read) delivers them in two reads of 4 k each,
//    with no register transposes.
//  * A ring of 4 LDS stages of BK = 32, refilled three stages ahead.
//  * MFMA shape: 16x16x32 rather than 32x32x16. Both have the same throughput, but a 32x32 tile reads and writes
//    16 accumulator registers per 32-cycle instruction where the 16x16 tile moves 4 per 16 cycles. Under the
//    board's power limit the smaller register traffic lets the clock run higher: measured on MI355X at 4096^3
//    U(-1,1), the same pipeline with 32x32x16 tiles ran at 1,243-1,265 TFLOP/s, this one at 1,344-1,375.
//  * Software pipeline: each stage's k-step is done in two phases over halves of the wave's B blocks; the next
//    phase's fragments are read from LDS while the current phase's MFMAs run. The reads (and, after the barrier,
//    the global->LDS loads of the stage three ahead) are placed between the MFMAs in fixed program order
//    (sched_barrier), so the matrix pipe is fed while LDS and global traffic are in flight. One s_barrier per
//    stage.
//  * Workgroups are remapped XCD-aware (consecutive tile ids on one XCD) and grouped along M for L2 reuse.
//  * Epilogue: the rounded tile is staged through LDS per wave and written with 16-byte stores; epilogue
//    operands are read with matching 16-byte loads.
#include <hip/hip_runtime.h>

#include <string>
#include <type_traits>
#include <utility>

#include "fh_common.h"
#include "fh_gemm.h"
#include "fh_mfma16.h"

namespace fh {
namespace {

using namespace mfma16;

// bf16 gelu by table for the add;gelu epilogue. With round_between the gelu input is a bf16 value, so gelu is a
// map of 16-bit patterns; the generated table holds the band of magnitudes [kGeluTabLo, kGeluTabHi) (2^-9 <= |x| < 8)
// for both signs, computed on the host as round(0.5 x (1 + erff(x / sqrt 2))) in fp32, and outside the band the
// function has closed forms (below: round(0.5 x); above: x for positive x, -0.0 for negative x; gelu(-inf) = NaN;
// NaN stays NaN). gen_gelu_table.cpp derives the band and checks the rules on all 65,536 inputs. This replaces
// ~30 VALU instructions per element (the erfc fit) with ~12 and one LDS read, and equals the fp32 formula with the
// C library's erff bit for bit.
#include "fh_gelu_table.inc"

__device__ __forceinline__ uint32_t gelu_bf16_tab(uint32_t b, const uint16_t* tab) {
  const uint32_t mag = b & 0x7fffu;
  const uint32_t neg = b >> 15;
  const uint32_t small = float_to_bf16_bits_hw(0.5f * __uint_as_float(b << 16));
  // the read is clamped into the band so every lane reads (no divergence); out-of-band lanes ignore it
  const uint32_t idx = min(max(mag, kGeluTabLo), kGeluTabHi - 1) - kGeluTabLo + neg * (kGeluTabHi - kGeluTabLo);
  const uint32_t t = tab[idx];
  uint32_t r = mag < kGeluTabLo ? small : mag < kGeluTabHi ? t : (neg ? 0x8000u : b);
  r = b == 0xff80u ? kGeluNegInf : r;
  return mag > 0x7f80u ? (b | 0x40u) : r;
}

// round(round(v + w) -> gelu) on one 16-byte vector of 8 bf16 (v: the staged rounded GEMM values, w: the operand)
__device__ __forceinline__ uint4 add_gelu_tab(uint4 v, uint4 w, const uint16_t* tab) {
  float a[8], o[8];
  unpack_vec<bf16_t>(v, a);
  unpack_vec<bf16_t>(w, o);
  uint32_t u[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const uint32_t s = store2<bf16_t>(a[2 * d] + o[2 * d], a[2 * d + 1] + o[2 * d + 1]);
    u[d] = gelu_bf16_tab(s & 0xffffu, tab) | (gelu_bf16_tab(s >> 16, tab) << 16);
  }
  return uint4{u[0], u[1], u[2], u[3]};
}

// A fragment set: a wave tile's A (all TM 16-row blocks) and NB of its 16-column B blocks, each B block as the low
// and high 4 k of the lane's 8.
template <int TM>
struct AFrags {
  u32x4_t a[TM];
};
template <int NB>
struct BFrags {
  u32x2_t lo[NB], hi[NB];
};

// Ties fragment registers to the preceding lgkmcnt(0) wait, so no consumer is scheduled above it (the LDS reads
// are inline asm the compiler's wait tracking does not see).
template <int TM>
__device__ __forceinline__ void tie(AFrags<TM>& f) {
#pragma unroll
  for (int i = 0; i < TM; ++i) asm volatile("" : "+v"(f.a[i]));
}
template <int NB>
__device__ __forceinline__ void tie(BFrags<NB>& f) {
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    asm volatile("" : "+v"(f.lo[j]));
    asm volatile("" : "+v"(f.hi[j]));
  }
}
__device__ __forceinline__ void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// One workgroup = WAVES_M x WAVES_N waves computing a BM x BN tile; each wave owns (BM/WAVES_M) x (BN/WAVES_N)
// as TM x TN MFMA tiles of 16 x 16. A stage (BK = 32) is one k-step of every tile. Large wave tiles run it in two
// phases over the halves of the wave's B blocks (fb0: [0, TN/2), fb1: [TN/2, TN)):
//   wait(fa, fb0); phase 0: MFMA(A, fb0) || read stage kt's B blocks [TN/2, TN) -> fb1;
//   wait vmcnt (this wave's loads of stage kt+1); s_barrier;
//   wait(fb1); phase 1: MFMA(A, fb1) || read stage kt+1's A -> fa' and B blocks [0, TN/2) -> fb0
//                      || load stage kt+3 into the slot of stage kt-1.
// Small wave tiles hold two full sets and run a stage as one phase:
//   wait vmcnt; s_barrier; wait(fa, fb); MFMA(A, B) || read stage kt+1 -> (fa', fb') || load stage kt+3.
// Sets alternate between stages (so the loop runs two stages per iteration). Ordering: stage kt+1 is read only
// after the barrier that follows every wave's vmcnt wait for it. The slot refilled after the barrier of step kt
// held stage kt-1, whose reads every wave waited for (lgkmcnt(0)) before arriving at that barrier. Stages past
// the end re-load the last stage (nobody reads them), so every step issues the same number of loads and the vmcnt
// counts hold on every path.
template <typename T, int BM, int BN, int WAVES_M, int WAVES_N, int E>
__global__ __launch_bounds__(WAVES_M* WAVES_N * 64) void gemm16_kernel(GemmArgs args) {
  using S = uint16_t;
  constexpr int NW = WAVES_M * WAVES_N;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int A_BYTES = BM * kBK * 2;
  constexpr int B_BYTES = BN * kBK * 2;
  constexpr int STAGE = A_BYTES + B_BYTES;
  constexpr int A_PER_WAVE = A_BYTES / 1024 / NW;  // global->LDS instructions per wave and stage
  constexpr int B_PER_WAVE = B_BYTES / 1024 / NW;
  constexpr int LOADS = A_PER_WAVE + B_PER_WAVE;
  constexpr int B_CHUNKS = BN / 8;  // 16-byte chunks per B row
  constexpr int B_ROWS_PER_INSTR = 64 / B_CHUNKS;
  static_assert((A_BYTES / 1024) % NW == 0 && (B_BYTES / 1024) % NW == 0, "stage loads split evenly over waves");
  static_assert(B_CHUNKS >= 8 && B_CHUNKS <= 64, "BN in [64, 512]");
  static_assert(TM >= 1 && TN >= 2 && TN % 2 == 0, "wave tile at least 16x32");
  static_assert(2 * LOADS <= 63, "vmcnt range");

  __shared__ __attribute__((aligned(1024))) unsigned char ring[kStages * STAGE];
  // add;gelu on bf16: the gelu table, loaded at the start with the first stages (its loads are older than every
  // stage's, so the prologue's vmcnt wait covers them)
  constexpr bool GELU_TAB = E == kEpiAddGelu && std::is_same_v<T, bf16_t>;
  __shared__ __attribute__((aligned(1024))) uint16_t gelu_lds[GELU_TAB ? kGeluTabN : 8];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS destinations become scalar math
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
  const bool grouped = args.groups > 0;
  const S* __restrict__ B = grouped ? static_cast<const S*>(args.group_b[blockIdx.y])
                                    : static_cast<const S*>(args.B) + blockIdx.y * args.stride_b;
  S* __restrict__ C = grouped ? static_cast<S*>(args.group_c[blockIdx.y]) : static_cast<S*>(args.C) + blockIdx.y * args.stride_c;
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
    a_src[j] = min(m0 + row, M - 1) * lda + chunk * 8;
  }
  int64_t b_src[B_PER_WAVE];
#pragma unroll
  for (int j = 0; j < B_PER_WAVE; ++j) {
    const int krow = (wave * B_PER_WAVE + j) * B_ROWS_PER_INSTR + lane / B_CHUNKS;
    const int chunk = (lane % B_CHUNKS) ^ b_swizzle16<B_CHUNKS>(krow);
    b_src[j] = static_cast<int64_t>(krow) * ldb + min(n0 + chunk * 8, N - 8);
  }

  // Load instruction J (< LOADS) of this wave's share of stage kt, into ring slot kt % kStages.
  auto load_one = [&]<int J>(int kt) {
    unsigned char* st = ring + (kt & (kStages - 1)) * STAGE;
    const int64_t k0 = static_cast<int64_t>(min(kt, KT - 1)) * kBK;
    if constexpr (J < A_PER_WAVE) {
      global_to_lds16(A + a_src[J] + k0, (FH_LDS void*)(st + (wave * A_PER_WAVE + J) * 1024));
    } else {
      constexpr int JB = J - A_PER_WAVE;
      global_to_lds16(B + b_src[JB] + k0 * ldb, (FH_LDS void*)(st + A_BYTES + (wave * B_PER_WAVE + JB) * 1024));
    }
  };
  auto issue_stage = [&](int kt) {
    [&]<int... J>(std::integer_sequence<int, J...>) {
      (load_one.template operator()<J>(kt), ...);
    }(std::make_integer_sequence<int, LOADS>{});
  };

  // ---- per-lane LDS read offsets (bytes within a stage) ----
  // A (16x16x32 operand: lane l holds row l % 16, k 8 (l / 16) .. + 7): one ds_read_b128 per 16-row block; block
  // i adds 16 rows = 1 KB (the swizzle depends on row bits 2-3 only).
  const int a_off = [&] {
    const int row = wm * WM + (lane & 15);
    return row * 64 + (((lane >> 4) ^ a_swizzle(row)) * 16);
  }();
  // B (lane l holds column l % 16, k 8 (l / 16) .. + 7): two transpose reads of 4 k each. In group g = l / 16,
  // lane r = q + 4 e points at row 8 g + e, columns 4 q .. 4 q + 3 of the block; the high read adds 4 rows.
  const int g = lane >> 4, r = lane & 15, q = r & 3, e = r >> 2;
  int b_off[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int ncol = wn * WN + j * 16 + 4 * q;
    const int krow = 8 * g + e;  // + 4 for the high read: krow & 3, krow & 1 and krow & 8 are unchanged
    const int chunk = (ncol >> 3) ^ b_swizzle16<B_CHUNKS>(krow);
    b_off[j] = A_BYTES + krow * (BN * 2) + chunk * 16 + (ncol & 7) * 2;
  }
  constexpr int B_HI = 4 * BN * 2;
  const uint32_t ring_addr = lds_addr((const FH_LDS void*)ring);

  f32x4_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int x = 0; x < 4; ++x) acc[i][j][x] = 0.0f;

  // Small wave tiles keep two full fragment sets (A and all B blocks) and run each stage as one phase that reads
  // the next stage; large ones split a stage into two phases over halves of the B blocks (one full set would not
  // leave registers for a second).
  constexpr bool ONE = (TM + 2 * TN) * 8 + TM * TN * 4 <= 160;
  constexpr int TB = ONE ? TN : TN / 2;  // B blocks per fragment set
  AFrags<TM> fa0, fa1;
  BFrags<TB> fb0, fb1;
  constexpr int NMFMA = TM * TB;  // MFMAs per phase
  // reads are spread over the first three quarters of a phase's MFMAs (so they land before it ends), global->LDS
  // loads over the first half
  constexpr int R_SPAN = NMFMA * 3 / 4 > 0 ? NMFMA * 3 / 4 : 1;
  constexpr int L_SPAN = NMFMA / 2 > 0 ? NMFMA / 2 : 1;

  // Read R of B blocks [J0, J0 + TB) of the stage at `base` into f (even R: low 4 k, odd R: high 4 k).
  auto read_b = [&]<int R, int J0>(uint32_t base, BFrags<TB>& f) {
    constexpr int j = R / 2;
    if constexpr (R % 2 == 0)
      f.lo[j] = lds_read_tr16_b64<0>(base + b_off[J0 + j]);
    else
      f.hi[j] = lds_read_tr16_b64<B_HI>(base + b_off[J0 + j]);
  };
  // Read R of a stage's first set: its A blocks into fa, then its B blocks [0, TB) into fb.
  auto read_set = [&]<int R>(uint32_t base, AFrags<TM>& fa, BFrags<TB>& fb) {
    if constexpr (R < TM)
      fa.a[R] = lds_read_b128<R * 1024>(base + a_off);
    else
      read_b.template operator()<R - TM, 0>(base, fb);
  };
  // The MFMAs of B blocks [J0, J0 + TB) (fragments fa, fb), with reads placed between them in fixed program order:
  // NEXT: the first set of the stage at `base` into (fa_n, fb_n) and the global->LDS loads of stage load_kt;
  // otherwise: B blocks [TB, 2 TB) of the stage at `base` into fb_n.
  auto phase = [&]<int J0, bool NEXT>(AFrags<TM>& fa, BFrags<TB>& fb, uint32_t base, AFrags<TM>& fa_n,
                                       BFrags<TB>& fb_n, int load_kt) {
    constexpr int NR = NEXT ? TM + 2 * TB : 2 * TB;
    [&]<int... M_>(std::integer_sequence<int, M_...>) {
      (
          [&] {
            constexpr int i = M_ / TB, j = M_ % TB;
            mfma16x<T>(fa.a[i], u32x4_t{fb.lo[j][0], fb.lo[j][1], fb.hi[j][0], fb.hi[j][1]}, acc[i][J0 + j]);
            constexpr int r0 = first(M_, NR, R_SPAN);
            [&]<int... R_>(std::integer_sequence<int, R_...>) {
              if constexpr (NEXT)
                (read_set.template operator()<r0 + R_>(base, fa_n, fb_n), ...);
              else
                (read_b.template operator()<r0 + R_, TB>(base, fb_n), ...);
            }(std::make_integer_sequence<int, share(M_, NR, R_SPAN)>{});
            if constexpr (NEXT) {
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
  auto barrier_next = [&] {
    wait_vmcnt<LOADS>();  // this wave's part of stage kt+1 has landed (stage kt+2 may be in flight)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  // Stage kt with its first set in (fa, fb). One phase: fb_n receives the next stage's B. Two phases: fb_n
  // receives this stage's second B half, and fb the next stage's first.
  auto step = [&](int kt, AFrags<TM>& fa, AFrags<TM>& fa_n, BFrags<TB>& fb, BFrags<TB>& fb_n) {
    const uint32_t cur = ring_addr + (kt & (kStages - 1)) * STAGE;
    const uint32_t nxt = ring_addr + ((kt + 1) & (kStages - 1)) * STAGE;
    if constexpr (ONE) {
      barrier_next();
      wait_lds();
      tie(fa);
      tie(fb);
      phase.template operator()<0, true>(fa, fb, nxt, fa_n, fb_n, kt + kStages - 1);
    } else {
      wait_lds();
      tie(fa);
      tie(fb);
      phase.template operator()<0, false>(fa, fb, cur, fa_n, fb_n, 0);
      barrier_next();
      wait_lds();
      tie(fb_n);
      phase.template operator()<TB, true>(fa, fb_n, nxt, fa_n, fb, kt + kStages - 1);
    }
  };

  // ---- prologue: stages 0..2 in flight, stage 0's first set in fa0 / fb0 ----
  if constexpr (GELU_TAB) {
    for (int j = wave; j < static_cast<int>(kGeluTabN / 512); j += NW)
      global_to_lds16(fh_gelu_table + j * 512 + lane * 8, (FH_LDS void*)(gelu_lds + j * 512));
  }
  issue_stage(0);
  issue_stage(1);
  issue_stage(2);
  wait_vmcnt<2 * LOADS>();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  [&]<int... R_>(std::integer_sequence<int, R_...>) {
    (read_set.template operator()<R_>(ring_addr, fa0, fb0), ...);
  }(std::make_integer_sequence<int, TM + 2 * TB>{});

  int kt = 0;
  for (; kt + 1 < KT; kt += 2) {
    step(kt, fa0, fa1, fb0, fb1);
    if constexpr (ONE)
      step(kt + 1, fa1, fa0, fb1, fb0);
    else
      step(kt + 1, fa1, fa0, fb0, fb1);
  }
  if (kt < KT) step(kt, fa0, fa1, fb0, fb1);
  // The last step read the next stage's fragments (past the end: unused). Those LDS reads are still in flight
  // and would write their registers after the compiler has reused them in the epilogue, so they are waited for
  // with the registers tied before anything else may use them.
  wait_lds();
  tie(fa0);
  tie(fa1);
  tie(fb0);
  tie(fb1);

  // ---- epilogue: round, stage each wave tile in LDS, then 16-byte coalesced read-modify-store ----
  wait_vmcnt<0>();  // the trailing re-loads must land before the ring is reused
  __syncthreads();
  constexpr int WTILE_BYTES = WM * WN * 2;
  static_assert(NW * WTILE_BYTES <= kStages * STAGE, "the wave tiles fit in the ring");
  S* wl = reinterpret_cast<S*>(ring + wave * WTILE_BYTES);
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int x = 0; x < 4; ++x) wl[(i * 16 + 4 * g + x) * WN + j * 16 + r] = Io<T>::store(acc[i][j][x]);
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's tile is in LDS (wave-private region)
  __builtin_amdgcn_wave_barrier();
  constexpr int V = 8;           // elements per 16-byte vector
  constexpr int LPR = WN / V;    // lanes per staged row
  constexpr int RPI = 64 / LPR;  // rows per wave-wide access
  static_assert(64 % LPR == 0 && WM % RPI == 0, "epilogue access shape");
  const int c = (lane % LPR) * V;
  const int64_t col = n0 + wn * WN + c;
  EpilogueArgs ep = args.ep;
  if (grouped)
#pragma unroll
    for (int sg = 0; sg < FH_MAX_SEGMENTS; ++sg) ep.ins[sg] = args.group_ins[blockIdx.y][sg];
  constexpr int ITERS = WM / RPI;
  constexpr int NOP = epi_operands<E>();
  if constexpr (NOP == 0) {
    for (int it = 0; it < ITERS; ++it) {
      const int rr = it * RPI + lane / LPR;
      const int64_t row = m0 + wm * WM + rr;
      if (row < M && col < N) {
        uint4 packed = *reinterpret_cast<const uint4*>(wl + rr * WN + c);
        const int64_t idx = row * ldc + col;
        packed = epi_vec<E, T>(ep, packed, idx);
        *reinterpret_cast<uint4*>(C + idx) = packed;
      }
    }
  } else {
    // programs with operands: the operand loads of a batch of rows are all issued before the first is used, so the
    // epilogue waits for memory once per batch rather than once per row. Rows and columns past the edge load the
    // last valid vector instead (never used), which keeps the loads free of branches the wait-count tracking
    // would have to join.
    constexpr int BATCH = ITERS < 8 ? ITERS : 8;
    const int64_t col_c = col < N ? col : N - V;
    for (int it0 = 0; it0 < ITERS; it0 += BATCH) {
      uint4 in[BATCH][NOP];
#pragma unroll
      for (int b = 0; b < BATCH; ++b) {
        const int64_t row = m0 + wm * WM + (it0 + b) * RPI + lane / LPR;
        epi_load<E, T>(ep, (row < M ? row : M - 1) * ldc + col_c, in[b]);
      }
#pragma unroll
      for (int b = 0; b < BATCH; ++b) {
        const int rr = (it0 + b) * RPI + lane / LPR;
        const int64_t row = m0 + wm * WM + rr;
        if (row < M && col < N) {
          const uint4 packed = *reinterpret_cast<const uint4*>(wl + rr * WN + c);
          const int64_t idx = row * ldc + col;
          if constexpr (GELU_TAB) {
            *reinterpret_cast<uint4*>(C + idx) =
                ep.round_between ? add_gelu_tab(packed, in[b][0], gelu_lds) : epi_apply<E, T>(ep, packed, in[b]);
          } else {
            *reinterpret_cast<uint4*>(C + idx) = epi_apply<E, T>(ep, packed, in[b]);
          }
        }
      }
    }
  }
}

template <typename T, int BM, int BN, int WAVES_M, int WAVES_N>
fh_status launch(GemmArgs args, int64_t batch, hipStream_t stream) {
  args.tiles_m = static_cast<int32_t>((args.M + BM - 1) / BM);
  args.tiles_n = static_cast<int32_t>((args.N + BN - 1) / BN);
  dim3 grid(static_cast<uint32_t>(args.tiles_m) * static_cast<uint32_t>(args.tiles_n), static_cast<uint32_t>(batch));
  auto go = [&]<int E>() {
    hipLaunchKernelGGL((gemm16_kernel<T, BM, BN, WAVES_M, WAVES_N, E>), grid, dim3(WAVES_M * WAVES_N * 64), 0, stream,
                       args);
    return launch_status("gemm16_kernel launch");
  };
  // bf16 (the configurations' type): the programs of C1-C5's GEMMs as kernels of their own; the rest (and f16)
  // take the interpreter (see EpiKind)
  if constexpr (std::is_same_v<T, bf16_t>) {
    switch (epi_kind(args.ep)) {
      case kEpiNone: return go.template operator()<kEpiNone>();
      case kEpiAdd: return go.template operator()<kEpiAdd>();
      case kEpiAddGelu: return go.template operator()<kEpiAddGelu>();
      case kEpiAddAdd: return go.template operator()<kEpiAddAdd>();
      default: break;
    }
  }
  return go.template operator()<kEpiAny>();
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Largest tile that still gives (nearly) every CU a workgroup (measured on MI355X, bf16 U(-1,1), M=N=K:
// 4096: 256x256/8 waves 1164 TFLOP/s; 2048: 128x128/8 waves 711-724; 1024: 64x64/4 waves 282). A 256x256 tile
// does the work of four 128x128 tiles at about 1.4 times their rate per CU, so it still wins with three quarters
// of the CUs busy: 4096 x 3072 x 1024 (192 tiles) 31.8 us against 33.3-34.0 us on 128x128 tiles.
template <typename T>
fh_status dispatch(const GemmArgs& args, int64_t batch, hipStream_t stream) {
  const int cus = device_cu_count();
  auto tiles = [&](int64_t bm, int64_t bn) { return ((args.M + bm - 1) / bm) * ((args.N + bn - 1) / bn) * batch; };
  if (args.M >= 256 && args.N >= 256 && tiles(256, 256) * 4 >= static_cast<int64_t>(cus) * 3)
    return launch<T, 256, 256, 4, 2>(args, batch, stream);
  if (args.M >= 128 && args.N >= 128 && tiles(128, 128) >= cus) return launch<T, 128, 128, 2, 4>(args, batch, stream);
  if (args.N >= 128 && tiles(64, 128) >= cus) return launch<T, 64, 128, 2, 2>(args, batch, stream);
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
  for (int g = 0; g < args.groups; ++g) {
    if (!aligned16(args.group_b[g]) || !aligned16(args.group_c[g])) return false;
    for (int s = 0; s < args.ep.nseg; ++s)
      if (ew_is_binary(args.ep.ops[s]) && !aligned16(args.group_ins[g][s])) return false;
  }
  *status = dtype == FH_BF16 ? dispatch<bf16_t>(args, batch, stream) : dispatch<f16_t>(args, batch, stream);
  return true;
}

}  // namespace fh
