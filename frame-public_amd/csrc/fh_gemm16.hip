// bf16 / f16 GEMM for gfx950: C[M,N] = A[M,K] · B[K,N], row-major, fp32 accumulation on
// v_mfma_f32_32x32x16_{bf16,f16}, one round-to-nearest-even per output, then the optional elementwise epilogue
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
//  * Software pipeline: each stage is multiplied as two k16 halves, and the fragments of the next half are
//    read from LDS while the current half's MFMAs run. The reads (and, after the barrier, the global->LDS
//    loads of the stage three ahead) are placed between the MFMAs in fixed program order (sched_barrier), so
//    the matrix pipe is fed while LDS and global traffic are in flight. One s_barrier per stage.
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

// The fragments of one k16 half of a wave tile.
template <int TM, int TN>
struct Fragments {
  u32x4_t a[TM];
  u32x2_t bl[TN], bh[TN];  // B fragment = 4 k from the low transpose read, 4 k from the high one
};

// Waits for every outstanding LDS read (they complete in order), then ties the fragment registers to the wait
// so no consumer is scheduled above it. The B halves are combined into MFMA operands only after this point.
template <int TM, int TN>
__device__ __forceinline__ void fence_fragments(Fragments<TM, TN>& f) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < TM; ++i) asm volatile("" : "+v"(f.a[i]));
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    asm volatile("" : "+v"(f.bl[j]));
    asm volatile("" : "+v"(f.bh[j]));
  }
}

// One workgroup = WAVES_M x WAVES_N waves computing a BM x BN tile; each wave owns (BM/WAVES_M) x (BN/WAVES_N)
// as TM x TN MFMA tiles of 32 x 32.
//
// Per stage kt (ring slot kt % 4), with f0 / f1 the fragment buffers of the two k16 halves:
//   fence(f0); MFMA(kt, half 0) || read(kt, half 1) -> f1;
//   wait vmcnt (this wave's loads of stage kt+1); s_barrier;
//   fence(f1); MFMA(kt, half 1) || read(kt+1, half 0) -> f0 || load stage kt+3 into the slot of stage kt-1.
// Ordering: stage kt+1 is read only after the barrier that follows every wave's vmcnt wait for it. The slot
// refilled after the barrier of step kt held stage kt-1, whose reads every wave fenced (lgkmcnt(0)) before
// arriving at that barrier. Stages past the end re-load the last stage (nobody reads them), so every step
// issues the same number of loads and the vmcnt counts hold on every path.
template <typename T, int BM, int BN, int WAVES_M, int WAVES_N, int E>
__global__ __launch_bounds__(WAVES_M* WAVES_N * 64) void gemm16_kernel(GemmArgs args) {
  using S = uint16_t;
  constexpr int NW = WAVES_M * WAVES_N;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int TM = WM / 32, TN = WN / 32;
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
  static_assert(TM >= 1 && TN >= 1, "wave tile at least 32x32");
  static_assert(2 * LOADS <= 63, "vmcnt range");

  __shared__ __attribute__((aligned(1024))) unsigned char ring[kStages * STAGE];

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
    const int chunk = (lane % B_CHUNKS) ^ b_swizzle<B_CHUNKS>(krow);
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
  const uint32_t ring_addr = lds_addr((const FH_LDS void*)ring);

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int x = 0; x < 16; ++x) acc[i][j][x] = 0.0f;

  Fragments<TM, TN> f0, f1;
  constexpr int NREAD = TM + 2 * TN;  // LDS reads per half
  constexpr int NMFMA = TM * TN;      // MFMAs per half

  // Read number R of half H of the stage at `base` into f.
  auto read_one = [&]<int H, int R>(uint32_t base, Fragments<TM, TN>& f) {
    if constexpr (R < TM) {
      f.a[R] = lds_read_b128<R * 2048>(base + a_off[H]);
    } else if constexpr ((R - TM) % 2 == 0) {
      f.bl[(R - TM) / 2] = lds_read_tr16_b64<H * B_S>(base + b_off[(R - TM) / 2]);
    } else {
      f.bh[(R - TM) / 2] = lds_read_tr16_b64<H * B_S + B_H>(base + b_off[(R - TM) / 2]);
    }
  };
  // The MFMAs of the half held in `cur`. After each come some of the reads of half H of the stage at `base`
  // into `nxt` (all within the first three quarters of the MFMAs, so they land before the half ends) and, with
  // LOADS_TOO, some of the global->LDS loads of stage load_kt (within the first half of the MFMAs).
  constexpr int R_SPAN = NMFMA * 3 / 4 > 0 ? NMFMA * 3 / 4 : 1;
  constexpr int L_SPAN = NMFMA / 2 > 0 ? NMFMA / 2 : 1;
  auto multiply_and_read = [&]<int H, bool LOADS_TOO>(Fragments<TM, TN>& cur, uint32_t base, Fragments<TM, TN>& nxt,
                                                      int load_kt) {
    [&]<int... M_>(std::integer_sequence<int, M_...>) {
      (
          [&] {
            constexpr int i = M_ / TN, j = M_ % TN;
            mfma32<T>(cur.a[i], u32x4_t{cur.bl[j][0], cur.bl[j][1], cur.bh[j][0], cur.bh[j][1]}, acc[i][j]);
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

  // ---- prologue: stages 0..2 in flight, half 0 of stage 0 in f0 ----
  issue_stage(0);
  issue_stage(1);
  issue_stage(2);
  wait_vmcnt<2 * LOADS>();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  [&]<int... R_>(std::integer_sequence<int, R_...>) {
    (read_one.template operator()<0, R_>(ring_addr, f0), ...);
  }(std::make_integer_sequence<int, NREAD>{});

  for (int kt = 0; kt < KT; ++kt) {
    const uint32_t cur = ring_addr + (kt & (kStages - 1)) * STAGE;
    const uint32_t nxt = ring_addr + ((kt + 1) & (kStages - 1)) * STAGE;
    fence_fragments(f0);
    multiply_and_read.template operator()<1, false>(f0, cur, f1, 0);
    wait_vmcnt<LOADS>();  // this wave's part of stage kt+1 has landed (stage kt+2 may be in flight)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    fence_fragments(f1);
    multiply_and_read.template operator()<0, true>(f1, nxt, f0, kt + kStages - 1);
  }
  // The last step read the next half's fragments (past the end: unused). Those LDS reads are still in flight
  // and would write their registers after the compiler has reused them in the epilogue, so they are fenced with
  // the registers tied before anything else may use them.
  fence_fragments(f0);

  // ---- epilogue: round, stage each wave tile in LDS, then 16-byte coalesced read-modify-store ----
  wait_vmcnt<0>();  // the trailing re-loads must land before the ring is reused
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __syncthreads();
  constexpr int WTILE_BYTES = WM * WN * 2;
  static_assert(NW * WTILE_BYTES <= kStages * STAGE, "the wave tiles fit in the ring");
  S* wl = reinterpret_cast<S*>(ring + wave * WTILE_BYTES);
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
          *reinterpret_cast<uint4*>(C + idx) = epi_apply<E, T>(ep, packed, in[b]);
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

// Largest tile that still gives every CU a workgroup (measured on MI355X, bf16 U(-1,1), M=N=K:
// 4096: 256x256/8 waves 1164 TFLOP/s; 2048: 128x128/8 waves 711-724; 1024: 64x64/4 waves 282).
template <typename T>
fh_status dispatch(const GemmArgs& args, int64_t batch, hipStream_t stream) {
  const int cus = device_cu_count();
  auto tiles = [&](int64_t bm, int64_t bn) { return ((args.M + bm - 1) / bm) * ((args.N + bn - 1) / bn) * batch; };
  if (args.M >= 256 && args.N >= 256 && tiles(256, 256) >= cus) return launch<T, 256, 256, 4, 2>(args, batch, stream);
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
