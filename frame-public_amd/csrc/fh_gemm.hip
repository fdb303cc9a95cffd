// Dense GEMM for gfx950: C[M,N] = A[M,K] · B[K,N], row-major, fp32 accumulation on MFMA.
//
// Semantics follow Frame's matmul (reference: src/backends/cpu/kernels/matmul.cpp:92-185): dtype in = out,
// products accumulated in fp32, one round-to-nearest-even store. The optional epilogue applies the
// elementwise segments Frame's graph would run next (bias add, ReLU, ...) on the rounded product before
// the single store, rounding between segments exactly like the unfused graph.
//
// Tile kernel layout (one workgroup = 4 waves = 256 threads):
//   * Block tile BM x BN, K staged in slices of 128 bytes per row (64 bf16/f16 or 32 fp32 values).
//   * A slice is stored in LDS row-major [BM][128 B]; B slice is stored transposed [BN][128 B] so both MFMA
//     operands read 16-byte k-contiguous fragments. B is transposed in registers (E x E blocks) between
//     the global load and the LDS store, so global reads stay fully coalesced.
//   * Every 16-byte chunk is XOR-swizzled inside its row by ((row ^ row>>3) & 7): fragment reads, A stores
//     and transposed B stores are all bank-conflict free.
//   * Two LDS stages: the global loads of slice k+1 are in flight while the MFMAs consume slice k.
//   * Waves are laid out 2 x 2; each owns a (BM/2) x (BN/2) sub-tile of 32x32 MFMA tiles.
//   * Workgroup ids are remapped so that consecutive tiles land on the same XCD (blocks are dispatched
//     round-robin over the 8 XCDs) and tiles are visited in groups of rows for L2 reuse.
#include <hip/hip_runtime.h>

#include <string>
#include <type_traits>

#include "fh_common.h"
#include "fh_gemm.h"

namespace fh {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

template <typename T>
struct GemmTraits;
template <>
struct GemmTraits<bf16_t> {
  static constexpr int E = 8;  // elements per 16-byte chunk
};
template <>
struct GemmTraits<f16_t> {
  static constexpr int E = 8;
};
template <>
struct GemmTraits<float> {
  static constexpr int E = 4;
};

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row ^ (row >> 3)) & 7); }

// Transposes an E x E block of 16-bit values held as E rows of 16 bytes.
__device__ __forceinline__ void transpose8x8_u16(const uint4 (&in)[8], uint4 (&out)[8]) {
  const uint32_t* src = reinterpret_cast<const uint32_t*>(in);  // src[r*4 + d]
  uint32_t* dst = reinterpret_cast<uint32_t*>(out);
#pragma unroll
  for (int c = 0; c < 8; ++c) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t a = src[(2 * q) * 4 + (c >> 1)];
      const uint32_t b = src[(2 * q + 1) * 4 + (c >> 1)];
      dst[c * 4 + q] = (c & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
    }
  }
}

__device__ __forceinline__ void transpose4x4_u32(const uint4 (&in)[4], uint4 (&out)[4]) {
  const uint32_t* src = reinterpret_cast<const uint32_t*>(in);
  uint32_t* dst = reinterpret_cast<uint32_t*>(out);
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int r = 0; r < 4; ++r) dst[c * 4 + r] = src[r * 4 + c];
}

template <typename T>
__device__ __forceinline__ void mfma_step(const uint4& a, const uint4& b, f32x16_t& acc);

template <>
__device__ __forceinline__ void mfma_step<bf16_t>(const uint4& a, const uint4& b, f32x16_t& acc) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                acc, 0, 0, 0);
}
template <>
__device__ __forceinline__ void mfma_step<f16_t>(const uint4& a, const uint4& b, f32x16_t& acc) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b),
                                               acc, 0, 0, 0);
}
// fp32: one 16-byte chunk holds 4 k-values; lane halves read different chunks and both operands use the
// same k assignment, so four 32x32x2 MFMAs consume the pair of chunks.
template <>
__device__ __forceinline__ void mfma_step<float>(const uint4& a, const uint4& b, f32x16_t& acc) {
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.x), __uint_as_float(b.x), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.y), __uint_as_float(b.y), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.z), __uint_as_float(b.z), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.w), __uint_as_float(b.w), acc, 0, 0, 0);
}

template <typename T, int BM, int BN, bool kGuard>
__global__ __launch_bounds__(256) void gemm_tile_kernel(GemmArgs args) {
  using S = typename Io<T>::storage;
  constexpr int E = GemmTraits<T>::E;
  constexpr int BK = 8 * E;  // 128 bytes of K per row
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int A_LOADS = BM * 8 / 256;
  constexpr int B_BLOCKS = 8 * BN / E;  // E x E blocks in a K slice
  constexpr int B_ITERS = (B_BLOCKS + 255) / 256;
  constexpr int NB_PER_ROW = BN / E;
  static_assert(A_LOADS >= 1, "BM too small");

  __shared__ uint4 lds[2][(BM + BN) * 8];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // --- tile scheduling: XCD-aware remap, then grouped row-major order ---
  const int tiles = args.tiles_m * args.tiles_n;
  int bid = blockIdx.x;
  if ((tiles & 7) == 0) bid = (bid & 7) * (tiles >> 3) + (bid >> 3);
  constexpr int GROUP_M = 4;
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
  const int64_t M = args.M, N = args.N, K = args.K;
  const int64_t lda = args.lda, ldb = args.ldb, ldc = args.ldc;

  uint4 ra[A_LOADS];
  uint4 rb[B_ITERS][E];

  auto load_slice = [&](int kt) {
    const int64_t k0 = static_cast<int64_t>(kt) * BK;
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int id = tid + 256 * i;
      const int row = id >> 3, c = id & 7;
      const int64_t gr = m0 + row, gk = k0 + c * E;
      if (!kGuard || (gr < M && gk < K)) {
        ra[i] = *reinterpret_cast<const uint4*>(A + gr * lda + gk);
      } else {
        ra[i] = make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int j = 0; j < B_ITERS; ++j) {
      const int blk = tid + 256 * j;
      const int kb = blk / NB_PER_ROW, nb = blk % NB_PER_ROW;
      const int64_t gn = n0 + nb * E;
#pragma unroll
      for (int r = 0; r < E; ++r) {
        const int64_t gk = k0 + kb * E + r;
        if ((B_BLOCKS % 256 == 0 || blk < B_BLOCKS) && (!kGuard || (gk < K && gn < N))) {
          rb[j][r] = *reinterpret_cast<const uint4*>(B + gk * ldb + gn);
        } else {
          rb[j][r] = make_uint4(0, 0, 0, 0);
        }
      }
    }
  };

  auto store_slice = [&](int buf) {
    uint4* As = lds[buf];
    uint4* Bs = lds[buf] + BM * 8;
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int id = tid + 256 * i;
      const int row = id >> 3, c = id & 7;
      As[row * 8 + swz(row, c)] = ra[i];
    }
#pragma unroll
    for (int j = 0; j < B_ITERS; ++j) {
      const int blk = tid + 256 * j;
      if (B_BLOCKS % 256 != 0 && blk >= B_BLOCKS) continue;
      const int kb = blk / NB_PER_ROW, nb = blk % NB_PER_ROW;
      uint4 t[E];
      if constexpr (E == 8) {
        transpose8x8_u16(rb[j], t);
      } else {
        transpose4x4_u32(rb[j], t);
      }
#pragma unroll
      for (int c = 0; c < E; ++c) {
        const int n = nb * E + c;
        Bs[n * 8 + swz(n, kb)] = t[c];
      }
    }
  };

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  const int KT = static_cast<int>((K + BK - 1) / BK);
  const int half = lane >> 5;
  const int l32 = lane & 31;

  load_slice(0);
  store_slice(0);
  __syncthreads();

  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) load_slice(kt + 1);
    const uint4* As = lds[cur];
    const uint4* Bs = lds[cur] + BM * 8;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int chunk = 2 * ks + half;
      uint4 a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = wm * WM + i * 32 + l32;
        a[i] = As[row * 8 + swz(row, chunk)];
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int row = wn * WN + j * 32 + l32;
        b[j] = Bs[row * 8 + swz(row, chunk)];
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) mfma_step<T>(a[i], b[j], acc[i][j]);
    }
    if (kt + 1 < KT) store_slice(cur ^ 1);
    __syncthreads();
  }

  // --- epilogue: stage the rounded tile through LDS (free after the last barrier), then each wave runs the
  // elementwise program on 16-byte vectors and stores them coalesced. Rounding the product to T before
  // staging loses nothing: the epilogue starts from the rounded product anyway. ---
  constexpr int V = 16 / static_cast<int>(sizeof(S));       // elements per 16-byte vector
  constexpr int CAP = (BM + BN) * 64 / static_cast<int>(sizeof(S));  // LDS elements owned by one wave
  constexpr int RP_RAW = (CAP / WN) / 32 * 32;
  constexpr int RP = RP_RAW < WM ? RP_RAW : WM;               // wave rows staged per pass
  constexpr int PASSES = WM / RP;
  constexpr int LPR = WN / V;                                  // lanes per staged row
  constexpr int RPI = 64 / LPR;                                // staged rows per wave-wide access
  static_assert(RP >= 32 && WM % RP == 0 && 64 % LPR == 0, "epilogue staging shape");
  S* wl = reinterpret_cast<S*>(&lds[0][0]) + wave * CAP;
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      if (i / (RP / 32) != p) continue;
      const int rbase = (i % (RP / 32)) * 32;
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int rr = rbase + 8 * (r >> 2) + 4 * half + (r & 3);
          wl[rr * WN + j * 32 + l32] = Io<T>::store(acc[i][j][r]);
        }
    }
    __syncthreads();
    const int c = (lane % LPR) * V;
    const int64_t col = n0 + wn * WN + c;
#pragma unroll 4
    for (int it = 0; it < RP / RPI; ++it) {
      const int rr = it * RPI + lane / LPR;
      const int64_t row = m0 + wm * WM + p * RP + rr;
      if (kGuard && (row >= M || col >= N)) continue;
      uint4 packed = *reinterpret_cast<const uint4*>(wl + rr * WN + c);
      const int64_t idx = row * ldc + col;
      if (args.ep.nseg > 0) packed = epilogue_vec<T>(args.ep, packed, idx);
      *reinterpret_cast<uint4*>(C + idx) = packed;
    }
    if (p + 1 < PASSES) __syncthreads();
  }
}

// Small and unaligned GEMMs (few output tiles, or rows/columns the tile kernels cannot take): one thread per
// output of a 16 x 16 tile, its k loop strictly sequential like the reference CPU kernel (fp32 products and sums,
// no contraction, one rounding), so the result is bit-identical to it. K is staged through LDS in chunks of kKC as
// fp32, A row-major and B transposed, both k-contiguous so each step reads 4 k-values per operand with one
// 16-byte LDS read; the next chunk's global loads are in flight while the current one is consumed.
constexpr int kSeqT = 16;   // output tile edge
constexpr int kKC = 128;    // k per LDS chunk
constexpr int kKP = kKC + 4;  // padded row: 16 consecutive B rows hit distinct 16-byte bank groups

template <typename T>
__global__ __launch_bounds__(256) void gemm_seq_kernel(GemmArgs args) {
  using S = typename Io<T>::storage;
  __shared__ __attribute__((aligned(16))) float As[2][kSeqT * kKP];
  __shared__ __attribute__((aligned(16))) float Bt[2][kSeqT * kKP];
  const S* __restrict__ A = static_cast<const S*>(args.A) + blockIdx.z * args.stride_a;
  const S* __restrict__ B = static_cast<const S*>(args.B) + blockIdx.z * args.stride_b;
  S* __restrict__ C = static_cast<S*>(args.C) + blockIdx.z * args.stride_c;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kSeqT, n0 = static_cast<int64_t>(blockIdx.x) * kSeqT;
  const int64_t M = args.M, N = args.N, K = args.K;
  const int t = threadIdx.x;
  const int r = t >> 4, c = t & 15;

  // chunk loads: A[16][kKC] and B[kKC][16], each with consecutive lanes on the operand's contiguous index: k for
  // row-major A and transposed B (thread -> row / column t/16, k t%16 + 16 i), the row or column otherwise
  // (thread -> k t/16 + 16 i, row / column t%16)
  float la[8], lb[8];
  const bool ta = args.trans_a != 0, tb = args.trans_b != 0;
  auto load_chunk = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t gm = m0 + (ta ? c : r), gk = k0 + (ta ? r : c) + 16 * i;
      la[i] = (gm < M && gk < K) ? Io<T>::load(A[ta ? gk * args.lda + gm : gm * args.lda + gk]) : 0.0f;
      const int64_t bk = k0 + (tb ? c : r) + 16 * i, bn = n0 + (tb ? r : c);
      lb[i] = (bk < K && bn < N) ? Io<T>::load(B[tb ? bn * args.ldb + bk : bk * args.ldb + bn]) : 0.0f;
    }
  };
  auto store_chunk = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      As[buf][ta ? c * kKP + r + 16 * i : r * kKP + c + 16 * i] = la[i];
      Bt[buf][tb ? r * kKP + c + 16 * i : c * kKP + r + 16 * i] = lb[i];
    }
  };

  float acc = 0.0f;
  const int chunks = static_cast<int>((K + kKC - 1) / kKC);
  if (chunks > 0) {
    load_chunk(0);
    store_chunk(0);
  }
  __syncthreads();
  for (int ch = 0; ch < chunks; ++ch) {
    const int buf = ch & 1;
    if (ch + 1 < chunks) load_chunk(static_cast<int64_t>(ch + 1) * kKC);
    const int kn = static_cast<int>(min<int64_t>(kKC, K - static_cast<int64_t>(ch) * kKC));
    const float* ar = &As[buf][r * kKP];
    const float* br = &Bt[buf][c * kKP];
    int kk = 0;
    // 16 k per step: the four LDS reads of each operand are issued before the sum uses them, so one LDS latency
    // covers 16 k instead of 4 (the sum itself is the same chain, in the same order)
    for (; kk + 16 <= kn; kk += 16) {
      float4 a[4], b[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        a[u] = *reinterpret_cast<const float4*>(ar + kk + 4 * u);
        b[u] = *reinterpret_cast<const float4*>(br + kk + 4 * u);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        acc = acc + a[u].x * b[u].x;
        acc = acc + a[u].y * b[u].y;
        acc = acc + a[u].z * b[u].z;
        acc = acc + a[u].w * b[u].w;
      }
    }
    for (; kk + 4 <= kn; kk += 4) {
      const float4 a = *reinterpret_cast<const float4*>(ar + kk);
      const float4 b = *reinterpret_cast<const float4*>(br + kk);
      acc = acc + a.x * b.x;
      acc = acc + a.y * b.y;
      acc = acc + a.z * b.z;
      acc = acc + a.w * b.w;
    }
    for (; kk < kn; ++kk) acc = acc + ar[kk] * br[kk];
    if (ch + 1 < chunks) store_chunk(buf ^ 1);
    __syncthreads();
  }
  const int64_t row = m0 + r, col = n0 + c;
  if (row < M && col < N) {
    float v = Io<T>::round(acc);
    const int64_t idx = row * args.ldc + col;
    if (args.ep.nseg > 0) v = epilogue_one<T>(args.ep, v, idx);
    C[idx] = Io<T>::store(v);
  }
}

// Small GEMMs whose k-sum may be reassociated (FH_GEMM_ANY_ORDER): the sequential kernel's few 16 x 16 tiles leave
// most CUs idle, and each output's k loop is one long dependent chain. Here a workgroup of 16 waves owns a 4 x 16
// output tile (four times as many workgroups) and splits K 16 ways. K is staged through LDS as fp32 in chunks of
// up to kSplitKC = 1024 (A row-major, B transposed; every global load of a chunk in flight at once, so C1's layers
// pay one memory latency); within a chunk wave w sums its own contiguous sixteenth of the k, one output per lane,
// products and sums in fp32 without contraction like the sequential kernel. The 16 partial sums are then added in
// wave order: deterministic, and different from the sequential order by fp32 reassociation only. (Measured at
// C1's shapes on MI355X: 64x784x256 6.4 us and 64x256x10 3.4 us against 10.2 / 4.4 us with 4 waves and 16.3 /
// 6.1 us sequential; a launch of any kernel costs ~3 us there.)
// With row_softmax (N <= 16, so every output row lies in one workgroup), the rounded outputs of each row then
// go through softmax exactly as fh_softmax_rows computes it (m = max, e = exp(x - m), s = sum e, y = round(e / s);
// the sum taken over 16 lanes instead of 64).
constexpr int kSplitTM = 4, kSplitTN = 16, kSplitKC = 1024, kSplitKP = kSplitKC + 4, kSplitWaves = 16;

template <typename T>
__global__ __launch_bounds__(kSplitWaves * 64) void gemm_split_kernel(GemmArgs args) {
  using S = typename Io<T>::storage;
  __shared__ __attribute__((aligned(16))) float As[kSplitTM * kSplitKP];
  __shared__ __attribute__((aligned(16))) float Bt[kSplitTN * kSplitKP];
  __shared__ float part[kSplitWaves][kSplitTM * kSplitTN];
  constexpr int NT = kSplitWaves * 64;
  const S* __restrict__ A = static_cast<const S*>(args.A) + blockIdx.z * args.stride_a;
  const S* __restrict__ B = static_cast<const S*>(args.B) + blockIdx.z * args.stride_b;
  S* __restrict__ C = static_cast<S*>(args.C) + blockIdx.z * args.stride_c;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kSplitTM, n0 = static_cast<int64_t>(blockIdx.x) * kSplitTN;
  const int64_t M = args.M, N = args.N, K = args.K;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int r = lane >> 4, c = lane & 15;  // this lane's output: (m0 + r, n0 + c)

  float acc = 0.0f;
  for (int64_t k0 = 0; k0 < K; k0 += kSplitKC) {
    const int kn = static_cast<int>(min<int64_t>(kSplitKC, K - k0));
    // every element of the chunk this thread stages is loaded into registers before the first is written to LDS,
    // so the loads overlap (a load-then-store loop waits for each load in turn)
    constexpr int AJ = kSplitTM * kSplitKC / NT, BJ = kSplitTN * kSplitKC / NT;
    static_assert(kSplitTM * kSplitKC % NT == 0 && kSplitTN * kSplitKC % NT == 0, "whole staging rounds");
    float av[AJ], bv[BJ];
#pragma unroll
    for (int j = 0; j < AJ; ++j) {
      const int i = t + j * NT, row = i / kSplitKC, kk = i - row * kSplitKC;
      av[j] = (kk < kn && m0 + row < M) ? Io<T>::load(A[(m0 + row) * args.lda + k0 + kk]) : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < BJ; ++j) {
      const int i = t + j * NT, kk = i >> 4, cc = i & 15;
      bv[j] = (kk < kn && n0 + cc < N) ? Io<T>::load(B[(k0 + kk) * args.ldb + n0 + cc]) : 0.0f;
    }
    if (k0 > 0) __syncthreads();  // the previous chunk has been read
#pragma unroll
    for (int j = 0; j < AJ; ++j) {
      const int i = t + j * NT, row = i / kSplitKC, kk = i - row * kSplitKC;
      if (kk < kn) As[row * kSplitKP + kk] = av[j];
    }
#pragma unroll
    for (int j = 0; j < BJ; ++j) {
      const int i = t + j * NT, kk = i >> 4, cc = i & 15;
      if (kk < kn) Bt[cc * kSplitKP + kk] = bv[j];
    }
    __syncthreads();
    const int per = (kn + kSplitWaves - 1) / kSplitWaves;
    const int q0 = wave * per;
    const int qn = max(0, min(per, kn - q0));
    const float* ar = &As[r * kSplitKP + q0];
    const float* br = &Bt[c * kSplitKP + q0];
    for (int kk = 0; kk < qn; ++kk) acc = acc + ar[kk] * br[kk];
  }
  part[wave][lane] = acc;
  __syncthreads();
  if (t < kSplitTM * kSplitTN) {
    const int64_t row = m0 + (t >> 4), col = n0 + (t & 15);
    const bool live = row < M && col < N;
    float sum = part[0][t];
#pragma unroll
    for (int w = 1; w < kSplitWaves; ++w) sum = sum + part[w][t];
    float v = Io<T>::round(sum);
    const int64_t idx = row * args.ldc + col;
    if (live && args.ep.nseg > 0) v = epilogue_one<T>(args.ep, v, idx);
    if (args.row_softmax) {  // N <= 16: the row's outputs are the 16 lanes of this lane's group
      float m = live ? v : -__builtin_inff();
#pragma unroll
      for (int o = 8; o > 0; o >>= 1) {
        const float other = __shfl_xor(m, o, 16);
        m = (other > m) ? other : m;
      }
      const float e = live ? expf(v - m) : 0.0f;
      float s = e;
#pragma unroll
      for (int o = 8; o > 0; o >>= 1) s += __shfl_xor(s, o, 16);
      v = e / s;
    }
    if (live) C[idx] = Io<T>::store(v);
  }
}

template <typename T, int BM, int BN>
fh_status launch_tile(GemmArgs args, int64_t batch, hipStream_t stream) {
  args.tiles_m = static_cast<int32_t>((args.M + BM - 1) / BM);
  args.tiles_n = static_cast<int32_t>((args.N + BN - 1) / BN);
  constexpr int BK = 8 * GemmTraits<T>::E;
  const bool full = (args.M % BM == 0) && (args.N % BN == 0) && (args.K % BK == 0);
  dim3 grid(static_cast<uint32_t>(args.tiles_m) * static_cast<uint32_t>(args.tiles_n),
            static_cast<uint32_t>(batch));
  if (full) {
    hipLaunchKernelGGL((gemm_tile_kernel<T, BM, BN, false>), grid, dim3(256), 0, stream, args);
  } else {
    hipLaunchKernelGGL((gemm_tile_kernel<T, BM, BN, true>), grid, dim3(256), 0, stream, args);
  }
  return launch_status("gemm_tile_kernel launch");
}

bool epilogue_aligned(const EpilogueArgs& ep) {
  for (int s = 0; s < ep.nseg; ++s)
    if (ew_is_binary(ep.ops[s]) && reinterpret_cast<uintptr_t>(ep.ins[s]) % 16 != 0) return false;
  return true;
}

template <typename T>
fh_status dispatch_gemm(GemmArgs args, int64_t batch, hipStream_t stream) {
  constexpr int E = GemmTraits<T>::E;
  const int cus = device_cu_count();
  // Few 64 x 64 tiles: the sequential kernel, whose 16 x 16 tiles spread further and whose latency is a handful
  // of K chunks. fp32 below a quarter of the CUs; 16-bit only below 16 tiles (its MFMA kernel stays faster down
  // to there: the C4 classifier, 16 tiles, 7.8 us there against 22 us sequential).
  const int64_t tiles64 = ((args.M + 63) / 64) * ((args.N + 63) / 64) * batch;
  const bool small = (std::is_same_v<T, float> ? tiles64 * 4 < cus : tiles64 < 16) && args.K <= 16384;
  if constexpr (!std::is_same_v<T, float>) {
    fh_status st = FH_OK;
    if (!small && gemm16_try_launch(std::is_same_v<T, bf16_t> ? FH_BF16 : FH_F16, args, batch, stream, &st)) return st;
  }
  const size_t esz = sizeof(typename Io<T>::storage);
  const bool aligned = (reinterpret_cast<uintptr_t>(args.A) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(args.B) % 16 == 0) && (args.K % E == 0) &&
                       (args.N % E == 0) && (args.lda % E == 0) && (args.ldb % E == 0) &&
                       ((args.stride_a * esz) % 16 == 0) && ((args.stride_b * esz) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(args.C) % 16 == 0) && (args.ldc % E == 0) &&
                       ((args.stride_c * esz) % 16 == 0) && epilogue_aligned(args.ep);
  const bool split_ok = args.any_order && !args.trans_a && !args.trans_b &&
                        (args.M + kSplitTM - 1) / kSplitTM <= 65535 && batch <= 65535;
  if (args.row_softmax && (!split_ok || args.N > kSplitTN))
    return fail(FH_INVALID_ARGUMENT, "fh_gemm_ex: FH_GEMM_ROW_SOFTMAX needs FH_GEMM_ANY_ORDER, N <= 16 and at most "
                                     "262,140 rows");
  if ((small || args.row_softmax) && split_ok) {
    dim3 grid(static_cast<uint32_t>((args.N + kSplitTN - 1) / kSplitTN),
              static_cast<uint32_t>((args.M + kSplitTM - 1) / kSplitTM), static_cast<uint32_t>(batch));
    hipLaunchKernelGGL((gemm_split_kernel<T>), grid, dim3(kSplitWaves * 64), 0, stream, args);
    return launch_status("gemm_split_kernel launch");
  }
  // small problems, or operands the tile kernels cannot take
  if (!aligned || small) {
    if ((args.M + kSeqT - 1) / kSeqT > 65535 || batch > 65535)
      return fail(FH_UNIMPLEMENTED, "fh_gemm: unaligned operands with more than 1,048,560 rows or 65,535 batches");
    dim3 grid(static_cast<uint32_t>((args.N + kSeqT - 1) / kSeqT), static_cast<uint32_t>((args.M + kSeqT - 1) / kSeqT),
              static_cast<uint32_t>(batch));
    hipLaunchKernelGGL((gemm_seq_kernel<T>), grid, dim3(256), 0, stream, args);
    return launch_status("gemm_seq_kernel launch");
  }
  auto tiles = [&](int64_t t) { return ((args.M + t - 1) / t) * ((args.N + t - 1) / t) * batch; };
  if (tiles(256) >= cus) return launch_tile<T, 256, 256>(args, batch, stream);
  if (tiles(128) >= cus / 2) return launch_tile<T, 128, 128>(args, batch, stream);
  return launch_tile<T, 64, 64>(args, batch, stream);
}

fh_status run_gemm(int32_t dtype, GemmArgs args, int64_t batch, hipStream_t stream) {
  switch (dtype) {
    case FH_F32:
      return dispatch_gemm<float>(args, batch, stream);
    case FH_BF16:
      return dispatch_gemm<bf16_t>(args, batch, stream);
    case FH_F16:
      return dispatch_gemm<f16_t>(args, batch, stream);
    default:
      return fail(FH_UNIMPLEMENTED, "fh_gemm: unsupported dtype code " + std::to_string(dtype));
  }
}

fh_status copy_epilogue(const fh_epilogue* in, EpilogueArgs& out) {
  out = EpilogueArgs{};
  if (in == nullptr) return FH_OK;
  if (in->nseg < 0 || in->nseg > FH_MAX_SEGMENTS)
    return fail(FH_INVALID_ARGUMENT, "epilogue: nseg out of range: " + std::to_string(in->nseg));
  out.nseg = in->nseg;
  out.round_between = in->round_between;
  for (int s = 0; s < in->nseg; ++s) {
    const uint8_t op = in->ops[s];
    if (!epilogue_op_ok(op))
      return fail(FH_INVALID_ARGUMENT, "epilogue: unknown op code " + std::to_string(op));
    if (ew_is_binary(op) && in->ins[s] == nullptr)
      return fail(FH_INVALID_ARGUMENT, "epilogue: binary segment " + std::to_string(s) + " has no operand");
    out.ops[s] = op;
    out.ins[s] = in->ins[s];
  }
  return FH_OK;
}

}  // namespace

fh_status gemm_with_epilogue_args(int32_t dtype, const void* A, const void* B, void* C, int64_t M, int64_t N,
                                  int64_t K, const fh_epilogue* epilogue, hipStream_t stream, int32_t flags) {
  if ((flags & ~(FH_GEMM_ANY_ORDER | FH_GEMM_ROW_SOFTMAX)) != 0)
    return fail(FH_INVALID_ARGUMENT, "fh_gemm_ex: unknown flags " + std::to_string(flags));
  if (!is_supported_float(dtype)) return fail(FH_UNIMPLEMENTED, "fh_gemm: unsupported dtype");
  if (M < 0 || N < 0 || K < 0) return fail(FH_INVALID_ARGUMENT, "fh_gemm: negative dimension");
  if (M == 0 || N == 0) return FH_OK;
  if (A == nullptr || B == nullptr || C == nullptr) {
    if (K > 0 || C == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_gemm: null operand");
  }
  GemmArgs args{};
  args.A = A;
  args.B = B;
  args.C = C;
  args.M = M;
  args.N = N;
  args.K = K;
  args.lda = K;
  args.ldb = N;
  args.ldc = N;
  args.any_order = (flags & FH_GEMM_ANY_ORDER) != 0;
  args.row_softmax = (flags & FH_GEMM_ROW_SOFTMAX) != 0;
  fh_status st = copy_epilogue(epilogue, args.ep);
  if (st != FH_OK) return st;
  return run_gemm(dtype, args, 1, stream);
}

}  // namespace fh

extern "C" fh_status fh_gemm_ex(int32_t dtype, const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                                const fh_epilogue* epilogue, int32_t flags, void* stream) {
  return fh::gemm_with_epilogue_args(dtype, A, B, C, M, N, K, epilogue, static_cast<hipStream_t>(stream), flags);
}

extern "C" fh_status fh_gemm_grouped(int32_t dtype, const void* A, int32_t groups, const void* const* B, void* const* C,
                                     int64_t M, int64_t N, int64_t K, const fh_epilogue* epilogues, int32_t flags,
                                     void* stream) {
  using namespace fh;
  if (groups < 1 || groups > kGemmMaxGroups)
    return fail(FH_INVALID_ARGUMENT, "fh_gemm_grouped: groups must be in [1, " + std::to_string(kGemmMaxGroups) + "]");
  if (B == nullptr || C == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_gemm_grouped: null operand arrays");
  if ((flags & ~FH_GEMM_ANY_ORDER) != 0) return fail(FH_INVALID_ARGUMENT, "fh_gemm_grouped: unknown flags");
  // every group must carry the same epilogue program (one kernel instance serves them all)
  for (int g = 1; g < groups && epilogues != nullptr; ++g) {
    if (epilogues[g].nseg != epilogues[0].nseg || epilogues[g].round_between != epilogues[0].round_between)
      return fail(FH_INVALID_ARGUMENT, "fh_gemm_grouped: groups with different epilogue programs");
    for (int s = 0; s < epilogues[0].nseg && s < FH_MAX_SEGMENTS; ++s)
      if (epilogues[g].ops[s] != epilogues[0].ops[s])
        return fail(FH_INVALID_ARGUMENT, "fh_gemm_grouped: groups with different epilogue programs");
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool sixteen = dtype == FH_BF16 || dtype == FH_F16;
  if (sixteen && M > 0 && N > 0 && K > 0 && A != nullptr) {
    GemmArgs args{};
    args.A = A;
    args.B = B[0];
    args.C = C[0];
    args.M = M;
    args.N = N;
    args.K = K;
    args.lda = K;
    args.ldb = N;
    args.ldc = N;
    args.any_order = (flags & FH_GEMM_ANY_ORDER) != 0;
    fh_status st = copy_epilogue(epilogues, args.ep);
    if (st != FH_OK) return st;
    args.groups = groups;
    for (int g = 0; g < groups; ++g) {
      if (B[g] == nullptr || C[g] == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_gemm_grouped: null operand");
      args.group_b[g] = B[g];
      args.group_c[g] = C[g];
      EpilogueArgs eg{};
      if (epilogues != nullptr && (st = copy_epilogue(&epilogues[g], eg)) != FH_OK) return st;
      for (int sg = 0; sg < FH_MAX_SEGMENTS; ++sg) args.group_ins[g][sg] = eg.ins[sg];
    }
    // the MFMA kernel takes the groups as its second grid axis when the problem is one it accepts and is not small
    const int64_t tiles64 = ((M + 63) / 64) * ((N + 63) / 64) * groups;
    if (tiles64 >= 16 && gemm16_try_launch(dtype, args, groups, s, &st)) return st;
  }
  // otherwise: one GEMM per group
  for (int g = 0; g < groups; ++g) {
    const fh_status st = fh_gemm_ex(dtype, A, B[g], C[g], M, N, K, epilogues != nullptr ? &epilogues[g] : nullptr,
                                    flags, stream);
    if (st != FH_OK) return st;
  }
  return FH_OK;
}

extern "C" fh_status fh_gemm(int32_t dtype, const void* A, const void* B, void* C, int64_t M, int64_t N,
                             int64_t K, const fh_epilogue* epilogue, void* stream) {
  return fh::gemm_with_epilogue_args(dtype, A, B, C, M, N, K, epilogue, static_cast<hipStream_t>(stream), 0);
}

extern "C" fh_status fh_gemm_batched(int32_t dtype, const void* A, const void* B, void* C, int64_t M,
                                     int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc,
                                     int64_t stride_a, int64_t stride_b, int64_t stride_c, int64_t batch,
                                     void* stream) {
  using namespace fh;
  if (!is_supported_float(dtype)) return fail(FH_UNIMPLEMENTED, "fh_gemm_batched: unsupported dtype");
  if (M < 0 || N < 0 || K < 0 || batch < 0)
    return fail(FH_INVALID_ARGUMENT, "fh_gemm_batched: negative dimension");
  if (M == 0 || N == 0 || batch == 0) return FH_OK;
  if (lda < K || ldb < N || ldc < N)
    return fail(FH_INVALID_ARGUMENT, "fh_gemm_batched: leading dimension smaller than the row width");
  if (batch > 65535) return fail(FH_INVALID_ARGUMENT, "fh_gemm_batched: batch above 65535");
  GemmArgs args{};
  args.A = A;
  args.B = B;
  args.C = C;
  args.M = M;
  args.N = N;
  args.K = K;
  args.lda = lda;
  args.ldb = ldb;
  args.ldc = ldc;
  args.stride_a = stride_a;
  args.stride_b = stride_b;
  args.stride_c = stride_c;
  return run_gemm(dtype, args, batch, static_cast<hipStream_t>(stream));
}

// matmul_grad_lhs_internal (rhs = 0): out [m,k] = gy [m,n] * b[k,n]^T; matmul_grad_rhs_internal (rhs = 1):
// out [k,n] = a[m,k]^T * gy [m,n]. The sequential kernel reads the transposed operand in place, so every output is
// one fp32 sum over the contraction index in ascending order (reference: src/backends/cpu/kernels/matmul.cpp:187-327).
extern "C" fh_status fh_matmul_grad(int32_t dtype, int32_t rhs, const void* p, const void* q, void* out, int64_t m,
                                    int64_t n, int64_t k, void* stream) {
  using namespace fh;
  if (!is_supported_float(dtype)) return fail(FH_UNIMPLEMENTED, "fh_matmul_grad: unsupported dtype");
  if (m < 0 || n < 0 || k < 0) return fail(FH_INVALID_ARGUMENT, "fh_matmul_grad: negative dimension");
  GemmArgs args{};
  if (rhs == 0) {  // A = gy [m,n] (contraction n), B(j, c) = b[c * n + j]
    args.A = p, args.B = q, args.M = m, args.N = k, args.K = n, args.lda = n, args.ldb = n, args.ldc = k;
    args.trans_b = 1;
  } else {  // A(c, i) = a[i * k + c], B = gy [m,n] (contraction m)
    args.A = p, args.B = q, args.M = k, args.N = n, args.K = m, args.lda = k, args.ldb = n, args.ldc = n;
    args.trans_a = 1;
  }
  args.C = out;
  if (args.M == 0 || args.N == 0) return FH_OK;
  if (p == nullptr || q == nullptr || out == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_matmul_grad: null pointer");
  if ((args.M + kSeqT - 1) / kSeqT > 65535) return fail(FH_UNIMPLEMENTED, "fh_matmul_grad: more than 1,048,560 rows");
  const dim3 grid(static_cast<uint32_t>((args.N + kSeqT - 1) / kSeqT), static_cast<uint32_t>((args.M + kSeqT - 1) / kSeqT), 1);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case FH_F32:
      hipLaunchKernelGGL((gemm_seq_kernel<float>), grid, dim3(256), 0, s, args);
      break;
    case FH_BF16:
      hipLaunchKernelGGL((gemm_seq_kernel<bf16_t>), grid, dim3(256), 0, s, args);
      break;
    default:
      hipLaunchKernelGGL((gemm_seq_kernel<f16_t>), grid, dim3(256), 0, s, args);
      break;
  }
  return launch_status("fh_matmul_grad");
}
