// Fused network stem for gfx950: y = max_pool2d(act(conv2d(x, w) + bias)) in one launch, NCHW in and out, with the
// convolution 7x7, stride 2, padding 3, Cin <= 4, Cout = 64, and the pool 3x3, stride 2, padding 1 (ResNet's stem;
// reference semantics: src/backends/cpu/kernels/conv.cpp:223-314 for the convolution, elementwise.cpp:329-331 for
// relu, pool.cpp:187-234 for the pool). The convolution output, 4x the pool output's size, never reaches HBM.
//
// Work decomposition: a workgroup owns one image and a run of pool rows; strip t is 7 pool columns, i.e. 16
// convolution columns (14t - 1 .. 14t + 14; 15 are read by the pool), and two waves own it, each with half of the
// output channels (two 16-channel tiles), so 16 waves share a CU (four per SIMD) to hide each other's LDS and memory
// waits. A wave walks down the rows, so the whole pool is done in registers: the horizontal 3-window inside each
// 16-lane row of the MFMA output, the vertical 3-window across the wave's consecutive rows. The per-row copies
// (raw rows in, unfolded rows, the pooled row out) move the same chunks every row, so their coordinates are
// worked out once per thread.
//
// GEMM per convolution row: C[64 cout][16 px] += W[64][K] * U[K][16 px] on v_mfma_f32_16x16x32_bf16, K ordered as
// (kh, c, kw) with kw padded from 7 to 8: each 8-k group of one (kh, c) is one lane's 16-byte fragment. The bias is
// one more group (7 Cin is never a multiple of 4, so the last k-step has room): its filter fragment holds the bias
// and its U fragment is {1, 0, ..., 0}, so bias x 1, exact, joins the fp32 sum. The filter fragments stay in
// registers for the whole kernel (the wave's 2 cout tiles x ceil(7 Cin / 4) k-steps); the U fragments come
// from LDS, where each input row is held "unfolded" per channel: for every output column ow the 8 values
// x[2 ow - 3 .. 2 ow + 3], 0 as one 16-byte chunk, so a fragment is one ds_read_b128. The zero in the eighth slot
// is in both operands, so no real pixel meets a zero weight (an infinite input stays finite where the reference's
// is). Unfolded input rows live in a 16-row LDS ring. Each pool row needs 4 new input rows: they are loaded from HBM
// (16-byte coalesced loads) two pool rows ahead while the MFMAs run, stored as raw rows with zero margins in LDS,
// and unfolded from there into the ring one pool row ahead, so the steady state needs no edge cases and one
// barrier per pool row.
//
// Numerics: the conv value of a pixel is the fp32 MFMA sum plus the bias (the reference adds the bias inside the fp32
// accumulator and rounds once). The pool takes the maximum of a window's fp32 sums and then applies the unfused
// chain's one rounding and relu to it: both are monotonic, so for values that are not NaN max(relu(round(x))) ==
// relu(round(max(x))), and only 2 of every 9 window cells are rounded. NaN follows the reference's scan (first valid
// element of the window in (kh, kw) order, then a strictly greater one replaces it): the result is NaN when the
// window's first valid cell is NaN, NaN cells are skipped otherwise. Between -0 and +0 of equal maxima the choice
// can differ from the first-occurrence rule (the matrix core's signed zeros already can).
#include <hip/hip_runtime.h>

#include <string>

#include "fh_common.h"

namespace fh {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kCout = 64;
constexpr int kMTiles = kCout / 16;
constexpr int kRing = 16;        // unfolded input rows resident in LDS
constexpr int kMaxStrips = 8;    // strips per workgroup: pool width up to 56
constexpr int kWps = 2;          // waves per strip, each with kMTiles / kWps of the output channel tiles
constexpr int kMt = kMTiles / kWps;
constexpr int kMaxCin = 3;
constexpr int kSlots = kMaxStrips * 16;  // unfolded chunks per row and channel (strip-major, 16 per strip)
constexpr int kRawPad = 8;               // zero elements left of a raw row (and at least 8 right of it)
constexpr int kMaxW = 224;               // input width bound (pool width 56)
constexpr int kRawStride = kMaxW + 2 * kRawPad;  // elements per raw row and channel
constexpr int kOutBytes = kCout * kMaxStrips * 7 * 2;  // one pool row, all channels

struct StemArgs {
  const uint16_t* x;
  const uint16_t* w;
  const uint16_t* bias;  // may be null
  uint16_t* y;
  int32_t cin, h, w_in;  // input
  int32_t oh, ow;        // convolution output
  int32_t ph, pw;        // pool output
  int32_t strips;        // waves = ceil(pw / 7)
  int32_t rows_per_wg;   // pool rows per workgroup
  int32_t wgs_per_img;
  int32_t relu;
};

template <typename T>
__device__ __forceinline__ f32x4_t mfma16(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
  if constexpr (std::is_same_v<T, bf16_t>) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                   0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
  }
}

// Lane l of a 16-lane row receives lane l + N's value (DPP row_shl:N; lanes past the row end keep their own).
template <int N>
__device__ __forceinline__ float from_right(float v) {
  const int i = __float_as_int(v);
  return __int_as_float(__builtin_amdgcn_update_dpp(i, i, 0x100 + N, 0xf, 0xf, false));
}

// Maximum of the operands that are not NaN (NaN when all are): v_max3_f32 / v_max_f32 in the kernel's IEEE mode,
// as inline asm so the compiler adds no canonicalising moves in front of them.
__device__ __forceinline__ float max3_nan_skip(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ float max2_nan_skip(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// The unfolded chunk x[2 ow - 3 .. 2 ow + 3], 0 from an 8-element window starting at column 2 ow - 4 held in
// four dwords (d[0] low half = column 2 ow - 4).
__device__ __forceinline__ uint4 unfold_window(const uint32_t (&d)[4]) {
  return uint4{__builtin_amdgcn_alignbit(d[1], d[0], 16), __builtin_amdgcn_alignbit(d[2], d[1], 16),
               __builtin_amdgcn_alignbit(d[3], d[2], 16), d[3] >> 16};
}

// Output column of unfolded slot `slot` (strip slot >> 4, lane slot & 15).
__device__ __forceinline__ int slot_ow(int slot) { return 14 * (slot >> 4) - 1 + (slot & 15); }

template <typename T, int CIN>
__global__ __launch_bounds__(kMaxStrips * kWps * 64, 1) void conv_stem_pool_kernel(StemArgs a) {
  constexpr int KS = (7 * CIN + 3) / 4;  // k-steps of 32
  constexpr int kRowBytes = CIN * kSlots * 16;            // one unfolded row, all channels
  constexpr int kRingBytes = kRing * kRowBytes;
  constexpr int kRawBytes = 4 * CIN * kRawStride * 2;     // the 4 raw input rows of one pool row
  constexpr int kPackedBytes = kMTiles * KS * 64 * 16;    // filter fragments, [m][s][lane]
  constexpr int OFF_ZERO = kRingBytes, OFF_ONE = OFF_ZERO + 16, OFF_RAW = OFF_ONE + 16;
  constexpr int OFF_OUT = OFF_RAW + 2 * kRawBytes, OFF_PACK = OFF_OUT + 2 * kOutBytes;
  constexpr int LDS_BYTES = OFF_PACK + kPackedBytes;
  static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
  __shared__ __attribute__((aligned(16))) unsigned char lds[LDS_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int strip = wave / kWps, m0 = (wave % kWps) * kMt;  // this wave's strip and first channel tile
  const int nthreads = a.strips * kWps * 64;
  const int i16 = lane & 15, g4 = lane >> 4;
  const int W = a.w_in, H = a.h;
  const int wchunks = W / 8;  // 16-byte chunks per input row and channel

  const int img = blockIdx.x / a.wgs_per_img;
  const int p_begin = (blockIdx.x - img * a.wgs_per_img) * a.rows_per_wg;
  const int p_end = min(p_begin + a.rows_per_wg, a.ph);
  const uint16_t* __restrict__ x_img = a.x + static_cast<int64_t>(img) * CIN * H * W;
  auto ring_off = [&](int ir, int c, int slot) { return ((ir & (kRing - 1)) * CIN + c) * (kSlots * 16) + slot * 16; };
  auto raw_off = [&](int buf, int rr, int c) { return OFF_RAW + buf * kRawBytes + ((rr * CIN + c) * kRawStride) * 2; };

  // ---- set-up: zero chunk, fp32 bias, zero raw margins, packed filter fragments ----
  // the zero chunk, and the "one" chunk {1, 0, ..., 0} that the bias group multiplies
  if (tid == 0) *reinterpret_cast<uint4*>(lds + OFF_ZERO) = uint4{0, 0, 0, 0};
  if (tid == 1) *reinterpret_cast<uint4*>(lds + OFF_ONE) = uint4{Io<T>::store(1.0f), 0, 0, 0};
  for (int i = tid; i < 2 * kRawBytes / 16; i += nthreads)
    *reinterpret_cast<uint4*>(lds + OFF_RAW + 16 * i) = uint4{0, 0, 0, 0};
  for (int idx = tid; idx < kMTiles * KS * 64; idx += nthreads) {
    const int l = idx & 63, ms = idx >> 6, m = ms / KS, s = ms - m * KS;
    const int co = 16 * m + (l & 15), g = 4 * s + (l >> 4);  // (kh, c) group of lane l's 8 k
    uint32_t e[4] = {0, 0, 0, 0};
    if (g < 7 * CIN) {
      const int kh = g / CIN, c = g - kh * CIN;
      const uint16_t* src = a.w + ((static_cast<int64_t>(co) * CIN + c) * 7 + kh) * 7;
      for (int k = 0; k < 7; ++k) e[k >> 1] |= static_cast<uint32_t>(src[k]) << (16 * (k & 1));
    } else if (g == 7 * CIN && a.bias != nullptr) {
      e[0] = a.bias[co];  // the bias group: bias x 1 (exact) joins the fp32 sum
    }
    *reinterpret_cast<uint4*>(lds + OFF_PACK + idx * 16) = uint4{e[0], e[1], e[2], e[3]};
  }
  // the unfolded rows of the first pool row (and of the row before it), straight from HBM with the image edges
  for (int qi = tid; qi < 11 * CIN * kSlots; qi += nthreads) {
    const int slot = qi % kSlots, rc = qi / kSlots, c = rc % CIN, ir = 4 * p_begin - 5 + rc / CIN;
    const int ow = slot_ow(slot);
    uint32_t o[4] = {0, 0, 0, 0};
    if (ir >= 0 && ir < H) {
      const uint16_t* row = x_img + (static_cast<int64_t>(c) * H + ir) * W;
      for (int k = 0; k < 7; ++k) {
        const int col = 2 * ow - 3 + k;
        if (col >= 0 && col < W) o[k >> 1] |= static_cast<uint32_t>(row[col]) << (16 * (k & 1));
      }
    }
    *reinterpret_cast<uint4*>(lds + ring_off(ir, c, slot)) = uint4{o[0], o[1], o[2], o[3]};
  }
  __syncthreads();  // zero margins before the raw rows below land between them; packed fragments complete

  // The per-row copies below move the same chunks every pool row, so each thread's chunk coordinates (integer
  // divisions by run-time sizes, some forty instructions each) are worked out once, here.
  // load_raw / store_raw: chunk lr_k of raw row lr_rr, channel lr_c; one 16-byte chunk per thread (4 rows x CIN x
  // W / 8 <= nthreads)
  const int lr_k = tid % wchunks, lr_rc = tid / wchunks;
  const int lr_c = lr_rc % CIN, lr_rr = lr_rc / CIN;
  const bool lr_on = tid < 4 * CIN * wchunks;
  const uint16_t* lr_src = x_img + (static_cast<int64_t>(lr_c) * H + lr_rr) * W + 8 * lr_k;  // + (4 p + 2) W
  const int lr_dst = raw_off(0, lr_rr, lr_c) + (kRawPad + 8 * lr_k) * 2;          // + buffer * kRawBytes
  // unfold_raw: the 4 CIN 16 strips = CIN nthreads / kWps chunks of a pool row, UF per thread (qi = tid + k nthreads,
  // the last ones only where qi is below that count); columns 2 ow - 4 .. 2 ow + 3 sit at raw elements 2 ow + 4 ..
  // (even: dword-aligned)
  constexpr int UF = (CIN + kWps - 1) / kWps;
  int uf_src[UF], uf_dst[UF], uf_rr[UF];
  bool uf_on[UF];
#pragma unroll
  for (int k = 0; k < UF; ++k) {
    const int qi = tid + k * nthreads;
    const int slot = qi % (16 * a.strips), rc = qi / (16 * a.strips), c = rc % CIN, rr = rc / CIN;
    uf_on[k] = qi < 64 * CIN * a.strips;
    uf_src[k] = raw_off(0, rr & 3, c) + (2 * slot_ow(slot) + kRawPad - 4) * 2;
    uf_dst[k] = ring_off(0, c, slot);  // + ring row * CIN * kSlots * 16
    uf_rr[k] = rr;
  }

  // raw input rows 4p + 6 .. 4p + 9 (the new rows of pool row p + 1) -> registers, then -> raw buffer (p + 1) & 1
  auto load_raw = [&](int p, uint4& v) -> bool {
    if (p >= p_end || !lr_on) return false;
    const int ir = 4 * p + 2 + lr_rr;
    v = uint4{0, 0, 0, 0};
    if (ir >= 0 && ir < H) v = *reinterpret_cast<const uint4*>(lr_src + static_cast<int64_t>(4 * p + 2) * W);
    return true;
  };
  auto store_raw = [&](int p, const uint4& v) {
    uint2* dst = reinterpret_cast<uint2*>(lds + lr_dst + (p & 1) * kRawBytes);
    dst[0] = uint2{v.x, v.y};
    dst[1] = uint2{v.z, v.w};
  };
  // raw buffer (p & 1), rows 4p + 2 .. 4p + 5 -> unfolded ring rows
  auto unfold_raw = [&](int p) {
#pragma unroll
    for (int k = 0; k < UF; ++k) {
      if (!uf_on[k]) continue;
      const uint32_t* src = reinterpret_cast<const uint32_t*>(lds + uf_src[k] + (p & 1) * kRawBytes);
      const uint32_t d[4] = {src[0], src[1], src[2], src[3]};
      const int row = (4 * p + 2 + uf_rr[k]) & (kRing - 1);
      *reinterpret_cast<uint4*>(lds + uf_dst[k] + row * (CIN * kSlots * 16)) = unfold_window(d);
    }
  };
  {
    uint4 v;
    if (load_raw(p_begin + 1, v)) store_raw(p_begin + 1, v);
  }
  __syncthreads();

  u32x4_t wf[kMt][KS];
#pragma unroll
  for (int m = 0; m < kMt; ++m)
#pragma unroll
    for (int s = 0; s < KS; ++s)
      wf[m][s] = *reinterpret_cast<const u32x4_t*>(lds + OFF_PACK + (((m0 + m) * KS + s) * 64 + lane) * 16);

  // ---- one convolution row r of this wave's strip: C[16 px][64 cout] on the matrix core with the pixels in M, so
  // lane l holds 4 consecutive pixel slots (4a .. 4a + 3, a = l / 16) of channel 16 m + l % 16 per tile m. The lane
  // then holds the row's part of two pool windows: pool column 2a (slots 4a, 4a + 1, 4a + 2) and 2a + 1 (slots
  // 4a + 2, 4a + 3 and 4a + 4, the next lane group's first). sink(m, w, h, first) gets for tile m and window w the
  // maximum of the window's valid cells in this row (fp32 sums, NaN cells skipped; NaN when none) and the window's
  // first valid cell in this row. ----
  const int base_col = 14 * strip - 1 + 4 * g4;  // convolution column of slot 4a
  const int lane_slot = 16 * strip + i16;        // the pixel slot whose unfolded input this lane supplies (MFMA A row)
  // whether a cell of this wave's windows lies outside the output (the first and the last strip): uniform per wave
  const bool wave_edge = __any(base_col < 0 || base_col + 4 >= a.ow) != 0;
  const float qnan = __builtin_nanf("");
  // per k-step s: this lane's (kh, c) group g = 4 s + g4 and the part of its fragment address that does not depend
  // on the row; groups past 7 CIN read the "one" chunk (the bias group g = 7 CIN, whose filter fragment holds the
  // bias: 7 CIN is never a multiple of 4 for CIN <= 3, so there is always a free group) or the zero chunk
  int frag_base[KS], frag_kh[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const int g = 4 * s + g4, kh = g / CIN, c = g - kh * CIN;
    frag_kh[s] = g >= 7 * CIN ? -1 : kh;
    frag_base[s] = g > 7 * CIN ? OFF_ZERO : g == 7 * CIN ? OFF_ONE : ring_off(0, c, lane_slot);
  }
  auto conv_row = [&](int r, auto&& sink) {
    // every fragment read of the row first, then the products (one LDS latency per row, not per k-step)
    u32x4_t px[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int off = frag_kh[s] < 0 ? frag_base[s]
                                     : frag_base[s] + ((2 * r - 3 + frag_kh[s]) & (kRing - 1)) * (CIN * kSlots * 16);
      px[s] = *reinterpret_cast<const u32x4_t*>(lds + off);
    }
    f32x4_t acc[kMt];
#pragma unroll
    for (int m = 0; m < kMt; ++m) acc[m] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int m = 0; m < kMt; ++m) acc[m] = mfma16<T>(px[s], wf[m][s], acc[m]);
    const bool row_ok = r < a.oh;
#pragma unroll
    for (int m = 0; m < kMt; ++m) {
      float v[5] = {acc[m][0], acc[m][1], acc[m][2], acc[m][3], 0.0f};
      v[4] = __shfl_down(v[0], 16);  // slot 4a + 4 (lanes 48..63: unused)
      float first_a = v[0];
      if (wave_edge) {  // cells outside the output are absent: NaN, which the maximum skips
#pragma unroll
        for (int j = 0; j < 5; ++j)
          if (base_col + j < 0 || base_col + j >= a.ow) v[j] = qnan;
        first_a = base_col < 0 ? v[1] : v[0];  // column -1 is absent
      }
      sink(m, 0, row_ok ? max3_nan_skip(v[0], v[1], v[2]) : qnan, first_a);
      sink(m, 1, row_ok ? max3_nan_skip(v[2], v[3], v[4]) : qnan, v[2]);
    }
  };

  // R: the running maximum of the current window's valid cells (NaN while there is none);
  // F: the window's first valid cell (in row 2p - 1, or in row 2p when p == 0): the result is NaN when it is
  float R[kMt][2], F[kMt][2];
#pragma unroll
  for (int m = 0; m < kMt; ++m)
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      R[m][w] = qnan;
      F[m][w] = 0.0f;
    }
  bool have_prev = p_begin > 0;
  if (have_prev)
    conv_row(2 * p_begin - 1, [&](int m, int w, float h, float first) {
      R[m][w] = h;
      F[m][w] = first;
    });

  // the output copy's first chunk per thread (pw % 8 == 0): channel oc_co, 8-column group oc_k, its staging offset
  // and its place in y less the pool row's
  const int oc_per_c = a.pw / 8;
  const int oc_co = oc_per_c > 0 ? tid / oc_per_c : 0, oc_k = tid - oc_co * oc_per_c;
  const bool oc_on = tid < kCout * oc_per_c;
  const int oc_lds = (oc_co * a.pw + 8 * oc_k) * 2;
  const int64_t cstride = static_cast<int64_t>(a.ph) * a.pw;
  uint16_t* const y_img = a.y + static_cast<int64_t>(img) * kCout * cstride;
  uint16_t* const oc_dst = y_img + oc_co * cstride + 8 * oc_k;  // + p pw
  const int q0 = 7 * strip + 2 * g4;  // pool columns q0 (window 0) and q0 + 1 (window 1, for a < 3)
  const bool write0 = q0 < a.pw, write1 = g4 < 3 && q0 + 1 < a.pw;
  int st_off[kMt];  // staging offset of this lane's window 0 in the wave's tile m (window 1 is 2 bytes on)
#pragma unroll
  for (int m = 0; m < kMt; ++m) st_off[m] = ((16 * (m0 + m) + i16) * a.pw + q0) * 2;
  for (int p = p_begin; p < p_end; ++p) {
    // Ring rows of pool row p (4p - 3 .. 4p + 5) are in place. Rows 4p + 6 .. 4p + 9 (pool row p + 1) are raw in
    // buffer (p + 1) & 1: unfold them into ring slots no row of this step reads; load the raw rows of p + 2.
    if (p + 1 < p_end) unfold_raw(p + 1);
    uint4 pre;
    const bool loaded = load_raw(p + 2, pre);
    __builtin_amdgcn_sched_barrier(0);
    if (!have_prev) {  // pool row 0: the window starts at row 0 (row -1 is padding)
      conv_row(2 * p, [&](int m, int w, float h, float first) {
        R[m][w] = h;
        F[m][w] = first;
      });
    } else {
      conv_row(2 * p, [&](int m, int w, float h, float) { R[m][w] = max2_nan_skip(R[m][w], h); });
    }
    unsigned char* ob = lds + OFF_OUT + (p & 1) * kOutBytes;
    __builtin_amdgcn_sched_barrier(0);
    conv_row(2 * p + 1, [&](int m, int w, float h, float first) {
      // the window's maximum, then the one rounding and relu of the unfused chain (both monotonic, so they commute
      // with the maximum); NaN when the window's first valid cell is NaN
      float best = Io<T>::round(max2_nan_skip(R[m][w], h));
      if (a.relu && best < 0.0f) best = 0.0f;
      if (F[m][w] != F[m][w]) best = qnan;
      if (w == 0 ? write0 : write1) *reinterpret_cast<uint16_t*>(ob + st_off[m] + 2 * w) = Io<T>::store(best);
      R[m][w] = h;  // row 2p + 1 opens the next window
      F[m][w] = first;
    });
    have_prev = true;
    __builtin_amdgcn_sched_barrier(0);
    if (loaded) store_raw(p + 2, pre);
    __syncthreads();
    // pool row p, all channels, from the staging buffer to y
    uint16_t* yrow = y_img + static_cast<int64_t>(p) * a.pw;
    if ((a.pw & 7) == 0) {
      // chunk i = tid (coordinates worked out before the loop) and, where 64 pw / 8 > nthreads, the rest
      if (oc_on) *reinterpret_cast<uint4*>(oc_dst + static_cast<int64_t>(p) * a.pw) = *reinterpret_cast<const uint4*>(ob + oc_lds);
      for (int i = tid + nthreads; i < kCout * oc_per_c; i += nthreads) {
        const int co = i / oc_per_c, k = i - co * oc_per_c;
        *reinterpret_cast<uint4*>(yrow + co * cstride + 8 * k) = *reinterpret_cast<const uint4*>(ob + (co * a.pw + 8 * k) * 2);
      }
    } else {
      for (int i = tid; i < kCout * a.pw; i += nthreads) {
        const int co = i / a.pw, k = i - co * a.pw;
        yrow[co * cstride + k] = *reinterpret_cast<const uint16_t*>(ob + (co * a.pw + k) * 2);
      }
    }
  }
}

template <typename T, int CIN>
fh_status launch_stem(const StemArgs& a, int grid, hipStream_t s) {
  hipLaunchKernelGGL((conv_stem_pool_kernel<T, CIN>), dim3(static_cast<uint32_t>(grid)),
                     dim3(static_cast<uint32_t>(a.strips * kWps * 64)), 0, s, a);
  return launch_status("conv_stem_pool_kernel launch");
}

}  // namespace
}  // namespace fh

using namespace fh;

extern "C" int32_t fh_conv2d_stem_pool_supported(int32_t dtype, const int64_t geom[12], const int64_t pool[6]) {
  if (dtype != FH_BF16 && dtype != FH_F16) return 0;
  if (geom == nullptr || pool == nullptr) return 0;
  const int64_t n = geom[0], cin = geom[1], h = geom[2], w = geom[3], cout = geom[4];
  if (n < 1 || cin < 1 || cin > kMaxCin || cout != kCout || geom[11] != 1) return 0;
  if (geom[5] != 7 || geom[6] != 7 || geom[7] != 2 || geom[8] != 2 || geom[9] != 3 || geom[10] != 3) return 0;
  if (pool[0] != 3 || pool[1] != 3 || pool[2] != 2 || pool[3] != 2 || pool[4] != 1 || pool[5] != 1) return 0;
  if (h < 1 || w < 8 || w % 8 != 0 || w > kMaxW || h > (1 << 20)) return 0;
  const int64_t oh = (h + 6 - 7) / 2 + 1, ow = (w + 6 - 7) / 2 + 1;
  const int64_t ph = (oh + 2 - 3) / 2 + 1, pw = (ow + 2 - 3) / 2 + 1;
  if (oh < 1 || ow < 1 || ph < 1 || pw < 1 || (pw + 6) / 7 > kMaxStrips) return 0;
  if (4 * cin * (w / 8) > 64 * ((pw + 6) / 7)) return 0;  // one raw 16-byte chunk per thread and pool row
  if (n * cin * h * w >= (int64_t{1} << 31) || n * cout * ph * pw >= (int64_t{1} << 31)) return 0;
  return 1;
}

extern "C" fh_status fh_conv2d_stem_pool(int32_t dtype, const void* x, const void* w, const void* bias, void* y,
                                         const int64_t geom[12], const int64_t pool[6], int32_t relu, void* stream) {
  if (fh_conv2d_stem_pool_supported(dtype, geom, pool) == 0)
    return fail(FH_UNIMPLEMENTED, "fh_conv2d_stem_pool: unsupported dtype or geometry (conv 7x7/2 pad 3, Cin <= 3, "
                                  "Cout 64, W % 8 == 0, W <= 224; pool 3x3/2 pad 1)");
  if (x == nullptr || w == nullptr || y == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_conv2d_stem_pool: null pointer");
  if ((reinterpret_cast<uintptr_t>(y) & 15) != 0 || (reinterpret_cast<uintptr_t>(x) & 15) != 0)
    return fail(FH_INVALID_ARGUMENT, "fh_conv2d_stem_pool: x and y must be 16-byte aligned");
  StemArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.w = static_cast<const uint16_t*>(w);
  a.bias = static_cast<const uint16_t*>(bias);
  a.y = static_cast<uint16_t*>(y);
  a.cin = static_cast<int32_t>(geom[1]);
  a.h = static_cast<int32_t>(geom[2]);
  a.w_in = static_cast<int32_t>(geom[3]);
  a.oh = (a.h + 6 - 7) / 2 + 1;
  a.ow = (a.w_in + 6 - 7) / 2 + 1;
  a.ph = (a.oh + 2 - 3) / 2 + 1;
  a.pw = (a.ow + 2 - 3) / 2 + 1;
  a.strips = (a.pw + 6) / 7;
  a.relu = relu != 0 ? 1 : 0;
  // pool rows per workgroup: about one workgroup per CU over the whole batch
  const int64_t n = geom[0];
  const int64_t cus = device_cu_count();
  int64_t rows = (n * a.ph + cus - 1) / cus;
  rows = rows < 1 ? 1 : (rows > a.ph ? a.ph : rows);
  a.rows_per_wg = static_cast<int32_t>(rows);
  a.wgs_per_img = static_cast<int32_t>((a.ph + rows - 1) / rows);
  const int64_t grid = n * a.wgs_per_img;
  if (grid >= (int64_t{1} << 31)) return fail(FH_INVALID_ARGUMENT, "fh_conv2d_stem_pool: grid too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool bf = dtype == FH_BF16;
  const int g = static_cast<int>(grid);
  switch (a.cin) {
    case 1: return bf ? launch_stem<bf16_t, 1>(a, g, s) : launch_stem<f16_t, 1>(a, g, s);
    case 2: return bf ? launch_stem<bf16_t, 2>(a, g, s) : launch_stem<f16_t, 2>(a, g, s);
    case 3: return bf ? launch_stem<bf16_t, 3>(a, g, s) : launch_stem<f16_t, 3>(a, g, s);
    default: return bf ? launch_stem<bf16_t, 3>(a, g, s) : launch_stem<f16_t, 3>(a, g, s);
  }
}
