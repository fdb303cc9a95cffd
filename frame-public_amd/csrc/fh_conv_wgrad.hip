// conv2d_grad_filter_internal on MFMA (bf16 / f16): the filter gradient as a GEMM over the batch-spatial positions,
//   dW[co][(a,b,ci)] = sum over p = (n, oh, ow) of dy[p][co] * x[n][oh*sh - ph + a][ow*sw - pw + b][ci],
// M = Cout, N = KH*KW*Cin, K = N*Ho*Wo, with both operands channels-last (dy [P][Cout], x [N][H][W][Cin]). K is
// the long dimension (batch times the output plane) and M*N is small, so K is split across workgroups: each
// writes an fp32 partial tile into a workspace, and a second kernel sums the partials in split order and writes
// dW in the reference's [Cout][Cin][KH][KW] layout with one rounding.
//
// Both operands are k-major (rows of p), so both MFMA fragments come from ds_read_b64_tr_b16 transpose reads of
// [BK][cols] LDS tiles (the B-operand path of the GEMM kernel, used for A as well). Tiles: WM (co) x 128 (a,b,ci)
// per workgroup with WM = 128 when Cout >= 128 (4 waves of 64 x 64, four 32x32x16 MFMA tiles each) and WM = 64
// otherwise (4 waves of 32 x 64, two tiles), register-staged loads with zero fill for rows past the split and
// taps in the padding, two LDS stages of 64 p-rows. The larger tile loads 1.5x fewer bytes per MFMA, which is
// what limits this kernel: operands come from L2 (x is read once per filter tap).
#include <algorithm>
#include <mutex>
#include <string>

#include "fh_mfma16.h"

namespace fh {
namespace {

using namespace mfma16;

constexpr int kWN = 128, kWK = 64;  // workgroup tile columns and rows per stage (WM is a template argument)
constexpr int kWThreads = 256;

struct WgradArgs {
  const void* x;   // [N][H][W][Cin] (Cin % 8 == 0)
  const void* dy;  // [P][Cout] (Cout % 8 == 0)
  float* part;     // [splits][Cout][NC]
  int32_t h, w, cin, cout, kw, sh, sw, ph, pw, oh, ow, nc, tiles_n;
  int64_t p, rows_per_split;
  uint64_t plane_m, ow_m;  // multiply-shift dividers for Ho*Wo and Wo (make_divider)
  uint32_t plane_s, ow_s;
};

// Division of 0 <= n < 2^31 by a fixed d >= 1 as floor(n * m / 2^s) (Granlund and Montgomery, "Division by
// invariant integers using multiplication", 1994, theorem 4.2 with N = 31): l = ceil(log2 d), s = 31 + l,
// m = floor(2^s / d) + 1, so 2^s < m d <= 2^s + 2^l and the quotient is exact. m <= 2^32, so n * m < 2^63.
inline void make_divider(int64_t d, uint64_t& m, uint32_t& s) {
  int l = 0;
  while ((int64_t{1} << l) < d) ++l;
  s = static_cast<uint32_t>(31 + l);
  m = (uint64_t{1} << s) / static_cast<uint64_t>(d) + 1;
}
__device__ __forceinline__ int32_t div_by(int32_t n, uint64_t m, uint32_t s) {
  return static_cast<int32_t>((static_cast<uint64_t>(static_cast<uint32_t>(n)) * m) >> s);
}

__device__ __forceinline__ int swz8(int krow) { return 2 * (krow & 3); }
__device__ __forceinline__ int swz16(int krow) { return (2 * (krow & 3)) ^ (8 * (krow & 1)); }

// Workgroup tile rows for a filter of cout output channels (the host's and the kernel's choice must agree).
inline int wgrad_wm(int64_t cout) { return cout >= 128 ? 128 : 64; }

template <typename T, int kWM>
__global__ __launch_bounds__(kWThreads) void conv_wgrad_kernel(WgradArgs a) {
  static_assert(kWM == 64 || kWM == 128, "tile rows");
  constexpr int MT = kWM / 64;  // 32-row MFMA tiles per wave
  using S = typename Io<T>::storage;
  __shared__ __attribute__((aligned(16))) S As[2][kWK * kWM];
  __shared__ __attribute__((aligned(16))) S Bs[2][kWK * kWN];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tm = blockIdx.x / a.tiles_n, tn = blockIdx.x % a.tiles_n;
  const int m0 = tm * kWM, n0 = tn * kWN;
  // p fits 32 bits (checked by the host)
  const int32_t p_begin = static_cast<int32_t>(static_cast<int64_t>(blockIdx.y) * a.rows_per_split);
  const int32_t p_end = static_cast<int32_t>(min(a.p, static_cast<int64_t>(p_begin) + a.rows_per_split));
  const S* __restrict__ X = static_cast<const S*>(a.x);
  const S* __restrict__ DY = static_cast<const S*>(a.dy);

  // A loads: kWK*(WM/8) chunks, rows t/(WM/8) + A_STEP i, column chunk t%(WM/8); B loads: kWK*16 chunks, rows
  // t/16 + 16 i, column chunk t%16 (a fixed filter tap and ci block per thread)
  constexpr int A_CH = kWM / 8, A_STEP = kWThreads / A_CH;
  // A rows of 8 chunks swizzle like the GEMM's A, rows of 16 chunks like B
  auto swza = [](int krow) { return kWM == 64 ? swz8(krow) : swz16(krow); };
  constexpr int A_LOADS = kWK * A_CH / kWThreads, B_LOADS = kWK * (kWN / 8) / kWThreads;
  const int a_row = tid / A_CH, a_chunk = tid % A_CH;
  const bool a_col_ok = m0 + 8 * a_chunk < a.cout;
  const int b_row = tid >> 4, b_chunk = tid & 15;
  const int ncol = n0 + 8 * b_chunk;
  const bool b_col_ok = ncol < a.nc;
  const int tap = b_col_ok ? ncol / a.cin : 0;
  const int ci = b_col_ok ? ncol - tap * a.cin : 0;
  const int ta = tap / a.kw, tb = tap - ta * a.kw;
  const int32_t plane = a.oh * a.ow;

  uint4 ra[A_LOADS], rb[B_LOADS];
  auto load = [&](int32_t p0) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int32_t p = p0 + a_row + A_STEP * i;
      ra[i] = (p < p_end && a_col_ok) ? *reinterpret_cast<const uint4*>(DY + static_cast<int64_t>(p) * a.cout + m0 + 8 * a_chunk)
                                      : uint4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const int32_t p = p0 + b_row + 16 * i;
      uint4 v{0, 0, 0, 0};
      if (p < p_end && b_col_ok) {
        const int32_t n = div_by(p, a.plane_m, a.plane_s);
        const int32_t rem = p - n * plane;
        const int32_t oh = div_by(rem, a.ow_m, a.ow_s), ow = rem - oh * a.ow;
        const int32_t ih = oh * a.sh - a.ph + ta, iw = ow * a.sw - a.pw + tb;
        if (ih >= 0 && ih < a.h && iw >= 0 && iw < a.w)
          v = *reinterpret_cast<const uint4*>(X + ((static_cast<int64_t>(n) * a.h + ih) * a.w + iw) * a.cin + ci);
      }
      rb[i] = v;
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int r = a_row + A_STEP * i;
      *reinterpret_cast<uint4*>(&As[buf][r * kWM + ((a_chunk ^ swza(r)) * 8)]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const int r = b_row + 16 * i;
      *reinterpret_cast<uint4*>(&Bs[buf][r * kWN + ((b_chunk ^ swz16(r)) * 8)]) = rb[i];
    }
  };

  // transpose-read addressing (bytes within a tile): lane group g = lane/16 covers 16 columns and 4 k rows;
  // lane q + 4e of the group points at row (kbase + e), columns 4q .. 4q+3 of the group's 16
  const int wm = wave >> 1, wn = wave & 1;
  const int g = lane >> 4, r16 = lane & 15, q = r16 & 3, e = r16 >> 2;
  const int krow0 = 8 * (g >> 1) + e;  // + 16 s + 4 h: krow & 3 and krow & 1 unchanged
  int a_off[MT], b_off[2];
  {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int col = wm * (kWM / 2) + 32 * mt + 16 * (g & 1) + 4 * q;
      a_off[mt] = krow0 * (kWM * 2) + ((col >> 3) ^ swza(krow0)) * 16 + (col & 7) * 2;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int c = wn * 64 + 32 * j + 16 * (g & 1) + 4 * q;
      b_off[j] = krow0 * (kWN * 2) + ((c >> 3) ^ swz16(krow0)) * 16 + (c & 7) * 2;
    }
  }

  f32x16_t acc[MT][2];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int x = 0; x < 16; ++x) acc[mt][j][x] = 0.0f;

  const int32_t steps = (p_end - p_begin + kWK - 1) / kWK;
  if (steps > 0) {
    load(p_begin);
    store(0);
  }
  __syncthreads();
  asm volatile("" ::: "memory");  // the transpose reads below are asm: keep them after the barrier
  for (int32_t it = 0; it < steps; ++it) {
    const int buf = it & 1;
    if (it + 1 < steps) load(p_begin + (it + 1) * kWK);
    const uint32_t abase = lds_addr((const FH_LDS void*)&As[buf][0]);
    const uint32_t bbase = lds_addr((const FH_LDS void*)&Bs[buf][0]);
    [&]<int... K_>(std::integer_sequence<int, K_...>) {
      (
          [&] {
            constexpr int s = K_;  // 16-row k-step within the stage
            u32x2_t al[MT], ah[MT], bl[2], bh[2];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              al[mt] = lds_read_tr16_b64<(16 * s) * kWM * 2>(abase + a_off[mt]);
              ah[mt] = lds_read_tr16_b64<(16 * s + 4) * kWM * 2>(abase + a_off[mt]);
            }
            bl[0] = lds_read_tr16_b64<(16 * s) * kWN * 2>(bbase + b_off[0]);
            bh[0] = lds_read_tr16_b64<(16 * s + 4) * kWN * 2>(bbase + b_off[0]);
            bl[1] = lds_read_tr16_b64<(16 * s) * kWN * 2>(bbase + b_off[1]);
            bh[1] = lds_read_tr16_b64<(16 * s + 4) * kWN * 2>(bbase + b_off[1]);
            if constexpr (MT == 1)
              asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(al[0]), "+v"(ah[0]), "+v"(bl[0]), "+v"(bh[0]), "+v"(bl[1]), "+v"(bh[1]));
            else
              asm volatile("s_waitcnt lgkmcnt(0)"
                           : "+v"(al[0]), "+v"(ah[0]), "+v"(al[1]), "+v"(ah[1]), "+v"(bl[0]), "+v"(bh[0]), "+v"(bl[1]),
                             "+v"(bh[1]));
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              const u32x4_t af{al[mt][0], al[mt][1], ah[mt][0], ah[mt][1]};
#pragma unroll
              for (int j = 0; j < 2; ++j) mfma32<T>(af, u32x4_t{bl[j][0], bl[j][1], bh[j][0], bh[j][1]}, acc[mt][j]);
            }
          }(),
          ...);
    }(std::make_integer_sequence<int, kWK / 16>{});
    // buf^1 was last read in the previous iteration, before its closing barrier: safe to refill now
    if (it + 1 < steps) store(buf ^ 1);
    __syncthreads();
    asm volatile("" ::: "memory");
  }

  // fp32 partial tile: row m = 8*(x/4) + 4*(lane/32) + x%4 of the wave's 32, column lane%32 of each 32-wide tile
  float* out = a.part + static_cast<int64_t>(blockIdx.y) * a.cout * a.nc;
  const int hi = lane >> 5, l32 = lane & 31;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + wn * 64 + 32 * j + l32;
      if (col >= a.nc) continue;
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        const int row = m0 + wm * (kWM / 2) + 32 * mt + 8 * (x >> 2) + 4 * hi + (x & 3);
        if (row < a.cout) out[static_cast<int64_t>(row) * a.nc + col] = acc[mt][j][x];
      }
    }
}

// dw[co][ci][kh][kw] = round(sum over splits, in order, of part[s][co][(kh*KW + kw)*cin_pad + ci]), ci < cin. One
// thread per workspace column in its natural (co, tap, ci) order, so the split-strided reads of a wave are
// contiguous; the scattered 2-byte writes are the small side.
template <typename T>
__global__ __launch_bounds__(64) void wgrad_reduce_kernel(const float* __restrict__ part, typename Io<T>::storage* __restrict__ dw,
                                                           int32_t splits, int32_t cout, int32_t cin, int32_t cin_pad,
                                                           int32_t taps, int64_t nc, int64_t total) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 64 + threadIdx.x;
  if (i >= total) return;
  const int32_t ci = static_cast<int32_t>(i % cin_pad);
  const int64_t r = i / cin_pad;
  const int32_t tap = static_cast<int32_t>(r % taps);
  const int32_t co = static_cast<int32_t>(r / taps);
  if (ci >= cin) return;
  const int64_t stride = static_cast<int64_t>(cout) * nc;
  // Sixteen partials in flight per batch, summed in split order (the order does not depend on the batching).
  constexpr int32_t kB = 16;
  float s = 0.0f;
  int32_t k = 0;
  for (; k + kB <= splits; k += kB) {
    float t[kB];
#pragma unroll
    for (int32_t u = 0; u < kB; ++u) t[u] = part[(k + u) * stride + i];
#pragma unroll
    for (int32_t u = 0; u < kB; ++u) s += t[u];
  }
  for (; k < splits; ++k) s += part[k * stride + i];
  dw[(static_cast<int64_t>(co) * cin + ci) * taps + tap] = Io<T>::store(s);
}

template <typename T>
fh_status run_wgrad(const WgradArgs& args, int32_t splits, int32_t cin_real, int32_t kh, void* dw, hipStream_t s) {
  const int wm = wgrad_wm(args.cout);
  const int tiles = ((args.cout + wm - 1) / wm) * args.tiles_n;
  const dim3 grid(static_cast<uint32_t>(tiles), static_cast<uint32_t>(splits));
  if (wm == 128)
    hipLaunchKernelGGL((conv_wgrad_kernel<T, 128>), grid, dim3(kWThreads), 0, s, args);
  else
    hipLaunchKernelGGL((conv_wgrad_kernel<T, 64>), grid, dim3(kWThreads), 0, s, args);
  if (fh_status st = launch_status("conv_wgrad_kernel"); st != FH_OK) return st;
  const int64_t total = static_cast<int64_t>(args.cout) * args.nc;  // every workspace column (co, tap, ci_pad)
  // 64-lane workgroups: the small layers' few thousand columns still spread over every CU
  hipLaunchKernelGGL((wgrad_reduce_kernel<T>), dim3(static_cast<uint32_t>((total + 63) / 64)), dim3(64), 0, s,
                     args.part, static_cast<typename Io<T>::storage*>(dw), splits, args.cout, cin_real, args.cin,
                     kh * args.kw, static_cast<int64_t>(args.nc), total);
  return launch_status("wgrad_reduce_kernel");
}

// ---- no-allocation variant -----------------------------------------------------------------------------------
// The split-K partials of fh_conv2d_wgrad_nhwc_noalloc live in this file-scope device array. Each device the
// library runs on holds its own copy until the process ends. In host code the name `scratch` is only a host-side
// stand-in: its device address is looked up once per device (hipGetSymbolAddress with that device current) and
// only that address is handed to kernels. Nothing in it needs to start at zero: the main kernel writes every
// partial of every split before the reduction reads it.
constexpr int64_t kWgradScratchBytes = int64_t{64} << 20;
constexpr int kScratchMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kWgradScratchBytes];

// Calls on one device are ordered through the array: each call's stream first waits for the event the previous
// call recorded after its kernels (on whatever stream that was), and the call records it again after its own.
// g_scratch_mu is held from the wait to the record, so the order is the order in which the host made the calls.
std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchMaxDevices] = {};
hipEvent_t g_scratch_done[kScratchMaxDevices] = {};

// Set-up, once per device with that device current (g_scratch_mu held): the array's device address and the
// ordering event. No device memory is allocated.
fh_status scratch_of_current_device_locked(int* dev_out, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return fail(FH_DEVICE_ERROR, "fh_conv2d_wgrad_nhwc_noalloc: hipGetDevice failed");
  if (dev < 0 || dev >= kScratchMaxDevices)
    return fail(FH_UNIMPLEMENTED, "fh_conv2d_wgrad_nhwc_noalloc: device index above 63");
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(FH_DEVICE_ERROR, std::string("fh_conv2d_wgrad_nhwc_noalloc: hipGetSymbolAddress(scratch): ") +
                                       hipGetErrorString(e));
    hipEvent_t ev = nullptr;
    const hipError_t ee = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (ee != hipSuccess)
      return fail(FH_DEVICE_ERROR, std::string("fh_conv2d_wgrad_nhwc_noalloc: hipEventCreateWithFlags: ") +
                                       hipGetErrorString(ee));
    g_scratch_done[dev] = ev;
    g_scratch_ptr[dev] = p;
  }
  *dev_out = dev;
  *out = g_scratch_ptr[dev];
  return FH_OK;
}

}  // namespace
}  // namespace fh

using namespace fh;

extern "C" int64_t fh_conv2d_wgrad_workspace(int32_t dtype, const int64_t geom[12], int32_t cin_pad, int32_t* splits) {
  if (dtype != FH_BF16 && dtype != FH_F16) return -1;
  if (geom == nullptr || geom[11] != 1 || cin_pad % 8 != 0 || cin_pad < geom[1] || geom[4] % 8 != 0) return -1;
  // every extent positive, strides positive, padding non-negative, each 31-bit; the padded input covers the filter
  for (int k = 0; k < 11; ++k)
    if (geom[k] < (k >= 9 ? 0 : 1) || geom[k] > 0x7fffffffLL) return -1;
  if (geom[2] + 2 * geom[9] < geom[5] || geom[3] + 2 * geom[10] < geom[6]) return -1;
  const int64_t oh = (geom[2] + 2 * geom[9] - geom[5]) / geom[7] + 1, ow = (geom[3] + 2 * geom[10] - geom[6]) / geom[8] + 1;
  const int64_t p = geom[0] * oh * ow, nc = geom[5] * geom[6] * cin_pad;
  if (p <= 0 || nc <= 0 || p >= (int64_t{1} << 31) - (int64_t{1} << 23) || nc > (1 << 30)) return -1;  // rows fit int32
  const int64_t wm = wgrad_wm(geom[4]);
  const int64_t tiles = ((geom[4] + wm - 1) / wm) * ((nc + kWN - 1) / kWN);
  // enough workgroups to fill the device twice over, each at least 512 p-rows, the workspace within 256 MiB
  int64_t sp = (2 * 256 + tiles - 1) / tiles;
  sp = std::min<int64_t>(sp, std::max<int64_t>(1, p / 512));
  sp = std::min<int64_t>(sp, std::max<int64_t>(1, (int64_t{256} << 20) / (4 * geom[4] * nc)));
  sp = std::max<int64_t>(1, std::min<int64_t>(sp, 65535));
  if (splits != nullptr) *splits = static_cast<int32_t>(sp);
  return sp * geom[4] * nc * 4;
}

extern "C" fh_status fh_conv2d_wgrad_nhwc(int32_t dtype, const void* x, const void* dy, void* dw, void* workspace,
                                          int64_t workspace_bytes, const int64_t geom[12], int32_t cin_pad, void* stream) {
  int32_t splits = 0;
  const int64_t need = fh_conv2d_wgrad_workspace(dtype, geom, cin_pad, &splits);
  if (need < 0) return fail(FH_UNIMPLEMENTED, "fh_conv2d_wgrad_nhwc: unsupported dtype or geometry");
  if (workspace_bytes < need) return fail(FH_INVALID_ARGUMENT, "fh_conv2d_wgrad_nhwc: workspace too small");
  for (int k = 0; k < 12; ++k)
    if (geom[k] < 0 || geom[k] > 0x7fffffffLL) return fail(FH_INVALID_ARGUMENT, "fh_conv2d_wgrad_nhwc: geometry out of range");
  if (x == nullptr || dy == nullptr || dw == nullptr || workspace == nullptr)
    return fail(FH_INVALID_ARGUMENT, "fh_conv2d_wgrad_nhwc: null pointer");
  WgradArgs a{};
  a.x = x, a.dy = dy, a.part = static_cast<float*>(workspace);
  a.h = static_cast<int32_t>(geom[2]), a.w = static_cast<int32_t>(geom[3]), a.cin = cin_pad;
  a.cout = static_cast<int32_t>(geom[4]), a.kw = static_cast<int32_t>(geom[6]);
  a.sh = static_cast<int32_t>(geom[7]), a.sw = static_cast<int32_t>(geom[8]);
  a.ph = static_cast<int32_t>(geom[9]), a.pw = static_cast<int32_t>(geom[10]);
  a.oh = static_cast<int32_t>((geom[2] + 2 * geom[9] - geom[5]) / geom[7] + 1);
  a.ow = static_cast<int32_t>((geom[3] + 2 * geom[10] - geom[6]) / geom[8] + 1);
  a.nc = static_cast<int32_t>(geom[5] * geom[6] * cin_pad);
  a.tiles_n = (a.nc + kWN - 1) / kWN;
  a.p = geom[0] * a.oh * a.ow;
  a.rows_per_split = ((a.p + splits - 1) / splits + kWK - 1) / kWK * kWK;
  if (a.oh <= 0 || a.ow <= 0) return fail(FH_INVALID_ARGUMENT, "fh_conv2d_wgrad_nhwc: empty output plane");
  make_divider(static_cast<int64_t>(a.oh) * a.ow, a.plane_m, a.plane_s);
  make_divider(a.ow, a.ow_m, a.ow_s);
  if (!(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(dy) % 16 == 0))
    return fail(FH_INVALID_ARGUMENT, "fh_conv2d_wgrad_nhwc: operands must be 16-byte aligned");
  if ((geom[4] * static_cast<int64_t>(a.nc) + 63) / 64 > 0xffffffffLL ||
      (geom[4] + wgrad_wm(geom[4]) - 1) / wgrad_wm(geom[4]) * static_cast<int64_t>(a.tiles_n) > 0xffffffffLL)
    return fail(FH_INVALID_ARGUMENT, "fh_conv2d_wgrad_nhwc: filter too large for one launch");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == FH_BF16) return run_wgrad<bf16_t>(a, splits, static_cast<int32_t>(geom[1]), static_cast<int32_t>(geom[5]), dw, s);
  return run_wgrad<f16_t>(a, splits, static_cast<int32_t>(geom[1]), static_cast<int32_t>(geom[5]), dw, s);
}

extern "C" fh_status fh_conv2d_wgrad_nhwc_noalloc(int32_t dtype, const void* x, const void* dy, void* dw,
                                                  const int64_t geom[12], int32_t cin_pad, void* stream) {
  const int64_t need = fh_conv2d_wgrad_workspace(dtype, geom, cin_pad, nullptr);
  if (need < 0) return fail(FH_UNIMPLEMENTED, "fh_conv2d_wgrad_nhwc_noalloc: unsupported dtype or geometry");
  if (need > kWgradScratchBytes)
    return fail(FH_INVALID_ARGUMENT, "fh_conv2d_wgrad_nhwc_noalloc: the split-K partials need " + std::to_string(need) +
                                         " bytes, above the " + std::to_string(kWgradScratchBytes) +
                                         "-byte no-allocation scratch (use fh_conv2d_wgrad_nhwc with a workspace)");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  void* ws = nullptr;
  int dev = -1;
  if (fh_status st = scratch_of_current_device_locked(&dev, &ws); st != FH_OK) return st;
  // Under graph capture the graph's own dependencies order the work (an event recorded outside the capture is not
  // waited on there): overlapping replays of such graphs on one device race.
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  FH_HIP_CHECK(hipStreamIsCapturing(s, &cap));
  const bool order = cap == hipStreamCaptureStatusNone;
  if (order) FH_HIP_CHECK(hipStreamWaitEvent(s, g_scratch_done[dev], 0));
  if (fh_status st = fh_conv2d_wgrad_nhwc(dtype, x, dy, dw, ws, need, geom, cin_pad, stream); st != FH_OK) return st;
  if (order) FH_HIP_CHECK(hipEventRecord(g_scratch_done[dev], s));
  return FH_OK;
}
