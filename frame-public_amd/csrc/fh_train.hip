// Training-path kernels: the gradient-only ops of compiler::build_backward_graph's graphs (pool gradients, conv
// gradients, sum and its gradient, mse_loss and its gradient). matmul_grad_{lhs,rhs} are lowered to a transpose
// plus the GEMM kernels by the backend, relu_grad_internal is an elementwise program op (FH_EW_RELU_GRAD).
//
// Where a result is a per-element sequential sum in the reference (pool gradients, conv gradients), each output is
// accumulated by one thread in the reference's order with the same fp32 operations, so fp32 results are
// bit-identical and 16-bit ones differ only if the reference's single final rounding does (it does not: same
// float, same rounding). sum and mse_loss are tree reductions in fp32 (deterministic, not in the reference's
// order); their parity is a tolerance.
#include <algorithm>

#include "fh_common.h"

namespace fh {
namespace {

constexpr int kThreads = 256;

int64_t blocks_for(int64_t n, int per = kThreads) { return (n + per - 1) / per; }

// ---- pool gradients (gather form) --------------------------------------------------------------------------

struct PoolG {
  int32_t n, c, h, w, kh, kw, sh, sw, ph, pw, oh, ow;
};

// One thread per input element. max: the covering windows in (oh, ow) ascending order, each window's argmax
// recomputed exactly as the forward (first strict maximum in (kh, kw) order over non-padding taps), dy added
// when the argmax is this element (reference: src/backends/cpu/kernels/pool.cpp:186-206, 358-388, where the
// windows scatter in that order into a float buffer). avg: kh then kw ascending over the covering windows, sum of
// dy, then / (KH*KW) (reference: pool.cpp:543-566). MODE 2 is max followed by relu_grad_internal against the
// pool's input: dx = x > 0 ? max-pool gradient : 0 (elementwise.cpp:407-414), both values as the separate ops
// store them.
template <typename T, int MODE>
__global__ __launch_bounds__(kThreads) void pool2d_grad_kernel(const typename Io<T>::storage* __restrict__ dy,
                                                               const typename Io<T>::storage* __restrict__ x,
                                                               typename Io<T>::storage* __restrict__ dx, PoolG g,
                                                               int64_t total) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= total) return;
  const int32_t iw = static_cast<int32_t>(i % g.w);
  const int32_t ih = static_cast<int32_t>((i / g.w) % g.h);
  const int64_t nc = i / (static_cast<int64_t>(g.w) * g.h);
  const auto* dyp = dy + nc * g.oh * g.ow;
  float acc = 0.0f;
  if constexpr (MODE != 1) {
    const auto* xp = x + nc * g.h * g.w;
    // windows whose rows cover ih: oh*sh - ph <= ih <= oh*sh - ph + kh - 1
    const int32_t th = ih + g.ph - g.kh + 1, tw = iw + g.pw - g.kw + 1;  // first window start reaching ih / iw
    const int32_t oh_lo = th <= 0 ? 0 : (th + g.sh - 1) / g.sh;
    const int32_t ow_lo = tw <= 0 ? 0 : (tw + g.sw - 1) / g.sw;
    const int32_t oh_hi = min(g.oh - 1, (ih + g.ph) / g.sh);
    const int32_t ow_hi = min(g.ow - 1, (iw + g.pw) / g.sw);
    for (int32_t oh = oh_lo; oh <= oh_hi; ++oh) {
      const int32_t h0 = oh * g.sh - g.ph;
      if (ih < h0 || ih >= h0 + g.kh) continue;
      for (int32_t ow = ow_lo; ow <= ow_hi; ++ow) {
        const int32_t w0 = ow * g.sw - g.pw;
        if (iw < w0 || iw >= w0 + g.kw) continue;
        bool found = false;
        float best = 0.0f;
        int32_t at = -1;
        for (int32_t a = 0; a < g.kh; ++a) {
          const int32_t hh = h0 + a;
          if (hh < 0 || hh >= g.h) continue;
          for (int32_t b = 0; b < g.kw; ++b) {
            const int32_t ww = w0 + b;
            if (ww < 0 || ww >= g.w) continue;
            const float v = Io<T>::load(xp[hh * g.w + ww]);
            if (!found || v > best) {
              found = true;
              best = v;
              at = hh * g.w + ww;
            }
          }
        }
        if (at == ih * g.w + iw) acc += Io<T>::load(dyp[oh * g.ow + ow]);
      }
    }
    if constexpr (MODE == 2) acc = Io<T>::load(xp[ih * g.w + iw]) > 0.0f ? acc : 0.0f;
    dx[i] = Io<T>::store(acc);
  } else {
    for (int32_t a = 0; a < g.kh; ++a) {
      const int32_t nh = ih + g.ph - a;
      if (nh < 0 || nh % g.sh != 0) continue;
      const int32_t oh = nh / g.sh;
      if (oh >= g.oh) continue;
      for (int32_t b = 0; b < g.kw; ++b) {
        const int32_t nw = iw + g.pw - b;
        if (nw < 0 || nw % g.sw != 0) continue;
        const int32_t ow = nw / g.sw;
        if (ow >= g.ow) continue;
        acc += Io<T>::load(dyp[oh * g.ow + ow]);
      }
    }
    dx[i] = Io<T>::store(acc / static_cast<float>(g.kh * g.kw));
  }
}

// max_pool2d_grad for the 3x3 / stride 2 / padding 1 window (the ResNet stem pool): one thread per 2x2 input block
// (rows 2i, 2i+1, columns 2j, 2j+1), whose covering windows are exactly (oh, ow) in {i, i+1} x {j, j+1}. Each of
// the four windows' argmax is found once (first strict maximum in (kh, kw) order, as the forward) and every input of
// the block adds the dy of the windows that chose it in (oh, ow) order: the same sums as the generic kernel.
// RELU: then relu_grad against x (dx = x > 0 ? sum : 0), as pool2d_grad_kernel's MODE 2.
template <typename T, bool RELU>
__global__ __launch_bounds__(kThreads) void maxpool3s2_grad_kernel(const typename Io<T>::storage* __restrict__ dy,
                                                                   const typename Io<T>::storage* __restrict__ x,
                                                                   typename Io<T>::storage* __restrict__ dx, int32_t h,
                                                                   int32_t w, int32_t oh, int32_t ow, int32_t bh,
                                                                   int32_t bw, int64_t total) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (t >= total) return;
  const int32_t bj = static_cast<int32_t>(t % bw);
  const int64_t r = t / bw;
  const int32_t bi = static_cast<int32_t>(r % bh);
  const int64_t nc = r / bh;
  const auto* xp = x + nc * h * w;
  const auto* dyp = dy + nc * oh * ow;
  int32_t arg[4];
  float g[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int32_t wh = bi + (k >> 1), ww = bj + (k & 1);
    arg[k] = -1;
    g[k] = 0.0f;
    if (wh >= oh || ww >= ow) continue;
    bool found = false;
    float best = 0.0f;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      const int32_t hh = 2 * wh - 1 + a;
      if (hh < 0 || hh >= h) continue;
#pragma unroll
      for (int b = 0; b < 3; ++b) {
        const int32_t cc = 2 * ww - 1 + b;
        if (cc < 0 || cc >= w) continue;
        const float v = Io<T>::load(xp[hh * w + cc]);
        if (!found || v > best) {
          found = true;
          best = v;
          arg[k] = hh * w + cc;
        }
      }
    }
    g[k] = Io<T>::load(dyp[wh * ow + ww]);
  }
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const int32_t ih = 2 * bi + (d >> 1), iw = 2 * bj + (d & 1);
    if (ih >= h || iw >= w) continue;
    const int32_t at = ih * w + iw;
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (arg[k] == at) acc += g[k];
    if constexpr (RELU) acc = Io<T>::load(xp[at]) > 0.0f ? acc : 0.0f;
    dx[nc * h * w + at] = Io<T>::store(acc);
  }
}

// The same gradient on 2 x 8 input blocks when W % 8 == 0: the ten covering windows (oh in {i, i+1}, ow in
// 4j .. 4j+4) are evaluated from one register tile of the 5 x 11 inputs they span (16-byte loads for the middle
// eight columns), and the block is written with two 16-byte stores. RELU as maxpool3s2_grad_kernel's.
template <typename T, bool RELU>
__global__ __launch_bounds__(kThreads) void maxpool3s2_grad8_kernel(const typename Io<T>::storage* __restrict__ dy,
                                                                    const typename Io<T>::storage* __restrict__ x,
                                                                    typename Io<T>::storage* __restrict__ dx, int32_t h,
                                                                    int32_t w, int32_t oh, int32_t ow, int32_t bh,
                                                                    int32_t bw, int64_t total) {
  using S = typename Io<T>::storage;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (t >= total) return;
  const int32_t bj = static_cast<int32_t>(t % bw);
  const int64_t r0 = t / bw;
  const int32_t bi = static_cast<int32_t>(r0 % bh);
  const int64_t nc = r0 / bh;
  const S* xp = x + nc * h * w;
  const S* dyp = dy + nc * oh * ow;
  const int32_t row0 = 2 * bi - 1, col0 = 8 * bj - 1;  // local (0, 0)
  float v[5][11];
  bool rv[5], cv[11];
#pragma unroll
  for (int c = 0; c < 11; ++c) cv[c] = col0 + c >= 0 && col0 + c < w;
#pragma unroll
  for (int r = 0; r < 5; ++r) {
    const int32_t gr = row0 + r;
    rv[r] = gr >= 0 && gr < h;
#pragma unroll
    for (int c = 0; c < 11; ++c) v[r][c] = 0.0f;
    if (!rv[r]) continue;
    const S* rowp = xp + static_cast<int64_t>(gr) * w;
    const uint4 mid = *reinterpret_cast<const uint4*>(rowp + 8 * bj);
    const S* m = reinterpret_cast<const S*>(&mid);
#pragma unroll
    for (int c = 0; c < 8; ++c) v[r][c + 1] = Io<T>::load(m[c]);
    if (cv[0]) v[r][0] = Io<T>::load(rowp[col0]);
    if (cv[9]) v[r][9] = Io<T>::load(rowp[col0 + 9]);
    if (cv[10]) v[r][10] = Io<T>::load(rowp[col0 + 10]);
  }
  int arg[10];
  float g[10];
#pragma unroll
  for (int k = 0; k < 10; ++k) {
    const int wr = k / 5, wc = k % 5;
    const int32_t woh = bi + wr, wow = 4 * bj + wc;
    arg[k] = -1;
    g[k] = 0.0f;
    if (woh >= oh || wow >= ow) continue;
    bool found = false;
    float best = 0.0f;
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
      for (int b = 0; b < 3; ++b) {
        const int lr = 2 * wr + a, lc = 2 * wc + b;
        if (!rv[lr] || !cv[lc]) continue;
        const float val = v[lr][lc];
        if (!found || val > best) {
          found = true;
          best = val;
          arg[k] = lr * 11 + lc;
        }
      }
    g[k] = Io<T>::load(dyp[woh * ow + wow]);
  }
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    const int32_t gr = 2 * bi + rr;
    if (gr >= h) continue;
    uint4 packed;
    S* o = reinterpret_cast<S*>(&packed);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int at = (rr + 1) * 11 + (c + 1);
      float acc = 0.0f;
#pragma unroll
      for (int k = 0; k < 10; ++k)
        if (arg[k] == at) acc += g[k];
      if constexpr (RELU) acc = v[rr + 1][c + 1] > 0.0f ? acc : 0.0f;
      o[c] = Io<T>::store(acc);
    }
    *reinterpret_cast<uint4*>(dx + nc * h * w + static_cast<int64_t>(gr) * w + 8 * bj) = packed;
  }
}

// The same 2 x 8 block gradient with one workgroup per (n, c) plane: the whole x plane and dy plane are first
// copied into LDS with coalesced 16-byte loads (the per-thread form issues 5 x 4 loads, 15 of them 2-byte halo
// columns, and 10 dy loads per block: ~130 us for ResNet's stem pool), then every block reads its 5 x 11 tile and
// its ten dy values from LDS. Window scan, ties and the order of each input's sum are the per-thread kernel's;
// RELU as maxpool3s2_grad_kernel's (x is already in registers: the fused relu gradient reads nothing more).
template <typename T, bool RELU>
__global__ __launch_bounds__(kThreads) void maxpool3s2_grad8_plane_kernel(const typename Io<T>::storage* __restrict__ dy,
                                                                          const typename Io<T>::storage* __restrict__ x,
                                                                          typename Io<T>::storage* __restrict__ dx,
                                                                          int32_t h, int32_t w, int32_t oh, int32_t ow,
                                                                          int32_t bh, int32_t bw, int32_t dy_vec) {
  using S = typename Io<T>::storage;
  extern __shared__ __attribute__((aligned(16))) unsigned char plane_lds[];
  S* xs = reinterpret_cast<S*>(plane_lds);
  S* ds = xs + h * w;  // h * w % 8 == 0: 16-byte aligned
  const int64_t nc = blockIdx.x;
  const S* xp = x + nc * h * w;
  const S* dyp = dy + nc * oh * ow;
  for (int i = threadIdx.x; i < h * w / 8; i += kThreads)
    reinterpret_cast<uint4*>(xs)[i] = reinterpret_cast<const uint4*>(xp)[i];
  if (dy_vec) {
    for (int i = threadIdx.x; i < oh * ow / 8; i += kThreads)
      reinterpret_cast<uint4*>(ds)[i] = reinterpret_cast<const uint4*>(dyp)[i];
  } else {
    for (int i = threadIdx.x; i < oh * ow; i += kThreads) ds[i] = dyp[i];
  }
  __syncthreads();
  // Blocks whose 5 x 11 tile and ten windows all lie inside the plane take a path with no validity logic; the
  // rest (the plane's border blocks) the general one. Both are enumerated compactly, so a wave runs one path.
  const int32_t bi_hi = min((h - 4) / 2, oh - 2), bj_hi = min((w - 10) / 8, (ow - 5) / 4);
  const int32_t ni = bi_hi >= 1 ? bi_hi : 0, nj = bj_hi >= 1 ? bj_hi : 0;  // interior rows 1 .. bi_hi, cols 1 .. bj_hi
  // one block: FULL = every tile position and window valid
  auto block = [&]<bool FULL>(int32_t bi, int32_t bj) {
    const int32_t row0 = 2 * bi - 1, col0 = 8 * bj - 1;  // local (0, 0)
    float v[5][11];
    bool rv[5], cv[11];
#pragma unroll
    for (int c = 0; c < 11; ++c) cv[c] = FULL || (col0 + c >= 0 && col0 + c < w);
#pragma unroll
    for (int r = 0; r < 5; ++r) {
      const int32_t gr = row0 + r;
      rv[r] = FULL || (gr >= 0 && gr < h);
      const S* rowp = xs + (FULL ? gr : min(max(gr, 0), h - 1)) * w;
      const uint4 mid = *reinterpret_cast<const uint4*>(rowp + 8 * bj);
      const S* m = reinterpret_cast<const S*>(&mid);
#pragma unroll
      for (int c = 0; c < 8; ++c) v[r][c + 1] = Io<T>::load(m[c]);
      v[r][0] = Io<T>::load(rowp[FULL ? col0 : max(col0, 0)]);
      v[r][9] = Io<T>::load(rowp[FULL ? col0 + 9 : min(col0 + 9, w - 1)]);
      v[r][10] = Io<T>::load(rowp[FULL ? col0 + 10 : min(col0 + 10, w - 1)]);
    }
    // per window: the first valid position, then a later one only when strictly greater (the reference's scan),
    // branch-free
    int arg[10];
    float g[10];
#pragma unroll
    for (int k = 0; k < 10; ++k) {
      const int wr = k / 5, wc = k % 5;
      const int32_t woh = bi + wr, wow = 4 * bj + wc;
      const bool wvalid = FULL || (woh < oh && wow < ow);
      bool found = false;
      float best = 0.0f;
      int at = -1;
#pragma unroll
      for (int a = 0; a < 3; ++a)
#pragma unroll
        for (int b = 0; b < 3; ++b) {
          const int lr = 2 * wr + a, lc = 2 * wc + b;
          const float val = v[lr][lc];
          if constexpr (FULL) {
            const bool take = (a == 0 && b == 0) || val > best;
            best = take ? val : best;
            at = take ? lr * 11 + lc : at;
          } else {
            const bool ok = rv[lr] && cv[lc];
            const bool take = ok && (!found || val > best);
            best = take ? val : best;
            at = take ? lr * 11 + lc : at;
            found = found || ok;
          }
        }
      arg[k] = wvalid ? at : -1;
      const float gv = Io<T>::load(ds[(FULL ? woh : min(woh, oh - 1)) * ow + (FULL ? wow : min(wow, ow - 1))]);
      g[k] = wvalid ? gv : 0.0f;
    }
    // input (1 + rr, 1 + c) of the tile is covered by windows wr with 2 wr <= 1 + rr <= 2 wr + 2 and wc with
    // 2 wc <= 1 + c <= 2 wc + 2; the others cannot have chosen it. Summed in window order; adding +0.0 for a
    // window that chose another input leaves the sum unchanged (it starts at +0.0, so it is never -0.0).
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int32_t gr = 2 * bi + rr;
      if (!FULL && gr >= h) continue;
      uint4 packed;
      S* o = reinterpret_cast<S*>(&packed);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const int lr = rr + 1, lc = c + 1, at = lr * 11 + lc;
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < 10; ++k) {
          const int wr = k / 5, wc = k % 5;
          if (2 * wr <= lr && lr <= 2 * wr + 2 && 2 * wc <= lc && lc <= 2 * wc + 2) acc += arg[k] == at ? g[k] : 0.0f;
        }
        if constexpr (RELU) acc = v[lr][lc] > 0.0f ? acc : 0.0f;
        o[c] = Io<T>::store(acc);
      }
      *reinterpret_cast<uint4*>(dx + nc * h * w + static_cast<int64_t>(gr) * w + 8 * bj) = packed;
    }
  };
  for (int e = threadIdx.x; e < ni * nj; e += kThreads) block.template operator()<true>(1 + e / nj, 1 + e % nj);
  // border blocks: rows 0 and bi_hi + 1 .. bh - 1 whole, the interior rows' columns 0 and bj_hi + 1 .. bw - 1
  const int32_t top = 1 + (bh - 1 - ni);                   // whole rows: row 0 and the rows below the interior
  const int32_t side = bw - nj;                            // border columns of an interior row
  const int32_t nb = top * bw + ni * side;
  for (int e = threadIdx.x; e < nb; e += kThreads) {
    int32_t bi, bj;
    if (e < top * bw) {
      const int32_t r = e / bw;
      bi = r == 0 ? 0 : ni + r;
      bj = e % bw;
    } else {
      const int32_t f = e - top * bw, r = f / side, c = f % side;
      bi = 1 + r;
      bj = c == 0 ? 0 : nj + c;
    }
    block.template operator()<false>(bi, bj);
  }
}

// ---- conv gradients (direct, reference order) ----------------------------------------------------------------

struct ConvG {
  int32_t n, cin, h, w, cout, kh, kw, sh, sw, ph, pw, groups, oh, ow;
};

// dx[n, cf, ih, iw] = sum over co of cf's group, kh, kw (ascending) of dy * w at the taps where ih + ph - kh is a
// multiple of the stride inside dy (reference: src/backends/cpu/kernels/conv.cpp:320-352).
template <typename T>
__global__ __launch_bounds__(kThreads) void conv_grad_input_kernel(const typename Io<T>::storage* __restrict__ dy,
                                                                   const typename Io<T>::storage* __restrict__ wt,
                                                                   typename Io<T>::storage* __restrict__ dx, ConvG g,
                                                                   int64_t total) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= total) return;
  const int32_t iw = static_cast<int32_t>(i % g.w);
  const int32_t ih = static_cast<int32_t>((i / g.w) % g.h);
  const int32_t cf = static_cast<int32_t>((i / (static_cast<int64_t>(g.w) * g.h)) % g.cin);
  const int64_t n = i / (static_cast<int64_t>(g.w) * g.h * g.cin);
  const int32_t cin_g = g.cin / g.groups, cout_g = g.cout / g.groups;
  const int32_t grp = cf / cin_g, ci = cf - grp * cin_g;
  float acc = 0.0f;
  for (int32_t co = grp * cout_g; co < (grp + 1) * cout_g; ++co) {
    const auto* dyc = dy + (n * g.cout + co) * g.oh * g.ow;
    const auto* wc = wt + (static_cast<int64_t>(co) * cin_g + ci) * g.kh * g.kw;
    for (int32_t a = 0; a < g.kh; ++a) {
      const int32_t nh = ih + g.ph - a;
      if (nh < 0 || nh % g.sh != 0) continue;
      const int32_t oh = nh / g.sh;
      if (oh >= g.oh) continue;
      for (int32_t b = 0; b < g.kw; ++b) {
        const int32_t nw = iw + g.pw - b;
        if (nw < 0 || nw % g.sw != 0) continue;
        const int32_t ow = nw / g.sw;
        if (ow >= g.ow) continue;
        acc += Io<T>::load(dyc[oh * g.ow + ow]) * Io<T>::load(wc[a * g.kw + b]);
      }
    }
  }
  dx[i] = Io<T>::store(acc);
}

// dw[co, ci, kh, kw] = sum over n, oh, ow (ascending) of x * dy, padding taps skipped
// (reference: src/backends/cpu/kernels/conv.cpp:423-451).
template <typename T>
__global__ __launch_bounds__(kThreads) void conv_grad_filter_kernel(const typename Io<T>::storage* __restrict__ x,
                                                                    const typename Io<T>::storage* __restrict__ dy,
                                                                    typename Io<T>::storage* __restrict__ dw, ConvG g,
                                                                    int64_t total) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= total) return;
  const int32_t cin_g = g.cin / g.groups, cout_g = g.cout / g.groups;
  const int32_t b = static_cast<int32_t>(i % g.kw);
  const int32_t a = static_cast<int32_t>((i / g.kw) % g.kh);
  const int32_t ci = static_cast<int32_t>((i / (static_cast<int64_t>(g.kw) * g.kh)) % cin_g);
  const int32_t co = static_cast<int32_t>(i / (static_cast<int64_t>(g.kw) * g.kh * cin_g));
  const int32_t cf = (co / cout_g) * cin_g + ci;
  float acc = 0.0f;
  for (int32_t n = 0; n < g.n; ++n) {
    const auto* xc = x + (static_cast<int64_t>(n) * g.cin + cf) * g.h * g.w;
    const auto* dyc = dy + (static_cast<int64_t>(n) * g.cout + co) * g.oh * g.ow;
    for (int32_t oh = 0; oh < g.oh; ++oh) {
      const int32_t ih = oh * g.sh - g.ph + a;
      if (ih < 0 || ih >= g.h) continue;
      for (int32_t ow = 0; ow < g.ow; ++ow) {
        const int32_t iw = ow * g.sw - g.pw + b;
        if (iw < 0 || iw >= g.w) continue;
        acc += Io<T>::load(xc[ih * g.w + iw]) * Io<T>::load(dyc[oh * g.ow + ow]);
      }
    }
  }
  dw[i] = Io<T>::store(acc);
}

// ---- operands of the transposed convolution (conv2d_grad_input on the implicit-GEMM conv) -----------------------

// out[ci][a][b][co] = w[co][ci][KH-1-a][KW-1-b]: the filter of dx = conv(dy, w') in the conv kernel's channels-last
// filter layout [Cout'][KH][KW][Cin'] with Cout' = Cin, Cin' = Cout.
template <typename S>
__global__ __launch_bounds__(kThreads) void filter_flip_kernel(const S* __restrict__ w, S* __restrict__ out, int32_t cout,
                                                               int32_t cin, int32_t kh, int32_t kw, int64_t total) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= total) return;
  const int32_t co = static_cast<int32_t>(i % cout);
  int64_t r = i / cout;
  const int32_t b = static_cast<int32_t>(r % kw);
  r /= kw;
  const int32_t a = static_cast<int32_t>(r % kh);
  const int32_t ci = static_cast<int32_t>(r / kh);
  out[i] = w[((static_cast<int64_t>(co) * cin + ci) * kh + (kh - 1 - a)) * kw + (kw - 1 - b)];
}

// The same permutation through LDS: a workgroup owns 64 output channels co and kFlipCi input channels ci. Each co's
// kFlipCi * taps source elements are one contiguous run of w, and each (ci, tap) destination row holds the 64 co
// contiguously, so the global writes are coalesced and neighbouring workgroups read neighbouring runs (the gather
// form above reads with a stride of cin * taps elements). One ci per workgroup: a 64x64x3x3 filter still spreads
// over 64 workgroups (with eight, its eight workgroups took longer than the gather form).
constexpr int kFlipCo = 64, kFlipCi = 1;
// Workgroup (bx, by) of one filter's flip: output channels [64 bx, 64 bx + 64), input channels
// [ci_per by, ci_per by + ci_per); the tile takes kFlipCo * (ci_per * taps + 1) elements of LDS. TAPS and CIP > 0:
// a whole tile (64 output and CIP input channels) of a TAPS-tap filter, whose index divisions become constant
// ones (the runtime divisions made the kernel bound by integer instructions).
template <typename S, int TAPS = 0, int CIP = 0>
__device__ __forceinline__ void filter_flip_tile(const S* __restrict__ w, S* __restrict__ out, int32_t cout, int32_t cin,
                                                 int32_t taps_rt, int32_t ci_per_rt, int32_t bx, int32_t by, S* tile) {
  constexpr bool FIXED = TAPS > 0 && CIP > 0;
  const int32_t taps = FIXED ? TAPS : taps_rt, ci_per = FIXED ? CIP : ci_per_rt;
  const int32_t co0 = bx * kFlipCo, ci0 = by * ci_per;
  const int32_t nco = FIXED ? kFlipCo : min(kFlipCo, cout - co0), nci = FIXED ? CIP : min(ci_per, cin - ci0);
  const int32_t run = nci * taps, pitch = ci_per * taps + 1;
  const S* src = w + static_cast<int64_t>(co0) * cin * taps + static_cast<int64_t>(ci0) * taps;
  for (int32_t e = threadIdx.x; e < nco * run; e += kThreads) {
    const int32_t c = e / run, j = e - c * run;
    tile[c * pitch + j] = src[static_cast<int64_t>(c) * cin * taps + j];
  }
  __syncthreads();
  // out[(ci * taps + t) * cout + co] = w[co][ci][taps - 1 - t] (the (a, b) flip is the tap reversal)
  for (int32_t e = threadIdx.x; e < run * nco; e += kThreads) {
    const int32_t q = e / nco, c = e - q * nco;
    const int32_t cl = q / taps, t = q - cl * taps;
    out[(static_cast<int64_t>(ci0 + cl) * taps + t) * cout + co0 + c] = tile[c * pitch + cl * taps + (taps - 1 - t)];
  }
}

template <typename S>
__global__ __launch_bounds__(kThreads) void filter_flip_tiled_kernel(const S* __restrict__ w, S* __restrict__ out,
                                                                     int32_t cout, int32_t cin, int32_t taps) {
  extern __shared__ uint32_t flip_smem[];
  filter_flip_tile<S>(w, out, cout, cin, taps, kFlipCi, static_cast<int32_t>(blockIdx.x),
                      static_cast<int32_t>(blockIdx.y), reinterpret_cast<S*>(flip_smem));
}

// Several filters' flips in one launch (a training graph's filters are all known before its first input gradient,
// and each flip alone is too small to be more than launch and memory latency): workgroup g belongs to filter i with
// first_block[i] <= g < first_block[i + 1] and runs that filter's workgroup (g - first_block[i]) of the tiled
// flip, over ci_per input channels (one launch has workgroups enough for larger tiles than a single small
// filter's: the reads become runs of ci_per * taps elements); each output is the same permutation, bit for bit.
struct FlipBatch {
  const void* w[FH_FLIP_MAX];
  void* out[FH_FLIP_MAX];
  int32_t cout[FH_FLIP_MAX], cin[FH_FLIP_MAX], taps[FH_FLIP_MAX];
  int32_t first_block[FH_FLIP_MAX + 1];
  int32_t count, ci_per;
};

template <typename S>
__global__ __launch_bounds__(kThreads) void filter_flip_multi_kernel(FlipBatch a) {
  extern __shared__ uint32_t flip_smem[];
  const int32_t g = static_cast<int32_t>(blockIdx.x);
  int i = 0;
  while (i + 1 < a.count && a.first_block[i + 1] <= g) ++i;
  const int32_t local = g - a.first_block[i];
  const int32_t tiles_co = (a.cout[i] + kFlipCo - 1) / kFlipCo;
  const int32_t by = local / tiles_co, bx = local - by * tiles_co;
  const S* w = static_cast<const S*>(a.w[i]);
  S* out = static_cast<S*>(a.out[i]);
  S* tile = reinterpret_cast<S*>(flip_smem);
  const bool whole = (bx + 1) * kFlipCo <= a.cout[i] && (by + 1) * a.ci_per <= a.cin[i] && a.ci_per == 8;
  if (whole && a.taps[i] == 9)
    filter_flip_tile<S, 9, 8>(w, out, a.cout[i], a.cin[i], 9, 8, bx, by, tile);
  else if (whole && a.taps[i] == 1)
    filter_flip_tile<S, 1, 8>(w, out, a.cout[i], a.cin[i], 1, 8, bx, by, tile);
  else
    filter_flip_tile<S>(w, out, a.cout[i], a.cin[i], a.taps[i], a.ci_per, bx, by, tile);
}

// out_i = x_i + round(s_i * y_i) for up to FH_AXPY_MAX tensors: workgroups are dealt to the tensors by
// first_block (a prefix over each tensor's workgroup count), each workgroup covers kAxpyVecs 16-byte vectors per
// thread. The product is rounded to the storage type before the add, as the separate mul node stores it.
constexpr int kAxpyVecs = 4;
struct AxpyBatch {
  const void* x[FH_AXPY_MAX];
  const void* y[FH_AXPY_MAX];
  void* out[FH_AXPY_MAX];
  int64_t n[FH_AXPY_MAX];
  float s[FH_AXPY_MAX];
  int32_t first_block[FH_AXPY_MAX + 1];
  int32_t count;
  uint32_t aligned;  // bit i: tensor i's three pointers are 16-byte aligned
};

template <typename T>
__device__ __forceinline__ typename Io<T>::storage axpy_one(typename Io<T>::storage x, typename Io<T>::storage y, float s) {
  const float step = Io<T>::load(Io<T>::store(s * Io<T>::load(y)));
  return Io<T>::store(Io<T>::load(x) + step);
}

template <typename T>
__global__ __launch_bounds__(kThreads) void axpy_multi_kernel(const AxpyBatch b) {
  using S = typename Io<T>::storage;
  constexpr int V = 16 / sizeof(S);
  const int32_t blk = static_cast<int32_t>(blockIdx.x);
  int32_t t = 0;
  while (t + 1 < b.count && b.first_block[t + 1] <= blk) ++t;
  const S* x = static_cast<const S*>(b.x[t]);
  const S* y = static_cast<const S*>(b.y[t]);
  S* out = static_cast<S*>(b.out[t]);
  const int64_t n = b.n[t];
  const float s = b.s[t];
  const bool vec = (b.aligned >> t) & 1u;
  const int64_t v0 = static_cast<int64_t>(blk - b.first_block[t]) * kThreads * kAxpyVecs + threadIdx.x;
#pragma unroll
  for (int u = 0; u < kAxpyVecs; ++u) {
    const int64_t e0 = (v0 + static_cast<int64_t>(u) * kThreads) * V;
    if (e0 >= n) break;
    if (vec && e0 + V <= n) {
      const uint4 xq = *reinterpret_cast<const uint4*>(x + e0), yq = *reinterpret_cast<const uint4*>(y + e0);
      S xs[V], ys[V], os[V];
      __builtin_memcpy(xs, &xq, 16);
      __builtin_memcpy(ys, &yq, 16);
#pragma unroll
      for (int e = 0; e < V; ++e) os[e] = axpy_one<T>(xs[e], ys[e], s);
      uint4 oq;
      __builtin_memcpy(&oq, os, 16);
      *reinterpret_cast<uint4*>(out + e0) = oq;
    } else {
      const int64_t end = min(e0 + V, n);
      for (int64_t e = e0; e < end; ++e) out[e] = axpy_one<T>(x[e], y[e], s);
    }
  }
}

// channels-last x [N,H,W,C] -> [N,Hu,Wu,C], the same placement, 16-byte vectors of channels (C % 8 == 0).
template <typename S>
__global__ __launch_bounds__(kThreads) void dilate_nhwc_vec_kernel(const S* __restrict__ x, S* __restrict__ out, int32_t c,
                                                                   int32_t h, int32_t w, int32_t sh, int32_t sw,
                                                                   int32_t hu, int32_t wu, int64_t total) {
  constexpr int V = 16 / sizeof(S);
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;  // vector index
  if (i >= total) return;
  const int32_t cv = c / V;
  const int32_t ch = static_cast<int32_t>(i % cv) * V;
  int64_t r = i / cv;
  const int32_t xw = static_cast<int32_t>(r % wu);
  r /= wu;
  const int32_t yh = static_cast<int32_t>(r % hu);
  const int64_t n = r / hu;
  uint4 v{0, 0, 0, 0};
  if (yh % sh == 0 && xw % sw == 0 && yh / sh < h && xw / sw < w)
    v = *reinterpret_cast<const uint4*>(x + ((n * h + yh / sh) * w + xw / sw) * c + ch);
  *reinterpret_cast<uint4*>(out + ((n * hu + yh) * wu + xw) * c + ch) = v;
}

// avg_pool2d_grad_internal on channels-last dy [N,Ho,Wo,C] -> dx [N,H,W,C]: per input element the covering windows
// in the reference's (kh, kw) order, sum of dy, then / (KH*KW), for a 16-byte vector of channels per lane.
template <typename T>
__global__ __launch_bounds__(kThreads) void avgpool_grad_nhwc_kernel(const typename Io<T>::storage* __restrict__ dy,
                                                                     typename Io<T>::storage* __restrict__ dx, PoolG g,
                                                                     int64_t total) {
  using S = typename Io<T>::storage;
  constexpr int V = 16 / sizeof(S);
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= total) return;
  const int32_t cv = g.c / V;
  const int32_t ch = static_cast<int32_t>(i % cv) * V;
  int64_t r = i / cv;
  const int32_t iw = static_cast<int32_t>(r % g.w);
  r /= g.w;
  const int32_t ih = static_cast<int32_t>(r % g.h);
  const int64_t n = r / g.h;
  float acc[V];
#pragma unroll
  for (int k = 0; k < V; ++k) acc[k] = 0.0f;
  for (int32_t a = 0; a < g.kh; ++a) {
    const int32_t nh = ih + g.ph - a;
    if (nh < 0 || nh % g.sh != 0) continue;
    const int32_t oh = nh / g.sh;
    if (oh >= g.oh) continue;
    for (int32_t b = 0; b < g.kw; ++b) {
      const int32_t nw = iw + g.pw - b;
      if (nw < 0 || nw % g.sw != 0) continue;
      const int32_t ow = nw / g.sw;
      if (ow >= g.ow) continue;
      const uint4 v = *reinterpret_cast<const uint4*>(dy + ((n * g.oh + oh) * g.ow + ow) * g.c + ch);
      const S* e = reinterpret_cast<const S*>(&v);
#pragma unroll
      for (int k = 0; k < V; ++k) acc[k] += Io<T>::load(e[k]);
    }
  }
  const float denom = static_cast<float>(g.kh * g.kw);
  uint4 o;
  S* oe = reinterpret_cast<S*>(&o);
#pragma unroll
  for (int k = 0; k < V; ++k) oe[k] = Io<T>::store(acc[k] / denom);
  *reinterpret_cast<uint4*>(dx + ((n * g.h + ih) * g.w + iw) * g.c + ch) = o;
}

// NCHW x [N,C,H,W] -> channels-last [N,Hu,Wu,C] with x[n][c][h][w] at (h*sh, w*sw) and zeros elsewhere.
template <typename S>
__global__ __launch_bounds__(kThreads) void dilate_nhwc_kernel(const S* __restrict__ x, S* __restrict__ out, int32_t c,
                                                               int32_t h, int32_t w, int32_t sh, int32_t sw, int32_t hu,
                                                               int32_t wu, int64_t total) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= total) return;
  const int32_t ch = static_cast<int32_t>(i % c);
  int64_t r = i / c;
  const int32_t xw = static_cast<int32_t>(r % wu);
  r /= wu;
  const int32_t yh = static_cast<int32_t>(r % hu);
  const int64_t n = r / hu;
  S v{};
  if (yh % sh == 0 && xw % sw == 0 && yh / sh < h && xw / sw < w)
    v = x[((n * c + ch) * h + yh / sh) * w + xw / sw];
  out[i] = v;
}

// ---- sum / sum_grad_internal -------------------------------------------------------------------------------

constexpr int kMaxDims = 8;

// x's dims split into kept (output) and reduced groups, adjacent dims of the same kind merged. Offsets in x are
// base(kept coordinates) + roff(reduced coordinates).
struct ReduceG {
  int32_t nk, nr;
  int64_t kdim[kMaxDims], kstride[kMaxDims];
  int64_t rdim[kMaxDims], rstride[kMaxDims];
  int64_t nout, nred;
};

__device__ inline int64_t decompose(int64_t idx, int32_t nd, const int64_t* dim, const int64_t* stride) {
  int64_t off = 0;
  for (int32_t d = nd - 1; d >= 0; --d) {
    const int64_t c = idx % dim[d];
    idx /= dim[d];
    off += c * stride[d];
  }
  return off;
}

constexpr int kSumThreads = 1024;

// One workgroup per output: fp32 partial sums strided over the reduced elements, then a fixed-shape tree. The
// reduced set is walked as (outer reduced coordinates) x (innermost reduced run): when that run is contiguous in x
// (the bias gradient's H*W planes, a row sum) each lane reads 16-byte vectors of it, and the outer coordinates are
// decoded once per run instead of once per element.
template <typename T>
__global__ __launch_bounds__(kSumThreads) void sum_kernel(const typename Io<T>::storage* __restrict__ x,
                                                          typename Io<T>::storage* __restrict__ out, ReduceG g) {
  using S = typename Io<T>::storage;
  constexpr int V = 16 / sizeof(S);
  __shared__ float part[kSumThreads / 64];
  const int64_t o = blockIdx.x;
  const int64_t base = decompose(o, g.nk, g.kdim, g.kstride);
  float acc = 0.0f;
  const bool inner_run = g.nr >= 1 && g.rstride[g.nr - 1] == 1;
  if (inner_run) {
    const int64_t len = g.rdim[g.nr - 1];
    const int64_t outer = len > 0 ? g.nred / len : 0;
    const bool vec = len % V == 0 && (reinterpret_cast<uintptr_t>(x) % 16) == 0 && (base % V) == 0 &&
                     (g.nr == 1 || g.rstride[g.nr - 2] % V == 0);
    if (vec && g.nr <= 2) {
      // flat index over (outer coordinate, vector within the run); four independent 16-byte loads in flight per
      // lane before they are accumulated (in index order)
      const int64_t per_row = len / V, total = outer * per_row;
      const int64_t ostride = g.nr == 2 ? g.rstride[0] : 0;
      auto at = [&](int64_t f) {
        const int64_t q = f / per_row;
        return reinterpret_cast<const uint4*>(x + base + q * ostride + (f - q * per_row) * V);
      };
      int64_t f = threadIdx.x;
      for (; f + 3 * kSumThreads < total; f += 4 * kSumThreads) {
        uint4 w[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) w[u] = *at(f + u * kSumThreads);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const S* e = reinterpret_cast<const S*>(&w[u]);
#pragma unroll
          for (int k = 0; k < V; ++k) acc += Io<T>::load(e[k]);
        }
      }
      for (; f < total; f += kSumThreads) {
        const uint4 w = *at(f);
        const S* e = reinterpret_cast<const S*>(&w);
#pragma unroll
        for (int k = 0; k < V; ++k) acc += Io<T>::load(e[k]);
      }
    } else {
      for (int64_t q = 0; q < outer; ++q) {
        const int64_t off = base + (g.nr > 1 ? decompose(q, g.nr - 1, g.rdim, g.rstride) : 0);
        for (int64_t r = threadIdx.x; r < len; r += kSumThreads) acc += Io<T>::load(x[off + r]);
      }
    }
  } else if (g.nr == 1) {
    for (int64_t r = threadIdx.x; r < g.nred; r += kSumThreads) acc += Io<T>::load(x[base + r * g.rstride[0]]);
  } else {
    for (int64_t r = threadIdx.x; r < g.nred; r += kSumThreads)
      acc += Io<T>::load(x[base + decompose(r, g.nr, g.rdim, g.rstride)]);
  }
  for (int m = 32; m >= 1; m >>= 1) acc += __shfl_xor(acc, m);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = 0.0f;
    for (int k = 0; k < kSumThreads / 64; ++k) s += part[k];
    out[o] = Io<T>::store(s);
  }
}

// Column sums of a dense [rows, cols] tensor (cols * itemsize % 16 == 0): the bias gradient of channels-last data.
// Stage 1: workgroup w sums rows [w*R, (w+1)*R) for every column, lanes holding 16-byte column vectors and striding
// over rows, then a fixed LDS tree over the lanes that share a column vector; fp32 partials to part[w][cols].
// Stage 2: out[c] = round(sum over w in order of part[w][c]).
template <typename T>
__global__ __launch_bounds__(kThreads) void sum_rows_partial_kernel(const typename Io<T>::storage* __restrict__ x,
                                                                    float* __restrict__ part, int64_t rows, int32_t cols,
                                                                    int64_t rows_per_wg) {
  using S = typename Io<T>::storage;
  constexpr int V = 16 / sizeof(S);
  __shared__ float red[kThreads * V];
  const int32_t cv = cols / V;                       // column vectors
  const int32_t lanes_per_row = min(cv, kThreads);   // threads covering one row
  const int32_t row_step = kThreads / lanes_per_row;  // rows in flight per iteration
  const int32_t t = threadIdx.x;
  const int32_t rsub = t / lanes_per_row, vcol = t % lanes_per_row;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * rows_per_wg, r1 = min(rows, r0 + rows_per_wg);
  // the same trip count for every thread (the loop holds barriers)
  for (int32_t base = 0; base < cv; base += lanes_per_row) {
    const int32_t vc = base + vcol;
    const bool col_ok = vc < cv;
    float acc[V];
#pragma unroll
    for (int k = 0; k < V; ++k) acc[k] = 0.0f;
    if (rsub < row_step && col_ok) {
      // rows r, r + row_step, ... added in order; the loads of 8 of them are issued before their sums, so one
      // memory latency covers 8 rows instead of one
      constexpr int U = 8;
      const S* xc = x + static_cast<int64_t>(vc) * V;
      int64_t r = r0 + rsub;
      for (; r + (U - 1) * row_step < r1; r += U * row_step) {
        uint4 w[U];
#pragma unroll
        for (int u = 0; u < U; ++u) w[u] = *reinterpret_cast<const uint4*>(xc + (r + u * row_step) * cols);
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const S* e = reinterpret_cast<const S*>(&w[u]);
#pragma unroll
          for (int k = 0; k < V; ++k) acc[k] += Io<T>::load(e[k]);
        }
      }
      for (; r < r1; r += row_step) {
        const uint4 w = *reinterpret_cast<const uint4*>(xc + r * cols);
        const S* e = reinterpret_cast<const S*>(&w);
#pragma unroll
        for (int k = 0; k < V; ++k) acc[k] += Io<T>::load(e[k]);
      }
    }
#pragma unroll
    for (int k = 0; k < V; ++k) red[t * V + k] = acc[k];
    __syncthreads();
    if (rsub == 0 && col_ok) {
      // lanes rsub = 0 .. row_step-1 with this vcol, added in rsub order
      for (int k = 0; k < V; ++k) {
        float s = 0.0f;
        for (int32_t q = 0; q < row_step; ++q) s += red[(q * lanes_per_row + vcol) * V + k];
        part[static_cast<int64_t>(blockIdx.x) * cols + static_cast<int64_t>(vc) * V + k] = s;
      }
    }
    __syncthreads();
  }
}

// One wave per column: lane l adds partials l, l+64, ... in order, then a fixed xor-shuffle tree.
template <typename T>
__global__ __launch_bounds__(kThreads) void sum_rows_final_kernel(const float* __restrict__ part,
                                                                  typename Io<T>::storage* __restrict__ out, int32_t wgs,
                                                                  int32_t cols) {
  const int32_t c = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  const int32_t lane = threadIdx.x & 63;
  if (c >= cols) return;
  float s = 0.0f;
  for (int32_t w = lane; w < wgs; w += 64) s += part[static_cast<int64_t>(w) * cols + c];
  for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m);
  if (lane == 0) out[c] = Io<T>::store(s);
}

// gx[i] = gy[projection of i]: a copy of the storage bits.
template <typename S>
__global__ __launch_bounds__(kThreads) void sum_grad_kernel(const S* __restrict__ gy, S* __restrict__ gx, ReduceG g,
                                                            int64_t total) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= total) return;
  // kdim holds every dim of x and kstride the matching stride in gy (0 for a reduced dim)
  gx[i] = gy[decompose(i, g.nk, g.kdim, g.kstride)];
}

// ---- mse_loss ----------------------------------------------------------------------------------------------

constexpr int kLossThreads = 1024;

template <typename T>
__global__ __launch_bounds__(kLossThreads) void mse_loss_kernel(const typename Io<T>::storage* __restrict__ p,
                                                                const typename Io<T>::storage* __restrict__ t,
                                                                typename Io<T>::storage* __restrict__ out, int64_t n) {
  __shared__ float part[kLossThreads / 64];
  float acc = 0.0f;
  // each thread sums elements threadIdx.x, + kLossThreads, ... in order; the loads of 16 of them are issued before
  // their sum, so one memory latency covers 16 elements instead of one
  constexpr int U = 16;
  int64_t i = threadIdx.x;
  for (; i + (U - 1) * kLossThreads < n; i += U * kLossThreads) {
    float d[U];
#pragma unroll
    for (int u = 0; u < U; ++u) d[u] = Io<T>::load(p[i + u * kLossThreads]) - Io<T>::load(t[i + u * kLossThreads]);
#pragma unroll
    for (int u = 0; u < U; ++u) acc += d[u] * d[u];
  }
  for (; i < n; i += kLossThreads) {
    const float d = Io<T>::load(p[i]) - Io<T>::load(t[i]);
    acc += d * d;
  }
  for (int m = 32; m >= 1; m >>= 1) acc += __shfl_xor(acc, m);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = 0.0f;
    for (int k = 0; k < kLossThreads / 64; ++k) s += part[k];
    out[0] = Io<T>::store(s / static_cast<float>(n));
  }
}

// gpred = (2 * gy / numel) * (pred - target), the reference's operations in its order
// (reference: src/backends/cpu/kernels/loss.cpp:230-262).
template <typename T>
__global__ __launch_bounds__(kThreads) void mse_loss_grad_kernel(const typename Io<T>::storage* __restrict__ p,
                                                                 const typename Io<T>::storage* __restrict__ t,
                                                                 const typename Io<T>::storage* __restrict__ gy,
                                                                 typename Io<T>::storage* __restrict__ out, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n) return;
  const float c = 2.0f * Io<T>::load(gy[0]) / static_cast<float>(n);
  out[i] = Io<T>::store(c * (Io<T>::load(p[i]) - Io<T>::load(t[i])));
}

// ---- host side ---------------------------------------------------------------------------------------------

template <template <typename> class K, typename... A>
fh_status dispatch(int32_t dtype, A&&... args) {
  switch (dtype) {
    case FH_F32:
      return K<float>::run(args...);
    case FH_BF16:
      return K<bf16_t>::run(args...);
    default:
      return K<f16_t>::run(args...);
  }
}

bool grid_ok(int64_t blocks) { return blocks <= 0x7fffffffLL; }

template <typename T>
struct PoolGradRun {
  static fh_status run(int32_t mode, const void* dy, const void* x, void* dx, const PoolG& g, int64_t total,
                       hipStream_t s) {
    using S = typename Io<T>::storage;
    const dim3 grid(static_cast<uint32_t>(blocks_for(total)));
    const bool aligned = reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(dx) % 16 == 0;
    const bool relu = mode == 2;
    if (mode != 1 && g.kh == 3 && g.kw == 3 && g.sh == 2 && g.sw == 2 && g.ph == 1 && g.pw == 1 && g.w % 8 == 0 &&
        (sizeof(S) == 2) && aligned) {
      const int32_t bh = (g.h + 1) / 2, bw = g.w / 8;
      const int64_t planes = static_cast<int64_t>(g.n) * g.c;
      const int64_t plane_bytes = (static_cast<int64_t>(g.h) * g.w + static_cast<int64_t>(g.oh) * g.ow) * 2;
      if (plane_bytes <= 64 * 1024 && planes <= 0x7fffffffLL) {
        const int32_t dy_vec = (static_cast<int64_t>(g.oh) * g.ow) % 8 == 0 && reinterpret_cast<uintptr_t>(dy) % 16 == 0;
        auto go = [&]<bool R>() {
          hipLaunchKernelGGL((maxpool3s2_grad8_plane_kernel<T, R>), dim3(static_cast<uint32_t>(planes)), dim3(kThreads),
                             static_cast<uint32_t>(plane_bytes), s, static_cast<const S*>(dy), static_cast<const S*>(x),
                             static_cast<S*>(dx), g.h, g.w, g.oh, g.ow, bh, bw, dy_vec);
        };
        relu ? go.template operator()<true>() : go.template operator()<false>();
      } else {
        const int64_t blocks = planes * bh * bw;
        auto go = [&]<bool R>() {
          hipLaunchKernelGGL((maxpool3s2_grad8_kernel<T, R>), dim3(static_cast<uint32_t>(blocks_for(blocks))),
                             dim3(kThreads), 0, s, static_cast<const S*>(dy), static_cast<const S*>(x), static_cast<S*>(dx),
                             g.h, g.w, g.oh, g.ow, bh, bw, blocks);
        };
        relu ? go.template operator()<true>() : go.template operator()<false>();
      }
    } else if (mode != 1 && g.kh == 3 && g.kw == 3 && g.sh == 2 && g.sw == 2 && g.ph == 1 && g.pw == 1) {
      const int32_t bh = (g.h + 1) / 2, bw = (g.w + 1) / 2;
      const int64_t blocks = static_cast<int64_t>(g.n) * g.c * bh * bw;
      auto go = [&]<bool R>() {
        hipLaunchKernelGGL((maxpool3s2_grad_kernel<T, R>), dim3(static_cast<uint32_t>(blocks_for(blocks))), dim3(kThreads),
                           0, s, static_cast<const S*>(dy), static_cast<const S*>(x), static_cast<S*>(dx), g.h, g.w, g.oh,
                           g.ow, bh, bw, blocks);
      };
      relu ? go.template operator()<true>() : go.template operator()<false>();
    } else if (mode == 0)
      hipLaunchKernelGGL((pool2d_grad_kernel<T, 0>), grid, dim3(kThreads), 0, s, static_cast<const S*>(dy),
                         static_cast<const S*>(x), static_cast<S*>(dx), g, total);
    else if (mode == 2)
      hipLaunchKernelGGL((pool2d_grad_kernel<T, 2>), grid, dim3(kThreads), 0, s, static_cast<const S*>(dy),
                         static_cast<const S*>(x), static_cast<S*>(dx), g, total);
    else
      hipLaunchKernelGGL((pool2d_grad_kernel<T, 1>), grid, dim3(kThreads), 0, s, static_cast<const S*>(dy),
                         static_cast<const S*>(x), static_cast<S*>(dx), g, total);
    return launch_status("fh_pool2d_grad");
  }
};

template <typename T>
struct ConvGradRun {
  static fh_status run(int filter, const void* p, const void* q, void* out, const ConvG& g, int64_t total, hipStream_t s) {
    using S = typename Io<T>::storage;
    const dim3 grid(static_cast<uint32_t>(blocks_for(total)));
    if (filter)
      hipLaunchKernelGGL((conv_grad_filter_kernel<T>), grid, dim3(kThreads), 0, s, static_cast<const S*>(p),
                         static_cast<const S*>(q), static_cast<S*>(out), g, total);
    else
      hipLaunchKernelGGL((conv_grad_input_kernel<T>), grid, dim3(kThreads), 0, s, static_cast<const S*>(p),
                         static_cast<const S*>(q), static_cast<S*>(out), g, total);
    return launch_status(filter ? "fh_conv2d_grad_filter" : "fh_conv2d_grad_input");
  }
};

template <typename T>
struct SumRun {
  static fh_status run(const void* x, void* out, const ReduceG& g, hipStream_t s) {
    using S = typename Io<T>::storage;
    hipLaunchKernelGGL((sum_kernel<T>), dim3(static_cast<uint32_t>(g.nout)), dim3(kSumThreads), 0, s,
                       static_cast<const S*>(x), static_cast<S*>(out), g);
    return launch_status("fh_sum");
  }
};

template <typename T>
struct MseRun {
  static fh_status run(int grad, const void* p, const void* t, const void* gy, void* out, int64_t n, hipStream_t s) {
    using S = typename Io<T>::storage;
    if (grad)
      hipLaunchKernelGGL((mse_loss_grad_kernel<T>), dim3(static_cast<uint32_t>(blocks_for(n))), dim3(kThreads), 0, s,
                         static_cast<const S*>(p), static_cast<const S*>(t), static_cast<const S*>(gy), static_cast<S*>(out),
                         n);
    else
      hipLaunchKernelGGL((mse_loss_kernel<T>), dim3(1), dim3(kLossThreads), 0, s, static_cast<const S*>(p),
                         static_cast<const S*>(t), static_cast<S*>(out), n);
    return launch_status(grad ? "fh_mse_loss_grad" : "fh_mse_loss");
  }
};

fh_status conv_geom(const char* who, int32_t dtype, const int64_t* geom, ConvG& g) {
  const std::string w(who);
  if (!is_supported_float(dtype)) return fail(FH_UNIMPLEMENTED, w + ": unsupported dtype");
  if (geom == nullptr) return fail(FH_INVALID_ARGUMENT, w + ": null geometry");
  for (int k = 0; k < 12; ++k)
    if (geom[k] < 0 || geom[k] > 0x7fffffffLL) return fail(FH_INVALID_ARGUMENT, w + ": geometry entry out of range");
  g = ConvG{static_cast<int32_t>(geom[0]), static_cast<int32_t>(geom[1]), static_cast<int32_t>(geom[2]),
            static_cast<int32_t>(geom[3]), static_cast<int32_t>(geom[4]), static_cast<int32_t>(geom[5]),
            static_cast<int32_t>(geom[6]), static_cast<int32_t>(geom[7]), static_cast<int32_t>(geom[8]),
            static_cast<int32_t>(geom[9]), static_cast<int32_t>(geom[10]), static_cast<int32_t>(geom[11]), 0, 0};
  if (g.kh <= 0 || g.kw <= 0 || g.sh <= 0 || g.sw <= 0 || g.groups <= 0 || g.cin % g.groups != 0 ||
      g.cout % g.groups != 0)
    return fail(FH_INVALID_ARGUMENT, w + ": invalid geometry");
  const int64_t oh = (static_cast<int64_t>(g.h) + 2 * g.ph - g.kh), ow = (static_cast<int64_t>(g.w) + 2 * g.pw - g.kw);
  if (oh < 0 || ow < 0) return fail(FH_INVALID_ARGUMENT, w + ": filter larger than the padded input");
  g.oh = static_cast<int32_t>(oh / g.sh + 1);
  g.ow = static_cast<int32_t>(ow / g.sw + 1);
  return FH_OK;
}

// Splits x's dims into merged kept / reduced groups (row-major strides).
void build_reduce(int32_t rank, const int64_t* dims, const uint8_t* reduced, ReduceG& g) {
  g = ReduceG{};
  int64_t stride = 1;
  int64_t kd[kMaxDims], ks[kMaxDims], rd[kMaxDims], rs[kMaxDims];
  int nk = 0, nr = 0;
  int last = -1;  // kind of the previous (inner) dim: 0 kept, 1 reduced
  for (int32_t d = rank - 1; d >= 0; --d) {
    const int kind = reduced[d] ? 1 : 0;
    if (dims[d] == 1) {  // size-1 dims contribute nothing
      continue;
    }
    if (kind == last) {  // merge with the adjacent inner dim of the same kind (contiguous in row-major order)
      if (kind) rd[nr - 1] *= dims[d];
      else kd[nk - 1] *= dims[d];
    } else if (kind) {
      rd[nr] = dims[d];
      rs[nr] = stride;
      ++nr;
    } else {
      kd[nk] = dims[d];
      ks[nk] = stride;
      ++nk;
    }
    last = kind;
    stride *= dims[d];
  }
  // stored outermost first
  g.nk = nk;
  g.nr = nr;
  g.nout = 1;
  g.nred = 1;
  for (int k = 0; k < nk; ++k) {
    g.kdim[k] = kd[nk - 1 - k];
    g.kstride[k] = ks[nk - 1 - k];
    g.nout *= g.kdim[k];
  }
  for (int k = 0; k < nr; ++k) {
    g.rdim[k] = rd[nr - 1 - k];
    g.rstride[k] = rs[nr - 1 - k];
    g.nred *= g.rdim[k];
  }
}

fh_status check_reduce(const char* who, int32_t rank, const int64_t* dims, const uint8_t* reduced) {
  const std::string w(who);
  if (rank < 0 || rank > kMaxDims) return fail(FH_UNIMPLEMENTED, w + ": rank above 8");
  if (rank > 0 && (dims == nullptr || reduced == nullptr)) return fail(FH_INVALID_ARGUMENT, w + ": null dims");
  for (int32_t d = 0; d < rank; ++d)
    if (dims[d] < 0) return fail(FH_INVALID_ARGUMENT, w + ": negative dimension");
  return FH_OK;
}

}  // namespace
}  // namespace fh

using namespace fh;

extern "C" fh_status fh_pool2d_grad(int32_t dtype, int32_t mode, const void* dy, const void* x, void* dx,
                                    const int64_t geom[10], void* stream) {
  if (!is_supported_float(dtype)) return fail(FH_UNIMPLEMENTED, "fh_pool2d_grad: unsupported dtype");
  if (mode < 0 || mode > 2)
    return fail(FH_INVALID_ARGUMENT, "fh_pool2d_grad: mode must be 0 (max), 1 (avg) or 2 (max, then relu_grad by x)");
  if (geom == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_pool2d_grad: null geometry");
  for (int k = 0; k < 10; ++k)
    if (geom[k] < 0 || geom[k] > 0x7fffffffLL) return fail(FH_INVALID_ARGUMENT, "fh_pool2d_grad: geometry entry out of range");
  PoolG g{static_cast<int32_t>(geom[0]), static_cast<int32_t>(geom[1]), static_cast<int32_t>(geom[2]),
          static_cast<int32_t>(geom[3]), static_cast<int32_t>(geom[4]), static_cast<int32_t>(geom[5]),
          static_cast<int32_t>(geom[6]), static_cast<int32_t>(geom[7]), static_cast<int32_t>(geom[8]),
          static_cast<int32_t>(geom[9]), 0, 0};
  if (g.kh <= 0 || g.kw <= 0 || g.sh <= 0 || g.sw <= 0 || g.h + 2 * g.ph < g.kh || g.w + 2 * g.pw < g.kw)
    return fail(FH_INVALID_ARGUMENT, "fh_pool2d_grad: invalid geometry");
  g.oh = (g.h + 2 * g.ph - g.kh) / g.sh + 1;
  g.ow = (g.w + 2 * g.pw - g.kw) / g.sw + 1;
  if (mode != 1 && (g.ph >= g.kh || g.pw >= g.kw || (g.oh - 1) * g.sh - g.ph >= g.h || (g.ow - 1) * g.sw - g.pw >= g.w))
    return fail(FH_INVALID_ARGUMENT, "fh_pool2d_grad: a max-pool window has no valid (non-padding) position");
  const int64_t total = static_cast<int64_t>(g.n) * g.c * g.h * g.w;
  if (total == 0) return FH_OK;
  if (dy == nullptr || dx == nullptr || (mode != 1 && x == nullptr))
    return fail(FH_INVALID_ARGUMENT, "fh_pool2d_grad: null pointer");
  if (!grid_ok(blocks_for(total))) return fail(FH_INVALID_ARGUMENT, "fh_pool2d_grad: tensor too large");
  return dispatch<PoolGradRun>(dtype, mode, dy, x, dx, g, total, static_cast<hipStream_t>(stream));
}

extern "C" fh_status fh_conv2d_grad_input(int32_t dtype, const void* dy, const void* w, void* dx,
                                          const int64_t geom[12], void* stream) {
  ConvG g{};
  if (fh_status st = conv_geom("fh_conv2d_grad_input", dtype, geom, g); st != FH_OK) return st;
  const int64_t total = static_cast<int64_t>(g.n) * g.cin * g.h * g.w;
  if (total == 0) return FH_OK;
  if (dy == nullptr || w == nullptr || dx == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_conv2d_grad_input: null pointer");
  if (!grid_ok(blocks_for(total))) return fail(FH_INVALID_ARGUMENT, "fh_conv2d_grad_input: tensor too large");
  return dispatch<ConvGradRun>(dtype, 0, dy, w, dx, g, total, static_cast<hipStream_t>(stream));
}

extern "C" fh_status fh_conv2d_grad_filter(int32_t dtype, const void* x, const void* dy, void* dw,
                                           const int64_t geom[12], void* stream) {
  ConvG g{};
  if (fh_status st = conv_geom("fh_conv2d_grad_filter", dtype, geom, g); st != FH_OK) return st;
  const int64_t total = static_cast<int64_t>(g.cout) * (g.cin / g.groups) * g.kh * g.kw;
  if (total == 0) return FH_OK;
  if (x == nullptr || dy == nullptr || dw == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_conv2d_grad_filter: null pointer");
  return dispatch<ConvGradRun>(dtype, 1, x, dy, dw, g, total, static_cast<hipStream_t>(stream));
}

extern "C" fh_status fh_sum(int32_t dtype, const void* x, void* out, int32_t rank, const int64_t* dims,
                            const uint8_t* reduced, void* stream) {
  if (!is_supported_float(dtype)) return fail(FH_UNIMPLEMENTED, "fh_sum: unsupported dtype");
  if (fh_status st = check_reduce("fh_sum", rank, dims, reduced); st != FH_OK) return st;
  uint8_t all[kMaxDims];
  for (int32_t d = 0; d < rank; ++d) all[d] = reduced[d];
  ReduceG g{};
  build_reduce(rank, dims, all, g);
  int64_t numel = 1;
  for (int32_t d = 0; d < rank; ++d) numel *= dims[d];
  if (g.nout == 0) return FH_OK;
  if (x == nullptr || out == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_sum: null pointer");
  if (numel == 0) g.nred = 0;  // an empty reduction writes zeros
  if (!grid_ok(g.nout)) return fail(FH_INVALID_ARGUMENT, "fh_sum: too many outputs");
  return dispatch<SumRun>(dtype, x, out, g, static_cast<hipStream_t>(stream));
}

extern "C" fh_status fh_sum_grad(int32_t dtype, const void* gy, void* gx, int32_t rank, const int64_t* dims,
                                 const uint8_t* reduced, void* stream) {
  if (!is_supported_float(dtype)) return fail(FH_UNIMPLEMENTED, "fh_sum_grad: unsupported dtype");
  if (fh_status st = check_reduce("fh_sum_grad", rank, dims, reduced); st != FH_OK) return st;
  // full dims of x with the output (gy) strides of each dim, reduced dims striding 0
  ReduceG g{};
  g.nk = rank;
  int64_t total = 1, ostride = 1;
  for (int32_t d = rank - 1; d >= 0; --d) {
    g.kdim[d] = dims[d];
    g.kstride[d] = reduced[d] ? 0 : ostride;
    if (!reduced[d]) ostride *= dims[d];
    total *= dims[d];
  }
  if (total == 0) return FH_OK;
  if (gy == nullptr || gx == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_sum_grad: null pointer");
  if (!grid_ok(blocks_for(total))) return fail(FH_INVALID_ARGUMENT, "fh_sum_grad: tensor too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>(blocks_for(total)));
  if (dtype == FH_F32)
    hipLaunchKernelGGL((sum_grad_kernel<uint32_t>), grid, dim3(kThreads), 0, s, static_cast<const uint32_t*>(gy),
                       static_cast<uint32_t*>(gx), g, total);
  else
    hipLaunchKernelGGL((sum_grad_kernel<uint16_t>), grid, dim3(kThreads), 0, s, static_cast<const uint16_t*>(gy),
                       static_cast<uint16_t*>(gx), g, total);
  return launch_status("fh_sum_grad");
}

extern "C" fh_status fh_mse_loss(int32_t dtype, const void* pred, const void* target, void* out, int64_t numel,
                                 void* stream) {
  if (!is_supported_float(dtype)) return fail(FH_UNIMPLEMENTED, "fh_mse_loss: unsupported dtype");
  if (numel <= 0) return fail(FH_INVALID_ARGUMENT, "fh_mse_loss: empty input (numel 0)");
  if (pred == nullptr || target == nullptr || out == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_mse_loss: null pointer");
  return dispatch<MseRun>(dtype, 0, pred, target, nullptr, out, numel, static_cast<hipStream_t>(stream));
}

extern "C" fh_status fh_mse_loss_grad(int32_t dtype, const void* pred, const void* target, const void* gy, void* out,
                                      int64_t numel, void* stream) {
  if (!is_supported_float(dtype)) return fail(FH_UNIMPLEMENTED, "fh_mse_loss_grad: unsupported dtype");
  if (numel <= 0) return fail(FH_INVALID_ARGUMENT, "fh_mse_loss_grad: empty input (numel 0)");
  if (pred == nullptr || target == nullptr || gy == nullptr || out == nullptr)
    return fail(FH_INVALID_ARGUMENT, "fh_mse_loss_grad: null pointer");
  if (!grid_ok(blocks_for(numel))) return fail(FH_INVALID_ARGUMENT, "fh_mse_loss_grad: tensor too large");
  return dispatch<MseRun>(dtype, 1, pred, target, gy, out, numel, static_cast<hipStream_t>(stream));
}

extern "C" fh_status fh_conv_filter_flip(int32_t dtype, const void* w, void* out, int64_t cout, int64_t cin, int64_t kh,
                                         int64_t kw, void* stream) {
  if (!is_supported_float(dtype)) return fail(FH_UNIMPLEMENTED, "fh_conv_filter_flip: unsupported dtype");
  if (cout < 0 || cin < 0 || kh < 0 || kw < 0 || cout > 0x7fffffffLL || cin > 0x7fffffffLL || kh > 0x7fffffffLL ||
      kw > 0x7fffffffLL)
    return fail(FH_INVALID_ARGUMENT, "fh_conv_filter_flip: invalid dims");
  const int64_t total = cout * cin * kh * kw;
  if (total == 0) return FH_OK;
  if (w == nullptr || out == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_conv_filter_flip: null pointer");
  if (!grid_ok(blocks_for(total))) return fail(FH_INVALID_ARGUMENT, "fh_conv_filter_flip: tensor too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>(blocks_for(total)));
  const int32_t a = static_cast<int32_t>(cout), b = static_cast<int32_t>(cin), c = static_cast<int32_t>(kh),
                d = static_cast<int32_t>(kw);
  const int64_t taps = kh * kw, esize = dtype_size(dtype);
  const int64_t lds = kFlipCo * (kFlipCi * taps + 1) * esize;
  const int64_t gy = (cin + kFlipCi - 1) / kFlipCi;
  if (lds <= 64 * 1024 && gy <= 65535) {
    const dim3 tgrid(static_cast<uint32_t>((cout + kFlipCo - 1) / kFlipCo), static_cast<uint32_t>(gy));
    const size_t shm = static_cast<size_t>((lds + 3) / 4 * 4);
    const int32_t t = static_cast<int32_t>(taps);
    if (dtype == FH_F32)
      hipLaunchKernelGGL((filter_flip_tiled_kernel<uint32_t>), tgrid, dim3(kThreads), shm, s,
                         static_cast<const uint32_t*>(w), static_cast<uint32_t*>(out), a, b, t);
    else
      hipLaunchKernelGGL((filter_flip_tiled_kernel<uint16_t>), tgrid, dim3(kThreads), shm, s,
                         static_cast<const uint16_t*>(w), static_cast<uint16_t*>(out), a, b, t);
    return launch_status("fh_conv_filter_flip");
  }
  if (dtype == FH_F32)
    hipLaunchKernelGGL((filter_flip_kernel<uint32_t>), grid, dim3(kThreads), 0, s, static_cast<const uint32_t*>(w),
                       static_cast<uint32_t*>(out), a, b, c, d, total);
  else
    hipLaunchKernelGGL((filter_flip_kernel<uint16_t>), grid, dim3(kThreads), 0, s, static_cast<const uint16_t*>(w),
                       static_cast<uint16_t*>(out), a, b, c, d, total);
  return launch_status("fh_conv_filter_flip");
}

extern "C" fh_status fh_conv_filter_flip_multi(int32_t dtype, int32_t count, const void* const* w, void* const* out,
                                               const int64_t* dims, void* stream) {
  if (!is_supported_float(dtype)) return fail(FH_UNIMPLEMENTED, "fh_conv_filter_flip_multi: unsupported dtype");
  if (count < 0 || count > FH_FLIP_MAX) return fail(FH_INVALID_ARGUMENT, "fh_conv_filter_flip_multi: count out of range");
  if (count == 0) return FH_OK;
  if (w == nullptr || out == nullptr || dims == nullptr)
    return fail(FH_INVALID_ARGUMENT, "fh_conv_filter_flip_multi: null pointer");
  const int64_t esize = dtype_size(dtype);
  int64_t max_taps = 1;
  for (int32_t i = 0; i < count; ++i) {
    const int64_t cout = dims[4 * i], cin = dims[4 * i + 1], kh = dims[4 * i + 2], kw = dims[4 * i + 3];
    if (cout < 0 || cin < 0 || kh < 0 || kw < 0 || cout > 0x7fffffffLL || cin > 0x7fffffffLL)
      return fail(FH_INVALID_ARGUMENT, "fh_conv_filter_flip_multi: invalid dims");
    if (kh * kw > FH_FLIP_MAX_TAPS)
      return fail(FH_INVALID_ARGUMENT, "fh_conv_filter_flip_multi: kh * kw above " + std::to_string(FH_FLIP_MAX_TAPS));
    if (cout * cin * kh * kw > 0) max_taps = std::max(max_taps, kh * kw);
  }
  // input channels per workgroup: up to 8, as many as keep the tile within 64 KB of LDS (at least one: 255 taps of
  // fp32 take 64 KB)
  const int32_t ci_per = static_cast<int32_t>(std::clamp<int64_t>((65536 / (kFlipCo * esize) - 1) / max_taps, 1, 8));
  FlipBatch b{};
  int64_t blocks = 0;
  for (int32_t i = 0; i < count; ++i) {
    const int64_t cout = dims[4 * i], cin = dims[4 * i + 1], kh = dims[4 * i + 2], kw = dims[4 * i + 3];
    const int64_t total = cout * cin * kh * kw;
    if (total > 0 && (w[i] == nullptr || out[i] == nullptr))
      return fail(FH_INVALID_ARGUMENT, "fh_conv_filter_flip_multi: null tensor pointer");
    b.w[i] = w[i], b.out[i] = out[i];
    b.cout[i] = static_cast<int32_t>(cout), b.cin[i] = static_cast<int32_t>(cin);
    b.taps[i] = static_cast<int32_t>(kh * kw);
    b.first_block[i] = static_cast<int32_t>(blocks);
    if (total > 0) blocks += (cout + kFlipCo - 1) / kFlipCo * ((cin + ci_per - 1) / ci_per);
    if (blocks > 0x7fffffffLL) return fail(FH_INVALID_ARGUMENT, "fh_conv_filter_flip_multi: filters too large for one launch");
  }
  b.first_block[count] = static_cast<int32_t>(blocks);
  b.count = count;
  b.ci_per = ci_per;
  if (blocks == 0) return FH_OK;
  const size_t shm = static_cast<size_t>((kFlipCo * (ci_per * max_taps + 1) * esize + 3) / 4 * 4);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == FH_F32)
    hipLaunchKernelGGL((filter_flip_multi_kernel<uint32_t>), dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), shm, s, b);
  else
    hipLaunchKernelGGL((filter_flip_multi_kernel<uint16_t>), dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), shm, s, b);
  return launch_status("fh_conv_filter_flip_multi");
}

extern "C" fh_status fh_axpy_multi(int32_t dtype, int32_t count, const void* const* x, const void* const* y,
                                   void* const* out, const int64_t* numel, const float* scales, void* stream) {
  if (!is_supported_float(dtype)) return fail(FH_UNIMPLEMENTED, "fh_axpy_multi: unsupported dtype");
  if (count < 0 || count > FH_AXPY_MAX) return fail(FH_INVALID_ARGUMENT, "fh_axpy_multi: count out of range");
  if (count == 0) return FH_OK;
  if (x == nullptr || y == nullptr || out == nullptr || numel == nullptr || scales == nullptr)
    return fail(FH_INVALID_ARGUMENT, "fh_axpy_multi: null pointer");
  const int64_t esize = dtype_size(dtype), per_block = int64_t{kThreads} * kAxpyVecs * (16 / esize);
  AxpyBatch b{};
  int64_t blocks = 0;
  for (int32_t i = 0; i < count; ++i) {
    if (numel[i] < 0) return fail(FH_INVALID_ARGUMENT, "fh_axpy_multi: negative numel");
    if (numel[i] > 0 && (x[i] == nullptr || y[i] == nullptr || out[i] == nullptr))
      return fail(FH_INVALID_ARGUMENT, "fh_axpy_multi: null tensor pointer");
    b.x[i] = x[i], b.y[i] = y[i], b.out[i] = out[i], b.n[i] = numel[i], b.s[i] = scales[i];
    b.first_block[i] = static_cast<int32_t>(blocks);
    const bool al = reinterpret_cast<uintptr_t>(x[i]) % 16 == 0 && reinterpret_cast<uintptr_t>(y[i]) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(out[i]) % 16 == 0;
    if (al) b.aligned |= 1u << i;
    blocks += (numel[i] + per_block - 1) / per_block;
    if (blocks > 0x7fffffffLL) return fail(FH_INVALID_ARGUMENT, "fh_axpy_multi: tensors too large for one launch");
  }
  b.first_block[count] = static_cast<int32_t>(blocks);
  b.count = count;
  if (blocks == 0) return FH_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>(blocks));
  switch (dtype) {
    case FH_F32: hipLaunchKernelGGL((axpy_multi_kernel<float>), grid, dim3(kThreads), 0, s, b); break;
    case FH_BF16: hipLaunchKernelGGL((axpy_multi_kernel<bf16_t>), grid, dim3(kThreads), 0, s, b); break;
    default: hipLaunchKernelGGL((axpy_multi_kernel<f16_t>), grid, dim3(kThreads), 0, s, b); break;
  }
  return launch_status("fh_axpy_multi");
}

extern "C" fh_status fh_dilate_nhwc(int32_t dtype, int32_t in_nhwc, const void* x, void* out, int64_t n, int64_t c,
                                    int64_t h, int64_t w, int64_t sh, int64_t sw, int64_t hu, int64_t wu, void* stream) {
  if (!is_supported_float(dtype)) return fail(FH_UNIMPLEMENTED, "fh_dilate_nhwc: unsupported dtype");
  const int64_t dims[] = {n, c, h, w, sh, sw, hu, wu};
  for (int64_t v : dims)
    if (v < 0 || v > 0x7fffffffLL) return fail(FH_INVALID_ARGUMENT, "fh_dilate_nhwc: invalid dims");
  if (sh == 0 || sw == 0) return fail(FH_INVALID_ARGUMENT, "fh_dilate_nhwc: zero stride");
  const int64_t total = n * hu * wu * c;
  if (total == 0) return FH_OK;
  if (x == nullptr || out == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_dilate_nhwc: null pointer");
  if (!grid_ok(blocks_for(total))) return fail(FH_INVALID_ARGUMENT, "fh_dilate_nhwc: tensor too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int32_t args[] = {static_cast<int32_t>(c), static_cast<int32_t>(h), static_cast<int32_t>(w), static_cast<int32_t>(sh),
                          static_cast<int32_t>(sw), static_cast<int32_t>(hu), static_cast<int32_t>(wu)};
  if (in_nhwc) {
    const int64_t vw = 16 / dtype_size(dtype);
    if (c % vw != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(out) % 16 != 0)
      return fail(FH_UNIMPLEMENTED, "fh_dilate_nhwc: a channels-last input needs 16-byte channel vectors");
    const int64_t vt = total / vw;
    const dim3 vgrid(static_cast<uint32_t>(blocks_for(vt)));
    if (dtype == FH_F32)
      hipLaunchKernelGGL((dilate_nhwc_vec_kernel<uint32_t>), vgrid, dim3(kThreads), 0, s, static_cast<const uint32_t*>(x),
                         static_cast<uint32_t*>(out), args[0], args[1], args[2], args[3], args[4], args[5], args[6], vt);
    else
      hipLaunchKernelGGL((dilate_nhwc_vec_kernel<uint16_t>), vgrid, dim3(kThreads), 0, s, static_cast<const uint16_t*>(x),
                         static_cast<uint16_t*>(out), args[0], args[1], args[2], args[3], args[4], args[5], args[6], vt);
    return launch_status("fh_dilate_nhwc");
  }
  const dim3 grid(static_cast<uint32_t>(blocks_for(total)));
  if (dtype == FH_F32)
    hipLaunchKernelGGL((dilate_nhwc_kernel<uint32_t>), grid, dim3(kThreads), 0, s, static_cast<const uint32_t*>(x),
                       static_cast<uint32_t*>(out), args[0], args[1], args[2], args[3], args[4], args[5], args[6], total);
  else
    hipLaunchKernelGGL((dilate_nhwc_kernel<uint16_t>), grid, dim3(kThreads), 0, s, static_cast<const uint16_t*>(x),
                       static_cast<uint16_t*>(out), args[0], args[1], args[2], args[3], args[4], args[5], args[6], total);
  return launch_status("fh_dilate_nhwc");
}

extern "C" fh_status fh_avg_pool2d_grad_nhwc(int32_t dtype, const void* dy, void* dx, const int64_t geom[10], void* stream) {
  if (!is_supported_float(dtype)) return fail(FH_UNIMPLEMENTED, "fh_avg_pool2d_grad_nhwc: unsupported dtype");
  if (geom == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_avg_pool2d_grad_nhwc: null geometry");
  for (int k = 0; k < 10; ++k)
    if (geom[k] < 0 || geom[k] > 0x7fffffffLL) return fail(FH_INVALID_ARGUMENT, "fh_avg_pool2d_grad_nhwc: geometry entry out of range");
  PoolG g{static_cast<int32_t>(geom[0]), static_cast<int32_t>(geom[1]), static_cast<int32_t>(geom[2]),
          static_cast<int32_t>(geom[3]), static_cast<int32_t>(geom[4]), static_cast<int32_t>(geom[5]),
          static_cast<int32_t>(geom[6]), static_cast<int32_t>(geom[7]), static_cast<int32_t>(geom[8]),
          static_cast<int32_t>(geom[9]), 0, 0};
  if (g.kh <= 0 || g.kw <= 0 || g.sh <= 0 || g.sw <= 0 || g.h + 2 * g.ph < g.kh || g.w + 2 * g.pw < g.kw)
    return fail(FH_INVALID_ARGUMENT, "fh_avg_pool2d_grad_nhwc: invalid geometry");
  g.oh = (g.h + 2 * g.ph - g.kh) / g.sh + 1;
  g.ow = (g.w + 2 * g.pw - g.kw) / g.sw + 1;
  const int64_t vw = 16 / dtype_size(dtype);
  if (g.c % vw != 0 || reinterpret_cast<uintptr_t>(dy) % 16 != 0 || reinterpret_cast<uintptr_t>(dx) % 16 != 0)
    return fail(FH_UNIMPLEMENTED, "fh_avg_pool2d_grad_nhwc: needs 16-byte channel vectors");
  const int64_t total = static_cast<int64_t>(g.n) * g.h * g.w * (g.c / vw);
  if (total == 0) return FH_OK;
  if (dy == nullptr || dx == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_avg_pool2d_grad_nhwc: null pointer");
  if (!grid_ok(blocks_for(total))) return fail(FH_INVALID_ARGUMENT, "fh_avg_pool2d_grad_nhwc: tensor too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>(blocks_for(total)));
  switch (dtype) {
    case FH_F32:
      hipLaunchKernelGGL((avgpool_grad_nhwc_kernel<float>), grid, dim3(kThreads), 0, s, static_cast<const float*>(dy),
                         static_cast<float*>(dx), g, total);
      break;
    case FH_BF16:
      hipLaunchKernelGGL((avgpool_grad_nhwc_kernel<bf16_t>), grid, dim3(kThreads), 0, s, static_cast<const uint16_t*>(dy),
                         static_cast<uint16_t*>(dx), g, total);
      break;
    default:
      hipLaunchKernelGGL((avgpool_grad_nhwc_kernel<f16_t>), grid, dim3(kThreads), 0, s, static_cast<const uint16_t*>(dy),
                         static_cast<uint16_t*>(dx), g, total);
      break;
  }
  return launch_status("fh_avg_pool2d_grad_nhwc");
}

namespace {
// rows per stage-1 workgroup: about 256 workgroups, 64 .. 65536 rows each
int64_t sum_rows_per_wg(int64_t rows) { return std::min<int64_t>(65536, std::max<int64_t>(64, (rows + 255) / 256)); }
}  // namespace

extern "C" int64_t fh_sum_rows_workspace(int32_t dtype, int64_t rows, int64_t cols) {
  if (!is_supported_float(dtype) || rows <= 0 || cols <= 0 || (cols * dtype_size(dtype)) % 16 != 0 || cols > (1 << 24))
    return -1;
  const int64_t per = sum_rows_per_wg(rows);
  const int64_t wgs = (rows + per - 1) / per;
  if (wgs > 0x7fffffffLL) return -1;
  return wgs * cols * 4;
}

extern "C" fh_status fh_sum_rows(int32_t dtype, const void* x, void* out, int64_t rows, int64_t cols, void* workspace,
                                 int64_t workspace_bytes, void* stream) {
  const int64_t need = fh_sum_rows_workspace(dtype, rows, cols);
  if (need < 0) return fail(FH_UNIMPLEMENTED, "fh_sum_rows: unsupported dtype or shape (cols*itemsize % 16 != 0)");
  if (workspace_bytes < need) return fail(FH_INVALID_ARGUMENT, "fh_sum_rows: workspace too small");
  if (x == nullptr || out == nullptr || workspace == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_sum_rows: null pointer");
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return fail(FH_INVALID_ARGUMENT, "fh_sum_rows: x must be 16-byte aligned");
  const int64_t per = sum_rows_per_wg(rows);
  const int32_t wgs = static_cast<int32_t>((rows + per - 1) / per);
  const int32_t c = static_cast<int32_t>(cols);
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* part = static_cast<float*>(workspace);
  const dim3 fgrid(static_cast<uint32_t>((cols + kThreads / 64 - 1) / (kThreads / 64)));
  switch (dtype) {
    case FH_F32:
      hipLaunchKernelGGL((sum_rows_partial_kernel<float>), dim3(wgs), dim3(kThreads), 0, s, static_cast<const float*>(x), part,
                         rows, c, per);
      hipLaunchKernelGGL((sum_rows_final_kernel<float>), fgrid, dim3(kThreads), 0, s, part, static_cast<float*>(out), wgs, c);
      break;
    case FH_BF16:
      hipLaunchKernelGGL((sum_rows_partial_kernel<bf16_t>), dim3(wgs), dim3(kThreads), 0, s, static_cast<const uint16_t*>(x),
                         part, rows, c, per);
      hipLaunchKernelGGL((sum_rows_final_kernel<bf16_t>), fgrid, dim3(kThreads), 0, s, part, static_cast<uint16_t*>(out), wgs, c);
      break;
    default:
      hipLaunchKernelGGL((sum_rows_partial_kernel<f16_t>), dim3(wgs), dim3(kThreads), 0, s, static_cast<const uint16_t*>(x),
                         part, rows, c, per);
      hipLaunchKernelGGL((sum_rows_final_kernel<f16_t>), fgrid, dim3(kThreads), 0, s, part, static_cast<uint16_t*>(out), wgs, c);
      break;
  }
  return launch_status("fh_sum_rows");
}
