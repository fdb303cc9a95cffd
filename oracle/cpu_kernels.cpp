// TEST INFRASTRUCTURE — parity oracle (see cpu_kernels.h). Never linked into the product.
//
// Written as plain loops on purpose: each function is a line-by-line statement of the arithmetic the
// reference CPU backend performs, so that summation order and rounding points are visible and identical.
// Compiled with -ffp-contract=off: the reference's a*b+c is a multiply followed by an add.
#include "cpu_kernels.h"

#include <cmath>
#include <cstring>
#include <vector>

namespace {

// ---- dtype bridge: IEEE binary16 / bfloat16 round-to-nearest-even (reference: include/frame/core/dtype.h:51-131)
uint32_t bits_of(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}
float float_of(uint32_t u) {
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

uint16_t to_bf16(float v) {
  const uint32_t u = bits_of(v);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);  // quiet NaN
  return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
float from_bf16(uint16_t b) { return float_of(static_cast<uint32_t>(b) << 16); }

// binary16 narrowing written from the IEEE-754 definition: normal numbers round the 13 dropped mantissa bits to
// nearest-even, values below the smallest normal are shifted into a subnormal with the same rule, overflow goes
// to infinity, NaN becomes the canonical quiet NaN with the sign kept.
uint16_t to_f16(float v) {
  const uint32_t u = bits_of(v);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t mag = u & 0x7fffffffu;
  if (mag > 0x7f800000u) return static_cast<uint16_t>(sign | 0x7e00u);
  if (mag == 0x7f800000u) return static_cast<uint16_t>(sign | 0x7c00u);
  const int exp = static_cast<int>(mag >> 23) - 127;  // unbiased
  if (exp >= 16) return static_cast<uint16_t>(sign | 0x7c00u);
  if (exp >= -14) {  // normal range of binary16
    const uint32_t mant = mag & 0x7fffffu;
    uint32_t h = (static_cast<uint32_t>(exp + 15) << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;  // carries into exponent / infinity correctly
    return static_cast<uint16_t>(sign | h);
  }
  if (exp < -25) return static_cast<uint16_t>(sign);  // below half of the smallest subnormal: zero
  // subnormal: value = mant24 * 2^(exp-23); target unit is 2^-24
  const uint32_t mant24 = (mag & 0x7fffffu) | 0x800000u;
  const int shift = -exp - 1;  // number of bits dropped: 14 - exp - 1 ... keeps units of 2^-24
  uint32_t h = mant24 >> shift;
  const uint32_t rem = mant24 & ((1u << shift) - 1u);
  const uint32_t halfway = 1u << (shift - 1);
  if (rem > halfway || (rem == halfway && (h & 1u))) ++h;
  return static_cast<uint16_t>(sign | h);
}

float from_f16(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t mant = h & 0x3ffu;
  if (exp == 0) {
    // subnormal or zero: mant * 2^-24, exact in binary32
    const float mag = static_cast<float>(mant) * 5.9604644775390625e-08f;
    return sign ? -mag : mag;
  }
  if (exp == 0x1f) return float_of(sign | 0x7f800000u | (mant << 13));
  return float_of(sign | ((exp + 112u) << 23) | (mant << 13));
}

// Typed load/store through fp32 (reference: src/backends/cpu/kernels/accum_cast.h:19-44)
struct F32 {
  using S = float;
  static float ld(S v) { return v; }
  static S st(float v) { return v; }
};
struct BF16 {
  using S = uint16_t;
  static float ld(S v) { return from_bf16(v); }
  static S st(float v) { return to_bf16(v); }
};
struct F16 {
  using S = uint16_t;
  static float ld(S v) { return from_f16(v); }
  static S st(float v) { return to_f16(v); }
};

template <typename Fn>
int with_dtype(int dtype, Fn&& fn) {
  switch (dtype) {
    case 0:
      return fn(F32{});
    case 2:
      return fn(F16{});
    case 3:
      return fn(BF16{});
    default:
      return 1;
  }
}

// Sub-op arithmetic (reference: src/backends/cpu/kernels/elementwise.cpp:146-331). relu is std::max(x, 0.0f):
// `x < 0 ? 0 : x`, which keeps NaN and -0.0. gelu is this build's exact-erf form.
float unary(uint8_t op, float x) {
  switch (op) {
    case 3:
      return (x < 0.0f) ? 0.0f : x;
    case 4:
      return x * x;
    case 5:
      return 0.5f * x * (1.0f + std::erf(x * 0.70710678118654752440f));
    case 7:  // sigmoid, the reference's overflow-free two-branch form (elementwise.cpp:342-353)
      if (x >= 0.0f) return 1.0f / (1.0f + std::exp(-x));
      return std::exp(x) / (1.0f + std::exp(x));
    case 8:  // tanh (elementwise.cpp:397)
      return std::tanh(x);
    case 9:  // rsqrt (elementwise.cpp:405)
      return 1.0f / std::sqrt(x);
    default:
      return x;
  }
}
// op 6 is relu_grad_internal(x, gy): gy where x > 0, else 0 (reference: src/backends/cpu/kernels/elementwise.cpp:407-414).
// op 10 is gelu_grad_internal(x, gy) = gy * (Phi(x) + x * phi(x)), this build's gelu derivative (no reference).
float binary(uint8_t op, float a, float b) {
  if (op == 6) return a > 0.0f ? b : 0.0f;
  if (op == 10)
    return b * (0.5f * (1.0f + std::erf(a * 0.70710678118654752440f)) + a * (std::exp(-0.5f * a * a) * 0.39894228040143267794f));
  return op == 2 ? a * b : a + b;
}
bool is_binary(uint8_t op) { return op == 1 || op == 2 || op == 6 || op == 10; }

template <typename D>
float matmul_element(const typename D::S* a, const typename D::S* b, int64_t n, int64_t k, int64_t i, int64_t j) {
  float acc = 0.0f;
  for (int64_t p = 0; p < k; ++p) acc += D::ld(a[i * k + p]) * D::ld(b[p * n + j]);
  return acc;
}

struct ConvG {
  int64_t n, cin, h, w, cout, kh, kw, sh, sw, ph, pw, groups, oh, ow;
};

bool read_conv(const int64_t* g, ConvG& c) {
  c = ConvG{g[0], g[1], g[2], g[3], g[4], g[5], g[6], g[7], g[8], g[9], g[10], g[11], 0, 0};
  if (c.groups <= 0 || c.sh <= 0 || c.sw <= 0 || c.cin % c.groups || c.cout % c.groups) return false;
  c.oh = (c.h + 2 * c.ph - c.kh) / c.sh + 1;  // floor formula (reference: src/backends/cpu/kernels/conv.cpp:209-210)
  c.ow = (c.w + 2 * c.pw - c.kw) / c.sw + 1;
  return true;
}

// One output of conv2d: products in (ci, kh, kw) order skipping padding, bias added last
// (reference: src/backends/cpu/kernels/conv.cpp:223-251).
template <typename D>
float conv_element(const ConvG& p, const typename D::S* x, const typename D::S* w, const typename D::S* bias,
                   int64_t idx) {
  const int64_t ow = idx % p.ow;
  const int64_t oh = (idx / p.ow) % p.oh;
  const int64_t co = (idx / (p.ow * p.oh)) % p.cout;
  const int64_t n = idx / (p.ow * p.oh * p.cout);
  const int64_t cin_g = p.cin / p.groups;
  const int64_t g = co / (p.cout / p.groups);
  float acc = 0.0f;
  for (int64_t ci = 0; ci < cin_g; ++ci) {
    const int64_t cf = g * cin_g + ci;
    for (int64_t a = 0; a < p.kh; ++a) {
      const int64_t ih = oh * p.sh - p.ph + a;
      if (ih < 0 || ih >= p.h) continue;
      for (int64_t b = 0; b < p.kw; ++b) {
        const int64_t iw = ow * p.sw - p.pw + b;
        if (iw < 0 || iw >= p.w) continue;
        acc += D::ld(x[((n * p.cin + cf) * p.h + ih) * p.w + iw]) * D::ld(w[((co * cin_g + ci) * p.kh + a) * p.kw + b]);
      }
    }
  }
  if (bias != nullptr) acc += D::ld(bias[co]);
  return acc;
}

}  // namespace

extern "C" {

uint16_t oracle_float_to_bf16(float v) { return to_bf16(v); }
float oracle_bf16_to_float(uint16_t b) { return from_bf16(b); }
uint16_t oracle_float_to_f16(float v) { return to_f16(v); }
float oracle_f16_to_float(uint16_t h) { return from_f16(h); }
void oracle_f32_to_bf16_array(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = to_bf16(in[i]);
}
void oracle_f32_to_f16_array(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = to_f16(in[i]);
}

// reference: src/backends/cpu/kernels/matmul.cpp:92-129 — i, j outer, p inner and sequential
int oracle_matmul(int dtype, const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t k) {
  return with_dtype(dtype, [&](auto d) {
    using D = decltype(d);
    const auto* A = static_cast<const typename D::S*>(a);
    const auto* B = static_cast<const typename D::S*>(b);
    auto* C = static_cast<typename D::S*>(c);
    for (int64_t i = 0; i < m; ++i)
      for (int64_t j = 0; j < n; ++j) C[i * n + j] = D::st(matmul_element<D>(A, B, n, k, i, j));
    return 0;
  });
}

int oracle_matmul_sample(int dtype, const void* a, const void* b, int64_t m, int64_t n, int64_t k,
                         const int64_t* rows, const int64_t* cols, int64_t count, void* out) {
  return with_dtype(dtype, [&](auto d) {
    using D = decltype(d);
    const auto* A = static_cast<const typename D::S*>(a);
    const auto* B = static_cast<const typename D::S*>(b);
    auto* O = static_cast<typename D::S*>(out);
    for (int64_t s = 0; s < count; ++s) {
      if (rows[s] < 0 || rows[s] >= m || cols[s] < 0 || cols[s] >= n) return 1;
      O[s] = D::st(matmul_element<D>(A, B, n, k, rows[s], cols[s]));
    }
    return 0;
  });
}

int oracle_conv2d(int dtype, const void* x, const void* w, const void* bias, void* y, const int64_t* geom) {
  ConvG p;
  if (!read_conv(geom, p)) return 1;
  return with_dtype(dtype, [&](auto d) {
    using D = decltype(d);
    using S = typename D::S;
    const int64_t total = p.n * p.cout * p.oh * p.ow;
    for (int64_t i = 0; i < total; ++i)
      static_cast<S*>(y)[i] = D::st(conv_element<D>(p, static_cast<const S*>(x), static_cast<const S*>(w),
                                                    static_cast<const S*>(bias), i));
    return 0;
  });
}

int oracle_conv2d_sample(int dtype, const void* x, const void* w, const void* bias, const int64_t* geom,
                         const int64_t* idx, int64_t count, void* out) {
  ConvG p;
  if (!read_conv(geom, p)) return 1;
  const int64_t total = p.n * p.cout * p.oh * p.ow;
  return with_dtype(dtype, [&](auto d) {
    using D = decltype(d);
    using S = typename D::S;
    for (int64_t s = 0; s < count; ++s) {
      if (idx[s] < 0 || idx[s] >= total) return 1;
      static_cast<S*>(out)[s] = D::st(conv_element<D>(p, static_cast<const S*>(x), static_cast<const S*>(w),
                                                      static_cast<const S*>(bias), idx[s]));
    }
    return 0;
  });
}

// Segments run one after another over the whole tensor, each rounding to the storage dtype, exactly like the
// reference's sequential sub-kernel execution with temporaries (reference: src/ops/fused_elementwise_utils.cpp:122-206).
int oracle_ew_program(int dtype, int nseg, const uint8_t* ops, const int8_t* arities, const void* const* ins,
                      int nin, void* out, int64_t numel) {
  int expected = 0;
  for (int s = 0; s < nseg; ++s) expected += (s == 0) ? arities[s] : arities[s] - 1;
  if (nseg < 1 || expected != nin) return 1;
  return with_dtype(dtype, [&](auto d) {
    using D = decltype(d);
    using S = typename D::S;
    std::vector<S> prev(static_cast<size_t>(numel)), cur(static_cast<size_t>(numel));
    int next = 0;
    for (int s = 0; s < nseg; ++s) {
      const S* in0 = (s == 0) ? static_cast<const S*>(ins[next++]) : prev.data();
      const S* in1 = nullptr;
      if (arities[s] == 2) in1 = static_cast<const S*>(ins[next++]);
      for (int64_t i = 0; i < numel; ++i) {
        const float a = D::ld(in0[i]);
        const float r = is_binary(ops[s]) ? binary(ops[s], a, D::ld(in1[i])) : unary(ops[s], a);
        cur[static_cast<size_t>(i)] = D::st(r);
      }
      prev.swap(cur);
    }
    std::memcpy(out, prev.data(), static_cast<size_t>(numel) * sizeof(S));
    return 0;
  });
}

// reference: src/backends/cpu/kernels/sequence.cpp:148-173
int oracle_softmax(int dtype, const void* x, void* y, int64_t rows, int64_t cols) {
  if (cols <= 0) return rows == 0 ? 0 : 1;
  return with_dtype(dtype, [&](auto d) {
    using D = decltype(d);
    using S = typename D::S;
    const S* X = static_cast<const S*>(x);
    S* Y = static_cast<S*>(y);
    std::vector<float> row(static_cast<size_t>(cols));
    for (int64_t i = 0; i < rows; ++i) {
      float mx = D::ld(X[i * cols]);
      row[0] = mx;
      for (int64_t j = 1; j < cols; ++j) {
        const float v = D::ld(X[i * cols + j]);
        row[static_cast<size_t>(j)] = v;
        if (v > mx) mx = v;
      }
      float sum = 0.0f;
      for (int64_t j = 0; j < cols; ++j) {
        const float e = std::exp(row[static_cast<size_t>(j)] - mx);
        row[static_cast<size_t>(j)] = e;
        sum += e;
      }
      for (int64_t j = 0; j < cols; ++j) Y[i * cols + j] = D::st(row[static_cast<size_t>(j)] / sum);
    }
    return 0;
  });
}

// reference: src/backends/cpu/kernels/sequence.cpp:254-276
int oracle_layer_norm(int dtype, const void* x, const void* gamma, const void* beta, void* y, int64_t rows,
                      int64_t cols, double eps_attr) {
  const float eps = static_cast<float>(eps_attr);
  return with_dtype(dtype, [&](auto d) {
    using D = decltype(d);
    using S = typename D::S;
    const S* X = static_cast<const S*>(x);
    const S* G = static_cast<const S*>(gamma);
    const S* B = static_cast<const S*>(beta);
    S* Y = static_cast<S*>(y);
    for (int64_t i = 0; i < rows; ++i) {
      const S* xr = X + i * cols;
      float sum = 0.0f;
      for (int64_t j = 0; j < cols; ++j) sum += D::ld(xr[j]);
      const float mean = sum / static_cast<float>(cols);
      float var_sum = 0.0f;
      for (int64_t j = 0; j < cols; ++j) {
        const float c = D::ld(xr[j]) - mean;
        var_sum += c * c;
      }
      const float variance = var_sum / static_cast<float>(cols);
      const float r = 1.0f / std::sqrt(variance + eps);
      for (int64_t j = 0; j < cols; ++j) {
        const float xhat = (D::ld(xr[j]) - mean) * r;
        Y[i * cols + j] = D::st(D::ld(G[j]) * xhat + D::ld(B[j]));
      }
    }
    return 0;
  });
}

// reference: src/backends/cpu/kernels/pool.cpp:178-237 (max) and :283-306 (avg)
int oracle_pool2d(int dtype, int mode, const void* x, void* y, const int64_t* g) {
  const int64_t N = g[0], C = g[1], H = g[2], W = g[3], KH = g[4], KW = g[5], SH = g[6], SW = g[7], PH = g[8],
                PW = g[9];
  if (SH <= 0 || SW <= 0 || KH <= 0 || KW <= 0) return 1;
  const int64_t OH = (H + 2 * PH - KH) / SH + 1, OW = (W + 2 * PW - KW) / SW + 1;
  return with_dtype(dtype, [&](auto d) {
    using D = decltype(d);
    using S = typename D::S;
    const S* X = static_cast<const S*>(x);
    S* Y = static_cast<S*>(y);
    const float denom = static_cast<float>(KH * KW);
    for (int64_t nc = 0; nc < N * C; ++nc)
      for (int64_t oh = 0; oh < OH; ++oh)
        for (int64_t ow = 0; ow < OW; ++ow) {
          float acc = 0.0f;
          bool found = false;
          for (int64_t a = 0; a < KH; ++a) {
            const int64_t ih = oh * SH - PH + a;
            if (ih < 0 || ih >= H) continue;
            for (int64_t b = 0; b < KW; ++b) {
              const int64_t iw = ow * SW - PW + b;
              if (iw < 0 || iw >= W) continue;
              const float v = D::ld(X[(nc * H + ih) * W + iw]);
              if (mode == 0) {
                if (!found || v > acc) acc = v;
                found = true;
              } else {
                acc += v;
              }
            }
          }
          if (mode == 0 && !found) return 2;
          Y[(nc * OH + oh) * OW + ow] = D::st(mode == 0 ? acc : acc / denom);
        }
    return 0;
  });
}

// reference: src/backends/cpu/kernels/shape.cpp:72-165 — output linear index decoded to coordinates, input
// offset through the permuted strides, one element copied at a time.
int oracle_transpose(int itemsize, const void* x, void* y, int rank, const int64_t* in_dims, const int64_t* perm) {
  std::vector<int64_t> in_strides(static_cast<size_t>(rank), 1), out_dims(static_cast<size_t>(rank));
  for (int d = rank - 2; d >= 0; --d) in_strides[d] = in_strides[d + 1] * in_dims[d + 1];
  int64_t numel = 1;
  for (int d = 0; d < rank; ++d) {
    if (perm[d] < 0 || perm[d] >= rank) return 1;
    out_dims[d] = in_dims[perm[d]];
    numel *= out_dims[d];
  }
  const char* X = static_cast<const char*>(x);
  char* Y = static_cast<char*>(y);
  for (int64_t lin = 0; lin < numel; ++lin) {
    int64_t rem = lin, src = 0;
    for (int d = rank - 1; d >= 0; --d) {
      const int64_t c = rem % out_dims[d];
      rem /= out_dims[d];
      src += c * in_strides[perm[d]];
    }
    std::memcpy(Y + lin * itemsize, X + src * itemsize, static_cast<size_t>(itemsize));
  }
  return 0;
}

// reference: src/backends/cpu/kernels/shape.cpp:275-392 — outer x (width * inner) contiguous segments
int oracle_slice(int itemsize, const void* x, void* y, int rank, const int64_t* in_dims, int64_t axis, int64_t start,
                 int64_t stop) {
  if (axis < 0 || axis >= rank || start < 0 || stop < start || stop > in_dims[axis]) return 1;
  int64_t outer = 1, inner = 1;
  for (int d = 0; d < axis; ++d) outer *= in_dims[d];
  for (int d = static_cast<int>(axis) + 1; d < rank; ++d) inner *= in_dims[d];
  const int64_t width = stop - start;
  const char* X = static_cast<const char*>(x);
  char* Y = static_cast<char*>(y);
  for (int64_t o = 0; o < outer; ++o)
    std::memcpy(Y + (o * width * inner) * itemsize, X + (o * in_dims[axis] + start) * inner * itemsize,
                static_cast<size_t>(width * inner * itemsize));
  return 0;
}

// reference: src/backends/cpu/kernels/shape.cpp:170-270
int oracle_concat(int itemsize, const void* const* xs, int count, void* y, int rank, const int64_t* dims,
                  int64_t axis) {
  if (count < 1 || axis < 0 || axis >= rank) return 1;
  int64_t outer = 1, inner = 1, total_axis = 0;
  for (int d = 0; d < axis; ++d) outer *= dims[d];
  for (int d = static_cast<int>(axis) + 1; d < rank; ++d) inner *= dims[d];
  for (int t = 0; t < count; ++t) total_axis += dims[t * rank + axis];
  char* Y = static_cast<char*>(y);
  for (int64_t o = 0; o < outer; ++o) {
    int64_t off = 0;
    for (int t = 0; t < count; ++t) {
      const int64_t wdt = dims[t * rank + axis];
      std::memcpy(Y + ((o * total_axis + off) * inner) * itemsize,
                  static_cast<const char*>(xs[t]) + (o * wdt * inner) * itemsize,
                  static_cast<size_t>(wdt * inner * itemsize));
      off += wdt;
    }
  }
  return 0;
}

// reference: src/ops/constant_utils.cpp (fill_tensor_from_constant_attrs): one value per element, double -> float
// -> storage rounding.
int oracle_constant(int dtype, const double* values, int64_t nvalues, void* out, int64_t numel) {
  if (nvalues != numel) return 1;
  return with_dtype(dtype, [&](auto d) {
    using D = decltype(d);
    for (int64_t i = 0; i < numel; ++i) static_cast<typename D::S*>(out)[i] = D::st(static_cast<float>(values[i]));
    return 0;
  });
}

}  // extern "C"

// ---- training path ----------------------------------------------------------------------------------------
extern "C" {

// reference: src/backends/cpu/kernels/matmul.cpp:187-231 (lhs: ga[i,p] = sum_j gy[i,j]*b[p,j]) and :285-327
// (rhs: gb[p,j] = sum_i a[i,p]*gy[i,j]); float accumulator, contraction index ascending, one rounding at the store.
int oracle_matmul_grad(int dtype, int rhs, const void* p, const void* q, void* out, int64_t m, int64_t n, int64_t k) {
  return with_dtype(dtype, [&](auto d) {
    using D = decltype(d);
    using S = typename D::S;
    const S* P = static_cast<const S*>(p);
    const S* Q = static_cast<const S*>(q);
    S* O = static_cast<S*>(out);
    if (!rhs) {  // P = gy [m,n], Q = b [k,n] -> [m,k]
      for (int64_t i = 0; i < m; ++i)
        for (int64_t c = 0; c < k; ++c) {
          float acc = 0.0f;
          for (int64_t j = 0; j < n; ++j) acc += D::ld(P[i * n + j]) * D::ld(Q[c * n + j]);
          O[i * k + c] = D::st(acc);
        }
    } else {  // P = a [m,k], Q = gy [m,n] -> [k,n]
      for (int64_t c = 0; c < k; ++c)
        for (int64_t j = 0; j < n; ++j) {
          float acc = 0.0f;
          for (int64_t i = 0; i < m; ++i) acc += D::ld(P[i * k + c]) * D::ld(Q[i * n + j]);
          O[c * n + j] = D::st(acc);
        }
    }
    return 0;
  });
}

// reference: src/backends/cpu/kernels/conv.cpp:320-352. Per input element, products over co (of its group), kh,
// kw ascending, taking only taps where (ih + pad - kh) is a multiple of the stride and lands inside dy.
int oracle_conv2d_grad_input(int dtype, const void* dy, const void* w, void* dx, const int64_t* geom) {
  ConvG p;
  if (!read_conv(geom, p)) return 1;
  return with_dtype(dtype, [&](auto d) {
    using D = decltype(d);
    using S = typename D::S;
    const S* DY = static_cast<const S*>(dy);
    const S* Wt = static_cast<const S*>(w);
    S* DX = static_cast<S*>(dx);
    const int64_t cin_g = p.cin / p.groups, cout_g = p.cout / p.groups;
    for (int64_t n = 0; n < p.n; ++n)
      for (int64_t cf = 0; cf < p.cin; ++cf) {
        const int64_t g = cf / cin_g, ci = cf - g * cin_g;
        for (int64_t ih = 0; ih < p.h; ++ih)
          for (int64_t iw = 0; iw < p.w; ++iw) {
            float acc = 0.0f;
            for (int64_t co = g * cout_g; co < (g + 1) * cout_g; ++co)
              for (int64_t a = 0; a < p.kh; ++a) {
                const int64_t nh = ih + p.ph - a;
                if (nh % p.sh != 0) continue;
                const int64_t oh = nh / p.sh;
                if (oh < 0 || oh >= p.oh) continue;
                for (int64_t b = 0; b < p.kw; ++b) {
                  const int64_t nw = iw + p.pw - b;
                  if (nw % p.sw != 0) continue;
                  const int64_t ow = nw / p.sw;
                  if (ow < 0 || ow >= p.ow) continue;
                  acc += D::ld(DY[((n * p.cout + co) * p.oh + oh) * p.ow + ow]) *
                         D::ld(Wt[((co * cin_g + ci) * p.kh + a) * p.kw + b]);
                }
              }
            DX[((n * p.cin + cf) * p.h + ih) * p.w + iw] = D::st(acc);
          }
      }
    return 0;
  });
}

// reference: src/backends/cpu/kernels/conv.cpp:423-451. Per filter element, products over n, oh, ow ascending,
// skipping taps in the padding.
int oracle_conv2d_grad_filter(int dtype, const void* x, const void* dy, void* dw, const int64_t* geom) {
  ConvG p;
  if (!read_conv(geom, p)) return 1;
  return with_dtype(dtype, [&](auto d) {
    using D = decltype(d);
    using S = typename D::S;
    const S* X = static_cast<const S*>(x);
    const S* DY = static_cast<const S*>(dy);
    S* DW = static_cast<S*>(dw);
    const int64_t cin_g = p.cin / p.groups, cout_g = p.cout / p.groups;
    for (int64_t co = 0; co < p.cout; ++co) {
      const int64_t g = co / cout_g;
      for (int64_t ci = 0; ci < cin_g; ++ci)
        for (int64_t a = 0; a < p.kh; ++a)
          for (int64_t b = 0; b < p.kw; ++b) {
            float acc = 0.0f;
            for (int64_t n = 0; n < p.n; ++n)
              for (int64_t oh = 0; oh < p.oh; ++oh) {
                const int64_t ih = oh * p.sh - p.ph + a;
                if (ih < 0 || ih >= p.h) continue;
                for (int64_t ow = 0; ow < p.ow; ++ow) {
                  const int64_t iw = ow * p.sw - p.pw + b;
                  if (iw < 0 || iw >= p.w) continue;
                  acc += D::ld(X[((n * p.cin + g * cin_g + ci) * p.h + ih) * p.w + iw]) *
                         D::ld(DY[((n * p.cout + co) * p.oh + oh) * p.ow + ow]);
                }
              }
            DW[((co * cin_g + ci) * p.kh + a) * p.kw + b] = D::st(acc);
          }
    }
    return 0;
  });
}

// mode 0 = max_pool2d_grad_internal (reference: src/backends/cpu/kernels/pool.cpp:186-206 window argmax, first
// strict maximum in (kh, kw) order; :358-388 windows in (n, c, oh, ow) order add dy into a float buffer at the
// argmax, one rounding at the end). mode 1 = avg_pool2d_grad_internal (:543-566: per input element, kh then kw
// ascending over covering windows, sum of dy, then / (KH*KW)). geom as oracle_pool2d (input dims).
int oracle_pool2d_grad(int dtype, int mode, const void* dy, const void* x, void* dx, const int64_t* g) {
  const int64_t N = g[0], C = g[1], H = g[2], W = g[3], KH = g[4], KW = g[5], SH = g[6], SW = g[7], PH = g[8],
                PW = g[9];
  if (SH <= 0 || SW <= 0 || KH <= 0 || KW <= 0) return 1;
  const int64_t OH = (H + 2 * PH - KH) / SH + 1, OW = (W + 2 * PW - KW) / SW + 1;
  return with_dtype(dtype, [&](auto d) {
    using D = decltype(d);
    using S = typename D::S;
    const S* DY = static_cast<const S*>(dy);
    const S* X = static_cast<const S*>(x);
    S* DX = static_cast<S*>(dx);
    if (mode == 0) {
      std::vector<float> acc(static_cast<size_t>(N * C * H * W), 0.0f);
      for (int64_t nc = 0; nc < N * C; ++nc)
        for (int64_t oh = 0; oh < OH; ++oh)
          for (int64_t ow = 0; ow < OW; ++ow) {
            bool found = false;
            float best = 0.0f;
            int64_t at = 0;
            for (int64_t a = 0; a < KH; ++a) {
              const int64_t ih = oh * SH - PH + a;
              if (ih < 0 || ih >= H) continue;
              for (int64_t b = 0; b < KW; ++b) {
                const int64_t iw = ow * SW - PW + b;
                if (iw < 0 || iw >= W) continue;
                const float v = D::ld(X[(nc * H + ih) * W + iw]);
                if (!found || v > best) {
                  found = true;
                  best = v;
                  at = ih * W + iw;
                }
              }
            }
            if (!found) return 2;
            acc[static_cast<size_t>(nc * H * W + at)] += D::ld(DY[(nc * OH + oh) * OW + ow]);
          }
      for (size_t i = 0; i < acc.size(); ++i) DX[i] = D::st(acc[i]);
      return 0;
    }
    const float denom = static_cast<float>(KH * KW);
    for (int64_t nc = 0; nc < N * C; ++nc)
      for (int64_t ih = 0; ih < H; ++ih)
        for (int64_t iw = 0; iw < W; ++iw) {
          float acc = 0.0f;
          for (int64_t a = 0; a < KH; ++a) {
            const int64_t nh = ih + PH - a;
            if (nh % SH != 0) continue;
            const int64_t oh = nh / SH;
            if (oh < 0 || oh >= OH) continue;
            for (int64_t b = 0; b < KW; ++b) {
              const int64_t nw = iw + PW - b;
              if (nw % SW != 0) continue;
              const int64_t ow = nw / SW;
              if (ow < 0 || ow >= OW) continue;
              acc += D::ld(DY[(nc * OH + oh) * OW + ow]);
            }
          }
          DX[(nc * H + ih) * W + iw] = D::st(acc / denom);
        }
    return 0;
  });
}

namespace {
// Linear index of x's element `i` in the reduced tensor (reduced axes dropped; reference:
// src/backends/cpu/kernels/reduction.cpp:87-116).
int64_t project(int rank, const int64_t* dims, const uint8_t* reduced, int64_t i) {
  int64_t out = 0, stride = 1;
  for (int d = rank - 1; d >= 0; --d) {
    const int64_t sz = dims[d] > 0 ? dims[d] : 1;
    const int64_t c = i % sz;
    i /= sz;
    if (!reduced[d]) {
      out += c * stride;
      stride *= dims[d];
    }
  }
  return out;
}
}  // namespace

// reference: src/backends/cpu/kernels/reduction.cpp:215-241 — one float accumulator per output, x visited in
// row-major order, one rounding per output. reduced[d] != 0 marks a reduced axis (every axis for axes = []).
int oracle_sum(int dtype, const void* x, void* out, int rank, const int64_t* dims, const uint8_t* reduced) {
  int64_t numel = 1, nout = 1;
  for (int d = 0; d < rank; ++d) {
    numel *= dims[d];
    if (!reduced[d]) nout *= dims[d];
  }
  return with_dtype(dtype, [&](auto dd) {
    using D = decltype(dd);
    using S = typename D::S;
    const S* X = static_cast<const S*>(x);
    S* O = static_cast<S*>(out);
    std::vector<float> acc(static_cast<size_t>(nout), 0.0f);
    for (int64_t i = 0; i < numel; ++i) acc[static_cast<size_t>(project(rank, dims, reduced, i))] += D::ld(X[i]);
    for (int64_t j = 0; j < nout; ++j) O[j] = D::st(acc[static_cast<size_t>(j)]);
    return 0;
  });
}

// reference: src/backends/cpu/kernels/reduction.cpp:378-388 — gx[i] = gy[project(i)], a bit copy.
int oracle_sum_grad(int itemsize, const void* gy, void* gx, int rank, const int64_t* dims, const uint8_t* reduced) {
  int64_t numel = 1;
  for (int d = 0; d < rank; ++d) numel *= dims[d];
  const auto* G = static_cast<const unsigned char*>(gy);
  auto* O = static_cast<unsigned char*>(gx);
  for (int64_t i = 0; i < numel; ++i)
    std::memcpy(O + i * itemsize, G + project(rank, dims, reduced, i) * itemsize, static_cast<size_t>(itemsize));
  return 0;
}

// reference: src/backends/cpu/kernels/loss.cpp:110-147 — sum of (p - t)^2 in index order, then / numel, one rounding.
int oracle_mse_loss(int dtype, const void* pred, const void* target, void* out, int64_t numel) {
  if (numel <= 0) return 1;
  return with_dtype(dtype, [&](auto d) {
    using D = decltype(d);
    using S = typename D::S;
    const S* P = static_cast<const S*>(pred);
    const S* T = static_cast<const S*>(target);
    float acc = 0.0f;
    for (int64_t i = 0; i < numel; ++i) {
      const float diff = D::ld(P[i]) - D::ld(T[i]);
      acc += diff * diff;
    }
    static_cast<S*>(out)[0] = D::st(acc / static_cast<float>(numel));
    return 0;
  });
}

// reference: src/backends/cpu/kernels/loss.cpp:230-262 — c = 2 * gy / numel (in that order), out = c * (p - t).
int oracle_mse_loss_grad(int dtype, const void* pred, const void* target, const void* gy, void* out, int64_t numel) {
  if (numel <= 0) return 1;
  return with_dtype(dtype, [&](auto d) {
    using D = decltype(d);
    using S = typename D::S;
    const S* P = static_cast<const S*>(pred);
    const S* T = static_cast<const S*>(target);
    const float c = 2.0f * D::ld(static_cast<const S*>(gy)[0]) / static_cast<float>(numel);
    S* O = static_cast<S*>(out);
    for (int64_t i = 0; i < numel; ++i) O[i] = D::st(c * (D::ld(P[i]) - D::ld(T[i])));
    return 0;
  });
}

}  // extern "C"
