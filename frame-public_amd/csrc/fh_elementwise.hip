// Memory-bound kernels: the one-pass fused elementwise program, fills and data movement
// (strided 2-D copies for slice/concat/reshape and the gather permute for transpose).
//
// The elementwise program reproduces Frame's fused_elementwise_internal semantics
// (reference: src/ops/fused_elementwise_utils.cpp:122-206): segment 0 takes its inputs from the external
// list, every later segment takes the previous result as input 0 and its remaining inputs from the external
// list in order; each segment's result is rounded to the storage dtype (the unfused graph stores every
// intermediate). Unlike the reference there is one pass over memory: every external input is read once
// and the result written once.
#include <hip/hip_runtime.h>

#include <string>
#include <utility>

#include "fh_common.h"

namespace fh {
namespace {

struct EwArgs {
  int32_t nseg;
  int32_t round_between;
  uint8_t ops[FH_MAX_SEGMENTS];
  int8_t arities[FH_MAX_SEGMENTS];
  const void* ins[FH_MAX_EW_INPUTS];
  void* out;
  int64_t numel;
};

constexpr int kEwThreads = 256;

// Evaluates the program on V consecutive elements starting at element `base`.
template <typename T, int V>
__device__ __forceinline__ void ew_eval(const EwArgs& a, int64_t base) {
  using S = typename Io<T>::storage;
  struct alignas(V * sizeof(S)) Vec {
    S e[V];
  };
  float v[V];
  int next_in = 0;
  for (int s = 0; s < a.nseg; ++s) {
    const uint8_t op = a.ops[s];
    const int arity = a.arities[s];
    if (s == 0) {
      const Vec x = *reinterpret_cast<const Vec*>(static_cast<const S*>(a.ins[0]) + base);
#pragma unroll
      for (int e = 0; e < V; ++e) v[e] = Io<T>::load(x.e[e]);
      next_in = 1;
      if (arity == 2) {
        const Vec y = *reinterpret_cast<const Vec*>(static_cast<const S*>(a.ins[1]) + base);
#pragma unroll
        for (int e = 0; e < V; ++e) v[e] = ew_binary(op, v[e], Io<T>::load(y.e[e]));
        next_in = 2;
      } else {
#pragma unroll
        for (int e = 0; e < V; ++e) v[e] = ew_unary(op, v[e]);
      }
    } else if (arity == 2) {
      const Vec y = *reinterpret_cast<const Vec*>(static_cast<const S*>(a.ins[next_in]) + base);
      ++next_in;
#pragma unroll
      for (int e = 0; e < V; ++e) v[e] = ew_binary(op, v[e], Io<T>::load(y.e[e]));
    } else {
#pragma unroll
      for (int e = 0; e < V; ++e) v[e] = ew_unary(op, v[e]);
    }
    if (a.round_between) {
#pragma unroll
      for (int e = 0; e < V; ++e) v[e] = Io<T>::round(v[e]);
    }
  }
  Vec out;
#pragma unroll
  for (int e = 0; e < V; ++e) out.e[e] = Io<T>::store(v[e]);
  *reinterpret_cast<Vec*>(static_cast<S*>(a.out) + base) = out;
}

// V elements per thread per step, 16-byte accesses for V*sizeof(S) == 16. The scalar tail is handled by
// the first threads of the grid.
template <typename T, int V>
__global__ __launch_bounds__(kEwThreads) void ew_program_kernel(EwArgs a) {
  const int64_t nvec = a.numel / V;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kEwThreads;
  int64_t i = static_cast<int64_t>(blockIdx.x) * kEwThreads + threadIdx.x;
  for (; i < nvec; i += stride) ew_eval<T, V>(a, i * V);
  if (V > 1) {
    const int64_t tail_start = nvec * V;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kEwThreads + threadIdx.x;
    if (tail_start + t < a.numel) ew_eval<T, 1>(a, tail_start + t);
  }
}

// ---- fast path: 16-byte vectors, NIN external inputs known at compile time ----------------------------------
// Per vector: the NIN input loads are issued first (non-temporal: each element is read once), then the program
// runs with the segment switch outside the element loop, then one non-temporal 16-byte store. Rounding between
// segments is skipped where it is provably the identity: after the last segment (the store rounds) and after
// relu of an already rounded value (relu returns its input or zero, both representable).
typedef unsigned int ew_u4 __attribute__((ext_vector_type(4)));

template <typename T>
struct Lanes;
template <>
struct Lanes<float> {
  static constexpr int V = 4;
  __device__ static void unpack(const ew_u4& w, float (&v)[4]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = __uint_as_float(w[e]);
  }
  __device__ static ew_u4 pack(const float (&v)[4]) {
    return ew_u4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])};
  }
  __device__ static void round(float (&)[4]) {}
};
template <>
struct Lanes<bf16_t> {
  static constexpr int V = 8;
  __device__ static void unpack(const ew_u4& w, float (&v)[8]) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      v[2 * d] = __uint_as_float(w[d] << 16);
      v[2 * d + 1] = __uint_as_float(w[d] & 0xffff0000u);
    }
  }
  // two floats -> one packed pair with a single v_cvt_pk_bf16_f32 (the hardware narrowing, see fh_common.h)
  __device__ static uint32_t pack2(float lo, float hi) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{lo, hi}, b2));
  }
  __device__ static ew_u4 pack(const float (&v)[8]) {
    ew_u4 w;
#pragma unroll
    for (int d = 0; d < 4; ++d) w[d] = pack2(v[2 * d], v[2 * d + 1]);
    return w;
  }
  __device__ static void round(float (&v)[8]) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t p = pack2(v[2 * d], v[2 * d + 1]);
      v[2 * d] = __uint_as_float(p << 16);
      v[2 * d + 1] = __uint_as_float(p & 0xffff0000u);
    }
  }
};
template <>
struct Lanes<f16_t> {
  static constexpr int V = 8;
  __device__ static void unpack(const ew_u4& w, float (&v)[8]) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      v[2 * d] = f16_bits_to_float(static_cast<uint16_t>(w[d] & 0xffffu));
      v[2 * d + 1] = f16_bits_to_float(static_cast<uint16_t>(w[d] >> 16));
    }
  }
  __device__ static ew_u4 pack(const float (&v)[8]) {
    ew_u4 w;
#pragma unroll
    for (int d = 0; d < 4; ++d)
      w[d] = static_cast<uint32_t>(float_to_f16_bits(v[2 * d])) | (static_cast<uint32_t>(float_to_f16_bits(v[2 * d + 1])) << 16);
    return w;
  }
  __device__ static void round(float (&v)[8]) {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = Io<f16_t>::round(v[e]);
  }
};

// The segment op codes as one scalar word: a runtime-indexed a.ops[s] becomes a per-iteration vector load of the
// kernel argument followed by a vmcnt(0) wait, which also drains the in-flight input loads.
__device__ __forceinline__ uint64_t ops_as_word(const EwArgs& a) {
  uint64_t w;
  __builtin_memcpy(&w, a.ops, sizeof(w));
  static_assert(sizeof(a.ops) == sizeof(w), "eight one-byte op codes");
  return w;
}

// Issues the NIN input loads of vector i. The empty asm statements take the loaded registers as operands, so all
// NIN loads are issued before the first wait (the compiler would otherwise sink a load to its first use). Plain
// (temporal) accesses: measured on MI355X for add;relu bf16 [64,64,56,56] with inputs rotated past the MALL,
// two vectors per thread in flight with plain loads and stores reach 5.72 TB/s, a plain copy of the same bytes
// 5.81 TB/s, and the non-temporal forms 5.45-5.67 TB/s.
template <int NIN>
__device__ __forceinline__ void ew_load(const EwArgs& a, int64_t i, ew_u4 (&in)[NIN]) {
#pragma unroll
  for (int k = 0; k < NIN; ++k) in[k] = static_cast<const ew_u4*>(a.ins[k])[i];
}

template <int NIN>
__device__ __forceinline__ void ew_issued(ew_u4 (&in)[NIN]) {
#pragma unroll
  for (int k = 0; k < NIN; ++k) asm volatile("" : "+v"(in[k]));
}

template <typename T, int NIN>
__global__ __launch_bounds__(kEwThreads) void ew_vec_kernel(EwArgs a) {
  using L = Lanes<T>;
  constexpr int V = L::V;
  const uint64_t ops_word = ops_as_word(a);
  const int64_t nvec = a.numel / V;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kEwThreads;
  int64_t i = static_cast<int64_t>(blockIdx.x) * kEwThreads + threadIdx.x;
  // one vector of look-ahead: the next grid-stride vector's loads are in flight while this one is computed
  ew_u4 cur[NIN], nxt[NIN];
  if (i < nvec) ew_load<NIN>(a, i, cur);
  for (; i < nvec; i += stride) {
    // unconditional (index clamped to the last vector, result unused past the end): a load under a per-lane
    // condition would make the wait counts unknowable and force a wait for every outstanding load
    ew_load<NIN>(a, min(i + stride, nvec - 1), nxt);
    ew_issued<NIN>(cur);
    float v[V], w[V];
    L::unpack(cur[0], v);
    int next = 1;
    bool rounded = true;  // v holds storage-representable values (it starts as a loaded input)
    for (int s = 0; s < a.nseg; ++s) {
      const uint8_t op = static_cast<uint8_t>(ops_word >> (8 * s));
      const bool last = s + 1 == a.nseg;
      switch (op) {
        case FH_EW_ADD:
        case FH_EW_MUL:
        case FH_EW_RELU_GRAD:
        case FH_EW_GELU_GRAD:
        case FH_EW_RELU_MASK: {
          ew_u4 t = cur[0];
#pragma unroll
          for (int k = 1; k < NIN; ++k)
            if (k == next) t = cur[k];
          ++next;
          L::unpack(t, w);
          if (op == FH_EW_ADD) {
#pragma unroll
            for (int e = 0; e < V; ++e) v[e] = v[e] + w[e];
          } else if (op != FH_EW_MUL) {
#pragma unroll
            for (int e = 0; e < V; ++e) v[e] = ew_binary(op, v[e], w[e]);
          } else {
#pragma unroll
            for (int e = 0; e < V; ++e) v[e] = v[e] * w[e];
          }
          rounded = false;
          break;
        }
        case FH_EW_RELU:
#pragma unroll
          for (int e = 0; e < V; ++e) v[e] = (v[e] < 0.0f) ? 0.0f : v[e];
          break;  // relu of a rounded value is rounded
        default:
#pragma unroll
          for (int e = 0; e < V; ++e) v[e] = ew_unary(op, v[e]);
          rounded = false;
          break;
      }
      if (a.round_between && !last && !rounded) {
        L::round(v);
        rounded = true;
      }
    }
    static_cast<ew_u4*>(a.out)[i] = L::pack(v);
#pragma unroll
    for (int k = 0; k < NIN; ++k) cur[k] = nxt[k];
  }
  // scalar tail (numel % V elements) on the first threads of the grid
  const int64_t tail_start = nvec * V;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kEwThreads + threadIdx.x;
  if (tail_start + t < a.numel) ew_eval<T, 1>(a, tail_start + t);
}

// Programs known at compile time (the common fused groups): no segment loop, no op switch, each segment's
// input fixed. OPS are fh_ew_op codes; NIN = 1 + the number of binary segments.
template <uint8_t... OPS>
constexpr int ew_inputs() {
  return 1 + ((ew_is_binary(OPS) ? 1 : 0) + ... + 0);
}

template <typename T, uint8_t... OPS>
__global__ __launch_bounds__(kEwThreads) void ew_fixed_kernel(EwArgs a) {
  using L = Lanes<T>;
  constexpr int V = L::V;
  constexpr int NIN = ew_inputs<OPS...>();
  constexpr uint8_t ops[] = {OPS...};
  constexpr int NSEG = sizeof...(OPS);
  const int64_t nvec = a.numel / V;
  // two vectors per thread and iteration (i and i + kEwThreads), all their loads issued before any use
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kEwThreads * 2;
  for (int64_t i0 = static_cast<int64_t>(blockIdx.x) * kEwThreads * 2 + threadIdx.x; i0 < nvec; i0 += stride) {
    ew_u4 in2[2][NIN];
    // unconditional (the second index clamped to the last vector, its result unused past the end): a load under a
    // per-lane condition would make the wait counts unknowable and force a wait for every outstanding load
    ew_load<NIN>(a, i0, in2[0]);
    ew_load<NIN>(a, min(i0 + kEwThreads, nvec - 1), in2[1]);
    ew_issued<NIN>(in2[0]);
    ew_issued<NIN>(in2[1]);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
    const int64_t i = i0 + u * kEwThreads;
    if (u == 1 && i >= nvec) break;
    ew_u4 (&cur)[NIN] = in2[u];
    float v[V], w[V];
    L::unpack(cur[0], v);
    [&]<int... S>(std::integer_sequence<int, S...>) {
      (
          [&] {
            constexpr uint8_t op = ops[S];
            constexpr bool binary = ew_is_binary(op);
            // input of segment S: 1 + the binary segments before it
            constexpr int in_idx = [] {
              int n = 1;
              for (int q = 0; q < S; ++q) n += ew_is_binary(ops[q]) ? 1 : 0;
              return n;
            }();
            if constexpr (binary) {
              L::unpack(cur[in_idx], w);
#pragma unroll
              for (int e = 0; e < V; ++e)
                v[e] = op == FH_EW_ADD ? v[e] + w[e] : op == FH_EW_MUL ? v[e] * w[e] : ew_binary(op, v[e], w[e]);
            } else if constexpr (op == FH_EW_RELU) {
#pragma unroll
              for (int e = 0; e < V; ++e) v[e] = (v[e] < 0.0f) ? 0.0f : v[e];
            } else {
#pragma unroll
              for (int e = 0; e < V; ++e) v[e] = ew_unary(op, v[e]);
            }
            // Rounded after every segment but the last (the store rounds). Every segment's input is representable
            // (a loaded value or a rounded / relu'd result), and relu returns its input or zero, so rounding after
            // relu is the identity as well.
            constexpr bool skip = S + 1 == NSEG || op == FH_EW_RELU;
            if constexpr (!skip) L::round(v);
          }(),
          ...);
    }(std::make_integer_sequence<int, NSEG>{});
    static_cast<ew_u4*>(a.out)[i] = L::pack(v);
    }
  }
  const int64_t tail_start = nvec * V;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kEwThreads + threadIdx.x;
  if (tail_start + t < a.numel) ew_eval<T, 1>(a, tail_start + t);
}

// Launches the compile-time kernel for a.ops when it is one of the common programs; false otherwise.
template <typename T>
bool launch_fixed(const EwArgs& a, dim3 grid, hipStream_t stream) {
  const uint8_t o0 = a.ops[0], o1 = a.nseg > 1 ? a.ops[1] : 0;
#define FH_EW_FIXED(...)                                                                       \
  do {                                                                                         \
    hipLaunchKernelGGL((ew_fixed_kernel<T, __VA_ARGS__>), grid, dim3(kEwThreads), 0, stream, a); \
    return true;                                                                               \
  } while (0)
  if (a.nseg == 1) {
    switch (o0) {
      case FH_EW_ADD: FH_EW_FIXED(FH_EW_ADD);
      case FH_EW_MUL: FH_EW_FIXED(FH_EW_MUL);
      case FH_EW_RELU: FH_EW_FIXED(FH_EW_RELU);
      case FH_EW_GELU: FH_EW_FIXED(FH_EW_GELU);
      case FH_EW_SQUARE: FH_EW_FIXED(FH_EW_SQUARE);
      case FH_EW_RELU_GRAD: FH_EW_FIXED(FH_EW_RELU_GRAD);
      case FH_EW_GELU_GRAD: FH_EW_FIXED(FH_EW_GELU_GRAD);
      case FH_EW_SIGMOID: FH_EW_FIXED(FH_EW_SIGMOID);
      case FH_EW_TANH: FH_EW_FIXED(FH_EW_TANH);
      case FH_EW_RSQRT: FH_EW_FIXED(FH_EW_RSQRT);
      default: return false;
    }
  }
  if (a.nseg == 2) {
    if (o0 == FH_EW_ADD && o1 == FH_EW_RELU) FH_EW_FIXED(FH_EW_ADD, FH_EW_RELU);
    if (o0 == FH_EW_ADD && o1 == FH_EW_GELU) FH_EW_FIXED(FH_EW_ADD, FH_EW_GELU);
    if (o0 == FH_EW_ADD && o1 == FH_EW_ADD) FH_EW_FIXED(FH_EW_ADD, FH_EW_ADD);
    if (o0 == FH_EW_MUL && o1 == FH_EW_ADD) FH_EW_FIXED(FH_EW_MUL, FH_EW_ADD);
    if (o0 == FH_EW_ADD && o1 == FH_EW_RELU_MASK) FH_EW_FIXED(FH_EW_ADD, FH_EW_RELU_MASK);
  }
#undef FH_EW_FIXED
  return false;
}

template <typename T>
fh_status launch_ew(const EwArgs& a, hipStream_t stream) {
  using S = typename Io<T>::storage;
  constexpr int V = 16 / sizeof(S);
  bool aligned = reinterpret_cast<uintptr_t>(a.out) % 16 == 0;
  int nin = 0;
  for (int s = 0; s < a.nseg; ++s) nin += (s == 0) ? a.arities[s] : a.arities[s] - 1;
  for (int k = 0; k < nin; ++k) aligned = aligned && (reinterpret_cast<uintptr_t>(a.ins[k]) % 16 == 0);
  const int64_t per_thread = aligned ? V : 1;
  const int64_t work = (a.numel + per_thread - 1) / per_thread;
  int64_t blocks = (work + kEwThreads - 1) / kEwThreads;
  const int64_t cap = static_cast<int64_t>(device_cu_count()) * 16;  // measured best for 25-100 MB operands
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  const dim3 grid(static_cast<uint32_t>(blocks));
  // compile-time programs need round_between (always set for 16-bit storage; rounding is the identity for fp32)
  if (aligned && (a.round_between || sizeof(S) == 4) && launch_fixed<T>(a, grid, stream)) {
    // launched
  } else if (aligned && nin >= 1 && nin <= 3) {
    switch (nin) {
      case 1:
        hipLaunchKernelGGL((ew_vec_kernel<T, 1>), grid, dim3(kEwThreads), 0, stream, a);
        break;
      case 2:
        hipLaunchKernelGGL((ew_vec_kernel<T, 2>), grid, dim3(kEwThreads), 0, stream, a);
        break;
      default:
        hipLaunchKernelGGL((ew_vec_kernel<T, 3>), grid, dim3(kEwThreads), 0, stream, a);
        break;
    }
  } else if (aligned) {
    hipLaunchKernelGGL((ew_program_kernel<T, V>), grid, dim3(kEwThreads), 0, stream, a);
  } else {
    hipLaunchKernelGGL((ew_program_kernel<T, 1>), grid, dim3(kEwThreads), 0, stream, a);
  }
  return launch_status("ew kernel launch");
}

// ---------------------------------------------------------------------------------------------
template <typename W>
__global__ void fill_kernel(W* dst, W value, int64_t count) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride)
    dst[i] = value;
}

// Row copy: each block copies rows; bytes moved in 16-byte units when both pitches and pointers allow.
template <typename W>
__global__ void copy2d_kernel(char* dst, int64_t dpitch, const char* src, int64_t spitch, int64_t wunits,
                              int64_t rows) {
  const int64_t total = wunits * rows;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t r = i / wunits, c = i % wunits;
    reinterpret_cast<W*>(dst + r * dpitch)[c] = reinterpret_cast<const W*>(src + r * spitch)[c];
  }
}

struct PermuteArgs {
  int32_t rank;
  int64_t out_dims[8];
  int64_t in_strides[8];
  int64_t numel;
};

template <typename W>
__global__ void permute_kernel(const W* __restrict__ x, W* __restrict__ y, PermuteArgs p) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < p.numel; i += stride) {
    int64_t rem = i, src = 0;
    for (int d = p.rank - 1; d >= 0; --d) {
      const int64_t coord = rem % p.out_dims[d];
      rem /= p.out_dims[d];
      src += coord * p.in_strides[d];
    }
    y[i] = x[src];
  }
}

// Rank-2 transpose through a 64x64 LDS tile: coalesced reads and writes on both sides.
template <typename W>
__global__ __launch_bounds__(256) void transpose2d_kernel(const W* __restrict__ x, W* __restrict__ y,
                                                          int64_t rows, int64_t cols) {
  __shared__ W tile[64][65];
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 64, c0 = static_cast<int64_t>(blockIdx.x) * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4) {
    const int64_t gr = r0 + r, gc = c0 + tx;
    if (gr < rows && gc < cols) tile[r][tx] = x[gr * cols + gc];
  }
  __syncthreads();
  for (int c = ty; c < 64; c += 4) {
    const int64_t gc = c0 + c, gr = r0 + tx;  // output row = input col
    if (gc < cols && gr < rows) y[gc * rows + gr] = tile[tx][c];
  }
}

int64_t grid_for(int64_t work, int64_t threads) {
  int64_t blocks = (work + threads - 1) / threads;
  const int64_t cap = static_cast<int64_t>(device_cu_count()) * 16;
  if (blocks > cap) blocks = cap;
  return blocks < 1 ? 1 : blocks;
}

}  // namespace
}  // namespace fh

using namespace fh;

extern "C" fh_status fh_ew_program(int32_t dtype, int32_t nseg, const uint8_t* ops, const int8_t* arities,
                                   const void* const* ins, int32_t nin, void* out, int64_t numel,
                                   int32_t round_between, void* stream) {
  if (!is_supported_float(dtype)) return fail(FH_UNIMPLEMENTED, "fh_ew_program: unsupported dtype");
  if (nseg < 1 || nseg > FH_MAX_SEGMENTS)
    return fail(FH_INVALID_ARGUMENT, "fh_ew_program: segment count out of range: " + std::to_string(nseg));
  if (ops == nullptr || arities == nullptr || ins == nullptr)
    return fail(FH_INVALID_ARGUMENT, "fh_ew_program: null argument");
  if (numel < 0) return fail(FH_INVALID_ARGUMENT, "fh_ew_program: negative numel");
  // empty tensors have no storage (null data): the program is still checked, nothing is launched
  if (out == nullptr && numel > 0) return fail(FH_INVALID_ARGUMENT, "fh_ew_program: null output");
  EwArgs a{};
  a.nseg = nseg;
  a.round_between = round_between;
  int expected = 0;
  for (int s = 0; s < nseg; ++s) {
    const uint8_t op = ops[s];
    if (op < FH_EW_ADD || op > FH_EW_RELU_MASK)
      return fail(FH_INVALID_ARGUMENT, "fh_ew_program: unknown op code " + std::to_string(op));
    const int want = ew_is_binary(op) ? 2 : 1;
    if (arities[s] != want)
      return fail(FH_INVALID_ARGUMENT, "fh_ew_program: segment " + std::to_string(s) + " arity " +
                                           std::to_string(arities[s]) + " does not match its op");
    a.ops[s] = op;
    a.arities[s] = arities[s];
    expected += (s == 0) ? arities[s] : arities[s] - 1;
  }
  if (expected != nin || nin > FH_MAX_EW_INPUTS)
    return fail(FH_INVALID_ARGUMENT, "fh_ew_program: arities imply " + std::to_string(expected) +
                                         " inputs, got " + std::to_string(nin));
  for (int k = 0; k < nin; ++k) {
    if (ins[k] == nullptr && numel > 0) return fail(FH_INVALID_ARGUMENT, "fh_ew_program: null input");
    a.ins[k] = ins[k];
  }
  a.out = out;
  a.numel = numel;
  if (numel == 0) return FH_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case FH_F32:
      return launch_ew<float>(a, s);
    case FH_BF16:
      return launch_ew<bf16_t>(a, s);
    default:
      return launch_ew<f16_t>(a, s);
  }
}

extern "C" fh_status fh_fill(void* dst, int32_t itemsize, uint64_t pattern, int64_t count, void* stream) {
  if (count < 0) return fail(FH_INVALID_ARGUMENT, "fh_fill: negative count");
  if (count == 0) return FH_OK;
  if (dst == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_fill: null destination");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>(grid_for(count, 256)));
  switch (itemsize) {
    case 1:
      hipLaunchKernelGGL(fill_kernel<uint8_t>, grid, dim3(256), 0, s, static_cast<uint8_t*>(dst),
                         static_cast<uint8_t>(pattern), count);
      break;
    case 2:
      hipLaunchKernelGGL(fill_kernel<uint16_t>, grid, dim3(256), 0, s, static_cast<uint16_t*>(dst),
                         static_cast<uint16_t>(pattern), count);
      break;
    case 4:
      hipLaunchKernelGGL(fill_kernel<uint32_t>, grid, dim3(256), 0, s, static_cast<uint32_t*>(dst),
                         static_cast<uint32_t>(pattern), count);
      break;
    case 8:
      hipLaunchKernelGGL(fill_kernel<uint64_t>, grid, dim3(256), 0, s, static_cast<uint64_t*>(dst), pattern,
                         count);
      break;
    default:
      return fail(FH_INVALID_ARGUMENT, "fh_fill: itemsize must be 1, 2, 4 or 8");
  }
  return launch_status("fill_kernel launch");
}

extern "C" fh_status fh_copy2d(void* dst, int64_t dst_pitch, const void* src, int64_t src_pitch,
                               int64_t width_bytes, int64_t rows, void* stream) {
  if (rows < 0 || width_bytes < 0) return fail(FH_INVALID_ARGUMENT, "fh_copy2d: negative size");
  if (rows == 0 || width_bytes == 0) return FH_OK;
  if (dst == nullptr || src == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_copy2d: null pointer");
  if (dst_pitch < width_bytes || src_pitch < width_bytes)
    return fail(FH_INVALID_ARGUMENT, "fh_copy2d: pitch smaller than width");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uintptr_t align_mask = reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src) |
                               static_cast<uintptr_t>(dst_pitch) | static_cast<uintptr_t>(src_pitch) |
                               static_cast<uintptr_t>(width_bytes);
  char* d = static_cast<char*>(dst);
  const char* sp = static_cast<const char*>(src);
  if (align_mask % 16 == 0) {
    const int64_t units = width_bytes / 16;
    hipLaunchKernelGGL(copy2d_kernel<uint4>, dim3(static_cast<uint32_t>(grid_for(units * rows, 256))), dim3(256),
                       0, s, d, dst_pitch, sp, src_pitch, units, rows);
  } else if (align_mask % 4 == 0) {
    const int64_t units = width_bytes / 4;
    hipLaunchKernelGGL(copy2d_kernel<uint32_t>, dim3(static_cast<uint32_t>(grid_for(units * rows, 256))),
                       dim3(256), 0, s, d, dst_pitch, sp, src_pitch, units, rows);
  } else if (align_mask % 2 == 0) {
    const int64_t units = width_bytes / 2;
    hipLaunchKernelGGL(copy2d_kernel<uint16_t>, dim3(static_cast<uint32_t>(grid_for(units * rows, 256))),
                       dim3(256), 0, s, d, dst_pitch, sp, src_pitch, units, rows);
  } else {
    hipLaunchKernelGGL(copy2d_kernel<uint8_t>, dim3(static_cast<uint32_t>(grid_for(width_bytes * rows, 256))),
                       dim3(256), 0, s, d, dst_pitch, sp, src_pitch, width_bytes, rows);
  }
  return launch_status("copy2d_kernel launch");
}

extern "C" fh_status fh_permute(int32_t itemsize, const void* x, void* y, int32_t rank, const int64_t* out_dims,
                                const int64_t* in_strides_permuted, void* stream) {
  if (rank < 0 || rank > 8) return fail(FH_INVALID_ARGUMENT, "fh_permute: rank must be in [0, 8]");
  if (rank > 0 && (out_dims == nullptr || in_strides_permuted == nullptr))
    return fail(FH_INVALID_ARGUMENT, "fh_permute: null shape arrays");
  PermuteArgs p{};
  p.rank = rank;
  p.numel = 1;
  for (int d = 0; d < rank; ++d) {
    if (out_dims[d] < 0) return fail(FH_INVALID_ARGUMENT, "fh_permute: negative dimension");
    p.out_dims[d] = out_dims[d];
    p.in_strides[d] = in_strides_permuted[d];
    p.numel *= out_dims[d];
  }
  if (p.numel == 0) return FH_OK;
  if (x == nullptr || y == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_permute: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  // rank-2 transpose (perm = [1, 0] on a dense input): tiled kernel.
  const bool is_t2 = rank == 2 && p.in_strides[0] == 1 && p.in_strides[1] == p.out_dims[0];
  const dim3 grid(static_cast<uint32_t>(grid_for(p.numel, 256)));
  if (is_t2) {
    const int64_t in_rows = p.out_dims[1], in_cols = p.out_dims[0];
    const dim3 g2(static_cast<uint32_t>((in_cols + 63) / 64), static_cast<uint32_t>((in_rows + 63) / 64));
    switch (itemsize) {
      case 2:
        hipLaunchKernelGGL(transpose2d_kernel<uint16_t>, g2, dim3(256), 0, s, static_cast<const uint16_t*>(x),
                           static_cast<uint16_t*>(y), in_rows, in_cols);
        return launch_status("transpose2d_kernel launch");
      case 4:
        hipLaunchKernelGGL(transpose2d_kernel<uint32_t>, g2, dim3(256), 0, s, static_cast<const uint32_t*>(x),
                           static_cast<uint32_t*>(y), in_rows, in_cols);
        return launch_status("transpose2d_kernel launch");
      default:
        break;
    }
  }
  switch (itemsize) {
    case 1:
      hipLaunchKernelGGL(permute_kernel<uint8_t>, grid, dim3(256), 0, s, static_cast<const uint8_t*>(x),
                         static_cast<uint8_t*>(y), p);
      break;
    case 2:
      hipLaunchKernelGGL(permute_kernel<uint16_t>, grid, dim3(256), 0, s, static_cast<const uint16_t*>(x),
                         static_cast<uint16_t*>(y), p);
      break;
    case 4:
      hipLaunchKernelGGL(permute_kernel<uint32_t>, grid, dim3(256), 0, s, static_cast<const uint32_t*>(x),
                         static_cast<uint32_t*>(y), p);
      break;
    case 8:
      hipLaunchKernelGGL(permute_kernel<uint64_t>, grid, dim3(256), 0, s, static_cast<const uint64_t*>(x),
                         static_cast<uint64_t*>(y), p);
      break;
    default:
      return fail(FH_INVALID_ARGUMENT, "fh_permute: itemsize must be 1, 2, 4 or 8");
  }
  return launch_status("permute_kernel launch");
}
