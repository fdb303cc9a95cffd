// The MI355X `hip` backend: HAL objects over the C ABI of libframe_hip_kernels.so (include/frame_hip_abi.h).
// Modelled on the plugin contract of the reference (include/frame/hal/backend.h:77-109); the design analog
// being replaced is src/backends/cuda/cuda_backend.{h,cpp}.
#pragma once

#include <cstddef>
#include <cstdint>
#include <deque>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <span>
#include <string>
#include <unordered_map>
#include <vector>

#include <frame/core/device.h>
#include <frame/core/status.h>
#include <frame/hal/allocator.h>
#include <frame/hal/backend.h>
#include <frame/hal/event.h>
#include <frame/hal/executable.h>
#include <frame/hal/stream.h>
#include <frame/ir/graph.h>
#include <frame/ops/kernel_registry.h>

#include "frame_hip_abi.h"

namespace frame::backends::hip {

// fh_status -> Status (the ABI's codes are frame::ErrorCode ordinals); the message comes from fh_last_error.
Status from_fh(fh_status code, std::string_view what);

#define FRAME_HIP_RETURN_IF_ERROR(expr, what)                                 \
  do {                                                                        \
    const fh_status frame_hip_st_ = (expr);                                   \
    if (frame_hip_st_ != FH_OK) return ::frame::backends::hip::from_fh(frame_hip_st_, (what)); \
  } while (0)

class HipStream final : public hal::Stream {
 public:
  HipStream(void* handle, int32_t device);
  ~HipStream() override;
  Status synchronize() override;
  Status record(hal::Event& event) override;
  Status wait(const hal::Event& event) override;
  void* native_handle() override { return handle_; }
  int32_t device() const { return device_; }
  // Process-unique, never reused (unlike the hipStream_t address): what executables key per-stream state by.
  uint64_t id() const { return id_; }

 private:
  void* handle_;
  int32_t device_;
  uint64_t id_;
};

// Whether the HipStream with this id still exists (ids of destroyed streams are never handed out again).
bool hip_stream_alive(uint64_t id);
// Calls fn(hipStream_t) for each live HipStream of `device` while holding the registry's lock (so none of them is
// destroyed meanwhile), until fn returns false; returns whether every call returned true.
bool for_each_live_stream(int32_t device, const std::function<bool(void*)>& fn);
// The id of `stream` if it is a live HipStream, else 0 (a stream of another backend): a lookup among the live
// HipStream objects, which needs no RTTI (the reference's sources are built without dynamic_cast / typeid).
uint64_t hip_stream_id(const hal::Stream& stream);

class HipEvent final : public hal::Event {
 public:
  HipEvent(void* handle, int32_t device) : handle_(handle), device_(device) {}
  ~HipEvent() override;
  bool query() const override;
  Status synchronize() override;
  void* handle() const { return handle_; }
  bool recorded() const { return recorded_; }
  void mark_recorded() { recorded_ = true; }

 private:
  void* handle_;
  int32_t device_;
  bool recorded_ = false;  // an event never recorded counts as complete
};

// Device memory with a size-class cache, so repeated runs do not call hipMalloc. deallocate() carries no stream
// (hal::Allocator), and kernels queued on any stream before the free may still read or write the block, so a
// freed block first goes to a pending list with a fence: an event recorded at the free on every live stream of the
// device and on the null stream. A request of that size class that finds no reusable block takes the oldest
// pending one after waiting for its fence's events (work queued after the free keeps running); a block freed
// while a stream was being captured has no fence and is released by one device-wide synchronisation, as is the
// whole pending list before a retry on out-of-memory. A block is therefore never handed out while work queued
// before its free can still touch it (the reference gets this from cudaFree, which synchronises on every free,
// src/backends/cuda/cuda_allocator.cpp:55-66).
class HipAllocator final : public hal::Allocator {
 public:
  explicit HipAllocator(int32_t device) : device_(device) {}
  ~HipAllocator() override;
  Result<void*> allocate(size_t bytes, size_t alignment) override;
  void deallocate(void* ptr) override;
  static constexpr size_t kGuaranteedAlignment = 256;

  // Bytes held by the cache (reusable + pending) and by live blocks; for tests of memory growth.
  struct Stats {
    size_t live_bytes = 0, cached_bytes = 0, pending_bytes = 0;
    uint64_t device_allocations = 0, device_syncs = 0, fence_waits = 0;
  };
  Stats stats();
  static size_t size_class(size_t bytes);

 private:
  struct PendingBlock {
    void* ptr;
    std::vector<void*> fence;  // events recorded at the free
    bool fenced;               // false: freed during a capture, released by a device-wide wait only
  };
  bool record_fence_locked(std::vector<void*>& fence);
  void recycle_fence_locked(std::vector<void*>& fence);
  Status release_pending_locked();               // device-wide wait, then every pending block -> reusable
  Result<void*> take_pending_locked(size_t cls);  // oldest pending block of the class once its fence passed
  int32_t device_;
  std::mutex mu_;
  std::unordered_map<void*, size_t> live_;                // pointer -> size class
  std::map<size_t, std::vector<void*>> free_lists_;       // size class -> reusable blocks
  std::map<size_t, std::deque<PendingBlock>> pending_;    // size class -> freed, oldest first
  std::vector<void*> event_pool_;                         // fence events ready for reuse
  Stats stats_;
};

// Test hooks behind the C API's frame_hip_run_tapped / frame_hip_executable_steps (no counterpart in the
// reference). `exe` must be an executable HipBackend::compile returned. Step i is the i-th non-input node of the
// lowered graph (frame_hip_lowered_text prints it).
struct HipStepTap {
  size_t step;    // plan step index
  size_t output;  // output index of that step
  void* host;     // destination, `bytes` long
  size_t bytes;   // must equal the output's size
};
Status hip_run_tapped(hal::Executable& exe, std::span<const Tensor> inputs, std::span<Tensor> outputs, hal::Stream& stream,
                      std::span<const HipStepTap> taps);
std::string hip_executable_steps(const hal::Executable& exe);

class HipBackend final : public hal::Backend {
 public:
  HipBackend();
  ~HipBackend() override;
  std::string_view name() const override { return kHipBackendName; }
  Result<int32_t> device_count() const override;
  Result<std::unique_ptr<hal::Stream>> create_stream(Device device) override;
  Result<std::unique_ptr<hal::Event>> create_event(Device device) override;
  hal::Allocator* allocator(Device device) override;
  Status copy(void* dst, Device dst_device, const void* src, Device src_device, size_t bytes,
              hal::Stream* stream) override;
  Result<std::unique_ptr<hal::Executable>> compile(const ir::Graph& graph, const hal::CompileOptions& options) override;
  Status launch(const hal::KernelInvocation& invocation, hal::Stream* stream) override;

 private:
  Status check_device(Device device) const;
  std::mutex mu_;
  std::vector<std::unique_ptr<HipAllocator>> allocators_;
};

// The stream handle a kernel enqueues on (nullptr = the device's null stream).
inline void* stream_handle(const ops::KernelContext& ctx) {
  return ctx.stream == nullptr ? nullptr : ctx.stream->native_handle();
}

// Internal op names produced by HipBackend::compile's lowering (never user-visible).
inline constexpr std::string_view kGemmEpilogueOp = "hip_matmul_epilogue_internal";
inline constexpr std::string_view kConvEpilogueOp = "hip_conv2d_epilogue_internal";
// Up to FH_GEMM_MAX_GROUPS matmuls (each optionally with the same epilogue program) that read one A operand, as one
// fh_gemm_grouped launch: inputs [A, B_0 .. B_{g-1}, epilogue operands of group 0, of group 1, ...], outputs C_0 ..
// C_{g-1}; attrs groups, ep_ops (possibly empty), any_order.
inline constexpr std::string_view kGemmGroupedOp = "hip_matmul_grouped_internal";
// [d0, d1, d2, d3] -> [d0, d2, d3, d1]: NCHW activations to NHWC, [Cout][Cin][KH][KW] filters to [Cout][KH][KW][Cin].
inline constexpr std::string_view kChannelsLastOp = "hip_channels_last_internal";
// conv2d (optionally with an epilogue program) on channels-last operands; output NCHW, or channels-last
// [N,Ho,Wo,Cout] with attribute out_nhwc = 1.
inline constexpr std::string_view kConvNhwcOp = "hip_conv2d_nhwc_internal";
// channels_last of up to kMultiMaxTensors tensors in one step (a graph's filters; each [d0,d1,d2,d3] ->
// [d0,d2,d3,d1] with d1*d2*d3 <= kMultiPlaneMax), see fh_transpose_planes_multi.
inline constexpr std::string_view kChannelsLastMultiOp = "hip_channels_last_multi_internal";
inline constexpr size_t kMultiMaxTensors = 32;
inline constexpr int64_t kMultiPlaneMax = 8192;
// max_pool2d / avg_pool2d on channels-last [N,H,W,C] activations (same attributes; see fh_pool2d_nhwc).
inline constexpr std::string_view kMaxPoolNhwcOp = "hip_max_pool2d_nhwc_internal";
inline constexpr std::string_view kAvgPoolNhwcOp = "hip_avg_pool2d_nhwc_internal";
// conv2d 7x7/2 (Cin <= 3, Cout 64) [-> relu] -> max_pool2d 3x3/2 as one launch, NCHW in and out (fh_conv2d_stem_pool):
// inputs x, w[, bias]; attrs stride, padding, groups (the conv's), kernel, pool_stride, pool_padding, relu.
inline constexpr std::string_view kConvStemPoolOp = "hip_conv2d_stem_pool_internal";
// Cin <= 8: x [N,C,H,W] -> [N,H,W,8] zero-padded; w [Cout,C,KH,KW] -> [Cout, K8] (see fh_conv_pack_*_c8).
inline constexpr std::string_view kPackInputC8Op = "hip_pack_input_c8_internal";
inline constexpr std::string_view kPackFilterC8Op = "hip_pack_filter_c8_internal";
// conv2d_grad_input_internal as a stride-1 convolution on the implicit-GEMM kernel: the flipped channels-last
// filter [Cin][KH][KW][Cout] (fh_conv_filter_flip) and dy zero-dilated by the stride into channels-last
// [N,Hu,Wu,Cout] (fh_dilate_nhwc; attribute stride).
inline constexpr std::string_view kFilterFlipOp = "hip_conv_filter_flip_internal";
// the flips of up to FH_FLIP_MAX filters in one launch (fh_conv_filter_flip_multi): input i w_i [Cout,Cin,KH,KW],
// output i [Cin,KH,KW,Cout]
inline constexpr std::string_view kFilterFlipMultiOp = "hip_conv_filter_flip_multi_internal";
inline constexpr std::string_view kDilateNhwcOp = "hip_dilate_nhwc_internal";  // attr in_nhwc = 1: dy channels-last
// relu_grad_internal(x, max_pool2d_grad_internal(dy, x)) as one launch (fh_pool2d_grad mode 2): inputs dy, x and
// the pool gradient's attributes
inline constexpr std::string_view kMaxPoolReluGradOp = "hip_max_pool2d_relu_grad_internal";
// an elementwise program of fh_ew_op codes (attr ew_ops), inputs in program order: programs the reference's fused
// chains cannot name (relu_grad(x, a + b) as add then FH_EW_RELU_MASK by x)
inline constexpr std::string_view kEwProgramOp = "hip_ew_program_internal";
// sum over every axis but the last (the bias gradient of channels-last data or of [rows, features]): outputs the
// sum and an fp32 workspace of per-workgroup partials (see fh_sum_rows).
inline constexpr std::string_view kSumRowsOp = "hip_sum_rows_internal";
// out_i = add(x_i, mul(constant s_i, y_i)) for up to FH_AXPY_MAX pairs in one launch (the SGD update graph's
// parameter updates; see fh_axpy_multi): inputs [x_0, y_0, x_1, y_1, ...], one output per pair, attr scales.
inline constexpr std::string_view kAxpyMultiOp = "hip_axpy_multi_internal";
// avg_pool2d_grad_internal on channels-last dy / dx (same attributes; see fh_avg_pool2d_grad_nhwc).
inline constexpr std::string_view kAvgPoolGradNhwcOp = "hip_avg_pool2d_grad_nhwc_internal";
// conv2d_grad_filter_internal on MFMA: inputs x channels-last [N,H,W,cin_pad] and dy channels-last [N,Ho,Wo,Cout];
// outputs dw [Cout,Cin,KH,KW] and an fp32 split-K workspace (see fh_conv2d_wgrad_nhwc); attrs stride, padding,
// groups, filter_shape.
inline constexpr std::string_view kConvWgradOp = "hip_conv2d_wgrad_nhwc_internal";
// attention(q, k, v) [batch*seq, heads*dh] -> [batch*seq, heads*dh]: the per-(batch, head) slice / matmul / mul /
// softmax / matmul / concat decomposition in one kernel (attrs batch, seq, heads, dh, scale; see fh_attention_fwd).
inline constexpr std::string_view kAttentionOp = "hip_attention_internal";

// The graph HipBackend::compile plans for `graph` (already through the pass pipeline): attention, epilogue
// (opt_level >= 1) and channels-last conv lowering applied to a copy. Host-only; used by compile and by
// frame_hip_lowered_text.
Result<ir::Graph> lower_for_hip(const ir::Graph& graph, int32_t opt_level);

// Elementwise op name -> fh_ew_op code (0 when the op has no device code).
uint8_t ew_code(std::string_view op);

}  // namespace frame::backends::hip
