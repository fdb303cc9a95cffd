// HAL objects of the `hip` backend: streams, events, the caching allocator, copies, eager launch and the
// registration (reference contract: include/frame/hal/backend.h:77-160; design analog replaced:
// src/backends/cuda/cuda_backend.cpp:42-320, cuda_allocator.cpp:26-66).
#include "hip_backend.h"

#include <atomic>
#include <bit>
#include <functional>
#include <string>
#include <unordered_map>
#include <unordered_set>

#include <frame/ir/graph.h>
#include <frame/ops/kernel_registry.h>

namespace frame::backends::hip {

Result<std::unique_ptr<hal::Executable>> compile_hip_executable(const ir::Graph& graph, const hal::CompileOptions& options,
                                                                 HipAllocator& allocator, Device device);

Status from_fh(fh_status code, std::string_view what) {
  if (code == FH_OK) return Status::ok();
  const char* msg = fh_last_error();
  return Status::make(static_cast<ErrorCode>(code), std::string(what) + ": " + (msg != nullptr ? msg : ""));
}

uint8_t ew_code(std::string_view op) {
  if (op == "add") return FH_EW_ADD;
  if (op == "mul") return FH_EW_MUL;
  if (op == "relu") return FH_EW_RELU;
  if (op == "square") return FH_EW_SQUARE;
  if (op == "gelu") return FH_EW_GELU;
  return 0;
}

// ---- stream / event ---------------------------------------------------------------------------------------

namespace {
std::mutex g_streams_mu;
std::unordered_set<uint64_t> g_live_streams;  // ids of live HipStreams
struct LiveStream {
  uint64_t id;
  void* handle;
  int32_t device;
};
std::unordered_map<const hal::Stream*, LiveStream> g_live_stream_objects;  // live HipStream objects
std::atomic<uint64_t> g_next_stream_id{1};
}  // namespace

bool hip_stream_alive(uint64_t id) {
  std::lock_guard<std::mutex> lock(g_streams_mu);
  return g_live_streams.count(id) != 0;
}

uint64_t hip_stream_id(const hal::Stream& stream) {
  std::lock_guard<std::mutex> lock(g_streams_mu);
  auto it = g_live_stream_objects.find(&stream);
  return it != g_live_stream_objects.end() ? it->second.id : 0;
}

bool for_each_live_stream(int32_t device, const std::function<bool(void*)>& fn) {
  std::lock_guard<std::mutex> lock(g_streams_mu);  // no stream of the list is destroyed meanwhile
  for (const auto& [obj, ls] : g_live_stream_objects)
    if (ls.device == device && !fn(ls.handle)) return false;
  return true;
}

HipStream::HipStream(void* handle, int32_t device) : handle_(handle), device_(device), id_(g_next_stream_id++) {
  std::lock_guard<std::mutex> lock(g_streams_mu);
  g_live_streams.insert(id_);
  g_live_stream_objects.emplace(this, LiveStream{id_, handle_, device_});
}

HipStream::~HipStream() {
  {
    std::lock_guard<std::mutex> lock(g_streams_mu);
    g_live_streams.erase(id_);
    g_live_stream_objects.erase(this);
  }
  (void)fh_stream_destroy(handle_);
}

Status HipStream::synchronize() {
  FRAME_HIP_RETURN_IF_ERROR(fh_stream_synchronize(handle_), "HipStream::synchronize");
  return Status::ok();
}

Status HipStream::record(hal::Event& event) {
  // Events handed to a hip stream come from HipBackend::create_event (same-backend contract of the HAL).
  auto* e = static_cast<HipEvent*>(&event);
  FRAME_HIP_RETURN_IF_ERROR(fh_event_record(e->handle(), handle_), "HipStream::record");
  e->mark_recorded();
  return Status::ok();
}

Status HipStream::wait(const hal::Event& event) {
  const auto* e = static_cast<const HipEvent*>(&event);
  if (!e->recorded()) return Status::ok();  // never recorded = already complete
  FRAME_HIP_RETURN_IF_ERROR(fh_stream_wait_event(handle_, e->handle()), "HipStream::wait");
  return Status::ok();
}

HipEvent::~HipEvent() { (void)fh_event_destroy(handle_); }

bool HipEvent::query() const {
  if (!recorded_) return true;
  int32_t done = 0;
  return fh_event_query(handle_, &done) == FH_OK && done != 0;
}

Status HipEvent::synchronize() {
  if (!recorded_) return Status::ok();
  FRAME_HIP_RETURN_IF_ERROR(fh_event_synchronize(handle_), "HipEvent::synchronize");
  return Status::ok();
}

// ---- allocator --------------------------------------------------------------------------------------------

size_t HipAllocator::size_class(size_t bytes) {
  // 512 B granularity up to 1 MiB, then powers of two split in 4 steps (<= 25% slack), so the cache serves
  // repeated shapes exactly and mixed shapes with bounded waste.
  if (bytes <= (1u << 20)) return (bytes + 511) & ~size_t{511};
  const size_t top = std::bit_floor(bytes);
  const size_t step = top / 4;
  return (bytes + step - 1) / step * step;
}

HipAllocator::~HipAllocator() {
  // Process teardown: return cached blocks (hipFree waits for the device) and the fence events. Live blocks belong
  // to Storage objects that may outlive us.
  for (auto& [cls, list] : free_lists_)
    for (void* p : list) (void)fh_free(p);
  for (auto& [cls, list] : pending_)
    for (PendingBlock& b : list) {
      (void)fh_free(b.ptr);
      for (void* e : b.fence) (void)fh_event_destroy(e);
    }
  for (void* e : event_pool_) (void)fh_event_destroy(e);
}

// Events recorded now on every live stream of the device and on the null stream: once they have all completed,
// every kernel or copy queued before this point (on any of those streams) has finished. False when a stream is
// being captured into a graph (nothing is recorded then; the caller falls back to a device-wide wait) or when an
// event cannot be had.
bool HipAllocator::record_fence_locked(std::vector<void*>& fence) {
  auto not_capturing = [](void* s) {
    int32_t capturing = 1;
    return fh_stream_capturing(s, &capturing) == FH_OK && capturing == 0;
  };
  auto record = [&](void* s) {
    void* e = nullptr;
    if (!event_pool_.empty()) {
      e = event_pool_.back();
      event_pool_.pop_back();
    } else if (fh_event_create(&e, device_) != FH_OK) {
      return false;
    }
    fence.push_back(e);
    return fh_event_record(e, s) == FH_OK;
  };
  return for_each_live_stream(device_, not_capturing) && for_each_live_stream(device_, record) && record(nullptr);
}

void HipAllocator::recycle_fence_locked(std::vector<void*>& fence) {
  event_pool_.insert(event_pool_.end(), fence.begin(), fence.end());
  fence.clear();
}

Status HipAllocator::release_pending_locked() {
  if (pending_.empty()) return Status::ok();
  FRAME_HIP_RETURN_IF_ERROR(fh_set_device(device_), "HipAllocator: set device");
  FRAME_HIP_RETURN_IF_ERROR(fh_device_synchronize(), "HipAllocator: wait for work on freed blocks");
  ++stats_.device_syncs;
  for (auto& [cls, list] : pending_) {
    auto& dst = free_lists_[cls];
    for (PendingBlock& b : list) {
      dst.push_back(b.ptr);
      recycle_fence_locked(b.fence);
    }
    stats_.pending_bytes -= cls * list.size();
    stats_.cached_bytes += cls * list.size();
  }
  pending_.clear();
  return Status::ok();
}

// The oldest pending block of a size class, once the work queued before its free has finished: a wait on its
// fence's events (usually complete already), which leaves work queued after the free running. Blocks freed while
// a stream was being captured carry no fence and take the device-wide wait.
Result<void*> HipAllocator::take_pending_locked(size_t cls) {
  auto it = pending_.find(cls);
  if (it == pending_.end() || it->second.empty()) return static_cast<void*>(nullptr);
  PendingBlock& b = it->second.front();
  if (!b.fenced) {
    FRAME_RETURN_IF_ERROR(release_pending_locked());
    auto& list = free_lists_[cls];
    void* p = list.back();
    list.pop_back();
    stats_.cached_bytes -= cls;
    return p;
  }
  for (void* e : b.fence) {
    int32_t done = 0;
    FRAME_HIP_RETURN_IF_ERROR(fh_event_query(e, &done), "HipAllocator: fence query");
    if (!done) {
      FRAME_HIP_RETURN_IF_ERROR(fh_event_synchronize(e), "HipAllocator: wait for work on a freed block");
      ++stats_.fence_waits;
    }
  }
  void* p = b.ptr;
  recycle_fence_locked(b.fence);
  it->second.pop_front();
  stats_.pending_bytes -= cls;
  return p;
}

HipAllocator::Stats HipAllocator::stats() {
  std::lock_guard<std::mutex> lock(mu_);
  return stats_;
}

Result<void*> HipAllocator::allocate(size_t bytes, size_t alignment) {
  if (bytes == 0) return Status::make(ErrorCode::kInvalidArgument, "HipAllocator::allocate: bytes must be > 0");
  if (alignment == 0 || (alignment & (alignment - 1)) != 0)
    return Status::make(ErrorCode::kInvalidArgument,
                        "HipAllocator::allocate: alignment " + std::to_string(alignment) + " is not a power of two");
  if (alignment > kGuaranteedAlignment)
    return Status::make(ErrorCode::kInvalidArgument, "HipAllocator::allocate: alignment " + std::to_string(alignment) +
                                                         " exceeds the guaranteed " + std::to_string(kGuaranteedAlignment));
  const size_t cls = size_class(bytes);
  std::lock_guard<std::mutex> lock(mu_);
  auto take = [&]() -> void* {
    auto it = free_lists_.find(cls);
    if (it == free_lists_.end() || it->second.empty()) return nullptr;
    void* p = it->second.back();
    it->second.pop_back();
    stats_.cached_bytes -= cls;
    return p;
  };
  void* p = take();
  if (p == nullptr) {
    Result<void*> r = take_pending_locked(cls);
    if (!r.is_ok()) return r.status();
    p = r.value();
  }
  if (p == nullptr) {
    fh_status st = fh_malloc(&p, cls, device_);
    if (st == FH_OUT_OF_MEMORY) {
      // Give the whole cache back to the device (pending blocks once their work is done) and retry once.
      FRAME_RETURN_IF_ERROR(release_pending_locked());
      for (auto& [c, list] : free_lists_)
        for (void* q : list) (void)fh_free(q);
      free_lists_.clear();
      stats_.cached_bytes = 0;
      st = fh_malloc(&p, cls, device_);
    }
    if (st != FH_OK) return from_fh(st, "HipAllocator::allocate(" + std::to_string(bytes) + " bytes)");
    ++stats_.device_allocations;
  }
  live_.emplace(p, cls);
  stats_.live_bytes += cls;
  return p;
}

void HipAllocator::deallocate(void* ptr) {
  if (ptr == nullptr) return;
  std::lock_guard<std::mutex> lock(mu_);
  auto it = live_.find(ptr);
  if (it == live_.end()) return;  // not ours: ignore rather than corrupt the cache
  PendingBlock b{ptr, {}, false};
  b.fenced = record_fence_locked(b.fence);
  if (!b.fenced) recycle_fence_locked(b.fence);
  pending_[it->second].push_back(std::move(b));
  stats_.live_bytes -= it->second;
  stats_.pending_bytes += it->second;
  live_.erase(it);
}

// ---- backend ----------------------------------------------------------------------------------------------

HipBackend::HipBackend() = default;
HipBackend::~HipBackend() = default;

Result<int32_t> HipBackend::device_count() const {
  int32_t n = 0;
  FRAME_HIP_RETURN_IF_ERROR(fh_device_count(&n), "HipBackend::device_count");
  return n;
}

Status HipBackend::check_device(Device device) const {
  if (device.backend != kHipBackendName)
    return Status::make(ErrorCode::kInvalidArgument,
                        "hip backend: device backend '" + std::string(device.backend) + "' is not 'hip'");
  Result<int32_t> n = device_count();
  if (!n.is_ok()) return n.status();
  if (device.index < 0 || device.index >= n.value())
    return Status::make(ErrorCode::kInvalidArgument, "hip backend: device index " + std::to_string(device.index) +
                                                         " out of range (device_count=" + std::to_string(n.value()) + ")");
  return Status::ok();
}

Result<std::unique_ptr<hal::Stream>> HipBackend::create_stream(Device device) {
  FRAME_RETURN_IF_ERROR(check_device(device));
  void* s = nullptr;
  FRAME_HIP_RETURN_IF_ERROR(fh_stream_create(&s, device.index), "HipBackend::create_stream");
  return std::unique_ptr<hal::Stream>(std::make_unique<HipStream>(s, device.index));
}

Result<std::unique_ptr<hal::Event>> HipBackend::create_event(Device device) {
  FRAME_RETURN_IF_ERROR(check_device(device));
  void* e = nullptr;
  FRAME_HIP_RETURN_IF_ERROR(fh_event_create(&e, device.index), "HipBackend::create_event");
  return std::unique_ptr<hal::Event>(std::make_unique<HipEvent>(e, device.index));
}

hal::Allocator* HipBackend::allocator(Device device) {
  if (!check_device(device).is_ok()) return nullptr;
  std::lock_guard<std::mutex> lock(mu_);
  if (allocators_.size() <= static_cast<size_t>(device.index)) allocators_.resize(static_cast<size_t>(device.index) + 1);
  auto& a = allocators_[static_cast<size_t>(device.index)];
  if (!a) a = std::make_unique<HipAllocator>(device.index);
  return a.get();
}

Status HipBackend::copy(void* dst, Device dst_device, const void* src, Device src_device, size_t bytes,
                        hal::Stream* stream) {
  if (bytes == 0) return Status::ok();
  if (dst == nullptr || src == nullptr) return Status::make(ErrorCode::kInvalidArgument, "HipBackend::copy: null pointer");
  const bool dst_host = dst_device.backend == kCpuBackendName;
  const bool src_host = src_device.backend == kCpuBackendName;
  if (!dst_host) FRAME_RETURN_IF_ERROR(check_device(dst_device));
  if (!src_host) FRAME_RETURN_IF_ERROR(check_device(src_device));
  const int32_t kind = dst_host ? (src_host ? FH_H2H : FH_D2H) : (src_host ? FH_H2D : FH_D2D);
  void* s = stream == nullptr ? nullptr : stream->native_handle();
  FRAME_HIP_RETURN_IF_ERROR(fh_memcpy(dst, src, bytes, kind, s), "HipBackend::copy");
  return Status::ok();
}

Result<std::unique_ptr<hal::Executable>> HipBackend::compile(const ir::Graph& graph, const hal::CompileOptions& options) {
  Device device{kHipBackendName, 0};
  for (const ir::Node* n : graph.topological_order())
    if (!n->outputs().empty()) {
      device = n->outputs()[0].type().device;
      break;
    }
  FRAME_RETURN_IF_ERROR(check_device(device));
  auto* alloc = static_cast<HipAllocator*>(allocator(device));
  if (alloc == nullptr) return Status::make(ErrorCode::kInternal, "HipBackend::compile: no allocator");
  return compile_hip_executable(graph, options, *alloc, device);
}

Status HipBackend::launch(const hal::KernelInvocation& inv, hal::Stream* stream) {
  FRAME_RETURN_IF_ERROR(check_device(inv.device));
  Result<ops::KernelFn> k = ops::KernelRegistry::instance().find(inv.op, kHipBackendName);
  if (!k.is_ok()) return Status::make(ErrorCode::kUnimplemented, std::string(k.status().message()));
  ops::KernelContext ctx{inv.inputs, inv.outputs, inv.attrs, inv.device, stream, nullptr};
  return k.value()(ctx);
}

}  // namespace frame::backends::hip

FRAME_REGISTER_BACKEND(frame::kHipBackendName, frame::backends::hip::HipBackend);
