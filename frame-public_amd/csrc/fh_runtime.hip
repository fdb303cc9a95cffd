// Runtime shims of the C ABI: devices, memory, copies, streams and events.
// These back HipBackend / HipAllocator / HipStream / HipEvent on the C++ side.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <string>

#include "fh_common.h"

namespace fh {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& message) { g_last_error = message; }

fh_status fail(fh_status code, const std::string& message) {
  set_error(message);
  return code;
}

fh_status check_hip(hipError_t err, const char* what) {
  if (err == hipSuccess) return FH_OK;
  std::string msg = std::string(what) + ": " + hipGetErrorName(err) + " (" + hipGetErrorString(err) + ")";
  set_error(msg);
  if (err == hipErrorOutOfMemory || err == hipErrorMemoryAllocation) return FH_OUT_OF_MEMORY;
  if (err == hipErrorInvalidValue || err == hipErrorInvalidDevicePointer || err == hipErrorInvalidDevice)
    return FH_INVALID_ARGUMENT;
  return FH_DEVICE_ERROR;
}

}  // namespace fh

using fh::fail;

extern "C" {

const char* fh_last_error(void) { return fh::g_last_error.c_str(); }

int32_t fh_abi_version(void) { return FH_ABI_VERSION; }

fh_status fh_device_count(int32_t* count) {
  if (count == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_device_count: count is null");
  int n = 0;
  hipError_t err = hipGetDeviceCount(&n);
  if (err == hipErrorNoDevice) {
    (void)hipGetLastError();
    *count = 0;
    return FH_OK;
  }
  FH_HIP_CHECK(err);
  *count = n;
  return FH_OK;
}

fh_status fh_set_device(int32_t device) {
  FH_HIP_CHECK(hipSetDevice(device));
  return FH_OK;
}

fh_status fh_malloc(void** ptr, size_t bytes, int32_t device) {
  if (ptr == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_malloc: ptr is null");
  if (bytes == 0) return fail(FH_INVALID_ARGUMENT, "fh_malloc: bytes must be > 0");
  FH_HIP_CHECK(hipSetDevice(device));
  void* p = nullptr;
  FH_HIP_CHECK(hipMalloc(&p, bytes));
  *ptr = p;
  return FH_OK;
}

fh_status fh_free(void* ptr) {
  if (ptr == nullptr) return FH_OK;
  FH_HIP_CHECK(hipFree(ptr));
  return FH_OK;
}

fh_status fh_host_alloc(void** ptr, size_t bytes) {
  if (ptr == nullptr || bytes == 0) return fail(FH_INVALID_ARGUMENT, "fh_host_alloc: bad arguments");
  FH_HIP_CHECK(hipHostMalloc(ptr, bytes, hipHostMallocDefault));
  return FH_OK;
}

fh_status fh_host_free(void* ptr) {
  if (ptr == nullptr) return FH_OK;
  FH_HIP_CHECK(hipHostFree(ptr));
  return FH_OK;
}

fh_status fh_memcpy(void* dst, const void* src, size_t bytes, int32_t kind, void* stream) {
  if (bytes == 0) return FH_OK;
  if (dst == nullptr || src == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_memcpy: null pointer");
  hipMemcpyKind k;
  switch (kind) {
    case FH_H2H:
      k = hipMemcpyHostToHost;
      break;
    case FH_H2D:
      k = hipMemcpyHostToDevice;
      break;
    case FH_D2H:
      k = hipMemcpyDeviceToHost;
      break;
    case FH_D2D:
      k = hipMemcpyDeviceToDevice;
      break;
    default:
      return fail(FH_INVALID_ARGUMENT, "fh_memcpy: unknown copy kind " + std::to_string(kind));
  }
  if (stream == nullptr) {
    FH_HIP_CHECK(hipMemcpy(dst, src, bytes, k));
  } else {
    FH_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, k, static_cast<hipStream_t>(stream)));
  }
  return FH_OK;
}

fh_status fh_stream_create(void** stream, int32_t device) {
  if (stream == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_stream_create: stream is null");
  FH_HIP_CHECK(hipSetDevice(device));
  hipStream_t s = nullptr;
  // Default priority on purpose: every stream of this library runs at the same priority.
  FH_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *stream = s;
  return FH_OK;
}

fh_status fh_stream_capturing(void* stream, int32_t* capturing) {
  if (capturing == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_stream_capturing: capturing is null");
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  FH_HIP_CHECK(hipStreamIsCapturing(static_cast<hipStream_t>(stream), &st));
  *capturing = st == hipStreamCaptureStatusNone ? 0 : 1;
  return FH_OK;
}

fh_status fh_stream_destroy(void* stream) {
  if (stream == nullptr) return FH_OK;
  FH_HIP_CHECK(hipStreamDestroy(static_cast<hipStream_t>(stream)));
  return FH_OK;
}

fh_status fh_stream_synchronize(void* stream) {
  FH_HIP_CHECK(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
  return FH_OK;
}

// Stream capture into a HIP graph (thread-local mode: other threads' HIP calls are unaffected) and replay.
fh_status fh_graph_begin_capture(void* stream) {
  if (stream == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_graph_begin_capture: the null stream cannot be captured");
  FH_HIP_CHECK(hipStreamBeginCapture(static_cast<hipStream_t>(stream), hipStreamCaptureModeThreadLocal));
  return FH_OK;
}

fh_status fh_graph_end_capture(void* stream, int32_t keep, void** exec) {
  if (stream == nullptr || exec == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_graph_end_capture: null argument");
  *exec = nullptr;
  hipGraph_t g = nullptr;
  FH_HIP_CHECK(hipStreamEndCapture(static_cast<hipStream_t>(stream), &g));
  if (!keep) {
    if (g != nullptr) FH_HIP_CHECK(hipGraphDestroy(g));
    return FH_OK;
  }
  hipGraphExec_t e = nullptr;
  const hipError_t err = hipGraphInstantiate(&e, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (err != hipSuccess) return fh::check_hip(err, "hipGraphInstantiate");
  *exec = e;
  return FH_OK;
}

fh_status fh_graph_launch(void* exec, void* stream) {
  if (exec == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_graph_launch: null graph");
  FH_HIP_CHECK(hipGraphLaunch(static_cast<hipGraphExec_t>(exec), static_cast<hipStream_t>(stream)));
  return FH_OK;
}

fh_status fh_graph_destroy(void* exec) {
  if (exec == nullptr) return FH_OK;
  FH_HIP_CHECK(hipGraphExecDestroy(static_cast<hipGraphExec_t>(exec)));
  return FH_OK;
}

fh_status fh_device_synchronize(void) {
  FH_HIP_CHECK(hipDeviceSynchronize());
  return FH_OK;
}

fh_status fh_event_create(void** event, int32_t device) {
  if (event == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_event_create: event is null");
  FH_HIP_CHECK(hipSetDevice(device));
  hipEvent_t e = nullptr;
  FH_HIP_CHECK(hipEventCreate(&e));
  *event = e;
  return FH_OK;
}

fh_status fh_event_destroy(void* event) {
  if (event == nullptr) return FH_OK;
  FH_HIP_CHECK(hipEventDestroy(static_cast<hipEvent_t>(event)));
  return FH_OK;
}

fh_status fh_event_record(void* event, void* stream) {
  if (event == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_event_record: event is null");
  FH_HIP_CHECK(hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream)));
  return FH_OK;
}

fh_status fh_stream_wait_event(void* stream, void* event) {
  if (event == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_stream_wait_event: event is null");
  FH_HIP_CHECK(hipStreamWaitEvent(static_cast<hipStream_t>(stream), static_cast<hipEvent_t>(event), 0));
  return FH_OK;
}

fh_status fh_event_query(void* event, int32_t* done) {
  if (event == nullptr || done == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_event_query: null argument");
  hipError_t err = hipEventQuery(static_cast<hipEvent_t>(event));
  if (err == hipSuccess) {
    *done = 1;
    return FH_OK;
  }
  if (err == hipErrorNotReady) {
    *done = 0;
    return FH_OK;
  }
  return fh::check_hip(err, "hipEventQuery");
}

fh_status fh_event_synchronize(void* event) {
  if (event == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_event_synchronize: event is null");
  FH_HIP_CHECK(hipEventSynchronize(static_cast<hipEvent_t>(event)));
  return FH_OK;
}

fh_status fh_event_elapsed_ms(void* start, void* stop, float* ms) {
  if (start == nullptr || stop == nullptr || ms == nullptr)
    return fail(FH_INVALID_ARGUMENT, "fh_event_elapsed_ms: null argument");
  FH_HIP_CHECK(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)));
  return FH_OK;
}

}  // extern "C"
