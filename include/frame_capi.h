/*
 * frame_capi.h — C entry points of the Frame host library (libframe.so) for foreign-function callers.
 *
 * It is the C counterpart of the reference's Python binding surface for the compiled-graph path
 * (reference: python/src/bind_runtime.cpp:30-56 — compile(graph, backend) and Executable.run over
 * runtime::run_with_allocated_outputs — and python/src/bind_core.cpp for tensors): graphs cross the boundary
 * as Frame IR text (the dump_text format), tensors and executables as opaque handles. No C++ type crosses it.
 *
 * Every function returning int returns 0 on success or a frame::ErrorCode ordinal; the message of the last
 * failure on the calling thread is frame_last_error(). Text outputs use the (out, cap, needed) convention:
 * *needed receives the size including the terminating NUL; with out == NULL or cap too small the call returns
 * -1 and writes nothing.
 */
#ifndef FRAME_CAPI_H_
#define FRAME_CAPI_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct frame_tensor frame_tensor;
typedef struct frame_stream frame_stream;
typedef struct frame_event frame_event;
typedef struct frame_executable frame_executable;

const char* frame_last_error(void);

/* Registered backend names, comma-separated (BackendRegistry::available). */
int frame_backends(char* out, int64_t cap, int64_t* needed);
int frame_device_count(const char* backend, int32_t* count);

/* Tensors: dtype codes are frame::DTypeCode ordinals (0 float32, 2 float16, 3 bfloat16, ...). */
int frame_tensor_empty(const char* backend, int32_t device, int32_t dtype, const int64_t* dims, int32_t rank,
                       frame_tensor** out);
/* A tensor that starts `byte_offset` bytes into a fresh block (a multiple of the element size): the view
 * Tensor::from_storage_slice makes (reference include/frame/core/tensor.h:30-45), e.g. to hand an executable
 * operands that are not 16-byte aligned. */
int frame_tensor_empty_at(const char* backend, int32_t device, int32_t dtype, const int64_t* dims, int32_t rank,
                          int64_t byte_offset, frame_tensor** out);
void frame_tensor_free(frame_tensor* t);
void* frame_tensor_data(frame_tensor* t);
int64_t frame_tensor_nbytes(const frame_tensor* t);
int frame_tensor_upload(frame_tensor* t, const void* host, size_t bytes);   /* synchronous */
int frame_tensor_download(const frame_tensor* t, void* host, size_t bytes); /* synchronous */

/* Streams and events of a backend (hal::Stream / hal::Event). */
int frame_stream_create(const char* backend, int32_t device, frame_stream** out);
void frame_stream_destroy(frame_stream* s);
int frame_stream_synchronize(frame_stream* s);
void* frame_stream_native(frame_stream* s); /* hipStream_t for the hip backend */
int frame_event_create(const char* backend, int32_t device, frame_event** out);
void frame_event_destroy(frame_event* e);
int frame_event_record(frame_event* e, frame_stream* s);
int frame_event_synchronize(frame_event* e);

/* runtime::compile of IR text for `backend` (opt_level as hal::CompileOptions::opt_level). */
int frame_compile(const char* ir_text, const char* backend, int32_t opt_level, frame_executable** out);
/* Backend::compile (include/frame/hal/backend.h:104-105) of the graph as given: no pass pipeline, no cache. An op
 * without a kernel on the backend fails with kUnimplemented naming the op (the HAL conformance contract,
 * reference tests/cpp/hal_conformance/test_hal_conformance.cpp:249-269). */
int frame_backend_compile(const char* ir_text, const char* backend, int32_t opt_level, frame_executable** out);
void frame_executable_free(frame_executable* e);
int32_t frame_executable_num_inputs(const frame_executable* e);
int32_t frame_executable_num_outputs(const frame_executable* e);
/* dims must hold 8 entries; writes dtype code and rank. */
int frame_executable_io_spec(const frame_executable* e, int32_t is_output, int32_t index, int32_t* dtype, int64_t* dims,
                             int32_t* rank);
/* Executable::run on `stream` (enqueue only). */
int frame_executable_run(frame_executable* e, frame_tensor* const* inputs, int32_t n_in, frame_tensor* const* outputs,
                         int32_t n_out, frame_stream* stream);
/* `iterations` back-to-back Executable::run calls on `stream` (enqueue only), run i reading input set i % n_sets
 * (input_sets holds n_sets x n_in tensors, set-major) and writing `outputs`. The benchmark's timed loop: the runs
 * are issued from native code, as the reference's google-benchmark loops call Executable::run from C++
 * (benchmarks/bench_matmul.cpp), so a short graph is not timed at the speed of a Python loop. Stops at the first
 * failing run and returns its status. */
int frame_executable_run_repeat(frame_executable* e, frame_tensor* const* input_sets, int32_t n_sets, int32_t n_in,
                                frame_tensor* const* outputs, int32_t n_out, frame_stream* stream, int32_t iterations);
/* runtime::run_with_allocated_outputs: allocates outputs on device 0 of the backend, runs, synchronises. */
int frame_run_with_allocated_outputs(frame_executable* e, frame_tensor* const* inputs, int32_t n_in,
                                     frame_tensor** outputs, int32_t n_out);
/* Test hooks for per-op parity inside a whole compiled graph (no counterpart in the reference). A hip executable's
 * plan step i is the i-th non-input node of the lowered graph (frame_hip_lowered_text of the same IR text and
 * opt_level); frame_hip_executable_steps lists them as lines "i op". frame_hip_run_tapped runs the executable like
 * frame_executable_run (on a transient arena, eager, synchronised at the end) and, after each step steps[t], copies
 * its output output_index[t] into host[t], which holds bytes[t] bytes (the output's exact size, else
 * kInvalidArgument). */
int frame_hip_run_tapped(frame_executable* e, frame_tensor* const* inputs, int32_t n_in, frame_tensor* const* outputs,
                         int32_t n_out, frame_stream* stream, int32_t n_taps, const int32_t* steps,
                         const int32_t* output_index, void* const* host, const int64_t* bytes);
int frame_hip_executable_steps(const frame_executable* e, char* out, int64_t cap, int64_t* needed);

/* Number of entries in the compile cache. */
int64_t frame_compile_cache_size(void);

/* Compiler observability: the standard pipeline (pass_name NULL or "") or one named pass applied to the
 * parsed text, dump_text round trip, and the memory plan as lines "topo out offset size def last" + "total N". */
int frame_transform_text(const char* ir_text, const char* pass_name, char* out, int64_t cap, int64_t* needed);
int frame_roundtrip_text(const char* ir_text, char* out, int64_t cap, int64_t* needed);
int frame_memory_plan_text(const char* ir_text, char* out, int64_t cap, int64_t* needed);

/* Training-graph construction (compiler::build_backward_graph / build_sgd_update_graph, reference
 * include/frame/compiler/autograd.h:45-67) on IR text. frame_backward_text: the forward graph's outputs, then the
 * gradients of output `loss_output_index` w.r.t. graph inputs wrt[0..n_wrt). frame_sgd_update_text: the update graph
 * for the types of graph inputs param_inputs[0..n_params) of `ir_text`. */
int frame_backward_text(const char* ir_text, int32_t loss_output_index, const int32_t* wrt, int32_t n_wrt, char* out,
                        int64_t cap, int64_t* needed);
int frame_sgd_update_text(const char* ir_text, const int32_t* param_inputs, int32_t n_params, double learning_rate,
                          char* out, int64_t cap, int64_t* needed);

/* The graph the hip backend plans for `ir_text`: the standard pipeline for "hip", then HipBackend::compile's
 * lowering (fused attention, matmul/conv epilogues at opt_level >= 1, channels-last conv), as IR text.
 * Host-only (no device needed); no counterpart in the reference, which has no backend lowering to inspect. */
int frame_hip_lowered_text(const char* ir_text, int32_t opt_level, char* out, int64_t cap, int64_t* needed);

/* Backend::copy (include/frame/hal/backend.h:100-102) between two devices named by backend and index; "cpu" means
 * host memory. The direction follows the two devices; asynchronous on `stream` when it is non-null, synchronous
 * otherwise (the reference's contract, src/backends/cuda/cuda_backend.cpp:185-204). */
int frame_backend_copy(const char* backend, void* dst, const char* dst_backend, int32_t dst_index, const void* src,
                       const char* src_backend, int32_t src_index, size_t bytes, frame_stream* stream);

/* Counters of the hip backend's caching allocator for `device`: out[0] live bytes, out[1] reusable cached bytes,
 * out[2] freed bytes whose queued work may still run, out[3] device allocations made, out[4] device-wide waits,
 * out[5] waits for one freed block's fence events. No counterpart in the reference (its allocator caches
 * nothing); for tests of memory growth and reuse. */
int frame_hip_allocator_stats(int32_t device, uint64_t out[6]);

/* ONNX weight exchange (interop::save_onnx_weights / load_onnx_weights, reference
 * include/frame/interop/onnx_weights.h:38,47): the graph.initializer subset of an ONNX ModelProto, dtypes
 * float32 / float16 / bfloat16 (DTypeCode ordinals 0 / 2 / 3), host buffers. frame_load_onnx_weights parses `path`
 * into host tensors owned by *out, read back with the frame_onnx_* accessors (file order) and released with
 * frame_onnx_free. */
typedef struct frame_onnx_weights frame_onnx_weights;
int frame_save_onnx_weights(const char* path, int32_t n, const char* const* names, const int32_t* dtypes,
                            const int64_t* const* dims, const int32_t* ranks, const void* const* data);
int frame_load_onnx_weights(const char* path, frame_onnx_weights** out);
int32_t frame_onnx_count(const frame_onnx_weights* w);
const char* frame_onnx_name(const frame_onnx_weights* w, int32_t i);
int32_t frame_onnx_dtype(const frame_onnx_weights* w, int32_t i);
int32_t frame_onnx_rank(const frame_onnx_weights* w, int32_t i);
int64_t frame_onnx_dim(const frame_onnx_weights* w, int32_t i, int32_t k);
const void* frame_onnx_data(const frame_onnx_weights* w, int32_t i);
void frame_onnx_free(frame_onnx_weights* w);

/* Eager single-op launch (Backend::launch) of the one operator node in `node_ir_text` (a graph whose
 * non-input nodes are exactly one op) on the given tensors. */
int frame_launch(const char* node_ir_text, const char* backend, frame_tensor* const* inputs, int32_t n_in,
                 frame_tensor* const* outputs, int32_t n_out, frame_stream* stream);

#ifdef __cplusplus
}
#endif

#endif /* FRAME_CAPI_H_ */
