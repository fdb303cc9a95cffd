#pragma once
// ONNX weight exchange: the initializer subset of an ONNX ModelProto (TensorProto name / dims / data_type /
// raw_data for FLOAT, FLOAT16 and BFLOAT16) inside a minimal valid model skeleton (ir_version, one opset_import,
// graph.name). No operator graph is read or written. Interface follows the reference's
// include/frame/interop/onnx_weights.h:1-57 so that callers written against Frame compile unchanged; interop
// depends on core only (the allocator is passed in, forward-declared here).

#include <span>
#include <string>
#include <vector>

#include <frame/core/macros.h>
#include <frame/core/status.h>
#include <frame/core/tensor.h>

namespace frame::hal {
class Allocator;
}  // namespace frame::hal

namespace frame::interop {

// An initializer: its name and its data (host cpu memory).
struct NamedTensor {
  std::string name;
  Tensor tensor;
};

// Writes `weights` to `path` as a minimal ONNX ModelProto holding them as graph initializers. Every tensor must live
// on the cpu device with dtype float32, float16 or bfloat16 (else kInvalidArgument naming the tensor); a path that
// cannot be opened gives kInvalidArgument, a failed write kInternal.
FRAME_API Status save_onnx_weights(const std::string& path, std::span<const NamedTensor> weights);

// Reads the graph initializers of the ONNX ModelProto at `path`, in file order, into cpu tensors allocated from
// `allocator` (which must outlive them). Missing file: kNotFound. Truncated or out-of-range fields and the
// deprecated group wire types are rejected with the offset or wire type in the message; a data_type outside the
// three supported ones gives kInvalidArgument naming the ONNX enum value. Unknown fields are skipped.
FRAME_API Result<std::vector<NamedTensor>> load_onnx_weights(const std::string& path, hal::Allocator& allocator);

}  // namespace frame::interop
