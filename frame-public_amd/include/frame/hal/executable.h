#pragma once
// hal::Executable: the product of Backend::compile; run() executes the whole graph on a stream
// (reference: include/frame/hal/executable.h:22-59).

#include <span>
#include <string_view>
#include <vector>

#include <frame/core/device.h>
#include <frame/core/dtype.h>
#include <frame/core/macros.h>
#include <frame/core/shape.h>
#include <frame/core/status.h>
#include <frame/core/tensor.h>

namespace frame::hal {

class Stream;

struct IoSpec {
  DType dtype{DTypeCode::kFloat32};
  Shape shape;
};

class FRAME_API Executable {
 public:
  virtual ~Executable() = default;
  virtual Status run(std::span<const Tensor> inputs, std::span<Tensor> outputs, Stream& stream) = 0;
  virtual std::vector<IoSpec> input_signature() const = 0;
  virtual std::vector<IoSpec> output_signature() const = 0;
};

// Element-wise comparison of tensors against a signature (count, dtype, shape). `label` prefixes messages.
FRAME_API Status validate_io_signature(std::span<const Tensor> values, const std::vector<IoSpec>& signature,
                                       std::string_view label);

// Every tensor must live on `expected`.
FRAME_API Status validate_tensor_devices(std::span<const Tensor> values, Device expected, std::string_view label);

}  // namespace frame::hal
