#pragma once
// Tensor: shallow-copy handle = shared Storage + row-major view metadata
// (reference: include/frame/core/tensor.h:22-75).

#include <cstdint>
#include <memory>
#include <type_traits>

#include <frame/core/device.h>
#include <frame/core/dtype.h>
#include <frame/core/macros.h>
#include <frame/core/shape.h>
#include <frame/core/status.h>
#include <frame/core/storage.h>

namespace frame::hal {
class Allocator;
}

namespace frame {

class FRAME_API Tensor {
 public:
  Tensor() = default;

  // Uninitialised tensor whose Storage comes from `allocator` (kDefaultAlignment).
  static Result<Tensor> empty(const Shape& shape, DType dtype, Device device, hal::Allocator& allocator);

  // View of bytes [byte_offset, byte_offset + numel*itemsize) of an existing Storage (arena slices).
  static Tensor from_storage_slice(std::shared_ptr<Storage> storage, size_t byte_offset, const Shape& shape,
                                   DType dtype, Device device);

  const Shape& shape() const { return shape_; }
  const Strides& strides() const { return strides_; }
  DType dtype() const { return dtype_; }
  Device device() const;
  int64_t numel() const { return shape_.numel(); }

  void* raw_data();
  const void* raw_data() const;

  template <ScalarType T>
  T* data() {
    FRAME_CHECK(dtype_traits<std::remove_cv_t<T>>::code == dtype_.code());
    return static_cast<T*>(raw_data());
  }

  // Same storage, new row-major shape with the same element count.
  Tensor view(const Shape& new_shape) const;

 private:
  std::shared_ptr<Storage> storage_;
  Shape shape_;
  Strides strides_;
  int64_t offset_ = 0;  // in elements
  DType dtype_{DTypeCode::kFloat32};
};

}  // namespace frame
