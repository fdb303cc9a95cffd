// Shape / Storage / Tensor implementations (reference behaviour: src/core/{shape,storage,tensor}.cpp).
#include <limits>
#include <string>
#include <utility>

#include <frame/core/shape.h>
#include <frame/core/storage.h>
#include <frame/core/tensor.h>
#include <frame/hal/allocator.h>

namespace frame {

Status Shape::verify() const {
  for (size_t i = 0; i < dims_.size(); ++i) {
    if (dims_[i] == kDynamicDim)
      return Status::make(ErrorCode::kInvalidArgument,
                          "Shape.verify: dimension " + std::to_string(i) + " is dynamic, static shape required");
    if (dims_[i] < 0)
      return Status::make(ErrorCode::kInvalidArgument, "Shape.verify: dimension " + std::to_string(i) +
                                                           " is negative (" + std::to_string(dims_[i]) + ")");
  }
  return Status::ok();
}

std::string Shape::to_string() const {
  std::string s = "[";
  for (size_t i = 0; i < dims_.size(); ++i) {
    if (i) s += ", ";
    s += std::to_string(dims_[i]);
  }
  return s + "]";
}

Strides row_major_strides(const Shape& shape) {
  std::vector<int64_t> st(static_cast<size_t>(shape.rank()));
  int64_t acc = 1;
  for (int64_t i = shape.rank() - 1; i >= 0; --i) {
    st[static_cast<size_t>(i)] = acc;
    acc *= shape.dim(i);
  }
  return Strides(std::move(st));
}

// ---- Storage ----------------------------------------------------------------------------------------------

void Storage::release() noexcept {
  if (data_ != nullptr && allocator_ != nullptr) allocator_->deallocate(data_);
  data_ = nullptr;
  nbytes_ = 0;
  device_ = Device{};
  allocator_ = nullptr;
}

Storage::Storage(Storage&& o) noexcept
    : data_(std::exchange(o.data_, nullptr)),
      nbytes_(std::exchange(o.nbytes_, 0)),
      device_(std::exchange(o.device_, Device{})),
      allocator_(std::exchange(o.allocator_, nullptr)) {}

Storage& Storage::operator=(Storage&& o) noexcept {
  if (this != &o) {
    release();
    data_ = std::exchange(o.data_, nullptr);
    nbytes_ = std::exchange(o.nbytes_, 0);
    device_ = std::exchange(o.device_, Device{});
    allocator_ = std::exchange(o.allocator_, nullptr);
  }
  return *this;
}

Storage::~Storage() { release(); }

Result<std::shared_ptr<Storage>> Storage::allocate(hal::Allocator& allocator, size_t bytes, size_t alignment,
                                                   Device device) {
  auto s = std::make_shared<Storage>();
  s->device_ = device;
  if (bytes == 0) return s;  // empty storage, nothing to return to the allocator
  Result<void*> p = allocator.allocate(bytes, alignment);
  if (!p.is_ok()) return p.status();
  s->data_ = p.value();
  s->nbytes_ = bytes;
  s->allocator_ = &allocator;
  return s;
}

// ---- Tensor -----------------------------------------------------------------------------------------------

Result<Tensor> Tensor::empty(const Shape& shape, DType dtype, Device device, hal::Allocator& allocator) {
  FRAME_RETURN_IF_ERROR(shape.verify());
  const size_t numel = static_cast<size_t>(shape.numel());
  const size_t item = dtype.itemsize();
  if (item != 0 && numel > std::numeric_limits<size_t>::max() / item)
    return Status::make(ErrorCode::kInvalidArgument, "Tensor.empty: numel * itemsize overflows size_t");
  Result<std::shared_ptr<Storage>> st = Storage::allocate(allocator, numel * item, kDefaultAlignment, device);
  if (!st.is_ok()) return st.status();
  Tensor t;
  t.storage_ = std::move(st.value());
  t.shape_ = shape;
  t.strides_ = row_major_strides(shape);
  t.dtype_ = dtype;
  return t;
}

Tensor Tensor::from_storage_slice(std::shared_ptr<Storage> storage, size_t byte_offset, const Shape& shape,
                                  DType dtype, Device device) {
  FRAME_CHECK(storage != nullptr);
  FRAME_CHECK(device == storage->device());
  const size_t item = dtype.itemsize();
  FRAME_CHECK(item > 0 && byte_offset % item == 0);
  FRAME_CHECK(shape.numel() >= 0);
  const size_t bytes = static_cast<size_t>(shape.numel()) * item;
  FRAME_CHECK(byte_offset <= storage->nbytes() && bytes <= storage->nbytes() - byte_offset);
  Tensor t;
  t.storage_ = std::move(storage);
  t.shape_ = shape;
  t.strides_ = row_major_strides(shape);
  t.offset_ = static_cast<int64_t>(byte_offset / item);
  t.dtype_ = dtype;
  return t;
}

Device Tensor::device() const { return storage_ ? storage_->device() : Device{}; }

void* Tensor::raw_data() {
  if (!storage_ || storage_->data() == nullptr) return nullptr;
  return static_cast<char*>(storage_->data()) + static_cast<size_t>(offset_) * dtype_.itemsize();
}

const void* Tensor::raw_data() const {
  if (!storage_ || storage_->data() == nullptr) return nullptr;
  return static_cast<const char*>(storage_->data()) + static_cast<size_t>(offset_) * dtype_.itemsize();
}

Tensor Tensor::view(const Shape& new_shape) const {
  FRAME_CHECK(new_shape.verify().is_ok() && new_shape.numel() == shape_.numel());
  Tensor t = *this;
  t.shape_ = new_shape;
  t.strides_ = row_major_strides(new_shape);
  return t;
}

}  // namespace frame
