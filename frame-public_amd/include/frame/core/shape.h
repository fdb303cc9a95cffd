#pragma once
// Shape and Strides value types (static shapes only; kDynamicDim is a reserved sentinel that verify()
// rejects). Interface as in the reference (include/frame/core/shape.h:21-82).

#include <cstddef>
#include <cstdint>
#include <initializer_list>
#include <string>
#include <utility>
#include <vector>

#include <frame/core/macros.h>
#include <frame/core/status.h>

namespace frame {

inline constexpr int64_t kDynamicDim = -1;

class Shape {
 public:
  Shape() = default;
  Shape(std::initializer_list<int64_t> dims) : dims_(dims) {}
  explicit Shape(std::vector<int64_t> dims) : dims_(std::move(dims)) {}

  int64_t rank() const { return static_cast<int64_t>(dims_.size()); }
  int64_t dim(int64_t i) const { return dims_[static_cast<size_t>(i)]; }
  const std::vector<int64_t>& dims() const { return dims_; }

  int64_t numel() const {
    int64_t n = 1;
    for (int64_t d : dims_) {
      if (d == kDynamicDim) return kDynamicDim;
      n *= d;
    }
    return n;
  }
  bool has_dynamic_dim() const {
    for (int64_t d : dims_)
      if (d == kDynamicDim) return true;
    return false;
  }
  FRAME_API Status verify() const;
  FRAME_API std::string to_string() const;  // "[d0, d1, ...]", for messages only
  bool operator==(const Shape&) const = default;

 private:
  std::vector<int64_t> dims_;
};

class Strides {
 public:
  Strides() = default;
  Strides(std::initializer_list<int64_t> strides) : strides_(strides) {}
  explicit Strides(std::vector<int64_t> strides) : strides_(std::move(strides)) {}
  int64_t rank() const { return static_cast<int64_t>(strides_.size()); }
  const std::vector<int64_t>& values() const { return strides_; }
  bool operator==(const Strides&) const = default;

 private:
  std::vector<int64_t> strides_;
};

FRAME_API Strides row_major_strides(const Shape& shape);

}  // namespace frame
