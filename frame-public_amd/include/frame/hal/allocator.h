#pragma once
// hal::Allocator: device memory for one device; pooling is the backend's choice
// (reference: include/frame/hal/allocator.h:13-21).

#include <cstddef>

#include <frame/core/macros.h>
#include <frame/core/status.h>

namespace frame::hal {

class FRAME_API Allocator {
 public:
  virtual ~Allocator() = default;
  virtual Result<void*> allocate(size_t bytes, size_t alignment) = 0;
  virtual void deallocate(void* ptr) = 0;
};

}  // namespace frame::hal
