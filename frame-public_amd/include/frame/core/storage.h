#pragma once
// Storage: one block of device (or host) memory plus the device it lives on. Move-only; shared through
// std::shared_ptr<Storage>. Memory comes from a hal::Allocator that must outlive the Storage
// (reference: include/frame/core/storage.h:28-55).

#include <cstddef>
#include <memory>

#include <frame/core/device.h>
#include <frame/core/macros.h>
#include <frame/core/status.h>

namespace frame::hal {
class Allocator;
}

namespace frame {

class FRAME_API Storage {
 public:
  Storage() = default;
  Storage(const Storage&) = delete;
  Storage& operator=(const Storage&) = delete;
  Storage(Storage&&) noexcept;
  Storage& operator=(Storage&&) noexcept;
  ~Storage();

  static Result<std::shared_ptr<Storage>> allocate(hal::Allocator& allocator, size_t bytes, size_t alignment,
                                                   Device device);

  void* data() { return data_; }
  const void* data() const { return data_; }
  size_t nbytes() const { return nbytes_; }
  Device device() const { return device_; }

 private:
  void release() noexcept;
  void* data_ = nullptr;
  size_t nbytes_ = 0;
  Device device_{};
  hal::Allocator* allocator_ = nullptr;  // non-owning; returns data_ on destruction
};

inline constexpr size_t kDefaultAlignment = 64;

}  // namespace frame
