#pragma once
// hal::Event. An event that was never recorded counts as complete: query() is true and synchronize() is Ok
// (reference: include/frame/hal/event.h:13-24).

#include <frame/core/macros.h>
#include <frame/core/status.h>

namespace frame::hal {

class FRAME_API Event {
 public:
  virtual ~Event() = default;
  virtual bool query() const = 0;
  virtual Status synchronize() = 0;
};

}  // namespace frame::hal
