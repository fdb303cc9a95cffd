#pragma once
// hal::Stream: ordered queue of asynchronous device work (reference: include/frame/hal/stream.h:13-29).

#include <frame/core/macros.h>
#include <frame/core/status.h>

namespace frame::hal {

class Event;

class FRAME_API Stream {
 public:
  virtual ~Stream() = default;
  virtual Status synchronize() = 0;            // block until all queued work finished
  virtual Status record(Event& event) = 0;     // mark the current position of the queue
  virtual Status wait(const Event& event) = 0;  // later work waits for `event`
  virtual void* native_handle() = 0;           // hipStream_t for the hip backend; backends only
};

}  // namespace frame::hal
