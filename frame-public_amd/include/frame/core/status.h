#pragma once
// Error model: Status and Result<T>. No exceptions cross the library or the HAL.
// Same enumerators, ordinals and member functions as the reference (include/frame/core/status.h:18-98): the
// C ABI of the kernel library (fh_status) reuses these ordinals.

#include <cstdint>
#include <optional>
#include <string>
#include <string_view>
#include <utility>

#include <frame/core/macros.h>

namespace frame {

enum class ErrorCode : uint8_t {
  kOk = 0,
  kInvalidArgument,
  kNotFound,
  kAlreadyExists,
  kUnimplemented,
  kOutOfMemory,
  kInternal,
  kDeviceError,
};

class FRAME_API Status {
 public:
  Status() = default;
  static Status ok() { return Status(); }
  static Status make(ErrorCode code, std::string_view message) {
    Status s;
    s.code_ = code;
    s.message_ = std::string(message);
    return s;
  }
  bool is_ok() const { return code_ == ErrorCode::kOk; }
  ErrorCode code() const { return code_; }
  std::string_view message() const { return message_; }

 private:
  ErrorCode code_ = ErrorCode::kOk;
  std::string message_;
};

template <typename T>
class Result {
 public:
  Result(T value) : status_(Status::ok()), value_(std::move(value)) {}
  Result(Status status) : status_(std::move(status)) {}

  bool is_ok() const { return status_.is_ok() && value_.has_value(); }
  const Status& status() const { return status_; }
  T& value() {
    FRAME_CHECK(value_.has_value());
    return *value_;
  }
  const T& value() const {
    FRAME_CHECK(value_.has_value());
    return *value_;
  }

 private:
  Status status_;
  std::optional<T> value_;
};

}  // namespace frame

#define FRAME_RETURN_IF_ERROR(expr)                   \
  do {                                                \
    ::frame::Status _frame_status = (expr);           \
    if (!_frame_status.is_ok()) return _frame_status; \
  } while (0)

#define FRAME_UNIMPLEMENTED() (::frame::Status::make(::frame::ErrorCode::kUnimplemented, __func__))
