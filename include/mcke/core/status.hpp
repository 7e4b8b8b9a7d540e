// mcke/core/status.hpp -- error vocabulary of the host API.
//
// Mirrors the reference's include/mcke/core/status.hpp:42-190: StatusCode (same
// numeric values, which are also the C-ABI's return codes), Status, StatusOr<T>,
// the *Error constructors and the MCKE_RETURN_IF_ERROR / MCKE_ASSIGN_OR_RETURN
// propagation macros.  The reference's kCudaError slot is kDeviceError here and
// carries HIP runtime errors; CudaError() is kept as an alias of DeviceError().
#pragma once

#include <cassert>
#include <cstdint>
#include <optional>
#include <stdexcept>
#include <string>
#include <string_view>
#include <utility>

namespace mcke {

enum class StatusCode : std::uint8_t {
  kOk = 0,
  kOutOfMemory = 1,
  kInvalidArgument = 2,
  kFailedPrecondition = 3,
  kUnimplemented = 4,
  kInternal = 5,
  kDeviceError = 6,
  kCudaError = kDeviceError,   // the reference's name for the same slot
};

[[nodiscard]] constexpr std::string_view to_string(StatusCode c) noexcept {
  switch (c) {
    case StatusCode::kOk: return "Ok";
    case StatusCode::kOutOfMemory: return "OutOfMemory";
    case StatusCode::kInvalidArgument: return "InvalidArgument";
    case StatusCode::kFailedPrecondition: return "FailedPrecondition";
    case StatusCode::kUnimplemented: return "Unimplemented";
    case StatusCode::kInternal: return "Internal";
    case StatusCode::kDeviceError: return "DeviceError";
  }
  return "Unknown";
}

class [[nodiscard]] Status {
 public:
  Status() = default;
  Status(StatusCode code, std::string message) : code_(code), message_(std::move(message)) {}

  [[nodiscard]] bool ok() const noexcept { return code_ == StatusCode::kOk; }
  [[nodiscard]] StatusCode code() const noexcept { return code_; }
  [[nodiscard]] const std::string& message() const noexcept { return message_; }
  [[nodiscard]] std::string to_string() const {
    return ok() ? std::string("Ok") : std::string(mcke::to_string(code_)) + ": " + message_;
  }
  void throw_if_error() const {
    if (!ok()) throw std::runtime_error(to_string());
  }

 private:
  StatusCode code_ = StatusCode::kOk;
  std::string message_;
};

[[nodiscard]] inline Status OkStatus() { return Status{}; }
[[nodiscard]] inline Status OutOfMemoryError(std::string m) { return {StatusCode::kOutOfMemory, std::move(m)}; }
[[nodiscard]] inline Status InvalidArgumentError(std::string m) { return {StatusCode::kInvalidArgument, std::move(m)}; }
[[nodiscard]] inline Status FailedPreconditionError(std::string m) { return {StatusCode::kFailedPrecondition, std::move(m)}; }
[[nodiscard]] inline Status UnimplementedError(std::string m) { return {StatusCode::kUnimplemented, std::move(m)}; }
[[nodiscard]] inline Status InternalError(std::string m) { return {StatusCode::kInternal, std::move(m)}; }
[[nodiscard]] inline Status DeviceError(std::string m) { return {StatusCode::kDeviceError, std::move(m)}; }
[[nodiscard]] inline Status CudaError(std::string m) { return DeviceError(std::move(m)); }

template <typename T>
class [[nodiscard]] StatusOr {
 public:
  StatusOr(T value) : value_(std::move(value)) {}   // NOLINT: implicit by design
  StatusOr(Status status) : status_(std::move(status)) {   // NOLINT
    assert(!status_.ok() && "StatusOr must not hold an OK status without a value");
  }
  [[nodiscard]] bool ok() const noexcept { return value_.has_value(); }
  [[nodiscard]] const Status& status() const noexcept { return status_; }
  [[nodiscard]] T& value() { return value_.value(); }
  [[nodiscard]] const T& value() const { return value_.value(); }
  [[nodiscard]] T& operator*() noexcept { return *value_; }
  [[nodiscard]] const T& operator*() const noexcept { return *value_; }
  T* operator->() noexcept { return &*value_; }
  const T* operator->() const noexcept { return &*value_; }
  [[nodiscard]] T value_or_throw() && {
    status_.throw_if_error();
    return std::move(*value_);
  }

 private:
  Status status_{};
  std::optional<T> value_{};
};

}  // namespace mcke

#define MCKE_RETURN_IF_ERROR(expr)                 \
  do {                                             \
    ::mcke::Status _mcke_status = (expr);          \
    if (!_mcke_status.ok()) return _mcke_status;   \
  } while (0)

#define MCKE_CONCAT_INNER(a, b) a##b
#define MCKE_CONCAT(a, b) MCKE_CONCAT_INNER(a, b)
#define MCKE_ASSIGN_OR_RETURN_IMPL(tmp, lhs, expr) \
  auto tmp = (expr);                               \
  if (!tmp.ok()) return tmp.status();              \
  lhs = std::move(*tmp)
#define MCKE_ASSIGN_OR_RETURN(lhs, expr) \
  MCKE_ASSIGN_OR_RETURN_IMPL(MCKE_CONCAT(_mcke_or_, __LINE__), lhs, expr)
