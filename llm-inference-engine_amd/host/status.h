// Status / StatusOr for the host layer: the reference's error taxonomy
// (src/core/status.h:52-64; values are shared with the C ABI's return codes)
// with a message, no exceptions.
#pragma once

#include <cstdint>
#include <string>
#include <utility>

namespace ehip::host {

enum class StatusCode : std::uint8_t {
  kOk = 0,
  kCancelled = 1,
  kInvalidArgument = 2,
  kNotFound = 3,
  kAlreadyExists = 4,
  kFailedPrecondition = 5,
  kOutOfRange = 6,
  kResourceExhausted = 7,
  kOutOfMemory = 8,
  kUnimplemented = 9,
  kUnavailable = 10,
  kInternal = 11,
};

class [[nodiscard]] Status {
 public:
  Status() = default;
  Status(StatusCode code, std::string message)
      : code_(code), message_(code == StatusCode::kOk ? std::string() : std::move(message)) {}
  static Status Ok() { return Status(); }
  bool ok() const { return code_ == StatusCode::kOk; }
  StatusCode code() const { return code_; }
  const std::string& message() const { return message_; }

 private:
  StatusCode code_ = StatusCode::kOk;
  std::string message_;
};

template <class T>
class [[nodiscard]] StatusOr {
 public:
  StatusOr(T value) : value_(std::move(value)) {}  // NOLINT(implicit)
  StatusOr(Status status) : status_(std::move(status)) {}  // NOLINT(implicit)
  bool ok() const { return status_.ok(); }
  const Status& status() const { return status_; }
  T& value() { return value_; }
  const T& value() const { return value_; }
  T& operator*() { return value_; }
  const T& operator*() const { return value_; }
  T* operator->() { return &value_; }

 private:
  Status status_;
  T value_{};
};

// printf-style message helper.
std::string Format(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

inline Status Error(StatusCode c, std::string msg) { return Status(c, std::move(msg)); }

}  // namespace ehip::host
