// llmi::Result<T> / llmi::Error / llmi::fail: the value-or-error type the
// reference's forward* and load signatures return
// (include/llmi/util/result.hpp:9-39 of the reference).
//
// Built inside the reference engine (LLMI_GPU_WITH_REFERENCE_MODEL, this
// directory ahead of the reference's include directory), the reference's own
// header is used, so both halves of the engine share one type.  Standalone,
// this is an implementation of the same interface: a Result holds either a T
// or an Error (never both), ok() / operator bool tell which, value() and the
// dereference operators reach the T, error() the message.
#pragma once

#if defined(LLMI_GPU_WITH_REFERENCE_MODEL)
#include_next <llmi/util/result.hpp>
#else

#include <optional>
#include <string>
#include <utility>

namespace llmi {

struct Error {
  std::string message;
};

template <typename T>
class Result {
 public:
  Result(T value) : val_(std::in_place, std::move(value)) {}  // NOLINT(google-explicit-constructor)
  Result(Error error) : err_(std::move(error.message)) {}     // NOLINT(google-explicit-constructor)

  [[nodiscard]] bool ok() const { return val_.has_value(); }
  explicit operator bool() const { return ok(); }

  // Reaching the value of a failed Result throws std::bad_optional_access.
  [[nodiscard]] T& value() & { return val_.value(); }
  [[nodiscard]] const T& value() const& { return val_.value(); }
  [[nodiscard]] T&& value() && { return std::move(val_.value()); }
  T* operator->() { return &value(); }
  const T* operator->() const { return &value(); }
  T& operator*() & { return value(); }
  const T& operator*() const& { return value(); }

  // The failure message; empty for a Result that holds a value.
  [[nodiscard]] const std::string& error() const { return err_; }

 private:
  std::optional<T> val_;
  std::string err_;
};

inline Error fail(std::string message) { return Error{std::move(message)}; }

}  // namespace llmi

#endif  // LLMI_GPU_WITH_REFERENCE_MODEL
