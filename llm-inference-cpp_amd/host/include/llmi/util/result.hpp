// Value-or-error type with the reference's interface
// (include/llmi/util/result.hpp:9-39): errors are values, never aborts.
#pragma once

#include <string>
#include <utility>
#include <variant>

namespace llmi {

struct Error {
  std::string message;
};

template <typename T>
class Result {
 public:
  Result(T value) : v_(std::move(value)) {}      // NOLINT(google-explicit-constructor)
  Result(Error error) : v_(std::move(error)) {}  // NOLINT(google-explicit-constructor)

  [[nodiscard]] bool ok() const { return v_.index() == 0; }
  explicit operator bool() const { return ok(); }

  [[nodiscard]] T& value() & { return std::get<0>(v_); }
  [[nodiscard]] const T& value() const& { return std::get<0>(v_); }
  [[nodiscard]] T&& value() && { return std::get<0>(std::move(v_)); }
  T* operator->() { return &value(); }
  const T* operator->() const { return &value(); }
  T& operator*() & { return value(); }
  const T& operator*() const& { return value(); }

  [[nodiscard]] const std::string& error() const { return std::get<1>(v_).message; }

 private:
  std::variant<T, Error> v_;
};

inline Error fail(std::string message) { return Error{std::move(message)}; }

}  // namespace llmi
