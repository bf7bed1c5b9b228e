// result.h -- value-or-error for the host layer.  The reference's seam
// returns std::expected<T, std::string> (runtime/executor/backend.h:82-166,
// STYLE.md:33-54: failures are values, nothing throws); this toolchain's
// C++ library predates <expected>, so the host layer carries the same
// contract in this small type: a T, or the failure's message.
#pragma once

#include <string>
#include <utility>
#include <variant>

namespace seeai::host {

struct Error {
  std::string message;
};

template <class T>
class Result {
 public:
  Result(T value) : v_(std::move(value)) {}  // NOLINT: implicit, like expected
  Result(Error e) : v_(std::move(e)) {}      // NOLINT
  explicit operator bool() const { return v_.index() == 0; }
  T& operator*() { return std::get<0>(v_); }
  const T& operator*() const { return std::get<0>(v_); }
  T* operator->() { return &std::get<0>(v_); }
  const T* operator->() const { return &std::get<0>(v_); }
  const std::string& error() const { return std::get<1>(v_).message; }

 private:
  std::variant<T, Error> v_;
};

template <>
class Result<void> {
 public:
  Result() = default;
  Result(Error e) : ok_(false), message_(std::move(e.message)) {}  // NOLINT
  explicit operator bool() const { return ok_; }
  const std::string& error() const { return message_; }

 private:
  bool ok_ = true;
  std::string message_;
};

inline Error Fail(std::string message) { return Error{std::move(message)}; }

}  // namespace seeai::host
