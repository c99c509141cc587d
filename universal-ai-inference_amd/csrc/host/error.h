// error.h — error convention of the host runtime.
//
// Same categories and numbering as the reference's uaii::Error / ErrorCode
// (include/uaii/core/error.hpp:12-55), which the C ABI maps 1:1 onto
// uaii_status (libs/uaii-capi/src/capi.cpp:27-39). No exceptions cross the API.
#pragma once

#include <hip/hip_runtime_api.h>

#include <string>
#include <utility>

namespace uaii {

enum class ErrorCode {
  Ok = 0,
  InvalidArgument = 1,
  NotFound = 2,
  IoError = 3,
  ConfigError = 4,
  PluginError = 5,
  AbiMismatch = 6,
  NotImplemented = 7,
  Internal = 8,
};

class Error {
 public:
  Error() = default;
  Error(ErrorCode code, std::string message) : code_(code), message_(std::move(message)) {}
  static Error success() { return Error{}; }
  static Error make(ErrorCode code, std::string message) { return Error{code, std::move(message)}; }
  bool ok() const noexcept { return code_ == ErrorCode::Ok; }
  ErrorCode code() const noexcept { return code_; }
  const std::string& message() const noexcept { return message_; }
  std::string to_string() const;

 private:
  ErrorCode code_ = ErrorCode::Ok;
  std::string message_;
};

const char* to_string(ErrorCode code) noexcept;

// HIP failures surface as Internal errors naming the call (the reference maps
// HIP status the same way, libs/uaii-backends/src/rocm_runtime_api.cpp:37-43).
inline Error hip_error(hipError_t st, const char* what) {
  if (st == hipSuccess) return Error::success();
  return Error::make(ErrorCode::Internal, std::string(what) + ": " + hipGetErrorString(st));
}

#define UAII_TRY(expr)                 \
  do {                                 \
    ::uaii::Error _e = (expr);         \
    if (!_e.ok()) return _e;           \
  } while (0)

#define UAII_HIP(expr)                                     \
  do {                                                     \
    hipError_t _st = (expr);                               \
    if (_st != hipSuccess) return ::uaii::hip_error(_st, #expr); \
  } while (0)

}  // namespace uaii
