// backend.h — the reference's backend interface, restated for the ROCm backend.
//
// These are the types IBackend::dispatch trades in, with the reference's names,
// members, enum values and declaration order, so that an object built here is
// called through the reference's vtable and hands the reference's TensorView /
// Attribute / Error objects back and forth unchanged:
//   DType, DeviceType               include/uaii/interfaces/types.hpp:13-37
//   quant::QuantFormat              include/uaii/quant/formats.hpp:11-30
//   kernels::TensorView             include/uaii/kernels/tensor_view.hpp:12-50
//   ir::AttributeType / Attribute   include/uaii/ir/attribute.hpp:11-31
//   BackendCapabilities, IBackend   include/uaii/interfaces/backend.hpp:15-87
// (Error and ErrorCode: error.h.) tests/test_backend_abi.py compiles a program
// against the reference's own headers that drives this library's backend
// through them.
#pragma once

#include "error.h"

#include <cstddef>
#include <cstdint>
#include <string>
#include <variant>
#include <vector>

namespace uaii {

enum class DType { Unknown = 0, F32, F16, BF16, I8, I32, I64, U8, U32, Bool };

enum class DeviceType { Unknown = 0, Cpu, Cuda, Metal, Vulkan, WebGpu, Rocm, Npu, Custom };

namespace quant {
enum class QuantFormat {
  F32 = 0, F16, BF16, INT8, INT4, NF4, MXFP4,
  Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K,
};
}  // namespace quant

namespace kernels {
struct TensorView {
  DType dtype = DType::Unknown;
  const std::int64_t* shape = nullptr;
  std::size_t rank = 0;
  void* data = nullptr;
  std::size_t nbytes = 0;
  // packed GGUF blocks in `data` when quant_format is Q4_0 .. Q6_K
  quant::QuantFormat quant_format = quant::QuantFormat::F32;
  std::int64_t quant_rows = 0;
  std::int64_t quant_cols = 0;

  std::int64_t dim(std::size_t i) const { return i < rank ? shape[i] : 1; }
  std::size_t numel() const {
    if (rank == 0) return 0;
    std::size_t n = 1;
    for (std::size_t i = 0; i < rank; ++i) {
      if (shape[i] < 0) return 0;
      n *= static_cast<std::size_t>(shape[i]);
    }
    return n;
  }
};
}  // namespace kernels

namespace ir {
enum class AttributeType { String = 0, Int, Float, Bool, IntArray, FloatArray };
using AttributeValue = std::variant<std::string, std::int64_t, double, bool, std::vector<std::int64_t>,
                                    std::vector<double>>;
struct Attribute {
  std::string key;
  AttributeType type = AttributeType::String;
  AttributeValue value = std::string{};
};
}  // namespace ir

struct BackendCapabilities {
  std::string name;
  DeviceType device_type = DeviceType::Unknown;
  std::vector<DType> supported_dtypes;
  bool supports_profiling = false;
  bool supports_async = false;
  bool host_fallback = false;
  bool native_available = false;
  bool attention_host_fallback = false;
  std::string details;
};

class IBackend {
 public:
  virtual ~IBackend() = default;
  virtual std::string name() const = 0;
  virtual DeviceType device_type() const = 0;
  virtual Error initialize() = 0;
  virtual void shutdown() noexcept = 0;
  virtual BackendCapabilities capabilities() const = 0;
  virtual Error allocate(std::size_t bytes, void** out_ptr) = 0;
  virtual Error free(void* ptr) noexcept = 0;
  virtual Error copy_h2d(const void* host, void* device, std::size_t bytes) {
    (void)host; (void)device; (void)bytes;
    return Error::make(ErrorCode::NotImplemented, "copy_h2d not implemented");
  }
  virtual Error copy_h2d_async(const void* host, void* device, std::size_t bytes) {
    (void)host; (void)device; (void)bytes;
    return Error::make(ErrorCode::NotImplemented, "copy_h2d_async not implemented");
  }
  virtual Error copy_d2h(const void* device, void* host, std::size_t bytes) {
    (void)device; (void)host; (void)bytes;
    return Error::make(ErrorCode::NotImplemented, "copy_d2h not implemented");
  }
  virtual Error copy_d2d(const void* src, void* dst, std::size_t bytes) {
    (void)src; (void)dst; (void)bytes;
    return Error::make(ErrorCode::NotImplemented, "copy_d2d not implemented");
  }
  virtual Error synchronize() = 0;
  virtual Error dispatch(const std::string& op_name, const std::string& op_version,
                         const std::vector<kernels::TensorView>& inputs,
                         std::vector<kernels::TensorView>* outputs,
                         const std::vector<ir::Attribute>& attrs) = 0;
  virtual bool uses_host_fallback() const noexcept { return false; }
  virtual bool attention_host_fallback() const noexcept { return false; }
};

}  // namespace uaii
