// rocm_backend.h — IBackend for one MI355X: the reference's operators, one per
// dispatch, on the HIP kernels of this library.
//
// Replaces RocmBackend (libs/uaii-backends/src/rocm_backend.cpp:8-132), whose
// native path never ran and whose dispatch staged everything through the host
// CPU kernels. Here every operator the reference's decoder graph emits
// (gguf.cpp:916-1209: Embedding, RMSNorm, MatMul with packed or f32 weights,
// Add, Mul, Silu, Gelu, RoPE, Attention with the KV cache, Softmax, Identity)
// runs on the device; an operator or form this backend does not run returns
// NotImplemented, never a host computation.
//
// Residency, as in the reference's CUDA backend (cuda_backend.cpp:166-207): a
// TensorView may hold device memory (used in place) or host memory, which the
// reference's Session allocates. Host activations are staged through a device
// arena per dispatch and host outputs copied back before dispatch returns.
// MatMul's B operand and Embedding's table are weights: uploaded (and re-laid
// out for the GEMV) once per (address, size, format, shape) and reused; a caller
// that rewrites such a buffer calls invalidate_weight.
//
// KV cache: the reference's Attention appends to the thread's active
// runtime::KvCache (dispatch.cpp:219-231), a host object this library cannot
// reach. The backend keeps the cache on the device instead (head-major
// [n_kv][max_seq][head_dim] per layer, f32 as the reference's or f16) with the
// reference's semantics: configure / reset / append at past_len per layer /
// commit_step (include/uaii/runtime/kv_cache.hpp:16-190). RoPE's default position
// is its past_len + row, as rope_f32 takes the active cache's (transformer.cpp:
// 176-178). A Session routes its KvCache calls to the hooks below.
#pragma once

#include "backend.h"

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <tuple>
#include <vector>

#define UAII_BACKEND_EXPORT __attribute__((visibility("default")))

struct uaii_hip_weight;

namespace uaii {
namespace backends {

class RocmBackend final : public IBackend {
 public:
  explicit RocmBackend(int device = 0);
  ~RocmBackend() override;
  RocmBackend(const RocmBackend&) = delete;
  RocmBackend& operator=(const RocmBackend&) = delete;

  std::string name() const override { return "rocm"; }
  DeviceType device_type() const override { return DeviceType::Rocm; }
  Error initialize() override;
  void shutdown() noexcept override;
  BackendCapabilities capabilities() const override;
  Error allocate(std::size_t bytes, void** out_ptr) override;
  Error free(void* ptr) noexcept override;
  Error copy_h2d(const void* host, void* device, std::size_t bytes) override;
  Error copy_h2d_async(const void* host, void* device, std::size_t bytes) override;
  Error copy_d2h(const void* device, void* host, std::size_t bytes) override;
  Error copy_d2d(const void* src, void* dst, std::size_t bytes) override;
  Error synchronize() override;
  Error dispatch(const std::string& op_name, const std::string& op_version,
                 const std::vector<kernels::TensorView>& inputs, std::vector<kernels::TensorView>* outputs,
                 const std::vector<ir::Attribute>& attrs) override;
  bool uses_host_fallback() const noexcept override { return false; }
  bool attention_host_fallback() const noexcept override { return false; }

  // runtime::KvCache on the device (kv_cache.hpp:27-55, :80-120, :122-125)
  Error configure_kv_cache(std::int64_t n_layers, std::int64_t max_seq, std::int64_t kv_dim,
                           std::int64_t n_kv_heads, bool f16);
  void reset_kv_cache() noexcept;
  void commit_kv_step() noexcept;
  std::int64_t kv_past_len() const noexcept { return past_len_; }
  void invalidate_weight(const void* ptr) noexcept;
  hipStream_t stream() const noexcept { return stream_; }

 private:
  struct Arena;
  struct WeightKey {
    const void* ptr;
    std::size_t nbytes;
    int format;
    std::int64_t rows, cols;
    bool transposed;
    bool operator<(const WeightKey& o) const {
      return std::tie(ptr, nbytes, format, rows, cols, transposed) <
             std::tie(o.ptr, o.nbytes, o.format, o.rows, o.cols, o.transposed);
    }
  };

  Error require_ready() const;
  bool on_device(const void* p) const;
  Error stage_in(const kernels::TensorView& t, Arena& ar, const float** dev);
  Error stage_out(kernels::TensorView& t, Arena& ar, float** dev, bool* copy_back);
  Error finish_outputs(std::vector<kernels::TensorView>* outputs, const std::vector<float*>& dev,
                       const std::vector<bool>& copy_back);
  Error weight_for(const kernels::TensorView& b, bool transpose_b, uaii_hip_weight** out);
  Error rope_table(float theta, int head_dim, std::int64_t max_pos, const float** table);

  Error op_matmul(const std::vector<kernels::TensorView>& in, std::vector<kernels::TensorView>* out,
                  const std::vector<ir::Attribute>& attrs);
  Error op_rmsnorm(const std::vector<kernels::TensorView>& in, std::vector<kernels::TensorView>* out,
                   const std::vector<ir::Attribute>& attrs);
  Error op_elementwise(const std::string& op, const std::vector<kernels::TensorView>& in,
                       std::vector<kernels::TensorView>* out);
  Error op_softmax(const std::vector<kernels::TensorView>& in, std::vector<kernels::TensorView>* out,
                   const std::vector<ir::Attribute>& attrs);
  Error op_embedding(const std::vector<kernels::TensorView>& in, std::vector<kernels::TensorView>* out);
  Error op_rope(const std::vector<kernels::TensorView>& in, std::vector<kernels::TensorView>* out,
                const std::vector<ir::Attribute>& attrs);
  Error op_attention(const std::vector<kernels::TensorView>& in, std::vector<kernels::TensorView>* out,
                     const std::vector<ir::Attribute>& attrs);

  int device_ = 0;
  bool ready_ = false;
  hipStream_t stream_ = nullptr;
  std::unique_ptr<Arena> arena_;
  std::vector<std::pair<void*, std::size_t>> device_allocs_;
  std::map<WeightKey, uaii_hip_weight*> weights_;
  // RoPE (cos, sin) tables per (theta bits, head_dim): device table and positions held
  std::map<std::pair<std::uint32_t, int>, std::pair<float*, std::int64_t>> rope_tabs_;
  // KV cache
  void* kv_ = nullptr;
  std::int64_t kv_layers_ = 0, kv_max_seq_ = 0, kv_dim_ = 0, kv_heads_ = 0;
  bool kv_f16_ = false;
  std::int64_t past_len_ = 0, pending_seq_ = 0;
};

// The factory branch create_backend("rocm") would take (factory.cpp:52-80).
UAII_BACKEND_EXPORT Error create_rocm_backend(std::unique_ptr<IBackend>* out, int device = 0);
// Session hooks for its KvCache calls (session.cpp:777-856: configure at
// ensure_kv_cache, reset at the start of generate, commit_step after run);
// InvalidArgument when `backend` is not this library's RocmBackend.
UAII_BACKEND_EXPORT Error rocm_configure_kv_cache(IBackend* backend, std::int64_t n_layers,
                                                  std::int64_t max_seq, std::int64_t kv_dim,
                                                  std::int64_t n_kv_heads, bool f16);
UAII_BACKEND_EXPORT Error rocm_reset_kv_cache(IBackend* backend);
UAII_BACKEND_EXPORT Error rocm_commit_kv_step(IBackend* backend);

}  // namespace backends
}  // namespace uaii
