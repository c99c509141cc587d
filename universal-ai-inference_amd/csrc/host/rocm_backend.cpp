// rocm_backend.cpp — the reference's operators on one MI355X, one per dispatch.
//
// Operator semantics (names, inputs, attributes and their defaults, shape checks,
// error codes) follow the reference's CPU dispatcher, libs/uaii-kernels/src/
// dispatch.cpp:67-272, and the kernels it calls; the arithmetic runs in this
// library's HIP kernels through the uaii_hip_* launch layer.
#include "rocm_backend.h"

#include "uaii_hip.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <utility>

namespace uaii {
namespace backends {

using kernels::TensorView;

namespace {

// dispatch.cpp:10-39: an attribute counts only with the expected type (floats
// also from ints)
bool attr_bool(const std::vector<ir::Attribute>& attrs, const char* key, bool def) {
  for (const auto& a : attrs)
    if (a.key == key && a.type == ir::AttributeType::Bool) return std::get<bool>(a.value);
  return def;
}

std::int64_t attr_int(const std::vector<ir::Attribute>& attrs, const char* key, std::int64_t def) {
  for (const auto& a : attrs)
    if (a.key == key && a.type == ir::AttributeType::Int) return std::get<std::int64_t>(a.value);
  return def;
}

float attr_float(const std::vector<ir::Attribute>& attrs, const char* key, float def) {
  for (const auto& a : attrs) {
    if (a.key == key && a.type == ir::AttributeType::Float) return static_cast<float>(std::get<double>(a.value));
    if (a.key == key && a.type == ir::AttributeType::Int) return static_cast<float>(std::get<std::int64_t>(a.value));
  }
  return def;
}

Error bad(const std::string& msg) { return Error::make(ErrorCode::InvalidArgument, msg); }
Error unsupported(const std::string& msg) { return Error::make(ErrorCode::NotImplemented, "rocm backend: " + msg); }

Error hip_rc(int rc, const char* what) {
  if (rc == 0) return Error::success();
  if (rc > 0) return hip_error(static_cast<hipError_t>(rc), what);
  return Error::make(rc == -2 ? ErrorCode::NotImplemented : ErrorCode::InvalidArgument,
                     std::string(what) + ": " + uaii_hip_error_string(rc));
}

// GGUF tensor type of a packed QuantFormat (formats.hpp:11-30 -> GGUF ids), -1 if none
int gguf_type(quant::QuantFormat f) {
  switch (f) {
    case quant::QuantFormat::Q4_0: return 2;
    case quant::QuantFormat::Q4_1: return 3;
    case quant::QuantFormat::Q5_0: return 6;
    case quant::QuantFormat::Q5_1: return 7;
    case quant::QuantFormat::Q8_0: return 8;
    case quant::QuantFormat::Q2_K: return 10;
    case quant::QuantFormat::Q3_K: return 11;
    case quant::QuantFormat::Q4_K: return 12;
    case quant::QuantFormat::Q5_K: return 13;
    case quant::QuantFormat::Q6_K: return 14;
    default: return -1;
  }
}

// bytes of one GGUF row of `cols` values (formats.hpp:81-102), 0 if unsupported
std::size_t gguf_row_bytes(int type, std::int64_t cols) {
  int be = 0, bb = 0;
  switch (type) {
    case 0: be = 1; bb = 4; break;
    case 1: be = 1; bb = 2; break;
    case 2: be = 32; bb = 18; break;
    case 3: be = 32; bb = 20; break;
    case 6: be = 32; bb = 22; break;
    case 7: be = 32; bb = 24; break;
    case 8: be = 32; bb = 34; break;
    case 10: be = 256; bb = 84; break;
    case 11: be = 256; bb = 110; break;
    case 12: be = 256; bb = 144; break;
    case 13: be = 256; bb = 176; break;
    case 14: be = 256; bb = 210; break;
    default: return 0;
  }
  if (cols % be) return 0;
  return static_cast<std::size_t>(cols / be) * static_cast<std::size_t>(bb);
}

std::size_t align256(std::size_t n) { return (n + 255) & ~static_cast<std::size_t>(255); }

bool is_f32(const TensorView& t) { return t.dtype == DType::F32 && t.data != nullptr; }

// parse_attn_shape (transformer.cpp:26-48): [batch, dim] or [batch, seq, dim]
struct AttnShape {
  std::int64_t batch = 0, seq = 0, dim = 0;
};
Error attn_shape(const TensorView& t, AttnShape* s, const char* name) {
  if (t.dtype != DType::F32 || t.data == nullptr) return bad(std::string(name) + " f32 required");
  if (t.rank == 2) { *s = {t.dim(0), 1, t.dim(1)}; return Error::success(); }
  if (t.rank == 3) { *s = {t.dim(0), t.dim(1), t.dim(2)}; return Error::success(); }
  return bad(std::string(name) + " expects [batch,seq,dim] or [batch,dim]");
}

}  // namespace

// Device arena for staged host tensors: grown (after the stream drains) when a
// dispatch needs more, bump-allocated within a dispatch.
struct RocmBackend::Arena {
  void* base = nullptr;
  std::size_t cap = 0, used = 0;
  Error reserve(std::size_t bytes, hipStream_t s) {
    used = 0;
    if (bytes <= cap) return Error::success();
    const std::size_t want = std::max(bytes, std::max<std::size_t>(2 * cap, 1 << 20));
    UAII_HIP(hipStreamSynchronize(s));
    if (base) (void)hipFree(base);
    base = nullptr;
    cap = 0;
    UAII_HIP(hipMalloc(&base, want));
    cap = want;
    return Error::success();
  }
  void* take(std::size_t bytes) {
    void* p = static_cast<char*>(base) + used;
    used += align256(bytes);
    return p;
  }
  ~Arena() {
    if (base) (void)hipFree(base);
  }
};

RocmBackend::RocmBackend(int device) : device_(device), arena_(new Arena()) {}

RocmBackend::~RocmBackend() { shutdown(); }

Error RocmBackend::initialize() {
  if (ready_) return Error::success();
  int n = 0;
  UAII_HIP(hipGetDeviceCount(&n));
  if (device_ < 0 || device_ >= n) return bad("rocm device " + std::to_string(device_) + " not present");
  UAII_TRY(hip_rc(uaii_hip_init(device_), "uaii_hip_init"));
  UAII_HIP(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
  ready_ = true;
  return Error::success();
}

void RocmBackend::shutdown() noexcept {
  if (!ready_) return;
  (void)hipStreamSynchronize(stream_);
  for (auto& kv : weights_) uaii_hip_weight_destroy(kv.second);
  weights_.clear();
  for (auto& kv : rope_tabs_) (void)hipFree(kv.second.first);
  rope_tabs_.clear();
  for (auto& a : device_allocs_) (void)hipFree(a.first);
  device_allocs_.clear();
  if (kv_) (void)hipFree(kv_);
  kv_ = nullptr;
  kv_layers_ = 0;
  arena_.reset(new Arena());
  (void)hipStreamDestroy(stream_);
  stream_ = nullptr;
  ready_ = false;
}

BackendCapabilities RocmBackend::capabilities() const {
  BackendCapabilities c;
  c.name = "rocm";
  c.device_type = DeviceType::Rocm;
  c.supported_dtypes = {DType::F32, DType::F16};
  c.supports_profiling = false;
  c.supports_async = true;
  c.host_fallback = false;
  c.native_available = ready_;
  c.attention_host_fallback = false;
  c.details = ready_ ? "ROCm backend (native, MI355X kernels); ops: Embedding RMSNorm MatMul Add Mul Silu "
                       "Gelu Identity Softmax RoPE Attention"
                     : "ROCm backend (not initialized)";
  return c;
}

Error RocmBackend::require_ready() const {
  if (!ready_) return bad("rocm backend not initialized");
  return Error::success();
}

Error RocmBackend::allocate(std::size_t bytes, void** out_ptr) {
  UAII_TRY(require_ready());
  if (!out_ptr) return bad("allocate out null");
  UAII_HIP(hipMalloc(out_ptr, bytes));
  device_allocs_.emplace_back(*out_ptr, bytes);
  return Error::success();
}

Error RocmBackend::free(void* ptr) noexcept {
  if (ptr == nullptr) return Error::success();
  for (auto it = device_allocs_.begin(); it != device_allocs_.end(); ++it) {
    if (it->first == ptr) {
      (void)hipStreamSynchronize(stream_);
      const hipError_t e = hipFree(ptr);
      device_allocs_.erase(it);
      return hip_error(e, "hipFree");
    }
  }
  return Error::make(ErrorCode::NotFound, "pointer not owned by ROCm backend");
}

Error RocmBackend::copy_h2d(const void* host, void* device, std::size_t bytes) {
  UAII_TRY(require_ready());
  UAII_HIP(hipMemcpyAsync(device, host, bytes, hipMemcpyHostToDevice, stream_));
  UAII_HIP(hipStreamSynchronize(stream_));
  return Error::success();
}

Error RocmBackend::copy_h2d_async(const void* host, void* device, std::size_t bytes) {
  UAII_TRY(require_ready());
  UAII_HIP(hipMemcpyAsync(device, host, bytes, hipMemcpyHostToDevice, stream_));
  return Error::success();
}

Error RocmBackend::copy_d2h(const void* device, void* host, std::size_t bytes) {
  UAII_TRY(require_ready());
  UAII_HIP(hipMemcpyAsync(host, device, bytes, hipMemcpyDeviceToHost, stream_));
  UAII_HIP(hipStreamSynchronize(stream_));
  return Error::success();
}

Error RocmBackend::copy_d2d(const void* src, void* dst, std::size_t bytes) {
  UAII_TRY(require_ready());
  UAII_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, stream_));
  return Error::success();
}

Error RocmBackend::synchronize() {
  UAII_TRY(require_ready());
  UAII_HIP(hipStreamSynchronize(stream_));
  return Error::success();
}

bool RocmBackend::on_device(const void* p) const {
  hipPointerAttribute_t a{};
  if (hipPointerGetAttributes(&a, p) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return a.type == hipMemoryTypeDevice || a.type == hipMemoryTypeManaged;
}

Error RocmBackend::stage_in(const TensorView& t, Arena& ar, const float** dev) {
  if (t.data == nullptr) return bad("dispatch: input without data");
  if (on_device(t.data)) {
    *dev = static_cast<const float*>(t.data);
    return Error::success();
  }
  void* d = ar.take(t.nbytes);
  UAII_HIP(hipMemcpyAsync(d, t.data, t.nbytes, hipMemcpyHostToDevice, stream_));
  *dev = static_cast<const float*>(d);
  return Error::success();
}

Error RocmBackend::stage_out(TensorView& t, Arena& ar, float** dev, bool* copy_back) {
  if (t.data == nullptr) return bad("dispatch: output without data");
  if (on_device(t.data)) {
    *dev = static_cast<float*>(t.data);
    *copy_back = false;
    return Error::success();
  }
  *dev = static_cast<float*>(ar.take(t.nbytes));
  *copy_back = true;
  return Error::success();
}

Error RocmBackend::finish_outputs(std::vector<TensorView>* outputs, const std::vector<float*>& dev,
                                  const std::vector<bool>& copy_back) {
  bool any = false;
  for (std::size_t i = 0; i < dev.size(); ++i) {
    if (!copy_back[i]) continue;
    TensorView& t = (*outputs)[i];
    UAII_HIP(hipMemcpyAsync(t.data, dev[i], t.nbytes, hipMemcpyDeviceToHost, stream_));
    any = true;
  }
  // host outputs are complete when dispatch returns; device-only dispatches stay
  // queued on the backend's stream (synchronize() waits for them)
  if (any) UAII_HIP(hipStreamSynchronize(stream_));
  return Error::success();
}

void RocmBackend::invalidate_weight(const void* ptr) noexcept {
  for (auto it = weights_.begin(); it != weights_.end();) {
    if (it->first.ptr == ptr) {
      (void)hipStreamSynchronize(stream_);
      uaii_hip_weight_destroy(it->second);
      it = weights_.erase(it);
    } else {
      ++it;
    }
  }
}

// A MatMul B operand or an Embedding table as a device weight [rows = N][cols = K].
Error RocmBackend::weight_for(const TensorView& b, bool transpose_b, uaii_hip_weight** out) {
  const int qt = gguf_type(b.quant_format);
  int type;
  std::int64_t N, K;
  bool transposed = false;
  if (qt >= 0) {
    if (!transpose_b) return bad("quant_gemm expects transpose_b=true (B is [N,K] packed)");
    type = qt;
    N = b.quant_rows > 0 ? b.quant_rows : b.dim(0);
    K = b.quant_cols > 0 ? b.quant_cols : b.dim(1);
  } else if ((b.dtype == DType::F32 || b.dtype == DType::F16) && b.rank == 2) {
    type = b.dtype == DType::F32 ? 0 : 1;
    N = transpose_b ? b.dim(0) : b.dim(1);
    K = transpose_b ? b.dim(1) : b.dim(0);
    transposed = !transpose_b;
  } else {
    return unsupported("MatMul B of dtype " + std::to_string(static_cast<int>(b.dtype)) + " rank " +
                       std::to_string(b.rank));
  }
  const std::size_t rb = gguf_row_bytes(type, K);
  if (N <= 0 || K <= 0 || rb == 0) return bad("weight shape " + std::to_string(N) + "x" + std::to_string(K));
  const std::size_t need = rb * static_cast<std::size_t>(N);
  if (b.data == nullptr || b.nbytes < need) return bad("weight buffer smaller than its shape");
  const WeightKey key{b.data, b.nbytes, type, N, K, transposed};
  auto it = weights_.find(key);
  if (it != weights_.end()) {
    *out = it->second;
    return Error::success();
  }
  // host bytes of the rows (device-resident weights are read back once)
  std::vector<std::uint8_t> host;
  const std::uint8_t* src = static_cast<const std::uint8_t*>(b.data);
  if (on_device(b.data)) {
    host.resize(need);
    UAII_HIP(hipStreamSynchronize(stream_));
    UAII_HIP(hipMemcpy(host.data(), b.data, need, hipMemcpyDeviceToHost));
    src = host.data();
  }
  std::vector<std::uint8_t> tr;
  if (transposed) {  // [K][N] -> [N][K]
    const std::size_t es = type == 0 ? 4 : 2;
    tr.resize(need);
    for (std::int64_t k = 0; k < K; ++k)
      for (std::int64_t n = 0; n < N; ++n)
        std::memcpy(&tr[(static_cast<std::size_t>(n) * K + k) * es], src + (static_cast<std::size_t>(k) * N + n) * es,
                    es);
    src = tr.data();
  }
  uaii_hip_weight* w = nullptr;
  UAII_TRY(hip_rc(uaii_hip_weight_create(type, src, N, K, &w), "uaii_hip_weight_create"));
  weights_[key] = w;
  *out = w;
  return Error::success();
}

Error RocmBackend::rope_table(float theta, int head_dim, std::int64_t max_pos, const float** table) {
  std::uint32_t tb;
  std::memcpy(&tb, &theta, 4);
  auto& slot = rope_tabs_[{tb, head_dim}];
  if (slot.second < max_pos) {
    std::int64_t cap = std::max<std::int64_t>(slot.second, 256);
    while (cap < max_pos) cap *= 2;
    UAII_HIP(hipStreamSynchronize(stream_));
    if (slot.first) (void)hipFree(slot.first);
    slot = {nullptr, 0};
    float* t = nullptr;
    UAII_HIP(hipMalloc(&t, static_cast<std::size_t>(cap) * static_cast<std::size_t>(head_dim) * 4));
    const int rc = uaii_hip_rope_table(theta, head_dim, cap, t);
    if (rc) {
      (void)hipFree(t);
      return hip_rc(rc, "uaii_hip_rope_table");
    }
    slot = {t, cap};
  }
  *table = slot.first;
  return Error::success();
}

Error RocmBackend::configure_kv_cache(std::int64_t n_layers, std::int64_t max_seq, std::int64_t kv_dim,
                                      std::int64_t n_kv_heads, bool f16) {
  UAII_TRY(require_ready());
  // KvCache::configure (kv_cache.hpp:27-55)
  if (n_layers <= 0 || max_seq <= 0 || kv_dim <= 0 || n_kv_heads <= 0)
    return bad("KvCache::configure invalid dims");
  if (kv_dim % n_kv_heads != 0) return bad("KvCache dim not divisible by n_heads");
  if (max_seq > INT32_MAX) return bad("KvCache max_seq beyond 2^31 positions");
  UAII_HIP(hipStreamSynchronize(stream_));
  if (kv_) (void)hipFree(kv_);
  kv_ = nullptr;
  kv_layers_ = 0;
  const std::size_t bytes = static_cast<std::size_t>(n_layers) * 2 * static_cast<std::size_t>(max_seq) *
                            static_cast<std::size_t>(kv_dim) * (f16 ? 2 : 4);
  UAII_HIP(hipMalloc(&kv_, bytes));
  UAII_HIP(hipMemsetAsync(kv_, 0, bytes, stream_));
  kv_layers_ = n_layers;
  kv_max_seq_ = max_seq;
  kv_dim_ = kv_dim;
  kv_heads_ = n_kv_heads;
  kv_f16_ = f16;
  past_len_ = 0;
  pending_seq_ = 0;
  return Error::success();
}

void RocmBackend::reset_kv_cache() noexcept {
  // KvCache::reset (kv_cache.hpp:57-62): positions forgotten (every read is
  // bounded by past_len, so the stale contents are never attended)
  past_len_ = 0;
  pending_seq_ = 0;
}

void RocmBackend::commit_kv_step() noexcept {
  past_len_ += pending_seq_;
  pending_seq_ = 0;
}

Error RocmBackend::dispatch(const std::string& op_name, const std::string& /*op_version*/,
                            const std::vector<TensorView>& inputs, std::vector<TensorView>* outputs,
                            const std::vector<ir::Attribute>& attrs) {
  UAII_TRY(require_ready());
  if (outputs == nullptr || outputs->empty()) return bad("dispatch outputs empty");
  if (op_name == "MatMul") return op_matmul(inputs, outputs, attrs);
  if (op_name == "RMSNorm") return op_rmsnorm(inputs, outputs, attrs);
  if (op_name == "Add" || op_name == "Mul" || op_name == "Silu" || op_name == "Gelu" || op_name == "Identity")
    return op_elementwise(op_name, inputs, outputs);
  if (op_name == "Softmax") return op_softmax(inputs, outputs, attrs);
  if (op_name == "Embedding") return op_embedding(inputs, outputs);
  if (op_name == "RoPE") return op_rope(inputs, outputs, attrs);
  if (op_name == "Attention") return op_attention(inputs, outputs, attrs);
  return unsupported("op '" + op_name + "' has no device kernel here");
}

Error RocmBackend::op_matmul(const std::vector<TensorView>& in, std::vector<TensorView>* out,
                             const std::vector<ir::Attribute>& attrs) {
  if (in.size() != 2 || out->size() != 1) return bad("MatMul expects 2 inputs / 1 output");
  if (attr_bool(attrs, "transpose_a", false)) return unsupported("MatMul transpose_a");
  const TensorView& a = in[0];
  TensorView& c = (*out)[0];
  if (!is_f32(a) || a.rank != 2) return bad("quant_gemm A must be f32 [M,K]");
  if (c.dtype != DType::F32 || c.rank != 2 || c.data == nullptr) return bad("quant_gemm C must be f32");
  uaii_hip_weight* w = nullptr;
  UAII_TRY(weight_for(in[1], attr_bool(attrs, "transpose_b", false), &w));
  const std::int64_t M = a.dim(0), K = a.dim(1);
  const TensorView& b = in[1];
  const bool q = gguf_type(b.quant_format) >= 0;
  const bool tb = attr_bool(attrs, "transpose_b", false);
  const std::int64_t N = q ? (b.quant_rows > 0 ? b.quant_rows : b.dim(0)) : (tb ? b.dim(0) : b.dim(1));
  const std::int64_t Bk = q ? (b.quant_cols > 0 ? b.quant_cols : b.dim(1)) : (tb ? b.dim(1) : b.dim(0));
  if (K != Bk || c.dim(0) != M || c.dim(1) != N) return bad("quant_gemm shape mismatch");
  if (a.nbytes < static_cast<std::size_t>(M * K) * 4 || c.nbytes < static_cast<std::size_t>(M * N) * 4)
    return bad("MatMul buffer smaller than its shape");
  Arena& ar = *arena_;
  UAII_TRY(ar.reserve(align256(a.nbytes) + align256(c.nbytes), stream_));
  const float* ad = nullptr;
  float* cd = nullptr;
  bool back = false;
  UAII_TRY(stage_in(a, ar, &ad));
  UAII_TRY(stage_out(c, ar, &cd, &back));
  if (M == 1) UAII_TRY(hip_rc(uaii_hip_gemv(w, ad, cd, stream_), "uaii_hip_gemv"));
  else UAII_TRY(hip_rc(uaii_hip_gemm(w, ad, M, cd, stream_), "uaii_hip_gemm"));
  return finish_outputs(out, {cd}, {back});
}

Error RocmBackend::op_rmsnorm(const std::vector<TensorView>& in, std::vector<TensorView>* out,
                              const std::vector<ir::Attribute>& attrs) {
  if (in.empty() || out->size() != 1) return bad("RMSNorm arity");
  const TensorView& x = in[0];
  TensorView& y = (*out)[0];
  // check_last_axis_norm (norm.cpp)
  if (!is_f32(x) || y.dtype != DType::F32 || y.data == nullptr || x.rank == 0 || x.numel() != y.numel())
    return bad("RMSNorm f32 shape");
  const std::int64_t axis = x.dim(x.rank - 1);
  const std::int64_t rows = axis > 0 ? static_cast<std::int64_t>(x.numel()) / axis : 0;
  const TensorView* w = in.size() > 1 ? &in[1] : nullptr;
  if (w && (w->dtype != DType::F32 || static_cast<std::int64_t>(w->numel()) != axis))
    return bad("RMSNorm weight shape");
  Arena& ar = *arena_;
  UAII_TRY(ar.reserve(align256(x.nbytes) + align256(y.nbytes) + (w ? align256(w->nbytes) : 0), stream_));
  const float *xd = nullptr, *wd = nullptr;
  float* yd = nullptr;
  bool back = false;
  UAII_TRY(stage_in(x, ar, &xd));
  if (w) UAII_TRY(stage_in(*w, ar, &wd));
  UAII_TRY(stage_out(y, ar, &yd, &back));
  UAII_TRY(hip_rc(uaii_hip_rmsnorm(xd, wd, yd, rows, axis, attr_float(attrs, "eps", 1e-5f), stream_),
                  "uaii_hip_rmsnorm"));
  return finish_outputs(out, {yd}, {back});
}

Error RocmBackend::op_elementwise(const std::string& op, const std::vector<TensorView>& in,
                                  std::vector<TensorView>* out) {
  const bool bin = op == "Add" || op == "Mul";
  if (in.size() != (bin ? 2u : 1u) || out->size() != 1) return bad(op + " arity");
  TensorView& y = (*out)[0];
  // check_same_f32 / check_unary_f32 (elementwise.cpp:10-41)
  if (!is_f32(in[0]) || (bin && !is_f32(in[1])) || y.dtype != DType::F32 || y.data == nullptr)
    return bad(bin ? "elementwise requires f32" : "unary requires f32");
  const std::size_t n = in[0].numel();
  if ((bin && in[1].numel() != n) || y.numel() != n)
    return bad(bin ? "elementwise numel mismatch" : "unary numel mismatch");
  Arena& ar = *arena_;
  UAII_TRY(ar.reserve(align256(in[0].nbytes) + (bin ? align256(in[1].nbytes) : 0) + align256(y.nbytes), stream_));
  const float *ad = nullptr, *bd = nullptr;
  float* yd = nullptr;
  bool back = false;
  UAII_TRY(stage_in(in[0], ar, &ad));
  if (bin) UAII_TRY(stage_in(in[1], ar, &bd));
  UAII_TRY(stage_out(y, ar, &yd, &back));
  const std::int64_t nn = static_cast<std::int64_t>(n);
  int rc = 0;
  if (op == "Add") rc = uaii_hip_add(ad, bd, yd, nn, stream_);
  else if (op == "Mul") rc = uaii_hip_mul(ad, bd, yd, nn, stream_);
  else if (op == "Silu") rc = uaii_hip_silu(ad, yd, nn, stream_);
  else if (op == "Gelu") rc = uaii_hip_gelu(ad, yd, nn, stream_);
  else if (ad != yd) rc = (int)hipMemcpyAsync(yd, ad, n * 4, hipMemcpyDeviceToDevice, stream_);
  UAII_TRY(hip_rc(rc, op.c_str()));
  return finish_outputs(out, {yd}, {back});
}

Error RocmBackend::op_softmax(const std::vector<TensorView>& in, std::vector<TensorView>* out,
                              const std::vector<ir::Attribute>& attrs) {
  if (in.size() != 1 || out->size() != 1) return bad("Softmax expects 1 in / 1 out");
  const TensorView& x = in[0];
  TensorView& y = (*out)[0];
  if (!is_f32(x) || y.dtype != DType::F32 || y.data == nullptr) return bad("softmax requires f32");
  if (x.rank == 0 || x.rank != y.rank) return bad("softmax rank mismatch");
  for (std::size_t i = 0; i < x.rank; ++i)
    if (x.dim(i) != y.dim(i)) return bad("softmax shape mismatch");
  int ax = static_cast<int>(attr_int(attrs, "axis", -1));
  if (ax < 0) ax += static_cast<int>(x.rank);
  if (ax < 0 || ax >= static_cast<int>(x.rank)) return bad("softmax axis out of range");
  if (ax != static_cast<int>(x.rank) - 1) return unsupported("Softmax over a non-last axis");
  const std::int64_t n = x.dim(x.rank - 1);
  const std::int64_t rows = n > 0 ? static_cast<std::int64_t>(x.numel()) / n : 0;
  Arena& ar = *arena_;
  UAII_TRY(ar.reserve(align256(x.nbytes) + align256(y.nbytes), stream_));
  const float* xd = nullptr;
  float* yd = nullptr;
  bool back = false;
  UAII_TRY(stage_in(x, ar, &xd));
  UAII_TRY(stage_out(y, ar, &yd, &back));
  for (std::int64_t r = 0; r < rows; ++r)
    UAII_TRY(hip_rc(uaii_hip_softmax(xd + r * n, yd + r * n, n, stream_), "uaii_hip_softmax"));
  return finish_outputs(out, {yd}, {back});
}

Error RocmBackend::op_embedding(const std::vector<TensorView>& in, std::vector<TensorView>* out) {
  if (in.size() != 2 || out->size() != 1) return bad("Embedding arity");
  const TensorView& tok = in[0];
  const TensorView& w = in[1];
  TensorView& y = (*out)[0];
  // embedding_f32 (transformer.cpp:61-142)
  if (tok.data == nullptr || w.data == nullptr || y.data == nullptr) return bad("embedding null");
  if (tok.dtype != DType::F32 || y.dtype != DType::F32) return bad("embedding requires f32 tokens/out");
  if (w.rank != 2 || tok.rank != 2) return bad("embedding rank (tokens/weight)");
  const std::int64_t vocab = w.quant_rows > 0 ? w.quant_rows : w.dim(0);
  const std::int64_t dim = w.quant_cols > 0 ? w.quant_cols : w.dim(1);
  const std::int64_t batch = tok.dim(0), seq = tok.dim(1);
  if (y.rank == 3) {
    if (y.dim(0) != batch || y.dim(1) != seq || y.dim(2) != dim) return bad("embedding out shape [B,S,D]");
  } else if (y.rank == 2) {
    if (seq == 1 && (y.dim(0) != batch || y.dim(1) != dim)) return bad("embedding out shape [B,D]");
    if (seq != 1 && (y.dim(0) != batch * seq || y.dim(1) != dim)) return bad("embedding out shape [B*S,D]");
  } else {
    return bad("embedding out rank must be 2 or 3");
  }
  const std::int64_t n = batch * seq;
  std::vector<float> idf(static_cast<std::size_t>(n));
  if (on_device(tok.data)) {
    UAII_HIP(hipStreamSynchronize(stream_));
    UAII_HIP(hipMemcpy(idf.data(), tok.data, static_cast<std::size_t>(n) * 4, hipMemcpyDeviceToHost));
  } else {
    std::memcpy(idf.data(), tok.data, static_cast<std::size_t>(n) * 4);
  }
  std::vector<std::int32_t> ids(static_cast<std::size_t>(n));
  for (std::int64_t i = 0; i < n; ++i) {
    const int id = static_cast<int>(idf[static_cast<std::size_t>(i)]);
    if (id < 0 || id >= static_cast<int>(vocab))
      return bad("embedding token id out of range: " + std::to_string(id) + " vocab=" + std::to_string(vocab));
    ids[static_cast<std::size_t>(i)] = id;
  }
  uaii_hip_weight* dw = nullptr;
  TensorView tv = w;
  if (gguf_type(w.quant_format) < 0 && w.dtype != DType::F32) return bad("embedding weight requires f32");
  UAII_TRY(weight_for(tv, true, &dw));
  Arena& ar = *arena_;
  UAII_TRY(ar.reserve(align256(static_cast<std::size_t>(n) * 4) + align256(y.nbytes), stream_));
  auto* idd = static_cast<std::int32_t*>(ar.take(static_cast<std::size_t>(n) * 4));
  UAII_HIP(hipMemcpyAsync(idd, ids.data(), static_cast<std::size_t>(n) * 4, hipMemcpyHostToDevice, stream_));
  float* yd = nullptr;
  bool back = false;
  UAII_TRY(stage_out(y, ar, &yd, &back));
  UAII_TRY(hip_rc(uaii_hip_embed(dw, idd, n, yd, stream_), "uaii_hip_embed"));
  return finish_outputs(out, {yd}, {back});
}

Error RocmBackend::op_rope(const std::vector<TensorView>& in, std::vector<TensorView>* out,
                           const std::vector<ir::Attribute>& attrs) {
  if (in.empty() || out->size() != 1) return bad("RoPE arity");
  const TensorView& x = in[0];
  TensorView& y = (*out)[0];
  // rope_f32 (transformer.cpp:144-220)
  if (x.data == nullptr || y.data == nullptr) return bad("rope null");
  if (x.dtype != DType::F32 || y.dtype != DType::F32) return bad("rope f32");
  if (x.numel() != y.numel() || x.rank < 2) return bad("rope shape");
  const std::int64_t dim = x.dim(x.rank - 1);
  if (dim % 2 != 0) return bad("rope dim must be even");
  const std::int64_t head_dim = attr_int(attrs, "head_dim", 0);
  const std::int64_t rd = head_dim > 0 ? head_dim : dim;
  if (rd <= 0 || dim % rd != 0 || rd % 2 != 0) return bad("rope head_dim invalid");
  const int mode = static_cast<int>(attr_int(attrs, "mode", 0));
  if (mode != 0 && mode != 2) return unsupported("RoPE mode " + std::to_string(mode));
  const float theta = attr_float(attrs, "theta", 10000.f);
  const std::int64_t rows = static_cast<std::int64_t>(x.numel()) / dim;
  // positions: the cache's past_len + row, or the positions input where it has one
  const std::int64_t base = kv_layers_ > 0 ? past_len_ : 0;
  std::vector<std::int32_t> pos(static_cast<std::size_t>(rows));
  std::vector<float> given;
  const TensorView* pt = in.size() > 1 ? &in[1] : nullptr;
  if (pt && pt->data) {
    given.resize(pt->numel());
    if (on_device(pt->data)) {
      UAII_HIP(hipStreamSynchronize(stream_));
      UAII_HIP(hipMemcpy(given.data(), pt->data, given.size() * 4, hipMemcpyDeviceToHost));
    } else {
      std::memcpy(given.data(), pt->data, given.size() * 4);
    }
  }
  std::int64_t max_pos = 0;
  for (std::int64_t r = 0; r < rows; ++r) {
    float p = static_cast<float>(base + r);
    if (static_cast<std::size_t>(r) < given.size()) p = given[static_cast<std::size_t>(r)];
    if (!(p >= 0.0f) || p != std::floor(p) || p > 2147483647.0f)
      return unsupported("RoPE position " + std::to_string(p) + " (integral positions only)");
    pos[static_cast<std::size_t>(r)] = static_cast<std::int32_t>(p);
    max_pos = std::max<std::int64_t>(max_pos, pos[static_cast<std::size_t>(r)]);
  }
  const float* tab = nullptr;
  UAII_TRY(rope_table(theta, static_cast<int>(rd), max_pos + 1, &tab));
  Arena& ar = *arena_;
  UAII_TRY(ar.reserve(align256(x.nbytes) + align256(y.nbytes) + align256(pos.size() * 4), stream_));
  const float* xd = nullptr;
  float* yd = nullptr;
  bool back = false;
  UAII_TRY(stage_in(x, ar, &xd));
  UAII_TRY(stage_out(y, ar, &yd, &back));
  auto* pd = static_cast<std::int32_t*>(ar.take(pos.size() * 4));
  UAII_HIP(hipMemcpyAsync(pd, pos.data(), pos.size() * 4, hipMemcpyHostToDevice, stream_));
  if (yd != xd) UAII_HIP(hipMemcpyAsync(yd, xd, x.numel() * 4, hipMemcpyDeviceToDevice, stream_));
  UAII_TRY(hip_rc(uaii_hip_rope(yd, rows, dim, static_cast<int>(rd), mode, pd, tab, stream_), "uaii_hip_rope"));
  return finish_outputs(out, {yd}, {back});
}

Error RocmBackend::op_attention(const std::vector<TensorView>& in, std::vector<TensorView>* out,
                                const std::vector<ir::Attribute>& attrs) {
  if (in.size() < 3 || out->empty()) return bad("Attention expects Q,K,V");
  AttnShape qs, ks, vs, os;
  UAII_TRY(attn_shape(in[0], &qs, "attn_q"));
  UAII_TRY(attn_shape(in[1], &ks, "attn_k"));
  UAII_TRY(attn_shape(in[2], &vs, "attn_v"));
  UAII_TRY(attn_shape((*out)[0], &os, "attn_out"));
  if (qs.batch != ks.batch || qs.batch != vs.batch || qs.batch != os.batch || qs.dim != os.dim ||
      ks.dim != vs.dim || qs.seq != os.seq || ks.seq != vs.seq || qs.seq != ks.seq)
    return bad("attention shape mismatch");
  if (qs.batch != 1) return unsupported("Attention with batch " + std::to_string(qs.batch));
  const int nh = static_cast<int>(attr_int(attrs, "num_heads", 1));
  const std::int64_t q_dim = qs.dim, kv_dim = ks.dim, S = qs.seq;
  if (nh <= 0 || q_dim % nh != 0) return bad("invalid num_heads");
  const std::int64_t hd = q_dim / nh;
  if (kv_dim % hd != 0) return bad("kv_dim not divisible by head_dim");
  const int nkv = static_cast<int>(kv_dim / hd);
  if (nkv <= 0 || nh % nkv != 0) return bad("invalid GQA head grouping");
  const float scale = attr_float(attrs, "scale", 0.f);
  if (scale > 0.0f && scale != 1.0f / std::sqrt(static_cast<float>(hd)))
    return unsupported("Attention scale other than 1/sqrt(head_dim)");
  const bool causal = attr_bool(attrs, "causal", true);
  const bool use_kv = attr_bool(attrs, "use_kv_cache", false);
  const std::int64_t layer = attr_int(attrs, "layer_id", -1);
  Arena& ar = *arena_;

  if (in.size() < 5 && use_kv && kv_layers_ > 0 && layer >= 0) {
    // the cache path (dispatch.cpp:219-231): attend over past_len cached keys and
    // the new ones, then the new K/V stay in the cache until commit_step
    if (layer >= kv_layers_) return bad("KvCache layer out of range");
    if (kv_dim != kv_dim_) return bad("KvCache append shape mismatch");
    if (nkv != kv_heads_) return bad("Attention kv heads differ from the KvCache's");
    if (past_len_ + S > kv_max_seq_)
      return bad("KvCache capacity exceeded: seq=" + std::to_string(past_len_ + S) +
                 " max_seq=" + std::to_string(kv_max_seq_));
    UAII_TRY(ar.reserve(align256(in[0].nbytes) + align256(in[1].nbytes) + align256(in[2].nbytes) +
                            align256((*out)[0].nbytes), stream_));
    const float *qd = nullptr, *kd = nullptr, *vd = nullptr;
    float* od = nullptr;
    bool back = false;
    UAII_TRY(stage_in(in[0], ar, &qd));
    UAII_TRY(stage_in(in[1], ar, &kd));
    UAII_TRY(stage_in(in[2], ar, &vd));
    UAII_TRY(stage_out((*out)[0], ar, &od, &back));
    const std::size_t es = kv_f16_ ? 2 : 4;
    const std::size_t layer_bytes = static_cast<std::size_t>(kv_max_seq_) * static_cast<std::size_t>(kv_dim_) * es;
    char* kc = static_cast<char*>(kv_) + static_cast<std::size_t>(layer) * 2 * layer_bytes;
    char* vc = kc + layer_bytes;
    UAII_TRY(hip_rc(uaii_hip_kv_append(kd, vd, kc, vc, S, kv_dim, static_cast<int>(hd), kv_max_seq_, past_len_,
                                       kv_f16_ ? 1 : 0, stream_),
                    "uaii_hip_kv_append"));
    for (std::int64_t i = 0; i < S; ++i) {
      const std::int64_t n_keys = causal ? past_len_ + i + 1 : past_len_ + S;
      UAII_TRY(hip_rc(uaii_hip_attention_decode(qd + i * q_dim, kc, vc, kv_f16_ ? 1 : 0, kv_max_seq_, nh, nkv,
                                                static_cast<int>(hd), n_keys, od + i * q_dim, stream_),
                      "uaii_hip_attention_decode"));
    }
    pending_seq_ = S;
    return finish_outputs(out, {od}, {back});
  }

  // explicit past K/V (5 inputs) or no cache: the keys are past rows then the new
  // ones, in a temporary head-major f32 cache
  std::int64_t P = 0;
  const TensorView *pk = nullptr, *pv = nullptr;
  if (in.size() >= 5) {
    AttnShape pks, pvs;
    UAII_TRY(attn_shape(in[3], &pks, "past_k"));
    UAII_TRY(attn_shape(in[4], &pvs, "past_v"));
    if (pks.batch != 1 || pvs.batch != 1 || pks.dim != kv_dim || pvs.dim != kv_dim || pks.seq != pvs.seq)
      return bad("attention past shape mismatch");
    P = pks.seq;
    pk = &in[3];
    pv = &in[4];
  }
  const std::int64_t T = P + S;
  const std::size_t cache_bytes = static_cast<std::size_t>(T) * static_cast<std::size_t>(kv_dim) * 4;
  const bool present = out->size() >= 3;
  std::size_t need = align256(in[0].nbytes) + align256(in[1].nbytes) + align256(in[2].nbytes) +
                     align256((*out)[0].nbytes) + 2 * align256(cache_bytes);
  if (pk) need += align256(pk->nbytes) + align256(pv->nbytes);
  if (present) need += align256((*out)[1].nbytes) + align256((*out)[2].nbytes);
  UAII_TRY(ar.reserve(need, stream_));
  const float *qd = nullptr, *kd = nullptr, *vd = nullptr, *pkd = nullptr, *pvd = nullptr;
  UAII_TRY(stage_in(in[0], ar, &qd));
  UAII_TRY(stage_in(in[1], ar, &kd));
  UAII_TRY(stage_in(in[2], ar, &vd));
  if (pk) {
    UAII_TRY(stage_in(*pk, ar, &pkd));
    UAII_TRY(stage_in(*pv, ar, &pvd));
  }
  std::vector<float*> dev(out->size(), nullptr);
  std::vector<bool> back(out->size(), false);
  {
    bool b0 = false;
    UAII_TRY(stage_out((*out)[0], ar, &dev[0], &b0));
    back[0] = b0;
  }
  void* kc = ar.take(cache_bytes);
  void* vc = ar.take(cache_bytes);
  if (P > 0)
    UAII_TRY(hip_rc(uaii_hip_kv_append(pkd, pvd, kc, vc, P, kv_dim, static_cast<int>(hd), T, 0, 0, stream_),
                    "uaii_hip_kv_append"));
  UAII_TRY(hip_rc(uaii_hip_kv_append(kd, vd, kc, vc, S, kv_dim, static_cast<int>(hd), T, P, 0, stream_),
                  "uaii_hip_kv_append"));
  for (std::int64_t i = 0; i < S; ++i) {
    const std::int64_t n_keys = causal ? P + i + 1 : T;
    UAII_TRY(hip_rc(uaii_hip_attention_decode(qd + i * q_dim, kc, vc, 0, T, nh, nkv, static_cast<int>(hd), n_keys,
                                              dev[0] + i * q_dim, stream_),
                    "uaii_hip_attention_decode"));
  }
  if (present) {
    // present K/V = concat(past, new) as [1, P+S, kv_dim] (transformer.cpp:378-420)
    for (int j = 1; j <= 2; ++j) {
      TensorView& t = (*out)[static_cast<std::size_t>(j)];
      if (t.dtype != DType::F32 || t.numel() != static_cast<std::size_t>(T * kv_dim))
        return bad("attention present shape mismatch");
      bool b = false;
      UAII_TRY(stage_out(t, ar, &dev[static_cast<std::size_t>(j)], &b));
      back[static_cast<std::size_t>(j)] = b;
      const float* past = j == 1 ? pkd : pvd;
      const float* cur = j == 1 ? kd : vd;
      float* dst = dev[static_cast<std::size_t>(j)];
      const std::size_t pb = static_cast<std::size_t>(P * kv_dim) * 4, cb = static_cast<std::size_t>(S * kv_dim) * 4;
      if (P > 0) UAII_HIP(hipMemcpyAsync(dst, past, pb, hipMemcpyDeviceToDevice, stream_));
      UAII_HIP(hipMemcpyAsync(dst + P * kv_dim, cur, cb, hipMemcpyDeviceToDevice, stream_));
    }
  }
  return finish_outputs(out, dev, back);
}

// ---- factory and Session hooks ----------------------------------------------------

Error create_rocm_backend(std::unique_ptr<IBackend>* out, int device) {
  if (out == nullptr) return bad("backend out null");
  out->reset(new RocmBackend(device));
  return Error::success();
}

namespace {
RocmBackend* as_rocm(IBackend* b) { return b ? dynamic_cast<RocmBackend*>(b) : nullptr; }
}  // namespace

Error rocm_configure_kv_cache(IBackend* backend, std::int64_t n_layers, std::int64_t max_seq,
                              std::int64_t kv_dim, std::int64_t n_kv_heads, bool f16) {
  RocmBackend* r = as_rocm(backend);
  if (!r) return bad("not the ROCm backend of libuaii_amd");
  return r->configure_kv_cache(n_layers, max_seq, kv_dim, n_kv_heads, f16);
}

Error rocm_reset_kv_cache(IBackend* backend) {
  RocmBackend* r = as_rocm(backend);
  if (!r) return bad("not the ROCm backend of libuaii_amd");
  r->reset_kv_cache();
  return Error::success();
}

Error rocm_commit_kv_step(IBackend* backend) {
  RocmBackend* r = as_rocm(backend);
  if (!r) return bad("not the ROCm backend of libuaii_amd");
  r->commit_kv_step();
  return Error::success();
}

}  // namespace backends
}  // namespace uaii
