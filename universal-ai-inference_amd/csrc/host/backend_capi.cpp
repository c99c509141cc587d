// backend_capi.cpp — uaii_backend.h over uaii::backends::RocmBackend.
#include "uaii/c_api/uaii_backend.h"

#include "capi_internal.h"
#include "rocm_backend.h"

#include <memory>
#include <string>
#include <vector>

struct uaii_backend {
  std::unique_ptr<uaii::IBackend> b;
};

namespace {

thread_local std::string g_details;

uaii::backends::RocmBackend* rocm(uaii_backend* h) {
  return h ? static_cast<uaii::backends::RocmBackend*>(h->b.get()) : nullptr;
}

uaii::kernels::TensorView view_of(const uaii_tensor_view& t) {
  uaii::kernels::TensorView v;
  v.dtype = static_cast<uaii::DType>(t.dtype);
  v.shape = t.shape;
  v.rank = t.rank;
  v.data = t.data;
  v.nbytes = t.nbytes;
  v.quant_format = static_cast<uaii::quant::QuantFormat>(t.quant_format);
  v.quant_rows = t.quant_rows;
  v.quant_cols = t.quant_cols;
  return v;
}

}  // namespace

extern "C" {

uaii_status uaii_backend_create(const char* name, int device, uaii_backend** out) {
  if (!out) return uaii_capi_fail(UAII_ERR_INVALID_ARGUMENT, "backend out null");
  *out = nullptr;
  if (!name || std::string(name) != "rocm")
    return uaii_capi_fail(UAII_ERR_NOT_FOUND, "unknown backend (this library provides 'rocm')");
  auto h = std::make_unique<uaii_backend>();
  uaii::Error e = uaii::backends::create_rocm_backend(&h->b, device);
  if (!e.ok()) return uaii_capi_status(e);
  *out = h.release();
  return uaii_capi_status(uaii::Error::success());
}

void uaii_backend_destroy(uaii_backend* backend) { delete backend; }

uaii_status uaii_backend_initialize(uaii_backend* backend) {
  if (!backend) return uaii_capi_fail(UAII_ERR_INVALID_ARGUMENT, "backend null");
  return uaii_capi_status(backend->b->initialize());
}

const char* uaii_backend_details(uaii_backend* backend) {
  g_details = backend ? backend->b->capabilities().details : std::string();
  return g_details.c_str();
}

int uaii_backend_uses_host_fallback(uaii_backend* backend) {
  return backend && backend->b->uses_host_fallback() ? 1 : 0;
}

uaii_status uaii_backend_dispatch(uaii_backend* backend, const char* op_name, const char* op_version,
                                  const uaii_tensor_view* inputs, size_t n_inputs, uaii_tensor_view* outputs,
                                  size_t n_outputs, const uaii_attribute* attrs, size_t n_attrs) {
  if (!backend || !op_name || (n_inputs && !inputs) || (n_outputs && !outputs) || (n_attrs && !attrs))
    return uaii_capi_fail(UAII_ERR_INVALID_ARGUMENT, "dispatch: null argument");
  std::vector<uaii::kernels::TensorView> in, out;
  for (size_t i = 0; i < n_inputs; ++i) in.push_back(view_of(inputs[i]));
  for (size_t i = 0; i < n_outputs; ++i) out.push_back(view_of(outputs[i]));
  std::vector<uaii::ir::Attribute> at;
  for (size_t i = 0; i < n_attrs; ++i) {
    uaii::ir::Attribute a;
    if (!attrs[i].key) return uaii_capi_fail(UAII_ERR_INVALID_ARGUMENT, "dispatch: attribute without key");
    a.key = attrs[i].key;
    switch (attrs[i].type) {
      case 0: a.type = uaii::ir::AttributeType::String; a.value = std::string(attrs[i].s ? attrs[i].s : ""); break;
      case 1: a.type = uaii::ir::AttributeType::Int; a.value = static_cast<std::int64_t>(attrs[i].i); break;
      case 2: a.type = uaii::ir::AttributeType::Float; a.value = attrs[i].f; break;
      case 3: a.type = uaii::ir::AttributeType::Bool; a.value = attrs[i].i != 0; break;
      default: return uaii_capi_fail(UAII_ERR_INVALID_ARGUMENT, "dispatch: attribute type");
    }
    at.push_back(std::move(a));
  }
  return uaii_capi_status(backend->b->dispatch(op_name, op_version ? op_version : "1", in, &out, at));
}

uaii_status uaii_backend_synchronize(uaii_backend* backend) {
  if (!backend) return uaii_capi_fail(UAII_ERR_INVALID_ARGUMENT, "backend null");
  return uaii_capi_status(backend->b->synchronize());
}

uaii_status uaii_backend_allocate(uaii_backend* backend, size_t bytes, void** out_ptr) {
  if (!backend) return uaii_capi_fail(UAII_ERR_INVALID_ARGUMENT, "backend null");
  return uaii_capi_status(backend->b->allocate(bytes, out_ptr));
}

uaii_status uaii_backend_free(uaii_backend* backend, void* ptr) {
  if (!backend) return uaii_capi_fail(UAII_ERR_INVALID_ARGUMENT, "backend null");
  return uaii_capi_status(backend->b->free(ptr));
}

uaii_status uaii_backend_copy_h2d(uaii_backend* backend, const void* host, void* device, size_t bytes) {
  if (!backend) return uaii_capi_fail(UAII_ERR_INVALID_ARGUMENT, "backend null");
  return uaii_capi_status(backend->b->copy_h2d(host, device, bytes));
}

uaii_status uaii_backend_copy_d2h(uaii_backend* backend, const void* device, void* host, size_t bytes) {
  if (!backend) return uaii_capi_fail(UAII_ERR_INVALID_ARGUMENT, "backend null");
  return uaii_capi_status(backend->b->copy_d2h(device, host, bytes));
}

uaii_status uaii_backend_configure_kv_cache(uaii_backend* backend, int64_t n_layers, int64_t max_seq,
                                            int64_t kv_dim, int64_t n_kv_heads, int kv_f16) {
  if (!backend) return uaii_capi_fail(UAII_ERR_INVALID_ARGUMENT, "backend null");
  return uaii_capi_status(rocm(backend)->configure_kv_cache(n_layers, max_seq, kv_dim, n_kv_heads, kv_f16 != 0));
}

uaii_status uaii_backend_reset_kv_cache(uaii_backend* backend) {
  if (!backend) return uaii_capi_fail(UAII_ERR_INVALID_ARGUMENT, "backend null");
  rocm(backend)->reset_kv_cache();
  return uaii_capi_status(uaii::Error::success());
}

uaii_status uaii_backend_commit_kv_step(uaii_backend* backend) {
  if (!backend) return uaii_capi_fail(UAII_ERR_INVALID_ARGUMENT, "backend null");
  rocm(backend)->commit_kv_step();
  return uaii_capi_status(uaii::Error::success());
}

int64_t uaii_backend_kv_past_len(uaii_backend* backend) {
  return backend ? rocm(backend)->kv_past_len() : -1;
}

}  // extern "C"
