/*
 * uaii_backend.h — C binding of libuaii_amd.so's ROCm IBackend.
 *
 * The reference's operators are dispatched through uaii::IBackend
 * (include/uaii/interfaces/backend.hpp:29-87), a C++ interface; this library's
 * implementation is uaii::backends::RocmBackend (C++ factory
 * uaii::backends::create_rocm_backend, the branch factory.cpp:52-80 would take
 * for "rocm"). These entry points bind the same object for C and ctypes callers,
 * one function per IBackend method, with TensorView and ir::Attribute as plain
 * structs:
 *   uaii_backend_create / _destroy        create_backend("rocm", ...) (factory.cpp:52-80)
 *   uaii_backend_initialize               IBackend::initialize
 *   uaii_backend_dispatch                 IBackend::dispatch (op semantics of
 *                                         libs/uaii-kernels/src/dispatch.cpp:67-272)
 *   uaii_backend_allocate / _free /
 *   _copy_h2d / _copy_d2h / _synchronize  the IBackend methods of those names
 *   uaii_backend_configure_kv_cache /     runtime::KvCache configure / reset /
 *   _reset_kv_cache / _commit_kv_step     commit_step (include/uaii/runtime/kv_cache.hpp)
 * Each returns a uaii_status and sets uaii_last_error() on failure. A backend is
 * used by one thread at a time.
 */
#ifndef UAII_C_API_UAII_BACKEND_H_
#define UAII_C_API_UAII_BACKEND_H_

#include "uaii/c_api/uaii.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct uaii_backend uaii_backend;

/* kernels::TensorView (include/uaii/kernels/tensor_view.hpp:12-24): dtype is
 * uaii::DType (0 unknown, 1 f32, 2 f16, ...); quant_format is quant::QuantFormat
 * (0 F32, 1 F16, ..., 7 Q4_0, 8 Q4_1, 9 Q5_0, 10 Q5_1, 11 Q8_0, 12 Q2_K, 13 Q3_K,
 * 14 Q4_K, 15 Q5_K, 16 Q6_K); data is host or device memory. */
typedef struct uaii_tensor_view {
  int32_t dtype;
  const int64_t* shape;
  size_t rank;
  void* data;
  size_t nbytes;
  int32_t quant_format;
  int64_t quant_rows;
  int64_t quant_cols;
} uaii_tensor_view;

/* ir::Attribute (include/uaii/ir/attribute.hpp:11-31): type 0 string (s),
 * 1 int (i), 2 float (f), 3 bool (i != 0). */
typedef struct uaii_attribute {
  const char* key;
  int32_t type;
  int64_t i;
  double f;
  const char* s;
} uaii_attribute;

UAII_CAPI_API uaii_status uaii_backend_create(const char* name, int device, uaii_backend** out);
UAII_CAPI_API void uaii_backend_destroy(uaii_backend* backend);
UAII_CAPI_API uaii_status uaii_backend_initialize(uaii_backend* backend);
/* IBackend::capabilities().details and uses_host_fallback(); the string is valid
 * until the next call on this thread. */
UAII_CAPI_API const char* uaii_backend_details(uaii_backend* backend);
UAII_CAPI_API int uaii_backend_uses_host_fallback(uaii_backend* backend);
UAII_CAPI_API uaii_status uaii_backend_dispatch(uaii_backend* backend, const char* op_name,
                                                const char* op_version, const uaii_tensor_view* inputs,
                                                size_t n_inputs, uaii_tensor_view* outputs, size_t n_outputs,
                                                const uaii_attribute* attrs, size_t n_attrs);
UAII_CAPI_API uaii_status uaii_backend_synchronize(uaii_backend* backend);
UAII_CAPI_API uaii_status uaii_backend_allocate(uaii_backend* backend, size_t bytes, void** out_ptr);
UAII_CAPI_API uaii_status uaii_backend_free(uaii_backend* backend, void* ptr);
UAII_CAPI_API uaii_status uaii_backend_copy_h2d(uaii_backend* backend, const void* host, void* device,
                                                size_t bytes);
UAII_CAPI_API uaii_status uaii_backend_copy_d2h(uaii_backend* backend, const void* device, void* host,
                                                size_t bytes);
UAII_CAPI_API uaii_status uaii_backend_configure_kv_cache(uaii_backend* backend, int64_t n_layers,
                                                          int64_t max_seq, int64_t kv_dim,
                                                          int64_t n_kv_heads, int kv_f16);
UAII_CAPI_API uaii_status uaii_backend_reset_kv_cache(uaii_backend* backend);
UAII_CAPI_API uaii_status uaii_backend_commit_kv_step(uaii_backend* backend);
UAII_CAPI_API int64_t uaii_backend_kv_past_len(uaii_backend* backend);

#ifdef __cplusplus
}
#endif

#endif /* UAII_C_API_UAII_BACKEND_H_ */
