/*
 * uaii.h — C ABI of the MI355X token-loop library (libuaii_amd.so).
 *
 * Drop-in for the reference's stable C ABI (include/uaii/c_api/uaii.h, C API
 * 0.3.0). Enum values, the uaii_session_options layout and every signature below
 * are identical to the reference; the library implements the "rocm" backend on a
 * device-resident decoder program built from a GGUF file.
 *
 * Entry point -> reference interface it replaces:
 *   uaii_session_options_init   capi.cpp:62-78   (defaults; backend "rocm" here)
 *   uaii_get_c_api_version*     capi.cpp:96-104
 *   uaii_status_name            capi.cpp:106-119
 *   uaii_last_error             capi.cpp:121-123, uaii.h:106-107 (thread-local)
 *   uaii_session_create         capi.cpp:125-183
 *   uaii_session_destroy        capi.cpp:185-187
 *   uaii_session_run            capi.cpp:226-233 (one token step at the current position)
 *   uaii_session_get_f32        capi.cpp:200-224 (named hidden-state / logits taps)
 *   uaii_session_generate       capi.cpp:235-259
 */
#ifndef UAII_C_API_UAII_H_
#define UAII_C_API_UAII_H_

#include "uaii/c_api/version.h"

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define UAII_CAPI_API __attribute__((visibility("default")))

typedef enum uaii_status {
  UAII_OK = 0,
  UAII_ERR_INVALID_ARGUMENT = 1,
  UAII_ERR_NOT_FOUND = 2,
  UAII_ERR_IO = 3,
  UAII_ERR_CONFIG = 4,
  UAII_ERR_PLUGIN = 5,
  UAII_ERR_ABI = 6,
  UAII_ERR_NOT_IMPLEMENTED = 7,
  UAII_ERR_INTERNAL = 8
} uaii_status;

typedef enum uaii_weight_init {
  UAII_WEIGHT_INIT_NONE = 0,
  UAII_WEIGHT_INIT_ZEROS = 1,
  UAII_WEIGHT_INIT_ONES = 2,
  UAII_WEIGHT_INIT_SEQUENCE = 3
} uaii_weight_init;

/* Activation storage dtype. F32 keeps the reference's f32 KV cache; F16 stores
 * the device KV cache in IEEE half (compute stays f32). */
typedef enum uaii_compute_dtype {
  UAII_COMPUTE_DTYPE_F32 = 0,
  UAII_COMPUTE_DTYPE_F16 = 1
} uaii_compute_dtype;

typedef struct uaii_session uaii_session;

typedef struct uaii_session_options {
  uint32_t struct_size;          /* sizeof(uaii_session_options) */
  const char* backend;           /* "rocm" (only backend of this library) */
  const char* weights_dir;       /* prefix for relative model paths (may be NULL) */
  uaii_weight_init weight_init;  /* a weight whose bytes the file lacks: NONE fails the create (NOT_FOUND); ZEROS / ONES / SEQUENCE fill its f32 values (Path A; packed Path B weights cannot be filled) */
  int enable_fusion;             /* accepted; the device program is always fused */
  int enable_memory_reuse;       /* non-zero (default): weights take the values of the
                                    reference's f32 weight load (its Path A: Q4_0 nibbles
                                    in pairwise order); 0 with keep_quantized_weights:
                                    those of its packed decode (Path B) */
  int enable_profiler;           /* non-zero: per-step device timing is recorded */
  const char* profile_trace_path;
  uint64_t budget_bytes;         /* device byte budget; 0 = unlimited; exceeding it
                                    fails with UAII_ERR_INVALID_ARGUMENT */
  int enable_streaming;          /* must be 0: the whole model is HBM resident */
  int allow_missing_weights;
  const char* weights_sandbox;
  int compute_dtype;             /* uaii_compute_dtype: KV cache storage */
  int keep_quantized_weights;    /* 0: Path A values as with enable_memory_reuse; the
                                    device keeps weights block-packed either way */
  int64_t max_context;           /* 0 = GGUF {arch}.context_length */
} uaii_session_options;

UAII_CAPI_API void uaii_session_options_init(uaii_session_options* opts);

UAII_CAPI_API uaii_status uaii_get_version(int* major, int* minor, int* patch);
UAII_CAPI_API const char* uaii_get_version_string(void);
UAII_CAPI_API void uaii_get_c_api_version(int* major, int* minor, int* patch);
UAII_CAPI_API const char* uaii_get_c_api_version_string(void);

UAII_CAPI_API const char* uaii_status_name(uaii_status status);
/** Thread-local last error message (valid until next C API call on this thread). */
UAII_CAPI_API const char* uaii_last_error(void);

/** Create a session from a GGUF decoder file. */
UAII_CAPI_API uaii_status uaii_session_create(const char* path,
                                              const uaii_session_options* opts,
                                              uaii_session** out);

UAII_CAPI_API void uaii_session_destroy(uaii_session* session);

UAII_CAPI_API uaii_status uaii_session_set_f32(uaii_session* session,
                                               const char* tensor_name,
                                               const float* data,
                                               size_t n);

/** Read a named tensor of the last step: "hidden", "blk.N.resid1", "blk.N.resid2",
 * "normed", "logits", "probs" (reference graph names, gguf.cpp:935-1209). */
UAII_CAPI_API uaii_status uaii_session_get_f32(uaii_session* session,
                                               const char* tensor_name,
                                               float* out,
                                               size_t capacity,
                                               size_t* out_n);

UAII_CAPI_API uaii_status uaii_session_run(uaii_session* session);

/** Greedy generate: prompt_tokens -> out_tokens (prompt echoed first); writes
 * min(capacity, prompt_n + max_new_tokens) ids and their count to *out_n. */
UAII_CAPI_API uaii_status uaii_session_generate(uaii_session* session,
                                                const int64_t* prompt_tokens,
                                                size_t prompt_n,
                                                int64_t max_new_tokens,
                                                int64_t* out_tokens,
                                                size_t capacity,
                                                size_t* out_n);

UAII_CAPI_API uaii_status uaii_session_profile_summary(uaii_session* session,
                                                       char* buf,
                                                       size_t capacity);

UAII_CAPI_API uaii_status uaii_session_write_trace(uaii_session* session,
                                                   const char* path);

/* Model conversion (include/uaii/c_api/uaii.h:154-155 in the reference) is not
 * part of this library: it returns UAII_ERR_NOT_IMPLEMENTED. Exported so callers
 * that bind the whole reference header (bindings/python/uaii/_backend.py:151-181)
 * load this library unchanged. */
UAII_CAPI_API uaii_status uaii_convert_model(const char* input_path,
                                             const char* output_path);

#ifdef __cplusplus
}
#endif

#endif /* UAII_C_API_UAII_H_ */
