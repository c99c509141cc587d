/*
 * uaii_ext.h — token-loop extensions of libuaii_amd.so beyond the reference ABI.
 *
 * No counterpart in the reference C API: these entry points expose the device
 * token loop step by step for streaming callers and for measurement (the
 * reference's uaii_session_run is synchronous and uaii_session_generate runs the
 * whole loop). They operate on the same session as uaii.h.
 */
#ifndef UAII_C_API_UAII_EXT_H_
#define UAII_C_API_UAII_EXT_H_

#include "uaii/c_api/uaii.h"

#ifdef __cplusplus
extern "C" {
#endif

/** Reset the session to position 0 with `prompt_n` prompt ids on the device
 * (KV capacity sized for `capacity` positions, 0 = max_context). */
UAII_CAPI_API uaii_status uaii_session_begin(uaii_session* session, const int64_t* prompt_tokens,
                                             size_t prompt_n, int64_t capacity);

/** Enqueue one token step at the current position without waiting. With
 * want_logits the step also runs the LM head and greedy argmax; without it the
 * next prompt token is fed (valid only inside the prompt). */
UAII_CAPI_API uaii_status uaii_session_step_async(uaii_session* session, int want_logits);

/** Run the next n prompt tokens (positions pos .. pos + n - 1, taken from the
 * prompt given to uaii_session_begin) through every layer at once on the matrix
 * cores: K/V are appended for each position and no logits are computed; the
 * following step feeds prompt token pos + n. The reference prefills token by
 * token (session.cpp:1005-1015); the results agree within float tolerance.
 * Returns UAII_ERR_NOT_IMPLEMENTED when the model is outside this path (see
 * uaii_session_prefill_supported). Synchronises with the device. */
UAII_CAPI_API uaii_status uaii_session_prefill(uaii_session* session, int64_t n);

/** *supported = 1 when uaii_session_prefill covers the model: weights in Q4_0,
 * Q8_0, Q4_K or Q6_K, dense SwiGLU/GELU FFNs, an f16 KV cache, head_dim 64 or
 * 128. uaii_session_generate uses it for the prompt whenever it is 1. */
UAII_CAPI_API uaii_status uaii_session_prefill_supported(uaii_session* session, int* supported);

/** Wait for all enqueued steps. */
UAII_CAPI_API uaii_status uaii_session_sync(uaii_session* session);

/** Current position (tokens processed so far). */
UAII_CAPI_API uaii_status uaii_session_position(uaii_session* session, int64_t* pos);

/** Copy ids[0..n) (prompt followed by generated ids) to `out`. */
UAII_CAPI_API uaii_status uaii_session_read_ids(uaii_session* session, int64_t* out, size_t n);

/** Move back to position `pos` (0 < pos <= current): ids and KV entries below
 * `pos` are kept, the token at `pos` is fed next. */
UAII_CAPI_API uaii_status uaii_session_seek(uaii_session* session, int64_t pos);

/** Per-kernel HIP event timing on (direct launches) or off (graph replay). */
UAII_CAPI_API uaii_status uaii_session_set_profiling(uaii_session* session, int on);

/** Greedy argmax margin of the last step: (best logit, runner-up logit). */
UAII_CAPI_API uaii_status uaii_session_last_margin(uaii_session* session, float* best,
                                                   float* second);

/** Sampling parameters (include/uaii/runtime/sampling.hpp:15-27 in the
 * reference). Greedy when temperature <= 0, top_k <= 0, top_p >= 1 and
 * repetition_penalty <= 1. */
typedef struct uaii_sample_params {
  uint32_t struct_size;
  float temperature;
  float top_p;
  int32_t top_k;
  float repetition_penalty;
  uint64_t seed;
  int has_seed; /* 0: seed from std::random_device, as the reference */
} uaii_sample_params;

UAII_CAPI_API void uaii_sample_params_init(uaii_sample_params* params);

/** uaii_session_generate with the reference's sampler (Session::generate's
 * SampleParams argument, session.cpp:910-1046): non-greedy draws are made on
 * the host from each step's logits row (session.cpp:974-978) with a seeded
 * mt19937_64. */
UAII_CAPI_API uaii_status uaii_session_generate_sampled(uaii_session* session,
                                                        const int64_t* prompt_tokens,
                                                        size_t prompt_n, int64_t max_new_tokens,
                                                        const uaii_sample_params* params,
                                                        int64_t* out_tokens, size_t capacity,
                                                        size_t* out_n);

/** Non-greedy draws of uaii_session_generate_sampled on the device (on != 0)
 * instead of on the host: the same parameters, penalty history and generator
 * draws (one uniform per generated token, taken from the seeded mt19937_64
 * before the run), with the pick made where the logits are, so only token ids
 * cross PCIe. The reference samples on the host; this switch has no
 * counterpart there. Ids equal the host sampler's except where a draw lands
 * within float rounding of a cumulative boundary, on tied scores, or with
 * top_k alone (walked in descending order rather than std::nth_element's, the
 * same distribution). UAII_ERR_NOT_IMPLEMENTED for vocabularies above 262144.
 * UAII_DEVICE_SAMPLER=1 in the environment turns it on for new sessions. */
UAII_CAPI_API uaii_status uaii_session_set_device_sampler(uaii_session* session, int on);

/** One draw of the sampler (sampling.cpp:22-125) over row[0..vocab) with a fresh
 * mt19937_64(params->seed); penalty ids as the reference's history. Host only. */
UAII_CAPI_API uaii_status uaii_sample_token(const float* row, size_t vocab,
                                            const uaii_sample_params* params,
                                            const int64_t* penalty_tokens, size_t n_penalty,
                                            int64_t* out_token);

/** Parse a GGUF file and derive the decoder the session would run, without
 * touching the GPU: a JSON object (arch, layer count, dims, heads, vocab,
 * context length, rope mode/theta, rms eps, tied embeddings, per-layer FFN kind
 * and tensor types) is written to buf (NUL-terminated, truncated to capacity). */
UAII_CAPI_API uaii_status uaii_model_describe(const char* path, char* buf, size_t capacity);

#ifdef __cplusplus
}
#endif

#endif /* UAII_C_API_UAII_EXT_H_ */
