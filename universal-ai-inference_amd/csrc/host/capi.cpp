// capi.cpp — the uaii.h C ABI over runtime::Session (libs/uaii-capi/src/capi.cpp).
#include "uaii/c_api/uaii.h"
#include "uaii/c_api/uaii_ext.h"

#include "session.h"

#include <algorithm>
#include <cstring>
#include <memory>
#include <random>
#include <string>
#include <vector>

namespace {

thread_local std::string g_last_error;

uaii_status to_status(uaii::ErrorCode code) {
  switch (code) {
    case uaii::ErrorCode::Ok: return UAII_OK;
    case uaii::ErrorCode::InvalidArgument: return UAII_ERR_INVALID_ARGUMENT;
    case uaii::ErrorCode::NotFound: return UAII_ERR_NOT_FOUND;
    case uaii::ErrorCode::IoError: return UAII_ERR_IO;
    case uaii::ErrorCode::ConfigError: return UAII_ERR_CONFIG;
    case uaii::ErrorCode::PluginError: return UAII_ERR_PLUGIN;
    case uaii::ErrorCode::AbiMismatch: return UAII_ERR_ABI;
    case uaii::ErrorCode::NotImplemented: return UAII_ERR_NOT_IMPLEMENTED;
    default: return UAII_ERR_INTERNAL;
  }
}

uaii_status from_error(const uaii::Error& err) {
  g_last_error = err.ok() ? std::string() : err.to_string();
  return to_status(err.code());
}

uaii_status fail(uaii_status st, const char* msg) {
  g_last_error = msg;
  return st;
}

struct SessionHandle {
  uaii::runtime::Session session;
};

}  // namespace

// The thread's last-error text and the status of an Error, for the other C
// entry points of this library (uaii_backend.h).
uaii_status uaii_capi_status(const uaii::Error& err) { return from_error(err); }
uaii_status uaii_capi_fail(uaii_status st, const char* msg) { return fail(st, msg); }

namespace {

}  // namespace

extern "C" {

void uaii_session_options_init(uaii_session_options* opts) {
  if (opts == nullptr) return;
  std::memset(opts, 0, sizeof(*opts));
  opts->struct_size = static_cast<uint32_t>(sizeof(uaii_session_options));
  opts->backend = "rocm";
  opts->weight_init = UAII_WEIGHT_INIT_NONE;
  opts->enable_fusion = 1;
  opts->enable_memory_reuse = 1;
  opts->compute_dtype = UAII_COMPUTE_DTYPE_F32;
  opts->keep_quantized_weights = 1;
  opts->max_context = 0;
}

uaii_status uaii_get_version(int* major, int* minor, int* patch) {
  if (major) *major = UAII_AMD_VERSION_MAJOR;
  if (minor) *minor = UAII_AMD_VERSION_MINOR;
  if (patch) *patch = UAII_AMD_VERSION_PATCH;
  return UAII_OK;
}

const char* uaii_get_version_string(void) { return UAII_AMD_VERSION_STRING; }

void uaii_get_c_api_version(int* major, int* minor, int* patch) {
  if (major) *major = UAII_C_API_VERSION_MAJOR;
  if (minor) *minor = UAII_C_API_VERSION_MINOR;
  if (patch) *patch = UAII_C_API_VERSION_PATCH;
}

const char* uaii_get_c_api_version_string(void) { return UAII_C_API_VERSION_STRING; }

const char* uaii_status_name(uaii_status status) {
  switch (status) {
    case UAII_OK: return "ok";
    case UAII_ERR_INVALID_ARGUMENT: return "invalid_argument";
    case UAII_ERR_NOT_FOUND: return "not_found";
    case UAII_ERR_IO: return "io";
    case UAII_ERR_CONFIG: return "config";
    case UAII_ERR_PLUGIN: return "plugin";
    case UAII_ERR_ABI: return "abi";
    case UAII_ERR_NOT_IMPLEMENTED: return "not_implemented";
    case UAII_ERR_INTERNAL: return "internal";
    default: return "unknown";
  }
}

const char* uaii_last_error(void) { return g_last_error.c_str(); }

uaii_status uaii_session_create(const char* path, const uaii_session_options* opts,
                                uaii_session** out) {
  if (path == nullptr || out == nullptr) return fail(UAII_ERR_INVALID_ARGUMENT, "path/out null");
  *out = nullptr;
  uaii_session_options local;
  uaii_session_options_init(&local);
  if (opts != nullptr) {
    // ABI-safe growth: copy only what the caller's struct holds (capi.cpp:132-139)
    if (opts->struct_size == 0 || opts->struct_size > sizeof(uaii_session_options))
      return fail(UAII_ERR_ABI, "uaii_session_options.struct_size invalid");
    std::memcpy(&local, opts, static_cast<size_t>(opts->struct_size));
    local.struct_size = static_cast<uint32_t>(sizeof(uaii_session_options));
  }
  uaii::runtime::SessionOptions so;
  so.backend_name = local.backend ? local.backend : "rocm";
  if (local.weights_dir) so.weights_dir = local.weights_dir;
  so.weight_init = static_cast<uaii::runtime::WeightInit>(
      (local.weight_init >= 0 && local.weight_init <= 3) ? local.weight_init : 0);
  so.enable_fusion = local.enable_fusion != 0;
  so.enable_memory_reuse = local.enable_memory_reuse != 0;
  so.enable_profiler = local.enable_profiler != 0;
  if (local.profile_trace_path) so.profile_trace_path = local.profile_trace_path;
  so.budget_bytes = local.budget_bytes;
  so.enable_streaming = local.enable_streaming != 0;
  so.allow_missing_weights = local.allow_missing_weights != 0;
  if (local.weights_sandbox) so.weights_sandbox = local.weights_sandbox;
  so.kv_f16 = local.compute_dtype == UAII_COMPUTE_DTYPE_F16;
  so.keep_quantized_weights = local.keep_quantized_weights != 0;
  so.max_context = local.max_context;
  auto h = std::make_unique<SessionHandle>();
  uaii::Error err = h->session.create(path, so);
  if (!err.ok()) return from_error(err);
  *out = reinterpret_cast<uaii_session*>(h.release());
  g_last_error.clear();
  return UAII_OK;
}

void uaii_session_destroy(uaii_session* session) {
  delete reinterpret_cast<SessionHandle*>(session);
}

uaii_status uaii_session_set_f32(uaii_session* session, const char* tensor_name,
                                 const float* data, size_t n) {
  if (session == nullptr || tensor_name == nullptr || data == nullptr)
    return fail(UAII_ERR_INVALID_ARGUMENT, "set_f32 null arg");
  auto* h = reinterpret_cast<SessionHandle*>(session);
  return from_error(h->session.set_tensor_f32(tensor_name, std::vector<float>(data, data + n)));
}

uaii_status uaii_session_get_f32(uaii_session* session, const char* tensor_name, float* out,
                                 size_t capacity, size_t* out_n) {
  if (session == nullptr || tensor_name == nullptr || out_n == nullptr)
    return fail(UAII_ERR_INVALID_ARGUMENT, "get_f32 null arg");
  auto* h = reinterpret_cast<SessionHandle*>(session);
  std::vector<float> values;
  uaii::Error err = h->session.get_tensor_f32(tensor_name, &values);
  if (!err.ok()) return from_error(err);
  *out_n = values.size();
  if (out == nullptr) return UAII_OK;
  if (capacity < values.size()) return fail(UAII_ERR_INVALID_ARGUMENT, "get_f32 buffer too small");
  std::memcpy(out, values.data(), values.size() * sizeof(float));
  g_last_error.clear();
  return UAII_OK;
}

uaii_status uaii_session_run(uaii_session* session) {
  if (session == nullptr) return fail(UAII_ERR_INVALID_ARGUMENT, "session null");
  return from_error(reinterpret_cast<SessionHandle*>(session)->session.run());
}

uaii_status uaii_session_generate(uaii_session* session, const int64_t* prompt_tokens,
                                  size_t prompt_n, int64_t max_new_tokens, int64_t* out_tokens,
                                  size_t capacity, size_t* out_n) {
  if (session == nullptr || out_tokens == nullptr || out_n == nullptr)
    return fail(UAII_ERR_INVALID_ARGUMENT, "generate null args");
  auto* h = reinterpret_cast<SessionHandle*>(session);
  std::vector<int64_t> prompt;
  if (prompt_tokens != nullptr && prompt_n > 0) prompt.assign(prompt_tokens, prompt_tokens + prompt_n);
  std::vector<int64_t> out;
  uaii::Error err = h->session.generate(prompt, max_new_tokens, &out);
  if (!err.ok()) return from_error(err);
  const size_t n = std::min(capacity, out.size());
  for (size_t i = 0; i < n; ++i) out_tokens[i] = out[i];
  *out_n = n;
  g_last_error.clear();
  return UAII_OK;
}

uaii_status uaii_session_profile_summary(uaii_session* session, char* buf, size_t capacity) {
  if (session == nullptr || buf == nullptr || capacity == 0)
    return fail(UAII_ERR_INVALID_ARGUMENT, "profile_summary null/empty");
  const std::string s = reinterpret_cast<SessionHandle*>(session)->session.profile_summary();
  if (s.size() + 1 > capacity) return fail(UAII_ERR_INVALID_ARGUMENT, "profile_summary buffer too small");
  std::memcpy(buf, s.c_str(), s.size() + 1);
  g_last_error.clear();
  return UAII_OK;
}

uaii_status uaii_session_write_trace(uaii_session* session, const char* path) {
  if (session == nullptr || path == nullptr) return fail(UAII_ERR_INVALID_ARGUMENT, "write_trace null");
  const std::string s = reinterpret_cast<SessionHandle*>(session)->session.profile_summary();
  FILE* f = std::fopen(path, "w");
  if (!f) return fail(UAII_ERR_IO, "cannot open trace path");
  std::fputs(s.c_str(), f);
  std::fclose(f);
  g_last_error.clear();
  return UAII_OK;
}

void uaii_sample_params_init(uaii_sample_params* params) {
  if (params == nullptr) return;
  std::memset(params, 0, sizeof(*params));
  params->struct_size = static_cast<uint32_t>(sizeof(uaii_sample_params));
  params->temperature = 0.0f;
  params->top_p = 1.0f;
  params->top_k = 0;
  params->repetition_penalty = 1.0f;
}

namespace {
bool to_params(const uaii_sample_params* in, uaii::runtime::SampleParams* out) {
  if (in == nullptr) return true;  // greedy
  if (in->struct_size == 0 || in->struct_size > sizeof(uaii_sample_params)) return false;
  uaii_sample_params p;
  uaii_sample_params_init(&p);
  std::memcpy(&p, in, in->struct_size);
  out->temperature = p.temperature;
  out->top_p = p.top_p;
  out->top_k = p.top_k;
  out->repetition_penalty = p.repetition_penalty;
  out->seed = p.seed;
  out->has_seed = p.has_seed != 0;
  return true;
}
}  // namespace

uaii_status uaii_session_generate_sampled(uaii_session* session, const int64_t* prompt_tokens,
                                          size_t prompt_n, int64_t max_new_tokens,
                                          const uaii_sample_params* params, int64_t* out_tokens,
                                          size_t capacity, size_t* out_n) {
  if (session == nullptr || out_tokens == nullptr || out_n == nullptr)
    return fail(UAII_ERR_INVALID_ARGUMENT, "generate_sampled null arg");
  if (prompt_n > 0 && prompt_tokens == nullptr) return fail(UAII_ERR_INVALID_ARGUMENT, "prompt null");
  uaii::runtime::SampleParams sp;
  if (!to_params(params, &sp)) return fail(UAII_ERR_ABI, "uaii_sample_params.struct_size invalid");
  std::vector<int64_t> prompt(prompt_tokens, prompt_tokens + prompt_n);
  std::vector<int64_t> out;
  uaii::Error err = reinterpret_cast<SessionHandle*>(session)->session.generate(
      prompt, max_new_tokens, &out, {}, {}, sp);
  if (!err.ok()) return from_error(err);
  const size_t n = std::min(capacity, out.size());
  std::copy(out.begin(), out.begin() + (std::ptrdiff_t)n, out_tokens);
  *out_n = n;
  g_last_error.clear();
  return UAII_OK;
}

uaii_status uaii_sample_token(const float* row, size_t vocab, const uaii_sample_params* params,
                              const int64_t* penalty_tokens, size_t n_penalty, int64_t* out_token) {
  if (row == nullptr || out_token == nullptr || (n_penalty > 0 && penalty_tokens == nullptr))
    return fail(UAII_ERR_INVALID_ARGUMENT, "sample_token null arg");
  uaii::runtime::SampleParams sp;
  if (!to_params(params, &sp)) return fail(UAII_ERR_ABI, "uaii_sample_params.struct_size invalid");
  std::vector<int64_t> pen(penalty_tokens, penalty_tokens + n_penalty);
  std::mt19937_64 rng(sp.seed);
  uaii::Error err = uaii::runtime::sample_token_f32(row, vocab, sp, pen, &rng, out_token);
  if (!err.ok()) return from_error(err);
  g_last_error.clear();
  return UAII_OK;
}

uaii_status uaii_model_describe(const char* path, char* buf, size_t capacity) {
  if (path == nullptr || buf == nullptr || capacity == 0)
    return fail(UAII_ERR_INVALID_ARGUMENT, "model_describe null arg");
  uaii::GgufFile file;
  uaii::DecoderSpec spec;
  uaii::Error err = file.open(path);
  if (err.ok()) err = uaii::derive_decoder(file, &spec);
  if (!err.ok()) return from_error(err);
  const std::string s = uaii::describe_decoder(spec);
  const size_t n = std::min(capacity - 1, s.size());
  std::memcpy(buf, s.data(), n);
  buf[n] = '\0';
  g_last_error.clear();
  return UAII_OK;
}

uaii_status uaii_convert_model(const char* input_path, const char* output_path) {
  (void)input_path;
  (void)output_path;
  return fail(UAII_ERR_NOT_IMPLEMENTED, "uaii_convert_model: model conversion is not part of the ROCm decode library");
}

// ---- uaii_ext.h ------------------------------------------------------------

uaii_status uaii_session_begin(uaii_session* session, const int64_t* prompt_tokens,
                               size_t prompt_n, int64_t capacity) {
  if (session == nullptr || (prompt_tokens == nullptr && prompt_n > 0))
    return fail(UAII_ERR_INVALID_ARGUMENT, "begin null args");
  auto* h = reinterpret_cast<SessionHandle*>(session);
  std::vector<int64_t> prompt(prompt_tokens, prompt_tokens + prompt_n);
  return from_error(h->session.begin(prompt, capacity));
}

uaii_status uaii_session_step_async(uaii_session* session, int want_logits) {
  if (session == nullptr) return fail(UAII_ERR_INVALID_ARGUMENT, "session null");
  return from_error(reinterpret_cast<SessionHandle*>(session)->session.step_async(want_logits != 0));
}

uaii_status uaii_session_prefill(uaii_session* session, int64_t n) {
  if (session == nullptr || n < 0) return fail(UAII_ERR_INVALID_ARGUMENT, "prefill args");
  return from_error(reinterpret_cast<SessionHandle*>(session)->session.prefill(n));
}

uaii_status uaii_session_prefill_supported(uaii_session* session, int* supported) {
  if (session == nullptr || supported == nullptr) return fail(UAII_ERR_INVALID_ARGUMENT, "null args");
  auto* p = reinterpret_cast<SessionHandle*>(session)->session.program();
  if (!p) return fail(UAII_ERR_INVALID_ARGUMENT, "session not ready");
  *supported = p->prefill_supported() ? 1 : 0;
  return UAII_OK;
}

uaii_status uaii_session_sync(uaii_session* session) {
  if (session == nullptr) return fail(UAII_ERR_INVALID_ARGUMENT, "session null");
  auto* p = reinterpret_cast<SessionHandle*>(session)->session.program();
  if (!p) return fail(UAII_ERR_INVALID_ARGUMENT, "session not ready");
  return from_error(p->synchronize());
}

uaii_status uaii_session_position(uaii_session* session, int64_t* pos) {
  if (session == nullptr || pos == nullptr) return fail(UAII_ERR_INVALID_ARGUMENT, "null args");
  auto* p = reinterpret_cast<SessionHandle*>(session)->session.program();
  if (!p) return fail(UAII_ERR_INVALID_ARGUMENT, "session not ready");
  uaii_hip::StepState st{};
  uaii::Error err = p->read_state(&st);
  if (!err.ok()) return from_error(err);
  *pos = st.pos;
  return UAII_OK;
}

uaii_status uaii_session_read_ids(uaii_session* session, int64_t* out, size_t n) {
  if (session == nullptr || (out == nullptr && n > 0)) return fail(UAII_ERR_INVALID_ARGUMENT, "null args");
  auto* p = reinterpret_cast<SessionHandle*>(session)->session.program();
  if (!p) return fail(UAII_ERR_INVALID_ARGUMENT, "session not ready");
  return from_error(p->read_ids(out, (int64_t)n));
}

uaii_status uaii_session_seek(uaii_session* session, int64_t pos) {
  if (session == nullptr) return fail(UAII_ERR_INVALID_ARGUMENT, "session null");
  auto* p = reinterpret_cast<SessionHandle*>(session)->session.program();
  if (!p) return fail(UAII_ERR_INVALID_ARGUMENT, "session not ready");
  return from_error(p->seek(pos));
}

uaii_status uaii_session_set_profiling(uaii_session* session, int on) {
  if (session == nullptr) return fail(UAII_ERR_INVALID_ARGUMENT, "session null");
  auto* p = reinterpret_cast<SessionHandle*>(session)->session.program();
  if (!p) return fail(UAII_ERR_INVALID_ARGUMENT, "session not ready");
  uaii::Error err = p->synchronize();
  if (!err.ok()) return from_error(err);
  p->set_profile(on != 0);
  if (on) p->reset_timings();
  return UAII_OK;
}

uaii_status uaii_session_set_device_sampler(uaii_session* session, int on) {
  if (session == nullptr) return fail(UAII_ERR_INVALID_ARGUMENT, "session null");
  auto& sess = reinterpret_cast<SessionHandle*>(session)->session;
  auto* p = sess.program();
  if (!p) return fail(UAII_ERR_INVALID_ARGUMENT, "session not ready");
  if (on && !p->sampler_supported())
    return fail(UAII_ERR_NOT_IMPLEMENTED, "device sampler: vocabulary too large");
  sess.set_device_sampler(on != 0);
  return UAII_OK;
}

uaii_status uaii_session_last_margin(uaii_session* session, float* best, float* second) {
  if (session == nullptr || best == nullptr || second == nullptr)
    return fail(UAII_ERR_INVALID_ARGUMENT, "null args");
  auto* p = reinterpret_cast<SessionHandle*>(session)->session.program();
  if (!p) return fail(UAII_ERR_INVALID_ARGUMENT, "session not ready");
  uaii_hip::StepState st{};
  uaii::Error err = p->read_state(&st);
  if (!err.ok()) return from_error(err);
  *best = st.max_logit;
  *second = st.second;
  return UAII_OK;
}

}  // extern "C"
