// session.cpp — see session.h.
#include "session.h"

#include <algorithm>
#include <random>
#include <cstdlib>

namespace uaii {
namespace runtime {

Error Session::create(const std::string& gguf_path, SessionOptions options) {
  options_ = std::move(options);
  ready_ = false;
  if (options_.backend_name != "rocm") {
    return Error::make(ErrorCode::NotImplemented,
                       "backend '" + options_.backend_name +
                           "' is not provided by this library (it implements 'rocm')");
  }
  if (options_.enable_streaming) {
    return Error::make(ErrorCode::NotImplemented,
                       "weight streaming is not supported: the model is HBM resident");
  }
  std::string path = gguf_path;
  if (!options_.weights_dir.empty() && !path.empty() && path[0] != '/')
    path = options_.weights_dir + "/" + path;
  UAII_TRY(file_.open(path));
  UAII_TRY(derive_decoder(file_, &spec_));
  ProgramOptions po;
  // The reference holds every weight as f32 from gguf_load_tensor_f32 (Path A)
  // when memory reuse is on (each weight's slot is sized for f32, so the packed
  // copy is refused: session.cpp:259-367, :420-443) or when quantized weights are
  // not kept (:342-366); only memory_reuse=0 with keep_quantized_weights=1 keeps
  // them packed (Path B). The values differ for Q4_0 (gguf.cpp:514-520); device
  // storage stays packed on both paths.
  po.f32_weight_load = options_.enable_memory_reuse || !options_.keep_quantized_weights;
  po.kv_f16 = options_.kv_f16;
  // UAII_NO_GRAPH=1 launches the step kernels directly instead of replaying the
  // captured graph (same kernels; for tools that cannot follow stream capture).
  const char* ng = std::getenv("UAII_NO_GRAPH");
  po.use_graph = options_.use_graph && !(ng && ng[0] == '1');
  po.profile = options_.enable_profiler;
  po.max_context = options_.max_context;
  po.budget_bytes = options_.budget_bytes;
  po.weight_init = static_cast<int>(options_.weight_init);
  po.allow_missing_weights = options_.allow_missing_weights;
  po.weight_source = path;
  if (const char* ds = std::getenv("UAII_DEVICE_SAMPLER")) options_.device_sampler = ds[0] == '1';
  program_ = std::make_unique<DecoderProgram>();
  UAII_TRY(program_->build(spec_, po));
  ready_ = true;
  return Error::success();
}

// max_context option, else GGUF context_length (session.cpp:936-946).
int64_t Session::resolve_max_context() const {
  if (options_.max_context > 0) return options_.max_context;
  return spec_.ctx_len;
}

Error Session::generate(const std::vector<int64_t>& prompt, int64_t max_new,
                        std::vector<int64_t>* out, const std::vector<int64_t>& stop_ids,
                        const OnNewToken& on_new_token, const SampleParams& sample) {
  if (!ready_) return Error::make(ErrorCode::InvalidArgument, "session not ready");
  if (out == nullptr) return Error::make(ErrorCode::InvalidArgument, "out_tokens null");
  if (prompt.empty()) return Error::make(ErrorCode::InvalidArgument, "prompt_tokens empty");
  if (max_new < 0) return Error::make(ErrorCode::InvalidArgument, "max_new_tokens < 0");
  const int64_t max_ctx = resolve_max_context();
  const int64_t n_prompt = (int64_t)prompt.size();
  const int64_t total = n_prompt + max_new;
  if (max_ctx > 0) {
    if (n_prompt > max_ctx)
      return Error::make(ErrorCode::InvalidArgument,
                         "prompt length exceeds max_context (" + std::to_string(n_prompt) + " > " +
                             std::to_string(max_ctx) + ")");
    if (total > max_ctx)
      return Error::make(ErrorCode::InvalidArgument,
                         "prompt+max_new_tokens exceeds max_context (" + std::to_string(total) +
                             " > " + std::to_string(max_ctx) + ")");
  }
  const int64_t kv_max =
      max_ctx > 0 ? max_ctx : std::max<int64_t>(total, n_prompt + std::max<int64_t>(max_new, 1));
  DecoderProgram& p = *program_;
  UAII_TRY(p.ensure_capacity(kv_max));
  UAII_TRY(p.begin(prompt.data(), n_prompt));
  run_started_ = true;

  // Non-greedy draws use a seeded mt19937_64 (session.cpp:989-995), one uniform
  // per generated token (sampling.cpp:111-112).
  std::mt19937_64 rng;
  if (!sample.greedy()) {
    if (sample.has_seed) {
      rng.seed(sample.seed);
    } else {
      std::random_device rd;
      rng.seed((static_cast<uint64_t>(rd()) << 32) ^ static_cast<uint64_t>(rd()));
    }
  }
  // The device sampler takes the draws up front and picks each token where its
  // logits are: only the ids come back, as on the greedy path.
  const bool dev_sample = !sample.greedy() && options_.device_sampler && p.sampler_supported();
  struct Disarm {
    DecoderProgram* p;
    ~Disarm() {
      if (p) p->disarm_sampler();
    }
  } disarm{nullptr};
  if (dev_sample) {
    std::uniform_real_distribution<float> dist(0.0f, 1.0f);
    std::vector<float> r((size_t)std::max<int64_t>(max_new, 1));
    for (auto& v : r) v = dist(rng);
    DecoderProgram::SamplerParams sp;
    sp.inv_t = 1.0f / std::max(sample.temperature, 1e-5f);
    sp.top_p = sample.top_p;
    sp.top_k = sample.top_k;
    sp.rep = sample.repetition_penalty;
    UAII_TRY(p.arm_sampler(sp, r.data(), (int64_t)r.size()));
    disarm.p = &p;
  }

  out->clear();
  // Prefill. The reference runs one step per prompt token; here all prompt
  // tokens but the last go through the matrix-core path as M-row products when
  // the model's formats allow it, and the last one runs the ordinary step with
  // the LM head. Otherwise one step per prompt token, logits only at the end.
  if (n_prompt > 1 && p.prefill_supported()) {
    UAII_TRY(p.prefill(n_prompt - 1));
    UAII_TRY(p.step(true));
  } else {
    for (int64_t i = 0; i < n_prompt; ++i) UAII_TRY(p.step(i == n_prompt - 1));
  }
  const bool per_token = (bool)on_new_token || !stop_ids.empty();
  auto is_stop = [&](int64_t t) { return std::find(stop_ids.begin(), stop_ids.end(), t) != stop_ids.end(); };
  if (!sample.greedy() && !dev_sample) {
    // Non-greedy on the host: the reference samples the pre-softmax `logits` row
    // (want_logits = !sample.greedy(), session.cpp:974-978) with the seeded
    // generator (:1018-1026); each step's logits come back from the device and
    // the chosen id is fed to the next step. The sampler applies its own
    // softmax, so the device's softmax kernel does not run on this path.
    out->assign(prompt.begin(), prompt.end());
    std::vector<float> logits;
    for (int64_t t = 0; t < max_new; ++t) {
      UAII_TRY(p.read_tap("logits", &logits));
      int64_t next = 0;
      UAII_TRY(sample_token_f32(logits.data(), logits.size(), sample, *out, &rng, &next));
      out->push_back(next);
      if (on_new_token && !on_new_token(next)) return Error::success();
      if (is_stop(next)) return Error::success();
      if (t + 1 >= max_new) break;
      UAII_TRY(p.set_token(next));
      UAII_TRY(p.step(true));
    }
    return Error::success();
  }
  if (!per_token) {
    // Whole decode on the device: every step's argmax (or draw) feeds the next step.
    for (int64_t t = 0; t + 1 < max_new; ++t) UAII_TRY(p.step(true));
    out->resize((size_t)total);
    UAII_TRY(p.read_ids(out->data(), total));
    return Error::success();
  }
  out->assign(prompt.begin(), prompt.end());
  for (int64_t t = 0; t < max_new; ++t) {
    // one 4-byte id per token: the one this step's argmax (or draw) appended
    int64_t next = 0;
    UAII_TRY(p.read_id(n_prompt + t, &next));
    out->push_back(next);
    if (on_new_token && !on_new_token(next)) return Error::success();
    if (is_stop(next)) return Error::success();
    if (t + 1 >= max_new) break;
    UAII_TRY(p.step(true));
  }
  return Error::success();
}

Error Session::begin(const std::vector<int64_t>& prompt, int64_t capacity) {
  if (!ready_) return Error::make(ErrorCode::InvalidArgument, "session not ready");
  if (prompt.empty()) return Error::make(ErrorCode::InvalidArgument, "prompt_tokens empty");
  int64_t cap = capacity > 0 ? capacity : resolve_max_context();
  if (cap <= 0) cap = (int64_t)prompt.size() + 1;
  const int64_t max_ctx = resolve_max_context();
  if (max_ctx > 0 && cap > max_ctx)
    return Error::make(ErrorCode::InvalidArgument, "capacity exceeds max_context");
  UAII_TRY(program_->ensure_capacity(cap));
  UAII_TRY(program_->begin(prompt.data(), (int64_t)prompt.size()));
  run_started_ = true;
  return Error::success();
}

Error Session::step_async(bool want_logits) {
  if (!ready_ || !run_started_) return Error::make(ErrorCode::InvalidArgument, "session not started");
  return program_->step(want_logits);
}

Error Session::prefill(int64_t n) {
  if (!ready_ || !run_started_) return Error::make(ErrorCode::InvalidArgument, "session not started");
  return program_->prefill(n);
}

Error Session::set_tensor_f32(const std::string& name, const std::vector<float>& values) {
  if (!ready_) return Error::make(ErrorCode::InvalidArgument, "session not ready");
  if (name != "tokens")
    return Error::make(ErrorCode::NotFound, "settable tensor is 'tokens' only: " + name);
  if (values.empty()) return Error::make(ErrorCode::InvalidArgument, "tokens buffer empty");
  // seq=1 graphs take the last id (session.cpp:858-873)
  pending_token_ = (int64_t)values.back();
  if (run_started_) return program_->set_token(pending_token_);
  return Error::success();
}

Error Session::run() {
  if (!ready_) return Error::make(ErrorCode::InvalidArgument, "session not ready");
  DecoderProgram& p = *program_;
  if (!run_started_) {
    const int64_t max_ctx = resolve_max_context();
    UAII_TRY(p.ensure_capacity(max_ctx > 0 ? max_ctx : 4096));
    const int64_t tok = pending_token_;
    UAII_TRY(p.begin(&tok, 1));
    run_started_ = true;
  }
  uaii_hip::StepState st{};
  UAII_TRY(p.read_state(&st));
  if (st.pos >= p.max_context())
    return Error::make(ErrorCode::InvalidArgument, "KvCache capacity exceeded");
  UAII_TRY(p.step(true));
  return p.synchronize();
}

Error Session::get_tensor_f32(const std::string& name, std::vector<float>* values) {
  if (!ready_) return Error::make(ErrorCode::InvalidArgument, "session not ready");
  if (values == nullptr) return Error::make(ErrorCode::InvalidArgument, "values null");
  return program_->read_tap(name, values);
}

}  // namespace runtime
}  // namespace uaii
