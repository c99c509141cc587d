// session.h — C++ session API of the MI355X token loop.
//
// Mirrors the reference's runtime::Session surface for this path
// (include/uaii/runtime/session.hpp:39-185): SessionOptions fields with the same
// meaning, create / generate / run / set_tensor_f32 / get_tensor_f32,
// OnNewToken returning false to stop, stop ids included in the output, and the
// same context-length checks and error codes as Session::generate
// (libs/uaii-runtime/src/session.cpp:910-1046). The graph it runs is the decoder
// derived from the GGUF file (DecoderSpec), executed by DecoderProgram on the GPU.
#pragma once

#include "error.h"
#include "gguf_file.h"
#include "program.h"
#include "sampling.h"

#include <cstdint>
#include <functional>
#include <memory>
#include <string>
#include <vector>

namespace uaii {
namespace runtime {

enum class WeightInit { None = 0, Zeros, Ones, Sequence };

struct SessionOptions {
  WeightInit weight_init = WeightInit::None;
  std::string weights_dir;
  bool allow_missing_weights = false;
  std::string weights_sandbox;
  std::string backend_name = "rocm";
  bool enable_fusion = true;
  bool enable_memory_reuse = true;
  bool enable_streaming = false;
  bool enable_profiler = false;
  std::string profile_trace_path;
  bool kv_f16 = false;               // compute_dtype == F16
  bool keep_quantized_weights = true;
  int64_t max_context = 0;
  uint64_t budget_bytes = 0;
  bool use_graph = true;             // replay captured step graphs
  // non-greedy draws on the device (sample.hip) instead of the host sampler;
  // UAII_DEVICE_SAMPLER=1 also turns it on
  bool device_sampler = false;
};


class Session {
 public:
  Session() = default;
  ~Session() = default;
  Session(const Session&) = delete;
  Session& operator=(const Session&) = delete;

  Error create(const std::string& gguf_path, SessionOptions options = {});
  bool ready() const noexcept { return ready_; }

  using OnNewToken = std::function<bool(int64_t token_id)>;
  Error generate(const std::vector<int64_t>& prompt_tokens, int64_t max_new_tokens,
                 std::vector<int64_t>* out_tokens, const std::vector<int64_t>& stop_token_ids = {},
                 const OnNewToken& on_new_token = {}, const SampleParams& sample = {});

  // One token step at the current position (token from set_tensor_f32("tokens")).
  Error run();
  Error set_tensor_f32(const std::string& name, const std::vector<float>& values);
  Error get_tensor_f32(const std::string& name, std::vector<float>* values);
  std::string profile_summary() const { return program_ ? program_->profile_summary() : "{}"; }

  // Step-level token loop (uaii_ext.h).
  Error begin(const std::vector<int64_t>& prompt, int64_t capacity);
  Error step_async(bool want_logits);
  // Prompt tokens [pos, pos + n) through the matrix-core path (no logits).
  Error prefill(int64_t n);
  DecoderProgram* program() { return program_.get(); }
  void set_device_sampler(bool on) { options_.device_sampler = on; }
  bool device_sampler() const { return options_.device_sampler; }
  const DecoderSpec& spec() const { return spec_; }

 private:
  int64_t resolve_max_context() const;

  bool ready_ = false;
  SessionOptions options_;
  GgufFile file_;
  DecoderSpec spec_;
  std::unique_ptr<DecoderProgram> program_;
  bool run_started_ = false;
  int64_t pending_token_ = 0;
};

}  // namespace runtime
}  // namespace uaii
