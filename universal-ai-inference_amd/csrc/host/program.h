// program.h — the device-resident decoder program behind Session.
//
// Owns every device allocation of a session: split-layout weights (HBM resident
// for the life of the session), the KV cache ([layer][kv_head][max_seq][hd], f16
// or f32), activations, RoPE tables, the decode state and the step graphs. One
// token step is a fixed kernel sequence whose dynamic inputs (position, token)
// live in device memory, so the sequence is captured once into a hipGraph and
// replayed per token; only the generated ids come back to the host.
#pragma once

#include "error.h"
#include "gguf_file.h"

#include "hip/uaii_hip_internal.h"

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace uaii {

// A weight in the split device layout (see csrc/hip/repack.hip).
struct DeviceWeight {
  uaii_hip::DevWeight view{};
  void* base = nullptr;
  size_t bytes = 0;
  DeviceWeight() = default;
  DeviceWeight(const DeviceWeight&) = delete;
  DeviceWeight& operator=(const DeviceWeight&) = delete;
  ~DeviceWeight();
};

// Upload `rows` GGUF rows of `cols` values and re-lay them out on the device.
// f32_load: the rows take the values the reference's f32 weight load gives them
// (gguf_load_tensor_f32, which orders Q4_0 nibbles pairwise) instead of those of
// its packed decode; the storage stays block-packed either way.
Error upload_weight(int type, const uint8_t* host, int64_t rows, int64_t cols, hipStream_t s,
                    DeviceWeight* out, bool f32_load = false);

struct ProgramOptions {
  // Weights carry the values of the reference's Path A, its f32 weight load
  // (session.cpp:420-443 -> gguf_load_tensor_f32), rather than of its packed
  // quant_gemm path. MoE models always do: the reference runs them on Path A only.
  bool f32_weight_load = false;
  bool kv_f16 = false;        // KV cache storage dtype
  bool use_graph = true;      // replay the captured step graph
  bool profile = false;       // per-kernel HIP event timing (direct launches)
  int64_t max_context = 0;    // 0: GGUF context_length
  // Device bytes the program may hold (weights, KV cache, activations, prompt
  // buffers); 0 = unlimited. Exceeding it is InvalidArgument "memory budget
  // exceeded", as the reference's MemoryBudget::reserve (libs/uaii-memory/src/budget.cpp:6-19).
  uint64_t budget_bytes = 0;
  // A weight whose bytes the file does not hold (session.cpp:510-544): with
  // weight_init 0 (None) the build fails; 1 zeros, 2 ones, 3 i * 0.01 fill the
  // weight's f32 values (packed Path B buffers cannot be filled).
  int weight_init = 0;
  bool allow_missing_weights = false;
  std::string weight_source;  // the file, for the reference's messages
};

struct KernelTiming {
  double total_ms = 0.0;
  int64_t launches = 0;
  double bytes = 0.0;  // algorithmic bytes per launch summed
  double flops = 0.0;  // algorithmic flops per launch summed (matrix-core kernels)
};

class DecoderProgram {
 public:
  DecoderProgram() = default;
  ~DecoderProgram();
  DecoderProgram(const DecoderProgram&) = delete;
  DecoderProgram& operator=(const DecoderProgram&) = delete;

  Error build(const DecoderSpec& spec, const ProgramOptions& opts);
  const DecoderSpec& spec() const { return spec_; }
  int64_t max_context() const { return max_ctx_; }

  // Size KV and the token buffer for `max_seq` positions (re-captures graphs on growth).
  Error ensure_capacity(int64_t max_seq);
  // Reset to position 0 with the given prompt (ids copied to the device).
  Error begin(const int64_t* prompt, int64_t n_prompt);
  // Enqueue one token step at the current position.
  Error step(bool want_logits);
  Error synchronize();
  // Copy ids[0..n) (prompt + generated) to the host.
  Error read_ids(int64_t* out, int64_t n);
  // one id of the history (the id generated at position index - 1 for index >= n_prompt)
  Error read_id(int64_t index, int64_t* id);
  Error read_state(uaii_hip::StepState* st);
  // Run the n tokens ids[pos .. pos + n) through every layer as M-row matrix
  // products on the matrix cores (K/V appended for each position, no logits),
  // then leave ids[pos + n] as the token the next step() feeds.
  Error prefill(int64_t n);
  // Whether prefill() covers this model (weight formats, FFN kind, f16 KV cache).
  bool prefill_supported() const { return pf_ok_; }
  // Overwrite the token fed at the current position.
  Error set_token(int64_t token);
  // Rewind to `pos` (ids and KV below it are kept; ids[pos] is fed next).
  Error seek(int64_t pos);
  // Token draws on the device (sample.hip) in place of the greedy argmax for the
  // steps that compute logits: the reference's sampler parameters, and r[t], the
  // uniform for the token generated at position n_prompt + t.
  struct SamplerParams {
    float inv_t = 1.0f;  // 1 / max(temperature, 1e-5)
    float top_p = 1.0f;
    int32_t top_k = 0;
    float rep = 1.0f;
    bool operator==(const SamplerParams& o) const {
      return inv_t == o.inv_t && top_p == o.top_p && top_k == o.top_k && rep == o.rep;
    }
  };
  bool sampler_supported() const { return spec_.vocab <= uaii_hip::sample_max_vocab(); }
  Error arm_sampler(const SamplerParams& p, const float* r, int64_t n);
  void disarm_sampler() { sampler_on_ = false; }
  void set_profile(bool on) { opts_.profile = on; }
  Error read_tap(const std::string& name, std::vector<float>* out);
  std::string profile_summary() const;
  const std::map<std::string, KernelTiming>& timings() const { return timing_; }
  void reset_timings() { timing_.clear(); }
  hipStream_t stream() const { return stream_; }

 private:
  struct Layer {
    DeviceWeight wq, wk, wv, wo, gate, up, down, gate_inp, gate_exps, up_exps, down_exps;
    DeviceWeight gate_sh, up_sh, down_sh;  // MoE shared expert (ffn_*_shexp)
    float *attn_norm = nullptr, *ffn_norm = nullptr, *bq = nullptr, *bk = nullptr, *bv = nullptr;
    bool shared = false;
    int64_t inter_sh = 0;
  };

  Error upload_f32(const GgufTensor* t, float** out);
  Error missing_weight(const GgufTensor* t, bool packed, std::vector<float>* fill);
  // Count `bytes` against the device budget in `pool` (static, dynamic or prompt buffers).
  Error charge(uint64_t& pool, uint64_t bytes);
  uint64_t used_static_ = 0, used_dyn_ = 0, used_pf_ = 0;
  // Profiling mode: each launch group records a start/stop event pair on its own
  // kernel dispatches (hipExtLaunchKernelGGL through UAII_LAUNCH), with no
  // synchronisation between kernels; collect_timings() reads the pairs.
  template <class F>
  Error timed(const char* name, double bytes, double flops, F&& launch);
  Error collect_timings();
  Error ensure_prefill_buffers(int64_t chunk);
  Error pf_gemm(const DeviceWeight* w[3], const int64_t cols0[3], int nw, const DeviceWeight* w2,
                int epi, int64_t m, float* y, int64_t ldy, int store_split = 1);
  int pf_store_split(const DeviceWeight* w[3], int nw, int64_t m, int64_t ldy);
  Error pf_prep(float* x, int64_t K, int64_t m, const float* norm_w, bool hi16 = false);
  template <class Prep, class Gemm>
  Error prefill_moe(const Layer& L, const LayerSpec& ls, int64_t m, Prep&& prep, Gemm&& gemm);
  Error encode_step(bool want_logits);
  void free_dynamic();

  DecoderSpec spec_;
  ProgramOptions opts_;
  hipStream_t stream_ = nullptr;
  std::vector<std::unique_ptr<Layer>> layers_;
  DeviceWeight tok_embd_, output_;
  float* out_norm_ = nullptr;
  std::vector<void*> allocs_;  // owned static allocations (norms, biases, activations)

  // activations
  float *x_ = nullptr, *q_ = nullptr, *attn_ = nullptr, *h_ = nullptr, *logits_ = nullptr,
        *probs_ = nullptr, *tap_hidden_ = nullptr, *tap_r1_ = nullptr, *tap_r2_ = nullptr,
        *tap_normed_ = nullptr, *moe_logits_ = nullptr, *moe_w_ = nullptr;
  int32_t* moe_ids_ = nullptr;
  float* lm_part_val_ = nullptr;
  int32_t* lm_part_idx_ = nullptr;
  int lm_blocks_ = 0;  // capacity of the LM-head partial buffers
  bool pf_h16_ = true;    // Q4_0 prefill GEMMs on PfAct::hi16 activations (UAII_PF_H16=0: off)
  // profiling mode: start/stop event pairs and their (kernel name, bytes) per launch group
  struct ProfTag {
    std::string name;
    double bytes = 0.0, flops = 0.0;
  };
  std::vector<std::pair<hipEvent_t, hipEvent_t>> prof_events_;
  std::vector<ProfTag> prof_tags_;
  size_t prof_used_ = 0;
  uaii_hip::StepState* state_ = nullptr;

  // sized by ensure_capacity
  int64_t max_ctx_ = 0;
  void* kv_ = nullptr;
  size_t kv_bytes_ = 0;
  int32_t* ids_ = nullptr;
  float2* rope_ = nullptr;
  float* attn_part_ = nullptr;
  // decode attention merged inside the split kernel: tickets + fail word
  // (AttnArgs::sync), null when the two-launch path runs
  int attn_splits_ = 1;

  // the residual-add GEMVs (O, down) through the LDS ring (ring_gemv.hip) where
  // the shapes allow: 1 (default) or 0 none
  int ring_mode_ = 0;
  bool splitk_ = true;  // O (with the split merge) and down split along K, atomic residual adds
  uint8_t* ring_pad_ = nullptr;

  // step graphs: no logits, greedy logits, sampled logits
  hipGraphExec_t graph_[3] = {nullptr, nullptr, nullptr};
  bool sampler_on_ = false;
  SamplerParams samp_{}, samp_graph_{};  // armed; baked into graph_[2]
  float* samp_r_ = nullptr;              // the draws
  int64_t samp_r_cap_ = 0, samp_n_ = 0;
  void* samp_ws_ = nullptr;              // sample_workspace_bytes(vocab)
  std::map<std::string, KernelTiming> timing_;
  hipEvent_t ev0_ = nullptr, ev1_ = nullptr;
  int64_t hid_max_ = 0;  // floats of the FFN hidden buffer (gate/up output)
  bool moe_ = false;

  // prefill: chunk buffers ([chunk][...] rows) and the prepared-activation scratch
  bool pf_ok_ = false;
  int64_t pf_chunk_ = 0, pf_kmax_ = 0;
  float *pf_x_ = nullptr, *pf_qkv_ = nullptr, *pf_q_ = nullptr, *pf_attn_ = nullptr,
        *pf_h_ = nullptr;
  float* pf_part_ = nullptr;  // [4][chunk][dim]: K-split partials of a residual-add GEMM
  // MoE prompt rows: routing [chunk][k], per-expert lists, expert outputs
  int32_t *pf_moe_ids_ = nullptr, *pf_moe_cnt_ = nullptr, *pf_moe_list_ = nullptr,
          *pf_moe_inv_ = nullptr, *pf_moe_tab_ = nullptr;
  int64_t pf_tab_cap_ = 0;             // int32 entries of pf_moe_tab_
  int64_t pf_part_cols_ = 0;           // columns per row of pf_part_
  std::vector<int32_t> pf_tab_host_;   // the grouped GEMMs' row tables before upload
  float *pf_moe_w_ = nullptr, *pf_moe_y_ = nullptr, *pf_hsh_ = nullptr;
  int pf_pending_ = 0;        // splits in pf_part_ still to be added into pf_x_
  int cus_ = 0;
  uaii_hip::PfAct pf_act_{};  // mpad: rows of the last prep (the GEMMs' tiling)
  int64_t pf_act_rows_ = 0;   // row capacity of pf_act_
  std::vector<void*> pf_allocs_;
};

template <class F>
Error DecoderProgram::timed(const char* name, double bytes, double flops, F&& launch) {
  if (!opts_.profile) {
    UAII_HIP(launch());
    return Error::success();
  }
  if (prof_used_ == prof_events_.size()) {
    hipEvent_t a = nullptr, b = nullptr;
    UAII_HIP(hipEventCreate(&a));
    UAII_HIP(hipEventCreate(&b));
    prof_events_.push_back({a, b});
    prof_tags_.push_back(ProfTag{});
  }
  uaii_hip::g_launch_events.start = prof_events_[prof_used_].first;
  uaii_hip::g_launch_events.stop = prof_events_[prof_used_].second;
  const hipError_t st = launch();
  uaii_hip::g_launch_events = uaii_hip::LaunchEvents{};
  UAII_HIP(st);
  prof_tags_[prof_used_] = ProfTag{name, bytes, flops};
  ++prof_used_;
  return Error::success();
}

}  // namespace uaii
