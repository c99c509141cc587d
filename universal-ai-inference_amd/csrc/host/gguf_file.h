// gguf_file.h — memory-mapped GGUF reader and decoder description.
//
// Header layout follows the reference reader (libs/uaii-loaders/src/gguf.cpp:
// 374-443): magic, version, tensor and KV counts, typed KV entries, tensor infos,
// data section at the next 32-byte boundary (general.alignment is ignored, as in
// the reference). Unlike the reference, which re-reads the whole file for every
// tensor (gguf.cpp:464-467, 592-595), the file is mapped once and tensors are
// served as pointers into the mapping.
//
// DecoderSpec is the decoder the reference's GgufLoader::load derives from the
// same file (gguf.cpp:801-1246): hyperparameter keys with arch / llama. /
// general. fallbacks, tied embeddings, optional Q/K/V biases, dense SwiGLU,
// GELU or MoE FFN, RoPE mode by architecture.
#pragma once

#include "error.h"

#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace uaii {

struct GgufTensor {
  std::string name;
  int type = 0;
  std::vector<uint64_t> ne;  // GGUF order (ne[0] = row length)
  uint64_t offset = 0;
  // null when the file ends before the tensor's bytes do: the header still
  // parses (as gguf_read_header, gguf.cpp:374-443) and the load fails, or takes
  // the session's weight_init fill (session.cpp:510-544)
  const uint8_t* data = nullptr;
  uint64_t nbytes = 0;
  // row-major view after the reference's dims reversal (gguf.cpp:272-280)
  int64_t cols() const { return ne.empty() ? 0 : (int64_t)ne[0]; }
  int64_t rows() const {
    int64_t r = 1;
    for (size_t i = 1; i < ne.size(); ++i) r *= (int64_t)ne[i];
    return r;
  }
};

struct GgufValue {
  uint32_t type = 0;
  int64_t i = 0;
  double f = 0.0;
  std::string s;
  bool is_int = false, is_float = false, is_str = false;
};

class GgufFile {
 public:
  GgufFile() = default;
  ~GgufFile();
  GgufFile(const GgufFile&) = delete;
  GgufFile& operator=(const GgufFile&) = delete;

  Error open(const std::string& path);
  const GgufTensor* find(const std::string& name) const;
  const GgufValue* kv(const std::string& key) const;
  int64_t kv_int(const std::string& key, int64_t def) const;
  float kv_float(const std::string& key, float def) const;
  std::string kv_string(const std::string& key) const;
  const std::vector<GgufTensor>& tensors() const { return tensors_; }
  const std::string& path() const { return path_; }

 private:
  std::string path_;
  uint8_t* map_ = nullptr;
  size_t len_ = 0;
  std::map<std::string, GgufValue> kv_;
  std::vector<GgufTensor> tensors_;
  std::map<std::string, size_t> index_;
};

// Whether the reference can dequantize a GGUF type (gguf.cpp:285-304).
bool gguf_type_supported(int type);
// Packed bytes of n values (include/uaii/quant/formats.hpp:81-102).
uint64_t gguf_nbytes(int type, uint64_t n);

struct LayerSpec {
  const GgufTensor* attn_norm = nullptr;
  const GgufTensor *wq = nullptr, *wk = nullptr, *wv = nullptr, *wo = nullptr;
  const GgufTensor *bq = nullptr, *bk = nullptr, *bv = nullptr;
  const GgufTensor* ffn_norm = nullptr;
  const GgufTensor *w_gate = nullptr, *w_up = nullptr, *w_down = nullptr;
  const GgufTensor *gate_inp = nullptr, *gate_exps = nullptr, *up_exps = nullptr,
                   *down_exps = nullptr;
  const GgufTensor *gate_sh = nullptr, *up_sh = nullptr, *down_sh = nullptr;
  enum Ffn { kNone, kSwiGLU, kGelu, kMoE } ffn = kNone;
  int64_t inter = 0;  // FFN intermediate size (per expert for MoE)
};

struct DecoderSpec {
  std::string arch;
  int64_t n_layers = 0, dim = 0, n_heads = 0, n_kv_heads = 0, head_dim = 0;
  int64_t q_dim = 0, kv_dim = 0, vocab = 0, ctx_len = 0;
  int64_t n_experts = 0, top_k = 0;
  float rope_theta = 10000.f, rms_eps = 1e-5f;
  int rope_mode = 0;
  bool tied = false;
  const GgufTensor* tok_embd = nullptr;
  const GgufTensor* out_norm = nullptr;
  const GgufTensor* output = nullptr;  // == tok_embd when tied
  std::vector<LayerSpec> layers;
};

// Derive the decoder; `max_layers_env` mirrors UAII_MAX_LAYERS (gguf.cpp:785-799).
Error derive_decoder(const GgufFile& f, DecoderSpec* out);

// JSON summary of a derived decoder (uaii_model_describe).
std::string describe_decoder(const DecoderSpec& d);

}  // namespace uaii
