// gguf_file.cpp — see gguf_file.h.
#include "gguf_file.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cctype>
#include <cstdio>
#include <cstdlib>
#include <cstring>

namespace uaii {

std::string Error::to_string() const {
  if (ok()) return "ok";
  return std::string(uaii::to_string(code_)) + ": " + message_;
}

const char* to_string(ErrorCode code) noexcept {
  switch (code) {
    case ErrorCode::Ok: return "ok";
    case ErrorCode::InvalidArgument: return "invalid_argument";
    case ErrorCode::NotFound: return "not_found";
    case ErrorCode::IoError: return "io_error";
    case ErrorCode::ConfigError: return "config_error";
    case ErrorCode::PluginError: return "plugin_error";
    case ErrorCode::AbiMismatch: return "abi_mismatch";
    case ErrorCode::NotImplemented: return "not_implemented";
    default: return "internal";
  }
}

namespace {

struct Cursor {
  const uint8_t* p;
  const uint8_t* end;
  bool bad = false;
  uint64_t u(int n) {
    if (p + n > end) { bad = true; p = end; return 0; }
    uint64_t v = 0;
    for (int i = 0; i < n; ++i) v |= (uint64_t)p[i] << (8 * i);
    p += n;
    return v;
  }
  std::string str() {
    const uint64_t n = u(8);
    if (bad || n > (uint64_t)(end - p)) { bad = true; return {}; }
    std::string s(reinterpret_cast<const char*>(p), (size_t)n);
    p += n;
    return s;
  }
};

int scalar_bytes(uint32_t t) {
  switch (t) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    default: return -1;
  }
}

// Typed KV value (value types 0-12, gguf.cpp:20-34). Arrays are skipped.
bool read_value(Cursor& c, uint32_t t, GgufValue* v, int depth = 0) {
  v->type = t;
  switch (t) {
    case 0: v->i = (int64_t)(uint8_t)c.u(1); v->is_int = true; break;
    case 1: v->i = (int64_t)(int8_t)c.u(1); v->is_int = true; break;
    case 2: v->i = (int64_t)(uint16_t)c.u(2); v->is_int = true; break;
    case 3: v->i = (int64_t)(int16_t)c.u(2); v->is_int = true; break;
    case 4: v->i = (int64_t)(uint32_t)c.u(4); v->is_int = true; break;
    case 5: v->i = (int64_t)(int32_t)c.u(4); v->is_int = true; break;
    case 6: { uint32_t b = (uint32_t)c.u(4); float f; std::memcpy(&f, &b, 4); v->f = f; v->is_float = true; break; }
    case 7: v->i = (int64_t)c.u(1); break;
    case 8: v->s = c.str(); v->is_str = true; break;
    case 9: {
      if (depth > 4) return false;
      const uint32_t et = (uint32_t)c.u(4);
      const uint64_t n = c.u(8);
      GgufValue tmp;
      for (uint64_t k = 0; k < n && !c.bad; ++k) {
        if (et == 8) { c.str(); continue; }
        const int sb = scalar_bytes(et);
        if (sb > 0) { if ((uint64_t)sb > (uint64_t)(c.end - c.p)) { c.bad = true; break; } c.p += sb; continue; }
        if (!read_value(c, et, &tmp, depth + 1)) return false;
      }
      break;
    }
    case 10: v->i = (int64_t)c.u(8); v->is_int = true; break;
    case 11: v->i = (int64_t)c.u(8); v->is_int = true; break;
    case 12: { uint64_t b = c.u(8); double d; std::memcpy(&d, &b, 8); v->f = d; v->is_float = true; break; }
    default: return false;
  }
  return !c.bad;
}

int block_elems(int t) {
  switch (t) {
    case 0: case 1: return 1;
    case 2: case 3: case 6: case 7: case 8: return 32;
    case 10: case 11: case 12: case 13: case 14: return 256;
    default: return 0;
  }
}

int block_bytes(int t) {
  switch (t) {
    case 0: return 4; case 1: return 2; case 2: return 18; case 3: return 20; case 6: return 22;
    case 7: return 24; case 8: return 34; case 10: return 84; case 11: return 110;
    case 12: return 144; case 13: return 176; case 14: return 210;
    default: return 0;
  }
}

}  // namespace

bool gguf_type_supported(int type) { return block_elems(type) != 0; }

uint64_t gguf_nbytes(int type, uint64_t n) {
  const int be = block_elems(type);
  return be ? (n / (uint64_t)be) * (uint64_t)block_bytes(type) : 0;
}

GgufFile::~GgufFile() {
  if (map_) munmap(map_, len_);
}

Error GgufFile::open(const std::string& path) {
  path_ = path;
  const int fd = ::open(path.c_str(), O_RDONLY);
  if (fd < 0) return Error::make(ErrorCode::NotFound, "cannot open " + path);
  struct stat st;
  if (fstat(fd, &st) != 0) { ::close(fd); return Error::make(ErrorCode::IoError, "stat " + path); }
  len_ = (size_t)st.st_size;
  void* m = len_ ? mmap(nullptr, len_, PROT_READ, MAP_PRIVATE, fd, 0) : MAP_FAILED;
  ::close(fd);
  if (m == MAP_FAILED) return Error::make(ErrorCode::IoError, "mmap failed: " + path);
  map_ = static_cast<uint8_t*>(m);
  Cursor c{map_, map_ + len_};
  if (len_ < 24 || std::memcmp(map_, "GGUF", 4) != 0)
    return Error::make(ErrorCode::InvalidArgument, "not a GGUF file");
  c.p += 4;
  c.u(4);  // version
  const uint64_t n_tensors = c.u(8), n_kv = c.u(8);
  // every tensor info takes at least 24 bytes (name length, rank, type, offset),
  // so a count beyond that cannot be real (and must not size an allocation)
  if (n_tensors > (uint64_t)len_ / 24 || n_kv > (uint64_t)len_ / 12)
    return Error::make(ErrorCode::InvalidArgument, "truncated binary read");
  for (uint64_t i = 0; i < n_kv; ++i) {
    std::string key = c.str();
    const uint32_t t = (uint32_t)c.u(4);
    GgufValue v;
    if (c.bad || !read_value(c, t, &v)) return Error::make(ErrorCode::InvalidArgument, "truncated binary read");
    kv_[key] = std::move(v);
  }
  tensors_.reserve((size_t)n_tensors);
  for (uint64_t i = 0; i < n_tensors; ++i) {
    GgufTensor t;
    t.name = c.str();
    const uint32_t nd = (uint32_t)c.u(4);
    if (nd > 8) return Error::make(ErrorCode::InvalidArgument, "bad tensor rank");
    for (uint32_t d = 0; d < nd; ++d) t.ne.push_back(c.u(8));
    t.type = (int)c.u(4);
    t.offset = c.u(8);
    if (c.bad) return Error::make(ErrorCode::InvalidArgument, "truncated binary read");
    tensors_.push_back(std::move(t));
  }
  const uint64_t data_off = ((uint64_t)(c.p - map_) + 31) & ~(uint64_t)31;
  for (size_t i = 0; i < tensors_.size(); ++i) {
    GgufTensor& t = tensors_[i];
    // element count, byte size and end offset with every product and sum checked
    // for uint64 wrap-around: a crafted header must not pass the end-of-file test
    uint64_t n = 1;
    bool wrap = false;
    for (auto d : t.ne) wrap = wrap || __builtin_mul_overflow(n, d, &n) || d > (uint64_t)INT64_MAX;
    const int be = block_elems(t.type);
    uint64_t end = 0;
    if (!wrap && be) {
      if (n % (uint64_t)be)
        return Error::make(ErrorCode::InvalidArgument,
                           "tensor " + t.name + " element count is not a multiple of its block size");
      wrap = __builtin_mul_overflow(n / (uint64_t)be, (uint64_t)block_bytes(t.type), &t.nbytes) ||
             __builtin_add_overflow(data_off, t.offset, &end) || __builtin_add_overflow(end, t.nbytes, &end);
    }
    if (wrap || n > (uint64_t)INT64_MAX)
      return Error::make(ErrorCode::InvalidArgument, "tensor " + t.name + " size overflows");
    // bytes past the end of the file: left unreadable (data null) for the load
    // to report, as the reference reads tensors only when it loads them
    const bool readable = be && data_off + t.offset <= (uint64_t)len_ && end <= (uint64_t)len_;
    t.data = readable ? map_ + data_off + t.offset : nullptr;
    index_[t.name] = i;
  }
  return Error::success();
}

const GgufTensor* GgufFile::find(const std::string& name) const {
  auto it = index_.find(name);
  return it == index_.end() ? nullptr : &tensors_[it->second];
}

const GgufValue* GgufFile::kv(const std::string& key) const {
  auto it = kv_.find(key);
  return it == kv_.end() ? nullptr : &it->second;
}

// kv_i64 accepts i64 / u64 / i32 / u32 (gguf.cpp:664-676).
int64_t GgufFile::kv_int(const std::string& key, int64_t def) const {
  const GgufValue* v = kv(key);
  if (!v) return def;
  if (v->type == 4 || v->type == 5 || v->type == 10 || v->type == 11) return v->i;
  return def;
}

// kv_float accepts f32 / f64 / i32 / i64 / u32 / u64 (gguf.cpp:693-707).
float GgufFile::kv_float(const std::string& key, float def) const {
  const GgufValue* v = kv(key);
  if (!v) return def;
  if (v->is_float) return (float)v->f;
  if (v->type == 4 || v->type == 5 || v->type == 10 || v->type == 11) return (float)v->i;
  return def;
}

std::string GgufFile::kv_string(const std::string& key) const {
  const GgufValue* v = kv(key);
  return (v && v->is_str) ? v->s : std::string();
}

namespace {

// {arch}.suffix, then llama.suffix, then general.suffix (gguf.cpp:734-763).
int64_t arch_int(const GgufFile& f, const std::string& arch, const char* suf, int64_t def) {
  if (!arch.empty()) {
    const int64_t v = f.kv_int(arch + "." + suf, -1);
    if (v >= 0) return v;
  }
  int64_t v = f.kv_int(std::string("llama.") + suf, -1);
  if (v >= 0) return v;
  v = f.kv_int(std::string("general.") + suf, -1);
  if (v >= 0) return v;
  return def;
}

float arch_float(const GgufFile& f, const std::string& arch, const char* suf, float def) {
  if (!arch.empty() && f.kv(arch + "." + suf)) return f.kv_float(arch + "." + suf, def);
  if (f.kv(std::string("llama.") + suf)) return f.kv_float(std::string("llama.") + suf, def);
  if (f.kv(std::string("general.") + suf)) return f.kv_float(std::string("general.") + suf, def);
  return def;
}

const GgufTensor* find_any(const GgufFile& f, std::initializer_list<const char*> names) {
  for (const char* n : names) if (const GgufTensor* t = f.find(n)) return t;
  return nullptr;
}

}  // namespace

Error derive_decoder(const GgufFile& f, DecoderSpec* o) {
  DecoderSpec d;
  d.tok_embd = find_any(f, {"token_embd.weight", "embed.weight", "model.embed_tokens.weight", "token_embd"});
  d.output = find_any(f, {"output.weight", "lm_head.weight", "output"});
  d.tied = d.output == nullptr && d.tok_embd != nullptr;
  if (d.tied) d.output = d.tok_embd;
  d.out_norm = find_any(f, {"output_norm.weight", "norm.weight", "output_norm"});
  const bool has_blk0 = f.find("blk.0.attn_q.weight") || f.find("blk.0.attn_norm.weight");
  if (!d.tok_embd || !d.output || !has_blk0)
    return Error::make(ErrorCode::NotImplemented, "GGUF file is not a blk.* transformer decoder");
  std::string arch = f.kv_string("general.architecture");
  for (char& ch : arch) ch = (char)std::tolower((unsigned char)ch);
  d.arch = arch;
  for (const GgufTensor* t : {d.tok_embd, d.output, d.out_norm}) {
    if (t && !gguf_type_supported(t->type))
      return Error::make(ErrorCode::NotImplemented, "unsupported GGUF quant type for weight " + t->name);
  }
  d.dim = d.tok_embd->cols();
  d.vocab = d.output->rows();
  d.n_heads = arch_int(f, arch, "attention.head_count", 0);
  if (d.n_heads <= 0) d.n_heads = 1;
  d.n_kv_heads = arch_int(f, arch, "attention.head_count_kv", d.n_heads);
  if (d.n_kv_heads <= 0) d.n_kv_heads = d.n_heads;
  const int64_t emb_len = arch_int(f, arch, "embedding_length", d.dim);
  d.head_dim = arch_int(f, arch, "attention.key_length", 0);
  if (d.head_dim <= 0) d.head_dim = (emb_len > 0 ? emb_len : d.dim) / d.n_heads;
  d.q_dim = d.n_heads * d.head_dim;
  d.kv_dim = d.n_kv_heads * d.head_dim;
  d.rope_theta = arch_float(f, arch, "rope.freq_base", 10000.f);
  static const char* kNeox[] = {"qwen2", "qwen2moe", "qwen3", "qwen", "phi2", "phi3", "falcon",
                                "stablelm", "starcoder2", "olmo2", "gemma", "gemma2", "gemma3"};
  d.rope_mode = 0;
  for (const char* a : kNeox) if (arch == a) d.rope_mode = 2;
  d.rms_eps = arch_float(f, arch, "attention.layer_norm_rms_epsilon", 1e-5f);
  int64_t n_layers = arch_int(f, arch, "block_count", 0);
  if (n_layers <= 0) {
    for (int64_t i = 0; i < 512; ++i) {
      const std::string p = "blk." + std::to_string(i) + ".";
      if (!f.find(p + "attn_norm.weight") && !f.find(p + "attn_q.weight")) { n_layers = i; break; }
    }
  }
  if (n_layers > 512) n_layers = 512;
  if (const char* env = std::getenv("UAII_MAX_LAYERS")) {
    const int cap = std::atoi(env);
    if (cap > 0 && n_layers > cap) n_layers = cap;
  }
  d.n_experts = arch_int(f, arch, "expert_count", 0);
  d.top_k = arch_int(f, arch, "expert_used_count", 2);
  if (d.top_k <= 0) d.top_k = 2;
  d.ctx_len = arch_int(f, arch, "context_length", 0);

  auto get = [&](const std::string& name, const GgufTensor** out) -> Error {
    *out = f.find(name);
    if (*out && !gguf_type_supported((*out)->type))
      return Error::make(ErrorCode::NotImplemented, "unsupported GGUF quant type for weight " + name);
    return Error::success();
  };
  for (int64_t li = 0; li < n_layers; ++li) {
    const std::string p = "blk." + std::to_string(li) + ".";
    LayerSpec L;
    UAII_TRY(get(p + "attn_norm.weight", &L.attn_norm));
    UAII_TRY(get(p + "attn_q.weight", &L.wq));
    UAII_TRY(get(p + "attn_k.weight", &L.wk));
    UAII_TRY(get(p + "attn_v.weight", &L.wv));
    UAII_TRY(get(p + "attn_q.bias", &L.bq));
    UAII_TRY(get(p + "attn_k.bias", &L.bk));
    UAII_TRY(get(p + "attn_v.bias", &L.bv));
    UAII_TRY(get(p + "attn_output.weight", &L.wo));
    UAII_TRY(get(p + "ffn_norm.weight", &L.ffn_norm));
    UAII_TRY(get(p + "ffn_gate.weight", &L.w_gate));
    UAII_TRY(get(p + "ffn_up.weight", &L.w_up));
    UAII_TRY(get(p + "ffn_down.weight", &L.w_down));
    UAII_TRY(get(p + "ffn_gate_inp.weight", &L.gate_inp));
    UAII_TRY(get(p + "ffn_gate_exps.weight", &L.gate_exps));
    UAII_TRY(get(p + "ffn_up_exps.weight", &L.up_exps));
    UAII_TRY(get(p + "ffn_down_exps.weight", &L.down_exps));
    UAII_TRY(get(p + "ffn_gate_shexp.weight", &L.gate_sh));
    UAII_TRY(get(p + "ffn_up_shexp.weight", &L.up_sh));
    UAII_TRY(get(p + "ffn_down_shexp.weight", &L.down_sh));
    if (!L.attn_norm || !L.wq || !L.wk || !L.wv || !L.wo) break;  // gguf.cpp:993-996
    if (L.gate_inp && L.gate_exps && L.up_exps && L.down_exps) {
      L.ffn = LayerSpec::kMoE;
      L.inter = L.gate_exps->ne.size() >= 2 ? (int64_t)L.gate_exps->ne[1] : 0;
      if (d.n_experts <= 0 && L.gate_exps->ne.size() >= 3) d.n_experts = (int64_t)L.gate_exps->ne[2];
    } else if (L.w_gate && L.w_up && L.w_down) {
      L.ffn = LayerSpec::kSwiGLU;
      L.inter = L.w_up->rows();
    } else if (L.w_up && L.w_down) {
      L.ffn = LayerSpec::kGelu;
      L.inter = L.w_up->rows();
    }
    d.layers.push_back(L);
  }
  d.n_layers = (int64_t)d.layers.size();
  if (d.n_experts > 0 && d.top_k > d.n_experts) d.top_k = d.n_experts;
  *o = std::move(d);
  return Error::success();
}

namespace {

const char* ffn_name(LayerSpec::Ffn f) {
  switch (f) {
    case LayerSpec::kSwiGLU: return "swiglu";
    case LayerSpec::kGelu: return "gelu";
    case LayerSpec::kMoE: return "moe";
    default: return "none";
  }
}

int tensor_type(const GgufTensor* t) { return t ? t->type : -1; }

}  // namespace

std::string describe_decoder(const DecoderSpec& d) {
  std::string s = "{";
  auto kv = [&](const char* k, const std::string& v, bool quote) {
    if (s.size() > 1) s += ", ";
    s += "\"";
    s += k;
    s += "\": ";
    if (quote) s += "\"" + v + "\"";
    else s += v;
  };
  char f[64];
  kv("arch", d.arch, true);
  kv("n_layers", std::to_string(d.n_layers), false);
  kv("dim", std::to_string(d.dim), false);
  kv("n_heads", std::to_string(d.n_heads), false);
  kv("n_kv_heads", std::to_string(d.n_kv_heads), false);
  kv("head_dim", std::to_string(d.head_dim), false);
  kv("q_dim", std::to_string(d.q_dim), false);
  kv("kv_dim", std::to_string(d.kv_dim), false);
  kv("vocab", std::to_string(d.vocab), false);
  kv("ctx_len", std::to_string(d.ctx_len), false);
  kv("n_experts", std::to_string(d.n_experts), false);
  kv("top_k", std::to_string(d.top_k), false);
  std::snprintf(f, sizeof f, "%.9g", (double)d.rope_theta);
  kv("rope_theta", f, false);
  std::snprintf(f, sizeof f, "%.9g", (double)d.rms_eps);
  kv("rms_eps", f, false);
  kv("rope_mode", std::to_string(d.rope_mode), false);
  kv("tied", d.tied ? "true" : "false", false);
  kv("tok_embd_type", std::to_string(tensor_type(d.tok_embd)), false);
  kv("output_type", std::to_string(tensor_type(d.output)), false);
  std::string layers = "[";
  for (size_t i = 0; i < d.layers.size(); ++i) {
    const LayerSpec& L = d.layers[i];
    if (i) layers += ", ";
    layers += "{\"ffn\": \"" + std::string(ffn_name(L.ffn)) + "\", \"inter\": " + std::to_string(L.inter) +
              ", \"wq\": " + std::to_string(tensor_type(L.wq)) + ", \"wk\": " + std::to_string(tensor_type(L.wk)) +
              ", \"wv\": " + std::to_string(tensor_type(L.wv)) + ", \"wo\": " + std::to_string(tensor_type(L.wo)) +
              ", \"bias\": " + ((L.bq || L.bk || L.bv) ? "true" : "false") +
              ", \"down\": " + std::to_string(tensor_type(L.w_down ? L.w_down : L.down_exps)) + "}";
  }
  layers += "]";
  kv("layers", layers, false);
  s += "}";
  return s;
}

}  // namespace uaii
