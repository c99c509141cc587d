// program.cpp — see program.h.
#include "program.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <sstream>

namespace uaii {

using namespace uaii_hip;

namespace {

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

double gguf_bpw(int type) {
  const int be = block_elems(type);
  return be ? (double)block_bytes(type) / (double)be : 0.0;
}

// Algorithmic bytes of one M=1 GEMV: packed weight + f32 input + f32 output.
double gemv_bytes(const DevWeight& w) {
  return (double)w.rows * (double)w.cols * gguf_bpw(w.type) + 4.0 * (double)w.cols +
         4.0 * (double)w.rows;
}

// RoPE angle table, computed with the reference's own float expressions
// (transformer.cpp:195-216): freq = 1/powf(theta, 2p/hd), angle = pos*freq.
std::vector<float2> rope_table(float theta, int hd, int64_t max_pos) {
  std::vector<float2> tab((size_t)max_pos * (size_t)(hd / 2));
  for (int p = 0; p < hd / 2; ++p) {
    const float freq = 1.0f / std::pow(theta, static_cast<float>(2 * p) / static_cast<float>(hd));
    for (int64_t pos = 0; pos < max_pos; ++pos) {
      const float ang = static_cast<float>(pos) * freq;
      tab[(size_t)pos * (size_t)(hd / 2) + (size_t)p] = make_float2(std::cos(ang), std::sin(ang));
    }
  }
  return tab;
}

}  // namespace

DeviceWeight::~DeviceWeight() {
  if (base) (void)hipFree(base);
}

Error upload_weight(int type, const uint8_t* host, int64_t rows, int64_t cols, hipStream_t s,
                    DeviceWeight* out, bool f32_load) {
  const int be = block_elems(type);
  if (be == 0) return Error::make(ErrorCode::NotImplemented, "unsupported GGUF type " + std::to_string(type));
  if (rows <= 0 || cols <= 0 || cols % be)
    return Error::make(ErrorCode::InvalidArgument, "weight cols not a multiple of the block size");
  int64_t rb[4];
  split_row_bytes(type, cols, rb);
  if (rb[0] % 16)
    return Error::make(ErrorCode::InvalidArgument, "weight row payload not a multiple of 16 bytes");
  size_t off[4], total = 0;
  for (int k = 0; k < 4; ++k) {
    off[k] = total;
    total = align_up(total + (size_t)(rows * rb[k]), 256);
  }
  UAII_HIP(hipMalloc(&out->base, total));
  out->bytes = total;
  DevWeight& v = out->view;
  v.type = type;
  v.rows = rows;
  v.cols = cols;
  uint8_t* b = static_cast<uint8_t*>(out->base);
  v.a = b + off[0]; v.b = b + off[1]; v.c = b + off[2]; v.d = b + off[3];
  v.a_row = rb[0]; v.b_row = rb[1]; v.c_row = rb[2]; v.d_row = rb[3];

  const int64_t raw_row = (int64_t)gguf_nbytes(type, (uint64_t)cols);
  const int64_t chunk_rows = std::max<int64_t>(1, std::min<int64_t>(rows, (64ll << 20) / raw_row));
  void* stage = nullptr;
  UAII_HIP(hipMalloc(&stage, (size_t)(chunk_rows * raw_row)));
  Error err;
  for (int64_t r0 = 0; r0 < rows && err.ok(); r0 += chunk_rows) {
    const int64_t n = std::min(chunk_rows, rows - r0);
    hipError_t st = hipMemcpyAsync(stage, host + r0 * raw_row, (size_t)(n * raw_row),
                                   hipMemcpyHostToDevice, s);
    if (st == hipSuccess) {
      DevWeight sub = v;
      sub.rows = n;
      sub.a += r0 * v.a_row; sub.b += r0 * v.b_row; sub.c += r0 * v.c_row; sub.d += r0 * v.d_row;
      st = launch_repack(sub, static_cast<const uint8_t*>(stage), s, f32_load);
    }
    if (st == hipSuccess) st = hipStreamSynchronize(s);
    err = hip_error(st, "weight upload");
  }
  (void)hipFree(stage);
  return err;
}

DecoderProgram::~DecoderProgram() {
  free_dynamic();
  if (samp_r_) (void)hipFree(samp_r_);
  for (void* p : pf_allocs_) (void)hipFree(p);
  for (void* p : allocs_) (void)hipFree(p);
  if (ev0_) (void)hipEventDestroy(ev0_);
  if (ev1_) (void)hipEventDestroy(ev1_);
  if (stream_) (void)hipStreamDestroy(stream_);
}

void DecoderProgram::free_dynamic() {
  for (auto& g : graph_) {
    if (g) (void)hipGraphExecDestroy(g);
    g = nullptr;
  }
  for (void* p : {(void*)kv_, (void*)ids_, (void*)rope_, (void*)attn_part_}) {
    if (p) (void)hipFree(p);
  }
  kv_ = nullptr; ids_ = nullptr; rope_ = nullptr; attn_part_ = nullptr;
  max_ctx_ = 0;
  used_dyn_ = 0;
}

Error DecoderProgram::charge(uint64_t& pool, uint64_t bytes) {
  const uint64_t used = used_static_ + used_dyn_ + used_pf_;
  if (opts_.budget_bytes != 0 && used + bytes > opts_.budget_bytes)
    return Error::make(ErrorCode::InvalidArgument,
                       "memory budget exceeded: used=" + std::to_string(used) + " need=" +
                           std::to_string(bytes) + " limit=" + std::to_string(opts_.budget_bytes));
  pool += bytes;
  return Error::success();
}

// The load of a weight whose bytes the file does not hold fails as the
// reference's load_or_init_weights does (session.cpp:510-544): an error unless
// weight_init asks for a synthetic fill of the f32 buffer (zeros, ones, or
// element i = i * 0.01 in row-major order); a packed buffer (Path B) has no f32
// values to fill.
Error DecoderProgram::missing_weight(const GgufTensor* t, bool packed, std::vector<float>* fill) {
  const std::string ref = opts_.weight_source + "#" + t->name;
  if (opts_.weight_init == 0) {
    if (!opts_.allow_missing_weights)
      return Error::make(ErrorCode::NotFound, "failed to load required weight '" + t->name + "' from '" + ref +
                                                  "': the file ends before the tensor's data");
    return Error::make(ErrorCode::NotFound, "failed to load weight '" + t->name + "' from '" + ref + "'");
  }
  if (packed) return Error::make(ErrorCode::NotFound, "failed to load packed weight '" + t->name + "'");
  uint64_t n = 1;
  for (auto d : t->ne) n *= d;
  fill->assign(n, 0.0f);
  if (opts_.weight_init == 2) {
    for (auto& v : *fill) v = 1.0f;
  } else if (opts_.weight_init == 3) {
    for (uint64_t i = 0; i < n; ++i) (*fill)[i] = static_cast<float>(i) * 0.01f;
  }
  return Error::success();
}

Error DecoderProgram::upload_f32(const GgufTensor* t, float** out) {
  *out = nullptr;
  if (!t) return Error::success();
  uint64_t n = 1;
  for (auto d : t->ne) n *= d;
  UAII_TRY(charge(used_static_, n * 4));
  std::vector<float> h(n);
  if (!t->data) {
    UAII_TRY(missing_weight(t, false, &h));
  } else if (t->type == T_F32) {
    std::memcpy(h.data(), t->data, n * 4);
  } else if (t->type == T_F16) {
    for (uint64_t i = 0; i < n; ++i) {
      uint16_t v;
      std::memcpy(&v, t->data + 2 * i, 2);
      // exact half -> float (same value as the reference's f16_to_f32)
      const uint32_t sign = (uint32_t)(v & 0x8000u) << 16;
      uint32_t e = (v >> 10) & 31u, m = v & 1023u, bits;
      if (e == 0 && m == 0) bits = sign;
      else if (e == 0) { int sh = 0; while (!(m & 0x400u)) { m <<= 1; ++sh; } bits = sign | ((uint32_t)(113 - sh) << 23) | ((m & 1023u) << 13); }
      else if (e == 31) bits = sign | 0x7f800000u | (m << 13);
      else bits = sign | ((e + 112u) << 23) | (m << 13);
      std::memcpy(&h[i], &bits, 4);
    }
  } else {
    return Error::make(ErrorCode::NotImplemented, "norm/bias tensor " + t->name + " must be F32 or F16");
  }
  void* p = nullptr;
  UAII_HIP(hipMalloc(&p, n * 4));
  allocs_.push_back(p);
  UAII_HIP(hipMemcpy(p, h.data(), n * 4, hipMemcpyHostToDevice));
  *out = static_cast<float*>(p);
  return Error::success();
}

Error DecoderProgram::build(const DecoderSpec& spec, const ProgramOptions& opts) {
  spec_ = spec;
  opts_ = opts;
  UAII_HIP(prepare_gemv());
  UAII_HIP(prepare_attention());
  UAII_HIP(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
  UAII_HIP(hipEventCreate(&ev0_));
  UAII_HIP(hipEventCreate(&ev1_));
  const DecoderSpec& d = spec_;
  if (d.n_layers <= 0) return Error::make(ErrorCode::InvalidArgument, "decoder has no layers");
  if (d.head_dim % 2 || d.head_dim > 256)
    return Error::make(ErrorCode::NotImplemented, "head_dim must be even and <= 256");
  if (d.n_heads % d.n_kv_heads)
    return Error::make(ErrorCode::InvalidArgument, "invalid GQA head grouping");
  if (d.dim % 4 || d.q_dim % 4)
    return Error::make(ErrorCode::InvalidArgument, "model dims must be multiples of 4");

  // Path A values (the reference's f32 weight load) when asked, and for MoE
  // models, whose expert kernel the reference runs on f32 weights only
  // (transformer.cpp:551-554)
  bool moe_model = d.n_experts > 0;
  for (const LayerSpec& s : d.layers) moe_model = moe_model || s.ffn == LayerSpec::kMoE;
  const bool f32_load = opts_.f32_weight_load || moe_model;
  auto up = [&](const GgufTensor* t, DeviceWeight* w) -> Error {
    if (t->cols() <= 0 || t->rows() <= 0)
      return Error::make(ErrorCode::InvalidArgument, "tensor " + t->name + " has no elements");
    if (!t->data) {
      // bytes past the end of the file: the reference's failed load or its fill
      std::vector<float> fill;
      const bool packed = !f32_load && t->type != T_F32 && t->type != T_F16;
      UAII_TRY(missing_weight(t, packed, &fill));
      UAII_TRY(upload_weight(T_F32, reinterpret_cast<const uint8_t*>(fill.data()), t->rows(), t->cols(), stream_, w,
                             f32_load));
      return charge(used_static_, w->bytes);
    }
    // the rows the upload copies must be exactly the bytes the file holds for
    // this tensor (the parser bounded those by the end of the mapping)
    if ((uint64_t)t->rows() * gguf_nbytes(t->type, (uint64_t)t->cols()) != t->nbytes)
      return Error::make(ErrorCode::InvalidArgument, "tensor " + t->name + " shape does not match its bytes");
    UAII_TRY(upload_weight(t->type, t->data, t->rows(), t->cols(), stream_, w, f32_load));
    return charge(used_static_, w->bytes);
  };
  UAII_TRY(up(d.tok_embd, &tok_embd_));
  if (!d.tied) UAII_TRY(up(d.output, &output_));
  UAII_TRY(upload_f32(d.out_norm, &out_norm_));
  for (int64_t li = 0; li < d.n_layers; ++li) {
    const LayerSpec& s = d.layers[(size_t)li];
    auto L = std::make_unique<Layer>();
    if (s.wq->cols() != d.dim || s.wq->rows() != d.q_dim || s.wk->rows() != d.kv_dim ||
        s.wv->rows() != d.kv_dim || s.wo->cols() != d.q_dim || s.wo->rows() != d.dim)
      return Error::make(ErrorCode::InvalidArgument, "attention weight shapes do not match hyperparameters");
    UAII_TRY(up(s.wq, &L->wq));
    UAII_TRY(up(s.wk, &L->wk));
    UAII_TRY(up(s.wv, &L->wv));
    UAII_TRY(up(s.wo, &L->wo));
    UAII_TRY(upload_f32(s.attn_norm, &L->attn_norm));
    UAII_TRY(upload_f32(s.ffn_norm, &L->ffn_norm));
    UAII_TRY(upload_f32(s.bq, &L->bq));
    UAII_TRY(upload_f32(s.bk, &L->bk));
    UAII_TRY(upload_f32(s.bv, &L->bv));
    if (s.ffn == LayerSpec::kSwiGLU) {
      if (s.w_gate->type != s.w_up->type)
        return Error::make(ErrorCode::NotImplemented, "ffn_gate and ffn_up must share a quant type");
      UAII_TRY(up(s.w_gate, &L->gate));
      UAII_TRY(up(s.w_up, &L->up));
      UAII_TRY(up(s.w_down, &L->down));
      hid_max_ = std::max(hid_max_, 2 * s.inter);
    } else if (s.ffn == LayerSpec::kGelu) {
      // dense GELU MLP (gguf.cpp:1156-1170)
      UAII_TRY(up(s.w_up, &L->up));
      UAII_TRY(up(s.w_down, &L->down));
      hid_max_ = std::max(hid_max_, s.inter);
    } else if (s.ffn == LayerSpec::kMoE) {
      // router + expert stacks [E, I, D] / [E, D, I] as 2-D weights of E*I (E*D) rows
      // (gguf.cpp:1076-1106), optional shared expert (:1107-1128)
      const int64_t E = d.n_experts, I = s.inter;
      if (E < 1 || E > 256 || d.top_k < 1 || d.top_k > 8)
        return Error::make(ErrorCode::NotImplemented, "MoE with more than 256 experts or top_k > 8");
      if (s.gate_exps->type != s.up_exps->type)
        return Error::make(ErrorCode::NotImplemented, "ffn_gate_exps and ffn_up_exps must share a quant type");
      if (s.gate_inp->rows() != E || s.gate_inp->cols() != d.dim || s.gate_exps->rows() != E * I ||
          s.up_exps->rows() != E * I || s.down_exps->rows() != E * d.dim || s.down_exps->cols() != I)
        return Error::make(ErrorCode::InvalidArgument, "MoE tensor shapes do not match expert_count");
      UAII_TRY(up(s.gate_inp, &L->gate_inp));
      UAII_TRY(up(s.gate_exps, &L->gate_exps));
      UAII_TRY(up(s.up_exps, &L->up_exps));
      UAII_TRY(up(s.down_exps, &L->down_exps));
      int64_t width = std::min<int64_t>(d.top_k, E) * I;
      if (s.gate_sh && s.up_sh && s.down_sh) {
        if (s.gate_sh->type != s.up_sh->type)
          return Error::make(ErrorCode::NotImplemented, "ffn_gate_shexp and ffn_up_shexp must share a quant type");
        UAII_TRY(up(s.gate_sh, &L->gate_sh));
        UAII_TRY(up(s.up_sh, &L->up_sh));
        UAII_TRY(up(s.down_sh, &L->down_sh));
        L->shared = true;
        L->inter_sh = s.up_sh->rows();
        width += L->inter_sh;
      }
      hid_max_ = std::max(hid_max_, width);
      moe_ = true;
    } else {
      // kNone: resid2 = resid1 (gguf.cpp:1171-1173)
    }
    layers_.push_back(std::move(L));
  }

  // activations and step state
  auto alloc = [&](size_t bytes, void** p) -> Error {
    UAII_TRY(charge(used_static_, std::max<size_t>(bytes, 256)));
    UAII_HIP(hipMalloc(p, std::max<size_t>(bytes, 256)));
    UAII_HIP(hipMemset(*p, 0, std::max<size_t>(bytes, 256)));
    allocs_.push_back(*p);
    return Error::success();
  };
  const size_t D = (size_t)d.dim, Q = (size_t)d.q_dim, V = (size_t)d.vocab, L = (size_t)d.n_layers;
  UAII_TRY(alloc(4 * D, (void**)&x_));
  UAII_TRY(alloc(4 * Q, (void**)&q_));
  UAII_TRY(alloc(4 * Q, (void**)&attn_));
  UAII_TRY(alloc(4 * (size_t)std::max<int64_t>(hid_max_, 1), (void**)&h_));
  if (moe_) {
    UAII_TRY(alloc(4 * (size_t)d.n_experts, (void**)&moe_logits_));
    UAII_TRY(alloc(4 * 8, (void**)&moe_ids_));
    UAII_TRY(alloc(4 * 8, (void**)&moe_w_));
  }
  UAII_TRY(alloc(4 * V, (void**)&logits_));
  UAII_TRY(alloc(4 * V, (void**)&probs_));
  UAII_TRY(alloc(4 * D, (void**)&tap_hidden_));
  UAII_TRY(alloc(4 * D * L, (void**)&tap_r1_));
  UAII_TRY(alloc(4 * D * L, (void**)&tap_r2_));
  UAII_TRY(alloc(4 * D, (void**)&tap_normed_));
  UAII_TRY(alloc(sizeof(StepState), (void**)&state_));
  GemvArgs lm{};  // same plan inputs as the LM-head launch in encode_step
  lm.nseg = 1;
  lm.epi = EPI_LOGITS;
  lm.K = d.dim;
  lm.seg[0].w = d.tied ? tok_embd_.view : output_.view;
  lm.seg[0].rows = d.vocab;
  lm_blocks_ = gemv_grid(lm);
  lm.rtap = tap_r2_;  // the launch after a split-K down takes the raw-tap kernel: its grid too
  lm_blocks_ = std::max(lm_blocks_, gemv_grid(lm));
  const int lm_blocks = lm_blocks_;
  UAII_TRY(alloc(4 * (size_t)lm_blocks, (void**)&lm_part_val_));
  UAII_TRY(alloc(4 * (size_t)lm_blocks, (void**)&lm_part_idx_));
  UAII_HIP(hipStreamSynchronize(stream_));
  int64_t want = opts_.max_context > 0 ? opts_.max_context : d.ctx_len;
  if (want > 0) UAII_TRY(ensure_capacity(want));

  // the matrix-core prompt path: block formats it decodes, dense FFNs, f16 cache
  pf_ok_ = opts_.kv_f16 && pf_attn_supported((int)d.head_dim, (int)d.n_heads, (int)d.n_kv_heads) &&
           d.dim % 64 == 0 && d.q_dim % 64 == 0;
  for (int64_t li = 0; pf_ok_ && li < d.n_layers; ++li) {
    const Layer& L = *layers_[(size_t)li];
    const LayerSpec& ls = d.layers[(size_t)li];
    std::vector<const DeviceWeight*> ws = {&L.wq, &L.wk, &L.wv, &L.wo};
    if (ls.ffn == LayerSpec::kSwiGLU) ws.insert(ws.end(), {&L.gate, &L.up, &L.down});
    if (ls.ffn == LayerSpec::kGelu) ws.insert(ws.end(), {&L.up, &L.down});
    if (ls.ffn == LayerSpec::kMoE) {
      ws.insert(ws.end(), {&L.gate_exps, &L.up_exps, &L.down_exps});
      if (L.shared) {
        ws.insert(ws.end(), {&L.gate_sh, &L.up_sh, &L.down_sh});
        if (L.inter_sh % 64) pf_ok_ = false;
      }
      if (!pf_router_supported(L.gate_inp.view.type)) pf_ok_ = false;
    }
    if (ls.ffn != LayerSpec::kNone && ls.inter % 64) pf_ok_ = false;
    for (const DeviceWeight* w : ws) pf_ok_ = pf_ok_ && pf_supported(w->view.type);
  }
  if (const char* env = std::getenv("UAII_PREFILL")) {
    if (std::string(env) == "0") pf_ok_ = false;
  }
  // Q4_0 GEMMs take their high nibbles in place (PfAct::hi16) where every
  // consumer of a prep is one; UAII_PF_H16=0 keeps the shifted decode
  if (const char* env = std::getenv("UAII_PF_H16")) pf_h16_ = std::string(env) != "0";
  UAII_TRY(alloc(1024, (void**)&ring_pad_));
  {
    // the ring kernel measures faster for the residual-add GEMVs (O, down; the
    // QKV and gate/up GEMVs measured slower on it, their RMSNorm staging waiting
    // behind the first loads, as did the LM head); UAII_RING=0 keeps every
    // projection on gemv.hip
    const char* env = std::getenv("UAII_RING");
    ring_mode_ = env ? std::atoi(env) : 1;
    if (prepare_ring_gemv() != hipSuccess) ring_mode_ = 0;
    (void)hipGetLastError();
  }
  // The projections that add into the residual stream run split along K, each
  // block adding its partial row sums with float atomics: the attention output
  // projection with the merge of the attention's key splits in its launch
  // (attn_out.hip; attention + merge + O 13.6 us against 18.0 us on the 8B
  // decode) and the FFN down projection (splitk_gemv.hip; 9.4 against 12.3 us).
  // The adds land in arrival order; UAII_SPLITK=0 keeps the merge kernel and the
  // whole-row O and down kernels, whose residual is the same bits on every run.
  if (const char* env = std::getenv("UAII_SPLITK")) splitk_ = std::string(env) != "0";
  return Error::success();
}

Error DecoderProgram::ensure_prefill_buffers(int64_t chunk) {
  if (chunk <= pf_chunk_) return Error::success();
  UAII_HIP(hipStreamSynchronize(stream_));
  for (void* p : pf_allocs_) (void)hipFree(p);
  pf_allocs_.clear();
  used_pf_ = 0;
  const DecoderSpec& d = spec_;
  int64_t inter = 1, inter_sh = 0;
  for (const LayerSpec& ls : d.layers) inter = std::max(inter, ls.inter);
  for (const auto& L : layers_) inter_sh = std::max(inter_sh, L->inter_sh);
  const int64_t topk = moe_ ? std::min<int64_t>(d.top_k, d.n_experts) : 1;
  const int64_t mpad = pf_mpad(chunk * topk);  // MoE: the experts' hidden rows
  const int64_t kmax = std::max({d.dim, d.q_dim, inter, inter_sh});
  auto alloc = [&](size_t bytes, void** p) -> Error {
    UAII_TRY(charge(used_pf_, std::max<size_t>(bytes, 256)));
    UAII_HIP(hipMalloc(p, std::max<size_t>(bytes, 256)));
    pf_allocs_.push_back(*p);
    return Error::success();
  };
  const size_t C = (size_t)chunk;
  UAII_TRY(alloc(4 * C * (size_t)d.dim, (void**)&pf_x_));
  UAII_TRY(alloc(4 * C * (size_t)(d.q_dim + 2 * d.kv_dim), (void**)&pf_qkv_));
  UAII_TRY(alloc(4 * C * (size_t)d.q_dim, (void**)&pf_q_));
  UAII_TRY(alloc(4 * C * (size_t)d.q_dim, (void**)&pf_attn_));
  UAII_TRY(alloc(4 * C * (size_t)inter, (void**)&pf_h_));
  // K-split partials: the residual stream's, or the QKV group's
  pf_part_cols_ = std::max(d.dim, d.q_dim + 2 * d.kv_dim);
  UAII_TRY(alloc(4 * 4 * C * (size_t)pf_part_cols_, (void**)&pf_part_));
  if (moe_) {
    const size_t CK = C * (size_t)topk;
    UAII_TRY(alloc(4 * CK, (void**)&pf_moe_ids_));
    UAII_TRY(alloc(4 * CK, (void**)&pf_moe_w_));
    UAII_TRY(alloc(4 * 2 * (size_t)d.n_experts, (void**)&pf_moe_cnt_));  // counts | offsets
    UAII_TRY(alloc(4 * CK, (void**)&pf_moe_list_));
    UAII_TRY(alloc(4 * CK, (void**)&pf_moe_inv_));
    UAII_TRY(alloc(4 * CK * (size_t)d.dim, (void**)&pf_moe_y_));
    // two grouped-GEMM row tables, each at most CK / 32 + E entries of 3
    pf_tab_cap_ = 2 * 3 * ((int64_t)CK / 32 + d.n_experts + 1);
    UAII_TRY(alloc(4 * (size_t)pf_tab_cap_, (void**)&pf_moe_tab_));
    // routed experts' hidden rows [chunk * k][inter]; the shared expert's [chunk][inter_sh]
    (void)hipFree(pf_h_);
    pf_allocs_.erase(std::find(pf_allocs_.begin(), pf_allocs_.end(), (void*)pf_h_));
    UAII_TRY(alloc(4 * CK * (size_t)inter, (void**)&pf_h_));
    if (inter_sh > 0) UAII_TRY(alloc(4 * C * (size_t)inter_sh, (void**)&pf_hsh_));
  }
  UAII_TRY(alloc(2 * (size_t)mpad * (size_t)kmax, (void**)&pf_act_.hi));
  UAII_TRY(alloc(2 * (size_t)mpad * (size_t)kmax, (void**)&pf_act_.lo));
  UAII_TRY(alloc(4 * (size_t)(kmax / 32) * (size_t)mpad, (void**)&pf_act_.sx));
  UAII_TRY(alloc(4 * (size_t)mpad, (void**)&pf_act_.rs));
  pf_act_.mpad = mpad;
  pf_act_rows_ = mpad;
  pf_chunk_ = chunk;
  pf_kmax_ = kmax;
  return Error::success();
}

// One MFMA GEMM launch per run of consecutive weights of the same block format
// (q, k and v may differ, e.g. Q6_K attn_v beside Q4_K attn_q).
Error DecoderProgram::pf_gemm(const DeviceWeight* w[3], const int64_t cols0[3], int nw,
                              const DeviceWeight* w2, int epi, int64_t m, float* y, int64_t ldy,
                              int store_split) {
  for (int i = 0; i < nw;) {
    PfGemmArgs a{};
    a.epi = epi;
    a.M = m;
    a.K = w[i]->view.cols;
    a.mpad = pf_act_.mpad;
    a.ahi = pf_act_.hi;
    a.alo = pf_act_.lo;
    a.sx = pf_act_.sx;
    a.rs = pf_act_.rs;
    a.y = y;
    a.ldy = ldy;
    a.hi16 = pf_act_.hi16;
    int j = i;
    while (j < nw && w[j]->view.type == w[i]->view.type) {
      PfSeg& sg = a.seg[a.nseg++];
      sg.w = w[j]->view;
      if (w2) sg.w2 = w2->view;
      sg.rows = w[j]->view.rows;
      sg.col0 = cols0[j];
      ++j;
    }
    if (cus_ == 0) {
      int dev = 0;
      UAII_HIP(hipGetDevice(&dev));
      UAII_HIP(hipDeviceGetAttribute(&cus_, hipDeviceAttributeMultiprocessorCount, dev));
    }
    // a residual add into the stream of a single-format launch may split K; its
    // partials are added by the next prep of the stream (pf_prep)
    a.ksplit = 1;
    if (epi == EPI_ADD && y == pf_x_ && i == 0 && j == nw && pf_pending_ == 0) {
      a.ksplit = pf_gemm_ksplit(a, cus_);
      a.part = pf_part_;
    }
    // a split store: every launch of the group writes partials with the same split
    if (store_split > 1) {
      a.ksplit = store_split;
      a.part = pf_part_;
    }
    UAII_HIP(launch_pf_gemm(a, stream_));
    if (epi == EPI_ADD && a.ksplit > 1) pf_pending_ = a.ksplit;
    i = j;
  }
  return Error::success();
}

// K split shared by the launches of a plain-store group (QKV): the largest any
// launch of the group asks for, halved until every launch's K range allows it.
int DecoderProgram::pf_store_split(const DeviceWeight* w[3], int nw, int64_t m, int64_t ldy) {
  if (cus_ == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus_, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return 1;
  }
  if ((int64_t)4 * pf_chunk_ * pf_part_cols_ < 4 * m * ldy) return 1;
  int ks = 1;
  int64_t kq = 64;
  for (int i = 0; i < nw;) {
    PfGemmArgs a{};
    a.epi = EPI_STORE;
    a.M = m;
    a.K = w[i]->view.cols;
    a.mpad = pf_act_.mpad;
    int j = i;
    while (j < nw && w[j]->view.type == w[i]->view.type) {
      PfSeg& sg = a.seg[a.nseg++];
      sg.w = w[j]->view;
      sg.rows = w[j]->view.rows;
      ++j;
    }
    const int t = w[i]->view.type;
    if (t == T_Q4_K || t == T_Q6_K) kq = 256;
    ks = std::max(ks, pf_gemm_ksplit(a, cus_));
    i = j;
  }
  const int64_t K = w[0]->view.cols;
  while (ks > 1 && K % (kq * ks) != 0) ks /= 2;
  return ks;
}

Error DecoderProgram::pf_prep(float* x, int64_t K, int64_t m, const float* norm_w, bool hi16) {
  if (pf_mpad(m) > pf_act_rows_ || K > pf_kmax_)
    return Error::make(ErrorCode::Internal, "prefill activation rows exceed their buffer");
  pf_act_.mpad = pf_mpad(m);
  pf_act_.hi16 = hi16 ? 1 : 0;  // the GEMMs that read these rows take the same layout
  PfAct act = pf_act_;
  act.K = K;
  const int pend = (x == pf_x_) ? pf_pending_ : 0;
  UAII_HIP(launch_pf_prep(x, K, m, norm_w, spec_.rms_eps, act, stream_, pend ? pf_part_ : nullptr, pend));
  if (pend) pf_pending_ = 0;
  return Error::success();
}

// MoE FFN over the chunk's rows (transformer.cpp:446-612, shared expert
// gguf.cpp:1107-1128): router + top-k per token, per-expert token lists, one
// gate/up GEMM per expert over its gathered tokens, one prep of all routed
// hidden rows, one down GEMM per expert, then x += w y in slot order and the
// shared expert's down as a residual add.
template <class Prep, class Gemm>
Error DecoderProgram::prefill_moe(const Layer& L, const LayerSpec& ls, int64_t m, Prep&& prep, Gemm&& gemm) {
  const DecoderSpec& d = spec_;
  hipStream_t s = stream_;
  const int E = (int)d.n_experts;
  const int k = (int)std::min<int64_t>(d.top_k, d.n_experts);
  const int64_t I = ls.inter;
  UAII_TRY(prep(pf_x_, d.dim, m, L.ffn_norm));
  UAII_TRY(timed("pf_moe_route", 4.0 * (double)(m * d.dim + E * d.dim), 2.0 * (double)(m * E * d.dim), [&] {
    return launch_pf_moe_route(pf_x_, m, d.dim, L.ffn_norm, d.rms_eps, L.gate_inp.view, E, k, pf_moe_ids_,
                               pf_moe_w_, s);
  }));
  UAII_TRY(timed("pf_moe_route", 0.0, 0.0, [&] {
    return launch_pf_moe_lists(pf_moe_ids_, m, k, E, pf_moe_cnt_, pf_moe_cnt_ + E, pf_moe_list_, pf_moe_inv_, s);
  }));
  std::vector<int32_t> co((size_t)(2 * E));
  UAII_HIP(hipMemcpyAsync(co.data(), pf_moe_cnt_, 8 * (size_t)E, hipMemcpyDeviceToHost, s));
  UAII_HIP(hipStreamSynchronize(s));
  // per-expert row tables of the two grouped launches: {expert, row0, row_end}
  // per grid row, rows in the packed (expert-major) order of the lists
  const int bm_gu = pf_gemm_group_rows(L.gate_exps.view.type);
  const int bm_dn = pf_gemm_group_rows(L.down_exps.view.type);
  std::vector<int32_t>& tab = pf_tab_host_;
  tab.clear();
  int n_used = 0;
  auto add_table = [&](int bm) {
    const int first = (int)(tab.size() / 3);
    for (int e = 0; e < E; ++e) {
      const int32_t c = co[(size_t)e], off = co[(size_t)(E + e)];
      for (int32_t r = 0; r < c; r += bm) {
        tab.push_back(e);
        tab.push_back(off + r);
        tab.push_back(off + c);
      }
    }
    return first;
  };
  for (int e = 0; e < E; ++e) n_used += co[(size_t)e] > 0 ? 1 : 0;
  const int t_gu = add_table(bm_gu);
  const int n_gu = (int)(tab.size() / 3) - t_gu;
  const int t_dn = add_table(bm_dn);
  const int n_dn = (int)(tab.size() / 3) - t_dn;
  if ((int64_t)tab.size() > pf_tab_cap_)
    return Error::make(ErrorCode::Internal, "MoE prefill row table exceeds its buffer");
  UAII_HIP(hipMemcpyAsync(pf_moe_tab_, tab.data(), 4 * tab.size(), hipMemcpyHostToDevice, s));
  auto grouped = [&](int64_t K, int epi, int bm, int t0, int nt) {
    PfGemmArgs g{};
    g.nseg = 1;
    g.epi = epi;
    g.M = m * k;
    g.K = K;
    g.mpad = pf_mpad(m * k);
    g.ahi = pf_act_.hi;
    g.alo = pf_act_.lo;
    g.sx = pf_act_.sx;
    g.rs = pf_act_.rs;
    g.sx_ld = pf_act_.mpad;
    g.gtab = pf_moe_tab_ + 3 * t0;
    g.ntab = nt;
    g.ngroups = E;
    g.gbm = bm;
    return g;
  };
  {
    // gathered token rows x gate / up of their experts -> routed hidden rows
    PfGemmArgs g = grouped(d.dim, EPI_SWIGLU, bm_gu, t_gu, n_gu);
    g.arow = pf_moe_list_;
    g.y = pf_h_;
    g.ldy = I;
    g.seg[0].w = L.gate_exps.view;
    g.seg[0].w2 = L.up_exps.view;
    g.seg[0].rows = I;
    const double bytes = 2.0 * (double)L.gate_exps.bytes * n_used / E;
    UAII_TRY(timed("pf_moe_gate_up", bytes, 4.0 * (double)(m * k * I * d.dim), [&] { return launch_pf_gemm(g, s); }));
  }
  const int64_t c00[3] = {0, 0, 0};
  if (L.shared) {  // the shared expert reads the same normalised rows
    const DeviceWeight* wg[3] = {&L.gate_sh, nullptr, nullptr};
    UAII_TRY(gemm("pf_gemm_shared_gate_up", wg, c00, 1, &L.up_sh, EPI_SWIGLU, m, pf_hsh_, L.inter_sh));
  }
  // the routed tokens' hidden rows, packed by expert
  UAII_TRY(prep(pf_h_, I, m * k, nullptr));
  {
    PfGemmArgs g = grouped(I, EPI_STORE, bm_dn, t_dn, n_dn);
    g.y = pf_moe_y_;
    g.ldy = d.dim;
    g.seg[0].w = L.down_exps.view;
    g.seg[0].rows = d.dim;
    const double bytes = (double)L.down_exps.bytes * n_used / E;
    UAII_TRY(timed("pf_moe_down", bytes, 2.0 * (double)(m * k * I * d.dim), [&] { return launch_pf_gemm(g, s); }));
  }
  UAII_TRY(timed("pf_moe_combine", 4.0 * (double)(m * d.dim * (k + 2)), 0.0, [&] {
    return launch_pf_moe_combine(pf_x_, m, d.dim, k, pf_moe_w_, pf_moe_inv_, pf_moe_y_, s);
  }));
  if (L.shared) {
    UAII_TRY(prep(pf_hsh_, L.inter_sh, m, nullptr));
    const DeviceWeight* wd[3] = {&L.down_sh, nullptr, nullptr};
    UAII_TRY(gemm("pf_gemm_shared_down", wd, c00, 1, nullptr, EPI_ADD, m, pf_x_, d.dim));
  }
  return Error::success();
}

Error DecoderProgram::prefill(int64_t n) {
  if (n <= 0) return Error::success();
  if (!pf_ok_) return Error::make(ErrorCode::NotImplemented, "prefill: model not covered by the matrix-core path");
  if (!kv_) return Error::make(ErrorCode::InvalidArgument, "KvCache not configured");
  const DecoderSpec& d = spec_;
  StepState st{};
  UAII_TRY(read_state(&st));
  const int64_t p0 = st.pos;
  if (p0 + n >= max_ctx_) return Error::make(ErrorCode::InvalidArgument, "prefill exceeds KV capacity");
  // 1024-token chunks: on the 8B prompt 25.1k tok/s against 22.5k for 512 (the
  // gate/up GEMM runs 8 % faster per token at M = 1024; 1536..4096 measured no
  // better); UAII_PREFILL_CHUNK overrides
  int64_t target = 1024;
  if (const char* env = std::getenv("UAII_PREFILL_CHUNK")) target = std::max<int64_t>(16, std::atoll(env));
  const int64_t chunk = std::min(n, target);
  UAII_TRY(ensure_prefill_buffers(chunk));
  hipStream_t s = stream_;
  const size_t layer_kv = (size_t)d.kv_dim * (size_t)max_ctx_ * 2;
  const int64_t ldqkv = d.q_dim + 2 * d.kv_dim;
  prof_used_ = 0;
  auto prep = [&](float* x, int64_t K, int64_t m, const float* norm_w, bool hi16 = false) -> Error {
    Error err = Error::success();
    Error launched = timed("pf_prep", 12.0 * (double)m * (double)K, 0.0, [&]() -> hipError_t {
      err = pf_prep(x, K, m, norm_w, hi16);
      return err.ok() ? hipSuccess : hipErrorInvalidValue;
    });
    if (!err.ok()) return err;
    return launched;
  };
  // algorithmic work of one GEMM launch group: weights once, A (hi + lo), C
  auto gemm_cost = [&](const DeviceWeight* const* w, int nw, int64_t m, int64_t outs, double* bytes,
                       double* flops) {
    *bytes = 0.0;
    *flops = 0.0;
    for (int i = 0; i < nw; ++i) {
      *bytes += (double)w[i]->bytes;
      *flops += 2.0 * (double)m * (double)w[i]->view.rows * (double)w[i]->view.cols;
    }
    *bytes += 4.0 * (double)m * (double)w[0]->view.cols + 4.0 * (double)m * (double)outs;
  };
  auto gemm = [&](const char* name, const DeviceWeight** w, const int64_t* cols0, int nw,
                  const DeviceWeight* w2, int epi, int64_t m, float* y, int64_t ldy,
                  int store_split = 1) -> Error {
    double bytes = 0.0, flops = 0.0;
    gemm_cost(w, nw, m, ldy, &bytes, &flops);
    if (w2) {
      bytes += (double)w2->bytes;
      flops *= 2.0;
    }
    Error err = Error::success();
    Error launched = timed(name, bytes, flops, [&]() -> hipError_t {
      err = pf_gemm(w, cols0, nw, w2, epi, m, y, ldy, store_split);
      return err.ok() ? hipSuccess : hipErrorInvalidValue;
    });
    if (!err.ok()) return err;
    return launched;
  };
  for (int64_t c0 = 0; c0 < n; c0 += chunk) {
    const int64_t m = std::min(chunk, n - c0);
    const int64_t p = p0 + c0;
    UAII_TRY(timed("pf_embed", 4.0 * (double)m * (double)d.dim, 0.0,
                   [&] { return launch_embed_rows(tok_embd_.view, ids_ + p, m, pf_x_, s); }));
    pf_pending_ = 0;  // a new chunk's stream: the last chunk's final partials are moot
    for (int64_t li = 0; li < d.n_layers; ++li) {
      const Layer& L = *layers_[(size_t)li];
      const LayerSpec& ls = d.layers[(size_t)li];
      uint8_t* kbase = static_cast<uint8_t*>(kv_) + (size_t)li * 2 * layer_kv;
      uint8_t* vbase = kbase + layer_kv;
      // each prep's layout: PfAct::hi16 when every GEMM reading it takes it
      auto h16 = [&](const DeviceWeight& w) { return pf_h16_ && pf_hi16_supported(w.view.type); };
      // attention block (gguf.cpp:1000-1060)
      UAII_TRY(prep(pf_x_, d.dim, m, L.attn_norm, h16(L.wq) && h16(L.wk) && h16(L.wv)));
      const DeviceWeight* qkv[3] = {&L.wq, &L.wk, &L.wv};
      const int64_t qkv_cols[3] = {0, d.q_dim, d.q_dim + d.kv_dim};
      const int qkv_split = pf_store_split(qkv, 3, m, ldqkv);
      UAII_TRY(gemm("pf_gemm_qkv", qkv, qkv_cols, 3, nullptr, EPI_STORE, m, pf_qkv_, ldqkv, qkv_split));
      PfQkvArgs qa{};
      qa.part = pf_part_;
      qa.nsplit = qkv_split;
      qa.qkv = pf_qkv_;
      qa.ldq = ldqkv;
      qa.M = m;
      qa.p0 = (int)p;
      qa.q_dim = (int)d.q_dim;
      qa.kv_dim = (int)d.kv_dim;
      qa.head_dim = (int)d.head_dim;
      qa.rope_mode = d.rope_mode;
      qa.rope = rope_;
      qa.bq = L.bq;
      qa.bk = L.bk;
      qa.bv = L.bv;
      qa.qout = pf_q_;
      qa.kcache = kbase;
      qa.vcache = vbase;
      qa.kv_f16 = 1;
      qa.max_seq = max_ctx_;
      UAII_TRY(timed("pf_qkv_rope", 4.0 * (double)m * (double)(ldqkv + d.q_dim + d.kv_dim), 0.0,
                     [&] { return launch_pf_qkv(qa, s); }));
      PfAttnArgs at{};
      at.q = pf_q_;
      at.ldq = d.q_dim;
      at.kcache = kbase;
      at.vcache = vbase;
      at.max_seq = max_ctx_;
      at.n_heads = (int)d.n_heads;
      at.n_kv = (int)d.n_kv_heads;
      at.hd = (int)d.head_dim;
      at.p0 = p;
      at.M = m;
      at.out = pf_attn_;
      at.ldo = d.q_dim;
      // causal (query, key) pairs x heads x (QK + PV) multiply-adds
      const double pairs = (double)m * (double)p + 0.5 * (double)m * (double)(m + 1);
      UAII_TRY(timed("pf_attention", 4.0 * pairs * (double)d.kv_dim, 4.0 * pairs * (double)d.q_dim, [&] {
        return launch_pf_attn(at, s);
      }));
      UAII_TRY(prep(pf_attn_, d.q_dim, m, nullptr, h16(L.wo)));
      const DeviceWeight* wo[3] = {&L.wo, nullptr, nullptr};
      const int64_t c00[3] = {0, 0, 0};
      UAII_TRY(gemm("pf_gemm_o", wo, c00, 1, nullptr, EPI_ADD, m, pf_x_, d.dim));
      // FFN block (gguf.cpp:1130-1173)
      if (ls.ffn == LayerSpec::kSwiGLU || ls.ffn == LayerSpec::kGelu) {
        const bool ffn16 = ls.ffn == LayerSpec::kSwiGLU ? h16(L.gate) && h16(L.up) : h16(L.up);
        UAII_TRY(prep(pf_x_, d.dim, m, L.ffn_norm, ffn16));
        if (ls.ffn == LayerSpec::kSwiGLU) {
          const DeviceWeight* wg[3] = {&L.gate, nullptr, nullptr};
          UAII_TRY(gemm("pf_gemm_gate_up", wg, c00, 1, &L.up, EPI_SWIGLU, m, pf_h_, ls.inter));
        } else {
          const DeviceWeight* wu[3] = {&L.up, nullptr, nullptr};
          UAII_TRY(gemm("pf_gemm_up", wu, c00, 1, nullptr, EPI_GELU, m, pf_h_, ls.inter));
        }
        UAII_TRY(prep(pf_h_, ls.inter, m, nullptr, h16(L.down)));
        const DeviceWeight* wd[3] = {&L.down, nullptr, nullptr};
        UAII_TRY(gemm("pf_gemm_down", wd, c00, 1, nullptr, EPI_ADD, m, pf_x_, d.dim));
      } else if (ls.ffn == LayerSpec::kMoE) {
        UAII_TRY(prefill_moe(L, ls, m, prep, gemm));
      }
    }
  }
  UAII_TRY(collect_timings());
  // the next step feeds ids[p0 + n] at position p0 + n
  UAII_HIP(hipStreamSynchronize(s));
  int32_t tok = 0;
  UAII_HIP(hipMemcpy(&tok, ids_ + p0 + n, 4, hipMemcpyDeviceToHost));
  st.pos = (int32_t)(p0 + n);
  st.token = tok;
  UAII_HIP(hipMemcpy(state_, &st, sizeof(st), hipMemcpyHostToDevice));
  return Error::success();
}

Error DecoderProgram::ensure_capacity(int64_t max_seq) {
  if (max_seq <= max_ctx_ && kv_) return Error::success();
  UAII_HIP(hipStreamSynchronize(stream_));
  free_dynamic();
  const DecoderSpec& d = spec_;
  const size_t elem = opts_.kv_f16 ? 2 : 4;
  kv_bytes_ = (size_t)d.n_layers * 2 * (size_t)d.kv_dim * (size_t)max_seq * elem;
  // slack past the end: the layer kernel fetches whole tiles of keys, masking
  // the ones past the cached length
  const size_t kv_slack = 64 << 10;
  const int hd = (int)d.head_dim;
  attn_splits_ = attention_splits(max_seq);
  const int G = (int)(d.n_heads / d.n_kv_heads);
  const size_t part = (size_t)d.n_kv_heads * attn_splits_ * G * (size_t)(hd + 2);
  UAII_TRY(charge(used_dyn_, kv_bytes_ + kv_slack + sizeof(int32_t) * (size_t)(max_seq + 2) +
                                 sizeof(float2) * (size_t)max_seq * (size_t)(hd / 2) + part * 4));
  UAII_HIP(hipMalloc(&kv_, kv_bytes_ + kv_slack));
  UAII_HIP(hipMemsetAsync(kv_, 0, kv_bytes_ + kv_slack, stream_));
  UAII_HIP(hipMalloc((void**)&ids_, sizeof(int32_t) * (size_t)(max_seq + 2)));
  UAII_HIP(hipMemsetAsync(ids_, 0, sizeof(int32_t) * (size_t)(max_seq + 2), stream_));
  std::vector<float2> tab = rope_table(d.rope_theta, hd, max_seq);
  UAII_HIP(hipMalloc((void**)&rope_, tab.size() * sizeof(float2)));
  UAII_HIP(hipMemcpy(rope_, tab.data(), tab.size() * sizeof(float2), hipMemcpyHostToDevice));
  UAII_HIP(hipMalloc((void**)&attn_part_, part * 4));
  UAII_HIP(hipStreamSynchronize(stream_));
  max_ctx_ = max_seq;
  return Error::success();
}

Error DecoderProgram::arm_sampler(const SamplerParams& prm, const float* r, int64_t n) {
  if (!sampler_supported())
    return Error::make(ErrorCode::NotImplemented, "device sampler: vocabulary above " +
                                                      std::to_string(sample_max_vocab()));
  if (n < 0 || (n > 0 && !r)) return Error::make(ErrorCode::InvalidArgument, "device sampler: draws");
  UAII_HIP(hipStreamSynchronize(stream_));
  if (!samp_ws_) {
    const size_t b = sample_workspace_bytes(spec_.vocab);
    UAII_TRY(charge(used_static_, b));
    UAII_HIP(hipMalloc(&samp_ws_, b));
    allocs_.push_back(samp_ws_);
  }
  if (n > samp_r_cap_) {
    if (samp_r_) (void)hipFree(samp_r_);
    samp_r_ = nullptr;
    samp_r_cap_ = 0;
    UAII_HIP(hipMalloc((void**)&samp_r_, sizeof(float) * (size_t)n));
    samp_r_cap_ = n;
    // the graph holds the old buffer's address
    if (graph_[2]) (void)hipGraphExecDestroy(graph_[2]);
    graph_[2] = nullptr;
  }
  if (n > 0) UAII_HIP(hipMemcpy(samp_r_, r, sizeof(float) * (size_t)n, hipMemcpyHostToDevice));
  if (graph_[2] && !(prm == samp_graph_ && n == samp_n_)) {
    (void)hipGraphExecDestroy(graph_[2]);
    graph_[2] = nullptr;
  }
  samp_ = prm;
  samp_graph_ = prm;
  samp_n_ = n;
  sampler_on_ = true;
  return Error::success();
}

Error DecoderProgram::begin(const int64_t* prompt, int64_t n_prompt) {
  if (n_prompt <= 0) return Error::make(ErrorCode::InvalidArgument, "prompt_tokens empty");
  if (n_prompt > max_ctx_) return Error::make(ErrorCode::InvalidArgument, "prompt exceeds KV capacity");
  std::vector<int32_t> ids((size_t)n_prompt);
  for (int64_t i = 0; i < n_prompt; ++i) {
    if (prompt[i] < 0 || prompt[i] >= tok_embd_.view.rows)
      return Error::make(ErrorCode::InvalidArgument,
                         "embedding token id out of range: " + std::to_string(prompt[i]) +
                             " vocab=" + std::to_string(tok_embd_.view.rows));
    ids[(size_t)i] = (int32_t)prompt[i];
  }
  UAII_HIP(hipStreamSynchronize(stream_));
  UAII_HIP(hipMemcpy(ids_, ids.data(), ids.size() * 4, hipMemcpyHostToDevice));
  StepState st{};
  st.pos = 0;
  st.token = ids[0];
  st.n_prompt = (int32_t)n_prompt;
  st.argmax = 0;
  UAII_HIP(hipMemcpy(state_, &st, sizeof(st), hipMemcpyHostToDevice));
  return Error::success();
}

Error DecoderProgram::set_token(int64_t token) {
  if (token < 0 || token >= tok_embd_.view.rows)
    return Error::make(ErrorCode::InvalidArgument, "embedding token id out of range: " + std::to_string(token));
  const int32_t t = (int32_t)token;
  UAII_HIP(hipStreamSynchronize(stream_));
  UAII_HIP(hipMemcpy(&state_->token, &t, 4, hipMemcpyHostToDevice));
  // the id history holds the token fed at each position
  int32_t pos = 0;
  UAII_HIP(hipMemcpy(&pos, &state_->pos, 4, hipMemcpyDeviceToHost));
  if (pos >= 0 && pos <= max_ctx_) UAII_HIP(hipMemcpy(ids_ + pos, &t, 4, hipMemcpyHostToDevice));
  return Error::success();
}

Error DecoderProgram::seek(int64_t pos) {
  StepState st{};
  UAII_TRY(read_state(&st));
  if (pos <= 0 || pos > st.pos || pos >= max_ctx_)
    return Error::make(ErrorCode::InvalidArgument, "seek position out of range");
  int32_t tok = 0;
  UAII_HIP(hipMemcpy(&tok, ids_ + pos, 4, hipMemcpyDeviceToHost));
  st.pos = (int32_t)pos;
  st.token = tok;
  UAII_HIP(hipMemcpy(state_, &st, sizeof(st), hipMemcpyHostToDevice));
  return Error::success();
}

Error DecoderProgram::read_state(StepState* st) {
  UAII_HIP(hipStreamSynchronize(stream_));
  UAII_HIP(hipMemcpy(st, state_, sizeof(StepState), hipMemcpyDeviceToHost));
  return Error::success();
}

Error DecoderProgram::synchronize() {
  UAII_HIP(hipStreamSynchronize(stream_));
  return Error::success();
}

Error DecoderProgram::read_ids(int64_t* out, int64_t n) {
  if (n > max_ctx_ + 1) return Error::make(ErrorCode::InvalidArgument, "read_ids beyond capacity");
  std::vector<int32_t> ids((size_t)n);
  UAII_HIP(hipStreamSynchronize(stream_));
  UAII_HIP(hipMemcpy(ids.data(), ids_, (size_t)n * 4, hipMemcpyDeviceToHost));
  for (int64_t i = 0; i < n; ++i) out[i] = ids[(size_t)i];
  return Error::success();
}

Error DecoderProgram::read_id(int64_t index, int64_t* id) {
  if (index < 0 || index > max_ctx_) return Error::make(ErrorCode::InvalidArgument, "read_id beyond capacity");
  int32_t v = 0;
  UAII_HIP(hipStreamSynchronize(stream_));
  UAII_HIP(hipMemcpy(&v, ids_ + index, 4, hipMemcpyDeviceToHost));
  *id = v;
  return Error::success();
}

Error DecoderProgram::collect_timings() {
  if (!opts_.profile) return Error::success();
  UAII_HIP(hipStreamSynchronize(stream_));
  for (size_t i = 0; i < prof_used_; ++i) {
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, prof_events_[i].first, prof_events_[i].second) != hipSuccess) {
      (void)hipGetLastError();  // a group that launched nothing records no time
      continue;
    }
    KernelTiming& t = timing_[prof_tags_[i].name];
    t.total_ms += ms;
    t.launches += 1;
    t.bytes += prof_tags_[i].bytes;
    t.flops += prof_tags_[i].flops;
  }
  prof_used_ = 0;
  return Error::success();
}

Error DecoderProgram::encode_step(bool want_logits) {
  const DecoderSpec& d = spec_;
  hipStream_t s = stream_;
  const size_t elem = opts_.kv_f16 ? 2 : 4;
  const size_t layer_kv = (size_t)d.kv_dim * (size_t)max_ctx_ * elem;

  prof_used_ = 0;
  auto timed = [&](const char* name, double bytes, auto&& launch) -> Error {
    return this->timed(name, bytes, 0.0, launch);
  };
  auto collect = [&]() -> Error { return collect_timings(); };

  UAII_TRY(timed("embed", 0.0, [&] { return launch_embed(tok_embd_.view, state_, x_, tap_hidden_, s); }));
  int32_t pos_host = 0;
  if (opts_.profile) {
    UAII_HIP(hipMemcpy(&pos_host, &state_->pos, 4, hipMemcpyDeviceToHost));
  }
  // A residual written by atomic adds has no launch that sees its final value,
  // so its tap (resid2) is written by the next GEMV's input staging.
  float* r2_pending = nullptr;
  for (int64_t li = 0; li < d.n_layers; ++li) {
    const Layer& L = *layers_[(size_t)li];
    const LayerSpec& ls = d.layers[(size_t)li];
    uint8_t* kbase = static_cast<uint8_t*>(kv_) + (size_t)li * 2 * layer_kv;
    uint8_t* vbase = kbase + layer_kv;

    GemvArgs a{};
    a.nseg = 3;
    a.epi = EPI_QKV;
    a.K = d.dim;
    a.x = x_;
    a.norm_w = L.attn_norm;
    a.eps = d.rms_eps;
    a.y = q_;
    a.seg[0].w = L.wq.view; a.seg[0].rows = d.q_dim; a.seg[0].kind = 0; a.seg[0].bias = L.bq;
    a.seg[1].w = L.wk.view; a.seg[1].rows = d.kv_dim; a.seg[1].kind = 1; a.seg[1].bias = L.bk;
    a.seg[2].w = L.wv.view; a.seg[2].rows = d.kv_dim; a.seg[2].kind = 2; a.seg[2].bias = L.bv;
    a.kcache = kbase;
    a.vcache = vbase;
    a.kv_f16 = opts_.kv_f16 ? 1 : 0;
    a.max_seq = max_ctx_;
    a.head_dim = (int)d.head_dim;
    a.rope_mode = d.rope_mode;
    a.rope = rope_;
    a.state = state_;
    a.rtap = r2_pending;
    r2_pending = nullptr;
    const double qkv_bytes = gemv_bytes(L.wq.view) + gemv_bytes(L.wk.view) + gemv_bytes(L.wv.view);
    UAII_TRY(timed("gemv_qkv", qkv_bytes, [&] { return launch_gemv(a, s); }));

    AttnArgs at{};
    at.q = q_;
    at.kcache = kbase;
    at.vcache = vbase;
    at.kv_f16 = opts_.kv_f16 ? 1 : 0;
    at.max_seq = max_ctx_;
    at.n_heads = (int)d.n_heads;
    at.n_kv = (int)d.n_kv_heads;
    at.hd = (int)d.head_dim;
    at.state = state_;
    at.fixed_len = 0;
    at.out = attn_;
    at.part = attn_part_;
    at.splits = attn_splits_;
    const double attn_bytes = 2.0 * (double)(pos_host + 1) * (double)d.kv_dim * (double)elem +
                              8.0 * (double)d.q_dim;
    // merge + O + residual in one launch (FFN layers whose first GEMV records
    // the residual tap resid1 from its input: gate/up, up, the first experts')
    MergeOArgs mo{};
    mo.at = at;
    mo.w = L.wo.view;
    mo.rows = d.dim;
    mo.y = x_;
    const bool fuse_o = splitk_ &&
                        (ls.ffn == LayerSpec::kSwiGLU || ls.ffn == LayerSpec::kGelu || ls.ffn == LayerSpec::kMoE) &&
                        merge_o_supported(mo);
    if (fuse_o) {
      UAII_TRY(timed("attention", attn_bytes, [&] { return launch_attention_splits(at, s); }));
    } else {
      UAII_TRY(timed("attention", attn_bytes, [&] { return launch_attention_decode(at, s); }));
    }

    GemvArgs o{};
    o.nseg = 1;
    o.epi = EPI_ADD;
    o.K = d.q_dim;
    o.x = attn_;
    o.y = x_;
    o.tap = tap_r1_ + li * d.dim;
    o.seg[0].w = L.wo.view;
    o.seg[0].rows = d.dim;
    o.state = state_;
    RingArgs ro{};
    ro.w = L.wo.view;
    ro.rows = d.dim;
    ro.epi = EPI_ADD;
    ro.K = d.q_dim;
    ro.x = attn_;
    ro.y = x_;
    ro.tap = o.tap;
    ro.pad = ring_pad_;
    if (fuse_o) {
      UAII_TRY(timed("gemv_o", gemv_bytes(L.wo.view), [&] { return launch_merge_o(mo, s); }));
    } else if (ring_mode_ >= 1 && ring_gemv_supported(ro)) {
      UAII_TRY(timed("gemv_o", gemv_bytes(L.wo.view), [&] { return launch_ring_gemv(ro, s); }));
    } else {
      UAII_TRY(timed("gemv_o", gemv_bytes(L.wo.view), [&] { return launch_gemv(o, s); }));
    }

    if (ls.ffn == LayerSpec::kSwiGLU) {
      GemvArgs g{};
      g.nseg = 1;
      g.epi = EPI_SWIGLU;
      g.K = d.dim;
      g.x = x_;
      g.norm_w = L.ffn_norm;  // null when the layer has no ffn_norm (gguf.cpp:1055-1062)
      g.eps = d.rms_eps;
      g.y = h_;
      g.seg[0].w = L.gate.view;
      g.seg[0].w2 = L.up.view;
      g.seg[0].rows = 2 * ls.inter;
      g.state = state_;
      if (fuse_o) g.rtap = tap_r1_ + li * d.dim;
      const double gu_bytes = gemv_bytes(L.gate.view) + gemv_bytes(L.up.view);
      UAII_TRY(timed("gemv_gate_up", gu_bytes, [&] { return launch_gemv(g, s); }));
      GemvArgs dn{};
      dn.nseg = 1;
      dn.epi = EPI_ADD;
      dn.K = ls.inter;
      dn.x = h_;
      dn.y = x_;
      dn.tap = tap_r2_ + li * d.dim;
      dn.seg[0].w = L.down.view;
      dn.seg[0].rows = d.dim;
      dn.state = state_;
      RingArgs rd{};
      rd.w = L.down.view;
      rd.rows = d.dim;
      rd.epi = EPI_ADD;
      rd.K = ls.inter;
      rd.x = h_;
      rd.y = x_;
      rd.tap = dn.tap;
      rd.pad = ring_pad_;
      SplitKArgs sk{};
      sk.w = L.down.view;
      sk.rows = d.dim;
      sk.x = h_;
      sk.y = x_;
      if (splitk_ && gemv_splitk_supported(sk)) {
        UAII_TRY(timed("gemv_down", gemv_bytes(L.down.view), [&] { return launch_gemv_splitk(sk, s); }));
        r2_pending = dn.tap;
      } else if (ring_mode_ >= 1 && ring_gemv_supported(rd)) {
        UAII_TRY(timed("gemv_down", gemv_bytes(L.down.view), [&] { return launch_ring_gemv(rd, s); }));
      } else {
        UAII_TRY(timed("gemv_down", gemv_bytes(L.down.view), [&] { return launch_gemv(dn, s); }));
      }
    } else if (ls.ffn == LayerSpec::kGelu) {
      GemvArgs g{};
      g.nseg = 1;
      g.epi = EPI_GELU;
      g.K = d.dim;
      g.x = x_;
      g.norm_w = L.ffn_norm;
      g.eps = d.rms_eps;
      g.y = h_;
      g.seg[0].w = L.up.view;
      g.seg[0].rows = ls.inter;
      g.state = state_;
      if (fuse_o) g.rtap = tap_r1_ + li * d.dim;
      UAII_TRY(timed("gemv_up_gelu", gemv_bytes(L.up.view), [&] { return launch_gemv(g, s); }));
      GemvArgs dn{};
      dn.nseg = 1;
      dn.epi = EPI_ADD;
      dn.K = ls.inter;
      dn.x = h_;
      dn.y = x_;
      dn.tap = tap_r2_ + li * d.dim;
      dn.seg[0].w = L.down.view;
      dn.seg[0].rows = d.dim;
      dn.state = state_;
      SplitKArgs sk{};
      sk.w = L.down.view;
      sk.rows = d.dim;
      sk.x = h_;
      sk.y = x_;
      if (splitk_ && gemv_splitk_supported(sk)) {
        UAII_TRY(timed("gemv_down", gemv_bytes(L.down.view), [&] { return launch_gemv_splitk(sk, s); }));
        r2_pending = dn.tap;
      } else {
        UAII_TRY(timed("gemv_down", gemv_bytes(L.down.view), [&] { return launch_gemv(dn, s); }));
      }
    } else if (ls.ffn == LayerSpec::kMoE) {
      // router logits on the ffn_norm'd input, then softmax / top-k / weights on
      // the device (transformer.cpp:446-481)
      const int64_t E = d.n_experts, I = ls.inter;
      const int k = (int)std::min<int64_t>(d.top_k, E);
      if (L.ffn_norm && pf_router_supported(L.gate_inp.view.type) && E <= 256 && k <= 8 && d.dim % 4 == 0) {
        // one block: RMSNorm, the E router logits and the top-k in one launch
        UAII_TRY(timed("moe_route", gemv_bytes(L.gate_inp.view), [&] {
          return launch_pf_moe_route(x_, 1, d.dim, L.ffn_norm, d.rms_eps, L.gate_inp.view, (int)E, k, moe_ids_,
                                     moe_w_, s);
        }));
      } else {
        GemvArgs r{};
        r.nseg = 1;
        r.epi = EPI_STORE;
        r.K = d.dim;
        r.x = x_;
        r.norm_w = L.ffn_norm;
        r.eps = d.rms_eps;
        r.y = moe_logits_;
        r.seg[0].w = L.gate_inp.view;
        r.seg[0].rows = E;
        r.state = state_;
        UAII_TRY(timed("moe_router", gemv_bytes(L.gate_inp.view), [&] { return launch_gemv(r, s); }));
        UAII_TRY(timed("moe_route", 0.0, [&] { return launch_moe_route(moe_logits_, (int)E, k, moe_ids_, moe_w_, s); }));
      }
      // gate/up of the k chosen experts (+ the shared expert): one segment each,
      // rows of expert moe_ids_[t], outputs at h_[t * I]
      const int nsegs = k + (L.shared ? 1 : 0);
      for (int t0 = 0; t0 < nsegs; t0 += 3) {
        GemvArgs g{};
        g.epi = EPI_SWIGLU;
        g.K = d.dim;
        g.x = x_;
        g.norm_w = L.ffn_norm;
        g.eps = d.rms_eps;
        g.y = h_;
        g.state = state_;
        if (fuse_o && t0 == 0) g.rtap = tap_r1_ + li * d.dim;
        double bytes = 0.0;
        for (int t = t0; t < std::min(nsegs, t0 + 3); ++t) {
          GemvSeg& sg = g.seg[g.nseg++];
          if (t < k) {
            sg.w = L.gate_exps.view;
            sg.w2 = L.up_exps.view;
            sg.rows = 2 * I;
            sg.row_base = (int64_t)t * I;
            sg.expert = moe_ids_ + t;
            sg.expert_rows = I;
            bytes += 2.0 * gemv_bytes(L.gate_exps.view) / (double)E;
          } else {
            sg.w = L.gate_sh.view;
            sg.w2 = L.up_sh.view;
            sg.rows = 2 * L.inter_sh;
            sg.row_base = (int64_t)k * I;
            bytes += gemv_bytes(L.gate_sh.view) + gemv_bytes(L.up_sh.view);
          }
        }
        UAII_TRY(timed("moe_gate_up", bytes, [&] { return launch_gemv(g, s); }));
      }
      // x += w_t * down_{e_t}(h_t) per chosen expert (then + shared down), the
      // residual tap after the last one
      for (int t = 0; t < nsegs; ++t) {
        GemvArgs dn{};
        dn.nseg = 1;
        dn.epi = EPI_ADD;
        dn.y = x_;
        dn.state = state_;
        if (t + 1 < k) {
          // two routed experts in one launch, added in their order
          dn.nseg = 2;
          dn.epi = EPI_ADD2;
          dn.K = I;
          dn.x = h_ + (int64_t)t * I;
          for (int h = 0; h < 2; ++h) {
            GemvSeg& sg = dn.seg[h];
            sg.x = h_ + (int64_t)(t + h) * I;
            sg.w = L.down_exps.view;
            sg.rows = d.dim;
            sg.expert = moe_ids_ + t + h;
            sg.expert_rows = d.dim;
            sg.scale = moe_w_ + t + h;
          }
          if (t + 2 == nsegs) dn.tap = tap_r2_ + li * d.dim;
          const double bytes = 2.0 * gemv_bytes(L.down_exps.view) / (double)E;
          UAII_TRY(timed("moe_down", bytes, [&] { return launch_gemv(dn, s); }));
          ++t;
          continue;
        }
        if (t + 1 == nsegs) dn.tap = tap_r2_ + li * d.dim;
        double bytes;
        if (t < k) {
          dn.K = I;
          dn.x = h_ + (int64_t)t * I;
          dn.seg[0].w = L.down_exps.view;
          dn.seg[0].rows = d.dim;
          dn.seg[0].expert = moe_ids_ + t;
          dn.seg[0].expert_rows = d.dim;
          dn.seg[0].scale = moe_w_ + t;
          bytes = gemv_bytes(L.down_exps.view) / (double)E;
        } else {
          dn.K = L.inter_sh;
          dn.x = h_ + (int64_t)k * I;
          dn.seg[0].w = L.down_sh.view;
          dn.seg[0].rows = d.dim;
          bytes = gemv_bytes(L.down_sh.view);
        }
        UAII_TRY(timed("moe_down", bytes, [&] { return launch_gemv(dn, s); }));
      }
    } else {
      UAII_HIP(hipMemcpyAsync(tap_r2_ + li * d.dim, x_, 4 * (size_t)d.dim, hipMemcpyDeviceToDevice, s));
    }
  }
  if (want_logits && sampler_on_) {
    // the normalised LM head into logits_, then the draw and the token advance
    GemvArgs lm{};
    lm.nseg = 1;
    lm.epi = EPI_STORE;
    lm.K = d.dim;
    lm.x = x_;
    lm.norm_w = out_norm_;
    lm.eps = d.rms_eps;
    lm.y = logits_;
    lm.xtap = tap_normed_;
    lm.rtap = r2_pending;
    lm.seg[0].w = d.tied ? tok_embd_.view : output_.view;
    lm.seg[0].rows = d.vocab;
    UAII_TRY(timed("gemv_lm_head", gemv_bytes(lm.seg[0].w), [&] { return launch_gemv(lm, s); }));
    SampleArgs sa{};
    sa.logits = logits_;
    sa.V = d.vocab;
    sa.inv_t = samp_.inv_t;
    sa.top_p = samp_.top_p;
    sa.top_k = samp_.top_k;
    sa.rep = samp_.rep;
    sa.state = state_;
    sa.ids = ids_;
    sa.rbuf = samp_r_;
    sa.nr = samp_n_;
    sa.ws = samp_ws_;
    UAII_TRY(timed("sample", 0.0, [&] { return launch_sample(sa, s); }));
  } else if (want_logits) {
    GemvArgs lm{};
    lm.nseg = 1;
    lm.epi = EPI_LOGITS;
    lm.K = d.dim;
    lm.x = x_;
    lm.norm_w = out_norm_;
    lm.eps = d.rms_eps;
    lm.y = logits_;
    lm.xtap = tap_normed_;
    lm.rtap = r2_pending;
    lm.seg[0].w = d.tied ? tok_embd_.view : output_.view;
    lm.seg[0].rows = d.vocab;
    lm.part_val = lm_part_val_;
    lm.part_idx = lm_part_idx_;
    lm.part_cap = lm_blocks_;
    lm.ids = ids_;
    lm.state = state_;
    UAII_TRY(timed("gemv_lm_head", gemv_bytes(lm.seg[0].w), [&] { return launch_gemv(lm, s); }));
  } else {
    if (r2_pending) UAII_HIP(hipMemcpyAsync(r2_pending, x_, 4 * (size_t)d.dim, hipMemcpyDeviceToDevice, s));
    UAII_TRY(timed("advance", 0.0, [&] { return launch_advance(state_, ids_, s); }));
  }
  return collect();
}

Error DecoderProgram::step(bool want_logits) {
  if (!kv_) return Error::make(ErrorCode::InvalidArgument, "KvCache not configured");
  if (opts_.profile || !opts_.use_graph) return encode_step(want_logits);
  hipGraphExec_t& ex = graph_[want_logits ? (sampler_on_ ? 2 : 1) : 0];
  if (!ex) {
    hipGraph_t g = nullptr;
    UAII_HIP(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
    Error err = encode_step(want_logits);
    hipError_t st = hipStreamEndCapture(stream_, &g);
    UAII_TRY(err);
    UAII_HIP(st);
    st = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    UAII_HIP(st);
  }
  UAII_HIP(hipGraphLaunch(ex, stream_));
  return Error::success();
}

Error DecoderProgram::read_tap(const std::string& name, std::vector<float>* out) {
  const DecoderSpec& d = spec_;
  const float* src = nullptr;
  size_t n = 0;
  if (name == "hidden") { src = tap_hidden_; n = (size_t)d.dim; }
  else if (name == "normed") { src = tap_normed_; n = (size_t)d.dim; }
  else if (name == "logits") { src = logits_; n = (size_t)d.vocab; }
  else if (name == "probs") {
    UAII_HIP(launch_softmax(logits_, probs_, d.vocab, stream_));
    src = probs_;
    n = (size_t)d.vocab;
  } else if (name.rfind("blk.", 0) == 0) {
    const size_t dot = name.find('.', 4);
    if (dot == std::string::npos) return Error::make(ErrorCode::NotFound, "tensor not found: " + name);
    const int64_t li = std::atoll(name.substr(4, dot - 4).c_str());
    const std::string what = name.substr(dot + 1);
    if (li < 0 || li >= d.n_layers) return Error::make(ErrorCode::NotFound, "tensor not found: " + name);
    if (what == "resid1") src = tap_r1_ + li * d.dim;
    else if (what == "resid2") src = tap_r2_ + li * d.dim;
    else return Error::make(ErrorCode::NotFound, "tensor not found: " + name);
    n = (size_t)d.dim;
  } else {
    return Error::make(ErrorCode::NotFound, "tensor not found: " + name);
  }
  out->resize(n);
  UAII_HIP(hipStreamSynchronize(stream_));
  UAII_HIP(hipMemcpy(out->data(), src, n * 4, hipMemcpyDeviceToHost));
  return Error::success();
}

std::string DecoderProgram::profile_summary() const {
  std::ostringstream os;
  os << "{";
  bool first = true;
  for (const auto& kv : timing_) {
    const KernelTiming& t = kv.second;
    if (!first) os << ",";
    first = false;
    const double avg_us = t.launches ? 1000.0 * t.total_ms / (double)t.launches : 0.0;
    const double gbs = t.total_ms > 0 ? t.bytes / (t.total_ms * 1e-3) / 1e9 : 0.0;
    const double tfs = t.total_ms > 0 ? t.flops / (t.total_ms * 1e-3) / 1e12 : 0.0;
    os << "\"" << kv.first << "\":{\"launches\":" << t.launches << ",\"total_ms\":" << t.total_ms
       << ",\"avg_us\":" << avg_us << ",\"bytes\":" << t.bytes << ",\"gbps\":" << gbs
       << ",\"flops\":" << t.flops << ",\"tflops\":" << tfs << "}";
  }
  os << "}";
  return os.str();
}

}  // namespace uaii
