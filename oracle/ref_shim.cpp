// ref_shim.cpp — extern "C" driver around the reference's own CPU kernels.
//
// TEST INFRASTRUCTURE ONLY. Built by `make -C oracle ref` together with the
// reference kernel sources (compiled in place from the reference tree) into
// oracle/_ref/libuaii_ref.so. Tests use it to pin the C oracle, and bench.py may
// time it as the CPU baseline ("kind": "reference"). The product never loads it.
//
// Per-op entry points call the reference functions directly. uref_generate
// re-drives the reference kernels in the order the reference GGUF graph wires
// them (libs/uaii-loaders/src/gguf.cpp:935-1209) with the dispatch decisions of
// libs/uaii-kernels/src/dispatch.cpp:82-237 and the token loop of
// libs/uaii-runtime/src/session.cpp:910-1164. GGUF header parsing for the
// graph wiring is borrowed from the C oracle (uaii_oracle.c), whose own parity is
// tested separately; weights that the reference holds as f32 (norms, biases,
// routers, every weight on Path A) come from the reference's own loader
// (gguf_read_header + gguf_load_tensor_f32, libs/uaii-loaders/src/gguf.cpp).

#include "uaii/kernels/kernels.hpp"
#include "uaii/loaders/gguf.hpp"
#include "uaii/kernels/quant_gemm.hpp"
#include "uaii/quant/gguf_dequant.hpp"
#include "uaii/runtime/kv_cache.hpp"

#include <immintrin.h>
#include "uaii/runtime/sampling.hpp"

extern "C" {
#include "uaii_oracle.h"
}

#include <chrono>
#include <cstdio>
#include <cstring>
#include <memory>
#include <random>
#include <string>
#include <vector>

using namespace uaii;
using kernels::TensorView;

namespace {

thread_local std::string g_err;

bool map_type(int t, quant::QuantFormat* f) {
  switch (t) {
    case 0: *f = quant::QuantFormat::F32; return true;
    case 1: *f = quant::QuantFormat::F16; return true;
    case 2: *f = quant::QuantFormat::Q4_0; return true;
    case 3: *f = quant::QuantFormat::Q4_1; return true;
    case 6: *f = quant::QuantFormat::Q5_0; return true;
    case 7: *f = quant::QuantFormat::Q5_1; return true;
    case 8: *f = quant::QuantFormat::Q8_0; return true;
    case 10: *f = quant::QuantFormat::Q2_K; return true;
    case 11: *f = quant::QuantFormat::Q3_K; return true;
    case 12: *f = quant::QuantFormat::Q4_K; return true;
    case 13: *f = quant::QuantFormat::Q5_K; return true;
    case 14: *f = quant::QuantFormat::Q6_K; return true;
    default: return false;
  }
}

// A tensor plus the shape storage its view points at.
struct Owned {
  std::int64_t shape[3] = {0, 0, 0};
  std::vector<float> f32;
  TensorView view;
};

std::unique_ptr<Owned> f32_tensor(std::vector<std::int64_t> dims) {
  auto t = std::make_unique<Owned>();
  std::size_t n = 1;
  for (std::size_t i = 0; i < dims.size(); ++i) {
    t->shape[i] = dims[i];
    n *= static_cast<std::size_t>(dims[i]);
  }
  t->f32.assign(n, 0.0f);
  t->view.dtype = DType::F32;
  t->view.shape = t->shape;
  t->view.rank = dims.size();
  t->view.data = t->f32.data();
  t->view.nbytes = n * sizeof(float);
  return t;
}

}  // namespace

extern "C" {

const char* uref_last_error(void) { return g_err.c_str(); }

int uref_dequant_row(int type, const std::uint8_t* packed, std::int64_t cols, float* out) {
  quant::QuantFormat f;
  if (!map_type(type, &f)) return -1;
  Error e = quant::dequant_gguf_row(f, packed, cols, out);
  if (!e.ok()) { g_err = e.message(); return -1; }
  return 0;
}

int uref_quant_gemm(int type, const float* A, std::int64_t M, std::int64_t K,
                    const std::uint8_t* B, std::int64_t N, float* C) {
  quant::QuantFormat f;
  if (!map_type(type, &f)) return -1;
  std::int64_t as[2] = {M, K}, bs[2] = {N, K}, cs[2] = {M, N};
  TensorView a, b, c;
  a.dtype = DType::F32; a.shape = as; a.rank = 2; a.data = const_cast<float*>(A);
  a.nbytes = static_cast<std::size_t>(M * K) * 4;
  b.dtype = DType::Unknown; b.shape = bs; b.rank = 2; b.data = const_cast<std::uint8_t*>(B);
  b.quant_format = f; b.quant_rows = N; b.quant_cols = K;
  b.nbytes = quant::packed_nbytes(f, static_cast<std::size_t>(N * K));
  c.dtype = DType::F32; c.shape = cs; c.rank = 2; c.data = C;
  c.nbytes = static_cast<std::size_t>(M * N) * 4;
  Error e = kernels::quant_gemm_f32(a, b, &c, true);
  if (!e.ok()) { g_err = e.message(); return -1; }
  return 0;
}

int uref_rmsnorm(const float* x, const float* w, float* y, std::int64_t n, float eps) {
  auto in = f32_tensor({1, n}), wt = f32_tensor({n}), out = f32_tensor({1, n});
  std::memcpy(in->f32.data(), x, n * 4);
  if (w) std::memcpy(wt->f32.data(), w, n * 4);
  Error e = kernels::rmsnorm_f32(in->view, w ? &wt->view : nullptr, &out->view, eps);
  if (!e.ok()) { g_err = e.message(); return -1; }
  std::memcpy(y, out->f32.data(), n * 4);
  return 0;
}

int uref_rope(float* x, std::int64_t dim, std::int64_t head_dim, float pos, float theta,
              int mode) {
  auto in = f32_tensor({1, dim}), out = f32_tensor({1, dim}), p = f32_tensor({1});
  std::memcpy(in->f32.data(), x, dim * 4);
  p->f32[0] = pos;
  Error e = kernels::rope_f32(in->view, &p->view, &out->view, theta, head_dim, mode);
  if (!e.ok()) { g_err = e.message(); return -1; }
  std::memcpy(x, out->f32.data(), dim * 4);
  return 0;
}

int uref_attention_decode(const float* q, const float* kc, const float* vc, std::int64_t past,
                          const float* kn, const float* vn, float* out, int n_heads,
                          int n_kv_heads, int hd) {
  const std::int64_t qd = static_cast<std::int64_t>(n_heads) * hd;
  const std::int64_t kvd = static_cast<std::int64_t>(n_kv_heads) * hd;
  auto Q = f32_tensor({1, qd}), K = f32_tensor({1, kvd}), V = f32_tensor({1, kvd});
  auto O = f32_tensor({1, qd});
  std::memcpy(Q->f32.data(), q, qd * 4);
  std::memcpy(K->f32.data(), kn, kvd * 4);
  std::memcpy(V->f32.data(), vn, kvd * 4);
  std::unique_ptr<Owned> PK, PV;
  if (past > 0) {
    PK = f32_tensor({1, past, kvd});
    PV = f32_tensor({1, past, kvd});
    std::memcpy(PK->f32.data(), kc, past * kvd * 4);
    std::memcpy(PV->f32.data(), vc, past * kvd * 4);
  }
  Error e = kernels::attention_kv_f32(Q->view, K->view, V->view, &O->view, n_heads, 0.0f, true,
                                      PK ? &PK->view : nullptr, PV ? &PV->view : nullptr,
                                      nullptr, nullptr);
  if (!e.ok()) { g_err = e.message(); return -1; }
  std::memcpy(out, O->f32.data(), qd * 4);
  return 0;
}

int uref_softmax(const float* x, float* y, std::int64_t n) {
  auto in = f32_tensor({1, n}), out = f32_tensor({1, n});
  std::memcpy(in->f32.data(), x, n * 4);
  Error e = kernels::softmax_f32(in->view, &out->view, -1);
  if (!e.ok()) { g_err = e.message(); return -1; }
  std::memcpy(y, out->f32.data(), n * 4);
  return 0;
}

int uref_silu(const float* x, float* y, std::int64_t n) {
  auto in = f32_tensor({1, n}), out = f32_tensor({1, n});
  std::memcpy(in->f32.data(), x, n * 4);
  Error e = kernels::silu_f32(in->view, &out->view);
  if (!e.ok()) { g_err = e.message(); return -1; }
  std::memcpy(y, out->f32.data(), n * 4);
  return 0;
}

std::int64_t uref_argmax(const float* row, std::int64_t n) {
  runtime::SampleParams greedy;
  std::mt19937_64 rng{0};
  std::int64_t tok = -1;
  Error e = runtime::sample_token_f32(row, static_cast<std::size_t>(n), greedy, {}, &rng, &tok);
  if (!e.ok()) { g_err = e.message(); return -1; }
  return tok;
}

// ------------------------------------------------------------------ generate

namespace {

struct Weight {
  std::int64_t shape[3] = {0, 0, 0};
  std::vector<float> f32;
  TensorView view;
  bool present = false;
};

// Path B keeps block-quant weights packed (session.cpp:342-358); Path A and
// non-block types are f32, as the reference's own loader gives them
// (gguf_load_tensor_f32, gguf.cpp:445-556, the load of session.cpp:434-443).
bool bind_weight(orc_model* m, const loaders::GgufFile& gf, const std::string& name,
                 bool f32_always, bool path_a, Weight* w) {
  int type = 0;
  std::int64_t ne[3];
  const std::uint8_t* data = nullptr;
  if (orc_model_tensor(m, name.c_str(), &type, ne, &data) != 0) return false;
  quant::QuantFormat f;
  if (!map_type(type, &f)) { g_err = "unsupported type for " + name; return false; }
  int rank = ne[2] > 1 ? 3 : (ne[1] > 1 || !f32_always ? 2 : 1);
  if (rank == 3) { w->shape[0] = ne[2]; w->shape[1] = ne[1]; w->shape[2] = ne[0]; }
  else if (rank == 2) { w->shape[0] = ne[1]; w->shape[1] = ne[0]; }
  else { w->shape[0] = ne[0]; }
  const std::int64_t rows = ne[1] * ne[2], cols = ne[0];
  w->view.shape = w->shape;
  w->view.rank = static_cast<std::size_t>(rank);
  const bool packed = quant::is_gguf_block_quant(f) && !f32_always && !path_a;
  if (packed) {
    w->view.dtype = DType::Unknown;
    w->view.data = const_cast<std::uint8_t*>(data);
    w->view.quant_format = f;
    w->view.quant_rows = rank == 3 ? 0 : rows;
    w->view.quant_cols = rank == 3 ? 0 : cols;
    w->view.nbytes = quant::packed_nbytes(f, static_cast<std::size_t>(rows * cols));
  } else {
    Shape sh;
    const Error e = loaders::gguf_load_tensor_f32(gf, name, &w->f32, &sh);
    if (!e.ok() || w->f32.size() != static_cast<std::size_t>(rows * cols)) {
      g_err = "gguf_load_tensor_f32 " + name + ": " + e.message();
      return false;
    }
    w->view.dtype = DType::F32;
    w->view.data = w->f32.data();
    w->view.nbytes = w->f32.size() * 4;
  }
  w->present = true;
  return true;
}

Error matmul(const TensorView& x, const Weight& w, TensorView* y) {
  // dispatch.cpp:82-100: packed + transpose_b -> quant_gemm, else f32 matmul
  if (kernels::supports_quant_gemm(w.view.quant_format)) {
    return kernels::quant_gemm_f32(x, w.view, y, true);
  }
  return kernels::matmul_f32(x, w.view, y, false, true);
}

// One GGUF decoder driven through the reference kernels: weights bound Path B
// (Path A for MoE, whose experts only work on f32, transformer.cpp:551-554), a
// reference KvCache, and run() = one Session::run() over the graph order of
// gguf.cpp:935-1209.
constexpr int NW = 19;  // weights per layer bound by RefRunner

// Each value through IEEE binary16 and back, round to nearest even, on the
// CPU's own conversion instructions (F16C, compiled for this function only):
// the fp16 KV cache mirror, independent of the oracle's integer conversion.
__attribute__((target("f16c"))) void round_f16_hw(float* p, std::int64_t n) {
  for (std::int64_t i = 0; i < n; ++i) p[i] = _cvtsh_ss(_cvtss_sh(p[i], _MM_FROUND_TO_NEAREST_INT));
}

struct RefRunner {
  orc_model* m = nullptr;
  std::int64_t L = 0, D = 0, H = 0, HKV = 0, hd = 0, V = 0, E = 0, topk = 0, rope_mode = 0,
               ctx = 0, qd = 0, kvd = 0, ff = 1;
  float theta = 0.f, eps = 0.f;
  bool path_a = false;
  bool kv_f16 = false;  // K (after RoPE) and V rounded to fp16 before attention and the append
  loaders::GgufFile gf;
  Weight emb, onorm, lm;
  std::vector<Weight> W;
  runtime::KvCache kv;
  std::unique_ptr<Owned> tokens, x, n1, res1, q, k, v, qb, kb, vb, qr, kr, att, ao, n2, g, u, ga,
      hid, fo, res2, normed, logits, probs, mp, mt, fi, fin;

  ~RefRunner() {
    kernels::set_active_kv_cache(nullptr);
    if (m) orc_model_close(m);
  }

  Error open(const char* path, int max_layers, std::int64_t kv_max_override,
             std::int64_t total_hint, std::int64_t n_prompt, bool force_path_a = false) {
    m = orc_model_open(path, max_layers);
    if (!m) return Error::make(ErrorCode::NotFound, orc_last_error());
    Error he = loaders::gguf_read_header(path, &gf);
    if (!he.ok()) return he;
    std::int64_t hp[12];
    float fp[2];
    orc_model_hparams(m, hp);
    orc_model_fparams(m, fp);
    L = hp[0]; D = hp[1]; H = hp[2]; HKV = hp[3]; hd = hp[4]; V = hp[5];
    E = hp[7]; topk = hp[8]; rope_mode = hp[9]; ctx = hp[10];
    theta = fp[0]; eps = fp[1];
    path_a = force_path_a || E > 0;
    qd = H * hd; kvd = HKV * hd;
    W.resize(static_cast<std::size_t>(L * NW));
    bind_weight(m, gf, "token_embd.weight", false, path_a, &emb);
    bind_weight(m, gf, "output_norm.weight", true, path_a, &onorm);
    if (!bind_weight(m, gf, "output.weight", false, path_a, &lm)) {
      bind_weight(m, gf, "token_embd.weight", false, path_a, &lm);  // tied (gguf.cpp:813-816)
    }
    // per layer: 0 attn_norm .. 8 ffn_down, 9-12 MoE router/experts, 13-15 q/k/v
    // biases, 16-18 shared expert gate/up/down (gguf.cpp:1107-1128)
    static const char* names[NW] = {"attn_norm", "attn_q", "attn_k", "attn_v", "attn_output",
                                    "ffn_norm", "ffn_gate", "ffn_up", "ffn_down",
                                    "ffn_gate_inp", "ffn_gate_exps", "ffn_up_exps",
                                    "ffn_down_exps", "attn_q.bias", "attn_k.bias",
                                    "attn_v.bias", "ffn_gate_shexp", "ffn_up_shexp",
                                    "ffn_down_shexp"};
    for (std::int64_t li = 0; li < L; ++li) {
      for (int kk = 0; kk < NW; ++kk) {
        std::string nm = "blk." + std::to_string(li) + "." + names[kk];
        if (kk < 13 || kk >= 16) nm += ".weight";
        const bool f32_always = (kk == 0 || kk == 5 || (kk >= 9 && kk < 16));
        bind_weight(m, gf, nm, f32_always, path_a, &W[li * NW + kk]);
      }
    }
    for (std::int64_t li = 0; li < L; ++li) {
      const Weight& up = W[li * NW + 7];
      const Weight& ge = W[li * NW + 10];
      const Weight& ush = W[li * NW + 17];
      if (up.present) ff = std::max<std::int64_t>(ff, up.shape[0]);
      if (ge.present) ff = std::max<std::int64_t>(ff, ge.shape[1]);
      if (ush.present) ff = std::max<std::int64_t>(ff, ush.shape[0]);
    }
    const std::int64_t kv_max =
        kv_max_override > 0 ? kv_max_override
                            : (ctx > 0 ? ctx : std::max<std::int64_t>(total_hint, n_prompt + 1));
    Error e = kv.configure(L, 1, kv_max, kvd, HKV);
    if (!e.ok()) return e;
    kernels::set_active_kv_cache(&kv);
    tokens = f32_tensor({1, 1});
    x = f32_tensor({1, D}); n1 = f32_tensor({1, D}); res1 = f32_tensor({1, D});
    q = f32_tensor({1, qd}); k = f32_tensor({1, kvd}); v = f32_tensor({1, kvd});
    qb = f32_tensor({1, qd}); kb = f32_tensor({1, kvd}); vb = f32_tensor({1, kvd});
    qr = f32_tensor({1, qd}); kr = f32_tensor({1, kvd});
    att = f32_tensor({1, qd}); ao = f32_tensor({1, D}); n2 = f32_tensor({1, D});
    g = f32_tensor({1, ff}); u = f32_tensor({1, ff}); ga = f32_tensor({1, ff});
    hid = f32_tensor({1, ff}); fo = f32_tensor({1, D}); res2 = f32_tensor({1, D});
    normed = f32_tensor({1, D}); logits = f32_tensor({1, V}); probs = f32_tensor({1, V});
    mp = f32_tensor({1, std::max<std::int64_t>(E, 1)}); mt = f32_tensor({1, 1});
    fi = f32_tensor({1, D}); fin = f32_tensor({1, D});
    return Error::success();
  }

  // Session::run() then KvCache::commit_step() (session.cpp:1048-1164).
  Error run(std::int64_t token, float* taps_resid2) {
    tokens->f32[0] = static_cast<float>(token);
    Error err = kernels::embedding_f32(tokens->view, emb.view, &x->view);
    if (!err.ok()) return err;
    std::memcpy(fi->f32.data(), x->f32.data(), D * 4);
    for (std::int64_t li = 0; li < L; ++li) {
      Weight* w = &W[li * NW];
      if (!(err = kernels::rmsnorm_f32(fi->view, &w[0].view, &n1->view, eps)).ok()) return err;
      if (!(err = matmul(n1->view, w[1], &q->view)).ok()) return err;
      if (!(err = matmul(n1->view, w[2], &k->view)).ok()) return err;
      if (!(err = matmul(n1->view, w[3], &v->view)).ok()) return err;
      TensorView qq = q->view, kk = k->view, vv = v->view;
      if (w[13].present) { (void)kernels::add_f32(q->view, w[13].view, &qb->view); qq = qb->view; }
      if (w[14].present) { (void)kernels::add_f32(k->view, w[14].view, &kb->view); kk = kb->view; }
      if (w[15].present) { (void)kernels::add_f32(v->view, w[15].view, &vb->view); vv = vb->view; }
      if (!(err = kernels::rope_f32(qq, nullptr, &qr->view, theta, hd,
                                    static_cast<int>(rope_mode))).ok()) return err;
      if (!(err = kernels::rope_f32(kk, nullptr, &kr->view, theta, hd,
                                    static_cast<int>(rope_mode))).ok()) return err;
      if (kv_f16) {
        // the fp16 cache holds the current token's K and V as every past one's
        round_f16_hw(kr->f32.data(), kvd);
        round_f16_hw(static_cast<float*>(vv.data), kvd);
      }
      // Attention with the active KV cache (dispatch.cpp:219-231)
      TensorView pk = kv.k_view(li), pv = kv.v_view(li);
      err = kernels::attention_kv_f32(qr->view, kr->view, vv, &att->view, static_cast<int>(H), 0.0f,
                                      true, pk.data ? &pk : nullptr, pv.data ? &pv : nullptr,
                                      nullptr, nullptr);
      if (!err.ok()) return err;
      if (!(err = kv.append_layer(li, kr->view, vv)).ok()) return err;
      if (!(err = matmul(att->view, w[4], &ao->view)).ok()) return err;
      if (!(err = kernels::add_f32(fi->view, ao->view, &res1->view)).ok()) return err;
      TensorView min = res1->view;
      if (w[5].present) {
        if (!(err = kernels::rmsnorm_f32(res1->view, &w[5].view, &n2->view, eps)).ok()) return err;
        min = n2->view;
      }
      auto set_width = [&](std::int64_t I) {
        g->shape[1] = u->shape[1] = ga->shape[1] = hid->shape[1] = I;
        g->view.nbytes = u->view.nbytes = ga->view.nbytes = hid->view.nbytes =
            static_cast<std::size_t>(I) * 4;
      };
      if (w[9].present && w[10].present) {
        if (!(err = kernels::moe_router_f32(min, w[9].view, &mp->view, &mt->view)).ok()) return err;
        err = kernels::moe_experts_swiglu_f32(min, w[10].view, w[11].view, w[12].view, mp->view,
                                              &fo->view, static_cast<int>(E), static_cast<int>(topk));
        if (!err.ok()) return err;
        if (w[16].present && w[17].present && w[18].present) {
          // shared expert: silu(min@gate_sh) * (min@up_sh) @ down_sh, added to ff_out
          set_width(w[17].shape[0]);
          if (!(err = matmul(min, w[16], &g->view)).ok()) return err;
          if (!(err = matmul(min, w[17], &u->view)).ok()) return err;
          if (!(err = kernels::silu_f32(g->view, &ga->view)).ok()) return err;
          if (!(err = kernels::mul_f32(ga->view, u->view, &hid->view)).ok()) return err;
          if (!(err = matmul(hid->view, w[18], &ao->view)).ok()) return err;
          if (!(err = kernels::add_f32(fo->view, ao->view, &n1->view)).ok()) return err;
          std::memcpy(fo->f32.data(), n1->f32.data(), D * 4);
        }
      } else if (!w[6].present && w[7].present && w[8].present) {
        // dense GELU MLP (gguf.cpp:1156-1170)
        set_width(w[7].shape[0]);
        if (!(err = matmul(min, w[7], &u->view)).ok()) return err;
        if (!(err = kernels::gelu_f32(u->view, &ga->view)).ok()) return err;
        if (!(err = matmul(ga->view, w[8], &fo->view)).ok()) return err;
      } else {
        const std::int64_t I = w[7].shape[0];
        g->shape[1] = u->shape[1] = ga->shape[1] = hid->shape[1] = I;
        g->view.nbytes = u->view.nbytes = ga->view.nbytes = hid->view.nbytes =
            static_cast<std::size_t>(I) * 4;
        if (!(err = matmul(min, w[6], &g->view)).ok()) return err;
        if (!(err = matmul(min, w[7], &u->view)).ok()) return err;
        if (!(err = kernels::silu_f32(g->view, &ga->view)).ok()) return err;
        if (!(err = kernels::mul_f32(ga->view, u->view, &hid->view)).ok()) return err;
        if (!(err = matmul(hid->view, w[8], &fo->view)).ok()) return err;
      }
      if (!(err = kernels::add_f32(res1->view, fo->view, &res2->view)).ok()) return err;
      std::memcpy(fi->f32.data(), res2->f32.data(), D * 4);
      if (taps_resid2) std::memcpy(taps_resid2 + li * D, res2->f32.data(), D * 4);
    }
    std::memcpy(fin->f32.data(), fi->f32.data(), D * 4);
    TensorView fv = fin->view;
    if (onorm.present) {
      if (!(err = kernels::rmsnorm_f32(fin->view, &onorm.view, &normed->view, eps)).ok()) return err;
      fv = normed->view;
    }
    if (!(err = matmul(fv, lm, &logits->view)).ok()) return err;
    if (!(err = kernels::softmax_f32(logits->view, &probs->view, -1)).ok()) return err;
    kv.commit_step();
    return Error::success();
  }
};

}  // namespace

namespace {

// Generate through the reference kernels with the reference's sampler
// (session.cpp:989-1044): greedy over the probs row when `sp` is greedy, else a
// seeded mt19937_64 over the logits row (want_logits = !sample.greedy(),
// session.cpp:974-978).
int generate_with(const char* path, int max_layers, const std::int64_t* prompt,
                  std::int64_t n_prompt, std::int64_t max_new, const runtime::SampleParams& sp,
                  std::int64_t* out, std::int64_t* out_n, float* taps_logits, float* taps_resid2,
                  bool path_a = false, bool kv_f16 = false) {
  RefRunner R;
  Error err = R.open(path, max_layers, 0, n_prompt + max_new, n_prompt, path_a);
  if (!err.ok()) { g_err = err.message(); return -1; }
  R.kv_f16 = kv_f16;
  std::vector<std::int64_t> hist;
  std::mt19937_64 rng{0};
  if (sp.has_seed) rng.seed(sp.seed);
  for (std::int64_t i = 0; i < n_prompt; ++i) {
    const bool last = max_new <= 1 && i == n_prompt - 1;
    err = R.run(prompt[i], last ? taps_resid2 : nullptr);
    if (!err.ok()) { g_err = err.message(); return -1; }
    hist.push_back(prompt[i]);
  }
  for (std::int64_t t = 0; t < max_new; ++t) {
    std::int64_t next = 0;
    const float* scores = sp.greedy() ? R.probs->f32.data() : R.logits->f32.data();
    err = runtime::sample_token_f32(scores, static_cast<std::size_t>(R.V), sp, hist, &rng, &next);
    if (!err.ok()) { g_err = err.message(); return -1; }
    hist.push_back(next);
    if (t + 1 >= max_new) break;
    err = R.run(next, t + 2 >= max_new ? taps_resid2 : nullptr);
    if (!err.ok()) { g_err = err.message(); return -1; }
  }
  if (taps_logits) std::memcpy(taps_logits, R.logits->f32.data(), R.V * 4);
  for (std::size_t i = 0; i < hist.size(); ++i) out[i] = hist[i];
  *out_n = static_cast<std::int64_t>(hist.size());
  return 0;
}

runtime::SampleParams make_params(float temperature, float top_p, int top_k, float rep,
                                  std::uint64_t seed) {
  runtime::SampleParams sp;
  sp.temperature = temperature;
  sp.top_p = top_p;
  sp.top_k = top_k;
  sp.repetition_penalty = rep;
  sp.seed = seed;
  sp.has_seed = true;
  return sp;
}

}  // namespace

// Greedy generate through the reference kernels. taps_logits (vocab floats) and
// taps_resid2 (n_layers*dim floats) receive the last run()'s values when non-NULL.
int uref_generate(const char* path, int max_layers, const std::int64_t* prompt,
                  std::int64_t n_prompt, std::int64_t max_new, std::int64_t* out,
                  std::int64_t* out_n, float* taps_logits, float* taps_resid2) {
  return generate_with(path, max_layers, prompt, n_prompt, max_new, runtime::SampleParams{}, out,
                       out_n, taps_logits, taps_resid2);
}

// Greedy generate on Path A (every weight f32 from gguf_load_tensor_f32, f32
// GEMM): the reference's route under its default options (session.cpp:259-367).
int uref_generate_path_a(const char* path, int max_layers, const std::int64_t* prompt,
                         std::int64_t n_prompt, std::int64_t max_new, std::int64_t* out,
                         std::int64_t* out_n, float* taps_logits, float* taps_resid2) {
  return generate_with(path, max_layers, prompt, n_prompt, max_new, runtime::SampleParams{}, out,
                       out_n, taps_logits, taps_resid2, true);
}

// Greedy generate through the reference kernels with K and V rounded to fp16
// (hardware conversion) before attention and the cache append: the reference's
// own attention and cache over the values an fp16 KV cache holds.
int uref_generate_kv16(const char* path, int max_layers, const std::int64_t* prompt,
                       std::int64_t n_prompt, std::int64_t max_new, std::int64_t* out,
                       std::int64_t* out_n, float* taps_logits, float* taps_resid2) {
  return generate_with(path, max_layers, prompt, n_prompt, max_new, runtime::SampleParams{}, out,
                       out_n, taps_logits, taps_resid2, false, true);
}

// One whole GGUF tensor through the reference's f32 load (gguf.cpp:445-556).
int uref_load_tensor_f32(const char* path, const char* name, float* out, std::int64_t cap,
                         std::int64_t* out_n) {
  loaders::GgufFile gf;
  Error e = loaders::gguf_read_header(path, &gf);
  std::vector<float> v;
  Shape sh;
  if (e.ok()) e = loaders::gguf_load_tensor_f32(gf, name, &v, &sh);
  if (!e.ok()) { g_err = e.message(); return -1; }
  *out_n = static_cast<std::int64_t>(v.size());
  if (out == nullptr) return 0;
  if (cap < *out_n) { g_err = "capacity"; return -1; }
  std::memcpy(out, v.data(), v.size() * 4);
  return 0;
}

// The same with the reference sampler: temperature / top_p / top_k / repetition
// penalty and a seeded mt19937_64.
int uref_generate_sampled(const char* path, const std::int64_t* prompt, std::int64_t n_prompt,
                          std::int64_t max_new, float temperature, float top_p, int top_k,
                          float rep, std::uint64_t seed, std::int64_t* out, std::int64_t* out_n) {
  return generate_with(path, 0, prompt, n_prompt, max_new,
                       make_params(temperature, top_p, top_k, rep, seed), out, out_n, nullptr,
                       nullptr);
}

// One reference draw (sampling.cpp:22-125) from a fresh mt19937_64(seed).
int uref_sample_token(const float* row, std::int64_t vocab, float temperature, float top_p,
                      int top_k, float rep, std::uint64_t seed, const std::int64_t* penalty,
                      std::int64_t n_penalty, std::int64_t* out) {
  std::vector<std::int64_t> pen(penalty, penalty + n_penalty);
  std::mt19937_64 rng(seed);
  const Error err = runtime::sample_token_f32(row, static_cast<std::size_t>(vocab),
                                              make_params(temperature, top_p, top_k, rep, seed),
                                              pen, &rng, out);
  if (!err.ok()) { g_err = err.message(); return -1; }
  return 0;
}

// CPU baseline window: `n_steps` decode runs at positions start_pos.. through the
// reference kernels, after filling the reference KvCache with start_pos
// deterministic K/V rows (values in [-0.5, 0.5)). Returns the wall seconds of the
// n_steps runs (the fill is not timed), or < 0 on error.
double uref_time_decode_window(const char* path, std::int64_t start_pos, std::int64_t n_steps) {
  RefRunner R;
  Error err = R.open(path, 0, start_pos + n_steps + 1, 0, 1);
  if (!err.ok()) { g_err = err.message(); return -1.0; }
  auto kt = f32_tensor({1, R.kvd}), vt = f32_tensor({1, R.kvd});
  for (std::int64_t p = 0; p < start_pos; ++p) {
    for (std::int64_t li = 0; li < R.L; ++li) {
      for (std::int64_t j = 0; j < R.kvd; ++j) {
        const std::uint32_t h = static_cast<std::uint32_t>((p * R.kvd + j) * 2654435761u + li * 40503u);
        kt->f32[j] = static_cast<float>(h & 0xffff) / 65536.0f - 0.5f;
        vt->f32[j] = static_cast<float>((h >> 16) & 0xffff) / 65536.0f - 0.5f;
      }
      err = R.kv.append_layer(li, kt->view, vt->view);
      if (!err.ok()) { g_err = err.message(); return -1.0; }
    }
    R.kv.commit_step();
  }
  const auto t0 = std::chrono::steady_clock::now();
  std::int64_t tok = 1;
  for (std::int64_t i = 0; i < n_steps; ++i) {
    err = R.run(tok, nullptr);
    if (!err.ok()) { g_err = err.message(); return -1.0; }
    runtime::SampleParams greedy;
    std::mt19937_64 rng{0};
    (void)runtime::sample_token_f32(R.probs->f32.data(), static_cast<std::size_t>(R.V), greedy, {},
                                    &rng, &tok);
  }
  const auto t1 = std::chrono::steady_clock::now();
  return std::chrono::duration<double>(t1 - t0).count();
}

// CPU baseline window (i): the first n prompt tokens fed one at a time through
// the reference kernels from an empty cache, as the reference prefills
// (session.cpp:1006-1016: one run() per prompt token). Returns the wall seconds
// of the n runs, or < 0 on error. report_every > 0 prints progress to stderr.
double uref_time_prompt_window(const char* path, const std::int64_t* prompt, std::int64_t n,
                               int report_every) {
  RefRunner R;
  Error err = R.open(path, 0, n + 1, 0, n);
  if (!err.ok()) { g_err = err.message(); return -1.0; }
  const auto t0 = std::chrono::steady_clock::now();
  for (std::int64_t i = 0; i < n; ++i) {
    err = R.run(prompt[i], nullptr);
    if (!err.ok()) { g_err = err.message(); return -1.0; }
    if (report_every > 0 && (i + 1) % report_every == 0) {
      const double s = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
      std::fprintf(stderr, "cpu prompt window: %lld/%lld tokens, %.1f s\n", (long long)(i + 1),
                   (long long)n, s);
      std::fflush(stderr);
    }
  }
  const auto t1 = std::chrono::steady_clock::now();
  return std::chrono::duration<double>(t1 - t0).count();
}

}  // extern "C"
