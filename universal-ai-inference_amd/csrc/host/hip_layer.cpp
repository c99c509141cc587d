// hip_layer.cpp — the extern "C" HIP launch layer declared in include/uaii_hip.h.
#include "uaii_hip.h"

#include "program.h"

#include <cmath>
#include <mutex>
#include <random>
#include <vector>

using namespace uaii_hip;

struct uaii_hip_weight {
  uaii::DeviceWeight w;
};

namespace {

constexpr int kErrArg = -1;      // invalid argument
constexpr int kErrNotImpl = -2;  // not implemented
constexpr int kErrScratch = -3;  // larger than the allocation-free scratch

std::mutex g_scratch_mu;
void* g_scratch = nullptr;       // attention partials for uaii_hip_attention_decode
size_t g_scratch_bytes = 0;

hipStream_t S(void* s) { return static_cast<hipStream_t>(s); }

int grow_scratch(size_t bytes) {
  if (bytes <= g_scratch_bytes) return 0;
  if (g_scratch) {
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return (int)e;
    (void)hipFree(g_scratch);
    g_scratch = nullptr;
    g_scratch_bytes = 0;
  }
  hipError_t e = hipMalloc(&g_scratch, bytes);
  if (e != hipSuccess) return (int)e;
  e = hipMemset(g_scratch, 0, bytes);
  if (e != hipSuccess) return (int)e;
  g_scratch_bytes = bytes;
  return 0;
}

}  // namespace

extern "C" {

int uaii_hip_init(int device) {
  hipError_t e = hipSetDevice(device);
  if (e != hipSuccess) return (int)e;
  e = prepare_gemv();
  if (e != hipSuccess) return (int)e;
  e = prepare_attention();
  if (e != hipSuccess) return (int)e;
  return (int)prepare_noalloc();
}

int uaii_hip_device_count(int* count) {
  if (!count) return kErrArg;
  return (int)hipGetDeviceCount(count);
}

const char* uaii_hip_error_string(int code) {
  if (code == kErrArg) return "invalid argument";
  if (code == kErrNotImpl) return "not implemented";
  if (code == kErrScratch)
    return "the call needs more device scratch than the allocation-free entry point holds";
  return hipGetErrorString(static_cast<hipError_t>(code));
}

int uaii_hip_malloc(void** ptr, size_t bytes) {
  if (!ptr) return kErrArg;
  return (int)hipMalloc(ptr, bytes);
}
int uaii_hip_free(void* ptr) { return (int)hipFree(ptr); }
int uaii_hip_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  return (int)hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice);
}
int uaii_hip_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  return (int)hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost);
}
int uaii_hip_memset(void* ptr, int value, size_t bytes) { return (int)hipMemset(ptr, value, bytes); }
int uaii_hip_synchronize(void) { return (int)hipDeviceSynchronize(); }

int uaii_hip_weight_create(int gguf_type, const void* host_packed, int64_t rows, int64_t cols,
                           uaii_hip_weight** out) {
  if (!host_packed || !out || rows <= 0 || cols <= 0) return kErrArg;
  auto* h = new uaii_hip_weight();
  uaii::Error err = uaii::upload_weight(gguf_type, static_cast<const uint8_t*>(host_packed), rows,
                                        cols, nullptr, &h->w);
  if (!err.ok()) {
    delete h;
    return err.code() == uaii::ErrorCode::NotImplemented ? kErrNotImpl : kErrArg;
  }
  *out = h;
  return 0;
}

int uaii_hip_weight_destroy(uaii_hip_weight* w) {
  delete w;
  return 0;
}

int64_t uaii_hip_weight_bytes(const uaii_hip_weight* w) { return w ? (int64_t)w->w.bytes : 0; }

int uaii_hip_dequant_rows(const uaii_hip_weight* w, int64_t row0, int64_t nrows, float* out,
                          void* stream) {
  if (!w || !out || row0 < 0 || nrows < 0 || row0 + nrows > w->w.view.rows) return kErrArg;
  return (int)launch_dequant(w->w.view, row0, nrows, out, S(stream));
}

static int gemv_common(const uaii_hip_weight* w, const float* x, const float* norm_w, float eps,
                       float* y, void* stream, int epi = EPI_STORE) {
  if (!w || !x || !y) return kErrArg;
  if (w->w.view.cols % 4) return kErrArg;
  GemvArgs a{};
  a.nseg = 1;
  a.epi = epi;
  a.K = w->w.view.cols;
  a.x = x;
  a.norm_w = norm_w;
  a.eps = eps;
  a.y = y;
  a.seg[0].w = w->w.view;
  a.seg[0].rows = w->w.view.rows;
  return (int)launch_gemv(a, S(stream));
}

int uaii_hip_gemv(const uaii_hip_weight* w, const float* x, float* y, void* stream) {
  return gemv_common(w, x, nullptr, 0.0f, y, stream);
}

int uaii_hip_gemv_rmsnorm(const uaii_hip_weight* w, const float* x, const float* norm_w,
                          float eps, float* y, void* stream) {
  if (!norm_w) return kErrArg;
  return gemv_common(w, x, norm_w, eps, y, stream);
}

int uaii_hip_gemv_add(const uaii_hip_weight* w, const float* x, const float* norm_w, float eps,
                      float* y, void* stream) {
  return gemv_common(w, x, norm_w, eps, y, stream, EPI_ADD);
}

int uaii_hip_gemv_swiglu(const uaii_hip_weight* wg, const uaii_hip_weight* wu, const float* x,
                         const float* norm_w, float eps, float* y, void* stream) {
  if (!wg || !wu || !x || !y) return kErrArg;
  const DevWeight& g = wg->w.view;
  const DevWeight& u = wu->w.view;
  if (g.type != u.type || g.rows != u.rows || g.cols != u.cols || g.cols % 4) return kErrArg;
  GemvArgs a{};
  a.nseg = 1;
  a.epi = EPI_SWIGLU;
  a.K = g.cols;
  a.x = x;
  a.norm_w = norm_w;
  a.eps = eps;
  a.y = y;
  a.seg[0].w = g;
  a.seg[0].w2 = u;
  a.seg[0].rows = 2 * g.rows;  // logical rows interleave (gate j, up j)
  return (int)launch_gemv(a, S(stream));
}

}  // extern "C"

namespace {

// M-row products: the MFMA kernel for the block formats it decodes, else one
// GEMV launch per row (same epilogue). Prepared activations live in g_scratch.
int gemm_common(const uaii_hip_weight* w, const uaii_hip_weight* w2, const float* x, int64_t m,
                const float* norm_w, float eps, float* y, int epi, void* stream) {
  if (!w || !x || !y || m <= 0) return kErrArg;
  const DevWeight& v = w->w.view;
  if (epi == EPI_SWIGLU) {
    if (!w2) return kErrArg;
    const DevWeight& u = w2->w.view;
    if (u.type != v.type || u.rows != v.rows || u.cols != v.cols) return kErrArg;
  }
  const int64_t K = v.cols, N = v.rows;
  if (!pf_supported(v.type) || K % 64) {
    for (int64_t i = 0; i < m; ++i) {
      const float* xi = x + i * K;
      float* yi = y + i * N;
      int rc = 0;
      if (epi == EPI_SWIGLU) rc = uaii_hip_gemv_swiglu(w, w2, xi, norm_w, eps, yi, stream);
      else rc = gemv_common(w, xi, norm_w, eps, yi, stream, epi);
      if (rc) return rc;
    }
    return 0;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  const int64_t mpad = pf_mpad(m);
  const size_t hb = (size_t)mpad * (size_t)K * 2, sxb = (size_t)(K / 32) * (size_t)mpad * 4;
  int rc = grow_scratch(2 * hb + sxb + (size_t)mpad * 4);
  if (rc) return rc;
  char* base = static_cast<char*>(g_scratch);
  PfAct act{};
  act.hi = reinterpret_cast<__half*>(base);
  act.lo = reinterpret_cast<__half*>(base + hb);
  act.sx = reinterpret_cast<float*>(base + 2 * hb);
  act.rs = reinterpret_cast<float*>(base + 2 * hb + sxb);
  act.mpad = mpad;
  act.K = K;
  act.hi16 = pf_hi16_supported(v.type) ? 1 : 0;  // this launch is the activations' only consumer
  hipError_t e = launch_pf_prep(const_cast<float*>(x), K, m, norm_w, eps, act, S(stream));
  if (e != hipSuccess) return (int)e;
  PfGemmArgs a{};
  a.nseg = 1;
  a.epi = epi;
  a.M = m;
  a.K = K;
  a.mpad = mpad;
  a.ahi = act.hi;
  a.alo = act.lo;
  a.sx = act.sx;
  a.rs = act.rs;
  a.y = y;
  a.ldy = N;
  a.seg[0].w = v;
  if (w2) a.seg[0].w2 = w2->w.view;
  a.seg[0].rows = N;
  a.seg[0].col0 = 0;
  a.hi16 = act.hi16;
  return (int)launch_pf_gemm(a, S(stream));
}

}  // namespace

extern "C" {

int uaii_hip_gemm(const uaii_hip_weight* w, const float* x, int64_t m, float* y, void* stream) {
  return gemm_common(w, nullptr, x, m, nullptr, 0.0f, y, EPI_STORE, stream);
}

int uaii_hip_gemm_rmsnorm(const uaii_hip_weight* w, const float* x, int64_t m, const float* norm_w,
                          float eps, float* y, void* stream) {
  if (!norm_w) return kErrArg;
  return gemm_common(w, nullptr, x, m, norm_w, eps, y, EPI_STORE, stream);
}

int uaii_hip_gemm_add(const uaii_hip_weight* w, const float* x, int64_t m, const float* norm_w,
                      float eps, float* y, void* stream) {
  return gemm_common(w, nullptr, x, m, norm_w, eps, y, EPI_ADD, stream);
}

int uaii_hip_gemm_swiglu(const uaii_hip_weight* wg, const uaii_hip_weight* wu, const float* x,
                         int64_t m, const float* norm_w, float eps, float* y, void* stream) {
  return gemm_common(wg, wu, x, m, norm_w, eps, y, EPI_SWIGLU, stream);
}

int uaii_hip_attention_prefill(const float* q, const void* kcache, const void* vcache,
                               int64_t max_seq, int n_heads, int n_kv_heads, int head_dim,
                               int64_t p0, int64_t m, float* out, void* stream) {
  if (!q || !kcache || !vcache || !out || m <= 0 || p0 < 0 || p0 + m > max_seq) return kErrArg;
  if (!pf_attn_supported(head_dim, n_heads, n_kv_heads)) return kErrNotImpl;
  PfAttnArgs a{};
  a.q = q;
  a.ldq = (int64_t)n_heads * head_dim;
  a.kcache = kcache;
  a.vcache = vcache;
  a.max_seq = max_seq;
  a.n_heads = n_heads;
  a.n_kv = n_kv_heads;
  a.hd = head_dim;
  a.p0 = p0;
  a.M = m;
  a.out = out;
  a.ldo = a.ldq;
  return (int)launch_pf_attn(a, S(stream));
}

int uaii_hip_rmsnorm(const float* x, const float* w, float* y, int64_t rows, int64_t n, float eps,
                     void* stream) {
  if (!x || !y || rows < 0 || n <= 0) return kErrArg;
  return (int)launch_rmsnorm(x, w, y, rows, n, eps, S(stream));
}

int uaii_hip_softmax(const float* x, float* y, int64_t n, void* stream) {
  if (!x || !y || n <= 0) return kErrArg;
  return (int)launch_softmax(x, y, n, S(stream));
}

int uaii_hip_add(const float* a, const float* b, float* y, int64_t n, void* stream) {
  if (!a || !b || !y || n < 0) return kErrArg;
  return (int)launch_elementwise(0, a, b, y, n, S(stream));
}

int uaii_hip_mul(const float* a, const float* b, float* y, int64_t n, void* stream) {
  if (!a || !b || !y || n < 0) return kErrArg;
  return (int)launch_elementwise(1, a, b, y, n, S(stream));
}

int uaii_hip_silu(const float* x, float* y, int64_t n, void* stream) {
  if (!x || !y || n < 0) return kErrArg;
  return (int)launch_elementwise(2, x, nullptr, y, n, S(stream));
}

int uaii_hip_gelu(const float* x, float* y, int64_t n, void* stream) {
  if (!x || !y || n < 0) return kErrArg;
  return (int)launch_elementwise(3, x, nullptr, y, n, S(stream));
}

int uaii_hip_embed(const uaii_hip_weight* w, const int32_t* ids, int64_t n, float* out, void* stream) {
  if (!w || !ids || !out || n < 0) return kErrArg;
  return (int)launch_embed_rows(w->w.view, ids, n, out, S(stream));
}

int uaii_hip_kv_append(const float* k, const float* v, void* kcache, void* vcache, int64_t rows,
                       int64_t kv_dim, int head_dim, int64_t max_seq, int64_t p0, int kv_f16,
                       void* stream) {
  if (!k || !v || !kcache || !vcache || rows < 0 || head_dim <= 0 || kv_dim <= 0 ||
      kv_dim % head_dim || p0 < 0 || p0 + rows > max_seq)
    return kErrArg;
  return (int)launch_kv_append(k, v, kcache, vcache, rows, kv_dim, head_dim, max_seq, p0, kv_f16 ? 1 : 0,
                               S(stream));
}

int uaii_hip_argmax(const float* x, int64_t n, int32_t* out_idx, void* stream) {
  if (!x || !out_idx || n <= 0) return kErrArg;
  return (int)launch_argmax(x, n, out_idx, S(stream));
}

int64_t uaii_hip_sample_workspace_bytes(int64_t vocab) {
  return (int64_t)sample_workspace_bytes(vocab);
}

int uaii_hip_sample(const float* logits, int64_t vocab, float temperature, float top_p, int top_k,
                    float repetition_penalty, const int32_t* pen, int64_t n_pen, float r, int32_t* out_idx,
                    void* workspace, void* stream) {
  if (!logits || !out_idx || !workspace || vocab <= 0 || vocab > sample_max_vocab() || n_pen < 0 ||
      (n_pen > 0 && !pen) || !(r >= 0.0f && r <= 1.0f))
    return kErrArg;
  SampleArgs a{};
  a.logits = logits;
  a.V = vocab;
  a.inv_t = 1.0f / std::max(temperature, 1e-5f);  // sampling.cpp:63
  a.top_p = top_p;
  a.top_k = top_k;
  a.rep = repetition_penalty;
  a.pen = pen;
  a.n_pen = n_pen;
  a.r_fixed = r;
  a.out = out_idx;
  a.ws = workspace;
  return (int)launch_sample(a, S(stream));
}

int uaii_sample_uniforms(uint64_t seed, int64_t n, float* out) {
  if (n < 0 || (n > 0 && !out)) return kErrArg;
  // the per-token draw of sample_token_f32 (sampling.cpp:111-112) from a seeded
  // mt19937_64 (session.cpp:989-995)
  std::mt19937_64 rng(seed);
  std::uniform_real_distribution<float> dist(0.0f, 1.0f);
  for (int64_t i = 0; i < n; ++i) out[i] = dist(rng);
  return 0;
}

int uaii_hip_rope_table(float theta, int head_dim, int64_t max_pos, float* table_dev) {
  if (!table_dev || head_dim <= 0 || head_dim % 2 || max_pos <= 0) return kErrArg;
  std::vector<float> tab((size_t)max_pos * (size_t)head_dim);
  for (int p = 0; p < head_dim / 2; ++p) {
    // transformer.cpp:195-216: freq = 1/powf(theta, 2p/hd), angle = pos*freq
    const float freq = 1.0f / std::pow(theta, static_cast<float>(2 * p) / static_cast<float>(head_dim));
    for (int64_t pos = 0; pos < max_pos; ++pos) {
      const float ang = static_cast<float>(pos) * freq;
      tab[((size_t)pos * (size_t)(head_dim / 2) + (size_t)p) * 2] = std::cos(ang);
      tab[((size_t)pos * (size_t)(head_dim / 2) + (size_t)p) * 2 + 1] = std::sin(ang);
    }
  }
  return (int)hipMemcpy(table_dev, tab.data(), tab.size() * 4, hipMemcpyHostToDevice);
}

int uaii_hip_rope(float* x, int64_t rows, int64_t dim, int head_dim, int mode,
                  const int32_t* pos_dev, const float* table_dev, void* stream) {
  if (!x || !pos_dev || !table_dev || head_dim <= 0 || head_dim % 2 || dim % head_dim) return kErrArg;
  return (int)launch_rope(x, rows, dim, head_dim, pos_dev, 1,
                          reinterpret_cast<const float2*>(table_dev), mode, S(stream));
}

int uaii_hip_attention_decode(const float* q, const void* kcache, const void* vcache, int kv_f16,
                              int64_t max_seq, int n_heads, int n_kv_heads, int head_dim,
                              int64_t n_keys, float* out, void* stream) {
  if (!q || !kcache || !vcache || !out || n_heads <= 0 || n_kv_heads <= 0 ||
      n_heads % n_kv_heads || head_dim <= 0 || n_keys <= 0 || n_keys > max_seq ||
      max_seq > INT32_MAX)  // key positions are 32-bit in the kernels
    return kErrArg;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  const int splits = uaii_hip::attention_splits(max_seq);
  const int G = n_heads / n_kv_heads;
  const size_t part = (size_t)n_kv_heads * splits * G * (size_t)(head_dim + 2) * 4;
  int rc = grow_scratch(part);
  if (rc) return rc;
  AttnArgs a{};
  a.q = q;
  a.kcache = kcache;
  a.vcache = vcache;
  a.kv_f16 = kv_f16;
  a.max_seq = max_seq;
  a.n_heads = n_heads;
  a.n_kv = n_kv_heads;
  a.hd = head_dim;
  a.state = nullptr;
  a.fixed_len = (int)n_keys;
  a.out = out;
  a.part = static_cast<float*>(g_scratch);
  a.splits = splits;
  return (int)launch_attention_decode(a, S(stream));
}

int uaii_hip_gemv_add_atomic(const uaii_hip_weight* w, const float* x, float* y, void* stream) {
  if (!w || !x || !y) return kErrArg;
  {
    // x is read while other blocks already add into y: the ranges must not overlap
    const uintptr_t x0 = (uintptr_t)x, x1 = x0 + (uintptr_t)w->w.view.cols * sizeof(float);
    const uintptr_t y0 = (uintptr_t)y, y1 = y0 + (uintptr_t)w->w.view.rows * sizeof(float);
    if (x0 < y1 && y0 < x1) return kErrArg;
  }
  SplitKArgs p{};
  p.w = w->w.view;
  p.rows = w->w.view.rows;
  p.x = x;
  p.y = y;
  if (!uaii_hip::gemv_splitk_supported(p)) return kErrArg;
  return (int)launch_gemv_splitk(p, S(stream));
}

int uaii_hip_attention_o(const float* q, const void* kcache, const void* vcache, int kv_f16,
                         int64_t max_seq, int n_heads, int n_kv_heads, int head_dim,
                         int64_t n_keys, const uaii_hip_weight* wo, float* out, float* y,
                         void* stream) {
  if (!q || !kcache || !vcache || !out || !y || !wo || n_heads <= 0 || n_kv_heads <= 0 ||
      n_heads % n_kv_heads || head_dim <= 0 || n_keys <= 0 || n_keys > max_seq ||
      max_seq > INT32_MAX)
    return kErrArg;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  const int splits = uaii_hip::attention_splits(max_seq);
  const int G = n_heads / n_kv_heads;
  MergeOArgs m{};
  AttnArgs& a = m.at;
  a.q = q;
  a.kcache = kcache;
  a.vcache = vcache;
  a.kv_f16 = kv_f16;
  a.max_seq = max_seq;
  a.n_heads = n_heads;
  a.n_kv = n_kv_heads;
  a.hd = head_dim;
  a.state = nullptr;
  a.fixed_len = (int)n_keys;
  a.out = out;
  a.splits = splits;
  m.w = wo->w.view;
  m.rows = wo->w.view.rows;
  m.y = y;
  if (!uaii_hip::merge_o_supported(m)) return kErrArg;
  {
    // blocks write `out` while others already add into y: the ranges must not overlap
    const uintptr_t o0 = (uintptr_t)out, o1 = o0 + (uintptr_t)n_heads * head_dim * sizeof(float);
    const uintptr_t y0 = (uintptr_t)y, y1 = y0 + (uintptr_t)m.rows * sizeof(float);
    if (o0 < y1 && y0 < o1) return kErrArg;
  }
  const size_t part = (size_t)n_kv_heads * splits * G * (size_t)(head_dim + 2) * 4;
  int rc = grow_scratch(part);
  if (rc) return rc;
  a.part = static_cast<float*>(g_scratch);
  const hipError_t st = launch_attention_splits(a, S(stream));
  if (st != hipSuccess) return (int)st;
  return (int)launch_merge_o(m, S(stream));
}

int uaii_hip_time_gemv(const uaii_hip_weight* w, const float* x, float* y, int iters,
                       float* avg_ms) {
  if (!w || !x || !y || iters <= 0 || !avg_ms) return kErrArg;
  hipEvent_t e0, e1;
  (void)hipEventCreate(&e0);
  (void)hipEventCreate(&e1);
  int rc = uaii_hip_gemv(w, x, y, nullptr);  // warm
  (void)hipEventRecord(e0, nullptr);
  for (int i = 0; i < iters && !rc; ++i) rc = uaii_hip_gemv(w, x, y, nullptr);
  (void)hipEventRecord(e1, nullptr);
  (void)hipEventSynchronize(e1);
  float ms = 0.0f;
  (void)hipEventElapsedTime(&ms, e0, e1);
  *avg_ms = ms / (float)iters;
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return rc;
}

int uaii_hip_time_gemv_rotate(const uaii_hip_weight* const* ws, int nw, const float* x, float* y,
                              int iters, float* avg_ms) {
  if (!ws || nw <= 0 || !x || !y || iters <= 0 || !avg_ms) return kErrArg;
  for (int i = 0; i < nw; ++i)
    if (!ws[i]) return kErrArg;
  hipEvent_t e0, e1;
  (void)hipEventCreate(&e0);
  (void)hipEventCreate(&e1);
  int rc = uaii_hip_gemv(ws[0], x, y, nullptr);  // warm
  (void)hipEventRecord(e0, nullptr);
  for (int i = 0; i < iters && !rc; ++i) rc = uaii_hip_gemv(ws[(i + 1) % nw], x, y, nullptr);
  (void)hipEventRecord(e1, nullptr);
  (void)hipEventSynchronize(e1);
  float ms = 0.0f;
  (void)hipEventElapsedTime(&ms, e0, e1);
  *avg_ms = ms / (float)iters;
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return rc;
}

int uaii_hip_time_gemm(const uaii_hip_weight* w, const float* x, int64_t m, float* y, int iters,
                       float* avg_ms) {
  if (!w || !x || !y || iters <= 0 || !avg_ms || m <= 0) return kErrArg;
  hipEvent_t e0, e1;
  (void)hipEventCreate(&e0);
  (void)hipEventCreate(&e1);
  int rc = uaii_hip_gemm(w, x, m, y, nullptr);
  (void)hipEventRecord(e0, nullptr);
  for (int i = 0; i < iters && !rc; ++i) rc = uaii_hip_gemm(w, x, m, y, nullptr);
  (void)hipEventRecord(e1, nullptr);
  (void)hipEventSynchronize(e1);
  float ms = 0.0f;
  (void)hipEventElapsedTime(&ms, e0, e1);
  *avg_ms = ms / (float)iters;
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return rc;
}

int uaii_hip_time_copy(const void* src, void* dst, size_t bytes, int iters, float* avg_ms) {
  if (!src || !dst || iters <= 0 || !avg_ms || bytes % 16) return kErrArg;
  hipEvent_t e0, e1;
  (void)hipEventCreate(&e0);
  (void)hipEventCreate(&e1);
  const int64_t n16 = (int64_t)(bytes / 16);
  int rc = (int)uaii_hip::launch_copy(src, dst, n16, nullptr);
  (void)hipEventRecord(e0, nullptr);
  for (int i = 0; i < iters && !rc; ++i) rc = (int)uaii_hip::launch_copy(src, dst, n16, nullptr);
  (void)hipEventRecord(e1, nullptr);
  (void)hipEventSynchronize(e1);
  float ms = 0.0f;
  (void)hipEventElapsedTime(&ms, e0, e1);
  *avg_ms = ms / (float)iters;
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return rc;
}

int uaii_hip_time_read(const void* const* srcs, int nsrc, size_t bytes, int iters, float* avg_ms) {
  if (!srcs || nsrc <= 0 || iters <= 0 || !avg_ms || bytes % 16 || bytes == 0) return kErrArg;
  for (int i = 0; i < nsrc; ++i)
    if (!srcs[i]) return kErrArg;
  uint32_t* sink = nullptr;
  hipError_t e = hipMalloc(&sink, 16);
  if (e != hipSuccess) return (int)e;
  hipEvent_t e0, e1;
  (void)hipEventCreate(&e0);
  (void)hipEventCreate(&e1);
  const int64_t n16 = (int64_t)(bytes / 16);
  int rc = (int)uaii_hip::launch_read(srcs[0], n16, sink, nullptr);
  (void)hipEventRecord(e0, nullptr);
  for (int i = 0; i < iters && !rc; ++i)
    rc = (int)uaii_hip::launch_read(srcs[(i + 1) % nsrc], n16, sink, nullptr);
  (void)hipEventRecord(e1, nullptr);
  (void)hipEventSynchronize(e1);
  float ms = 0.0f;
  (void)hipEventElapsedTime(&ms, e0, e1);
  *avg_ms = ms / (float)iters;
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  (void)hipFree(sink);
  return rc;
}

}  // extern "C"
