/*
 * uaii_hip.h — extern "C" HIP launch layer of libuaii_amd.so (gfx950).
 *
 * Plain pointers and sizes only. Device pointers come from uaii_hip_malloc (or
 * any hipMalloc'd memory of the same process); `stream` is a hipStream_t or
 * NULL for the null stream. Every call returns 0 on success or a hipError_t /
 * negative validation code (see uaii_hip_error_string).
 *
 * Entry point -> reference interface it replaces:
 *   uaii_hip_weight_create     gguf_load_tensor_raw (libs/uaii-loaders/src/gguf.cpp:558-602)
 *                              + Session packed weight buffers (session.cpp:342-358):
 *                              GGUF block rows uploaded and re-laid out for HBM once
 *   uaii_hip_dequant_rows      dequant_gguf_row (libs/uaii-quant/src/gguf_dequant.cpp:420-439)
 *   uaii_hip_gemv              quant_gemm_f32 at M=1 (libs/uaii-kernels/src/quant_gemm.cpp:22-70)
 *   uaii_hip_gemv_rmsnorm      rmsnorm_f32 (norm.cpp:89-130) feeding quant_gemm_f32
 *   uaii_hip_gemm              quant_gemm_f32 at M>1 (prefill; same file)
 *   uaii_hip_add / _mul /      add_f32, mul_f32, silu_f32, gelu_f32
 *   _silu / _gelu              (libs/uaii-kernels/src/elementwise.cpp:56-110)
 *   uaii_hip_embed             embedding_f32 (libs/uaii-kernels/src/transformer.cpp:61-142)
 *   uaii_hip_kv_append         KvCache::append_layer (include/uaii/runtime/kv_cache.hpp:80-120)
 *   uaii_hip_rmsnorm           rmsnorm_f32 (libs/uaii-kernels/src/norm.cpp:89-130)
 *   uaii_hip_softmax           softmax_f32 (libs/uaii-kernels/src/softmax.cpp:11-77)
 *   uaii_hip_argmax            greedy sample_token_f32 (libs/uaii-runtime/src/sampling.cpp:38-50)
 *   uaii_hip_sample            non-greedy sample_token_f32 (sampling.cpp:53-125) on the device
 *   uaii_hip_rope              rope_f32 (libs/uaii-kernels/src/transformer.cpp:144-220)
 *   uaii_hip_attention_decode  attention_kv_f32, q_seq=1 (transformer.cpp:222-433)
 *   uaii_hip_attention_o       attention_kv_f32 + quant_gemm_f32 of the attention
 *                              output + residual add_f32 (quant_gemm.cpp:22-70,
 *                              elementwise.cpp:99-110), the decode layer's attention half
 *   uaii_hip_gemv_add          quant_gemm_f32 + residual add_f32 (elementwise.cpp:86-97)
 *   uaii_hip_gemv_add_atomic   the same, split along K with float-atomic adds (Q4_0, Q6_K)
 *   uaii_hip_gemv_swiglu       two quant_gemm_f32 + silu_f32 * mul_f32
 *                              (elementwise.cpp:73-110), the graph's FFN gate/up
 *   uaii_hip_gemm_rmsnorm/_add/_swiglu  the same three at M>1 (prefill)
 *   uaii_hip_attention_prefill attention_kv_f32 for a run of prompt positions
 *                              (the reference feeds them one per step)
 * and the reference ROCm stub's launchers it supersedes
 * (libs/uaii-backends/src/rocm_kernels.hpp:10-14: launch_add_f32, launch_rmsnorm_f32).
 */
#ifndef UAII_HIP_H_
#define UAII_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define UAII_HIP_API __attribute__((visibility("default")))

typedef struct uaii_hip_weight uaii_hip_weight;

/* ---- device and memory ---------------------------------------------------- */
UAII_HIP_API int uaii_hip_init(int device);
UAII_HIP_API int uaii_hip_device_count(int* count);
UAII_HIP_API const char* uaii_hip_error_string(int code);
UAII_HIP_API int uaii_hip_malloc(void** ptr, size_t bytes);
UAII_HIP_API int uaii_hip_free(void* ptr);
UAII_HIP_API int uaii_hip_memcpy_h2d(void* dst, const void* src, size_t bytes);
UAII_HIP_API int uaii_hip_memcpy_d2h(void* dst, const void* src, size_t bytes);
UAII_HIP_API int uaii_hip_memset(void* ptr, int value, size_t bytes);
UAII_HIP_API int uaii_hip_synchronize(void);

/* ---- weights ---------------------------------------------------------------- */
/* gguf_type: GGUF tensor type id (0 F32, 1 F16, 2 Q4_0, 3 Q4_1, 6 Q5_0, 7 Q5_1,
 * 8 Q8_0, 10 Q2_K, 11 Q3_K, 12 Q4_K, 13 Q5_K, 14 Q6_K); host_packed holds `rows`
 * GGUF rows of `cols` values. */
UAII_HIP_API int uaii_hip_weight_create(int gguf_type, const void* host_packed, int64_t rows,
                                        int64_t cols, uaii_hip_weight** out);
UAII_HIP_API int uaii_hip_weight_destroy(uaii_hip_weight* w);
UAII_HIP_API int64_t uaii_hip_weight_bytes(const uaii_hip_weight* w);

/* ---- kernels ---------------------------------------------------------------- */
UAII_HIP_API int uaii_hip_dequant_rows(const uaii_hip_weight* w, int64_t row0, int64_t nrows,
                                       float* out, void* stream);
UAII_HIP_API int uaii_hip_gemv(const uaii_hip_weight* w, const float* x, float* y,
                               void* stream);
UAII_HIP_API int uaii_hip_gemv_rmsnorm(const uaii_hip_weight* w, const float* x,
                                       const float* norm_w, float eps, float* y, void* stream);
/* y[i] += (W . x')[i], x' = x or RMSNorm(x) * norm_w when norm_w is non-NULL. */
UAII_HIP_API int uaii_hip_gemv_add(const uaii_hip_weight* w, const float* x,
                                   const float* norm_w, float eps, float* y, void* stream);
/* y[j] = silu((Wg . x')[j]) * (Wu . x')[j]; wg and wu share type and shape. */
UAII_HIP_API int uaii_hip_gemv_swiglu(const uaii_hip_weight* wg, const uaii_hip_weight* wu,
                                      const float* x, const float* norm_w, float eps, float* y,
                                      void* stream);
/* M > 1: y[i][:] = W . x[i][:] for i < m (x [m][cols], y [m][rows]). Q4_0, Q8_0,
 * Q4_K and Q6_K run on the matrix cores (weights decoded to their exact small
 * integers, x split into f16 hi + lo, block scales applied to the f32 partials);
 * other formats run one GEMV per row. Q4_0 and Q8_0 need m (rounded up to 64)
 * * cols * 2 < 2^31 (their kernels address the f16 activation rows by 32-bit
 * byte offsets); larger calls return hipErrorInvalidValue. */
UAII_HIP_API int uaii_hip_gemm(const uaii_hip_weight* w, const float* x, int64_t m, float* y,
                               void* stream);
UAII_HIP_API int uaii_hip_gemm_rmsnorm(const uaii_hip_weight* w, const float* x, int64_t m,
                                       const float* norm_w, float eps, float* y, void* stream);
/* y[i][:] += W . x'[i][:], x' = x or RMSNorm(x) * norm_w when norm_w is non-NULL. */
UAII_HIP_API int uaii_hip_gemm_add(const uaii_hip_weight* w, const float* x, int64_t m,
                                   const float* norm_w, float eps, float* y, void* stream);
/* y[i][j] = silu((Wg . x'[i])[j]) * (Wu . x'[i])[j], y [m][rows]. */
UAII_HIP_API int uaii_hip_gemm_swiglu(const uaii_hip_weight* wg, const uaii_hip_weight* wu,
                                      const float* x, int64_t m, const float* norm_w, float eps,
                                      float* y, void* stream);
UAII_HIP_API int uaii_hip_rmsnorm(const float* x, const float* w, float* y, int64_t rows,
                                  int64_t n, float eps, void* stream);
UAII_HIP_API int uaii_hip_softmax(const float* x, float* y, int64_t n, void* stream);
/* Elementwise f32 over n values (y may alias an input): add_f32, mul_f32,
 * silu_f32, gelu_f32 (libs/uaii-kernels/src/elementwise.cpp:56-110). */
UAII_HIP_API int uaii_hip_add(const float* a, const float* b, float* y, int64_t n, void* stream);
UAII_HIP_API int uaii_hip_mul(const float* a, const float* b, float* y, int64_t n, void* stream);
UAII_HIP_API int uaii_hip_silu(const float* x, float* y, int64_t n, void* stream);
UAII_HIP_API int uaii_hip_gelu(const float* x, float* y, int64_t n, void* stream);
/* Embedding rows (embedding_f32, libs/uaii-kernels/src/transformer.cpp:61-142):
 * out[i][:] = dequantized row ids[i] of w; ids are device int32, in range. */
UAII_HIP_API int uaii_hip_embed(const uaii_hip_weight* w, const int32_t* ids, int64_t n, float* out,
                                void* stream);
/* K and V rows ([rows][kv_dim] f32) into the head-major caches of
 * uaii_hip_attention_decode at positions p0 .. p0 + rows - 1, as f16 (kv_f16 = 1)
 * or f32 (KvCache::append_layer, include/uaii/runtime/kv_cache.hpp:80-120). */
UAII_HIP_API int uaii_hip_kv_append(const float* k, const float* v, void* kcache, void* vcache,
                                    int64_t rows, int64_t kv_dim, int head_dim, int64_t max_seq,
                                    int64_t p0, int kv_f16, void* stream);
UAII_HIP_API int uaii_hip_argmax(const float* x, int64_t n, int32_t* out_idx, void* stream);
/* Device sampling: one draw of sample_token_f32's non-greedy path
 * (libs/uaii-runtime/src/sampling.cpp:53-125) from a device logits row of
 * `vocab` floats (at most 262144), with the reference's temperature, top_p,
 * top_k and repetition penalty over the `n_pen` device ids `pen`, and the draw
 * `r` in [0, 1] that the reference takes from its generator (uaii_sample_uniforms
 * gives the same sequence). The reference samples on the host; this entry has no
 * counterpart there and serves token loops that keep the logits on the device.
 * workspace: device memory of uaii_hip_sample_workspace_bytes(vocab) bytes,
 * 256-byte aligned; calls sharing one workspace must not overlap. The id is
 * written to the device int32 at out_idx. */
UAII_HIP_API int64_t uaii_hip_sample_workspace_bytes(int64_t vocab);
UAII_HIP_API int uaii_hip_sample(const float* logits, int64_t vocab, float temperature, float top_p,
                                 int top_k, float repetition_penalty, const int32_t* pen,
                                 int64_t n_pen, float r, int32_t* out_idx, void* workspace,
                                 void* stream);
/* Host: n draws of std::uniform_real_distribution<float>(0, 1) from
 * std::mt19937_64(seed), the per-token draws of sample_token_f32
 * (sampling.cpp:111-112) in order. */
UAII_HIP_API int uaii_sample_uniforms(uint64_t seed, int64_t n, float* out);
/* table: [max_pos][head_dim/2] (cos, sin) float pairs, filled on the host with
 * the reference's angle formula, uploaded to `table_dev`. */
UAII_HIP_API int uaii_hip_rope_table(float theta, int head_dim, int64_t max_pos,
                                     float* table_dev);
UAII_HIP_API int uaii_hip_rope(float* x, int64_t rows, int64_t dim, int head_dim, int mode,
                               const int32_t* pos_dev, const float* table_dev, void* stream);
/* kcache/vcache: head-major [n_kv_heads][max_seq][head_dim], f16 (kv_f16=1) or f32;
 * attends over keys 0..n_keys-1. The split partials go to one device buffer the
 * library owns (grown on demand, kept until the process ends; growing it waits
 * for the device), shared with uaii_hip_attention_o: calls that run at the same
 * time on different streams race on it, so issue them on one stream. */
UAII_HIP_API int uaii_hip_attention_decode(const float* q, const void* kcache,
                                           const void* vcache, int kv_f16, int64_t max_seq,
                                           int n_heads, int n_kv_heads, int head_dim,
                                           int64_t n_keys, float* out, void* stream);

/* y += W . x for Q4_0 or Q6_K W [rows][cols], split along K: each block multiplies a
 * 1024-column slice of W by the matching inputs and adds its row sums into y
 * with float atomics, so y's rows take cols / 1024 adds in an order the
 * hardware picks (runs can differ in their last bits). cols a multiple of
 * 1024, rows a multiple of 16; other shapes or types return -1 and launch
 * nothing. x and y must not overlap: blocks still reading x run beside blocks
 * already adding into y. */
UAII_HIP_API int uaii_hip_gemv_add_atomic(const uaii_hip_weight* w, const float* x, float* y,
                                          void* stream);

/* uaii_hip_attention_decode, then y += W_o . out (residual add), in two
 * launches: the key-split kernel, then one launch that merges the splits of
 * 256 / head_dim heads per block, writes them to `out` and adds its share of
 * the W_o product into y with float atomics. out is the same bits as
 * uaii_hip_attention_decode's; each y row is a sum whose adds arrive in an
 * order the hardware picks, so runs can differ in its last bits. W_o: Q4_0,
 * Q8_0 or Q4_K, [rows][n_heads * head_dim] with n_heads * head_dim a multiple of 256,
 * head_dim 64 or 128, rows (y's length) a multiple of 32; other shapes return
 * -1 and launch nothing, as do `out` and y overlapping (merge blocks write
 * `out` while others add into y). Its split partials share uaii_hip_attention_decode's
 * library-owned buffer (the same one-stream rule applies). */
UAII_HIP_API int uaii_hip_attention_o(const float* q, const void* kcache, const void* vcache,
                                      int kv_f16, int64_t max_seq, int n_heads,
                                      int n_kv_heads, int head_dim, int64_t n_keys,
                                      const uaii_hip_weight* wo, float* out, float* y,
                                      void* stream);

/* uaii_hip_attention_decode without any allocation. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * stream capture, allocation-free serving loops). Same arguments, kernels and
 * results as uaii_hip_attention_decode; the split partials live in a fixed
 * 2 MiB device array per GPU (held until the process ends) instead of a
 * hipMalloc'd buffer, so n_kv_heads * splits * (n_heads / n_kv_heads) *
 * (head_dim + 2) * 4 bytes must fit in 2 MiB (splits = min(32, ceil(max_seq /
 * 128))); larger calls return -3 and launch nothing. Calls that overlap on one
 * GPU share that array and race. */
UAII_HIP_API int uaii_hip_attention_decode_noalloc(const float* q, const void* kcache,
                                                   const void* vcache, int kv_f16,
                                                   int64_t max_seq, int n_heads, int n_kv_heads,
                                                   int head_dim, int64_t n_keys, float* out,
                                                   void* stream);

/* Causal attention of m queries at positions p0 .. p0 + m - 1 (q, out:
 * [m][n_heads * head_dim]) over an f16 cache holding keys 0 .. p0 + m - 1;
 * head_dim 64 or 128 (attention_kv_f32 applied to each query in turn,
 * libs/uaii-kernels/src/transformer.cpp:222-433). */
UAII_HIP_API int uaii_hip_attention_prefill(const float* q, const void* kcache,
                                            const void* vcache, int64_t max_seq, int n_heads,
                                            int n_kv_heads, int head_dim, int64_t p0, int64_t m,
                                            float* out, void* stream);

/* ---- timing (HIP events on `stream`) ---------------------------------------- */
/* Average device time of `iters` back-to-back uaii_hip_gemv launches, in ms. */
UAII_HIP_API int uaii_hip_time_gemv(const uaii_hip_weight* w, const float* x, float* y,
                                    int iters, float* avg_ms);
/* The same over `nw` weights of one shape taken in turn (uaii_hip_gemv each),
 * so that a rotation larger than the last-level cache reads HBM every launch.
 * No counterpart in the reference: measurement only. */
UAII_HIP_API int uaii_hip_time_gemv_rotate(const uaii_hip_weight* const* ws, int nw,
                                           const float* x, float* y, int iters, float* avg_ms);
UAII_HIP_API int uaii_hip_time_gemm(const uaii_hip_weight* w, const float* x, int64_t m,
                                    float* y, int iters, float* avg_ms);
/* Device-to-device copy with the library's plain copy kernel (bytes % 16 == 0). */
UAII_HIP_API int uaii_hip_time_copy(const void* src, void* dst, size_t bytes, int iters,
                                    float* avg_ms);
/* Per-launch floor of the decode kernels: a plain read of `bytes` (% 16 == 0)
 * in their launch shape (one 512-thread block per CU, eight 16-byte loads in
 * flight per thread), `iters` launches rotating over the `nsrc` buffers so that
 * a rotation larger than the last-level cache reads HBM every launch.
 * No counterpart in the reference: measurement only. */
UAII_HIP_API int uaii_hip_time_read(const void* const* srcs, int nsrc, size_t bytes, int iters,
                                    float* avg_ms);

#ifdef __cplusplus
}
#endif

#endif /* UAII_HIP_H_ */
