/*
 * uaii_oracle.h — CPU oracle for the GGUF token loop.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker the parity tests,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg compare the HIP
 * path against. The product (libuaii_amd.so) never links, loads or calls it.
 *
 * Every function restates the reference algorithm in plain C and cites the
 * reference file:line it follows (paths relative to the reference root).
 *
 * Parity pinning (what checks each function against something other than its
 * own formula) is listed per function below; see tests/test_oracle_*.py.
 */
#ifndef UAII_ORACLE_H_
#define UAII_ORACLE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF tensor type ids (include/uaii/loaders/gguf.hpp:18-36). */
enum {
  ORC_F32 = 0, ORC_F16 = 1, ORC_Q4_0 = 2, ORC_Q4_1 = 3, ORC_Q5_0 = 6, ORC_Q5_1 = 7,
  ORC_Q8_0 = 8, ORC_Q2_K = 10, ORC_Q3_K = 11, ORC_Q4_K = 12, ORC_Q5_K = 13, ORC_Q6_K = 14
};

/* IEEE half -> float, exact incl. subnormals (libs/uaii-quant/src/gguf_dequant.cpp:79-105).
 * Pinned: exhaustive 65536-value check against numpy float16 and oracle/_ref. */
float orc_half_to_float(uint16_t h);

/* float -> IEEE half bits, round to nearest even; overflow to +-inf, NaN stays a
 * quiet NaN. The fp16 KV cache mode of orc_generate stores every cached K/V
 * element as orc_half_to_float(orc_float_to_half(x)).
 * Pinned: every float32 bit pattern against numpy float16, closed-form ties,
 * subnormals and overflows (tests/test_oracle_f16.py). */
uint16_t orc_float_to_half(float f);
void orc_float_to_half_n(const float* in, uint16_t* out, int64_t n);

/* Bytes of one packed row of `cols` values (include/uaii/quant/formats.hpp:81-102). */
size_t orc_row_bytes(int type, int64_t cols);

/* Elements per block and bytes per block for a GGUF type; 0 if unsupported. */
int orc_block_elems(int type);
int orc_block_bytes(int type);

/* Dequantize one packed row (libs/uaii-quant/src/gguf_dequant.cpp:117-439).
 * Returns 0 on success, -1 on unsupported type or cols not a block multiple.
 * Pinned: reference Q4_0 known-answer block (tests/unit/quant_dequant_test.cpp:37-80),
 * closed-form hand-built blocks for each format, and oracle/_ref. */
int orc_dequant_row(int type, const uint8_t* packed, int64_t cols, float* out);

/* One row as the reference's f32 weight load gives it (gguf_load_tensor_f32,
 * libs/uaii-loaders/src/gguf.cpp:445-556), the values every weight takes on
 * Path A: Q4_0 byte j of a block gives elements 2j (low nibble) and 2j+1 (high
 * nibble) (gguf.cpp:514-520); Q8_0, F32 and F16 decode as orc_dequant_row, and
 * the other block formats go through it (gguf.cpp:528-546).
 * Pinned: against the reference's gguf_load_tensor_f32 on whole GGUF tensors
 * (oracle/_ref, tests/test_oracle_path_a.py). */
int orc_load_row_f32(int type, const uint8_t* packed, int64_t cols, float* out);

/* C[M,N] = A[M,K] * dequant(B[N,K])^T, per-row dequant then sequential f32 dot
 * (libs/uaii-kernels/src/quant_gemm.cpp:22-70). nthreads<=0 -> all cores.
 * Pinned: benchmark pattern known answer (benchmarks/src/uaii_bench.cpp:505-518)
 * computed in f64, and oracle/_ref. */
int orc_quant_gemm(int type, const float* A, int64_t M, int64_t K, const uint8_t* B,
                   int64_t N, float* C, int nthreads);

/* y = x * (1/sqrt(mean(x^2)+eps)) * w (libs/uaii-kernels/src/norm.cpp:89-130). */
void orc_rmsnorm(const float* x, const float* w, float* y, int64_t n, float eps);

/* In-place RoPE over `dim` values split into heads of `head_dim`
 * (libs/uaii-kernels/src/transformer.cpp:144-220). mode 0 = interleaved pairs,
 * mode 2 = NeoX half pairs. */
void orc_rope(float* x, int64_t dim, int64_t head_dim, float pos, float theta, int mode);

/* Seq=1 decode attention over a [past,kv_dim] cache plus the current k/v row
 * (libs/uaii-kernels/src/transformer.cpp:222-433). Scale 1/sqrt(head_dim). */
void orc_attention_decode(const float* q, const float* kcache, const float* vcache,
                          int64_t past, const float* k_new, const float* v_new,
                          float* out, int n_heads, int n_kv_heads, int head_dim);

/* Softmax over n (libs/uaii-kernels/src/softmax.cpp:11-77). */
void orc_softmax(const float* x, float* y, int64_t n);

/* Greedy argmax, strict '>' so the lowest index wins ties
 * (libs/uaii-runtime/src/sampling.cpp:38-50). */
int64_t orc_argmax(const float* row, int64_t n);

/* SiLU v/(1+exp(-v)) (libs/uaii-kernels/src/elementwise.cpp:73-84). */
float orc_silu(float v);

/* MoE router: logits = x . gate^T, softmax, top-1 (transformer.cpp:446-481). */
void orc_moe_router(const float* x, const float* gate, int64_t D, int64_t E, float* probs);

/* Top-k experts by prob, renormalised weights (transformer.cpp:565-580). */
void orc_moe_topk(const float* probs, int64_t E, int k, int* ids, float* weights);

/* ------------------------------------------------------------------ GGUF model */

typedef struct orc_model orc_model;

/* Open a GGUF decoder (header layout libs/uaii-loaders/src/gguf.cpp:374-443, graph
 * derivation gguf.cpp:801-1246). max_layers>0 caps the layer count like
 * UAII_MAX_LAYERS (gguf.cpp:785-799). Returns NULL on failure (orc_last_error()). */
orc_model* orc_model_open(const char* path, int max_layers);
/* The same; path_a != 0 runs every model on the reference's Path A (all weights
 * loaded as f32 by gguf_load_tensor_f32 and multiplied by the f32 GEMM), which
 * the reference takes under its default options (enable_memory_reuse=1:
 * session.cpp:259-367, :420-443) or keep_quantized_weights=0. MoE models take
 * Path A either way (their expert kernel reads f32 only, transformer.cpp:551-554). */
orc_model* orc_model_open_ex(const char* path, int max_layers, int path_a);
void orc_model_close(orc_model* m);
const char* orc_last_error(void);

/* Hyperparameters: [n_layers, dim, n_heads, n_kv_heads, head_dim, vocab, ffn,
 * n_experts, top_k, rope_mode, ctx_len, tied] */
void orc_model_hparams(const orc_model* m, int64_t* out12);
void orc_model_fparams(const orc_model* m, float* out2); /* [rope_theta, rms_eps] */

/* Raw view of one GGUF tensor: type, ne[0..2] (GGUF order, ne0 = row length) and
 * a pointer into the mapped file. Returns 0 if found, -1 otherwise. */
int orc_model_tensor(const orc_model* m, const char* name, int* type, int64_t* ne3,
                     const uint8_t** data);

/* Taps filled after each run(): copies of the last step's named tensors. */
typedef struct orc_taps {
  float* hidden;   /* [dim]           embedding output            */
  float* resid1;   /* [n_layers, dim] after attention residual    */
  float* resid2;   /* [n_layers, dim] after FFN residual          */
  float* normed;   /* [dim]           output RMSNorm              */
  float* logits;   /* [vocab]                                      */
  float* probs;    /* [vocab]                                      */
} orc_taps;

/* Greedy generate (libs/uaii-runtime/src/session.cpp:910-1046): token-by-token
 * prefill, then argmax over probs. kv_f16 != 0 rounds cached K/V to fp16 (to
 * mirror a device fp16 cache); 0 keeps the reference's f32 cache.
 * out receives prompt+generated ids; *out_n the count. taps may be NULL.
 * Returns 0 on success, -1 on error. nthreads for the GEMVs. */
int orc_generate(orc_model* m, const int64_t* prompt, int64_t n_prompt, int64_t max_new,
                 int kv_f16, int nthreads, int64_t* out, int64_t* out_n, orc_taps* taps);

/* orc_generate with prompt_block > 0: prompt tokens 0 .. n_prompt-2 run layer by
 * layer in blocks of prompt_block tokens (each weight row dequantized once per
 * block), the last prompt token and the decode as token steps. Same ids and taps
 * as orc_generate bit for bit (tests/test_oracle_prompt.py); for long prompts. */
int orc_generate_ex(orc_model* m, const int64_t* prompt, int64_t n_prompt, int64_t max_new,
                    int kv_f16, int nthreads, int64_t prompt_block, int64_t* out,
                    int64_t* out_n, orc_taps* taps);

/* Run `n_steps` decode steps feeding `tokens` at positions start_pos.. with a KV
 * cache pre-filled with deterministic values for positions < start_pos (timing
 * window for the CPU baseline). Returns elapsed seconds, <0 on error. */
double orc_time_decode_window(orc_model* m, int64_t start_pos, int64_t n_steps,
                              int nthreads);

#ifdef __cplusplus
}
#endif

#endif /* UAII_ORACLE_H_ */
