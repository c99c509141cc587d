// uaii_synth.h — seeded synthetic GGUF decoder writer (weights, quantizers, file).
//
// The reference ships no GGUF block quantizer or quantized GGUF writer
// (libs/uaii-quant/src/codec.cpp:93-178 packs only F32/F16/BF16/INT*/NF4/MXFP4;
// libs/uaii-loaders/src/gguf.cpp:604-662 writes F32 only), so the synthetic
// models the benchmarks and tests run on come from this writer. The packed
// bytes it emits are the specification: only dequantization (reading) is pinned
// against the reference.
//
// Values: element i of tensor t (tensors numbered in file order from 0) is
//   key  = splitmix64(seed + 0x632BE59BD9B4E019 * (t + 1))
//   a, b = splitmix64(key + 2i), splitmix64(key + 2i + 1)
//   u1   = ((a >> 11) + 1) * 2^-53,  u2 = (b >> 11) * 2^-53
//   n    = sqrt(-2 ln u1) * cos(2 pi u2)            (Box-Muller, double)
//   w    = (float)(n * std)
// Norm weights are 1.0 f32. The MoE router (ffn_gate_inp) is f32 with its own
// std. The file is GGUF v3 with a 32-byte aligned data section (the reference
// ignores general.alignment and always aligns to 32, gguf.cpp:436-440).
#ifndef UAII_SYNTH_H_
#define UAII_SYNTH_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct uaii_synth_config {
  int64_t n_layers;
  int64_t dim;
  int64_t n_heads;
  int64_t n_kv_heads;
  int64_t head_dim;      /* 0 -> dim / n_heads */
  int64_t ffn;
  int64_t vocab;
  int64_t ctx_len;
  float rope_theta;
  float rms_eps;
  int tied;              /* 1: no output.weight (lm_head = token_embd) */
  int n_experts;         /* 0: dense SwiGLU FFN */
  int top_k;
  int type_default;      /* GGUF type ids: 0 F32, 1 F16, 2 Q4_0, 8 Q8_0, 12 Q4_K, ... */
  int type_embd;         /* -1 -> type_default */
  int type_output;       /* -1 -> type_default */
  int type_attn_v;       /* -1 -> type_default */
  int type_ffn_down;     /* -1 -> type_default */
  uint64_t seed;
  float std;             /* weight std, e.g. 0.02 */
  float router_std;      /* ffn_gate_inp std */
  const char* arch;      /* general.architecture, NULL -> "llama" */
  int gelu;              /* 1: dense FFN without gate (ffn_up, ffn_down; GELU) */
  int qkv_bias;          /* 1: attn_q/k/v.bias f32 tensors */
  int64_t shared_ffn;    /* MoE: shared expert width (ffn_*_shexp), 0 = none */
} uaii_synth_config;

/* Write the model. nthreads <= 0 uses all cores. Returns 0 or -1 (see
 * uaii_synth_last_error). */
int uaii_synth_write_gguf(const char* path, const uaii_synth_config* cfg, int nthreads);
const char* uaii_synth_last_error(void);

/* The value generator above, for tests: n values of tensor t starting at i0. */
void uaii_synth_normals(uint64_t seed, uint64_t tensor, uint64_t i0, int64_t n, float std,
                        float* out);

/* Quantize one row of n values (n a multiple of the block size) to GGUF `type`.
 * Returns bytes written or -1. */
int64_t uaii_synth_quantize_row(int type, const float* x, int64_t n, uint8_t* out);

/* float -> IEEE half, round to nearest even. */
uint16_t uaii_synth_f32_to_f16(float f);

#ifdef __cplusplus
}
#endif

#endif /* UAII_SYNTH_H_ */
