// uaii_hip_internal.h — launch helpers shared by the HIP translation units and
// the host runtime. Not part of the public C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace uaii_hip {

// Bytes per row of the split arrays a, b, c, d for `type` at `cols`.
void split_row_bytes(int type, int64_t cols, int64_t out[4]);

// q4_0_pairwise: Q4_0 rows take the values of the reference's f32 weight load
// (gguf.cpp:514-520) rather than its packed decode (gguf_dequant.cpp:117-134).
hipError_t launch_repack(const DevWeight& w, const uint8_t* src_dev, hipStream_t s,
                         bool q4_0_pairwise = false);
hipError_t launch_dequant(const DevWeight& w, int64_t row0, int64_t nrows, float* out,
                          hipStream_t s);

// ---- fused GEMV (decode, M = 1) ----------------------------------------------

enum Epilogue : int {
  EPI_STORE = 0,   // y[row] = dot
  EPI_ADD = 1,     // y[row] = y[row] + dot        (residual add)
  EPI_QKV = 2,     // bias, RoPE pairs, q -> y, k/v -> KV cache at pos
  EPI_SWIGLU = 3,  // rows (gate i, up i) -> y[i] = silu(g) * u
  EPI_LOGITS = 4,  // y[row] = dot, block argmax partials (+ final argmax/advance kernel)
  EPI_GELU = 5,    // y[row] = gelu(dot) (tanh form, elementwise.cpp:57-71)
  // two MoE experts' down rows in one launch: segments 0 and 1 cover the same
  // output rows with their own input (seg.x), expert and weight (seg.scale);
  // y[row] = (y[row] + s0 * dot0) + s1 * dot1, the order of two EPI_ADD launches
  EPI_ADD2 = 6,
};

// Persistent decode state shared by the step kernels (device memory).
struct StepState {
  int32_t pos;       // position of the token being processed (= KV past_len)
  int32_t token;     // token id fed at `pos`
  int32_t n_prompt;  // prompt length
  int32_t argmax;    // last greedy argmax
  float max_logit;   // its logit
  float second;      // runner-up logit (parity margin diagnostics)
  int32_t pad[2];
};

struct GemvSeg {
  DevWeight w;   // for EPI_SWIGLU: gate rows; w2 = up rows
  DevWeight w2;
  const float* bias;   // optional per-row bias (EPI_QKV)
  int64_t rows;        // logical rows in this segment
  int64_t row_base;    // first logical row in the epilogue's output space
  int kind;            // EPI_QKV: 0 = q, 1 = k, 2 = v
  int block0;          // first block of this segment
  // MoE: the weight rows of expert *expert (device memory) of a [E * expert_rows]
  // stack: physical row = *expert * expert_rows + row (w and w2 alike)
  const int32_t* expert;
  int64_t expert_rows;
  const float* scale;  // EPI_ADD: y += *scale * dot (device memory), or null
  const float* x;      // this segment's input vector, or null for GemvArgs::x
  // set by launch_gemv (the kernel's integer setup, done once on the host):
  // row groups of the segment, groups per block (gq, plus one for blocks below
  // gr), and 64-chunk columns per wave of a K split
  int32_t ngroups, gq, gr, per;
};

// The fields a GEMV block needs first (its input and RMSNorm weight) lead the
// struct, so the launch's first scalar-cache line holds them and the input
// loads go out before anything else is read.
struct GemvArgs {
  const float* x;        // input vector [K]
  const float* norm_w;   // RMSNorm weight [K] (prologue) or null
  int64_t K;
  float eps;
  int nseg;
  int epi;
  // set by launch_gemv: waves of a block that split one row set's K (1, 2 or 4)
  int ksplit;
  float* y;              // EPI_STORE/ADD/QKV(q)/SWIGLU/LOGITS output
  float* tap;            // optional copy of each written value (EPI_ADD)
  float* xtap;           // optional copy of the staged (normalised) input, block 0
  float* rtap;           // optional copy of the raw input (before any RMSNorm), block 0
  // EPI_QKV
  void* kcache;          // layer base, [n_kv][max_seq][hd] (f16 or f32)
  void* vcache;
  int64_t max_seq;
  int head_dim;
  int rope_mode;
  const float2* rope;    // [max_seq][hd/2] (cos, sin)
  // EPI_LOGITS
  float* part_val;       // [part_cap] block partials of the argmax
  int32_t* part_idx;
  int part_cap;          // capacity of part_val/part_idx (launch fails if the grid exceeds it)
  int kv_f16;            // EPI_QKV: f16 cache (beside part_cap: no padding after either)
  int32_t* ids;          // token history [max_seq + 1]
  // shared
  StepState* state;
  GemvSeg seg[3];
};

hipError_t launch_gemv(const GemvArgs& a, hipStream_t s);
// Raise the dynamic-LDS limit of the GEMV kernel (call once per device, outside capture).
hipError_t prepare_gemv();
// Number of blocks launch_gemv will use for the given args (for partial buffers).
int gemv_grid(const GemvArgs& a);

// MoE routing (transformer.cpp:446-481, :565-580): probs = softmax(logits[E]),
// the k largest (ties: lower expert first), weights renormalised over them.
hipError_t launch_moe_route(const float* logits, int n_experts, int k, int32_t* ids, float* w,
                            hipStream_t s);

// ---- small ops -------------------------------------------------------------------

hipError_t launch_embed(const DevWeight& w, const StepState* st, float* x, float* tap,
                        hipStream_t s);
hipError_t launch_embed_rows(const DevWeight& w, const int32_t* ids, int64_t n, float* x,
                             hipStream_t s);
hipError_t launch_advance(StepState* st, int32_t* ids, hipStream_t s);
// Elementwise operators of the op-by-op backend: op 0 add, 1 mul (a, b), 2 SiLU,
// 3 GELU (a only); y may alias a.
hipError_t launch_elementwise(int op, const float* a, const float* b, float* y, int64_t n,
                              hipStream_t s);
// K and V rows [rows][kv_dim] into head-major caches [n_kv][max_seq][hd] at p0..
hipError_t launch_kv_append(const float* k, const float* v, void* kc, void* vc, int64_t rows,
                            int64_t kv_dim, int hd, int64_t max_seq, int64_t p0, int f16,
                            hipStream_t s);
hipError_t launch_rmsnorm(const float* x, const float* w, float* y, int64_t rows, int64_t n,
                          float eps, hipStream_t s);
hipError_t launch_softmax(const float* x, float* y, int64_t n, hipStream_t s);
hipError_t launch_argmax(const float* x, int64_t n, int32_t* out_idx, hipStream_t s);
hipError_t launch_rope(float* x, int64_t rows, int64_t dim, int head_dim, const int32_t* pos,
                       int64_t pos_stride, const float2* tab, int mode, hipStream_t s);
// Plain device copy of n16 16-byte words (the yardstick for HBM rates and counters).
hipError_t launch_copy(const void* src, void* dst, int64_t n16, hipStream_t s);
// Plain read of n16 16-byte words, one 512-thread block per CU (the per-launch
// floor of the decode kernels); `sink` receives a word only by a 2^-32 chance.
hipError_t launch_read(const void* src, int64_t n16, uint32_t* sink, hipStream_t s);

// ---- attention -----------------------------------------------------------------

// Everything a block needs to issue its first loads sits in the first 64 bytes.
struct AttnArgs {
  const float* q;        // [n_heads * hd] (post-RoPE)
  const StepState* state;  // keys 0..state->pos inclusive
  const void* kcache;    // layer base [n_kv][max_seq][hd]
  const void* vcache;
  int64_t max_seq;
  int fixed_len;           // >0: use this key count instead of state->pos + 1
  int kv_f16;
  int n_heads, n_kv, hd;
  int splits;
  float* out;            // [n_heads * hd]
  float* part;           // [n_kv][splits][group][hd + 2]
};

int attention_splits(int64_t max_seq);
hipError_t launch_attention_decode(const AttnArgs& a, hipStream_t s);
// The split kernel alone: partials into a.part, a.out untouched (a.splits <= 32).
hipError_t launch_attention_splits(const AttnArgs& a, hipStream_t s);

// ---- split merge + output projection + residual add (attn_out.hip) -----------------

struct MergeOArgs {
  AttnArgs at;      // the split partials (part, splits, heads, hd); merged values also to at.out
  DevWeight w;      // W_o [rows][n_heads * hd], Q4_0
  int64_t rows;     // output rows
  float* y;         // residual stream: y[r] += W_o[r] . merged
};

bool merge_o_supported(const MergeOArgs& p);  // shapes and weight layout (not the pointers)
hipError_t launch_merge_o(const MergeOArgs& p, hipStream_t s);

// ---- split-K GEMV with a float-atomic residual add (splitk_gemv.hip) --------------

struct SplitKArgs {
  DevWeight w;      // Q4_0 [rows][K]
  int64_t rows;     // output rows
  const float* x;   // input [K]
  float* y;         // y[r] += W[r] . x
};

bool gemv_splitk_supported(const SplitKArgs& p);  // shapes and weight layout (not the pointers)
hipError_t launch_gemv_splitk(const SplitKArgs& p, hipStream_t s);
hipError_t prepare_attention();
// Resolves the allocation-free attention scratch of the current device (noalloc.hip).
hipError_t prepare_noalloc();
size_t noalloc_scratch_bytes();

// ---- one decode GEMV with its weights streamed through an LDS ring ----------------

// Loader waves fetch the block's rows global -> LDS while compute waves take
// stages out of LDS (ring_gemv.hip), so the dot products never hold back the
// next loads. Q4_0 only, EPI_STORE / EPI_ADD; see ring_gemv_supported for the
// shapes. The input fields lead (the kernel loads its input before anything else).
struct RingArgs {
  const float* x;        // input [K]
  const float* norm_w;   // RMSNorm weight or null
  int64_t K;
  float eps;
  int epi;               // EPI_STORE or EPI_ADD
  // set by launch_ring_gemv: stages per block (tq, plus one for blocks below tr)
  int32_t tq, tr;
  DevWeight w;
  int64_t rows;          // output rows (<= w.rows)
  float* y;              // output
  float* tap;            // EPI_ADD: copy of each written value, or null
  const uint8_t* pad;    // >= 1 KiB of device memory read by the padding DMA lines
};

bool ring_gemv_supported(const RingArgs& a);
hipError_t prepare_ring_gemv();
hipError_t launch_ring_gemv(const RingArgs& a, hipStream_t s);

// ---- sampling (sample.hip) ------------------------------------------------------------

// One draw from the logits row (sample_token_f32's non-greedy path,
// libs/uaii-runtime/src/sampling.cpp:53-125). With `state`, the penalised ids are
// ids[0 .. pos], the draw is rbuf[pos + 1 - n_prompt] and the pick kernel
// advances the token as k_argmax_final does; without it, pen[0 .. n_pen) and
// r_fixed. `ws`: sample_workspace_bytes(V), 256-byte aligned.
struct SampleArgs {
  const float* logits;
  int64_t V;
  float inv_t;           // 1 / max(temperature, 1e-5)
  float top_p;           // active when 0 < top_p < 1 - 1e-6
  int32_t top_k;         // active when 0 < top_k < V
  float rep;             // repetition penalty, active when > 1 + 1e-6
  StepState* state;
  int32_t* ids;          // history [max_seq + 2]
  const float* rbuf;     // uniform draws, one per generated token
  int64_t nr;
  const int32_t* pen;    // standalone: penalised ids
  int64_t n_pen;
  float r_fixed;         // standalone: the draw
  int32_t* out;          // the sampled id, or null
  void* ws;
};
int sample_max_vocab();
size_t sample_workspace_bytes(int64_t V);
hipError_t launch_sample(const SampleArgs& a, hipStream_t s);

// The final argmax + token advance over `nparts` partials (k_argmax_final).
hipError_t launch_argmax_final(float* part_val, int32_t* part_idx, int nparts, StepState* state,
                               int32_t* ids, hipStream_t s);


// ---- prefill (M > 1 prompt tokens, matrix cores) ---------------------------------------

// Activation rows prepared for the MFMA GEMM: x * 2^e = hi + lo in f16 (each
// aligned group of 4 stored as k0, k2, k1, k3), per-32 sums of x * 2^e, and 2^-e.
struct PfAct {
  __half* hi;     // [mpad][K]
  __half* lo;     // [mpad][K]
  float* sx;      // [K / 32][mpad]
  float* rs;      // [mpad]
  int64_t mpad;   // rows allocated (multiple of 64); rows >= M are zero
  int64_t K;
  // 1: the layout the Q4_0 direct-to-LDS GEMM takes with its high nibbles
  // decoded in place (elements 16..31 of every 32-block stored times 1/16);
  // only for activations every consumer of which is such a launch
  int hi16;
};

struct PfSeg {
  DevWeight w;      // weight rows (EPI_SWIGLU: gate)
  DevWeight w2;     // EPI_SWIGLU: up rows
  int64_t rows;     // output columns of this segment
  int64_t col0;     // first output column in y
  int tile0;        // set by launch_pf_gemm
};

struct PfGemmArgs {
  PfSeg seg[3];
  int nseg;
  int epi;              // EPI_STORE, EPI_ADD, EPI_SWIGLU, EPI_GELU
  int64_t M, K, mpad;
  const __half* ahi;
  const __half* alo;
  const float* sx;
  const float* rs;
  float* y;             // [M][ldy]
  int64_t ldy;
  // EPI_ADD split over K: ksplit > 1 blocks along grid z each take K / ksplit
  // and store their partial to part[z][M][ldy] instead of adding into y; the
  // next launch_pf_prep of y adds the partials (z in order) into y
  int ksplit;
  float* part;
  // optional activation-row map: output row t reads activation row arow[t]
  // (MoE experts gather their tokens); rows are those of ahi/alo/sx/rs
  const int32_t* arow;
  int64_t sx_ld;  // row stride of sx (the activations' padded row count); 0: mpad
  // optional expert grouping (MoE): grid row y computes output rows
  // [gtab[3y + 1], gtab[3y + 2]) against expert gtab[3y] of the weight stacks,
  // whose rows e * seg.rows .. (e + 1) * seg.rows - 1 are that expert's;
  // at most gbm rows per entry (pf_gemm_group_rows of the format)
  const int32_t* gtab;
  int ntab, ngroups, gbm;
  int hi16;       // the activations carry PfAct::hi16's layout (Q4_0 only)
};

struct PfQkvArgs {
  const float* qkv;     // [M][ldq]: q | k | v before bias and RoPE
  int64_t ldq, M;
  int p0;               // position of row 0
  int q_dim, kv_dim, head_dim, rope_mode;
  const float2* rope;   // [max_seq][head_dim / 2]
  const float *bq, *bk, *bv;
  float* qout;          // [M][q_dim]
  void* kcache;         // layer base [n_kv][max_seq][hd]
  void* vcache;
  int kv_f16;
  int64_t max_seq;
  // K-split GEMM output instead of qkv when nsplit > 1: [nsplit][M][ldq]
  const float* part;
  int nsplit;
};

struct PfAttnArgs {
  const float* q;       // [M][ldq] post-RoPE
  int64_t ldq;
  const void* kcache;   // f16 layer base [n_kv][max_seq][hd]
  const void* vcache;
  int64_t max_seq;
  int n_heads, n_kv, hd;
  int64_t p0, M;        // queries at positions p0 .. p0 + M - 1 (keys 0 .. p0 + M - 1)
  float* out;           // [M][ldo]
  int64_t ldo;
};

// MoE prompt rows (transformer.cpp:446-612 applied to M tokens):
// router logits of RMSNorm(x[t]) . Wr^T (Wr F32 or F16, [E][K]), softmax, top-k
// (ties: lower expert), weights renormalised: ids[t][k], w[t][k].
hipError_t launch_pf_moe_route(const float* x, int64_t M, int64_t K, const float* norm_w, float eps,
                               const DevWeight& router, int E, int k, int32_t* ids, float* w,
                               hipStream_t s);
// Per-expert token lists from ids[M][k]: counts[E], offsets[E] (prefix sums),
// list[offsets[e] + j] = token of the j-th (token, slot) routed to e (token
// order), inv[t * k + slot] = its packed row.
hipError_t launch_pf_moe_lists(const int32_t* ids, int64_t M, int k, int E, int32_t* counts,
                               int32_t* offsets, int32_t* list, int32_t* inv, hipStream_t s);
// x[t] += w[t][0] y[inv[t][0]], then + w[t][1] y[inv[t][1]], ... (slot order).
hipError_t launch_pf_moe_combine(float* x, int64_t M, int64_t D, int k, const float* w,
                                 const int32_t* inv, const float* y, hipStream_t s);
bool pf_router_supported(int type);

bool pf_supported(int type);
bool pf_attn_supported(int head_dim, int n_heads, int n_kv);
int64_t pf_mpad(int64_t m);
// x [M][ldx] -> act. With nsplit > 0, x first becomes x + sum_z part[z][M][ldx]
// (written back: x is the residual stream).
hipError_t launch_pf_prep(float* x, int64_t ldx, int64_t M, const float* norm_w, float eps,
                          const PfAct& act, hipStream_t s, const float* part = nullptr,
                          int nsplit = 0);
// Whether a weight format's prefill GEMM takes PfAct::hi16 activations.
bool pf_hi16_supported(int type);
hipError_t launch_pf_gemm(PfGemmArgs a, hipStream_t s);
// K split launch_pf_gemm can take for `a` (EPI_ADD only; 1 = none) on `cus` CUs.
int pf_gemm_ksplit(const PfGemmArgs& a, int cus);
// rows per entry of an expert-grouped GEMM's table for this block format
int pf_gemm_group_rows(int type);
hipError_t launch_pf_qkv(const PfQkvArgs& a, hipStream_t s);
hipError_t launch_pf_attn(const PfAttnArgs& a, hipStream_t s);

}  // namespace uaii_hip
