// attn_out.hip — the merge of the decode attention's key splits, the attention
// output projection and its residual add in one launch (gfx950).
//
// Replaces, at M = 1, quant_gemm_f32 of the attention output
// (libs/uaii-kernels/src/quant_gemm.cpp:22-70) and the residual add_f32
// (elementwise.cpp:99-110) for Q4_0, Q8_0 and Q4_K weights, together with the second step of
// the split-K decode attention: out = sum_s w_s o_s / sum_s w_s l_s with
// w_s = exp(m_s - max_s m_s), which makes the per-split softmaxes one softmax
// over all keys as attention_kv_f32 computes it (transformer.cpp:222-433).
//
// Split along K by heads: block (r, c) owns column slice c of W_o (SC = 256
// columns: 8 blocks of 32 or one Q4_K super-block; 256 / hd query heads, hd 64
// or 128) and RB = 32 J consecutive rows r RB ... The row block is the grid's
// x index, so the slices of one row block (its blocks r + R c) land on one XCD
// and their atomic adds to a row meet in that XCD's L2 (13.8 MB fetched per 8B
// launch against 17.8 MB with the slices of a row spread over the XCDs; the
// split partials are then fetched by every XCD).
// Each wave merges 64 of the slice's dims from the split partials with the
// arithmetic of k_attn_merge (same bits), the block keeps them in LDS, and lane
// (g, b) of a wave multiplies weight block b of rows g, g + 8, ... (J rows) by
// them; the eight blocks of a row are summed with DPP and the row's sum is
// added into the residual stream with one float atomic. The partial loads are
// issued first and the weight loads right behind them, so the merge runs while
// the weight bytes are in flight. Block (0, c) also writes the merged slice to
// the attention output buffer.
//
// A residual row is the sum of 1 + q_dim / SC terms added in the order the
// atomics arrive, so two runs may differ in the last bits of those f32 adds;
// every other value is computed in a fixed order.

#include "common.h"
#include "block_dot.h"
#include "uaii_hip_internal.h"

namespace uaii_hip {
namespace {

constexpr int SC = 256;  // weight columns per block
constexpr int NW = 4;    // waves per block
constexpr int CH = 32;   // most key splits (attention_splits)

template <int FMT, int J>
__global__ void __launch_bounds__(NW * 64) k_merge_o(MergeOArgs p) {
  constexpr int QW = FMT == T_Q4_0 ? 1 : 2;  // 16-byte payload words per block
  __shared__ float xs[SC];
  const AttnArgs& a = p.at;
  const int c = blockIdx.y, w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int hd = a.hd, G = a.n_heads / a.n_kv, SB = a.splits;

  // the split partials of query dim col (hd is 64 or 128: a wave lies in one head)
  const int col = c * SC + w * 64 + lane;
  const int hq = col / hd, d = col - hq * hd;
  const int kvh = hq / G, g = hq - kvh * G;
  const int64_t ks = (int64_t)G * (hd + 2);  // split stride
  const float* hp = a.part + ((int64_t)kvh * SB * G + g) * (hd + 2);
  const int kl = lane < SB ? lane : SB - 1;
  const float mk = hp[kl * ks + hd], lk = hp[kl * ks + hd + 1];
  float ov[CH];
#pragma unroll
  for (int s = 0; s < CH; ++s) ov[s] = hp[(s < SB ? s : SB - 1) * ks + d];

  // the lane's weights: block b of rows r0 + 8 j: 16 (Q4_0) or 32 (Q8_0) payload
  // bytes and the f16 scale, or for Q4_K (one 256-element super-block per slice)
  // the 32 quant bytes holding sub-block b and the super-block's 16 scale bytes
  const int b = lane & 7;
  const int64_t r0 = (int64_t)blockIdx.x * (NW * 8 * J) + w * (8 * J) + (lane >> 3);
  uint4 qv[J][QW];
  uint32_t sv[J];
  uint4 mt[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int64_t r = r0 + 8 * j;
    const int64_t off = FMT == T_Q4_K ? c * 128 + (b >> 1) * 32 : (c * SC + b * 32) * QW / 2;
    const uint4* src = reinterpret_cast<const uint4*>(p.w.a + r * p.w.a_row + off);
#pragma unroll
    for (int k = 0; k < QW; ++k) qv[j][k] = src[k];
    if constexpr (FMT == T_Q4_K) mt[j] = *reinterpret_cast<const uint4*>(p.w.b + r * p.w.b_row + c * 16);
    else sv[j] = *reinterpret_cast<const uint16_t*>(p.w.b + r * p.w.b_row + c * (SC / 16) + b * 2);
  }
  // every load is issued before the merge waits for the first of them
  __builtin_amdgcn_sched_barrier(0);

  // merge: splits past SB weigh 0 (their loads repeat split SB - 1)
  const float mv = lane < SB ? mk : -INFINITY;
  const float M = wave_max_dpp(mv);
  const float wk = (lane < SB && mv != -INFINITY) ? expf(mv - M) : 0.0f;
  const float den = wave_sum_dpp(wk * (lane < SB ? lk : 0.0f));
  float num = 0.0f;
#pragma unroll
  for (int s = 0; s < CH; ++s) num += lane_val(wk, s) * ov[s];
  const float o = num * (den > 0.0f ? 1.0f / den : 0.0f);
  xs[w * 64 + lane] = o;
  if (blockIdx.x == 0) a.out[col] = o;
  // block barrier ordering LDS only (no wait for the weight loads in flight)
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  __builtin_amdgcn_sched_barrier(0);

  // block b's 32 inputs
  float xv[32];
#pragma unroll
  for (int k = 0; k < 32; k += 4) {
    const float4 t = *reinterpret_cast<const float4*>(&xs[b * 32 + k]);
    xv[k] = t.x; xv[k + 1] = t.y; xv[k + 2] = t.z; xv[k + 3] = t.w;
  }
  float sx = 0.0f;
#pragma unroll
  for (int k = 0; k < 32; ++k) sx += xv[k];

  float rs[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    float v;
    if constexpr (FMT == T_Q8_0) v = q8_0_dot(qv[j], sv[j], xv);
    else if constexpr (FMT == T_Q4_K) v = q4_k_dot(qv[j], mt[j], b, xv, sx);
    else v = q4_0_dot(qv[j][0], sv[j], xv, sx);
    // the row's eight blocks: lanes b = 0..7 of the row group
    v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_mov<0x141>(v);  // row_half_mirror
    rs[j] = v;
  }
  float v = rs[0];
#pragma unroll
  for (int j = 1; j < J; ++j) v = b == j ? rs[j] : v;
  if (b < J) atomicAdd(p.y + r0 + 8 * b, v);
}

int pick_j(const MergeOArgs& p) {
  const int64_t slices = p.at.n_heads * (int64_t)p.at.hd / SC;
  for (int j : {4, 2, 1})
    if (p.rows % (NW * 8 * j) == 0 && slices * (p.rows / (NW * 8 * j)) >= 512) return j;
  return p.rows % (NW * 8) == 0 ? 1 : 0;
}

}  // namespace

bool merge_o_supported(const MergeOArgs& p) {
  const AttnArgs& a = p.at;
  if (a.n_kv < 1 || a.n_heads % a.n_kv) return false;
  if (a.hd != 64 && a.hd != 128) return false;  // whole waves per head, whole heads per slice
  if (a.splits < 1 || a.splits > CH) return false;
  const int64_t K = (int64_t)a.n_heads * a.hd;
  if (K % SC) return false;
  const DevWeight& w = p.w;
  if (w.cols != K || w.b_row != K / 16) return false;
  // a slice is 8 blocks of 32 (Q4_0, Q8_0) or one 256-element super-block (Q4_K)
  if (!(w.type == T_Q4_0 && w.a_row == K / 2) && !(w.type == T_Q8_0 && w.a_row == K) &&
      !(w.type == T_Q4_K && w.a_row == K / 2))
    return false;
  if (p.rows <= 0 || w.rows < p.rows) return false;
  return pick_j(p) > 0;
}

hipError_t launch_merge_o(const MergeOArgs& p, hipStream_t s) {
  if (!merge_o_supported(p) || !p.at.part || !p.at.out || !p.y) return hipErrorInvalidValue;
  const int J = pick_j(p);
  dim3 grid((unsigned)(p.rows / (NW * 8 * J)), (unsigned)((int64_t)p.at.n_heads * p.at.hd / SC));
#define UAII_MO(F)                                                                          \
  do {                                                                                      \
    if (J == 4) UAII_LAUNCH((k_merge_o<F, 4>), grid, dim3(NW * 64), 0, s, p);                \
    else if (J == 2) UAII_LAUNCH((k_merge_o<F, 2>), grid, dim3(NW * 64), 0, s, p);           \
    else UAII_LAUNCH((k_merge_o<F, 1>), grid, dim3(NW * 64), 0, s, p);                       \
  } while (0)
  if (p.w.type == T_Q8_0) UAII_MO(T_Q8_0);
  else if (p.w.type == T_Q4_K) UAII_MO(T_Q4_K);
  else UAII_MO(T_Q4_0);
#undef UAII_MO
  return hipGetLastError();
}

}  // namespace uaii_hip
