// attention.hip — GQA decode attention over the device KV cache (gfx950).
//
// Replaces attention_kv_f32 at q_seq = 1 (libs/uaii-kernels/src/transformer.cpp:
// 222-433): scores q.k * (1/sqrt(hd)), softmax over all cached keys plus the
// current one, then P.V, with kv head h serving q heads h*G .. h*G+G-1
// (transformer.cpp:334). The cache is head-major [n_kv][max_seq][hd] (f16 or f32),
// so one kv head's keys are one contiguous stream.
//
// Split-K over the sequence: block (h, s) takes a contiguous slice of keys for
// kv head h, stages K and V tiles in LDS, and keeps an online-softmax running
// max / sum / output for all G query heads of the group (K/V read once per
// group). Each block writes (o, m, l) partials; a second small kernel merges the
// splits of every query head. (A last-block ticket merge inside the split kernel
// costs more than the extra launch: with a device-scope release per block, an L2
// write-back on CDNA4; with write-through (sc1) partial stores and sc1 loads in
// the merging block, 409 against 451 tok/s on the 8B decode, the merge code
// raising the kernel to 214 VGPRs; with the splits of a kv head on one XCD and
// the ticket and partials in its L2, 518 against 526 tok/s.)

#include "common.h"
#include "uaii_hip_internal.h"

namespace uaii_hip {
namespace {

constexpr int NT = 256;    // threads per block
constexpr int MAXG = 16;   // max q heads per kv head

template <bool F16>
__device__ inline float ld_kv(const void* p, int64_t i) {
  if constexpr (F16) return __half2float(reinterpret_cast<const __half*>(p)[i]);
  else return reinterpret_cast<const float*>(p)[i];
}

// TILE keys per LDS tile (64 for head_dim <= 64, 32 above, keeping K+V tiles
// within 64 KiB of LDS).
template <bool F16, int TILE>
__global__ void __launch_bounds__(NT) k_attn(AttnArgs a) {
  extern __shared__ float sm[];
  const int hd = a.hd, G = a.n_heads / a.n_kv;
  const int ld = hd + 1;  // padded row stride (conflict-free column reads)
  float* q_s = sm;                      // [G][hd]
  float* k_s = q_s + G * hd;            // [TILE][ld]
  float* v_s = k_s + TILE * ld;         // [TILE][ld]
  float* p_s = v_s + TILE * ld;         // [G][TILE]
  __shared__ float m_run[MAXG], l_run[MAXG], alpha[MAXG];

  const int h = blockIdx.x, s = blockIdx.y, S = gridDim.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = NT / 64;
  const int64_t n = a.fixed_len > 0 ? (int64_t)a.fixed_len : (int64_t)a.state->pos + 1;
  const int64_t C = (n + S - 1) / S;
  const int64_t j0 = (int64_t)s * C, j1 = (j0 + C < n) ? j0 + C : n;
  const float scale = 1.0f / sqrtf((float)hd);

  for (int i = tid; i < G * hd; i += NT) q_s[i] = a.q[(int64_t)h * G * hd + i];
  if (tid < G) { m_run[tid] = -INFINITY; l_run[tid] = 0.0f; }
  // each thread owns outputs (g, d) = idx, idx + NT, ...
  constexpr int OWN = MAXG * 256 / NT;
  float o_acc[OWN];
  const int nown = (G * hd + NT - 1) / NT;
#pragma unroll
  for (int k = 0; k < OWN; ++k) o_acc[k] = 0.0f;
  __syncthreads();

  const void* kc = reinterpret_cast<const char*>(a.kcache) +
                   ((int64_t)h * a.max_seq) * hd * (F16 ? 2 : 4);
  const void* vc = reinterpret_cast<const char*>(a.vcache) +
                   ((int64_t)h * a.max_seq) * hd * (F16 ? 2 : 4);

  for (int64_t t0 = j0; t0 < j1; t0 += TILE) {
    const int tn = (int)((j1 - t0 < TILE) ? (j1 - t0) : TILE);
    for (int i = tid; i < tn * hd; i += NT) {
      const int j = i / hd, d = i % hd;
      k_s[j * ld + d] = ld_kv<F16>(kc, (t0 + j) * hd + d);
      v_s[j * ld + d] = ld_kv<F16>(vc, (t0 + j) * hd + d);
    }
    __syncthreads();
    for (int i = tid; i < G * TILE; i += NT) {
      const int g = i / TILE, j = i % TILE;
      float sc = -INFINITY;
      if (j < tn) {
        float dot = 0.0f;
        for (int d = 0; d < hd; ++d) dot += q_s[g * hd + d] * k_s[j * ld + d];
        sc = dot * scale;
      }
      p_s[g * TILE + j] = sc;
    }
    __syncthreads();
    // per-head online softmax update, one wave per head
    for (int g = wave; g < G; g += nw) {
      const float v = (lane < TILE) ? p_s[g * TILE + lane] : -INFINITY;
      const float tmax = wave_max(v);
      const float mold = m_run[g];
      const float mnew = fmaxf(mold, tmax);
      const float e = (lane < tn) ? expf(v - mnew) : 0.0f;
      if (lane < TILE) p_s[g * TILE + lane] = e;
      const float es = wave_sum(e);
      if (lane == 0) {
        const float al = (mold == -INFINITY) ? 0.0f : expf(mold - mnew);
        alpha[g] = al;
        l_run[g] = l_run[g] * al + es;
        m_run[g] = mnew;
      }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < OWN; ++k) {
      const int idx = tid + k * NT;
      if (k >= nown || idx >= G * hd) continue;
      const int g = idx / hd, d = idx % hd;
      float acc = o_acc[k] * alpha[g];
      for (int j = 0; j < tn; ++j) acc += p_s[g * TILE + j] * v_s[j * ld + d];
      o_acc[k] = acc;
    }
    __syncthreads();
  }

  // write partials: part[(h*S + s)*G + g][hd + 2] = (o[hd], m, l)
  const int64_t pstride = hd + 2;
  float* part = a.part + ((int64_t)h * S + s) * G * pstride;
#pragma unroll
  for (int k = 0; k < OWN; ++k) {
    const int idx = tid + k * NT;
    if (k >= nown || idx >= G * hd) continue;
    const int g = idx / hd, d = idx % hd;
    part[g * pstride + d] = o_acc[k];
  }
  if (tid < G) {
    part[tid * pstride + hd] = m_run[tid];
    part[tid * pstride + hd + 1] = l_run[tid];
  }
}

// ---- fast path: head_dim 64 / 128, group size 1 / 2 / 4 / 8 ----------------------
//
// Block (h, s) of 4 waves owns a contiguous key range of kv head h; each wave
// takes a quarter and walks it in tiles of 64 keys. Scores: lane = key, the
// lane's K row is read in 16-byte chunks and dotted with the G query rows held in
// LDS (same-address reads broadcast). P.V: lane = slice of head_dim, V rows read
// coalesced (64 lanes x HD/64 elements per key). Online softmax per wave, the 4
// wave states merged in LDS into one block partial; k_attn_merge combines the
// block partials.

template <bool F16>
__device__ inline void load8(const void* base, int64_t elem, float* out) {
  if constexpr (F16) {
    const uint4 r = *reinterpret_cast<const uint4*>(reinterpret_cast<const __half*>(base) + elem);
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = __half2float(__ushort_as_half((uint16_t)(w[i] & 0xffff)));
      out[2 * i + 1] = __half2float(__ushort_as_half((uint16_t)(w[i] >> 16)));
    }
  } else {
    const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + elem);
    const float4 a = p[0], b = p[1];
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
  }
}

template <bool F16, int DPL>
__device__ inline void load_slice(const void* base, int64_t elem, float* out) {
  if constexpr (F16) {
    const __half* p = reinterpret_cast<const __half*>(base) + elem;
    if constexpr (DPL == 2) {
      const uint32_t w = *reinterpret_cast<const uint32_t*>(p);
      out[0] = __half2float(__ushort_as_half((uint16_t)(w & 0xffff)));
      out[1] = __half2float(__ushort_as_half((uint16_t)(w >> 16)));
    } else {
#pragma unroll
      for (int e = 0; e < DPL; ++e) out[e] = __half2float(p[e]);
    }
  } else {
    const float* p = reinterpret_cast<const float*>(base) + elem;
#pragma unroll
    for (int e = 0; e < DPL; ++e) out[e] = p[e];
  }
}

template <bool F16, int HD, int G>
__global__ void __launch_bounds__(256) k_attn_fast(AttnArgs a) {
  constexpr int DPL = HD / 64;  // head-dim elements per lane in P.V
  constexpr int NW = 4;
  __shared__ float q_s[G * HD];
  __shared__ float p_s[NW][G][64];
  __shared__ float wm[NW][G], wl[NW][G];
  __shared__ float wo[NW][G * HD];

  const int h = blockIdx.x, sblk = blockIdx.y, SB = gridDim.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t n = a.fixed_len > 0 ? (int64_t)a.fixed_len : (int64_t)a.state->pos + 1;
  const int64_t CB = (n + SB - 1) / SB;                  // keys per block
  const int64_t b0 = (int64_t)sblk * CB, b1 = (b0 + CB < n) ? b0 + CB : n;
  const int64_t CW = (CB + NW - 1) / NW;                  // keys per wave
  const int64_t w0 = b0 + (int64_t)wave * CW;
  const int64_t w1 = (w0 + CW < b1) ? w0 + CW : b1;
  const float scale = 1.0f / sqrtf((float)HD);

  for (int i = tid; i < G * HD; i += 256) q_s[i] = a.q[(int64_t)h * G * HD + i];
  __syncthreads();

  const size_t esz = F16 ? 2 : 4;
  const char* kc = reinterpret_cast<const char*>(a.kcache) + (size_t)h * a.max_seq * HD * esz;
  const char* vc = reinterpret_cast<const char*>(a.vcache) + (size_t)h * a.max_seq * HD * esz;

  float m[G], l[G], o[G][DPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) o[g][e] = 0.0f;
  }

  for (int64_t t0 = w0; t0 < w1; t0 += 64) {
    const int tn = (int)((w1 - t0 < 64) ? (w1 - t0) : 64);
    // scores, lane = key
    float sc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) sc[g] = 0.0f;
    if (lane < tn) {
      const int64_t row = (t0 + lane) * HD;
#pragma unroll 4
      for (int c = 0; c < HD / 8; ++c) {
        float kf[8];
        load8<F16>(kc, row + 8 * c, kf);
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float4 qa = *reinterpret_cast<const float4*>(&q_s[g * HD + 8 * c]);
          const float4 qb = *reinterpret_cast<const float4*>(&q_s[g * HD + 8 * c + 4]);
          sc[g] += qa.x * kf[0] + qa.y * kf[1] + qa.z * kf[2] + qa.w * kf[3] +
                   qb.x * kf[4] + qb.y * kf[5] + qb.z * kf[6] + qb.w * kf[7];
        }
      }
    }
    float alpha[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float sv = (lane < tn) ? sc[g] * scale : -INFINITY;
      const float mnew = fmaxf(m[g], wave_max(sv));
      const float pv = (lane < tn) ? expf(sv - mnew) : 0.0f;
      alpha[g] = (m[g] == -INFINITY) ? 0.0f : expf(m[g] - mnew);
      l[g] = l[g] * alpha[g] + wave_sum(pv);
      m[g] = mnew;
      p_s[wave][g][lane] = pv;
    }
    // the probabilities are read back by other lanes of this wave (in-order LDS)
    __builtin_amdgcn_wave_barrier();
    // P.V, lane = head-dim slice
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < DPL; ++e) o[g][e] *= alpha[g];
#pragma unroll 8
    for (int jj = 0; jj < tn; ++jj) {
      float vf[DPL];
      load_slice<F16, DPL>(vc, (t0 + jj) * HD + lane * DPL, vf);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float pg = p_s[wave][g][jj];
#pragma unroll
        for (int e = 0; e < DPL; ++e) o[g][e] += pg * vf[e];
      }
    }
    __builtin_amdgcn_wave_barrier();
  }

  // combine the 4 wave states of this block
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if (lane == 0) { wm[wave][g] = m[g]; wl[wave][g] = l[g]; }
#pragma unroll
    for (int e = 0; e < DPL; ++e) wo[wave][g * HD + lane * DPL + e] = o[g][e];
  }
  __syncthreads();
  const int64_t pstride = HD + 2;
  float* part = a.part + ((int64_t)h * SB + sblk) * G * pstride;
  for (int i = tid; i < G * HD; i += 256) {
    const int g = i / HD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, wm[w][g]);
    float acc = 0.0f, den = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = (wm[w][g] == -INFINITY) ? 0.0f : expf(wm[w][g] - M);
      acc += f * wo[w][i];
      den += f * wl[w][g];
    }
    part[g * pstride + (i % HD)] = acc;
    if (i % HD == 0) {
      part[g * pstride + HD] = M;
      part[g * pstride + HD + 1] = den;
    }
  }
}

// ---- f16 KV, head_dim 64 / 128: one memory round trip per 32-key tile ---------------
//
// A wave takes tiles of TK = 32 keys. All K and V loads of a tile are issued
// back to back before any arithmetic (16-byte loads, each lane group reading a
// contiguous 64-byte (K) or 16-byte (V) run of a key row), so a block's keys cost
// one memory round trip. Scores: LK = HD/32 lanes per key, each owning 32 dims;
// v_dot2_f32_f16 on the exact f16 keys against q * scale split into f16 hi + lo
// pairs (about 22 significant bits of q), sums f32, reduced over the LK lanes.
// Online softmax per query head over the tile. P.V: LV = HD/8 lanes per key, 8
// dims each, 64/LV keys per instruction; the key groups are reduced once at the
// end. Partials as for the other kernels.
typedef _Float16 attn_h2 __attribute__((ext_vector_type(2)));

__device__ inline float adot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(attn_h2, a), __builtin_bit_cast(attn_h2, b), c, false);
}

__device__ inline uint32_t ah_bits(_Float16 h) { return (uint32_t)__builtin_bit_cast(uint16_t, h); }

template <int HD, int G, int TK, int NW>
__global__ void __launch_bounds__(NW * 64) k_attn_h16(AttnArgs a) {
  static_assert(TK == 16 || TK == 32, "tile of 16 or 32 keys");
  static_assert(TK >= 64 / (HD / 32), "at least one key per lane group in the scores");
  constexpr int LK = HD / 32;            // lanes per key (scores)
  static_assert(LK == 2 || LK == 4, "score lanes reduced with quad_perm moves");
  constexpr int KPI = 64 / LK;           // keys per K instruction
  constexpr int KJ = TK / KPI;           // keys per lane per tile (scores)
  constexpr int LV = HD / 8;             // lanes per key (P.V)
  constexpr int VPI = 64 / LV;           // keys per V instruction
  constexpr int VJ = TK / VPI;           // keys per lane per tile (P.V)
  __shared__ uint4 qh_s[G][HD / 8], ql_s[G][HD / 8];  // (q * scale) as f16 pairs, 4 pairs per uint4
  __shared__ float p_s[NW][G][TK];       // layout [key % VPI][key / VPI] per g
  __shared__ float wm[NW][G], wl[NW][G];
  __shared__ float wo[NW][G][HD];

  const int h = blockIdx.x, sblk = blockIdx.y, SB = gridDim.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // key range of this block in 32-bit arithmetic (positions < max_seq < 2^31):
  // the K/V loads wait for it, and a 64-bit division is a long emulated sequence
  const int n = a.fixed_len > 0 ? a.fixed_len : a.state->pos + 1;
  const int CB = (int)(((unsigned)n + (unsigned)SB - 1u) / (unsigned)SB);
  const int b0 = sblk * CB, b1 = (b0 + CB < n) ? b0 + CB : n;
  // Scores in base-2 units (q scaled by log2(e) / sqrt(hd)), so each softmax
  // exponential is one v_exp_f32 instead of expf's range reduction around it:
  // attention + merge 11.7 -> 11.0 us on the 8B decode. The partials' maxima
  // are written back in natural units for the merge.
  const float scale = 1.44269504088896341f / sqrtf((float)HD);

  // q of the group first: waiting for it does not wait for the K/V loads below
  constexpr int NT = NW * 64;
  constexpr int QPT = (G * HD + NT - 1) / NT;
  float qv[QPT];
#pragma unroll
  for (int k = 0; k < QPT; ++k) {
    const int i = tid + NT * k;
    qv[k] = (i < G * HD) ? a.q[(int64_t)h * G * HD + i] : 0.0f;
  }

  const __half* kc = reinterpret_cast<const __half*>(a.kcache) + (int64_t)h * a.max_seq * HD;
  const __half* vc = reinterpret_cast<const __half*>(a.vcache) + (int64_t)h * a.max_seq * HD;
  const int kq = lane % LK, kk = lane / LK;   // scores: dims [32 kq, 32 kq + 32) of key kk + KPI j
  const int vd = lane % LV, vk = lane / LV;   // P.V: dims [8 vd, 8 vd + 8) of key vk + VPI j

  // Two register sets, used in turn: a wave's next tile is in flight while it
  // computes one. (A loop that loads its tile at the top of every pass but the
  // first joins two load paths at the loop head, and the compiler then waited
  // there for the whole first tile, K and V, before the first score. With one
  // tile per wave, as at 4096 positions, the straight-line path below measured
  // attention + merge 12.1 against 12.7 us on the 8B decode, the waits for V
  // falling inside the score and softmax work.)
  uint4 kr[KJ][4], vr[VJ], kn[KJ][4], vn[VJ];
  auto load_tile = [&](int t0, uint4 (&K)[KJ][4], uint4 (&V)[VJ]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
      int key = t0 + kk + KPI * j;
      key = key < b1 ? key : b1 - 1;  // in bounds; masked below
      const uint4* src = reinterpret_cast<const uint4*>(kc + (int64_t)key * HD + 32 * kq);
#pragma unroll
      for (int c = 0; c < 4; ++c) K[j][c] = src[c];
    }
#pragma unroll
    for (int j = 0; j < VJ; ++j) {
      int key = t0 + vk + VPI * j;
      key = key < b1 ? key : b1 - 1;
      V[j] = *reinterpret_cast<const uint4*>(vc + (int64_t)key * HD + 8 * vd);
    }
  };

  const int first = b0 + wave * TK;
  if (first < b1) load_tile(first, kr, vr);

  // q * scale -> f16 (hi, lo) pairs in LDS
#pragma unroll
  for (int k = 0; k < QPT; ++k) {
    const int i = tid + NT * k;
    const float v = qv[k] * scale;
    const _Float16 hi = (_Float16)v;
    const _Float16 lo = (_Float16)(v - (float)hi);
    if (i < G * HD) {
      reinterpret_cast<uint16_t*>(&qh_s[0][0])[i] = (uint16_t)ah_bits(hi);
      reinterpret_cast<uint16_t*>(&ql_s[0][0])[i] = (uint16_t)ah_bits(lo);
    }
  }
  __syncthreads();

  float m[G], l[G], o[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[g][e] = 0.0f;
  }

  auto tile = [&](int t0, const uint4 (&K)[KJ][4], const uint4 (&V)[VJ]) __attribute__((always_inline)) {
    // scores
    float sc[KJ][G];
#pragma unroll
    for (int j = 0; j < KJ; ++j)
#pragma unroll
      for (int g = 0; g < G; ++g) sc[j][g] = 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint4 qh = qh_s[g][4 * kq + c], ql = ql_s[g][4 * kq + c];
#pragma unroll
        for (int j = 0; j < KJ; ++j) {
          float t = sc[j][g];
          t = adot2(K[j][c].x, qh.x, t); t = adot2(K[j][c].x, ql.x, t);
          t = adot2(K[j][c].y, qh.y, t); t = adot2(K[j][c].y, ql.y, t);
          t = adot2(K[j][c].z, qh.z, t); t = adot2(K[j][c].z, ql.z, t);
          t = adot2(K[j][c].w, qh.w, t); t = adot2(K[j][c].w, ql.w, t);
          sc[j][g] = t;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float t = sc[j][g];
        t += dpp_mov<0xB1>(t);                  // xor 1
        if constexpr (LK == 4) t += dpp_mov<0x4E>(t);  // xor 2
        sc[j][g] = (t0 + kk + KPI * j < b1) ? t : -INFINITY;
      }
    }
    // online softmax over the tile, per query head
    float alpha[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mx = sc[0][g];
#pragma unroll
      for (int j = 1; j < KJ; ++j) mx = fmaxf(mx, sc[j][g]);
      const float mnew = fmaxf(m[g], wave_max_dpp(mx));
      float ps = 0.0f;
#pragma unroll
      for (int j = 0; j < KJ; ++j) {
        const float pv = (sc[j][g] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(sc[j][g] - mnew);
        ps += pv;
        const int key = kk + KPI * j;
        if (kq == 0) p_s[wave][g][(key % VPI) * VJ + key / VPI] = pv;
      }
      alpha[g] = (m[g] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m[g] - mnew);
      l[g] = l[g] * alpha[g] + wave_sum_dpp(kq == 0 ? ps : 0.0f);
      m[g] = mnew;
    }
    __builtin_amdgcn_wave_barrier();
    // P.V
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) o[g][e] *= alpha[g];
#pragma unroll
    for (int j = 0; j < VJ; ++j) {
      float vf[8];
      const uint32_t w4[4] = {V[j].x, V[j].y, V[j].z, V[j].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vf[2 * e] = __half2float(__ushort_as_half((uint16_t)(w4[e] & 0xffffu)));
        vf[2 * e + 1] = __half2float(__ushort_as_half((uint16_t)(w4[e] >> 16)));
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float pg = p_s[wave][g][vk * VJ + j];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[g][e] += pg * vf[e];
      }
    }
    __builtin_amdgcn_wave_barrier();
  };

  const int step = NW * TK;
  if (b1 - b0 <= step) {
    // at most one tile per wave (every split of a cache up to 4096 positions):
    // no next-tile code ahead of the first scores
    if (first < b1) tile(first, kr, vr);
  } else {
    for (int t0 = first; t0 < b1; t0 += 2 * step) {
      if (t0 + step < b1) load_tile(t0 + step, kn, vn);
      tile(t0, kr, vr);
      if (t0 + step >= b1) break;
      if (t0 + 2 * step < b1) load_tile(t0 + 2 * step, kr, vr);
      tile(t0 + step, kn, vn);
    }
  }

  // reduce the key groups of P.V (lanes vd, vd + LV, ...)
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float t = o[g][e];
#pragma unroll
      for (int o2 = LV; o2 < 64; o2 <<= 1) t += __shfl_xor(t, o2, 64);
      o[g][e] = t;
    }
  // combine the 4 wave states of this block
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if (lane == 0) { wm[wave][g] = m[g]; wl[wave][g] = l[g]; }
    if (lane < LV) {
#pragma unroll
      for (int e = 0; e < 8; ++e) wo[wave][g][8 * lane + e] = o[g][e];
    }
  }
  __syncthreads();
  const int64_t pstride = HD + 2;
  float* part = a.part + ((int64_t)h * SB + sblk) * G * pstride;
  for (int i = tid; i < G * HD; i += NT) {
    const int g = i / HD, d = i % HD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, wm[w][g]);
    float acc = 0.0f, den = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = (wm[w][g] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(wm[w][g] - M);
      acc += f * wo[w][g][d];
      den += f * wl[w][g];
    }
    part[g * pstride + d] = acc;
    if (d == 0) {
      part[g * pstride + HD] = M * 0.693147180559945309f;  // ln 2: natural units
      part[g * pstride + HD + 1] = den;
    }
  }
}

// Tiles of 32 keys per wave: a block covers 128 keys per pass. (16-key tiles
// with twice the splits measured slower end to end: more blocks and a wider
// merge cost more than the shorter per-block chain saves.)
// (Eight waves of 16-key tiles per block measured within 2 % of this.)
template <int HD>
bool launch_h16(const AttnArgs& a, int G, hipStream_t s) {
  constexpr int TK = 32, NW = 4;
  dim3 grid(a.n_kv, a.splits);
  switch (G) {
    case 1: UAII_LAUNCH((k_attn_h16<HD, 1, TK, NW>), grid, dim3(NW * 64), 0, s, a); return true;
    case 2: UAII_LAUNCH((k_attn_h16<HD, 2, TK, NW>), grid, dim3(NW * 64), 0, s, a); return true;
    case 4: UAII_LAUNCH((k_attn_h16<HD, 4, TK, NW>), grid, dim3(NW * 64), 0, s, a); return true;
    case 8: UAII_LAUNCH((k_attn_h16<HD, 8, TK, NW>), grid, dim3(NW * 64), 0, s, a); return true;
    default: return false;
  }
}


// Merge the SB (<= 32) block partials of every query head (one block per head,
// one thread per output dim): out = sum_s w_s o_s / sum_s w_s l_s with
// w_s = exp(m_s - max_s m_s). Split s's m and l sit on lane s of every wave,
// which derives the weights itself (DPP max and sum) and reads w_s from lane s
// with readlane; a thread's dims of the splits' o are loaded together with
// them, before any arithmetic, so the merge costs one memory round trip (where
// loading the weights first, through LDS, and then the o values cost three).
// The sums and their order are those of a loop s = 0 .. SB-1.
__global__ void __launch_bounds__(256) k_attn_merge(AttnArgs a) {
  constexpr int CH = 32;  // most splits (attention_splits)
  const int hq = blockIdx.x, hd = a.hd, G = a.n_heads / a.n_kv, SB = a.splits;
  const int kvh = hq / G, g = hq % G, lane = threadIdx.x & 63;
  const int d = threadIdx.x < hd ? (int)threadIdx.x : hd - 1;  // lanes past hd repeat the last dim
  const int64_t ks = (int64_t)G * (hd + 2);                      // split stride
  const float* hp = a.part + ((int64_t)kvh * SB * G + g) * (hd + 2);
  const int kl = lane < SB ? lane : SB - 1;
  const float mk = hp[kl * ks + hd], lk = hp[kl * ks + hd + 1];
  float ov[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) ov[c] = hp[(c < SB ? c : SB - 1) * ks + d];
  const float mv = lane < SB ? mk : -INFINITY;
  const float M = wave_max_dpp(mv);
  const float wk = (lane < SB && mv != -INFINITY) ? expf(mv - M) : 0.0f;
  const float den = wave_sum_dpp(wk * (lane < SB ? lk : 0.0f));
  // splits past SB weigh 0 (their loads repeat split SB - 1): adding 0 * o
  // leaves the sum as it is, and the FMAs stay on a straight line
  float num = 0.0f;
#pragma unroll
  for (int c = 0; c < CH; ++c) num += lane_val(wk, c) * ov[c];
  if ((int)threadIdx.x < hd) a.out[(int64_t)hq * hd + d] = num * (den > 0.0f ? 1.0f / den : 0.0f);
}


}  // namespace

hipError_t prepare_attention() {
  const int lim = lds_limit();
  const void* fns[] = {(const void*)k_attn<true, 64>, (const void*)k_attn<false, 64>,
                       (const void*)k_attn<true, 32>, (const void*)k_attn<false, 32>};
  for (const void* f : fns) {
    (void)hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, lim - 1024);
    (void)hipGetLastError();
  }
  return hipSuccess;
}

template <bool F16, int HD>
bool launch_fast_hd(const AttnArgs& a, int G, hipStream_t s) {
  dim3 grid(a.n_kv, a.splits);
  switch (G) {
    case 1: UAII_LAUNCH((k_attn_fast<F16, HD, 1>), grid, dim3(256), 0, s, a); return true;
    case 2: UAII_LAUNCH((k_attn_fast<F16, HD, 2>), grid, dim3(256), 0, s, a); return true;
    case 4: UAII_LAUNCH((k_attn_fast<F16, HD, 4>), grid, dim3(256), 0, s, a); return true;
    case 8: UAII_LAUNCH((k_attn_fast<F16, HD, 8>), grid, dim3(256), 0, s, a); return true;
    default: return false;
  }
}

// Key splits of the decode attention for a cache of max_seq positions: one per
// 128 keys, at most 32 (one 32-key tile per wave at 4096 positions).
int attention_splits(int64_t max_seq) {
  const int64_t s = (max_seq + 127) / 128;
  return (int)(s < 1 ? 1 : (s > 32 ? 32 : s));
}

hipError_t launch_attention_splits(const AttnArgs& a, hipStream_t s) {
  const int G = a.n_heads / a.n_kv;
  if (G < 1 || G > MAXG || a.hd > 256 || a.hd % 2 || a.n_heads % a.n_kv) return hipErrorInvalidValue;
  if (a.splits < 1 || a.splits > 32) return hipErrorInvalidValue;  // attention_splits: <= 32
  if ((a.hd == 64 || a.hd == 128) && (G == 1 || G == 2 || G == 4 || G == 8)) {
    bool ok;
    if (a.kv_f16) ok = (a.hd == 64) ? launch_h16<64>(a, G, s) : launch_h16<128>(a, G, s);
    else if (a.hd == 64) ok = launch_fast_hd<false, 64>(a, G, s);
    else ok = launch_fast_hd<false, 128>(a, G, s);
    if (ok) return hipGetLastError();
  }
  const int tile = a.hd > 64 ? 32 : 64;
  const size_t lds = sizeof(float) * ((size_t)G * a.hd + 2 * tile * (size_t)(a.hd + 1) + (size_t)G * tile);
  if ((int)lds > lds_limit() - 1024) return hipErrorInvalidValue;
  dim3 grid(a.n_kv, a.splits);
  if (tile == 64) {
    if (a.kv_f16) UAII_LAUNCH((k_attn<true, 64>), grid, dim3(NT), lds, s, a);
    else UAII_LAUNCH((k_attn<false, 64>), grid, dim3(NT), lds, s, a);
  } else {
    if (a.kv_f16) UAII_LAUNCH((k_attn<true, 32>), grid, dim3(NT), lds, s, a);
    else UAII_LAUNCH((k_attn<false, 32>), grid, dim3(NT), lds, s, a);
  }
  return hipGetLastError();
}

hipError_t launch_attention_decode(const AttnArgs& a, hipStream_t s) {
  const hipError_t st = launch_attention_splits(a, s);
  if (st != hipSuccess) return st;
  UAII_LAUNCH(k_attn_merge, dim3(a.n_heads), dim3((a.hd + 63) / 64 * 64), 0, s, a);
  return hipGetLastError();
}

}  // namespace uaii_hip
