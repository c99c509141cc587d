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
// group). Each block writes (o, m, l) partials; the last block of head h to
// finish (atomic ticket) merges the splits and writes the output, then re-arms
// the ticket so the kernel can be replayed from a graph.

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
  __shared__ int last;

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
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = atomicAdd(&a.ticket[h], 1u);
    last = (prev == (uint32_t)S - 1);
  }
  __syncthreads();
  if (!last) return;
  __threadfence();

  // merge the S splits of kv head h
  const volatile float* hp = a.part + (int64_t)h * S * G * pstride;
  for (int idx = tid; idx < G * hd; idx += NT) {
    const int g = idx / hd, d = idx % hd;
    float M = -INFINITY;
    for (int k = 0; k < S; ++k) M = fmaxf(M, hp[(k * G + g) * pstride + hd]);
    float num = 0.0f, den = 0.0f;
    for (int k = 0; k < S; ++k) {
      const float mk = hp[(k * G + g) * pstride + hd];
      if (mk == -INFINITY) continue;
      const float w = expf(mk - M);
      num += w * hp[(k * G + g) * pstride + d];
      den += w * hp[(k * G + g) * pstride + hd + 1];
    }
    a.out[((int64_t)h * G + g) * hd + d] = den > 0.0f ? num / den : 0.0f;
  }
  if (tid == 0) a.ticket[h] = 0u;
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

hipError_t launch_attention_decode(const AttnArgs& a, hipStream_t s) {
  const int G = a.n_heads / a.n_kv;
  if (G < 1 || G > MAXG || a.hd > 256 || a.hd % 2 || a.n_heads % a.n_kv) return hipErrorInvalidValue;
  const int tile = a.hd > 64 ? 32 : 64;
  const size_t lds = sizeof(float) * ((size_t)G * a.hd + 2 * tile * (size_t)(a.hd + 1) + (size_t)G * tile);
  if ((int)lds > lds_limit() - 1024) return hipErrorInvalidValue;
  dim3 grid(a.n_kv, a.splits);
  if (tile == 64) {
    if (a.kv_f16) hipLaunchKernelGGL((k_attn<true, 64>), grid, dim3(NT), lds, s, a);
    else hipLaunchKernelGGL((k_attn<false, 64>), grid, dim3(NT), lds, s, a);
  } else {
    if (a.kv_f16) hipLaunchKernelGGL((k_attn<true, 32>), grid, dim3(NT), lds, s, a);
    else hipLaunchKernelGGL((k_attn<false, 32>), grid, dim3(NT), lds, s, a);
  }
  return hipGetLastError();
}

}  // namespace uaii_hip
