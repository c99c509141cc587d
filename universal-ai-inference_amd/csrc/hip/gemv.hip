// gemv.hip — fused dequant-GEMV for the decode step (M = 1), gfx950.
//
// Replaces the reference's per-row dequant + sequential dot
// (libs/uaii-kernels/src/quant_gemm.cpp:22-70) and the surrounding elementwise
// graph ops that read the GEMV result (gguf.cpp:1000-1209): RMSNorm prologue
// (norm.cpp:89-130), bias + RoPE + KV append epilogue (transformer.cpp:144-220,
// kv_cache.hpp:80-120), residual Add (elementwise.cpp:86-97), SiLU*up
// (elementwise.cpp:73-110) and greedy argmax (sampling.cpp:38-50).
//
// Work decomposition: a block is WPB waves; each wave owns RPW output rows and
// walks their split-layout payload in 16-byte chunks, lane l taking chunks
// l, l+64, ... . The input vector is staged once per block in LDS as f32 (after
// the optional RMSNorm), each lane reads the x values of its chunk once and
// reuses them for all RPW rows, and the per-chunk sum of x folds the
// quantization offsets/mins out of the inner loop. Partial dots are reduced with
// 64-lane xor shuffles (DPP on CDNA4).

#include "common.h"
#include "uaii_hip_internal.h"

#include <algorithm>

namespace uaii_hip {
namespace {

constexpr int WPB = 4;  // waves per block
constexpr int RPW = 4;  // rows per wave (even: RoPE / SwiGLU pairs share a wave)

// ---- per-format chunk decode-dot ------------------------------------------------

// x values of chunk t: up to four 16-runs (or one short run for F32/F16).
template <int FMT>
__device__ inline int x_runs(int64_t t, int64_t base[4]) {
  if constexpr (FMT == T_Q4_0 || FMT == T_Q4_1 || FMT == T_Q5_0 || FMT == T_Q5_1) {
    base[0] = 32 * t; base[1] = 32 * t + 16; return 2;
  } else if constexpr (FMT == T_Q8_0) {
    base[0] = 16 * t; return 1;
  } else if constexpr (FMT == T_Q4_K || FMT == T_Q5_K) {
    const int64_t sb = t / 8; const int tt = (int)(t % 8), cc = tt / 2, hh = tt % 2;
    base[0] = 256 * sb + 64 * cc + 16 * hh; base[1] = base[0] + 32; return 2;
  } else if constexpr (FMT == T_Q6_K) {
    const int64_t sb = t / 8; const int h = (int)((t % 8) / 4), u = (int)(t % 4);
    base[0] = 256 * sb + 128 * h + 16 * u; base[1] = base[0] + 64; return 2;
  } else if constexpr (FMT == T_Q2_K || FMT == T_Q3_K) {
    const int64_t sb = t / 4; const int h = (int)((t % 4) / 2), g = (int)(t % 2);
    for (int p = 0; p < 4; ++p) base[p] = 256 * sb + 128 * h + 32 * p + 16 * g;
    return 4;
  } else {
    return 0;
  }
}

// Wave-uniform base pointers of one weight row in the split layout.
struct RowPtr {
  const uint8_t* a;
  const uint8_t* b;
  const uint8_t* c;
  const uint8_t* d;
};

__device__ inline RowPtr row_ptr(const DevWeight& w, int64_t r) {
  RowPtr p;
  p.a = w.a + r * w.a_row;
  p.b = w.b + r * w.b_row;
  p.c = w.c + r * w.c_row;
  p.d = w.d + r * w.d_row;
  return p;
}

// Raw per-row data of one chunk (only the fields a format uses stay live).
struct Raw {
  uint4 q;     // 16 payload bytes
  uint4 aux;   // side data (format specific)
  uint4 aux2;  // high-bit planes (Q5_K qh, Q3_K hmask)
  float s0, s1;
};

__device__ inline float byte_f(uint32_t w, int k) { return (float)((w >> (8 * k)) & 0xffu); }

template <int FMT>
__device__ inline void load_raw(const RowPtr& p, int64_t t, Raw& o) {
  o.q = *reinterpret_cast<const uint4*>(p.a + t * 16);
  if constexpr (FMT == T_Q4_0) {
    o.s0 = h2f(ld_u16(p.b + t * 2));
  } else if constexpr (FMT == T_Q8_0) {
    o.s0 = h2f(ld_u16(p.b + (t >> 1) * 2));
  } else if constexpr (FMT == T_Q4_1) {
    const uint32_t dm = *reinterpret_cast<const uint32_t*>(p.b + t * 4);
    o.s0 = h2f((uint16_t)(dm & 0xffff)); o.s1 = h2f((uint16_t)(dm >> 16));
  } else if constexpr (FMT == T_Q5_0) {
    o.aux.x = *reinterpret_cast<const uint32_t*>(p.b + t * 4);
    o.s0 = h2f(ld_u16(p.c + t * 2));
  } else if constexpr (FMT == T_Q5_1) {
    o.aux.x = *reinterpret_cast<const uint32_t*>(p.b + t * 4);
    const uint32_t dm = *reinterpret_cast<const uint32_t*>(p.c + t * 4);
    o.s0 = h2f((uint16_t)(dm & 0xffff)); o.s1 = h2f((uint16_t)(dm >> 16));
  } else if constexpr (FMT == T_Q4_K || FMT == T_Q5_K) {
    o.aux = *reinterpret_cast<const uint4*>(p.b + (t >> 3) * 16);
    if constexpr (FMT == T_Q5_K) {
      // the 16 qh bytes covering this chunk's lanes l = 16*(t&1) + i
      o.aux2 = *reinterpret_cast<const uint4*>(p.c + (t >> 3) * 32 + 16 * (t & 1));
    }
  } else if constexpr (FMT == T_Q6_K) {
    const int64_t sb = t >> 3; const int h = (int)((t & 7) >> 2), u = (int)(t & 3);
    o.aux = *reinterpret_cast<const uint4*>(p.b + sb * 64 + h * 32 + 16 * (u & 1));
    const int8_t* sc = reinterpret_cast<const int8_t*>(p.c + sb * 16 + h * 8);
    const float d = h2f(ld_u16(p.d + sb * 2));
    o.s0 = d * (float)sc[u];
    o.s1 = d * (float)sc[u + 4];
  } else if constexpr (FMT == T_Q2_K) {
    o.aux = *reinterpret_cast<const uint4*>(p.b + (t >> 2) * 16);  // scales
    const uint32_t dd = *reinterpret_cast<const uint32_t*>(p.c + (t >> 2) * 4);
    o.s0 = h2f((uint16_t)(dd & 0xffff)); o.s1 = h2f((uint16_t)(dd >> 16));
  } else if constexpr (FMT == T_Q3_K) {
    o.aux = *reinterpret_cast<const uint4*>(p.c + (t >> 2) * 16);  // scales12, d
    o.aux2 = *reinterpret_cast<const uint4*>(p.b + (t >> 2) * 32 + 16 * (t & 1));
  }
}

__device__ inline uint32_t word(const uint4& v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

// Byte i of a 16-byte register value (no memory round trip for runtime i).
__device__ inline int bget(const uint4& v, int i) {
  return (int)((word(v, i >> 2) >> (8 * (i & 3))) & 0xffu);
}

// K-quant 6-bit (scale, min) pair j from the meta word (scales at bytes 4..15),
// same unpacking as gguf_dequant.cpp:107-115.
__device__ inline void kscale_reg(int j, const uint4& meta, int& sc, int& mn) {
  if (j < 4) {
    sc = bget(meta, 4 + j) & 63;
    mn = bget(meta, 8 + j) & 63;
  } else {
    sc = (bget(meta, 8 + j) & 15) | ((bget(meta, j) >> 6) << 4);
    mn = (bget(meta, 8 + j) >> 4) | ((bget(meta, 4 + j) >> 6) << 4);
  }
}

// Dot of one chunk with its x values. xv holds the runs back to back (16 each),
// xs the per-run sums.
template <int FMT>
__device__ inline float chunk_dot(const Raw& o, int64_t t, const float* xv,
                                  const float* xs) {
  if constexpr (FMT == T_Q4_0 || FMT == T_Q4_1) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t wq = word(o.q, i);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        s += byte_f(wq & 0x0f0f0f0fu, k) * xv[4 * i + k];
        s += byte_f((wq >> 4) & 0x0f0f0f0fu, k) * xv[16 + 4 * i + k];
      }
    }
    if constexpr (FMT == T_Q4_0) return o.s0 * (s - 8.0f * (xs[0] + xs[1]));
    else return o.s0 * s + o.s1 * (xs[0] + xs[1]);
  } else if constexpr (FMT == T_Q5_0 || FMT == T_Q5_1) {
    const uint32_t hb = o.aux.x;
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t b = (word(o.q, j >> 2) >> (8 * (j & 3))) & 0xffu;
      const uint32_t lo = (b & 15u) | (((hb >> j) & 1u) << 4);
      const uint32_t hi = (b >> 4) | (((hb >> (j + 16)) & 1u) << 4);
      s += (float)lo * xv[j] + (float)hi * xv[16 + j];
    }
    if constexpr (FMT == T_Q5_0) return o.s0 * (s - 16.0f * (xs[0] + xs[1]));
    else return o.s0 * s + o.s1 * (xs[0] + xs[1]);
  } else if constexpr (FMT == T_Q8_0) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t wq = word(o.q, i);
#pragma unroll
      for (int k = 0; k < 4; ++k) s += (float)(int8_t)((wq >> (8 * k)) & 0xffu) * xv[4 * i + k];
    }
    return o.s0 * s;
  } else if constexpr (FMT == T_Q4_K || FMT == T_Q5_K) {
    const int tt = (int)(t & 7), cc = tt >> 1;
    const float d = h2f((uint16_t)(o.aux.x & 0xffff)), dmin = h2f((uint16_t)(o.aux.x >> 16));
    int sc, mn;
    kscale_reg(2 * cc, o.aux, sc, mn);
    const float d1 = d * (float)sc, m1 = dmin * (float)mn;
    kscale_reg(2 * cc + 1, o.aux, sc, mn);
    const float d2 = d * (float)sc, m2 = dmin * (float)mn;
    float slo = 0.0f, shi = 0.0f;
    if constexpr (FMT == T_Q4_K) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t wq = word(o.q, i);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          slo += byte_f(wq & 0x0f0f0f0fu, k) * xv[4 * i + k];
          shi += byte_f((wq >> 4) & 0x0f0f0f0fu, k) * xv[16 + 4 * i + k];
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const uint32_t b = (word(o.q, j >> 2) >> (8 * (j & 3))) & 0xffu;
        const uint32_t h = (word(o.aux2, j >> 2) >> (8 * (j & 3))) & 0xffu;
        const uint32_t lo = (b & 15u) + 16u * ((h >> (2 * cc)) & 1u);
        const uint32_t hi = (b >> 4) + 16u * ((h >> (2 * cc + 1)) & 1u);
        slo += (float)lo * xv[j];
        shi += (float)hi * xv[16 + j];
      }
    }
    return d1 * slo - m1 * xs[0] + d2 * shi - m2 * xs[1];
  } else if constexpr (FMT == T_Q6_K) {
    const int u = (int)(t & 3), sh = 2 * (u >> 1);
    float slo = 0.0f, shi = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t b = (word(o.q, j >> 2) >> (8 * (j & 3))) & 0xffu;
      const uint32_t h = (word(o.aux, j >> 2) >> (8 * (j & 3))) & 0xffu;
      const uint32_t lo = (b & 15u) | (((h >> sh) & 3u) << 4);
      const uint32_t hi = (b >> 4) | (((h >> (sh + 4)) & 3u) << 4);
      slo += (float)lo * xv[j];
      shi += (float)hi * xv[16 + j];
    }
    return o.s0 * (slo - 32.0f * xs[0]) + o.s1 * (shi - 32.0f * xs[1]);
  } else if constexpr (FMT == T_Q2_K) {
    const int h = (int)((t & 3) >> 1), g = (int)(t & 1);
    float tot = 0.0f;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int s = bget(o.aux, 8 * h + 2 * p + g);
      float sq = 0.0f;
#pragma unroll
      for (int l = 0; l < 16; ++l) {
        const uint32_t b = (word(o.q, l >> 2) >> (8 * (l & 3))) & 0xffu;
        sq += (float)((b >> (2 * p)) & 3u) * xv[16 * p + l];
      }
      tot += (o.s0 * (float)(s & 15)) * sq - (o.s1 * (float)(s >> 4)) * xs[p];
    }
    return tot;
  } else if constexpr (FMT == T_Q3_K) {
    const int h = (int)((t & 3) >> 1), g = (int)(t & 1);
    const float dall = h2f((uint16_t)(o.aux.w & 0xffff));
    float tot = 0.0f;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int j = 8 * h + 2 * p + g;
      const int lo4 = (j < 8) ? (bget(o.aux, j) & 15) : (bget(o.aux, j - 8) >> 4);
      const int hi2b = (bget(o.aux, 8 + (j % 4)) >> (2 * (j / 4))) & 3;
      const float dl = dall * (float)((lo4 | (hi2b << 4)) - 32);
      const uint32_t mbit = 1u << (4 * h + p);
      float sq = 0.0f;
#pragma unroll
      for (int l = 0; l < 16; ++l) {
        const uint32_t b = (word(o.q, l >> 2) >> (8 * (l & 3))) & 0xffu;
        const uint32_t m = (word(o.aux2, l >> 2) >> (8 * (l & 3))) & 0xffu;
        const int qq = (int)((b >> (2 * p)) & 3u) - ((m & mbit) ? 0 : 4);
        sq += (float)qq * xv[16 * p + l];
      }
      tot += dl * sq;
    }
    return tot;
  } else if constexpr (FMT == T_F32) {
    return __uint_as_float(o.q.x) * xv[0] + __uint_as_float(o.q.y) * xv[1] +
           __uint_as_float(o.q.z) * xv[2] + __uint_as_float(o.q.w) * xv[3];
  } else if constexpr (FMT == T_F16) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t wq = word(o.q, i);
      s += h2f((uint16_t)(wq & 0xffff)) * xv[2 * i] + h2f((uint16_t)(wq >> 16)) * xv[2 * i + 1];
    }
    return s;
  } else {
    return 0.0f;
  }
}

// x floats per chunk for a format.
template <int FMT>
constexpr int xn() {
  return (FMT == T_Q2_K || FMT == T_Q3_K) ? 64 : (FMT == T_Q8_0 ? 16 : (FMT == T_F32 ? 4 : (FMT == T_F16 ? 8 : 32)));
}

template <int FMT>
__device__ inline void load_x(const float* __restrict__ xsm, int64_t t, float* xv, float* xsum) {
  if constexpr (FMT == T_F32 || FMT == T_F16) {
    constexpr int n = (FMT == T_F32) ? 4 : 8;
#pragma unroll
    for (int i = 0; i < n; ++i) xv[i] = xsm[n * t + i];
    xsum[0] = 0.0f;
  } else {
    int64_t base[4];
    const int nr = x_runs<FMT>(t, base);
#pragma unroll
    for (int rr = 0; rr < xn<FMT>() / 16; ++rr) {
      if (rr < nr) {
        const float4* p = reinterpret_cast<const float4*>(xsm + base[rr]);
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float4 v = p[k];
          xv[16 * rr + 4 * k + 0] = v.x; xv[16 * rr + 4 * k + 1] = v.y;
          xv[16 * rr + 4 * k + 2] = v.z; xv[16 * rr + 4 * k + 3] = v.w;
          s += (v.x + v.y) + (v.z + v.w);
        }
        xsum[rr] = s;
      }
    }
  }
}

// Accumulate RPW row dots over the row payloads; lane l takes chunks l, l+64, ...
// Two chunks per iteration so each lane has 2*RPW 16-byte loads in flight.
template <int FMT>
__device__ inline void rows_dot(const RowPtr* P, int64_t nch, const float* xsm, int lane,
                                float* acc) {
  for (int64_t t = lane; t < nch; t += 128) {
    const bool two = t + 64 < nch;
    Raw r0[RPW], r1[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) load_raw<FMT>(P[r], t, r0[r]);
    if (two) {
#pragma unroll
      for (int r = 0; r < RPW; ++r) load_raw<FMT>(P[r], t + 64, r1[r]);
    }
    float xv[xn<FMT>()];
    float xsum[4];
    load_x<FMT>(xsm, t, xv, xsum);
#pragma unroll
    for (int r = 0; r < RPW; ++r) acc[r] += chunk_dot<FMT>(r0[r], t, xv, xsum);
    if (two) {
      load_x<FMT>(xsm, t + 64, xv, xsum);
#pragma unroll
      for (int r = 0; r < RPW; ++r) acc[r] += chunk_dot<FMT>(r1[r], t + 64, xv, xsum);
    }
  }
}

// ---- prologue ---------------------------------------------------------------------

// Stage x (optionally RMS-normalised: x * (1/sqrt(mean(x^2)+eps)) * w, two
// roundings per element as in norm.cpp:122-127) into LDS.
__device__ inline void stage_x(const GemvArgs& a, float* xsm, float* red) {
  // Loads are issued in unrolled batches of 8 float4 per thread so a block pays
  // one memory round trip per batch (a plain strided loop serialises them).
  constexpr int B = 8;
  const int tid = threadIdx.x, nt = blockDim.x;
  const int nv = (int)(a.K / 4);
  const float4* x4 = reinterpret_cast<const float4*>(a.x);
  const float4* w4 = reinterpret_cast<const float4*>(a.norm_w);
  float4* s4 = reinterpret_cast<float4*>(xsm);
  const bool tap = a.xtap && blockIdx.x == 0;
  const bool norm = a.norm_w != nullptr;
  const bool w_in_regs = norm && nv <= B * nt;
  float4 wr[B];
  float ss = 0.0f;
  for (int base = 0; base < nv; base += B * nt) {
    float4 xr[B];
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const int i = base + j * nt + tid;
      if (i < nv) {
        xr[j] = x4[i];
        if (w_in_regs) wr[j] = w4[i];
      }
    }
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const int i = base + j * nt + tid;
      if (i < nv) {
        const float4 v = xr[j];
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        if (!w_in_regs) {
          s4[i] = v;
          if (!norm && tap) reinterpret_cast<float4*>(a.xtap)[i] = v;
        } else {
          xr[j] = v;  // kept for the normalisation below
        }
      }
    }
    if (w_in_regs) {
      // single batch: finish the norm from registers after the reduction
      ss = wave_sum(ss);
      if ((tid & 63) == 0) red[tid >> 6] = ss;
      __syncthreads();
      float tot = 0.0f;
      for (int k = 0; k < (nt >> 6); ++k) tot += red[k];
      const float inv = 1.0f / sqrtf(tot / (float)a.K + a.eps);
#pragma unroll
      for (int j = 0; j < B; ++j) {
        const int i = base + j * nt + tid;
        if (i < nv) {
          float4 v = xr[j];
          const float4 w = wr[j];
          v.x = fmul_rn(fmul_rn(v.x, inv), w.x);
          v.y = fmul_rn(fmul_rn(v.y, inv), w.y);
          v.z = fmul_rn(fmul_rn(v.z, inv), w.z);
          v.w = fmul_rn(fmul_rn(v.w, inv), w.w);
          s4[i] = v;
          if (tap) reinterpret_cast<float4*>(a.xtap)[i] = v;
        }
      }
      __syncthreads();
      return;
    }
  }
  if (!norm) {
    __syncthreads();
    return;
  }
  // RMSNorm with K > 8 * 4 * blockDim: second pass over LDS with batched weight loads
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.0f;
  for (int k = 0; k < (nt >> 6); ++k) tot += red[k];
  const float inv = 1.0f / sqrtf(tot / (float)a.K + a.eps);
  for (int base = 0; base < nv; base += B * nt) {
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const int i = base + j * nt + tid;
      if (i < nv) wr[j] = w4[i];
    }
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const int i = base + j * nt + tid;
      if (i < nv) {
        float4 v = s4[i];
        const float4 w = wr[j];
        v.x = fmul_rn(fmul_rn(v.x, inv), w.x);
        v.y = fmul_rn(fmul_rn(v.y, inv), w.y);
        v.z = fmul_rn(fmul_rn(v.z, inv), w.z);
        v.w = fmul_rn(fmul_rn(v.w, inv), w.w);
        s4[i] = v;
        if (tap) reinterpret_cast<float4*>(a.xtap)[i] = v;
      }
    }
  }
  __syncthreads();
}

// ---- epilogues ----------------------------------------------------------------------

// Logical row L of a QKV segment -> physical row (RoPE pairs adjacent in L).
__device__ inline int64_t qkv_phys(int64_t L, int mode, int hd) {
  if (mode != 2) return L;
  const int64_t P = L >> 1;
  const int64_t h = P / (hd / 2), p = P % (hd / 2);
  return h * hd + p + (L & 1) * (hd / 2);
}

template <int FMT, int EPI>
__global__ void __launch_bounds__(WPB * 64) k_gemv(GemvArgs a) {
  extern __shared__ float xsm[];
  __shared__ float red[WPB];
  __shared__ float bval[WPB];
  __shared__ int32_t bidx[WPB];

  // segment lookup (uniform per block)
  int si = 0;
  for (int k = 1; k < a.nseg; ++k) if ((int)blockIdx.x >= a.seg[k].block0) si = k;
  const GemvSeg& seg = a.seg[si];
  const int nblk = (si + 1 < a.nseg ? a.seg[si + 1].block0 : (int)gridDim.x) - seg.block0;
  const int64_t ngroups = (seg.rows + WPB * RPW - 1) / (WPB * RPW);

  stage_x(a, xsm, red);

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  float best_v = -INFINITY;
  int32_t best_i = 0x7fffffff;

  // persistent loop: this block takes row groups blk, blk + nblk, ...
  for (int64_t grp = blockIdx.x - seg.block0; grp < ngroups; grp += nblk) {
    const int64_t lrow0 = (grp * WPB + wave) * RPW;
    RowPtr P[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      int64_t l = lrow0 + r;
      if (l >= seg.rows) l = seg.rows - 1;  // clamp: duplicate work, result dropped
      if constexpr (EPI == EPI_SWIGLU) {
        P[r] = row_ptr((l & 1) ? seg.w2 : seg.w, l >> 1);
      } else if constexpr (EPI == EPI_QKV) {
        P[r] = row_ptr(seg.w, seg.kind == 2 ? l : qkv_phys(l, a.rope_mode, a.head_dim));
      } else {
        P[r] = row_ptr(seg.w, l);
      }
    }
    float acc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;
    rows_dot<FMT>(P, seg.w.a_row / 16, xsm, lane, acc);
#pragma unroll
    for (int r = 0; r < RPW; ++r) acc[r] = wave_sum(acc[r]);

    if constexpr (EPI == EPI_STORE || EPI == EPI_ADD || EPI == EPI_LOGITS) {
      if (lane < RPW) {
        float v = 0.0f;
#pragma unroll
        for (int r = 0; r < RPW; ++r) if (r == lane) v = acc[r];
        const int64_t l = lrow0 + lane;
        if (l < seg.rows) {
          const int64_t o = seg.row_base + l;
          if constexpr (EPI == EPI_ADD) v = a.y[o] + v;
          a.y[o] = v;
          if (a.tap) a.tap[o] = v;
        }
      }
      if constexpr (EPI == EPI_LOGITS) {
        // running greedy argmax of this wave (rows ascend, strict '>' keeps the lowest)
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
          const int64_t l = lrow0 + r;
          if (l < seg.rows && (best_i == 0x7fffffff || acc[r] > best_v)) { best_v = acc[r]; best_i = (int32_t)l; }
        }
      }
    } else if constexpr (EPI == EPI_SWIGLU) {
      // pairs (gate, up) at logical rows (2j, 2j+1)
      if (lane < RPW / 2) {
        float g = 0.0f, u = 0.0f;
#pragma unroll
        for (int r = 0; r < RPW; r += 2) if (r == 2 * lane) { g = acc[r]; u = acc[r + 1]; }
        const int64_t l = lrow0 + 2 * lane;
        if (l < seg.rows) {
          const float act = g / (1.0f + expf(-g));  // silu (elementwise.cpp:73-84)
          a.y[seg.row_base + (l >> 1)] = act * u;
        }
      }
    } else if constexpr (EPI == EPI_QKV) {
      if (lane < RPW / 2) {
        float v0 = 0.0f, v1 = 0.0f;
#pragma unroll
        for (int r = 0; r < RPW; r += 2) if (r == 2 * lane) { v0 = acc[r]; v1 = acc[r + 1]; }
        const int64_t l = lrow0 + 2 * lane;
        if (l < seg.rows) {
          const int64_t r0 = (seg.kind == 2) ? l : qkv_phys(l, a.rope_mode, a.head_dim);
          const int64_t r1 = (seg.kind == 2) ? l + 1 : qkv_phys(l + 1, a.rope_mode, a.head_dim);
          if (seg.bias) { v0 = v0 + seg.bias[r0]; v1 = v1 + seg.bias[r1]; }
          const int pos = a.state->pos;
          if (seg.kind != 2) {
            // rotate pair p of its head by the host-built angle table
            const int64_t p = (a.rope_mode == 2) ? (r0 % a.head_dim) : ((r0 % a.head_dim) >> 1);
            const float2 cs = a.rope[(int64_t)pos * (a.head_dim / 2) + p];
            const float n0 = v0 * cs.x - v1 * cs.y;
            const float n1 = v0 * cs.y + v1 * cs.x;
            v0 = n0; v1 = n1;
          }
          if (seg.kind == 0) {
            a.y[r0] = v0;
            a.y[r1] = v1;
          } else {
            // K after RoPE and raw V go to the cache at `pos` (gguf.cpp:1043, dispatch.cpp:218)
            void* cache = (seg.kind == 1) ? a.kcache : a.vcache;
            const int64_t hd = a.head_dim;
            const int64_t o0 = ((r0 / hd) * a.max_seq + pos) * hd + (r0 % hd);
            const int64_t o1 = ((r1 / hd) * a.max_seq + pos) * hd + (r1 % hd);
            if (a.kv_f16) {
              reinterpret_cast<__half*>(cache)[o0] = __float2half(v0);
              reinterpret_cast<__half*>(cache)[o1] = __float2half(v1);
            } else {
              reinterpret_cast<float*>(cache)[o0] = v0;
              reinterpret_cast<float*>(cache)[o1] = v1;
            }
          }
        }
      }
    }
  }

  if constexpr (EPI == EPI_LOGITS) {
    // block partial of the greedy argmax; k_argmax_final reduces the partials
    if (lane == 0) { bval[wave] = best_v; bidx[wave] = best_i; }
    __syncthreads();
    if (threadIdx.x == 0) {
      float bv = bval[0];
      int32_t bi = bidx[0];
      for (int k = 1; k < WPB; ++k) {
        if (bidx[k] == 0x7fffffff) continue;
        if (bi == 0x7fffffff || bval[k] > bv || (bval[k] == bv && bidx[k] < bi)) { bv = bval[k]; bi = bidx[k]; }
      }
      a.part_val[blockIdx.x] = bv;
      a.part_idx[blockIdx.x] = bi;
    }
  }
}

// Final greedy argmax over the LM-head block partials (lowest index wins ties,
// sampling.cpp:38-50), then the token advance: inside the prompt the next token
// is the prompt's, afterwards the argmax (session.cpp:1006-1044).
__global__ void __launch_bounds__(1024) k_argmax_final(GemvArgs a, int nparts) {
  __shared__ float fv[16], f2[16];
  __shared__ int32_t fi[16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float bv = -INFINITY, b2 = -INFINITY;
  int32_t bi = 0x7fffffff;
  for (int k = threadIdx.x; k < nparts; k += blockDim.x) {
    const float v = a.part_val[k];
    const int32_t ix = a.part_idx[k];
    if (ix == 0x7fffffff) continue;
    if (bi == 0x7fffffff || v > bv || (v == bv && ix < bi)) { b2 = fmaxf(b2, bv); bv = v; bi = ix; }
    else b2 = fmaxf(b2, v);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int32_t oi = __shfl_xor(bi, o, 64);
    const float o2 = __shfl_xor(b2, o, 64);
    if (oi != 0x7fffffff && (bi == 0x7fffffff || ov > bv || (ov == bv && oi < bi))) {
      b2 = fmaxf(fmaxf(b2, o2), bv); bv = ov; bi = oi;
    } else {
      b2 = fmaxf(fmaxf(b2, o2), ov);
    }
  }
  if (lane == 0) { fv[wave] = bv; fi[wave] = bi; f2[wave] = b2; }
  __syncthreads();
  if (threadIdx.x == 0) {
    float v = fv[0], s2 = f2[0];
    int32_t ix = fi[0];
    for (int k = 1; k < (int)(blockDim.x >> 6); ++k) {
      if (fi[k] != 0x7fffffff && (ix == 0x7fffffff || fv[k] > v || (fv[k] == v && fi[k] < ix))) {
        s2 = fmaxf(fmaxf(s2, f2[k]), v); v = fv[k]; ix = fi[k];
      } else {
        s2 = fmaxf(fmaxf(s2, f2[k]), fv[k]);
      }
    }
    StepState* st = a.state;
    st->argmax = ix;
    st->max_logit = v;
    st->second = s2;
    const int p = st->pos + 1;
    const int next = (p < st->n_prompt) ? a.ids[p] : ix;
    a.ids[p] = next;
    st->token = next;
    st->pos = p;
  }
}

using KernelFn = void (*)(GemvArgs);

template <int EPI>
KernelFn pick_fmt(int type) {
  switch (type) {
    case T_Q4_0: return k_gemv<T_Q4_0, EPI>;
    case T_Q8_0: return k_gemv<T_Q8_0, EPI>;
    case T_Q4_K: return k_gemv<T_Q4_K, EPI>;
    case T_Q6_K: return k_gemv<T_Q6_K, EPI>;
    case T_Q4_1: return k_gemv<T_Q4_1, EPI>;
    case T_Q5_0: return k_gemv<T_Q5_0, EPI>;
    case T_Q5_1: return k_gemv<T_Q5_1, EPI>;
    case T_Q5_K: return k_gemv<T_Q5_K, EPI>;
    case T_Q2_K: return k_gemv<T_Q2_K, EPI>;
    case T_Q3_K: return k_gemv<T_Q3_K, EPI>;
    case T_F32: return k_gemv<T_F32, EPI>;
    case T_F16: return k_gemv<T_F16, EPI>;
    default: return nullptr;
  }
}

KernelFn pick(int epi, int type) {
  switch (epi) {
    case EPI_STORE: return pick_fmt<EPI_STORE>(type);
    case EPI_ADD: return pick_fmt<EPI_ADD>(type);
    case EPI_QKV: return pick_fmt<EPI_QKV>(type);
    case EPI_SWIGLU: return pick_fmt<EPI_SWIGLU>(type);
    case EPI_LOGITS: return pick_fmt<EPI_LOGITS>(type);
    default: return nullptr;
  }
}

}  // namespace

// Raise each instantiation's dynamic-LDS limit to what the device allows per
// block (where the runtime accepts the attribute; otherwise its default holds).
hipError_t prepare_gemv() {
  const int epis[] = {EPI_STORE, EPI_ADD, EPI_QKV, EPI_SWIGLU, EPI_LOGITS};
  const int types[] = {T_Q4_0, T_Q8_0, T_Q4_K, T_Q6_K, T_Q4_1, T_Q5_0,
                       T_Q5_1, T_Q5_K, T_Q2_K, T_Q3_K, T_F32,  T_F16};
  const int lim = lds_limit();
  for (int e : epis) {
    for (int t : types) {
      (void)hipFuncSetAttribute((const void*)pick(e, t), hipFuncAttributeMaxDynamicSharedMemorySize,
                                lim - 1024);
      (void)hipGetLastError();
    }
  }
  return hipSuccess;
}

int cu_count() {
  static int n = 0;
  if (n == 0) {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
      n = v;
    else
      n = 256;
  }
  return n;
}

// Blocks per segment: one per row group, capped so a launch holds at most
// kBlocksPerCU blocks per CU in total (the rest loop), shared out by group count.
constexpr int kBlocksPerCU = 4;

void plan_blocks(const GemvArgs& a, int* per_seg) {
  const int rpb = WPB * RPW;
  int64_t total = 0;
  for (int k = 0; k < a.nseg; ++k) total += (a.seg[k].rows + rpb - 1) / rpb;
  const int64_t cap = (int64_t)cu_count() * kBlocksPerCU;
  for (int k = 0; k < a.nseg; ++k) {
    const int64_t g = (a.seg[k].rows + rpb - 1) / rpb;
    int64_t b = g;
    if (total > cap) {
      b = std::max<int64_t>(1, (g * cap + total - 1) / total);
      const int64_t per = (g + b - 1) / b;  // groups per block, then even out the blocks
      b = (g + per - 1) / per;
    }
    per_seg[k] = (int)std::min<int64_t>(b, g);
  }
}

int gemv_grid(const GemvArgs& a) {
  int per[3] = {0, 0, 0};
  plan_blocks(a, per);
  int blocks = 0;
  for (int k = 0; k < a.nseg; ++k) blocks += per[k];
  return blocks;
}

// One launch per run of segments sharing a weight type (the kernel is
// specialised per type); QKV with mixed types therefore takes several launches.
hipError_t launch_gemv(const GemvArgs& in, hipStream_t s) {
  const size_t lds = (size_t)in.K * sizeof(float);
  if ((int)lds > lds_limit() - 1024 || in.K % 4) return hipErrorInvalidValue;
  if (in.epi == EPI_LOGITS && in.nseg != 1) return hipErrorInvalidValue;
  for (int k = 0; k < in.nseg; ++k) {
    if (in.epi == EPI_SWIGLU && in.seg[k].w2.type != in.seg[k].w.type) return hipErrorInvalidValue;
    if ((in.epi == EPI_SWIGLU || in.epi == EPI_QKV) && (in.seg[k].rows % 2)) return hipErrorInvalidValue;
    if (in.seg[k].w.cols != in.K) return hipErrorInvalidValue;
  }
  int k0 = 0;
  while (k0 < in.nseg) {
    int k1 = k0 + 1;
    while (k1 < in.nseg && in.seg[k1].w.type == in.seg[k0].w.type) ++k1;
    GemvArgs a = in;
    a.nseg = k1 - k0;
    for (int k = 0; k < a.nseg; ++k) a.seg[k] = in.seg[k0 + k];
    int per[3] = {0, 0, 0};
    plan_blocks(a, per);
    int blocks = 0;
    for (int k = 0; k < a.nseg; ++k) {
      a.seg[k].block0 = blocks;
      blocks += per[k];
    }
    if (k0 > 0) a.xtap = nullptr;
    KernelFn fn = pick(a.epi, a.seg[0].w.type);
    if (!fn) return hipErrorInvalidValue;
    if (blocks > 0) {
      hipLaunchKernelGGL(fn, dim3(blocks), dim3(WPB * 64), lds, s, a);
      const hipError_t st = hipGetLastError();
      if (st != hipSuccess) return st;
      if (a.epi == EPI_LOGITS) {
        hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(1024), 0, s, a, blocks);
        const hipError_t st2 = hipGetLastError();
        if (st2 != hipSuccess) return st2;
      }
    }
    k0 = k1;
  }
  return hipSuccess;
}

}  // namespace uaii_hip
