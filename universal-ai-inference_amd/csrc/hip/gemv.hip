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
// l, l+64, ... . The input vector is staged once per block in LDS (after the
// optional RMSNorm): as f32, or for the f16-pair formats (Q4_0, Q4_1, Q4_K,
// Q6_K) as f16 hi/lo pairs in the order the nibble masks produce, with a
// power-of-two scale per chunk. Each lane reads the x values of its chunk once and
// reuses them for all RPW rows, and the per-chunk sum of x folds the
// quantization offsets/mins out of the inner loop. Partial dots are reduced with
// 64-lane xor shuffles (DPP on CDNA4).

#include "common.h"
#include "uaii_hip_internal.h"

#include <algorithm>
#include <mutex>
#include <vector>

namespace uaii_hip {
namespace {

// Tuning knobs (compile-time): resident-block cap per CU for the persistent
// grid (0 = the runtime's occupancy figure) and the number of units whose
// weight loads are issued together (1 or 2).
#ifndef UAII_GEMV_BLOCKS_PER_CU
#define UAII_GEMV_BLOCKS_PER_CU 0
#endif
#ifndef UAII_GEMV_BATCH
#define UAII_GEMV_BATCH 1
#endif


// Waves per block (measured per role on the 8B decode step): 4 in general; 8 for
// the QKV epilogue (6144 rows of K = 4096: more row sets share one staged
// input); 16 for the K-split long rows of the residual-add GEMV (the down
// projection, whose staged input is as large as a 4-wave block's weight bytes).
constexpr int WPB = 4;
#ifndef UAII_WPB_QKV
#define UAII_WPB_QKV 8
#endif
#ifndef UAII_WPB_SWIGLU
#define UAII_WPB_SWIGLU 4
#endif
constexpr int WPB_QKV = UAII_WPB_QKV;
constexpr int WPB_SWIGLU = UAII_WPB_SWIGLU;
constexpr int WPB_LONG = 16;
constexpr int NB = UAII_GEMV_BATCH;
static_assert(NB == 1 || NB == 2, "UAII_GEMV_BATCH must be 1 or 2");
constexpr int RPW_MAX = 4;  // rows per wave (even: RoPE / SwiGLU pairs share a wave)

// Rows per wave by format: the K-quants carry more side data per chunk, so they
// take two rows per wave to stay within 128 VGPRs.
__host__ __device__ constexpr int rpw_of(int fmt) {
  return (fmt == T_Q2_K || fmt == T_Q3_K || fmt == T_Q4_K || fmt == T_Q5_K || fmt == T_Q6_K) ? 2 : 4;
}

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

// Raw per-row data of one chunk (only the fields a format uses stay live). Only
// bits are loaded here; every conversion happens where the chunk is decoded, so
// a unit's loads issue back to back with nothing waiting on them.
struct Raw {
  uint4 q;     // 16 payload bytes
  uint4 aux;   // side data (format specific)
  uint4 aux2;  // Q5_K qh, Q3_K hmask; Q6_K: the 8 scale bytes of the half block
  uint32_t s;  // f16 scale bits: d in the low half, m / dmin in the high half
};

__device__ inline float byte_f(uint32_t w, int k) { return (float)((w >> (8 * k)) & 0xffu); }
__device__ inline float lo_h(uint32_t s) { return h2f((uint16_t)(s & 0xffffu)); }
__device__ inline float hi_h(uint32_t s) { return h2f((uint16_t)(s >> 16)); }

template <int FMT>
__device__ inline void load_raw(const RowPtr& p, int64_t t, Raw& o) {
  o.q = *reinterpret_cast<const uint4*>(p.a + t * 16);
  if constexpr (FMT == T_Q4_0) {
    o.s = ld_u16(p.b + t * 2);
  } else if constexpr (FMT == T_Q8_0) {
    o.s = ld_u16(p.b + (t >> 1) * 2);
  } else if constexpr (FMT == T_Q4_1) {
    o.s = *reinterpret_cast<const uint32_t*>(p.b + t * 4);
  } else if constexpr (FMT == T_Q5_0) {
    o.aux.x = *reinterpret_cast<const uint32_t*>(p.b + t * 4);
    o.s = ld_u16(p.c + t * 2);
  } else if constexpr (FMT == T_Q5_1) {
    o.aux.x = *reinterpret_cast<const uint32_t*>(p.b + t * 4);
    o.s = *reinterpret_cast<const uint32_t*>(p.c + t * 4);
  } else if constexpr (FMT == T_Q4_K || FMT == T_Q5_K) {
    o.aux = *reinterpret_cast<const uint4*>(p.b + (t >> 3) * 16);
    if constexpr (FMT == T_Q5_K) {
      // the 16 qh bytes covering this chunk's lanes l = 16*(t&1) + i
      o.aux2 = *reinterpret_cast<const uint4*>(p.c + (t >> 3) * 32 + 16 * (t & 1));
    }
  } else if constexpr (FMT == T_Q6_K) {
    const int64_t sb = t >> 3; const int h = (int)((t & 7) >> 2), u = (int)(t & 3);
    o.aux = *reinterpret_cast<const uint4*>(p.b + sb * 64 + h * 32 + 16 * (u & 1));
    const uint2 sc = *reinterpret_cast<const uint2*>(p.c + sb * 16 + h * 8);
    o.aux2.x = sc.x; o.aux2.y = sc.y;
    o.s = ld_u16(p.d + sb * 2);
  } else if constexpr (FMT == T_Q2_K) {
    o.aux = *reinterpret_cast<const uint4*>(p.b + (t >> 2) * 16);  // scales
    o.s = *reinterpret_cast<const uint32_t*>(p.c + (t >> 2) * 4);
  } else if constexpr (FMT == T_Q3_K) {
    o.aux = *reinterpret_cast<const uint4*>(p.c + (t >> 2) * 16);  // scales12, d
    o.aux2 = *reinterpret_cast<const uint4*>(p.b + (t >> 2) * 32 + 16 * (t & 1));
  }
}

// Per-chunk float scales from the raw bits: s0 = d (Q6_K: d * scale of the
// chunk's low run), s1 = m / dmin (Q6_K: d * scale of the high run).
template <int FMT>
__device__ inline void raw_scales(const Raw& o, int64_t t, float& s0, float& s1) {
  s0 = 0.0f;
  s1 = 0.0f;
  if constexpr (FMT == T_Q4_0 || FMT == T_Q8_0 || FMT == T_Q5_0) {
    s0 = lo_h(o.s);
  } else if constexpr (FMT == T_Q4_1 || FMT == T_Q5_1 || FMT == T_Q2_K) {
    s0 = lo_h(o.s);
    s1 = hi_h(o.s);
  } else if constexpr (FMT == T_Q6_K) {
    const int u = (int)(t & 3);
    const float d = lo_h(o.s);
    s0 = d * (float)(int8_t)((o.aux2.x >> (8 * u)) & 0xffu);
    s1 = d * (float)(int8_t)((o.aux2.y >> (8 * u)) & 0xffu);
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
  float s0, s1;
  raw_scales<FMT>(o, t, s0, s1);
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
    if constexpr (FMT == T_Q4_0) return s0 * (s - 8.0f * (xs[0] + xs[1]));
    else return s0 * s + s1 * (xs[0] + xs[1]);
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
    if constexpr (FMT == T_Q5_0) return s0 * (s - 16.0f * (xs[0] + xs[1]));
    else return s0 * s + s1 * (xs[0] + xs[1]);
  } else if constexpr (FMT == T_Q8_0) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t wq = word(o.q, i);
#pragma unroll
      for (int k = 0; k < 4; ++k) s += (float)(int8_t)((wq >> (8 * k)) & 0xffu) * xv[4 * i + k];
    }
    return s0 * s;
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
    return s0 * (slo - 32.0f * xs[0]) + s1 * (shi - 32.0f * xs[1]);
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
      tot += (s0 * (float)(s & 15)) * sq - (s1 * (float)(s >> 4)) * xs[p];
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

// The staged input lives in LDS as planes: plane g holds the g-th float4 of
// every chunk's x values, indexed by chunk. The 64 lanes of a wave work on 64
// consecutive chunks, so each plane read is 64 consecutive float4 (no bank
// conflicts), where a chunk-contiguous layout would put every lane on the same
// banks.
template <int FMT>
constexpr int xgroups() { return xn<FMT>() / 4; }

// float4 index i of the input (elements 4i..4i+3) -> (chunk t, plane g); the
// inverse of x_runs: plane g is float4 (g % 4) of run g / 4.
template <int FMT>
__device__ inline void plane_of(int64_t i, int64_t& t, int& g) {
  if constexpr (FMT == T_Q4_0 || FMT == T_Q4_1 || FMT == T_Q5_0 || FMT == T_Q5_1) {
    t = i >> 3; g = (int)(i & 7);
  } else if constexpr (FMT == T_Q8_0) {
    t = i >> 2; g = (int)(i & 3);
  } else if constexpr (FMT == T_Q4_K || FMT == T_Q5_K) {
    // i = 64 sb + 16 cc + 8 rr + 4 hh + k
    const int64_t sb = i >> 6; const int r = (int)(i & 63);
    t = 8 * sb + 2 * (r >> 4) + ((r >> 2) & 1); g = 4 * ((r >> 3) & 1) + (r & 3);
  } else if constexpr (FMT == T_Q6_K) {
    // i = 64 sb + 32 h + 16 rr + 4 u + k
    const int64_t sb = i >> 6; const int r = (int)(i & 63);
    t = 8 * sb + 4 * (r >> 5) + ((r >> 2) & 3); g = 4 * ((r >> 4) & 1) + (r & 3);
  } else if constexpr (FMT == T_Q2_K || FMT == T_Q3_K) {
    // i = 64 sb + 32 h + 8 p + 4 g' + k
    const int64_t sb = i >> 6; const int r = (int)(i & 63);
    t = 4 * sb + 2 * (r >> 5) + ((r >> 2) & 1); g = 4 * ((r >> 3) & 3) + (r & 3);
  } else if constexpr (FMT == T_F16) {
    t = i >> 1; g = (int)(i & 1);
  } else {
    t = i; g = 0;
  }
}

template <int FMT>
__device__ inline int64_t plane_index(int64_t i, int64_t nch) {
  int64_t t;
  int g;
  plane_of<FMT>(i, t, g);
  return (int64_t)g * nch + t;
}

// x values of chunk t (runs back to back, 16 each) and the per-run sums.
template <int FMT>
__device__ inline void load_x(const float* __restrict__ xsm, int64_t nch, int64_t t, float* xv,
                              float* xsum) {
  const float4* pl = reinterpret_cast<const float4*>(xsm);
#pragma unroll
  for (int rr = 0; rr < (xgroups<FMT>() + 3) / 4; ++rr) {
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int g = 4 * rr + k;
      if (g < xgroups<FMT>()) {
        const float4 v = pl[(int64_t)g * nch + t];
        xv[4 * g + 0] = v.x; xv[4 * g + 1] = v.y;
        xv[4 * g + 2] = v.z; xv[4 * g + 3] = v.w;
        s += (v.x + v.y) + (v.z + v.w);
      }
    }
    xsum[rr] = s;
  }
}

// Logical row L of a QKV segment -> physical row (RoPE pairs adjacent in L).
__device__ inline int64_t qkv_phys(int64_t L, int mode, int hd) {
  if (mode != 2) return L;
  const int64_t P = L >> 1;
  const int64_t h = P / (hd / 2), p = P % (hd / 2);
  return h * hd + p + (L & 1) * (hd / 2);
}

// ---- f16-pair dot for the 4-bit and 6-bit formats (Q4_0, Q4_1, Q4_K, Q6_K) --------
//
// The dot runs on v_dot2_f32_f16. A payload word q (bytes 4i..4i+3 of a chunk)
// gives four f16 pairs by masking alone: q & 0x000F000F holds the low nibbles of
// bytes 0 and 2 as the subnormal halves n * 2^-24 (exact), q & 0x00F000F0 their
// high nibbles as n * 2^-20, and the same masks on q >> 8 give bytes 1 and 3.
// For Q6_K the two high bits of each 6-bit value are OR-ed in above the nibble
// (bits 4-5 of a low-nibble half, bits 8-9 of a high-nibble half), still an
// exact subnormal. Every chunk covers two runs of 16 inputs, run 0 against the
// low nibbles and run 1 against the high nibbles. The input is scaled per chunk
// by a power of two S (the chunk's largest |x| * S in [2^14, 2^15); run 1 by
// S / 16) and split into f16 hi (on a grid of 2^-10 of the chunk's largest
// value) + lo (the rest), so every x keeps about 22 significant bits relative
// to its chunk; both products per element are exact, the hi sums are exact in
// f32 and the lo sums round. A run's sum of n * x is then (acc_hi + acc_lo) * c
// with c = 2^24 / S.
//
// LDS: 8 uint4 planes indexed by chunk (word i: plane 2i = hi pairs, 2i+1 = lo
// pairs, in the order (r0[4i], r0[4i+2]), (r1[4i], r1[4i+2]) / 16,
// (r0[4i+1], r0[4i+3]), (r1[4i+1], r1[4i+3]) / 16 for runs r0, r1), then the
// chunk's side data: float2 (sum of both runs' unscaled inputs, c) for the
// single-scale formats, float4 (sum of run 0, sum of run 1, c, 0) for the
// K-quants, whose two runs carry their own scales.

#ifndef UAII_GEMV_KPAIR
#define UAII_GEMV_KPAIR 1  // 0: Q4_K / Q6_K on the f32 cvt + FMA path
#endif

typedef _Float16 h2v __attribute__((ext_vector_type(2)));

template <int FMT>
__host__ __device__ constexpr bool pair_fmt() {
  return FMT == T_Q4_0 || FMT == T_Q4_1 || (UAII_GEMV_KPAIR && (FMT == T_Q4_K || FMT == T_Q6_K));
}

// f32 slots of side data per chunk in the LDS staging.
template <int FMT>
__host__ __device__ constexpr int pair_side() { return (FMT == T_Q4_0 || FMT == T_Q4_1) ? 2 : 4; }

// float4 index of run 0 of chunk t in the input (x_runs in float4 units) and
// the float4 offset of run 1 from it.
template <int FMT>
__device__ inline int64_t pair_run0(int64_t t) {
  if constexpr (FMT == T_Q4_K) return 64 * (t >> 3) + 16 * ((t & 7) >> 1) + 4 * (t & 1);
  else if constexpr (FMT == T_Q6_K) return 64 * (t >> 3) + 32 * ((t & 7) >> 2) + 4 * (t & 3);
  else return 8 * t;
}
template <int FMT>
__host__ __device__ constexpr int pair_run1() { return FMT == T_Q4_K ? 8 : (FMT == T_Q6_K ? 16 : 4); }

__device__ inline float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2v, a), __builtin_bit_cast(h2v, b), c, false);
}

// 2^k for -126 <= k <= 127
__device__ inline float pow2f(int k) { return __uint_as_float((uint32_t)(k + 127) << 23); }

__device__ inline uint32_t hbits(_Float16 h) { return (uint32_t)__builtin_bit_cast(uint16_t, h); }

// (a, b) -> f16 pairs hi = (A, B), lo = (f16(a - A), f16(b - B)) with A, B the
// nearest multiples of the grid G. The callers pass G = |max| * 2^-10
// (rounded down to a power of two), so |A| / g <= 2048 is exact in f16, and every
// partial sum of nibble * hi products over a chunk is a multiple of g * 2^-24
// below 2^24 of them: exact in f32, whatever rounding v_dot2_f32_f16 applies to
// its accumulator. (With hi = f16(a) those sums round, and the accumulator's
// rounding was measured to bias them downward: on positive-scale formats such
// as Q4_K a row-wide offset of ~3e-5 relative.) Only the lo sums, ~2^-11 of the
// total, round.
template <int G>
__device__ inline float grid_round(float a) {
  static_assert(G == 1 || G == 16, "grid 1 or 16");
  if constexpr (G == 1) return rintf(a);
  // nearest multiple of 16 for |a| < 2^26: the ulp of 1.5 * 2^27 is 16
  else return (a + 201326592.0f) - 201326592.0f;
}

template <int G>
__device__ inline void split2(float a, float b, uint32_t& hi, uint32_t& lo) {
  const float ar = grid_round<G>(a), br = grid_round<G>(b);
  const _Float16 ah = (_Float16)ar, bh = (_Float16)br;
  const _Float16 al = (_Float16)(a - ar), bl = (_Float16)(b - br);
  hi = hbits(ah) | (hbits(bh) << 16);
  lo = hbits(al) | (hbits(bl) << 16);
}

// The chunk's x pairs and side data: xc = (sum of both runs, -, c, -) for the
// single-scale formats, (sum of run 0, sum of run 1, c, -) for the K-quants.
template <int FMT>
__device__ inline void load_xpairs(const float* __restrict__ xsm, int64_t nch, int64_t t, uint4* xp,
                                   float4& xc) {
  const uint4* pl = reinterpret_cast<const uint4*>(xsm);
#pragma unroll
  for (int g = 0; g < 8; ++g) xp[g] = pl[(int64_t)g * nch + t];
  if constexpr (pair_side<FMT>() == 2) {
    const float2 v = reinterpret_cast<const float2*>(pl + 8 * nch)[t];
    xc = make_float4(v.x, 0.0f, v.y, 0.0f);
  } else {
    xc = reinterpret_cast<const float4*>(pl + 8 * nch)[t];
  }
}

// Q4_K (scale, min) 6-bit pairs of sub-blocks 2cc and 2cc + 1 (kscale_reg for
// j = 2cc, 2cc + 1 on whole words): sc / mn hold the two scales / mins in bytes
// 0 and 1.
__device__ inline void kscale_pair(int cc, const uint4& meta, uint32_t& sc, uint32_t& mn) {
  const int sh = 16 * (cc & 1);
  const uint32_t a = meta.y >> sh, b = meta.z >> sh, c = meta.w >> sh;
  if (cc < 2) {
    sc = a & 0x3f3fu;
    mn = b & 0x3f3fu;
  } else {
    sc = (c & 0x0f0fu) | ((a >> 2) & 0x3030u);
    mn = ((c >> 4) & 0x0f0fu) | ((b >> 2) & 0x3030u);
  }
}

template <int FMT>
__device__ inline float chunk_dot_pairs(const Raw& o, int64_t t, const uint4* xp, float4 xc) {
  const float c = xc.z;
  if constexpr (FMT == T_Q4_0 || FMT == T_Q4_1) {
    float sh = 0.0f, sl = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t q = word(o.q, i), q8 = q >> 8;
      const uint32_t p0 = q & 0x000F000Fu, p1 = q & 0x00F000F0u;
      const uint32_t p2 = q8 & 0x000F000Fu, p3 = q8 & 0x00F000F0u;
      const uint4 H = xp[2 * i], L = xp[2 * i + 1];
      sh = dot2(p0, H.x, sh); sl = dot2(p0, L.x, sl);
      sh = dot2(p1, H.y, sh); sl = dot2(p1, L.y, sl);
      sh = dot2(p2, H.z, sh); sl = dot2(p2, L.z, sl);
      sh = dot2(p3, H.w, sh); sl = dot2(p3, L.w, sl);
    }
    const float s = (sh + sl) * c;  // sum of n * x
    if constexpr (FMT == T_Q4_0) return lo_h(o.s) * (s - 8.0f * xc.x);
    else return lo_h(o.s) * s + hi_h(o.s) * xc.x;
  } else {
    // K-quants: run 0 (low nibbles) and run 1 (high nibbles) summed apart, hi
    // and lo parts in their own accumulators (the hi sums stay exact)
    float s0 = 0.0f, s1 = 0.0f, l0 = 0.0f, l1 = 0.0f;
    const int qsh = 2 * (int)((t & 3) >> 1);  // Q6_K: qh bit pair of the chunk's runs
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t q = word(o.q, i), q8 = q >> 8;
      uint32_t p0 = q & 0x000F000Fu, p1 = q & 0x00F000F0u;
      uint32_t p2 = q8 & 0x000F000Fu, p3 = q8 & 0x00F000F0u;
      if constexpr (FMT == T_Q6_K) {
        // bits qsh, qsh+1 (run 0) and qsh+4, qsh+5 (run 1) of each qh byte to
        // bits 4-5 and 8-9 of its f16 half
        const uint32_t h = word(o.aux, i);
        const uint32_t hs = h << (4 - qsh), h8 = h >> (4 + qsh);
        p0 |= hs & 0x00300030u; p1 |= hs & 0x03000300u;
        p2 |= h8 & 0x00300030u; p3 |= h8 & 0x03000300u;
      }
      const uint4 H = xp[2 * i], L = xp[2 * i + 1];
      s0 = dot2(p0, H.x, s0); l0 = dot2(p0, L.x, l0);
      s1 = dot2(p1, H.y, s1); l1 = dot2(p1, L.y, l1);
      s0 = dot2(p2, H.z, s0); l0 = dot2(p2, L.z, l0);
      s1 = dot2(p3, H.w, s1); l1 = dot2(p3, L.w, l1);
    }
    s0 += l0;
    s1 += l1;
    if constexpr (FMT == T_Q4_K) {
      const float d = lo_h(o.aux.x), dmin = hi_h(o.aux.x);
      uint32_t sc, mn;
      kscale_pair((int)((t & 7) >> 1), o.aux, sc, mn);
      const float dc = d * c;
      return (dc * (float)(sc & 0xffu)) * s0 - (dmin * (float)(mn & 0xffu)) * xc.x +
             (dc * (float)(sc >> 8)) * s1 - (dmin * (float)(mn >> 8)) * xc.y;
    } else {
      float a0, a1;
      raw_scales<FMT>(o, t, a0, a1);
      return a0 * (s0 * c - 32.0f * xc.x) + a1 * (s1 * c - 32.0f * xc.y);
    }
  }
}

// ---- walk over row groups ------------------------------------------------------------
//
// A block's WPB waves form WPB/ks row sets of RPW rows; the ks waves of one row set
// split the row's 64-chunk columns between them (ks > 1 for long rows, so a row
// group costs one memory round trip, not several). A wave's work is a sequence of
// units (row group, step); one step covers two chunk columns, i.e. chunks t and
// t + 64 of each of its rows for lane l = t % 64. Units go in batches of NB: the
// loads of a whole batch are issued before any of it is decoded (and the first
// unit's before the input vector is staged), and no loaded data is carried from
// one batch to the next, so the compiler never has to wait to reuse registers.

struct Walk {
  int64_t nch;     // 16-byte chunks per row
  int cbeg, cend;  // this wave's chunk columns [cbeg, cend)
  int steps;       // steps per row group (the same for every wave of the block)
};

struct EpiIn {
  float v0, v1;  // EPI_ADD: residual, expert weight (1 when absent); EPI_QKV: bias pair
  float2 cs;     // EPI_QKV: rotation of the pair
};

template <int FMT>
struct UnitBuf {
  Raw r[2][rpw_of(FMT)];
  EpiIn e;  // the group's epilogue inputs (epi_load)
};

// Wave-uniform row pointers of logical rows l0 .. l0+R-1 of a segment.
// `ebase` is the first physical row of the segment's expert (0 without MoE).
template <int EPI, int R>
__device__ inline void unit_rows(const GemvArgs& a, const GemvSeg& seg, int64_t ebase, int64_t l0,
                                 RowPtr* P) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    int64_t l = l0 + r;
    if (l >= seg.rows) l = seg.rows - 1;  // clamp: duplicate work, result dropped
    if constexpr (EPI == EPI_SWIGLU) {
      P[r] = row_ptr((l & 1) ? seg.w2 : seg.w, ebase + (l >> 1));
    } else if constexpr (EPI == EPI_QKV) {
      P[r] = row_ptr(seg.w, seg.kind == 2 ? l : qkv_phys(l, a.rope_mode, a.head_dim));
    } else {
      P[r] = row_ptr(seg.w, ebase + l);
    }
  }
}

// Global inputs of one row group's epilogue, read by epi_load with the group's
// weights (reading them after the dot would add a dependent round trip to
// memory at the end of every group): EPI_ADD the residual value of this lane's
// row (lanes < R) and the MoE expert weight; EPI_QKV the bias pair and the RoPE
// (cos, sin) of this lane's pair (lanes < R/2). Every load is unconditional
// (clamped rows, a valid stand-in pointer where an input is absent), so the
// compiler's waits for the weight loads stay exact.
template <int EPI, int R>
__device__ inline void epi_load(const GemvArgs& a, const GemvSeg& seg, int64_t lrow0, int lane, int pos, EpiIn& e) {
  if constexpr (EPI == EPI_ADD) {
    const int64_t l = min(lrow0 + min(lane, R - 1), seg.rows - 1);
    e.v0 = a.y[seg.row_base + l];
    const float* sp = seg.scale ? seg.scale : a.y;
    e.v1 = sp[0];
  } else if constexpr (EPI == EPI_QKV) {
    const int64_t l = min(lrow0 + 2 * min(lane, R / 2 - 1), seg.rows - 2);
    const int64_t r0 = (seg.kind == 2) ? l : qkv_phys(l, a.rope_mode, a.head_dim);
    const int64_t r1 = (seg.kind == 2) ? l + 1 : qkv_phys(l + 1, a.rope_mode, a.head_dim);
    const float* bp = seg.bias ? seg.bias : a.y;
    e.v0 = bp[seg.bias ? r0 : 0];
    e.v1 = bp[seg.bias ? r1 : 0];
    const int64_t p = (a.rope_mode == 2) ? (r0 % a.head_dim) : ((r0 % a.head_dim) >> 1);
    e.cs = a.rope[(int64_t)pos * (a.head_dim / 2) + p];
  }
}

// Position of the token being decoded (QKV epilogue only), read once per launch.
template <int EPI>
__device__ inline int epi_pos(const GemvArgs& a) {
  if constexpr (EPI == EPI_QKV) return a.state->pos;
  return 0;
}

template <int FMT, int EPI>
__device__ inline void load_unit(const GemvArgs& a, const GemvSeg& seg, int64_t ebase, const Walk& wk,
                                 int64_t l0, int step, int lane, int pos, UnitBuf<FMT>& U) {
  constexpr int R = rpw_of(FMT);
  RowPtr P[R];
  unit_rows<EPI, R>(a, seg, ebase, l0, P);
  // Straight-line loads: a column past the wave's range, or a lane past the row's
  // last chunk, loads an in-bounds chunk again and compute_unit drops it. (A
  // branch around some of the loads would make the compiler's wait counts
  // conservative at the join and serialise the unit's loads.)
  const int ncol = (int)((wk.nch + 63) / 64);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int col = min(wk.cbeg + 2 * step + j, ncol - 1);
    const int64_t t = min((int64_t)col * 64 + lane, wk.nch - 1);
#pragma unroll
    for (int r = 0; r < R; ++r) load_raw<FMT>(P[r], t, U.r[j][r]);
  }
  epi_load<EPI, R>(a, seg, l0, lane, pos, U.e);
}

template <int FMT>
__device__ inline void compute_unit(const Walk& wk, int step, int lane, const float* xsm,
                                    const UnitBuf<FMT>& U, float* acc) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int col = wk.cbeg + 2 * step + j;  // wave-uniform
    {
      const int64_t t0 = (int64_t)min(col, (int)((wk.nch + 63) / 64) - 1) * 64 + lane;
      const bool ok = col < wk.cend && t0 < wk.nch;
      const int64_t t = t0 < wk.nch ? t0 : wk.nch - 1;
      if constexpr (pair_fmt<FMT>()) {
        uint4 xp[8];
        float4 xc;
        load_xpairs<FMT>(xsm, wk.nch, t, xp, xc);
#pragma unroll
        for (int r = 0; r < rpw_of(FMT); ++r) {
          const float v = chunk_dot_pairs<FMT>(U.r[j][r], t, xp, xc);
          acc[r] += ok ? v : 0.0f;
        }
      } else {
        float xv[xn<FMT>()];
        float xsum[4];
        load_x<FMT>(xsm, wk.nch, t, xv, xsum);
#pragma unroll
        for (int r = 0; r < rpw_of(FMT); ++r) {
          const float v = chunk_dot<FMT>(U.r[j][r], t, xv, xsum);
          acc[r] += ok ? v : 0.0f;
        }
      }
    }
  }
}

// ---- prologue ---------------------------------------------------------------------

// Stage x (optionally RMS-normalised: x * (1/sqrt(mean(x^2)+eps)) * w, two
// roundings per element as in norm.cpp:122-127) into LDS.
template <int FMT, int NT, bool RT>
__device__ inline void stage_x(const GemvArgs& a, const float* xin, int64_t nch, float* xsm, float* red) {
  // Loads are issued in unrolled batches of 4 float4 per thread so a block pays
  // one memory round trip per batch (a plain strided loop serialises them).
  constexpr int B = 4;
  const int tid = threadIdx.x, nt = NT;  // threads per block
  const int nv = (int)(a.K / 4);
  const float4* x4 = reinterpret_cast<const float4*>(xin);
  const float4* w4 = reinterpret_cast<const float4*>(a.norm_w);
  float4* s4 = reinterpret_cast<float4*>(xsm);
  const bool tap = a.xtap && blockIdx.x == 0;
  const bool rtap = RT && a.rtap && blockIdx.x == 0;
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
        if (rtap) reinterpret_cast<float4*>(a.rtap)[i] = v;
        if (!w_in_regs) {
          s4[plane_index<FMT>(i, nch)] = v;
          if (!norm && tap) reinterpret_cast<float4*>(a.xtap)[i] = v;
        } else {
          xr[j] = v;  // kept for the normalisation below
        }
      }
    }
    if (w_in_regs) {
      // single batch: finish the norm from registers after the reduction
      ss = wave_sum_dpp(ss);
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
          s4[plane_index<FMT>(i, nch)] = v;
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
  // RMSNorm with K > 4 * 4 * NT: second pass over LDS with batched weight loads
  ss = wave_sum_dpp(ss);
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
        const int64_t pi = plane_index<FMT>(i, nch);
        float4 v = s4[pi];
        const float4 w = wr[j];
        v.x = fmul_rn(fmul_rn(v.x, inv), w.x);
        v.y = fmul_rn(fmul_rn(v.y, inv), w.y);
        v.z = fmul_rn(fmul_rn(v.z, inv), w.z);
        v.w = fmul_rn(fmul_rn(v.w, inv), w.w);
        s4[pi] = v;
        if (tap) reinterpret_cast<float4*>(a.xtap)[i] = v;
      }
    }
  }
  __syncthreads();
}

// Staging of a pair format. Item (t, w) is float4 w of each of chunk t's two runs
// (x4[pair_run0(t) + w] and x4[pair_run0(t) + pair_run1 + w]); the four items of
// chunk t sit on four consecutive lanes. The first PB items per thread are loaded into registers by
// stage_pairs_issue, before the block's first weight loads, so waiting for them
// never waits for the weights.
constexpr int PB = 4;   // items per thread in the register batch
constexpr int PBW = 2;  // items per thread whose RMSNorm weights ride along

struct PairStage {
  float4 xa[PB], xb[PB];
  float4 wa[PBW], wb[PBW];
};

template <int FMT, int NT>
__device__ inline void stage_pairs_issue(const GemvArgs& a, const float* xin, int64_t nch, PairStage& ps) {
  constexpr int R1 = pair_run1<FMT>();
  const int tid = threadIdx.x, nt = NT;  // threads per block
  const int64_t items = nch * 4;
  const float4* x4 = reinterpret_cast<const float4*>(xin);
  const float4* w4 = reinterpret_cast<const float4*>(a.norm_w);
#pragma unroll
  for (int k = 0; k < PB; ++k) {
    const int64_t it = (int64_t)k * nt + tid;
    if (it < items) {
      const int64_t i0 = pair_run0<FMT>(it >> 2) + (it & 3);
      ps.xa[k] = x4[i0];
      ps.xb[k] = x4[i0 + R1];
    }
  }
  if (w4 && items <= (int64_t)PBW * nt) {
#pragma unroll
    for (int k = 0; k < PBW; ++k) {
      const int64_t it = (int64_t)k * nt + tid;
      if (it < items) {
        const int64_t i0 = pair_run0<FMT>(it >> 2) + (it & 3);
        ps.wa[k] = w4[i0];
        ps.wb[k] = w4[i0 + R1];
      }
    }
  }
}

// One item: RMSNorm (two roundings, norm.cpp:122-127), the optional tap, the
// chunk's power-of-two scale (max over the chunk's four lanes), the hi/lo split
// into the planes, and the chunk's side data from the lane holding word 0.
template <int FMT, bool RT>
__device__ inline void emit_pair_item(const GemvArgs& a, int64_t nch, int64_t it, bool valid, float4 u,
                                      float4 v, float4 uw, float4 vw, bool norm, float inv, bool tap,
                                      bool rtap, float* xsm) {
  const int64_t t = it >> 2;
  const int w = (int)(it & 3);
  if (RT && rtap && valid) {
    const int64_t r0 = pair_run0<FMT>(t) + w;
    reinterpret_cast<float4*>(a.rtap)[r0] = u;
    reinterpret_cast<float4*>(a.rtap)[r0 + pair_run1<FMT>()] = v;
  }
  if (norm) {
    u.x = fmul_rn(fmul_rn(u.x, inv), uw.x); u.y = fmul_rn(fmul_rn(u.y, inv), uw.y);
    u.z = fmul_rn(fmul_rn(u.z, inv), uw.z); u.w = fmul_rn(fmul_rn(u.w, inv), uw.w);
    v.x = fmul_rn(fmul_rn(v.x, inv), vw.x); v.y = fmul_rn(fmul_rn(v.y, inv), vw.y);
    v.z = fmul_rn(fmul_rn(v.z, inv), vw.z); v.w = fmul_rn(fmul_rn(v.w, inv), vw.w);
  }
  constexpr bool two = pair_side<FMT>() == 4;  // the runs' sums kept apart
  float m = 0.0f, pu = 0.0f, pv = 0.0f;
  if (valid) {
    m = fmaxf(fmaxf(fmaxf(fabsf(u.x), fabsf(u.y)), fmaxf(fabsf(u.z), fabsf(u.w))),
              fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    pu = (u.x + u.y) + (u.z + u.w);
    pv = (v.x + v.y) + (v.z + v.w);
    if constexpr (!two) { pu += pv; pv = 0.0f; }
  }
  // the chunk's four lanes (quad xor 1, 2) on DPP moves, not LDS permutes
  m = fmaxf(m, dpp_mov<0xB1>(m));
  m = fmaxf(m, dpp_mov<0x4E>(m));
  pu += dpp_mov<0xB1>(pu);
  pu += dpp_mov<0x4E>(pu);
  if constexpr (two) {
    pv += dpp_mov<0xB1>(pv);
    pv += dpp_mov<0x4E>(pv);
  }
  if (!valid) return;
  const int64_t i0 = pair_run0<FMT>(t) + w;
  if (tap) {
    reinterpret_cast<float4*>(a.xtap)[i0] = u;
    reinterpret_cast<float4*>(a.xtap)[i0 + pair_run1<FMT>()] = v;
  }
  // S = 2^sh with m * S in [2^14, 2^15) (m = m' * 2^e, m' in [0.5, 1), read from
  // the bits; the small margin covers rounding); c = 2^24 / S
  const int e = (int)((__float_as_uint(m * 1.001f) >> 23) & 0xffu) - 126;
  const int sh = (m > 0.0f) ? max(-100, min(100, 15 - e)) : 0;
  const float sl_ = pow2f(sh), sh_ = pow2f(sh - 4);
  uint32_t h0, l0, h1, l1, h2, l2, h3, l3;
  // grids: run 0 scaled below 2^15 -> 16; run 1 (a further / 16) -> 1
  split2<16>(u.x * sl_, u.z * sl_, h0, l0);
  split2<1>(v.x * sh_, v.z * sh_, h1, l1);
  split2<16>(u.y * sl_, u.w * sl_, h2, l2);
  split2<1>(v.y * sh_, v.w * sh_, h3, l3);
  uint4* pl = reinterpret_cast<uint4*>(xsm);
  pl[(int64_t)(2 * w) * nch + t] = make_uint4(h0, h1, h2, h3);
  pl[(int64_t)(2 * w + 1) * nch + t] = make_uint4(l0, l1, l2, l3);
  if (w == 0) {
    if constexpr (two) reinterpret_cast<float4*>(pl + 8 * nch)[t] = make_float4(pu, pv, pow2f(24 - sh), 0.0f);
    else reinterpret_cast<float2*>(pl + 8 * nch)[t] = make_float2(pu, pow2f(24 - sh));
  }
}

template <int FMT, int NT, bool RT>
__device__ inline void stage_pairs_finish(const GemvArgs& a, const float* xin, int64_t nch, const PairStage& ps,
                                          float* xsm, float* red) {
  constexpr int R1 = pair_run1<FMT>();
  const int tid = threadIdx.x, nt = NT;  // threads per block
  const int64_t items = nch * 4;
  const float4* x4 = reinterpret_cast<const float4*>(xin);
  const float4* w4 = reinterpret_cast<const float4*>(a.norm_w);
  const bool norm = w4 != nullptr;
  const bool wregs = items <= (int64_t)PBW * nt;  // norm weights of every item in registers
  const bool tap = a.xtap && blockIdx.x == 0;
  const bool rtap = RT && a.rtap && blockIdx.x == 0;
  const float4 one = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
  float inv = 1.0f;
  if (norm) {
    float ss = 0.0f;
    if (wregs) {
#pragma unroll
      for (int k = 0; k < PBW; ++k) {
        if ((int64_t)k * nt + tid < items) {
          const float4 u = ps.xa[k], v = ps.xb[k];
          ss += (u.x * u.x + u.y * u.y) + (u.z * u.z + u.w * u.w) + (v.x * v.x + v.y * v.y) +
                (v.z * v.z + v.w * v.w);
        }
      }
    } else {
      for (int64_t it = tid; it < items; it += nt) {
        const int64_t i0 = pair_run0<FMT>(it >> 2) + (it & 3);
        const float4 u = x4[i0], v = x4[i0 + R1];
        ss += (u.x * u.x + u.y * u.y) + (u.z * u.z + u.w * u.w) + (v.x * v.x + v.y * v.y) +
              (v.z * v.z + v.w * v.w);
      }
    }
    ss = wave_sum_dpp(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (int k = 0; k < (nt >> 6); ++k) tot += red[k];
    inv = 1.0f / sqrtf(tot / (float)a.K + a.eps);
  }
  // register batch
#pragma unroll
  for (int k = 0; k < PB; ++k) {
    const int64_t it = (int64_t)k * nt + tid;
    if ((int64_t)k * nt < items) {  // block-uniform; the shuffles need all lanes
      float4 uw = one, vw = one;
      if (norm) {
        if (k < PBW && wregs) { uw = ps.wa[k < PBW ? k : 0]; vw = ps.wb[k < PBW ? k : 0]; }
        else if (it < items) {
          const int64_t i0 = pair_run0<FMT>(it >> 2) + (it & 3);
          uw = w4[i0]; vw = w4[i0 + R1];
        }
      }
      emit_pair_item<FMT, RT>(a, nch, it, it < items, ps.xa[k], ps.xb[k], uw, vw, norm, inv, tap, rtap, xsm);
    }
  }
  // the rest (rows longer than PB * 4 * 32 * nt / 4 elements)
  for (int64_t base = (int64_t)PB * nt; base < items; base += nt) {
    const int64_t it = base + tid;
    const bool valid = it < items;
    float4 u = one, v = one, uw = one, vw = one;
    if (valid) {
      const int64_t i0 = pair_run0<FMT>(it >> 2) + (it & 3);
      u = x4[i0]; v = x4[i0 + R1];
      if (norm) { uw = w4[i0]; vw = w4[i0 + R1]; }
    }
    emit_pair_item<FMT, RT>(a, nch, it, valid, u, v, uw, vw, norm, inv, tap, rtap, xsm);
  }
  __syncthreads();
}

// ---- epilogues ----------------------------------------------------------------------

// Output side of one finished row group; acc[] holds the wave-uniform full dots
// of logical rows lrow0 .. lrow0+R-1.
template <int EPI, int R>
__device__ inline void epilogue(const GemvArgs& a, const GemvSeg& seg, int64_t lrow0, int lane,
                                const float* acc, const EpiIn& e, int pos, float& best_v, int32_t& best_i) {
  if constexpr (EPI == EPI_STORE || EPI == EPI_ADD || EPI == EPI_LOGITS || EPI == EPI_GELU) {
    if (lane < R) {
      float v = 0.0f;
#pragma unroll
      for (int r = 0; r < R; ++r) if (r == lane) v = acc[r];
      const int64_t l = lrow0 + lane;
      if (l < seg.rows) {
        const int64_t o = seg.row_base + l;
        if constexpr (EPI == EPI_ADD) {
          if (seg.scale) v = e.v1 * v;  // MoE expert weight (transformer.cpp:600-608)
          v = e.v0 + v;
        }
        if constexpr (EPI == EPI_GELU) {
          // tanh-form GELU (elementwise.cpp:57-71)
          const float inner = 0.7978845608f * (v + 0.044715f * v * v * v);
          v = 0.5f * v * (1.0f + tanhf(inner));
        }
        a.y[o] = v;
        if (a.tap) a.tap[o] = v;
      }
    }
    if constexpr (EPI == EPI_LOGITS) {
      // running greedy argmax of this wave (rows ascend, strict '>' keeps the lowest)
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int64_t l = lrow0 + r;
        if (l < seg.rows && (best_i == 0x7fffffff || acc[r] > best_v)) { best_v = acc[r]; best_i = (int32_t)l; }
      }
    }
  } else if constexpr (EPI == EPI_SWIGLU) {
    // pairs (gate, up) at logical rows (2j, 2j+1)
    if (lane < R / 2) {
      float g = 0.0f, u = 0.0f;
#pragma unroll
      for (int r = 0; r < R; r += 2) if (r == 2 * lane) { g = acc[r]; u = acc[r + 1]; }
      const int64_t l = lrow0 + 2 * lane;
      if (l < seg.rows) {
        const float act = g / (1.0f + expf(-g));  // silu (elementwise.cpp:73-84)
        a.y[seg.row_base + (l >> 1)] = act * u;
      }
    }
  } else if constexpr (EPI == EPI_QKV) {
    if (lane < R / 2) {
      float v0 = 0.0f, v1 = 0.0f;
#pragma unroll
      for (int r = 0; r < R; r += 2) if (r == 2 * lane) { v0 = acc[r]; v1 = acc[r + 1]; }
      const int64_t l = lrow0 + 2 * lane;
      if (l < seg.rows) {
        const int64_t r0 = (seg.kind == 2) ? l : qkv_phys(l, a.rope_mode, a.head_dim);
        const int64_t r1 = (seg.kind == 2) ? l + 1 : qkv_phys(l + 1, a.rope_mode, a.head_dim);
        if (seg.bias) { v0 = v0 + e.v0; v1 = v1 + e.v1; }
        if (seg.kind != 2) {
          // rotate pair p of its head by the host-built angle table
          const float2 cs = e.cs;
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

// The whole kernel for one format (the dynamic LDS, xsm, holds the staged input).
template <int FMT, int EPI, int W, bool RT>
__device__ __forceinline__ void gemv_body(GemvArgs a, float* xsm) {
  __shared__ float red[2 * W];
  __shared__ float kred[2][W][RPW_MAX];
  __shared__ float bval[W];
  __shared__ int32_t bidx[W];
  // EPI_ADD2: the block's waves form two halves, half h computing the rows of
  // segment h (same output rows, own input staged in its own LDS region)
  constexpr bool PAIR = EPI == EPI_ADD2;
  constexpr int HW = PAIR ? W / 2 : W;  // waves per segment in a block
  __shared__ float pexch[2][PAIR ? HW : 1][RPW_MAX];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int half = PAIR ? wave / HW : 0, hw = PAIR ? wave % HW : wave;

  // The input's loads go out first, from the leading fields of the arguments
  // (for a pair format a row of K values is K / 32 chunks): the launch's input
  // is its first memory request, before the segment and group setup below.
  PairStage ps0;
  if constexpr (pair_fmt<FMT>() && !PAIR) stage_pairs_issue<FMT, W * 64>(a, a.x, a.K >> 5, ps0);

  // segment lookup (uniform per block; per half for EPI_ADD2)
  int si = 0;
  if constexpr (PAIR) {
    si = half;
  } else {
    for (int k = 1; k < a.nseg; ++k) if ((int)blockIdx.x >= a.seg[k].block0) si = k;
  }
  const GemvSeg& seg = a.seg[si];
  const int nblk = PAIR ? (int)gridDim.x
                        : (si + 1 < a.nseg ? a.seg[si + 1].block0 : (int)gridDim.x) - seg.block0;

  constexpr int RPW = rpw_of(FMT);
  const int ks = a.ksplit;
  const int nrs = HW / ks;  // row sets per block (per half)
  const int rs = hw / ks, kp = hw % ks;

  Walk wk;
  wk.nch = seg.w.a_row >> 4;
  const int ncol = (int)((wk.nch + 63) >> 6);
  const int per = seg.per;
  wk.cbeg = kp * per;
  wk.cend = min(ncol, wk.cbeg + per);
  wk.steps = (per + 1) >> 1;

  const float* xin = seg.x ? seg.x : a.x;
  const int64_t ebase = seg.expert ? (int64_t)seg.expert[0] * seg.expert_rows : 0;
  const int pos = epi_pos<EPI>(a);
  const int g0 = (int)blockIdx.x - (PAIR ? 0 : seg.block0);
  // this half's staged input (the LDS holds one region per segment for EPI_ADD2)
  const int64_t region = pair_fmt<FMT>() ? wk.nch * (32 + pair_side<FMT>()) : a.K;
  float* const xs = xsm + (PAIR ? half * region : 0);
  // groups g0, g0 + nblk, ... below ngroups (counts computed on the host)
  const int mine = (g0 < seg.ngroups) ? seg.gq + (g0 < seg.gr ? 1 : 0) : 0;
  const int nunits = mine * wk.steps;

  auto unit_l0 = [&](int u) {
    return ((int64_t)(g0 + (u / wk.steps) * nblk) * nrs + rs) * RPW;
  };
  auto unit_step = [&](int u) { return u % wk.steps; };

  // input loads first; the first unit's weight loads go out before the staging
  // arithmetic for the register-staged formats, after it for the pair formats
  UnitBuf<FMT> U0;
  if constexpr (PAIR) {
    // both inputs staged by the whole block, one after the other (for the pair
    // formats before the first weight loads: their staging registers and a
    // unit's would not fit together under the 16-wave block's register limit)
    if constexpr (!pair_fmt<FMT>())
      if (nunits > 0) load_unit<FMT, EPI>(a, seg, ebase, wk, unit_l0(0), 0, lane, pos, U0);
#pragma unroll 1
    for (int h = 0; h < 2; ++h) {
      if constexpr (pair_fmt<FMT>()) {
        PairStage ps;
        stage_pairs_issue<FMT, W * 64>(a, a.seg[h].x, wk.nch, ps);
        stage_pairs_finish<FMT, W * 64, RT>(a, a.seg[h].x, wk.nch, ps, xsm + h * region, red);
      } else {
        stage_x<FMT, W * 64, RT>(a, a.seg[h].x, wk.nch, xsm + h * region, red);
      }
    }
    if constexpr (pair_fmt<FMT>())
      if (nunits > 0) load_unit<FMT, EPI>(a, seg, ebase, wk, unit_l0(0), 0, lane, pos, U0);
  } else if constexpr (pair_fmt<FMT>()) {
    // The weight loads go out only after the input is staged. The input vector
    // was just written by the previous launch; every CU's request for it is
    // served behind whatever the grid has already asked of memory, so issuing
    // the first unit's weights ahead of it (here, or once this wave's own input
    // has arrived, or after a short sleep) delayed the input to 6-10 us after
    // the launch against ~3 us, measured by per-wave clock stamps on the 8B
    // decode (gate/up 19.3 -> 17.9 us, LM head 61 -> 55 us, QKV unchanged;
    // 461 -> 471 tok/s).
    stage_pairs_finish<FMT, W * 64, RT>(a, xin, wk.nch, ps0, xsm, red);
    if (nunits > 0) load_unit<FMT, EPI>(a, seg, ebase, wk, unit_l0(0), 0, lane, pos, U0);
  } else if constexpr (FMT == T_Q8_0) {
    // input first here too: 8B Q8_0 decode 368.4 -> 372.2 tok/s (QKV 13.0 -> 12.0
    // us); the same order for the K-quants measured slower (1B 935 -> 917 tok/s)
    stage_x<FMT, W * 64, RT>(a, xin, wk.nch, xsm, red);
    if (nunits > 0) load_unit<FMT, EPI>(a, seg, ebase, wk, unit_l0(0), 0, lane, pos, U0);
  } else {
    if (nunits > 0) load_unit<FMT, EPI>(a, seg, ebase, wk, unit_l0(0), 0, lane, pos, U0);
    stage_x<FMT, W * 64, RT>(a, xin, wk.nch, xsm, red);
  }

  float best_v = -INFINITY;
  int32_t best_i = 0x7fffffff;
  float acc[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;

  // unit u -> (group index i = u / steps, step = u % steps); row group g0 + i * nblk
  auto finish = [&](int u, const EpiIn& e) {
    const int i = u / wk.steps;
    if (u - i * wk.steps != wk.steps - 1) return;
#pragma unroll
    for (int r = 0; r < RPW; ++r) acc[r] = wave_sum_dpp(acc[r]);
    if (ks > 1) {
      const int par = (int)(i & 1);
      if (lane == 0) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) kred[par][wave][r] = acc[r];
      }
      // LDS only: a full __syncthreads() would also wait for the weight loads
      // already in flight for the next unit
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
      __builtin_amdgcn_s_barrier();
      if (kp == 0) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
          float s = kred[par][wave][r];
          for (int k = 1; k < ks; ++k) s += kred[par][wave + k][r];
          acc[r] = s;
        }
      }
    }
    if constexpr (PAIR) {
      // half 1 hands its dots to half 0, which adds both in segment order
      const int par = (int)(i & 1);
      if (kp == 0 && half == 1 && lane == 0) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) pexch[par][rs][r] = acc[r];
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
      __builtin_amdgcn_s_barrier();
      if (kp == 0 && half == 0 && lane < RPW) {
        float v0 = 0.0f, v1 = 0.0f;
#pragma unroll
        for (int r = 0; r < RPW; ++r) if (r == lane) { v0 = acc[r]; v1 = pexch[par][rs][r]; }
        const int64_t l = ((int64_t)(g0 + i * nblk) * nrs + rs) * RPW + lane;
        if (l < seg.rows) {
          const int64_t o = seg.row_base + l;
          float v = a.y[o] + a.seg[0].scale[0] * v0;  // transformer.cpp:600-608, expert by expert
          v = v + a.seg[1].scale[0] * v1;
          a.y[o] = v;
          if (a.tap) a.tap[o] = v;
        }
      }
    } else if (kp == 0) {
      epilogue<EPI, RPW>(a, seg, ((int64_t)(g0 + i * nblk) * nrs + rs) * RPW, lane, acc, e, pos, best_v, best_i);
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;
  };
  // first batch: unit 0 (already in flight) and, for NB = 2, unit 1
  if constexpr (NB == 1) {
    if (nunits > 0) {
      compute_unit<FMT>(wk, 0, lane, xs, U0, acc);
      finish(0, U0.e);
    }
    for (int u = 1; u < nunits; ++u) {
      UnitBuf<FMT> V;
      load_unit<FMT, EPI>(a, seg, ebase, wk, unit_l0(u), unit_step(u), lane, pos, V);
      compute_unit<FMT>(wk, unit_step(u), lane, xs, V, acc);
      finish(u, V.e);
    }
  } else {
    if (nunits > 0) {
      UnitBuf<FMT> U1;
      if (nunits > 1) load_unit<FMT, EPI>(a, seg, ebase, wk, unit_l0(1), unit_step(1), lane, pos, U1);
      compute_unit<FMT>(wk, 0, lane, xs, U0, acc);
      finish(0, U0.e);
      if (nunits > 1) {
        compute_unit<FMT>(wk, unit_step(1), lane, xs, U1, acc);
        finish(1, U1.e);
      }
    }
    for (int u = 2; u < nunits; u += 2) {
      UnitBuf<FMT> V0, V1;
      const bool two = u + 1 < nunits;  // block-uniform
      load_unit<FMT, EPI>(a, seg, ebase, wk, unit_l0(u), unit_step(u), lane, pos, V0);
      if (two) load_unit<FMT, EPI>(a, seg, ebase, wk, unit_l0(u + 1), unit_step(u + 1), lane, pos, V1);
      compute_unit<FMT>(wk, unit_step(u), lane, xs, V0, acc);
      finish(u, V0.e);
      if (two) {
        compute_unit<FMT>(wk, unit_step(u + 1), lane, xs, V1, acc);
        finish(u + 1, V1.e);
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
      for (int k = 1; k < W; ++k) {
        if (bidx[k] == 0x7fffffff) continue;
        if (bi == 0x7fffffff || bval[k] > bv || (bval[k] == bv && bidx[k] < bi)) { bv = bval[k]; bi = bidx[k]; }
      }
      a.part_val[blockIdx.x] = bv;
      a.part_idx[blockIdx.x] = bi;
    }
  }
}

// 8-wave blocks (QKV) ask for 4 waves per SIMD, i.e. two blocks per CU: Q4_K
// took 130 VGPRs and held one block per CU; capped at 128 (2 spilled) the
// Mixtral-shape QKV ran 12.8 -> 9.6 us. The two-format kernel keeps its 132:
// capped, its 6 spills made the 1B QKV slower.
template <int FMT, int EPI, int W, bool RT>
__global__ void __launch_bounds__(W * 64, W == 8 ? 4 : 1) k_gemv(GemvArgs a) {
  extern __shared__ float xsm[];
  gemv_body<FMT, EPI, W, RT>(a, xsm);
}

// Segments of two formats in one launch (a QKV whose V projection is stored in
// another format, as in Q4_K_M files: Q4_K Q/K, Q6_K V). Blocks belong to one
// segment, so each block stages and walks in its own segment's format; the
// per-format launches this replaces each paid their own ramp and input staging.
template <int FA, int FB, int EPI, int W, bool RT>
__global__ void __launch_bounds__(W * 64) k_gemv_mix(GemvArgs a) {
  extern __shared__ float xsm[];
  int si = 0;
  for (int k = 1; k < a.nseg; ++k) if ((int)blockIdx.x >= a.seg[k].block0) si = k;
  if (a.seg[si].w.type == FB) gemv_body<FB, EPI, W, RT>(a, xsm);
  else gemv_body<FA, EPI, W, RT>(a, xsm);
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

template <int EPI, int W, bool RT>
KernelFn pick_fmt(int type) {
  switch (type) {
    case T_Q4_0: return k_gemv<T_Q4_0, EPI, W, RT>;
    case T_Q8_0: return k_gemv<T_Q8_0, EPI, W, RT>;
    case T_Q4_K: return k_gemv<T_Q4_K, EPI, W, RT>;
    case T_Q6_K: return k_gemv<T_Q6_K, EPI, W, RT>;
    case T_Q4_1: return k_gemv<T_Q4_1, EPI, W, RT>;
    case T_Q5_0: return k_gemv<T_Q5_0, EPI, W, RT>;
    case T_Q5_1: return k_gemv<T_Q5_1, EPI, W, RT>;
    case T_Q5_K: return k_gemv<T_Q5_K, EPI, W, RT>;
    case T_Q2_K: return k_gemv<T_Q2_K, EPI, W, RT>;
    case T_Q3_K: return k_gemv<T_Q3_K, EPI, W, RT>;
    case T_F32: return k_gemv<T_F32, EPI, W, RT>;
    case T_F16: return k_gemv<T_F16, EPI, W, RT>;
    default: return nullptr;
  }
}

// Kernel for (epilogue, format, waves per block, raw input tap): WPB for every
// epilogue, WPB_QKV for the QKV epilogue, WPB_LONG for the residual add. The
// raw tap (GemvArgs::rtap, the residual a split-K launch left) is compiled into
// its own instances of the epilogues that take a residual as input: the copy in
// the staging slowed every launch that carried it, taken or not (1B decode
// 1220 -> 1193 tok/s).
KernelFn pick(int epi, int type, int w, bool rt) {
  if (rt) {
    if (epi == EPI_SWIGLU && w == WPB_SWIGLU) return pick_fmt<EPI_SWIGLU, WPB_SWIGLU, true>(type);
    if (epi == EPI_QKV && w == WPB_QKV) return pick_fmt<EPI_QKV, WPB_QKV, true>(type);
    if (w != WPB) return nullptr;
    switch (epi) {
      case EPI_STORE: return pick_fmt<EPI_STORE, WPB, true>(type);
      case EPI_QKV: return pick_fmt<EPI_QKV, WPB, true>(type);
      case EPI_SWIGLU: return pick_fmt<EPI_SWIGLU, WPB, true>(type);
      case EPI_LOGITS: return pick_fmt<EPI_LOGITS, WPB, true>(type);
      case EPI_GELU: return pick_fmt<EPI_GELU, WPB, true>(type);
      default: return nullptr;
    }
  }
  if (epi == EPI_SWIGLU && w == WPB_SWIGLU) return pick_fmt<EPI_SWIGLU, WPB_SWIGLU, false>(type);
  if (epi == EPI_QKV && w == WPB_QKV) return pick_fmt<EPI_QKV, WPB_QKV, false>(type);
  if (w == WPB_LONG) {
    if (epi == EPI_ADD) return pick_fmt<EPI_ADD, WPB_LONG, false>(type);
    if (epi == EPI_ADD2) return pick_fmt<EPI_ADD2, WPB_LONG, false>(type);
    return nullptr;
  }
  if (w != WPB) return nullptr;
  switch (epi) {
    case EPI_STORE: return pick_fmt<EPI_STORE, WPB, false>(type);
    case EPI_ADD: return pick_fmt<EPI_ADD, WPB, false>(type);
    case EPI_QKV: return pick_fmt<EPI_QKV, WPB, false>(type);
    case EPI_SWIGLU: return pick_fmt<EPI_SWIGLU, WPB, false>(type);
    case EPI_LOGITS: return pick_fmt<EPI_LOGITS, WPB, false>(type);
    case EPI_GELU: return pick_fmt<EPI_GELU, WPB, false>(type);
    default: return nullptr;
  }
}

// The two-format kernel: QKV with Q4_K and Q6_K segments.
KernelFn pick_mix(int epi, int w, bool rt) {
  if (epi == EPI_QKV && w == WPB_QKV)
    return rt ? k_gemv_mix<T_Q4_K, T_Q6_K, EPI_QKV, WPB_QKV, true> : k_gemv_mix<T_Q4_K, T_Q6_K, EPI_QKV, WPB_QKV, false>;
  return nullptr;
}

// Waves per block for a launch of epilogue `epi` whose rows split K over `ks` waves.
int pick_waves(int epi, int ks) {
  if (epi == EPI_ADD2) return WPB_LONG;
  if (epi == EPI_ADD && ks == 4) return WPB_LONG;
  if (epi == EPI_QKV) return WPB_QKV;
  if (epi == EPI_SWIGLU) return WPB_SWIGLU;
  return WPB;
}

}  // namespace

// Raise each instantiation's dynamic-LDS limit to what the device allows per
// block (where the runtime accepts the attribute; otherwise its default holds).
hipError_t prepare_gemv() {
  const int epis[] = {EPI_STORE, EPI_ADD, EPI_QKV, EPI_SWIGLU, EPI_LOGITS, EPI_GELU, EPI_ADD2};
  const int types[] = {T_Q4_0, T_Q8_0, T_Q4_K, T_Q6_K, T_Q4_1, T_Q5_0,
                       T_Q5_1, T_Q5_K, T_Q2_K, T_Q3_K, T_F32,  T_F16};
  const int lim = lds_limit();
  for (int e : epis) {
    for (int w : {WPB, WPB_QKV, WPB_SWIGLU, WPB_LONG}) {
      for (bool rt : {false, true}) {
        for (int t : types) {
          const KernelFn fn = pick(e, t, w, rt);
          if (!fn) continue;
          (void)hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, lim - 1024);
          (void)hipGetLastError();
        }
        if (const KernelFn fn = pick_mix(e, w, rt)) {
          (void)hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, lim - 1024);
          (void)hipGetLastError();
        }
      }
    }
  }
  return hipSuccess;
}

namespace {

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

// Blocks of `fn` that stay resident on one CU with `lds` bytes of dynamic LDS
// (registers, LDS and wave slots all counted by the runtime); cached per pair.
int resident_blocks(KernelFn fn, size_t lds, int waves) {
  struct Entry { KernelFn fn; size_t lds; int n; };
  static std::mutex mu;
  static std::vector<Entry> cache;
  std::lock_guard<std::mutex> lock(mu);
  for (const Entry& e : cache)
    if (e.fn == fn && e.lds == lds) return e.n;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, waves * 64, lds) != hipSuccess || n <= 0) {
    (void)hipGetLastError();
    n = 2;
  }
  cache.push_back({fn, lds, n});
  return n;
}

// Waves of a block that share one row set's K: enough that a wave walks at most
// two 64-chunk columns of a row per group.
int pick_ksplit(const DevWeight& w) {
  const int64_t ncol = (w.a_row / 16 + 63) / 64;
  int ks = 1;
  while (ks < 4 && (ncol + ks - 1) / ks > 2) ks *= 2;
  return ks;
}

// Dynamic LDS of one block: the staged input (f32 planes, or f16 hi/lo pair
// planes plus side data per chunk for the pair formats).
size_t lds_bytes(int type, int64_t K) {
  if (type == T_Q4_0 || type == T_Q4_1) return (size_t)(K / 32) * (128 + 8);
  if (UAII_GEMV_KPAIR && (type == T_Q4_K || type == T_Q6_K)) return (size_t)(K / 32) * (128 + 16);
  return (size_t)K * sizeof(float);
}

struct Plan {
  KernelFn fn = nullptr;
  size_t lds = 0;
  int ks = 1;
  int waves = WPB;
  int per[3] = {0, 0, 0};  // blocks per segment
  int blocks = 0;
};

// Blocks per segment: one per row group, capped at what stays resident (the
// rest loop), shared out by group count.
// Segments of a run in more than one format (the two-format kernel's case).
bool mixed_run(const GemvArgs& a) {
  for (int k = 1; k < a.nseg; ++k)
    if (a.seg[k].w.type != a.seg[0].w.type) return true;
  return false;
}

Plan make_plan(const GemvArgs& a) {
  Plan p;
  const bool pair = a.epi == EPI_ADD2;  // two segments over the same rows, one staged input each
  const bool mix = mixed_run(a);
  p.lds = (pair ? 2 : 1) * lds_bytes(a.seg[0].w.type, a.K);
  for (int k = 1; k < a.nseg; ++k) p.lds = std::max(p.lds, lds_bytes(a.seg[k].w.type, a.K));
  p.ks = pick_ksplit(a.seg[0].w);
  p.waves = pick_waves(a.epi, p.ks);
  const bool rt = a.rtap != nullptr;
  p.fn = mix ? pick_mix(a.epi, p.waves, rt) : pick(a.epi, a.seg[0].w.type, p.waves, rt);
  if (!p.fn) return p;
  const int rpg = (p.waves / (pair ? 2 : 1) / p.ks) * rpw_of(a.seg[0].w.type);
  if (pair) {
    const int64_t g = (a.seg[0].rows + rpg - 1) / rpg;
    const int per_cu = resident_blocks(p.fn, p.lds, p.waves);
    p.per[0] = (int)std::min<int64_t>(g, (int64_t)cu_count() * per_cu);
    p.per[1] = 0;
    p.blocks = p.per[0];
    return p;
  }
  int64_t total = 0;
  for (int k = 0; k < a.nseg; ++k) total += (a.seg[k].rows + rpg - 1) / rpg;
  const int per_cu = UAII_GEMV_BLOCKS_PER_CU > 0 ? UAII_GEMV_BLOCKS_PER_CU : resident_blocks(p.fn, p.lds, p.waves);
  // The LM head streams 296 MB (8B shape) through one launch: with every
  // resident block (5 per CU) its loads queue in the per-CU memory path (the
  // address unit waits on the cache 5x as long as a plain read's); 3 blocks per
  // CU measured 61.4 us against 65.0 with the argmax epilogue (1: 95.6, 2: 67.7,
  // 4: 64.1), 55.0 against 56.5 storing the logits for the device sampler;
  // 101.9 against 107.3 for the 558 MB Q8_0 head. Smaller heads keep every
  // resident block: 70.7 against 76.7 us for a 148 MB Q4_K head (2048 columns),
  // 28.7 against 29.4 for a 74 MB one.
  const DevWeight& w0 = a.seg[0].w;
  const int64_t head_bytes = w0.rows * (w0.a_row + w0.b_row + w0.c_row + w0.d_row);
  const bool lm_head = a.epi == EPI_LOGITS || (a.epi == EPI_STORE && a.nseg == 1 && a.seg[0].rows >= 65536);
  const int cap_cu = lm_head && head_bytes >= (256ll << 20) ? std::min(per_cu, 3) : per_cu;
  const int64_t cap = (int64_t)cu_count() * cap_cu;
  for (int k = 0; k < a.nseg; ++k) {
    const int64_t g = (a.seg[k].rows + rpg - 1) / rpg;
    int64_t b = g;
    // more groups than resident blocks: the segment's share of the cap. The
    // block count is not evened out to equal groups per block: with a whole
    // number of blocks per CU, block b takes groups b, b + nblk, ... and the
    // blocks one CU holds (b, b + CUs, ...) add up to equal work per CU, where
    // 896 evened-out blocks of two groups put four blocks on half the CUs and
    // three on the rest (8B gate/up 21.8 -> 19.8 us)
    if (total > cap) b = std::max<int64_t>(1, (g * cap + total - 1) / total);
    p.per[k] = (int)std::min<int64_t>(b, g);
    p.blocks += p.per[k];
  }
  return p;
}

// Whether segments of types ta and tb (the same K) share the two-format kernel:
// Q4_K and Q6_K, whose chunks (16 payload bytes, 32 inputs), rows per wave and
// staged-input side data agree.
bool mix_pair(int epi, int ta, int tb) {
  auto kq = [](int t) { return t == T_Q4_K || t == T_Q6_K; };
  return UAII_GEMV_KPAIR && epi == EPI_QKV && kq(ta) && kq(tb);
}

// Runs of consecutive segments sharing a weight type: one launch each (the
// kernel is specialised per type), so QKV with mixed types takes several, apart
// from the mixes the two-format kernel covers.
template <typename F>
hipError_t for_each_run(const GemvArgs& in, F&& f) {
  int k0 = 0;
  while (k0 < in.nseg) {
    int k1 = k0 + 1;
    while (k1 < in.nseg && (in.seg[k1].w.type == in.seg[k0].w.type ||
                            (mix_pair(in.epi, in.seg[k0].w.type, in.seg[k1].w.type) &&
                             in.seg[k1].w.a_row == in.seg[k0].w.a_row)))
      ++k1;
    GemvArgs a = in;
    a.nseg = k1 - k0;
    for (int k = 0; k < a.nseg; ++k) a.seg[k] = in.seg[k0 + k];
    if (k0 > 0) a.xtap = a.rtap = nullptr;
    const hipError_t st = f(a);
    if (st != hipSuccess) return st;
    k0 = k1;
  }
  return hipSuccess;
}

}  // namespace

int gemv_grid(const GemvArgs& in) {
  int most = 0;
  (void)for_each_run(in, [&](const GemvArgs& a) {
    most = std::max(most, make_plan(a).blocks);
    return hipSuccess;
  });
  return most;
}

hipError_t launch_gemv(const GemvArgs& in, hipStream_t s) {
  if (in.K % 4) return hipErrorInvalidValue;
  if (in.epi == EPI_LOGITS && in.nseg != 1) return hipErrorInvalidValue;
  if (in.epi == EPI_ADD2) {
    // one launch (one type), the same output rows, each segment its own input,
    // expert and weight
    const GemvSeg &s0 = in.seg[0], &s1 = in.seg[1];
    if (in.nseg != 2 || s0.w.type != s1.w.type || s0.rows != s1.rows || s0.row_base != s1.row_base ||
        !s0.x || !s1.x || !s0.scale || !s1.scale)
      return hipErrorInvalidValue;
  }
  for (int k = 0; k < in.nseg; ++k) {
    if (in.epi == EPI_SWIGLU && in.seg[k].w2.type != in.seg[k].w.type) return hipErrorInvalidValue;
    if ((in.epi == EPI_SWIGLU || in.epi == EPI_QKV) && (in.seg[k].rows % 2)) return hipErrorInvalidValue;
    if (in.seg[k].w.cols != in.K) return hipErrorInvalidValue;
    // every row a segment can touch lies inside its weight (and up-weight)
    const GemvSeg& g = in.seg[k];
    const int64_t need = (in.epi == EPI_SWIGLU) ? g.rows / 2 : g.rows;
    if (g.expert) {
      if (g.expert_rows <= 0 || need > g.expert_rows || g.w.rows % g.expert_rows) return hipErrorInvalidValue;
      if (in.epi == EPI_SWIGLU && g.w2.rows != g.w.rows) return hipErrorInvalidValue;
    } else if (in.epi != EPI_QKV) {
      if (need > g.w.rows) return hipErrorInvalidValue;
      if (in.epi == EPI_SWIGLU && need > g.w2.rows) return hipErrorInvalidValue;
    }
  }
  return for_each_run(in, [&](const GemvArgs& run) {
    GemvArgs a = run;
    const Plan p = make_plan(a);
    if (!p.fn) return hipErrorInvalidValue;
    a.ksplit = p.ks;
    const bool pair = a.epi == EPI_ADD2;
    if (!pair) {
      // one input for the run, at GemvArgs::x (the kernel issues it first)
      const float* x = a.seg[0].x ? a.seg[0].x : a.x;
      for (int k = 0; k < a.nseg; ++k) {
        if (a.seg[k].x && a.seg[k].x != x) return hipErrorInvalidValue;
        a.seg[k].x = nullptr;
      }
      a.x = x;
    }
    int blocks = 0;
    for (int k = 0; k < a.nseg; ++k) {
      a.seg[k].block0 = blocks;
      blocks += p.per[k];
    }
    if (blocks == 0) return hipSuccess;
    // the kernel's integer setup: row groups, groups per block, chunk columns per wave
    const int rpg = (p.waves / (pair ? 2 : 1) / p.ks) * rpw_of(a.seg[0].w.type);
    for (int k = 0; k < a.nseg; ++k) {
      GemvSeg& g = a.seg[k];
      const int64_t ngroups = (g.rows + rpg - 1) / rpg;
      const int nblk = pair ? blocks : p.per[k];
      if (ngroups > INT32_MAX || nblk <= 0) return hipErrorInvalidValue;
      g.ngroups = (int32_t)ngroups;
      g.gq = (int32_t)(ngroups / nblk);
      g.gr = (int32_t)(ngroups % nblk);
      const int64_t ncol = (g.w.a_row / 16 + 63) / 64;
      g.per = (int32_t)((ncol + p.ks - 1) / p.ks);
    }
    if ((int64_t)p.lds > lds_limit() - 1024) return hipErrorInvalidValue;
    if (a.epi == EPI_LOGITS && blocks > a.part_cap) return hipErrorInvalidValue;
    UAII_LAUNCH(p.fn, dim3(blocks), dim3(p.waves * 64), p.lds, s, a);
    hipError_t st = hipGetLastError();
    if (st == hipSuccess && a.epi == EPI_LOGITS) {
      UAII_LAUNCH(k_argmax_final, dim3(1), dim3(1024), 0, s, a, blocks);
      st = hipGetLastError();
    }
    return st;
  });
}

hipError_t launch_argmax_final(float* part_val, int32_t* part_idx, int nparts, StepState* state,
                               int32_t* ids, hipStream_t s) {
  if (!part_val || !part_idx || !state || !ids || nparts < 1) return hipErrorInvalidValue;
  GemvArgs a{};
  a.part_val = part_val;
  a.part_idx = part_idx;
  a.state = state;
  a.ids = ids;
  UAII_LAUNCH(k_argmax_final, dim3(1), dim3(1024), 0, s, a, nparts);
  return hipGetLastError();
}

}  // namespace uaii_hip
