// block_dot.h — one 32-element block (Q4_0, Q8_0, or a Q4_K sub-block) dotted
// with 32 f32 inputs, for the kernels that hold a block's inputs in registers
// (attn_out.hip, splitk_gemv.hip).
#pragma once

#include "common.h"

namespace uaii_hip {

// Q4_0 (libs/uaii-quant/src/gguf_dequant.cpp:117-134): element k is the low nibble of payload byte k,
// element k + 16 its high nibble, value (nibble - 8) * d. The nibbles go through
// f32 FMAs against the inputs in element order; the -8 offset is applied once,
// as 8 times the inputs' sum sx.
__device__ __forceinline__ float q4_0_dot(const uint4& q, uint32_t d16, const float (&xv)[32], float sx) {
  const uint32_t q4[4] = {q.x, q.y, q.z, q.w};
  float acc = 0.0f;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t lo = q4[t] & 0x0F0F0F0Fu, hi = (q4[t] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc = fmaf((float)((lo >> (8 * e)) & 0xFFu), xv[4 * t + e], acc);
      acc = fmaf((float)((hi >> (8 * e)) & 0xFFu), xv[16 + 4 * t + e], acc);
    }
  }
  return __half2float(__ushort_as_half((unsigned short)d16)) * (acc - 8.0f * sx);
}

// Q8_0 (gguf_dequant.cpp:203-217): element k is the signed payload byte k, value
// byte * d; f32 FMAs in element order.
__device__ __forceinline__ float q8_0_dot(const uint4 (&q)[2], uint32_t d16, const float (&xv)[32]) {
  const uint32_t w8[8] = {q[0].x, q[0].y, q[0].z, q[0].w, q[1].x, q[1].y, q[1].z, q[1].w};
  float acc = 0.0f;
#pragma unroll
  for (int t = 0; t < 8; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) acc = fmaf((float)(int8_t)((w8[t] >> (8 * e)) & 0xFFu), xv[4 * t + e], acc);
  return __half2float(__ushort_as_half((unsigned short)d16)) * acc;
}

// Sub-block j (0..7) of a Q4_K super-block (gguf_dequant.cpp:308-340): its 32
// elements are the low (j even) or high (j odd) nibbles of quant bytes
// 32 (j / 2) .. 32 (j / 2) + 31, here q; value d1 * nibble - m1 with d1 = d * sc,
// m1 = dmin * mn and (sc, mn) the 6-bit pair j of the 12 scale bytes
// (get_scale_min_k4, gguf_dequant.cpp:107-115). meta holds the super-block's
// d, dmin and scale bytes as the file stores them (16 bytes).
__device__ __forceinline__ float q4_k_dot(const uint4 (&q)[2], const uint4& meta, int j, const float (&xv)[32],
                                          float sx) {
  const int sh = 4 * (j & 1);
  const uint32_t w8[8] = {q[0].x, q[0].y, q[0].z, q[0].w, q[1].x, q[1].y, q[1].z, q[1].w};
  float acc = 0.0f;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const uint32_t n = (w8[t] >> sh) & 0x0F0F0F0Fu;
#pragma unroll
    for (int e = 0; e < 4; ++e) acc = fmaf((float)((n >> (8 * e)) & 0xFFu), xv[4 * t + e], acc);
  }
  const uint32_t mw[4] = {meta.x, meta.y, meta.z, meta.w};
  auto sbyte = [&](int k) { return (int)((mw[(4 + k) >> 2] >> (8 * ((4 + k) & 3))) & 0xFFu); };  // scales[k]
  int sc, mn;
  if (j < 4) {
    sc = sbyte(j) & 63;
    mn = sbyte(j + 4) & 63;
  } else {
    sc = (sbyte(j + 4) & 15) | ((sbyte(j - 4) >> 6) << 4);
    mn = (sbyte(j + 4) >> 4) | ((sbyte(j) >> 6) << 4);
  }
  const float d = __half2float(__ushort_as_half((unsigned short)(meta.x & 0xFFFFu)));
  const float dmin = __half2float(__ushort_as_half((unsigned short)(meta.x >> 16)));
  return (d * (float)sc) * acc - (dmin * (float)mn) * sx;
}

// Elements 32 m .. 32 m + 31 (m = 0..3) of one 128-element half of a Q6_K
// super-block (gguf_dequant.cpp:381-416): element l takes the low (m < 2) or
// high (m >= 2) nibble of quant byte 32 (m & 1) + l of the half's 64 (ql) and
// bits 2m, 2m + 1 of its high-bit byte l (qh), value d * scale * (q - 32), the
// int8 scale of elements l < 16 in byte 0 of sc2 and of l >= 16 in byte 1.
__device__ __forceinline__ float q6_k_dot(const uint4 (&ql)[2], const uint4 (&qh)[2], int m, uint32_t sc2,
                                          uint32_t d16, const float (&xv)[32], float sx0, float sx1) {
  const int nsh = 4 * (m >> 1), hsh = 2 * m;
  const uint32_t wl[8] = {ql[0].x, ql[0].y, ql[0].z, ql[0].w, ql[1].x, ql[1].y, ql[1].z, ql[1].w};
  const uint32_t wh[8] = {qh[0].x, qh[0].y, qh[0].z, qh[0].w, qh[1].x, qh[1].y, qh[1].z, qh[1].w};
  float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const uint32_t q = ((wl[t] >> nsh) & 0x0F0F0F0Fu) | (((wh[t] >> hsh) & 0x03030303u) << 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float v = (float)((q >> (8 * e)) & 0xFFu) * xv[4 * t + e];
      if (t < 4) a0 += v; else a1 += v;
    }
  }
  const float s0 = (float)(int8_t)(sc2 & 0xFFu), s1 = (float)(int8_t)((sc2 >> 8) & 0xFFu);
  const float d = __half2float(__ushort_as_half((unsigned short)d16));
  return d * (s0 * (a0 - 32.0f * sx0) + s1 * (a1 - 32.0f * sx1));
}

}  // namespace uaii_hip
