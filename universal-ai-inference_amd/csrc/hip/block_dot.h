// block_dot.h — one Q4_0 or Q8_0 block dotted with 32 f32 inputs, for the
// kernels that hold a block's inputs in registers (attn_out.hip, splitk_gemv.hip).
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

}  // namespace uaii_hip
