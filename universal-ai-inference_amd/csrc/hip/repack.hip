// repack.hip — GGUF block rows -> split device layout, and the bit-exact
// dequant kernels that read it back.
//
// Split layout per tensor [rows, cols] (byte arrays, each [rows][x_row]):
//   type   a (16-byte chunks)      b                 c                   d
//   F32    values                  -                 -                   -
//   F16    values                  -                 -                   -
//   Q4_0   qs (16 B / block)       d (2 B / block)   -                   -
//   Q4_1   qs                      d,m (4 B / block) -                   -
//   Q5_0   qs                      qh (4 B / block)  d (2 B / block)     -
//   Q5_1   qs                      qh (4 B / block)  d,m (4 B / block)   -
//   Q8_0   qs (32 B / block)       d (2 B / block)   -                   -
//   Q2_K   qs (64 B / sb)          scales (16 B/sb)  d,dmin (4 B / sb)   -
//   Q3_K   qs (64 B / sb)          hmask (32 B / sb) scales12,d,pad (16) -
//   Q4_K   qs (128 B / sb)         d,dmin,scales12 (16 B / sb) -         -
//   Q5_K   qs (128 B / sb)         d,dmin,scales12   qh (32 B / sb)      -
//   Q6_K   ql (128 B / sb)         qh (64 B / sb)    scales (16 B / sb)  d (2 B / sb)
// GGUF block layouts: libs/uaii-quant/src/gguf_dequant.cpp:12-77.

#include "common.h"
#include "uaii_hip_internal.h"

namespace uaii_hip {

void split_row_bytes(int type, int64_t cols, int64_t out[4]) {
  const int64_t nb32 = cols / 32, nb256 = cols / 256;
  out[0] = out[1] = out[2] = out[3] = 0;
  switch (type) {
    case T_F32: out[0] = cols * 4; break;
    case T_F16: out[0] = cols * 2; break;
    case T_Q4_0: out[0] = nb32 * 16; out[1] = nb32 * 2; break;
    case T_Q4_1: out[0] = nb32 * 16; out[1] = nb32 * 4; break;
    case T_Q5_0: out[0] = nb32 * 16; out[1] = nb32 * 4; out[2] = nb32 * 2; break;
    case T_Q5_1: out[0] = nb32 * 16; out[1] = nb32 * 4; out[2] = nb32 * 4; break;
    case T_Q8_0: out[0] = nb32 * 32; out[1] = nb32 * 2; break;
    case T_Q2_K: out[0] = nb256 * 64; out[1] = nb256 * 16; out[2] = nb256 * 4; break;
    case T_Q3_K: out[0] = nb256 * 64; out[1] = nb256 * 32; out[2] = nb256 * 16; break;
    case T_Q4_K: out[0] = nb256 * 128; out[1] = nb256 * 16; break;
    case T_Q5_K: out[0] = nb256 * 128; out[1] = nb256 * 16; out[2] = nb256 * 32; break;
    case T_Q6_K: out[0] = nb256 * 128; out[1] = nb256 * 64; out[2] = nb256 * 16; out[3] = nb256 * 2; break;
    default: break;
  }
}

namespace {

__device__ inline void cp(uint8_t* dst, const uint8_t* src, int n) {
  for (int i = 0; i < n; ++i) dst[i] = src[i];
}

// Q4_0 payload whose ggml decode (element k = low nibble of byte k, element
// k + 16 = its high nibble) gives the values of the reference's f32 load, which
// takes elements 2j and 2j + 1 from the low and high nibbles of byte j
// (libs/uaii-loaders/src/gguf.cpp:514-520).
__device__ inline void q4_0_from_pairwise(uint8_t* dst, const uint8_t* qs) {
  for (int k = 0; k < 16; ++k) {
    const int sh = 4 * (k & 1);
    const uint32_t lo = (qs[k >> 1] >> sh) & 15u;        // element k
    const uint32_t hi = (qs[8 + (k >> 1)] >> sh) & 15u;  // element k + 16
    dst[k] = (uint8_t)(lo | (hi << 4));
  }
}

// One thread per GGUF block. q4_0_pairwise: Q4_0 blocks take the values of the
// reference's f32 load instead of its packed decode.
__global__ void k_repack(DevWeight w, const uint8_t* __restrict__ src, int64_t nblocks_row,
                         int64_t total_blocks, int q4_0_pairwise) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= total_blocks) return;
  const int64_t r = gid / nblocks_row, i = gid % nblocks_row;
  const int bb = block_bytes(w.type);
  const uint8_t* s = src + gid * bb;
  uint8_t* a = const_cast<uint8_t*>(w.a) + r * w.a_row;
  uint8_t* b = const_cast<uint8_t*>(w.b) + r * w.b_row;
  uint8_t* c = const_cast<uint8_t*>(w.c) + r * w.c_row;
  uint8_t* d = const_cast<uint8_t*>(w.d) + r * w.d_row;
  switch (w.type) {
    case T_F32: cp(a + i * 4, s, 4); break;
    case T_F16: cp(a + i * 2, s, 2); break;
    case T_Q4_0:
      cp(b + i * 2, s, 2);
      if (q4_0_pairwise) q4_0_from_pairwise(a + i * 16, s + 2);
      else cp(a + i * 16, s + 2, 16);
      break;
    case T_Q4_1: cp(b + i * 4, s, 4); cp(a + i * 16, s + 4, 16); break;
    case T_Q5_0: cp(c + i * 2, s, 2); cp(b + i * 4, s + 2, 4); cp(a + i * 16, s + 6, 16); break;
    case T_Q5_1: cp(c + i * 4, s, 4); cp(b + i * 4, s + 4, 4); cp(a + i * 16, s + 8, 16); break;
    case T_Q8_0: cp(b + i * 2, s, 2); cp(a + i * 32, s + 2, 32); break;
    case T_Q2_K: cp(b + i * 16, s, 16); cp(a + i * 64, s + 16, 64); cp(c + i * 4, s + 80, 4); break;
    case T_Q3_K:
      cp(b + i * 32, s, 32); cp(a + i * 64, s + 32, 64); cp(c + i * 16, s + 96, 12);
      cp(c + i * 16 + 12, s + 108, 2); c[i * 16 + 14] = 0; c[i * 16 + 15] = 0;
      break;
    case T_Q4_K: cp(b + i * 16, s, 16); cp(a + i * 128, s + 16, 128); break;
    case T_Q5_K: cp(b + i * 16, s, 16); cp(c + i * 32, s + 16, 32); cp(a + i * 128, s + 48, 128); break;
    case T_Q6_K:
      cp(a + i * 128, s, 128); cp(b + i * 64, s + 128, 64); cp(c + i * 16, s + 192, 16);
      cp(d + i * 2, s + 208, 2);
      break;
    default: break;
  }
}

// One thread per 16-byte chunk; writes the decoded values to out[r - row0][idx].
template <int FMT>
__global__ void k_dequant(DevWeight w, int64_t row0, int64_t nrows, float* __restrict__ out) {
  const int64_t nchunks = w.a_row / 16;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= nrows * nchunks) return;
  const int64_t rr = gid / nchunks, t = gid % nchunks;
  ChunkOut o;
  decode_chunk<FMT>(w, row0 + rr, t, o);
  float* dst = out + rr * w.cols;
#pragma unroll
  for (int i = 0; i < 64; ++i)
    if (i < o.n) dst[o.idx[i]] = o.v[i];
}

}  // namespace

hipError_t launch_repack(const DevWeight& w, const uint8_t* src_dev, hipStream_t s, bool q4_0_pairwise) {
  const int64_t nbr = w.cols / block_elems(w.type);
  const int64_t total = nbr * w.rows;
  if (total == 0) return hipSuccess;
  const int threads = 256;
  const int64_t grid = (total + threads - 1) / threads;
  hipLaunchKernelGGL(k_repack, dim3((unsigned)grid), dim3(threads), 0, s, w, src_dev, nbr, total,
                     q4_0_pairwise ? 1 : 0);
  return hipGetLastError();
}

hipError_t launch_dequant(const DevWeight& w, int64_t row0, int64_t nrows, float* out,
                          hipStream_t s) {
  const int64_t total = nrows * (w.a_row / 16);
  if (total == 0) return hipSuccess;
  const int threads = 256;
  const int64_t grid = (total + threads - 1) / threads;
  UAII_FOR_TYPE(w.type, hipLaunchKernelGGL(k_dequant<FT>, dim3((unsigned)grid), dim3(threads), 0, s,
                                           w, row0, nrows, out));
  return hipGetLastError();
}

}  // namespace uaii_hip
