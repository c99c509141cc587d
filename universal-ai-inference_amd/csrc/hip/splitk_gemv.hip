// splitk_gemv.hip — a decode GEMV with a residual add, split along K, whose
// blocks add their partial row sums into the output with float atomics (gfx950).
//
// Replaces quant_gemm_f32 at M = 1 (libs/uaii-kernels/src/quant_gemm.cpp:22-70)
// plus the residual add_f32 (elementwise.cpp:99-110) for Q4_0 and Q6_K weights:
// the FFN down projection, y += W_down . h.
//
// Block (r, c) owns column slice c (SC = 1024 columns: 32 Q4_0 blocks, or 4 Q6_K
// super-blocks of which each lane takes 32 elements) of
// RB = 8 J consecutive rows r RB ... The row block is the grid's x index, so the
// slices of one row block land on one XCD and their atomic adds to a row meet
// in that XCD's L2 (33.6 MB fetched per 8B down launch, 33.1 MB algorithmic,
// against 37.3 MB with the slices of a row spread over the XCDs). Lane (g, b) of a wave (b = lane % 32) loads the 32
// inputs of block b of the slice straight from global memory (no LDS, no block
// barrier), then block b of rows g, g + 2, ... (J rows, 16 payload bytes and the
// f16 scale each), all of it before the first dot product. The 32 blocks of a
// row are summed across the half-wave (DPP within rows of 16 lanes, one swizzle
// across them) and the row's sum goes into y with one float atomic. Only the
// slice's 4 KiB of inputs is read per block, where a whole-row kernel stages all
// K inputs in every block.
//
// Each y row receives K / 1024 atomic adds in the order they arrive, so two runs
// may differ in the last bits of those f32 adds; each slice's sum is computed
// in a fixed order.

#include "common.h"
#include "block_dot.h"
#include "uaii_hip_internal.h"

namespace uaii_hip {
namespace {

constexpr int LPR = 32;        // lanes per row (Q4_0 blocks per slice)
constexpr int SC = 32 * LPR;   // columns per slice
constexpr int RPI = 64 / LPR;  // rows per wave instruction
constexpr int NW = 4;          // waves per block

template <int FMT, int J>
__global__ void __launch_bounds__(NW * 64) k_gemv_splitk(SplitKArgs p) {
  const int c = blockIdx.y, w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int b = lane % LPR;
  const int64_t r0 = (int64_t)blockIdx.x * (NW * RPI * J) + w * (RPI * J) + lane / LPR;

  // block b's 32 inputs, then the weights of its J rows
  float xv[32];
  const float4* xp = reinterpret_cast<const float4*>(p.x + (int64_t)c * SC + b * 32);
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float4 t = xp[k];
    xv[4 * k] = t.x; xv[4 * k + 1] = t.y; xv[4 * k + 2] = t.z; xv[4 * k + 3] = t.w;
  }
  // Q4_0: block b (16 payload bytes, f16 scale). Q6_K: elements 32 m .. 32 m + 31
  // of half hf of super-block sb (4 per slice): 32 ql and 32 qh bytes, the two
  // int8 scales and d
  constexpr int QW = FMT == T_Q6_K ? 2 : 1;
  const int64_t sb = (int64_t)c * (SC / 256) + (b >> 3);
  const int hf = (b & 7) >> 2, m = b & 3;
  uint4 qv[J][QW], hv[J][QW];
  uint32_t sv[J], dv[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int64_t r = r0 + RPI * j;
    if constexpr (FMT == T_Q6_K) {
      const uint4* ql = reinterpret_cast<const uint4*>(p.w.a + r * p.w.a_row + sb * 128 + hf * 64 + 32 * (m & 1));
      const uint4* qh = reinterpret_cast<const uint4*>(p.w.b + r * p.w.b_row + sb * 64 + hf * 32);
#pragma unroll
      for (int k = 0; k < QW; ++k) {
        qv[j][k] = ql[k];
        hv[j][k] = qh[k];
      }
      sv[j] = *reinterpret_cast<const uint16_t*>(p.w.c + r * p.w.c_row + sb * 16 + hf * 8 + 2 * m);
      dv[j] = *reinterpret_cast<const uint16_t*>(p.w.d + r * p.w.d_row + sb * 2);
    } else {
      qv[j][0] = *reinterpret_cast<const uint4*>(p.w.a + r * p.w.a_row + c * (SC / 2) + b * 16);
      sv[j] = *reinterpret_cast<const uint16_t*>(p.w.b + r * p.w.b_row + c * (SC / 16) + b * 2);
    }
  }
  // every load is issued before the first product waits for the inputs
  __builtin_amdgcn_sched_barrier(0);

  float sx0 = 0.0f, sx1 = 0.0f;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    sx0 += xv[k];
    sx1 += xv[16 + k];
  }
  float rs[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    float v;
    if constexpr (FMT == T_Q6_K) v = q6_k_dot(qv[j], hv[j], m, sv[j], dv[j], xv, sx0, sx1);
    else v = q4_0_dot(qv[j][0], sv[j], xv, sx0 + sx1);
    v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_mov<0x141>(v);  // row_half_mirror
    v += dpp_mov<0x140>(v);  // row_mirror: the 16 lanes of a row
    v += __shfl_xor(v, 16);  // the two rows of a half-wave
    rs[j] = v;
  }
  float v = rs[0];
#pragma unroll
  for (int j = 1; j < J; ++j) v = b == j ? rs[j] : v;
  if (b < J) atomicAdd(p.y + r0 + RPI * b, v);
}

// Rows per lane: the most (fewest blocks, fewest redundant input loads) that
// still gives 512 blocks; 8 on the 8B down projection (896 blocks; 4 and 16
// measured slower). Q6_K carries four payload words per row: at most 4.
int pick_j(const SplitKArgs& p) {
  const int64_t slices = p.w.cols / SC;
  const int most = p.w.type == T_Q6_K ? 4 : 8;
  for (int j : {8, 4, 2})
    if (j <= most && p.rows % (NW * RPI * j) == 0 && slices * (p.rows / (NW * RPI * j)) >= 512) return j;
  for (int j : {8, 4, 2})
    if (j <= most && p.rows % (NW * RPI * j) == 0) return j;
  return 0;
}

}  // namespace

bool gemv_splitk_supported(const SplitKArgs& p) {
  const DevWeight& w = p.w;
  if (w.cols <= 0 || w.cols % SC) return false;
  const bool q4 = w.type == T_Q4_0 && w.a_row == w.cols / 2 && w.b_row == w.cols / 16;
  const bool q6 = w.type == T_Q6_K && w.a_row == w.cols / 2 && w.b_row == w.cols / 4 &&
                  w.c_row == w.cols / 16 && w.d_row == w.cols / 128;
  if (!q4 && !q6) return false;
  if (p.rows <= 0 || w.rows < p.rows) return false;
  return pick_j(p) > 0;
}

hipError_t launch_gemv_splitk(const SplitKArgs& p, hipStream_t s) {
  if (!gemv_splitk_supported(p) || !p.x || !p.y) return hipErrorInvalidValue;
  const int J = pick_j(p);
  dim3 grid((unsigned)(p.rows / (NW * RPI * J)), (unsigned)(p.w.cols / SC));
  if (p.w.type == T_Q6_K) {
    if (J == 4) UAII_LAUNCH((k_gemv_splitk<T_Q6_K, 4>), grid, dim3(NW * 64), 0, s, p);
    else UAII_LAUNCH((k_gemv_splitk<T_Q6_K, 2>), grid, dim3(NW * 64), 0, s, p);
  } else {
    if (J == 8) UAII_LAUNCH((k_gemv_splitk<T_Q4_0, 8>), grid, dim3(NW * 64), 0, s, p);
    else if (J == 4) UAII_LAUNCH((k_gemv_splitk<T_Q4_0, 4>), grid, dim3(NW * 64), 0, s, p);
    else UAII_LAUNCH((k_gemv_splitk<T_Q4_0, 2>), grid, dim3(NW * 64), 0, s, p);
  }
  return hipGetLastError();
}

}  // namespace uaii_hip
