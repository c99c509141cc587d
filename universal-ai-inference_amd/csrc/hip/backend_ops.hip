// backend_ops.hip — the elementwise operators of the op-by-op backend (gfx950).
//
// The decoder's own step fuses these into the GEMV prologues and epilogues; the
// backend (host/rocm_backend.cpp) runs one reference operator per dispatch and
// needs them on their own:
//   k_ew<OP>      Add / Mul of two equal-sized f32 tensors, SiLU, GELU (tanh form)
//                 (libs/uaii-kernels/src/elementwise.cpp:56-110)
//   k_kv_append   rows of K and V written into a head-major cache
//                 [n_kv][max_seq][head_dim] at positions p0 .. p0+rows-1, f32 or f16
//                 (KvCache::append_layer, include/uaii/runtime/kv_cache.hpp:80-120,
//                 in the decode attention's layout)
// All are memory-bound streams: 16-byte loads and stores where the size allows,
// a grid-stride loop over 4-float groups, the tail element by element.

#include "common.h"
#include "uaii_hip_internal.h"

namespace uaii_hip {
namespace {

enum { EW_ADD = 0, EW_MUL = 1, EW_SILU = 2, EW_GELU = 3 };

template <int OP>
__device__ inline float ew1(float a, float b) {
  if constexpr (OP == EW_ADD) return a + b;
  if constexpr (OP == EW_MUL) return a * b;
  if constexpr (OP == EW_SILU) return a / (1.0f + expf(-a));
  // GELU, tanh approximation with the reference's constants
  const float u = 0.7978845608f * (a + 0.044715f * a * a * a);
  return 0.5f * a * (1.0f + tanhf(u));
}

template <int OP>
__global__ void __launch_bounds__(256) k_ew(const float* __restrict__ a, const float* __restrict__ b,
                                            float* __restrict__ y, int64_t n) {
  constexpr bool BIN = OP == EW_ADD || OP == EW_MUL;
  const int64_t n4 = n / 4;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const bool vec = ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(y) |
                     (BIN ? reinterpret_cast<uintptr_t>(b) : 0)) & 15) == 0;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (vec) {
    for (; i < n4; i += stride) {
      const float4 x = reinterpret_cast<const float4*>(a)[i];
      const float4 z = BIN ? reinterpret_cast<const float4*>(b)[i] : float4{0, 0, 0, 0};
      reinterpret_cast<float4*>(y)[i] = float4{ew1<OP>(x.x, z.x), ew1<OP>(x.y, z.y), ew1<OP>(x.z, z.z),
                                               ew1<OP>(x.w, z.w)};
    }
    i = 4 * n4 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  }
  for (; i < n; i += stride) y[i] = ew1<OP>(a[i], BIN ? b[i] : 0.0f);
}

__global__ void __launch_bounds__(256) k_kv_append(const float* __restrict__ k, const float* __restrict__ v,
                                                   void* kc, void* vc, int64_t rows, int64_t kv_dim,
                                                   int hd, int64_t max_seq, int64_t p0, int f16) {
  const int64_t n = rows * kv_dim;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / kv_dim, c = i % kv_dim;
    const int64_t dst = ((c / hd) * max_seq + p0 + r) * hd + c % hd;
    if (f16) {
      reinterpret_cast<__half*>(kc)[dst] = __float2half(k[i]);
      reinterpret_cast<__half*>(vc)[dst] = __float2half(v[i]);
    } else {
      reinterpret_cast<float*>(kc)[dst] = k[i];
      reinterpret_cast<float*>(vc)[dst] = v[i];
    }
  }
}

unsigned ew_blocks(int64_t n) {
  const int64_t b = (n / 4 + 255) / 256;
  return (unsigned)(b < 1 ? 1 : (b > 2048 ? 2048 : b));
}

}  // namespace

hipError_t launch_elementwise(int op, const float* a, const float* b, float* y, int64_t n,
                              hipStream_t s) {
  if (n <= 0) return hipSuccess;
  const dim3 g(ew_blocks(n)), blk(256);
  switch (op) {
    case EW_ADD: UAII_LAUNCH(k_ew<EW_ADD>, g, blk, 0, s, a, b, y, n); break;
    case EW_MUL: UAII_LAUNCH(k_ew<EW_MUL>, g, blk, 0, s, a, b, y, n); break;
    case EW_SILU: UAII_LAUNCH(k_ew<EW_SILU>, g, blk, 0, s, a, b, y, n); break;
    case EW_GELU: UAII_LAUNCH(k_ew<EW_GELU>, g, blk, 0, s, a, b, y, n); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_kv_append(const float* k, const float* v, void* kc, void* vc, int64_t rows,
                            int64_t kv_dim, int hd, int64_t max_seq, int64_t p0, int f16,
                            hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  const int64_t n = rows * kv_dim;
  const int64_t b = (n + 255) / 256;
  UAII_LAUNCH(k_kv_append, dim3((unsigned)(b > 4096 ? 4096 : b)), dim3(256), 0, s, k, v, kc, vc, rows,
              kv_dim, hd, max_seq, p0, f16);
  return hipGetLastError();
}

}  // namespace uaii_hip
