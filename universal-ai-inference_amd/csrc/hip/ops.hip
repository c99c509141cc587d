// ops.hip — small memory-bound kernels of the token loop (gfx950).
//
//   k_embed       token row gather + dequant (transformer.cpp:61-142)
//   k_advance     token/position advance when no lm_head runs (session.cpp:1006-1016)
//   k_rmsnorm     standalone RMSNorm rows (norm.cpp:89-130)
//   k_softmax     probabilities over the vocab (softmax.cpp:11-77)
//   k_argmax      greedy argmax, lowest index wins ties (sampling.cpp:38-50)
//   k_rope        standalone RoPE rows (transformer.cpp:144-220)
//   k_stream_copy plain 16-byte-word copy: the yardstick for HBM rates and for
//                 scaling the memory counters of the other kernels
//   k_stream_read plain read in the decode launch shape: the per-launch floor
//   k_moe_route   router softmax, top-k, renormalised weights (transformer.cpp:446-481,
//                 :565-580)

#include "common.h"
#include "uaii_hip_internal.h"

namespace uaii_hip {
namespace {

// One block per row: each thread decodes chunks of the embedding row. Bit-exact
// with the reference's dequant of the token's row.
template <int FMT>
__global__ void k_embed(DevWeight w, const StepState* st, const int32_t* ids, float* x,
                        float* tap) {
  const int64_t row = blockIdx.x;
  const int64_t tok = st ? (int64_t)st->token : (int64_t)ids[row];
  float* dst = x + row * w.cols;
  if (tok < 0 || tok >= w.rows) {
    // out-of-range ids are rejected on the host; keep the device path in bounds
    for (int64_t i = threadIdx.x; i < w.cols; i += blockDim.x) dst[i] = 0.0f;
    return;
  }
  const int64_t nch = w.a_row / 16;
  for (int64_t t = threadIdx.x; t < nch; t += blockDim.x) {
    ChunkOut o;
    decode_chunk<FMT>(w, tok, t, o);
#pragma unroll
    for (int i = 0; i < 64; ++i) {
      if (i < o.n) {
        dst[o.idx[i]] = o.v[i];
        if (tap) tap[row * w.cols + o.idx[i]] = o.v[i];
      }
    }
  }
}

__global__ void k_advance(StepState* st, int32_t* ids) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  const int p = st->pos + 1;
  // inside the prompt the next token is the prompt's; otherwise the last argmax
  const int next = (p < st->n_prompt) ? ids[p] : st->argmax;
  ids[p] = next;
  st->token = next;
  st->pos = p;
}

__global__ void k_rmsnorm(const float* x, const float* w, float* y, int64_t n, float eps) {
  __shared__ float red[16];
  const float* xr = x + (int64_t)blockIdx.x * n;
  float* yr = y + (int64_t)blockIdx.x * n;
  float ss = 0.0f;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) ss += xr[i] * xr[i];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.0f;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) tot += red[i];
  const float inv = 1.0f / sqrtf(tot / (float)n + eps);
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
    float v = fmul_rn(xr[i], inv);
    if (w) v = fmul_rn(v, w[i]);
    yr[i] = v;
  }
}

// Single block, 1024 threads: max, exp-sum, normalise.
__global__ void k_softmax(const float* x, float* y, int64_t n) {
  __shared__ float red[16];
  __shared__ float bc;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  float m = -INFINITY;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) m = fmaxf(m, x[i]);
  m = wave_max(m);
  if (lane == 0) red[wave] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = red[0];
    for (int i = 1; i < nw; ++i) t = fmaxf(t, red[i]);
    bc = t;
  }
  __syncthreads();
  const float mx = bc;
  float s = 0.0f;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
    const float e = expf(x[i] - mx);
    y[i] = e;
    s += e;
  }
  s = wave_sum(s);
  __syncthreads();
  if (lane == 0) red[wave] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.0f;
    for (int i = 0; i < nw; ++i) t += red[i];
    bc = t > 0.0f ? 1.0f / t : 0.0f;
  }
  __syncthreads();
  const float inv = bc;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) y[i] = y[i] * inv;
}

__global__ void k_argmax(const float* x, int64_t n, int32_t* out) {
  __shared__ float fv[16];
  __shared__ int32_t fi[16];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  float bv = -INFINITY;
  int32_t bi = 0x7fffffff;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
    if (bi == 0x7fffffff || x[i] > bv) { bv = x[i]; bi = (int32_t)i; }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int32_t oi = __shfl_xor(bi, o, 64);
    if (oi != 0x7fffffff && (bi == 0x7fffffff || ov > bv || (ov == bv && oi < bi))) { bv = ov; bi = oi; }
  }
  if (lane == 0) { fv[wave] = bv; fi[wave] = bi; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < nw; ++k) {
      if (fi[k] != 0x7fffffff && (bi == 0x7fffffff || fv[k] > bv || (fv[k] == bv && fi[k] < bi))) {
        bv = fv[k]; bi = fi[k];
      }
    }
    *out = bi;
  }
}

// One thread per rotation pair; row r uses position pos[r * pos_stride].
__global__ void k_rope(float* x, int64_t rows, int64_t dim, int hd, const int32_t* pos,
                       int64_t pos_stride, const float2* tab, int mode) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t pairs_row = dim / 2;
  if (gid >= rows * pairs_row) return;
  const int64_t r = gid / pairs_row, P = gid % pairs_row;
  const int64_t h = P / (hd / 2), p = P % (hd / 2);
  float* v = x + r * dim + h * hd;
  const int64_t i0 = (mode == 2) ? p : 2 * p;
  const int64_t i1 = (mode == 2) ? p + hd / 2 : 2 * p + 1;
  const float2 cs = tab[(int64_t)pos[r * pos_stride] * (hd / 2) + p];
  const float a = v[i0], b = v[i1];
  v[i0] = a * cs.x - b * cs.y;
  v[i1] = a * cs.y + b * cs.x;
}

// Grid-stride copy, 16 bytes per lane per iteration, four loads in flight.
__global__ void __launch_bounds__(256) k_stream_copy(const uint4* __restrict__ src,
                                                     uint4* __restrict__ dst, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + 3 * stride < n; i += 4 * stride) {
    const uint4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
    dst[i] = a; dst[i + stride] = b; dst[i + 2 * stride] = c; dst[i + 3 * stride] = d;
  }
  for (; i < n; i += stride) dst[i] = src[i];
}

// Plain read with the decode GEMVs' launch shape (one block of 512 threads per
// CU, eight independent 16-byte loads in flight per thread, no dependence on
// earlier results): the per-launch floor a kernel reading `n` words could reach.
__global__ void __launch_bounds__(512) k_stream_read(const uint4* __restrict__ src, int64_t n,
                                                    uint32_t* __restrict__ sink) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t acc = 0;
  for (int64_t base = 0; base < n; base += 8 * stride) {
    uint4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t i = base + j * stride + tid;
      v[j] = src[i < n ? i : n - 1];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) acc += v[j].x ^ v[j].w;
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;  // keeps the loads; practically never taken
}

// One wave, E <= 256 router logits: probs = softmax (exp(l - max), times 1/sum,
// softmax.cpp:11-77), then k rounds of the largest remaining prob (ties: the
// lower expert), weights = p / (sum of the k chosen probs). Writes ids[k], w[k].
__global__ void __launch_bounds__(64) k_moe_route(const float* __restrict__ logits, int E, int k,
                                                  int32_t* __restrict__ ids, float* __restrict__ w) {
  const int lane = threadIdx.x;
  float p[4];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane + 64 * j;
    p[j] = e < E ? logits[e] : -INFINITY;
    mx = fmaxf(mx, p[j]);
  }
  mx = wave_max(mx);
  float sum = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane + 64 * j;
    p[j] = e < E ? expf(p[j] - mx) : 0.0f;
    sum += p[j];
  }
  sum = wave_sum(sum);
  const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) p[j] = (lane + 64 * j < E) ? p[j] * inv : -1.0f;
  float mass = 0.0f;
  for (int t = 0; t < k; ++t) {
    // lane-local best (lowest index on ties), then across the wave
    float bv = -1.0f;
    int be = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (p[j] > bv) { bv = p[j]; be = lane + 64 * j; }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int oe = __shfl_xor(be, o, 64);
      if (ov > bv || (ov == bv && oe < be)) { bv = ov; be = oe; }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (lane + 64 * j == be) p[j] = -1.0f;  // taken
    if (lane == 0) {
      ids[t] = (be >= 0 && be < E) ? be : 0;
      w[t] = bv;
    }
    mass += bv;
  }
  if (!(mass > 0.0f)) mass = 1.0f;
  if (lane == 0) {
    for (int t = 0; t < k; ++t) w[t] = w[t] / mass;
  }
}

}  // namespace

thread_local LaunchEvents g_launch_events;

hipError_t launch_moe_route(const float* logits, int n_experts, int k, int32_t* ids, float* w,
                            hipStream_t s) {
  if (n_experts < 1 || n_experts > 256 || k < 1 || k > 8 || k > n_experts) return hipErrorInvalidValue;
  UAII_LAUNCH(k_moe_route, dim3(1), dim3(64), 0, s, logits, n_experts, k, ids, w);
  return hipGetLastError();
}

hipError_t launch_read(const void* src, int64_t n16, uint32_t* sink, hipStream_t s) {
  if (n16 <= 0) return hipSuccess;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return hipErrorInvalidDevice;
  UAII_LAUNCH(k_stream_read, dim3((unsigned)cus), dim3(512), 0, s, (const uint4*)src, n16, sink);
  return hipGetLastError();
}

hipError_t launch_copy(const void* src, void* dst, int64_t n16, hipStream_t s) {
  if (n16 <= 0) return hipSuccess;
  int64_t blocks = (n16 + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  UAII_LAUNCH(k_stream_copy, dim3((unsigned)blocks), dim3(256), 0, s,
                     (const uint4*)src, (uint4*)dst, n16);
  return hipGetLastError();
}

hipError_t launch_embed(const DevWeight& w, const StepState* st, float* x, float* tap,
                        hipStream_t s) {
  UAII_FOR_TYPE(w.type, UAII_LAUNCH(k_embed<FT>, dim3(1), dim3(256), 0, s, w, st,
                                           (const int32_t*)nullptr, x, tap));
  return hipGetLastError();
}

hipError_t launch_embed_rows(const DevWeight& w, const int32_t* ids, int64_t n, float* x,
                             hipStream_t s) {
  if (n <= 0) return hipSuccess;
  UAII_FOR_TYPE(w.type, UAII_LAUNCH(k_embed<FT>, dim3((unsigned)n), dim3(256), 0, s, w,
                                           (const StepState*)nullptr, ids, x, (float*)nullptr));
  return hipGetLastError();
}

hipError_t launch_advance(StepState* st, int32_t* ids, hipStream_t s) {
  UAII_LAUNCH(k_advance, dim3(1), dim3(64), 0, s, st, ids);
  return hipGetLastError();
}

hipError_t launch_rmsnorm(const float* x, const float* w, float* y, int64_t rows, int64_t n,
                          float eps, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  UAII_LAUNCH(k_rmsnorm, dim3((unsigned)rows), dim3(256), 0, s, x, w, y, n, eps);
  return hipGetLastError();
}

hipError_t launch_softmax(const float* x, float* y, int64_t n, hipStream_t s) {
  UAII_LAUNCH(k_softmax, dim3(1), dim3(1024), 0, s, x, y, n);
  return hipGetLastError();
}

hipError_t launch_argmax(const float* x, int64_t n, int32_t* out, hipStream_t s) {
  UAII_LAUNCH(k_argmax, dim3(1), dim3(1024), 0, s, x, n, out);
  return hipGetLastError();
}

hipError_t launch_rope(float* x, int64_t rows, int64_t dim, int head_dim, const int32_t* pos,
                       int64_t pos_stride, const float2* tab, int mode, hipStream_t s) {
  const int64_t total = rows * (dim / 2);
  if (total <= 0) return hipSuccess;
  UAII_LAUNCH(k_rope, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, x, rows,
                     dim, head_dim, pos, pos_stride, tab, mode);
  return hipGetLastError();
}

}  // namespace uaii_hip
