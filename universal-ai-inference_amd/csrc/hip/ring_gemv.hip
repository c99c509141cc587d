// ring_gemv.hip — one decode GEMV with its weights streamed through an LDS ring (gfx950).
//
// Replaces quant_gemm_f32 at M = 1 (libs/uaii-kernels/src/quant_gemm.cpp:22-70)
// plus the residual add_f32 (elementwise.cpp:99-110) for the projections whose
// output is added to the residual stream (attention output O and FFN down), on
// Q4_0 weights with K a multiple of 2048 (up to 16384).
//
// One block per CU, 12 waves. Waves 8..11 (loaders) only move bytes: the block
// owns a contiguous run of stages of R = 16 / ncp consecutive rows (ncol = K /
// 2048 chunk columns of 64 16-byte chunks, ncp the next power of two), each
// stage 16 lines of 1 KiB (global_load_lds_dwordx4, 64 lanes x 16 bytes) and 8
// lines of 256 bytes (global_load_lds_dword) of the split weight layout, 4 + 2
// DMA instructions per loader wave; a stage that needs fewer lines pads with
// reads of a small resident buffer, so every stage costs each loader the same
// vmcnt and the waits are immediates. Waves 0..7 compute: compute wave w takes
// chunk column w % ncp of rows 2 (w / ncp), +1, with the x values of its column
// held in registers as f16 hi + lo pairs scaled by a power of two per chunk
// (v_dot2_f32_f16 on the nibbles as f16 subnormals, exact products, f32 sums),
// and reduces two stages at a time with DPP row operations. The loaders never
// wait for the dot products: the first two stages go out with the input loads,
// then stages are consumed in pairs and the ring deepens to NS - 2 stages ahead.
// Partial row sums per column go to LDS; the epilogue adds the columns in order
// and the residual, and writes the output (and its tap).

#include "common.h"
#include "uaii_hip_internal.h"

#include <mutex>

namespace uaii_hip {
namespace {

constexpr int NCW = 8;             // compute waves
constexpr int NLW = 4;             // loader waves
constexpr int NTH = (NCW + NLW) * 64;
constexpr int SQ = 16384;          // 16-byte-line region of a stage
constexpr int SB = SQ + 2048;      // stage bytes
constexpr int LX4 = 4, LX1 = 2;    // DMA instructions per loader wave per stage
constexpr int ND = LX4 + LX1;
constexpr int PART_MAX = 2048;     // partial row sums per block (floats)

// Compiler-only ordering point (no instruction).
__device__ __forceinline__ void cfence() { __atomic_signal_fence(__ATOMIC_SEQ_CST); }

// Block barrier ordering LDS only: no wait for the loaders' DMA stages in flight.
__device__ __forceinline__ void block_sync() {
  cfence();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  cfence();
}

// s_waitcnt vmcnt(N) (0 <= N < 64), expcnt / lgkmcnt untouched.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt immediate");
  cfence();
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
  cfence();
}

// LDS DMA: the LDS address is the asm's M0 operand (the compiler writes M0);
// s_nop 0 is the wait state an LDS DMA needs after an M0 write.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"{m0}"(lds), "v"(g) : "memory");
}
__device__ __forceinline__ void dma4(const void* g, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %1, off" ::"{m0}"(lds), "v"(g) : "memory");
}
// LDS byte address of a pointer into LDS: the low half of its generic address
// (the LDS aperture base is the high half); no address-space cast, whose null
// check the backend fails to select here.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)reinterpret_cast<uintptr_t>(p));
}

typedef _Float16 lh2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(lh2, a), __builtin_bit_cast(lh2, b), c, false);
}
__device__ __forceinline__ float pow2f(int k) { return __uint_as_float((uint32_t)(k + 127) << 23); }
__device__ __forceinline__ uint32_t hbits(_Float16 h) { return (uint32_t)__builtin_bit_cast(uint16_t, h); }

// hi = the nearest multiples of the grid G (|hi| / G <= 2048, exact in f16, so
// the nibble * hi sums of a chunk are exact in f32), lo = the rest in f16
template <int G>
__device__ __forceinline__ float grid_round(float a) {
  static_assert(G == 1 || G == 16, "grid 1 or 16");
  if constexpr (G == 1) return rintf(a);
  else return (a + 201326592.0f) - 201326592.0f;  // |a| < 2^26: the ulp of 1.5 * 2^27 is 16
}
template <int G>
__device__ __forceinline__ void split2(float a, float b, uint32_t& hi, uint32_t& lo) {
  const float ar = grid_round<G>(a), br = grid_round<G>(b);
  const _Float16 ah = (_Float16)ar, bh = (_Float16)br;
  const _Float16 al = (_Float16)(a - ar), bl = (_Float16)(b - br);
  hi = hbits(ah) | (hbits(bh) << 16);
  lo = hbits(al) | (hbits(bl) << 16);
}

// ---- plan -----------------------------------------------------------------------------

// Stage geometry of a Q4_0 matrix with K columns (K % 2048 == 0, K <= 16384).
struct Geo {
  int ncol, ncp, R;     // chunk columns, its power-of-two cover, rows per stage
  int64_t arow, brow;   // payload / scale bytes per row
  int nl, sl;           // 1 KiB and 256-byte lines per stage
};

__host__ __device__ __forceinline__ Geo geo_of(int64_t K) {
  Geo g;
  g.ncol = (int)(K / 2048);
  g.ncp = 1;
  while (g.ncp < g.ncol) g.ncp <<= 1;
  g.R = 16 / g.ncp;
  g.arow = K / 2;
  g.brow = K / 16;
  g.nl = (int)(g.R * K / 2048);
  g.sl = (int)(g.R * K / 4096);
  return g;
}


struct Seg {
  const uint8_t* p16[LX4];       // this wave's 1 KiB lines
  const uint8_t* p4[LX1];        // and 256-byte lines
  uint32_t o16[LX4], o4[LX1];    // byte offset in the stage, or ~0u for a padding line
  int64_t s16, s4;               // per-stage advance of the real lines
  int left;                      // stages left in the run
};


// One stage's lines into the stage at LDS address slot_lds; the run advances.
__device__ __forceinline__ void issue_fast(Seg& sg, uint32_t slot_lds, uint32_t pad_lds, int lane) {
#pragma unroll
  for (int u = 0; u < LX4; ++u) {
    const bool real = sg.o16[u] != ~0u;
    dma16(sg.p16[u] + 16 * lane, real ? slot_lds + sg.o16[u] : pad_lds);
    if (real) sg.p16[u] += sg.s16;
  }
#pragma unroll
  for (int u = 0; u < LX1; ++u) {
    const bool real = sg.o4[u] != ~0u;
    dma4(sg.p4[u] + 4 * lane, real ? slot_lds + sg.o4[u] : pad_lds);
    if (real) sg.p4[u] += sg.s4;
  }
}


// Cross-lane sums and maxima with DPP row operations (full-rate VALU) instead
// of LDS permutes: within each 16-lane row xor 1, xor 2 (quad_perm), then the
// half-row and row mirrors; across the 4 rows with readlane.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float rl(float v, int k) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), k));
}
template <int N>  // N = 8 or 16 lanes
__device__ __forceinline__ float group_sum(float v) {
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp<0x141>(v);  // row_half_mirror
  if (N == 16) v += dpp<0x140>(v);  // row_mirror
  return v;
}
__device__ __forceinline__ float wave_total(float v) {
  v = group_sum<16>(v);
  return (rl(v, 0) + rl(v, 16)) + (rl(v, 32) + rl(v, 48));
}

// x values of one 32-element chunk as f16 hi/lo pairs (the order the Q4_0 nibble
// masks produce: word i -> (x[4i], x[4i+2]), (x[16+4i], x[16+4i+2]) / 16,
// (x[4i+1], x[4i+3]), (x[16+4i+1], x[16+4i+3]) / 16), scaled by 2^sh with the
// chunk's largest |x| * 2^sh in [2^14, 2^15); c = (sum of the 32 x, 2^(24 - sh)).
struct XP {
  uint4 p[8];
  float2 c;
};

__device__ __forceinline__ void make_pairs(const float* v, XP& xp) {
  float m = 0.0f, s0 = 0.0f, s1 = 0.0f;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    m = fmaxf(m, fmaxf(fabsf(v[k]), fabsf(v[k + 16])));
    s0 += v[k];
    s1 += v[k + 16];
  }
  const int e = (int)((__float_as_uint(m * 1.001f) >> 23) & 0xffu) - 126;
  const int sh = (m > 0.0f) ? max(-100, min(100, 15 - e)) : 0;
  const float S = pow2f(sh), S16 = pow2f(sh - 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t h0, l0, h1, l1, h2, l2, h3, l3;
    split2<16>(v[4 * i] * S, v[4 * i + 2] * S, h0, l0);
    split2<1>(v[16 + 4 * i] * S16, v[16 + 4 * i + 2] * S16, h1, l1);
    split2<16>(v[4 * i + 1] * S, v[4 * i + 3] * S, h2, l2);
    split2<1>(v[16 + 4 * i + 1] * S16, v[16 + 4 * i + 3] * S16, h3, l3);
    xp.p[2 * i] = make_uint4(h0, h1, h2, h3);
    xp.p[2 * i + 1] = make_uint4(l0, l1, l2, l3);
  }
  xp.c = make_float2(s0 + s1, pow2f(24 - sh));
}

// One Q4_0 block (16 nibble bytes, f16 scale d) against its chunk:
// d * sum (q - 8) x = d * (sum q x - 8 sum x)  (gguf_dequant.cpp Q4_0 decode).
__device__ __forceinline__ float dot_q4(uint4 qv, uint32_t sbits, const XP& xp) {
  float sh = 0.0f, sl = 0.0f;
  const uint32_t w4[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t q = w4[i], q8 = q >> 8;
    const uint32_t p0 = q & 0x000F000Fu, p1 = q & 0x00F000F0u;
    const uint32_t p2 = q8 & 0x000F000Fu, p3 = q8 & 0x00F000F0u;
    const uint4 H = xp.p[2 * i], L = xp.p[2 * i + 1];
    sh = dot2(p0, H.x, sh); sl = dot2(p0, L.x, sl);
    sh = dot2(p1, H.y, sh); sl = dot2(p1, L.y, sl);
    sh = dot2(p2, H.z, sh); sl = dot2(p2, L.z, sl);
    sh = dot2(p3, H.w, sh); sl = dot2(p3, L.w, sl);
  }
  const float s = (sh + sl) * xp.c.y;
  return h2f((uint16_t)(sbits & 0xffffu)) * (s - 8.0f * xp.c.x);
}


// The RMSNorm weights of this wave's chunk, loaded ahead of the device-wide
// wait that precedes their phase (they do not depend on it).
__device__ __forceinline__ void load_norm(const float* norm_w, const Geo& ge, bool comp, int wave, int lane,
                                          float* w) {
  const int c = wave % ge.ncp;
  const int64_t t = (int64_t)c * 64 + lane;
  if (comp && c < ge.ncol && norm_w) {
    const float4* w4 = reinterpret_cast<const float4*>(norm_w + 32 * t);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float4 f = w4[k];
      w[4 * k] = f.x; w[4 * k + 1] = f.y; w[4 * k + 2] = f.z; w[4 * k + 3] = f.w;
    }
  } else {
#pragma unroll
    for (int k = 0; k < 32; ++k) w[k] = 0.0f;
  }
}

// This wave's chunk of src (zeros for an idle column).
__device__ __forceinline__ void stage_load(const float* src, const Geo& ge, bool comp, int wave, int lane, float* v) {
  const int c = wave % ge.ncp;
  const int64_t t = (int64_t)c * 64 + lane;
  if (comp && c < ge.ncol) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float4 f = reinterpret_cast<const float4*>(src)[8 * t + k];
      v[4 * k] = f.x; v[4 * k + 1] = f.y; v[4 * k + 2] = f.z; v[4 * k + 3] = f.w;
    }
  } else {
#pragma unroll
    for (int k = 0; k < 32; ++k) v[k] = 0.0f;
  }
}

// RMSNorm (one block barrier when norm) and the pairs of the loaded chunk v.
__device__ __forceinline__ void stage_finish(float* v, bool norm, const float* w, float eps, int64_t K, const Geo& ge,
                                             bool comp, int wave, int lane, float* red, XP& xp) {
  const int c = wave % ge.ncp;
  const bool act = comp && c < ge.ncol;
  if (norm) {
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < 32; ++k) ss += v[k] * v[k];
    ss = wave_total(ss);
    if (comp && wave < ge.ncp && c < ge.ncol && lane == 0) red[c] = ss;
    block_sync();
    float tot = 0.0f;
    for (int k = 0; k < ge.ncol; ++k) tot += red[k];
    const float inv = 1.0f / sqrtf(tot / (float)K + eps);
#pragma unroll
    for (int k = 0; k < 32; ++k) v[k] = fmul_rn(fmul_rn(v[k], inv), w[k]);
  }
  if (act) {
    make_pairs(v, xp);
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) xp.p[k] = make_uint4(0u, 0u, 0u, 0u);
    xp.c = make_float2(0.0f, 0.0f);
  }
}


__device__ __forceinline__ float row_sum(const float* part, const Geo& ge, int i, int r) {
  float v = part[(i * ge.R + r) * ge.ncol];
  for (int c = 1; c < ge.ncol; ++c) v += part[(i * ge.R + r) * ge.ncol + c];
  return v;
}


constexpr int RING_NS = 8;
#ifndef UAII_RING_PRO
#define UAII_RING_PRO 2
#endif
constexpr int RING_PRO = UAII_RING_PRO;

// Wait until at most k stages' DMA lines (k * ND instructions) are outstanding.
__device__ __forceinline__ void wait_stages(int k) {
  switch (k) {
    case 0: wait_vm<0>(); break;
    case 1: wait_vm<ND>(); break;
    case 2: wait_vm<2 * ND>(); break;
    case 3: wait_vm<3 * ND>(); break;
    case 4: wait_vm<4 * ND>(); break;
    case 5: wait_vm<5 * ND>(); break;
    case 6: wait_vm<6 * ND>(); break;
    default: wait_vm<7 * ND>(); break;
  }
}

// Partial row sums of two consecutive stages (the second only if `two`): all
// four rows' bytes are read before any dot, so the dependent chains of the
// reductions overlap.
__device__ __forceinline__ void gemv_stage2(const uint8_t* st0, const uint8_t* st1, bool two, const Geo& ge,
                                            int si, const XP& xp, float* part, int wave, int lane) {
  const int c = wave % ge.ncp, rg = wave / ge.ncp;
  if (c >= ge.ncol) return;
  const int t = c * 64 + lane;
  uint4 qv[4];
  uint32_t sb[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint8_t* st = k < 2 ? st0 : (two ? st1 : st0);
    const int r = 2 * rg + (k & 1);
    qv[k] = *reinterpret_cast<const uint4*>(st + r * ge.arow + 16 * t);
    sb[k] = *reinterpret_cast<const uint16_t*>(st + SQ + r * ge.brow + 2 * t);
  }
  float d[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) d[k] = dot_q4(qv[k], sb[k], xp);
#pragma unroll
  for (int k = 0; k < 4; ++k) d[k] = group_sum<16>(d[k]);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float v = (rl(d[k], 0) + rl(d[k], 16)) + (rl(d[k], 32) + rl(d[k], 48));
    const int r = 2 * rg + (k & 1);
    if (lane == 0 && (k < 2 || two)) part[((si + (k >> 1)) * ge.R + r) * ge.ncol + c] = v;
  }
}

// Stages of a ring GEMV (R rows each).
__host__ __device__ __forceinline__ int64_t ring_stages_of(const RingArgs& a, const Geo& ge) { return a.rows / ge.R; }

// The run of stages that starts at global stage gs and ends at the block's
// last stage gend: each loader wave's lines of the first stage and their
// per-stage advance.
__device__ __forceinline__ void ring_seg(const RingArgs& a, const Geo& ge, int64_t gs, int64_t gend, int lw,
                                         Seg& sg) {
  const int64_t row0 = gs * ge.R;
  const uint8_t* A0 = a.w.a + row0 * ge.arow;
  const uint8_t* B0 = a.w.b + row0 * ge.brow;
#pragma unroll
  for (int u = 0; u < LX4; ++u) {
    const int j = lw + NLW * u;
    sg.p16[u] = j < ge.nl ? A0 + (int64_t)j * 1024 : a.pad;
    sg.o16[u] = j < ge.nl ? (uint32_t)(j * 1024) : ~0u;
  }
#pragma unroll
  for (int u = 0; u < LX1; ++u) {
    const int j = lw + NLW * u;
    sg.p4[u] = j < ge.sl ? B0 + (int64_t)j * 256 : a.pad;
    sg.o4[u] = j < ge.sl ? (uint32_t)(SQ + j * 256) : ~0u;
  }
  sg.s16 = ge.R * ge.arow;
  sg.s4 = ge.R * ge.brow;
  sg.left = (int)(gend - gs);
}

__global__ void __launch_bounds__(NTH, 1) k_ring_gemv(RingArgs a) {
  constexpr int NS = RING_NS;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  __shared__ float red[64];
  uint8_t* ring = lds;
  float* part = reinterpret_cast<float*>(lds + NS * SB + 1024);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool comp = wave < NCW;
  const int lw = wave - NCW;
  const int b = blockIdx.x;
  const Geo ge = geo_of(a.K);
  // The input vector's loads go out first (its fields lead the arguments),
  // ahead of the stage bookkeeping below.
  float w[32];
  load_norm(a.norm_w, ge, comp, wave, lane, w);
  float v[32];
  stage_load(a.x, ge, comp, wave, lane, v);
  // this block's run of stages (counts from the host): f .. f + n - 1
  const int n = a.tq + (b < a.tr ? 1 : 0);
  const int64_t f = (int64_t)b * a.tq + (b < a.tr ? b : a.tr);
  const uint32_t ring_lds = lds_addr(ring), pad_lds = lds_addr(lds + NS * SB);

  Seg sg;
  int issued = 0, islot = 0, cslot = 0;
  auto issue_next = [&]() __attribute__((always_inline)) {
    issue_fast(sg, ring_lds + (uint32_t)(islot * SB), pad_lds, lane);
    ++issued;
    islot = islot + 1 == NS ? 0 : islot + 1;
    if (--sg.left == 0 && issued < n) ring_seg(a, ge, f + issued, f + n, lw, sg);
  };
  // After the input's loads, the first RING_PRO stages: every CU's first
  // requests of a launch complete only when the whole grid's burst has been
  // served, so a small first burst gets the first data (and the input) back
  // sooner. Stages then go in pairs; each pair waits for its two stages, and the
  // loaders refill up to 4 stages per pair (the ring deepens to NS-2 stages ahead).
  block_sync();
  if (!comp && n > 0) {
    ring_seg(a, ge, f, f + n, lw, sg);
    for (int k = 0; k < RING_PRO; ++k)
      if (issued < n) issue_next();
  }
  XP xp;
  stage_finish(v, a.norm_w != nullptr, w, a.eps, a.K, ge, comp, wave, lane, red, xp);
  for (int i = 0; i < n; i += 2) {
    if (!comp) {
      // stages i and i + 1 are in flight (a one-stage first burst leaves i + 1
      // to here), then wait until both have landed
      while (issued < min(i + 2, n)) issue_next();
      wait_stages(issued - min(i + 2, n));
    }
    block_sync();
    if (!comp) {
      const int cap = min(n, i + NS);  // stages below i + NS have a free slot
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (issued < cap) issue_next();
    }
    const uint8_t* st0 = ring + cslot * SB;
    cslot = cslot + 1 == NS ? 0 : cslot + 1;
    const uint8_t* st1 = ring + cslot * SB;
    cslot = cslot + 1 == NS ? 0 : cslot + 1;
    if (comp) gemv_stage2(st0, st1, i + 1 < n, ge, i, xp, part, wave, lane);
  }
  block_sync();
  if (!comp) return;
  // epilogue (gemv.hip's EPI_STORE / EPI_ADD on the block's rows)
  for (int t = tid; t < n * ge.R; t += NCW * 64) {
    const int i = t / ge.R, r = t % ge.R;
    const int64_t gr = (f + i) * ge.R + r;
    float v = row_sum(part, ge, i, r);
    if (a.epi == EPI_ADD) v = a.y[gr] + v;
    a.y[gr] = v;
    if (a.tap) a.tap[gr] = v;
  }
}

int dev_cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  return n;
}

constexpr size_t ring_lds() { return (size_t)RING_NS * SB + 1024 + PART_MAX * 4; }

}  // namespace

bool ring_gemv_supported(const RingArgs& a) {
  if (a.K <= 0 || a.K % 2048 || a.K > 16384 || !a.x || !a.y || !a.pad) return false;
  if (a.epi != EPI_STORE && a.epi != EPI_ADD) return false;
  const Geo ge = geo_of(a.K);
  const DevWeight& w = a.w;
  if (w.type != T_Q4_0 || w.cols != a.K || w.a_row != ge.arow || w.b_row != ge.brow) return false;
  if (a.rows <= 0 || a.rows % ge.R || w.rows < a.rows) return false;
  const int64_t T = a.rows / ge.R;
  const int nblk = dev_cus();
  if (nblk < 1) return false;
  const int64_t most = (T + nblk - 1) / nblk;
  if (most * ge.R * ge.ncol > PART_MAX) return false;
  // the device's per-block LDS less a margin for the static arrays
  return ring_lds() <= (size_t)lds_limit() - 1024;
}

hipError_t prepare_ring_gemv() {
  static std::once_flag once;
  static hipError_t prep = hipSuccess;
  std::call_once(once, [] {
    prep = hipFuncSetAttribute((const void*)k_ring_gemv, hipFuncAttributeMaxDynamicSharedMemorySize, (int)ring_lds());
    int per_cu = 0;
    if (prep == hipSuccess) prep = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_ring_gemv, NTH, ring_lds());
    if (prep == hipSuccess && per_cu < 1) prep = hipErrorInvalidConfiguration;
  });
  return prep;
}

hipError_t launch_ring_gemv(const RingArgs& in, hipStream_t s) {
  if (!ring_gemv_supported(in)) return hipErrorInvalidValue;
  const hipError_t prep = prepare_ring_gemv();
  if (prep != hipSuccess) return prep;
  const int nblk = dev_cus();
  if (nblk <= 0) return hipErrorInvalidDevice;
  RingArgs a = in;
  const int64_t T = ring_stages_of(a, geo_of(a.K));
  a.tq = (int32_t)(T / nblk);
  a.tr = (int32_t)(T % nblk);
  UAII_LAUNCH(k_ring_gemv, dim3(nblk), dim3(NTH), ring_lds(), s, a);
  return hipGetLastError();
}

}  // namespace uaii_hip
