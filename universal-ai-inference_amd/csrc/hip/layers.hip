// layers.hip — every transformer layer of a decode step in one persistent launch (gfx950).
//
// Replaces, for dense SwiGLU decoders whose seven layer matrices share the Q4_0
// block format, the per-layer chain of the token step (gguf.cpp:1000-1209 built
// once per token; transformer.cpp:144-433 attention; quant_gemm.cpp:22-70 for
// every projection): RMSNorm -> QKV (+bias) -> RoPE / KV append -> attention ->
// O + residual -> RMSNorm -> gate/up SwiGLU -> down + residual, layer after layer.
//
// Why one launch: a decode GEMV is 9-66 MB of weights, and a launch per matrix
// loses ~5-8 us to the first memory round trip and the tail of the grid. Here
// one block per CU (all resident) streams its share of every matrix of every
// layer, and of the KV cache, through a ring of LDS stages that runs up to NS-1
// stages ahead, across the points where the layer waits for the whole device.
//
// Block = 12 waves. Waves 8..11 (loaders) only move bytes: each 18 KiB stage is
// 16 lines of 1 KiB (global_load_lds_dwordx4, 64 lanes x 16 bytes) and 8 lines
// of 256 bytes (global_load_lds_dword), 4 + 2 instructions per loader wave; a
// stage that needs fewer lines pads with reads of a small resident buffer, so
// every stage costs each loader the same vmcnt and the waits are immediates.
// Waves 0..7 compute; they never have an LDS load in flight, so their own
// global loads and stores (input vectors, epilogue outputs, device-wide
// counters) return without waiting behind the weight stream.
//
// A matrix of K columns is cut into stages of R = 16 / ncp consecutive rows
// (ncol = K / 2048 columns of 64 16-byte chunks, ncp the next power of two):
// compute wave w takes chunk column w % ncp of rows 2 (w / ncp), +1, with the x
// values of its column held in registers for the whole phase as f16 hi + lo
// pairs scaled by a power of two per chunk (the GEMV's exact v_dot2 scheme:
// v_dot2_f32_f16 on the nibbles as f16 subnormals). Partial row sums per column
// go to LDS; the phase's epilogue adds the columns in order.
//
// Attention: block b < n_kv * S takes kv head b / S, keys [s CB, (s+1) CB) of
// the cached positions 0 .. pos-1 (stages of 32 (hd 128) or 64 (hd 64) keys, K
// then V), online softmax per wave, the 8 wave states merged into one partial
// (o, m, l) per query head. The last block of a kv head to finish (a ticket
// counter) merges the S partials and the new token's own key and value: it
// applies RoPE to k, rounds k and v to f16, appends them to the cache at pos
// and computes their score in f32 — the cached keys the stages read never
// include pos, so the stages can be fetched before the QKV projections exist.
//
// Cross-block data (x, qkv, attn, h, partials) is written with device-scope
// (sc1) stores and read with sc1 loads; a compute wave waits for its stores
// (vmcnt 0; it has no LDS loads in flight) before its block arrives at a
// counter. Device-wide waits: 8 group counters, the last arrival of a group
// bumping a global one (~2 us per barrier), polled by one lane with a bounded
// spin (a timeout sets `fail` and the launch finishes with garbage, which the
// host reports). The last block to finish resets the counters.

#include "common.h"
#include "uaii_hip_internal.h"

#include <algorithm>
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
constexpr int PART_MAX = 2048;     // GEMV partial sums per phase per block (floats)
constexpr int RESID_MAX = 512;     // residual rows per phase per block

typedef unsigned long long u64;

// LayersSync word indices (one 128-byte line each)
constexpr int SY_FAIL = 0;
constexpr int SY_GROUP = 16;       // + 16 g, g < 8
constexpr int SY_ALL = 16 * 9;
constexpr int SY_MERGED = 16 * 10;
constexpr int SY_DONE = 16 * 11;
constexpr int SY_TICK = 16 * 16;   // + 16 h, h < 64

__device__ __forceinline__ u64 ld_ag(const u64* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void st_ag(u64* p, u64 v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ u64 add_ag(u64* p, u64 v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stf(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// Reads of data other blocks wrote in this launch: device-coherent (sc1)
// buffer loads, which skip this XCD's possibly stale L2 copy. They are plain
// (non-atomic) loads, so the compiler issues a batch of them back to back; an
// acquire fence with ordinary loads instead (buffer_inv sc1, invalidating the
// whole L2 under the weight stream) measured ~15 us per phase.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_of(const float* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, 0x7fffffff, 0x00020000);
}
// base wave-uniform (it becomes the buffer resource, held in scalar registers;
// a per-lane base would need a loop over the distinct values), i per lane
__device__ __forceinline__ float ldf(const float* base, int64_t i) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc_of(base), (int)(i * 4), 0, 16));
}
__device__ __forceinline__ float4 ldf4(const float* base, int64_t i) {
  return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rsrc_of(base), (int)(i * 4), 0, 16));
}

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
// (a, b) -> hi = (f16(a), f16(b)), lo = the rest in f16 (attention's q)
__device__ __forceinline__ void split2(float a, float b, uint32_t& hi, uint32_t& lo) {
  const _Float16 ah = (_Float16)a, bh = (_Float16)b;
  const _Float16 al = (_Float16)(a - (float)ah), bl = (_Float16)(b - (float)bh);
  hi = hbits(ah) | (hbits(bh) << 16);
  lo = hbits(al) | (hbits(bl) << 16);
}
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

// Block b's share of T stages: a contiguous run (the first T % nblk blocks
// take one more), so a CU streams consecutive rows of a matrix.
__host__ __device__ __forceinline__ int share(int64_t T, int b, int nblk) {
  return (int)(T / nblk + (b < T % nblk ? 1 : 0));
}
__host__ __device__ __forceinline__ int64_t first_stage(int64_t T, int b, int nblk) {
  return (int64_t)b * (T / nblk) + (b < T % nblk ? b : T % nblk);
}

struct Plan {
  Geo gq, go, gg, gd;         // QKV (K = dim), O (K = q_dim), gate/up (K = dim), down (K = inter)
  int nq, na, no, ng, nd;     // this block's stages per phase
  int64_t fq, fo, fg, fd;     // global index of its first stage per GEMV phase
  int e0, e1, e2, e3, T;      // ends of the QKV, attention, O, gate/up phases; stages per layer
  int64_t total;              // stages of the launch
  int att, ah, S;             // attention unit: kv head ah, split (b % S)
  int64_t k0, k1;             // its cached keys [k0, k1)
  int pos;
};

template <int HD>
__device__ __forceinline__ Plan make_plan(const LayersArgs& a, int b, int nblk, int pos) {
  constexpr int KT = 4096 / HD;  // keys per attention stage
  Plan p;
  p.gq = geo_of(a.dim);
  p.go = geo_of(a.q_dim);
  p.gg = geo_of(a.dim);
  p.gd = geo_of(a.inter);
  p.nq = share((a.q_dim + 2 * a.kv_dim) / p.gq.R, b, nblk);
  p.no = share(a.dim / p.go.R, b, nblk);
  p.ng = share(a.inter / (p.gg.R / 2), b, nblk);
  p.nd = share(a.dim / p.gd.R, b, nblk);
  p.fq = first_stage((a.q_dim + 2 * a.kv_dim) / p.gq.R, b, nblk);
  p.fo = first_stage(a.dim / p.go.R, b, nblk);
  p.fg = first_stage(a.inter / (p.gg.R / 2), b, nblk);
  p.fd = first_stage(a.dim / p.gd.R, b, nblk);
  p.S = a.splits;
  p.pos = pos;
  p.att = b < a.n_kv * p.S;
  p.ah = p.att ? b / p.S : 0;
  p.k0 = p.k1 = 0;
  p.na = 0;
  if (p.att && pos > 0) {
    const int64_t per = (pos + p.S - 1) / p.S;
    const int64_t CB = (per + KT - 1) / KT * KT;
    p.k0 = min((int64_t)(b % p.S) * CB, (int64_t)pos);
    p.k1 = min(p.k0 + CB, (int64_t)pos);
    p.na = (int)((p.k1 - p.k0 + KT - 1) / KT);
  }
  p.e0 = p.nq;
  p.e1 = p.e0 + p.na;
  p.e2 = p.e1 + p.no;
  p.e3 = p.e2 + p.ng;
  p.T = p.e3 + p.nd;
  p.total = (int64_t)p.T * a.n_layers;
  return p;
}

// Payload / scale base addresses of every layer's seven matrices, copied into
// LDS at the start (wq, wk, wv, wo, gate, up, down; a then b): the loaders
// read them there instead of through the scalar cache, whose misses would
// stall the issue of a stage.
constexpr int PT = 14;

// ---- loader side -------------------------------------------------------------------------------
//
// The stages of a phase (and of each matrix within the QKV phase) are a run
// whose lines advance by fixed strides, so the loaders keep, per run, the
// source of each of their lines and add the stride per stage; only at the
// start of a run (7-8 per layer) do they work out addresses from the layer
// table. (Working them out per stage took ~1.1 us of a loader's time per
// 0.7 us stage.)
struct Seg {
  const uint8_t* p16[LX4];       // this wave's 1 KiB lines
  const uint8_t* p4[LX1];        // and 256-byte lines
  uint32_t o16[LX4], o4[LX1];    // byte offset in the stage, or ~0u for a padding line
  int64_t s16, s4;               // per-stage advance of the real lines
  int left;                      // stages left in the run
};

// The run that starts at stage r of layer l (phases end at Plan::e0..e3 and T).
template <int HD>
__device__ __forceinline__ void seg_setup(const LayersArgs& a, const uint64_t* ptab, const Plan& p, int l, int r,
                                          int lw, Seg& sg) {
  const uint64_t* pt = ptab + l * PT;
  // 1 KiB lines: j < c16 from A0 + 1024 j, then from A1; 256-byte lines likewise
  const uint8_t *A0 = a.pad, *A1 = a.pad, *B0 = a.pad, *B1 = a.pad;
  int n16 = 0, c16 = 0, n4 = 0, c4 = 0, run = 1;
  int64_t da = 0, db = 0;
  auto single = [&](int m, int64_t row0, const Geo& ge, int stages) {
    A0 = reinterpret_cast<const uint8_t*>(pt[2 * m]) + row0 * ge.arow;
    B0 = reinterpret_cast<const uint8_t*>(pt[2 * m + 1]) + row0 * ge.brow;
    n16 = c16 = ge.nl;
    n4 = c4 = ge.sl;
    da = ge.R * ge.arow;
    db = ge.R * ge.brow;
    run = stages;
  };
  if (r < p.e0) {
    const int64_t row0 = (p.fq + r) * p.gq.R;
    const int left = p.e0 - r;
    if (row0 < a.q_dim) {
      single(0, row0, p.gq, min((int64_t)left, (a.q_dim - row0) / p.gq.R));
    } else if (row0 < a.q_dim + a.kv_dim) {
      single(1, row0 - a.q_dim, p.gq, min((int64_t)left, (a.q_dim + a.kv_dim - row0) / p.gq.R));
    } else {
      single(2, row0 - a.q_dim - a.kv_dim, p.gq, left);
    }
  } else if (r < p.e1) {
    constexpr int KT = 4096 / HD;
    const int64_t layer_bytes = a.kv_dim * a.max_seq * 2;
    const uint8_t* kb = static_cast<const uint8_t*>(a.kv) + (int64_t)l * 2 * layer_bytes;
    const int64_t off = ((int64_t)p.ah * a.max_seq + p.k0 + (int64_t)(r - p.e0) * KT) * HD * 2;
    A0 = kb + off;
    A1 = kb + layer_bytes + off;
    n16 = 16;
    c16 = 8;
    da = KT * HD * 2;
    run = p.e1 - r;
  } else if (r < p.e2) {
    single(3, (p.fo + (r - p.e1)) * p.go.R, p.go, p.e2 - r);
  } else if (r < p.e3) {
    const int64_t j0 = (p.fg + (r - p.e2)) * (p.gg.R / 2);
    A0 = reinterpret_cast<const uint8_t*>(pt[8]) + j0 * p.gg.arow;
    A1 = reinterpret_cast<const uint8_t*>(pt[10]) + j0 * p.gg.arow;
    B0 = reinterpret_cast<const uint8_t*>(pt[9]) + j0 * p.gg.brow;
    B1 = reinterpret_cast<const uint8_t*>(pt[11]) + j0 * p.gg.brow;
    n16 = p.gg.nl;
    c16 = p.gg.nl / 2;
    n4 = p.gg.sl;
    c4 = p.gg.sl / 2;
    da = (p.gg.R / 2) * p.gg.arow;
    db = (p.gg.R / 2) * p.gg.brow;
    run = p.e3 - r;
  } else {
    single(6, (p.fd + (r - p.e3)) * p.gd.R, p.gd, p.T - r);
  }
#pragma unroll
  for (int u = 0; u < LX4; ++u) {
    const int j = lw + NLW * u;
    sg.p16[u] = j < n16 ? (j < c16 ? A0 + (int64_t)j * 1024 : A1 + (int64_t)(j - c16) * 1024) : a.pad;
    sg.o16[u] = j < n16 ? (uint32_t)(j * 1024) : ~0u;
  }
#pragma unroll
  for (int u = 0; u < LX1; ++u) {
    const int j = lw + NLW * u;
    sg.p4[u] = j < n4 ? (j < c4 ? B0 + (int64_t)j * 256 : B1 + (int64_t)(j - c4) * 256) : a.pad;
    sg.o4[u] = j < n4 ? (uint32_t)(SQ + j * 256) : ~0u;
  }
  sg.s16 = da;
  sg.s4 = db;
  sg.left = run;
}

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

// ---- compute side ---------------------------------------------------------------------------

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
__device__ __forceinline__ float wave_top(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  return fmaxf(fmaxf(rl(v, 0), rl(v, 16)), fmaxf(rl(v, 32), rl(v, 48)));
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

// Phase input: this compute wave's chunk column of src (optionally RMSNorm'd,
// norm.cpp:89-130: x * (1 / sqrt(mean(x^2) + eps)) * w, two roundings). Every
// wave of the block calls it (one block barrier when norm_w is set).
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
template <bool SC1>
__device__ __forceinline__ void stage_load(const float* src, const Geo& ge, bool comp, int wave, int lane, float* v) {
  const int c = wave % ge.ncp;
  const int64_t t = (int64_t)c * 64 + lane;
  if (comp && c < ge.ncol) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float4 f = SC1 ? ldf4(src, 32 * t + 4 * k) : reinterpret_cast<const float4*>(src)[8 * t + k];
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

// w: this wave's RMSNorm weights from load_norm (norm set) or unused. SC1:
// src was written in this launch by other blocks (device-coherent loads).
template <bool SC1 = true>
__device__ __forceinline__ void stage_in(const float* src, bool norm, const float* w, float eps, int64_t K,
                                         const Geo& ge, bool comp, int wave, int lane, float* red, XP& xp) {
  const int c = wave % ge.ncp;
  const bool act = comp && c < ge.ncol;
  float v[32];
  const int64_t t = (int64_t)c * 64 + lane;
  if (act) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float4 f = SC1 ? ldf4(src, 32 * t + 4 * k) : reinterpret_cast<const float4*>(src)[8 * t + k];
      v[4 * k] = f.x; v[4 * k + 1] = f.y; v[4 * k + 2] = f.z; v[4 * k + 3] = f.w;
    }
  } else {
#pragma unroll
    for (int k = 0; k < 32; ++k) v[k] = 0.0f;
  }
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
  } else {  // an idle column: defined values, so no earlier phase's pairs stay live
#pragma unroll
    for (int k = 0; k < 8; ++k) xp.p[k] = make_uint4(0u, 0u, 0u, 0u);
    xp.c = make_float2(0.0f, 0.0f);
  }
}

// Partial row sums of one GEMV stage: wave -> (column w % ncp, rows 2 (w / ncp), +1).
__device__ __forceinline__ void gemv_stage(const uint8_t* st, const Geo& ge, int si, const XP& xp, float* part, int wave,
                                  int lane) {
  const int c = wave % ge.ncp, rg = wave / ge.ncp;
  if (c >= ge.ncol) return;
  const int t = c * 64 + lane;
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    const int r = 2 * rg + rr;
    const uint4 qv = *reinterpret_cast<const uint4*>(st + r * ge.arow + 16 * t);
    const uint32_t sb = *reinterpret_cast<const uint16_t*>(st + SQ + r * ge.brow + 2 * t);
    const float d = wave_total(dot_q4(qv, sb, xp));
    if (lane == 0) part[(si * ge.R + r) * ge.ncol + c] = d;
  }
}

__device__ __forceinline__ float row_sum(const float* part, const Geo& ge, int i, int r) {
  float v = part[(i * ge.R + r) * ge.ncol];
  for (int c = 1; c < ge.ncol; ++c) v += part[(i * ge.R + r) * ge.ncol + c];
  return v;
}

// RoPE (transformer.cpp:144-220): element d of a head after rotation by the
// angle table of position pos; mode 0 pairs (2i, 2i+1), mode 2 pairs (i, i + hd/2).
// `base` is wave-uniform; the head starts at element h0 of it.
__device__ __forceinline__ float rope_at(const float* base, int64_t h0, int d, int hd, int mode, const float2* rope,
                                         int pos) {
  if (mode == 2) {
    const int half = hd / 2, i = d % half;
    const float x0 = ldf(base, h0 + i), x1 = ldf(base, h0 + i + half);
    const float2 cs = rope[(int64_t)pos * half + i];
    return d < half ? x0 * cs.x - x1 * cs.y : x0 * cs.y + x1 * cs.x;
  }
  const int d0 = d & ~1;
  const float x0 = ldf(base, h0 + d0), x1 = ldf(base, h0 + d0 + 1);
  const float2 cs = rope[(int64_t)pos * (hd / 2) + (d0 >> 1)];
  return (d & 1) ? x0 * cs.y + x1 * cs.x : x0 * cs.x - x1 * cs.y;
}

// Attention state of one compute lane: lanes lk = lane % LK own dims
// 8 lk .. 8 lk + 7 of key lane / LK of the wave's KW keys per stage.
template <int HD, int G>
struct Att {
  static constexpr int LK = HD / 8, KW = 64 / LK;
  float m[G], l[G], o[G][8];
};

// (q * scale) of the group's G heads after RoPE as f16 hi / lo pairs in LDS:
// qp[(g * LK + lk) * 8 + i] = hi pair i, + 4 + i = lo pair i of dims 8 lk .. 8 lk + 7.
// Compute thread t < G * LK fills (g, lk) = (t / LK, t % LK); a block barrier follows.
template <int HD, int G>
__device__ __forceinline__ void att_prep_q(const LayersArgs& a, const Plan& p, uint32_t* qp, int t) {
  constexpr int LK = HD / 8;
  if (t >= G * LK) return;
  const int g = t / LK, lk = t % LK;
  const float scale = 1.0f / sqrtf((float)HD);
  const int64_t h0 = (int64_t)(p.ah * G + g) * HD;
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = rope_at(a.qkv, h0, 8 * lk + e, HD, a.rope_mode, a.rope, p.pos) * scale;
  uint32_t hi[4], lo[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) split2(v[2 * i], v[2 * i + 1], hi[i], lo[i]);
  uint4* dst = reinterpret_cast<uint4*>(qp + t * 8);
  dst[0] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
  dst[1] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
}

template <int HD, int G>
__device__ __forceinline__ void att_init(Att<HD, G>& s) {
#pragma unroll
  for (int g = 0; g < G; ++g) {
    s.m[g] = -INFINITY;
    s.l[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s.o[g][e] = 0.0f;
  }
}

template <int HD, int G>
__device__ __forceinline__ void att_stage(const uint8_t* st, int64_t t0, int64_t k1, const uint32_t* qp, Att<HD, G>& s,
                                          int wave, int lane) {
  constexpr int LK = Att<HD, G>::LK, KW = Att<HD, G>::KW;
  const int lk = lane % LK, kq = lane / LK;
  const int kw = wave * KW + kq;
  const bool valid = t0 + kw < k1;
  const uint4 kk = *reinterpret_cast<const uint4*>(st + kw * HD * 2 + 16 * lk);
  const uint4 vv = *reinterpret_cast<const uint4*>(st + 8192 + kw * HD * 2 + 16 * lk);
  float sc[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const uint4 qh = reinterpret_cast<const uint4*>(qp)[(g * LK + lk) * 2];
    const uint4 ql = reinterpret_cast<const uint4*>(qp)[(g * LK + lk) * 2 + 1];
    float t = 0.0f;
    t = dot2(kk.x, qh.x, t); t = dot2(kk.x, ql.x, t);
    t = dot2(kk.y, qh.y, t); t = dot2(kk.y, ql.y, t);
    t = dot2(kk.z, qh.z, t); t = dot2(kk.z, ql.z, t);
    t = dot2(kk.w, qh.w, t); t = dot2(kk.w, ql.w, t);
    t = group_sum<LK>(t);
    sc[g] = valid ? t : -INFINITY;
  }
  float vf[8];
  const uint32_t w4[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    vf[2 * e] = h2f((uint16_t)(w4[e] & 0xffffu));
    vf[2 * e + 1] = h2f((uint16_t)(w4[e] >> 16));
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float mnew = fmaxf(s.m[g], wave_top(sc[g]));
    const float pv = valid ? expf(sc[g] - mnew) : 0.0f;
    const float alpha = (s.m[g] == -INFINITY) ? 0.0f : expf(s.m[g] - mnew);
    s.l[g] = s.l[g] * alpha + wave_total(lk == 0 ? pv : 0.0f);
#pragma unroll
    for (int e = 0; e < 8; ++e) s.o[g][e] = s.o[g][e] * alpha + (valid ? pv * vf[e] : 0.0f);
    s.m[g] = mnew;
  }
}

// ---- the kernel -------------------------------------------------------------------------------

// Bytes of the region shared by the GEMV partials / residuals and the
// attention's q pairs, wave states and merge values.
template <int HD, int G>
__host__ __device__ constexpr int layers_misc() {
  return (2 * NCW * G + NCW * G * HD) * 4 > (PART_MAX + RESID_MAX) * 4 ? (2 * NCW * G + NCW * G * HD) * 4
                                                                       : (PART_MAX + RESID_MAX) * 4;
}

template <int HD, int G, int NS>
__global__ void __launch_bounds__(NTH, 1) k_layers(LayersArgs a) {
  static_assert((NS - 2) * ND < 64, "vmcnt immediate");
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  __shared__ float red[64];
  __shared__ int s_flag;
  uint8_t* ring = lds;
  uint8_t* pad_lds = lds + NS * SB;
  float* misc = reinterpret_cast<float*>(pad_lds + 1024);
  float* part = misc;               // GEMV partial sums
  float* resid = misc + PART_MAX;   // residual values of the phase's rows
  float* wm = misc;                 // attention wave states (aliases part / resid)
  float* wl = misc + NCW * G;
  float* wo = misc + 2 * NCW * G;
  float* mls = misc;                // merge: (m, l) of every split (after the wave states are used)
  uint32_t* qp = reinterpret_cast<uint32_t*>(misc);  // attention q pairs (before the wave states)

  int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool comp = wave < NCW;
  const int lw = wave - NCW;
  const int nblk = gridDim.x, b = blockIdx.x;
  const int pos = __builtin_amdgcn_readfirstlane(a.state->pos);
  const Plan p = make_plan<HD>(a, b, nblk, pos);
  uint64_t* ptab = reinterpret_cast<uint64_t*>(misc + (layers_misc<HD, G>() / 4));
  // norms and biases through the constant address space: scalar loads, which a
  // loader wave's vmcnt does not count
  typedef const __attribute__((address_space(4))) LayerW CLayerW;
  CLayerW* lws = (CLayerW*)a.layers;
  u64* sy = a.sync->w;
  const int ngrp = nblk < 8 ? nblk : 8;
  const int grp = b & 7;
  const u64 in_grp = (u64)((nblk - grp + 7) / 8);
  u64 nbar = 0;
  bool dead = false;

  // loaders: the run being fetched and the position (layer il, stage ir, slot
  // islot) of the next stage; everyone: the slot of the stage consumed next
  Seg sg;
  int il = 0, ir = 0, islot = 0;
  const uint32_t ring_lds = lds_addr(ring), pad_lds_addr = lds_addr(pad_lds);
  int cslot = 0;
  int64_t issued = 0;
  auto issue_next = [&]() __attribute__((always_inline)) {
    issue_fast(sg, ring_lds + (uint32_t)(islot * SB), pad_lds_addr, lane);
    ++issued;
    islot = islot + 1 == NS ? 0 : islot + 1;
    if (++ir == p.T) { ir = 0; ++il; }
    if (--sg.left == 0 && issued < p.total) seg_setup<HD>(a, ptab, p, il, ir, lw, sg);
  };
  // Stage gi: the loaders wait for their lines of it (at most NS-2 later stages
  // outstanding), one block barrier, then they refill the slot of stage gi-1,
  // which every compute wave finished reading before this barrier.
  auto stage_begin = [&](int64_t gi) __attribute__((always_inline)) -> const uint8_t* {
    if (!comp) {
      if (gi + NS - 2 < p.total) wait_vm<(NS - 2) * ND>();
      else wait_vm<0>();
    }
    block_sync();
    if (!comp && issued < p.total) issue_next();
    const uint8_t* st = ring + cslot * SB;
    cslot = cslot + 1 == NS ? 0 : cslot + 1;
    return st;
  };
  auto stage_end = [&](int64_t) __attribute__((always_inline)) {};
  // bounded poll of one counter by lane 0 of wave 0 (a compute wave)
  auto poll = [&](int idx, u64 target) __attribute__((always_inline)) {
    if (tid == 0 && !dead) {
      const u64 t0 = __builtin_amdgcn_s_memrealtime();
      while (ld_ag(&sy[idx]) < target) {
        __builtin_amdgcn_s_sleep(1);
        if (__builtin_amdgcn_s_memrealtime() - t0 > a.timeout) {
          st_ag(&sy[SY_FAIL], 1);
          dead = true;
          break;
        }
      }
    }
  };
  // compute waves' global stores complete, then the whole grid
  auto grid_sync = [&]() __attribute__((always_inline)) {
    if (comp) wait_vm<0>();
    block_sync();
    ++nbar;
    if (tid == 0) {
      const u64 old = add_ag(&sy[SY_GROUP + 16 * grp], 1);
      if (old + 1 == nbar * in_grp) add_ag(&sy[SY_ALL], 1);
    }
    poll(SY_ALL, nbar * (u64)ngrp);
    block_sync();
  };

  // the pointer table, then the first NS-1 stages
  for (int t = tid; t < a.n_layers * PT; t += NTH) {
    const int l = t / PT, k = t % PT;
    const LayerW& w = a.layers[l];
    const DevWeight& m = k < 2 ? w.wq : k < 4 ? w.wk : k < 6 ? w.wv : k < 8 ? w.wo : k < 10 ? w.gate
                       : k < 12 ? w.up : w.down;
    ptab[t] = reinterpret_cast<uint64_t>((k & 1) ? m.b : m.a);
  }
  wait_vm<0>();
  block_sync();
  if (!comp && p.total > 0) {
    seg_setup<HD>(a, ptab, p, 0, 0, lw, sg);
    for (int k = 0; k < NS - 1; ++k)
      if (issued < p.total) issue_next();
  }

  int64_t g = 0;
  XP xp;
  float wpre[32];  // RMSNorm weights of the next normalised phase
  for (int l = 0; l < a.n_layers; ++l) {
    // per-lane values are recomputed inside each layer instead of being kept
    // live (or spilled) across the whole loop
    asm volatile("" : "+v"(tid), "+v"(lane));
    const float* attn_norm = lws[l].attn_norm;
    const float* ffn_norm = lws[l].ffn_norm;
    const float* bq = lws[l].bq;
    const float* bk = lws[l].bk;
    const float* bv = lws[l].bv;

    // ---- Q, K, V projections (raw, + bias) ----
    if (l == 0) load_norm(attn_norm, p.gq, comp, wave, lane, wpre);
    stage_in(a.x, attn_norm != nullptr, wpre, a.eps, a.dim, p.gq, comp, wave, lane, red, xp);
    for (int i = 0; i < p.nq; ++i, ++g) {
      const uint8_t* st = stage_begin(g);
      if (comp) gemv_stage(st, p.gq, i, xp, part, wave, lane);
      stage_end(g);
    }
    block_sync();
    if (comp) {
      const int n = p.nq * p.gq.R;
      for (int t = tid; t < n; t += NCW * 64) {
        const int i = t / p.gq.R, r = t % p.gq.R;
        float v = row_sum(part, p.gq, i, r);
        const int64_t gr = (p.fq + i) * p.gq.R + r;
        const float* bias = gr < a.q_dim ? bq : (gr < a.q_dim + a.kv_dim ? bk : bv);
        const int64_t bi = gr < a.q_dim ? gr : (gr < a.q_dim + a.kv_dim ? gr - a.q_dim : gr - a.q_dim - a.kv_dim);
        if (bias) v = v + bias[bi];
        stf(a.qkv + gr, v);
      }
    }
    grid_sync();

    // ---- attention over the cached keys, merged by the head's last block ----
    if (p.att) {
      Att<HD, G> s;
      if (comp) att_prep_q<HD, G>(a, p, qp, tid);
      att_init<HD, G>(s);
      block_sync();
      constexpr int KT = 4096 / HD;
      for (int i = 0; i < p.na; ++i, ++g) {
        const uint8_t* st = stage_begin(g);
        if (comp) att_stage<HD, G>(st, p.k0 + (int64_t)i * KT, p.k1, qp, s, wave, lane);
        stage_end(g);
      }
      if (comp) {
        constexpr int LK = Att<HD, G>::LK;
#pragma unroll
        for (int gg = 0; gg < G; ++gg)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            float t = s.o[gg][e];
#pragma unroll
            for (int o2 = LK; o2 < 64; o2 <<= 1) t += __shfl_xor(t, o2, 64);
            s.o[gg][e] = t;
          }
#pragma unroll
        for (int gg = 0; gg < G; ++gg) {
          if (lane == 0) {
            wm[wave * G + gg] = s.m[gg];
            wl[wave * G + gg] = s.l[gg];
          }
          if (lane < LK) {
#pragma unroll
            for (int e = 0; e < 8; ++e) wo[(wave * G + gg) * HD + 8 * lane + e] = s.o[gg][e];
          }
        }
      }
      block_sync();
      const int S = p.S;
      float* pbase = a.part + ((int64_t)p.ah * S + (b % S)) * G * (HD + 2);
      if (comp) {
        for (int i = tid; i < G * HD; i += NCW * 64) {
          const int gg = i / HD, d = i % HD;
          float M = -INFINITY;
#pragma unroll
          for (int w = 0; w < NCW; ++w) M = fmaxf(M, wm[w * G + gg]);
          float acc = 0.0f, den = 0.0f;
#pragma unroll
          for (int w = 0; w < NCW; ++w) {
            const float f = (wm[w * G + gg] == -INFINITY) ? 0.0f : expf(wm[w * G + gg] - M);
            acc += f * wo[(w * G + gg) * HD + d];
            den += f * wl[w * G + gg];
          }
          stf(pbase + gg * (HD + 2) + d, acc);
          if (d == 0) {
            stf(pbase + gg * (HD + 2) + HD, M);
            stf(pbase + gg * (HD + 2) + HD + 1, den);
          }
        }
        wait_vm<0>();
      }
      block_sync();
      if (tid == 0) {
        const u64 old = add_ag(&sy[SY_TICK + 16 * p.ah], 1);
        s_flag = (old + 1 == (u64)(l + 1) * (u64)S) ? 1 : 0;
      }
      block_sync();
      if (s_flag) {
        // the new token's key / value (position pos) and the S partials of kv head ah
        const float scale = 1.0f / sqrtf((float)HD);
        const float* kraw = a.qkv + a.q_dim + (int64_t)p.ah * HD;
        const float* vraw = kraw + a.kv_dim;
        const int64_t layer_elems = a.kv_dim * a.max_seq;
        __half* kc = static_cast<__half*>(a.kv) + (int64_t)l * 2 * layer_elems;
        __half* vc = kc + layer_elems;
        const float* hb = a.part + (int64_t)p.ah * S * G * (HD + 2);
        if (comp) {
          for (int i = tid; i < G * HD; i += NCW * 64) {
            const int gg = i / HD, d = i % HD;
            const float qv = rope_at(a.qkv, (int64_t)(p.ah * G + gg) * HD, d, HD, a.rope_mode, a.rope, pos) * scale;
            const __half k16 = __float2half(rope_at(kraw, 0, d, HD, a.rope_mode, a.rope, pos));
            const float prod = wave_sum(qv * __half2float(k16));
            if (lane == 0) red[i / 64] = prod;
            if (gg == 0) {
              kc[((int64_t)p.ah * a.max_seq + pos) * HD + d] = k16;
              vc[((int64_t)p.ah * a.max_seq + pos) * HD + d] = __float2half(ldf(vraw, d));
            }
          }
          for (int i = tid; i < S * G; i += NCW * 64) {
            mls[2 * i] = ldf(hb, (int64_t)i * (HD + 2) + HD);
            mls[2 * i + 1] = ldf(hb, (int64_t)i * (HD + 2) + HD + 1);
          }
        }
        block_sync();
        if (comp) {
          for (int i = tid; i < G * HD; i += NCW * 64) {
            const int gg = i / HD, d = i % HD;
            float snew = 0.0f;
            for (int j = 0; j < HD / 64; ++j) snew += red[gg * (HD / 64) + j];
            const float vnew = __half2float(__float2half(ldf(vraw, d)));
            float M = snew;
            for (int k = 0; k < S; ++k) M = fmaxf(M, mls[2 * (k * G + gg)]);
            float num = 0.0f, den = 0.0f;
            for (int k0 = 0; k0 < S; k0 += 16) {
              // 16 splits' values requested together (clamped index, weight 0 past S)
              float ov[16];
#pragma unroll
              for (int u = 0; u < 16; ++u)
                ov[u] = ldf(hb, (int64_t)(min(k0 + u, S - 1) * G + gg) * (HD + 2) + d);
#pragma unroll
              for (int u = 0; u < 16; ++u) {
                const int k = min(k0 + u, S - 1);
                const float mk = mls[2 * (k * G + gg)];
                const float f = (mk == -INFINITY || k0 + u >= S) ? 0.0f : expf(mk - M);
                num += f * ov[u];
                den += f * mls[2 * (k * G + gg) + 1];
              }
            }
            const float fn = expf(snew - M);
            num += fn * vnew;
            den += fn;
            stf(a.attn + (int64_t)(p.ah * G + gg) * HD + d, num / den);
          }
          wait_vm<0>();
        }
        block_sync();
        if (tid == 0) add_ag(&sy[SY_MERGED], 1);
      }
    }
    poll(SY_MERGED, (u64)(l + 1) * (u64)a.n_kv);
    block_sync();

    // ---- O projection + residual ----
    if (comp) {
      for (int t = tid; t < p.no * p.go.R; t += NCW * 64)
        resid[t] = ldf(a.x, (p.fo + t / p.go.R) * p.go.R + t % p.go.R);
    }
    stage_in(a.attn, false, wpre, 0.0f, a.q_dim, p.go, comp, wave, lane, red, xp);
    for (int i = 0; i < p.no; ++i, ++g) {
      const uint8_t* st = stage_begin(g);
      if (comp) gemv_stage(st, p.go, i, xp, part, wave, lane);
      stage_end(g);
    }
    block_sync();
    if (comp) {
      for (int t = tid; t < p.no * p.go.R; t += NCW * 64) {
        const int i = t / p.go.R, r = t % p.go.R;
        const int64_t gr = (p.fo + i) * p.go.R + r;
        const float v = resid[t] + row_sum(part, p.go, i, r);
        stf(a.x + gr, v);
        if (a.tap_r1) a.tap_r1[(int64_t)l * a.dim + gr] = v;
      }
    }
    load_norm(ffn_norm, p.gg, comp, wave, lane, wpre);
    grid_sync();

    // ---- gate / up, SwiGLU ----
    stage_in(a.x, ffn_norm != nullptr, wpre, a.eps, a.dim, p.gg, comp, wave, lane, red, xp);
    for (int i = 0; i < p.ng; ++i, ++g) {
      const uint8_t* st = stage_begin(g);
      if (comp) gemv_stage(st, p.gg, i, xp, part, wave, lane);
      stage_end(g);
    }
    block_sync();
    if (comp) {
      const int hr = p.gg.R / 2;
      for (int t = tid; t < p.ng * hr; t += NCW * 64) {
        const int i = t / hr, r = t % hr;
        const float gv = row_sum(part, p.gg, i, r), uv = row_sum(part, p.gg, i, r + hr);
        const int64_t j = (p.fg + i) * hr + r;
        stf(a.h + j, gv / (1.0f + expf(-gv)) * uv);  // silu(g) * u (elementwise.cpp:73-84)
      }
    }
    grid_sync();

    // ---- down + residual ----
    if (comp) {
      for (int t = tid; t < p.nd * p.gd.R; t += NCW * 64)
        resid[t] = ldf(a.x, (p.fd + t / p.gd.R) * p.gd.R + t % p.gd.R);
    }
    stage_in(a.h, false, wpre, 0.0f, a.inter, p.gd, comp, wave, lane, red, xp);
    for (int i = 0; i < p.nd; ++i, ++g) {
      const uint8_t* st = stage_begin(g);
      if (comp) gemv_stage(st, p.gd, i, xp, part, wave, lane);
      stage_end(g);
    }
    block_sync();
    if (comp) {
      for (int t = tid; t < p.nd * p.gd.R; t += NCW * 64) {
        const int i = t / p.gd.R, r = t % p.gd.R;
        const int64_t gr = (p.fd + i) * p.gd.R + r;
        const float v = resid[t] + row_sum(part, p.gd, i, r);
        stf(a.x + gr, v);
        if (a.tap_r2) a.tap_r2[(int64_t)l * a.dim + gr] = v;
      }
    }
    if (l + 1 < a.n_layers) {
      load_norm(lws[l + 1].attn_norm, p.gq, comp, wave, lane, wpre);
      grid_sync();
    }
  }

  // every DMA landed (none is outstanding once the last stage was consumed)
  wait_vm<0>();
  block_sync();
  if (tid == 0) {
    const u64 old = add_ag(&sy[SY_DONE], 1);
    if (old + 1 == (u64)nblk) {
      for (int k = 0; k < 8; ++k) st_ag(&sy[SY_GROUP + 16 * k], 0);
      st_ag(&sy[SY_ALL], 0);
      st_ag(&sy[SY_MERGED], 0);
      for (int h = 0; h < a.n_kv; ++h) st_ag(&sy[SY_TICK + 16 * h], 0);
      st_ag(&sy[SY_DONE], 0);
    }
  }
}

// ---- one GEMV through the ring (decode, between ordinary launches) -----------------------------

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

// Stages of a ring GEMV (R rows each; EPI_SWIGLU: R/2 gate + R/2 up rows).
__host__ __device__ __forceinline__ int64_t ring_stages_of(const RingArgs& a, const Geo& ge) {
  if (a.epi == EPI_SWIGLU) return a.rows[0] / (ge.R / 2);
  int64_t rows = 0;
  for (int k = 0; k < a.nseg; ++k) rows += a.rows[k];
  return rows / ge.R;
}

// The run of stages that starts at global stage gs and ends at the block's
// last stage gend or at a segment boundary.
__device__ __forceinline__ void ring_seg(const RingArgs& a, const Geo& ge, int64_t gs, int64_t gend, int lw,
                                         Seg& sg) {
  const uint8_t *A0 = a.pad, *A1 = a.pad, *B0 = a.pad, *B1 = a.pad;
  int n16, c16, n4, c4;
  int64_t da, db, run;
  if (a.epi == EPI_SWIGLU) {
    const int64_t j0 = gs * (ge.R / 2);
    A0 = a.w[0].a + j0 * ge.arow;
    A1 = a.w[1].a + j0 * ge.arow;
    B0 = a.w[0].b + j0 * ge.brow;
    B1 = a.w[1].b + j0 * ge.brow;
    n16 = ge.nl; c16 = ge.nl / 2;
    n4 = ge.sl; c4 = ge.sl / 2;
    da = (ge.R / 2) * ge.arow;
    db = (ge.R / 2) * ge.brow;
    run = gend - gs;
  } else {
    int64_t row0 = gs * ge.R;
    int k = 0;
    while (k + 1 < a.nseg && row0 >= a.rows[k]) { row0 -= a.rows[k]; ++k; }
    const DevWeight& w = a.w[k];
    A0 = w.a + row0 * ge.arow;
    B0 = w.b + row0 * ge.brow;
    n16 = c16 = ge.nl;
    n4 = c4 = ge.sl;
    da = ge.R * ge.arow;
    db = ge.R * ge.brow;
    run = min(gend - gs, (a.rows[k] - row0) / ge.R);
  }
#pragma unroll
  for (int u = 0; u < LX4; ++u) {
    const int j = lw + NLW * u;
    sg.p16[u] = j < n16 ? (j < c16 ? A0 + (int64_t)j * 1024 : A1 + (int64_t)(j - c16) * 1024) : a.pad;
    sg.o16[u] = j < n16 ? (uint32_t)(j * 1024) : ~0u;
  }
#pragma unroll
  for (int u = 0; u < LX1; ++u) {
    const int j = lw + NLW * u;
    sg.p4[u] = j < n4 ? (j < c4 ? B0 + (int64_t)j * 256 : B1 + (int64_t)(j - c4) * 256) : a.pad;
    sg.o4[u] = j < n4 ? (uint32_t)(SQ + j * 256) : ~0u;
  }
  sg.s16 = da;
  sg.s4 = db;
  sg.left = (int)run;
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
  stage_load<false>(a.x, ge, comp, wave, lane, v);
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
  if (a.xtap && b == 0 && comp && wave < ge.ncol) {  // the staged input, once (chunk column = wave)
    float4* dst = reinterpret_cast<float4*>(a.xtap) + 8 * ((int64_t)wave * 64 + lane);
#pragma unroll
    for (int k = 0; k < 8; ++k) dst[k] = make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
  }
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
  // epilogues (gemv.hip's, on the block's rows)
  if (a.epi == EPI_SWIGLU) {
    const int hr = ge.R / 2;
    for (int t = tid; t < n * hr; t += NCW * 64) {
      const int i = t / hr, r = t % hr;
      const float gv = row_sum(part, ge, i, r), uv = row_sum(part, ge, i, r + hr);
      a.y[(f + i) * hr + r] = gv / (1.0f + expf(-gv)) * uv;  // silu(g) * u (elementwise.cpp:73-84)
    }
  } else if (a.epi == EPI_QKV) {
    const int pos = a.state->pos;
    const int hr = ge.R / 2;
    for (int t = tid; t < n * hr; t += NCW * 64) {
      const int i = t / hr, r0 = 2 * (t % hr);
      int64_t l = (f + i) * ge.R + r0;
      int k = 0;
      while (k + 1 < a.nseg && l >= a.rows[k]) { l -= a.rows[k]; ++k; }
      float v0 = row_sum(part, ge, i, r0), v1 = row_sum(part, ge, i, r0 + 1);
      if (a.bias[k]) { v0 = v0 + a.bias[k][l]; v1 = v1 + a.bias[k][l + 1]; }
      const int64_t hd = a.head_dim;
      if (k != 2) {  // RoPE mode 0 on q and k (transformer.cpp:144-220)
        const float2 cs = a.rope[(int64_t)pos * (hd / 2) + ((l % hd) >> 1)];
        const float n0 = v0 * cs.x - v1 * cs.y;
        const float n1 = v0 * cs.y + v1 * cs.x;
        v0 = n0; v1 = n1;
      }
      if (k == 0) {
        a.y[l] = v0;
        a.y[l + 1] = v1;
      } else {  // K after RoPE and raw V into the cache at pos (kv_cache.hpp:80-120)
        void* cache = k == 1 ? a.kcache : a.vcache;
        const int64_t o0 = ((l / hd) * a.max_seq + pos) * hd + (l % hd);
        if (a.kv_f16) {
          reinterpret_cast<__half*>(cache)[o0] = __float2half(v0);
          reinterpret_cast<__half*>(cache)[o0 + 1] = __float2half(v1);
        } else {
          reinterpret_cast<float*>(cache)[o0] = v0;
          reinterpret_cast<float*>(cache)[o0 + 1] = v1;
        }
      }
    }
  } else if (a.epi == EPI_LOGITS) {
    // logits, and this wave's greedy argmax partial: a thread's rows ascend, so
    // strict '>' keeps the lowest index; lanes combine on (larger value, then
    // lower index), as k_argmax_final does across the partials
    float bv = -INFINITY;
    int32_t bi = 0x7fffffff;
    for (int t = tid; t < n * ge.R; t += NCW * 64) {
      const int i = t / ge.R, r = t % ge.R;
      const int64_t gr = (f + i) * ge.R + r;
      const float v = row_sum(part, ge, i, r);
      a.y[gr] = v;
      if (bi == 0x7fffffff || v > bv) { bv = v; bi = (int32_t)gr; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int32_t oi = __shfl_xor(bi, o, 64);
      if (oi != 0x7fffffff && (bi == 0x7fffffff || ov > bv || (ov == bv && oi < bi))) { bv = ov; bi = oi; }
    }
    if (lane == 0) {
      a.part_val[b * NCW + wave] = bv;
      a.part_idx[b * NCW + wave] = bi;
    }
  } else {
    for (int t = tid; t < n * ge.R; t += NCW * 64) {
      const int i = t / ge.R, r = t % ge.R;
      const int64_t gr = (f + i) * ge.R + r;
      float v = row_sum(part, ge, i, r);
      if (a.epi == EPI_ADD) v = a.y[gr] + v;
      a.y[gr] = v;
      if (a.tap) a.tap[gr] = v;
    }
  }
}

int dev_cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  return n;
}

template <int HD, int G>
constexpr int ring_stages() { return (G * HD > 512) ? 6 : 7; }

// Dynamic LDS: ring, padding line, shared region (the merge's (m, l) pairs,
// 2 S G <= 512 G floats, fit in the wave states' space), pointer table.
template <int HD, int G>
size_t layers_lds(int n_layers) {
  return (size_t)ring_stages<HD, G>() * SB + 1024 + (size_t)layers_misc<HD, G>() + (size_t)n_layers * PT * 8;
}

// Dynamic LDS the kernel may take: the device's per-block limit less a
// margin for the static arrays.
inline size_t layers_lds_cap() { return (size_t)lds_limit() - 1024; }

// Raise the kernel's dynamic-LDS limit and check that a block fits on a CU
// (once per process; the device count check is per launch).
template <int HD, int G>
hipError_t prep_hg() {
  constexpr int NS = ring_stages<HD, G>();
  static std::once_flag once;
  static hipError_t prep = hipSuccess;
  std::call_once(once, [] {
    const size_t lds = layers_lds_cap();
    prep = hipFuncSetAttribute((const void*)k_layers<HD, G, NS>, hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)lds);
    int per_cu = 0;
    if (prep == hipSuccess)
      prep = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_layers<HD, G, NS>, NTH, lds);
    if (prep == hipSuccess && per_cu < 1) prep = hipErrorInvalidConfiguration;
  });
  return prep;
}

template <int HD, int G>
hipError_t launch_hg(const LayersArgs& a, int nblk, hipStream_t s) {
  constexpr int NS = ring_stages<HD, G>();
  const size_t lds = layers_lds<HD, G>(a.n_layers);
  if (lds > layers_lds_cap()) return hipErrorInvalidValue;
  const hipError_t prep = prep_hg<HD, G>();
  if (prep != hipSuccess) return prep;
  UAII_LAUNCH((k_layers<HD, G, NS>), dim3(nblk), dim3(NTH), lds, s, a);
  return hipGetLastError();
}

}  // namespace

int layers_splits(int n_kv) {
  const int n = dev_cus();
  return n_kv > 0 && n >= n_kv ? std::min(256, n / n_kv) : 0;
}

bool layers_supported(int type, int n_layers, int64_t dim, int64_t q_dim, int64_t kv_dim, int64_t inter,
                      int n_heads, int n_kv, int head_dim) {
  if (type != T_Q4_0 || n_layers < 1) return false;
  if (head_dim != 64 && head_dim != 128) return false;
  if (n_kv < 1 || n_kv > 64 || n_heads % n_kv) return false;
  const int G = n_heads / n_kv;
  if (G != 1 && G != 2 && G != 4 && G != 8) return false;
  if ((int64_t)n_heads * head_dim != q_dim || (int64_t)n_kv * head_dim != kv_dim) return false;
  for (int64_t K : {dim, q_dim, inter})
    if (K <= 0 || K % 2048 || K > 16384) return false;
  const int nblk = dev_cus();
  if (nblk < 1 || layers_splits(n_kv) < 1) return false;
  const Geo gq = geo_of(dim), go = geo_of(q_dim), gd = geo_of(inter);
  const int64_t Tq = (q_dim + 2 * kv_dim) / gq.R, To = dim / go.R, Tg = inter / (gq.R / 2), Td = dim / gd.R;
  if ((q_dim + 2 * kv_dim) % gq.R || dim % go.R || inter % (gq.R / 2) || dim % gd.R) return false;
  if (q_dim % gq.R || kv_dim % gq.R) return false;  // a stage never straddles two matrices
  auto most = [&](int64_t T) { return (T + nblk - 1) / nblk; };
  if (most(Tq) * gq.R * gq.ncol > PART_MAX || most(To) * go.R * go.ncol > PART_MAX ||
      most(Tg) * gq.R * gq.ncol > PART_MAX || most(Td) * gd.R * gd.ncol > PART_MAX)
    return false;
  if (most(To) * go.R > RESID_MAX || most(Td) * gd.R > RESID_MAX) return false;
  size_t lds = 0;
  if (head_dim == 128) lds = G == 8 ? layers_lds<128, 8>(n_layers) : layers_lds<128, 4>(n_layers);
  else lds = G == 8 ? layers_lds<64, 8>(n_layers) : layers_lds<64, 4>(n_layers);
  return lds <= layers_lds_cap();
}

int ring_logits_parts() { return dev_cus() * NCW; }

bool ring_gemv_supported(const RingArgs& a) {
  if (a.nseg < 1 || a.nseg > 3 || a.K <= 0 || a.K % 2048 || a.K > 16384 || !a.x || !a.y || !a.pad) return false;
  if (a.epi != EPI_STORE && a.epi != EPI_ADD && a.epi != EPI_QKV && a.epi != EPI_SWIGLU && a.epi != EPI_LOGITS)
    return false;
  if (a.epi == EPI_LOGITS && (a.nseg != 1 || !a.part_val || !a.part_idx || a.rows[0] > INT32_MAX)) return false;
  if (a.epi == EPI_SWIGLU && a.nseg != 2) return false;
  if (a.epi == EPI_QKV && (a.nseg != 3 || a.head_dim < 2 || a.head_dim % 2 || !a.rope || !a.state || !a.kcache ||
                           !a.vcache))
    return false;
  const Geo ge = geo_of(a.K);
  int64_t T = 0;
  for (int k = 0; k < a.nseg; ++k) {
    const DevWeight& w = a.w[k];
    if (w.type != T_Q4_0 || w.cols != a.K || w.a_row != ge.arow || w.b_row != ge.brow) return false;
    const int64_t unit = a.epi == EPI_SWIGLU ? ge.R / 2 : ge.R;
    const int64_t rows = a.epi == EPI_SWIGLU ? a.rows[0] : a.rows[k];
    if (rows <= 0 || rows % unit || w.rows < rows) return false;
    if (a.epi != EPI_SWIGLU) T += rows / ge.R;
  }
  if (a.epi == EPI_SWIGLU) T = a.rows[0] / (ge.R / 2);
  if (a.epi == EPI_QKV && a.head_dim % 2) return false;
  const int nblk = dev_cus();
  if (nblk < 1) return false;
  const int64_t most = (T + nblk - 1) / nblk;
  if (most * ge.R * ge.ncol > PART_MAX) return false;
  return (size_t)RING_NS * SB + 1024 + PART_MAX * 4 <= layers_lds_cap();
}

hipError_t prepare_ring_gemv() {
  static std::once_flag once;
  static hipError_t prep = hipSuccess;
  std::call_once(once, [] {
    const size_t lds = (size_t)RING_NS * SB + 1024 + PART_MAX * 4;
    prep = hipFuncSetAttribute((const void*)k_ring_gemv, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    int per_cu = 0;
    if (prep == hipSuccess) prep = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_ring_gemv, NTH, lds);
    if (prep == hipSuccess && per_cu < 1) prep = hipErrorInvalidConfiguration;
  });
  return prep;
}

hipError_t launch_ring_gemv(const RingArgs& in, hipStream_t s) {
  if (!ring_gemv_supported(in)) return hipErrorInvalidValue;
  const hipError_t prep = prepare_ring_gemv();
  if (prep != hipSuccess) return prep;
  const size_t lds = (size_t)RING_NS * SB + 1024 + PART_MAX * 4;
  const int nblk = dev_cus();
  if (nblk <= 0) return hipErrorInvalidDevice;
  RingArgs a = in;
  const int64_t T = ring_stages_of(a, geo_of(a.K));
  a.tq = (int32_t)(T / nblk);
  a.tr = (int32_t)(T % nblk);
  UAII_LAUNCH(k_ring_gemv, dim3(nblk), dim3(NTH), lds, s, a);
  return hipGetLastError();
}

hipError_t prepare_layers(int head_dim, int G) {
  if (head_dim == 128) {
    switch (G) {
      case 1: return prep_hg<128, 1>();
      case 2: return prep_hg<128, 2>();
      case 4: return prep_hg<128, 4>();
      case 8: return prep_hg<128, 8>();
      default: return hipErrorInvalidValue;
    }
  }
  if (head_dim == 64) {
    switch (G) {
      case 1: return prep_hg<64, 1>();
      case 2: return prep_hg<64, 2>();
      case 4: return prep_hg<64, 4>();
      case 8: return prep_hg<64, 8>();
      default: return hipErrorInvalidValue;
    }
  }
  return hipErrorInvalidValue;
}

hipError_t launch_layers(const LayersArgs& in, int type, hipStream_t s) {
  if (!layers_supported(type, in.n_layers, in.dim, in.q_dim, in.kv_dim, in.inter, in.n_heads, in.n_kv,
                        in.head_dim) ||
      !in.layers || in.n_layers < 1 || !in.x || !in.qkv || !in.attn || !in.h || !in.part || !in.kv ||
      !in.rope || !in.state || !in.sync || !in.pad || in.max_seq < 1)
    return hipErrorInvalidValue;
  LayersArgs a = in;
  a.splits = layers_splits(a.n_kv);
  const int nblk = dev_cus();
  const int G = a.n_heads / a.n_kv;
  if (a.head_dim == 128) {
    switch (G) {
      case 1: return launch_hg<128, 1>(a, nblk, s);
      case 2: return launch_hg<128, 2>(a, nblk, s);
      case 4: return launch_hg<128, 4>(a, nblk, s);
      default: return launch_hg<128, 8>(a, nblk, s);
    }
  }
  switch (G) {
    case 1: return launch_hg<64, 1>(a, nblk, s);
    case 2: return launch_hg<64, 2>(a, nblk, s);
    case 4: return launch_hg<64, 4>(a, nblk, s);
    default: return launch_hg<64, 8>(a, nblk, s);
  }
}

}  // namespace uaii_hip
