// prefill.hip — the prompt path (M > 1 tokens at once) on gfx950 matrix cores.
//
// The reference prefills one token at a time through quant_gemm_f32
// (libs/uaii-quant/src/quant_gemm.cpp:22-70: per weight row, dequantise to f32
// and dot with every activation row) and attention_kv_f32
// (libs/uaii-kernels/src/transformer.cpp:222-433). Here a chunk of M prompt
// tokens runs layer by layer as dense contractions:
//
//   k_pf_prep   RMSNorm (optional) of each activation row, a power-of-two row
//               scale 2^e, and the split x * 2^e = hi + lo into two f16 values
//               (together ~22 significant bits), plus per-32 sums for formats
//               whose blocks carry an offset.
//   k_pf_gemm   C[M][N] = A . W^T with W read in its split GGUF layout: the
//               weights of one (sub-)block decode in registers to their small
//               integers, which f16 holds exactly; v_mfma_f32_16x16x32_f16
//               (16x16x16 for 16-element sub-blocks) multiplies them with hi
//               and with lo, and the block's scale (and offset times the row
//               sum) is applied to the f32 partial. The only roundings are the
//               f32 accumulations, so results match the f32 reference to
//               ~1e-6 relative. Epilogues: store, residual add, SwiGLU, GELU.
//   k_pf_qkv    Q/K/V bias, RoPE and the KV-cache append for M positions.
//   k_pf_attn   causal attention of M queries over the f16 cache on MFMA:
//               S^T = K . Q^T, online softmax, O^T += V^T . P^T, with q * scale
//               and P split into f16 hi + lo against the exact f16 keys/values.
//
// Operand layout of the 16x16xK f16 MFMAs used here (CDNA3/CDNA4): lane l
// supplies row (l % 16) of A and column (l % 16) of B with k-group (l / 16);
// the f32 result D[4 * (l / 16) + r][l % 16] sits in element r of lane l. The
// order of k inside a lane's group only has to agree between A and B: the
// activation rows are stored with each aligned group of 4 values as
// (k0, k2, k1, k3), the order in which the weight decode below produces them
// from bytes 0 and 2, then 1 and 3, of a 32-bit word.
#include <type_traits>

#include "common.h"
#include "uaii_hip_internal.h"

namespace uaii_hip {
namespace {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

__device__ inline h2_t as_h2(uint32_t u) { return __builtin_bit_cast(h2_t, u); }
// (v & m) | c in one v_and_or_b32. Written out because gfx9's three-operand
// encoding takes no literal constants, so the compiler splits the expression
// into v_and + v_or; here the mask sits in a scalar register and the constant
// in a vector register, both loop-invariant.
__device__ inline uint32_t and_or(uint32_t v, uint32_t m, uint32_t c) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(m), "v"(c));
  return r;
}
// low nibbles of bytes 0 and 2 as f16 (1024 + q)
__device__ inline uint32_t nib_pair(uint32_t v) { return and_or(v, 0x000F000Fu, 0x64006400u); }
// The same with the mask in a vector register: 0x000F000F gives 1024 + q from
// the low nibbles, 0x00F000F0 gives 1024 + 16 q from the high ones in place
__device__ inline uint32_t and_or_v(uint32_t v, uint32_t m, uint32_t c) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "v"(m), "v"(c));
  return r;
}
// bytes 0 and 2 as f16 (1024 + b)
__device__ inline uint32_t byte_pair(uint32_t v) { return and_or(v, 0x00FF00FFu, 0x64006400u); }

__device__ inline h8_t cat8(h2_t a, h2_t b, h2_t c, h2_t d) {
  return h8_t{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

__device__ inline f4_t mfma32(h8_t a, h8_t b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ inline float pow2f_i(int e) { return __uint_as_float((uint32_t)(e + 127) << 23); }

// ---- activation prep ----------------------------------------------------------------

// One block per row; rows >= M (tile padding) are written as zeros.
__global__ void __launch_bounds__(256) k_pf_prep(float* __restrict__ x, int64_t ldx,
                                                 int64_t M, const float* __restrict__ norm_w,
                                                 float eps, PfAct act, const float* __restrict__ part,
                                                 int nsplit) {
  extern __shared__ float row[];
  __shared__ float red[4];
  const int64_t t = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t K = act.K;
  const int nv = (int)(K / 4);
  uint2* hi2 = reinterpret_cast<uint2*>(act.hi + t * K);
  uint2* lo2 = reinterpret_cast<uint2*>(act.lo + t * K);
  if (t >= M) {
    for (int i = tid; i < nv; i += 256) { hi2[i] = make_uint2(0, 0); lo2[i] = make_uint2(0, 0); }
    for (int64_t b = tid; b < K / 32; b += 256) act.sx[b * act.mpad + t] = 0.0f;
    if (tid == 0) act.rs[t] = 0.0f;
    return;
  }
  float4* r4 = reinterpret_cast<float4*>(row);
  float4* x4 = reinterpret_cast<float4*>(x + t * ldx);
  float ss = 0.0f, amax = 0.0f;
  for (int i = tid; i < nv; i += 256) {
    float4 v = x4[i];
    if (nsplit > 0) {
      // residual add of a K-split GEMM's partials, in split order
      float4 p = reinterpret_cast<const float4*>(part + t * ldx)[i];
      for (int z = 1; z < nsplit; ++z) {
        const float4 q = reinterpret_cast<const float4*>(part + ((int64_t)z * M + t) * ldx)[i];
        p.x += q.x; p.y += q.y; p.z += q.z; p.w += q.w;
      }
      v.x += p.x; v.y += p.y; v.z += p.z; v.w += p.w;
      x4[i] = v;
    }
    r4[i] = v;
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
  }
  if (norm_w) {
    // x * (1/sqrt(mean(x^2)+eps)) * w with two roundings (norm.cpp:122-127)
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    const float tot = red[0] + red[1] + red[2] + red[3];
    const float inv = 1.0f / sqrtf(tot / (float)K + eps);
    const float4* w4 = reinterpret_cast<const float4*>(norm_w);
    amax = 0.0f;
    for (int i = tid; i < nv; i += 256) {
      float4 v = r4[i];
      const float4 w = w4[i];
      v.x = fmul_rn(fmul_rn(v.x, inv), w.x);
      v.y = fmul_rn(fmul_rn(v.y, inv), w.y);
      v.z = fmul_rn(fmul_rn(v.z, inv), w.z);
      v.w = fmul_rn(fmul_rn(v.w, inv), w.w);
      r4[i] = v;
      amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    __syncthreads();  // red[] is reused below
  }
  amax = wave_max(amax);
  if ((tid & 63) == 0) red[tid >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  // scale so that max |x| * 2^e lies in [2^14, 2^15): hi keeps 11 bits of every
  // element near the top of the row and lo the next 11
  int e = 0;
  if (amax > 0.0f) {
    const int ex = (int)((__float_as_uint(amax) >> 23) & 0xff) - 126;  // amax in [2^(ex-1), 2^ex)
    e = min(100, max(-100, 15 - ex));
  }
  const float s = pow2f_i(e);
  if (tid == 0) act.rs[t] = pow2f_i(-e);
  for (int base = 0; base < nv; base += 256) {
    const int i = base + tid;
    float sum = 0.0f;
    if (i < nv) {
      const float4 v = r4[i];
      const float y0 = v.x * s, y1 = v.y * s, y2 = v.z * s, y3 = v.w * s;
      // hi16 layout: elements 16..31 of the 32-block (float4 slots 4..7) times
      // 1/16, exactly (a power of two), before the split
      const float q = (act.hi16 && (i & 7) >= 4) ? 0.0625f : 1.0f;
      const float z0 = y0 * q, z1 = y1 * q, z2 = y2 * q, z3 = y3 * q;
      const _Float16 h0 = (_Float16)z0, h1 = (_Float16)z1, h2 = (_Float16)z2, h3 = (_Float16)z3;
      const _Float16 l0 = (_Float16)(z0 - (float)h0), l1 = (_Float16)(z1 - (float)h1);
      const _Float16 l2 = (_Float16)(z2 - (float)h2), l3 = (_Float16)(z3 - (float)h3);
      // stored order (k0, k2, k1, k3)
      hi2[i] = make_uint2(__builtin_bit_cast(uint32_t, h2_t{h0, h2}),
                          __builtin_bit_cast(uint32_t, h2_t{h1, h3}));
      lo2[i] = make_uint2(__builtin_bit_cast(uint32_t, h2_t{l0, l2}),
                          __builtin_bit_cast(uint32_t, h2_t{l1, l3}));
      sum = (y0 + y1) + (y2 + y3);
    }
    // 8 consecutive float4 = one 32-block (K % 32 == 0, so groups are whole)
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    sum += __shfl_xor(sum, 4, 64);
    if (i < nv && (i & 7) == 0) act.sx[(int64_t)(i >> 3) * act.mpad + t] = sum;
  }
}

// ---- weight fragments -----------------------------------------------------------------

// A stage is two consecutive 32-blocks of k (kb = 2 st, 2 st + 1). PfRaw holds
// the bytes of one weight row's stage that lane group g needs, loaded one stage
// ahead of use; pf_decode() turns one block of it into the MFMA B operand (the
// block's small integers) and its scale (and offset).
template <int FMT>
struct PfRaw;
template <>
struct PfRaw<T_Q4_0> {
  uint2 q[2];   // qs bytes 8 (g & 1) .. +7 of each block
  uint32_t d;   // the two f16 scales
};
template <>
struct PfRaw<T_Q8_0> {
  uint2 q[2];   // qs bytes 8 g .. +7 of each block
  uint32_t d;
};
template <>
struct PfRaw<T_Q4_K> {
  uint2 q;      // qs bytes 8 g .. +7 of the pair: low nibbles block 0, high block 1
  uint4 meta;   // d, dmin, scales[12] of the super-block
};
template <>
struct PfRaw<T_Q6_K> {
  uint2 ql[2];     // ql bytes 8 g .. +7 of blocks 0 and 1 (low or high nibbles by stage)
  uint2 qh;        // qh bytes 8 g .. +7 (shared by both blocks)
  uint32_t sc;     // the four int8 sub-block scales of the stage
  uint32_t d;
};

template <int FMT>
struct PfFrag {
  h8_t b;         // the block's weight integers (Q6_K: the high part of sc (q - 32))
  h8_t blo;       // Q6_K: the remainder of sc (q - 32) after b (0 or +-1)
  float sc[1];
  float off;
};

// Q6_K folds each 16-element sub-block's int8 scale into the MFMA operand:
// sc (q - 32) is an integer of magnitude <= 4096, which the f16 pair (b, blo)
// holds exactly, so a 32-element block (two sub-blocks) takes one 16x16x32 MFMA
// per operand pair and only the super-block scale d remains for the f32 partial.
template <int FMT>
__device__ constexpr bool pf_split_b() {
  return FMT == T_Q6_K;
}
template <int FMT>
__device__ constexpr bool pf_offset() {
  return FMT == T_Q4_K;
}

// The lane's row pointers into the split arrays, lane-group offsets folded in.
struct PfRow {
  const uint8_t* a;
  const uint8_t* b;
  const uint8_t* c;
  const uint8_t* d;
};

template <int FMT>
__device__ inline PfRow pf_row(const DevWeight& w, int64_t row, int g) {
  PfRow p{};
  p.a = w.a + row * w.a_row;
  p.b = w.b + row * w.b_row;
  if constexpr (FMT == T_Q4_0) {
    p.a += 8 * (g & 1);
  } else if constexpr (FMT == T_Q8_0 || FMT == T_Q4_K) {
    p.a += 8 * g;
  } else if constexpr (FMT == T_Q6_K) {
    p.a += 8 * g;
    p.b += 8 * g;
    p.c = w.c + row * w.c_row;
    p.d = w.d + row * w.d_row;
  }
  return p;
}

template <int FMT>
__device__ inline void pf_load(const PfRow& p, int64_t st, PfRaw<FMT>& r) {
  if constexpr (FMT == T_Q4_0) {
    const uint8_t* q = p.a + st * 32;
    r.q[0] = *reinterpret_cast<const uint2*>(q);
    r.q[1] = *reinterpret_cast<const uint2*>(q + 16);
    r.d = *reinterpret_cast<const uint32_t*>(p.b + st * 4);
  } else if constexpr (FMT == T_Q8_0) {
    const uint8_t* q = p.a + st * 64;
    r.q[0] = *reinterpret_cast<const uint2*>(q);
    r.q[1] = *reinterpret_cast<const uint2*>(q + 32);
    r.d = *reinterpret_cast<const uint32_t*>(p.b + st * 4);
  } else if constexpr (FMT == T_Q4_K) {
    r.q = *reinterpret_cast<const uint2*>(p.a + st * 32);
    r.meta = *reinterpret_cast<const uint4*>(p.b + (st >> 2) * 16);
  } else if constexpr (FMT == T_Q6_K) {
    // super-block st / 4, half (st % 4) / 2, elements 64 (st % 2) .. +63 of the half
    const uint8_t* ql = p.a + (st >> 1) * 64;
    r.ql[0] = *reinterpret_cast<const uint2*>(ql);
    r.ql[1] = *reinterpret_cast<const uint2*>(ql + 32);
    r.qh = *reinterpret_cast<const uint2*>(p.b + (st >> 1) * 32);
    r.sc = *reinterpret_cast<const uint32_t*>(p.c + st * 4);
    r.d = ld_u16(p.d + (st >> 2) * 2);
  }
}

// Block s (0 or 1) of stage st for lane group g. H16 (Q4_0, PfAct::hi16
// activations): lane groups 2 and 3, which hold elements 16..31, decode their
// high nibbles in place as 16 (q - 8), exact in f16, and the activations of
// those elements carry the factor 1/16; this saves the per-lane shift.
template <int FMT, bool H16 = false>
__device__ inline void pf_decode(const PfRaw<FMT>& r, int64_t st, int s, int g, PfFrag<FMT>& f) {
  if constexpr (FMT == T_Q4_0 && H16) {
    const bool up = g >= 2;
    const uint32_t m = up ? 0x00F000F0u : 0x000F000Fu;
    const _Float16 bv = up ? (_Float16)1152.0f : (_Float16)1032.0f;  // 1024 + 16 * 8 : 1024 + 8
    const h2_t bias = {bv, bv};
    const uint32_t c = 0x64006400u;
    const uint32_t v0 = r.q[s].x, v1 = r.q[s].y;
    f.b = cat8(as_h2(and_or_v(v0, m, c)) - bias, as_h2(and_or_v(v0 >> 8, m, c)) - bias,
               as_h2(and_or_v(v1, m, c)) - bias, as_h2(and_or_v(v1 >> 8, m, c)) - bias);
    f.sc[0] = h2f((uint16_t)(r.d >> (16 * s)));
  } else if constexpr (FMT == T_Q4_0) {
    const int sh = (g >> 1) * 4;
    const uint32_t v0 = r.q[s].x >> sh, v1 = r.q[s].y >> sh;
    const h2_t bias = {(_Float16)1032.0f, (_Float16)1032.0f};
    f.b = cat8(as_h2(nib_pair(v0)) - bias, as_h2(nib_pair(v0 >> 8)) - bias,
               as_h2(nib_pair(v1)) - bias, as_h2(nib_pair(v1 >> 8)) - bias);
    f.sc[0] = h2f((uint16_t)(r.d >> (16 * s)));
  } else if constexpr (FMT == T_Q8_0) {
    const uint32_t v0 = r.q[s].x ^ 0x80808080u, v1 = r.q[s].y ^ 0x80808080u;
    const h2_t bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    f.b = cat8(as_h2(byte_pair(v0)) - bias, as_h2(byte_pair(v0 >> 8)) - bias,
               as_h2(byte_pair(v1)) - bias, as_h2(byte_pair(v1 >> 8)) - bias);
    f.sc[0] = h2f((uint16_t)(r.d >> (16 * s)));
  } else if constexpr (FMT == T_Q4_K) {
    const int j = 2 * (int)(st & 3) + s;  // sub-block of the super-block
    const uint32_t v0 = r.q.x >> (4 * s), v1 = r.q.y >> (4 * s);
    const h2_t bias = {(_Float16)1024.0f, (_Float16)1024.0f};
    f.b = cat8(as_h2(nib_pair(v0)) - bias, as_h2(nib_pair(v0 >> 8)) - bias,
               as_h2(nib_pair(v1)) - bias, as_h2(nib_pair(v1 >> 8)) - bias);
    // 6-bit (scale, min) pair j of the 12-byte field (gguf_dequant.cpp:107-115):
    // bytes j & 3 of the three words hold s[j & 3], s[4 + (j & 3)], s[8 + (j & 3)]
    const int bsh = 8 * (j & 3);
    const int by = (int)((r.meta.y >> bsh) & 0xff), bz = (int)((r.meta.z >> bsh) & 0xff);
    const int bw = (int)((r.meta.w >> bsh) & 0xff);
    int sc, mn;
    if (j < 4) {
      sc = by & 63;
      mn = bz & 63;
    } else {
      sc = (bw & 15) | ((by >> 6) << 4);
      mn = (bw >> 4) | ((bz >> 6) << 4);
    }
    const float d = h2f((uint16_t)(r.meta.x & 0xffff)), dmin = h2f((uint16_t)(r.meta.x >> 16));
    f.sc[0] = fmul_rn(d, (float)sc);
    f.off = fmul_rn(dmin, (float)mn);
  } else if constexpr (FMT == T_Q6_K) {
    // element e = 64 (st % 2) + 32 s + 8 g + i of the half: ql byte e % 64 (high
    // nibble when e >= 64), qh byte e % 32 at bit 2 (e / 32), sub-block e / 16 of
    // the stage, i.e. 2 s + g / 2. b = RN(sc (q - 32)) and blo = sc (q - 32) - b
    // by one fused multiply-add, exact: the integer is at most 4096 in magnitude
    const int nib = (int)(st & 1) * 4;
    const int qsh = 4 * (int)(st & 1) + 2 * s;
    const h2_t bias = {(_Float16)1056.0f, (_Float16)1056.0f};
    const _Float16 scv = (_Float16)(float)(int8_t)((r.sc >> (8 * (2 * s + (g >> 1)))) & 0xff);
    const h2_t sc2 = {scv, scv};
    const uint32_t w[2] = {r.ql[s].x, r.ql[s].y}, hq[2] = {r.qh.x, r.qh.y};
    h2_t hi[4], lo[4];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const uint32_t q6 = ((w[t] >> nib) & 0x0F0F0F0Fu) | (((hq[t] >> qsh) & 0x03030303u) << 4);
      const h2_t p0 = as_h2(byte_pair(q6)) - bias, p1 = as_h2(byte_pair(q6 >> 8)) - bias;
      hi[2 * t] = p0 * sc2;
      lo[2 * t] = __builtin_elementwise_fma(p0, sc2, -hi[2 * t]);
      hi[2 * t + 1] = p1 * sc2;
      lo[2 * t + 1] = __builtin_elementwise_fma(p1, sc2, -hi[2 * t + 1]);
    }
    f.b = cat8(hi[0], hi[1], hi[2], hi[3]);
    f.blo = cat8(lo[0], lo[1], lo[2], lo[3]);
    f.sc[0] = h2f((uint16_t)r.d);
  }
}

// ---- GEMM -------------------------------------------------------------------------------

#ifndef UAII_PF_DMA
#define UAII_PF_DMA 1  // Q4_0 / Q8_0 through the direct-to-LDS kernel
#endif
#ifndef UAII_PF_TILE
#define UAII_PF_TILE 0  // wave tile: 0 chosen per launch, 2 64x32, 3 32x32
#endif
constexpr int PF_WAVES = 4;   // waves per block, side by side along N
#ifndef UAII_PF_KTILE
#define UAII_PF_KTILE 1  // Q4_K takes the 64 x 32 wave tile too (0: always 32 x 32)
#endif
#ifndef UAII_PF_ROW
#define UAII_PF_ROW 40
#endif
#ifndef UAII_PF_KS_BPC
// K split target: four-wave block equivalents per CU. 4 (two 8-wave blocks per
// CU) measured 26.2k against 25.5k tok/s for 2 on the 8B prompt (down, O and
// QKV 3-12 % faster, the partial fold in the next prep 1.4 ms slower); 8 25.2k
#define UAII_PF_KS_BPC 4
#endif
#ifndef UAII_PF_K6TILE
// Q6_K takes the 64 x 32 wave tile where the grid allows (0: always 32 x 32):
// 1B down 14.3 -> 11.3 ms per prompt with the former 16x16x16 decode
#define UAII_PF_K6TILE 1
#endif
#ifndef UAII_PF_DW
#define UAII_PF_DW 8  // waves per block of the direct-to-LDS kernel (4 or 8)
#endif
#ifndef UAII_PF_XCD
#define UAII_PF_XCD 1  // XCD-aware block order in the direct-to-LDS kernel
#endif
constexpr int PF_ROW = UAII_PF_ROW;  // halfs per staged 32-k row (32 + 8 pad)

// LDS: [buffer 2][block 2][hi/lo 2][BM rows][PF_ROW halfs]
template <int MT>
constexpr int pf_lds_halfs() { return 2 * 2 * 2 * 16 * MT * PF_ROW; }

// Output rows [m0, mend) of this grid row and the first weight row of its
// expert (0 without grouping).
struct PfRange {
  int64_t m0, mend, mfirst, wrow0;
};
__device__ inline PfRange pf_range(const PfGemmArgs& a, int bm, int64_t seg_rows, int gy = -1) {
  if (gy < 0) gy = blockIdx.y;
  PfRange r;
  if (a.gtab) {
    const int32_t* e = a.gtab + 3 * gy;
    r.wrow0 = (int64_t)e[0] * seg_rows;
    r.m0 = e[1];
    r.mend = e[2];
    r.mfirst = r.m0;
  } else {
    r.wrow0 = 0;
    r.m0 = (int64_t)gy * bm;
    r.mend = a.M;
    r.mfirst = 0;
  }
  return r;
}
// Activation row of output row t. Rows past the range read its first row (the
// map's first entry without grouping); their results are dropped. Unmapped,
// ungrouped rows below mpad are read as they are.
__device__ inline int64_t pf_arow(const PfGemmArgs& a, const PfRange& r, int64_t t) {
  if (!a.arow && !a.gtab) return t;
  const int64_t tc = t < r.mend ? t : r.mfirst;
  return a.arow ? (int64_t)a.arow[tc] : tc;
}

// Block tile: 16 MT activation rows x PF_WAVES * 16 NT weight rows (for SwiGLU
// each wave's NT subtiles are NT / 2 gate and NT / 2 up subtiles of the same
// rows). K advances one stage (64) at a time; activations are staged in LDS
// (double-buffered), each lane loads its weight bytes one stage ahead.
template <int FMT, int EPI, int MT, int NT>
__global__ void __launch_bounds__(PF_WAVES * 64, 2) k_pf_gemm(PfGemmArgs a) {
  constexpr int BM = 16 * MT;
  constexpr bool OFF = pf_offset<FMT>();
  constexpr int NQ = (EPI == EPI_SWIGLU) ? NT / 2 : NT;  // distinct row subtiles
  __shared__ _Float16 lds[pf_lds_halfs<MT>()];

  // segment of this column tile
  const int tile = blockIdx.x;
  int si = 0;
  for (int k = 1; k < a.nseg; ++k) if (tile >= a.seg[k].tile0) si = k;
  const PfSeg& seg = a.seg[si];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int col = lane & 15, g = lane >> 4;
  const int64_t n0 = ((int64_t)(tile - seg.tile0) * PF_WAVES + wave) * (16 * NQ);
  const PfRange mr = pf_range(a, BM, seg.rows);
  const int64_t m0 = mr.m0;
  const int64_t K = a.K, nst = K / 64 / a.ksplit;  // stages of this block's K range
  const int64_t sbase = (int64_t)blockIdx.z * nst;  // its first stage

  // weight rows of this lane per subtile (clamped: rows past the end are loaded, not stored)
  PfRow prow[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int64_t r = n0 + 16 * (j % NQ) + col;
    const DevWeight& w = (EPI == EPI_SWIGLU && j >= NQ) ? seg.w2 : seg.w;
    prow[j] = pf_row<FMT>(w, mr.wrow0 + (r < seg.rows ? r : seg.rows - 1), g);
  }

  f4_t acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

  auto arow_of = [&](int64_t t) __attribute__((always_inline)) -> int64_t { return pf_arow(a, mr, t); };
  // activation stage: BM rows x 2 blocks x (hi, lo) x 4 pieces of 16 B
  constexpr int PIECES = BM * 2 * 2 * 4;
  constexpr int PPT = PIECES / (PF_WAVES * 64);
  static_assert(PIECES % (PF_WAVES * 64) == 0, "stage pieces per thread");
  // activation pieces one stage ahead (stored to the other LDS buffer after the
  // compute), weight bytes two stages ahead in a ring of 3; ring indices are
  // compile-time constants
  uint4 stg[PPT];
  PfRaw<FMT> raw[3][NT];
  // this thread's activation pieces at stage 0 of the block's K range (a stage
  // adds 64 halfs); row offsets and the row map are read once, not per stage
  const __half* abase[PPT];
#pragma unroll
  for (int u = 0; u < PPT; ++u) {
    const int c = threadIdx.x + u * PF_WAVES * 64;
    const int q = c & 3, r = (c >> 2) % BM, kbh = (c >> 2) / BM;  // kbh = block * 2 + hi/lo
    abase[u] = ((kbh & 1) ? a.alo : a.ahi) + arow_of(m0 + r) * K + (2 * sbase + (kbh >> 1)) * 32 + q * 8;
  }
  // Q4_K: the activation block sums of the stage's two blocks, staged beside the
  // activations (threads < 2 BM, one value each) instead of read from memory
  // inside the compute, where the wait for them would also wait for every load
  // in flight
  __shared__ float sxs[OFF ? 2 * 2 * BM : 1];
  float stg_sx = 0.0f;
  const float* sxbase = nullptr;
  if constexpr (OFF) {
    const int t = threadIdx.x < 2 * BM ? threadIdx.x : 0;
    sxbase = a.sx + (2 * sbase + t / BM) * a.sx_ld + arow_of(m0 + t % BM);
  }
  auto load_stage = [&](uint4 (&dst)[PPT], int64_t st) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < PPT; ++u) {
      // element-wise: a whole-struct copy here is turned into a memcpy into a
      // stack array (scratch memory)
      const uint4 v = *reinterpret_cast<const uint4*>(abase[u] + st * 64);
      dst[u].x = v.x;
      dst[u].y = v.y;
      dst[u].z = v.z;
      dst[u].w = v.w;
    }
    if constexpr (OFF) stg_sx = sxbase[st * 2 * a.sx_ld];
  };
  auto store_stage = [&](const uint4 (&src)[PPT], int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < PPT; ++u) {
      const int c = threadIdx.x + u * PF_WAVES * 64;
      const int q = c & 3, r = (c >> 2) % BM, kbh = (c >> 2) / BM;
      _Float16* dst = lds + (((buf * 4) + kbh) * BM + r) * PF_ROW + q * 8;
      *reinterpret_cast<uint4*>(dst) = src[u];
    }
    if constexpr (OFF) {
      if (threadIdx.x < 2 * BM) sxs[buf * 2 * BM + threadIdx.x] = stg_sx;
    }
  };
  auto load_w = [&](PfRaw<FMT>(&dst)[NT], int64_t st) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < NT; ++j) pf_load<FMT>(prow[j], sbase + st, dst[j]);
  };
  // LDS writes done, then the block barrier. No memory fence: a fence would also
  // wait for the weight and activation loads in flight for later stages.
  auto lds_barrier = []() __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt, expcnt untouched
    __builtin_amdgcn_s_barrier();
  };
  auto compute = [&](const PfRaw<FMT>(&rw)[NT], int64_t stl, int buf) __attribute__((always_inline)) {
    const int64_t st = sbase + stl;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      PfFrag<FMT> fr[NT];
#pragma unroll
      for (int j = 0; j < NT; ++j) pf_decode<FMT>(rw[j], st, s, g, fr[j]);
      const _Float16* base = lds + ((buf * 2 + s) * 2) * BM * PF_ROW;
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const _Float16* ph = base + (16 * i + col) * PF_ROW;
        const _Float16* pl = ph + BM * PF_ROW;
        f4_t sxv = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (OFF) {
          const float4 s4 = *reinterpret_cast<const float4*>(sxs + (buf * 2 + s) * BM + 16 * i + 4 * g);
          sxv = f4_t{s4.x, s4.y, s4.z, s4.w};
        }
        const h8_t ahi = *reinterpret_cast<const h8_t*>(ph + 8 * g);
        const h8_t alo = *reinterpret_cast<const h8_t*>(pl + 8 * g);
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          f4_t p = mfma32(ahi, fr[j].b, f4_t{0.0f, 0.0f, 0.0f, 0.0f});
          p = mfma32(alo, fr[j].b, p);
          if constexpr (pf_split_b<FMT>()) p = mfma32(ahi, fr[j].blo, p);  // (hi, lo) x lo: ~2^-21
          acc[i][j] += fr[j].sc[0] * p;
          if constexpr (OFF) acc[i][j] -= fr[j].off * sxv;
        }
      }
    }
  };
  // one stage: prefetch activations of st + 1 and weights of st + 2, compute
  // stage st, move stage st + 1 into the other LDS buffer
  auto step = [&](auto ws, int64_t st) __attribute__((always_inline)) {
    constexpr int W = decltype(ws)::value;
    if (st + 1 < nst) load_stage(stg, st + 1);
    if (st + 2 < nst) load_w(raw[(W + 2) % 3], st + 2);
    compute(raw[W], st, (int)(st & 1));
    if (st + 1 < nst) store_stage(stg, (int)((st + 1) & 1));
    lds_barrier();
  };

  load_w(raw[0], 0);
  if (nst > 1) load_w(raw[1], 1);
  load_stage(stg, 0);
  store_stage(stg, 0);
  lds_barrier();
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  for (int64_t st = 0; st < nst; st += 3) {
    step(I0{}, st);
    if (st + 1 >= nst) break;
    step(I1{}, st + 1);
    if (st + 2 >= nst) break;
    step(I2{}, st + 2);
  }

  // epilogue: lane holds rows m0 + 16i + 4g + r of column n0 + 16j + col
#pragma unroll
  for (int i = 0; i < MT; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t t = m0 + 16 * i + 4 * g + r;
      if (t >= mr.mend) continue;
      const float rs = a.rs[pf_arow(a, mr, t)];
      float* yrow = a.y + t * a.ldy + seg.col0;
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        const int64_t n = n0 + 16 * j + col;
        if (n >= seg.rows) continue;
        const float v = acc[i][j][r] * rs;
        if constexpr (EPI == EPI_STORE) {
          if (a.ksplit > 1) a.part[((int64_t)blockIdx.z * a.M + t) * a.ldy + seg.col0 + n] = v;
          else yrow[n] = v;
        } else if constexpr (EPI == EPI_ADD) {
          if (a.ksplit > 1) a.part[((int64_t)blockIdx.z * a.M + t) * a.ldy + seg.col0 + n] = v;
          else yrow[n] = yrow[n] + v;
        } else if constexpr (EPI == EPI_SWIGLU) {
          const float u = acc[i][j + NQ][r] * rs;
          const float act = v / (1.0f + expf(-v));  // silu (elementwise.cpp:73-84)
          yrow[n] = act * u;
        } else if constexpr (EPI == EPI_GELU) {
          const float inner = 0.7978845608f * (v + 0.044715f * v * v * v);
          yrow[n] = 0.5f * v * (1.0f + tanhf(inner));
        }
      }
    }
  }
}

// ---- GEMM with direct-to-LDS loads (Q4_0, Q8_0) -----------------------------------------
//
// Same tile math as k_pf_gemm, but activations and weight bytes travel global ->
// LDS with global_load_lds_dwordx4 / _dword (lane i of an instruction writes the
// 16 (4) bytes at M0 + 16 i (4 i)), so no registers hold data in flight and a
// ring of three LDS stages keeps two stages of loads outstanding. The loads are
// issued from inline assembly and their completion is waited for with explicit
// vmcnt counts: the compiler would otherwise wait for every outstanding LDS
// load before each LDS read. Both operands stay row-major in LDS (the lanes
// of one DMA instruction that share a row fetch its contiguous bytes), with
// the 16-byte pieces of each row XOR-permuted so that the fragment reads are
// free of bank conflicts on gfx950: activation piece p of row r sits in slot
// p ^ ((r >> 1) & 3); weight part p of row r (32- or 64-byte rows) in slot
// p ^ ((r >> 3) & 1) for Q4_0, p ^ ((r >> 2) & 3) for Q8_0. Measured with
// SQ_LDS_BANK_CONFLICT: unpermuted rows cost 4 conflict cycles per 16-byte
// activation read and 2 (Q4_0) or 6 (Q8_0) per 8-byte weight read, as does
// the permutation p ^ (((r >> 1) ^ (r >> 3)) & 3) for the activations.
//
// The LDS address goes to the asm as an M0 operand ("{m0}"), so the compiler
// writes M0 itself and knows it holds that value; the s_nop gives the one wait
// state an LDS DMA needs after an M0 write.

__device__ inline void dma16(const void* g, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"{m0}"(lds), "v"(g) : "memory");
}
__device__ inline void dma4(const void* g, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %1, off" ::"{m0}"(lds), "v"(g) : "memory");
}
// The same 16-byte copy from a wave-uniform base (scalar registers) plus the
// lane's 32-bit byte offset: no per-lane 64-bit address arithmetic per stage.
__device__ inline void dma16s(const void* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"{m0}"(lds), "v"(voff), "s"(sbase)
               : "memory");
}
// A pointer the wave holds in common, made visibly uniform so that it lives in
// scalar registers.
__device__ inline const uint8_t* uniform_ptr(const void* p) {
  const uint64_t u = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  return reinterpret_cast<const uint8_t*>((uintptr_t)(((uint64_t)hi << 32) | lo));
}
__device__ inline uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p);
}
__device__ inline int pf_swz(int r) { return (r >> 1) & 3; }
template <int FMT>
__device__ inline int pf_wswz(int r) { return FMT == T_Q4_0 ? (r >> 3) & 1 : (r >> 2) & 3; }

template <int FMT>
constexpr int dma_qbytes() { return FMT == T_Q8_0 ? 64 : 32; }  // payload bytes per row per stage
template <int MT>
constexpr int dma_a_bytes() { return 2 * 2 * 16 * MT * 64; }      // [block][hi/lo][row][64 B]
// per wave: the payload of its 16 NT rows, then a 256-byte scale area (a dword per row)
template <int FMT, int NT>
constexpr int dma_wave_w_bytes() { return 16 * NT * dma_qbytes<FMT>() + 256; }
// Waves per block of the direct-to-LDS kernel, side by side along N: 8, so
// that with two blocks per CU each SIMD holds four waves.
constexpr int PF_DW = UAII_PF_DW;
template <int FMT, int MT, int NT>
constexpr int dma_stage_bytes() { return dma_a_bytes<MT>() + PF_DW * dma_wave_w_bytes<FMT, NT>(); }
// Activation DMA instructions per wave and stage: the 4 MT (block, hi/lo,
// subtile) copies spread over the waves
template <int MT>
constexpr int dma_a_per_wave() { return 4 * MT / PF_DW; }
// DMA instructions each wave issues per stage (the vmcnt unit)
template <int FMT, int MT, int NT>
constexpr int dma_per_stage() { return dma_a_per_wave<MT>() + 16 * NT * dma_qbytes<FMT>() / 1024 + 1; }
// Weight subtiles per wave: 2 (32 rows). 64-row waves (4) spilled registers at
// the 64 x 64 wave tile.
template <int FMT>
constexpr int dma_nt() { return 2; }

template <int FMT, int EPI, int MT, int NT, bool H16>
__global__ void __launch_bounds__(PF_DW * 64, 2) k_pf_gemm_dma(PfGemmArgs a) {
  static_assert(NT == 2 || NT == 4, "weight subtiles per wave");
  static_assert((4 * MT) % PF_DW == 0, "activation copies per wave");
  constexpr int NA = dma_a_per_wave<MT>();
  constexpr int BM = 16 * MT;
  constexpr int NQ = (EPI == EPI_SWIGLU) ? NT / 2 : NT;
  constexpr int NR = 16 * NT;  // weight rows per wave
  constexpr int QB = dma_qbytes<FMT>();
  constexpr int WB = dma_wave_w_bytes<FMT, NT>();
  constexpr int SB = dma_stage_bytes<FMT, MT, NT>();
  constexpr int ND = dma_per_stage<FMT, MT, NT>();
  static_assert(ND <= 15, "vmcnt immediate");
  __shared__ __attribute__((aligned(16))) uint8_t lds[3 * SB];

  // Grid position. Blocks go to the XCDs round-robin in dispatch order; with
  // the column-tile count a multiple of 8, XCD x takes the column tiles
  // 8 c + x, and within an XCD the blocks are renumbered row tile fastest, so
  // that the blocks resident on one XCD share their weight columns in its L2.
  int tile = blockIdx.x, gy = blockIdx.y;
#if UAII_PF_XCD
  if ((gridDim.x & 7) == 0) {
    const int id = blockIdx.y * gridDim.x + blockIdx.x;
    const int loc = id >> 3;
    gy = loc % gridDim.y;
    tile = (loc / gridDim.y) * 8 + (id & 7);
  }
#endif
  int si = 0;
  for (int k = 1; k < a.nseg; ++k) if (tile >= a.seg[k].tile0) si = k;
  const PfSeg& seg = a.seg[si];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int col = lane & 15, g = lane >> 4;
  const int64_t n0 = ((int64_t)(tile - seg.tile0) * PF_DW + wave) * (16 * NQ);
  const PfRange mr = pf_range(a, BM, seg.rows, gy);
  const int64_t m0 = mr.m0;
  const int64_t K = a.K;
  const int nst = (int)(K / 64 / a.ksplit);         // stages of this block's K range
  const int64_t sbase = (int64_t)blockIdx.z * nst;  // its first stage

  // this lane's DMA sources. Activations: wave w copies (block (w >> 1) & 1,
  // hi/lo w & 1) of the row subtiles NA (w >> 2) .. NA (w >> 2) + NA - 1;
  // instruction u covers rows 16 u' .. 16 u' + 15 of its subtile u', lane ->
  // (row, slot).
  const int arow_l = lane >> 2, aslot = lane & 3;
  const __half* asrc = (wave & 1) ? a.alo : a.ahi;
  const int ablk = (wave >> 1) & 1;
  const int asub0 = NA * (wave >> 2);
  // the lane's byte offset of its row's piece (stage independent; the launch
  // checks that the activation array spans under 2^31 bytes) and the wave's
  // scalar base, to which stage st adds 128 st bytes (64 k of f16)
  uint32_t aoff[NA];
#pragma unroll
  for (int u = 0; u < NA; ++u) {
    const int r = 16 * (asub0 + u) + arow_l;
    const int piece = aslot ^ pf_swz(r);
    aoff[u] = (uint32_t)(pf_arow(a, mr, m0 + r) * K * 2) + (uint32_t)(ablk * 64 + piece * 16);
  }
  const uint8_t* abase = uniform_ptr(asrc);
  // Weights: the wave's 32 rows (subtile j = row / 16; SwiGLU: j = 1 is the up
  // tensor); a row's stage payload is WP 16-byte parts, and LDS slot
  // q = 64 u + lane of the payload is slot q % WP of row q / WP. One dword per
  // row of scales.
  constexpr int WP = QB / 16;
  constexpr int NWQ = NR * QB / 1024;  // payload DMA instructions per stage
  const uint8_t* wsrc_q[NWQ];
#pragma unroll
  for (int u = 0; u < NWQ; ++u) {
    const int q = lane + 64 * u;
    const int rl = q / WP, part = (q % WP) ^ pf_wswz<FMT>(rl);
    const int j = rl >> 4;
    const DevWeight& w = (EPI == EPI_SWIGLU && j >= NQ) ? seg.w2 : seg.w;
    int64_t r = n0 + 16 * (j % NQ) + (rl & 15);
    r = mr.wrow0 + (r < seg.rows ? r : seg.rows - 1);
    wsrc_q[u] = w.a + r * w.a_row + 16 * part;
  }
  const uint8_t* wsrc_s;
  {
    const int rl = lane & (NR - 1);
    const int j = rl >> 4;
    const DevWeight& w = (EPI == EPI_SWIGLU && j >= NQ) ? seg.w2 : seg.w;
    int64_t r = n0 + 16 * (j % NQ) + (rl & 15);
    r = mr.wrow0 + (r < seg.rows ? r : seg.rows - 1);
    wsrc_s = w.b + r * w.b_row;
  }

  auto issue = [&](int stl, int slot) __attribute__((always_inline)) {
    const int64_t st = sbase + stl;
    uint8_t* base = lds + slot * SB;
    // activations
#pragma unroll
    for (int u = 0; u < NA; ++u)
      dma16s(uniform_ptr(abase + st * 128), aoff[u],
             lds_addr(base + ((ablk * 2 + (wave & 1)) * BM + 16 * (asub0 + u)) * 64));
    // weight payload and scales of this wave's rows
    uint8_t* wb = base + dma_a_bytes<MT>() + wave * WB;
#pragma unroll
    for (int u = 0; u < NWQ; ++u) dma16(wsrc_q[u] + st * QB, lds_addr(wb + u * 1024));
    dma4(wsrc_s + st * 4, lds_addr(wb + NR * QB));
  };
  auto wait_stage = [&](int st) __attribute__((always_inline)) {
    // stage st is complete when at most the next stage's loads are outstanding
    if (st + 1 < nst) __builtin_amdgcn_s_waitcnt(0x0f70 | ND);  // vmcnt(ND), lgkm/exp untouched
    else __builtin_amdgcn_s_waitcnt(0x0f70);                    // vmcnt(0)
    __builtin_amdgcn_s_barrier();
  };

  f4_t acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

  auto compute = [&](int stl, int slot) __attribute__((always_inline)) {
    const int64_t st = sbase + stl;
    const uint8_t* base = lds + slot * SB;
    const uint8_t* wb = base + dma_a_bytes<MT>() + wave * WB;
    PfRaw<FMT> rw[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      // block s of the row: part s (Q4_0: 16 bytes, lane half g & 1) or parts
      // 2 s, 2 s + 1 (Q8_0: 32 bytes, lane quarter g)
      const uint8_t* rowp = wb + (16 * j + col) * QB;
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        const int part = (FMT == T_Q4_0) ? sb : 2 * sb + (g >> 1);
        rw[j].q[sb] = *reinterpret_cast<const uint2*>(rowp + 16 * (part ^ pf_wswz<FMT>(col)) + 8 * (g & 1));
      }
      rw[j].d = *reinterpret_cast<const uint32_t*>(wb + NR * QB + 4 * (16 * j + col));
    }
    // Steps (block sb, subtile i) in order, each fenced from the next so that
    // the registers live at once stay bounded: a step reads the next step's A
    // fragments, issues its own matrix-core ops, then applies the previous
    // step's block scales while those ops run.
    auto afrag = [&](int sb, int i, h8_t& hi, h8_t& lo) __attribute__((always_inline)) {
      const int r = 16 * i + col;
      const int off = r * 64 + 16 * (g ^ pf_swz(r));
      hi = *reinterpret_cast<const h8_t*>(base + ((sb * 2 + 0) * BM) * 64 + off);
      lo = *reinterpret_cast<const h8_t*>(base + ((sb * 2 + 1) * BM) * 64 + off);
    };
    h8_t nhi, nlo;
    afrag(0, 0, nhi, nlo);
    f4_t pp[NT];
    float psc[NT];
    PfFrag<FMT> fr[NT];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
#pragma unroll
      for (int j = 0; j < NT; ++j) pf_decode<FMT, H16>(rw[j], st, sb, g, fr[j]);
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const int step = sb * MT + i;
        const h8_t ahi = nhi, alo = nlo;
        if (step + 1 < 2 * MT) afrag((step + 1) / MT, (step + 1) % MT, nhi, nlo);
        f4_t pc[NT];
#pragma unroll
        for (int j = 0; j < NT; ++j) pc[j] = mfma32(ahi, fr[j].b, f4_t{0.0f, 0.0f, 0.0f, 0.0f});
#pragma unroll
        for (int j = 0; j < NT; ++j) pc[j] = mfma32(alo, fr[j].b, pc[j]);
        if (step > 0) {
#pragma unroll
          for (int j = 0; j < NT; ++j) acc[(step - 1) % MT][j] += psc[j] * pp[j];
        }
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          pp[j] = pc[j];
          psc[j] = fr[j].sc[0];
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[MT - 1][j] += psc[j] * pp[j];
  };

  issue(0, 0);
  if (nst > 1) issue(1, 1);
  for (int st = 0; st < nst; st += 3) {
    wait_stage(st);
    if (st + 2 < nst) issue(st + 2, 2);
    compute(st, 0);
    if (st + 1 >= nst) break;
    wait_stage(st + 1);
    if (st + 3 < nst) issue(st + 3, 0);
    compute(st + 1, 1);
    if (st + 2 >= nst) break;
    wait_stage(st + 2);
    if (st + 4 < nst) issue(st + 4, 1);
    compute(st + 2, 2);
  }

  // epilogue: lane holds rows m0 + 16i + 4g + r of column n0 + 16j + col
#pragma unroll
  for (int i = 0; i < MT; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t t = m0 + 16 * i + 4 * g + r;
      if (t >= mr.mend) continue;
      const float rs = a.rs[pf_arow(a, mr, t)];
      float* yrow = a.y + t * a.ldy + seg.col0;
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        const int64_t n = n0 + 16 * j + col;
        if (n >= seg.rows) continue;
        const float v = acc[i][j][r] * rs;
        if constexpr (EPI == EPI_STORE) {
          if (a.ksplit > 1) a.part[((int64_t)blockIdx.z * a.M + t) * a.ldy + seg.col0 + n] = v;
          else yrow[n] = v;
        } else if constexpr (EPI == EPI_ADD) {
          if (a.ksplit > 1) a.part[((int64_t)blockIdx.z * a.M + t) * a.ldy + seg.col0 + n] = v;
          else yrow[n] = yrow[n] + v;
        } else if constexpr (EPI == EPI_SWIGLU) {
          const float u = acc[i][j + NQ][r] * rs;
          const float act = v / (1.0f + expf(-v));  // silu (elementwise.cpp:73-84)
          yrow[n] = act * u;
        } else if constexpr (EPI == EPI_GELU) {
          const float inner = 0.7978845608f * (v + 0.044715f * v * v * v);
          yrow[n] = 0.5f * v * (1.0f + tanhf(inner));
        }
      }
    }
  }
}

// ---- QKV post-processing ------------------------------------------------------------------

// One block per token: bias, RoPE of q and k pairs (host-built angle table, as
// the decode epilogue), q -> qout, k and v -> cache at position p0 + t.
__global__ void __launch_bounds__(256) k_pf_qkv(PfQkvArgs a) {
  const int64_t t = blockIdx.x;
  const int pos = a.p0 + (int)t;
  const float* row = a.qkv + t * a.ldq;
  // value x of this row: the GEMM's output, or the sum of its K-split partials
  // in split order
  auto val = [&](int x) -> float {
    if (a.nsplit <= 1) return row[x];
    float v = a.part[t * a.ldq + x];
    for (int z = 1; z < a.nsplit; ++z) v = v + a.part[((int64_t)z * a.M + t) * a.ldq + x];
    return v;
  };
  const int hd = a.head_dim, half = hd / 2;
  const int npair = (a.q_dim + a.kv_dim) / 2;
  for (int u = threadIdx.x; u < npair; u += blockDim.x) {
    const bool isq = u < a.q_dim / 2;
    const int uu = isq ? u : u - a.q_dim / 2;
    const int head = uu / half, p = uu % half;
    const int r0 = head * hd + (a.rope_mode == 2 ? p : 2 * p);
    const int r1 = r0 + (a.rope_mode == 2 ? half : 1);
    const int base = isq ? 0 : a.q_dim;
    float v0 = val(base + r0), v1 = val(base + r1);
    const float* bias = isq ? a.bq : a.bk;
    if (bias) { v0 = v0 + bias[r0]; v1 = v1 + bias[r1]; }
    const float2 cs = a.rope[(int64_t)pos * half + p];
    const float n0 = v0 * cs.x - v1 * cs.y;
    const float n1 = v0 * cs.y + v1 * cs.x;
    if (isq) {
      a.qout[t * a.q_dim + r0] = n0;
      a.qout[t * a.q_dim + r1] = n1;
    } else {
      const int64_t o0 = ((int64_t)(r0 / hd) * a.max_seq + pos) * hd + (r0 % hd);
      const int64_t o1 = ((int64_t)(r1 / hd) * a.max_seq + pos) * hd + (r1 % hd);
      if (a.kv_f16) {
        reinterpret_cast<__half*>(a.kcache)[o0] = __float2half(n0);
        reinterpret_cast<__half*>(a.kcache)[o1] = __float2half(n1);
      } else {
        reinterpret_cast<float*>(a.kcache)[o0] = n0;
        reinterpret_cast<float*>(a.kcache)[o1] = n1;
      }
    }
  }
  for (int r = threadIdx.x; r < a.kv_dim; r += blockDim.x) {
    float v = val(a.q_dim + a.kv_dim + r);
    if (a.bv) v = v + a.bv[r];
    const int64_t o = ((int64_t)(r / hd) * a.max_seq + pos) * hd + (r % hd);
    if (a.kv_f16) reinterpret_cast<__half*>(a.vcache)[o] = __float2half(v);
    else reinterpret_cast<float*>(a.vcache)[o] = v;
  }
}

// ---- causal attention over the f16 cache ---------------------------------------------------

constexpr int PA_TK = 64;  // keys per LDS tile
// 16-query subtiles per wave. 2 halves the K/V staging per matrix-core op but
// needs 430 registers at head_dim 128 (one wave per SIMD): measured 1.6x slower
// than 1 on the 8B prefill.
#ifndef UAII_PA_QW
#define UAII_PA_QW 1
#endif
constexpr int PA_QW = UAII_PA_QW;

// Block: 4 waves on kv head blockIdx.y / (G / GW); wave w takes q head
// (w % GW) of the block's GW heads and query subtiles PA_QW (w / GW) ..
// PA_QW (w / GW) + PA_QW - 1 (16 queries each). K tiles and transposed V tiles
// of 64 keys are double-buffered in LDS; each thread loads the next tile's K/V
// pieces into registers while the current tile is computed.
template <int HD>
__global__ void __launch_bounds__(256, 2) k_pf_attn(PfAttnArgs a) {
  constexpr int KP = HD + 8;        // K tile row (halfs)
  constexpr int VP = PA_TK + 8;     // V^T tile row (halfs)
  constexpr int NC = HD / 32;       // 32-wide hd chunks (S)
  constexpr int ND = HD / 16;       // 16-row hd subtiles (O)
  constexpr int KPIECES = PA_TK * (HD / 8) / 256;       // 16-byte K pieces per thread
  constexpr int VPAIRS = PA_TK / 2 * (HD / 8) / 256;    // (2 keys x 8 dims) V pieces per thread
  __shared__ _Float16 ks[2][PA_TK * KP];
  __shared__ _Float16 vt[2][HD * VP];

  const int G = a.n_heads / a.n_kv;
  const int GW = G < 4 ? G : 4;
  const int QS = 4 / GW;
  const int hb = blockIdx.y;
  const int kvh = hb / (G / GW);
  const int hbase = kvh * G + (hb % (G / GW)) * GW;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, col = lane & 15, g = lane >> 4;
  const bool active = wave < GW * QS;
  const int head = hbase + (wave % GW);
  const int64_t q0 = (int64_t)blockIdx.x * (16 * PA_QW * QS);
  const int64_t qw0 = q0 + 16 * PA_QW * (wave / GW);   // this wave's first query
  const int64_t qend = min((int64_t)a.M, q0 + 16 * PA_QW * QS);
  const int64_t nkeys = a.p0 + qend;  // keys the block needs (causal)

  // q * scale * 2^e as f16 hi + lo per query subtile u: lane (query col, group g)
  // holds hd 32c + 8g .. +7 of chunk c; the matrix cores flush f16 subnormals,
  // so each query row is scaled to put its largest element in [2^14, 2^15)
  const float scale = 1.0f / sqrtf((float)HD);
  h8_t qhi[PA_QW][NC], qlo[PA_QW][NC];
  float qrs[PA_QW];
  bool qvalid[PA_QW];
  int64_t qpos[PA_QW];
#pragma unroll
  for (int u = 0; u < PA_QW; ++u) {
    const int64_t qrow = qw0 + 16 * u + col;
    qvalid[u] = active && qrow < a.M;
    qpos[u] = a.p0 + qrow;
    float qv[NC][8];
    float qmax = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if (qvalid[u]) {
        const float4* qp = reinterpret_cast<const float4*>(a.q + qrow * a.ldq + (int64_t)head * HD + 32 * c + 8 * g);
        const float4 x0 = qp[0], x1 = qp[1];
        qv[c][0] = x0.x; qv[c][1] = x0.y; qv[c][2] = x0.z; qv[c][3] = x0.w;
        qv[c][4] = x1.x; qv[c][5] = x1.y; qv[c][6] = x1.z; qv[c][7] = x1.w;
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) qv[c][k] = 0.0f;
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        qv[c][k] = qv[c][k] * scale;
        qmax = fmaxf(qmax, fabsf(qv[c][k]));
      }
    }
    qmax = fmaxf(qmax, __shfl_xor(qmax, 16, 64));
    qmax = fmaxf(qmax, __shfl_xor(qmax, 32, 64));
    int qe = 0;
    if (qmax > 0.0f) qe = min(100, max(-100, 15 - ((int)((__float_as_uint(qmax) >> 23) & 0xff) - 126)));
    const float qs = pow2f_i(qe);
    qrs[u] = pow2f_i(-qe);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float v = qv[c][k] * qs;
        const _Float16 h = (_Float16)v;
        qhi[u][c][k] = h;
        qlo[u][c][k] = (_Float16)(v - (float)h);
      }
    }
  }

  // scale of the raw scores into base-2 exponent units, and the causal limits
  // in 32-bit positions (a cache holds < 2^31 keys)
  float l2s[PA_QW];
  int qposi[PA_QW];
#pragma unroll
  for (int u = 0; u < PA_QW; ++u) {
    l2s[u] = qrs[u] * 1.4426950408889634f;
    qposi[u] = (int)qpos[u];
  }
  const int64_t qpos0 = a.p0 + qw0;  // the wave's first query position
  f4_t o[PA_QW][ND];
  float mrun[PA_QW], lrun[PA_QW];
#pragma unroll
  for (int u = 0; u < PA_QW; ++u) {
    mrun[u] = -INFINITY;
    lrun[u] = 0.0f;
#pragma unroll
    for (int d = 0; d < ND; ++d) o[u][d] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
  }

  const __half* kbase = reinterpret_cast<const __half*>(a.kcache) + (int64_t)kvh * a.max_seq * HD;
  const __half* vbase = reinterpret_cast<const __half*>(a.vcache) + (int64_t)kvh * a.max_seq * HD;

  // tile staging: K pieces (key, 8 dims) and V pairs (keys 2k, 2k + 1, 8 dims);
  // keys past nkeys read as zeros. Offsets inside a tile are 32-bit and fixed
  // per thread; only the last tile checks them against nkeys.
  uint4 kreg[KPIECES], vreg[VPAIRS][2];
  auto load_tile = [&](int64_t kt) __attribute__((always_inline)) {
    const __half* kt_base = reinterpret_cast<const __half*>(uniform_ptr(kbase + kt * HD));
    const __half* vt_base = reinterpret_cast<const __half*>(uniform_ptr(vbase + kt * HD));
    const bool full = kt + PA_TK <= nkeys;  // block-uniform
#pragma unroll
    for (int u = 0; u < KPIECES; ++u) {
      const int c = threadIdx.x + 256 * u;
      const int key = c / (HD / 8), p = c % (HD / 8);
      kreg[u] = make_uint4(0, 0, 0, 0);
      if (full || kt + key < nkeys) kreg[u] = *reinterpret_cast<const uint4*>(kt_base + (key * HD + 8 * p));
    }
#pragma unroll
    for (int u = 0; u < VPAIRS; ++u) {
      const int c = threadIdx.x + 256 * u;
      const int kp = c / (HD / 8), p = c % (HD / 8);
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        vreg[u][e] = make_uint4(0, 0, 0, 0);
        if (full || kt + 2 * kp + e < nkeys)
          vreg[u][e] = *reinterpret_cast<const uint4*>(vt_base + ((2 * kp + e) * HD + 8 * p));
      }
    }
  };
  auto store_tile = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < KPIECES; ++u) {
      const int c = threadIdx.x + 256 * u;
      const int key = c / (HD / 8), p = c % (HD / 8);
      *reinterpret_cast<uint4*>(&ks[buf][key * KP + 8 * p]) = kreg[u];
    }
#pragma unroll
    for (int u = 0; u < VPAIRS; ++u) {
      const int c = threadIdx.x + 256 * u;
      const int kp = c / (HD / 8), p = c % (HD / 8);
      const uint32_t w0[4] = {vreg[u][0].x, vreg[u][0].y, vreg[u][0].z, vreg[u][0].w};
      const uint32_t w1[4] = {vreg[u][1].x, vreg[u][1].y, vreg[u][1].z, vreg[u][1].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // dims 8p + 2e and 8p + 2e + 1 of keys 2kp and 2kp + 1, as key pairs
        const uint32_t lo = (w0[e] & 0xffffu) | (w1[e] << 16);
        const uint32_t hi = (w0[e] >> 16) | (w1[e] & 0xffff0000u);
        *reinterpret_cast<uint32_t*>(&vt[buf][(8 * p + 2 * e) * VP + 2 * kp]) = lo;
        *reinterpret_cast<uint32_t*>(&vt[buf][(8 * p + 2 * e + 1) * VP + 2 * kp]) = hi;
      }
    }
  };
  auto lds_barrier = []() __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
  };

  auto compute = [&](int64_t kt, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < PA_QW; ++u) {
      // S^T for 4 key subtiles: lane holds keys kt + 16s + 4g + r of query col
      // raw scores (q pre-scaled by 2^qe); the running max and the exponentials
      // are in base 2: score * log2(e) = acc * l2s, p = 2^(acc * l2s - m)
      f4_t sc[4];
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        f4_t acc = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const h8_t kf = *reinterpret_cast<const h8_t*>(&ks[buf][(16 * s4 + col) * KP + 32 * c + 8 * g]);
          acc = mfma32(kf, qhi[u][c], acc);
          acc = mfma32(kf, qlo[u][c], acc);
        }
        sc[s4] = acc;
      }
      // causal mask only on tiles that reach past the wave's first query
      // (rows past M are never stored and need none)
      if (kt + PA_TK - 1 > qpos0) {
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int key = (int)kt + 16 * s4 + 4 * g + r;
            if (key > qposi[u]) sc[s4][r] = -INFINITY;
          }
      }
      float tmax = -INFINITY;
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
        for (int r = 0; r < 4; ++r) tmax = fmaxf(tmax, sc[s4][r]);
      tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
      const float mnew = fmaxf(mrun[u], tmax * l2s[u]);
      const float alpha = (mrun[u] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mrun[u] - mnew);
      const float mref = (mnew == -INFINITY) ? 0.0f : mnew;  // a fully masked row so far: p = 0
      float psum = 0.0f;
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = __builtin_amdgcn_exp2f(fmaf(sc[s4][r], l2s[u], -mref));
          sc[s4][r] = p;
          psum += p;
        }
      psum += __shfl_xor(psum, 16, 64);
      psum += __shfl_xor(psum, 32, 64);
      lrun[u] = lrun[u] * alpha + psum;
      mrun[u] = mnew;
      if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int d = 0; d < ND; ++d) o[u][d] *= alpha;
      }
      // O^T += V^T . (2^14 P)^T over two 32-key chunks (p <= 1, so 2^14 p keeps
      // hi and lo normal); lane's keys: 32c + 4g + r (r < 4), 32c + 16 + 4g + (r - 4)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        h8_t phi, plo;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          const float p = sc[2 * c + (r >> 2)][r & 3] * 16384.0f;
          const _Float16 h = (_Float16)p;
          phi[r] = h;
          plo[r] = (_Float16)(p - (float)h);
        }
#pragma unroll
        for (int d = 0; d < ND; ++d) {
          const _Float16* vr = &vt[buf][(16 * d + col) * VP + 32 * c + 4 * g];
          const h4_t v0 = *reinterpret_cast<const h4_t*>(vr);
          const h4_t v1 = *reinterpret_cast<const h4_t*>(vr + 16);
          const h8_t vf = h8_t{v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
          o[u][d] = mfma32(vf, phi, o[u][d]);
          o[u][d] = mfma32(vf, plo, o[u][d]);
        }
      }
    }
  };

  load_tile(0);
  store_tile(0);
  lds_barrier();
  int buf = 0;
  for (int64_t kt = 0; kt < nkeys; kt += PA_TK) {
    const bool more = kt + PA_TK < nkeys;  // block-uniform
    if (more) load_tile(kt + PA_TK);
    if (active) compute(kt, buf);
    if (more) store_tile(buf ^ 1);
    lds_barrier();
    buf ^= 1;
  }

#pragma unroll
  for (int u = 0; u < PA_QW; ++u) {
    if (!qvalid[u]) continue;
    const int64_t qrow = qw0 + 16 * u + col;
    const float inv = (1.0f / 16384.0f) / lrun[u];
    float* out = a.out + qrow * a.ldo + (int64_t)head * HD;
#pragma unroll
    for (int d = 0; d < ND; ++d) {
      const float4 v = make_float4(o[u][d][0] * inv, o[u][d][1] * inv, o[u][d][2] * inv, o[u][d][3] * inv);
      *reinterpret_cast<float4*>(out + 16 * d + 4 * g) = v;
    }
  }
}

// ---- MoE over prompt rows ----------------------------------------------------------------

// Routing of token t on one wave from its E router logits (LDS): softmax
// (exp(l - max) * 1/sum), k rounds of the largest remaining probability (ties:
// the lower expert), weights renormalised over the chosen k
// (transformer.cpp:446-481, :565-580).
__device__ inline void moe_topk(const float* logit, int E, int k, int32_t* __restrict__ ids,
                                float* __restrict__ wout, int64_t t, int lane) {
  float p[4];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane + 64 * j;
    p[j] = e < E ? logit[e] : -INFINITY;
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
  const float isum = sum > 0.0f ? 1.0f / sum : 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) p[j] = (lane + 64 * j < E) ? p[j] * isum : -1.0f;
  float mass = 0.0f;
  float wsel[8];
  int32_t esel[8];
  for (int q = 0; q < k; ++q) {
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
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (j == q) { wsel[j] = bv; esel[j] = (be >= 0 && be < E) ? be : 0; }
    mass += bv;
  }
  if (!(mass > 0.0f)) mass = 1.0f;
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (j < k) {
        ids[t * k + j] = esel[j];
        wout[t * k + j] = wsel[j] / mass;
      }
    }
  }
}

// One block per token: RMSNorm of x[t] (the k_pf_prep arithmetic), router
// logits against F32 / F16 rows, then the routing of k_moe_route on wave 0:
// softmax (exp(l - max) * 1/sum), k rounds of the largest remaining probability
// (ties: the lower expert), weights renormalised over the chosen k
// (transformer.cpp:446-481, :565-580).
template <int RT>
__global__ void __launch_bounds__(256) k_pf_moe_route(const float* __restrict__ x, int64_t K,
                                                      const float* __restrict__ norm_w, float eps,
                                                      DevWeight router, int E, int k,
                                                      int32_t* __restrict__ ids, float* __restrict__ wout) {
  extern __shared__ float row[];
  __shared__ float red[4];
  __shared__ float logit[256];
  const int64_t t = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nv = (int)(K / 4);
  float4* r4 = reinterpret_cast<float4*>(row);
  const float4* x4 = reinterpret_cast<const float4*>(x + t * K);
  float ss = 0.0f;
  for (int i = tid; i < nv; i += 256) {
    const float4 v = x4[i];
    r4[i] = v;
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  }
  ss = wave_sum(ss);
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  const float tot = red[0] + red[1] + red[2] + red[3];
  const float inv = 1.0f / sqrtf(tot / (float)K + eps);
  const float4* w4 = reinterpret_cast<const float4*>(norm_w);
  for (int i = tid; i < nv; i += 256) {
    float4 v = r4[i];
    const float4 w = w4[i];
    v.x = fmul_rn(fmul_rn(v.x, inv), w.x);
    v.y = fmul_rn(fmul_rn(v.y, inv), w.y);
    v.z = fmul_rn(fmul_rn(v.z, inv), w.z);
    v.w = fmul_rn(fmul_rn(v.w, inv), w.w);
    r4[i] = v;
  }
  __syncthreads();
  // logits: wave w takes experts w, w + 4, ...; each lane 4 consecutive inputs
  // per step, the router loads of 8 steps issued before their arithmetic (one
  // memory round trip per 8 steps, not per step)
  constexpr int RB = 8;
  for (int e = wave; e < E; e += 4) {
    float acc = 0.0f;
    const uint8_t* wr = router.a + (int64_t)e * router.a_row;
    for (int base = 0; base < nv; base += 64 * RB) {
      float4 wv[RB];
#pragma unroll
      for (int j = 0; j < RB; ++j) {
        const int i = min(base + 64 * j + lane, nv - 1);
        if constexpr (RT == T_F32) {
          wv[j] = reinterpret_cast<const float4*>(wr)[i];
        } else {
          const uint2 h = reinterpret_cast<const uint2*>(wr)[i];
          wv[j] = make_float4(h2f((uint16_t)(h.x & 0xffff)), h2f((uint16_t)(h.x >> 16)),
                              h2f((uint16_t)(h.y & 0xffff)), h2f((uint16_t)(h.y >> 16)));
        }
      }
#pragma unroll
      for (int j = 0; j < RB; ++j) {
        const int i = base + 64 * j + lane;
        if (i < nv) {
          const float4 xv = r4[i];
          acc += xv.x * wv[j].x + xv.y * wv[j].y + xv.z * wv[j].z + xv.w * wv[j].w;
        }
      }
    }
    acc = wave_sum(acc);
    if (lane == 0) logit[e] = acc;
  }
  __syncthreads();
  if (wave == 0) moe_topk(logit, E, k, ids, wout, t, lane);
}

// The same routing for one token (the decode step) on a 16-wave block: the
// router row of expert e is cut into P parts of up to 512 float4 (8 per lane),
// wave w takes the parts w, w + 16, ..., and its first part's router loads are
// issued before the RMSNorm, so the weight fetch overlaps the input's. The
// parts' sums are added in part order. dynamic LDS: K normalised inputs, then
// the E * P part sums.
template <int RT>
__global__ void __launch_bounds__(1024) k_moe_route_dec(const float* __restrict__ x, int64_t K,
                                                        const float* __restrict__ norm_w, float eps,
                                                        DevWeight router, int E, int k,
                                                        int32_t* __restrict__ ids, float* __restrict__ wout) {
  extern __shared__ float row[];
  __shared__ float red[16];
  __shared__ float logit[256];
  constexpr int RB = 8;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nv = (int)(K / 4);
  const int P = (nv + 64 * RB - 1) / (64 * RB);
  const int items = E * P;
  float* psum = row + K;
  using Raw = typename std::conditional<RT == T_F32, float4, uint2>::type;
  auto load_item = [&](int it, Raw (&wv)[RB]) __attribute__((always_inline)) {
    const int e = it / P, part = it % P;
    const Raw* wr = reinterpret_cast<const Raw*>(router.a + (int64_t)e * router.a_row);
#pragma unroll
    for (int j = 0; j < RB; ++j) wv[j] = wr[min(part * 64 * RB + 64 * j + lane, nv - 1)];
  };
  auto dot_item = [&](int it, const Raw (&wv)[RB]) __attribute__((always_inline)) {
    const int part = it % P;
    const float4* r4 = reinterpret_cast<const float4*>(row);
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < RB; ++j) {
      const int i = part * 64 * RB + 64 * j + lane;
      if (i < nv) {
        float4 w;
        if constexpr (RT == T_F32) {
          w = wv[j];
        } else {
          w = make_float4(h2f((uint16_t)(wv[j].x & 0xffff)), h2f((uint16_t)(wv[j].x >> 16)),
                          h2f((uint16_t)(wv[j].y & 0xffff)), h2f((uint16_t)(wv[j].y >> 16)));
        }
        const float4 xv = r4[i];
        acc += xv.x * w.x + xv.y * w.y + xv.z * w.z + xv.w * w.w;
      }
    }
    acc = wave_sum(acc);
    if (lane == 0) psum[it] = acc;
  };
  Raw w0[RB];
  if (wave < items) load_item(wave, w0);
  // RMSNorm (the k_pf_prep arithmetic) into LDS
  float4* r4 = reinterpret_cast<float4*>(row);
  const float4* x4 = reinterpret_cast<const float4*>(x);
  float ss = 0.0f;
  for (int i = tid; i < nv; i += 1024) {
    const float4 v = x4[i];
    r4[i] = v;
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  }
  ss = wave_sum(ss);
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int w = 0; w < 16; ++w) tot += red[w];
  const float inv = 1.0f / sqrtf(tot / (float)K + eps);
  const float4* n4 = reinterpret_cast<const float4*>(norm_w);
  for (int i = tid; i < nv; i += 1024) {
    float4 v = r4[i];
    const float4 w = n4[i];
    v.x = fmul_rn(fmul_rn(v.x, inv), w.x);
    v.y = fmul_rn(fmul_rn(v.y, inv), w.y);
    v.z = fmul_rn(fmul_rn(v.z, inv), w.z);
    v.w = fmul_rn(fmul_rn(v.w, inv), w.w);
    r4[i] = v;
  }
  __syncthreads();
  if (wave < items) dot_item(wave, w0);
  for (int it = wave + 16; it < items; it += 16) {
    Raw wv[RB];
    load_item(it, wv);
    dot_item(it, wv);
  }
  __syncthreads();
  if (wave != 0) return;
  for (int e = lane; e < E; e += 64) {
    float l = 0.0f;
    for (int q = 0; q < P; ++q) l += psum[e * P + q];
    logit[e] = l;
  }
  moe_topk(logit, E, k, ids, wout, 0, lane);
}

// One block lists each expert's (token, slot) entries in entry order (entry
// i = token * k + slot): counts[e], offsets[e] (exclusive prefix), list[pos] =
// token and inv[i] = pos. Wave w owns the entry range [w n / 4, (w + 1) n / 4):
// range counts by LDS atomics, then each wave walks its range 64 entries at a
// time, a lane's position within its expert being the number of same-expert
// lanes below it (ballot + popcount) past the range's running base.
__global__ void __launch_bounds__(256) k_pf_moe_lists(const int32_t* __restrict__ ids, int64_t M, int k,
                                                      int E, int32_t* counts, int32_t* offsets,
                                                      int32_t* list, int32_t* inv) {
  __shared__ int32_t cnt[4][256], base[4][256];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t n = M * k;
  const int64_t per = (n + 3) / 4;
  const int64_t r0 = min(n, (int64_t)wave * per), r1 = min(n, r0 + per);
  for (int j = tid; j < 4 * 256; j += 256) cnt[j >> 8][j & 255] = 0;
  __syncthreads();
  for (int64_t i = r0 + lane; i < r1; i += 64) atomicAdd(&cnt[wave][ids[i]], 1);
  __syncthreads();
  if (tid == 0) {
    int32_t acc = 0;
    for (int e = 0; e < E; ++e) {
      counts[e] = cnt[0][e] + cnt[1][e] + cnt[2][e] + cnt[3][e];
      offsets[e] = acc;
      for (int r = 0; r < 4; ++r) {
        base[r][e] = acc;
        acc += cnt[r][e];
      }
    }
  }
  __syncthreads();
  for (int64_t g = r0; g < r1; g += 64) {
    const int64_t i = g + lane;
    const bool act = i < r1;
    const int x = act ? ids[i] : -1;
    uint64_t pending = __ballot(act);
    while (pending) {
      const int e0 = __shfl(x, __ffsll((long long)pending) - 1, 64);  // wave-uniform
      const uint64_t m = __ballot(x == e0) & pending;
      const int32_t b = base[wave][e0];
      if (x == e0) {
        const int32_t pos = b + __popcll(m & ((1ull << lane) - 1ull));
        list[pos] = (int32_t)(i / k);
        inv[i] = pos;
      }
      if (lane == 0) base[wave][e0] = b + __popcll(m);
      pending &= ~m;
    }
  }
}

// One block per token: x[t] += w y in slot order (each slot one expert).
__global__ void __launch_bounds__(256) k_pf_moe_combine(float* __restrict__ x, int64_t D, int k,
                                                        const float* __restrict__ w,
                                                        const int32_t* __restrict__ inv,
                                                        const float* __restrict__ y) {
  const int64_t t = blockIdx.x;
  float* xr = x + t * D;
  for (int64_t i = threadIdx.x; i < D; i += 256) {
    float v = xr[i];
    for (int q = 0; q < k; ++q) v = v + w[t * k + q] * y[(int64_t)inv[t * k + q] * D + i];
    xr[i] = v;
  }
}

}  // namespace

// ---- launchers ------------------------------------------------------------------------------

bool pf_supported(int type) {
  return type == T_Q4_0 || type == T_Q8_0 || type == T_Q4_K || type == T_Q6_K;
}

int64_t pf_mpad(int64_t m) { return (m + 63) / 64 * 64; }

hipError_t launch_pf_prep(float* x, int64_t ldx, int64_t M, const float* norm_w, float eps,
                          const PfAct& act, hipStream_t s, const float* part, int nsplit) {
  if (nsplit < 0 || (nsplit > 0 && !part)) return hipErrorInvalidValue;
  if (M <= 0 || M > act.mpad || act.K % 32 || act.mpad % 64 || ldx % 4) return hipErrorInvalidValue;
  const size_t lds = (size_t)act.K * 4;
  if ((int64_t)lds > lds_limit()) return hipErrorInvalidValue;
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_pf_prep),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  UAII_LAUNCH(k_pf_prep, dim3((unsigned)act.mpad), dim3(256), lds, s, x, ldx, M, norm_w, eps, act,
              part, nsplit);
  return hipGetLastError();
}

namespace {
template <int FMT, int EPI, int MT, int NT>
hipError_t pf_gemm_go(PfGemmArgs a, hipStream_t s) {
  const int per_tile = PF_WAVES * 16 * (EPI == EPI_SWIGLU ? NT / 2 : NT);
  int ntiles = 0;
  for (int k = 0; k < a.nseg; ++k) {
    a.seg[k].tile0 = ntiles;
    ntiles += (int)((a.seg[k].rows + per_tile - 1) / per_tile);
  }
  if (a.gtab && a.gbm != 16 * MT) return hipErrorInvalidValue;
  dim3 grid((unsigned)ntiles, (unsigned)(a.gtab ? a.ntab : a.mpad / (16 * MT)), (unsigned)a.ksplit);
  UAII_LAUNCH((k_pf_gemm<FMT, EPI, MT, NT>), grid, dim3(PF_WAVES * 64), 0, s, a);
  return hipGetLastError();
}

template <int FMT, int EPI, int MT>
hipError_t pf_gemm_dma_go(PfGemmArgs a, hipStream_t s) {
  constexpr int NT = dma_nt<FMT>();
  const int per_tile = PF_DW * 16 * (EPI == EPI_SWIGLU ? NT / 2 : NT);
  int ntiles = 0;
  for (int k = 0; k < a.nseg; ++k) {
    a.seg[k].tile0 = ntiles;
    ntiles += (int)((a.seg[k].rows + per_tile - 1) / per_tile);
  }
  if (a.gtab && a.gbm != 16 * MT) return hipErrorInvalidValue;
  dim3 grid((unsigned)ntiles, (unsigned)(a.gtab ? a.ntab : a.mpad / (16 * MT)), (unsigned)a.ksplit);
  if constexpr (FMT == T_Q4_0) {
    if (a.hi16) {
      UAII_LAUNCH((k_pf_gemm_dma<FMT, EPI, MT, NT, true>), grid, dim3(PF_DW * 64), 0, s, a);
      return hipGetLastError();
    }
  }
  UAII_LAUNCH((k_pf_gemm_dma<FMT, EPI, MT, NT, false>), grid, dim3(PF_DW * 64), 0, s, a);
  return hipGetLastError();
}

// Wave tile per launch: 64 x 32 (measured best at M = 512 for the 8B shapes,
// ahead of 64 x 64 and 32 x 32; for Q4_K 232 against 196 TFLOP/s on the 1B
// gate/up; for Q6_K 85 against 67 TFLOP/s on the 1B down with the former
// 16x16x16 decode) unless that leaves the grid under one block per CU; then
// 32 x 32.
template <int FMT, int EPI>
hipError_t pf_gemm_tile(const PfGemmArgs& a, hipStream_t s) {
  int64_t rows = 0;
  for (int k = 0; k < a.nseg; ++k) rows += a.seg[k].rows;
  if (EPI == EPI_SWIGLU) rows *= 2;
  const int64_t mid = (rows / 128) * (a.mpad / 64);
  constexpr bool wide = FMT == T_Q4_0 || FMT == T_Q8_0;
  const int want = UAII_PF_TILE;
  if (a.gtab) {  // expert groups: the tile height their table was built for
    if constexpr (wide) {
      if (UAII_PF_DMA) return pf_gemm_dma_go<FMT, EPI, 4>(a, s);
      return pf_gemm_go<FMT, EPI, 4, 2>(a, s);
    }
    if constexpr (FMT == T_Q4_K) {
      if (UAII_PF_KTILE) return pf_gemm_go<FMT, EPI, 4, 2>(a, s);
    }
    return pf_gemm_go<FMT, EPI, 2, 2>(a, s);
  }
  if constexpr (wide) {
    if (UAII_PF_DMA) {
      if (want == 2 || (want == 0 && mid >= 256)) return pf_gemm_dma_go<FMT, EPI, 4>(a, s);
      return pf_gemm_dma_go<FMT, EPI, 2>(a, s);
    }
    if (want == 2 || (want == 0 && mid >= 256)) return pf_gemm_go<FMT, EPI, 4, 2>(a, s);
  }
  if constexpr (FMT == T_Q4_K) {
    if (UAII_PF_KTILE && (want == 2 || (want == 0 && mid >= 256))) return pf_gemm_go<FMT, EPI, 4, 2>(a, s);
  }
  if constexpr (FMT == T_Q6_K) {
    if (UAII_PF_K6TILE && (want == 2 || (want == 0 && mid >= 256))) return pf_gemm_go<FMT, EPI, 4, 2>(a, s);
  }
  return pf_gemm_go<FMT, EPI, 2, 2>(a, s);
}

template <int FMT>
hipError_t pf_gemm_epi(const PfGemmArgs& a, hipStream_t s) {
  switch (a.epi) {
    case EPI_STORE: return pf_gemm_tile<FMT, EPI_STORE>(a, s);
    case EPI_ADD: return pf_gemm_tile<FMT, EPI_ADD>(a, s);
    case EPI_SWIGLU: return pf_gemm_tile<FMT, EPI_SWIGLU>(a, s);
    case EPI_GELU: return pf_gemm_tile<FMT, EPI_GELU>(a, s);
    default: return hipErrorInvalidValue;
  }
}
}  // namespace

// K split for a residual-add or plain-store launch: enough blocks for two per CU
// (each block's K range a whole number of stages and, for the K-quants,
// super-blocks).
int pf_gemm_ksplit(const PfGemmArgs& a, int cus) {
  if ((a.epi != EPI_ADD && a.epi != EPI_STORE) || a.nseg < 1) return 1;
  const int type = a.seg[0].w.type;
  if (!pf_supported(type)) return 1;
  int64_t rows = 0;
  for (int k = 0; k < a.nseg; ++k) rows += a.seg[k].rows;
  const bool wide = type == T_Q4_0 || type == T_Q8_0;
  const bool tall = wide || (type == T_Q4_K && UAII_PF_KTILE);  // formats with the 64 x 32 wave tile
  const int64_t mid = (rows / 128) * (a.mpad / 64);
  const bool big_tile = tall && (UAII_PF_TILE == 2 || (UAII_PF_TILE == 0 && mid >= 256));
  const int nw = (wide && UAII_PF_DMA) ? PF_DW : PF_WAVES;  // waves per block
  const int64_t tiles = (rows + nw * 32 - 1) / (nw * 32);     // 32 weight rows per wave
  const int64_t blocks = tiles * (a.mpad / (big_tile ? 64 : 32));
  const int64_t kq = wide ? 64 : 256;
  int ks = 1;
  const int64_t want = (int64_t)cus * UAII_PF_KS_BPC * PF_WAVES / nw;  // blocks (of PF_WAVES-wave units)
  while (ks < 4 && blocks * ks < want && a.K % (kq * ks * 2) == 0) ks *= 2;
  return ks;
}

int pf_gemm_group_rows(int type) {
  return (type == T_Q4_0 || type == T_Q8_0 || (type == T_Q4_K && UAII_PF_KTILE)) ? 64 : 32;
}

bool pf_hi16_supported(int type) { return type == T_Q4_0 && UAII_PF_DMA; }

hipError_t launch_pf_gemm(PfGemmArgs a, hipStream_t s) {
  if (a.ksplit < 1) a.ksplit = 1;
  if (a.sx_ld <= 0) a.sx_ld = a.mpad;
  if (!a.arow && !a.gtab && a.sx_ld != a.mpad) return hipErrorInvalidValue;
  if (a.nseg < 1 || a.nseg > 3 || a.M <= 0 || a.M > a.mpad || a.mpad % 64 || a.K % 64)
    return hipErrorInvalidValue;
  if (a.gtab) {
    // every table entry lies inside [0, M) and names an expert below ngroups (the
    // caller builds it on the host); here the launch itself is checked
    if (a.ntab < 1 || a.ngroups < 1 || a.ksplit != 1 || a.nseg != 1 ||
        a.gbm != pf_gemm_group_rows(a.seg[0].w.type) || (!a.arow && a.sx_ld < a.mpad))
      return hipErrorInvalidValue;
    const PfSeg& sg = a.seg[0];
    if (sg.rows * a.ngroups > sg.w.rows || (a.epi == EPI_SWIGLU && sg.rows * a.ngroups > sg.w2.rows))
      return hipErrorInvalidValue;
  }
  const int type = a.seg[0].w.type;
  if (!pf_supported(type)) return hipErrorInvalidValue;
  // the direct-to-LDS kernels (Q4_0, Q8_0) address activation rows by 32-bit
  // byte offsets: their activation arrays must span under 2^31 bytes
  if ((type == T_Q4_0 || type == T_Q8_0) && UAII_PF_DMA && a.sx_ld * a.K * 2 >= (int64_t(1) << 31))
    return hipErrorInvalidValue;
  if (a.hi16 && !pf_hi16_supported(type)) return hipErrorInvalidValue;
  const int64_t kq = (type == T_Q4_K || type == T_Q6_K) ? 256 : 64;  // K granule of a block's range
  if (a.K % (kq * a.ksplit)) return hipErrorInvalidValue;
  if (a.ksplit > 1 && ((a.epi != EPI_ADD && a.epi != EPI_STORE) || !a.part)) return hipErrorInvalidValue;
  for (int k = 0; k < a.nseg; ++k) {
    const PfSeg& sg = a.seg[k];
    if (sg.w.type != type || sg.w.cols != a.K || sg.rows <= 0 || sg.rows > sg.w.rows)
      return hipErrorInvalidValue;
    if (a.epi == EPI_SWIGLU &&
        (sg.w2.type != type || sg.w2.cols != a.K || sg.rows > sg.w2.rows))
      return hipErrorInvalidValue;
  }
  switch (type) {
    case T_Q4_0: return pf_gemm_epi<T_Q4_0>(a, s);
    case T_Q8_0: return pf_gemm_epi<T_Q8_0>(a, s);
    case T_Q4_K: return pf_gemm_epi<T_Q4_K>(a, s);
    case T_Q6_K: return pf_gemm_epi<T_Q6_K>(a, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_pf_qkv(const PfQkvArgs& a, hipStream_t s) {
  if (a.M <= 0 || a.head_dim <= 0 || a.head_dim % 2 || a.q_dim % a.head_dim ||
      a.kv_dim % a.head_dim || a.p0 < 0 || a.p0 + a.M > a.max_seq)
    return hipErrorInvalidValue;
  UAII_LAUNCH(k_pf_qkv, dim3((unsigned)a.M), dim3(256), 0, s, a);
  return hipGetLastError();
}

bool pf_attn_supported(int head_dim, int n_heads, int n_kv) {
  if (head_dim != 64 && head_dim != 128) return false;
  if (n_kv <= 0 || n_heads % n_kv) return false;
  const int G = n_heads / n_kv;
  const int GW = G < 4 ? G : 4;
  return G % GW == 0;
}

hipError_t launch_pf_attn(const PfAttnArgs& a, hipStream_t s) {
  if (a.M <= 0 || a.p0 < 0 || a.p0 + a.M > a.max_seq || !pf_attn_supported(a.hd, a.n_heads, a.n_kv) ||
      a.ldq % 4 || a.ldo % 4)
    return hipErrorInvalidValue;
  const int G = a.n_heads / a.n_kv;
  const int GW = G < 4 ? G : 4;
  const int QS = 4 / GW;
  const int QT = 16 * PA_QW * QS;  // queries per block
  dim3 grid((unsigned)((a.M + QT - 1) / QT), (unsigned)(a.n_kv * (G / GW)));
  if (a.hd == 64) UAII_LAUNCH(k_pf_attn<64>, grid, dim3(256), 0, s, a);
  else UAII_LAUNCH(k_pf_attn<128>, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

bool pf_router_supported(int type) { return type == T_F32 || type == T_F16; }

hipError_t launch_pf_moe_route(const float* x, int64_t M, int64_t K, const float* norm_w, float eps,
                               const DevWeight& router, int E, int k, int32_t* ids, float* w,
                               hipStream_t s) {
  if (M <= 0 || K % 4 || !norm_w || E < 1 || E > 256 || k < 1 || k > 8 || k > E ||
      router.rows < E || router.cols != K || !pf_router_supported(router.type))
    return hipErrorInvalidValue;
  if (M == 1) {
    // the decode step: the 16-wave kernel
    const int64_t P = (K / 4 + 511) / 512;
    const size_t lds1 = (size_t)(K + E * P) * 4;
    if ((int64_t)lds1 > lds_limit()) return hipErrorInvalidValue;
    const void* fn = router.type == T_F32 ? reinterpret_cast<const void*>(&k_moe_route_dec<T_F32>)
                                          : reinterpret_cast<const void*>(&k_moe_route_dec<T_F16>);
    if (lds1 > 64 * 1024) {
      const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds1);
      if (e != hipSuccess) return e;
    }
    if (router.type == T_F32)
      UAII_LAUNCH(k_moe_route_dec<T_F32>, dim3(1), dim3(1024), lds1, s, x, K, norm_w, eps, router, E, k, ids, w);
    else
      UAII_LAUNCH(k_moe_route_dec<T_F16>, dim3(1), dim3(1024), lds1, s, x, K, norm_w, eps, router, E, k, ids, w);
    return hipGetLastError();
  }
  const size_t lds = (size_t)K * 4;
  if ((int64_t)lds > lds_limit()) return hipErrorInvalidValue;
  if (router.type == T_F32) {
    if (lds > 64 * 1024) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_pf_moe_route<T_F32>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return e;
    }
    UAII_LAUNCH(k_pf_moe_route<T_F32>, dim3((unsigned)M), dim3(256), lds, s, x, K, norm_w, eps, router, E,
                k, ids, w);
  } else {
    if (lds > 64 * 1024) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_pf_moe_route<T_F16>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return e;
    }
    UAII_LAUNCH(k_pf_moe_route<T_F16>, dim3((unsigned)M), dim3(256), lds, s, x, K, norm_w, eps, router, E,
                k, ids, w);
  }
  return hipGetLastError();
}

hipError_t launch_pf_moe_lists(const int32_t* ids, int64_t M, int k, int E, int32_t* counts,
                               int32_t* offsets, int32_t* list, int32_t* inv, hipStream_t s) {
  if (M <= 0 || k < 1 || k > 8 || E < 1 || E > 256) return hipErrorInvalidValue;
  UAII_LAUNCH(k_pf_moe_lists, dim3(1), dim3(256), 0, s, ids, M, k, E, counts, offsets, list, inv);
  return hipGetLastError();
}

hipError_t launch_pf_moe_combine(float* x, int64_t M, int64_t D, int k, const float* w,
                                 const int32_t* inv, const float* y, hipStream_t s) {
  if (M <= 0 || D <= 0 || k < 1 || k > 8) return hipErrorInvalidValue;
  UAII_LAUNCH(k_pf_moe_combine, dim3((unsigned)M), dim3(256), 0, s, x, D, k, w, inv, y);
  return hipGetLastError();
}

}  // namespace uaii_hip
