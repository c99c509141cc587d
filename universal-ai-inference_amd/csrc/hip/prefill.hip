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
#include "common.h"
#include "uaii_hip_internal.h"

namespace uaii_hip {
namespace {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

__device__ inline h2_t as_h2(uint32_t u) { return __builtin_bit_cast(h2_t, u); }
// low nibbles of bytes 0 and 2 as f16 (1024 + q)
__device__ inline uint32_t nib_pair(uint32_t v) { return (v & 0x000F000Fu) | 0x64006400u; }
// bytes 0 and 2 as f16 (1024 + b)
__device__ inline uint32_t byte_pair(uint32_t v) { return (v & 0x00FF00FFu) | 0x64006400u; }

__device__ inline h8_t cat8(h2_t a, h2_t b, h2_t c, h2_t d) {
  return h8_t{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

__device__ inline f4_t mfma32(h8_t a, h8_t b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ inline f4_t mfma16(h4_t a, h4_t b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ inline float pow2f_i(int e) { return __uint_as_float((uint32_t)(e + 127) << 23); }

// ---- activation prep ----------------------------------------------------------------

// One block per row; rows >= M (tile padding) are written as zeros.
__global__ void __launch_bounds__(256) k_pf_prep(const float* __restrict__ x, int64_t ldx,
                                                 int64_t M, const float* __restrict__ norm_w,
                                                 float eps, PfAct act) {
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
  const float4* x4 = reinterpret_cast<const float4*>(x + t * ldx);
  float ss = 0.0f, amax = 0.0f;
  for (int i = tid; i < nv; i += 256) {
    const float4 v = x4[i];
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
      const _Float16 h0 = (_Float16)y0, h1 = (_Float16)y1, h2 = (_Float16)y2, h3 = (_Float16)y3;
      const _Float16 l0 = (_Float16)(y0 - (float)h0), l1 = (_Float16)(y1 - (float)h1);
      const _Float16 l2 = (_Float16)(y2 - (float)h2), l3 = (_Float16)(y3 - (float)h3);
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

// Raw bytes of one 32-weight block of one row for lane group g, loaded one stage
// ahead of their use; decode() turns them into MFMA B operands and scales.
template <int FMT>
struct PfRaw {
  uint2 q;        // Q4_0/Q8_0/Q4_K payload bytes; Q6_K: (ql word s=0, ql word s=1)
  uint2 h;        // Q6_K: (qh word s=0, qh word s=1)
  uint4 meta;     // Q4_K: d, dmin, scales[12]
  uint32_t d;     // Q4_0/Q8_0: f16 d; Q6_K: f16 d | (two int8 scales << 16)
};

template <int FMT>
struct PfFrag {
  h8_t b;         // K=32 formats
  h4_t b16[2];    // K=16 formats: sub-blocks 0 and 1
  float sc[2];
  float off;
};

template <int FMT>
__device__ constexpr int pf_ksub() {
  return FMT == T_Q6_K ? 16 : 32;
}
template <int FMT>
__device__ constexpr bool pf_offset() {
  return FMT == T_Q4_K;
}

// Row `row`, 32-block `kb`, lane group g (k = 8g..8g+7 of the block, or for
// 16-element sub-blocks k = 16s + 4g..4g+3).
template <int FMT>
__device__ inline void pf_load(const DevWeight& w, int64_t row, int64_t kb, int g, PfRaw<FMT>& r) {
  if constexpr (FMT == T_Q4_0) {
    r.q = *reinterpret_cast<const uint2*>(w.a + row * w.a_row + kb * 16 + 8 * (g & 1));
    r.d = ld_u16(w.b + row * w.b_row + kb * 2);
  } else if constexpr (FMT == T_Q8_0) {
    r.q = *reinterpret_cast<const uint2*>(w.a + row * w.a_row + kb * 32 + 8 * g);
    r.d = ld_u16(w.b + row * w.b_row + kb * 2);
  } else if constexpr (FMT == T_Q4_K) {
    const int64_t sb = kb >> 3;
    const int j = (int)(kb & 7);
    r.q = *reinterpret_cast<const uint2*>(w.a + row * w.a_row + sb * 128 + 32 * (j >> 1) + 8 * g);
    r.meta = *reinterpret_cast<const uint4*>(w.b + row * w.b_row + sb * 16);
  } else if constexpr (FMT == T_Q6_K) {
    const int64_t sb = kb >> 3;
    const int e0 = 32 * (int)(kb & 7);
    const int hh = e0 >> 7, e = e0 & 127;
    const uint8_t* ql = w.a + row * w.a_row + sb * 128 + 64 * hh + (e & 63) + 4 * g;
    const uint8_t* qh = w.b + row * w.b_row + sb * 64 + 32 * hh + 4 * g;
    r.q = make_uint2(*reinterpret_cast<const uint32_t*>(ql), *reinterpret_cast<const uint32_t*>(ql + 16));
    r.h = make_uint2(*reinterpret_cast<const uint32_t*>(qh), *reinterpret_cast<const uint32_t*>(qh + 16));
    const uint32_t sc2 = ld_u16(w.c + row * w.c_row + sb * 16 + 8 * hh + (e >> 4));
    r.d = ld_u16(w.d + row * w.d_row + sb * 2) | (sc2 << 16);
  }
}

template <int FMT>
__device__ inline void pf_decode(const PfRaw<FMT>& r, int64_t kb, int g, PfFrag<FMT>& f) {
  if constexpr (FMT == T_Q4_0) {
    const int sh = (g >> 1) * 4;
    const uint32_t v0 = r.q.x >> sh, v1 = r.q.y >> sh;
    const h2_t bias = {(_Float16)1032.0f, (_Float16)1032.0f};
    f.b = cat8(as_h2(nib_pair(v0)) - bias, as_h2(nib_pair(v0 >> 8)) - bias,
               as_h2(nib_pair(v1)) - bias, as_h2(nib_pair(v1 >> 8)) - bias);
    f.sc[0] = h2f((uint16_t)r.d);
  } else if constexpr (FMT == T_Q8_0) {
    const uint32_t v0 = r.q.x ^ 0x80808080u, v1 = r.q.y ^ 0x80808080u;
    const h2_t bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    f.b = cat8(as_h2(byte_pair(v0)) - bias, as_h2(byte_pair(v0 >> 8)) - bias,
               as_h2(byte_pair(v1)) - bias, as_h2(byte_pair(v1 >> 8)) - bias);
    f.sc[0] = h2f((uint16_t)r.d);
  } else if constexpr (FMT == T_Q4_K) {
    const int j = (int)(kb & 7);
    const int sh = (j & 1) * 4;
    const uint32_t v0 = r.q.x >> sh, v1 = r.q.y >> sh;
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
    const int e = (32 * (int)(kb & 7)) & 127;
    const int nib = (e >= 64) ? 4 : 0, qsh = 2 * (e >> 5);
    const h2_t bias = {(_Float16)1056.0f, (_Float16)1056.0f};
    const float d = h2f((uint16_t)(r.d & 0xffff));
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const uint32_t ql = s ? r.q.y : r.q.x, qh = s ? r.h.y : r.h.x;
      const uint32_t q6 = ((ql >> nib) & 0x0F0F0F0Fu) | (((qh >> qsh) & 0x03030303u) << 4);
      const h2_t p0 = as_h2(byte_pair(q6)) - bias, p1 = as_h2(byte_pair(q6 >> 8)) - bias;
      f.b16[s] = h4_t{p0.x, p0.y, p1.x, p1.y};
      f.sc[s] = fmul_rn(d, (float)(int8_t)((r.d >> (16 + 8 * s)) & 0xff));
    }
  }
}

// ---- GEMM -------------------------------------------------------------------------------

constexpr int PF_WAVES = 4;   // waves per block, side by side along N
constexpr int PF_NT = 4;      // 16-column subtiles per wave
constexpr int PF_KB = 2;      // 32-blocks of k per LDS stage
constexpr int PF_ROW = 40;    // halfs per staged 32-k row (32 + 8 pad: conflict-free reads)

template <int MT>
constexpr int pf_bm() { return 16 * MT; }

// LDS: [stage 2][kb PF_KB][hi/lo 2][BM rows][PF_ROW halfs]
template <int MT>
constexpr int pf_lds_halfs() { return 2 * PF_KB * 2 * pf_bm<MT>() * PF_ROW; }

template <int FMT, int EPI, int MT>
__global__ void __launch_bounds__(PF_WAVES * 64) k_pf_gemm(PfGemmArgs a) {
  constexpr int BM = pf_bm<MT>();
  constexpr int KS = pf_ksub<FMT>();
  constexpr bool OFF = pf_offset<FMT>();
  constexpr int NQ = (EPI == EPI_SWIGLU) ? PF_NT / 2 : PF_NT;  // distinct row subtiles
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
  const int64_t m0 = (int64_t)blockIdx.y * BM;
  const int64_t K = a.K, nkb = K / 32;

  // weight rows of this lane per subtile (clamped: rows past the end are loaded but not stored)
  int64_t wrow[PF_NT];
#pragma unroll
  for (int j = 0; j < PF_NT; ++j) {
    const int64_t r = n0 + 16 * (j % NQ) + col;
    wrow[j] = r < seg.rows ? r : seg.rows - 1;
  }
  auto wt = [&](int j) -> const DevWeight& { return (EPI == EPI_SWIGLU && j >= NQ) ? seg.w2 : seg.w; };

  f4_t acc[MT][PF_NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < PF_NT; ++j) acc[i][j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // activation stage copy: BM rows x PF_KB blocks x (hi, lo) x 4 pieces of 16 B
  constexpr int PIECES = BM * PF_KB * 2 * 4;
  constexpr int PPT = (PIECES + PF_WAVES * 64 - 1) / (PF_WAVES * 64);
  uint4 stg[PPT];
  auto load_stage = [&](int64_t kb0) {
#pragma unroll
    for (int u = 0; u < PPT; ++u) {
      const int c = threadIdx.x + u * PF_WAVES * 64;
      stg[u] = make_uint4(0, 0, 0, 0);
      if (c < PIECES) {
        const int q = c & 3, r = (c >> 2) % BM, kbh = (c >> 2) / BM;  // kbh = kb * 2 + h
        const int kb = kbh >> 1, h = kbh & 1;
        if (kb0 + kb < nkb) {
          const __half* src = (h ? a.alo : a.ahi) + (m0 + r) * K + (kb0 + kb) * 32 + q * 8;
          stg[u] = *reinterpret_cast<const uint4*>(src);
        }
      }
    }
  };
  auto store_stage = [&](int buf) {
#pragma unroll
    for (int u = 0; u < PPT; ++u) {
      const int c = threadIdx.x + u * PF_WAVES * 64;
      if (c < PIECES) {
        const int q = c & 3, r = (c >> 2) % BM, kbh = (c >> 2) / BM;
        _Float16* dst = lds + (((buf * PF_KB * 2) + kbh) * BM + r) * PF_ROW + q * 8;
        *reinterpret_cast<uint4*>(dst) = stg[u];
      }
    }
  };

  // weight bytes: rc for the stage being computed, rn for the next one (register
  // arrays are only ever indexed by compile-time constants)
  PfRaw<FMT> rc[PF_KB][PF_NT], rn[PF_KB][PF_NT];
  auto load_w = [&](PfRaw<FMT> (&dst)[PF_KB][PF_NT], int64_t kb0) {
#pragma unroll
    for (int kb = 0; kb < PF_KB; ++kb) {
      const int64_t b = (kb0 + kb < nkb) ? kb0 + kb : nkb - 1;
#pragma unroll
      for (int j = 0; j < PF_NT; ++j) pf_load<FMT>(wt(j), wrow[j], b, g, dst[kb][j]);
    }
  };

  const int64_t nst = (nkb + PF_KB - 1) / PF_KB;
  load_stage(0);
  load_w(rc, 0);
  store_stage(0);
  __syncthreads();

  for (int64_t st = 0; st < nst; ++st) {
    const int cur = (int)(st & 1);
    if (st + 1 < nst) {
      load_stage((st + 1) * PF_KB);
      load_w(rn, (st + 1) * PF_KB);
    }
#pragma unroll
    for (int kb = 0; kb < PF_KB; ++kb) {
      const int64_t kbg = st * PF_KB + kb;
      if (kbg < nkb) {
        PfFrag<FMT> fr[PF_NT];
#pragma unroll
        for (int j = 0; j < PF_NT; ++j) pf_decode<FMT>(rc[kb][j], kbg, g, fr[j]);
        const _Float16* base = lds + ((cur * PF_KB + kb) * 2) * BM * PF_ROW;
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          const _Float16* ph = base + (16 * i + col) * PF_ROW;
          const _Float16* pl = ph + BM * PF_ROW;
          f4_t sxv = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
          if constexpr (OFF) {
            const float4 s4 = *reinterpret_cast<const float4*>(a.sx + kbg * a.mpad + m0 + 16 * i + 4 * g);
            sxv = f4_t{s4.x, s4.y, s4.z, s4.w};
          }
          if constexpr (KS == 32) {
            const h8_t ahi = *reinterpret_cast<const h8_t*>(ph + 8 * g);
            const h8_t alo = *reinterpret_cast<const h8_t*>(pl + 8 * g);
#pragma unroll
            for (int j = 0; j < PF_NT; ++j) {
              f4_t p = mfma32(ahi, fr[j].b, f4_t{0.0f, 0.0f, 0.0f, 0.0f});
              p = mfma32(alo, fr[j].b, p);
              acc[i][j] += fr[j].sc[0] * p;
              if constexpr (OFF) acc[i][j] -= fr[j].off * sxv;
            }
          } else {
#pragma unroll
            for (int s = 0; s < 2; ++s) {
              const h4_t ahi = *reinterpret_cast<const h4_t*>(ph + 16 * s + 4 * g);
              const h4_t alo = *reinterpret_cast<const h4_t*>(pl + 16 * s + 4 * g);
#pragma unroll
              for (int j = 0; j < PF_NT; ++j) {
                f4_t p = mfma16(ahi, fr[j].b16[s], f4_t{0.0f, 0.0f, 0.0f, 0.0f});
                p = mfma16(alo, fr[j].b16[s], p);
                acc[i][j] += fr[j].sc[s] * p;
              }
            }
          }
        }
      }
    }
    if (st + 1 < nst) {
      store_stage(cur ^ 1);
#pragma unroll
      for (int kb = 0; kb < PF_KB; ++kb)
#pragma unroll
        for (int j = 0; j < PF_NT; ++j) rc[kb][j] = rn[kb][j];
      __syncthreads();
    }
  }

  // epilogue: lane holds rows m0 + 16i + 4g + r of column n0 + 16j + col
#pragma unroll
  for (int i = 0; i < MT; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t t = m0 + 16 * i + 4 * g + r;
      if (t >= a.M) continue;
      const float rs = a.rs[t];
      float* yrow = a.y + t * a.ldy + seg.col0;
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        const int64_t n = n0 + 16 * j + col;
        if (n >= seg.rows) continue;
        const float v = acc[i][j][r] * rs;
        if constexpr (EPI == EPI_STORE) {
          yrow[n] = v;
        } else if constexpr (EPI == EPI_ADD) {
          yrow[n] = yrow[n] + v;
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
  const int hd = a.head_dim, half = hd / 2;
  const int npair = (a.q_dim + a.kv_dim) / 2;
  for (int u = threadIdx.x; u < npair; u += blockDim.x) {
    const bool isq = u < a.q_dim / 2;
    const int uu = isq ? u : u - a.q_dim / 2;
    const int head = uu / half, p = uu % half;
    const int r0 = head * hd + (a.rope_mode == 2 ? p : 2 * p);
    const int r1 = r0 + (a.rope_mode == 2 ? half : 1);
    const int base = isq ? 0 : a.q_dim;
    float v0 = row[base + r0], v1 = row[base + r1];
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
    float v = row[a.q_dim + a.kv_dim + r];
    if (a.bv) v = v + a.bv[r];
    const int64_t o = ((int64_t)(r / hd) * a.max_seq + pos) * hd + (r % hd);
    if (a.kv_f16) reinterpret_cast<__half*>(a.vcache)[o] = __float2half(v);
    else reinterpret_cast<float*>(a.vcache)[o] = v;
  }
}

// ---- causal attention over the f16 cache ---------------------------------------------------

constexpr int PA_TK = 64;  // keys per LDS tile

// Block: 4 waves on kv head blockIdx.y / (G / GW); wave w takes q head
// (w % GW) of the block's GW heads and query subtile w / GW (16 queries each).
template <int HD>
__global__ void __launch_bounds__(256) k_pf_attn(PfAttnArgs a) {
  constexpr int KP = HD + 8;        // K tile row (halfs)
  constexpr int VP = PA_TK + 8;     // V^T tile row (halfs)
  constexpr int NC = HD / 32;       // 32-wide hd chunks (S)
  constexpr int ND = HD / 16;       // 16-row hd subtiles (O)
  __shared__ _Float16 ks[PA_TK * KP];
  __shared__ _Float16 vt[HD * VP];

  const int G = a.n_heads / a.n_kv;
  const int GW = G < 4 ? G : 4;
  const int QS = 4 / GW;
  const int hb = blockIdx.y;                 // head block
  const int kvh = hb / (G / GW);
  const int hbase = kvh * G + (hb % (G / GW)) * GW;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, col = lane & 15, g = lane >> 4;
  const bool active = wave < GW * QS;
  const int head = hbase + (wave % GW);
  const int64_t q0 = (int64_t)blockIdx.x * (16 * QS);
  const int64_t qrow = q0 + 16 * (wave / GW) + col;  // this lane's query (column)
  const bool qvalid = active && qrow < a.M;
  const int64_t qpos = a.p0 + qrow;
  const int64_t qend = min((int64_t)a.M, q0 + 16 * QS);
  const int64_t nkeys = a.p0 + qend;  // keys the block needs (causal)

  // q * scale * 2^e as f16 hi + lo, natural hd order: lane (query col, group g)
  // holds hd 32c + 8g .. +7 of chunk c. The matrix cores flush f16 subnormals,
  // so each query row is scaled to put its largest element in [2^14, 2^15)
  // (lo stays normal) and the scores are scaled back by 2^-e.
  const float scale = 1.0f / sqrtf((float)HD);
  float qv[NC][8];
  float qmax = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    if (qvalid) {
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
  const float qs = pow2f_i(qe), qrs = pow2f_i(-qe);
  h8_t qhi[NC], qlo[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float s = qv[c][k] * qs;
      const _Float16 h = (_Float16)s;
      qhi[c][k] = h;
      qlo[c][k] = (_Float16)(s - (float)h);
    }
  }

  f4_t o[ND];
#pragma unroll
  for (int d = 0; d < ND; ++d) o[d] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
  float mrun = -INFINITY, lrun = 0.0f;

  const __half* kbase = reinterpret_cast<const __half*>(a.kcache) + (int64_t)kvh * a.max_seq * HD;
  const __half* vbase = reinterpret_cast<const __half*>(a.vcache) + (int64_t)kvh * a.max_seq * HD;

  for (int64_t kt = 0; kt < nkeys; kt += PA_TK) {
    // stage K rows and V transposed (keys past nkeys read as zeros)
    __syncthreads();
    for (int c = threadIdx.x; c < PA_TK * (HD / 8); c += 256) {
      const int key = c / (HD / 8), p = c % (HD / 8);
      uint4 kv = make_uint4(0, 0, 0, 0), vv = make_uint4(0, 0, 0, 0);
      if (kt + key < nkeys) {
        kv = *reinterpret_cast<const uint4*>(kbase + (kt + key) * HD + 8 * p);
        vv = *reinterpret_cast<const uint4*>(vbase + (kt + key) * HD + 8 * p);
      }
      *reinterpret_cast<uint4*>(ks + key * KP + 8 * p) = kv;
      const _Float16* ve = reinterpret_cast<const _Float16*>(&vv);
#pragma unroll
      for (int e = 0; e < 8; ++e) vt[(8 * p + e) * VP + key] = ve[e];
    }
    __syncthreads();
    if (!active) continue;

    // S^T for 4 key subtiles: lane holds keys kt + 16s + 4g + r of query col
    f4_t sc[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      f4_t acc = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const h8_t kf = *reinterpret_cast<const h8_t*>(ks + (16 * s + col) * KP + 32 * c + 8 * g);
        acc = mfma32(kf, qhi[c], acc);
        acc = mfma32(kf, qlo[c], acc);
      }
      sc[s] = acc * qrs;
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t key = kt + 16 * s + 4 * g + r;
        if (!qvalid || key > qpos) sc[s][r] = -INFINITY;
        tmax = fmaxf(tmax, sc[s][r]);
      }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float mnew = fmaxf(mrun, tmax);
    const float alpha = (mrun == -INFINITY) ? 0.0f : expf(mrun - mnew);
    float psum = 0.0f;
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = (sc[s][r] == -INFINITY) ? 0.0f : expf(sc[s][r] - mnew);
        sc[s][r] = p;
        psum += p;
      }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    lrun = lrun * alpha + psum;
    mrun = mnew;
#pragma unroll
    for (int d = 0; d < ND; ++d) o[d] *= alpha;

    // O^T += V^T . (2^14 P)^T over two 32-key chunks (p <= 1, so 2^14 p keeps
    // hi and lo normal); lane's keys: 32c + 4g + r (r < 4) and 32c + 16 + 4g + (r - 4)
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
        const _Float16* vr = vt + (16 * d + col) * VP + 32 * c + 4 * g;
        const h4_t v0 = *reinterpret_cast<const h4_t*>(vr);
        const h4_t v1 = *reinterpret_cast<const h4_t*>(vr + 16);
        const h8_t vf = h8_t{v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        o[d] = mfma32(vf, phi, o[d]);
        o[d] = mfma32(vf, plo, o[d]);
      }
    }
  }
  if (!qvalid) return;
  const float inv = (1.0f / 16384.0f) / lrun;
  float* out = a.out + qrow * a.ldo + (int64_t)head * HD;
#pragma unroll
  for (int d = 0; d < ND; ++d) {
    float4 v = make_float4(o[d][0] * inv, o[d][1] * inv, o[d][2] * inv, o[d][3] * inv);
    *reinterpret_cast<float4*>(out + 16 * d + 4 * g) = v;
  }
}

}  // namespace

// ---- launchers ------------------------------------------------------------------------------

bool pf_supported(int type) {
  return type == T_Q4_0 || type == T_Q8_0 || type == T_Q4_K || type == T_Q6_K;
}

int64_t pf_mpad(int64_t m) { return (m + 63) / 64 * 64; }

hipError_t launch_pf_prep(const float* x, int64_t ldx, int64_t M, const float* norm_w, float eps,
                          const PfAct& act, hipStream_t s) {
  if (M <= 0 || M > act.mpad || act.K % 32 || act.mpad % 64 || ldx % 4) return hipErrorInvalidValue;
  const size_t lds = (size_t)act.K * 4;
  if ((int64_t)lds > lds_limit()) return hipErrorInvalidValue;
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_pf_prep),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  UAII_LAUNCH(k_pf_prep, dim3((unsigned)act.mpad), dim3(256), lds, s, x, ldx, M, norm_w, eps, act);
  return hipGetLastError();
}

namespace {
template <int FMT, int EPI, int MT>
hipError_t pf_gemm_go(const PfGemmArgs& a, int ntiles, hipStream_t s) {
  dim3 grid((unsigned)ntiles, (unsigned)(a.mpad / pf_bm<MT>()));
  UAII_LAUNCH((k_pf_gemm<FMT, EPI, MT>), grid, dim3(PF_WAVES * 64), 0, s, a);
  return hipGetLastError();
}

template <int FMT, int MT>
hipError_t pf_gemm_epi(const PfGemmArgs& a, int ntiles, hipStream_t s) {
  switch (a.epi) {
    case EPI_STORE: return pf_gemm_go<FMT, EPI_STORE, MT>(a, ntiles, s);
    case EPI_ADD: return pf_gemm_go<FMT, EPI_ADD, MT>(a, ntiles, s);
    case EPI_SWIGLU: return pf_gemm_go<FMT, EPI_SWIGLU, MT>(a, ntiles, s);
    case EPI_GELU: return pf_gemm_go<FMT, EPI_GELU, MT>(a, ntiles, s);
    default: return hipErrorInvalidValue;
  }
}
}  // namespace

hipError_t launch_pf_gemm(PfGemmArgs a, hipStream_t s) {
  if (a.nseg < 1 || a.nseg > 3 || a.M <= 0 || a.M > a.mpad || a.mpad % 64 || a.K % 32)
    return hipErrorInvalidValue;
  const int type = a.seg[0].w.type;
  if (!pf_supported(type)) return hipErrorInvalidValue;
  if (type == T_Q4_K || type == T_Q6_K) {
    if (a.K % 256) return hipErrorInvalidValue;
  }
  const int per_tile = PF_WAVES * 16 * (a.epi == EPI_SWIGLU ? PF_NT / 2 : PF_NT);
  int ntiles = 0;
  for (int k = 0; k < a.nseg; ++k) {
    const PfSeg& sg = a.seg[k];
    if (sg.w.type != type || sg.w.cols != a.K || sg.rows <= 0 || sg.rows > sg.w.rows)
      return hipErrorInvalidValue;
    if (a.epi == EPI_SWIGLU &&
        (sg.w2.type != type || sg.w2.cols != a.K || sg.rows > sg.w2.rows))
      return hipErrorInvalidValue;
    a.seg[k].tile0 = ntiles;
    ntiles += (int)((sg.rows + per_tile - 1) / per_tile);
  }
  // 32-row tiles when 64-row tiles leave most of the chip idle
  const bool small = (int64_t)ntiles * (a.mpad / 64) < 512;
  switch (type) {
    case T_Q4_0: return small ? pf_gemm_epi<T_Q4_0, 2>(a, ntiles, s) : pf_gemm_epi<T_Q4_0, 4>(a, ntiles, s);
    case T_Q8_0: return small ? pf_gemm_epi<T_Q8_0, 2>(a, ntiles, s) : pf_gemm_epi<T_Q8_0, 4>(a, ntiles, s);
    case T_Q4_K: return small ? pf_gemm_epi<T_Q4_K, 2>(a, ntiles, s) : pf_gemm_epi<T_Q4_K, 4>(a, ntiles, s);
    case T_Q6_K: return small ? pf_gemm_epi<T_Q6_K, 2>(a, ntiles, s) : pf_gemm_epi<T_Q6_K, 4>(a, ntiles, s);
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
  dim3 grid((unsigned)((a.M + 16 * QS - 1) / (16 * QS)), (unsigned)(a.n_kv * (G / GW)));
  if (a.hd == 64) UAII_LAUNCH(k_pf_attn<64>, grid, dim3(256), 0, s, a);
  else UAII_LAUNCH(k_pf_attn<128>, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace uaii_hip
