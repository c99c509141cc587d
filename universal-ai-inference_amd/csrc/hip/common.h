// common.h — shared device-side definitions for the gfx950 token-loop kernels.
//
// Weights live in HBM in a "split" layout built once at load time from the GGUF
// bytes (repack.hip): per tensor, the quantized payload of every row is stored
// as one contiguous byte array (16-byte chunks, so a wave's 64 lanes read 1 KiB
// with one fully coalesced global_load_dwordx4), and the per-block scales sit in
// separate small arrays. The bytes per weight are unchanged (Q3_K pads its 12
// scale bytes + d to 16 bytes); the decoded values are bit-identical to the
// reference decoder (libs/uaii-quant/src/gguf_dequant.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <hip/hip_ext.h>

namespace uaii_hip {
// Per-thread event pair for kernel timing: while `stop` is set, UAII_LAUNCH
// launches through hipExtLaunchKernelGGL so the events are recorded on the
// kernel's own dispatch (start on the first kernel after it is set, stop on
// every one, so a group of launches is timed as a whole). Unset: plain launches.
struct LaunchEvents {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};
extern thread_local LaunchEvents g_launch_events;
}  // namespace uaii_hip

#define UAII_LAUNCH(K, G, B, LDS, S, ...)                                                      \
  do {                                                                                     \
    if (::uaii_hip::g_launch_events.stop) {                                                \
      hipExtLaunchKernelGGL(K, G, B, LDS, S, ::uaii_hip::g_launch_events.start,            \
                            ::uaii_hip::g_launch_events.stop, 0, __VA_ARGS__);             \
      ::uaii_hip::g_launch_events.start = nullptr;                                         \
    } else {                                                                               \
      hipLaunchKernelGGL(K, G, B, LDS, S, __VA_ARGS__);                                    \
    }                                                                                      \
  } while (0)

namespace uaii_hip {

// GGUF type ids (include/uaii/loaders/gguf.hpp:18-36).
enum : int {
  T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q4_1 = 3, T_Q5_0 = 6, T_Q5_1 = 7, T_Q8_0 = 8,
  T_Q2_K = 10, T_Q3_K = 11, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14
};

// Per-block LDS the current device allows (queried once; 64 KiB if unknown).
inline int lds_limit() {
  static int lim = 0;
  if (lim == 0) {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess &&
        v > 0) {
      lim = v;
    } else {
      lim = 64 * 1024;
    }
  }
  return lim;
}

// Device view of one split-layout weight [rows, cols]. `a` is the 16-byte
// chunked payload, `b`/`c`/`d` side arrays (format specific, see repack.hip).
struct DevWeight {
  int type;
  int64_t rows, cols;
  const uint8_t* a;  // payload, rows * a_row bytes
  const uint8_t* b;
  const uint8_t* c;
  const uint8_t* d;
  int64_t a_row, b_row, c_row, d_row;  // bytes per row of each array
};

// Chunks of 16 payload bytes per row; each chunk decodes to `chunk_elems` values.
__host__ __device__ inline int chunk_elems(int t) {
  switch (t) {
    case T_Q8_0: return 16;
    case T_F32: return 4;
    case T_F16: return 8;
    case T_Q2_K: case T_Q3_K: return 64;
    default: return 32;  // Q4_0 Q4_1 Q5_0 Q5_1 Q4_K Q5_K Q6_K
  }
}

__host__ __device__ inline int block_elems(int t) {
  switch (t) {
    case T_F32: case T_F16: return 1;
    case T_Q4_0: case T_Q4_1: case T_Q5_0: case T_Q5_1: case T_Q8_0: return 32;
    case T_Q2_K: case T_Q3_K: case T_Q4_K: case T_Q5_K: case T_Q6_K: return 256;
    default: return 0;
  }
}

__host__ __device__ inline int block_bytes(int t) {
  switch (t) {
    case T_F32: return 4; case T_F16: return 2; case T_Q4_0: return 18; case T_Q4_1: return 20;
    case T_Q5_0: return 22; case T_Q5_1: return 24; case T_Q8_0: return 34; case T_Q2_K: return 84;
    case T_Q3_K: return 110; case T_Q4_K: return 144; case T_Q5_K: return 176; case T_Q6_K: return 210;
    default: return 0;
  }
}

__device__ inline float h2f(uint16_t h) {
  // v_cvt_f32_f16 is an exact conversion (subnormals included).
  return __half2float(__ushort_as_half(h));
}

__device__ inline uint16_t ld_u16(const uint8_t* p) {
  return *reinterpret_cast<const uint16_t*>(p);
}

// Invoke f.template operator()<T>() for the runtime GGUF type `type`.
#define UAII_FOR_TYPE(type, BODY)                      \
  switch (type) {                                      \
    case T_F32: { constexpr int FT = T_F32; BODY; } break;   \
    case T_F16: { constexpr int FT = T_F16; BODY; } break;   \
    case T_Q4_0: { constexpr int FT = T_Q4_0; BODY; } break; \
    case T_Q4_1: { constexpr int FT = T_Q4_1; BODY; } break; \
    case T_Q5_0: { constexpr int FT = T_Q5_0; BODY; } break; \
    case T_Q5_1: { constexpr int FT = T_Q5_1; BODY; } break; \
    case T_Q8_0: { constexpr int FT = T_Q8_0; BODY; } break; \
    case T_Q2_K: { constexpr int FT = T_Q2_K; BODY; } break; \
    case T_Q3_K: { constexpr int FT = T_Q3_K; BODY; } break; \
    case T_Q4_K: { constexpr int FT = T_Q4_K; BODY; } break; \
    case T_Q5_K: { constexpr int FT = T_Q5_K; BODY; } break; \
    case T_Q6_K: { constexpr int FT = T_Q6_K; BODY; } break; \
    default: break;                                    \
  }

// Exact-rounding helpers: the reference evaluates dequant products and
// differences as separate f32 operations; these keep the compiler from fusing
// them into an FMA where bit-exactness is required.
__device__ inline float fmul_rn(float a, float b) { return __fmul_rn(a, b); }
__device__ inline float fsub_rn(float a, float b) { return __fsub_rn(a, b); }
__device__ inline float fadd_rn(float a, float b) { return __fadd_rn(a, b); }

// Full 64-lane sum; every lane returns the total.
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ inline float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Wave reductions on DPP moves instead of LDS permutes: within each 16-lane row
// xor 1 and xor 2 (quad_perm), then the half-row and row mirrors; across the 4
// rows with readlane (the result is wave-uniform). Call them with all
// 64 lanes active: readlane reads its lane whatever the exec mask holds.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_val(float v, int k) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), k));
}
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_mov<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_mov<0x141>(v));  // row_half_mirror
  v = fmaxf(v, dpp_mov<0x140>(v));  // row_mirror
  return fmaxf(fmaxf(lane_val(v, 0), lane_val(v, 16)), fmaxf(lane_val(v, 32), lane_val(v, 48)));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_mov<0xB1>(v);
  v += dpp_mov<0x4E>(v);
  v += dpp_mov<0x141>(v);
  v += dpp_mov<0x140>(v);
  return (lane_val(v, 0) + lane_val(v, 16)) + (lane_val(v, 32) + lane_val(v, 48));
}

// 6-bit (scale, min) pair j of the K-quant 12-byte field (gguf_dequant.cpp:107-115).
__device__ inline void kscale(int j, const uint8_t* s, int& sc, int& mn) {
  if (j < 4) {
    sc = s[j] & 63;
    mn = s[j + 4] & 63;
  } else {
    sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
    mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
}

// Decode chunk `t` of row `r` into 32 (or chunk_elems) values `v` with the element
// indices (within the row) written to `idx`. Bit-exact with the reference
// decoder. Used by the dequant kernels and the embedding gather; the GEMV
// kernels use algebraically regrouped forms of the same decode.
struct ChunkOut {
  float v[64];
  int idx[64];
  int n;
};

// FMT is the weight type as a template constant so every loop bound and array
// index folds to a constant (no scratch spills).
template <int FMT>
__device__ inline void decode_chunk(const DevWeight& w, int64_t r, int64_t t, ChunkOut& o) {
  const uint8_t* a = w.a + r * w.a_row + t * 16;
  uint8_t q[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) q[i] = a[i];
  switch (FMT) {
    case T_F32: {
      const float* f = reinterpret_cast<const float*>(q);
      for (int i = 0; i < 4; ++i) { o.v[i] = f[i]; o.idx[i] = (int)(4 * t + i); }
      o.n = 4;
      break;
    }
    case T_F16: {
      for (int i = 0; i < 8; ++i) {
        o.v[i] = h2f((uint16_t)(q[2 * i] | (q[2 * i + 1] << 8)));
        o.idx[i] = (int)(8 * t + i);
      }
      o.n = 8;
      break;
    }
    case T_Q4_0: {  // b: f16 d per block
      const float d = h2f(ld_u16(w.b + r * w.b_row + t * 2));
      for (int j = 0; j < 16; ++j) {
        o.v[j] = fmul_rn((float)((q[j] & 15) - 8), d);
        o.v[j + 16] = fmul_rn((float)((q[j] >> 4) - 8), d);
        o.idx[j] = (int)(32 * t + j);
        o.idx[j + 16] = (int)(32 * t + j + 16);
      }
      o.n = 32;
      break;
    }
    case T_Q4_1: {  // b: (d, m) f16 pair per block
      const uint8_t* dm = w.b + r * w.b_row + t * 4;
      const float d = h2f(ld_u16(dm)), m = h2f(ld_u16(dm + 2));
      for (int j = 0; j < 16; ++j) {
        o.v[j] = fadd_rn(fmul_rn((float)(q[j] & 15), d), m);
        o.v[j + 16] = fadd_rn(fmul_rn((float)(q[j] >> 4), d), m);
        o.idx[j] = (int)(32 * t + j);
        o.idx[j + 16] = (int)(32 * t + j + 16);
      }
      o.n = 32;
      break;
    }
    case T_Q5_0:
    case T_Q5_1: {  // b: 4-byte high bits per block, c: d (Q5_0) or (d, m) (Q5_1)
      const uint32_t hb = *reinterpret_cast<const uint32_t*>(w.b + r * w.b_row + t * 4);
      const bool one = FMT == T_Q5_1;
      const uint8_t* dm = w.c + r * w.c_row + t * (one ? 4 : 2);
      const float d = h2f(ld_u16(dm));
      const float m = one ? h2f(ld_u16(dm + 2)) : 0.0f;
      for (int j = 0; j < 16; ++j) {
        const int lo = (q[j] & 15) | (int)(((hb >> j) & 1u) << 4);
        const int hi = (q[j] >> 4) | (int)(((hb >> (j + 16)) & 1u) << 4);
        if (one) {
          o.v[j] = fadd_rn(fmul_rn((float)lo, d), m);
          o.v[j + 16] = fadd_rn(fmul_rn((float)hi, d), m);
        } else {
          o.v[j] = fmul_rn((float)(lo - 16), d);
          o.v[j + 16] = fmul_rn((float)(hi - 16), d);
        }
        o.idx[j] = (int)(32 * t + j);
        o.idx[j + 16] = (int)(32 * t + j + 16);
      }
      o.n = 32;
      break;
    }
    case T_Q8_0: {  // chunk = half block; b: f16 d per block
      const float d = h2f(ld_u16(w.b + r * w.b_row + (t / 2) * 2));
      for (int j = 0; j < 16; ++j) {
        o.v[j] = fmul_rn((float)(int8_t)q[j], d);
        o.idx[j] = (int)(16 * t + j);
      }
      o.n = 16;
      break;
    }
    case T_Q4_K:
    case T_Q5_K: {  // b: 16-byte meta (d, dmin, scales[12]) per super-block;
                    // Q5_K c: 32-byte qh per super-block
      const int64_t sb = t / 8;
      const int tt = (int)(t % 8), cc = tt / 2, hh = tt % 2;
      const uint8_t* meta = w.b + r * w.b_row + sb * 16;
      const float d = h2f(ld_u16(meta)), dmin = h2f(ld_u16(meta + 2));
      int sc, mn;
      kscale(2 * cc, meta + 4, sc, mn);
      const float d1 = fmul_rn(d, (float)sc), m1 = fmul_rn(dmin, (float)mn);
      kscale(2 * cc + 1, meta + 4, sc, mn);
      const float d2 = fmul_rn(d, (float)sc), m2 = fmul_rn(dmin, (float)mn);
      const uint8_t* qh = (FMT == T_Q5_K) ? w.c + r * w.c_row + sb * 32 : nullptr;
      for (int i = 0; i < 16; ++i) {
        const int l = 16 * hh + i;
        int lo = q[i] & 15, hi = q[i] >> 4;
        if (qh) {
          lo += 16 * ((qh[l] >> (2 * cc)) & 1);
          hi += 16 * ((qh[l] >> (2 * cc + 1)) & 1);
        }
        o.v[i] = fsub_rn(fmul_rn(d1, (float)lo), m1);
        o.v[i + 16] = fsub_rn(fmul_rn(d2, (float)hi), m2);
        o.idx[i] = (int)(256 * sb + 64 * cc + l);
        o.idx[i + 16] = (int)(256 * sb + 64 * cc + 32 + l);
      }
      o.n = 32;
      break;
    }
    case T_Q6_K: {  // b: qh (64 B / sb), c: int8 scales (16 / sb), d: f16 d (per sb)
      const int64_t sb = t / 8;
      const int h = (int)((t % 8) / 4), u = (int)(t % 4);
      const uint8_t* qh = w.b + r * w.b_row + sb * 64 + h * 32 + 16 * (u % 2);
      const int8_t* sc = reinterpret_cast<const int8_t*>(w.c + r * w.c_row + sb * 16 + h * 8);
      const float d = h2f(ld_u16(w.d + r * w.d_row + sb * 2));
      const int sh = 2 * (u / 2);
      const float s_lo = fmul_rn(d, (float)sc[u]), s_hi = fmul_rn(d, (float)sc[u + 4]);
      for (int i = 0; i < 16; ++i) {
        const int lo = (q[i] & 15) | (((qh[i] >> sh) & 3) << 4);
        const int hi = (q[i] >> 4) | (((qh[i] >> (sh + 4)) & 3) << 4);
        o.v[i] = fmul_rn(s_lo, (float)(lo - 32));
        o.v[i + 16] = fmul_rn(s_hi, (float)(hi - 32));
        o.idx[i] = (int)(256 * sb + 128 * h + 16 * u + i);
        o.idx[i + 16] = (int)(256 * sb + 128 * h + 64 + 16 * u + i);
      }
      o.n = 32;
      break;
    }
    case T_Q2_K:
    case T_Q3_K: {
      // chunk = 16 payload bytes of one 128-half group g (4 bit-planes x 16 lanes)
      // -> 64 values. Q2_K b: scales (16 B / sb), c: (d, dmin) (4 B / sb).
      // Q3_K b: hmask (32 B / sb), c: meta 16 B (scales[12], d, pad).
      const int64_t sb = t / 4;
      const int h = (int)((t % 4) / 2), g = (int)(t % 2);
      if (FMT == T_Q2_K) {
        const uint8_t* scl = w.b + r * w.b_row + sb * 16;
        const uint8_t* dd = w.c + r * w.c_row + sb * 4;
        const float d = h2f(ld_u16(dd)), dmin = h2f(ld_u16(dd + 2));
        for (int p = 0; p < 4; ++p) {
          const int s = scl[8 * h + 2 * p + g];
          const float dl = fmul_rn(d, (float)(s & 15)), ml = fmul_rn(dmin, (float)(s >> 4));
          for (int l = 0; l < 16; ++l) {
            o.v[16 * p + l] = fsub_rn(fmul_rn(dl, (float)((q[l] >> (2 * p)) & 3)), ml);
            o.idx[16 * p + l] = (int)(256 * sb + 128 * h + 32 * p + 16 * g + l);
          }
        }
      } else {
        const uint8_t* hm = w.b + r * w.b_row + sb * 32 + 16 * g;
        const uint8_t* meta = w.c + r * w.c_row + sb * 16;
        const float dall = h2f(ld_u16(meta + 12));
        for (int p = 0; p < 4; ++p) {
          const int j = 8 * h + 2 * p + g;
          const int lo4 = (j < 8) ? (meta[j] & 15) : (meta[j - 8] >> 4);
          const int hi2 = (meta[8 + (j % 4)] >> (2 * (j / 4))) & 3;
          const float dl = fmul_rn(dall, (float)((lo4 | (hi2 << 4)) - 32));
          const int mbit = 1 << (4 * h + p);
          for (int l = 0; l < 16; ++l) {
            const int qq = (q[l] >> (2 * p)) & 3;
            const int sub = (hm[l] & mbit) ? 0 : 4;
            o.v[16 * p + l] = fmul_rn(dl, (float)(qq - sub));
            o.idx[16 * p + l] = (int)(256 * sb + 128 * h + 32 * p + 16 * g + l);
          }
        }
      }
      o.n = 64;
      break;
    }
    default:
      o.n = 0;
  }
}

}  // namespace uaii_hip
