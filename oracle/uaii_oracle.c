/*
 * uaii_oracle.c — CPU oracle for the GGUF token loop.
 *
 * TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg as the checker. The product library never uses it.
 *
 * This is a plain-C restatement of the reference CPU path ("Path B": packed
 * GGUF weights, per-row dequant then sequential f32 dot). MoE models follow the
 * reference's Path A instead (f32-dequantized weights through the 64-tiled ref
 * GEMM), because the reference's MoE experts only work on f32 weights
 * (libs/uaii-kernels/src/transformer.cpp:551-554). Citations are relative to
 * the reference root.
 */
#define _GNU_SOURCE
#include "uaii_oracle.h"

#include <fcntl.h>
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <time.h>
#include <unistd.h>

static __thread char g_err[512];
static void set_err(const char* msg) { snprintf(g_err, sizeof g_err, "%s", msg); }
const char* orc_last_error(void) { return g_err; }

/* ------------------------------------------------------------------ half */

/* gguf_dequant.cpp:79-105: explicit bit assembly, subnormals renormalised. */
float orc_half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 31u;
  uint32_t m = h & 1023u;
  uint32_t bits;
  if (e == 0 && m == 0) {
    bits = sign;
  } else if (e == 0) {
    /* subnormal: shift the mantissa up until the implicit bit appears */
    uint32_t exp32 = 113; /* 127 - 15 + 1 */
    while (!(m & 0x400u)) { m <<= 1; exp32--; }
    bits = sign | (exp32 << 23) | ((m & 1023u) << 13);
  } else if (e == 31) {
    bits = sign | 0x7f800000u | (m << 13);
  } else {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline float rdh(const uint8_t* p) { return orc_half_to_float(rd16(p)); }

/* ------------------------------------------------------------------ formats */

int orc_block_elems(int t) {
  switch (t) {
    case ORC_F32: case ORC_F16: return 1;
    case ORC_Q4_0: case ORC_Q4_1: case ORC_Q5_0: case ORC_Q5_1: case ORC_Q8_0: return 32;
    case ORC_Q2_K: case ORC_Q3_K: case ORC_Q4_K: case ORC_Q5_K: case ORC_Q6_K: return 256;
    default: return 0;
  }
}

/* formats.hpp:81-102 */
int orc_block_bytes(int t) {
  switch (t) {
    case ORC_F32: return 4;
    case ORC_F16: return 2;
    case ORC_Q4_0: return 18;
    case ORC_Q4_1: return 20;
    case ORC_Q5_0: return 22;
    case ORC_Q5_1: return 24;
    case ORC_Q8_0: return 34;
    case ORC_Q2_K: return 84;
    case ORC_Q3_K: return 110;
    case ORC_Q4_K: return 144;
    case ORC_Q5_K: return 176;
    case ORC_Q6_K: return 210;
    default: return 0;
  }
}

size_t orc_row_bytes(int t, int64_t cols) {
  int be = orc_block_elems(t);
  if (be == 0) return 0;
  return (size_t)(cols / be) * (size_t)orc_block_bytes(t);
}

/* 6-bit scale/min unpack of the K-quant 12-byte scale field
 * (gguf_dequant.cpp:107-115). */
static void kscale(int j, const uint8_t* s, int* sc, int* mn) {
  if (j < 4) {
    *sc = s[j] & 63;
    *mn = s[j + 4] & 63;
  } else {
    *sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
    *mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
}

/* Q4_0 block = f16 d, 16 nibble bytes: low nibbles are elements 0..15, high
 * nibbles 16..31, value (q-8)*d (gguf_dequant.cpp:117-134). */
static void dq_q4_0(const uint8_t* b, float* y) {
  float d = rdh(b);
  for (int j = 0; j < 16; j++) {
    y[j] = (float)((b[2 + j] & 15) - 8) * d;
    y[j + 16] = (float)((b[2 + j] >> 4) - 8) * d;
  }
}

/* Q4_1: d, m (f16), 16 bytes; q*d + m (gguf_dequant.cpp:136-154). */
static void dq_q4_1(const uint8_t* b, float* y) {
  float d = rdh(b), m = rdh(b + 2);
  for (int j = 0; j < 16; j++) {
    y[j] = (float)(b[4 + j] & 15) * d + m;
    y[j + 16] = (float)(b[4 + j] >> 4) * d + m;
  }
}

/* Q5_0: d, 4 bytes of 5th bits, 16 nibble bytes; (q|hb<<4)-16 times d
 * (gguf_dequant.cpp:156-177). */
static void dq_q5_0(const uint8_t* b, float* y) {
  float d = rdh(b);
  uint32_t hb = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) |
                ((uint32_t)b[5] << 24);
  const uint8_t* qs = b + 6;
  for (int j = 0; j < 16; j++) {
    int lo = (qs[j] & 15) | (int)(((hb >> j) & 1u) << 4);
    int hi = (qs[j] >> 4) | (int)(((hb >> (j + 16)) & 1u) << 4);
    y[j] = (float)(lo - 16) * d;
    y[j + 16] = (float)(hi - 16) * d;
  }
}

/* Q5_1: d, m, qh[4], qs[16]; q*d + m (gguf_dequant.cpp:179-201). */
static void dq_q5_1(const uint8_t* b, float* y) {
  float d = rdh(b), m = rdh(b + 2);
  uint32_t hb = (uint32_t)b[4] | ((uint32_t)b[5] << 8) | ((uint32_t)b[6] << 16) |
                ((uint32_t)b[7] << 24);
  const uint8_t* qs = b + 8;
  for (int j = 0; j < 16; j++) {
    int lo = (qs[j] & 15) | (int)(((hb >> j) & 1u) << 4);
    int hi = (qs[j] >> 4) | (int)(((hb >> (j + 16)) & 1u) << 4);
    y[j] = (float)lo * d + m;
    y[j + 16] = (float)hi * d + m;
  }
}

/* Q8_0: d, 32 int8; q*d (gguf_dequant.cpp:203-217). */
static void dq_q8_0(const uint8_t* b, float* y) {
  float d = rdh(b);
  for (int j = 0; j < 32; j++) y[j] = (float)(int8_t)b[2 + j] * d;
}

/* Q2_K: scales[16], qs[64], d, dmin. Each 128-half has 4 bit-planes (shift
 * 0,2,4,6) over two 16-element groups (gguf_dequant.cpp:219-255). */
static void dq_q2_k(const uint8_t* b, float* y) {
  const uint8_t* sc = b;
  const uint8_t* q = b + 16;
  float d = rdh(b + 80), dmin = rdh(b + 82);
  int is = 0;
  for (int half = 0; half < 2; half++) {
    for (int plane = 0; plane < 4; plane++) {
      int shift = 2 * plane;
      for (int g = 0; g < 2; g++) {
        int s = sc[is++];
        float dl = d * (float)(s & 15);
        float ml = dmin * (float)(s >> 4);
        for (int l = 0; l < 16; l++) *y++ = dl * (float)((q[16 * g + l] >> shift) & 3) - ml;
      }
    }
    q += 32;
  }
}

/* Q3_K: hmask[32], qs[64], scales[12] (16 packed 6-bit signed), d
 * (gguf_dequant.cpp:257-306). The 6-bit scale j is low nibble (j<8: byte j low,
 * j>=8: byte j-8 high) plus two high bits from byte 8+(j%4) at shift 2*(j/4). */
static void dq_q3_k(const uint8_t* b, float* y) {
  const uint8_t* hm = b;
  const uint8_t* q = b + 32;
  const uint8_t* s12 = b + 96;
  float dall = rdh(b + 108);
  int scales[16];
  for (int j = 0; j < 16; j++) {
    int lo = (j < 8) ? (s12[j] & 15) : (s12[j - 8] >> 4);
    int hi = (s12[8 + (j % 4)] >> (2 * (j / 4))) & 3;
    scales[j] = (lo | (hi << 4)) - 32;
  }
  int is = 0;
  uint8_t mbit = 1;
  for (int half = 0; half < 2; half++) {
    for (int plane = 0; plane < 4; plane++) {
      int shift = 2 * plane;
      for (int g = 0; g < 2; g++) {
        float dl = dall * (float)scales[is++];
        for (int l = 0; l < 16; l++) {
          int qq = (q[16 * g + l] >> shift) & 3;
          int sub = (hm[16 * g + l] & mbit) ? 0 : 4;
          *y++ = dl * (float)(qq - sub);
        }
      }
      mbit = (uint8_t)(mbit << 1);
    }
    q += 32;
  }
}

/* Q4_K: d, dmin, scales[12], qs[128]; four 64-chunks, low nibbles then high
 * nibbles, y = (d*sc)*q - (dmin*m) with both products rounded
 * (gguf_dequant.cpp:308-340). */
static void dq_q4_k(const uint8_t* b, float* y) {
  float d = rdh(b), dmin = rdh(b + 2);
  const uint8_t* s = b + 4;
  const uint8_t* q = b + 16;
  for (int c = 0; c < 4; c++) {
    int sc, mn;
    kscale(2 * c, s, &sc, &mn);
    float d1 = d * (float)sc, m1 = dmin * (float)mn;
    kscale(2 * c + 1, s, &sc, &mn);
    float d2 = d * (float)sc, m2 = dmin * (float)mn;
    for (int l = 0; l < 32; l++) y[64 * c + l] = d1 * (float)(q[32 * c + l] & 15) - m1;
    for (int l = 0; l < 32; l++) y[64 * c + 32 + l] = d2 * (float)(q[32 * c + l] >> 4) - m2;
  }
}

/* Q5_K: like Q4_K plus qh[32] carrying a 5th bit per element, bit pair (2c, 2c+1)
 * for chunk c (gguf_dequant.cpp:342-379). */
static void dq_q5_k(const uint8_t* b, float* y) {
  float d = rdh(b), dmin = rdh(b + 2);
  const uint8_t* s = b + 4;
  const uint8_t* qh = b + 16;
  const uint8_t* q = b + 48;
  for (int c = 0; c < 4; c++) {
    int sc, mn;
    kscale(2 * c, s, &sc, &mn);
    float d1 = d * (float)sc, m1 = dmin * (float)mn;
    kscale(2 * c + 1, s, &sc, &mn);
    float d2 = d * (float)sc, m2 = dmin * (float)mn;
    for (int l = 0; l < 32; l++) {
      int hb = (qh[l] >> (2 * c)) & 1;
      y[64 * c + l] = d1 * (float)((q[32 * c + l] & 15) + 16 * hb) - m1;
    }
    for (int l = 0; l < 32; l++) {
      int hb = (qh[l] >> (2 * c + 1)) & 1;
      y[64 * c + 32 + l] = d2 * (float)((q[32 * c + l] >> 4) + 16 * hb) - m2;
    }
  }
}

/* Q6_K: ql[128], qh[64], int8 scales[16], d. Per 128-half, element e in 0..127
 * takes its low nibble from ql[e%64] (low nibble for e<64, high for e>=64), its
 * 2 high bits from qh[e%32] at shift 2*(e/32), minus 32, and scale sc[e/16]:
 * y = (d*sc)*q (gguf_dequant.cpp:381-416). */
static void dq_q6_k(const uint8_t* b, float* y) {
  const uint8_t* ql = b;
  const uint8_t* qh = b + 128;
  const int8_t* sc = (const int8_t*)(b + 192);
  float d = rdh(b + 208);
  for (int half = 0; half < 2; half++) {
    for (int e = 0; e < 128; e++) {
      int lo = (e < 64) ? (ql[e] & 15) : (ql[e - 64] >> 4);
      int hi = (qh[e % 32] >> (2 * (e / 32))) & 3;
      int q = (lo | (hi << 4)) - 32;
      y[e] = d * (float)sc[e / 16] * (float)q;
    }
    y += 128;
    ql += 64;
    qh += 32;
    sc += 8;
  }
}

/* dequant_gguf_row dispatch (gguf_dequant.cpp:420-439) plus F32/F16 rows for
 * unquantized tensors (gguf.cpp:471-482). */
int orc_dequant_row(int t, const uint8_t* p, int64_t cols, float* out) {
  if (!p || !out) return -1;
  if (t == ORC_F32) { memcpy(out, p, (size_t)cols * 4); return 0; }
  if (t == ORC_F16) { for (int64_t i = 0; i < cols; i++) out[i] = rdh(p + 2 * i); return 0; }
  int be = orc_block_elems(t), bb = orc_block_bytes(t);
  if (be == 0 || cols % be) return -1;
  int64_t nb = cols / be;
  for (int64_t i = 0; i < nb; i++) {
    const uint8_t* b = p + i * bb;
    float* y = out + i * be;
    switch (t) {
      case ORC_Q4_0: dq_q4_0(b, y); break;
      case ORC_Q4_1: dq_q4_1(b, y); break;
      case ORC_Q5_0: dq_q5_0(b, y); break;
      case ORC_Q5_1: dq_q5_1(b, y); break;
      case ORC_Q8_0: dq_q8_0(b, y); break;
      case ORC_Q2_K: dq_q2_k(b, y); break;
      case ORC_Q3_K: dq_q3_k(b, y); break;
      case ORC_Q4_K: dq_q4_k(b, y); break;
      case ORC_Q5_K: dq_q5_k(b, y); break;
      case ORC_Q6_K: dq_q6_k(b, y); break;
      default: return -1;
    }
  }
  return 0;
}

/* Row values of the reference's f32 weight load (gguf.cpp:445-556). */
int orc_load_row_f32(int t, const uint8_t* p, int64_t cols, float* out) {
  if (t != ORC_Q4_0) return orc_dequant_row(t, p, cols, out);
  if (!p || !out || cols % 32) return -1;
  for (int64_t b = 0; b < cols / 32; b++) {
    const uint8_t* blk = p + b * 18;
    const float d = rdh(blk);
    for (int i = 0; i < 32; i += 2) { /* gguf.cpp:514-520 */
      const uint8_t byte = blk[2 + i / 2];
      out[b * 32 + i] = d * (float)((int)(byte & 0x0f) - 8);
      out[b * 32 + i + 1] = d * (float)((int)(byte >> 4) - 8);
    }
  }
  return 0;
}

/* ------------------------------------------------------------------ threads */

typedef struct {
  void (*fn)(void* ctx, int64_t i, float* scratch);
  void* ctx;
  int64_t n;
  atomic_llong next;
  size_t scratch_floats;
} orc_pfor;

static void* pfor_body(void* arg) {
  orc_pfor* pf = (orc_pfor*)arg;
  float* scratch = pf->scratch_floats ? (float*)malloc(pf->scratch_floats * 4) : NULL;
  for (;;) {
    int64_t i = atomic_fetch_add(&pf->next, 1);
    if (i >= pf->n) break;
    pf->fn(pf->ctx, i, scratch);
  }
  free(scratch);
  return NULL;
}

static int ncores(void) {
  long n = sysconf(_SC_NPROCESSORS_ONLN);
  const char* env = getenv("UAII_NUM_THREADS"); /* thread_pool.cpp:13-22 */
  if (env && atoi(env) > 0) n = atoi(env);
  return n < 1 ? 1 : (int)n;
}

/* Dynamic work distribution over [0,n) like parallel_for (thread_pool.cpp:25-54);
 * each index is computed by exactly one thread, so results are order-free. */
static void parallel_for(int64_t n, int nthreads, size_t scratch_floats,
                         void (*fn)(void*, int64_t, float*), void* ctx) {
  if (nthreads <= 0) nthreads = ncores();
  if (nthreads > n) nthreads = (int)n;
  orc_pfor pf = {fn, ctx, n, 0, scratch_floats};
  atomic_init(&pf.next, 0);
  if (nthreads <= 1) { pfor_body(&pf); return; }
  pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)nthreads);
  for (int t = 1; t < nthreads; t++) pthread_create(&th[t], NULL, pfor_body, &pf);
  pfor_body(&pf);
  for (int t = 1; t < nthreads; t++) pthread_join(th[t], NULL);
  free(th);
}

/* ------------------------------------------------------------------ GEMV */

typedef struct {
  int type;
  const float* A;
  int64_t M, K, N;
  const uint8_t* B;
  size_t stride;
  float* C;
} qg_ctx;

/* quant_gemm.cpp:55-68: one output column j: dequant row j, then for each A row a
 * left-to-right f32 sum. */
static void qg_row(void* vctx, int64_t j, float* row) {
  qg_ctx* c = (qg_ctx*)vctx;
  if (orc_dequant_row(c->type, c->B + (size_t)j * c->stride, c->K, row) != 0) return;
  for (int64_t i = 0; i < c->M; i++) {
    const float* a = c->A + i * c->K;
    float s = 0.0f;
    for (int64_t k = 0; k < c->K; k++) s += a[k] * row[k];
    c->C[i * c->N + j] = s;
  }
}

int orc_quant_gemm(int type, const float* A, int64_t M, int64_t K, const uint8_t* B,
                   int64_t N, float* C, int nthreads) {
  if (orc_block_elems(type) == 0 || K % orc_block_elems(type)) return -1;
  qg_ctx c = {type, A, M, K, N, B, orc_row_bytes(type, K), C};
  parallel_for(N, nthreads, (size_t)K, qg_row, &c);
  return 0;
}

/* ------------------------------------------------------------------ small ops */

void orc_rmsnorm(const float* x, const float* w, float* y, int64_t n, float eps) {
  float ss = 0.0f;
  for (int64_t i = 0; i < n; i++) ss += x[i] * x[i];
  ss /= (float)n;
  float inv = 1.0f / sqrtf(ss + eps);
  for (int64_t i = 0; i < n; i++) {
    float v = x[i] * inv;
    if (w) v *= w[i];
    y[i] = v;
  }
}

void orc_rope(float* x, int64_t dim, int64_t head_dim, float pos, float theta, int mode) {
  int64_t rd = head_dim > 0 ? head_dim : dim;
  int64_t half = rd / 2;
  for (int64_t h = 0; h < dim / rd; h++) {
    float* v = x + h * rd;
    if (mode == 2) {
      for (int64_t i = 0; i < half; i++) {
        float freq = 1.0f / powf(theta, (2.0f * (float)i) / (float)rd);
        float ang = pos * freq;
        float c = cosf(ang), s = sinf(ang);
        float a = v[i], b = v[i + half];
        v[i] = a * c - b * s;
        v[i + half] = a * s + b * c;
      }
    } else {
      for (int64_t i = 0; i < rd; i += 2) {
        float freq = 1.0f / powf(theta, (float)i / (float)rd);
        float ang = pos * freq;
        float c = cosf(ang), s = sinf(ang);
        float a = v[i], b = v[i + 1];
        v[i] = a * c - b * s;
        v[i + 1] = a * s + b * c;
      }
    }
  }
}

/* transformer.cpp:332-374 specialised to q_seq=1: scores, softmax with the max
 * subtracted, probabilities normalised, then P.V summed key by key. Each score is
 * one left-to-right sum over d (four keys' sums advance together: independent
 * chains), and each output element one left-to-right sum over the keys (taken
 * key-outer across a head's elements), so the values are those of the plain
 * loops in the reference's order. */
typedef float orc_v4a __attribute__((vector_size(16), aligned(4)));

void orc_attention_decode(const float* q, const float* kc, const float* vc, int64_t past,
                          const float* kn, const float* vn, float* out, int n_heads,
                          int n_kv_heads, int hd) {
  int64_t kvd = (int64_t)n_kv_heads * hd;
  int64_t n = past + 1;
  int group = n_heads / n_kv_heads;
  float scale = 1.0f / sqrtf((float)hd);
  float* p = (float*)malloc((size_t)n * 4);
  float* acc = (float*)malloc((size_t)hd * 4);
  for (int h = 0; h < n_heads; h++) {
    int kh = h / group;
    const float* qh = q + (int64_t)h * hd;
    float mx = -INFINITY;
#define ORC_KROW(j) (((j) < past) ? kc + (j) * kvd + kh * hd : kn + kh * hd)
    int64_t j = 0;
    for (; j + 4 <= n; j += 4) {
      const float *k0 = ORC_KROW(j), *k1 = ORC_KROW(j + 1), *k2 = ORC_KROW(j + 2), *k3 = ORC_KROW(j + 3);
      float d0 = 0.0f, d1 = 0.0f, d2 = 0.0f, d3 = 0.0f;
      for (int d = 0; d < hd; d++) {
        d0 += qh[d] * k0[d];
        d1 += qh[d] * k1[d];
        d2 += qh[d] * k2[d];
        d3 += qh[d] * k3[d];
      }
      p[j] = d0 * scale; p[j + 1] = d1 * scale; p[j + 2] = d2 * scale; p[j + 3] = d3 * scale;
    }
    for (; j < n; j++) {
      const float* kr = ORC_KROW(j);
      float dot = 0.0f;
      for (int d = 0; d < hd; d++) dot += qh[d] * kr[d];
      p[j] = dot * scale;
    }
#undef ORC_KROW
    for (j = 0; j < n; j++) if (p[j] > mx) mx = p[j];
    float sum = 0.0f;
    for (j = 0; j < n; j++) { p[j] = expf(p[j] - mx); sum += p[j]; }
    float inv = sum > 0 ? 1.0f / sum : 0.0f;
    for (j = 0; j < n; j++) p[j] *= inv;
    for (int d = 0; d < hd; d++) acc[d] = 0.0f;
    for (j = 0; j < n; j++) {
      const float* vr = (j < past) ? vc + j * kvd + kh * hd : vn + kh * hd;
      const float pj = p[j];
      int d = 0;
      if ((hd & 3) == 0) {
        const orc_v4a pb = {pj, pj, pj, pj};
        for (; d < hd; d += 4) {
          orc_v4a a = *(const orc_v4a*)(acc + d), b = *(const orc_v4a*)(vr + d);
          *(orc_v4a*)(acc + d) = a + pb * b;
        }
      }
      for (; d < hd; d++) acc[d] += pj * vr[d];
    }
    for (int d = 0; d < hd; d++) out[(int64_t)h * hd + d] = acc[d];
  }
  free(acc);
  free(p);
}

void orc_softmax(const float* x, float* y, int64_t n) {
  float mx = -INFINITY;
  for (int64_t i = 0; i < n; i++) if (x[i] > mx) mx = x[i];
  float sum = 0.0f;
  for (int64_t i = 0; i < n; i++) { y[i] = expf(x[i] - mx); sum += y[i]; }
  float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
  for (int64_t i = 0; i < n; i++) y[i] *= inv;
}

int64_t orc_argmax(const float* row, int64_t n) {
  int64_t best = 0;
  float bv = row[0];
  for (int64_t i = 1; i < n; i++) if (row[i] > bv) { bv = row[i]; best = i; }
  return best;
}

float orc_silu(float v) { return v / (1.0f + expf(-v)); }

/* Ref GEMM inner order for one output (gemm_ref.cpp:55-73): k in tiles of 64,
 * each tile summed from zero, then added to the running output. */
static float dot_tiled64(const float* a, const float* b, int64_t k) {
  float c = 0.0f;
  for (int64_t k0 = 0; k0 < k; k0 += 64) {
    int64_t k1 = k0 + 64 < k ? k0 + 64 : k;
    float s = 0.0f;
    for (int64_t kk = k0; kk < k1; kk++) s += a[kk] * b[kk];
    c += 1.0f * s;
  }
  return c;
}

void orc_moe_router(const float* x, const float* gate, int64_t D, int64_t E, float* probs) {
  float* lg = (float*)malloc((size_t)E * 4);
  for (int64_t e = 0; e < E; e++) lg[e] = dot_tiled64(x, gate + e * D, D);
  orc_softmax(lg, probs, E);
  free(lg);
}

/* partial_sort by descending prob (transformer.cpp:565-570); equal probs keep the
 * lower expert first (a deterministic choice: std::partial_sort leaves their order
 * unspecified). Weights = p / sum of the top-k probs (:571-580). */
void orc_moe_topk(const float* probs, int64_t E, int k, int* ids, float* w) {
  int used[256] = {0};
  if (k > E) k = (int)E;
  float mass = 0.0f;
  for (int t = 0; t < k; t++) {
    int best = -1;
    for (int64_t e = 0; e < E; e++) {
      if (used[e]) continue;
      if (best < 0 || probs[e] > probs[best]) best = (int)e;
    }
    used[best] = 1;
    ids[t] = best;
    mass += probs[best];
  }
  if (!(mass > 0.0f)) mass = 1.0f;
  for (int t = 0; t < k; t++) w[t] = probs[ids[t]] / mass;
}

/* ------------------------------------------------------------------ GGUF */

typedef struct {
  char name[96];
  int type;
  int n_dims;
  uint64_t ne[4];
  uint64_t offset;
  const uint8_t* data;
} orc_tensor;

typedef struct {
  int type;            /* GGUF type */
  int64_t rows, cols;  /* row-major [rows, cols] (dims reversed, gguf.cpp:272-280) */
  int64_t n3;          /* leading expert dim for 3-D stacks, else 1 */
  const uint8_t* data;
  float* f32;          /* dequantized copy (norms always; all weights on Path A) */
} orc_w;

typedef struct {
  orc_w attn_norm, wq, wk, wv, wo, bq, bk, bv, ffn_norm, w_gate, w_up, w_down;
  orc_w gate_inp, gate_exps, up_exps, down_exps, gate_sh, up_sh, down_sh;
  int has_bias_q, has_bias_k, has_bias_v, moe, shared, gelu, has_ffn_norm, has_ffn;
} orc_layer;

struct orc_model {
  uint8_t* map;
  size_t map_len;
  int n_tensors;
  orc_tensor* t;
  char arch[64];
  int64_t n_layers, dim, n_heads, n_kv, head_dim, vocab, ffn, n_experts, top_k, ctx;
  int rope_mode, tied, path_a;
  float theta, eps;
  orc_w tok_embd, out_norm, output;
  int has_out_norm;
  orc_layer* L;
};

typedef struct {
  const uint8_t* p;
  const uint8_t* end;
  int bad;
} rdr;

static uint64_t rd_u(rdr* r, int n) {
  if (r->p + n > r->end) { r->bad = 1; return 0; }
  uint64_t v = 0;
  for (int i = 0; i < n; i++) v |= (uint64_t)r->p[i] << (8 * i);
  r->p += n;
  return v;
}

/* KV value sizes by GGUF value type (gguf.cpp:20-34). */
static int scalar_size(uint32_t vt) {
  switch (vt) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    default: return -1;
  }
}

typedef struct {
  char key[128];
  uint32_t vt;
  const uint8_t* val; /* points at the value bytes (not for arrays) */
  uint64_t slen;      /* string length */
} orc_kv;

static int skip_value(rdr* r, uint32_t vt) {
  if (vt == 8) { uint64_t n = rd_u(r, 8); if (r->p + n > r->end) return -1; r->p += n; return 0; }
  if (vt == 9) {
    uint32_t et = (uint32_t)rd_u(r, 4);
    uint64_t n = rd_u(r, 8);
    for (uint64_t i = 0; i < n && !r->bad; i++) if (skip_value(r, et)) return -1;
    return r->bad ? -1 : 0;
  }
  int s = scalar_size(vt);
  if (s < 0 || r->p + s > r->end) return -1;
  r->p += s;
  return 0;
}

static int64_t kv_int(const orc_kv* kv, int nkv, const char* key, int64_t def) {
  for (int i = 0; i < nkv; i++) {
    if (strcmp(kv[i].key, key)) continue;
    rdr r = {kv[i].val, kv[i].val + 8, 0};
    switch (kv[i].vt) { /* kv_i64 accepts i64/u64/i32/u32 (gguf.cpp:664-676) */
      case 4: return (int64_t)(uint32_t)rd_u(&r, 4);
      case 5: return (int64_t)(int32_t)rd_u(&r, 4);
      case 10: return (int64_t)rd_u(&r, 8);
      case 11: return (int64_t)rd_u(&r, 8);
      default: return def;
    }
  }
  return def;
}

static int kv_has(const orc_kv* kv, int nkv, const char* key) {
  for (int i = 0; i < nkv; i++) if (!strcmp(kv[i].key, key)) return 1;
  return 0;
}

static float kv_flt(const orc_kv* kv, int nkv, const char* key, float def) {
  for (int i = 0; i < nkv; i++) {
    if (strcmp(kv[i].key, key)) continue;
    rdr r = {kv[i].val, kv[i].val + 8, 0};
    switch (kv[i].vt) { /* kv_float (gguf.cpp:693-707) */
      case 6: { uint32_t b = (uint32_t)rd_u(&r, 4); float f; memcpy(&f, &b, 4); return f; }
      case 12: { uint64_t b = rd_u(&r, 8); double d; memcpy(&d, &b, 8); return (float)d; }
      case 5: return (float)(int32_t)rd_u(&r, 4);
      case 11: return (float)(int64_t)rd_u(&r, 8);
      case 4: return (float)(uint32_t)rd_u(&r, 4);
      case 10: return (float)rd_u(&r, 8);
      default: return def;
    }
  }
  return def;
}

/* Arch-prefixed, then llama., then general. (gguf.cpp:734-763). */
static int64_t kv_int_arch(const orc_kv* kv, int n, const char* arch, const char* suf,
                           int64_t def) {
  char k[192];
  if (arch[0]) {
    snprintf(k, sizeof k, "%s.%s", arch, suf);
    int64_t v = kv_int(kv, n, k, -1);
    if (v >= 0) return v;
  }
  snprintf(k, sizeof k, "llama.%s", suf);
  int64_t v = kv_int(kv, n, k, -1);
  if (v >= 0) return v;
  snprintf(k, sizeof k, "general.%s", suf);
  v = kv_int(kv, n, k, -1);
  if (v >= 0) return v;
  return def;
}

static float kv_flt_arch(const orc_kv* kv, int n, const char* arch, const char* suf,
                         float def) {
  char k[192];
  if (arch[0]) {
    snprintf(k, sizeof k, "%s.%s", arch, suf);
    if (kv_has(kv, n, k)) return kv_flt(kv, n, k, def);
  }
  snprintf(k, sizeof k, "llama.%s", suf);
  if (kv_has(kv, n, k)) return kv_flt(kv, n, k, def);
  snprintf(k, sizeof k, "general.%s", suf);
  if (kv_has(kv, n, k)) return kv_flt(kv, n, k, def);
  return def;
}

static const orc_tensor* find_t(const orc_model* m, const char* name) {
  for (int i = 0; i < m->n_tensors; i++) if (!strcmp(m->t[i].name, name)) return &m->t[i];
  return NULL;
}

static int type_supported(int t) { return orc_block_elems(t) != 0; }

static size_t tensor_bytes(const orc_tensor* t) {
  uint64_t n = 1;
  for (int d = 0; d < t->n_dims; d++) n *= t->ne[d];
  return orc_row_bytes(t->type, (int64_t)n);
}

/* f32 copy of a weight: the f32 load's values on Path A, else the dequant's */
static float* dequant_all(const orc_w* w, int path_a) {
  int64_t per = w->rows * w->cols;
  float* f = (float*)malloc((size_t)(per * w->n3) * 4);
  size_t rb = orc_row_bytes(w->type, w->cols);
  for (int64_t r = 0; r < w->rows * w->n3; r++) {
    if (path_a) orc_load_row_f32(w->type, w->data + r * rb, w->cols, f + r * w->cols);
    else orc_dequant_row(w->type, w->data + r * rb, w->cols, f + r * w->cols);
  }
  return f;
}

static int bind_w(orc_model* m, const char* name, orc_w* w, int want_f32) {
  memset(w, 0, sizeof *w);
  const orc_tensor* t = find_t(m, name);
  if (!t) return 0;
  if (!type_supported(t->type)) {
    snprintf(g_err, sizeof g_err, "unsupported GGUF quant type for weight %s", name);
    return -1;
  }
  w->type = t->type;
  w->cols = (int64_t)t->ne[0];
  w->rows = t->n_dims > 1 ? (int64_t)t->ne[1] : 1;
  w->n3 = t->n_dims > 2 ? (int64_t)t->ne[2] : 1;
  w->data = t->data;
  if (want_f32 || t->type == ORC_F32 || t->type == ORC_F16) w->f32 = dequant_all(w, m->path_a);
  return 1;
}

static void free_w(orc_w* w) { free(w->f32); w->f32 = NULL; }

orc_model* orc_model_open(const char* path, int max_layers) {
  return orc_model_open_ex(path, max_layers, 0);
}

orc_model* orc_model_open_ex(const char* path, int max_layers, int path_a) {
  int fd = open(path, O_RDONLY);
  if (fd < 0) { set_err("cannot open gguf"); return NULL; }
  struct stat st;
  fstat(fd, &st);
  uint8_t* map = (uint8_t*)mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (map == MAP_FAILED) { set_err("mmap failed"); return NULL; }
  orc_model* m = (orc_model*)calloc(1, sizeof *m);
  m->map = map;
  m->map_len = (size_t)st.st_size;
  rdr r = {map, map + st.st_size, 0};
  if (st.st_size < 24 || memcmp(map, "GGUF", 4)) { set_err("not a GGUF file"); goto fail; }
  r.p += 4;
  rd_u(&r, 4); /* version */
  uint64_t nt = rd_u(&r, 8), nkv = rd_u(&r, 8);
  orc_kv* kv = (orc_kv*)calloc(nkv ? nkv : 1, sizeof(orc_kv));
  for (uint64_t i = 0; i < nkv; i++) {
    uint64_t kl = rd_u(&r, 8);
    if (r.bad || r.p + kl > r.end) { free(kv); set_err("truncated kv"); goto fail; }
    size_t cl = kl < sizeof(kv[i].key) - 1 ? kl : sizeof(kv[i].key) - 1;
    memcpy(kv[i].key, r.p, cl);
    r.p += kl;
    kv[i].vt = (uint32_t)rd_u(&r, 4);
    kv[i].val = r.p;
    if (kv[i].vt == 8) { kv[i].slen = 0; memcpy(&kv[i].slen, r.p, 8); kv[i].val = r.p + 8; }
    if (skip_value(&r, kv[i].vt)) { free(kv); set_err("bad kv value"); goto fail; }
  }
  m->n_tensors = (int)nt;
  m->t = (orc_tensor*)calloc(nt ? nt : 1, sizeof(orc_tensor));
  for (uint64_t i = 0; i < nt; i++) {
    orc_tensor* t = &m->t[i];
    uint64_t nl = rd_u(&r, 8);
    if (r.bad || r.p + nl > r.end) { free(kv); set_err("truncated tensor info"); goto fail; }
    size_t cl = nl < sizeof(t->name) - 1 ? nl : sizeof(t->name) - 1;
    memcpy(t->name, r.p, cl);
    r.p += nl;
    t->n_dims = (int)rd_u(&r, 4);
    for (int d = 0; d < t->n_dims && d < 4; d++) t->ne[d] = rd_u(&r, 8);
    t->type = (int)rd_u(&r, 4);
    t->offset = rd_u(&r, 8);
  }
  if (r.bad) { free(kv); set_err("truncated header"); goto fail; }
  /* data section forced to 32-byte alignment (gguf.cpp:436-440) */
  size_t data_off = ((size_t)(r.p - map) + 31) & ~(size_t)31;
  for (uint64_t i = 0; i < nt; i++) {
    m->t[i].data = map + data_off + m->t[i].offset;
    if (type_supported(m->t[i].type) &&
        data_off + m->t[i].offset + tensor_bytes(&m->t[i]) > m->map_len) {
      free(kv); set_err("tensor data past end of file"); goto fail;
    }
  }

  /* hyperparameters (gguf.cpp:835-885) */
  {
    const orc_kv* a = NULL;
    for (uint64_t i = 0; i < nkv; i++) if (!strcmp(kv[i].key, "general.architecture")) a = &kv[i];
    if (a && a->vt == 8) {
      size_t n = a->slen < sizeof(m->arch) - 1 ? a->slen : sizeof(m->arch) - 1;
      for (size_t i = 0; i < n; i++) {
        char c = (char)a->val[i];
        m->arch[i] = (c >= 'A' && c <= 'Z') ? (char)(c + 32) : c;
      }
    }
  }
  int n = (int)nkv;
  const orc_tensor* emb = find_t(m, "token_embd.weight");
  const orc_tensor* lm = find_t(m, "output.weight");
  if (!emb) { free(kv); set_err("no token_embd.weight"); goto fail; }
  m->tied = lm == NULL;
  m->dim = (int64_t)emb->ne[0];
  m->vocab = lm ? (int64_t)lm->ne[1] : (int64_t)emb->ne[1];
  m->n_heads = kv_int_arch(kv, n, m->arch, "attention.head_count", 0);
  if (m->n_heads <= 0) m->n_heads = 1;
  m->n_kv = kv_int_arch(kv, n, m->arch, "attention.head_count_kv", m->n_heads);
  if (m->n_kv <= 0) m->n_kv = m->n_heads;
  int64_t emb_len = kv_int_arch(kv, n, m->arch, "embedding_length", m->dim);
  m->head_dim = kv_int_arch(kv, n, m->arch, "attention.key_length", 0);
  if (m->head_dim <= 0) m->head_dim = (emb_len > 0 ? emb_len : m->dim) / m->n_heads;
  m->theta = kv_flt_arch(kv, n, m->arch, "rope.freq_base", 10000.f);
  {
    static const char* neox[] = {"qwen2", "qwen2moe", "qwen3", "qwen", "phi2", "phi3",
                                 "falcon", "stablelm", "starcoder2", "olmo2", "gemma",
                                 "gemma2", "gemma3"};
    m->rope_mode = 0;
    for (size_t i = 0; i < sizeof neox / sizeof *neox; i++)
      if (!strcmp(m->arch, neox[i])) m->rope_mode = 2;
  }
  m->eps = kv_flt_arch(kv, n, m->arch, "attention.layer_norm_rms_epsilon", 1e-5f);
  m->n_layers = kv_int_arch(kv, n, m->arch, "block_count", 0);
  m->ctx = kv_int_arch(kv, n, m->arch, "context_length", 0);
  m->n_experts = kv_int_arch(kv, n, m->arch, "expert_count", 0);
  m->top_k = kv_int_arch(kv, n, m->arch, "expert_used_count", 2);
  if (m->top_k <= 0) m->top_k = 2;
  free(kv);
  if (m->n_layers <= 0) {
    char nm[96];
    for (int i = 0; i < 512; i++) {
      snprintf(nm, sizeof nm, "blk.%d.attn_norm.weight", i);
      char nq[96];
      snprintf(nq, sizeof nq, "blk.%d.attn_q.weight", i);
      if (!find_t(m, nm) && !find_t(m, nq)) { m->n_layers = i; break; }
    }
  }
  if (m->n_layers > 512) m->n_layers = 512;
  if (max_layers > 0 && m->n_layers > max_layers) m->n_layers = max_layers;
  m->path_a = path_a || find_t(m, "blk.0.ffn_gate_exps.weight") != NULL || m->n_experts > 0;

  if (bind_w(m, "token_embd.weight", &m->tok_embd, 0) < 0) goto fail;
  if (!m->tied && bind_w(m, "output.weight", &m->output, m->path_a) < 0) goto fail;
  if (m->tied) {
    /* lm_head reuses the embedding weight (gguf.cpp:813-816); own f32 copy if needed */
    m->output = m->tok_embd;
    int need = m->path_a || m->tok_embd.type == ORC_F32 || m->tok_embd.type == ORC_F16;
    m->output.f32 = need ? dequant_all(&m->tok_embd, m->path_a) : NULL;
  }
  m->has_out_norm = bind_w(m, "output_norm.weight", &m->out_norm, 1);
  if (m->has_out_norm < 0) goto fail;

  m->L = (orc_layer*)calloc((size_t)(m->n_layers ? m->n_layers : 1), sizeof(orc_layer));
  for (int64_t li = 0; li < m->n_layers; li++) {
    orc_layer* L = &m->L[li];
    char nm[128];
    int pa = m->path_a;
#define BIND(field, suffix, f32)                                      \
  snprintf(nm, sizeof nm, "blk.%ld." suffix, (long)li);               \
  if (bind_w(m, nm, &L->field, f32) < 0) goto fail;
    BIND(attn_norm, "attn_norm.weight", 1)
    BIND(wq, "attn_q.weight", pa) BIND(wk, "attn_k.weight", pa) BIND(wv, "attn_v.weight", pa)
    BIND(bq, "attn_q.bias", 1) BIND(bk, "attn_k.bias", 1) BIND(bv, "attn_v.bias", 1)
    BIND(wo, "attn_output.weight", pa) BIND(ffn_norm, "ffn_norm.weight", 1)
    BIND(w_gate, "ffn_gate.weight", pa) BIND(w_up, "ffn_up.weight", pa)
    BIND(w_down, "ffn_down.weight", pa) BIND(gate_inp, "ffn_gate_inp.weight", 1)
    BIND(gate_exps, "ffn_gate_exps.weight", 1) BIND(up_exps, "ffn_up_exps.weight", 1)
    BIND(down_exps, "ffn_down_exps.weight", 1) BIND(gate_sh, "ffn_gate_shexp.weight", pa)
    BIND(up_sh, "ffn_up_shexp.weight", pa) BIND(down_sh, "ffn_down_shexp.weight", pa)
#undef BIND
    if (!L->attn_norm.data || !L->wq.data || !L->wk.data || !L->wv.data || !L->wo.data) {
      m->n_layers = li; /* incomplete layer stops the stack (gguf.cpp:993-996) */
      break;
    }
    L->has_bias_q = L->bq.data != NULL;
    L->has_bias_k = L->bk.data != NULL;
    L->has_bias_v = L->bv.data != NULL;
    L->has_ffn_norm = L->ffn_norm.data != NULL;
    L->moe = L->gate_inp.data && L->gate_exps.data && L->up_exps.data && L->down_exps.data;
    L->shared = L->moe && L->gate_sh.data && L->up_sh.data && L->down_sh.data;
    L->has_ffn = L->moe || (L->w_gate.data && L->w_up.data && L->w_down.data) ||
                 (L->w_up.data && L->w_down.data);
    L->gelu = !L->moe && !L->w_gate.data && L->w_up.data && L->w_down.data;
    if (L->moe && m->n_experts <= 0) m->n_experts = L->gate_exps.n3;
    if (L->w_up.data && !m->ffn) m->ffn = L->w_up.rows;
    if (L->moe && !m->ffn) m->ffn = L->gate_exps.rows;
  }
  if (m->top_k > m->n_experts && m->n_experts > 0) m->top_k = m->n_experts;
  return m;
fail:
  orc_model_close(m);
  return NULL;
}

void orc_model_close(orc_model* m) {
  if (!m) return;
  if (m->L) {
    for (int64_t i = 0; i < m->n_layers; i++) {
      orc_w* ws = (orc_w*)&m->L[i];
      for (size_t k = 0; k < 19; k++) free_w(&ws[k]);
    }
    free(m->L);
  }
  if (m->tied) { free(m->output.f32); } else { free_w(&m->output); }
  free_w(&m->tok_embd);
  free_w(&m->out_norm);
  free(m->t);
  if (m->map) munmap(m->map, m->map_len);
  free(m);
}

void orc_model_hparams(const orc_model* m, int64_t* o) {
  o[0] = m->n_layers; o[1] = m->dim; o[2] = m->n_heads; o[3] = m->n_kv; o[4] = m->head_dim;
  o[5] = m->vocab; o[6] = m->ffn; o[7] = m->n_experts; o[8] = m->top_k;
  o[9] = m->rope_mode; o[10] = m->ctx; o[11] = m->tied;
}

void orc_model_fparams(const orc_model* m, float* o) { o[0] = m->theta; o[1] = m->eps; }

int orc_model_tensor(const orc_model* m, const char* name, int* type, int64_t* ne3,
                     const uint8_t** data) {
  const orc_tensor* t = find_t(m, name);
  if (!t) return -1;
  *type = t->type;
  for (int d = 0; d < 3; d++) ne3[d] = d < t->n_dims ? (int64_t)t->ne[d] : 1;
  *data = t->data;
  return 0;
}

/* ------------------------------------------------------------------ forward */

/* y[N] = W[N,K] . x. Path B: quant_gemm (per-row dequant + sequential dot).
 * Path A: f32 weights through the 64-tiled ref GEMM order. */
typedef struct {
  const orc_w* w;
  const float* x;
  float* y;
  int64_t row0;
} mv_ctx;

static void mv_row_a(void* v, int64_t j, float* scratch) {
  (void)scratch;
  mv_ctx* c = (mv_ctx*)v;
  c->y[j] = dot_tiled64(c->x, c->w->f32 + (c->row0 + j) * c->w->cols, c->w->cols);
}

static void matvec(const orc_model* m, const orc_w* w, const float* x, float* y,
                   int64_t row0, int64_t nrows, int nthreads) {
  if (m->path_a || w->type == ORC_F32 || w->type == ORC_F16) {
    mv_ctx c = {w, x, y, row0};
    if (!w->f32) return;
    parallel_for(nrows, nthreads, 0, mv_row_a, &c);
    return;
  }
  size_t rb = orc_row_bytes(w->type, w->cols);
  orc_quant_gemm(w->type, x, 1, w->cols, w->data + row0 * rb, nrows, y, nthreads);
}

typedef struct {
  orc_model* m;
  int kv_f16;
  int64_t max_seq;
  float* kc;  /* [L][max_seq][kv_dim] */
  float* vc;
  float *x, *n1, *q, *k, *v, *att, *tmp, *g, *u, *hid, *logits, *probs, *eout;
} orc_state;

/* float -> half bits, round to nearest even (IEEE 754 binary16): the value the
 * fp16 KV cache holds for each cached K/V element. Overflow goes to +-inf, values
 * below half the smallest subnormal to a signed zero, NaN stays NaN (quiet, sign
 * kept). Pinned by tests/test_oracle_f16.py against numpy's IEEE conversion on
 * every float32 bit pattern and by closed-form ties, subnormals and overflows. */
uint16_t orc_float_to_half(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  uint32_t sign = (b >> 16) & 0x8000u;
  int32_t e = (int32_t)((b >> 23) & 255) - 127 + 15;
  uint32_t mant = b & 0x7fffffu;
  uint16_t h;
  if (((b >> 23) & 255) == 255) {
    h = (uint16_t)(sign | 0x7c00u | (mant ? 0x200u : 0));
  } else if (e >= 31) {
    h = (uint16_t)(sign | 0x7c00u);
  } else if (e <= 0) {
    if (e < -10) {
      h = (uint16_t)sign;
    } else {
      uint32_t mm = mant | 0x800000u;
      int shift = 14 - e;
      uint32_t hm = mm >> shift;
      uint32_t rem = mm & ((1u << shift) - 1), halfway = 1u << (shift - 1);
      if (rem > halfway || (rem == halfway && (hm & 1))) hm++;
      h = (uint16_t)(sign | hm);
    }
  } else {
    uint32_t hm = mant >> 13, rem = mant & 0x1fffu;
    uint32_t hv = sign | ((uint32_t)e << 10) | hm;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1))) hv++;
    h = (uint16_t)hv;
  }
  return h;
}

void orc_float_to_half_n(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = orc_float_to_half(in[i]);
}

/* float -> half -> float, for the fp16 cache mirror */
static float round_f16(float f) { return orc_half_to_float(orc_float_to_half(f)); }

static void state_free(orc_state* s) {
  free(s->kc); free(s->vc); free(s->x); free(s->n1); free(s->q); free(s->k); free(s->v);
  free(s->att); free(s->tmp); free(s->g); free(s->u); free(s->hid); free(s->logits);
  free(s->probs); free(s->eout);
}

static int state_init(orc_state* s, orc_model* m, int64_t max_seq, int kv_f16) {
  memset(s, 0, sizeof *s);
  s->m = m;
  s->kv_f16 = kv_f16;
  s->max_seq = max_seq;
  int64_t kvd = m->n_kv * m->head_dim, qd = m->n_heads * m->head_dim;
  int64_t ff = m->ffn > 0 ? m->ffn : 4 * m->dim;
  size_t kvn = (size_t)(m->n_layers ? m->n_layers : 1) * (size_t)max_seq * (size_t)kvd;
  s->kc = (float*)calloc(kvn, 4);
  s->vc = (float*)calloc(kvn, 4);
  s->x = (float*)calloc((size_t)m->dim, 4);
  s->n1 = (float*)calloc((size_t)m->dim, 4);
  s->q = (float*)calloc((size_t)qd, 4);
  s->k = (float*)calloc((size_t)kvd, 4);
  s->v = (float*)calloc((size_t)kvd, 4);
  s->att = (float*)calloc((size_t)qd, 4);
  s->tmp = (float*)calloc((size_t)(m->dim > qd ? m->dim : qd), 4);
  s->g = (float*)calloc((size_t)ff, 4);
  s->u = (float*)calloc((size_t)ff, 4);
  s->hid = (float*)calloc((size_t)ff, 4);
  s->eout = (float*)calloc((size_t)m->dim, 4);
  s->logits = (float*)calloc((size_t)m->vocab, 4);
  s->probs = (float*)calloc((size_t)m->vocab, 4);
  if (!s->kc || !s->vc || !s->logits) { state_free(s); set_err("oom"); return -1; }
  return 0;
}

/* MoE FFN on f32 expert stacks (transformer.cpp:522-612): for each selected
 * expert, gate/up rows summed over D, SiLU*up, down rows summed over I, then
 * Y += w*out, experts in descending-prob order. Rows run on parallel_for; each
 * row's sum is one thread's sequential loop, so the result does not depend on
 * the thread count. */
typedef struct {
  const float *xin, *G, *U, *Dn;
  float *hid, *y;
  int64_t D, I;
  float w;
} moe_ctx;

static void moe_gate_up_row(void* v, int64_t i, float* scratch) {
  (void)scratch;
  moe_ctx* c = (moe_ctx*)v;
  float gs = 0.0f, us = 0.0f;
  for (int64_t d = 0; d < c->D; d++) {
    gs += c->xin[d] * c->G[i * c->D + d];
    us += c->xin[d] * c->U[i * c->D + d];
  }
  float sig = 1.0f / (1.0f + expf(-gs));
  c->hid[i] = (gs * sig) * us;
}

static void moe_down_row(void* v, int64_t o, float* scratch) {
  (void)scratch;
  moe_ctx* c = (moe_ctx*)v;
  float acc = 0.0f;
  for (int64_t i = 0; i < c->I; i++) acc += c->hid[i] * c->Dn[o * c->I + i];
  c->y[o] += c->w * acc;
}

static void moe_ffn(orc_state* s, const orc_layer* L, const float* xin, float* y,
                    int nthreads) {
  orc_model* m = s->m;
  int64_t D = m->dim, I = L->gate_exps.rows, E = L->gate_exps.n3;
  float probs[256];
  int ids[256];
  float w[256];
  orc_moe_router(xin, L->gate_inp.f32, D, E, probs);
  orc_moe_topk(probs, E, (int)m->top_k, ids, w);
  for (int64_t o = 0; o < D; o++) y[o] = 0.0f;
  for (int t = 0; t < (int)(m->top_k < E ? m->top_k : E); t++) {
    int e = ids[t];
    moe_ctx c = {xin, L->gate_exps.f32 + (int64_t)e * I * D, L->up_exps.f32 + (int64_t)e * I * D,
                 L->down_exps.f32 + (int64_t)e * D * I, s->hid, y, D, I, w[t]};
    parallel_for(I, nthreads, 0, moe_gate_up_row, &c);
    parallel_for(D, nthreads, 0, moe_down_row, &c);
  }
}

/* One Session::run() (session.cpp:1048-1164) over the graph gguf.cpp:935-1209. */
static int forward(orc_state* s, int64_t token, int64_t pos, int nthreads, orc_taps* tp,
                   int want_logits) {
  orc_model* m = s->m;
  int64_t D = m->dim, hd = m->head_dim, qd = m->n_heads * hd, kvd = m->n_kv * hd;
  if (token < 0 || token >= m->tok_embd.rows) { set_err("embedding token id out of range"); return -1; }
  if (pos >= s->max_seq) { set_err("KvCache capacity exceeded"); return -1; }
  /* Embedding (transformer.cpp:61-142): one dequantized row (Path A: the row of
   * the f32-loaded table) */
  size_t erb = orc_row_bytes(m->tok_embd.type, D);
  if (m->path_a) orc_load_row_f32(m->tok_embd.type, m->tok_embd.data + token * erb, D, s->x);
  else orc_dequant_row(m->tok_embd.type, m->tok_embd.data + token * erb, D, s->x);
  if (tp && tp->hidden) memcpy(tp->hidden, s->x, (size_t)D * 4);
  for (int64_t li = 0; li < m->n_layers; li++) {
    orc_layer* L = &m->L[li];
    orc_rmsnorm(s->x, L->attn_norm.f32, s->n1, D, m->eps);
    matvec(m, &L->wq, s->n1, s->q, 0, L->wq.rows, nthreads);
    matvec(m, &L->wk, s->n1, s->k, 0, L->wk.rows, nthreads);
    matvec(m, &L->wv, s->n1, s->v, 0, L->wv.rows, nthreads);
    if (L->has_bias_q) for (int64_t i = 0; i < qd; i++) s->q[i] = s->q[i] + L->bq.f32[i];
    if (L->has_bias_k) for (int64_t i = 0; i < kvd; i++) s->k[i] = s->k[i] + L->bk.f32[i];
    if (L->has_bias_v) for (int64_t i = 0; i < kvd; i++) s->v[i] = s->v[i] + L->bv.f32[i];
    orc_rope(s->q, qd, hd, (float)pos, m->theta, m->rope_mode);
    orc_rope(s->k, kvd, hd, (float)pos, m->theta, m->rope_mode);
    float* kc = s->kc + (size_t)li * (size_t)s->max_seq * (size_t)kvd;
    float* vc = s->vc + (size_t)li * (size_t)s->max_seq * (size_t)kvd;
    if (s->kv_f16) {
      for (int64_t i = 0; i < kvd; i++) { s->k[i] = round_f16(s->k[i]); s->v[i] = round_f16(s->v[i]); }
    }
    orc_attention_decode(s->q, kc, vc, pos, s->k, s->v, s->att, (int)m->n_heads,
                         (int)m->n_kv, (int)hd);
    /* KvCache::append_layer (kv_cache.hpp:80-120): after the attention math */
    memcpy(kc + pos * kvd, s->k, (size_t)kvd * 4);
    memcpy(vc + pos * kvd, s->v, (size_t)kvd * 4);
    matvec(m, &L->wo, s->att, s->tmp, 0, L->wo.rows, nthreads);
    for (int64_t i = 0; i < D; i++) s->x[i] = s->x[i] + s->tmp[i];
    if (tp && tp->resid1) memcpy(tp->resid1 + li * D, s->x, (size_t)D * 4);
    const float* min = s->x;
    if (L->has_ffn_norm) { orc_rmsnorm(s->x, L->ffn_norm.f32, s->n1, D, m->eps); min = s->n1; }
    if (L->moe) {
      moe_ffn(s, L, min, s->eout, nthreads);
      if (L->shared) {
        int64_t I = L->up_sh.rows;
        matvec(m, &L->gate_sh, min, s->g, 0, I, nthreads);
        matvec(m, &L->up_sh, min, s->u, 0, I, nthreads);
        for (int64_t i = 0; i < I; i++) s->hid[i] = orc_silu(s->g[i]) * s->u[i];
        matvec(m, &L->down_sh, s->hid, s->tmp, 0, D, nthreads);
        for (int64_t i = 0; i < D; i++) s->eout[i] = s->eout[i] + s->tmp[i];
      }
      for (int64_t i = 0; i < D; i++) s->x[i] = s->x[i] + s->eout[i];
    } else if (L->has_ffn && !L->gelu) {
      int64_t I = L->w_up.rows;
      matvec(m, &L->w_gate, min, s->g, 0, I, nthreads);
      matvec(m, &L->w_up, min, s->u, 0, I, nthreads);
      for (int64_t i = 0; i < I; i++) s->hid[i] = orc_silu(s->g[i]) * s->u[i];
      matvec(m, &L->w_down, s->hid, s->tmp, 0, D, nthreads);
      for (int64_t i = 0; i < D; i++) s->x[i] = s->x[i] + s->tmp[i];
    } else if (L->gelu) {
      /* Dense GELU MLP (gguf.cpp:1156-1170, elementwise.cpp:57-71) */
      int64_t I = L->w_up.rows;
      matvec(m, &L->w_up, min, s->u, 0, I, nthreads);
      for (int64_t i = 0; i < I; i++) {
        float v = s->u[i];
        float uu = 0.7978845608f * (v + 0.044715f * v * v * v);
        s->hid[i] = 0.5f * v * (1.0f + tanhf(uu));
      }
      matvec(m, &L->w_down, s->hid, s->tmp, 0, D, nthreads);
      for (int64_t i = 0; i < D; i++) s->x[i] = s->x[i] + s->tmp[i];
    }
    if (tp && tp->resid2) memcpy(tp->resid2 + li * D, s->x, (size_t)D * 4);
  }
  if (!want_logits) return 0;
  const float* fin = s->x;
  if (m->has_out_norm) { orc_rmsnorm(s->x, m->out_norm.f32, s->n1, D, m->eps); fin = s->n1; }
  if (tp && tp->normed) memcpy(tp->normed, fin, (size_t)D * 4);
  matvec(m, &m->output, fin, s->logits, 0, m->vocab, nthreads);
  orc_softmax(s->logits, s->probs, m->vocab);
  if (tp && tp->logits) memcpy(tp->logits, s->logits, (size_t)m->vocab * 4);
  if (tp && tp->probs) memcpy(tp->probs, s->probs, (size_t)m->vocab * 4);
  return 0;
}

/* ---------------------------------------------------------- layer-major prompt */

/* Y[i][j] = W_j . X_i for M rows of X at once, in tiles of 4 weight rows x 16
 * rows of X: the 4 weight rows are dequantized once per tile, X is held
 * transposed in groups of 16 rows ([group][k][16]), and the 64 sums of a tile
 * advance together over k in 4-wide vectors. Each vector lane is one (row of X,
 * weight row) sum taken left to right as s = s + x[k] * w[k] (a product rounded
 * to f32, then the add: no contraction), the order of qg_row's loop, so every
 * output equals the M = 1 call's bit for bit. Path A / F32 / F16 weights:
 * dot_tiled64 per (row of X, weight row), as mv_row_a. */
typedef float orc_v4 __attribute__((vector_size(16)));

typedef struct {
  const orc_model* m;
  const orc_w* w;
  const float* AT;  /* [ceil(M/16)][K][16] */
  const float* A;   /* [M][K] (f32-weight path) */
  int64_t M, K, N;
  float* Y;         /* [M][N] */
} mm_ctx;

#define MM_ROWS 4
#define MM_COLS 16

static void mm_tile(void* v, int64_t tile, float* rows) {
  mm_ctx* c = (mm_ctx*)v;
  const orc_w* w = c->w;
  const int64_t K = c->K;
  const int64_t j0 = tile * MM_ROWS;
  const int nr = (int)(c->N - j0 < MM_ROWS ? c->N - j0 : MM_ROWS);
  if (c->m->path_a || w->type == ORC_F32 || w->type == ORC_F16) {
    for (int r = 0; r < nr; r++) {
      const float* wr = w->f32 + (j0 + r) * w->cols;
      for (int64_t i = 0; i < c->M; i++) c->Y[i * c->N + j0 + r] = dot_tiled64(c->A + i * K, wr, K);
    }
    return;
  }
  size_t rb = orc_row_bytes(w->type, w->cols);
  for (int r = 0; r < MM_ROWS; r++) {
    if (r < nr) {
      if (orc_dequant_row(w->type, w->data + (size_t)(j0 + r) * rb, K, rows + r * K) != 0) return;
    } else {
      memset(rows + r * K, 0, (size_t)K * 4);
    }
  }
  for (int64_t g = 0; g * MM_COLS < c->M; g++) {
    const orc_v4* at = (const orc_v4*)(c->AT + g * K * MM_COLS);
    orc_v4 acc[MM_ROWS][MM_COLS / 4];
    for (int r = 0; r < MM_ROWS; r++)
      for (int q = 0; q < MM_COLS / 4; q++) acc[r][q] = (orc_v4){0.0f, 0.0f, 0.0f, 0.0f};
    for (int64_t k = 0; k < K; k++) {
      const orc_v4 a0 = at[k * 4 + 0], a1 = at[k * 4 + 1], a2 = at[k * 4 + 2], a3 = at[k * 4 + 3];
      for (int r = 0; r < MM_ROWS; r++) {
        const float wv = rows[r * K + k];
        const orc_v4 wb = {wv, wv, wv, wv};
        acc[r][0] = acc[r][0] + a0 * wb;
        acc[r][1] = acc[r][1] + a1 * wb;
        acc[r][2] = acc[r][2] + a2 * wb;
        acc[r][3] = acc[r][3] + a3 * wb;
      }
    }
    for (int r = 0; r < nr; r++)
      for (int ii = 0; ii < MM_COLS && g * MM_COLS + ii < c->M; ii++)
        c->Y[(g * MM_COLS + ii) * c->N + j0 + r] = acc[r][ii / 4][ii % 4];
  }
}

static void matmat(const orc_model* m, const orc_w* w, const float* X, int64_t M, float* Y,
                   float* at_buf, int nthreads) {
  int64_t K = w->cols;
  if (!(m->path_a || w->type == ORC_F32 || w->type == ORC_F16)) {
    for (int64_t g = 0; g * MM_COLS < M; g++)
      for (int64_t k = 0; k < K; k++)
        for (int ii = 0; ii < MM_COLS; ii++) {
          int64_t i = g * MM_COLS + ii;
          at_buf[(g * K + k) * MM_COLS + ii] = i < M ? X[i * K + k] : 0.0f;
        }
  } else if (!w->f32) {
    return;
  }
  mm_ctx c = {m, w, at_buf, X, M, K, w->rows, Y};
  parallel_for((w->rows + MM_ROWS - 1) / MM_ROWS, nthreads, (size_t)(MM_ROWS * K), mm_tile, &c);
}

typedef struct {
  const float *Q, *K, *V, *kc, *vc;
  float* ATT;
  int64_t p0, qd, kvd;
  int nh, nkv, hd;
} att_ctx;

static void att_row(void* v, int64_t b, float* scratch) {
  (void)scratch;
  att_ctx* c = (att_ctx*)v;
  orc_attention_decode(c->Q + b * c->qd, c->kc, c->vc, c->p0 + b, c->K + b * c->kvd,
                       c->V + b * c->kvd, c->ATT + b * c->qd, c->nh, c->nkv, c->hd);
}

/* Prompt tokens at positions p0 .. p0+nb-1 run layer by layer: per layer the
 * block's rows go through each projection together (matmat), and the block's K/V
 * are appended before its attentions, where token b reads positions < p0+b from
 * the cache and its own K/V, as forward() does. Every value equals what nb calls of
 * forward() (without the LM head, whose values are not read for these tokens)
 * give, bit for bit; tests/test_oracle_prompt.py checks that on every variant. */
static int forward_block(orc_state* s, const int64_t* tokens, int64_t nb, int64_t p0,
                         int nthreads) {
  orc_model* m = s->m;
  int64_t D = m->dim, hd = m->head_dim, qd = m->n_heads * hd, kvd = m->n_kv * hd;
  int64_t ff = m->ffn > 0 ? m->ffn : 4 * m->dim;
  for (int64_t li = 0; li < m->n_layers; li++) {
    const orc_layer* L = &m->L[li];
    if (L->has_ffn && L->w_up.rows > ff) ff = L->w_up.rows;
    if (L->shared && L->up_sh.rows > ff) ff = L->up_sh.rows;
  }
  int64_t kmax = D > qd ? D : qd;
  if (ff > kmax) kmax = ff;
  if (p0 + nb > s->max_seq) { set_err("KvCache capacity exceeded"); return -1; }
  size_t nbz = (size_t)nb;
  float* X = (float*)malloc(nbz * (size_t)D * 4);
  float* N1 = (float*)malloc(nbz * (size_t)D * 4);
  float* Q = (float*)malloc(nbz * (size_t)qd * 4);
  float* K = (float*)malloc(nbz * (size_t)kvd * 4);
  float* V = (float*)malloc(nbz * (size_t)kvd * 4);
  float* ATT = (float*)malloc(nbz * (size_t)qd * 4);
  float* T = (float*)malloc(nbz * (size_t)D * 4);
  float* G = (float*)malloc(nbz * (size_t)ff * 4);
  float* U = (float*)malloc(nbz * (size_t)ff * 4);
  float* H = (float*)malloc(nbz * (size_t)ff * 4);
  float* AT = (float*)malloc(((nbz + MM_COLS - 1) / MM_COLS * MM_COLS) * (size_t)kmax * 4);
  int rc = -1;
  if (!X || !N1 || !Q || !K || !V || !ATT || !T || !G || !U || !H || !AT) { set_err("oom"); goto done; }
  size_t erb = orc_row_bytes(m->tok_embd.type, D);
  for (int64_t b = 0; b < nb; b++) {
    int64_t token = tokens[b];
    if (token < 0 || token >= m->tok_embd.rows) { set_err("embedding token id out of range"); goto done; }
    if (m->path_a) orc_load_row_f32(m->tok_embd.type, m->tok_embd.data + token * erb, D, X + b * D);
    else orc_dequant_row(m->tok_embd.type, m->tok_embd.data + token * erb, D, X + b * D);
  }
  for (int64_t li = 0; li < m->n_layers; li++) {
    orc_layer* L = &m->L[li];
    for (int64_t b = 0; b < nb; b++) orc_rmsnorm(X + b * D, L->attn_norm.f32, N1 + b * D, D, m->eps);
    matmat(m, &L->wq, N1, nb, Q, AT, nthreads);
    matmat(m, &L->wk, N1, nb, K, AT, nthreads);
    matmat(m, &L->wv, N1, nb, V, AT, nthreads);
    float* kc = s->kc + (size_t)li * (size_t)s->max_seq * (size_t)kvd;
    float* vc = s->vc + (size_t)li * (size_t)s->max_seq * (size_t)kvd;
    for (int64_t b = 0; b < nb; b++) {
      float *q = Q + b * qd, *k = K + b * kvd, *v = V + b * kvd;
      if (L->has_bias_q) for (int64_t i = 0; i < qd; i++) q[i] = q[i] + L->bq.f32[i];
      if (L->has_bias_k) for (int64_t i = 0; i < kvd; i++) k[i] = k[i] + L->bk.f32[i];
      if (L->has_bias_v) for (int64_t i = 0; i < kvd; i++) v[i] = v[i] + L->bv.f32[i];
      orc_rope(q, qd, hd, (float)(p0 + b), m->theta, m->rope_mode);
      orc_rope(k, kvd, hd, (float)(p0 + b), m->theta, m->rope_mode);
      if (s->kv_f16) {
        for (int64_t i = 0; i < kvd; i++) { k[i] = round_f16(k[i]); v[i] = round_f16(v[i]); }
      }
      memcpy(kc + (p0 + b) * kvd, k, (size_t)kvd * 4);
      memcpy(vc + (p0 + b) * kvd, v, (size_t)kvd * 4);
    }
    att_ctx ac = {Q, K, V, kc, vc, ATT, p0, qd, kvd, (int)m->n_heads, (int)m->n_kv, (int)hd};
    parallel_for(nb, nthreads, 0, att_row, &ac);
    matmat(m, &L->wo, ATT, nb, T, AT, nthreads);
    for (int64_t i = 0; i < nb * D; i++) X[i] = X[i] + T[i];
    const float* min = X;
    if (L->has_ffn_norm) {
      for (int64_t b = 0; b < nb; b++) orc_rmsnorm(X + b * D, L->ffn_norm.f32, N1 + b * D, D, m->eps);
      min = N1;
    }
    if (L->moe) {
      for (int64_t b = 0; b < nb; b++) {
        moe_ffn(s, L, min + b * D, s->eout, nthreads);
        if (L->shared) {
          int64_t I = L->up_sh.rows;
          matvec(m, &L->gate_sh, min + b * D, s->g, 0, I, nthreads);
          matvec(m, &L->up_sh, min + b * D, s->u, 0, I, nthreads);
          for (int64_t i = 0; i < I; i++) s->hid[i] = orc_silu(s->g[i]) * s->u[i];
          matvec(m, &L->down_sh, s->hid, s->tmp, 0, D, nthreads);
          for (int64_t i = 0; i < D; i++) s->eout[i] = s->eout[i] + s->tmp[i];
        }
        for (int64_t i = 0; i < D; i++) X[b * D + i] = X[b * D + i] + s->eout[i];
      }
    } else if (L->has_ffn && !L->gelu) {
      int64_t I = L->w_up.rows;
      matmat(m, &L->w_gate, min, nb, G, AT, nthreads);
      matmat(m, &L->w_up, min, nb, U, AT, nthreads);
      for (int64_t i = 0; i < nb * I; i++) H[i] = orc_silu(G[i]) * U[i];
      matmat(m, &L->w_down, H, nb, T, AT, nthreads);
      for (int64_t i = 0; i < nb * D; i++) X[i] = X[i] + T[i];
    } else if (L->gelu) {
      int64_t I = L->w_up.rows;
      matmat(m, &L->w_up, min, nb, U, AT, nthreads);
      for (int64_t i = 0; i < nb * I; i++) {
        float v = U[i];
        float uu = 0.7978845608f * (v + 0.044715f * v * v * v);
        H[i] = 0.5f * v * (1.0f + tanhf(uu));
      }
      matmat(m, &L->w_down, H, nb, T, AT, nthreads);
      for (int64_t i = 0; i < nb * D; i++) X[i] = X[i] + T[i];
    }
  }
  rc = 0;
done:
  free(X); free(N1); free(Q); free(K); free(V); free(ATT); free(T); free(G); free(U); free(H); free(AT);
  return rc;
}

int orc_generate(orc_model* m, const int64_t* prompt, int64_t n_prompt, int64_t max_new,
                 int kv_f16, int nthreads, int64_t* out, int64_t* out_n, orc_taps* taps) {
  return orc_generate_ex(m, prompt, n_prompt, max_new, kv_f16, nthreads, 0, out, out_n, taps);
}

int orc_generate_ex(orc_model* m, const int64_t* prompt, int64_t n_prompt, int64_t max_new,
                    int kv_f16, int nthreads, int64_t prompt_block, int64_t* out, int64_t* out_n,
                    orc_taps* taps) {
  if (!m || !out || !out_n) { set_err("null args"); return -1; }
  if (n_prompt <= 0) { set_err("prompt_tokens empty"); return -1; }
  if (max_new < 0) { set_err("max_new_tokens < 0"); return -1; }
  int64_t total = n_prompt + max_new;
  int64_t max_ctx = m->ctx;
  if (max_ctx > 0 && (n_prompt > max_ctx || total > max_ctx)) {
    set_err("prompt+max_new_tokens exceeds max_context");
    return -1;
  }
  int64_t kv_max = max_ctx > 0 ? max_ctx : (total > n_prompt + 1 ? total : n_prompt + 1);
  orc_state s;
  if (state_init(&s, m, kv_max, kv_f16)) return -1;
  int64_t n = 0, pos = 0;
  /* prompt_block > 0: prompt tokens 0 .. n_prompt-2 layer-major in blocks of that
   * many tokens (same values as the token steps below) */
  if (prompt_block > 0) {
    while (pos < n_prompt - 1) {
      int64_t nb = n_prompt - 1 - pos < prompt_block ? n_prompt - 1 - pos : prompt_block;
      if (forward_block(&s, prompt + pos, nb, pos, nthreads)) { state_free(&s); return -1; }
      for (int64_t b = 0; b < nb; b++) out[n++] = prompt[pos + b];
      pos += nb;
    }
  }
  /* prefill: one run() per prompt token (session.cpp:1006-1016) */
  for (int64_t i = pos; i < n_prompt; i++) {
    int last = (i == n_prompt - 1);
    /* the LM head of the earlier prompt tokens is computed by the reference and
     * never read; skipping it here changes no value that is read */
    if (forward(&s, prompt[i], pos, nthreads, last ? taps : NULL, last)) { state_free(&s); return -1; }
    pos++;
    out[n++] = prompt[i];
  }
  /* decode: argmax over probs, strict '>' (session.cpp:1018-1044) */
  for (int64_t t = 0; t < max_new; t++) {
    int64_t next = orc_argmax(s.probs, m->vocab);
    out[n++] = next;
    if (t + 1 >= max_new) break;
    if (forward(&s, next, pos, nthreads, taps, 1)) { state_free(&s); return -1; }
    pos++;
  }
  *out_n = n;
  state_free(&s);
  return 0;
}

static double now_s(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

double orc_time_decode_window(orc_model* m, int64_t start_pos, int64_t n_steps, int nthreads) {
  int64_t kv_max = start_pos + n_steps + 1;
  orc_state s;
  if (state_init(&s, m, kv_max, 0)) return -1.0;
  /* deterministic past K/V (values in [-0.5,0.5)) standing in for a prefilled cache */
  int64_t kvd = m->n_kv * m->head_dim;
  for (int64_t li = 0; li < m->n_layers; li++)
    for (int64_t j = 0; j < start_pos * kvd; j++) {
      size_t idx = (size_t)li * (size_t)kv_max * (size_t)kvd + (size_t)j;
      uint32_t h = (uint32_t)(j * 2654435761u + (uint64_t)li * 40503u);
      s.kc[idx] = (float)(h & 0xffff) / 65536.0f - 0.5f;
      s.vc[idx] = (float)((h >> 16) & 0xffff) / 65536.0f - 0.5f;
    }
  double t0 = now_s();
  int64_t tok = 1;
  for (int64_t i = 0; i < n_steps; i++) {
    if (forward(&s, tok, start_pos + i, nthreads, NULL, 1)) { state_free(&s); return -1.0; }
    tok = orc_argmax(s.probs, m->vocab);
  }
  double dt = now_s() - t0;
  state_free(&s);
  return dt;
}
