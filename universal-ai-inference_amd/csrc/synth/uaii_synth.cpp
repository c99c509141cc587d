// uaii_synth.cpp — seeded synthetic GGUF decoder writer. See uaii_synth.h.
//
// Quantizers are this build's own round-to-nearest block encoders for the ggml
// block layouts the reference decodes (libs/uaii-quant/src/gguf_dequant.cpp).
// Every encoder quantizes against the scale exactly as the decoder will rebuild
// it (f16-rounded super-scales, f32 products), so a value's round trip error is
// at most half a quantization step.

#include "uaii_synth.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

namespace {

thread_local std::string g_err;

std::uint64_t splitmix64(std::uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

float half_to_float(std::uint16_t h) {
  const std::uint32_t sign = static_cast<std::uint32_t>(h & 0x8000u) << 16;
  std::uint32_t e = (h >> 10) & 31u, m = h & 1023u, bits;
  if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else {
      int sh = 0;
      while (!(m & 0x400u)) { m <<= 1; ++sh; }
      bits = sign | (static_cast<std::uint32_t>(113 - sh) << 23) | ((m & 1023u) << 13);
    }
  } else if (e == 31) {
    bits = sign | 0x7f800000u | (m << 13);
  } else {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

std::uint16_t to_half(float f) {
  std::uint32_t b;
  std::memcpy(&b, &f, 4);
  const std::uint32_t sign = (b >> 16) & 0x8000u;
  const std::uint32_t ex = (b >> 23) & 255u;
  const std::uint32_t mant = b & 0x7fffffu;
  if (ex == 255) return static_cast<std::uint16_t>(sign | 0x7c00u | (mant ? 0x200u : 0u));
  const int e = static_cast<int>(ex) - 127 + 15;
  if (e >= 31) return static_cast<std::uint16_t>(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return static_cast<std::uint16_t>(sign);
    const std::uint32_t mm = mant | 0x800000u;
    const int shift = 14 - e;
    std::uint32_t hm = mm >> shift;
    const std::uint32_t rem = mm & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (hm & 1u))) ++hm;
    return static_cast<std::uint16_t>(sign | hm);
  }
  std::uint32_t hv = sign | (static_cast<std::uint32_t>(e) << 10) | (mant >> 13);
  const std::uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (hv & 1u))) ++hv;
  return static_cast<std::uint16_t>(hv);
}

void put16(std::uint8_t* p, std::uint16_t v) {
  p[0] = static_cast<std::uint8_t>(v & 0xff);
  p[1] = static_cast<std::uint8_t>(v >> 8);
}

// f16-rounded scale and its decoded value (what the decoder will use).
float stored_scale(float s, std::uint8_t* dst) {
  const std::uint16_t h = to_half(s);
  put16(dst, h);
  return half_to_float(h);
}

int clampi(long v, int lo, int hi) { return static_cast<int>(std::min<long>(hi, std::max<long>(lo, v))); }

// Element of largest magnitude, keeping its sign.
float signed_absmax(const float* x, int n) {
  float best = 0.0f;
  for (int i = 0; i < n; ++i) if (std::fabs(x[i]) > std::fabs(best)) best = x[i];
  return best;
}

// ---- 32-element blocks -------------------------------------------------------

void q4_0(const float* x, std::uint8_t* b) {
  const float d = stored_scale(signed_absmax(x, 32) / -8.0f, b);
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  for (int j = 0; j < 16; ++j) {
    const int lo = clampi(std::lround(x[j] * id) + 8, 0, 15);
    const int hi = clampi(std::lround(x[j + 16] * id) + 8, 0, 15);
    b[2 + j] = static_cast<std::uint8_t>(lo | (hi << 4));
  }
}

void q4_1(const float* x, std::uint8_t* b) {
  float mn = x[0], mx = x[0];
  for (int i = 1; i < 32; ++i) { mn = std::min(mn, x[i]); mx = std::max(mx, x[i]); }
  const float d = stored_scale((mx - mn) / 15.0f, b);
  const float m = stored_scale(mn, b + 2);
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  for (int j = 0; j < 16; ++j) {
    const int lo = clampi(std::lround((x[j] - m) * id), 0, 15);
    const int hi = clampi(std::lround((x[j + 16] - m) * id), 0, 15);
    b[4 + j] = static_cast<std::uint8_t>(lo | (hi << 4));
  }
}

void q5_0(const float* x, std::uint8_t* b) {
  const float d = stored_scale(signed_absmax(x, 32) / -16.0f, b);
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  std::uint32_t qh = 0;
  for (int j = 0; j < 16; ++j) {
    const int lo = clampi(std::lround(x[j] * id) + 16, 0, 31);
    const int hi = clampi(std::lround(x[j + 16] * id) + 16, 0, 31);
    b[6 + j] = static_cast<std::uint8_t>((lo & 15) | ((hi & 15) << 4));
    qh |= static_cast<std::uint32_t>(lo >> 4) << j;
    qh |= static_cast<std::uint32_t>(hi >> 4) << (j + 16);
  }
  for (int k = 0; k < 4; ++k) b[2 + k] = static_cast<std::uint8_t>(qh >> (8 * k));
}

void q5_1(const float* x, std::uint8_t* b) {
  float mn = x[0], mx = x[0];
  for (int i = 1; i < 32; ++i) { mn = std::min(mn, x[i]); mx = std::max(mx, x[i]); }
  const float d = stored_scale((mx - mn) / 31.0f, b);
  const float m = stored_scale(mn, b + 2);
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  std::uint32_t qh = 0;
  for (int j = 0; j < 16; ++j) {
    const int lo = clampi(std::lround((x[j] - m) * id), 0, 31);
    const int hi = clampi(std::lround((x[j + 16] - m) * id), 0, 31);
    b[8 + j] = static_cast<std::uint8_t>((lo & 15) | ((hi & 15) << 4));
    qh |= static_cast<std::uint32_t>(lo >> 4) << j;
    qh |= static_cast<std::uint32_t>(hi >> 4) << (j + 16);
  }
  for (int k = 0; k < 4; ++k) b[4 + k] = static_cast<std::uint8_t>(qh >> (8 * k));
}

void q8_0(const float* x, std::uint8_t* b) {
  float amax = 0.0f;
  for (int i = 0; i < 32; ++i) amax = std::max(amax, std::fabs(x[i]));
  const float d = stored_scale(amax / 127.0f, b);
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  for (int j = 0; j < 32; ++j) {
    b[2 + j] = static_cast<std::uint8_t>(static_cast<std::int8_t>(clampi(std::lround(x[j] * id), -127, 127)));
  }
}

// ---- 256-element super-blocks --------------------------------------------------

// Asymmetric sub-block scales for Q4_K/Q5_K/Q2_K: per sub-block a positive step
// and a non-negative offset, quantized against f16 super-scales d and dmin.
struct Affine {
  std::vector<float> step, off;
};

Affine sub_affine(const float* x, int nsub, int len, int qmax) {
  Affine a;
  a.step.resize(nsub);
  a.off.resize(nsub);
  for (int j = 0; j < nsub; ++j) {
    float mn = 0.0f, mx = x[j * len];
    for (int i = 0; i < len; ++i) { mn = std::min(mn, x[j * len + i]); mx = std::max(mx, x[j * len + i]); }
    a.step[j] = (mx - mn) / static_cast<float>(qmax);
    a.off[j] = -mn;
  }
  return a;
}

// Pack eight 6-bit (scale, min) pairs into the 12-byte K-quant field, the inverse
// of the decoder's unpack (gguf_dequant.cpp:107-115).
void pack_k_scales(const int* sc, const int* mn, std::uint8_t* s) {
  for (int j = 0; j < 4; ++j) {
    s[j] = static_cast<std::uint8_t>((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
    s[j + 4] = static_cast<std::uint8_t>((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
    s[j + 8] = static_cast<std::uint8_t>((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
  }
}

// Shared Q4_K / Q5_K encoder; bits = 4 or 5. Writes d, dmin, scales; returns the
// 256 integer levels in q.
void k_affine(const float* x, int bits, std::uint8_t* hdr, int* q) {
  const int qmax = (1 << bits) - 1;
  Affine a = sub_affine(x, 8, 32, qmax);
  const float smax = *std::max_element(a.step.begin(), a.step.end());
  const float omax = *std::max_element(a.off.begin(), a.off.end());
  const float d = stored_scale(smax / 63.0f, hdr);
  const float dmin = stored_scale(omax / 63.0f, hdr + 2);
  int sc[8], mn[8];
  for (int j = 0; j < 8; ++j) {
    sc[j] = d > 0.0f ? clampi(std::lround(a.step[j] / d), 0, 63) : 0;
    mn[j] = dmin > 0.0f ? clampi(std::lround(a.off[j] / dmin), 0, 63) : 0;
  }
  pack_k_scales(sc, mn, hdr + 4);
  for (int j = 0; j < 8; ++j) {
    const float d1 = d * static_cast<float>(sc[j]);
    const float m1 = dmin * static_cast<float>(mn[j]);
    for (int i = 0; i < 32; ++i) {
      const float v = x[32 * j + i];
      q[32 * j + i] = d1 > 0.0f ? clampi(std::lround((v + m1) / d1), 0, qmax) : 0;
    }
  }
}

void q4_k(const float* x, std::uint8_t* b) {
  int q[256];
  k_affine(x, 4, b, q);
  std::uint8_t* qs = b + 16;
  for (int c = 0; c < 4; ++c)
    for (int l = 0; l < 32; ++l)
      qs[32 * c + l] = static_cast<std::uint8_t>(q[64 * c + l] | (q[64 * c + 32 + l] << 4));
}

void q5_k(const float* x, std::uint8_t* b) {
  int q[256];
  k_affine(x, 5, b, q);
  std::uint8_t* qh = b + 16;
  std::uint8_t* qs = b + 48;
  std::memset(qh, 0, 32);
  for (int c = 0; c < 4; ++c) {
    for (int l = 0; l < 32; ++l) {
      const int lo = q[64 * c + l], hi = q[64 * c + 32 + l];
      qs[32 * c + l] = static_cast<std::uint8_t>((lo & 15) | ((hi & 15) << 4));
      qh[l] |= static_cast<std::uint8_t>(((lo >> 4) & 1) << (2 * c));
      qh[l] |= static_cast<std::uint8_t>(((hi >> 4) & 1) << (2 * c + 1));
    }
  }
}

// Element e of a 256-block in the Q2_K/Q3_K bit-plane layout: half h = e/128,
// plane p = (e%128)/32, group g = (e%32)/16, lane l = e%16 -> byte 32h+16g+l,
// shift 2p; sub-block scale index e/16.
inline int plane_byte(int e) { return 32 * (e / 128) + 16 * ((e % 32) / 16) + (e % 16); }
inline int plane_shift(int e) { return 2 * ((e % 128) / 32); }

void q2_k(const float* x, std::uint8_t* b) {
  Affine a = sub_affine(x, 16, 16, 3);
  const float smax = *std::max_element(a.step.begin(), a.step.end());
  const float omax = *std::max_element(a.off.begin(), a.off.end());
  const float d = stored_scale(smax / 15.0f, b + 80);
  const float dmin = stored_scale(omax / 15.0f, b + 82);
  std::memset(b, 0, 80);
  for (int j = 0; j < 16; ++j) {
    const int sc = d > 0.0f ? clampi(std::lround(a.step[j] / d), 0, 15) : 0;
    const int mn = dmin > 0.0f ? clampi(std::lround(a.off[j] / dmin), 0, 15) : 0;
    b[j] = static_cast<std::uint8_t>(sc | (mn << 4));
    const float dl = d * static_cast<float>(sc), ml = dmin * static_cast<float>(mn);
    for (int i = 0; i < 16; ++i) {
      const int e = 16 * j + i;
      const int q = dl > 0.0f ? clampi(std::lround((x[e] + ml) / dl), 0, 3) : 0;
      b[16 + plane_byte(e)] |= static_cast<std::uint8_t>(q << plane_shift(e));
    }
  }
}

void q3_k(const float* x, std::uint8_t* b) {
  float scale[16];
  for (int j = 0; j < 16; ++j) scale[j] = signed_absmax(x + 16 * j, 16) / -4.0f;
  float smax = 0.0f;
  for (int j = 0; j < 16; ++j) smax = std::max(smax, std::fabs(scale[j]));
  const float d = stored_scale(smax / 31.0f, b + 108);
  std::memset(b, 0, 108);
  std::uint8_t* hm = b;
  std::uint8_t* qs = b + 32;
  std::uint8_t* s12 = b + 96;
  for (int j = 0; j < 16; ++j) {
    const int sc = d > 0.0f ? clampi(std::lround(scale[j] / d), -32, 31) : 0;
    const int u = sc + 32;  // 6-bit stored value
    if (j < 8) s12[j] |= static_cast<std::uint8_t>(u & 15);
    else s12[j - 8] |= static_cast<std::uint8_t>((u & 15) << 4);
    s12[8 + (j % 4)] |= static_cast<std::uint8_t>(((u >> 4) & 3) << (2 * (j / 4)));
    const float dl = d * static_cast<float>(sc);
    for (int i = 0; i < 16; ++i) {
      const int e = 16 * j + i;
      const int q = dl != 0.0f ? clampi(std::lround(x[e] / dl), -4, 3) : 0;
      const int q2 = q >= 0 ? q : q + 4;
      qs[plane_byte(e)] |= static_cast<std::uint8_t>(q2 << plane_shift(e));
      if (q >= 0) hm[16 * ((e % 32) / 16) + (e % 16)] |= static_cast<std::uint8_t>(1u << (4 * (e / 128) + (e % 128) / 32));
    }
  }
}

void q6_k(const float* x, std::uint8_t* b) {
  float scale[16];
  for (int j = 0; j < 16; ++j) scale[j] = signed_absmax(x + 16 * j, 16) / -32.0f;
  float smax = 0.0f;
  for (int j = 0; j < 16; ++j) smax = std::max(smax, std::fabs(scale[j]));
  const float d = stored_scale(smax / 127.0f, b + 208);
  std::memset(b, 0, 208);
  std::uint8_t* ql = b;
  std::uint8_t* qh = b + 128;
  auto* sc8 = reinterpret_cast<std::int8_t*>(b + 192);
  for (int j = 0; j < 16; ++j) {
    const int sc = d > 0.0f ? clampi(std::lround(scale[j] / d), -128, 127) : 0;
    sc8[j] = static_cast<std::int8_t>(sc);
    const float dl = d * static_cast<float>(sc);
    for (int i = 0; i < 16; ++i) {
      const int e = 16 * j + i;  // 0..255
      const int h = e / 128, k = e % 128;
      const int q = (dl != 0.0f ? clampi(std::lround(x[e] / dl), -32, 31) : 0) + 32;
      std::uint8_t* qlh = ql + 64 * h;
      std::uint8_t* qhh = qh + 32 * h;
      if (k < 64) qlh[k] |= static_cast<std::uint8_t>(q & 15);
      else qlh[k - 64] |= static_cast<std::uint8_t>((q & 15) << 4);
      qhh[k % 32] |= static_cast<std::uint8_t>(((q >> 4) & 3) << (2 * (k / 32)));
    }
  }
}

int block_elems(int t) {
  switch (t) {
    case 0: case 1: return 1;
    case 2: case 3: case 6: case 7: case 8: return 32;
    case 10: case 11: case 12: case 13: case 14: return 256;
    default: return 0;
  }
}

int block_bytes(int t) {
  switch (t) {
    case 0: return 4; case 1: return 2; case 2: return 18; case 3: return 20; case 6: return 22;
    case 7: return 24; case 8: return 34; case 10: return 84; case 11: return 110;
    case 12: return 144; case 13: return 176; case 14: return 210;
    default: return 0;
  }
}

std::int64_t row_bytes(int t, std::int64_t n) {
  const int be = block_elems(t);
  return be ? (n / be) * block_bytes(t) : 0;
}

// ---- GGUF writing -------------------------------------------------------------

struct TensorSpec {
  std::string name;
  int type;
  std::vector<std::uint64_t> ne;  // GGUF order: ne[0] = row length
  int fill;                       // 0 normal(std), 1 ones, 2 normal(router_std)
  std::uint64_t offset = 0;
  std::int64_t nbytes = 0;
};

struct Writer {
  std::vector<std::uint8_t> buf;
  void raw(const void* p, std::size_t n) {
    const auto* c = static_cast<const std::uint8_t*>(p);
    buf.insert(buf.end(), c, c + n);
  }
  void u32(std::uint32_t v) { raw(&v, 4); }
  void u64(std::uint64_t v) { raw(&v, 8); }
  void str(const std::string& s) { u64(s.size()); raw(s.data(), s.size()); }
  void kv_u32(const std::string& k, std::uint32_t v) { str(k); u32(4); u32(v); }
  void kv_f32(const std::string& k, float v) { str(k); u32(6); raw(&v, 4); }
  void kv_str(const std::string& k, const std::string& v) { str(k); u32(8); str(v); }
};

}  // namespace

extern "C" {

const char* uaii_synth_last_error(void) { return g_err.c_str(); }

uint16_t uaii_synth_f32_to_f16(float f) { return to_half(f); }

void uaii_synth_normals(uint64_t seed, uint64_t tensor, uint64_t i0, int64_t n, float std,
                        float* out) {
  const std::uint64_t key = splitmix64(seed + 0x632BE59BD9B4E019ull * (tensor + 1));
  const double two_pi = 6.283185307179586476925286766559;
  for (int64_t k = 0; k < n; ++k) {
    const std::uint64_t i = i0 + static_cast<std::uint64_t>(k);
    const std::uint64_t a = splitmix64(key + 2 * i), b = splitmix64(key + 2 * i + 1);
    const double u1 = static_cast<double>((a >> 11) + 1) * 0x1.0p-53;
    const double u2 = static_cast<double>(b >> 11) * 0x1.0p-53;
    const double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(two_pi * u2);
    out[k] = static_cast<float>(z * static_cast<double>(std));
  }
}

int64_t uaii_synth_quantize_row(int type, const float* x, int64_t n, uint8_t* out) {
  const int be = block_elems(type);
  if (be == 0 || n % be) return -1;
  const int bb = block_bytes(type);
  for (int64_t i = 0; i < n / be; ++i) {
    const float* xb = x + i * be;
    std::uint8_t* ob = out + i * bb;
    switch (type) {
      case 0: std::memcpy(ob, xb, 4); break;
      case 1: put16(ob, to_half(xb[0])); break;
      case 2: q4_0(xb, ob); break;
      case 3: q4_1(xb, ob); break;
      case 6: q5_0(xb, ob); break;
      case 7: q5_1(xb, ob); break;
      case 8: q8_0(xb, ob); break;
      case 10: q2_k(xb, ob); break;
      case 11: q3_k(xb, ob); break;
      case 12: q4_k(xb, ob); break;
      case 13: q5_k(xb, ob); break;
      case 14: q6_k(xb, ob); break;
      default: return -1;
    }
  }
  return (n / be) * bb;
}

int uaii_synth_write_gguf(const char* path, const uaii_synth_config* c, int nthreads) {
  if (path == nullptr || c == nullptr) { g_err = "null args"; return -1; }
  if (c->n_layers < 0 || c->dim <= 0 || c->n_heads <= 0 || c->vocab <= 0) {
    g_err = "invalid config";
    return -1;
  }
  const std::int64_t hd = c->head_dim > 0 ? c->head_dim : c->dim / c->n_heads;
  const std::int64_t nkv = c->n_kv_heads > 0 ? c->n_kv_heads : c->n_heads;
  const std::int64_t qd = c->n_heads * hd, kvd = nkv * hd;
  auto pick = [&](int t) { return t >= 0 ? t : c->type_default; };
  const auto D = static_cast<std::uint64_t>(c->dim), Q = static_cast<std::uint64_t>(qd);
  const auto KV = static_cast<std::uint64_t>(kvd), F = static_cast<std::uint64_t>(c->ffn);
  const auto V = static_cast<std::uint64_t>(c->vocab), E = static_cast<std::uint64_t>(c->n_experts);

  std::vector<TensorSpec> ts;
  ts.push_back({"token_embd.weight", pick(c->type_embd), {D, V}, 0});
  for (std::int64_t l = 0; l < c->n_layers; ++l) {
    const std::string p = "blk." + std::to_string(l) + ".";
    ts.push_back({p + "attn_norm.weight", 0, {D}, 1});
    ts.push_back({p + "attn_q.weight", c->type_default, {D, Q}, 0});
    ts.push_back({p + "attn_k.weight", c->type_default, {D, KV}, 0});
    ts.push_back({p + "attn_v.weight", pick(c->type_attn_v), {D, KV}, 0});
    if (c->qkv_bias) {
      ts.push_back({p + "attn_q.bias", 0, {Q}, 0});
      ts.push_back({p + "attn_k.bias", 0, {KV}, 0});
      ts.push_back({p + "attn_v.bias", 0, {KV}, 0});
    }
    ts.push_back({p + "attn_output.weight", c->type_default, {Q, D}, 0});
    ts.push_back({p + "ffn_norm.weight", 0, {D}, 1});
    if (c->n_experts > 0) {
      ts.push_back({p + "ffn_gate_inp.weight", 0, {D, E}, 2});
      ts.push_back({p + "ffn_gate_exps.weight", c->type_default, {D, F, E}, 0});
      ts.push_back({p + "ffn_up_exps.weight", c->type_default, {D, F, E}, 0});
      ts.push_back({p + "ffn_down_exps.weight", pick(c->type_ffn_down), {F, D, E}, 0});
      if (c->shared_ffn > 0) {
        const auto S = static_cast<std::uint64_t>(c->shared_ffn);
        ts.push_back({p + "ffn_gate_shexp.weight", c->type_default, {D, S}, 0});
        ts.push_back({p + "ffn_up_shexp.weight", c->type_default, {D, S}, 0});
        ts.push_back({p + "ffn_down_shexp.weight", pick(c->type_ffn_down), {S, D}, 0});
      }
    } else if (c->gelu) {
      ts.push_back({p + "ffn_up.weight", c->type_default, {D, F}, 0});
      ts.push_back({p + "ffn_down.weight", pick(c->type_ffn_down), {F, D}, 0});
    } else {
      ts.push_back({p + "ffn_gate.weight", c->type_default, {D, F}, 0});
      ts.push_back({p + "ffn_up.weight", c->type_default, {D, F}, 0});
      ts.push_back({p + "ffn_down.weight", pick(c->type_ffn_down), {F, D}, 0});
    }
  }
  ts.push_back({"output_norm.weight", 0, {D}, 1});
  if (!c->tied) ts.push_back({"output.weight", pick(c->type_output), {D, V}, 0});

  std::uint64_t off = 0;
  for (auto& t : ts) {
    const std::int64_t be = block_elems(t.type);
    if (be == 0 || static_cast<std::int64_t>(t.ne[0]) % be) {
      g_err = "tensor " + t.name + " row length not a multiple of its block size";
      return -1;
    }
    std::int64_t rows = 1;
    for (std::size_t d = 1; d < t.ne.size(); ++d) rows *= static_cast<std::int64_t>(t.ne[d]);
    t.nbytes = rows * row_bytes(t.type, static_cast<std::int64_t>(t.ne[0]));
    t.offset = off;
    off = (off + static_cast<std::uint64_t>(t.nbytes) + 31) & ~31ull;
  }

  Writer w;
  w.raw("GGUF", 4);
  w.u32(3);
  w.u64(ts.size());
  const bool moe = c->n_experts > 0;
  const bool key_len = hd * c->n_heads != c->dim;
  w.u64(11 + (moe ? 2 : 0) + (key_len ? 1 : 0));
  w.kv_str("general.architecture", c->arch ? c->arch : "llama");
  w.kv_str("general.name", "uaii-synth");
  w.kv_u32("general.alignment", 32);
  const std::string a = std::string(c->arch ? c->arch : "llama") + ".";
  w.kv_u32(a + "block_count", static_cast<std::uint32_t>(c->n_layers));
  w.kv_u32(a + "context_length", static_cast<std::uint32_t>(c->ctx_len));
  w.kv_u32(a + "embedding_length", static_cast<std::uint32_t>(c->dim));
  w.kv_u32(a + "feed_forward_length", static_cast<std::uint32_t>(c->ffn));
  w.kv_u32(a + "attention.head_count", static_cast<std::uint32_t>(c->n_heads));
  w.kv_u32(a + "attention.head_count_kv", static_cast<std::uint32_t>(nkv));
  w.kv_f32(a + "rope.freq_base", c->rope_theta);
  w.kv_f32(a + "attention.layer_norm_rms_epsilon", c->rms_eps);
  if (moe) {
    w.kv_u32(a + "expert_count", static_cast<std::uint32_t>(c->n_experts));
    w.kv_u32(a + "expert_used_count", static_cast<std::uint32_t>(c->top_k));
  }
  if (key_len) w.kv_u32(a + "attention.key_length", static_cast<std::uint32_t>(hd));
  for (const auto& t : ts) {
    w.str(t.name);
    w.u32(static_cast<std::uint32_t>(t.ne.size()));
    for (auto d : t.ne) w.u64(d);
    w.u32(static_cast<std::uint32_t>(t.type));
    w.u64(t.offset);
  }
  while (w.buf.size() % 32) w.buf.push_back(0);

  std::FILE* f = std::fopen(path, "wb");
  if (!f) { g_err = std::string("cannot create ") + path; return -1; }
  bool ok = std::fwrite(w.buf.data(), 1, w.buf.size(), f) == w.buf.size();

  unsigned nt = nthreads > 0 ? static_cast<unsigned>(nthreads) : std::thread::hardware_concurrency();
  if (nt == 0) nt = 1;
  std::vector<std::uint8_t> data;
  std::uint64_t written = 0;
  for (std::size_t ti = 0; ti < ts.size() && ok; ++ti) {
    const TensorSpec& t = ts[ti];
    while (written < t.offset) { std::fputc(0, f); ++written; }
    const std::int64_t cols = static_cast<std::int64_t>(t.ne[0]);
    const std::int64_t rows = t.nbytes / row_bytes(t.type, cols);
    const std::int64_t rb = row_bytes(t.type, cols);
    data.assign(static_cast<std::size_t>(t.nbytes), 0);
    std::atomic<std::int64_t> next{0};
    auto body = [&]() {
      std::vector<float> row(static_cast<std::size_t>(cols));
      for (;;) {
        const std::int64_t r0 = next.fetch_add(16);
        if (r0 >= rows) break;
        for (std::int64_t r = r0; r < std::min(rows, r0 + 16); ++r) {
          if (t.fill == 1) {
            std::fill(row.begin(), row.end(), 1.0f);
          } else {
            uaii_synth_normals(c->seed, ti, static_cast<std::uint64_t>(r * cols), cols,
                               t.fill == 2 ? c->router_std : c->std, row.data());
          }
          uaii_synth_quantize_row(t.type, row.data(), cols, data.data() + r * rb);
        }
      }
    };
    std::vector<std::thread> th;
    for (unsigned k = 1; k < nt; ++k) th.emplace_back(body);
    body();
    for (auto& x : th) x.join();
    ok = std::fwrite(data.data(), 1, data.size(), f) == data.size();
    written += static_cast<std::uint64_t>(t.nbytes);
  }
  if (std::fclose(f) != 0) ok = false;
  if (!ok) { g_err = "write failed"; return -1; }
  return 0;
}

}  // extern "C"
