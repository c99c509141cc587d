// sample.hip — temperature / top-k / top-p / repetition-penalty sampling on the
// device (gfx950).
//
// Replaces sample_token_f32's non-greedy path (libs/uaii-runtime/src/
// sampling.cpp:53-125) for the token loop, so a sampled decode needs no copy of
// the 128k-float logits row to the host per token: score_i = rep(logit_i) *
// (1 / max(T, 1e-5)) with rep() the HF-style penalty on ids already in the
// history; the top_k largest scores kept; softmax; the smallest prefix in
// descending-probability order whose mass reaches top_p kept and renormalised;
// one uniform r in [0, 1) (drawn on the host from the seeded mt19937_64, one per
// token, as the reference draws) walks the kept ids to the first whose
// cumulative probability reaches r.
//
// Order of the walk: descending probability with top_p (the reference's
// std::sort order), index order with neither top_k nor top_p (the reference's
// row order). With top_k alone the reference walks std::nth_element's
// arrangement of the k ids, which no device order reproduces; here it walks
// them in descending order, the same distribution.
//
// Arithmetic. Scores are the reference's float expressions. Each id's weight
// exp(score - max) becomes an integer mass round(w * 2^40), and every sum,
// prefix and threshold is an integer: results do not depend on the order of the
// additions, and equal the reference's draw unless r lies within the float
// rounding of the reference's sequential sums (about 1e-7 of the mass) of a
// cumulative boundary. Ties: at the top-k boundary the lowest ids stay (k in
// all); at the top-p cut all tied ids stay; tied ids are walked in id order.
//
// Three launches over a workspace (sample_workspace_bytes):
//   k_samp_keys  per 1024-id slice: scores as order-preserving 32-bit keys, the
//                slice's largest key;
//   k_samp_hist  per slice: integer masses against the global max, the slice's
//                mass and a 1024-bin histogram of the keys' top 10 bits (counts
//                and masses), added into the global one;
//   k_samp_pick  one block: the top-k, top-p and draw thresholds as radix selects
//                over the keys (top digit from the global histogram, then 11 and
//                11 bits from passes over the keys that only the matching ids
//                join), or the index-order walk; then the token advance.

#include "common.h"
#include "uaii_hip_internal.h"

namespace uaii_hip {
namespace {

constexpr int P_NT = 256;              // threads of the per-slice kernels
constexpr int P_EPT = 4;               // ids per thread
constexpr int SLICE = P_NT * P_EPT;    // ids per slice
constexpr int MAXV = 1 << 18;          // vocabulary limit
constexpr int MAXB = MAXV / SLICE;     // slices
constexpr int F_NT = 1024;             // threads of the pick kernel (== SLICE)
constexpr int D1 = 10, D2 = 11, D3 = 11;  // key digits, top first
constexpr int NB1 = 1 << D1, NB2 = 1 << D2, NB3 = 1 << D3;
constexpr double MASS_SCALE = 1099511627776.0;  // 2^40
static_assert(F_NT == SLICE, "the index walk gives each thread one id of a slice");
static_assert(D1 + D2 + D3 == 32, "digits cover the key");

struct Ws {
  uint32_t* keys;   // [V] order-preserving keys of the scores
  uint32_t* bmax;   // [MAXB] largest key per slice
  uint64_t* bmass;  // [MAXB] mass per slice
  uint32_t* h1c;    // [NB1] counts per top digit
  uint64_t* h1m;    // [NB1] masses per top digit
};

__host__ __device__ constexpr size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

__host__ __device__ inline size_t ws_bytes(int64_t V) {
  return align256((size_t)V * 4) + align256(MAXB * 4) + align256(MAXB * 8) + align256(NB1 * 4) +
         align256(NB1 * 8);
}

__device__ inline Ws carve(void* base, int64_t V) {
  char* p = static_cast<char*>(base);
  Ws w;
  w.keys = reinterpret_cast<uint32_t*>(p);
  p += align256((size_t)V * 4);
  w.bmax = reinterpret_cast<uint32_t*>(p);
  p += align256(MAXB * 4);
  w.bmass = reinterpret_cast<uint64_t*>(p);
  p += align256(MAXB * 8);
  w.h1c = reinterpret_cast<uint32_t*>(p);
  p += align256(NB1 * 4);
  w.h1m = reinterpret_cast<uint64_t*>(p);
  return w;
}

__device__ __forceinline__ uint32_t key_of(float s) {
  const uint32_t u = __float_as_uint(s);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);  // ascending in s
}

__device__ __forceinline__ float score_of(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// round(exp(s - smax) * 2^40); 0 for NaN (an infinite or NaN maximum)
__device__ __forceinline__ uint64_t mass_of(uint32_t key, float smax) {
  const float w = expf(score_of(key) - smax);
  return w > 0.0f ? (uint64_t)((double)w * MASS_SCALE + 0.5) : 0;
}

// The penalised history and the draw of this call: with a step state, ids[0 ..
// pos] and rbuf[pos + 1 - n_prompt]; standalone, pen[0 .. n_pen) and r_fixed.
__device__ __forceinline__ void history(const SampleArgs& a, const int32_t** h, int* n) {
  if (a.state) {
    *h = a.ids;
    *n = a.state->pos + 1;
  } else {
    *h = a.pen;
    *n = (int)a.n_pen;
  }
}

__device__ __forceinline__ uint64_t shfl_up64(uint64_t v, int o) {
  return (uint64_t)__shfl_up((long long)v, (unsigned)o, 64);
}
__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int o) {
  return (uint64_t)__shfl_xor((long long)v, o, 64);
}

template <int NT>
__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, uint32_t* red) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int o = 32; o > 0; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o, 64));
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  uint32_t t = 0;
  for (int k = 0; k < NT / 64; ++k) t = max(t, red[k]);
  return t;
}

template <int NT>
__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, uint64_t* red) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int o = 32; o > 0; o >>= 1) v += shfl_xor64(v, o);
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  uint64_t t = 0;
  for (int k = 0; k < NT / 64; ++k) t += red[k];
  return t;
}

// ---- per-slice kernels -------------------------------------------------------------------

__global__ void __launch_bounds__(P_NT) k_samp_keys(SampleArgs a) {
  __shared__ uint32_t seen[SLICE / 32];
  __shared__ uint32_t red[P_NT / 64];
  const Ws w = carve(a.ws, a.V);
  const int tid = threadIdx.x;
  const int64_t base = (int64_t)blockIdx.x * SLICE;
  // the global histogram k_samp_hist fills (it runs after this kernel)
  if (blockIdx.x == 0) {
    for (int b = tid; b < NB1; b += P_NT) {
      w.h1c[b] = 0u;
      w.h1m[b] = 0u;
    }
  }
  const bool rep_on = a.rep > 1.0f + 1e-6f;
  if (rep_on) {
    for (int k = tid; k < SLICE / 32; k += P_NT) seen[k] = 0u;
    __syncthreads();
    const int32_t* h;
    int n;
    history(a, &h, &n);
    for (int k = tid; k < n; k += P_NT) {
      const int64_t j = (int64_t)h[k] - base;
      if (j >= 0 && j < SLICE) atomicOr(&seen[j >> 5], 1u << (j & 31));
    }
    __syncthreads();
  }
  uint32_t mx = 0u;
#pragma unroll
  for (int e = 0; e < P_EPT; ++e) {
    const int j = e * P_NT + tid;
    const int64_t i = base + j;
    if (i < a.V) {
      float l = a.logits[i];
      if (rep_on && ((seen[j >> 5] >> (j & 31)) & 1u)) l = l > 0.0f ? l / a.rep : l * a.rep;
      const uint32_t k = key_of(l * a.inv_t);
      w.keys[i] = k;
      mx = max(mx, k);
    }
  }
  mx = block_max_u32<P_NT>(mx, red);
  if (tid == 0) w.bmax[blockIdx.x] = mx;
}

__global__ void __launch_bounds__(P_NT) k_samp_hist(SampleArgs a) {
  __shared__ uint32_t hc[NB1];
  __shared__ uint64_t hm[NB1];
  __shared__ uint32_t redu[P_NT / 64];
  __shared__ uint64_t red[P_NT / 64];
  const Ws w = carve(a.ws, a.V);
  const int tid = threadIdx.x;
  const int nb = (int)((a.V + SLICE - 1) / SLICE);
  uint32_t g = 0u;
  for (int b = tid; b < nb; b += P_NT) g = max(g, w.bmax[b]);
  const float smax = score_of(block_max_u32<P_NT>(g, redu));
  for (int b = tid; b < NB1; b += P_NT) {
    hc[b] = 0u;
    hm[b] = 0u;
  }
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * SLICE;
  uint64_t sum = 0;
#pragma unroll
  for (int e = 0; e < P_EPT; ++e) {
    const int64_t i = base + e * P_NT + tid;
    if (i < a.V) {
      const uint32_t k = w.keys[i];
      const uint64_t m = mass_of(k, smax);
      sum += m;
      atomicAdd(&hc[k >> (32 - D1)], 1u);
      atomicAdd((unsigned long long*)&hm[k >> (32 - D1)], (unsigned long long)m);
    }
  }
  __syncthreads();
  for (int b = tid; b < NB1; b += P_NT) {
    if (hc[b]) {
      atomicAdd(&w.h1c[b], hc[b]);
      atomicAdd((unsigned long long*)&w.h1m[b], (unsigned long long)hm[b]);
    }
  }
  sum = block_sum_u64<P_NT>(sum, red);
  if (tid == 0) w.bmass[blockIdx.x] = sum;
}

// ---- the pick kernel ---------------------------------------------------------------------

struct CM {
  uint64_t c, m;  // count, mass
};
__device__ __forceinline__ CM operator+(CM x, CM y) { return CM{x.c + y.c, x.m + y.m}; }
__device__ __forceinline__ CM operator-(CM x, CM y) { return CM{x.c - y.c, x.m - y.m}; }

struct PickLds {
  uint32_t hc[NB2];
  uint64_t hm[NB2];
  uint32_t hmin[NB2];  // lowest id per bin
  CM wsum[F_NT / 64];
  int s_item;
  CM s_acc;
};
static_assert(NB3 <= NB2, "level-3 histograms reuse the level-2 arrays");

// Over n logical items (item j's weights from `item(j)`), the first j (order
// 0..n-1) at which the running weight, starting at acc0, reaches the target: by
// mass when `by_mass`, else by count. Target 0, or a mass target where no item
// has mass, selects the first item with a count; targets beyond the total are
// clamped to it. Returns j (-1 when no item has a count) and, in *acc, acc0 plus
// the weights of the items before j.
template <class Item>
__device__ int find_first(int n, Item item, CM acc0, bool by_mass, uint64_t target, PickLds& s, CM* acc) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int per = (n + F_NT - 1) / F_NT;
  const int j0 = min(n, tid * per), j1 = min(n, j0 + per);
  CM own{};
  for (int j = j0; j < j1; ++j) own = own + item(j);
  // exclusive block scan of (count, mass) in item order
  CM x = own;
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t yc = shfl_up64(x.c, o), ym = shfl_up64(x.m, o);
    if (lane >= o) { x.c += yc; x.m += ym; }
  }
  __syncthreads();  // earlier readers of s are done
  if (lane == 63) s.wsum[wv] = x;
  if (tid == 0) s.s_item = -1;
  __syncthreads();
  CM before{}, tot{};
  for (int k = 0; k < F_NT / 64; ++k) {
    if (k < wv) before = before + s.wsum[k];
    tot = tot + s.wsum[k];
  }
  const CM excl = acc0 + before + (x - own);
  const CM end = acc0 + tot;
  bool use_m = by_mass && target != 0;
  uint64_t t = target;
  if (use_m) {
    if (t > end.m) t = end.m;
    if (t <= acc0.m) use_m = false;  // no mass left: the first item with a count
  }
  if (!use_m) {
    t = (by_mass || target == 0) ? acc0.c + 1 : target;
    if (t > end.c) t = end.c;
  }
  // t lies in (acc0, end]: exactly one thread's range holds the crossing
  const uint64_t lo = use_m ? excl.m : excl.c;
  const uint64_t hi = lo + (use_m ? own.m : own.c);
  if (t > (use_m ? acc0.m : acc0.c) && lo < t && hi >= t) {
    CM run = excl;
    for (int j = j0; j < j1; ++j) {
      const CM v = item(j);
      if ((use_m ? run.m + v.m : run.c + v.c) >= t) {
        s.s_item = j;
        s.s_acc = run;
        break;
      }
      run = run + v;
    }
  }
  __syncthreads();
  *acc = s.s_acc;
  return s.s_item;
}

struct Filter {
  bool on = false;
  uint32_t lo = 0u;               // kept: keys above lo, and lo itself ...
  uint32_t id_max = 0xffffffffu;  // ... for ids up to id_max
  CM part{};                      // kept weight inside lo's top-digit bin
};

__device__ __forceinline__ bool kept(const Filter& f, uint32_t k, int64_t i) {
  return k > f.lo || (k == f.lo && (uint64_t)i <= (uint64_t)f.id_max);
}

// Histogram (count, mass, lowest id) of the digit at `dshift` over the kept ids
// whose key matches `prefix` above `pshift`: one pass over the keys, where only
// the matching ids touch the LDS.
__device__ void pass_hist(const Ws& w, int64_t V, float smax, uint32_t prefix, int pshift, int dshift,
                          uint32_t dmask, const Filter& f, PickLds& s) {
  const int tid = threadIdx.x;
  __syncthreads();  // earlier readers of the histogram are done
  for (int b = tid; b < NB2; b += F_NT) {
    s.hc[b] = 0u;
    s.hm[b] = 0u;
    s.hmin[b] = 0xffffffffu;
  }
  __syncthreads();
  auto one = [&](uint32_t k, int64_t i) {
    if ((k >> pshift) == prefix && kept(f, k, i)) {
      const uint32_t d = (k >> dshift) & dmask;
      atomicAdd(&s.hc[d], 1u);
      atomicAdd((unsigned long long*)&s.hm[d], (unsigned long long)mass_of(k, smax));
      atomicMin(&s.hmin[d], (uint32_t)i);
    }
  };
  const int64_t n4 = V >> 2;
  const uint4* k4 = reinterpret_cast<const uint4*>(w.keys);
  for (int64_t q = tid; q < n4; q += F_NT) {
    const uint4 v = k4[q];
    one(v.x, 4 * q);
    one(v.y, 4 * q + 1);
    one(v.z, 4 * q + 2);
    one(v.w, 4 * q + 3);
  }
  for (int64_t i = 4 * n4 + tid; i < V; i += F_NT) one(w.keys[i], i);
  __syncthreads();
}

struct Sel {
  bool ok = false;
  uint32_t key = 0u;    // the selected key
  uint32_t min_id = 0u; // the lowest kept id with that key
  CM ge{};              // kept weight with key >= key
  CM eq{};              // kept weight with key == key
  CM part{};            // kept weight with key >= key inside key's top-digit bin
};

// Radix select from the top over the kept ids: the largest key K
// whose kept weight at or above it reaches the target (find_first's rules).
__device__ Sel select(const Ws& w, int64_t V, float smax, bool by_mass, uint64_t target, const Filter& f,
                      PickLds& s) {
  Sel r;
  const int fb1 = (int)(f.lo >> (32 - D1));
  CM acc1{}, acc2{}, acc3{};
  const int j1 = find_first(
      NB1,
      [&](int j) {
        const int b = NB1 - 1 - j;
        if (f.on && b < fb1) return CM{};
        if (f.on && b == fb1) return f.part;
        return CM{w.h1c[b], w.h1m[b]};
      },
      CM{}, by_mass, target, s, &acc1);
  if (j1 < 0) return r;
  const uint32_t B1 = (uint32_t)(NB1 - 1 - j1);
  pass_hist(w, V, smax, B1, 32 - D1, D3, NB2 - 1, f, s);
  const int j2 = find_first(
      NB2, [&](int j) { const int b = NB2 - 1 - j; return CM{s.hc[b], s.hm[b]}; }, acc1, by_mass, target, s,
      &acc2);
  if (j2 < 0) return r;
  const uint32_t B2 = (uint32_t)(NB2 - 1 - j2);
  const CM w2{s.hc[B2], s.hm[B2]};
  if (w2.c == 1) {
    // one id in the sub-bin: its key is the answer
    r.min_id = s.hmin[B2];
    r.key = w.keys[r.min_id];
    r.eq = w2;
    r.ge = acc2 + w2;
  } else {
    pass_hist(w, V, smax, (B1 << D2) | B2, D3, 0, NB3 - 1, f, s);
    const int j3 = find_first(
        NB3, [&](int j) { const int b = NB3 - 1 - j; return CM{s.hc[b], s.hm[b]}; }, acc2, by_mass, target, s,
        &acc3);
    if (j3 < 0) return r;
    const uint32_t B3 = (uint32_t)(NB3 - 1 - j3);
    r.key = (B1 << (D2 + D3)) | (B2 << D3) | B3;
    r.min_id = s.hmin[B3];
    r.eq = CM{s.hc[B3], s.hm[B3]};
    r.ge = acc3 + r.eq;
  }
  r.part = r.ge - acc1;
  r.ok = true;
  return r;
}

// The need-th lowest id (need >= 1) up to id_max whose key is `key`: per-thread
// counts over contiguous id ranges, their scan, then a walk of the one range
// that holds it.
__device__ uint32_t nth_tied_id(const Ws& w, int64_t V, uint32_t key, uint32_t id_max, uint64_t need,
                                PickLds& s) {
  const int64_t per = (V + F_NT - 1) / F_NT;
  const int64_t c0 = min(V, (int64_t)threadIdx.x * per);
  const int64_t c1 = min(min(V, c0 + per), (int64_t)id_max + 1);
  uint64_t cnt = 0;
  for (int64_t i = c0; i < c1; ++i) cnt += w.keys[i] == key ? 1u : 0u;
  CM acc{};
  const int t = find_first(F_NT, [&](int) { return CM{cnt, 0u}; }, CM{}, false, need, s, &acc);
  __syncthreads();
  if ((int)threadIdx.x == t) {
    uint64_t seen = acc.c;
    for (int64_t i = c0; i < c1; ++i) {
      if (w.keys[i] == key && ++seen == need) {
        s.s_item = (int)i;
        break;
      }
    }
  }
  __syncthreads();
  const int id = s.s_item;
  return id < 0 ? 0xffffffffu : (uint32_t)id;
}

__device__ __forceinline__ uint64_t ceil_mul(float x, uint64_t m) {
  return (uint64_t)ceil((double)x * (double)m);
}

__global__ void __launch_bounds__(F_NT) k_samp_pick(SampleArgs a) {
  __shared__ PickLds s;
  __shared__ uint32_t redu[F_NT / 64];
  __shared__ uint64_t red[F_NT / 64];
  const Ws w = carve(a.ws, a.V);
  const int tid = threadIdx.x;
  const int64_t V = a.V;
  const int nb = (int)((V + SLICE - 1) / SLICE);
  uint32_t g = 0u;
  for (int b = tid; b < nb; b += F_NT) g = max(g, w.bmax[b]);
  const float smax = score_of(block_max_u32<F_NT>(g, redu));
  const uint64_t total = block_sum_u64<F_NT>(tid < nb ? w.bmass[tid] : 0u, red);

  int p = 0;
  float r = a.r_fixed;
  if (a.state) {
    p = a.state->pos + 1;
    const int64_t t = (int64_t)p - a.state->n_prompt;
    r = (a.rbuf && t >= 0 && t < a.nr) ? a.rbuf[t] : 0.0f;
  }
  const bool use_k = a.top_k > 0 && (int64_t)a.top_k < V;
  const bool use_p = a.top_p > 0.0f && a.top_p < 1.0f - 1e-6f;
  int64_t pick = 0;
  if (total == 0) {
    pick = 0;  // no finite weight (an infinite or NaN maximum): the reference's degenerate first id
  } else if (use_k || use_p) {
    Filter f;
    uint64_t kept = total;
    if (use_k) {
      const Sel sk = select(w, V, smax, false, (uint64_t)a.top_k, f, s);
      f.on = true;
      f.lo = sk.key;
      f.part = sk.part;
      kept = sk.ge.m;
      // ties at the k-th score beyond k: the lowest ids stay
      const uint64_t need = (uint64_t)a.top_k - (sk.ge.c - sk.eq.c);
      if (sk.eq.c > need) {
        f.id_max = nth_tied_id(w, V, sk.key, 0xffffffffu, need, s);
        const CM drop{sk.eq.c - need, (sk.eq.m / sk.eq.c) * (sk.eq.c - need)};
        f.part = f.part - drop;
        kept -= drop.m;
      }
    }
    if (use_p) {
      const Sel sp = select(w, V, smax, true, ceil_mul(a.top_p, kept), f, s);
      if (sp.key != f.lo) f.id_max = 0xffffffffu;  // ties at the top-p cut stay together
      f.on = true;
      f.lo = sp.key;
      f.part = sp.part;
      kept = sp.ge.m;
    }
    const uint64_t tgt = ceil_mul(r, kept);
    const Sel sd = select(w, V, smax, true, tgt, f, s);
    pick = sd.ok ? (int64_t)sd.min_id : 0;
    if (sd.ok && sd.eq.c > 1) {
      // a draw inside tied scores: the tied ids in id order, each its share
      const uint64_t each = sd.eq.m / sd.eq.c, above = sd.ge.m - sd.eq.m;
      const uint64_t t = min(tgt, kept);
      uint64_t nth = 1;
      if (each > 0 && t > above) nth = min(sd.eq.c, (t - above + each - 1) / each);
      if (nth > 1) pick = nth_tied_id(w, V, sd.key, sd.key == f.lo ? f.id_max : 0xffffffffu, nth, s);
    }
  } else {
    // index order: the slice, then the id, where the prefix mass reaches r
    const uint64_t tgt = ceil_mul(r, total);
    CM acc{}, acc2{};
    const int js = find_first(
        nb,
        [&](int j) {
          const int64_t n = min((int64_t)SLICE, V - (int64_t)j * SLICE);
          return CM{(uint64_t)n, w.bmass[j]};
        },
        CM{}, true, tgt, s, &acc);
    const int64_t base = (int64_t)(js < 0 ? 0 : js) * SLICE;
    const int jj = find_first(
        SLICE,
        [&](int j) {
          const int64_t i = base + j;
          return i < V ? CM{1u, mass_of(w.keys[i], smax)} : CM{};
        },
        acc, true, tgt, s, &acc2);
    pick = base + (jj < 0 ? 0 : jj);
  }
  if (pick < 0 || pick >= V) pick = 0;  // every path above yields an id in range; the feed stays in range regardless
  if (tid == 0) {
    if (a.out) *a.out = (int32_t)pick;
    if (a.state) {
      // the token advance of k_argmax_final: inside the prompt the prompt's id
      StepState* st = a.state;
      const int next = (p < st->n_prompt) ? a.ids[p] : (int)pick;
      a.ids[p] = next;
      st->argmax = (int)pick;
      st->token = next;
      st->pos = p;
    }
  }
}

}  // namespace

int sample_max_vocab() { return MAXV; }

size_t sample_workspace_bytes(int64_t V) { return V > 0 && V <= MAXV ? ws_bytes(V) : 0; }

hipError_t launch_sample(const SampleArgs& a, hipStream_t s) {
  if (a.V <= 0 || a.V > MAXV || !a.logits || !a.ws) return hipErrorInvalidValue;
  if (a.state ? !a.ids : (a.n_pen > 0 && !a.pen)) return hipErrorInvalidValue;
  if (reinterpret_cast<uintptr_t>(a.ws) % 256) return hipErrorInvalidValue;
  const int nb = (int)((a.V + SLICE - 1) / SLICE);
  UAII_LAUNCH(k_samp_keys, dim3(nb), dim3(P_NT), 0, s, a);
  hipError_t st = hipGetLastError();
  if (st != hipSuccess) return st;
  UAII_LAUNCH(k_samp_hist, dim3(nb), dim3(P_NT), 0, s, a);
  st = hipGetLastError();
  if (st != hipSuccess) return st;
  UAII_LAUNCH(k_samp_pick, dim3(1), dim3(F_NT), 0, s, a);
  return hipGetLastError();
}

}  // namespace uaii_hip
