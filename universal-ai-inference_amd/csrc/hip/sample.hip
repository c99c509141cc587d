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
// Four launches over a workspace (sample_workspace_bytes). Scores are handled
// as order-preserving 32-bit keys, split into digits of 10, 11 and 11 bits.
//   k_samp_keys    per 1024-id slice: the keys, the slice's largest;
//   k_samp_hist    per slice: integer masses against the global max, the
//                  slice's mass, and the keys' top digits (count and mass per
//                  digit) added into a global histogram;
//   k_samp_bucket  per slice: from that histogram, the lowest top digit a kept
//                  id can have (the top-k boundary's, else the top-p cut's);
//                  the ids at or above it copied out grouped by top digit;
//   k_samp_pick    one block: the top-k, top-p and draw thresholds as radix
//                  selects (top digit from the histogram, the two lower digits
//                  from LDS histograms over one digit's group), a short kept
//                  list sorted in LDS, or the index-order walk; then the token
//                  advance. A single CU reads a 128k-key row in ~20 us, so it
//                  only reads the groups.

#include "common.h"
#include "uaii_hip_internal.h"

namespace uaii_hip {
namespace {

constexpr int P_NT = 256;              // threads of the per-slice kernels
constexpr int P_EPT = 4;               // ids per thread
constexpr int SLICE = P_NT * P_EPT;    // ids per slice
constexpr int MAXV = 1 << 18;          // vocabulary limit
constexpr int MAXB = MAXV / SLICE;     // slices
constexpr int F_NT = 512;              // threads of the pick kernel
constexpr int CAPG = 2048;             // kept ids the pick kernel sorts in LDS
constexpr int D1 = 10, D2 = 11, D3 = 11;  // key digits, top first
constexpr int SH1 = 32 - D1;
constexpr int NB1 = 1 << D1, NB2 = 1 << D2, NB3 = 1 << D3;
constexpr double MASS_SCALE = 1099511627776.0;  // 2^40
static_assert(D1 + D2 + D3 == 32, "digits cover the key");
static_assert(NB3 <= NB2, "level-3 histograms reuse the level-2 arrays");

struct Ws {
  uint32_t* keys;   // [V] order-preserving keys of the scores
  uint32_t* ckeys;  // [V] keys at or above the lowest kept top digit, grouped by
                    // top digit, highest first
  uint32_t* cids;   // [V] their ids
  uint32_t* bmax;   // [MAXB] largest key per slice
  uint64_t* bmass;  // [MAXB] mass per slice
  uint32_t* h1c;    // [NB1] counts per top digit
  uint64_t* h1m;    // [NB1] masses per top digit
  uint32_t* fill;   // [NB1] ids copied per top digit
  uint32_t* ctl;    // [0]: the lowest kept top digit (NB1: no groups)
};

__host__ __device__ constexpr size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

__host__ __device__ inline size_t ws_bytes(int64_t V) {
  return 3 * align256((size_t)V * 4) + align256(MAXB * 4) + align256(MAXB * 8) + align256(NB1 * 4) +
         align256(NB1 * 8) + align256(NB1 * 4) + 256;
}

__device__ inline Ws carve(void* base, int64_t V) {
  char* p = static_cast<char*>(base);
  Ws w;
  const size_t row = align256((size_t)V * 4);
  w.keys = reinterpret_cast<uint32_t*>(p);
  w.ckeys = reinterpret_cast<uint32_t*>(p + row);
  w.cids = reinterpret_cast<uint32_t*>(p + 2 * row);
  p += 3 * row;
  w.bmax = reinterpret_cast<uint32_t*>(p);
  p += align256(MAXB * 4);
  w.bmass = reinterpret_cast<uint64_t*>(p);
  p += align256(MAXB * 8);
  w.h1c = reinterpret_cast<uint32_t*>(p);
  p += align256(NB1 * 4);
  w.h1m = reinterpret_cast<uint64_t*>(p);
  p += align256(NB1 * 8);
  w.fill = reinterpret_cast<uint32_t*>(p);
  p += align256(NB1 * 4);
  w.ctl = reinterpret_cast<uint32_t*>(p);
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

__device__ __forceinline__ uint64_t ceil_mul(float x, uint64_t m) {
  return (uint64_t)ceil((double)x * (double)m);
}

struct Mode {
  bool use_k, use_p;
};

__device__ __forceinline__ Mode mode_of(const SampleArgs& a) {
  return Mode{a.top_k > 0 && (int64_t)a.top_k < a.V, a.top_p > 0.0f && a.top_p < 1.0f - 1e-6f};
}

// The penalised history: with a step state ids[0 .. pos], standalone pen[0 .. n_pen).
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

template <int NT>
__device__ __forceinline__ float global_max_score(const uint32_t* bmax, int nb, uint32_t* red) {
  uint32_t g = 0u;
  for (int b = threadIdx.x; b < nb; b += NT) g = max(g, bmax[b]);
  return score_of(block_max_u32<NT>(g, red));
}

struct CM {
  uint64_t c, m;  // count, mass
};
__device__ __forceinline__ CM operator+(CM x, CM y) { return CM{x.c + y.c, x.m + y.m}; }
__device__ __forceinline__ CM operator-(CM x, CM y) { return CM{x.c - y.c, x.m - y.m}; }

template <int NT>
struct ScanLds {
  CM wsum[NT / 64];
  int item;
  CM acc;
};

// Over n logical items (item j's weights from `item(j)`), the first j (order
// 0..n-1) at which the running weight, starting at acc0, reaches the target: by
// mass when `by_mass`, else by count. Target 0, or a mass target where no item
// has mass, selects the first item with a count; targets beyond the total are
// clamped to it. Returns j (-1 when no item has a count) and, in *acc, acc0 plus
// the weights of the items before j. Every thread of the block calls it.
template <int NT, class Item>
__device__ int find_first(int n, Item item, CM acc0, bool by_mass, uint64_t target, ScanLds<NT>& s,
                          CM* acc) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int per = (n + NT - 1) / NT;
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
  if (tid == 0) s.item = -1;
  __syncthreads();
  CM before{}, tot{};
  for (int k = 0; k < NT / 64; ++k) {
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
        s.item = j;
        s.acc = run;
        break;
      }
      run = run + v;
    }
  }
  __syncthreads();
  *acc = s.acc;
  return s.item;
}

// The lowest top digit a kept id can have, from the global histogram: the
// top-k boundary's (a count select), else the top-p cut's (a mass select).
// NB1 when no digit qualifies. The pick kernel's first select reproduces it.
template <int NT>
__device__ int lowest_digit(const SampleArgs& a, const Ws& w, uint64_t total, Mode md, ScanLds<NT>& s) {
  CM acc{};
  const uint64_t target = md.use_k ? (uint64_t)a.top_k : ceil_mul(a.top_p, total);
  const int j = find_first<NT>(
      NB1, [&](int jj) { const int b = NB1 - 1 - jj; return CM{w.h1c[b], w.h1m[b]}; }, CM{}, !md.use_k,
      target, s, &acc);
  return j < 0 ? NB1 : NB1 - 1 - j;
}

// ---- per-slice kernels -------------------------------------------------------------------

__global__ void __launch_bounds__(P_NT) k_samp_keys(SampleArgs a) {
  __shared__ uint32_t seen[SLICE / 32];
  __shared__ uint32_t red[P_NT / 64];
  const Ws w = carve(a.ws, a.V);
  const int tid = threadIdx.x;
  const int64_t base = (int64_t)blockIdx.x * SLICE;
  // what the next kernels accumulate into (they run after this one)
  if (blockIdx.x == 0) {
    for (int b = tid; b < NB1; b += P_NT) {
      w.h1c[b] = 0u;
      w.h1m[b] = 0u;
      w.fill[b] = 0u;
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
  const float smax = global_max_score<P_NT>(w.bmax, nb, redu);
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
      atomicAdd(&hc[k >> SH1], 1u);
      atomicAdd((unsigned long long*)&hm[k >> SH1], (unsigned long long)m);
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

__global__ void __launch_bounds__(P_NT) k_samp_bucket(SampleArgs a) {
  __shared__ ScanLds<P_NT> sc;
  __shared__ uint32_t lc[NB1];     // this slice's ids per top digit
  __shared__ uint32_t lbase[NB1];  // their place within the digit's group
  __shared__ uint32_t off[NB1];    // start of each digit's group
  __shared__ uint64_t red[P_NT / 64];
  const Ws w = carve(a.ws, a.V);
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const Mode md = mode_of(a);
  if (!md.use_k && !md.use_p) {
    if (blockIdx.x == 0 && tid == 0) w.ctl[0] = NB1;
    return;
  }
  uint64_t t = 0;
  for (int b = tid; b < NB1; b += P_NT) t += w.h1m[b];
  const uint64_t total = block_sum_u64<P_NT>(t, red);
  const int blo = lowest_digit<P_NT>(a, w, total, md, sc);
  if (blockIdx.x == 0 && tid == 0) w.ctl[0] = (uint32_t)blo;
  if (blo >= NB1) return;
  // group starts: counts of the higher digits (an exclusive scan from the top)
  constexpr int PER = NB1 / P_NT;
  uint32_t own = 0;
  for (int q = 0; q < PER; ++q) own += w.h1c[NB1 - 1 - (tid * PER + q)];
  uint32_t x = own;
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = (uint32_t)__shfl_up((int)x, (unsigned)o, 64);
    if (lane >= o) x += y;
  }
  __syncthreads();
  if (lane == 63) sc.wsum[wv].c = x;
  for (int b = tid; b < NB1; b += P_NT) lc[b] = 0u;
  __syncthreads();
  uint32_t run = x - own;
  for (int k = 0; k < wv; ++k) run += (uint32_t)sc.wsum[k].c;
  for (int q = 0; q < PER; ++q) {
    const int b = NB1 - 1 - (tid * PER + q);
    off[b] = run;
    run += w.h1c[b];
  }
  // this slice's ids at or above the lowest kept digit, ranked per digit
  const int64_t base = (int64_t)blockIdx.x * SLICE;
  uint32_t kk[P_EPT];
  int rank[P_EPT];
#pragma unroll
  for (int e = 0; e < P_EPT; ++e) {
    const int64_t i = base + e * P_NT + tid;
    rank[e] = -1;
    kk[e] = 0u;
    if (i < a.V) {
      kk[e] = w.keys[i];
      if ((int)(kk[e] >> SH1) >= blo) rank[e] = (int)atomicAdd(&lc[kk[e] >> SH1], 1u);
    }
  }
  __syncthreads();
  for (int b = tid; b < NB1; b += P_NT) {
    if (b >= blo && lc[b]) lbase[b] = atomicAdd(&w.fill[b], lc[b]);
  }
  __syncthreads();
#pragma unroll
  for (int e = 0; e < P_EPT; ++e) {
    if (rank[e] >= 0) {
      const uint32_t b = kk[e] >> SH1;
      const uint32_t pos = off[b] + lbase[b] + (uint32_t)rank[e];
      if (pos < (uint32_t)a.V) {
        w.ckeys[pos] = kk[e];
        w.cids[pos] = (uint32_t)(base + e * P_NT + tid);
      }
    }
  }
}

// ---- the pick kernel ---------------------------------------------------------------------

struct PickLds {
  uint32_t hc[NB2];
  uint64_t hm[NB2];
  uint32_t hmin[NB2];   // lowest id per bin
  uint64_t list[CAPG];  // gathered kept ids: key << 32 | ~id
  ScanLds<F_NT> sc;
  int cnt;
};

struct Filter {
  bool on = false;
  uint32_t lo = 0u;               // kept: keys above lo, and lo itself ...
  uint32_t id_max = 0xffffffffu;  // ... for ids up to id_max
  CM part{};                      // kept weight inside lo's top-digit bin
};

__device__ __forceinline__ bool kept(const Filter& f, uint32_t k, int i) {
  return k > f.lo || (k == f.lo && (uint32_t)i <= f.id_max);
}

// Keys to scan: the whole row (ids null: the id is the index) or a run of the
// grouped copy.
struct Src {
  const uint32_t* keys;
  const uint32_t* ids;
  int n;
  int V;  // ids at or above V are skipped
};

// fn(key, id) over the entries whose key passes the cheap test pre(key), by
// one block, several loads in flight per thread before any is used.
template <class Pre, class Fn>
__device__ __forceinline__ void for_src(const Src& src, Pre&& pre, Fn&& fn) {
  if (!src.ids) {
    constexpr int U = 8;
    const int n4 = src.n >> 2;
    const uint4* k4 = reinterpret_cast<const uint4*>(src.keys);
    for (int q0 = threadIdx.x; q0 < n4; q0 += F_NT * U) {
      uint4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int q = q0 + u * F_NT;
        v[u] = q < n4 ? k4[q] : make_uint4(0u, 0u, 0u, 0u);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int q = q0 + u * F_NT;
        const bool px = pre(v[u].x), py = pre(v[u].y), pz = pre(v[u].z), pw = pre(v[u].w);
        if (q < n4 && (px | py | pz | pw)) {
          if (px) fn(v[u].x, 4 * q);
          if (py) fn(v[u].y, 4 * q + 1);
          if (pz) fn(v[u].z, 4 * q + 2);
          if (pw) fn(v[u].w, 4 * q + 3);
        }
      }
    }
    for (int i = 4 * n4 + (int)threadIdx.x; i < src.n; i += F_NT) {
      const uint32_t k = src.keys[i];
      if (pre(k)) fn(k, i);
    }
  } else {
    constexpr int U = 4;
    for (int j0 = threadIdx.x; j0 < src.n; j0 += F_NT * U) {
      uint32_t k[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int j = j0 + u * F_NT;
        k[u] = j < src.n ? src.keys[j] : 0u;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int j = j0 + u * F_NT;
        if (j < src.n && pre(k[u])) {
          const uint32_t id = src.ids[j];
          if (id < (uint32_t)src.V) fn(k[u], (int)id);
        }
      }
    }
  }
}

// Histogram (count, mass, lowest id) of the digit at `dshift` over the kept
// entries whose key matches `prefix` above `pshift`.
__device__ void pass_hist(const Src& src, float smax, uint32_t prefix, int pshift, int dshift, uint32_t dmask,
                          const Filter& f, PickLds& s) {
  const int tid = threadIdx.x;
  __syncthreads();  // earlier readers of the histogram are done
  for (int b = tid; b < NB2; b += F_NT) {
    s.hc[b] = 0u;
    s.hm[b] = 0u;
    s.hmin[b] = 0xffffffffu;
  }
  __syncthreads();
  for_src(src, [&](uint32_t k) { return (k >> pshift) == prefix; }, [&](uint32_t k, int i) {
    if (kept(f, k, i)) {
      const uint32_t d = (k >> dshift) & dmask;
      atomicAdd(&s.hc[d], 1u);
      atomicAdd((unsigned long long*)&s.hm[d], (unsigned long long)mass_of(k, smax));
      atomicMin(&s.hmin[d], (uint32_t)i);
    }
  });
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

struct Ctx {
  Ws w;
  int64_t V;
  float smax;
  int blo;  // the lowest top digit with a group (NB1: none)
};

// The entries with top digit b: its group when there is one, else the row.
__device__ __forceinline__ Src source_of(const Ctx& c, int b, uint64_t above) {
  const uint64_t n = c.w.h1c[b];
  if (b >= c.blo && above + n <= (uint64_t)c.V) return Src{c.w.ckeys + above, c.w.cids + above, (int)n, (int)c.V};
  return Src{c.w.keys, nullptr, (int)c.V, (int)c.V};
}

// Radix select from the top over the kept ids: the largest key K whose kept
// weight at or above it reaches the target (find_first's rules).
__device__ Sel select(const Ctx& c, bool by_mass, uint64_t target, const Filter& f, PickLds& s) {
  Sel r;
  const Ws& w = c.w;
  const int fb1 = (int)(f.lo >> SH1);
  CM acc1{}, acc2{}, acc3{};
  const int j1 = find_first<F_NT>(
      NB1,
      [&](int j) {
        const int b = NB1 - 1 - j;
        if (f.on && b < fb1) return CM{};
        if (f.on && b == fb1) return f.part;
        return CM{w.h1c[b], w.h1m[b]};
      },
      CM{}, by_mass, target, s.sc, &acc1);
  if (j1 < 0) return r;
  const uint32_t B1 = (uint32_t)(NB1 - 1 - j1);
  // acc1.c counts every id above B1 (the filter only trims digits at or below
  // its own, and B1 is not below it): the start of B1's group
  const Src src = source_of(c, (int)B1, acc1.c);
  pass_hist(src, c.smax, B1, SH1, D3, NB2 - 1, f, s);
  const int j2 = find_first<F_NT>(
      NB2, [&](int j) { const int b = NB2 - 1 - j; return CM{s.hc[b], s.hm[b]}; }, acc1, by_mass, target,
      s.sc, &acc2);
  if (j2 < 0) return r;
  const uint32_t B2 = (uint32_t)(NB2 - 1 - j2);
  const CM w2{s.hc[B2], s.hm[B2]};
  if (w2.c == 1) {
    // one id in the sub-bin: its key is the answer
    r.min_id = s.hmin[B2];
    if (r.min_id >= (uint32_t)c.V) return r;
    r.key = w.keys[r.min_id];
    r.eq = w2;
    r.ge = acc2 + w2;
  } else {
    pass_hist(src, c.smax, (B1 << D2) | B2, D3, 0, NB3 - 1, f, s);
    const int j3 = find_first<F_NT>(
        NB3, [&](int j) { const int b = NB3 - 1 - j; return CM{s.hc[b], s.hm[b]}; }, acc2, by_mass, target,
        s.sc, &acc3);
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
// counts over contiguous id ranges of the row, their scan, then a walk of the
// one range that holds it. Only ties at a boundary come here.
__device__ uint32_t nth_tied_id(const Ctx& c, uint32_t key, uint32_t id_max, uint64_t need, PickLds& s) {
  const int64_t V = c.V;
  const int64_t per = (V + F_NT - 1) / F_NT;
  const int64_t c0 = min(V, (int64_t)threadIdx.x * per);
  const int64_t c1 = min(min(V, c0 + per), (int64_t)id_max + 1);
  uint64_t cnt = 0;
  for (int64_t i = c0; i < c1; ++i) cnt += c.w.keys[i] == key ? 1u : 0u;
  CM acc{};
  const int t = find_first<F_NT>(F_NT, [&](int) { return CM{cnt, 0u}; }, CM{}, false, need, s.sc, &acc);
  __syncthreads();
  if ((int)threadIdx.x == t) {
    uint64_t seen = acc.c;
    for (int64_t i = c0; i < c1; ++i) {
      if (c.w.keys[i] == key && ++seen == need) {
        s.sc.item = (int)i;
        break;
      }
    }
  }
  __syncthreads();
  const int id = s.sc.item;
  return id < 0 ? 0xffffffffu : (uint32_t)id;
}

// The n (<= CAPG) kept ids gathered into s.list as key << 32 | ~id and sorted
// descending (bitonic, in LDS): descending score, ascending id among ties.
__device__ void gather_sorted(const Ctx& c, const Filter& f, int n, PickLds& s, uint64_t* red) {
  const int tid = threadIdx.x;
  const int fb1 = (int)(f.lo >> SH1);
  Src src{c.w.keys, nullptr, (int)c.V, (int)c.V};
  if (fb1 >= c.blo) {
    // the groups of the digits at and above the filter's
    uint64_t part = 0;
    for (int b = fb1 + tid; b < NB1; b += F_NT) part += c.w.h1c[b];
    const uint64_t n = block_sum_u64<F_NT>(part, red);
    if (n <= (uint64_t)c.V) src = Src{c.w.ckeys, c.w.cids, (int)n, (int)c.V};
  }
  __syncthreads();
  if (tid == 0) s.cnt = 0;
  __syncthreads();
  for_src(src, [&](uint32_t k) { return k >= f.lo; }, [&](uint32_t k, int i) {
    if (kept(f, k, i)) {
      const int slot = atomicAdd(&s.cnt, 1);
      if (slot < n) s.list[slot] = ((uint64_t)k << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
    }
  });
  int N = 2;
  while (N < n) N <<= 1;
  __syncthreads();
  for (int i = n + tid; i < N; i += F_NT) s.list[i] = 0u;
  __syncthreads();
  for (int k = 2; k <= N; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < N; i += F_NT) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const uint64_t x = s.list[i], y = s.list[ixj];
          if (((i & k) == 0) ? (x < y) : (x > y)) {
            s.list[i] = y;
            s.list[ixj] = x;
          }
        }
      }
      __syncthreads();
    }
  }
}

// Top-p (when use_p) and the draw over the n sorted kept ids of s.list.
__device__ int64_t finish_sorted(int n, bool use_p, float top_p, float r, float smax, PickLds& s,
                                 uint64_t* red) {
  auto key_at = [&](int j) { return (uint32_t)(s.list[j] >> 32); };
  auto item = [&](int j) { return CM{1u, mass_of(key_at(j), smax)}; };
  uint64_t part = 0;
  for (int j = threadIdx.x; j < n; j += F_NT) part += item(j).m;
  uint64_t kept_m = block_sum_u64<F_NT>(part, red);
  int m = n;
  CM acc{};
  if (use_p) {
    const int jc = find_first<F_NT>(n, item, CM{}, true, ceil_mul(top_p, kept_m), s.sc, &acc);
    if (jc >= 0) {
      // ties at the cut stay: through the last id with the cut's score
      const uint32_t kc = key_at(jc);
      m = jc + 1;
      while (m < n && key_at(m) == kc) ++m;
      kept_m = acc.m + (uint64_t)(m - jc) * mass_of(kc, smax);
    }
  }
  const int jp = find_first<F_NT>(m, item, CM{}, true, ceil_mul(r, kept_m), s.sc, &acc);
  if (jp < 0) return 0;
  return (int64_t)(0xffffffffu - (uint32_t)(s.list[jp] & 0xffffffffu));
}

__global__ void __launch_bounds__(F_NT) k_samp_pick(SampleArgs a) {
  __shared__ PickLds s;
  __shared__ uint32_t redu[F_NT / 64];
  __shared__ uint64_t red[F_NT / 64];
  const int tid = threadIdx.x;
  Ctx c;
  c.w = carve(a.ws, a.V);
  c.V = a.V;
  const Ws& w = c.w;
  const int64_t V = a.V;
  const int nb = (int)((V + SLICE - 1) / SLICE);
  c.smax = global_max_score<F_NT>(w.bmax, nb, redu);
  c.blo = (int)w.ctl[0];
  uint64_t bm = 0;
  for (int b = tid; b < nb; b += F_NT) bm += w.bmass[b];
  const uint64_t total = block_sum_u64<F_NT>(bm, red);

  int p = 0;
  float r = a.r_fixed;
  if (a.state) {
    p = a.state->pos + 1;
    const int64_t t = (int64_t)p - a.state->n_prompt;
    r = (a.rbuf && t >= 0 && t < a.nr) ? a.rbuf[t] : 0.0f;
  }
  const Mode md = mode_of(a);
  int64_t pick = 0;
  if (total == 0) {
    pick = 0;  // no finite weight (an infinite or NaN maximum): the reference's degenerate first id
  } else if (md.use_k || md.use_p) {
    Filter f;
    uint64_t kept_m = total, kept_n = (uint64_t)V;
    if (md.use_k) {
      const Sel sk = select(c, false, (uint64_t)a.top_k, f, s);
      f.on = true;
      f.lo = sk.key;
      f.part = sk.part;
      kept_m = sk.ge.m;
      kept_n = sk.ge.c;
      // ties at the k-th score beyond k: the lowest ids stay
      const uint64_t need = (uint64_t)a.top_k - (sk.ge.c - sk.eq.c);
      if (sk.eq.c > need) {
        f.id_max = nth_tied_id(c, sk.key, 0xffffffffu, need, s);
        const CM drop{sk.eq.c - need, (sk.eq.m / sk.eq.c) * (sk.eq.c - need)};
        f.part = f.part - drop;
        kept_m -= drop.m;
        kept_n -= drop.c;
      }
    }
    if (md.use_k && kept_n <= (uint64_t)CAPG) {
      // a short kept list: top-p and the draw in LDS
      gather_sorted(c, f, (int)kept_n, s, red);
      pick = finish_sorted((int)kept_n, md.use_p, a.top_p, r, c.smax, s, red);
    } else {
      if (md.use_p) {
        const Sel sp = select(c, true, ceil_mul(a.top_p, kept_m), f, s);
        if (sp.key != f.lo) f.id_max = 0xffffffffu;  // ties at the top-p cut stay together
        f.on = true;
        f.lo = sp.key;
        f.part = sp.part;
        kept_m = sp.ge.m;
        kept_n = sp.ge.c;
      }
      if (kept_n <= (uint64_t)CAPG) {
        gather_sorted(c, f, (int)kept_n, s, red);
        pick = finish_sorted((int)kept_n, false, 1.0f, r, c.smax, s, red);
      } else {
        const uint64_t tgt = ceil_mul(r, kept_m);
        const Sel sd = select(c, true, tgt, f, s);
        pick = sd.ok ? (int64_t)sd.min_id : 0;
        if (sd.ok && sd.eq.c > 1) {
          // a draw inside tied scores: the tied ids in id order, each its share
          const uint64_t each = sd.eq.m / sd.eq.c, above = sd.ge.m - sd.eq.m;
          const uint64_t t = min(tgt, kept_m);
          uint64_t nth = 1;
          if (each > 0 && t > above) nth = min(sd.eq.c, (t - above + each - 1) / each);
          if (nth > 1) pick = nth_tied_id(c, sd.key, sd.key == f.lo ? f.id_max : 0xffffffffu, nth, s);
        }
      }
    }
  } else {
    // index order: the slice, then the id, where the prefix mass reaches r
    const uint64_t tgt = ceil_mul(r, total);
    CM acc{}, acc2{};
    const int js = find_first<F_NT>(
        nb,
        [&](int j) {
          const int64_t n = min((int64_t)SLICE, V - (int64_t)j * SLICE);
          return CM{(uint64_t)n, w.bmass[j]};
        },
        CM{}, true, tgt, s.sc, &acc);
    const int64_t base = (int64_t)(js < 0 ? 0 : js) * SLICE;
    const int jj = find_first<F_NT>(
        SLICE,
        [&](int j) {
          const int64_t i = base + j;
          return i < V ? CM{1u, mass_of(w.keys[i], c.smax)} : CM{};
        },
        acc, true, tgt, s.sc, &acc2);
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
  UAII_LAUNCH(k_samp_bucket, dim3(nb), dim3(P_NT), 0, s, a);
  st = hipGetLastError();
  if (st != hipSuccess) return st;
  UAII_LAUNCH(k_samp_pick, dim3(1), dim3(F_NT), 0, s, a);
  return hipGetLastError();
}

}  // namespace uaii_hip
