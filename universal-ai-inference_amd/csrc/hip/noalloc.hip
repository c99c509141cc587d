// noalloc.hip — decode attention that allocates nothing (uaii_hip_attention_decode_noalloc).
//
// uaii_hip_attention_decode keeps its split-K partials in a library buffer that
// grows with hipMalloc. Callers that may not allocate (code under stream capture,
// allocation-free serving loops) use this variant instead: the same kernels, with
// the partials in `scratch`, a file-scope device array of kScratchBytes that each
// GPU holds for the life of the process.
//
// The array's name is a host-side stand-in in host code; the device address comes
// from hipGetSymbolAddress, taken once per device with that device current (in
// uaii_hip_init, or on the entry point's first call on a device) and kept in
// g_scratch_dev. Only that address is ever passed to a kernel.
//
// Every call on a GPU shares that GPU's array: two calls that overlap on one GPU
// (different streams, no ordering between them) race on it. The kernels write
// every partial they read within one call, so nothing needs clearing between calls.
#include "uaii_hip.h"

#include "uaii_hip_internal.h"

#include <mutex>

namespace {

constexpr size_t kScratchBytes = size_t(2) << 20;  // 2 MiB of split partials per GPU
constexpr int kMaxDevices = 64;
constexpr int kErrArg = -1;
constexpr int kErrScratch = -3;  // the call needs more than kScratchBytes

// `used`: no kernel names the array, and the device compiler would otherwise drop it
// (hipGetSymbolAddress then finds nothing).
static __device__ __attribute__((used)) __align__(256) float scratch[kScratchBytes / sizeof(float)];

std::mutex g_mu;
float* g_scratch_dev[kMaxDevices] = {};

// Device address of `scratch` on the current device (resolved on first use).
hipError_t scratch_ptr(float** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_scratch_dev[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_dev[dev];
  return hipSuccess;
}

}  // namespace

namespace uaii_hip {

// Called by uaii_hip_init with `device` current.
hipError_t prepare_noalloc() {
  float* p = nullptr;
  return scratch_ptr(&p);
}

size_t noalloc_scratch_bytes() { return kScratchBytes; }

}  // namespace uaii_hip

extern "C" {

int uaii_hip_attention_decode_noalloc(const float* q, const void* kcache, const void* vcache,
                                      int kv_f16, int64_t max_seq, int n_heads, int n_kv_heads,
                                      int head_dim, int64_t n_keys, float* out, void* stream) {
  if (!q || !kcache || !vcache || !out || n_heads <= 0 || n_kv_heads <= 0 ||
      n_heads % n_kv_heads || head_dim <= 0 || n_keys <= 0 || n_keys > max_seq ||
      max_seq > INT32_MAX)  // key positions are 32-bit in the kernels
    return kErrArg;
  const int splits = uaii_hip::attention_splits(max_seq);
  const int G = n_heads / n_kv_heads;
  const size_t part = (size_t)n_kv_heads * (size_t)splits * (size_t)G * (size_t)(head_dim + 2) * 4;
  if (part > kScratchBytes) return kErrScratch;
  float* p = nullptr;
  const hipError_t e = scratch_ptr(&p);
  if (e != hipSuccess) return (int)e;
  uaii_hip::AttnArgs a{};
  a.q = q;
  a.kcache = kcache;
  a.vcache = vcache;
  a.kv_f16 = kv_f16;
  a.max_seq = max_seq;
  a.n_heads = n_heads;
  a.n_kv = n_kv_heads;
  a.hd = head_dim;
  a.state = nullptr;
  a.fixed_len = (int)n_keys;
  a.out = out;
  a.part = p;
  a.splits = splits;
  return (int)uaii_hip::launch_attention_decode(a, static_cast<hipStream_t>(stream));
}

}  // extern "C"
