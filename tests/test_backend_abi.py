"""The ROCm IBackend of libuaii_amd.so seen through the reference's own headers.

uaii::backends::RocmBackend implements the reference's uaii::IBackend
(include/uaii/interfaces/backend.hpp:29-87) from this build's restatement of
that interface (csrc/host/backend.h). A caller of the reference (its Session,
factory.cpp:52-80) is compiled against the reference's header, so the object
must be usable through the reference's vtable and types. This test compiles a
program with g++ against /root/reference/include only, links it against
libuaii_amd.so, creates the backend with the exported factory and, without a
GPU:
* calls every IBackend virtual through the reference's declaration and checks
  the result each one must give before initialize (name, device type,
  capabilities, host-fallback flags, allocate / free / copies / synchronize /
  dispatch refusing with the reference's Error codes and messages);
* calls the KvCache hooks and destroys the object through unique_ptr<IBackend>;
* prints sizeof / offsetof of TensorView, Attribute, BackendCapabilities and
  Error from the reference's headers, which must equal this build's.
Skipped when /root/reference is absent.
"""
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
REF_INCLUDE = Path("/root/reference/include")
PKG = ROOT / "universal-ai-inference_amd"
LIB = PKG / "lib" / "libuaii_amd.so"

LAYOUT = r'''
#include <cstddef>
#include <cstdio>
#define FIELD(T, m) std::printf("%s.%s %zu\n", #T, #m, offsetof(T, m))
int main() {
  using uaii::kernels::TensorView;
  using uaii::ir::Attribute;
  using uaii::BackendCapabilities;
  std::printf("TensorView %zu\n", sizeof(TensorView));
  FIELD(TensorView, dtype); FIELD(TensorView, shape); FIELD(TensorView, rank); FIELD(TensorView, data);
  FIELD(TensorView, nbytes); FIELD(TensorView, quant_format); FIELD(TensorView, quant_rows);
  FIELD(TensorView, quant_cols);
  std::printf("Attribute %zu\n", sizeof(Attribute));
  FIELD(Attribute, key); FIELD(Attribute, type); FIELD(Attribute, value);
  std::printf("BackendCapabilities %zu\n", sizeof(BackendCapabilities));
  FIELD(BackendCapabilities, name); FIELD(BackendCapabilities, device_type);
  FIELD(BackendCapabilities, supported_dtypes); FIELD(BackendCapabilities, supports_profiling);
  FIELD(BackendCapabilities, supports_async); FIELD(BackendCapabilities, host_fallback);
  FIELD(BackendCapabilities, native_available); FIELD(BackendCapabilities, attention_host_fallback);
  FIELD(BackendCapabilities, details);
  std::printf("Error %zu\n", sizeof(uaii::Error));
  return 0;
}
'''

DRIVER = r'''
#include "uaii/interfaces/backend.hpp"

#include <cstdio>
#include <memory>
#include <string>
#include <vector>

namespace uaii::backends {
// exported by libuaii_amd.so (csrc/host/rocm_backend.h)
Error create_rocm_backend(std::unique_ptr<IBackend>* out, int device);
Error rocm_configure_kv_cache(IBackend* backend, std::int64_t n_layers, std::int64_t max_seq,
                              std::int64_t kv_dim, std::int64_t n_kv_heads, bool f16);
Error rocm_reset_kv_cache(IBackend* backend);
Error rocm_commit_kv_step(IBackend* backend);
}  // namespace uaii::backends

static void show(const char* what, const uaii::Error& e) {
  std::printf("%s %d %s\n", what, static_cast<int>(e.code()), e.message().c_str());
}

int main() {
  using namespace uaii;
  std::unique_ptr<IBackend> b;
  show("create", backends::create_rocm_backend(&b, 0));
  std::printf("name %s\n", b->name().c_str());
  std::printf("device_type %d\n", static_cast<int>(b->device_type()));
  std::printf("uses_host_fallback %d\n", b->uses_host_fallback() ? 1 : 0);
  std::printf("attention_host_fallback %d\n", b->attention_host_fallback() ? 1 : 0);
  BackendCapabilities c = b->capabilities();
  std::printf("caps %s %d %zu %d %d %d %d|%s\n", c.name.c_str(), static_cast<int>(c.device_type),
              c.supported_dtypes.size(), c.supports_async ? 1 : 0, c.host_fallback ? 1 : 0,
              c.native_available ? 1 : 0, c.attention_host_fallback ? 1 : 0, c.details.c_str());
  void* p = nullptr;
  show("allocate", b->allocate(64, &p));
  show("free_null", b->free(nullptr));
  int x = 0;
  show("free_foreign", b->free(&x));
  float h[4] = {1, 2, 3, 4};
  show("copy_h2d", b->copy_h2d(h, h, 16));
  show("copy_h2d_async", b->copy_h2d_async(h, h, 16));
  show("copy_d2h", b->copy_d2h(h, h, 16));
  show("copy_d2d", b->copy_d2d(h, h, 16));
  show("synchronize", b->synchronize());
  std::int64_t shape[2] = {1, 4};
  kernels::TensorView v;
  v.dtype = DType::F32;
  v.shape = shape;
  v.rank = 2;
  v.data = h;
  v.nbytes = 16;
  std::vector<kernels::TensorView> in = {v, v}, out = {v};
  std::vector<ir::Attribute> attrs = {ir::make_bool_attr("transpose_b", true)};
  show("dispatch", b->dispatch("Add", "1", in, &out, attrs));
  show("configure_kv", backends::rocm_configure_kv_cache(b.get(), 2, 16, 64, 1, false));
  show("reset_kv", backends::rocm_reset_kv_cache(b.get()));
  show("commit_kv", backends::rocm_commit_kv_step(b.get()));
  show("reset_kv_null", backends::rocm_reset_kv_cache(nullptr));
  b->shutdown();
  b.reset();
  std::printf("destroyed\n");
  return 0;
}
'''


def _compile(tmp_path, name, src, includes, link=False):
    exe = tmp_path / name
    cpp = tmp_path / f"{name}.cpp"
    cpp.write_text(src)
    cmd = ["g++", "-std=c++17", "-O1", *[f"-I{i}" for i in includes], str(cpp), "-o", str(exe)]
    if link:
        cmd += [str(LIB), f"-Wl,-rpath,{LIB.parent}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    return exe


def _run(exe):
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, (r.returncode, r.stdout[-2000:], r.stderr[-2000:])
    return r.stdout


needs_ref = pytest.mark.skipif(not REF_INCLUDE.is_dir(), reason="reference headers absent")


@needs_ref
def test_layouts_equal_reference(tmp_path):
    ref = _compile(tmp_path, "layout_ref", '#include "uaii/interfaces/backend.hpp"\n' + LAYOUT,
                   [REF_INCLUDE])
    ours = _compile(tmp_path, "layout_ours",
                    '#define __HIP_PLATFORM_AMD__ 1\n#include "backend.h"\n' + LAYOUT,
                    [PKG / "csrc" / "host", "/opt/rocm/include"])
    a, b = _run(ref), _run(ours)
    assert a == b, f"reference:\n{a}\nthis build:\n{b}"


@needs_ref
def test_backend_through_reference_vtable(tmp_path):
    if not LIB.exists():
        pytest.skip("libuaii_amd.so not built")
    out = _run(_compile(tmp_path, "drive", DRIVER, [REF_INCLUDE], link=True))
    lines = dict(line.split(" ", 1) for line in out.strip().splitlines() if " " in line)
    assert lines["create"] == "0 "
    assert lines["name"] == "rocm"
    assert lines["device_type"] == "6"              # DeviceType::Rocm
    assert lines["uses_host_fallback"] == "0"
    assert lines["attention_host_fallback"] == "0"
    assert lines["caps"].startswith("rocm 6 2 1 0 0 0|ROCm backend (not initialized)")
    for k in ("allocate", "copy_h2d", "copy_h2d_async", "copy_d2h", "copy_d2d", "synchronize",
              "dispatch", "configure_kv"):
        assert lines[k] == "1 rocm backend not initialized", (k, lines[k])  # InvalidArgument
    assert lines["free_null"] == "0 "
    assert lines["free_foreign"] == "2 pointer not owned by ROCm backend"  # NotFound
    assert lines["reset_kv"] == "0 " and lines["commit_kv"] == "0 "
    assert lines["reset_kv_null"] == "1 not the ROCm backend of libuaii_amd"
    assert "destroyed" in out
