"""The C++ Session route of the repository's integration notes builds and links.

Section 3 of the integration notes at the repository root gives the branch a
maintainer would add to the reference's `Session::generate`
(include/uaii/runtime/session.hpp:131-136, routing `backend_name == "rocm"`,
session.hpp:50) so that it calls this build's `uaii_session_generate`. This test
takes that snippet out of the notes themselves, so the document and the test
cannot drift apart. It compiles the snippet with
g++ against the reference's own headers, links it against libuaii_amd.so and
runs it on the CPU:
* with `backend_name = "cpu"` the branch is skipped (the driver then returns
  its own NotImplemented marker);
* with `"rocm"` and a null session handle, the C ABI's status
  (UAII_ERR_INVALID_ARGUMENT, capi.cpp:235-259) comes back as the reference's
  `Error` with `ErrorCode::InvalidArgument` (error.hpp:12-55) and the ABI's
  message.
No GPU call is made. Skipped when /root/reference is absent.
"""
import os
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
REF_INCLUDE = Path("/root/reference/include")
LIB = ROOT / "universal-ai-inference_amd" / "lib" / "libuaii_amd.so"

DRIVER = r'''
#include "uaii/runtime/session.hpp"
#include "uaii/c_api/uaii.h"

#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

namespace uaii::runtime {
// The members the snippet reads (options_, rocm_session_) and the arguments of
// Session::generate, bound as parameters of a free function.
Error routed_generate(const SessionOptions& options_, uaii_session* rocm_session_,
                      const std::vector<std::int64_t>& prompt_tokens, std::int64_t max_new_tokens,
                      std::vector<std::int64_t>* out_tokens) {
@SNIPPET@
  return Error::make(ErrorCode::NotImplemented, "not routed");
}
}  // namespace uaii::runtime

int main() {
  using namespace uaii;
  runtime::SessionOptions o;
  std::vector<std::int64_t> prompt = {1, 2, 3}, out;
  o.backend_name = "cpu";
  const Error a = runtime::routed_generate(o, nullptr, prompt, 4, &out);
  o.backend_name = "rocm";
  const Error b = runtime::routed_generate(o, nullptr, prompt, 4, &out);
  std::printf("cpu %d rocm %d %s\n", static_cast<int>(a.code()), static_cast<int>(b.code()),
              b.message().c_str());
  return 0;
}
'''


def snippet() -> str:
    text = (ROOT / "INTEGRATION.md").read_text()
    sec = text.split("## 3.", 1)[1].split("\n## 4.", 1)[0]
    m = re.search(r"```cpp\n(.*?)```", sec, re.S)
    assert m, "section 3 of the integration notes holds no cpp block"
    return m.group(1)


@pytest.mark.skipif(not REF_INCLUDE.is_dir(), reason="reference headers absent")
def test_session_route_snippet_builds_links_and_maps_status(tmp_path):
    if not LIB.exists():
        pytest.skip("libuaii_amd.so not built")
    body = snippet()
    assert "uaii_session_generate" in body and 'backend_name == "rocm"' in body
    src = tmp_path / "route.cpp"
    src.write_text(DRIVER.replace("@SNIPPET@", body))
    exe = tmp_path / "route"
    cmd = ["g++", "-std=c++17", "-Wall", "-Werror=return-type", f"-I{REF_INCLUDE}", f"-I{ROOT / 'include'}",
           str(src), "-o", str(exe), f"-L{LIB.parent}", "-luaii_amd", f"-Wl,-rpath,{LIB.parent}",
           "-Wl,-rpath,/opt/rocm/lib", "-L/opt/rocm/lib", "-lamdhip64"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    env = dict(os.environ)
    env.setdefault("HIP_VISIBLE_DEVICES", "")
    r = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=60)
    assert r.returncode == 0, r.stderr[-2000:]
    parts = r.stdout.split(maxsplit=4)
    # the unrouted call falls through to the driver's marker (NotImplemented = 7);
    # the routed one returns the ABI's status as InvalidArgument = 1 with its message
    assert parts[:4] == ["cpu", "7", "rocm", "1"], r.stdout
    assert "null" in parts[4], r.stdout
