"""Kernel microbenchmark through the uaii_hip C ABI.

Times one fused GEMV (plain, RMSNorm, residual add or gate/up SwiGLU) of a given
GGUF type and shape on random block bytes (or, with --m > 1, the prefill MFMA
GEMM with the same epilogues), rotating over enough weight copies
(> 256 MiB in total, the MI355X last-level cache) that each launch reads its
weights from HBM, plus the plain 1 GiB copy kernel. Meant to run alone or under
``rocprofv3 --kernel-trace --stats`` / ``--pmc`` to pin a kernel's time and
memory traffic.

    python3 -m uaii_amd.kbench --epi swiglu --type q4_0 --rows 14336 --cols 4096

``--floor`` instead times the per-launch floor: a plain read kernel in the
decode GEMVs' launch shape over each decode kernel's byte count of the 8B Q4_0
step (rotating over buffers that together exceed the last-level cache).

    python3 -m uaii_amd.kbench --floor
"""
from __future__ import annotations

import argparse
import ctypes as C
import sys
import time

import numpy as np

from . import (BLOCK, DeviceBuffer, DeviceWeight, TYPE_NAMES, check_hip, lib, row_bytes)

BPW = {k: BLOCK[k][1] / BLOCK[k][0] for k in BLOCK}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--epi", choices=["plain", "rmsnorm", "add", "swiglu"], default="swiglu")
    ap.add_argument("--type", default="q4_0")
    ap.add_argument("--rows", type=int, default=14336, help="output rows (per weight for swiglu)")
    ap.add_argument("--cols", type=int, default=4096)
    ap.add_argument("--iters", type=int, default=40)
    ap.add_argument("--copy-mib", type=int, default=1024)
    ap.add_argument("--m", type=int, default=1,
                    help="activation rows: 1 = decode GEMV, > 1 = prefill MFMA GEMM (TFLOP/s)")
    ap.add_argument("--floor", action="store_true",
                    help="plain-read per-launch floor over the 8B decode kernels' byte counts")
    ap.add_argument("--floor-case", help="with --floor: only the case of this name (e.g. 'LM head')")
    a = ap.parse_args(argv)
    if a.floor:
        return floor(a.iters, a.floor_case)
    names = {v.lower(): k for k, v in TYPE_NAMES.items()}
    t = names[a.type.lower()]
    L = lib()
    check_hip(L.uaii_hip_init(0), "init")
    rng = np.random.default_rng(0)
    nw = 2 if a.epi == "swiglu" else 1
    wbytes = nw * a.rows * row_bytes(t, a.cols)
    copies = max(2, int(np.ceil(320 * 2 ** 20 / wbytes)))
    ws = []
    for c in range(copies):
        group = []
        for _ in range(nw):
            p = rng.integers(0, 256, size=a.rows * row_bytes(t, a.cols), dtype=np.uint8)
            blk = p.reshape(-1, BLOCK[t][1])
            blk[:, 1] &= 0x3b  # small finite f16 scales at byte 0..1 for the 32-blocks
            group.append(DeviceWeight(t, p, a.rows, a.cols))
        ws.append(group)
    x = DeviceBuffer.from_array(rng.normal(0, 1, a.m * a.cols).astype(np.float32))
    nrm = DeviceBuffer.from_array(np.ones(a.cols, np.float32))
    y = DeviceBuffer.from_array(np.zeros(a.m * a.rows, np.float32))

    def launch(g):
        if a.m > 1:
            if a.epi == "plain":
                return L.uaii_hip_gemm(g[0].h, x.ptr, a.m, y.ptr, None)
            if a.epi == "rmsnorm":
                return L.uaii_hip_gemm_rmsnorm(g[0].h, x.ptr, a.m, nrm.ptr, 1e-5, y.ptr, None)
            if a.epi == "add":
                return L.uaii_hip_gemm_add(g[0].h, x.ptr, a.m, None, 1e-5, y.ptr, None)
            return L.uaii_hip_gemm_swiglu(g[0].h, g[1].h, x.ptr, a.m, nrm.ptr, 1e-5, y.ptr, None)
        if a.epi == "plain":
            return L.uaii_hip_gemv(g[0].h, x.ptr, y.ptr, None)
        if a.epi == "rmsnorm":
            return L.uaii_hip_gemv_rmsnorm(g[0].h, x.ptr, nrm.ptr, 1e-5, y.ptr, None)
        if a.epi == "add":
            return L.uaii_hip_gemv_add(g[0].h, x.ptr, None, 1e-5, y.ptr, None)
        return L.uaii_hip_gemv_swiglu(g[0].h, g[1].h, x.ptr, nrm.ptr, 1e-5, y.ptr, None)

    for g in ws:  # warm
        check_hip(launch(g), "gemv")
    check_hip(L.uaii_hip_synchronize())
    t0 = time.perf_counter()
    for i in range(a.iters):
        check_hip(launch(ws[i % copies]), "gemv")
    check_hip(L.uaii_hip_synchronize())
    dt = (time.perf_counter() - t0) / a.iters
    if a.m > 1:
        flops = 2.0 * nw * a.m * a.rows * a.cols
        print(f"gemm {a.epi} {TYPE_NAMES[t]} M={a.m} {nw}x{a.rows}x{a.cols}: {dt * 1e6:.1f} us/launch "
              f"wall (activation prep included), {flops / dt / 1e12:.1f} TFLOP/s algorithmic", flush=True)
        return 0
    algo = nw * (a.rows * a.cols * BPW[t] + 4 * a.cols + 4 * a.rows)
    print(f"gemv {a.epi} {TYPE_NAMES[t]} {nw}x{a.rows}x{a.cols}: {dt * 1e6:.2f} us/launch wall, "
          f"{algo / dt / 1e9:.0f} GB/s algorithmic ({algo:.0f} B), {copies} weight copies", flush=True)
    nb = a.copy_mib * 2 ** 20
    src, dst = DeviceBuffer(nb), DeviceBuffer(nb)
    ms = C.c_float()
    check_hip(L.uaii_hip_time_copy(src.ptr, dst.ptr, nb, 10, C.byref(ms)), "copy")
    print(f"copy {a.copy_mib} MiB: {ms.value * 1e3:.1f} us, {2 * nb / (ms.value * 1e-3) / 1e9:.0f} GB/s (r+w)",
          flush=True)
    return 0


# Bytes per launch of the 8B Q4_0 decode kernels at ctx 4096 (algorithmic bytes).
FLOOR_CASES = [("O", 9.44e6), ("QKV", 14.17e6), ("attention K+V", 16.8e6), ("down", 33.0e6),
               ("gate+up", 66.1e6), ("LM head", 295.5e6)]


def floor(iters: int, only: str | None = None) -> int:
    """Average time of a plain read of each case's bytes, one launch after
    another, rotating over enough buffers (> 320 MiB) that every launch reads
    HBM. Prints one line per case and the per-token sum (32 layers of the five
    layer reads + the LM head)."""
    L = lib()
    check_hip(L.uaii_hip_init(0), "init")
    total_us = 0.0
    for name, nbytes in FLOOR_CASES:
        if only and name != only:
            continue
        nb = int(nbytes) // 16 * 16
        copies = max(2, int(np.ceil(320 * 2 ** 20 / nb)))
        bufs = [DeviceBuffer(nb) for _ in range(copies)]
        for b in bufs:
            b.zero()
        ptrs = (C.c_void_p * copies)(*[b.ptr for b in bufs])
        ms = C.c_float()
        check_hip(L.uaii_hip_time_read(ptrs, copies, nb, iters, C.byref(ms)), "read")
        us = ms.value * 1e3
        total_us += us * (1 if name == "LM head" else 32)
        print(f"floor {name:14s} {nb / 1e6:7.2f} MB: {us:7.2f} us/launch, {nb / us / 1e3:6.0f} GB/s, "
              f"{copies} buffers", flush=True)
        del bufs
    print(f"floor per token (32 x (O + QKV + attention + down + gate+up) + LM head): {total_us / 1e3:.3f} ms "
          f"= {1e6 / total_us:.0f} tok/s", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
