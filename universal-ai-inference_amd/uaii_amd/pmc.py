"""HBM traffic per launch from rocprofv3 counter runs.

Two runs of the same command, one with ``--pmc FETCH_SIZE`` and one with
``--pmc WRITE_SIZE`` (kilobytes per dispatch), each scaled by what the same
counter reads for the plain copy kernel ``k_stream_copy`` of known size (read
bytes = write bytes = the copy's size), give the measured bytes per launch of a
kernel; compared with its algorithmic bytes, excess traffic means re-reads.

    python3 -m uaii_amd.pmc --fetch F.csv --write W.csv --kernel 'k_gemv<2, 3>' \\
        --copy-bytes 1073741824 --algo-bytes 66207714 --out traffic.json

Decode mode splits the counter runs of one eager decode (UAII_NO_GRAPH=1
bench.py) into the step's roles by kernel symbol (the ring kernel's dispatches
alternate O, down) and writes profiles/traffic_<role>_<tag>.json for each, with
the algorithmic bytes per launch from a bench.py JSON line of the same build
and the sha1 of the role's kernel sources, which bench.py checks before it
quotes a file:

    python3 -m uaii_amd.pmc --fetch F.csv --write W.csv --decode bench.json \\
        --copy-bytes 1073741824 --out-dir profiles --tag 8b_q4_0
"""
from __future__ import annotations

import argparse
import csv
import json
import statistics
import sys


def per_dispatch(path: str, counter: str):
    """{kernel name: [value per dispatch]} for one counter of a counter CSV."""
    out = {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if r.get("Counter_Name") != counter:
                continue
            out.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
    return out


def per_dispatch_ordered(path: str, counter: str):
    """{kernel name: [(dispatch id, value)]} in dispatch order."""
    out = {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if r.get("Counter_Name") != counter:
                continue
            out.setdefault(r["Kernel_Name"], []).append((int(r.get("Dispatch_Id", 0) or 0),
                                                         float(r["Counter_Value"])))
    for v in out.values():
        v.sort()
    return out


# The decode step's roles: (bench.py timing name, kernel symbol patterns, which
# dispatches of the first pattern). The attention role is the key-split kernel;
# the split merge runs in the O projection's launch (k_merge_o); the down
# projection is the split-K kernel (k_gemv_splitk).
DECODE_ROLES = [
    ("gemv_qkv", ["k_gemv<2, 2,"], None),
    ("attention", ["k_attn_h16"], None),
    ("gemv_o", ["k_merge_o"], None),
    ("gemv_gate_up", ["k_gemv<2, 3,"], None),
    ("gemv_down", ["k_gemv_splitk"], None),
    ("gemv_lm_head", ["k_gemv<2, 4,"], None),
]

# Sources each role's kernels are built from (relative to the package's csrc/hip).
ROLE_SOURCES = {
    "gemv_qkv": ["gemv.hip"], "gemv_gate_up": ["gemv.hip"], "gemv_lm_head": ["gemv.hip"],
    "gemv_o": ["attn_out.hip", "block_dot.h"], "gemv_down": ["splitk_gemv.hip", "block_dot.h"],
    "attention": ["attention.hip"],
}


def source_sha(role: str) -> str:
    """sha1 over a role's kernel sources and the headers they share."""
    import hashlib
    from pathlib import Path
    hip = Path(__file__).resolve().parent.parent / "csrc" / "hip"
    h = hashlib.sha1()
    for name in ROLE_SOURCES.get(role, []) + ["common.h", "uaii_hip_internal.h"]:
        h.update(name.encode())
        h.update((hip / name).read_bytes())
    return h.hexdigest()


def _values(d: dict, pattern: str, parity):
    hits = [k for k in d if pattern in k]
    if not hits:
        raise SystemExit(f"no kernel matching {pattern!r}; have {sorted(d)[:12]}")
    vals = sorted(v for k in hits for v in d[k])
    if parity is not None:
        vals = vals[parity::2]
    return [v for _, v in vals], hits


def decode_roles(a) -> int:
    import os
    fetch = per_dispatch_ordered(a.fetch, "FETCH_SIZE")
    write = per_dispatch_ordered(a.write, "WRITE_SIZE")
    copy_f = statistics.median(_values(fetch, a.copy_kernel, None)[0]) * 1024.0
    copy_w = statistics.median(_values(write, a.copy_kernel, None)[0]) * 1024.0
    f_scale, w_scale = a.copy_bytes / copy_f, a.copy_bytes / copy_w
    with open(a.decode) as f:
        bench = json.loads(f.read().strip().splitlines()[-1])
    kernels = bench["kernels"]
    summary = {}
    for role, patterns, parity in DECODE_ROLES:
        if role not in kernels:
            continue
        kf = kw = 0.0
        symbols, n = [], 0
        for pat in patterns:
            fv, hits = _values(fetch, pat, parity)
            wv, _ = _values(write, pat, parity)
            kf += statistics.median(fv) * 1024.0
            kw += statistics.median(wv) * 1024.0
            symbols += hits
            n = len(fv)
        algo = kernels[role]["bytes_per_launch"]
        res = {
            "role": role, "bench_kernel": role, "kernel_symbols": sorted(set(symbols)),
            "source_sha1": source_sha(role), "dispatches": n,
            "fetch_bytes_raw": kf, "write_bytes_raw": kw,
            "copy_fetch_bytes_raw": copy_f, "copy_write_bytes_raw": copy_w,
            "fetch_scale": f_scale, "write_scale": w_scale,
            "traffic_bytes": kf * f_scale + kw * w_scale, "algorithmic_bytes": algo,
            "avg_launch_us_bench": kernels[role]["avg_us"],
            "workload": bench["config"]["workload"],
            "command": a.command,
        }
        res["traffic_over_algorithmic"] = res["traffic_bytes"] / algo
        summary[role] = {"traffic_MB": round(res["traffic_bytes"] / 1e6, 3),
                         "algorithmic_MB": round(algo / 1e6, 3),
                         "ratio": round(res["traffic_over_algorithmic"], 4)}
        if a.out_dir:
            with open(os.path.join(a.out_dir, f"traffic_{role}_{a.tag}.json"), "w") as f:
                f.write(json.dumps(res, indent=1) + "\n")
    print(json.dumps(summary, indent=1))
    return 0


def pick(d: dict, pattern: str):
    hits = [k for k in d if pattern in k]
    if not hits:
        raise SystemExit(f"no kernel matching {pattern!r}; have {sorted(d)[:8]}")
    vals = []
    for k in hits:
        vals += d[k]
    return vals


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--fetch", required=True)
    ap.add_argument("--write", required=True)
    ap.add_argument("--kernel")
    ap.add_argument("--decode", help="bench.py JSON line of the same build: split by decode role")
    ap.add_argument("--out-dir")
    ap.add_argument("--tag", default="8b_q4_0")
    ap.add_argument("--command", default="")
    ap.add_argument("--copy-kernel", default="k_stream_copy")
    ap.add_argument("--copy-bytes", type=float, required=True)
    ap.add_argument("--algo-bytes", type=float)
    ap.add_argument("--out")
    a = ap.parse_args(argv)
    if a.decode:
        return decode_roles(a)
    if not a.kernel or a.algo_bytes is None:
        ap.error("--kernel and --algo-bytes are required without --decode")
    fetch = per_dispatch(a.fetch, "FETCH_SIZE")
    write = per_dispatch(a.write, "WRITE_SIZE")
    copy_f = statistics.median(pick(fetch, a.copy_kernel)) * 1024.0
    copy_w = statistics.median(pick(write, a.copy_kernel)) * 1024.0
    k_f = statistics.median(pick(fetch, a.kernel)) * 1024.0
    k_w = statistics.median(pick(write, a.kernel)) * 1024.0
    f_scale, w_scale = a.copy_bytes / copy_f, a.copy_bytes / copy_w
    res = {
        "kernel": a.kernel,
        "dispatches": len(pick(fetch, a.kernel)),
        "fetch_bytes_raw": k_f, "write_bytes_raw": k_w,
        "copy_fetch_bytes_raw": copy_f, "copy_write_bytes_raw": copy_w,
        "fetch_scale": f_scale, "write_scale": w_scale,
        "traffic_bytes": k_f * f_scale + k_w * w_scale,
        "algorithmic_bytes": a.algo_bytes,
    }
    res["traffic_over_algorithmic"] = res["traffic_bytes"] / a.algo_bytes
    js = json.dumps(res, indent=1)
    if a.out:
        with open(a.out, "w") as f:
            f.write(js + "\n")
    print(js)
    return 0


if __name__ == "__main__":
    sys.exit(main())
