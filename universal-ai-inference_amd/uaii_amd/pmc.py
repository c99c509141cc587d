"""HBM traffic per launch from rocprofv3 counter runs.

Two runs of the same command, one with ``--pmc FETCH_SIZE`` and one with
``--pmc WRITE_SIZE`` (kilobytes per dispatch), each scaled by what the same
counter reads for the plain copy kernel ``k_stream_copy`` of known size (read
bytes = write bytes = the copy's size), give the measured bytes per launch of a
kernel; compared with its algorithmic bytes, excess traffic means re-reads.

    python3 -m uaii_amd.pmc --fetch F.csv --write W.csv --kernel 'k_gemv<2, 3>' \\
        --copy-bytes 1073741824 --algo-bytes 66207714 --out traffic.json
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
    ap.add_argument("--kernel", required=True)
    ap.add_argument("--copy-kernel", default="k_stream_copy")
    ap.add_argument("--copy-bytes", type=float, required=True)
    ap.add_argument("--algo-bytes", type=float, required=True)
    ap.add_argument("--out")
    a = ap.parse_args(argv)
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
