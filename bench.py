#!/usr/bin/env python3
"""Decode throughput of the GGUF token loop on one MI355X.

Workload: Llama-3-8B-shape decoder, Q4_0 weights, fp16 KV
cache, bs=1. A seeded random prompt fills the context to 3840 tokens, then the
timed region is K greedy decode steps ending at ctx 4096 (one step = one token
through all 32 layers + LM head + argmax, replayed from the captured hipGraph).

Also reported: the prompt prefill rate (matrix-core path, with its dominant
GEMM's fp16 MFMA roofline fraction), per-kernel device time from HIP
events on the session stream (a profiled replay of the same decode window right
after the timed region), the dominant kernel's HBM roofline fraction, a
device-to-device copy rate, the reference's CPU path timed on a bounded
window (reference kernels built from the reference sources, oracle/_ref), and
the device GEMV at the reference's one published kernel figure (Q4_0 2048x4096
on its benchmark's inputs) beside the reference kernel timed on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "universal-ai-inference_amd"))

METRIC = "decode tok/s bs1 Llama-3-8B-shape Q4_0 @ctx4096; GEMV+attn HBM GB/s % peak"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFS = 2500.0  # dense fp16 matrix-core peak of one MI355X


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def traffic_record(kernel: str):
    """The committed counter record of a step role, when it was taken on kernel
    sources identical to this tree's (sha1 of the role's sources); else None."""
    from uaii_amd import pmc
    try:
        sha = pmc.source_sha(kernel)
    except OSError:
        return None
    for f in sorted((ROOT / "profiles").glob(f"traffic_{kernel}_*.json")):
        try:
            t = json.loads(f.read_text())
        except (OSError, ValueError):
            continue
        if t.get("bench_kernel") == kernel and t.get("source_sha1") == sha:
            return t
    return None


def measured_traffic(kernel: str, algo_bytes: float):
    """HBM bytes per launch of the step role `kernel` from the committed counter
    runs (profiles/traffic_<role>_*.json: FETCH_SIZE + WRITE_SIZE, scaled by the
    copy kernel), when they were taken on the same shape and on kernel sources
    identical to this tree's (sha1 of the role's sources); else None."""
    from uaii_amd import pmc
    try:
        sha = pmc.source_sha(kernel)
    except OSError:
        return None
    for f in sorted((ROOT / "profiles").glob(f"traffic_{kernel}_*.json")):
        try:
            t = json.loads(f.read_text())
        except (OSError, ValueError):
            continue
        if (t.get("bench_kernel") == kernel and t.get("source_sha1") == sha
                and abs(t["algorithmic_bytes"] - algo_bytes) <= 1e-3 * algo_bytes):
            return round(t["traffic_bytes"])
    return None


def cpu_info():
    """Host CPU model, logical CPUs of the machine, and the CPUs this process may run on."""
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count() or 0
    return model, os.cpu_count() or 0, usable


def cpu_baseline(path: str, start_pos: int, n_steps: int, threads: int):
    """Reference CPU path on a bounded decode window (rank 0, N=1)."""
    sys.path.insert(0, str(ROOT))
    import oracle  # checker / baseline only
    import ctypes as C
    os.environ["UAII_NUM_THREADS"] = str(threads)  # reference thread_pool.cpp:13-22
    R = oracle.ref()
    if R is not None:
        R.uref_time_decode_window.restype = C.c_double
        R.uref_time_decode_window.argtypes = [C.c_char_p, C.c_int64, C.c_int64]
        secs = R.uref_time_decode_window(path.encode(), start_pos, n_steps)
        kind = "reference"
        what = ("the reference's own CPU kernels (quant_gemm_f32 Path B, rmsnorm, rope, attention_kv_f32, "
                "softmax; compiled from its sources into oracle/_ref) driven op by op by this build's "
                "restatement of the gguf.cpp decode graph, not the reference's Session::run")
    else:
        secs = oracle.Model(path).time_decode_window(start_pos, n_steps, threads)
        kind = "port"
        what = "the C restatement of the reference's CPU path (oracle/uaii_oracle.c)"
    if secs <= 0:
        raise RuntimeError("cpu baseline failed")
    model, ncpu, usable = cpu_info()
    return {"value": n_steps / secs, "unit": "tok/s", "cores": threads, "kind": kind,
            "threads": threads, "nproc": ncpu, "usable_cpus": usable, "cpu_model": model,
            "sample": f"{n_steps} decode steps at ctx {start_pos}..{start_pos + n_steps} "
                      f"(KV filled with deterministic values), {secs:.1f} s wall; {what}"}


PUBLISHED_GEMV = {"shape": "Q4_0 M=1 N=2048 K=4096", "median_ms": 4.495, "trials": 10,
                  "hardware": "Intel Core i9-14900HX, 32 threads, WSL2",
                  "source": "benchmarks/results/local_wsl.json:103-111 (uaii_bench.cpp:494-566)"}


def cpu_prompt_window(path: str, prompt, n_tokens: int, threads: int, report_every: int = 0):
    """Window (i): the first n prompt tokens fed one at a time through the
    reference's compiled kernels from an empty cache (session.cpp:1006-1016)."""
    sys.path.insert(0, str(ROOT))
    import numpy as np
    import oracle  # baseline only
    import ctypes as C
    os.environ["UAII_NUM_THREADS"] = str(threads)
    R = oracle.ref()
    if R is None:
        raise RuntimeError("reference kernels not built")
    R.uref_time_prompt_window.restype = C.c_double
    R.uref_time_prompt_window.argtypes = [C.c_char_p, C.POINTER(C.c_int64), C.c_int64, C.c_int]
    p = np.ascontiguousarray(prompt[:n_tokens], dtype=np.int64)
    secs = R.uref_time_prompt_window(path.encode(), p.ctypes.data_as(C.POINTER(C.c_int64)), len(p),
                                     report_every)
    if secs <= 0:
        raise RuntimeError("cpu prompt window failed")
    return {"tokens": len(p), "seconds": round(secs, 2), "tok_s": round(len(p) / secs, 4),
            "sample": f"prompt tokens 0..{len(p) - 1} of the benchmark prompt, one run() each from an "
                      f"empty cache (the reference's prefill), the start of the 256-token window (i)"}


def cpu_full_runs(uaii_amd, threads: int, lengths):
    """Whole greedy generate runs (prompt, then decode) on the small configs: the
    reference's compiled kernels on the host cores and this build on the GPU,
    same GGUF file and prompt, ids compared."""
    sys.path.insert(0, str(ROOT))
    import numpy as np
    import oracle  # baseline only
    from uaii_amd import synth
    os.environ["UAII_NUM_THREADS"] = str(threads)
    out = {}
    for name, (n_prompt, n_new) in lengths.items():
        cfg = synth.PRESETS[name]
        path = synth.cached_model(cfg, nthreads=16)
        prompt = np.random.default_rng(cfg.seed + 1).integers(0, cfg.vocab, n_prompt).astype(np.int64)
        t0 = time.perf_counter()
        want = oracle.ref_generate(path, prompt, n_new)[0]
        cpu_s = time.perf_counter() - t0
        with uaii_amd.Session(path) as sess:
            sess.generate(prompt, n_new)  # graphs captured
            t0 = time.perf_counter()
            got = sess.generate(prompt, n_new)
            gpu_s = time.perf_counter() - t0
        out[name] = {"prompt": n_prompt, "new": n_new, "cpu_s": round(cpu_s, 3),
                     "cpu_tok_s": round((n_prompt + n_new) / cpu_s, 2), "gpu_s": round(gpu_s, 4),
                     "gpu_tok_s": round((n_prompt + n_new) / gpu_s, 1),
                     "ids_match": bool(np.array_equal(np.asarray(got), np.asarray(want)))}
    return out


def published_gemv_inputs(np):
    """The inputs of the reference's quant GEMV benchmark (uaii_bench.cpp:505-518):
    Q4_0 blocks in row-major order with d = 1.0 (0x3c00) and qs[i] = (i + block) & 0xff,
    activations a[i] = 0.01f * ((i % 17) + 1). Returns the packed rows, a, and the
    exact product (f64 over the ggml nibble order, low nibbles first)."""
    n, k = 2048, 4096
    nb = n * k // 32
    blk = np.zeros((nb, 18), np.uint8)
    blk[:, 1] = 0x3C
    blk[:, 2:] = (np.arange(16)[None, :] + np.arange(nb)[:, None]) & 0xFF
    a = np.float32(0.01) * ((np.arange(k) % 17) + 1).astype(np.float32)
    qs = blk[:, 2:].astype(np.int64)
    w = (np.concatenate([qs & 15, qs >> 4], axis=1) - 8).reshape(n, k).astype(np.float64)
    return blk.reshape(-1), a.astype(np.float32), w @ a.astype(np.float64)


def published_gemv(np, uaii_amd, iters: int = 200):
    """The device GEMV at the reference's one published hot-path shape, on that
    benchmark's inputs: HIP-event time per launch over the one matrix back to back
    (the reference benchmark reuses its matrix too) and over copies taken in turn
    that together exceed the last-level cache (each launch reads HBM), and the
    result's largest relative error against the exact product."""
    import ctypes as C
    L = uaii_amd.lib()
    packed, a, exact = published_gemv_inputs(np)
    n, k = 2048, 4096
    copies = int(np.ceil(320 * 2 ** 20 / packed.nbytes))
    ws = [uaii_amd.DeviceWeight(uaii_amd.Q4_0, packed, n, k) for _ in range(copies)]
    x = uaii_amd.DeviceBuffer.from_array(a)
    y = uaii_amd.DeviceBuffer(4 * n)
    ms_hot, ms_hbm = C.c_float(), C.c_float()
    uaii_amd.check_hip(L.uaii_hip_time_gemv(ws[0].h, x.ptr, y.ptr, iters, C.byref(ms_hot)), "time_gemv")
    hs = (C.c_void_p * copies)(*[w.h for w in ws])
    uaii_amd.check_hip(L.uaii_hip_time_gemv_rotate(hs, copies, x.ptr, y.ptr, iters, C.byref(ms_hbm)),
                       "time_gemv_rotate")
    uaii_amd.check_hip(L.uaii_hip_gemv(ws[0].h, x.ptr, y.ptr, None), "gemv")
    uaii_amd.check_hip(L.uaii_hip_synchronize())
    got = y.to_array(np.float32, n).astype(np.float64)
    err = float(np.abs(got - exact).max() / np.abs(exact).max())
    for w in ws:
        w.free()
    algo = packed.nbytes + 4 * k + 4 * n
    return {**PUBLISHED_GEMV, "reference_ms": PUBLISHED_GEMV["median_ms"],
            "gpu_us_same_matrix": round(ms_hot.value * 1e3, 2),
            "gpu_us_from_hbm": round(ms_hbm.value * 1e3, 2),
            "gpu_gbps_from_hbm": round(algo / (ms_hbm.value * 1e-3) / 1e9, 1),
            "algorithmic_bytes": algo, "weight_copies": copies,
            "max_rel_err_vs_exact": err,
            "speedup_vs_published": round(PUBLISHED_GEMV["median_ms"] / ms_hbm.value, 1)}


def published_gemv_cpu(np, threads: int):
    """The reference's quant_gemm_f32 (compiled from its sources into oracle/_ref)
    on the same inputs on this host: median of 10 trials after 5 warm-up calls, as
    uaii_bench.cpp:84-94 and :643 time it."""
    sys.path.insert(0, str(ROOT))
    import oracle  # baseline only
    import ctypes as C
    os.environ["UAII_NUM_THREADS"] = str(threads)
    R = oracle.ref()
    if R is None:
        return None
    packed, a, exact = published_gemv_inputs(np)
    n, k = 2048, 4096
    out = np.zeros(n, np.float32)
    fp = C.POINTER(C.c_float)
    args = (2, a.ctypes.data_as(fp), 1, k, packed.ctypes.data_as(C.c_void_p), n, out.ctypes.data_as(fp))
    for _ in range(5):
        if R.uref_quant_gemm(*args) != 0:
            raise RuntimeError(R.uref_last_error().decode())
    samples = []
    for _ in range(10):
        t0 = time.perf_counter()
        R.uref_quant_gemm(*args)
        samples.append((time.perf_counter() - t0) * 1e3)
    err = float(np.abs(out.astype(np.float64) - exact).max() / np.abs(exact).max())
    return {"median_ms": round(float(np.median(samples)), 4), "min_ms": round(min(samples), 4),
            "threads": threads, "max_rel_err_vs_exact": err}


def parity_check(path: str, n_prompt: int, n_new: int, layers: int, threads: int):
    """Greedy ids of the benchmarked GGUF file truncated to its first `layers`
    layers (UAII_MAX_LAYERS, gguf.cpp:785-799): the device session (f16 KV, the
    prompt on the matrix cores) against the CPU oracle with an f16 KV cache."""
    sys.path.insert(0, str(ROOT))
    import numpy as np
    import oracle  # checker only
    import uaii_amd
    prompt = np.random.default_rng(1234).integers(0, 32000, n_prompt).astype(np.int64)
    os.environ["UAII_MAX_LAYERS"] = str(layers)
    try:
        with uaii_amd.Session(path, kv_f16=True, max_context=n_prompt + n_new + 8) as s:
            got = s.generate(prompt, n_new)
    finally:
        del os.environ["UAII_MAX_LAYERS"]
    want, _ = oracle.Model(path, max_layers=layers).generate(prompt, n_new, kv_f16=True, nthreads=threads,
                                                             taps=False)
    return {"layers": layers, "prompt": n_prompt, "decoded": n_new,
            "ids_match": bool(np.array_equal(got, want)), "against": "oracle (f16 KV)"}


def sampled_rates(uaii_amd, sess, prompt, ctx: int, K: int):
    """Sampled decode rate at the headline context, host sampler (the
    reference's method: the logits row to the host each token, session.cpp:974-978)
    and device sampler (uaii_session_set_device_sampler): two seeded
    generate_sampled runs of `base` and `base + K` new tokens over the same
    prompt; K over the difference of their wall times is the per-token rate with
    the prefill cancelled out."""
    base = 8
    pr = prompt[: ctx - base - K]
    out = {"method": f"{K} tokens: wall time of generate_sampled(+{base + K}) minus (+{base}), "
                     f"prompt {len(pr)}"}
    for name, (t, tp, tk, rp) in (("T0.8_p0.9_k40", (0.8, 0.9, 40, 1.0)), ("T1_p0.9", (1.0, 0.9, 0, 1.0))):
        res, ids = {}, {}
        for mode in ("host", "device"):
            sess.set_device_sampler(mode == "device")
            prm = uaii_amd.sample_params(t, tp, tk, rp, seed=1234)
            sess.generate_sampled(pr, base, prm)  # graphs captured, buffers sized
            t0 = time.perf_counter()
            sess.generate_sampled(pr, base, prm)
            ta = time.perf_counter() - t0
            t0 = time.perf_counter()
            ids[mode] = sess.generate_sampled(pr, base + K, prm)
            tb = time.perf_counter() - t0
            res[f"{mode}_tok_s"] = round(K / (tb - ta), 1)
        sess.set_device_sampler(False)
        gh, gd = ids["host"][len(pr):].tolist(), ids["device"][len(pr):].tolist()
        same = 0
        while same < min(len(gh), len(gd)) and gh[same] == gd[same]:
            same += 1
        res["equal_leading_ids"] = same
        res["tokens"] = base + K
        out[name] = res
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=240)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--config", default="8b")
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--profile-steps", type=int, default=32)
    ap.add_argument("--cpu-steps", type=int, default=3)
    ap.add_argument("--cpu-threads", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-profile", action="store_true")
    ap.add_argument("--no-parity", action="store_true")
    ap.add_argument("--no-sampled", action="store_true")
    ap.add_argument("--cpu-prompt-tokens", type=int, default=8,
                    help="window (i): the first N prompt tokens through the reference CPU kernels")
    ap.add_argument("--cpu-1b", default="16,16", help="prompt,new tokens of the full 1B CPU run (0 skips)")
    ap.add_argument("--cpu-only", action="store_true",
                    help="only the CPU baseline windows (with --cpu-prompt-tokens / --cpu-steps)")
    ap.add_argument("--sampled-steps", type=int, default=128)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); "
              "the path has no multi-GPU mode", file=sys.stderr)
        return 2

    import numpy as np
    import uaii_amd
    from uaii_amd import synth

    cfg = synth.PRESETS[args.config]
    ctx = min(args.ctx, cfg.ctx_len)
    K, W = args.steps, args.warmup
    n_prompt = ctx - K - W
    if n_prompt < 1:
        raise SystemExit("steps + warmup must be below the context length")

    t = time.time()
    path = synth.cached_model(cfg, nthreads=16)
    log(f"model {path} ready in {time.time() - t:.1f}s")
    if args.cpu_only:
        prompt = np.random.default_rng(cfg.seed + 1).integers(0, cfg.vocab, n_prompt)
        res = {"decode_window": cpu_baseline(path, n_prompt + W + K // 2, args.cpu_steps, args.cpu_threads)}
        log(f"cpu decode window {res['decode_window']}")
        res["prompt_window"] = cpu_prompt_window(path, prompt, args.cpu_prompt_tokens, args.cpu_threads,
                                                 report_every=16)
        print(json.dumps(res), flush=True)
        return 0

    # device copy rate (HBM read+write) for context
    L = uaii_amd.lib()
    uaii_amd.check_hip(L.uaii_hip_init(0), "init")
    nb = 1 << 30
    src, dst = uaii_amd.DeviceBuffer(nb), uaii_amd.DeviceBuffer(nb)
    ms = __import__("ctypes").c_float()
    uaii_amd.check_hip(L.uaii_hip_time_copy(src.ptr, dst.ptr, nb, 10, __import__("ctypes").byref(ms)))
    copy_gbs = 2 * nb / (ms.value * 1e-3) / 1e9
    src.free(), dst.free()
    log(f"d2d copy {copy_gbs:.0f} GB/s (read+write)")
    pub = published_gemv(np, uaii_amd)
    log(f"published GEMV shape {pub}")

    t = time.perf_counter()
    sess = uaii_amd.Session(path, kv_f16=True, max_context=ctx)
    load_s = time.perf_counter() - t
    file_bytes = os.path.getsize(path)
    load = {"seconds": round(load_s, 3), "file_bytes": file_bytes,
            "gbps": round(file_bytes / load_s / 1e9, 2) if load_s > 0 else None,
            "method": "Session() on the mapped GGUF file (written on this box, so in the page cache): "
                      "per weight, 64 MB chunks copied from the mapping to a device stage and "
                      "repacked on the device; KV cache and scratch for the context included"}
    log(f"session created in {load_s:.2f}s ({load['gbps']} GB/s of GGUF file)")
    prompt = np.random.default_rng(cfg.seed + 1).integers(0, cfg.vocab, n_prompt)

    # prefill (untimed for `value`): prompt tokens 0..n-2 as M-row products on the
    # matrix cores, the last prompt token as an ordinary step with the LM head
    prefill = {}
    if sess.prefill_supported():
        sess.begin(prompt, ctx)
        sess.prefill(n_prompt - 1)  # first pass allocates the chunk buffers
        sess.begin(prompt, ctx)
        sess.sync()
        t0 = time.perf_counter()
        sess.prefill(n_prompt - 1)
        sess.step_async(True)
        sess.sync()
        prefill_s = time.perf_counter() - t0
        # the chunk DecoderProgram::prefill uses: 1024 rows, or UAII_PREFILL_CHUNK (at least 16)
        env_chunk = os.environ.get("UAII_PREFILL_CHUNK")
        chunk = max(16, int(env_chunk)) if env_chunk else 1024
        prefill["method"] = f"matrix cores (MFMA), {min(chunk, n_prompt - 1)}-token chunks"
        if not args.no_profile:
            # the same prefill profiled per kernel; it rebuilds the same KV state
            sess.begin(prompt, ctx)
            sess.set_profiling(True)
            sess.prefill(n_prompt - 1)
            pk = json.loads(sess.profile_summary())
            sess.set_profiling(False)
            sess.step_async(True)
            sess.sync()
            flops = sum(v["flops"] for v in pk.values())
            gemms = {n: v for n, v in pk.items() if n.startswith("pf_gemm")}
            dom = max(gemms, key=lambda n: gemms[n]["total_ms"])
            d = gemms[dom]
            prefill["kernel_ms"] = round(sum(v["total_ms"] for v in pk.values()), 2)
            prefill["algorithmic_tflops"] = round(flops / (prefill_s * 1e12), 1)
            prefill["roofline"] = {"bound": "mfma", "kernel": dom, "achieved": round(d["tflops"], 1),
                                   "peak": MFMA_F16_PEAK_TFS, "unit": "TFLOP/s",
                                   "frac": round(d["tflops"] / MFMA_F16_PEAK_TFS, 4),
                                   "flops_per_launch": d["flops"] / d["launches"],
                                   "avg_launch_us": round(d["avg_us"], 2)}
            prefill["kernels"] = {n: {"total_ms": round(v["total_ms"], 2), "avg_us": round(v["avg_us"], 2),
                                      "tflops": round(v["tflops"], 1), "gbps": round(v["gbps"], 1)}
                                  for n, v in pk.items()}
    else:
        # one step per prompt token (the reference's method)
        sess.begin(prompt, ctx)
        sess.sync()
        t0 = time.perf_counter()
        for i in range(n_prompt):
            sess.step_async(i == n_prompt - 1)
        sess.sync()
        prefill_s = time.perf_counter() - t0
        prefill["method"] = "token steps"
    prefill["tok_s"] = round(n_prompt / prefill_s, 1)
    prefill["seconds"] = round(prefill_s, 4)
    log(f"prefill {n_prompt} tokens in {prefill_s:.3f}s ({n_prompt / prefill_s:.0f} tok/s, "
        f"{prefill['method']}) {json.dumps({k: v for k, v in prefill.items() if k != 'kernels'})}")

    for _ in range(W):
        sess.step_async(True)
    sess.sync()

    # timed region: K decode steps (graph replays), synchronised on both sides
    uaii_amd.check_hip(L.uaii_hip_synchronize())
    t0 = time.perf_counter()
    for _ in range(K):
        sess.step_async(True)
    sess.sync()
    uaii_amd.check_hip(L.uaii_hip_synchronize())
    dt = time.perf_counter() - t0
    tok_s = K / dt
    log(f"decode {K} steps in {dt:.3f}s -> {tok_s:.1f} tok/s ({1e3 * dt / K:.3f} ms/step)")
    ids = sess.read_ids(ctx + 1)  # the prompt, then every generated id
    best, second = sess.last_margin()

    kernels = {}
    roofline = None
    P = 0
    if not args.no_profile:
        P = min(args.profile_steps, K)
        sess.seek(n_prompt + W)
        sess.set_profiling(True)
        for _ in range(P):
            sess.step_async(True)
        sess.sync()
        kernels = json.loads(sess.profile_summary())
        sess.set_profiling(False)
        ids2 = sess.read_ids(n_prompt + W + P + 1)
        replay_ok = bool(len(ids2) == n_prompt + W + P + 1 and
                         np.array_equal(ids2, ids[: n_prompt + W + P + 1]))
        log(f"profiled replay of {P} steps reproduces the ids: {replay_ok}")
        # dominant kernel by device time
        dom = max(kernels, key=lambda k: kernels[k]["total_ms"])
        k = kernels[dom]
        achieved = k["bytes"] / (k["total_ms"] * 1e-3) / 1e9
        gemv_attn = [v for n, v in kernels.items() if n.startswith("gemv") or n == "attention"]
        agg_b = sum(v["bytes"] for v in gemv_attn)
        agg_ms = sum(v["total_ms"] for v in gemv_attn)
        step_ms = sum(v["total_ms"] for v in kernels.values()) / P
        roofline = {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1),
                    "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                    "traffic": measured_traffic(dom, k["bytes"] / k["launches"]),
                    "bytes_per_launch": k["bytes"] / k["launches"],
                    "avg_launch_us": round(k["avg_us"], 2),
                    "gemv_attn_achieved": round(agg_b / (agg_ms * 1e-3) / 1e9, 1),
                    "gemv_attn_frac": round(agg_b / (agg_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                    "kernel_ms_per_step": round(step_ms, 4),
                    "profiled_steps": P, "profiled_replay_ids_match": replay_ok,
                    "traffic_over_algorithmic_by_role": {
                        n: (round(t["traffic_over_algorithmic"], 4) if t else None)
                        for n, t in ((n, traffic_record(n)) for n, v in kernels.items() if v["bytes"] > 0)}}
    sampled = None
    if not args.no_sampled:
        try:
            sampled = sampled_rates(uaii_amd, sess, prompt, ctx, args.sampled_steps)
            log(f"sampled decode {sampled}")
        except Exception as e:
            log(f"sampled decode unavailable: {e}")
            sampled = {"error": str(e)}
    sess.close()

    parity = None
    if not args.no_parity:
        try:
            parity = parity_check(path, 16, 8, 2, args.cpu_threads)
            log(f"parity {parity}")
        except Exception as e:
            log(f"parity check failed to run: {e}")
            parity = {"error": str(e)}

    cpu = None
    if not args.no_cpu_baseline:
        try:
            cpu = cpu_baseline(path, n_prompt + W + K // 2, args.cpu_steps, args.cpu_threads)
            log(f"cpu baseline {cpu}")
        except Exception as e:  # the GPU figure stands on its own
            log(f"cpu baseline unavailable: {e}")
        if cpu is not None and args.cpu_prompt_tokens > 0:
            try:
                cpu["prompt_window"] = cpu_prompt_window(path, prompt, args.cpu_prompt_tokens, args.cpu_threads)
                log(f"cpu prompt window {cpu['prompt_window']}")
            except Exception as e:
                log(f"cpu prompt window unavailable: {e}")
        if cpu is not None:
            lengths = {"tiny": (32, 64)}
            if args.cpu_1b and args.cpu_1b != "0":
                p1, n1 = (int(v) for v in args.cpu_1b.split(","))
                lengths["1b"] = (p1, n1)
            try:
                cpu["full_runs"] = cpu_full_runs(uaii_amd, args.cpu_threads, lengths)
                log(f"cpu full runs {cpu['full_runs']}")
            except Exception as e:
                log(f"cpu full runs unavailable: {e}")
        try:
            pub["cpu_reference_here"] = published_gemv_cpu(np, args.cpu_threads)
            log(f"published GEMV shape on this host {pub['cpu_reference_here']}")
        except Exception as e:
            log(f"published GEMV shape on this host unavailable: {e}")

    out = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": K,
        "warmup": W, "ms_per_step": round(1e3 * dt / K, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded N(0,0.02) weights quantized to GGUF blocks, random prompt ids)",
        "config": {"workload": f"{args.config} decode bs1, prompt {n_prompt} + {W} warmup, "
                               f"timed ctx {n_prompt + W}->{n_prompt + W + K}",
                   "weights": uaii_amd.TYPE_NAMES[cfg.type_default], "kv_cache": "f16",
                   "n_layers": cfg.n_layers, "dim": cfg.dim, "heads": f"{cfg.n_heads}/{cfg.n_kv_heads}",
                   "ffn": cfg.ffn, "vocab": cfg.vocab},
        "prefill_tok_s": round(n_prompt / prefill_s, 1),
        "prefill": prefill,
        "copy_gbps": round(copy_gbs, 1),
        "load": load,
        "published_gemv": pub,
        "argmax_margin_last": round(best - second, 6),
        "roofline": roofline,
        "kernels": {n: {"avg_us": round(v["avg_us"], 2), "gbps": round(v["gbps"], 1),
                        "bytes_per_launch": round(v["bytes"] / max(1, v["launches"])),
                        "launches_per_step": v["launches"] / max(1, P)}
                    for n, v in kernels.items()},
        "sampled_tok_s": sampled,
        "parity": parity,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
