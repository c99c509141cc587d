"""Every BASELINE workload shape under GPU parity, through the C ABI.

* Decode attention at the headline context: max_seq 4096 gives 32 key splits
  per kv head (the merge of 32 partials), checked against the oracle's
  attention_kv_f32 restatement (transformer.cpp:222-433) at 1, 2049, 4090 and
  4096 keys, 32 or 64 query heads over 8 kv heads, head_dim 64 / 128, f16 and
  f32 caches.
* The split merge fused with the O projection and residual add
  (uaii_hip_attention_o) at the 8B, 1B and wider shapes: the merged output the
  same bits as the two-launch attention's, y within 1e-5 of the oracle's
  quant_gemm_f32 of it plus the residual.
* The Llama-3-8B shape (Q4_0 and Q8_0), two layers of it at full width with a
  4096-position KV cache: a 96-token prompt on the matrix cores, then 64 greedy
  tokens; ids identical to the oracle with an fp16 cache, logits and the
  residual taps within 2e-3 of it, and of the oracle's f32-cache path (the
  reference's own cache type) over a shorter run.
* The Llama-3.2-1B shape at full depth (16 layers, Q4_K + Q6_K, tied):
  128-token prompt, 64 greedy tokens.
* The same two layers at the headline length: a 4032-token prompt on the matrix
  cores, then 64 greedy tokens to a full 4096-position cache.
* The Mixtral shape (8 experts, top-2, Q4_K, d 4096, ffn 14336), one layer:
  64-token prompt, 64 greedy tokens against the oracle's Path A MoE (the only
  path on which the reference's experts run, transformer.cpp:522-612).

Reference loop for every model: session.cpp:1006-1044 (prompt, then greedy
argmax over probs, lowest index on ties).
"""
import ctypes as C
import dataclasses
import os

import numpy as np
import pytest

import oracle
import uaii_amd
from uaii_amd import synth, DeviceBuffer, check_hip

pytestmark = pytest.mark.gpu

THREADS = max(1, min(16, os.cpu_count() or 1))

SHAPES = {
    "8b_q4_0": dataclasses.replace(synth.PRESETS["8b"], n_layers=2),
    "8b_q8_0": dataclasses.replace(synth.PRESETS["8b_q8"], n_layers=2),
    "1b": synth.PRESETS["1b"],
    "mx": dataclasses.replace(synth.PRESETS["mx"], n_layers=1),
}


def maxrel(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max() / max(np.abs(b).max(), 1e-30))


def check_attention_decode(hip, nh, nkv, hd, kv_f16, max_seq, n_keys, seed):
    """uaii_hip_attention_decode on seeded q, K, V against the oracle's
    attention_kv_f32 restatement (the past n_keys - 1 keys, then the current one)."""
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal((nkv, max_seq, hd)).astype(np.float32)
    v = rng.standard_normal((nkv, max_seq, hd)).astype(np.float32)
    if kv_f16:
        k, v = k.astype(np.float16), v.astype(np.float16)
    dq, dk, dv = DeviceBuffer.from_array(q), DeviceBuffer.from_array(k), DeviceBuffer.from_array(v)
    do = DeviceBuffer(nh * hd * 4)
    check_hip(hip.uaii_hip_attention_decode(dq.ptr, dk.ptr, dv.ptr, kv_f16, max_seq, nh, nkv, hd,
                                            n_keys, do.ptr, None))
    got = do.to_array(np.float32, nh * hd)
    # oracle layout [seq][kv_dim]: the past n_keys - 1 keys, then the current one
    kf = k.astype(np.float32).transpose(1, 0, 2).reshape(max_seq, nkv * hd)
    vf = v.astype(np.float32).transpose(1, 0, 2).reshape(max_seq, nkv * hd)
    past = max(n_keys - 1, 1)
    kc, vc = np.ascontiguousarray(kf[:past]), np.ascontiguousarray(vf[:past])
    kn, vn = np.ascontiguousarray(kf[n_keys - 1]), np.ascontiguousarray(vf[n_keys - 1])
    want = np.zeros(nh * hd, np.float32)
    oracle.oracle().orc_attention_decode(oracle._fp(q), oracle._fp(kc), oracle._fp(vc), n_keys - 1,
                                         oracle._fp(kn), oracle._fp(vn), oracle._fp(want), nh, nkv, hd)
    assert maxrel(got, want) < 1e-5
    if n_keys == 1:
        assert maxrel(got, np.repeat(vf[0].reshape(nkv, hd), nh // nkv, axis=0).reshape(-1)) < 1e-6


@pytest.mark.parametrize("kv_f16", [1, 0])
@pytest.mark.parametrize("heads", [(32, 8, 128), (64, 8, 128), (32, 8, 64)], ids=str)
@pytest.mark.parametrize("n_keys", [1, 2049, 4090, 4096])
def test_attention_decode_32_splits(hip, kv_f16, heads, n_keys):
    nh, nkv, hd = heads
    check_attention_decode(hip, nh, nkv, hd, kv_f16, 4096, n_keys, n_keys * 13 + nh + hd)


@pytest.mark.parametrize("heads", [(32, 8, 128), (32, 8, 64)], ids=str)
@pytest.mark.parametrize("n_keys", [4097, 4224, 6000, 8192, 12289])
def test_attention_decode_several_tiles_per_wave(hip, heads, n_keys):
    """A cache past 4096 positions (12800): 32 splits of 129 .. 385 keys, so the
    f16 kernel's waves walk 2 to 4 tiles with their two register sets in turn
    (odd and even tile counts, a last pass with a single key)."""
    nh, nkv, hd = heads
    check_attention_decode(hip, nh, nkv, hd, 1, 12800, n_keys, n_keys * 13 + nh + hd + 1)


def check_attention_o(hip, nh, nkv, hd, kv_f16, max_seq, n_keys, rows, seed, t=uaii_amd.Q4_0):
    """uaii_hip_attention_o: its attention output the same bits as
    uaii_hip_attention_decode's, and y = y0 + W_o . out within 1e-5 of the
    oracle's quant_gemm_f32 of that output plus y0 (quant_gemm.cpp:22-70,
    elementwise.cpp:99-110). A second call from the same y0 agrees with the
    first to 1e-6 (its float atomics add in arrival order)."""
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal((nkv, max_seq, hd)).astype(np.float32)
    v = rng.standard_normal((nkv, max_seq, hd)).astype(np.float32)
    if kv_f16:
        k, v = k.astype(np.float16), v.astype(np.float16)
    packed = synth.quantize(t, synth.normals(seed, 0, 0, rows * nh * hd, 0.02))
    w = uaii_amd.DeviceWeight(t, packed, rows, nh * hd)
    y0 = rng.standard_normal(rows).astype(np.float32)
    dq, dk, dv = DeviceBuffer.from_array(q), DeviceBuffer.from_array(k), DeviceBuffer.from_array(v)
    do, do2 = DeviceBuffer(nh * hd * 4), DeviceBuffer(nh * hd * 4)
    ys = []
    for _ in range(2):
        dy = DeviceBuffer.from_array(y0)
        check_hip(hip.uaii_hip_attention_o(dq.ptr, dk.ptr, dv.ptr, kv_f16, max_seq, nh, nkv, hd, n_keys,
                                           w.h, do.ptr, dy.ptr, None), "attention_o")
        ys.append(dy.to_array(np.float32, rows))
    check_hip(hip.uaii_hip_attention_decode(dq.ptr, dk.ptr, dv.ptr, kv_f16, max_seq, nh, nkv, hd,
                                            n_keys, do2.ptr, None), "attention_decode")
    out, out2 = do.to_array(np.float32, nh * hd), do2.to_array(np.float32, nh * hd)
    assert np.array_equal(out.view(np.uint32), out2.view(np.uint32))
    want = y0 + oracle.quant_gemm(t, out2, packed, rows, nthreads=THREADS)[0]
    assert maxrel(ys[0], want) < 1e-5
    assert maxrel(ys[1], ys[0]) < 1e-6


@pytest.mark.parametrize("case", [
    (32, 8, 128, 1, 4096, 4096, 4096),     # 8B: 16 slices of 2 heads, 128-row blocks
    (32, 8, 128, 1, 4096, 1, 4096),        # one key: the merge of a single split
    (32, 8, 64, 1, 4096, 4090, 2048),      # 1B: 8 slices of 4 heads, 32-row blocks
    (64, 8, 128, 0, 4096, 2049, 8192),     # G = 8, f32 cache, q_dim 8192
    (8, 8, 128, 1, 12800, 12289, 96),      # G = 1, 4 slices, 3 row blocks
    (16, 2, 128, 1, 640, 300, 160),        # G = 8 over 5 splits, 5 row blocks
], ids=str)
def test_attention_o(hip, case):
    nh, nkv, hd, kv_f16, max_seq, n_keys, rows = case
    check_attention_o(hip, nh, nkv, hd, kv_f16, max_seq, n_keys, rows, nh * 7 + hd + n_keys + rows)


@pytest.mark.parametrize("case", [
    (32, 8, 128, 1, 4096, 4096, 4096),     # the 8B shape with Q8_0 weights
    (32, 8, 64, 1, 4096, 2049, 2048),      # 4 heads per slice
    (32, 8, 128, 0, 4096, 300, 96),        # f32 cache, 3 row blocks
], ids=str)
def test_attention_o_q8_0(hip, case):
    """uaii_hip_attention_o with a Q8_0 W_o (32 payload bytes per block)."""
    nh, nkv, hd, kv_f16, max_seq, n_keys, rows = case
    check_attention_o(hip, nh, nkv, hd, kv_f16, max_seq, n_keys, rows, nh * 5 + hd + n_keys + rows,
                      t=uaii_amd.Q8_0)


@pytest.mark.parametrize("case", [
    (32, 8, 64, 1, 2048, 1800, 2048),      # the 1B shape: one super-block per 4-head slice
    (32, 8, 128, 1, 4096, 4096, 4096),     # 2 heads per super-block
    (32, 8, 128, 0, 4096, 300, 96),        # f32 cache, 3 row blocks
], ids=str)
def test_attention_o_q4_k(hip, case):
    """uaii_hip_attention_o with a Q4_K W_o: each lane takes one 32-element
    sub-block (its own 6-bit scale and min) of the slice's super-block."""
    nh, nkv, hd, kv_f16, max_seq, n_keys, rows = case
    check_attention_o(hip, nh, nkv, hd, kv_f16, max_seq, n_keys, rows, nh * 3 + hd + n_keys + rows,
                      t=uaii_amd.Q4_K)


def test_attention_o_refuses_unsupported_shapes(hip):
    """W_o other than Q4_0, Q8_0 or Q4_K, rows not a multiple of 32, head_dim
    other than 64 or 128, n_heads * head_dim not a multiple of 256, or `out`
    overlapping y: -1 before any launch."""
    nh, nkv, hd, max_seq = 32, 8, 128, 256
    buf = DeviceBuffer(nkv * max_seq * hd * 4)
    out, y = DeviceBuffer(nh * hd * 4), DeviceBuffer(8192 * 4)
    x = synth.normals(3, 0, 0, 96 * nh * hd, 0.02)
    bad = [uaii_amd.DeviceWeight(uaii_amd.Q6_K, synth.quantize(uaii_amd.Q6_K, x[: 64 * nh * hd]), 64, nh * hd),
           uaii_amd.DeviceWeight(uaii_amd.Q4_0, synth.quantize(uaii_amd.Q4_0, x[: 48 * nh * hd]), 48, nh * hd)]
    for w in bad:
        assert hip.uaii_hip_attention_o(buf.ptr, buf.ptr, buf.ptr, 1, max_seq, nh, nkv, hd, 10, w.h, out.ptr,
                                        y.ptr, None) == -1
    w96 = uaii_amd.DeviceWeight(uaii_amd.Q4_0, synth.quantize(uaii_amd.Q4_0, x[: 32 * 24 * 96]), 32, 24 * 96)
    assert hip.uaii_hip_attention_o(buf.ptr, buf.ptr, buf.ptr, 1, max_seq, 24, 8, 96, 10, w96.h, out.ptr,
                                    y.ptr, None) == -1  # head_dim 96
    w4 = uaii_amd.DeviceWeight(uaii_amd.Q4_0, synth.quantize(uaii_amd.Q4_0, x[: 32 * 6 * 64]), 32, 6 * 64)
    assert hip.uaii_hip_attention_o(buf.ptr, buf.ptr, buf.ptr, 1, max_seq, 6, 2, 64, 10, w4.h, out.ptr,
                                    y.ptr, None) == -1  # q_dim 384
    w256 = uaii_amd.DeviceWeight(uaii_amd.Q4_0, synth.quantize(uaii_amd.Q4_0, x[: 32 * 4 * 256]), 32, 4 * 256)
    assert hip.uaii_hip_attention_o(buf.ptr, buf.ptr, buf.ptr, 1, max_seq, 4, 2, 256, 10, w256.h, out.ptr,
                                    y.ptr, None) == -1  # head_dim 256
    # a supported shape whose `out` and y overlap (merge blocks write `out` while
    # others add into y)
    wok = uaii_amd.DeviceWeight(uaii_amd.Q4_0, synth.quantize(uaii_amd.Q4_0, x[: 64 * nh * hd]), 64, nh * hd)
    assert hip.uaii_hip_attention_o(buf.ptr, buf.ptr, buf.ptr, 1, max_seq, nh, nkv, hd, 10, wok.h, y.ptr,
                                    y.ptr, None) == -1
    assert hip.uaii_hip_attention_o(buf.ptr, buf.ptr, buf.ptr, 1, max_seq, nh, nkv, hd, 10, wok.h, y.ptr,
                                    C.c_void_p(y.ptr.value + 4 * 100), None) == -1
    check_hip(hip.uaii_hip_synchronize())


def run_device(path, prompt, n_new, n_layers, kv_f16=True, max_context=0):
    with uaii_amd.Session(path, kv_f16=kv_f16, max_context=max_context) as s:
        if kv_f16:
            assert s.prefill_supported(), "the prompt should run on the matrix cores"
        ids = s.generate(prompt, n_new)
        taps = {k: s.get(k) for k in ("logits", "normed")}
        for li in range(n_layers):
            taps[f"r1_{li}"] = s.get(f"blk.{li}.resid1")
            taps[f"r2_{li}"] = s.get(f"blk.{li}.resid2")
    return ids, taps


def check_taps(taps, want, n_layers, bar=2e-3):
    errs = {"logits": maxrel(taps["logits"], want["logits"]),
            "normed": maxrel(taps["normed"], want["normed"])}
    for li in range(n_layers):
        errs[f"r1_{li}"] = maxrel(taps[f"r1_{li}"], want["resid1"][li])
        errs[f"r2_{li}"] = maxrel(taps[f"r2_{li}"], want["resid2"][li])
    print("max rel errors", {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    for k, e in errs.items():
        assert e < bar, (k, e)


@pytest.mark.parametrize("name", ["8b_q4_0", "8b_q8_0"])
def test_8b_shape_two_layers(name):
    cfg = SHAPES[name]
    path = synth.cached_model(cfg, nthreads=THREADS)
    prompt = np.random.default_rng(cfg.seed + 100).integers(0, cfg.vocab, 96).astype(np.int64)
    m = oracle.Model(path)
    assert m.n_layers == 2 and m.dim == 4096 and m.ffn == 14336 and m.vocab == 128256
    ids, taps = run_device(path, prompt, 64, 2, max_context=4096)
    want_ids, want = m.generate(prompt, 64, kv_f16=True, nthreads=THREADS)
    print(name, "gpu", ids[96:].tolist(), flush=True)
    print(name, "cpu", want_ids[96:].tolist(), flush=True)
    assert np.array_equal(ids, want_ids)
    check_taps(taps, want, 2)
    # the reference's f32 KV cache: the device's fp16 cache within the same bars
    ids8, taps8 = run_device(path, prompt, 8, 2, max_context=4096)
    want_ids32, want32 = m.generate(prompt, 8, kv_f16=False, nthreads=THREADS)
    assert np.array_equal(ids8, want_ids32)
    check_taps(taps8, want32, 2)


def test_8b_shape_headline_context():
    """The headline length: two 8B-shape layers (Q4_0, vocab 128256), a 4032-token
    prompt prefilled on the matrix cores (1024-row chunks), then 64 greedy tokens
    that fill the 4096-position fp16 cache (decode attention over 4033 .. 4096
    keys, 32 key splits). Against the oracle with an fp16 cache (its prompt run
    layer by layer, bit-identical to its token steps): all 64 ids identical,
    logits and every residual tap of the last step within 2e-3."""
    cfg = SHAPES["8b_q4_0"]
    path = synth.cached_model(cfg, nthreads=THREADS)
    n_prompt, n_new = 4032, 64
    prompt = np.random.default_rng(cfg.seed + 200).integers(0, cfg.vocab, n_prompt).astype(np.int64)
    print("8b headline context: device", flush=True)
    ids, taps = run_device(path, prompt, n_new, 2, max_context=4096)
    print("8b headline context: oracle", flush=True)
    want_ids, want = oracle.Model(path).generate(prompt, n_new, kv_f16=True, nthreads=THREADS,
                                                 prompt_block=256)
    print("8b ctx4096 gpu", ids[n_prompt:].tolist(), flush=True)
    print("8b ctx4096 cpu", want_ids[n_prompt:].tolist(), flush=True)
    assert len(ids) == 4096
    assert np.array_equal(ids, want_ids)
    check_taps(taps, want, 2)


def test_1b_shape_full_depth():
    cfg = SHAPES["1b"]
    path = synth.cached_model(cfg, nthreads=THREADS)
    prompt = np.random.default_rng(cfg.seed + 100).integers(0, cfg.vocab, 128).astype(np.int64)
    ids, taps = run_device(path, prompt, 64, cfg.n_layers)
    want_ids, want = oracle.Model(path).generate(prompt, 64, kv_f16=True, nthreads=THREADS)
    print("1b gpu", ids[128:].tolist(), flush=True)
    print("1b cpu", want_ids[128:].tolist(), flush=True)
    assert np.array_equal(ids, want_ids)
    check_taps(taps, want, cfg.n_layers)


def test_mixtral_shape_one_layer():
    cfg = SHAPES["mx"]
    path = synth.cached_model(cfg, nthreads=THREADS)
    prompt = np.random.default_rng(cfg.seed + 100).integers(0, cfg.vocab, 64).astype(np.int64)
    ids, taps = run_device(path, prompt, 64, 1)
    m = oracle.Model(path)
    assert m.n_experts == 8 and m.top_k == 2 and m.ffn == 14336
    want_ids, want = m.generate(prompt, 64, kv_f16=True, nthreads=THREADS, prompt_block=64)
    print("mx gpu", ids[64:].tolist(), flush=True)
    print("mx cpu", want_ids[64:].tolist(), flush=True)
    assert np.array_equal(ids, want_ids)
    check_taps(taps, want, 1)
