"""Prompt (M > 1) path on the matrix cores against the CPU oracle, through the
uaii_hip_* C ABI and the session.

* MFMA dequant-GEMM (uaii_hip_gemm*) against the oracle's per-row dequant +
  sequential f32 dot (quant_gemm.cpp:22-70) for M = 1 .. 512, the config-2
  shapes (N x K = 4096x4096, 4096x14336, 14336x4096) at M = 512, ragged M and
  N, the RMSNorm prologue and the residual-add / SwiGLU epilogues. Bar: max
  relative error (tensor scale) < 1e-4; the path keeps ~22-bit activations and
  exact integer weights, so it lands near 1e-6.
* The reference benchmark's Q4_0 pattern (uaii_bench.cpp:505-518) at M = 4
  against the exact f64 product.
* Causal prefill attention over an f16 cache against the oracle's decode
  attention applied to each query in turn (transformer.cpp:222-433). Bar 2e-5.
* Sessions: greedy generate with the prompt prefilled on the matrix cores gives
  the same ids as the oracle (f16 cache) over 64 decoded tokens, with logits and
  hidden states within 2e-3; chunked prefill (several chunks, p0 > 0) equals a
  single chunk.
"""
import numpy as np
import pytest

import oracle
import uaii_amd
from uaii_amd import synth, DeviceBuffer, DeviceWeight, check_hip

pytestmark = pytest.mark.gpu

MFMA_TYPES = [uaii_amd.Q4_0, uaii_amd.Q8_0, uaii_amd.Q4_K, uaii_amd.Q6_K]


def maxrel(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max() / max(np.abs(b).max(), 1e-30))


def packed(t, rows, cols, seed):
    return synth.quantize(t, synth.normals(seed, 0, 0, rows * cols, 0.02))


def run_gemm(hip, w, x, rows, norm=None, eps=1e-5):
    m, cols = x.shape
    dx, dy = DeviceBuffer.from_array(x), DeviceBuffer(m * rows * 4)
    if norm is None:
        check_hip(hip.uaii_hip_gemm(w.h, dx.ptr, m, dy.ptr, None), "gemm")
    else:
        dn = DeviceBuffer.from_array(norm.astype(np.float32))
        check_hip(hip.uaii_hip_gemm_rmsnorm(w.h, dx.ptr, m, dn.ptr, eps, dy.ptr, None), "gemm_rmsnorm")
    check_hip(hip.uaii_hip_synchronize())
    return dy.to_array(np.float32, m * rows).reshape(m, rows)


def oracle_rmsnorm_rows(x, nw, eps=1e-5):
    out = np.zeros_like(x)
    for i in range(x.shape[0]):
        row = np.ascontiguousarray(x[i])
        oracle.oracle().orc_rmsnorm(oracle._fp(row), oracle._fp(np.ascontiguousarray(nw)),
                                    oracle._fp(out[i]), x.shape[1], eps)
    return out


@pytest.mark.parametrize("t", MFMA_TYPES, ids=lambda t: uaii_amd.TYPE_NAMES[t])
@pytest.mark.parametrize("m,rows,cols", [(1, 256, 256), (3, 96, 512), (77, 1000, 1024),
                                         (130, 300, 2048), (512, 4096, 4096), (1024, 640, 1024)],
                         ids=str)
def test_gemm_against_oracle(hip, t, m, rows, cols):
    p = packed(t, rows, cols, seed=rows + cols + m)
    x = synth.normals(71, m, 0, m * cols, 1.0).reshape(m, cols)
    w = DeviceWeight(t, p, rows, cols)
    got = run_gemm(hip, w, x, rows)
    want = oracle.quant_gemm(t, x, p, rows, nthreads=0)
    print("gemm maxrel", uaii_amd.TYPE_NAMES[t], m, rows, cols, maxrel(got, want))
    assert maxrel(got, want) < 1e-4
    # every row on its own scale: a row 2^20 times smaller is just as accurate
    if m >= 3:
        xs = x.copy()
        xs[1] *= 2.0 ** -20
        got = run_gemm(hip, w, xs, rows)
        want = oracle.quant_gemm(t, xs, p, rows, nthreads=0)
        assert maxrel(got[1], want[1]) < 1e-4


@pytest.mark.parametrize("t", [uaii_amd.Q4_0, uaii_amd.Q8_0, uaii_amd.Q4_K],
                         ids=lambda t: uaii_amd.TYPE_NAMES[t])
@pytest.mark.parametrize("shape", [(4096, 14336), (14336, 4096)], ids=lambda s: f"{s[0]}x{s[1]}")
@pytest.mark.parametrize("act", ["f32", "f16"])
def test_gemm_config_shapes(hip, t, shape, act):
    """Config 2 at M=512; the oracle checks a sample of 24 activation rows. N(0,1)
    activations in f32 and as fp16 values (entering as their exact f32 values, the
    reference's row type)."""
    rows, cols = shape
    m = 512
    p = packed(t, rows, cols, seed=7)
    x = synth.normals(72, m, 0, m * cols, 1.0).reshape(m, cols)
    if act == "f16":
        x = x.astype(np.float16).astype(np.float32)
    w = DeviceWeight(t, p, rows, cols)
    got = run_gemm(hip, w, x, rows)
    pick = np.random.default_rng(5).choice(m, 24, replace=False)
    pick[0], pick[1] = 0, m - 1
    want = oracle.quant_gemm(t, x[pick], p, rows, nthreads=0)
    assert maxrel(got[pick], want) < 1e-4


def test_gemm_bench_pattern_known_answer(hip):
    """uaii_bench.cpp:505-518 Q4_0 pattern (d = 1, qs[i] = (i + block) & 0xff,
    a[i] = 0.01 ((i % 17) + 1)), N=2048, K=4096, four scaled copies of a."""
    rows, cols = 2048, 4096
    nb = rows * cols // 32
    blk = np.zeros((nb, 18), dtype=np.uint8)
    blk[:, 0], blk[:, 1] = 0x00, 0x3c
    b = np.arange(nb, dtype=np.int64)[:, None]
    blk[:, 2:] = ((np.arange(16)[None, :] + b) & 0xff).astype(np.uint8)
    a = (0.01 * ((np.arange(cols) % 17) + 1)).astype(np.float32)
    x = np.stack([a, -a, 3.0 * a, a * 2.0 ** -7]).astype(np.float32)
    w = DeviceWeight(uaii_amd.Q4_0, blk.reshape(-1), rows, cols)
    got = run_gemm(hip, w, x, rows)
    q = blk[:, 2:].astype(np.int64)
    vals = np.concatenate([(q & 15) - 8, (q >> 4) - 8], axis=1).reshape(rows, cols).astype(np.float64)
    exact = x.astype(np.float64) @ vals.T
    for i in range(4):
        assert maxrel(got[i], exact[i]) < 1e-5


@pytest.mark.parametrize("t", MFMA_TYPES, ids=lambda t: uaii_amd.TYPE_NAMES[t])
def test_gemm_rmsnorm_add_swiglu(hip, t):
    rows, cols, m = 768, 2048, 100
    x = synth.normals(73, m, 0, m * cols, 2.0).reshape(m, cols)
    nw = 1.0 + synth.normals(74, 1, 0, cols, 0.1)
    xn = oracle_rmsnorm_rows(x, nw)
    pg, pu = packed(t, rows, cols, 21), packed(t, rows, cols, 22)
    wg, wu = DeviceWeight(t, pg, rows, cols), DeviceWeight(t, pu, rows, cols)
    g = oracle.quant_gemm(t, xn, pg, rows, nthreads=0).astype(np.float64)
    u = oracle.quant_gemm(t, xn, pu, rows, nthreads=0).astype(np.float64)
    # RMSNorm prologue
    assert maxrel(run_gemm(hip, wg, x, rows, norm=nw), g) < 1e-4
    dx, dn = DeviceBuffer.from_array(x), DeviceBuffer.from_array(nw)
    # residual add
    y0 = synth.normals(75, m, 0, m * rows, 1.0).reshape(m, rows)
    dy = DeviceBuffer.from_array(y0)
    check_hip(hip.uaii_hip_gemm_add(wg.h, dx.ptr, m, dn.ptr, 1e-5, dy.ptr, None))
    assert maxrel(dy.to_array(np.float32, m * rows).reshape(m, rows), y0 + g) < 1e-4
    # SwiGLU pairs
    dh = DeviceBuffer(m * rows * 4)
    check_hip(hip.uaii_hip_gemm_swiglu(wg.h, wu.h, dx.ptr, m, dn.ptr, 1e-5, dh.ptr, None))
    want = g / (1.0 + np.exp(-g)) * u
    assert maxrel(dh.to_array(np.float32, m * rows).reshape(m, rows), want) < 1e-4


@pytest.mark.parametrize("t", MFMA_TYPES, ids=lambda t: uaii_amd.TYPE_NAMES[t])
def test_gemm_add_swiglu_wide_tile(hip, t):
    """The residual-add and SwiGLU launches on a grid large enough for the 64-row
    wave tile (4096 rows at M = 512), for every matrix-core format (Q6_K's tile
    spills registers there); the oracle checks 24 sampled activation rows."""
    rows, cols, m = 4096, 1024, 512
    x = synth.normals(77, m, 0, m * cols, 2.0).reshape(m, cols)
    nw = 1.0 + synth.normals(78, 1, 0, cols, 0.1)
    pick = np.random.default_rng(9).choice(m, 24, replace=False)
    pick[0], pick[1] = 0, m - 1
    xn = oracle_rmsnorm_rows(x[pick], nw)
    pg, pu = packed(t, rows, cols, 31), packed(t, rows, cols, 32)
    wg, wu = DeviceWeight(t, pg, rows, cols), DeviceWeight(t, pu, rows, cols)
    g = oracle.quant_gemm(t, xn, pg, rows, nthreads=0).astype(np.float64)
    u = oracle.quant_gemm(t, xn, pu, rows, nthreads=0).astype(np.float64)
    assert maxrel(run_gemm(hip, wg, x, rows, norm=nw)[pick], g) < 1e-4
    dx, dn = DeviceBuffer.from_array(x), DeviceBuffer.from_array(nw)
    y0 = synth.normals(79, m, 0, m * rows, 1.0).reshape(m, rows)
    dy = DeviceBuffer.from_array(y0)
    check_hip(hip.uaii_hip_gemm_add(wg.h, dx.ptr, m, dn.ptr, 1e-5, dy.ptr, None))
    got = dy.to_array(np.float32, m * rows).reshape(m, rows)[pick]
    assert maxrel(got, y0[pick] + g) < 1e-4
    dh = DeviceBuffer(m * rows * 4)
    check_hip(hip.uaii_hip_gemm_swiglu(wg.h, wu.h, dx.ptr, m, dn.ptr, 1e-5, dh.ptr, None))
    want = g / (1.0 + np.exp(-g)) * u
    assert maxrel(dh.to_array(np.float32, m * rows).reshape(m, rows)[pick], want) < 1e-4


def test_gemm_other_formats_run_row_by_row(hip):
    """Formats outside the MFMA decoder go through the GEMV per row, same results."""
    t, rows, cols, m = uaii_amd.Q5_K, 200, 512, 5
    p = packed(t, rows, cols, 23)
    x = synth.normals(76, m, 0, m * cols, 1.0).reshape(m, cols)
    got = run_gemm(hip, DeviceWeight(t, p, rows, cols), x, rows)
    assert maxrel(got, oracle.quant_gemm(t, x, p, rows, nthreads=0)) < 1e-4


@pytest.mark.parametrize("heads", [(8, 8, 64), (32, 8, 128), (16, 2, 64), (12, 4, 64), (6, 2, 128)],
                         ids=str)
@pytest.mark.parametrize("p0,m", [(0, 1), (0, 17), (0, 64), (100, 37), (5, 200)], ids=str)
def test_attention_prefill(hip, heads, p0, m):
    nh, nkv, hd = heads
    max_seq = 512
    rng = np.random.default_rng(p0 * 131 + m + nh)
    q = rng.standard_normal((m, nh * hd)).astype(np.float32)
    k = rng.standard_normal((nkv, max_seq, hd)).astype(np.float16)
    v = rng.standard_normal((nkv, max_seq, hd)).astype(np.float16)
    dq, dk, dv = DeviceBuffer.from_array(q), DeviceBuffer.from_array(k), DeviceBuffer.from_array(v)
    do = DeviceBuffer(m * nh * hd * 4)
    check_hip(hip.uaii_hip_attention_prefill(dq.ptr, dk.ptr, dv.ptr, max_seq, nh, nkv, hd, p0, m,
                                             do.ptr, None))
    check_hip(hip.uaii_hip_synchronize())
    got = do.to_array(np.float32, m * nh * hd).reshape(m, nh * hd)
    kf = k.astype(np.float32).transpose(1, 0, 2).reshape(max_seq, nkv * hd)
    vf = v.astype(np.float32).transpose(1, 0, 2).reshape(max_seq, nkv * hd)
    err = 0.0
    for i in range(m):
        n = p0 + i + 1  # query i sees keys 0 .. p0 + i
        past = max(n - 1, 1)
        kc = np.ascontiguousarray(kf[:past]) if n > 1 else np.zeros((1, nkv * hd), np.float32)
        vc = np.ascontiguousarray(vf[:past]) if n > 1 else np.zeros((1, nkv * hd), np.float32)
        want = np.zeros(nh * hd, np.float32)
        oracle.oracle().orc_attention_decode(oracle._fp(np.ascontiguousarray(q[i])), oracle._fp(kc),
                                             oracle._fp(vc), n - 1,
                                             oracle._fp(np.ascontiguousarray(kf[n - 1])),
                                             oracle._fp(np.ascontiguousarray(vf[n - 1])),
                                             oracle._fp(want), nh, nkv, hd)
        err = max(err, maxrel(got[i], want))
        assert maxrel(got[i], want) < 2e-5, f"query {i}"
    print("attention maxrel", heads, p0, m, err)


PREFILL_CFGS = {
    "gqa_q4_0": synth.ModelConfig(n_layers=3, dim=512, n_heads=8, n_kv_heads=2, ffn=1024,
                                  vocab=3000, ctx_len=512, type_default=uaii_amd.Q4_0,
                                  type_attn_v=uaii_amd.Q8_0, seed=41),
    "kmix_tied": synth.ModelConfig(n_layers=2, dim=512, n_heads=8, n_kv_heads=2, ffn=1536,
                                   vocab=2048, ctx_len=512, rope_theta=500000.0, tied=True,
                                   type_default=uaii_amd.Q4_K, type_attn_v=uaii_amd.Q6_K,
                                   type_ffn_down=uaii_amd.Q6_K, seed=42),
    "neox_hd128": synth.ModelConfig(n_layers=2, dim=512, n_heads=4, n_kv_heads=2, ffn=1024,
                                    vocab=1500, ctx_len=512, type_default=uaii_amd.Q8_0,
                                    arch="qwen2", seed=43),
    "gelu_bias": synth.ModelConfig(n_layers=2, dim=512, n_heads=8, n_kv_heads=4, ffn=1024,
                                   vocab=1500, ctx_len=512, type_default=uaii_amd.Q8_0, gelu=True,
                                   qkv_bias=True, seed=44),
    # MoE: 4 experts top-2 over Q4_K experts; every expert's token list a gather
    "moe_k": synth.ModelConfig(n_layers=2, dim=512, n_heads=8, n_kv_heads=2, ffn=512,
                               vocab=1200, ctx_len=512, type_default=uaii_amd.Q4_K, n_experts=4,
                               top_k=2, router_std=1.0 / 22, seed=45),
    # MoE 8 experts top-2 beside a shared expert, Q4_0
    "moe_shared": synth.ModelConfig(n_layers=2, dim=256, n_heads=4, n_kv_heads=4, ffn=320,
                                    vocab=700, ctx_len=512, type_default=uaii_amd.Q4_0,
                                    n_experts=8, top_k=2, router_std=1.0 / 16, shared_ffn=192,
                                    seed=46),
    # MoE 32 experts top-4: a 64-entry group of the token lists spans many
    # experts, so the per-expert ranking takes several rounds per group
    "moe_wide": synth.ModelConfig(n_layers=2, dim=256, n_heads=4, n_kv_heads=2, ffn=128,
                                  vocab=700, ctx_len=512, type_default=uaii_amd.Q4_0,
                                  n_experts=32, top_k=4, router_std=1.0 / 16, seed=47),
}


@pytest.mark.parametrize("name", list(PREFILL_CFGS))
def test_generate_with_prefill(name):
    cfg = PREFILL_CFGS[name]
    path = synth.cached_model(cfg)
    prompt = np.random.default_rng(cfg.seed).integers(0, cfg.vocab, 96).astype(np.int64)
    with uaii_amd.Session(path, kv_f16=True) as s:
        assert s.prefill_supported()
        ids = s.generate(prompt, 64)
        taps = {k: s.get(k) for k in ("logits", "normed")}
        r2 = [s.get(f"blk.{li}.resid2") for li in range(cfg.n_layers)]
    want_ids, want = oracle.Model(path).generate(prompt, 64, kv_f16=True)
    print(name, "gpu", ids[96:].tolist())
    print(name, "cpu", want_ids[96:].tolist())
    assert np.array_equal(ids, want_ids)
    assert maxrel(taps["logits"], want["logits"]) < 2e-3
    assert maxrel(taps["normed"], want["normed"]) < 2e-3
    for li in range(cfg.n_layers):
        assert maxrel(r2[li], want["resid2"][li]) < 2e-3


@pytest.mark.parametrize("name", ["moe_k", "moe_shared", "moe_wide"])
def test_moe_prefill_long_prompt(name):
    """A 400-token prompt: each expert's gathered rows span several row tiles
    of the grouped expert GEMMs, the last one partial."""
    cfg = PREFILL_CFGS[name]
    path = synth.cached_model(cfg)
    prompt = np.random.default_rng(cfg.seed + 7).integers(0, cfg.vocab, 400).astype(np.int64)
    with uaii_amd.Session(path, kv_f16=True) as s:
        assert s.prefill_supported()
        ids = s.generate(prompt, 8)
        taps = {k: s.get(k) for k in ("logits", "normed")}
        r2 = [s.get(f"blk.{li}.resid2") for li in range(cfg.n_layers)]
    want_ids, want = oracle.Model(path).generate(prompt, 8, kv_f16=True)
    assert np.array_equal(ids, want_ids)
    assert maxrel(taps["logits"], want["logits"]) < 2e-3
    assert maxrel(taps["normed"], want["normed"]) < 2e-3
    for li in range(cfg.n_layers):
        assert maxrel(r2[li], want["resid2"][li]) < 2e-3


@pytest.mark.parametrize("name", ["gqa_q4_0", "moe_shared"])
def test_prefill_chunks_and_offsets(monkeypatch, name):
    """A 150-token prompt in 32-token chunks (queries at p0 > 0 over earlier
    chunks' keys; MoE token lists rebuilt per chunk), after 5 tokens stepped one
    at a time, equals the token-by-token run: same ids, logits within 2e-3."""
    cfg = PREFILL_CFGS[name]
    path = synth.cached_model(cfg)
    prompt = np.random.default_rng(3).integers(0, cfg.vocab, 150).astype(np.int64)
    monkeypatch.setenv("UAII_PREFILL", "0")
    with uaii_amd.Session(path, kv_f16=True) as s:
        assert not s.prefill_supported()
        ref_ids = s.generate(prompt, 24)
        ref_logits = s.get("logits")
    monkeypatch.delenv("UAII_PREFILL")
    monkeypatch.setenv("UAII_PREFILL_CHUNK", "32")
    with uaii_amd.Session(path, kv_f16=True) as s:
        s.begin(prompt, 256)
        for _ in range(5):
            s.step_async(False)
        s.prefill(len(prompt) - 1 - 5)
        assert s.position() == len(prompt) - 1
        s.step_async(True)
        for _ in range(23):
            s.step_async(True)
        s.sync()
        ids = s.read_ids(len(prompt) + 24)
        logits = s.get("logits")
    assert np.array_equal(ids, ref_ids)
    assert maxrel(logits, ref_logits) < 2e-3


def test_generate_long_prompt_two_chunks():
    """An 1100-token prompt: one 1024-token chunk (the default chunk) and a
    75-token one at p0 = 1024, then 16 greedy tokens, against the oracle."""
    cfg = synth.ModelConfig(n_layers=2, dim=512, n_heads=8, n_kv_heads=2, ffn=1024, vocab=2000,
                            ctx_len=2048, type_default=uaii_amd.Q4_0, type_attn_v=uaii_amd.Q8_0,
                            seed=47)
    path = synth.cached_model(cfg)
    prompt = np.random.default_rng(cfg.seed).integers(0, cfg.vocab, 1100).astype(np.int64)
    with uaii_amd.Session(path, kv_f16=True) as s:
        assert s.prefill_supported()
        ids = s.generate(prompt, 16)
        taps = {k: s.get(k) for k in ("logits", "normed")}
        r2 = [s.get(f"blk.{li}.resid2") for li in range(cfg.n_layers)]
    want_ids, want = oracle.Model(path).generate(prompt, 16, kv_f16=True)
    assert np.array_equal(ids, want_ids)
    assert maxrel(taps["logits"], want["logits"]) < 2e-3
    assert maxrel(taps["normed"], want["normed"]) < 2e-3
    for li in range(cfg.n_layers):
        assert maxrel(r2[li], want["resid2"][li]) < 2e-3
