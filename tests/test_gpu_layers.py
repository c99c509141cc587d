"""The one-launch decode layer kernel (layers.hip) through the C ABI.

With UAII_LAYERS=1 (opt-in), models whose shapes the kernel takes (K a
multiple of 2048, Q4_0 layer matrices, fp16 KV cache) decode every token with
one launch for all layers.
Bars as for the other generate tests: greedy ids identical to the CPU oracle
(fp16-cache flavour) over the decoded tokens, logits and per-layer hidden
states within 2e-3 max relative error; and the same against the per-layer
launches of the same step (UAII_LAYERS=0), which the rest of the suite pins.
"""
import os

import numpy as np
import pytest

import oracle
import uaii_amd
from uaii_amd import synth

pytestmark = pytest.mark.gpu

CFGS = {
    # head_dim 128 with the 8B grouping (4 query heads per kv head)
    "g4_hd128": synth.ModelConfig(n_layers=2, dim=2048, n_heads=16, n_kv_heads=4, ffn=4096,
                                  vocab=1024, ctx_len=512, type_default=uaii_amd.Q4_0,
                                  type_attn_v=uaii_amd.Q4_0, seed=51),
    # head_dim 64, 2:1 grouping, NeoX RoPE (qwen2) with Q/K/V biases, K = 2048 in one column
    "g2_hd64_neox_bias": synth.ModelConfig(n_layers=2, dim=2048, n_heads=32, n_kv_heads=16,
                                           ffn=2048, vocab=1024, ctx_len=512, arch="qwen2",
                                           qkv_bias=True, type_default=uaii_amd.Q4_0,
                                           type_attn_v=uaii_amd.Q4_0, seed=52),
    # multi-head attention and an FFN of three chunk columns (K = 6144)
    "g1_hd128_ffn6144": synth.ModelConfig(n_layers=2, dim=2048, n_heads=16, n_kv_heads=16,
                                          ffn=6144, vocab=1024, ctx_len=512,
                                          type_default=uaii_amd.Q4_0, type_attn_v=uaii_amd.Q4_0,
                                          seed=53),
    # 8 query heads per kv head
    "g8_hd128": synth.ModelConfig(n_layers=2, dim=2048, n_heads=16, n_kv_heads=2, ffn=4096,
                                  vocab=1024, ctx_len=512, type_default=uaii_amd.Q4_0,
                                  type_attn_v=uaii_amd.Q4_0, seed=54),
    # head_dim 64 MHA: 8 splits per kv head, several 64-key stages per split at long context
    "g1_hd64_long": synth.ModelConfig(n_layers=2, dim=2048, n_heads=32, n_kv_heads=32, ffn=2048,
                                      vocab=1024, ctx_len=1024, type_default=uaii_amd.Q4_0,
                                      type_attn_v=uaii_amd.Q4_0, seed=55),
}


def maxrel(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max() / max(np.abs(b).max(), 1e-30))


def run(path, cfg, prompt, n_new, layers=True, profile=False, ring="1", ring_lm="0"):
    saved = {k: os.environ.get(k) for k in ("UAII_LAYERS", "UAII_RING", "UAII_RING_LM")}
    os.environ["UAII_LAYERS"] = "1" if layers else "0"
    os.environ["UAII_RING"] = ring
    os.environ["UAII_RING_LM"] = ring_lm
    try:
        with uaii_amd.Session(path, kv_f16=True, profile=profile) as s:
            ids = s.generate(prompt, n_new)
            taps = {"logits": s.get("logits"), "normed": s.get("normed")}
            for li in range(cfg.n_layers):
                taps[f"r1_{li}"] = s.get(f"blk.{li}.resid1")
                taps[f"r2_{li}"] = s.get(f"blk.{li}.resid2")
            summary = s.profile_summary() if profile else ""
    finally:
        for k, v in saved.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v
    return ids, taps, summary


@pytest.mark.parametrize("name", [n for n in CFGS if n != "g1_hd64_long"])
def test_layers_match_oracle(name):
    cfg = CFGS[name]
    path = synth.cached_model(cfg)
    prompt = np.random.default_rng(cfg.seed).integers(0, cfg.vocab, 40).astype(np.int64)
    print(name, flush=True)
    ids, taps, summary = run(path, cfg, prompt, 24, profile=True)
    assert "layers" in summary  # the one-launch kernel ran
    want_ids, want = oracle.Model(path).generate(prompt, 24, kv_f16=True)
    print(name, "gpu", ids[40:].tolist())
    print(name, "cpu", want_ids[40:].tolist())
    assert np.array_equal(ids, want_ids)
    assert maxrel(taps["logits"], want["logits"]) < 2e-3
    for li in range(cfg.n_layers):
        assert maxrel(taps[f"r1_{li}"], want["resid1"][li]) < 2e-3
        assert maxrel(taps[f"r2_{li}"], want["resid2"][li]) < 2e-3


@pytest.mark.parametrize("name", ["g4_hd128", "g2_hd64_neox_bias"])
def test_layers_match_per_layer_launches(name):
    cfg = CFGS[name]
    path = synth.cached_model(cfg)
    prompt = np.random.default_rng(cfg.seed + 7).integers(0, cfg.vocab, 3).astype(np.int64)
    print(name, flush=True)
    ids, taps, _ = run(path, cfg, prompt, 48, layers=True)
    ids0, taps0, summary0 = run(path, cfg, prompt, 48, layers=False, profile=True)
    assert "layers" not in summary0
    assert np.array_equal(ids, ids0)
    for k in taps:
        assert maxrel(taps[k], taps0[k]) < 1e-4, k


def test_layers_long_context():
    """600-token prompt (matrix-core prefill fills the cache) then 32 decode steps whose
    attention splits hold several key stages each; repeated generate on one session."""
    cfg = CFGS["g1_hd64_long"]
    path = synth.cached_model(cfg)
    prompt = np.random.default_rng(cfg.seed).integers(0, cfg.vocab, 600).astype(np.int64)
    print("g1_hd64_long", flush=True)
    ids, taps, _ = run(path, cfg, prompt, 32)
    want_ids, want = oracle.Model(path).generate(prompt, 32, kv_f16=True)
    assert np.array_equal(ids, want_ids)
    assert maxrel(taps["logits"], want["logits"]) < 2e-3
    for li in range(cfg.n_layers):
        assert maxrel(taps[f"r2_{li}"], want["resid2"][li]) < 2e-3
    # a second, shorter generate on a fresh session state gives the oracle's ids too
    short = prompt[:5]
    ids2, _, _ = run(path, cfg, short, 8)
    want2, _ = oracle.Model(path).generate(short, 8, kv_f16=True)
    assert np.array_equal(ids2, want2)


@pytest.mark.parametrize("mode", ["1", "2"])
@pytest.mark.parametrize("name", [n for n in CFGS if n != "g1_hd64_long"])
def test_ring_gemv_match_oracle(name, mode):
    """Per-layer launches with Q4_0 GEMVs on the LDS-ring kernel: mode 1 (default) the
    O and down projections, mode 2 also QKV (RoPE mode 0 only) and gate/up."""
    cfg = CFGS[name]
    path = synth.cached_model(cfg)
    prompt = np.random.default_rng(cfg.seed + 3).integers(0, cfg.vocab, 40).astype(np.int64)
    print(name, mode, flush=True)
    ids, taps, _ = run(path, cfg, prompt, 24, layers=False, ring=mode)
    want_ids, want = oracle.Model(path).generate(prompt, 24, kv_f16=True)
    assert np.array_equal(ids, want_ids)
    assert maxrel(taps["logits"], want["logits"]) < 2e-3
    for li in range(cfg.n_layers):
        assert maxrel(taps[f"r1_{li}"], want["resid1"][li]) < 2e-3
        assert maxrel(taps[f"r2_{li}"], want["resid2"][li]) < 2e-3


def test_ring_gemv_matches_gemv():
    cfg = CFGS["g4_hd128"]
    path = synth.cached_model(cfg)
    prompt = np.random.default_rng(cfg.seed + 11).integers(0, cfg.vocab, 5).astype(np.int64)
    ids, taps, _ = run(path, cfg, prompt, 40, layers=False, ring="2")
    ids0, taps0, _ = run(path, cfg, prompt, 40, layers=False, ring="0")
    assert np.array_equal(ids, ids0)
    for k in taps:
        assert maxrel(taps[k], taps0[k]) < 1e-4, k


@pytest.mark.parametrize("name", ["g4_hd128", "g1_hd128_ffn6144"])
def test_ring_lm_head(name):
    """The LM head on the ring GEMV (UAII_RING_LM=1: final RMSNorm staging, logits,
    argmax partials per compute wave, then the final argmax + token advance)
    against the oracle: ids, logits and the normed input."""
    cfg = CFGS[name]
    path = synth.cached_model(cfg)
    prompt = np.random.default_rng(cfg.seed + 3).integers(0, cfg.vocab, 20).astype(np.int64)
    print(name, flush=True)
    ids, taps, _ = run(path, cfg, prompt, 32, layers=False, ring_lm="1")
    want_ids, want = oracle.Model(path).generate(prompt, 32, kv_f16=True)
    assert np.array_equal(ids, want_ids)
    assert maxrel(taps["logits"], want["logits"]) < 2e-3
    assert maxrel(taps["normed"], want["normed"]) < 2e-3
