"""The residual-add projections through the C ABI, on each of their kernels.

By default (UAII_SPLITK=1) the Q4_0 attention output O runs with the merge of
the attention's key splits in its launch (attn_out.hip) and the FFN down split
along K (splitk_gemv.hip), both adding into the residual with float atomics.
UAII_SPLITK=0 keeps the whole-row kernels: the merge kernel, then O and down on
k_ring_gemv where the shapes allow (K a multiple of 2048; UAII_RING=1) or on
gemv.hip (UAII_RING=0). Bars as for the other generate tests: greedy ids
identical to the CPU oracle (fp16-cache flavour) over the decoded tokens,
logits and per-layer hidden states within 2e-3 max relative error; and the
kernels within 1e-4 of each other.
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


def run(path, cfg, prompt, n_new, ring="1", splitk="0"):
    env = {"UAII_RING": ring, "UAII_SPLITK": splitk}
    saved = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        with uaii_amd.Session(path, kv_f16=True) as s:
            ids = s.generate(prompt, n_new)
            taps = {"logits": s.get("logits"), "normed": s.get("normed")}
            for li in range(cfg.n_layers):
                taps[f"r1_{li}"] = s.get(f"blk.{li}.resid1")
                taps[f"r2_{li}"] = s.get(f"blk.{li}.resid2")
    finally:
        for k, v in saved.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v
    return ids, taps


@pytest.mark.parametrize("splitk", ["0", "1"], ids=["ring", "splitk"])
@pytest.mark.parametrize("name", [n for n in CFGS if n != "g1_hd64_long"])
def test_ring_gemv_match_oracle(name, splitk):
    """Per-layer launches with the O and down projections on the ring kernel
    (after the merge kernel), or split along K (the merge in O's launch)."""
    cfg = CFGS[name]
    path = synth.cached_model(cfg)
    prompt = np.random.default_rng(cfg.seed + 3).integers(0, cfg.vocab, 40).astype(np.int64)
    print(name, "splitk", splitk, flush=True)
    ids, taps = run(path, cfg, prompt, 24, splitk=splitk)
    want_ids, want = oracle.Model(path).generate(prompt, 24, kv_f16=True)
    assert np.array_equal(ids, want_ids)
    assert maxrel(taps["logits"], want["logits"]) < 2e-3
    for li in range(cfg.n_layers):
        assert maxrel(taps[f"r1_{li}"], want["resid1"][li]) < 2e-3
        assert maxrel(taps[f"r2_{li}"], want["resid2"][li]) < 2e-3


def test_ring_gemv_long_context():
    """600-token prompt (matrix-core prefill fills the cache) then 32 decode steps;
    repeated generate on one model."""
    cfg = CFGS["g1_hd64_long"]
    path = synth.cached_model(cfg)
    prompt = np.random.default_rng(cfg.seed).integers(0, cfg.vocab, 600).astype(np.int64)
    ids, taps = run(path, cfg, prompt, 32)
    want_ids, want = oracle.Model(path).generate(prompt, 32, kv_f16=True, prompt_block=128)
    assert np.array_equal(ids, want_ids)
    assert maxrel(taps["logits"], want["logits"]) < 2e-3
    for li in range(cfg.n_layers):
        assert maxrel(taps[f"r2_{li}"], want["resid2"][li]) < 2e-3
    short = prompt[:5]
    ids2, _ = run(path, cfg, short, 8)
    want2, _ = oracle.Model(path).generate(short, 8, kv_f16=True)
    assert np.array_equal(ids2, want2)


@pytest.mark.parametrize("name", ["g4_hd128", "g2_hd64_neox_bias"])
def test_splitk_matches_whole_row(name):
    """The split-K O (with the merge in its launch) and down against the
    whole-row kernels (merge kernel, ring O and down) on the same prompt: ids
    identical, every tap within 1e-4 (the atomic adds change only the order
    of the residual's f32 sums)."""
    cfg = CFGS[name]
    path = synth.cached_model(cfg)
    prompt = np.random.default_rng(cfg.seed + 17).integers(0, cfg.vocab, 9).astype(np.int64)
    ids, taps = run(path, cfg, prompt, 40, splitk="1")
    ids0, taps0 = run(path, cfg, prompt, 40, splitk="0")
    assert np.array_equal(ids, ids0)
    for k in taps:
        assert maxrel(taps[k], taps0[k]) < 1e-4, k


@pytest.mark.parametrize("name", ["g4_hd128", "g1_hd128_ffn6144"])
def test_ring_gemv_matches_gemv(name):
    cfg = CFGS[name]
    path = synth.cached_model(cfg)
    prompt = np.random.default_rng(cfg.seed + 11).integers(0, cfg.vocab, 5).astype(np.int64)
    ids, taps = run(path, cfg, prompt, 40, ring="1")
    ids0, taps0 = run(path, cfg, prompt, 40, ring="0")
    assert np.array_equal(ids, ids0)
    for k in taps:
        assert maxrel(taps[k], taps0[k]) < 1e-4, k
