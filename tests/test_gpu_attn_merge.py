"""Decode attention with the split merge inside the split kernel.

With 8 kv heads and an f16 cache, the decode attention merges its key splits in
the split kernel (the last split block of each kv head, through its XCD's L2)
when the device places all blocks (h, s) of one kv head h on one XCD, which
uaii_hip_xcd_merge_supported probes, and UAII_ATTN_MERGE=1 asks for it (off by
default: it measures no faster than the separate merge kernel). The merge's arithmetic and order are the merge kernel's, so both paths
must give the same ids, logits and residual taps bit for bit; both are also
checked against the CPU oracle (fp16 cache).
"""
import ctypes as C
import os

import numpy as np
import pytest

import oracle
import uaii_amd
from uaii_amd import synth

pytestmark = pytest.mark.gpu

CFGS = {
    # the 8B grouping (4 query heads per kv head) at head_dim 64, 8 key splits
    "g4_hd64": synth.ModelConfig(n_layers=2, dim=2048, n_heads=32, n_kv_heads=8, ffn=2048, vocab=1024,
                                 ctx_len=1024, type_default=uaii_amd.Q4_0, type_attn_v=uaii_amd.Q8_0,
                                 seed=71),
    # head_dim 128, 2 query heads per kv head
    "g2_hd128": synth.ModelConfig(n_layers=2, dim=2048, n_heads=16, n_kv_heads=8, ffn=2048, vocab=1024,
                                  ctx_len=512, type_default=uaii_amd.Q4_0, type_attn_v=uaii_amd.Q4_0,
                                  seed=72),
    # multi-head (1 query head per kv head), 32 key splits over 4096 positions
    "g1_hd128_ctx4096": synth.ModelConfig(n_layers=1, dim=1024, n_heads=8, n_kv_heads=8, ffn=2048,
                                          vocab=1024, ctx_len=4096, type_default=uaii_amd.Q4_0,
                                          type_attn_v=uaii_amd.Q4_0, seed=73),
}


def run(path, prompt, n_new, merge, n_layers):
    saved = os.environ.get("UAII_ATTN_MERGE")
    os.environ["UAII_ATTN_MERGE"] = "1" if merge else "0"
    try:
        with uaii_amd.Session(path, kv_f16=True) as s:
            ids = s.generate(prompt, n_new)
            taps = {"logits": s.get("logits")}
            for li in range(n_layers):
                taps[f"r1_{li}"] = s.get(f"blk.{li}.resid1")
                taps[f"r2_{li}"] = s.get(f"blk.{li}.resid2")
    finally:
        if saved is None:
            os.environ.pop("UAII_ATTN_MERGE", None)
        else:
            os.environ["UAII_ATTN_MERGE"] = saved
    return ids, taps


def test_placement_probe_on_mi355x(hip):
    v = C.c_int(-1)
    assert uaii_amd.lib().uaii_hip_xcd_merge_supported(C.byref(v)) == 0
    assert v.value == 1, "grid (8, 32) did not keep the blocks of one kv head on one XCD"


@pytest.mark.parametrize("name", list(CFGS))
def test_merge_in_split_kernel_matches_merge_kernel(name):
    cfg = CFGS[name]
    path = synth.cached_model(cfg)
    n_prompt = 300 if cfg.ctx_len <= 1024 else 3000
    prompt = np.random.default_rng(cfg.seed).integers(0, cfg.vocab, n_prompt).astype(np.int64)
    ids_m, taps_m = run(path, prompt, 24, True, cfg.n_layers)
    ids_k, taps_k = run(path, prompt, 24, False, cfg.n_layers)
    assert np.array_equal(ids_m, ids_k)
    for k in taps_k:
        assert np.array_equal(taps_m[k].view(np.uint32), taps_k[k].view(np.uint32)), k
    want_ids, want = oracle.Model(path).generate(prompt, 24, kv_f16=True, prompt_block=128)
    assert np.array_equal(ids_m, want_ids)
    err = float(np.abs(taps_m["logits"] - want["logits"]).max() / np.abs(want["logits"]).max())
    assert err < 2e-3, err
