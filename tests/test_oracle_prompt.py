"""The oracle's layer-major prompt path against its token steps (CPU only).

orc_generate_ex(prompt_block=B) runs the prompt (all but its last token) layer by
layer in blocks of B tokens: each projection over a block's rows at once, the
block's K/V appended before its attentions. It exists so that prompts of several
thousand tokens fit a test's time; it must give the token steps' ids and taps bit
for bit. Checked on every architecture variant the oracle runs (dense GQA, NeoX
with Q/K/V biases, GELU MLP, MoE with and without a shared expert, Path A f32
weights, K-quant formats), both KV caches, and blocks of 1, 5, 8 and 64 tokens
(ragged last blocks, blocks larger than the prompt).
"""
import numpy as np
import pytest

import oracle
import uaii_amd
from uaii_amd import synth

MODELS = {
    "gqa_q4_0": dict(n_heads=8, n_kv_heads=2, dim=256),
    "neox_bias": dict(n_heads=4, n_kv_heads=2, arch="qwen2", qkv_bias=True),
    "gelu": dict(gelu=True),
    "moe_shared": dict(n_experts=4, top_k=2, router_std=1.0 / 16, shared_ffn=192),
    "q4_k_q6_k": dict(dim=256, ffn=512, type_default=uaii_amd.Q4_K, type_attn_v=uaii_amd.Q6_K,
                      type_ffn_down=uaii_amd.Q6_K),
}


def model_for(name, tmp_path):
    base = dict(n_layers=2, dim=256, n_heads=4, n_kv_heads=4, ffn=320, vocab=500, ctx_len=160,
                type_default=uaii_amd.Q4_0, type_attn_v=uaii_amd.Q8_0, seed=150)
    base.update(MODELS[name])
    cfg = synth.ModelConfig(**base)
    return cfg, synth.write_model(tmp_path / f"{name}.gguf", cfg)


def same(a, b):
    return np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


@pytest.mark.parametrize("name", list(MODELS))
@pytest.mark.parametrize("kv_f16", [False, True], ids=["f32kv", "f16kv"])
def test_prompt_blocks_equal_token_steps(name, kv_f16, tmp_path):
    cfg, path = model_for(name, tmp_path)
    prompt = np.random.default_rng(7).integers(0, cfg.vocab, 37).astype(np.int64)
    m = oracle.Model(path)
    ids, taps = m.generate(prompt, 6, kv_f16=kv_f16)
    for block in (1, 5, 8, 64):
        bids, btaps = m.generate(prompt, 6, kv_f16=kv_f16, prompt_block=block)
        assert np.array_equal(ids, bids), block
        for k in taps:
            assert same(taps[k], btaps[k]), (block, k)


def test_prompt_blocks_path_a(tmp_path):
    cfg, path = model_for("gqa_q4_0", tmp_path)
    prompt = np.random.default_rng(8).integers(0, cfg.vocab, 21).astype(np.int64)
    m = oracle.Model(path, path_a=True)
    ids, taps = m.generate(prompt, 5)
    bids, btaps = m.generate(prompt, 5, prompt_block=8)
    assert np.array_equal(ids, bids)
    for k in taps:
        assert same(taps[k], btaps[k]), k


def test_prompt_blocks_one_token_prompt(tmp_path):
    cfg, path = model_for("gqa_q4_0", tmp_path)
    m = oracle.Model(path)
    ids, taps = m.generate([3], 4)
    bids, btaps = m.generate([3], 4, prompt_block=8)
    assert np.array_equal(ids, bids) and same(taps["logits"], btaps["logits"])
