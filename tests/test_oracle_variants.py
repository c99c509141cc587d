"""The oracle's architecture variants against the reference's own kernels
(oracle/_ref, built from the reference sources): MoE router + experts (Path A,
transformer.cpp:446-612), a shared expert (gguf.cpp:1107-1128), the dense GELU
MLP (gguf.cpp:1156-1170, elementwise.cpp:56-71) and Q/K/V bias adds
(gguf.cpp:1014-1029). Greedy ids, last-step logits and every layer's resid2
must be bit-identical. CPU only; skipped where the reference is not built."""
import numpy as np
import pytest

import oracle
import uaii_amd
from uaii_amd import synth

VARIANTS = {
    "moe4_top2": dict(n_experts=4, top_k=2, router_std=1.0 / 16),
    "moe4_top2_shared": dict(n_experts=4, top_k=2, router_std=1.0 / 16, shared_ffn=192),
    "gelu": dict(gelu=True),
    "qkv_bias": dict(qkv_bias=True, n_kv_heads=2),
}


def cfg_for(name):
    base = dict(n_layers=2, dim=256, n_heads=4, n_kv_heads=4, ffn=320, vocab=700, ctx_len=128,
                type_default=uaii_amd.Q4_0, type_attn_v=uaii_amd.Q8_0, seed=90)
    base.update(VARIANTS[name])
    return synth.ModelConfig(**base)


@pytest.mark.parametrize("name", list(VARIANTS))
def test_oracle_matches_reference_kernels(name, tmp_path):
    if oracle.ref() is None:
        pytest.skip("reference kernels not built (make -C oracle ref needs /root/reference)")
    cfg = cfg_for(name)
    path = synth.write_model(tmp_path / f"{name}.gguf", cfg)
    prompt = np.random.default_rng(5).integers(0, cfg.vocab, 6).astype(np.int64)
    m = oracle.Model(path)
    ids, taps = m.generate(prompt, 10)
    rids, rlogits, rres = oracle.ref_generate(path, prompt, 10, n_layers=m.n_layers, dim=m.dim,
                                              vocab=m.vocab)
    assert np.array_equal(ids, rids)
    assert np.array_equal(taps["logits"].view(np.uint32), rlogits.view(np.uint32))
    assert np.array_equal(taps["resid2"].view(np.uint32), rres.view(np.uint32))
