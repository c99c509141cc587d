"""The oracle against golden vectors written by the reference's own kernels
(tests/golden/make_golden.py over oracle/_ref): bit-exact dequant for the 10
block formats, and greedy ids, last-step logits and per-layer resid2 for the
tiny config. CPU only; the files travel with the repository."""
import hashlib
from pathlib import Path

import numpy as np
import pytest

import oracle
import uaii_amd
from uaii_amd import synth

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_dequant_matches_reference_vectors():
    g = np.load(GOLDEN / "dequant_blocks.npz")
    types = sorted(int(k.split("_")[1]) for k in g.files if k.startswith("bytes_"))
    assert len(types) == 10
    for t in types:
        p, want = g[f"bytes_{t}"], g[f"values_{t}"]
        got = oracle.dequant(t, p, want.shape[0], want.shape[1])
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), uaii_amd.TYPE_NAMES[t]


def tiny_model_or_skip():
    g = np.load(GOLDEN / "tiny_generate.npz")
    path = synth.cached_model(synth.PRESETS["tiny"])
    if hashlib.sha1(Path(path).read_bytes()).hexdigest() != str(g["gguf_sha1"]):
        pytest.fail("the synthetic tiny GGUF no longer matches the golden vectors' model")
    return g, path


def test_oracle_generate_matches_reference_vectors():
    g, path = tiny_model_or_skip()
    m = oracle.Model(path)
    ids, taps = m.generate(g["prompt"], 64, kv_f16=False)
    assert np.array_equal(ids, g["ids"])
    assert np.array_equal(taps["logits"].view(np.uint32), g["logits"].view(np.uint32))
    assert np.array_equal(taps["resid2"].view(np.uint32), g["resid2"].view(np.uint32))
