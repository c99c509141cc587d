"""The reference's Path A in the oracle: weights as its f32 load gives them.

Under the reference's default options (enable_memory_reuse=1,
libs/uaii-capi/src/capi.cpp:62-78) every weight gets an f32 buffer, the packed
copy does not fit it, and the weight comes from gguf_load_tensor_f32
(libs/uaii-runtime/src/session.cpp:259-367, :420-443), which orders Q4_0
nibbles pairwise (libs/uaii-loaders/src/gguf.cpp:514-520: byte j of a block
gives elements 2j and 2j+1) where the packed decode uses the ggml order
(gguf_dequant.cpp:117-134: elements j and j+16). The oracle's orc_load_row_f32
and its Path A generate are pinned here against the reference's own loader and
kernels (oracle/_ref), bit for bit. CPU only.
"""
import numpy as np
import pytest

import oracle
import uaii_amd
from uaii_amd import synth

TYPES = [uaii_amd.Q4_0, uaii_amd.Q8_0, uaii_amd.Q4_1, uaii_amd.Q5_0, uaii_amd.Q5_1, uaii_amd.Q2_K,
         uaii_amd.Q3_K, uaii_amd.Q4_K, uaii_amd.Q5_K, uaii_amd.Q6_K]


def needs_ref():
    if oracle.ref() is None:
        pytest.skip("reference kernels not built (make -C oracle ref needs /root/reference)")


def test_q4_0_pairwise_order_closed_form():
    # one block, d = 1: byte j = j | (15 - j) << 4
    blk = np.zeros(18, np.uint8)
    blk[:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[2:] = [j | ((15 - j) << 4) for j in range(16)]
    got = oracle.load_f32(uaii_amd.Q4_0, blk, 1, 32)[0]
    want = np.empty(32, np.float32)
    want[0::2] = np.arange(16) - 8          # low nibble of byte j -> element 2j
    want[1::2] = (15 - np.arange(16)) - 8   # high nibble -> element 2j + 1
    assert np.array_equal(got, want)
    ggml = oracle.dequant(uaii_amd.Q4_0, blk, 1, 32)[0]
    assert np.array_equal(ggml[:16], np.arange(16) - 8)          # ggml: elements j ...
    assert np.array_equal(ggml[16:], (15 - np.arange(16)) - 8)   # ... and j + 16
    assert np.array_equal(np.sort(got), np.sort(ggml))           # same values, other order


@pytest.mark.parametrize("t", TYPES, ids=lambda t: uaii_amd.TYPE_NAMES[t])
def test_load_row_f32_matches_reference_loader(t, tmp_path):
    needs_ref()
    cfg = synth.ModelConfig(n_layers=1, dim=256, n_heads=4, n_kv_heads=4, ffn=512, vocab=300,
                            ctx_len=64, type_default=t, type_embd=t, type_output=t, seed=70 + t)
    path = synth.write_model(tmp_path / "m.gguf", cfg)
    m = oracle.Model(path)
    for name in ("token_embd.weight", "blk.0.attn_q.weight", "blk.0.ffn_down.weight", "output.weight"):
        typ, rows, cols, raw = m.tensor(name)
        assert typ == t
        got = oracle.load_f32(t, raw, rows, cols).reshape(-1)
        want = oracle.ref_load_tensor_f32(path, name)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), name
    m.close()


@pytest.mark.parametrize("types", [(uaii_amd.Q4_0, uaii_amd.Q8_0), (uaii_amd.Q4_K, uaii_amd.Q6_K)],
                         ids=["q4_0", "q4_k"])
def test_path_a_generate_matches_reference(types, tmp_path):
    needs_ref()
    cfg = synth.ModelConfig(n_layers=2, dim=256, n_heads=4, n_kv_heads=2, ffn=512, vocab=900,
                            ctx_len=128, type_default=types[0], type_attn_v=types[1], seed=77)
    path = synth.write_model(tmp_path / "m.gguf", cfg)
    prompt = np.random.default_rng(9).integers(0, cfg.vocab, 7).astype(np.int64)
    m = oracle.Model(path, path_a=True)
    ids, taps = m.generate(prompt, 12)
    rids, rlogits, rres = oracle.ref_generate(path, prompt, 12, n_layers=m.n_layers, dim=m.dim,
                                              vocab=m.vocab, path_a=True)
    assert np.array_equal(ids, rids)
    assert np.array_equal(taps["logits"].view(np.uint32), rlogits.view(np.uint32))
    assert np.array_equal(taps["resid2"].view(np.uint32), rres.view(np.uint32))
    # Path B on the same file: the packed decode order changes Q4_0 values
    ids_b, taps_b = oracle.Model(path).generate(prompt, 12)
    if types[0] == uaii_amd.Q4_0:
        assert not np.array_equal(taps_b["hidden"], taps["hidden"])
    else:
        assert np.array_equal(taps_b["hidden"], taps["hidden"])
