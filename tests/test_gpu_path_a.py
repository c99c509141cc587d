"""Reference default options on the device: Path A weight values, and the budget.

With the C ABI's default options (enable_memory_reuse=1, the reference's
default, libs/uaii-capi/src/capi.cpp:62-78) or keep_quantized_weights=0, the
reference holds every weight as its f32 load gives it (session.cpp:259-367,
:420-443 -> gguf_load_tensor_f32), which orders Q4_0 nibbles pairwise
(gguf.cpp:514-520). The device keeps the blocks packed with their nibbles
permuted at upload, so its values are those f32 values bit for bit. Bars as in
test_gpu_session.py: greedy ids identical over the decoded tokens, the embedding
row (`hidden`) bit-exact, hidden states and logits within 2e-3 of the oracle's
Path A, which the CPU tests pin to the reference's own loader and kernels.
"""
import numpy as np
import pytest

import oracle
import uaii_amd
from uaii_amd import synth

pytestmark = pytest.mark.gpu

CFG = synth.ModelConfig(n_layers=3, dim=512, n_heads=8, n_kv_heads=2, ffn=1024, vocab=3000,
                        ctx_len=256, type_default=uaii_amd.Q4_0, type_attn_v=uaii_amd.Q8_0, seed=31)


def maxrel(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max() / max(np.abs(b).max(), 1e-30))


def run(path, prompt, n_new, **kw):
    with uaii_amd.Session(path, **kw) as s:
        ids = s.generate(prompt, n_new)
        taps = {k: s.get(k) for k in ("hidden", "logits")}
        taps["resid2"] = np.stack([s.get(f"blk.{li}.resid2") for li in range(CFG.n_layers)])
    return ids, taps


@pytest.mark.parametrize("opts", [dict(memory_reuse=True), dict(keep_quantized=False)],
                         ids=["memory_reuse", "f32_weights"])
@pytest.mark.parametrize("kv_f16", [False, True], ids=["kv_f32", "kv_f16_prefill"])
def test_path_a_generate(opts, kv_f16):
    path = synth.cached_model(CFG)
    prompt = np.random.default_rng(3).integers(0, CFG.vocab, 24).astype(np.int64)
    print("path A", opts, "kv_f16", kv_f16, flush=True)
    ids, taps = run(path, prompt, 64, kv_f16=kv_f16, **opts)
    want_ids, want = oracle.Model(path, path_a=True).generate(prompt, 64, kv_f16=kv_f16)
    assert np.array_equal(ids, want_ids)
    assert np.array_equal(taps["hidden"], want["hidden"])
    assert maxrel(taps["logits"], want["logits"]) < 2e-3
    for li in range(CFG.n_layers):
        assert maxrel(taps["resid2"][li], want["resid2"][li]) < 2e-3


def test_path_a_matches_reference_loader_and_kernels():
    """Ids and logits against the reference's own Path A: its gguf_load_tensor_f32
    and its kernels (oracle/_ref)."""
    if oracle.ref() is None:
        pytest.skip("oracle/_ref not built")
    path = synth.cached_model(CFG)
    prompt = np.random.default_rng(4).integers(0, CFG.vocab, 10).astype(np.int64)
    ids, taps = run(path, prompt, 16, memory_reuse=True)
    m = oracle.Model(path, path_a=True)
    rids, rlog, rres = oracle.ref_generate(path, prompt, 16, n_layers=m.n_layers, dim=m.dim,
                                           vocab=m.vocab, path_a=True)
    assert np.array_equal(ids, rids)
    assert maxrel(taps["logits"], rlog) < 2e-3
    for li in range(CFG.n_layers):
        assert maxrel(taps["resid2"][li], rres[li]) < 2e-3


def test_path_b_embedding_differs_from_path_a():
    """The same Q4_0 file on the two paths: the first token's embedding row is the
    packed decode's (Path B) or the f32 load's (Path A), each bit-exact."""
    path = synth.cached_model(CFG)
    prompt = np.array([17, 3], dtype=np.int64)
    _, a = run(path, prompt, 1, memory_reuse=True)
    _, b = run(path, prompt, 1)
    _, wa = oracle.Model(path, path_a=True).generate(prompt, 1)
    _, wb = oracle.Model(path).generate(prompt, 1)
    assert np.array_equal(a["hidden"], wa["hidden"])
    assert np.array_equal(b["hidden"], wb["hidden"])
    assert not np.array_equal(a["hidden"], b["hidden"])


def test_budget_bytes():
    """A device budget below the model's bytes fails the create with the
    reference's budget error (libs/uaii-memory/src/budget.cpp:6-19); a large one
    changes nothing."""
    path = synth.cached_model(CFG)
    with pytest.raises(uaii_amd.UaiiError, match="invalid_argument.*memory budget exceeded"):
        uaii_amd.Session(path, budget_bytes=1 << 20)
    prompt = np.array([1, 2, 3], dtype=np.int64)
    with uaii_amd.Session(path, budget_bytes=1 << 34) as s:
        ids = s.generate(prompt, 4)
    want, _ = oracle.Model(path).generate(prompt, 4)
    assert np.array_equal(ids, want)
    # the KV cache counts too: the smallest budget that holds a 16-slot session
    # refuses a 256-slot one
    b16 = _smallest_budget(path, 16)
    with uaii_amd.Session(path, budget_bytes=b16, max_context=16) as s:
        assert np.array_equal(s.generate(prompt, 4), want)
    with pytest.raises(uaii_amd.UaiiError, match="memory budget exceeded"):
        uaii_amd.Session(path, budget_bytes=b16, max_context=256)


def _smallest_budget(path, max_context):
    """Smallest budget (to 4 KiB) that lets the create pass, by bisection."""
    lo, hi = 1 << 20, 1 << 34
    while hi - lo > 4096:
        mid = (lo + hi) // 2
        try:
            uaii_amd.Session(path, budget_bytes=mid, max_context=max_context).close()
            hi = mid
        except uaii_amd.UaiiError:
            lo = mid
    return hi
