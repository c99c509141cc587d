"""Pins the oracle's fp16 KV cache mode (CPU only).

`orc_generate(kv_f16=1)` differs from the f32 path only in that every K (after
RoPE) and V element passes through float -> half -> float before attention and
the cache append. Checks that do not restate the oracle's own conversion:
  * orc_float_to_half against an IEEE binary16 conversion (torch's CPU
    conversion, round to nearest even): every pattern of the bits it rounds at
    every exponent, every mantissa where halves are subnormal, random patterns,
    and on request (UAII_F16_EXHAUSTIVE=1) all 2^32 float32 bit patterns; NaN
    kept as a NaN of the same sign;
  * closed-form ties, subnormals, overflow to infinity and signed zeros;
  * the whole mode against the reference's own kernels (oracle/_ref) with K and
    V rounded by the CPU's F16C conversion instructions: greedy ids, last logits
    and every layer's resid2 bit-identical, on dense GQA, NeoX and bias models.
"""
import os

import numpy as np
import pytest

import oracle
import uaii_amd
from uaii_amd import synth


def to_half(x):
    O = oracle.oracle()
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    O.orc_float_to_half_n(x.ctypes.data, out.ctypes.data, x.size)
    return out


def ieee_half_bits(x):
    """IEEE binary16 bits of float32 x, round to nearest even (torch's CPU
    conversion: the F16C instructions where the host has them)."""
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(torch.float16).view(torch.int16).numpy().view(np.uint16)


def check_bits(bits):
    x = bits.view(np.float32)
    got = to_half(x)
    want = ieee_half_bits(x)
    nan = np.isnan(x)
    if nan.any():
        g = got[nan]
        assert np.all((g & 0x7C00) == 0x7C00) and np.all((g & 0x03FF) != 0), "NaN lost"
        assert np.array_equal(g & 0x8000, (bits[nan] >> 16).astype(np.uint16) & 0x8000)
    bad = np.nonzero(got[~nan] != want[~nan])[0]
    assert bad.size == 0, f"{bad.size} mismatches, first input bits {bits[~nan][bad[0]]:#010x}"


def test_float_to_half_rounding_bits():
    """Every float32 whose half is subnormal or rounds into the subnormal range
    (exponents 2^-26 .. 2^-14, all 2^23 mantissas, both signs); for every sign
    and exponent, all 2^13 patterns of the bits that the conversion rounds away
    under nine patterns of the 10 it keeps; 2^24 random patterns."""
    mant = np.arange(1 << 23, dtype=np.uint32)
    for sign in (0, 1):
        for e in range(127 - 26, 127 - 13):
            check_bits(mant | np.uint32((sign << 31) | (e << 23)))
    low = np.arange(1 << 13, dtype=np.uint32)
    for high in (0x000, 0x001, 0x002, 0x155, 0x1FF, 0x200, 0x2AA, 0x3FE, 0x3FF):
        se = np.arange(512, dtype=np.uint32) << 23
        check_bits((se[:, None] | np.uint32(high << 13) | low[None, :]).ravel())
    check_bits(np.random.default_rng(3).integers(0, 1 << 32, 1 << 24, dtype=np.uint64).astype(np.uint32))


@pytest.mark.skipif(not os.environ.get("UAII_F16_EXHAUSTIVE"),
                    reason="all 2^32 patterns take ~90 s; UAII_F16_EXHAUSTIVE=1 runs them")
def test_float_to_half_every_float32():
    chunk = 1 << 24
    base = np.arange(chunk, dtype=np.uint32)
    for c in range(1 << 32 >> 24):
        check_bits(base + np.uint32(c * chunk))


@pytest.mark.parametrize("x, h", [
    (0.0, 0x0000), (-0.0, 0x8000),
    (1.0, 0x3C00), (-2.0, 0xC000),
    (1.0 + 2.0 ** -11, 0x3C00),                  # tie below an even mantissa: stays
    (1.0 + 3 * 2.0 ** -11, 0x3C02),              # tie above an odd mantissa: up to even
    (1.0 + 2.0 ** -11 + 2.0 ** -23, 0x3C01),     # just past the tie: up
    (65504.0, 0x7BFF),                           # largest finite half
    (65519.99, 0x7BFF),                          # below the overflow tie
    (65520.0, 0x7C00),                           # the overflow tie rounds to infinity
    (-1e6, 0xFC00),
    (2.0 ** -14, 0x0400),                        # smallest normal
    (2.0 ** -24, 0x0001),                        # smallest subnormal
    (2.0 ** -25, 0x0000),                        # tie between 0 and 2^-24: even (0)
    (3 * 2.0 ** -25, 0x0002),                    # tie between 2^-24 and 2^-23: even
    (2.0 ** -25 + 2.0 ** -40, 0x0001),           # past the tie: up
    (-(2.0 ** -26), 0x8000),                     # below half the smallest subnormal: -0
    (2.0 ** -14 - 2.0 ** -25, 0x0400),           # largest subnormal + half ulp ties up to the normal
])
def test_float_to_half_closed_forms(x, h):
    O = oracle.oracle()
    assert O.orc_float_to_half(float(np.float32(x))) == h
    assert to_half(np.array([x], np.float32))[0] == h


def test_float_to_half_infinities():
    O = oracle.oracle()
    assert O.orc_float_to_half(float("inf")) == 0x7C00
    assert O.orc_float_to_half(float("-inf")) == 0xFC00


KV16_MODELS = {
    "gqa4_hd64": dict(n_heads=8, n_kv_heads=2, dim=512),
    "neox_bias": dict(n_heads=4, n_kv_heads=2, dim=256, arch="qwen2", qkv_bias=True),
    "hd128_q4k": dict(n_heads=4, n_kv_heads=1, dim=512, ffn=512, type_default=uaii_amd.Q4_K,
                      type_attn_v=uaii_amd.Q6_K),
}


@pytest.mark.parametrize("name", list(KV16_MODELS))
def test_kv_f16_mode_matches_reference_kernels(name, tmp_path):
    if oracle.ref() is None:
        pytest.skip("reference kernels not built (make -C oracle ref needs /root/reference)")
    base = dict(n_layers=2, dim=256, n_heads=4, n_kv_heads=4, ffn=384, vocab=600, ctx_len=64,
                type_default=uaii_amd.Q4_0, type_attn_v=uaii_amd.Q8_0, seed=131)
    base.update(KV16_MODELS[name])
    cfg = synth.ModelConfig(**base)
    path = synth.write_model(tmp_path / f"{name}.gguf", cfg)
    prompt = np.random.default_rng(17).integers(0, cfg.vocab, 9).astype(np.int64)
    m = oracle.Model(path)
    ids, taps = m.generate(prompt, 12, kv_f16=True)
    rids, rlogits, rres = oracle.ref_generate(path, prompt, 12, n_layers=m.n_layers, dim=m.dim,
                                              vocab=m.vocab, kv_f16=True)
    assert np.array_equal(ids, rids)
    assert np.array_equal(taps["logits"].view(np.uint32), rlogits.view(np.uint32))
    assert np.array_equal(taps["resid2"].view(np.uint32), rres.view(np.uint32))
    # the rounding is exercised: the f32-cache run's logits differ
    _, taps32 = m.generate(prompt, 12, kv_f16=False)
    assert not np.array_equal(taps32["logits"].view(np.uint32), taps["logits"].view(np.uint32))
