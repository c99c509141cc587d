"""Pins the oracle's half conversion and GGUF block decoders (CPU only).

Checks that do not restate the oracle's own formula:
  * exhaustive half -> float over all 65536 codes against numpy's IEEE float16;
  * the reference's own Q4_0 known-answer block (tests/unit/quant_dequant_test.cpp:37-80);
  * special blocks whose value is fixed by the format (unit scales, zero mins);
  * random bytes of every format against the reference's compiled decoder
    (oracle/_ref, libs/uaii-quant/src/gguf_dequant.cpp), bit for bit;
  * round trips through the build's quantizers stay within half a step.
"""
import numpy as np
import pytest

import oracle
import uaii_amd
from uaii_amd import synth

BLOCKQ = [uaii_amd.Q4_0, uaii_amd.Q4_1, uaii_amd.Q5_0, uaii_amd.Q5_1, uaii_amd.Q8_0,
          uaii_amd.Q2_K, uaii_amd.Q3_K, uaii_amd.Q4_K, uaii_amd.Q5_K, uaii_amd.Q6_K]


def test_half_to_float_exhaustive():
    O = oracle.oracle()
    codes = np.arange(65536, dtype=np.uint16)
    want = codes.view(np.float16).astype(np.float32)
    got = np.array([O.orc_half_to_float(int(c)) for c in codes], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_reference_q4_0_known_answer():
    # quant_dequant_test.cpp:37-47: d = 0.5, qs[j] = ((j+1)%8) | ((j+4)%8) << 4
    blk = np.zeros(18, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    for j in range(16):
        blk[2 + j] = ((j + 1) % 8) | (((j + 4) % 8) << 4)
    got = oracle.dequant(uaii_amd.Q4_0, blk, 1, 32)[0]
    want = np.array([(((j + 1) % 8) - 8) * 0.5 for j in range(16)] +
                    [(((j + 4) % 8) - 8) * 0.5 for j in range(16)], np.float32)
    assert np.array_equal(got, want)


def test_q8_0_unit_scale_is_identity():
    blk = np.zeros(34, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    q = np.arange(-16, 16, dtype=np.int8)
    blk[2:] = q.view(np.uint8)
    assert np.array_equal(oracle.dequant(uaii_amd.Q8_0, blk, 1, 32)[0], q.astype(np.float32))


def test_q4_k_unit_scales_zero_mins_give_nibbles():
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)  # d
    blk[2:4] = np.frombuffer(np.float16(0.0).tobytes(), np.uint8)  # dmin
    # scale 1 and min 0 for all 8 sub-blocks: 6-bit fields j<4 in bytes 0..7, j>=4 in 8..11
    blk[4:8] = 1
    blk[8:12] = 0
    blk[12:16] = 1
    rng = np.random.default_rng(1)
    qs = rng.integers(0, 256, 128, dtype=np.uint8)
    blk[16:] = qs
    got = oracle.dequant(uaii_amd.Q4_K, blk, 1, 256)[0]
    want = np.concatenate([np.concatenate([qs[32 * c:32 * c + 32] & 15, qs[32 * c:32 * c + 32] >> 4])
                           for c in range(4)]).astype(np.float32)
    assert np.array_equal(got, want)


def test_q6_k_unit_scales_give_codes_minus_32():
    blk = np.zeros(210, np.uint8)
    blk[192:208] = 1  # int8 scales
    blk[208:210] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    # all-zero low/high bits -> every code is 0 - 32
    assert np.array_equal(oracle.dequant(uaii_amd.Q6_K, blk, 1, 256)[0], np.full(256, -32.0, np.float32))
    blk[0:128] = 0xff  # low nibbles 15, high bits 0 -> 15 - 32
    assert np.array_equal(oracle.dequant(uaii_amd.Q6_K, blk, 1, 256)[0], np.full(256, -17.0, np.float32))


@pytest.mark.parametrize("t", BLOCKQ, ids=lambda t: uaii_amd.TYPE_NAMES[t])
def test_random_bytes_match_reference_decoder(t):
    if oracle.ref() is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    rng = np.random.default_rng(1000 + t)
    cols, rows = 1024, 16
    p = rng.integers(0, 256, rows * uaii_amd.row_bytes(t, cols), dtype=np.uint8)
    got = oracle.dequant(t, p, rows, cols)
    want = oracle.dequant(t, p, rows, cols, use_ref=True)
    both_nan = np.isnan(got) & np.isnan(want)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[~both_nan].view(np.uint32), want[~both_nan].view(np.uint32))


@pytest.mark.parametrize("t", BLOCKQ, ids=lambda t: uaii_amd.TYPE_NAMES[t])
def test_quantizer_round_trip_within_half_step(t):
    x = synth.normals(3, 0, 0, 4096, 0.02)
    p = synth.quantize(t, x)
    assert p.nbytes == uaii_amd.row_bytes(t, 4096)
    y = oracle.dequant(t, p, 1, 4096)[0]
    err = np.abs(y - x)
    # a generous per-format bound relative to the block range (4-bit ~ 1/15 of range)
    bits = {uaii_amd.Q4_0: 4, uaii_amd.Q4_1: 4, uaii_amd.Q5_0: 5, uaii_amd.Q5_1: 5, uaii_amd.Q8_0: 8,
            uaii_amd.Q2_K: 2, uaii_amd.Q3_K: 3, uaii_amd.Q4_K: 4, uaii_amd.Q5_K: 5, uaii_amd.Q6_K: 6}[t]
    rng = np.abs(x).max() * 2
    assert err.max() <= rng / (2 ** bits - 1) * 1.01
    assert np.corrcoef(x, y)[0, 1] > {2: 0.8, 3: 0.9}.get(bits, 0.97)
