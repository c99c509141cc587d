"""The allocation-free decode attention entry point against the allocating one.

uaii_hip_attention_decode_noalloc runs the same kernels as
uaii_hip_attention_decode with the split partials in a fixed per-GPU device
array, so on identical inputs the outputs must be identical bit for bit. Two
calls in a row, the second with a smaller input (fewer heads, a shorter cache,
fewer keys, the other cache dtype), check that the array keeps no state that
matters between calls; the first call is also checked against the CPU oracle.
A call whose partials exceed the array is refused on the host (-3, nothing
launched).
"""
import numpy as np
import pytest

import oracle
from uaii_amd import DeviceBuffer, check_hip

pytestmark = pytest.mark.gpu


def _inputs(nh, nkv, hd, max_seq, kv_f16, seed):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal((nkv, max_seq, hd)).astype(np.float32)
    v = rng.standard_normal((nkv, max_seq, hd)).astype(np.float32)
    if kv_f16:
        k, v = k.astype(np.float16), v.astype(np.float16)
    return q, k, v


def _run(hip, fn, q, k, v, kv_f16, max_seq, nh, nkv, hd, n_keys):
    dq, dk, dv = DeviceBuffer.from_array(q), DeviceBuffer.from_array(k), DeviceBuffer.from_array(v)
    do = DeviceBuffer(nh * hd * 4)
    check_hip(fn(dq.ptr, dk.ptr, dv.ptr, kv_f16, max_seq, nh, nkv, hd, n_keys, do.ptr, None), fn.__name__)
    check_hip(hip.uaii_hip_synchronize())
    return do.to_array(np.float32, nh * hd)


def _oracle(q, k, v, nh, nkv, hd, n_keys):
    max_seq = k.shape[1]
    kf = k.astype(np.float32).transpose(1, 0, 2).reshape(max_seq, nkv * hd)
    vf = v.astype(np.float32).transpose(1, 0, 2).reshape(max_seq, nkv * hd)
    kc, vc = np.ascontiguousarray(kf[: n_keys - 1]), np.ascontiguousarray(vf[: n_keys - 1])
    kn, vn = np.ascontiguousarray(kf[n_keys - 1]), np.ascontiguousarray(vf[n_keys - 1])
    want = np.zeros(nh * hd, np.float32)
    oracle.oracle().orc_attention_decode(oracle._fp(q), oracle._fp(kc), oracle._fp(vc), n_keys - 1,
                                         oracle._fp(kn), oracle._fp(vn), oracle._fp(want), nh, nkv, hd)
    return want


CASES = [
    # (n_heads, n_kv_heads, head_dim, max_seq, n_keys, kv_f16): the 8B decode shape at
    # 32 key splits, then a smaller one (8 splits, no GQA, f32 cache)
    (32, 8, 128, 4096, 4090, 1),
    (8, 8, 64, 1000, 333, 0),
]


def test_noalloc_matches_allocating_entry_point_twice(hip):
    for i, (nh, nkv, hd, max_seq, n_keys, kv_f16) in enumerate(CASES):
        print(f"noalloc case {i}: heads {nh}/{nkv} hd {hd} max_seq {max_seq} keys {n_keys} f16 {kv_f16}",
              flush=True)
        q, k, v = _inputs(nh, nkv, hd, max_seq, kv_f16, seed=40 + i)
        ref = _run(hip, hip.uaii_hip_attention_decode, q, k, v, kv_f16, max_seq, nh, nkv, hd, n_keys)
        got = _run(hip, hip.uaii_hip_attention_decode_noalloc, q, k, v, kv_f16, max_seq, nh, nkv, hd,
                   n_keys)
        assert np.array_equal(got, ref), f"case {i}: allocation-free output differs"
        want = _oracle(q, k, v, nh, nkv, hd, n_keys)
        err = float(np.abs(got.astype(np.float64) - want).max() / np.abs(want).max())
        assert err < 1e-5, f"case {i}: max rel err {err:.3e} against the oracle"


def test_noalloc_refuses_partials_beyond_its_array(hip):
    # 64 kv heads x 32 splits x 258 floats x 4 B = 2.1 MB > 2 MiB: refused before launch
    nh = nkv = 64
    hd, max_seq = 256, 4096
    buf = DeviceBuffer(16)
    rc = hip.uaii_hip_attention_decode_noalloc(buf.ptr, buf.ptr, buf.ptr, 1, max_seq, nh, nkv, hd, 1,
                                               buf.ptr, None)
    assert rc == -3
    assert b"scratch" in hip.uaii_hip_error_string(rc)
    # key positions are 32-bit in the kernels: a cache of 2^31 or more positions
    # (or 2^32 keys, which a 32-bit count would read as 0) is refused by both
    # entry points before any launch
    for max_seq, n_keys in ((1 << 31, 1), (1 << 32, 1 << 32)):
        for fn in (hip.uaii_hip_attention_decode_noalloc, hip.uaii_hip_attention_decode):
            rc = fn(buf.ptr, buf.ptr, buf.ptr, 1, max_seq, 8, 8, 64, n_keys, buf.ptr, None)
            assert rc == -1, (fn.__name__, max_seq, n_keys, rc)
