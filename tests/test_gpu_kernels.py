"""HIP kernel parity against the CPU oracle (through the uaii_hip_* C ABI).

Bars: dequantized weights bit-exact; GEMV within 2e-3 max relative error
(max |gpu - cpu| / max |cpu|, the tensor-scale relative error) of the oracle's
per-row dequant + sequential f32 dot; small ops within 1e-5 of the oracle.
"""
import ctypes as C

import numpy as np
import pytest

import oracle
import uaii_amd
from uaii_amd import synth, DeviceBuffer, DeviceWeight, check_hip

pytestmark = pytest.mark.gpu

ALL_TYPES = [uaii_amd.Q4_0, uaii_amd.Q8_0, uaii_amd.Q4_K, uaii_amd.Q6_K, uaii_amd.Q4_1,
             uaii_amd.Q5_0, uaii_amd.Q5_1, uaii_amd.Q5_K, uaii_amd.Q2_K, uaii_amd.Q3_K,
             uaii_amd.F32, uaii_amd.F16]


def maxrel(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max() / max(np.abs(b).max(), 1e-30))


def random_packed(t, rows, cols, seed):
    """Seeded weights quantized by the build's writer, plus random raw bytes for
    the payload formats so every bit pattern is exercised."""
    x = synth.normals(seed, 0, 0, rows * cols, 0.02)
    if t in (uaii_amd.F32, uaii_amd.F16):
        return (x.astype(np.float32 if t == uaii_amd.F32 else np.float16)).view(np.uint8).copy()
    return synth.quantize(t, x)


def raw_random_blocks(t, rows, cols, seed):
    """Uniformly random block bytes with finite f16 scales (exercises all codes)."""
    rng = np.random.default_rng(seed)
    rb = uaii_amd.row_bytes(t, cols)
    p = rng.integers(0, 256, size=rows * rb, dtype=np.uint8)
    be, bb = uaii_amd.BLOCK[t]
    blocks = p.reshape(-1, bb)
    # keep f16 scale fields finite (exponent < 31) at their offsets
    offs = {uaii_amd.Q4_0: [0], uaii_amd.Q8_0: [0], uaii_amd.Q4_1: [0, 2], uaii_amd.Q5_0: [0],
            uaii_amd.Q5_1: [0, 2], uaii_amd.Q4_K: [0, 2], uaii_amd.Q5_K: [0, 2],
            uaii_amd.Q6_K: [208], uaii_amd.Q2_K: [80, 82], uaii_amd.Q3_K: [108]}[t]
    for o in offs:
        blocks[:, o + 1] &= 0x7b  # exponent bits < 0x1f
    return p


@pytest.mark.parametrize("t", ALL_TYPES[:10], ids=lambda t: uaii_amd.TYPE_NAMES[t])
def test_dequant_bit_exact_random_bytes(hip, t):
    rows, cols = 24, 512
    p = raw_random_blocks(t, rows, cols, seed=100 + t)
    w = DeviceWeight(t, p, rows, cols)
    out = DeviceBuffer(rows * cols * 4)
    check_hip(hip.uaii_hip_dequant_rows(w.h, 0, rows, out.ptr, None), "dequant")
    check_hip(hip.uaii_hip_synchronize())
    got = out.to_array(np.float32, rows * cols).reshape(rows, cols)
    want = oracle.dequant(t, p, rows, cols)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), "dequant not bit-exact"


@pytest.mark.parametrize("t", ALL_TYPES, ids=lambda t: uaii_amd.TYPE_NAMES[t])
def test_dequant_bit_exact_row_window(hip, t):
    rows, cols = 40, 1024
    p = random_packed(t, rows, cols, seed=7)
    w = DeviceWeight(t, p, rows, cols)
    out = DeviceBuffer(8 * cols * 4)
    check_hip(hip.uaii_hip_dequant_rows(w.h, 17, 8, out.ptr, None), "dequant")
    got = out.to_array(np.float32, 8 * cols).reshape(8, cols)
    want = oracle.dequant(t, p, rows, cols)[17:25]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def run_gemv(hip, t, rows, cols, x, p, norm=None, eps=1e-5):
    w = DeviceWeight(t, p, rows, cols)
    dx = DeviceBuffer.from_array(x.astype(np.float32))
    dy = DeviceBuffer(rows * 4)
    if norm is None:
        check_hip(hip.uaii_hip_gemv(w.h, dx.ptr, dy.ptr, None), "gemv")
    else:
        dn = DeviceBuffer.from_array(norm.astype(np.float32))
        check_hip(hip.uaii_hip_gemv_rmsnorm(w.h, dx.ptr, dn.ptr, eps, dy.ptr, None), "gemv_rmsnorm")
    check_hip(hip.uaii_hip_synchronize())
    return dy.to_array(np.float32, rows)


@pytest.mark.parametrize("t", ALL_TYPES, ids=lambda t: uaii_amd.TYPE_NAMES[t])
def test_gemv_small_all_formats(hip, t):
    rows, cols = 96, 1536
    p = random_packed(t, rows, cols, seed=21)
    x = synth.normals(99, 1, 0, cols, 1.0)
    got = run_gemv(hip, t, rows, cols, x, p)
    want = oracle.quant_gemm(t, x, p, rows)[0]
    assert maxrel(got, want) < 2e-5


def positive_scales(t, p, rows, cols):
    """The same blocks with every scale made non-negative (and the Q4_K mins
    zeroed), so all of a row's weights share a sign per block: rounding errors of
    the kernel's partial sums then add up coherently across the row instead of
    averaging out over random-sign scales."""
    be, bb = uaii_amd.BLOCK[t]
    b = p.reshape(-1, bb).copy()
    if t == uaii_amd.Q4_0:
        b[:, 1] &= 0x7f                       # d
    elif t == uaii_amd.Q4_K:
        b[:, 1] &= 0x7f                       # d
        b[:, 2:4] = 0                         # dmin
    elif t == uaii_amd.Q6_K:
        b[:, 192:208] &= 0x7f                 # int8 sub-block scales
        b[:, 209] &= 0x7f                     # d
    return b.reshape(-1)


@pytest.mark.parametrize("t", [uaii_amd.Q4_0, uaii_amd.Q4_K, uaii_amd.Q6_K],
                         ids=lambda t: uaii_amd.TYPE_NAMES[t])
def test_gemv_pair_formats_unbiased(hip, t):
    """The f16-pair GEMV (v_dot2 on nibbles as f16 subnormals) against the oracle
    on same-sign scales. With the activation's hi part rounded to f16 alone, the
    hi partial sums rounded in the dot instruction's accumulator, biased
    downward; on Q4_K's positive scales every row was off by the same ~3e-5
    (relative), with random-sign scales the error looked like noise. Both the
    largest error and the mean error over rows are bounded."""
    rows, cols = 256, 4096
    p = positive_scales(t, random_packed(t, rows, cols, seed=41), rows, cols)
    x = synth.normals(42, 1, 0, cols, 1.0)
    got = run_gemv(hip, t, rows, cols, x, p).astype(np.float64)
    want = oracle.quant_gemm(t, x, p, rows)[0].astype(np.float64)
    scale = np.abs(want).max()
    assert maxrel(got, want) < 4e-6
    assert abs((got - want).mean()) / scale < 1e-6


@pytest.mark.parametrize("t", [uaii_amd.Q4_0, uaii_amd.Q4_1, uaii_amd.Q4_K, uaii_amd.Q6_K],
                         ids=lambda t: uaii_amd.TYPE_NAMES[t])
def test_gemv_pair_formats_chunk_scales(hip, t):
    """The f16-pair GEMV scales each 32-input chunk by its own power of two: chunks
    from 1e-20 to 1e20 and all-zero chunks in one input (no chunk's scale may
    overflow, underflow or poison the sum). The error is measured against the
    largest output, which the 1e20 chunks dominate, so the small chunks are only
    held to finiteness here; their own precision is what the other GEMV tests
    check at unit scale. A kernel chunk is 32 consecutive inputs for Q4_0/Q4_1,
    but two 16-input runs 32 (Q4_K) or 64 (Q6_K) apart, so the scales are set
    per aligned span of 32, 64 or 128 inputs: every format then gets chunks
    that are all zero and chunks under one scale."""
    rows, cols = 64, 2048
    span = {uaii_amd.Q4_0: 32, uaii_amd.Q4_1: 32, uaii_amd.Q4_K: 64, uaii_amd.Q6_K: 128}[t]
    p = random_packed(t, rows, cols, seed=51)
    x = synth.normals(52, 1, 0, cols, 1.0).astype(np.float64)
    rng = np.random.default_rng(53)
    expo = rng.integers(-20, 21, cols // span)
    expo[::7] = -99  # all-zero spans
    scale = np.where(expo == -99, 0.0, 10.0 ** expo.astype(np.float64))
    x = (x.reshape(-1, span) * scale[:, None]).reshape(-1).astype(np.float32)
    got = run_gemv(hip, t, rows, cols, x, p)
    want = oracle.quant_gemm(t, x, p, rows)[0]
    assert np.all(np.isfinite(got))
    assert maxrel(got, want) < 2e-5


@pytest.mark.parametrize("t", [uaii_amd.Q4_0, uaii_amd.Q4_K, uaii_amd.Q6_K],
                         ids=lambda t: uaii_amd.TYPE_NAMES[t])
def test_gemv_pair_formats_outlier_channels(hip, t):
    """Inputs with a few 30-100x channels per 64 (as after an RMSNorm with large
    norm weights). A kernel chunk's power-of-two scale follows its largest input,
    so unit-scale inputs that share a chunk with an outlier are held on a coarser
    hi grid and rely on the lo part; each row's error is bounded against that
    row's non-outlier contribution (sum of |w x| over the unit channels), against
    the exact product of the dequantized weights in f64."""
    rows, cols = 512, 4096
    p = random_packed(t, rows, cols, seed=61)
    rng = np.random.default_rng(62)
    x = rng.standard_normal(cols)
    out_idx = np.concatenate([64 * g + rng.choice(64, 3, replace=False) for g in range(cols // 64)])
    x[out_idx] = rng.choice([-1.0, 1.0], out_idx.size) * rng.uniform(30.0, 100.0, out_idx.size)
    x = x.astype(np.float32)
    got = run_gemv(hip, t, rows, cols, x, p).astype(np.float64)
    w = oracle.dequant(t, p, rows, cols).astype(np.float64)
    exact = w @ x.astype(np.float64)
    rest = np.ones(cols, bool)
    rest[out_idx] = False
    l1_rest = np.abs(w[:, rest]) @ np.abs(x[rest].astype(np.float64))
    err = np.abs(got - exact) / l1_rest
    assert err.max() < 2e-5, f"worst row error {err.max():.3e} of its unit-channel L1"
    # the oracle (sequential f32) is held to the same bar, so the device is no worse
    want = oracle.quant_gemm(t, x, p, rows)[0].astype(np.float64)
    assert (np.abs(want - exact) / l1_rest).max() < 2e-5


@pytest.mark.parametrize("t", [uaii_amd.Q4_0, uaii_amd.Q8_0, uaii_amd.Q4_K, uaii_amd.Q6_K],
                         ids=lambda t: uaii_amd.TYPE_NAMES[t])
@pytest.mark.parametrize("shape", [(4096, 4096), (4096, 14336), (14336, 4096)],
                         ids=lambda s: f"{s[0]}x{s[1]}")
@pytest.mark.parametrize("act", ["f32", "f16"])
def test_gemv_config_shapes(hip, t, shape, act):
    """Config 2 shapes (N x K) at M=1 against the oracle's CPU dequant-matmul, with
    N(0,1) activations in f32 and as fp16 values (the reference takes f32 rows, so
    fp16 activations enter as their exact f32 values)."""
    rows, cols = shape
    p = random_packed(t, rows, cols, seed=3)
    x = synth.normals(98, 1, 0, cols, 1.0)
    if act == "f16":
        x = x.astype(np.float16).astype(np.float32)
    got = run_gemv(hip, t, rows, cols, x, p)
    want = oracle.quant_gemm(t, x, p, rows, nthreads=0)[0]
    assert maxrel(got, want) < 2e-3
    assert maxrel(got, want) < 1e-4  # in practice ~1e-6: f32 sums in a different order


def test_gemv_bench_pattern_known_answer(hip):
    """The reference benchmark's Q4_0 pattern (uaii_bench.cpp:505-518): d = 1.0,
    qs[i] = (i + block) & 0xff, a[i] = 0.01 * ((i % 17) + 1), N=2048, K=4096;
    compared with the exact f64 sum."""
    rows, cols = 2048, 4096
    nb = rows * cols // 32
    blk = np.zeros((nb, 18), dtype=np.uint8)
    blk[:, 0], blk[:, 1] = 0x00, 0x3c
    b = np.arange(nb, dtype=np.int64)[:, None]
    blk[:, 2:] = ((np.arange(16)[None, :] + b) & 0xff).astype(np.uint8)
    a = (0.01 * ((np.arange(cols) % 17) + 1)).astype(np.float32)
    got = run_gemv(hip, uaii_amd.Q4_0, rows, cols, a, blk.reshape(-1))
    q = blk[:, 2:].astype(np.int64)
    vals = np.concatenate([(q & 15) - 8, (q >> 4) - 8], axis=1).reshape(rows, cols).astype(np.float64)
    exact = vals @ a.astype(np.float64)
    assert maxrel(got, exact) < 1e-5


def test_timing_entries(hip):
    """The other measurement entries (bench.py, kbench): each returns a positive
    time, the copy leaves dst equal to src, the timed GEMM leaves the plain GEMM's
    output, the read floor accepts a rotation of buffers, and each refuses bad
    arguments."""
    rng = np.random.default_rng(92)
    nb = 1 << 20
    src = DeviceBuffer.from_array(rng.integers(0, 256, nb, dtype=np.uint8))
    dst = DeviceBuffer(nb)
    ms = C.c_float()
    check_hip(hip.uaii_hip_time_copy(src.ptr, dst.ptr, nb, 3, C.byref(ms)), "time_copy")
    assert ms.value > 0
    assert np.array_equal(dst.to_array(np.uint8, nb), src.to_array(np.uint8, nb))
    assert hip.uaii_hip_time_copy(src.ptr, dst.ptr, nb - 4, 3, C.byref(ms)) != 0  # bytes % 16
    bufs = [DeviceBuffer(nb) for _ in range(3)]
    ptrs = (C.c_void_p * 3)(*[b.ptr for b in bufs])
    check_hip(hip.uaii_hip_time_read(ptrs, 3, nb, 4, C.byref(ms)), "time_read")
    assert ms.value > 0
    assert hip.uaii_hip_time_read(ptrs, 0, nb, 4, C.byref(ms)) != 0
    assert hip.uaii_hip_time_read(ptrs, 3, 0, 4, C.byref(ms)) != 0
    rows, cols, m = 128, 256, 64
    p = rng.integers(0, 256, rows * uaii_amd.row_bytes(uaii_amd.Q4_0, cols), dtype=np.uint8)
    p.reshape(-1, 18)[:, 1] &= 0x3B
    w = DeviceWeight(uaii_amd.Q4_0, p, rows, cols)
    x = DeviceBuffer.from_array(rng.normal(0, 1, m * cols).astype(np.float32))
    y, y0 = DeviceBuffer(4 * m * rows), DeviceBuffer(4 * m * rows)
    check_hip(hip.uaii_hip_time_gemm(w.h, x.ptr, m, y.ptr, 2, C.byref(ms)), "time_gemm")
    assert ms.value > 0
    check_hip(hip.uaii_hip_gemm(w.h, x.ptr, m, y0.ptr, None), "gemm")
    check_hip(hip.uaii_hip_synchronize())
    assert np.array_equal(y.to_array(np.float32, m * rows), y0.to_array(np.float32, m * rows))
    assert hip.uaii_hip_time_gemm(w.h, x.ptr, 0, y.ptr, 2, C.byref(ms)) != 0


def test_time_gemv_rotate(hip):
    """The measurement entry that takes GEMV weights in turn (bench.py's
    published-shape figure): a positive time, the last launch's output equal to
    a plain GEMV of that weight, and bad arguments refused."""
    rng = np.random.default_rng(91)
    rows, cols = 256, 1024
    ws = []
    for _ in range(3):
        p = rng.integers(0, 256, rows * uaii_amd.row_bytes(uaii_amd.Q4_0, cols), dtype=np.uint8)
        p.reshape(-1, 18)[:, 1] &= 0x3B
        ws.append(DeviceWeight(uaii_amd.Q4_0, p, rows, cols))
    x = DeviceBuffer.from_array(rng.normal(0, 1, cols).astype(np.float32))
    y, y0 = DeviceBuffer(4 * rows), DeviceBuffer(4 * rows)
    hs = (C.c_void_p * 3)(*[w.h for w in ws])
    ms = C.c_float()
    check_hip(hip.uaii_hip_time_gemv_rotate(hs, 3, x.ptr, y.ptr, 4, C.byref(ms)), "rotate")
    assert ms.value > 0
    # launches 1..4 take weights 1, 2, 0, 1: the output is weight 1's
    check_hip(hip.uaii_hip_gemv(ws[1].h, x.ptr, y0.ptr, None), "gemv")
    check_hip(hip.uaii_hip_synchronize())
    assert np.array_equal(y.to_array(np.float32, rows), y0.to_array(np.float32, rows))
    assert hip.uaii_hip_time_gemv_rotate(hs, 0, x.ptr, y.ptr, 4, C.byref(ms)) != 0


@pytest.mark.parametrize("t", [uaii_amd.Q4_0, uaii_amd.Q4_K, uaii_amd.Q6_K],
                         ids=lambda t: uaii_amd.TYPE_NAMES[t])
def test_gemv_rmsnorm_prologue(hip, t):
    rows, cols = 512, 2048
    p = random_packed(t, rows, cols, seed=5)
    x = synth.normals(97, 1, 0, cols, 3.0)
    nw = 1.0 + synth.normals(96, 1, 0, cols, 0.1)
    got = run_gemv(hip, t, rows, cols, x, p, norm=nw, eps=1e-5)
    xn = np.zeros(cols, np.float32)
    oracle.oracle().orc_rmsnorm(oracle._fp(x), oracle._fp(nw), oracle._fp(xn), cols, 1e-5)
    want = oracle.quant_gemm(t, xn, p, rows)[0]
    assert maxrel(got, want) < 1e-4


def oracle_rmsnorm(x, nw, eps=1e-5):
    xn = np.zeros(x.size, np.float32)
    oracle.oracle().orc_rmsnorm(oracle._fp(np.ascontiguousarray(x, np.float32)),
                                oracle._fp(np.ascontiguousarray(nw, np.float32)),
                                oracle._fp(xn), x.size, eps)
    return xn


@pytest.mark.parametrize("t,rows,cols", [
    (uaii_amd.Q4_0, 4096, 14336),   # the 8B down projection (K split over 4 waves)
    (uaii_amd.Q8_0, 1000, 14336),   # two steps per row group
    (uaii_amd.Q4_0, 333, 11008),    # 6 chunk columns over 4 waves (one wave idle)
    (uaii_amd.Q6_K, 512, 14336),
    (uaii_amd.Q4_0, 70, 256),       # one partial column, fewer rows than a group
], ids=lambda v: str(v))
@pytest.mark.parametrize("norm", [False, True], ids=["plain", "rmsnorm"])
def test_gemv_add_epilogue(hip, t, rows, cols, norm):
    """y += W . x' (residual add of the graph, elementwise.cpp:86-97)."""
    p = random_packed(t, rows, cols, seed=rows + cols)
    x = synth.normals(95, 1, 0, cols, 1.0)
    nw = 1.0 + synth.normals(94, 1, 0, cols, 0.1)
    y0 = synth.normals(93, 1, 0, rows, 1.0)
    w = DeviceWeight(t, p, rows, cols)
    dx, dn, dy = DeviceBuffer.from_array(x), DeviceBuffer.from_array(nw), DeviceBuffer.from_array(y0)
    check_hip(hip.uaii_hip_gemv_add(w.h, dx.ptr, dn.ptr if norm else None, 1e-5, dy.ptr, None))
    got = dy.to_array(np.float32, rows)
    xin = oracle_rmsnorm(x, nw) if norm else x
    want = y0 + oracle.quant_gemm(t, xin, p, rows, nthreads=0)[0]
    assert maxrel(got, want) < 1e-4


@pytest.mark.parametrize("t,rows,cols", [
    (uaii_amd.Q4_0, 4096, 14336),   # the 8B down projection: 14 slices x 64 row blocks of 64 rows
    (uaii_amd.Q4_0, 2048, 8192),    # 8 slices, 32-row blocks
    (uaii_amd.Q4_0, 4096, 4096),
    (uaii_amd.Q4_0, 48, 1024),      # one slice, 16-row blocks
    (uaii_amd.Q6_K, 2048, 8192),    # the 1B down projection: 4 super-blocks per slice
    (uaii_amd.Q6_K, 4096, 14336),
    (uaii_amd.Q6_K, 48, 1024),
], ids=lambda v: uaii_amd.TYPE_NAMES.get(v, str(v)) if isinstance(v, int) and v in uaii_amd.TYPE_NAMES and v < 64 else str(v))
def test_gemv_add_atomic(hip, t, rows, cols):
    """y += W . x split along K with float-atomic adds (the residual add of the
    graph, elementwise.cpp:86-97, on quant_gemm_f32, quant_gemm.cpp:22-70):
    within 1e-5 of the oracle, within 1e-6 of the whole-row kernel, and two
    calls from the same y0 within 1e-6 of each other (the adds land in arrival
    order)."""
    p = random_packed(t, rows, cols, seed=rows + cols + 1)
    x = synth.normals(92, 1, 0, cols, 1.0)
    y0 = synth.normals(91, 1, 0, rows, 1.0)
    w = DeviceWeight(t, p, rows, cols)
    dx = DeviceBuffer.from_array(x)
    got = []
    for _ in range(2):
        dy = DeviceBuffer.from_array(y0)
        check_hip(hip.uaii_hip_gemv_add_atomic(w.h, dx.ptr, dy.ptr, None), "gemv_add_atomic")
        got.append(dy.to_array(np.float32, rows))
    dy = DeviceBuffer.from_array(y0)
    check_hip(hip.uaii_hip_gemv_add(w.h, dx.ptr, None, 1e-5, dy.ptr, None), "gemv_add")
    whole = dy.to_array(np.float32, rows)
    want = y0 + oracle.quant_gemm(t, x, p, rows, nthreads=0)[0]
    assert maxrel(got[0], want) < 1e-5
    assert maxrel(got[0], whole) < 1e-6
    assert maxrel(got[1], got[0]) < 1e-6


def test_gemv_add_atomic_refuses_unsupported_shapes(hip):
    """Types other than Q4_0 and Q6_K, columns not a multiple of 1024, rows not
    a multiple of 16 and overlapping x and y return -1 before any launch."""
    x, y = DeviceBuffer(4 * 4096), DeviceBuffer(4 * 4096)
    for t, rows, cols in [(uaii_amd.Q4_K, 64, 1024), (uaii_amd.Q8_0, 64, 1024), (uaii_amd.Q4_0, 64, 1536),
                          (uaii_amd.Q4_0, 24, 1024)]:
        w = DeviceWeight(t, random_packed(t, rows, cols, seed=7), rows, cols)
        assert hip.uaii_hip_gemv_add_atomic(w.h, x.ptr, y.ptr, None) == -1, (t, rows, cols)
    # a supported shape whose x and y overlap (x is read while y takes adds)
    w = DeviceWeight(uaii_amd.Q4_0, random_packed(uaii_amd.Q4_0, 64, 1024, seed=7), 64, 1024)
    assert hip.uaii_hip_gemv_add_atomic(w.h, x.ptr, x.ptr, None) == -1
    assert hip.uaii_hip_gemv_add_atomic(w.h, x.ptr, C.c_void_p(x.ptr.value + 4 * 1000), None) == -1
    check_hip(hip.uaii_hip_synchronize())


@pytest.mark.parametrize("t", [uaii_amd.Q4_0, uaii_amd.Q8_0, uaii_amd.Q4_K, uaii_amd.Q6_K],
                         ids=lambda t: uaii_amd.TYPE_NAMES[t])
def test_gemv_swiglu_epilogue(hip, t):
    """y = silu(Wg . x') * (Wu . x') (elementwise.cpp:73-110) with the RMSNorm prologue."""
    rows, cols = 1536, 4096
    pg = random_packed(t, rows, cols, seed=11)
    pu = random_packed(t, rows, cols, seed=12)
    x = synth.normals(92, 1, 0, cols, 2.0)
    nw = 1.0 + synth.normals(91, 1, 0, cols, 0.1)
    wg, wu = DeviceWeight(t, pg, rows, cols), DeviceWeight(t, pu, rows, cols)
    dx, dn, dy = DeviceBuffer.from_array(x), DeviceBuffer.from_array(nw), DeviceBuffer(rows * 4)
    check_hip(hip.uaii_hip_gemv_swiglu(wg.h, wu.h, dx.ptr, dn.ptr, 1e-5, dy.ptr, None))
    got = dy.to_array(np.float32, rows)
    xn = oracle_rmsnorm(x, nw)
    g = oracle.quant_gemm(t, xn, pg, rows, nthreads=0)[0].astype(np.float64)
    u = oracle.quant_gemm(t, xn, pu, rows, nthreads=0)[0].astype(np.float64)
    want = g / (1.0 + np.exp(-g)) * u
    assert maxrel(got, want) < 1e-4
    # mismatched gate/up shapes are rejected before any launch
    wsmall = DeviceWeight(t, pg[: len(pg) // 2], rows // 2, cols)
    assert hip.uaii_hip_gemv_swiglu(wg.h, wsmall.h, dx.ptr, dn.ptr, 1e-5, dy.ptr, None) != 0


def test_rmsnorm_softmax_argmax(hip):
    n = 5000
    x = synth.normals(1, 2, 0, 3 * n, 2.0).reshape(3, n)
    w = 1.0 + synth.normals(1, 3, 0, n, 0.1)
    dx, dw, dy = DeviceBuffer.from_array(x), DeviceBuffer.from_array(w), DeviceBuffer(x.nbytes)
    check_hip(hip.uaii_hip_rmsnorm(dx.ptr, dw.ptr, dy.ptr, 3, n, 1e-5, None))
    got = dy.to_array(np.float32, 3 * n).reshape(3, n)
    for r in range(3):
        want = np.zeros(n, np.float32)
        oracle.oracle().orc_rmsnorm(oracle._fp(np.ascontiguousarray(x[r])), oracle._fp(w),
                                    oracle._fp(want), n, 1e-5)
        assert maxrel(got[r], want) < 1e-6
    v = np.ascontiguousarray(x[0])
    dv, dp = DeviceBuffer.from_array(v), DeviceBuffer(v.nbytes)
    check_hip(hip.uaii_hip_softmax(dv.ptr, dp.ptr, n, None))
    probs = dp.to_array(np.float32, n)
    want = np.zeros(n, np.float32)
    oracle.oracle().orc_softmax(oracle._fp(v), oracle._fp(want), n)
    assert maxrel(probs, want) < 1e-5
    assert abs(float(probs.astype(np.float64).sum()) - 1.0) < 1e-5
    # argmax with a planted tie: lowest index wins (sampling.cpp:38-50)
    v2 = v.copy()
    v2[4321] = v2[123] = v2.max() + 1.0
    dv2, di = DeviceBuffer.from_array(v2), DeviceBuffer(4)
    check_hip(hip.uaii_hip_argmax(dv2.ptr, n, di.ptr, None))
    assert int(di.to_array(np.int32, 1)[0]) == 123 == oracle.oracle().orc_argmax(oracle._fp(v2), n)


@pytest.mark.parametrize("mode", [0, 2])
def test_rope(hip, mode):
    rows, hd, nh = 5, 64, 4
    dim = hd * nh
    x = synth.normals(3, 4, 0, rows * dim, 1.0).reshape(rows, dim)
    pos = np.array([0, 1, 17, 1000, 4095], dtype=np.int32)
    tab = DeviceBuffer(4096 * hd * 4)
    check_hip(hip.uaii_hip_rope_table(500000.0, hd, 4096, tab.ptr))
    dx, dp = DeviceBuffer.from_array(x), DeviceBuffer.from_array(pos)
    check_hip(hip.uaii_hip_rope(dx.ptr, rows, dim, hd, mode, dp.ptr, tab.ptr, None))
    got = dx.to_array(np.float32, rows * dim).reshape(rows, dim)
    for r in range(rows):
        want = np.ascontiguousarray(x[r]).copy()
        oracle.oracle().orc_rope(oracle._fp(want), dim, hd, float(pos[r]), 500000.0, mode)
        assert maxrel(got[r], want) < 1e-6
    assert np.array_equal(got[0], x[0])  # position 0 is the identity


@pytest.mark.parametrize("kv_f16", [0, 1])
@pytest.mark.parametrize("heads", [(8, 8, 64), (32, 8, 128), (16, 2, 64)], ids=str)
@pytest.mark.parametrize("n_keys", [1, 7, 100, 1500])
def test_attention_decode(hip, kv_f16, heads, n_keys):
    nh, nkv, hd = heads
    max_seq = 2048
    rng = np.random.default_rng(n_keys * 7 + nh)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal((nkv, max_seq, hd)).astype(np.float32)
    v = rng.standard_normal((nkv, max_seq, hd)).astype(np.float32)
    if kv_f16:
        k, v = k.astype(np.float16), v.astype(np.float16)
    dq, dk, dv = DeviceBuffer.from_array(q), DeviceBuffer.from_array(k), DeviceBuffer.from_array(v)
    do = DeviceBuffer(nh * hd * 4)
    check_hip(hip.uaii_hip_attention_decode(dq.ptr, dk.ptr, dv.ptr, kv_f16, max_seq, nh, nkv, hd,
                                            n_keys, do.ptr, None))
    got = do.to_array(np.float32, nh * hd)
    # oracle layout: [seq][kv_dim]; past = n_keys - 1, current = the last key
    kf = k.astype(np.float32).transpose(1, 0, 2).reshape(max_seq, nkv * hd)
    vf = v.astype(np.float32).transpose(1, 0, 2).reshape(max_seq, nkv * hd)
    kc, vc = np.ascontiguousarray(kf[: n_keys - 1]), np.ascontiguousarray(vf[: n_keys - 1])
    kn, vn = np.ascontiguousarray(kf[n_keys - 1]), np.ascontiguousarray(vf[n_keys - 1])
    want = np.zeros(nh * hd, np.float32)
    if n_keys == 1:
        kc = np.zeros((1, nkv * hd), np.float32)
        vc = np.zeros((1, nkv * hd), np.float32)
    oracle.oracle().orc_attention_decode(oracle._fp(q), oracle._fp(kc), oracle._fp(vc), n_keys - 1,
                                         oracle._fp(kn), oracle._fp(vn), oracle._fp(want), nh, nkv, hd)
    assert maxrel(got, want) < 1e-5
    if n_keys == 1:  # one key: the output is that key's V for every head of its group
        assert maxrel(got, np.repeat(vf[0].reshape(nkv, hd), nh // nkv, axis=0).reshape(-1)) < 1e-6
