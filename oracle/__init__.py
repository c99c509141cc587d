"""CPU oracle bindings — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, and only as the checker. The product library never loads it.

`liboracle.so` is the plain-C restatement of the reference CPU path
(uaii_oracle.c). `libuaii_ref.so`, built from the reference's own kernel sources
where the reference tree is present (oracle/Makefile, target `ref`), pins the
restatement; it is optional at run time.

Parity status per oracle function (what pins it):
  orc_half_to_float      exhaustive 65536-value check vs numpy float16 + _ref
  orc_float_to_half      every float32 bit pattern vs numpy float16 (IEEE round to
                         nearest even), closed-form ties / subnormals / overflow;
                         with orc_half_to_float this pins orc_generate's kv_f16 mode
  orc_dequant_row        reference Q4_0 known-answer block, hand-built closed-form
                         blocks for every format, synth round-trip bounds, _ref
  orc_load_row_f32       _ref's gguf_load_tensor_f32 (the reference loader itself)
                         on whole tensors of every format, bit for bit
  orc_quant_gemm         benchmark-pattern known answer in f64, _ref
  orc_rmsnorm            unit-RMS invariant with w=1, numpy f64, _ref
  orc_rope               pos 0 identity, pair-norm preservation, numpy f64, _ref
  orc_attention_decode   ctx=1 returns V, uniform-score closed form, numpy f64, _ref
  orc_softmax/argmax     sum-to-1, lowest-index tie rule, _ref
  orc_moe_router/topk    numpy f64 softmax/top-k, renormalised weights sum to 1
  orc_generate           _ref end-to-end greedy ids + taps (reference kernels)
  orc_generate_ex        layer-major prompt blocks: bit-identical ids and taps to
                         orc_generate on every architecture variant and both caches
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "_build" / "liboracle.so"
REF_SO = HERE / "_ref" / "libuaii_ref.so"

_o = None
_r = None


class OracleError(RuntimeError):
    pass


class Taps(C.Structure):
    _fields_ = [("hidden", C.POINTER(C.c_float)), ("resid1", C.POINTER(C.c_float)),
                ("resid2", C.POINTER(C.c_float)), ("normed", C.POINTER(C.c_float)),
                ("logits", C.POINTER(C.c_float)), ("probs", C.POINTER(C.c_float))]


def _fp(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def oracle():
    global _o
    if _o is None:
        if not ORACLE_SO.exists():
            raise OracleError(f"{ORACLE_SO} missing: make -C oracle")
        L = C.CDLL(str(ORACLE_SO))
        vp, i64, f = C.c_void_p, C.c_int64, C.POINTER(C.c_float)
        L.orc_half_to_float.restype = C.c_float
        L.orc_half_to_float.argtypes = [C.c_uint16]
        L.orc_float_to_half.restype = C.c_uint16
        L.orc_float_to_half.argtypes = [C.c_float]
        L.orc_float_to_half_n.restype = None
        L.orc_float_to_half_n.argtypes = [vp, vp, i64]
        L.orc_row_bytes.restype = C.c_size_t
        L.orc_row_bytes.argtypes = [C.c_int, i64]
        L.orc_dequant_row.restype = C.c_int
        L.orc_dequant_row.argtypes = [C.c_int, vp, i64, f]
        L.orc_quant_gemm.restype = C.c_int
        L.orc_quant_gemm.argtypes = [C.c_int, f, i64, i64, vp, i64, f, C.c_int]
        L.orc_rmsnorm.restype = None
        L.orc_rmsnorm.argtypes = [f, f, f, i64, C.c_float]
        L.orc_rope.restype = None
        L.orc_rope.argtypes = [f, i64, i64, C.c_float, C.c_float, C.c_int]
        L.orc_attention_decode.restype = None
        L.orc_attention_decode.argtypes = [f, f, f, i64, f, f, f, C.c_int, C.c_int, C.c_int]
        L.orc_softmax.restype = None
        L.orc_softmax.argtypes = [f, f, i64]
        L.orc_argmax.restype = i64
        L.orc_argmax.argtypes = [f, i64]
        L.orc_silu.restype = C.c_float
        L.orc_silu.argtypes = [C.c_float]
        L.orc_moe_router.restype = None
        L.orc_moe_router.argtypes = [f, f, i64, i64, f]
        L.orc_moe_topk.restype = None
        L.orc_moe_topk.argtypes = [f, i64, C.c_int, C.POINTER(C.c_int), f]
        L.orc_model_open.restype = vp
        L.orc_model_open.argtypes = [C.c_char_p, C.c_int]
        L.orc_model_open_ex.restype = vp
        L.orc_model_open_ex.argtypes = [C.c_char_p, C.c_int, C.c_int]
        L.orc_load_row_f32.restype = C.c_int
        L.orc_load_row_f32.argtypes = [C.c_int, vp, i64, f]
        L.orc_model_close.restype = None
        L.orc_model_close.argtypes = [vp]
        L.orc_last_error.restype = C.c_char_p
        L.orc_model_hparams.restype = None
        L.orc_model_hparams.argtypes = [vp, C.POINTER(i64)]
        L.orc_model_tensor.restype = C.c_int
        L.orc_model_tensor.argtypes = [vp, C.c_char_p, C.POINTER(C.c_int), C.POINTER(i64),
                                       C.POINTER(C.c_void_p)]
        L.orc_model_fparams.restype = None
        L.orc_model_fparams.argtypes = [vp, f]
        L.orc_generate.restype = C.c_int
        L.orc_generate.argtypes = [vp, C.POINTER(i64), i64, i64, C.c_int, C.c_int, C.POINTER(i64),
                                   C.POINTER(i64), C.POINTER(Taps)]
        L.orc_generate_ex.restype = C.c_int
        L.orc_generate_ex.argtypes = [vp, C.POINTER(i64), i64, i64, C.c_int, C.c_int, i64,
                                      C.POINTER(i64), C.POINTER(i64), C.POINTER(Taps)]
        L.orc_time_decode_window.restype = C.c_double
        L.orc_time_decode_window.argtypes = [vp, i64, i64, C.c_int]
        _o = L
    return _o


def ref():
    """The reference-kernel library, or None when it was not built."""
    global _r
    if _r is None:
        if not REF_SO.exists():
            return None
        L = C.CDLL(str(REF_SO))
        vp, i64, f = C.c_void_p, C.c_int64, C.POINTER(C.c_float)
        L.uref_last_error.restype = C.c_char_p
        L.uref_dequant_row.restype = C.c_int
        L.uref_dequant_row.argtypes = [C.c_int, vp, i64, f]
        L.uref_quant_gemm.restype = C.c_int
        L.uref_quant_gemm.argtypes = [C.c_int, f, i64, i64, vp, i64, f]
        L.uref_rmsnorm.restype = C.c_int
        L.uref_rmsnorm.argtypes = [f, f, f, i64, C.c_float]
        L.uref_rope.restype = C.c_int
        L.uref_rope.argtypes = [f, i64, i64, C.c_float, C.c_float, C.c_int]
        L.uref_attention_decode.restype = C.c_int
        L.uref_attention_decode.argtypes = [f, f, f, i64, f, f, f, C.c_int, C.c_int, C.c_int]
        L.uref_softmax.restype = C.c_int
        L.uref_softmax.argtypes = [f, f, i64]
        L.uref_silu.restype = C.c_int
        L.uref_silu.argtypes = [f, f, i64]
        L.uref_argmax.restype = i64
        L.uref_argmax.argtypes = [f, i64]
        L.uref_sample_token.restype = C.c_int
        L.uref_sample_token.argtypes = [f, i64, C.c_float, C.c_float, C.c_int, C.c_float, C.c_uint64,
                                        C.POINTER(i64), i64, C.POINTER(i64)]
        L.uref_generate_sampled.restype = C.c_int
        L.uref_generate_sampled.argtypes = [C.c_char_p, C.POINTER(i64), i64, i64, C.c_float,
                                            C.c_float, C.c_int, C.c_float, C.c_uint64,
                                            C.POINTER(i64), C.POINTER(i64)]
        L.uref_generate.restype = C.c_int
        L.uref_generate.argtypes = [C.c_char_p, C.c_int, C.POINTER(i64), i64, i64, C.POINTER(i64),
                                    C.POINTER(i64), f, f]
        L.uref_generate_path_a.restype = C.c_int
        L.uref_generate_path_a.argtypes = L.uref_generate.argtypes
        L.uref_generate_kv16.restype = C.c_int
        L.uref_generate_kv16.argtypes = L.uref_generate.argtypes
        L.uref_load_tensor_f32.restype = C.c_int
        L.uref_load_tensor_f32.argtypes = [C.c_char_p, C.c_char_p, f, i64, C.POINTER(i64)]
        _r = L
    return _r


# ---------------------------------------------------------------- numpy helpers

def dequant(gguf_type: int, packed, rows: int, cols: int, use_ref: bool = False):
    import numpy as np
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.empty((rows, cols), dtype=np.float32)
    rb = oracle().orc_row_bytes(gguf_type, cols)
    fn = ref().uref_dequant_row if use_ref else oracle().orc_dequant_row
    for r in range(rows):
        rc = fn(gguf_type, C.c_void_p(p.ctypes.data + r * rb), cols, _fp(out[r]))
        if rc != 0:
            raise OracleError("dequant failed")
    return out


def load_f32(gguf_type: int, packed, rows: int, cols: int):
    """Rows as the reference's f32 weight load gives them (orc_load_row_f32)."""
    import numpy as np
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.empty((rows, cols), dtype=np.float32)
    rb = oracle().orc_row_bytes(gguf_type, cols)
    for r in range(rows):
        if oracle().orc_load_row_f32(gguf_type, C.c_void_p(p.ctypes.data + r * rb), cols, _fp(out[r])):
            raise OracleError("load_f32 failed")
    return out


def quant_gemm(gguf_type: int, a, packed, n: int, nthreads: int = 0, use_ref: bool = False):
    import numpy as np
    a = np.ascontiguousarray(a, dtype=np.float32)
    if a.ndim == 1:
        a = a[None, :]
    m, k = a.shape
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    c = np.empty((m, n), dtype=np.float32)
    if use_ref:
        rc = ref().uref_quant_gemm(gguf_type, _fp(a), m, k, p.ctypes.data_as(C.c_void_p), n, _fp(c))
    else:
        rc = oracle().orc_quant_gemm(gguf_type, _fp(a), m, k, p.ctypes.data_as(C.c_void_p), n, _fp(c),
                                     nthreads)
    if rc != 0:
        raise OracleError("quant_gemm failed")
    return c


class Model:
    """An oracle model (orc_model_open_ex) with greedy generate and taps.

    path_a=True runs the reference's Path A (weights as its f32 load gives them,
    f32 GEMM): what the reference does under its default options
    (enable_memory_reuse=1) or keep_quantized_weights=0. MoE models run Path A
    either way."""

    def __init__(self, path: str, max_layers: int = 0, path_a: bool = False):
        self.path = str(path)
        self.h = oracle().orc_model_open_ex(self.path.encode(), max_layers, int(path_a))
        if not self.h:
            raise OracleError(oracle().orc_last_error().decode())
        hp = (C.c_int64 * 12)()
        oracle().orc_model_hparams(self.h, hp)
        (self.n_layers, self.dim, self.n_heads, self.n_kv, self.head_dim, self.vocab, self.ffn,
         self.n_experts, self.top_k, self.rope_mode, self.ctx, self.tied) = list(hp)

    def generate(self, prompt, max_new: int, kv_f16: bool = False, nthreads: int = 0,
                 taps: bool = True, prompt_block: int = 0):
        """Greedy generate; prompt_block > 0 runs the prompt (all but its last
        token) layer by layer in blocks of that many tokens, with the same result
        bit for bit (faster for long prompts)."""
        import numpy as np
        p = np.ascontiguousarray(prompt, dtype=np.int64)
        out = np.zeros(len(p) + max_new + 1, dtype=np.int64)
        n = C.c_int64()
        t = None
        bufs = {}
        if taps:
            bufs = {"hidden": np.zeros(self.dim, np.float32),
                    "resid1": np.zeros((self.n_layers, self.dim), np.float32),
                    "resid2": np.zeros((self.n_layers, self.dim), np.float32),
                    "normed": np.zeros(self.dim, np.float32),
                    "logits": np.zeros(self.vocab, np.float32),
                    "probs": np.zeros(self.vocab, np.float32)}
            t = Taps(*[_fp(bufs[k]) for k in ("hidden", "resid1", "resid2", "normed", "logits", "probs")])
        rc = oracle().orc_generate_ex(self.h, p.ctypes.data_as(C.POINTER(C.c_int64)), len(p), max_new,
                                      int(kv_f16), nthreads, prompt_block,
                                      out.ctypes.data_as(C.POINTER(C.c_int64)),
                                      C.byref(n), C.byref(t) if t is not None else None)
        if rc != 0:
            raise OracleError(oracle().orc_last_error().decode())
        return out[: n.value], bufs

    def tensor(self, name: str):
        """(GGUF type, rows, cols, a copy of the raw bytes) of one tensor."""
        import numpy as np
        t = C.c_int()
        ne = (C.c_int64 * 3)()
        data = C.c_void_p()
        if oracle().orc_model_tensor(self.h, name.encode(), C.byref(t), ne, C.byref(data)) != 0:
            raise OracleError(f"tensor not found: {name}")
        cols, rows = ne[0], ne[1] * ne[2]
        nbytes = rows * oracle().orc_row_bytes(t.value, cols)
        raw = np.ctypeslib.as_array((C.c_uint8 * nbytes).from_address(data.value)).copy()
        return t.value, rows, cols, raw

    def time_decode_window(self, start_pos: int, n_steps: int, nthreads: int = 0) -> float:
        s = oracle().orc_time_decode_window(self.h, start_pos, n_steps, nthreads)
        if s < 0:
            raise OracleError(oracle().orc_last_error().decode())
        return s

    def close(self):
        if self.h:
            oracle().orc_model_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def ref_generate(path: str, prompt, max_new: int, max_layers: int = 0, n_layers: int = 0,
                 dim: int = 0, vocab: int = 0, path_a: bool = False, kv_f16: bool = False):
    """Greedy generate through the reference's compiled kernels (needs _ref);
    path_a=True loads every weight with the reference's gguf_load_tensor_f32;
    kv_f16=True rounds K and V to fp16 (the CPU's F16C conversion) before the
    reference's attention and cache append."""
    import numpy as np
    R = ref()
    if R is None:
        raise OracleError("reference kernels not built (make -C oracle ref)")
    p = np.ascontiguousarray(prompt, dtype=np.int64)
    out = np.zeros(len(p) + max_new + 1, dtype=np.int64)
    n = C.c_int64()
    logits = np.zeros(max(vocab, 1), np.float32)
    resid2 = np.zeros(max(n_layers * dim, 1), np.float32)
    fn = R.uref_generate_path_a if path_a else (R.uref_generate_kv16 if kv_f16 else R.uref_generate)
    rc = fn(str(path).encode(), max_layers, p.ctypes.data_as(C.POINTER(C.c_int64)),
                         len(p), max_new, out.ctypes.data_as(C.POINTER(C.c_int64)), C.byref(n),
                         _fp(logits) if vocab else None, _fp(resid2) if n_layers else None)
    if rc != 0:
        raise OracleError(R.uref_last_error().decode())
    return out[: n.value], logits, resid2.reshape(max(n_layers, 1), -1) if n_layers else None


def ref_load_tensor_f32(path: str, name: str):
    """A whole GGUF tensor through the reference's gguf_load_tensor_f32 (needs _ref)."""
    import numpy as np
    R = ref()
    n = C.c_int64()
    if R.uref_load_tensor_f32(str(path).encode(), name.encode(), None, 0, C.byref(n)) != 0:
        raise OracleError(R.uref_last_error().decode())
    out = np.zeros(n.value, np.float32)
    if R.uref_load_tensor_f32(str(path).encode(), name.encode(), _fp(out), n.value, C.byref(n)) != 0:
        raise OracleError(R.uref_last_error().decode())
    return out


def ref_sample_token(row, temperature, top_p, top_k, rep, seed, penalty=()):
    """One draw of the reference's sample_token_f32 with mt19937_64(seed) (needs _ref)."""
    import numpy as np
    r = np.ascontiguousarray(row, dtype=np.float32)
    pen = np.ascontiguousarray(list(penalty) or [0], dtype=np.int64)
    out = C.c_int64()
    rc = ref().uref_sample_token(_fp(r), r.size, temperature, top_p, top_k, rep, seed,
                                 pen.ctypes.data_as(C.POINTER(C.c_int64)), len(penalty), C.byref(out))
    if rc != 0:
        raise OracleError(ref().uref_last_error().decode())
    return out.value


def ref_generate_sampled(path: str, prompt, max_new: int, temperature, top_p, top_k, rep, seed):
    """Generate through the reference kernels with the reference's sampler (needs _ref)."""
    import numpy as np
    p = np.ascontiguousarray(prompt, dtype=np.int64)
    out = np.zeros(len(p) + max_new + 1, dtype=np.int64)
    n = C.c_int64()
    rc = ref().uref_generate_sampled(str(path).encode(), p.ctypes.data_as(C.POINTER(C.c_int64)), len(p),
                                     max_new, temperature, top_p, top_k, rep, seed,
                                     out.ctypes.data_as(C.POINTER(C.c_int64)), C.byref(n))
    if rc != 0:
        raise OracleError(ref().uref_last_error().decode())
    return out[: n.value]
