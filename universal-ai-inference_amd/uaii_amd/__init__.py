"""ctypes bindings of libuaii_amd.so (the MI355X GGUF token loop) and the
synthetic GGUF writer.

The C ABI is the product boundary (include/uaii/c_api/uaii.h and
include/uaii_hip.h); these bindings exist for tests, the smoke check and the
benchmark. Loading fails loudly when the built library is missing: there is no
CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent.parent
LIB_DIR = PKG_DIR / "lib"
# UAII_AMD_LIB selects another build of the same library (A/B timing of builds).
LIB_PATH = Path(os.environ["UAII_AMD_LIB"]) if os.environ.get("UAII_AMD_LIB") else LIB_DIR / "libuaii_amd.so"
SYNTH_PATH = LIB_DIR / "libuaii_synth.so"

# GGUF tensor type ids (reference include/uaii/loaders/gguf.hpp:18-36)
F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 0, 1, 2, 3, 6, 7, 8, 10, 11, 12, 13, 14
TYPE_NAMES = {F32: "f32", F16: "f16", Q4_0: "q4_0", Q4_1: "q4_1", Q5_0: "q5_0", Q5_1: "q5_1",
              Q8_0: "q8_0", Q2_K: "q2_k", Q3_K: "q3_k", Q4_K: "q4_k", Q5_K: "q5_k", Q6_K: "q6_k"}
BLOCK = {F32: (1, 4), F16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20), Q5_0: (32, 22), Q5_1: (32, 24),
         Q8_0: (32, 34), Q2_K: (256, 84), Q3_K: (256, 110), Q4_K: (256, 144), Q5_K: (256, 176),
         Q6_K: (256, 210)}


def row_bytes(t: int, cols: int) -> int:
    be, bb = BLOCK[t]
    return cols // be * bb


class UaiiError(RuntimeError):
    pass


class SessionOptions(C.Structure):
    """uaii_session_options (identical layout to the reference's C API 0.3.0)."""
    _fields_ = [
        ("struct_size", C.c_uint32),
        ("backend", C.c_char_p),
        ("weights_dir", C.c_char_p),
        ("weight_init", C.c_int),
        ("enable_fusion", C.c_int),
        ("enable_memory_reuse", C.c_int),
        ("enable_profiler", C.c_int),
        ("profile_trace_path", C.c_char_p),
        ("budget_bytes", C.c_uint64),
        ("enable_streaming", C.c_int),
        ("allow_missing_weights", C.c_int),
        ("weights_sandbox", C.c_char_p),
        ("compute_dtype", C.c_int),
        ("keep_quantized_weights", C.c_int),
        ("max_context", C.c_int64),
    ]


_lib = None


class TensorView(C.Structure):
    """uaii_tensor_view: the fields of the reference's kernels::TensorView
    (include/uaii/kernels/tensor_view.hpp:12-24)."""
    _fields_ = [("dtype", C.c_int32), ("shape", C.POINTER(C.c_int64)), ("rank", C.c_size_t),
                ("data", C.c_void_p), ("nbytes", C.c_size_t), ("quant_format", C.c_int32),
                ("quant_rows", C.c_int64), ("quant_cols", C.c_int64)]


class Attribute(C.Structure):
    """uaii_attribute: ir::Attribute (include/uaii/ir/attribute.hpp:11-31)."""
    _fields_ = [("key", C.c_char_p), ("type", C.c_int32), ("i", C.c_int64), ("f", C.c_double),
                ("s", C.c_char_p)]


# uaii::DType and quant::QuantFormat values (include/uaii/interfaces/types.hpp:13-24,
# include/uaii/quant/formats.hpp:11-30)
DTYPE_F32, DTYPE_F16 = 1, 2
QUANT_FORMAT = {F32: 0, F16: 1, Q4_0: 7, Q4_1: 8, Q5_0: 9, Q5_1: 10, Q8_0: 11, Q2_K: 12, Q3_K: 13,
                Q4_K: 14, Q5_K: 15, Q6_K: 16}


class SampleParams(C.Structure):
    """uaii_sample_params (include/uaii/c_api/uaii_ext.h)."""
    _fields_ = [("struct_size", C.c_uint32), ("temperature", C.c_float), ("top_p", C.c_float),
                ("top_k", C.c_int32), ("repetition_penalty", C.c_float), ("seed", C.c_uint64),
                ("has_seed", C.c_int)]


def sample_params(temperature=0.0, top_p=1.0, top_k=0, repetition_penalty=1.0, seed=None):
    p = SampleParams()
    lib().uaii_sample_params_init(C.byref(p))
    p.temperature, p.top_p, p.top_k, p.repetition_penalty = temperature, top_p, top_k, repetition_penalty
    if seed is not None:
        p.seed, p.has_seed = seed, 1
    return p


def sample_uniforms(seed: int, n: int):
    """The first n draws of uniform_real_distribution<float>(0, 1) over
    mt19937_64(seed): the uniforms the reference's sampler takes, in order."""
    import numpy as np
    out = np.zeros(max(n, 1), dtype=np.float32)
    rc = lib().uaii_sample_uniforms(C.c_uint64(seed % (1 << 64)), n,
                                    out.ctypes.data_as(C.POINTER(C.c_float)))
    if rc != 0:
        raise UaiiError(f"uaii_sample_uniforms: {rc}")
    return out[:n]


def sample_token(row, params: "SampleParams", penalty=()):
    """One host draw of the sampler (fresh mt19937_64(params.seed))."""
    import numpy as np
    r = np.ascontiguousarray(row, dtype=np.float32)
    pen = np.ascontiguousarray(list(penalty) or [0], dtype=np.int64)
    out = C.c_int64()
    L = lib()
    rc = L.uaii_sample_token(r.ctypes.data_as(C.POINTER(C.c_float)), r.size, C.byref(params),
                             pen.ctypes.data_as(C.POINTER(C.c_int64)), len(penalty), C.byref(out))
    if rc != 0:
        raise UaiiError(f"uaii_sample_token: {L.uaii_last_error().decode()}")
    return out.value


def lib() -> C.CDLL:
    """Load libuaii_amd.so (raises if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise UaiiError(f"{LIB_PATH} is missing: run __graft_entry__.build() first")
    L = C.CDLL(str(LIB_PATH))
    vp, i64, i32, f32p = C.c_void_p, C.c_int64, C.c_int32, C.POINTER(C.c_float)
    sig = {
        "uaii_session_options_init": (None, [C.POINTER(SessionOptions)]),
        "uaii_status_name": (C.c_char_p, [C.c_int]),
        "uaii_last_error": (C.c_char_p, []),
        "uaii_get_c_api_version_string": (C.c_char_p, []),
        "uaii_get_version_string": (C.c_char_p, []),
        "uaii_session_create": (C.c_int, [C.c_char_p, C.POINTER(SessionOptions), C.POINTER(vp)]),
        "uaii_session_destroy": (None, [vp]),
        "uaii_session_run": (C.c_int, [vp]),
        "uaii_session_set_f32": (C.c_int, [vp, C.c_char_p, f32p, C.c_size_t]),
        "uaii_session_get_f32": (C.c_int, [vp, C.c_char_p, f32p, C.c_size_t, C.POINTER(C.c_size_t)]),
        "uaii_session_generate": (C.c_int, [vp, C.POINTER(i64), C.c_size_t, i64, C.POINTER(i64),
                                            C.c_size_t, C.POINTER(C.c_size_t)]),
        "uaii_session_profile_summary": (C.c_int, [vp, C.c_char_p, C.c_size_t]),
        "uaii_session_begin": (C.c_int, [vp, C.POINTER(i64), C.c_size_t, i64]),
        "uaii_session_step_async": (C.c_int, [vp, C.c_int]),
        "uaii_session_sync": (C.c_int, [vp]),
        "uaii_session_prefill": (C.c_int, [vp, i64]),
        "uaii_session_prefill_supported": (C.c_int, [vp, C.POINTER(C.c_int)]),
        "uaii_session_position": (C.c_int, [vp, C.POINTER(i64)]),
        "uaii_session_read_ids": (C.c_int, [vp, C.POINTER(i64), C.c_size_t]),
        "uaii_session_seek": (C.c_int, [vp, i64]),
        "uaii_session_set_profiling": (C.c_int, [vp, C.c_int]),
        "uaii_session_last_margin": (C.c_int, [vp, f32p, f32p]),
        "uaii_session_set_device_sampler": (C.c_int, [vp, C.c_int]),
        "uaii_sample_params_init": (None, [C.POINTER(SampleParams)]),
        "uaii_session_generate_sampled": (C.c_int, [vp, C.POINTER(i64), C.c_size_t, i64,
                                                    C.POINTER(SampleParams), C.POINTER(i64),
                                                    C.c_size_t, C.POINTER(C.c_size_t)]),
        "uaii_sample_token": (C.c_int, [f32p, C.c_size_t, C.POINTER(SampleParams), C.POINTER(i64),
                                        C.c_size_t, C.POINTER(i64)]),
        "uaii_model_describe": (C.c_int, [C.c_char_p, C.c_char_p, C.c_size_t]),
        "uaii_hip_init": (C.c_int, [C.c_int]),
        "uaii_hip_device_count": (C.c_int, [C.POINTER(C.c_int)]),
        "uaii_hip_error_string": (C.c_char_p, [C.c_int]),
        "uaii_hip_malloc": (C.c_int, [C.POINTER(vp), C.c_size_t]),
        "uaii_hip_free": (C.c_int, [vp]),
        "uaii_hip_memcpy_h2d": (C.c_int, [vp, vp, C.c_size_t]),
        "uaii_hip_memcpy_d2h": (C.c_int, [vp, vp, C.c_size_t]),
        "uaii_hip_memset": (C.c_int, [vp, C.c_int, C.c_size_t]),
        "uaii_hip_synchronize": (C.c_int, []),
        "uaii_hip_weight_create": (C.c_int, [C.c_int, vp, i64, i64, C.POINTER(vp)]),
        "uaii_hip_weight_destroy": (C.c_int, [vp]),
        "uaii_hip_weight_bytes": (i64, [vp]),
        "uaii_hip_dequant_rows": (C.c_int, [vp, i64, i64, vp, vp]),
        "uaii_hip_gemv": (C.c_int, [vp, vp, vp, vp]),
        "uaii_hip_gemv_rmsnorm": (C.c_int, [vp, vp, vp, C.c_float, vp, vp]),
        "uaii_hip_gemv_add": (C.c_int, [vp, vp, vp, C.c_float, vp, vp]),
        "uaii_hip_gemv_swiglu": (C.c_int, [vp, vp, vp, vp, C.c_float, vp, vp]),
        "uaii_hip_gemm": (C.c_int, [vp, vp, i64, vp, vp]),
        "uaii_hip_gemm_rmsnorm": (C.c_int, [vp, vp, i64, vp, C.c_float, vp, vp]),
        "uaii_hip_gemm_add": (C.c_int, [vp, vp, i64, vp, C.c_float, vp, vp]),
        "uaii_hip_gemm_swiglu": (C.c_int, [vp, vp, vp, i64, vp, C.c_float, vp, vp]),
        "uaii_hip_attention_prefill": (C.c_int, [vp, vp, vp, i64, C.c_int, C.c_int, C.c_int, i64,
                                                 i64, vp, vp]),
        "uaii_hip_rmsnorm": (C.c_int, [vp, vp, vp, i64, i64, C.c_float, vp]),
        "uaii_hip_softmax": (C.c_int, [vp, vp, i64, vp]),
        "uaii_hip_argmax": (C.c_int, [vp, i64, vp, vp]),
        "uaii_hip_sample_workspace_bytes": (i64, [i64]),
        "uaii_hip_sample": (C.c_int, [vp, i64, C.c_float, C.c_float, C.c_int, C.c_float, vp, i64,
                                      C.c_float, vp, vp, vp]),
        "uaii_sample_uniforms": (C.c_int, [C.c_uint64, i64, f32p]),
        "uaii_hip_rope_table": (C.c_int, [C.c_float, C.c_int, i64, vp]),
        "uaii_hip_rope": (C.c_int, [vp, i64, i64, C.c_int, C.c_int, vp, vp, vp]),
        "uaii_hip_attention_decode": (C.c_int, [vp, vp, vp, C.c_int, i64, C.c_int, C.c_int, C.c_int,
                                                i64, vp, vp]),
        "uaii_hip_attention_decode_noalloc": (C.c_int, [vp, vp, vp, C.c_int, i64, C.c_int, C.c_int,
                                                        C.c_int, i64, vp, vp]),
        "uaii_hip_attention_o": (C.c_int, [vp, vp, vp, C.c_int, i64, C.c_int, C.c_int, C.c_int,
                                           i64, vp, vp, vp, vp]),
        "uaii_hip_gemv_add_atomic": (C.c_int, [vp, vp, vp, vp]),
        "uaii_hip_time_gemv": (C.c_int, [vp, vp, vp, C.c_int, f32p]),
        "uaii_hip_time_gemv_rotate": (C.c_int, [vp, C.c_int, vp, vp, C.c_int, f32p]),
        "uaii_hip_time_gemm": (C.c_int, [vp, vp, i64, vp, C.c_int, f32p]),
        "uaii_hip_time_copy": (C.c_int, [vp, vp, C.c_size_t, C.c_int, f32p]),
        "uaii_hip_time_read": (C.c_int, [vp, C.c_int, C.c_size_t, C.c_int, f32p]),
        "uaii_hip_add": (C.c_int, [vp, vp, vp, i64, vp]),
        "uaii_hip_mul": (C.c_int, [vp, vp, vp, i64, vp]),
        "uaii_hip_silu": (C.c_int, [vp, vp, i64, vp]),
        "uaii_hip_gelu": (C.c_int, [vp, vp, i64, vp]),
        "uaii_hip_embed": (C.c_int, [vp, vp, i64, vp, vp]),
        "uaii_hip_kv_append": (C.c_int, [vp, vp, vp, vp, i64, i64, C.c_int, i64, i64, C.c_int, vp]),
        "uaii_backend_create": (C.c_int, [C.c_char_p, C.c_int, C.POINTER(vp)]),
        "uaii_backend_destroy": (None, [vp]),
        "uaii_backend_initialize": (C.c_int, [vp]),
        "uaii_backend_details": (C.c_char_p, [vp]),
        "uaii_backend_uses_host_fallback": (C.c_int, [vp]),
        "uaii_backend_dispatch": (C.c_int, [vp, C.c_char_p, C.c_char_p, C.POINTER(TensorView),
                                            C.c_size_t, C.POINTER(TensorView), C.c_size_t,
                                            C.POINTER(Attribute), C.c_size_t]),
        "uaii_backend_synchronize": (C.c_int, [vp]),
        "uaii_backend_allocate": (C.c_int, [vp, C.c_size_t, C.POINTER(vp)]),
        "uaii_backend_free": (C.c_int, [vp, vp]),
        "uaii_backend_copy_h2d": (C.c_int, [vp, vp, vp, C.c_size_t]),
        "uaii_backend_copy_d2h": (C.c_int, [vp, vp, vp, C.c_size_t]),
        "uaii_backend_configure_kv_cache": (C.c_int, [vp, i64, i64, i64, i64, C.c_int]),
        "uaii_backend_reset_kv_cache": (C.c_int, [vp]),
        "uaii_backend_commit_kv_step": (C.c_int, [vp]),
        "uaii_backend_kv_past_len": (i64, [vp]),
    }
    for name, (res, args) in sig.items():
        try:
            fn = getattr(L, name)
        except AttributeError:
            # an older build without this entry point: calling it raises
            def missing(*_a, _n=name):
                raise UaiiError(f"{LIB_PATH} does not export {_n}")
            setattr(L, name, missing)
            continue
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def check_hip(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = lib().uaii_hip_error_string(rc).decode()
        raise UaiiError(f"{what}: HIP layer error {rc} ({msg})")


class DeviceBuffer:
    """A device allocation owned from Python (numpy <-> device copies)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = C.c_void_p()
        check_hip(lib().uaii_hip_malloc(C.byref(self.ptr), max(self.nbytes, 4)), "malloc")

    @classmethod
    def from_array(cls, arr):
        import numpy as np
        a = np.ascontiguousarray(arr)
        buf = cls(a.nbytes)
        check_hip(lib().uaii_hip_memcpy_h2d(buf.ptr, a.ctypes.data_as(C.c_void_p), a.nbytes), "h2d")
        return buf

    def to_array(self, dtype, count):
        import numpy as np
        out = np.empty(count, dtype=dtype)
        check_hip(lib().uaii_hip_memcpy_d2h(out.ctypes.data_as(C.c_void_p), self.ptr, out.nbytes), "d2h")
        return out

    def zero(self):
        check_hip(lib().uaii_hip_memset(self.ptr, 0, self.nbytes), "memset")

    def free(self):
        if self.ptr:
            lib().uaii_hip_free(self.ptr)
            self.ptr = C.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class DeviceWeight:
    """GGUF rows uploaded to the device split layout (uaii_hip_weight_create)."""

    def __init__(self, gguf_type: int, packed, rows: int, cols: int):
        import numpy as np
        p = np.ascontiguousarray(packed, dtype=np.uint8)
        if p.nbytes != rows * row_bytes(gguf_type, cols):
            raise UaiiError("packed size does not match rows x cols")
        self.type, self.rows, self.cols = gguf_type, rows, cols
        self.h = C.c_void_p()
        check_hip(lib().uaii_hip_weight_create(gguf_type, p.ctypes.data_as(C.c_void_p), rows, cols,
                                               C.byref(self.h)), "weight_create")

    def free(self):
        if self.h:
            lib().uaii_hip_weight_destroy(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Session:
    """uaii_session_* through the C ABI."""

    def __init__(self, path: str, *, kv_f16: bool = False, max_context: int = 0,
                 profile: bool = False, backend: str = "rocm", memory_reuse: bool = False,
                 keep_quantized: bool = True, budget_bytes: int = 0, weight_init: int = 0,
                 allow_missing_weights: bool = False):
        """memory_reuse / keep_quantized select the reference's weight path: the
        defaults here (memory_reuse off, quantized weights kept) are its packed
        Path B, the quant_gemm path; memory_reuse=True (the C ABI's default, as in
        the reference) or keep_quantized=False give the values of its Path A (the
        f32 weight load, Q4_0 nibbles in pairwise order)."""
        L = lib()
        opts = SessionOptions()
        L.uaii_session_options_init(C.byref(opts))
        self._backend = backend.encode()
        opts.backend = self._backend
        opts.enable_memory_reuse = 1 if memory_reuse else 0
        opts.keep_quantized_weights = 1 if keep_quantized else 0
        opts.budget_bytes = budget_bytes
        opts.weight_init = weight_init  # 0 none, 1 zeros, 2 ones, 3 sequence (uaii_weight_init)
        opts.allow_missing_weights = 1 if allow_missing_weights else 0
        opts.compute_dtype = 1 if kv_f16 else 0
        opts.max_context = max_context
        opts.enable_profiler = 1 if profile else 0
        self.h = C.c_void_p()
        rc = L.uaii_session_create(str(path).encode(), C.byref(opts), C.byref(self.h))
        if rc != 0:
            raise UaiiError(f"uaii_session_create: {L.uaii_status_name(rc).decode()}: "
                            f"{L.uaii_last_error().decode()}")

    def generate(self, prompt, max_new: int):
        import numpy as np
        L = lib()
        p = np.ascontiguousarray(prompt, dtype=np.int64)
        cap = len(p) + max(max_new, 0)
        out = np.zeros(max(cap, 1), dtype=np.int64)
        n = C.c_size_t()
        rc = L.uaii_session_generate(self.h, p.ctypes.data_as(C.POINTER(C.c_int64)), len(p), max_new,
                                     out.ctypes.data_as(C.POINTER(C.c_int64)), cap, C.byref(n))
        if rc != 0:
            raise UaiiError(f"uaii_session_generate: {L.uaii_status_name(rc).decode()}: "
                            f"{L.uaii_last_error().decode()}")
        return out[: n.value]

    def generate_sampled(self, prompt, max_new: int, params: "SampleParams"):
        import numpy as np
        L = lib()
        p = np.ascontiguousarray(prompt, dtype=np.int64)
        cap = len(p) + max(max_new, 0)
        out = np.zeros(max(cap, 1), dtype=np.int64)
        n = C.c_size_t()
        rc = L.uaii_session_generate_sampled(self.h, p.ctypes.data_as(C.POINTER(C.c_int64)), len(p),
                                             max_new, C.byref(params),
                                             out.ctypes.data_as(C.POINTER(C.c_int64)), cap, C.byref(n))
        if rc != 0:
            raise UaiiError(f"uaii_session_generate_sampled: {L.uaii_status_name(rc).decode()}: "
                            f"{L.uaii_last_error().decode()}")
        return out[: n.value]

    def get(self, name: str):
        import numpy as np
        L = lib()
        n = C.c_size_t()
        rc = L.uaii_session_get_f32(self.h, name.encode(), None, 0, C.byref(n))
        if rc != 0:
            raise UaiiError(f"get_f32({name}): {L.uaii_last_error().decode()}")
        out = np.zeros(n.value, dtype=np.float32)
        rc = L.uaii_session_get_f32(self.h, name.encode(), out.ctypes.data_as(C.POINTER(C.c_float)),
                                    n.value, C.byref(n))
        if rc != 0:
            raise UaiiError(f"get_f32({name}): {L.uaii_last_error().decode()}")
        return out

    def _ok(self, rc, what):
        if rc != 0:
            L = lib()
            raise UaiiError(f"{what}: {L.uaii_status_name(rc).decode()}: {L.uaii_last_error().decode()}")

    def begin(self, prompt, capacity: int = 0):
        import numpy as np
        p = np.ascontiguousarray(prompt, dtype=np.int64)
        self._ok(lib().uaii_session_begin(self.h, p.ctypes.data_as(C.POINTER(C.c_int64)), len(p),
                                          capacity), "begin")

    def step_async(self, want_logits: bool = True):
        self._ok(lib().uaii_session_step_async(self.h, int(want_logits)), "step_async")

    def prefill(self, n: int):
        """Next n prompt tokens through the matrix-core path (synchronises)."""
        self._ok(lib().uaii_session_prefill(self.h, int(n)), "prefill")

    def prefill_supported(self) -> bool:
        v = C.c_int()
        self._ok(lib().uaii_session_prefill_supported(self.h, C.byref(v)), "prefill_supported")
        return bool(v.value)

    def sync(self):
        self._ok(lib().uaii_session_sync(self.h), "sync")

    def position(self) -> int:
        v = C.c_int64()
        self._ok(lib().uaii_session_position(self.h, C.byref(v)), "position")
        return v.value

    def read_ids(self, n: int):
        import numpy as np
        out = np.zeros(max(n, 1), dtype=np.int64)
        self._ok(lib().uaii_session_read_ids(self.h, out.ctypes.data_as(C.POINTER(C.c_int64)), n),
                 "read_ids")
        return out[:n]

    def seek(self, pos: int):
        self._ok(lib().uaii_session_seek(self.h, pos), "seek")

    def set_device_sampler(self, on: bool):
        """generate_sampled's non-greedy draws on the device (True) or the host."""
        self._ok(lib().uaii_session_set_device_sampler(self.h, int(on)), "set_device_sampler")

    def set_profiling(self, on: bool):
        self._ok(lib().uaii_session_set_profiling(self.h, int(on)), "set_profiling")

    def last_margin(self):
        b, s2 = C.c_float(), C.c_float()
        self._ok(lib().uaii_session_last_margin(self.h, C.byref(b), C.byref(s2)), "last_margin")
        return b.value, s2.value

    def profile_summary(self) -> str:
        buf = C.create_string_buffer(1 << 16)
        rc = lib().uaii_session_profile_summary(self.h, buf, len(buf))
        if rc != 0:
            raise UaiiError("profile_summary failed")
        return buf.value.decode()

    def close(self):
        if self.h:
            lib().uaii_session_destroy(self.h)
            self.h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Backend:
    """The ROCm IBackend through uaii_backend.h: dispatch of the reference's
    operators (libs/uaii-kernels/src/dispatch.cpp:67-272) on the device.

    Tensors are numpy arrays (host memory, staged by the backend, as the
    reference's Session hands over its host buffers) or DeviceBuffer objects
    with an explicit shape (device memory, used in place)."""

    def __init__(self, device: int = 0, initialize: bool = True):
        L = lib()
        self.h = C.c_void_p()
        self._ok(L.uaii_backend_create(b"rocm", device, C.byref(self.h)), "uaii_backend_create")
        if initialize:
            self._ok(L.uaii_backend_initialize(self.h), "uaii_backend_initialize")

    @staticmethod
    def _ok(rc, what):
        if rc != 0:
            L = lib()
            raise UaiiError(f"{what}: {L.uaii_status_name(rc).decode()}: {L.uaii_last_error().decode()}")

    @staticmethod
    def view(t, shape=None, quant=None):
        """A TensorView of a numpy array or of (DeviceBuffer, shape, dtype);
        quant = (gguf_type, rows, cols) marks packed GGUF rows (dtype Unknown)."""
        import numpy as np
        keep = []
        if isinstance(t, tuple):  # (DeviceBuffer, shape, numpy dtype)
            buf, shp, dt = t
            data, nbytes = buf.ptr.value, buf.nbytes
            dtype = DTYPE_F32 if np.dtype(dt) == np.float32 else DTYPE_F16 if np.dtype(dt) == np.float16 else 0
        else:
            a = np.ascontiguousarray(t)
            keep.append(a)
            shp = a.shape if shape is None else shape
            data, nbytes = a.ctypes.data, a.nbytes
            dtype = DTYPE_F32 if a.dtype == np.float32 else DTYPE_F16 if a.dtype == np.float16 else 0
        shape_arr = (C.c_int64 * max(len(shp), 1))(*shp)
        keep.append(shape_arr)
        v = TensorView(dtype, C.cast(shape_arr, C.POINTER(C.c_int64)), len(shp), data, nbytes, 0, 0, 0)
        if quant is not None:
            gt, rows, cols = quant
            v.dtype = 0
            v.quant_format, v.quant_rows, v.quant_cols = QUANT_FORMAT[gt], rows, cols
        return v, keep

    def dispatch(self, op: str, inputs, outputs, attrs=None):
        """inputs / outputs: lists of (TensorView, keep) pairs from view();
        attrs: {key: value} with bool / int / float / str values."""
        ins = (TensorView * max(len(inputs), 1))(*[v for v, _ in inputs])
        outs = (TensorView * max(len(outputs), 1))(*[v for v, _ in outputs])
        al = []
        for k, val in (attrs or {}).items():
            a = Attribute(k.encode(), 0, 0, 0.0, None)
            if isinstance(val, bool):
                a.type, a.i = 3, int(val)
            elif isinstance(val, int):
                a.type, a.i = 1, val
            elif isinstance(val, float):
                a.type, a.f = 2, val
            else:
                a.type, a.s = 0, str(val).encode()
            al.append(a)
        arr = (Attribute * max(len(al), 1))(*al)
        self._ok(lib().uaii_backend_dispatch(self.h, op.encode(), b"1", ins, len(inputs), outs,
                                             len(outputs), arr, len(al)), f"dispatch {op}")

    def configure_kv_cache(self, n_layers, max_seq, kv_dim, n_kv_heads, f16=False):
        self._ok(lib().uaii_backend_configure_kv_cache(self.h, n_layers, max_seq, kv_dim, n_kv_heads,
                                                       int(f16)), "configure_kv_cache")

    def reset_kv_cache(self):
        self._ok(lib().uaii_backend_reset_kv_cache(self.h), "reset_kv_cache")

    def commit_kv_step(self):
        self._ok(lib().uaii_backend_commit_kv_step(self.h), "commit_kv_step")

    def past_len(self) -> int:
        return lib().uaii_backend_kv_past_len(self.h)

    def synchronize(self):
        self._ok(lib().uaii_backend_synchronize(self.h), "synchronize")

    def details(self) -> str:
        return lib().uaii_backend_details(self.h).decode()

    def close(self):
        if self.h:
            lib().uaii_backend_destroy(self.h)
            self.h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
