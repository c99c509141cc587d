"""Seeded synthetic GGUF decoders (ctypes over libuaii_synth.so).

Presets follow the configurations the benchmark is quoted on (Llama-style
`blk.*` decoders written with the reference's tensor and key names); the value
generator and quantizers are specified in csrc/synth/uaii_synth.h.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field, asdict

from . import SYNTH_PATH, UaiiError, F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K


class _Cfg(C.Structure):
    _fields_ = [
        ("n_layers", C.c_int64), ("dim", C.c_int64), ("n_heads", C.c_int64),
        ("n_kv_heads", C.c_int64), ("head_dim", C.c_int64), ("ffn", C.c_int64),
        ("vocab", C.c_int64), ("ctx_len", C.c_int64), ("rope_theta", C.c_float),
        ("rms_eps", C.c_float), ("tied", C.c_int), ("n_experts", C.c_int), ("top_k", C.c_int),
        ("type_default", C.c_int), ("type_embd", C.c_int), ("type_output", C.c_int),
        ("type_attn_v", C.c_int), ("type_ffn_down", C.c_int), ("seed", C.c_uint64),
        ("std", C.c_float), ("router_std", C.c_float), ("arch", C.c_char_p),
        ("gelu", C.c_int), ("qkv_bias", C.c_int), ("shared_ffn", C.c_int64),
    ]


@dataclass
class ModelConfig:
    n_layers: int
    dim: int
    n_heads: int
    n_kv_heads: int
    ffn: int
    vocab: int
    ctx_len: int
    head_dim: int = 0
    rope_theta: float = 10000.0
    rms_eps: float = 1e-5
    tied: bool = False
    n_experts: int = 0
    top_k: int = 2
    type_default: int = Q8_0
    type_embd: int = -1
    type_output: int = -1
    type_attn_v: int = -1
    type_ffn_down: int = -1
    seed: int = 1
    std: float = 0.02
    router_std: float = 0.0
    arch: str = "llama"
    gelu: bool = False
    qkv_bias: bool = False
    shared_ffn: int = 0

    def key(self) -> str:
        d = asdict(self)
        # the three newest fields join the key only when set, so the files of
        # configs without them keep their cache names
        for k in ("gelu", "qkv_bias", "shared_ffn"):
            if not d[k]:
                d.pop(k)
        return "_".join(f"{k}{v}" for k, v in d.items())


# Configurations of the benchmark; prompt/decode lengths with them.
PRESETS = {
    # 4 layers, d512, 8x64 heads, SwiGLU 1408, vocab 32000, Q8_0, theta 1e4
    "tiny": ModelConfig(n_layers=4, dim=512, n_heads=8, n_kv_heads=8, ffn=1408, vocab=32000,
                        ctx_len=2048, rope_theta=10000.0, type_default=Q8_0, seed=11),
    # Llama-3.2-1B shape: Q4_K with Q6_K attn_v / ffn_down, tied embeddings
    "1b": ModelConfig(n_layers=16, dim=2048, n_heads=32, n_kv_heads=8, ffn=8192, vocab=128256,
                      ctx_len=2048, rope_theta=500000.0, tied=True, type_default=Q4_K,
                      type_attn_v=Q6_K, type_ffn_down=Q6_K, seed=12),
    # Llama-3-8B shape, Q4_0 (headline) and Q8_0
    "8b": ModelConfig(n_layers=32, dim=4096, n_heads=32, n_kv_heads=8, ffn=14336, vocab=128256,
                      ctx_len=4096, rope_theta=500000.0, type_default=Q4_0, seed=13),
    "8b_q8": ModelConfig(n_layers=32, dim=4096, n_heads=32, n_kv_heads=8, ffn=14336, vocab=128256,
                         ctx_len=4096, rope_theta=500000.0, type_default=Q8_0, seed=14),
    # Mixtral-8x7B shape: 8 experts top-2, Q4_K, router logits ~ N(0,1)
    "mx": ModelConfig(n_layers=32, dim=4096, n_heads=32, n_kv_heads=8, ffn=14336, vocab=32000,
                      ctx_len=4096, rope_theta=1000000.0, n_experts=8, top_k=2,
                      type_default=Q4_K, seed=15, router_std=1.0 / 64.0),
}

RUN_LENGTHS = {"tiny": (32, 64), "1b": (512, 256), "8b": (3840, 256), "8b_q8": (3840, 256),
               "mx": (1024, 256)}

_slib = None


def _synth():
    global _slib
    if _slib is None:
        if not SYNTH_PATH.exists():
            raise UaiiError(f"{SYNTH_PATH} is missing: run __graft_entry__.build() first")
        L = C.CDLL(str(SYNTH_PATH))
        L.uaii_synth_write_gguf.restype = C.c_int
        L.uaii_synth_write_gguf.argtypes = [C.c_char_p, C.POINTER(_Cfg), C.c_int]
        L.uaii_synth_last_error.restype = C.c_char_p
        L.uaii_synth_normals.restype = None
        L.uaii_synth_normals.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, C.c_int64, C.c_float,
                                         C.POINTER(C.c_float)]
        L.uaii_synth_quantize_row.restype = C.c_int64
        L.uaii_synth_quantize_row.argtypes = [C.c_int, C.POINTER(C.c_float), C.c_int64, C.c_void_p]
        L.uaii_synth_f32_to_f16.restype = C.c_uint16
        L.uaii_synth_f32_to_f16.argtypes = [C.c_float]
        _slib = L
    return _slib


def write_model(path: str, cfg: ModelConfig, nthreads: int = 0) -> str:
    c = _Cfg()
    for name, _ in _Cfg._fields_:
        v = getattr(cfg, name)
        if name == "arch":
            v = v.encode()
        elif name in ("tied", "gelu", "qkv_bias"):
            v = int(v)
        setattr(c, name, v)
    rc = _synth().uaii_synth_write_gguf(str(path).encode(), C.byref(c), nthreads)
    if rc != 0:
        raise UaiiError(f"synth write failed: {_synth().uaii_synth_last_error().decode()}")
    return str(path)


def cached_model(cfg: ModelConfig, directory: str | None = None, nthreads: int = 0) -> str:
    """Write (once) and return the path of the GGUF for `cfg`."""
    import hashlib
    d = directory or os.environ.get("UAII_MODEL_CACHE", "/tmp/uaii_models")
    os.makedirs(d, exist_ok=True)
    h = hashlib.sha1(cfg.key().encode()).hexdigest()[:16]
    path = os.path.join(d, f"synth_{h}.gguf")
    if not os.path.exists(path):
        tmp = path + f".tmp{os.getpid()}"
        write_model(tmp, cfg, nthreads)
        os.replace(tmp, path)
    return path


def normals(seed: int, tensor: int, i0: int, n: int, std: float):
    import numpy as np
    out = np.empty(n, dtype=np.float32)
    _synth().uaii_synth_normals(seed, tensor, i0, n, std, out.ctypes.data_as(C.POINTER(C.c_float)))
    return out


def quantize(gguf_type: int, x) -> "np.ndarray":
    import numpy as np
    from . import BLOCK
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    be, bb = BLOCK[gguf_type]
    out = np.zeros(x.size // be * bb, dtype=np.uint8)
    n = _synth().uaii_synth_quantize_row(gguf_type, x.ctypes.data_as(C.POINTER(C.c_float)), x.size,
                                         out.ctypes.data_as(C.c_void_p))
    if n < 0:
        raise UaiiError("quantize failed (size not a block multiple?)")
    return out


def f32_to_f16_bits(v: float) -> int:
    return int(_synth().uaii_synth_f32_to_f16(v))
