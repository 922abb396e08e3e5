"""ctypes binding of librotor_hip.so (the C ABI in include/rotor_hip.h).

Follows the reference's ctypes pattern for its native core
(src/rotor/bitnet_fast.py:15-48 library search, :86-102 argtypes/restype), with two
differences: every call's status is checked and turned into ``RuntimeError`` with the
library's own message, and a missing library is an error, never a silent fallback.

Library search order: ``$ROTOR_HIP_LIB`` if set, else ``rotor/lib/librotor_hip.so``
next to this file (built in-tree by ``rotor-rag_amd/csrc/build.py``).
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "librotor_hip.so"
ABI_VERSION = 108  # rt_version() of the library this table binds

class RtSrc(ctypes.Structure):
    """rt_src of include/rotor_hip.h"""
    _fields_ = [("mode", ctypes.c_int), ("x", ctypes.c_void_p), ("aux", ctypes.c_void_p), ("aux2", ctypes.c_void_p),
                ("eps", ctypes.c_float), ("attn_head_dim", ctypes.c_int), ("attn_max_len", ctypes.c_int)]


SRC_QUANT, SRC_RMSNORM, SRC_RELU2MUL, SRC_RELU2MUL_NORM, SRC_ATTN_NORM, SRC_RMSNORM_SSQ = 0, 2, 3, 4, 5, 6
LAUNCH_GEMV, LAUNCH_GEMV_FUSED, LAUNCH_SPLITK, LAUNCH_TILES = 0, 1, 2, 3

# name -> (restype, argtypes); every entry point of include/rotor_hip.h
_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
SIGNATURES = {
    "rt_last_error": (ctypes.c_char_p, []),
    "rt_version": (_I, []),
    "rt_device_count": (_I, [ctypes.POINTER(_I)]),
    "rt_ctx_create": (_I, [_I, ctypes.POINTER(_P)]),
    "rt_ctx_destroy": (_I, [_P]),
    "rt_ctx_set_stream": (_I, [_P, _P]),
    "rt_sync": (_I, [_P]),
    "rt_weights_upload": (_I, [_P, _P, _I, _I, _F, ctypes.POINTER(_P)]),
    "rt_weights_upload_device": (_I, [_P, _P, _I, _I, _F, ctypes.POINTER(_P)]),
    "rt_weights_download": (_I, [_P, _P, _P]),
    "rt_weights_info": (_I, [_P, ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_F)]),
    "rt_weights_free": (_I, [_P]),
    "rt_quantize_rows": (_I, [_P, _P, _I, _I, _P, _P]),
    "rt_linear_i32": (_I, [_P, _P, _P, _I, _P]),
    "rt_linear_f32": (_I, [_P, _P, _P, _I, _P]),
    "rt_linear_f32_rowscale": (_I, [_P, _P, _P, _I, _P, _P]),
    "rt_linear_f32_noalloc": (_I, [_P, _P, _P, _I, _P]),
    "rt_plan_create": (_I, [_P, _I, ctypes.POINTER(_P), ctypes.POINTER(_P), _I, ctypes.POINTER(_P),
                            ctypes.POINTER(_P)]),
    "rt_plan_run": (_I, [_P, _P]),
    "rt_plan_quantize": (_I, [_P, _P]),
    "rt_plan_gemv": (_I, [_P, _P]),
    "rt_plan_free": (_I, [_P]),
    "rt_plan_describe": (_I, [_P, ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "rt_act_create": (_I, [_P, _I, _I, ctypes.POINTER(_P)]),
    "rt_act_free": (_I, [_P]),
    "rt_act_quantize": (_I, [_P, _P, _I, _P]),
    "rt_act_rmsnorm_quantize": (_I, [_P, _P, _P, _F, _I, _P, _P]),
    "rt_act_relu2_mul_quantize": (_I, [_P, _P, _P, _I, _P, _P]),
    "rt_act_relu2_mul_norm_quantize": (_I, [_P, _P, _P, _P, _F, _I, _P, _P]),
    "rt_act_export": (_I, [_P, _P, _P, _P]),
    "rt_linear_act_f32": (_I, [_P, _P, _P, _P, _P]),
    "rt_plan_create_act": (_I, [_P, _I, ctypes.POINTER(_P), ctypes.POINTER(_P), _I, ctypes.POINTER(_P),
                                ctypes.POINTER(_P)]),
    "rt_plan_create_fused": (_I, [_P, _I, ctypes.POINTER(_P), ctypes.POINTER(RtSrc), ctypes.POINTER(_P),
                                  ctypes.POINTER(_P), ctypes.POINTER(_P)]),
    "rt_plan_create_gate_up": (_I, [_P, _P, _F, _F, ctypes.POINTER(RtSrc), _P, _P, _P, _P, ctypes.POINTER(_P)]),
    "rt_plan_create_act_gate_up": (_I, [_P, _P, _F, _F, _P, _I, _P, ctypes.POINTER(_P)]),
    "rt_plan_attach_attention": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P, _P, ctypes.c_size_t]),
    "rt_plan_attention_combine": (_I, [_P, _P, _P]),
    "rt_plan_attention_timeouts": (_I, [_P, _P]),
    "rt_plan_set_output_ssq": (_I, [_P, _P]),
    "rt_embed": (_I, [_P, _P, _I, _I, _P, _I, _P]),
    "rt_rope_kv_append": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "rt_attention": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "rt_attention_decode_workspace": (ctypes.c_size_t, [_I, _I, _I]),
    "rt_attention_decode": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P, ctypes.c_size_t]),
    "rt_attention_decode_partials": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P, _P, ctypes.c_size_t]),
    "rt_attention_decode_combine": (_I, [_P, _P, ctypes.c_size_t, _I, _I, _I, _P]),
    "rt_rope_attention_decode": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P, ctypes.c_size_t, _P]),
    "rt_lm_head_argmax": (_I, [_P, _P, _P, _P, _F, _I, _I, _P, _P, _P, _P, _I, _P, _P, _I, _I, _P]),
}

_lib = None


def lib_path() -> Path:
    env = os.environ.get("ROTOR_HIP_LIB")
    return Path(env) if env else LIB_PATH


def load():
    """Load (once) and return the library; raises RuntimeError when it cannot be loaded."""
    global _lib
    if _lib is not None:
        return _lib
    path = lib_path()
    if not path.exists():
        raise RuntimeError(f"librotor_hip.so not found at {path} (build it with rotor-rag_amd/csrc/build.py)")
    try:
        lib = ctypes.CDLL(str(path))
    except OSError as e:
        raise RuntimeError(f"cannot load {path}: {e}") from e
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError here = ABI mismatch, let it surface
        fn.restype = res
        fn.argtypes = args
    if lib.rt_version() != ABI_VERSION:
        raise RuntimeError(f"{path} has ABI version {lib.rt_version()}, this binding expects {ABI_VERSION} "
                           "(rebuild the library)")
    _lib = lib
    return lib


def last_error() -> str:
    return load().rt_last_error().decode(errors="replace")


def check(rc: int, what: str = "") -> None:
    """Raise RuntimeError with the library's message for a non-zero status."""
    if rc != 0:
        raise RuntimeError(f"{what or 'librotor_hip'} failed (status {rc}): {last_error()}")
