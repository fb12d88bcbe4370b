"""ctypes declarations for include/qff/qff.h (libqff_hip.so)."""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
LIB_PATH = os.path.join(PKG, "lib", "libqff_hip.so")

F32, BF16, F16 = 0, 1, 2

STATUS = {0: "ok", -1: "invalid argument", -2: "unsupported shape", -3: "HIP runtime error",
          -4: "request exceeds the context workspace", -5: "out of device memory"}


class QffError(RuntimeError):
    def __init__(self, fn: str, status: int):
        super().__init__(f"{fn} failed: {STATUS.get(status, status)} ({status})")
        self.status = status


_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float


class DeltaNetParams(ctypes.Structure):
    _fields_ = [("a_log", _vp), ("dt_bias", _vp), ("conv_w", _vp), ("norm_w", _vp), ("eps", _f)]


class GqaParams(ctypes.Structure):
    _fields_ = [("q_norm_w", _vp), ("k_norm_w", _vp), ("rope_theta", _f), ("rotary_dim", _i),
                ("scale", _f), ("eps", _f), ("kv_f16", _i)]


class Q4Part(ctypes.Structure):
    _fields_ = [("w", _vp), ("scales", _vp), ("biases", _vp), ("rows", _i), ("y", _vp), ("y_dtype", _i),
                ("residual", _vp)]


Q4_MAX_PARTS = 8


class CtxCfg(ctypes.Structure):
    _fields_ = [("max_batch", _i), ("max_ctx", _i), ("max_prefill_tokens", _i)]


# Every symbol include/qff/qff.h declares, with its argument types.
SIGNATURES = {
    "qff_ctx_create": [ctypes.POINTER(_vp), _i, ctypes.POINTER(CtxCfg)],
    "qff_ctx_destroy": [_vp],
    "qff_workspace_size": [ctypes.POINTER(CtxCfg), ctypes.POINTER(ctypes.c_size_t)],
    "qff_status_string": [_i],
    "qff_version": [],
    "qff_q4_dequant": [_vp, _vp, _vp, _vp, _vp, _i, _vp, _i, _i],
    "qff_q4_matmul": [_vp, _vp, _vp, _vp, _vp, _i, _vp, _i, _vp, _i, _i, _i, _i],
    "qff_q4_matmul_parts": [_vp, _vp, ctypes.POINTER(Q4Part), _i, _i, _vp, _i, _i, _i],
    "qff_q4_norm_matmul_parts": [_vp, _vp, ctypes.POINTER(Q4Part), _i, _i, _vp, _i, _vp, _i, _f, _i, _i],
    "qff_q8_dequant": [_vp, _vp, _vp, _vp, _vp, _i, _vp, _i, _i],
    "qff_router_top8": [_vp, _vp, _vp, _vp, _vp, _i, _vp, _i, _vp, _vp, _vp, _i, _i, _i],
    "qff_deltanet_decode": [_vp, _vp, ctypes.POINTER(DeltaNetParams), _vp, _vp, _i, _vp, _vp, _vp,
                            _vp, _vp, _i, _i],
    "qff_deltanet_prefill": [_vp, _vp, ctypes.POINTER(DeltaNetParams), _vp, _vp, _i, _vp, _vp,
                             _vp, _vp, _vp, _i, _i, _i],
    "qff_gqa_decode": [_vp, _vp, ctypes.POINTER(GqaParams), _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp,
                       _i, _i, _i],
    "qff_gqa_decode_static": [_vp, ctypes.POINTER(GqaParams), _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _i, _i,
                              _i],
    "qff_gqa_prefill": [_vp, _vp, ctypes.POINTER(GqaParams), _vp, _vp, _vp, _i, _vp, _vp, _i, _vp,
                        _i, _i, _i],
    "qff_kv_append": [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i],
    "qff_attention_gate": [_vp, _vp, _vp, _vp, _vp, _i],
    "qff_profile_enable": [_vp, _i],
    "qff_profile_read": [_vp, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_f), _i,
                         ctypes.POINTER(_i)],
}

_lib = None


def lib():
    """Load the in-tree HIP library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise QffError("load " + LIB_PATH, -3)
        L = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = ctypes.c_char_p if name == "qff_status_string" else _i
        _lib = L
    return _lib


def check(fn: str, status: int):
    if status != 0:
        raise QffError(fn, status)
