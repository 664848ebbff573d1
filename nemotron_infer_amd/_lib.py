"""ctypes binding of the C ABI in include/nmi_fp8_linear.h (libnmi.so).

There is no CPU fallback: if the library is missing, ``lib()`` raises.  Build it with
``python -m nemotron_infer_amd.build``.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libnmi.so")

NMI_OK = 0
NMI_ERR_INVALID_ARG = -1
NMI_ERR_ALIGNMENT = -2
NMI_ERR_UNSUPPORTED = -3
NMI_ERR_WORKSPACE = -4
NMI_ERR_ALLOC = -5
NMI_ERR_ASYNC = -6            # an earlier launch's asynchronous error (stream-K wait gave up)
NMI_WS_ERROR_OFFSET = 65532   # byte offset of the stream-K error word in a linear workspace

# Every symbol the header declares, with its ctypes signature.
_vp, _i, _i64, _sz, _f = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_float
SIGNATURES = {
    "nmi_abi_version": ([], _i),
    "nmi_last_error": ([], ctypes.c_char_p),
    "nmi_gemv_fp8": ([_vp, _vp, _vp, _vp, _i, _i, _vp], _i),
    "nmi_linear_fp8_w8a16": ([_vp, _i64, _vp, _i64, _vp, _vp, _i64, _i, _i, _i, _vp], _i),
    "nmi_linear_fp8_w8a16_ws": ([_vp, _i64, _vp, _i64, _vp, _vp, _i64, _i, _i, _i, _vp, _sz, _vp], _i),
    "nmi_linear_fp8_w8a16_grouped": ([_vp, _i64, _i, _i, _vp, _i, _vp, _sz, _vp], _i),
    "nmi_linear_workspace_bytes": ([_i, _i64, _i], _sz),
    "nmi_gemm_fp8_w8a16": ([_vp, _i64, _vp, _i64, _vp, _vp, _i64, _i, _i, _i, _vp, _sz, _vp], _i),
    "nmi_fp8_e4m3_decode": ([_vp, _vp, _vp, _vp, _f, _i, _vp], _i),
    "nmi_rmsnorm_bf16": ([_vp, _vp, _vp, _i, _i, _f, _vp], _i),
    "nmi_mlp_workspace_bytes": ([_i, _i, _i], _sz),
    "nmi_mlp_forward_fp8": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _f, _vp, _sz, _vp], _i),
    "nmi_mlp_noalloc_scratch_bytes": ([], _sz),
    "nmi_sdpa_decode_workspace_bytes": ([_i, _i, _i], _sz),
    "nmi_sdpa_decode_bf16": ([_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _sz, _vp], _i),
    "nmi_attn_decode_workspace_bytes": ([_i, _i, _i, _i], _sz),
    "nmi_mamba_decode_workspace_bytes": ([_i] * 6, _sz),
    "nmi_sdpa_prefill_workspace_bytes": ([_i, _i], _sz),
    "nmi_mamba_forward_workspace_bytes": ([_i] * 7, _sz),
    "nmi_mamba_forward_fp8": ([_vp] * 13 + [_i, _i, _vp, _vp] + [_i] * 6 + [_f, _vp, _sz, _vp], _i),
    "nmi_sdpa_prefill_bf16": ([_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i, _i, _i, _vp, _sz, _vp], _i),
    "nmi_attn_forward_workspace_bytes": ([_i] * 4, _sz),
    "nmi_attn_forward_fp8": ([_vp] * 11 + [_i, _vp, _vp, _i, _i, _i, _i, _f, _vp, _sz, _vp], _i),
    "nmi_mamba_mixer_decode": ([_vp, _i64] + [_vp] * 10 + [_i] * 6 + [_f, _vp], _i),
    "nmi_mamba_decode_fp8": ([_vp] * 15 + [_i] * 7 + [_f, _vp, _sz, _vp], _i),
    "nmi_attn_decode_fp8": ([_vp] * 12 + [_i, _i, _vp, _i, _i, _i, _f, _vp, _sz, _vp], _i),
    "nmi_mlp_forward_fp8_noalloc": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _f, _vp], _i),
    "nmi_tuning_set": ([ctypes.c_char_p, _i], _i),
    "nmi_alloc": ([_sz, ctypes.POINTER(_vp)], _i),
    "nmi_alloc_rewind": ([], _i),
    "nmi_alloc_reset": ([], _i),
    "nmi_alloc_stats": ([ctypes.POINTER(_sz), ctypes.POINTER(_sz)], _i),
    "nmi_sync": ([], _i),
    "nmi_async_status": ([], _i),
    "nmi_linear_fp8_w8a16_batch": ([_vp, _i, _i, _vp], _i),
    "nmi_gemv_chain_create": ([_vp, _i, ctypes.POINTER(_vp)], _i),
    "nmi_gemv_chain_workspace_bytes": ([_i], _sz),
    "nmi_gemv_chain_launch": ([_vp, _vp, _sz, _vp], _i),
    "nmi_gemv_chain_destroy": ([_vp], _i),
}

MAX_GROUPS = 4


class LinearGroup(ctypes.Structure):
    """nmi_linear_group of include/nmi_fp8_linear.h."""
    _fields_ = [("w_e4m3", _vp), ("ldw", _i64), ("w_scale", _vp), ("y_bf16", _vp), ("ldy", _i64),
                ("N", _i)]


MAX_BATCH = 8


class LinearJob(ctypes.Structure):
    """nmi_linear_job of include/nmi_fp8_linear.h."""
    _fields_ = [("x_bf16", _vp), ("ldx", _i64), ("K", _i), ("w", LinearGroup)]


class GemvPhase(ctypes.Structure):
    """nmi_gemv_phase of include/nmi_fp8_linear.h."""
    _fields_ = [("x_bf16", _vp), ("K", _i), ("ngroups", _i), ("wait_prev", _i),
                ("groups", LinearGroup * MAX_GROUPS)]


_lib = None


class NmiError(RuntimeError):
    def __init__(self, code: int, where: str, msg: str):
        super().__init__(f"{where} failed with status {code}: {msg}")
        self.code = code


def lib():
    """Load libnmi.so once; raise if it is missing (no fallback path exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `python -m nemotron_infer_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
        # NMI_TUNING="knob=value,knob=value": tuning knobs applied at load (for sweeps and
        # profiles of one variant from an unchanged command line)
        for item in filter(None, os.environ.get("NMI_TUNING", "").split(",")):
            knob, _, value = item.partition("=")
            tuning_set(knob.strip(), int(value))
    return _lib


def check(rc: int, where: str) -> None:
    if rc != NMI_OK:
        raise NmiError(rc, where, lib().nmi_last_error().decode())


def tuning_set(knob: str, value: int) -> None:
    check(lib().nmi_tuning_set(knob.encode(), int(value)), "nmi_tuning_set")
