"""torch-tensor front end of the C ABI: passes data_ptr()s and the current HIP stream.

    y = linear_fp8_w8a16(x_bf16, w_e4m3, w_scale)           # y = bf16((x . W^T) * s)

``x`` is bf16 [M, K] (or [K]), ``w`` is [N, K] in ``torch.float8_e4m3fn`` or ``torch.uint8``
(raw e4m3 codes), ``w_scale`` float32 [N]; all on the same GPU.  Calls go through
include/nmi_fp8_linear.h; there is no torch or CPU fallback.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _check_w(w: torch.Tensor) -> torch.Tensor:
    if w.dtype == torch.float8_e4m3fn:
        return w.view(torch.uint8)
    if w.dtype != torch.uint8:
        raise TypeError(f"weights must be float8_e4m3fn or uint8 codes, got {w.dtype}")
    return w


def linear_fp8_w8a16(x: torch.Tensor, w: torch.Tensor, w_scale: torch.Tensor,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """y[M, N] = bf16_rne((x[M, K] . e4m3(W[N, K])^T) * w_scale[N]) on the GPU."""
    w = _check_w(w)
    squeeze = x.dim() == 1
    x2 = x.unsqueeze(0) if squeeze else x
    if x2.dtype != torch.bfloat16 or w_scale.dtype != torch.float32:
        raise TypeError("x must be bfloat16 and w_scale float32")
    if x2.stride(-1) != 1 or w.stride(-1) != 1 or not w_scale.is_contiguous():
        raise ValueError("x, W rows and w_scale must be contiguous in the last dimension")
    M, K = x2.shape
    N = w.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    y2 = out.view(M, N) if squeeze and out.dim() == 1 else out
    rc = _lib.lib().nmi_linear_fp8_w8a16(
        x2.data_ptr(), x2.stride(0), w.data_ptr(), w.stride(0), w_scale.data_ptr(),
        y2.data_ptr(), y2.stride(0), M, N, K, _stream())
    _lib.check(rc, "nmi_linear_fp8_w8a16")
    return out[0] if squeeze and out.dim() == 2 else out


def gemv_fp8(x: torch.Tensor, w: torch.Tensor, w_scale: torch.Tensor,
             out: torch.Tensor | None = None) -> torch.Tensor:
    """M = 1 GEMV (ops/gemv.cuh:92-104 semantics): y[N] = bf16((W . x) * s)."""
    w = _check_w(w)
    N, K = w.shape
    if out is None:
        out = torch.empty((N,), dtype=torch.bfloat16, device=x.device)
    rc = _lib.lib().nmi_gemv_fp8(x.data_ptr(), w.data_ptr(), w_scale.data_ptr(), out.data_ptr(),
                                 N, K, _stream())
    _lib.check(rc, "nmi_gemv_fp8")
    return out


def gemm_fp8_w8a16(x: torch.Tensor, w: torch.Tensor, w_scale: torch.Tensor,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """Prefill GEMM on bf16 MFMA for any M (ops/gemm.cuh:325-403 replacement)."""
    w = _check_w(w)
    M, K = x.shape
    N = w.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    rc = _lib.lib().nmi_gemm_fp8_w8a16(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0),
                                       w_scale.data_ptr(), out.data_ptr(), out.stride(0), M, N, K,
                                       None, 0, _stream())
    _lib.check(rc, "nmi_gemm_fp8_w8a16")
    return out


def decode_e4m3(codes: torch.Tensor, scale: float):
    """Device decode of uint8 codes through the kernels' conversion helpers.
    Returns (f32 values, f32 values * scale, bf16 values)."""
    n = codes.numel()
    f = torch.empty(n, dtype=torch.float32, device=codes.device)
    fs = torch.empty_like(f)
    b = torch.empty(n, dtype=torch.bfloat16, device=codes.device)
    rc = _lib.lib().nmi_fp8_e4m3_decode(codes.data_ptr(), f.data_ptr(), fs.data_ptr(), b.data_ptr(),
                                        float(scale), n, _stream())
    _lib.check(rc, "nmi_fp8_e4m3_decode")
    return f, fs, b
