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


def _check_w(w: torch.Tensor, K: int | None = None) -> torch.Tensor:
    """e4m3 weights [N, K] as uint8 codes; rows must be contiguous (stride(-1) == 1)."""
    if w.dtype == torch.float8_e4m3fn:
        w = w.view(torch.uint8)
    elif w.dtype != torch.uint8:
        raise TypeError(f"weights must be float8_e4m3fn or uint8 codes, got {w.dtype}")
    if w.dim() != 2 or w.stride(-1) != 1:
        raise ValueError(f"weights must be a 2-D [N, K] matrix with contiguous rows (shape {tuple(w.shape)}, "
                         f"strides {w.stride()})")
    if K is not None and w.shape[1] != K:
        raise ValueError(f"weights have K = {w.shape[1]}, activations K = {K}")
    return w


def _check_s(s: torch.Tensor, N: int) -> torch.Tensor:
    """Per-row scales: contiguous float32 [N]."""
    if s.dtype != torch.float32:
        raise TypeError(f"w_scale must be float32, got {s.dtype}")
    if s.dim() != 1 or s.numel() != N or not s.is_contiguous():
        raise ValueError(f"w_scale must be a contiguous float32 vector of N = {N} values (shape {tuple(s.shape)})")
    return s


def _check_out(y: torch.Tensor, M: int, N: int, name: str = "out") -> torch.Tensor:
    """An output buffer: contiguous bf16 holding exactly [M, N] (or [N] when M == 1), returned
    as a 2-D view.  Anything else raises: a strided or copied view would silently receive
    the wrong elements or lose the results."""
    if y.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16, got {y.dtype}")
    ok_shape = tuple(y.shape) == (M, N) or (M == 1 and tuple(y.shape) == (N,))
    if not ok_shape or not y.is_contiguous():
        raise ValueError(f"{name} must be a contiguous bf16 tensor of shape ({M}, {N}) "
                         f"(got shape {tuple(y.shape)}, strides {y.stride()})")
    return y.view(M, N)


def _check_device(*ts: torch.Tensor) -> None:
    dev = ts[0].device
    if dev.type != "cuda":
        raise ValueError(f"tensors must be on a GPU, got {dev}")
    for t in ts[1:]:
        if t.device != dev:
            raise ValueError(f"all tensors must be on {dev}, got {t.device}")


_WORKSPACE: dict[int, torch.Tensor] = {}


def workspace(device: torch.device, nbytes: int) -> torch.Tensor | None:
    """Per-device workspace of the skinny kernel's K split: zero-filled when (re)allocated,
    kept for the process; every launch leaves it ready for the next.  Calls on one device
    share it, so they must be ordered on one stream (as torch's current stream orders them).
    Grows on demand -- make one eager call of the largest shape before capturing a graph."""
    if nbytes <= 0:
        return None
    idx = torch.device(device).index or 0
    ws = _WORKSPACE.get(idx)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _WORKSPACE[idx] = ws
    return ws


def _as_2d(x: torch.Tensor):
    x2 = x.unsqueeze(0) if x.dim() == 1 else x
    if x2.dtype != torch.bfloat16:
        raise TypeError("x must be bfloat16")
    if x2.stride(-1) != 1:
        raise ValueError("x must be contiguous in the last dimension")
    return x2


def linear_fp8_w8a16(x: torch.Tensor, w: torch.Tensor, w_scale: torch.Tensor,
                     out: torch.Tensor | None = None, use_workspace: bool = True) -> torch.Tensor:
    """y[M, N] = bf16_rne((x[M, K] . e4m3(W[N, K])^T) * w_scale[N]) on the GPU."""
    squeeze = x.dim() == 1
    x2 = _as_2d(x)
    M, K = x2.shape
    w = _check_w(w, K)
    N = w.shape[0]
    _check_s(w_scale, N)
    if out is None:
        out = torch.empty((N,) if squeeze else (M, N), dtype=torch.bfloat16, device=x.device)
    y2 = _check_out(out, M, N)
    _check_device(x2, w, w_scale, y2)
    L = _lib.lib()
    ws = workspace(x.device, L.nmi_linear_workspace_bytes(M, N, K)) if use_workspace else None
    rc = L.nmi_linear_fp8_w8a16_ws(
        x2.data_ptr(), x2.stride(0), w.data_ptr(), w.stride(0), w_scale.data_ptr(),
        y2.data_ptr(), y2.stride(0), M, N, K,
        None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(), _stream())
    _lib.check(rc, "nmi_linear_fp8_w8a16_ws")
    return out


def linear_fp8_w8a16_grouped(x: torch.Tensor, weights, outs=None, use_workspace: bool = True):
    """Several (W_i, s_i) sharing x in one dispatch: returns [y_i] with
    y_i = bf16((x . e4m3(W_i)^T) * s_i) (e.g. q/k/v of an attention block)."""
    x2 = _as_2d(x)
    M, K = x2.shape
    n = len(weights)
    if not 1 <= n <= _lib.MAX_GROUPS:
        raise ValueError(f"1..{_lib.MAX_GROUPS} groups")
    if outs is None:
        outs = [torch.empty((M, w.shape[0]), dtype=torch.bfloat16, device=x.device) for w, _ in weights]
    if len(outs) != n:
        raise ValueError(f"{n} weight groups but {len(outs)} outputs")
    arr = (_lib.LinearGroup * n)()
    for i, ((w, s), y) in enumerate(zip(weights, outs)):
        w = _check_w(w, K)
        _check_s(s, w.shape[0])
        y2 = _check_out(y, M, w.shape[0], f"outs[{i}]")
        _check_device(x2, w, s, y2)
        arr[i] = _lib.LinearGroup(w.data_ptr(), w.stride(0), s.data_ptr(), y2.data_ptr(), y2.stride(0),
                                  w.shape[0])
    L = _lib.lib()
    total = sum(w.shape[0] for w, _ in weights)
    ws = workspace(x.device, L.nmi_linear_workspace_bytes(M, total, K)) if use_workspace else None
    rc = L.nmi_linear_fp8_w8a16_grouped(x2.data_ptr(), x2.stride(0), M, K, arr, n,
                                        None if ws is None else ws.data_ptr(),
                                        0 if ws is None else ws.numel(), _stream())
    _lib.check(rc, "nmi_linear_fp8_w8a16_grouped")
    return outs


def linear_fp8_w8a16_batch(jobs, outs=None):
    """Independent linears (x_i, W_i, s_i) with the same M in one dispatch (one launch of the
    skinny kernel for 2 <= M <= 16): returns [y_i] with y_i = bf16((x_i . e4m3(W_i)^T) * s_i)."""
    n = len(jobs)
    if not 1 <= n <= _lib.MAX_BATCH:
        raise ValueError(f"1..{_lib.MAX_BATCH} jobs")
    xs = [_as_2d(x) for x, _, _ in jobs]
    M = xs[0].shape[0]
    if any(x2.shape[0] != M for x2 in xs):
        raise ValueError("every job's x must have the same number of rows M")
    if outs is None:
        outs = [torch.empty((M, w.shape[0]), dtype=torch.bfloat16, device=x.device) for x, w, _ in jobs]
    if len(outs) != n:
        raise ValueError(f"{n} jobs but {len(outs)} outputs")
    arr = (_lib.LinearJob * n)()
    for i, ((_, w, s), x2, y) in enumerate(zip(jobs, xs, outs)):
        K = x2.shape[1]
        w = _check_w(w, K)
        _check_s(s, w.shape[0])
        y2 = _check_out(y, M, w.shape[0], f"outs[{i}]")
        _check_device(x2, w, s, y2)
        arr[i] = _lib.LinearJob(x2.data_ptr(), x2.stride(0), K,
                                _lib.LinearGroup(w.data_ptr(), w.stride(0), s.data_ptr(), y2.data_ptr(),
                                                 y2.stride(0), w.shape[0]))
    _lib.check(_lib.lib().nmi_linear_fp8_w8a16_batch(arr, n, M, _stream()), "nmi_linear_fp8_w8a16_batch")
    return outs


def gemv_fp8(x: torch.Tensor, w: torch.Tensor, w_scale: torch.Tensor,
             out: torch.Tensor | None = None) -> torch.Tensor:
    """M = 1 GEMV (ops/gemv.cuh:92-104 semantics): y[N] = bf16((W . x) * s).  x is a contiguous
    bf16 [K] vector, W [N, K] with row stride K."""
    w = _check_w(w)
    N, K = w.shape
    if w.stride(0) != K:
        raise ValueError("gemv_fp8 takes W with row stride K (use linear_fp8_w8a16 for strided rows)")
    if x.dtype != torch.bfloat16 or x.numel() != K or not x.is_contiguous():
        raise ValueError(f"x must be a contiguous bf16 vector of K = {K} values (shape {tuple(x.shape)})")
    _check_s(w_scale, N)
    if out is None:
        out = torch.empty((N,), dtype=torch.bfloat16, device=x.device)
    _check_out(out, 1, N)
    _check_device(x, w, w_scale, out)
    rc = _lib.lib().nmi_gemv_fp8(x.data_ptr(), w.data_ptr(), w_scale.data_ptr(), out.data_ptr(),
                                 N, K, _stream())
    _lib.check(rc, "nmi_gemv_fp8")
    return out


def gemm_fp8_w8a16(x: torch.Tensor, w: torch.Tensor, w_scale: torch.Tensor,
                   out: torch.Tensor | None = None, use_workspace: bool = True) -> torch.Tensor:
    """Prefill GEMM on bf16 MFMA for any M (ops/gemm.cuh:325-403 replacement).  With the
    per-device workspace the large-tile kernels may split K between workgroups (stream-K)."""
    if x.dim() != 2:
        raise ValueError("x must be a 2-D [M, K] bf16 matrix")
    x2 = _as_2d(x)
    M, K = x2.shape
    w = _check_w(w, K)
    N = w.shape[0]
    _check_s(w_scale, N)
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    y2 = _check_out(out, M, N)
    _check_device(x2, w, w_scale, y2)
    L = _lib.lib()
    ws = workspace(x.device, L.nmi_linear_workspace_bytes(M, N, K)) if use_workspace else None
    rc = L.nmi_gemm_fp8_w8a16(x2.data_ptr(), x2.stride(0), w.data_ptr(), w.stride(0),
                              w_scale.data_ptr(), y2.data_ptr(), y2.stride(0), M, N, K,
                              None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(),
                              _stream())
    _lib.check(rc, "nmi_gemm_fp8_w8a16")
    return out


def rmsnorm_bf16(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-5,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """RMSNorm of bf16 rows (ops/reduce.cuh:229-244): y = bf16(x * (1/sqrt(mean(x^2) + eps) * w))."""
    x2 = _as_2d(x)
    if not x2.is_contiguous() or w.dtype != torch.float32 or not w.is_contiguous():
        raise ValueError("x must be contiguous bf16 and w contiguous float32")
    M, K = x2.shape
    if tuple(w.shape) != (K,):
        raise ValueError(f"w must hold K = {K} values")
    if out is None:
        out = torch.empty_like(x)
    _check_out(out, M, K) if x.dim() == 2 else _check_out(out, 1, K)
    _check_device(x2, w, out)
    rc = _lib.lib().nmi_rmsnorm_bf16(x2.data_ptr(), w.data_ptr(), out.data_ptr(), M, K, eps, _stream())
    _lib.check(rc, "nmi_rmsnorm_bf16")
    return out


_BLOCK_WS: dict[int, torch.Tensor] = {}


def mlp_forward_fp8(x: torch.Tensor, norm_w: torch.Tensor, up_w: torch.Tensor, up_s: torch.Tensor,
                    down_w: torch.Tensor, down_s: torch.Tensor, out: torch.Tensor | None = None,
                    eps: float = 1e-5, use_workspace: bool = True) -> torch.Tensor:
    """The fp8 MLP block (model/mlp_block.cuh:121-176): out = x + down(relu(up(rmsnorm(x)))^2).
    x, out: [M, hidden] bf16; up_w [inter, hidden], down_w [hidden, inter] e4m3 with per-row
    float32 scales.  The transient buffers come from a per-device tensor kept for the process
    (or, with use_workspace=False, from the library's bump allocator)."""
    x2 = _as_2d(x)
    if not x2.is_contiguous():
        raise ValueError("x must be contiguous")
    M, hidden = x2.shape
    up_w = _check_w(up_w, hidden)
    inter = up_w.shape[0]
    down_w = _check_w(down_w, inter)
    if down_w.shape[0] != hidden:
        raise ValueError(f"down_proj has {down_w.shape[0]} rows, hidden size is {hidden}")
    _check_s(up_s, inter)
    _check_s(down_s, hidden)
    if norm_w.dtype != torch.float32 or tuple(norm_w.shape) != (hidden,) or not norm_w.is_contiguous():
        raise ValueError(f"norm_w must be a contiguous float32 vector of {hidden} values")
    if out is None:
        out = torch.empty_like(x)
    _check_out(out, M, hidden) if x.dim() == 2 else _check_out(out, 1, hidden)
    _check_device(x2, norm_w, up_w, up_s, down_w, down_s, out)
    L = _lib.lib()
    ws = _block_ws(x.device, L.nmi_mlp_workspace_bytes(M, hidden, inter)) if use_workspace else None
    rc = L.nmi_mlp_forward_fp8(x2.data_ptr(), norm_w.data_ptr(), up_w.data_ptr(), up_s.data_ptr(),
                               down_w.data_ptr(), down_s.data_ptr(), out.data_ptr(), M, hidden, inter, eps,
                               None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(),
                               _stream())
    _lib.check(rc, "nmi_mlp_forward_fp8")
    return out


def _block_ws(device: torch.device, need: int) -> torch.Tensor:
    idx = device.index or 0
    ws = _BLOCK_WS.get(idx)
    if ws is None or ws.numel() < need:
        ws = torch.empty(max(need, 1 << 20), dtype=torch.uint8, device=device)
        _BLOCK_WS[idx] = ws
    return ws


def _check_bf16(t: torch.Tensor, shape, name: str) -> None:
    if t.dtype != torch.bfloat16 or tuple(t.shape) != tuple(shape) or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous bf16 tensor of shape {tuple(shape)}, "
                         f"got {t.dtype} {tuple(t.shape)}")


def _check_caches(k_cache: torch.Tensor, v_cache: torch.Tensor, S_cache: int):
    if k_cache.dim() != 3 or k_cache.shape[2] != 128:
        raise ValueError(f"k_cache must be [n_kv_heads, cache_cap, 128], got {tuple(k_cache.shape)}")
    n_kv, cap, _ = k_cache.shape
    _check_bf16(k_cache, (n_kv, cap, 128), "k_cache")
    _check_bf16(v_cache, (n_kv, cap, 128), "v_cache")
    if not 0 <= S_cache < cap:
        raise ValueError(f"S_cache={S_cache} must be in [0, cache_cap={cap})")
    return n_kv, cap


def sdpa_decode_bf16(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, k_new: torch.Tensor,
                     v_new: torch.Tensor, S_cache: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """Attention decode (ops/attention/sdpa_decode.cuh:267-285): q [H, 128] against the caches
    [H_KV, cap, 128] over positions [0, S_cache), then k_new / v_new [H_KV, 128] stored at
    position S_cache.  Returns o [H, 128] bf16."""
    n_kv, cap = _check_caches(k_cache, v_cache, S_cache)
    if q.dim() != 2 or q.shape[1] != 128:
        raise ValueError(f"q must be [n_heads, 128], got {tuple(q.shape)}")
    H = q.shape[0]
    _check_bf16(q, (H, 128), "q")
    _check_bf16(k_new, (n_kv, 128), "k_new")
    _check_bf16(v_new, (n_kv, 128), "v_new")
    if out is None:
        out = torch.empty_like(q)
    _check_bf16(out, (H, 128), "out")
    _check_device(q, k_cache, v_cache, k_new, v_new, out)
    L = _lib.lib()
    need = L.nmi_sdpa_decode_workspace_bytes(H, n_kv, S_cache)
    ws = _block_ws(q.device, need) if need else None
    rc = L.nmi_sdpa_decode_bf16(q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr(),
                                k_new.data_ptr(), v_new.data_ptr(), S_cache, cap, H, n_kv,
                                None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(), _stream())
    _lib.check(rc, "nmi_sdpa_decode_bf16")
    return out


def attn_decode_fp8(x: torch.Tensor, norm_w: torch.Tensor, q_w, q_s, k_w, k_s, v_w, v_s, o_w, o_s,
                    k_cache: torch.Tensor, v_cache: torch.Tensor, S_cache: int, out: torch.Tensor | None = None,
                    eps: float = 1e-5, use_workspace: bool = True) -> torch.Tensor:
    """The fp8 attention block at decode (model/attention_block.cuh:371-414):
    out = x + o_proj(sdpa_decode(q_proj(h), caches, S_cache)), h = rmsnorm(x), with this token's
    k_proj(h) / v_proj(h) stored in the caches at position S_cache.  x, out [1, hidden] (or
    [hidden]) bf16; weights e4m3 [rows, cols] with per-row float32 scales; caches
    [n_kv_heads, cap, 128] bf16."""
    x2 = _as_2d(x)
    if x2.shape[0] != 1 or not x2.is_contiguous() or x2.dtype != torch.bfloat16:
        raise ValueError("x must be one contiguous bf16 row")
    hidden = x2.shape[1]
    n_kv, cap = _check_caches(k_cache, v_cache, S_cache)
    q_w = _check_w(q_w, hidden)
    if q_w.shape[0] % 128:
        raise ValueError(f"q_proj has {q_w.shape[0]} rows, not a multiple of the head dim 128")
    H = q_w.shape[0] // 128
    k_w, v_w = _check_w(k_w, hidden), _check_w(v_w, hidden)
    for name, w in (("k_proj", k_w), ("v_proj", v_w)):
        if w.shape[0] != n_kv * 128:
            raise ValueError(f"{name} has {w.shape[0]} rows, the caches hold {n_kv} heads of 128")
    o_w = _check_w(o_w, H * 128)
    if o_w.shape[0] != hidden:
        raise ValueError(f"o_proj has {o_w.shape[0]} rows, hidden size is {hidden}")
    _check_s(q_s, H * 128)
    _check_s(k_s, n_kv * 128)
    _check_s(v_s, n_kv * 128)
    _check_s(o_s, hidden)
    if norm_w.dtype != torch.float32 or tuple(norm_w.shape) != (hidden,) or not norm_w.is_contiguous():
        raise ValueError(f"norm_w must be a contiguous float32 vector of {hidden} values")
    if out is None:
        out = torch.empty_like(x)
    _check_out(out, 1, hidden)
    _check_device(x2, norm_w, q_w, q_s, k_w, k_s, v_w, v_s, o_w, o_s, k_cache, v_cache, out)
    L = _lib.lib()
    ws = None
    if use_workspace:
        ws = _block_ws(x.device, L.nmi_attn_decode_workspace_bytes(hidden, H, n_kv, S_cache))
    rc = L.nmi_attn_decode_fp8(x2.data_ptr(), norm_w.data_ptr(), q_w.data_ptr(), q_s.data_ptr(), k_w.data_ptr(),
                               k_s.data_ptr(), v_w.data_ptr(), v_s.data_ptr(), o_w.data_ptr(), o_s.data_ptr(),
                               k_cache.data_ptr(), v_cache.data_ptr(), S_cache, cap, out.data_ptr(), hidden, H, n_kv,
                               eps, None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(),
                               _stream())
    _lib.check(rc, "nmi_attn_decode_fp8")
    return out


def _check_rows(t: torch.Tensor, S: int, cols: int, name: str) -> None:
    if t.dtype != torch.bfloat16 or t.dim() != 2 or t.shape[0] != S or t.shape[1] < cols or t.stride(1) != 1:
        raise ValueError(f"{name} must be a bf16 [S={S}, >= {cols}] tensor with contiguous rows, "
                         f"got {t.dtype} {tuple(t.shape)} strides {t.stride()}")


def sdpa_prefill_bf16(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, n_heads: int, n_kv_heads: int,
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """Causal attention over a prompt (ops/attention/sdpa_prefill.cuh:364-395), token-major: q
    [S, >= n_heads * 128], k, v [S, >= n_kv_heads * 128] (row-strided views allowed).  Returns o
    [S, n_heads * 128] bf16."""
    S = q.shape[0]
    _check_rows(q, S, n_heads * 128, "q")
    _check_rows(k, S, n_kv_heads * 128, "k")
    _check_rows(v, S, n_kv_heads * 128, "v")
    if out is None:
        out = torch.empty((S, n_heads * 128), dtype=torch.bfloat16, device=q.device)
    _check_rows(out, S, n_heads * 128, "out")
    _check_device(q, k, v, out)
    L = _lib.lib()
    need = L.nmi_sdpa_prefill_workspace_bytes(n_kv_heads, S)     # 0: the kernel reads q, k, v in place
    ws = _block_ws(q.device, need) if need else None
    rc = L.nmi_sdpa_prefill_bf16(q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), v.data_ptr(), v.stride(0),
                                 out.data_ptr(), out.stride(0), S, n_heads, n_kv_heads,
                                 ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0,
                                 _stream())
    _lib.check(rc, "nmi_sdpa_prefill_bf16")
    return out


def attn_forward_fp8(x: torch.Tensor, norm_w: torch.Tensor, q_w, q_s, k_w, k_s, v_w, v_s, o_w, o_s,
                     k_cache: torch.Tensor | None = None, v_cache: torch.Tensor | None = None,
                     out: torch.Tensor | None = None, eps: float = 1e-5, use_workspace: bool = True) -> torch.Tensor:
    """The fp8 attention block over a prompt (model/attention_block.cuh:289-366): x, out
    [S, hidden] bf16; with k_cache and v_cache ([n_kv_heads, cap, 128] bf16) positions [0, S)
    receive this prompt's k and v."""
    x2 = _as_2d(x)
    if not x2.is_contiguous() or x2.dtype != torch.bfloat16:
        raise ValueError("x must be a contiguous bf16 tensor")
    S, hidden = x2.shape
    q_w, k_w, v_w = _check_w(q_w, hidden), _check_w(k_w, hidden), _check_w(v_w, hidden)
    if q_w.shape[0] % 128 or k_w.shape[0] % 128 or k_w.shape[0] != v_w.shape[0]:
        raise ValueError("q/k/v projections must have whole 128-row heads, k and v the same count")
    H, n_kv = q_w.shape[0] // 128, k_w.shape[0] // 128
    o_w = _check_w(o_w, H * 128)
    if o_w.shape[0] != hidden:
        raise ValueError(f"o_proj has {o_w.shape[0]} rows, hidden size is {hidden}")
    _check_s(q_s, H * 128)
    _check_s(k_s, n_kv * 128)
    _check_s(v_s, n_kv * 128)
    _check_s(o_s, hidden)
    if norm_w.dtype != torch.float32 or tuple(norm_w.shape) != (hidden,) or not norm_w.is_contiguous():
        raise ValueError(f"norm_w must be a contiguous float32 vector of {hidden} values")
    cap = 0
    if k_cache is not None or v_cache is not None:
        if k_cache is None or v_cache is None:
            raise ValueError("give both caches or neither")
        if k_cache.dim() != 3 or k_cache.shape[0] != n_kv or k_cache.shape[2] != 128 or k_cache.shape[1] < S:
            raise ValueError(f"k_cache must be [{n_kv}, cap >= {S}, 128], got {tuple(k_cache.shape)}")
        cap = k_cache.shape[1]
        _check_bf16(k_cache, (n_kv, cap, 128), "k_cache")
        _check_bf16(v_cache, (n_kv, cap, 128), "v_cache")
    if out is None:
        out = torch.empty_like(x)
    _check_out(out, S, hidden) if x.dim() == 2 else _check_out(out, 1, hidden)
    _check_device(x2, norm_w, q_w, q_s, k_w, k_s, v_w, v_s, o_w, o_s, out)
    L = _lib.lib()
    ws = _block_ws(x.device, L.nmi_attn_forward_workspace_bytes(S, hidden, H, n_kv)) if use_workspace else None
    rc = L.nmi_attn_forward_fp8(x2.data_ptr(), norm_w.data_ptr(), q_w.data_ptr(), q_s.data_ptr(), k_w.data_ptr(),
                                k_s.data_ptr(), v_w.data_ptr(), v_s.data_ptr(), o_w.data_ptr(), o_s.data_ptr(),
                                out.data_ptr(), S, None if k_cache is None else k_cache.data_ptr(),
                                None if v_cache is None else v_cache.data_ptr(), cap, hidden, H, n_kv, eps,
                                None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(), _stream())
    _lib.check(rc, "nmi_attn_forward_fp8")
    return out


def _check_f32(t: torch.Tensor, shape, name: str) -> None:
    if t.dtype != torch.float32 or tuple(t.shape) != tuple(shape) or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous float32 tensor of shape {tuple(shape)}, "
                         f"got {t.dtype} {tuple(t.shape)}")


def _mamba_params(n_heads, head_dim, n_groups, conv_w, conv_b, A_log, D, dt_bias, gnorm_w, conv_state, ssm_state,
                  batch):
    inter = n_heads * head_dim
    conv_dim = inter + 2 * n_groups * 128
    _check_f32(conv_w, (conv_dim, 4), "conv_w")
    _check_f32(conv_b, (conv_dim,), "conv_b")
    for name, t in (("A_log", A_log), ("D", D), ("dt_bias", dt_bias)):
        _check_f32(t, (n_heads,), name)
    _check_f32(gnorm_w, (inter,), "gnorm_w")
    _check_f32(conv_state, (batch, conv_dim, 3), "conv_state")
    _check_f32(ssm_state, (batch, n_heads, head_dim, 128), "ssm_state")
    return inter, conv_dim


def mamba_mixer_decode(proj: torch.Tensor, conv_w, conv_b, A_log, D, dt_bias, gnorm_w, conv_state, ssm_state,
                       n_heads: int, head_dim: int, n_groups: int, eps: float = 1e-5):
    """The Mamba-2 mixer between the projections at decode (nmi_mamba_mixer_decode): proj
    [batch, >= PROJ] bf16 = [z | xBC | dt]; conv_state [batch, conv_dim, 3] and ssm_state
    [batch, n_heads, head_dim, 128] float32, updated in place.  Returns (y, g), both
    [batch, n_heads * head_dim] bf16: the SSM output and the gated-norm output."""
    if proj.dim() != 2 or proj.dtype != torch.bfloat16 or proj.stride(-1) != 1:
        raise ValueError("proj must be a 2-D bf16 tensor with contiguous rows")
    batch = proj.shape[0]
    inter, _ = _mamba_params(n_heads, head_dim, n_groups, conv_w, conv_b, A_log, D, dt_bias, gnorm_w, conv_state,
                             ssm_state, batch)
    y = torch.empty((batch, inter), dtype=torch.bfloat16, device=proj.device)
    g = torch.empty_like(y)
    _check_device(proj, conv_w, conv_b, A_log, D, dt_bias, gnorm_w, conv_state, ssm_state)
    L = _lib.lib()
    rc = L.nmi_mamba_mixer_decode(proj.data_ptr(), proj.stride(0), conv_w.data_ptr(), conv_b.data_ptr(),
                                  A_log.data_ptr(), D.data_ptr(), dt_bias.data_ptr(), gnorm_w.data_ptr(),
                                  conv_state.data_ptr(), ssm_state.data_ptr(), y.data_ptr(), g.data_ptr(), batch,
                                  n_heads, head_dim, n_groups, 128, 4, eps, _stream())
    _lib.check(rc, "nmi_mamba_mixer_decode")
    return y, g


def mamba_decode_fp8(x: torch.Tensor, norm_w: torch.Tensor, in_w, in_s, conv_w, conv_b, A_log, D, dt_bias, gnorm_w,
                     out_w, out_s, conv_state, ssm_state, n_heads: int, head_dim: int, n_groups: int,
                     out: torch.Tensor | None = None, eps: float = 1e-5, use_workspace: bool = True) -> torch.Tensor:
    """The fp8 Mamba-2 block at decode (model/mamba_block.cuh:436-515): x, out [batch, hidden]
    bf16; in_w [PROJ, hidden], out_w [hidden, n_heads * head_dim] e4m3 with per-row float32 scales;
    the states are updated in place."""
    x2 = _as_2d(x)
    if not x2.is_contiguous() or x2.dtype != torch.bfloat16:
        raise ValueError("x must be a contiguous bf16 tensor")
    batch, hidden = x2.shape
    inter, conv_dim = _mamba_params(n_heads, head_dim, n_groups, conv_w, conv_b, A_log, D, dt_bias, gnorm_w,
                                    conv_state, ssm_state, batch)
    in_w = _check_w(in_w, hidden)
    if in_w.shape[0] != inter + conv_dim + n_heads:
        raise ValueError(f"in_proj has {in_w.shape[0]} rows, expected {inter + conv_dim + n_heads}")
    out_w = _check_w(out_w, inter)
    if out_w.shape[0] != hidden:
        raise ValueError(f"out_proj has {out_w.shape[0]} rows, hidden size is {hidden}")
    _check_s(in_s, in_w.shape[0])
    _check_s(out_s, hidden)
    if norm_w.dtype != torch.float32 or tuple(norm_w.shape) != (hidden,) or not norm_w.is_contiguous():
        raise ValueError(f"norm_w must be a contiguous float32 vector of {hidden} values")
    if out is None:
        out = torch.empty_like(x)
    _check_out(out, batch, hidden) if x.dim() == 2 else _check_out(out, 1, hidden)
    _check_device(x2, norm_w, in_w, in_s, conv_w, conv_b, A_log, D, dt_bias, gnorm_w, out_w, out_s, conv_state,
                  ssm_state, out)
    L = _lib.lib()
    ws = None
    if use_workspace:
        ws = _block_ws(x.device, L.nmi_mamba_decode_workspace_bytes(batch, hidden, n_heads, head_dim, n_groups, 128))
    rc = L.nmi_mamba_decode_fp8(x2.data_ptr(), norm_w.data_ptr(), in_w.data_ptr(), in_s.data_ptr(), conv_w.data_ptr(),
                                conv_b.data_ptr(), A_log.data_ptr(), D.data_ptr(), dt_bias.data_ptr(),
                                gnorm_w.data_ptr(), out_w.data_ptr(), out_s.data_ptr(), conv_state.data_ptr(),
                                ssm_state.data_ptr(), out.data_ptr(), batch, hidden, n_heads, head_dim, n_groups, 128, 4,
                                eps, None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(), _stream())
    _lib.check(rc, "nmi_mamba_decode_fp8")
    return out


def mamba_forward_fp8(x: torch.Tensor, norm_w: torch.Tensor, in_w, in_s, conv_w, conv_b, A_log, D, dt_bias, gnorm_w,
                      out_w, out_s, n_heads: int, head_dim: int, n_groups: int, batch: int = 1,
                      conv_state_out: torch.Tensor | None = None, ssm_state_out: torch.Tensor | None = None,
                      out: torch.Tensor | None = None, eps: float = 1e-5, use_workspace: bool = True) -> torch.Tensor:
    """The fp8 Mamba-2 block over prompts (model/mamba_block.cuh:346-425): x, out [batch * S,
    hidden] bf16 (batch sequences of S tokens), each from a zero state; the final states go to
    conv_state_out [batch, conv_dim, 3] / ssm_state_out [batch, n_heads, head_dim, 128] when given."""
    x2 = _as_2d(x)
    if not x2.is_contiguous() or x2.dtype != torch.bfloat16:
        raise ValueError("x must be a contiguous bf16 tensor")
    M, hidden = x2.shape
    if batch < 1 or M % batch:
        raise ValueError(f"{M} rows do not split into {batch} sequences")
    S = M // batch
    inter = n_heads * head_dim
    conv_dim = inter + 2 * n_groups * 128
    _check_f32(conv_w, (conv_dim, 4), "conv_w")
    _check_f32(conv_b, (conv_dim,), "conv_b")
    for name, t in (("A_log", A_log), ("D", D), ("dt_bias", dt_bias)):
        _check_f32(t, (n_heads,), name)
    _check_f32(gnorm_w, (inter,), "gnorm_w")
    if conv_state_out is not None:
        _check_f32(conv_state_out, (batch, conv_dim, 3), "conv_state_out")
    if ssm_state_out is not None:
        _check_f32(ssm_state_out, (batch, n_heads, head_dim, 128), "ssm_state_out")
    in_w = _check_w(in_w, hidden)
    if in_w.shape[0] != inter + conv_dim + n_heads:
        raise ValueError(f"in_proj has {in_w.shape[0]} rows, expected {inter + conv_dim + n_heads}")
    out_w = _check_w(out_w, inter)
    if out_w.shape[0] != hidden:
        raise ValueError(f"out_proj has {out_w.shape[0]} rows, hidden size is {hidden}")
    _check_s(in_s, in_w.shape[0])
    _check_s(out_s, hidden)
    if norm_w.dtype != torch.float32 or tuple(norm_w.shape) != (hidden,) or not norm_w.is_contiguous():
        raise ValueError(f"norm_w must be a contiguous float32 vector of {hidden} values")
    if out is None:
        out = torch.empty_like(x)
    _check_out(out, M, hidden) if x.dim() == 2 else _check_out(out, 1, hidden)
    _check_device(x2, norm_w, in_w, in_s, conv_w, conv_b, A_log, D, dt_bias, gnorm_w, out_w, out_s, out)
    L = _lib.lib()
    ws = None
    if use_workspace:
        ws = _block_ws(x.device, L.nmi_mamba_forward_workspace_bytes(batch, S, hidden, n_heads, head_dim, n_groups,
                                                                     128))
    rc = L.nmi_mamba_forward_fp8(x2.data_ptr(), norm_w.data_ptr(), in_w.data_ptr(), in_s.data_ptr(), conv_w.data_ptr(),
                                 conv_b.data_ptr(), A_log.data_ptr(), D.data_ptr(), dt_bias.data_ptr(),
                                 gnorm_w.data_ptr(), out_w.data_ptr(), out_s.data_ptr(), out.data_ptr(), batch, S,
                                 None if conv_state_out is None else conv_state_out.data_ptr(),
                                 None if ssm_state_out is None else ssm_state_out.data_ptr(), hidden, n_heads, head_dim,
                                 n_groups, 128, 4, eps, None if ws is None else ws.data_ptr(),
                                 0 if ws is None else ws.numel(), _stream())
    _lib.check(rc, "nmi_mamba_forward_fp8")
    return out


class GemvChain:
    """The GEMVs of a decode step with as few launches as the dependencies allow
    (nmi_gemv_chain_*; M = 1).

    phases: a list of (x, groups, wait_prev): x a [K] (or [1, K]) bf16 tensor, groups a list of
    up to four (w, s, y) -- w [N, K] e4m3 codes (uint8), s [N] float32, y [N] bf16 output -- and
    wait_prev whether the phase reads x only after the previous phase has completed (x may be an
    earlier phase's output; the phase then starts a new launch).  The plan holds raw pointers:
    the tensors are kept referenced here and must not be reallocated while the chain is in use.
    Launches go on torch's current stream and are graph-capturable."""

    def __init__(self, phases):
        L = _lib.lib()
        n = len(phases)
        arr = (_lib.GemvPhase * n)()
        self._keep = []
        for i, (x, groups, wait_prev) in enumerate(phases):
            if x.dtype != torch.bfloat16 or not x.is_contiguous() or not (
                    x.dim() == 1 or (x.dim() == 2 and x.shape[0] == 1)):
                raise ValueError(f"phase {i}: x must be a contiguous bf16 [K] (or [1, K]) vector")
            x1 = x.view(-1)
            if not 1 <= len(groups) <= _lib.MAX_GROUPS:
                raise ValueError(f"1..{_lib.MAX_GROUPS} groups per phase")
            K = x1.numel()
            arr[i].x_bf16 = x1.data_ptr()
            arr[i].K = K
            arr[i].ngroups = len(groups)
            arr[i].wait_prev = 1 if wait_prev else 0
            for j, (w, sc, y) in enumerate(groups):
                w = _check_w(w, K)
                _check_s(sc, w.shape[0])
                y1 = _check_out(y, 1, w.shape[0], f"phase {i} group {j} y").view(-1)
                _check_device(x1, w, sc, y1)
                arr[i].groups[j] = _lib.LinearGroup(w.data_ptr(), w.stride(0), sc.data_ptr(), y1.data_ptr(),
                                                    y1.numel(), w.shape[0])
                self._keep += [w, sc, y1]
            self._keep.append(x1)
        h = ctypes.c_void_p()
        _lib.check(L.nmi_gemv_chain_create(arr, n, ctypes.byref(h)), "nmi_gemv_chain_create")
        self._h = h
        self.nphases = n
        self.launches = 1 + sum(1 for _, _, w in phases[1:] if w)

    def launch(self):
        _lib.check(_lib.lib().nmi_gemv_chain_launch(self._h, None, 0, _stream()), "nmi_gemv_chain_launch")

    def close(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            _lib.lib().nmi_gemv_chain_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


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
