"""fp8 (e4m3) W8A16 linear oracle: y = bf16_rne( (x_bf16 . W_e4m3^T) * s[n] ).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Notation: W is [N, K] e4m3 codes (uint8, row-major), s is [N] float32 per-row scale,
x is [M, K] bf16 (uint16 bit patterns or torch.bfloat16), y is [M, N] bf16.

* ``linear_fp8_w8a16``      -- the reference's CPU oracle numerics:
  ``F.linear(x.float(), W.float() * s[:, None])`` then ``.to(torch.bfloat16)``
  (tools/ref_full_model.py:44-49 dequantizes ``w.float() * scale``; :137 applies F.linear).
* ``linear_fp64``           -- exact-as-possible brute force in float64 (small shapes).
* ``gemv_fp32_sequential``  -- numpy restatement of tests/ops/test_gemm.cu:505-513
  (fp32 sum in k order, then ``* w_scale[n]``), vectorised over rows.
* ``bf16_rne``              -- float32 -> bf16 round-to-nearest-even closed form.
* ``parity``                -- the gate: rel_l2 and max-abs in bf16 ulp with a floor.
"""
from __future__ import annotations

import numpy as np

from . import e4m3


# ---------------------------------------------------------------------------------------
# bf16 helpers (closed form; no torch)
# ---------------------------------------------------------------------------------------
def bf16_rne(f: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest, ties to even; NaN -> 0x7FC0
    with the sign kept.  This is ``__float2bfloat16_rn`` (gemv.cuh:88) / ``.to(bfloat16)``."""
    f = np.ascontiguousarray(f, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(f)
    r[nan] = (0x7FC0 | ((u[nan] >> 16) & 0x8000)).astype(np.uint16)
    return r


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(f: np.ndarray) -> np.ndarray:
    return bf16_rne(f)


# ---------------------------------------------------------------------------------------
# Oracles
# ---------------------------------------------------------------------------------------
def dequant_f32(w_codes: np.ndarray, s: np.ndarray) -> np.ndarray:
    """W_f32[n, k] = LUT[W[n, k]] * s[n] in float32 (ref_full_model.py:48 ``w.float()*s``)."""
    lut = e4m3.decode_lut()
    return (lut[np.asarray(w_codes, dtype=np.uint8)] * np.asarray(s, np.float32)[:, None]).astype(np.float32)


def linear_fp8_w8a16(x_bf16_bits: np.ndarray, w_codes: np.ndarray, s: np.ndarray,
                     threads: int | None = None, return_f32: bool = False):
    """The torch CPU reference path, restated: dequant W to fp32 with its per-row scale,
    ``F.linear`` in fp32 on ``x.float()``, round the result to bf16.

    ``x_bf16_bits`` is uint16 [M, K] (or [K]); ``w_codes`` uint8 [N, K]; ``s`` float32 [N].
    Returns uint16 bf16 bits [M, N] (and the fp32 result when ``return_f32``)."""
    import torch
    import torch.nn.functional as F

    if threads is not None:
        torch.set_num_threads(threads)
    x = np.ascontiguousarray(x_bf16_bits, dtype=np.uint16)
    squeeze = x.ndim == 1
    if squeeze:
        x = x[None, :]
    xt = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16)
    wt = torch.from_numpy(np.ascontiguousarray(w_codes, dtype=np.uint8)).view(torch.float8_e4m3fn)
    st = torch.from_numpy(np.ascontiguousarray(s, dtype=np.float32))
    with torch.no_grad():
        wf = wt.float() * st[:, None]
        yf = F.linear(xt.float(), wf)
        yb = yf.to(torch.bfloat16)
    out = yb.view(torch.int16).numpy().view(np.uint16)
    yf = yf.numpy()
    if squeeze:
        out, yf = out[0], yf[0]
    return (out, yf) if return_f32 else out


def linear_fp64(x_bf16_bits: np.ndarray, w_codes: np.ndarray, s: np.ndarray) -> np.ndarray:
    """float64 brute force: y = (sum_k LUT[W]*x) * s, everything in double.  Returns fp64
    [M, N] (unrounded).  For small shapes: the reference point for pinning the oracles."""
    x = bf16_to_f32(np.atleast_2d(x_bf16_bits)).astype(np.float64)
    w = e4m3.decode_lut().astype(np.float64)[np.asarray(w_codes, np.uint8)]
    acc = x @ w.T
    return acc * np.asarray(s, np.float64)[None, :]


def gemv_fp32_sequential(x_bf16_bits: np.ndarray, w_codes: np.ndarray, s: np.ndarray) -> np.ndarray:
    """tests/ops/test_gemm.cu:505-513: ``sum += float(W[n,k]) * float(x[k])`` in k order in
    float32, then ``y[n] = sum * w_scale[n]`` in float32.  Returns float32 [N]."""
    x = bf16_to_f32(np.asarray(x_bf16_bits)).astype(np.float32)
    w = e4m3.decode_lut()[np.asarray(w_codes, np.uint8)]
    acc = np.zeros(w.shape[0], dtype=np.float32)
    for k in range(w.shape[1]):
        acc = (acc + (w[:, k] * x[k]).astype(np.float32)).astype(np.float32)
    return (acc * np.asarray(s, np.float32)).astype(np.float32)


# ---------------------------------------------------------------------------------------
# Parity gate
# ---------------------------------------------------------------------------------------
def bf16_ulp(a: np.ndarray) -> np.ndarray:
    """Spacing of bf16 numbers at magnitude ``a`` (8 significant bits): 2^(floor(log2 a) - 7).
    Magnitudes below the smallest normal use the subnormal spacing 2^-133."""
    a = np.abs(np.asarray(a, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return np.exp2(e - 7)


def parity(y_bits: np.ndarray, ref_bits: np.ndarray, ulp_tol: float = 2.0,
           rel_l2_tol: float = 1e-3, floor_frac: float = 2.0 ** -8, flip_frac: float = 0.01,
           mag: np.ndarray | None = None, rel_l2_all_tol: float | None = None):
    """Compare a bf16 result with the bf16-rounded oracle.

    * max |y - ref| <= ``ulp_tol`` bf16 ulp taken at ``max(|ref|, floor_frac * rms(ref))``
      (the floor keeps float32 accumulation-order noise on near-zero outputs from failing);
    * rounding flips -- elements that differ by at most one ulp, which a different float32
      summation order produces when the exact value lies next to a bf16 rounding boundary --
      are at most ``flip_frac`` of the elements (order noise flips ~0.03%; a wrong rounding
      mode or a sub-ulp systematic error flips far more);
    * rel_l2 over the differences larger than one ulp, ||y - ref||_2 / ||ref||_2, must be
      <= ``rel_l2_tol`` (every systematic error -- a dropped term, a wrong scale or index --
      shows there);
    * NaN positions must agree exactly.
    Also returned: ``rel_l2_all``, the plain rel_l2 over every element, which must be
    <= ``rel_l2_all_tol`` when one is given.  Gate it wherever the scales are per tensor; with
    per-row scales spread over two decades (log-uniform) one rounding flip on an element that
    dominates ||ref|| can alone exceed 1e-3, so those cases rely on the flip-exempt rel_l2.

    ``mag`` (optional, float, shape of ``ref``) replaces |ref| as the magnitude at which ulps
    are taken: for a rounded sum such as a residual add, the larger summand, since a one-ulp
    difference in a summand is many ulps of a result that cancels towards zero."""
    y = bf16_to_f32(y_bits).astype(np.float64)
    r = bf16_to_f32(ref_bits).astype(np.float64)
    nan_y, nan_r = np.isnan(y), np.isnan(r)
    nan_ok = bool(np.array_equal(nan_y, nan_r))
    fin = ~(nan_y | nan_r)
    y, r = y[fin], r[fin]
    m = np.abs(r) if mag is None else np.maximum(np.abs(np.asarray(mag, np.float64)[fin]), np.abs(r))
    if r.size == 0:
        return dict(ok=nan_ok, rel_l2=0.0, rel_l2_all=0.0, max_ulp=0.0, nan_ok=nan_ok, n=0,
                    n_diff=0, n_flip=0)
    denom = np.linalg.norm(r)
    d = y - r
    rms = float(np.sqrt(np.mean(r * r)))
    ulps = np.abs(d) / bf16_ulp(np.maximum(m, floor_frac * rms))
    exact_ulp = np.abs(d) / bf16_ulp(m)                  # at the reference's own magnitude
    flip = (d != 0) & (exact_ulp <= 1.0)
    big = np.where(flip, 0.0, d)
    rel_all = float(np.linalg.norm(d) / denom) if denom > 0 else float(np.linalg.norm(d))
    rel = float(np.linalg.norm(big) / denom) if denom > 0 else float(np.linalg.norm(big))
    max_ulp = float(ulps.max()) if ulps.size else 0.0
    n_flip = int(np.count_nonzero(flip))
    ok = (nan_ok and rel <= rel_l2_tol and max_ulp <= ulp_tol and n_flip <= flip_frac * r.size
          and (rel_l2_all_tol is None or rel_all <= rel_l2_all_tol))
    return dict(ok=ok, rel_l2=rel, rel_l2_all=rel_all, max_ulp=max_ulp, nan_ok=nan_ok, n=int(r.size),
                n_diff=int(np.count_nonzero(d)), n_flip=n_flip)
