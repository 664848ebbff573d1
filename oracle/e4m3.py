"""OCP 8-bit floating point, E4M3 variant ("e4m3fn"): decode table and quantizers.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Format (OCP 8-bit Floating Point Specification, E4M3): 1 sign bit, 4 exponent bits with
bias 7, 3 mantissa bits.  Exponent field 0 encodes subnormals m * 2^-9; the pattern
S.1111.111 (0x7F / 0xFF) is NaN; there is no infinity; the largest finite magnitude is
1.75 * 2^8 = 448.  The reference reads codes through ``static_cast<float>(__nv_fp8_e4m3)``
(nemotron_infer/csrc/include/ops/gemv.cuh:40-42) and torch ``float8_e4m3fn`` on the CPU
side (tools/ref_full_model.py:46-48); both implement this format.
"""
from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0
NAN_CODES = (0x7F, 0xFF)


def decode_code(b: int) -> float:
    """Decode one e4m3 code with the closed form (pure Python, used to build the table)."""
    sign = -1.0 if (b >> 7) & 1 else 1.0
    e = (b >> 3) & 0xF
    m = b & 0x7
    if e == 0xF and m == 0x7:
        return float("nan")
    if e == 0:
        return sign * m * 2.0 ** -9
    return sign * (1.0 + m / 8.0) * 2.0 ** (e - 7)


def decode_lut() -> np.ndarray:
    """256-entry float32 table: ``lut[b]`` is the value of code ``b``.

    NaN entries use the canonical quiet NaN 0x7FC00000 (sign kept for 0xFF)."""
    lut = np.array([decode_code(b) for b in range(256)], dtype=np.float32)
    bits = lut.view(np.uint32)
    bits[0x7F] = 0x7FC00000
    bits[0xFF] = 0xFFC00000
    return lut


def quantize_rne(q: np.ndarray) -> np.ndarray:
    """float32 -> e4m3 code, round-to-nearest-even, for inputs already clamped to +-448.

    This is the conversion ``static_cast<__nv_fp8_e4m3>(float)`` that the reference applies
    after its explicit clamp (tests/ops/test_gemm.cu:524-526, ops/gemm.cuh:285-287).  Since
    the magnitude ordering of the 127 non-negative finite codes matches their integer
    ordering and the code's low bit is the mantissa's low bit, RNE means: nearest table
    entry, ties to the even code.  NaN inputs map to 0x7F (sign kept).  Inputs beyond 448
    are rejected: the reference never converts them.
    """
    q = np.asarray(q, dtype=np.float32)
    if np.any(np.abs(q[~np.isnan(q)]) > E4M3_MAX):
        raise ValueError("quantize_rne: input must be clamped to +-448 first")
    mags = decode_lut()[:0x7F].astype(np.float64)          # codes 0..126, increasing
    a = np.abs(q.astype(np.float64))
    hi = np.searchsorted(mags, a, side="left")            # first table entry >= a
    hi = np.clip(hi, 0, 0x7E)
    lo = np.clip(hi - 1, 0, 0x7E)
    d_lo = a - mags[lo]
    d_hi = mags[hi] - a
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & ((hi & 1) == 0))
    code = np.where(pick_hi, hi, lo).astype(np.uint8)
    code = np.where(a == mags[hi], hi, code).astype(np.uint8)
    sign = (np.signbit(q)).astype(np.uint8) << 7
    out = (code | sign).astype(np.uint8)
    out[np.isnan(q)] = 0x7F | (sign[np.isnan(q)])
    return out


def quant_weight_perrow(wf: np.ndarray):
    """Per-row quantizer of tests/ops/test_gemm.cu:516-529 (and ops/gemm.cuh:198-216).

    For each output row n: ``s = rowmax|W| / 448`` (float32), ``s = 1/448`` when
    ``s < 1e-10``, ``inv = 1/s``, ``q = clamp(W * inv, -448, 448)``, code = RNE(q).
    Returns (codes uint8 [N,K], scales float32 [N])."""
    wf = np.asarray(wf, dtype=np.float32)
    rowmax = np.max(np.abs(wf), axis=1).astype(np.float32)
    s = (rowmax / np.float32(448.0)).astype(np.float32)
    s = np.where(s < np.float32(1e-10), np.float32(1.0) / np.float32(448.0), s).astype(np.float32)
    inv = (np.float32(1.0) / s).astype(np.float32)
    q = (wf * inv[:, None]).astype(np.float32)
    q = np.clip(q, np.float32(-448.0), np.float32(448.0))
    return quantize_rne(q), s


def quant_per_tensor(wf: np.ndarray):
    """Per-tensor quantizer of the synthetic configs: ``s = amax/448``,
    ``codes = RNE(clamp(W / s, +-448))``; the engine broadcasts ``s`` to a per-row vector
    (nemotron_infer/engine.py:117-121).  Returns (codes uint8 [N,K], scales float32 [N])."""
    wf = np.asarray(wf, dtype=np.float32)
    s = np.float32(np.max(np.abs(wf)) / np.float32(448.0))
    if s < np.float32(1e-10):
        s = np.float32(1.0) / np.float32(448.0)
    q = np.clip((wf / s).astype(np.float32), np.float32(-448.0), np.float32(448.0))
    return quantize_rne(q), np.full((wf.shape[0],), s, dtype=np.float32)
