"""Helpers shared by the GPU parity tests: move numpy bit patterns to the device and back,
run the product through the C ABI, and compare against the CPU oracle."""
from __future__ import annotations

import sys

import numpy as np
import torch

from oracle import linear

DEV = "cuda:0"


def announce(*parts) -> None:
    """Name the case before it touches the GPU (a fault may cut the log short)."""
    print("[case]", *parts, flush=True)
    sys.stdout.flush()


def x_to_dev(x_bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x_bits, np.uint16).view(np.int16)).view(torch.bfloat16).to(DEV)


def w_to_dev(codes: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(codes, np.uint8)).to(DEV)


def s_to_dev(s: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(s, np.float32)).to(DEV)


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def t_to_np_x(t: torch.Tensor) -> np.ndarray:
    return bits(t)


def oracle_bits(x_bits, codes, s) -> np.ndarray:
    return linear.linear_fp8_w8a16(x_bits, codes, s)


# Outputs of at least this many elements are also gated on rel_l2 over all elements: below it a
# single legitimate rounding flip (the oracle's own float32 summation order differs) on one
# large element can reach 1e-3 by itself (one flip of 2^-8 |y| on an element at 4 rms gives
# 0.016 / sqrt(n)).
STRICT_MIN_ELEMENTS = 2048


def assert_parity(y_bits, ref_bits, label="", per_row_scales=False, **kw):
    """The parity gate of oracle.linear.parity, plus rel_l2 over all elements <= 1e-3 on outputs
    of at least STRICT_MIN_ELEMENTS elements, unless the case has per-row scales spread over
    decades (log-uniform), where one rounding flip on a dominant element can exceed that alone
    and the flip-exempt rel_l2 is the systematic-error gate."""
    if not per_row_scales and np.asarray(ref_bits).size >= STRICT_MIN_ELEMENTS:
        kw.setdefault("rel_l2_all_tol", 1e-3)
    r = linear.parity(y_bits, ref_bits, **kw)
    assert r["ok"], f"{label}: {r}"
    return r
