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


def assert_parity(y_bits, ref_bits, label="", **kw):
    r = linear.parity(y_bits, ref_bits, **kw)
    assert r["ok"], f"{label}: {r}"
    return r
