"""CPU oracle for the fp8 MLP block and its bf16 element-wise steps -- TEST INFRASTRUCTURE ONLY.

Restates, in numpy/torch on the CPU, the data flow of nemotron_infer's fp8 MLP block
(csrc/include/model/mlp_block.cuh:121-176) so that the HIP block can be checked against it.
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg use it.

bf16 tensors are uint16 bit patterns, as in ``oracle.linear``.

* ``rmsnorm_bf16``   -- ops/reduce.cuh:135-214 (``rmsnorm_kernel_bf16``): per row
  r = 1 / sqrt(sum_k x^2 / K + eps), y = bf16_rne(x * (r * w)).  The sum of squares is taken
  in float64 and rounded to float32 once (the reference and the kernel both sum in float32, each
  in its own order; the float64 sum is the order-free value they approximate), then the float32
  steps in the reference's order with correctly rounded '/' and sqrt.
* ``relu2_bf16``     -- ops/elementwise.cuh:256-272: ``__hfma2_relu(x, 1, 0)`` then
  ``__hmul2(r, r)``, i.e. the bf16 rounding of max(x, 0)^2.
* ``add_bf16``       -- ops/elementwise.cuh:241-244: ``__hadd2``, the bf16 rounding of a + b.
* ``bf16_round_exact`` -- round-to-nearest-even of a float64 value to bf16 (8 significant bits,
  subnormal spacing 2^-133, overflow to inf); pins the two element-wise steps above.
* ``mlp_block_fp8``  -- the block at every M with bf16 activations into both projections:
  rmsnorm -> linear(up) -> relu^2 -> linear(down) -> residual add, each step rounded to bf16
  as the reference's M == 1 path does (mlp_block.cuh:140-148, 173-175); the projections in
  torch fp32 or (``precise``) float64.  The reference's
  M > 1 path quantizes the activations to e4m3 first (mlp_block.cuh:151-171); the library
  under test does not, and neither does this oracle.
* ``mlp_block_hf_f32`` -- the HF fp32 block of tools/dump_mlp_block.py:28-53
  (``plain_rmsnorm`` then ``down(relu(up(h))^2)`` plus the residual), all float32, no
  quantization: the expectation of the reference's FP8_MatchHF test (test_mlp_block.cu:155-185).
"""
from __future__ import annotations

import numpy as np

from . import linear

F32 = np.float32


def bf16_round_exact(v: np.ndarray) -> np.ndarray:
    """float64 -> bf16 bit patterns, round to nearest, ties to even, from the float64 value
    (no intermediate float32 rounding).  NaN -> 0x7FC0 (sign kept)."""
    v = np.asarray(v, dtype=np.float64)
    out = np.empty(v.shape, dtype=np.float64)
    a = np.abs(v)
    fin = np.isfinite(v) & (a > 0)
    _, e = np.frexp(np.where(fin, a, 1.0))              # a = m * 2^e, m in [0.5, 1)
    spacing = np.exp2(np.maximum(e - 8, -133).astype(np.float64))
    out[:] = v
    out[fin] = np.rint(v[fin] / spacing[fin]) * spacing[fin]
    big = np.abs(out) >= 2.0 ** 128
    out[big] = np.copysign(np.inf, out[big])
    with np.errstate(over="ignore"):
        f = out.astype(np.float32)                       # exact: 8 significant bits
    return linear.bf16_rne(f)


def rmsnorm_bf16(x_bits: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """x [M, K] bf16 bits, w [K] float32 -> y [M, K] bf16 bits (ops/reduce.cuh:135-214)."""
    x = linear.bf16_to_f32(np.atleast_2d(x_bits))
    K = x.shape[1]
    ss = (x.astype(np.float64) ** 2).sum(axis=1).astype(F32)
    with np.errstate(divide="ignore"):
        r = (F32(1.0) / np.sqrt((ss / F32(K) + F32(eps)).astype(F32))).astype(F32)
    rw = (r[:, None] * np.asarray(w, F32)[None, :]).astype(F32)
    return linear.bf16_rne((x * rw).astype(F32))


def relu2_bf16(v_bits: np.ndarray) -> np.ndarray:
    """bf16 rounding of max(v, 0)^2 (ops/elementwise.cuh:256-272); NaN stays NaN."""
    with np.errstate(invalid="ignore", over="ignore"):
        v = linear.bf16_to_f32(v_bits).astype(np.float64)
        r = np.where(v < 0, 0.0, v)                      # -0 -> -0, squared -> +0
        return bf16_round_exact(r * r)


def add_bf16(a_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    """bf16 rounding of a + b (ops/elementwise.cuh:241-244)."""
    with np.errstate(invalid="ignore", over="ignore"):
        a = linear.bf16_to_f32(a_bits).astype(np.float64)
        b = linear.bf16_to_f32(b_bits).astype(np.float64)
        return bf16_round_exact(a + b)


def mlp_block_fp8(x_bits, norm_w, up_codes, up_s, down_codes, down_s, eps=1e-5, return_stages=False,
                  precise=False):
    """The block on bf16 activations: x [M, hidden] bf16 bits, up [inter, hidden] e4m3 codes with
    up_s [inter], down [hidden, inter] codes with down_s [hidden].  Returns out bf16 bits.

    The projections are the torch fp32 ``F.linear`` of ``oracle.linear`` (the reference's CPU
    path), or with ``precise`` float64 sums rounded once to bf16: at K = 12544 with relu^2
    activations (all non-negative) the float32 sum of the former is off by up to ~3.5 bf16 ulp
    on outputs that cancel towards zero, which the latter is not."""
    x_bits = np.atleast_2d(np.asarray(x_bits, np.uint16))

    def proj(a, codes, s):
        if precise:
            return bf16_round_exact(linear.linear_fp64(a, codes, s))
        return linear.linear_fp8_w8a16(a, codes, s)

    h = rmsnorm_bf16(x_bits, norm_w, eps)
    up = proj(h, up_codes, up_s)
    act = relu2_bf16(up)
    down = proj(act, down_codes, down_s)
    out = add_bf16(x_bits, down)
    if return_stages:
        return out, dict(normed=h, up=up, act=act, down=down)
    return out


def mlp_block_hf_f32(x, norm_w, up_w, down_w, eps=1e-5):
    """tools/dump_mlp_block.py:28-53 in float32 torch: fp32 input and weights, no rounding to
    bf16 and no quantization.  Returns float32 [M, hidden]."""
    import torch
    import torch.nn.functional as F

    xt = torch.from_numpy(np.ascontiguousarray(x, F32))
    with torch.no_grad():
        var = xt.pow(2).mean(-1, keepdim=True)
        hs = (xt * torch.rsqrt(var + eps)) * torch.from_numpy(np.ascontiguousarray(norm_w, F32))
        up = F.linear(hs, torch.from_numpy(np.ascontiguousarray(up_w, F32)))
        act = F.relu(up).pow(2)
        down = F.linear(act, torch.from_numpy(np.ascontiguousarray(down_w, F32)))
        return (xt + down).numpy()
