"""GPU parity of the 16x16x32 skinny kernel (skinny16_fp8.hip: M <= 16, one row tile per
workgroup, K split between its waves whose sums are added in wave order; the DMA form, which
brings weights and activations into LDS with global_load_lds and reads them back in the MFMA
layout, and the row-run form, which loads 4 rows x 256 bytes per instruction into registers and
turns them into the MFMA layout through LDS), against the torch fp32 dequant-then-F.linear
oracle.

Tolerance: rel_l2 <= 1e-3 and max |diff| <= 2 bf16 ulp at max(|ref|, 2^-8 rms(ref)) (plus
rel_l2 over all elements where the scales are per tensor).  Size-independent properties:
repeated calls are bit-identical (fixed summation order), graph replays equal the eager call,
and nothing outside the output views is written.
"""
import numpy as np
import pytest
import torch

from nemotron_infer_amd import _lib, ops, synth
from tests.gpu_util import (DEV, announce, assert_parity, bits, oracle_bits, s_to_dev, w_to_dev,
                            x_to_dev)

pytestmark = pytest.mark.gpu

KNOBS = ("s16", "s16.r", "s16.t", "s16.w", "skinny.path")


@pytest.fixture(autouse=True)
def _reset_tuning():
    for k in KNOBS:
        _lib.tuning_set(k, 0)
    yield
    for k in KNOBS:
        _lib.tuning_set(k, 0)


def _case(M, N, K, seed, scales="log_uniform", act="normal"):
    w, s = synth.make_weight(N, K, seed, "cpu", scales=scales)
    x = synth.make_act(M, K, seed + 1, "cpu", kind=act)
    return x.view(torch.int16).numpy().view(np.uint16), w.numpy(), s.numpy()


def _check(M, N, K, seed, label, scales="log_uniform", act="normal"):
    x, w, s = _case(M, N, K, seed, scales=scales, act=act)
    xd, wd, sd = x_to_dev(x), w_to_dev(w), s_to_dev(s)
    y1 = ops.linear_fp8_w8a16(xd, wd, sd)
    y2 = ops.linear_fp8_w8a16(xd, wd, sd)
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16)), f"{label}: not deterministic"
    assert_parity(bits(y1), oracle_bits(x, w, s), label, per_row_scales=scales != "per_tensor")
    return bits(y1)


@pytest.mark.parametrize("M", [5, 8, 12, 16])
def test_config2_decode_shapes(M):
    """Config 2's decode shapes (q, k, v, o, up, down) at M from 5 to 16 (the default form),
    per-row log-uniform scales (K from 3136 to 12544)."""
    for lin in synth.SKINNY_SET:
        announce("s16_config2", M, lin.name, lin.N, lin.K)
        _check(M, lin.N, lin.K, 5000 + M + lin.N % 97, f"M={M} {lin.name}", act=lin.act)


@pytest.mark.parametrize("M", [2, 3, 4])
def test_small_m_when_forced(M):
    """s16 = 1 takes M = 2 .. 4 too (columns m >= M of the MFMA read row M - 1 and are dropped);
    M = 2 reaches it with skinny.path = 2 (otherwise the GEMV kernel takes M = 2)."""
    _lib.tuning_set("s16", 1)
    _lib.tuning_set("skinny.path", 2)
    for N, K in [(3136, 3136), (1000, 12544), (37, 64)]:
        announce("s16_small_m", M, N, K)
        _check(M, N, K, 5100 + M + N, f"M={M} N={N} K={K}")


@pytest.mark.parametrize("T,R,W", [(t, r, w) for t in (1, 0) for r in (1, 2) for w in (0, 2, 4)])
def test_ragged_shapes_each_form(T, R, W):
    """Both load forms (row runs through registers, T = 1; DMA into LDS, the default) with row
    tiles of 16 or 32 and two or four waves or as chosen (W = 0), on ragged N (partial last
    tiles), K of one slab (waves with nothing to do), K whose slabs do not divide between the
    waves or into 256-k groups, runs longer than two groups, many tiles, and 8 or 16 staged
    activation rows (M <= 8 or not)."""
    _lib.tuning_set("s16", 1)
    _lib.tuning_set("s16.t", T)
    _lib.tuning_set("s16.r", R)
    _lib.tuning_set("s16.w", W)
    for M, N, K in [(16, 37, 64), (7, 1000, 3136), (16, 300, 12544), (9, 20000, 192), (16, 16, 128),
                    (6, 257, 6272), (13, 2048, 1088), (5, 100, 576), (11, 64, 2112)]:
        announce("s16_ragged", T, R, W, M, N, K)
        _check(M, N, K, 5200 + 7 * R + W + M + N + K, f"T={T} R={R} W={W} M={M} N={N} K={K}")


@pytest.mark.parametrize("R,W", [(1, 2), (1, 4), (2, 2), (2, 4)])
def test_dma_form_equals_row_runs(R, W):
    """The DMA form splits K between the waves as the row-run form does and feeds the MFMAs the
    same operands in the same order: the same bytes, with 16 activation rows staged (M from 9 to
    16) or 8 (M <= 8), on ragged N and K."""
    for M, N, K in [(16, 3136, 12544), (9, 1000, 3136), (13, 300, 1088), (16, 37, 64), (8, 3136, 12544),
                    (5, 1000, 3136), (3, 300, 1088), (8, 37, 64)]:
        announce("s16_dma_eq_rows", R, W, M, N, K)
        _lib.tuning_set("s16", 1)
        _lib.tuning_set("s16.r", R)
        _lib.tuning_set("s16.w", W)
        _lib.tuning_set("s16.t", 1)
        y_rows = _check(M, N, K, 5260 + M + K, f"rows R={R} W={W} M={M} N={N} K={K}")
        _lib.tuning_set("s16.t", 0)
        y_dma = _check(M, N, K, 5260 + M + K, f"dma R={R} W={W} M={M} N={N} K={K}")
        assert np.array_equal(y_rows, y_dma), (R, W, M, N, K)


@pytest.mark.parametrize("T", [1, 0])
def test_row_tiles_agree(T):
    """Within a load form, row tiles of 16 or 32 sum each output over the same waves' runs in the
    same order: the same bytes."""
    M, N, K = 16, 3136, 12544
    announce("s16_forms_agree", T, M, N, K)
    _lib.tuning_set("s16", 1)
    _lib.tuning_set("s16.t", T)
    ys = []
    for R in (1, 2):
        _lib.tuning_set("s16.r", R)
        ys.append(_check(M, N, K, 5250, f"T={T} R={R}"))
    assert np.array_equal(ys[0], ys[1])


def test_per_tensor_scales_and_relu2_activations():
    """Per-tensor scales (the strict all-element rel_l2 gate applies) on down_proj's shape with
    relu^2-distributed activations (many exact zeros)."""
    announce("s16_per_tensor")
    _check(16, 3136, 12544, 5301, "per-tensor down_proj", scales="per_tensor", act="relu2")


def test_grouped_qkv_strided_outputs():
    """q | k | v in one launch, each output a column view of one [M, sum N] buffer with ragged
    widths (scalar stores where a view is not 8-byte aligned): every group matches the oracle and
    equals its separate call bit for bit (the launch takes row tiles of 32 for its 7120 rows, the
    k and v calls alone 16: the same sums), and nothing past the views is written."""
    M, K = 11, 3136
    Ns = (5120, 1000, 1000)
    announce("s16_grouped", M, Ns, K)
    cases = [_case(M, N, K, 5400 + i) for i, N in enumerate(Ns)]
    x = cases[0][0]
    xd = x_to_dev(x)
    wd = [(w_to_dev(w), s_to_dev(s)) for _, w, s in cases]
    total = sum(Ns)
    offs = np.cumsum((0,) + Ns)
    ybig = torch.full((M, total + 8), 3.0, dtype=torch.bfloat16, device=DEV)
    outs = [ybig[:, offs[i]:offs[i + 1]] for i in range(len(Ns))]
    L = _lib.lib()
    arr = (_lib.LinearGroup * len(Ns))()
    for i, ((w, s), y) in enumerate(zip(wd, outs)):
        arr[i] = _lib.LinearGroup(w.data_ptr(), w.stride(0), s.data_ptr(), y.data_ptr(), y.stride(0), w.shape[0])
    _lib.check(L.nmi_linear_fp8_w8a16_grouped(xd.data_ptr(), K, M, K, arr, len(Ns), None, 0, None), "grouped")
    separate = [ops.linear_fp8_w8a16(xd, w, s) for w, s in wd]
    torch.cuda.synchronize()
    assert torch.all(ybig[:, total:] == 3.0)
    for i, (_, w, s) in enumerate(cases):
        assert np.array_equal(bits(outs[i]), bits(separate[i])), f"group {i}"
        assert_parity(bits(outs[i]), oracle_bits(x, w, s), f"grouped {i}", per_row_scales=True)


@pytest.mark.parametrize("T", [1, 0])
@pytest.mark.parametrize("M", [3, 8, 16])
def test_strided_operands(T, M):
    """ldx > K, ldw > K, ldy > N (slices of wider buffers, 16-byte aligned) through both load
    forms: the DMA and register loads follow the strides, the results equal the contiguous
    call's bit for bit, and nothing outside the output slice is written."""
    N, K = 1000, 3136
    _lib.tuning_set("s16", 1)
    _lib.tuning_set("s16.t", T)
    announce("s16_strided", T, M, N, K)
    x, w, s = _case(M, N, K, 5700 + M)
    xbig = torch.zeros((M, K + 64), dtype=torch.bfloat16, device=DEV)
    xbig[:, 32:32 + K] = x_to_dev(x)
    wbig = torch.zeros((N, K + 48), dtype=torch.uint8, device=DEV)
    wbig[:, 16:16 + K] = w_to_dev(w)
    ybig = torch.full((M, N + 40), 7.0, dtype=torch.bfloat16, device=DEV)
    sd = s_to_dev(s)
    L = _lib.lib()
    xv, wv, yv = xbig[:, 32:], wbig[:, 16:], ybig[:, 8:]
    _lib.check(L.nmi_linear_fp8_w8a16(xv.data_ptr(), xbig.stride(0), wv.data_ptr(), wbig.stride(0), sd.data_ptr(),
                                      yv.data_ptr(), ybig.stride(0), M, N, K, None), "strided")
    y = ops.linear_fp8_w8a16(x_to_dev(x), w_to_dev(w), sd)
    torch.cuda.synchronize()
    assert np.array_equal(bits(ybig[:, 8:8 + N]), bits(y))
    assert_parity(bits(y), oracle_bits(x, w, s), f"strided T={T} M={M}")
    assert torch.all(ybig[:, :8] == 7.0) and torch.all(ybig[:, 8 + N:] == 7.0)


def test_k_not_a_multiple_of_64_goes_to_the_4x4x4_kernel():
    """K not a multiple of 64 runs the 4x4x4 kernel instead: the same bytes as with s16 = 2, within
    the parity gate of the oracle."""
    for M, N, K in [(8, 300, 3152), (12, 1000, 80)]:
        announce("s16_fallback", M, N, K)
        x, w, s = _case(M, N, K, 5500 + K)
        xd, wd, sd = x_to_dev(x), w_to_dev(w), s_to_dev(s)
        y = ops.linear_fp8_w8a16(xd, wd, sd)
        _lib.tuning_set("s16", 2)
        y4 = ops.linear_fp8_w8a16(xd, wd, sd)
        _lib.tuning_set("s16", 0)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), y4.view(torch.int16))
        assert_parity(bits(y), oracle_bits(x, w, s), f"fallback K={K}", per_row_scales=True)


def test_graph_replays_equal_eager():
    """A captured launch replayed with eager work in between: every replay equals the eager
    result."""
    M, N, K = 16, 12544, 3136
    announce("s16_graph", M, N, K)
    x, w, s = _case(M, N, K, 5600)
    xd, wd, sd = x_to_dev(x), w_to_dev(w), s_to_dev(s)
    y = ops.linear_fp8_w8a16(xd, wd, sd)
    torch.cuda.synchronize()
    eager = bits(y).copy()
    assert_parity(eager, oracle_bits(x, w, s), "eager", per_row_scales=True)
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            ops.linear_fp8_w8a16(xd, wd, sd, out=y)
    for rep in range(3):
        y.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bits(y), eager), rep
        ops.linear_fp8_w8a16(xd, wd, sd)                      # eager work between replays
        torch.cuda.synchronize()
