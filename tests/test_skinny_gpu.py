"""GPU parity of the 4x4x4 skinny kernel (1 <= M <= 16, bf16 MFMA over e4m3 weights converted in
registers; the 16x16x32 kernel, which takes M >= 3 by default, has its own tests and is switched
off here unless a test names it), of the small-M GEMV forms and of the grouped entry point,
against the torch fp32 dequant-then-F.linear oracle.

Tolerance: rel_l2 <= 1e-3 and max |diff| <= 2 bf16 ulp at max(|ref|, 2^-8 rms(ref)).
Size-independent properties: repeated calls are bit-identical, a grouped call equals the
separate calls under the same schedule, and M = 1 through this kernel agrees with the GEMV kernel
within the tolerance.
"""
import ctypes

import numpy as np
import pytest
import torch

from nemotron_infer_amd import _lib, ops, synth
from oracle import linear
from tests.conftest import load_golden
from tests.gpu_util import (DEV, announce, assert_parity, bits, oracle_bits, s_to_dev, w_to_dev,
                            x_to_dev)

pytestmark = pytest.mark.gpu

KNOBS = ("m1.path", "gemv.ks", "skinny.path", "s4.ks", "s4.t", "s4.u")


@pytest.fixture(autouse=True)
def _reset_tuning():
    """Default schedule, except that the 16x16x32 kernel (which takes M >= 3 by default and has
    its own tests) is switched off, so that M = 3 .. 16 here run the 4x4x4 kernel."""
    for k in KNOBS:
        _lib.tuning_set(k, 0)
    _lib.tuning_set("s16", 2)
    yield
    for k in KNOBS + ("s16",):
        _lib.tuning_set(k, 0)


def _case(M, N, K, seed, scales="log_uniform", act="normal"):
    w, s = synth.make_weight(N, K, seed, "cpu", scales=scales)
    x = synth.make_act(M, K, seed + 1, "cpu", kind=act)
    return x.view(torch.int16).numpy().view(np.uint16), w.numpy(), s.numpy()


def _run(x, w, s, use_ws):
    return bits(ops.linear_fp8_w8a16(x_to_dev(x), w_to_dev(w), s_to_dev(s), use_workspace=use_ws))


@pytest.mark.parametrize("name", ["kat_gemv_n64_k3136", "tiny_m4_n8_k16", "ragged_m3_n37_k208",
                                  "skinny_m16_n48_k3136", "special_nan_zero"])
@pytest.mark.parametrize("use_ws", [False, True])
@pytest.mark.parametrize("kernel", ["4x4x4", "16x16x32"])
def test_fixtures_all_m(name, use_ws, kernel):
    """Every fixture, every leading-row count 1..M of it, through both skinny kernels (the 4x4x4
    kernel, M = 1 forced onto it with m1.path = 3; the 16x16x32 kernel for 2 <= M <= 16 with
    s16 = 1, M = 1 on the GEMV kernel; fixtures whose K is not a multiple of 64 fall back to the
    4x4x4 kernel there)."""
    g = load_golden(name)
    x, w, s = g["x_bf16"], g["w_codes"], g["w_scale"]
    ref64 = linear.bf16_rne(g["y_f64"].astype(np.float32))
    if kernel == "4x4x4":
        _lib.tuning_set("m1.path", 3)
    else:
        _lib.tuning_set("s16", 1)
    for M in range(1, x.shape[0] + 1):
        announce("skinny_fixture", name, M, use_ws)
        y = _run(x[:M], w, s, use_ws)
        assert_parity(y, ref64[:M], f"{name} M={M} ws={use_ws} vs fp64")


@pytest.mark.parametrize("M", list(range(1, 17)))
def test_every_m_ragged(M):
    """Ragged N (not a multiple of 4, 16 or 64) and K (not a multiple of 64), both kernels (the
    4x4x4 one, M = 1 included; the 16x16x32 one with s16 = 1, path 1) and both workspace modes."""
    _lib.tuning_set("m1.path", 3)
    _lib.tuning_set("skinny.path", 2)
    for N, K in [(37, 208), (1000, 3136), (130, 12544 + 16)]:
        x, w, s = _case(M, N, K, 17 * M + N + K)
        ref = oracle_bits(x, w, s)
        for path in (0, 1):
            _lib.tuning_set("s16", 1 if path == 1 else 2)
            for use_ws in (False, True):
                announce("skinny_ragged", M, N, K, path, use_ws)
                assert_parity(_run(x, w, s, use_ws), ref, f"M={M} N={N} K={K} path={path} ws={use_ws}")


@pytest.mark.parametrize("ks", [1, 2, 4])
@pytest.mark.parametrize("t", [1, 2, 4])
@pytest.mark.parametrize("u", [2, 4, 8])
def test_s4_every_schedule(ks, t, u):
    """Each (waves splitting K, row groups per wave, chunks per lane) instantiation of the 4x4x4
    kernel (two LDS-DMA windows in flight; knob choices whose windows would not fit the LDS are
    narrowed), for M in {2, 5, 8, 16} (1, 2 and 4 groups of activation rows), with one, two, three
    and many windows (the loop over window pairs and both tails, partial last windows) and N not a
    multiple of the rows per workgroup."""
    _lib.tuning_set("s4.ks", ks)
    _lib.tuning_set("s4.t", t)
    _lib.tuning_set("s4.u", u)
    for M, N, K in [(2, 300, 3136), (5, 77, 5120), (8, 130, 1040), (16, 264, 3136), (13, 72, 208),
                    (3, 90, 12544 + 16), (9, 40, 16 * 16 * 3)]:
        announce("s4_schedule", ks, t, u, M, N, K)
        x, w, s = _case(M, N, K, 100 * ks + 10 * t + u + M)
        assert_parity(_run(x, w, s, False), oracle_bits(x, w, s), f"ks={ks} t={t} u={u} M={M}")


@pytest.mark.parametrize("M", [2, 4, 8, 16])
def test_config2_shapes(M):
    """Config 2 (M in {2,4,8,16}, the six decode shapes, per-row log-uniform scales) on the
    4x4x4 kernel (M = 2 too, with skinny.path = 2)."""
    _lib.tuning_set("skinny.path", 2)
    for lin in synth.SKINNY_SET:
        announce("skinny_config2", M, lin.name)
        x, w, s = _case(M, lin.N, lin.K, 2000 + M + lin.N % 53, act=lin.act)
        assert_parity(_run(x, w, s, True), oracle_bits(x, w, s), f"M={M} {lin.name}")


def test_new_inputs_each_call():
    """The same shape with new inputs each call: every result must match its own oracle (nothing
    from an earlier call -- LDS windows, registers -- leaks into the next)."""
    M, N, K = 4, 5120, 3136
    w, s = synth.make_weight(N, K, 5, "cpu", scales="log_uniform")
    wd, sd = w.to(DEV), s.to(DEV)
    for i in range(4):
        announce("stale_partials", i)
        x = synth.make_act(M, K, 300 + i, "cpu")
        y = ops.linear_fp8_w8a16(x.to(DEV), wd, sd)
        xb = x.view(torch.int16).numpy().view(np.uint16)
        assert_parity(bits(y), oracle_bits(xb, w.numpy(), s.numpy()), f"call {i}")


def test_grouped_qkv_matches_separate():
    """q|k|v in one launch (attention_block.cuh:400-402 runs them as three GEMVs) equals the
    three separate calls under the same (pinned) schedule, bit for bit, for M = 1 on the GEMV
    and 4x4x4 kernels and M = 4."""
    lins = synth.DECODE_SET[:3]
    for M in (1, 4):
        for path in (1, 3):
            if M > 1 and path == 1:
                continue
            _lib.tuning_set("m1.path", path)
            _lib.tuning_set("gemv.ks", 2)
            _lib.tuning_set("s4.t", 1)
            _lib.tuning_set("s4.ks", 1)
            announce("grouped_qkv", M, path)
            x = synth.make_act(M, 3136, 77, "cpu")
            ws = [synth.make_weight(l.N, l.K, 70 + i, "cpu", scales="log_uniform") for i, l in enumerate(lins)]
            xd = x.to(DEV)
            wd = [(w.to(DEV), s.to(DEV)) for w, s in ws]
            grouped = ops.linear_fp8_w8a16_grouped(xd, wd)
            separate = [ops.linear_fp8_w8a16(xd, w, s) for w, s in wd]
            torch.cuda.synchronize()
            xb = x.view(torch.int16).numpy().view(np.uint16)
            for (w, s), yg, ys, l in zip(ws, grouped, separate, lins):
                assert np.array_equal(bits(yg), bits(ys)), f"{l.name} M={M} path={path}"
                assert_parity(bits(yg), oracle_bits(xb, w.numpy(), s.numpy()), f"grouped {l.name}")


def test_grouped_rejects_bad_groups():
    L = _lib.lib()
    arr = (_lib.LinearGroup * 5)()
    assert L.nmi_linear_fp8_w8a16_grouped(0x10000, 64, 1, 64, arr, 5, None, 0, None) == _lib.NMI_ERR_INVALID_ARG
    assert L.nmi_linear_fp8_w8a16_grouped(0x10000, 64, 1, 64, arr, 0, None, 0, None) == _lib.NMI_ERR_INVALID_ARG


def test_m1_mfma_path_vs_gemv_full_size():
    """M = 1 at config 0's full size through the GEMV and 4x4x4 kernels: both within tolerance
    of the oracle."""
    N, K = 12544, 3136
    announce("m1_paths", N, K)
    x, w, s = _case(1, N, K, 5, scales="per_tensor")
    ref = oracle_bits(x[0], w, s)
    for path in (1, 3):
        _lib.tuning_set("m1.path", path)
        y = bits(ops.linear_fp8_w8a16(x_to_dev(x[0]), w_to_dev(w), s_to_dev(s)))
        assert_parity(y, ref, f"m1.path={path}")


@pytest.mark.parametrize("ks", [1, 2, 4])
@pytest.mark.parametrize("t", [1, 2, 4])
@pytest.mark.parametrize("p", [2, 3, 4])
def test_gemv_kernel_small_m(ks, t, p):
    """The multi-row GEMV kernel computing 2..4 activation rows at once (skinny.path = 3 with
    gemv.multirow = 1): every (K-split, rows per wave, chunks per lane) instantiation, M = 3 on the
    4-row variant, K past one LDS window (K = 10000 at M = 4 -> 625 chunks > 256), ragged N."""
    for k, v in (("skinny.path", 3), ("gemv.multirow", 1), ("gemv.ks", ks), ("gemv.t", t), ("gemv.p", p)):
        _lib.tuning_set(k, v)
    try:
        for M, N, K in [(2, 300, 3136), (3, 77, 5120), (4, 130, 10000), (4, 1000, 208)]:
            announce("gemv_small_m", ks, t, p, M, N, K)
            x, w, s = _case(M, N, K, 1000 * ks + 100 * t + 10 * p + M)
            assert_parity(_run(x, w, s, False), oracle_bits(x, w, s), f"ks={ks} t={t} p={p} M={M} N={N} K={K}")
    finally:
        for k in ("gemv.ks", "gemv.t", "gemv.p", "gemv.multirow"):
            _lib.tuning_set(k, 0)


@pytest.mark.parametrize("M", [2, 3, 4])
def test_stream_kernel_small_m(M):
    """The GEMV path at M = 2 (the stream kernel with two activation rows per weight step, every
    staging size: 2, 4, 8 pieces per thread and row) and at M = 3, 4 (skinny.path = 3: the
    multi-row kernel): ragged N, grouped matrices, strided x and y, against the oracle; nothing
    stored past the groups' columns."""
    _lib.tuning_set("skinny.path", 3)
    try:
        for N, K in [(300, 3136), (77, 5120), (1000, 208), (130, 8192), (3136, 1040)] + ([(50, 16384)] if M == 2 else []):
            announce("stream_small_m", M, N, K)
            x, w, s = _case(M, N, K, 500 * M + N + K)
            assert_parity(_run(x, w, s, False), oracle_bits(x, w, s), f"M={M} N={N} K={K}", per_row_scales=True)
        # grouped, strided x (ldx = K + 64) and y (ldy = sum N + 24)
        K, Ns = 3136, (1000, 37, 517)
        x, w0, s0 = _case(M, Ns[0], K, 9000 + M)
        xbig = torch.zeros((M, K + 64), dtype=torch.bfloat16, device=DEV)
        xbig[:, :K] = x_to_dev(x)
        mats = [(w0, s0)] + [_case(M, n, K, 9100 + M + n)[1:] for n in Ns[1:]]
        ldy = sum(Ns) + 24
        ybig = torch.full((M, ldy), 9.0, dtype=torch.bfloat16, device=DEV)
        L = _lib.lib()
        groups = (_lib.LinearGroup * 4)()
        devw = []
        off = 0
        for i, ((w, s), n) in enumerate(zip(mats, Ns)):
            wd, sd = w_to_dev(w), s_to_dev(s)
            devw.append((wd, sd))
            groups[i].w_e4m3, groups[i].ldw, groups[i].w_scale = wd.data_ptr(), K, sd.data_ptr()
            groups[i].y_bf16, groups[i].ldy, groups[i].N = ybig.data_ptr() + 2 * off, ldy, n
            off += n
        _lib.check(L.nmi_linear_fp8_w8a16_grouped(xbig.data_ptr(), K + 64, M, K, groups, len(Ns), None, 0, None),
                   "grouped")
        torch.cuda.synchronize()
        off = 0
        for (w, s), n in zip(mats, Ns):
            assert_parity(bits(ybig[:, off:off + n]), oracle_bits(x, w, s), f"grouped M={M} N={n}", per_row_scales=True)
            off += n
        assert torch.all(ybig[:, off:] == 9.0)
    finally:
        _lib.tuning_set("skinny.path", 0)


@pytest.mark.parametrize("M", [3, 5, 16])
def test_s4_strided_operands(M):
    """ldx > K, ldw > K, ldy > N (slices of wider buffers) through the 4x4x4 kernel: the DMA
    offsets and the loads follow the strides, and nothing outside the output slice is written."""
    N, K = 200, 3136
    announce("s4_strided", M)
    x, w, s = _case(M, N, K, 900 + M, scales="log_uniform")
    xbig = torch.zeros((M, K + 64), dtype=torch.bfloat16, device=DEV)
    xbig[:, 32:32 + K] = x_to_dev(x)
    wbig = torch.zeros((N, K + 48), dtype=torch.uint8, device=DEV)
    wbig[:, 16:16 + K] = w_to_dev(w)
    ybig = torch.full((M, N + 40), 7.0, dtype=torch.bfloat16, device=DEV)
    sd = s_to_dev(s)
    L = _lib.lib()
    nbytes = L.nmi_linear_workspace_bytes(M, N, K)
    ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=DEV)
    xv, wv, yv = xbig[:, 32:], wbig[:, 16:], ybig[:, 8:]
    _lib.check(L.nmi_linear_fp8_w8a16_ws(xv.data_ptr(), xbig.stride(0), wv.data_ptr(), wbig.stride(0), sd.data_ptr(),
                                         yv.data_ptr(), ybig.stride(0), M, N, K, ws.data_ptr(), nbytes, None), "ws")
    torch.cuda.synchronize()
    assert_parity(bits(ybig[:, 8:8 + N]), oracle_bits(x, w, s), f"strided M={M}")
    assert torch.all(ybig[:, :8] == 7.0) and torch.all(ybig[:, 8 + N:] == 7.0)
