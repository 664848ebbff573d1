"""GPU parity of the M = 1 GEMV and of the device e4m3 decode (gfx950), through the C ABI.

Gates: (1) the 256-code decode and decode*scale are bit-exact against the committed table;
(2) outputs agree with bf16_rne(torch fp32 dequant-then-F.linear) within rel_l2 <= 1e-3 and
max |diff| <= 2 bf16 ulp taken at max(|ref|, 2^-8 rms(ref)).  Size-independent properties
(power-of-two linearity, row-slice invariance, determinism) are checked at full size.
"""
import numpy as np
import pytest
import torch

from nemotron_infer_amd import _lib, ops, synth
from oracle import e4m3, linear
from tests.conftest import load_golden
from tests.gpu_util import (DEV, announce, assert_parity, bits, oracle_bits, s_to_dev, w_to_dev,
                            x_to_dev)

pytestmark = pytest.mark.gpu

FIXTURES = ["kat_gemv_n64_k3136", "tiny_m4_n8_k16", "ragged_m3_n37_k208",
            "skinny_m16_n48_k3136", "special_nan_zero"]


GEMV_KNOBS = ("gemv.ks", "gemv.t", "gemv.p", "gemv.xg", "gemv.wgs", "gemv.multirow", "gemv.grid", "gemv.balance")


@pytest.fixture(autouse=True)
def _reset_tuning():
    for k in GEMV_KNOBS:
        _lib.tuning_set(k, 0)
    yield
    for k in GEMV_KNOBS:
        _lib.tuning_set(k, 0)


# ------------------------------------------------------------------------------- decode
@pytest.mark.parametrize("scale", [1.0, 0.0078125, 3.7e-3, 1.2345e-4, 2.0 ** -20, 65504.0])
def test_decode_256_codes_bit_exact(scale):
    announce("decode_256", scale)
    lut = load_golden("e4m3_lut")["lut_bits"].view(np.float32)
    # every code at every byte position of a dword
    codes = np.concatenate([np.roll(np.arange(256, dtype=np.uint8), r) for r in range(4)])
    f, fs, b = ops.decode_e4m3(w_to_dev(codes), scale)
    torch.cuda.synchronize()
    f, fs, b = f.cpu().numpy(), fs.cpu().numpy(), bits(b)
    ref = lut[codes]
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(f), nan) and np.array_equal(np.isnan(fs), nan)
    assert np.array_equal(f.view(np.uint32)[~nan], ref.view(np.uint32)[~nan])
    ref_s = (ref * np.float32(scale)).astype(np.float32)
    assert np.array_equal(fs.view(np.uint32)[~nan], ref_s.view(np.uint32)[~nan])
    # GEMM weight-tile dequant: e4m3 -> bf16 is exact
    bref = linear.bf16_rne(ref)
    assert np.array_equal(b[~nan], bref[~nan])
    assert np.all((b[nan] & 0x7FFF) > 0x7F80)


# ------------------------------------------------------------------------------- fixtures
@pytest.mark.parametrize("name", FIXTURES)
def test_gemv_fixture_rows(name):
    """Each activation row of each fixture through the M = 1 GEMV entry point."""
    g = load_golden(name)
    x, w, s = g["x_bf16"], g["w_codes"], g["w_scale"]
    announce("gemv_fixture", name, x.shape, w.shape)
    wd, sd = w_to_dev(w), s_to_dev(s)
    ref64 = linear.bf16_rne(g["y_f64"].astype(np.float32))
    for m in range(x.shape[0]):
        y = ops.gemv_fp8(x_to_dev(x[m]), wd, sd)
        yb = bits(y)
        assert_parity(yb, ref64[m], f"{name} row {m} vs fp64")
        assert_parity(yb, oracle_bits(x[m], w, s), f"{name} row {m} vs torch oracle")


def test_kat_reference_tolerance():
    """GemvFP8Test.MatchesReference's own bound (test_gemm.cu:572-576) on the same inputs."""
    from oracle import cref

    g = load_golden("kat_gemv_n64_k3136")
    announce("kat_reference_tolerance")
    y = linear.bf16_to_f32(bits(ops.gemv_fp8(x_to_dev(g["x_bf16"][0]), w_to_dev(g["w_codes"]),
                                             s_to_dev(g["w_scale"]))))
    ref = cref.gemv_fp8_seq(g["x_bf16"][0], g["w_codes"], g["w_scale"])
    assert np.all(np.abs(y - ref) <= np.maximum(0.02, 0.02 * np.abs(ref)))


def test_special_values_gemv():
    g = load_golden("special_nan_zero")
    announce("special_values")
    wd, sd = w_to_dev(g["w_codes"]), s_to_dev(g["w_scale"])
    y0 = linear.bf16_to_f32(bits(ops.gemv_fp8(x_to_dev(g["x_bf16"][0]), wd, sd)))
    y1 = bits(ops.gemv_fp8(x_to_dev(g["x_bf16"][1]), wd, sd))
    assert np.isnan(y0[1]) and np.isnan(y0[2])
    assert y0[3] == 0.0
    # all-zero activation: +0 exactly, except rows holding NaN codes
    assert np.all(y1[[0, 3, 4, 5, 6, 7]] == 0x0000)


# ------------------------------------------------------------------------------- real shapes
def _case(N, K, seed, scales="per_tensor", act="normal"):
    w, s = synth.make_weight(N, K, seed, "cpu", scales=scales)
    x = synth.make_act(1, K, seed + 1, "cpu", kind=act)[0]
    return (x.view(torch.int16).numpy().view(np.uint16), w.numpy(), s.numpy())


SHAPES = [("config0_up_proj", 12544, 3136, "normal")] + [
    (f"config1_{l.name}", l.N, l.K, l.act) for l in synth.DECODE_SET] + [
    ("config4_in_proj_ragged", synth.MAMBA_IN, 3136, "normal"),
    ("config4_out_proj", 3136, synth.MAMBA_OUT_K, "normal"),
]


@pytest.mark.parametrize("label,N,K,act", SHAPES)
def test_gemv_real_shapes(label, N, K, act):
    announce("gemv_shape", label, N, K)
    x, w, s = _case(N, K, 1000 + N % 97 + K % 89, act=act)
    y = bits(ops.gemv_fp8(x_to_dev(x), w_to_dev(w), s_to_dev(s)))
    r = assert_parity(y, oracle_bits(x, w, s), label)
    assert r["n"] == N


# K values that exercise every slice layout of the stream kernel: one partial chunk group
# (16, 48), exactly 256 chunks (4096), 257 chunks (two slices of 129), the decode shapes (one,
# two and four slices of 196 / 160 chunks), 20000 (five slices), the LDS limit (32768, eight
# slices) and K past it (40000: the multi-row kernel takes over)
STREAM_K = [16, 48, 1024, 3136, 4096, 4112, 5120, 6272, 12544, 20000, 32768, 40000]


@pytest.mark.parametrize("K", STREAM_K)
@pytest.mark.parametrize("knobs", [{}, {"gemv.wgs": 2}, {"gemv.balance": 2}, {"gemv.grid": 3}])
def test_stream_gemv_slices(K, knobs):
    """The M = 1 stream kernel against the oracle at every slice layout, with row counts that
    leave a half row group (odd N), a single row and fewer row groups than waves, per-row
    log-uniform scales (a wrong scale index shows), and several grids: the default (sized so
    that waves get equal row counts), two workgroups per CU, the plain capped grid, and three
    workgroups walking everything."""
    for k, v in knobs.items():
        _lib.tuning_set(k, v)
    for N in (1, 3, 37, 1000):
        announce("stream_gemv", K, N, knobs)
        x, w, s = _case(N, K, 11 * N + K, scales="log_uniform")
        y = bits(ops.gemv_fp8(x_to_dev(x), w_to_dev(w), s_to_dev(s)))
        assert_parity(y, oracle_bits(x, w, s), f"stream K={K} N={N} {knobs}", per_row_scales=True)


def test_stream_gemv_matches_grouped_and_strided():
    """Grouped launch (q|k|v sharing x) == three separate launches bit for bit, and strided
    weight rows (ldw > K) and strided outputs (ldy > N) give the same bits as contiguous ones."""
    K = 3136
    x, _, _ = _case(8, K, 3)
    xd = x_to_dev(x)
    groups = [_case(N, K, 40 + N, scales="log_uniform")[1:] for N in (5120, 1024, 1000)]
    wd = [(w_to_dev(w), s_to_dev(s)) for w, s in groups]
    announce("stream_grouped", K)
    ys = ops.linear_fp8_w8a16_grouped(xd, wd)
    for (w, s), yg, (wh, sh) in zip(wd, ys, groups):
        yone = ops.linear_fp8_w8a16(xd, w, s)
        assert np.array_equal(bits(yg).reshape(-1), bits(yone).reshape(-1))
        assert_parity(bits(yone), oracle_bits(x, wh, sh), "grouped", per_row_scales=True)
    # strided rows and outputs through the C ABI
    w, s = wd[2]
    N = w.shape[0]
    wpad = torch.zeros((N, K + 64), dtype=torch.uint8, device=DEV)
    wpad[:, :K] = w
    ypad = torch.full((1, 2 * N + 8), float("nan"), dtype=torch.bfloat16, device=DEV)
    L = _lib.lib()
    announce("stream_strided", N, K)
    _lib.check(L.nmi_linear_fp8_w8a16(xd.data_ptr(), K, wpad.data_ptr(), K + 64, s.data_ptr(),
                                      ypad.data_ptr(), 2 * N + 8, 1, N, K, None), "strided")
    torch.cuda.synchronize()
    assert np.array_equal(bits(ypad)[0, :N], bits(ys[2]).reshape(-1))
    assert np.all(np.isnan(ypad[0, N:].float().cpu().numpy()))         # nothing past N written


@pytest.mark.parametrize("ks", [1, 2, 4])
@pytest.mark.parametrize("t", [1, 2, 4])
@pytest.mark.parametrize("p", [2, 3, 4])
def test_gemv_every_schedule(ks, t, p):
    """The multi-row GEMV kernel (M = 2 and, with tuning knob gemv.multirow = 1, M = 1): every
    (K-split waves, rows per wave, chunks per lane) instantiation with x from LDS and from
    global memory, against the oracle: K beyond one LDS window (K = 20000 -> 1250 chunks > the
    1024-chunk window), slices longer than one batch (K = 12544 at ks = 1), short K (one partial
    chunk group) and N not a multiple of the rows per workgroup."""
    _lib.tuning_set("gemv.multirow", 1)
    _lib.tuning_set("gemv.ks", ks)
    _lib.tuning_set("gemv.t", t)
    _lib.tuning_set("gemv.p", p)
    for xg in (0, 1):
        _lib.tuning_set("gemv.xg", xg)
        for N, K in [(1000, 3136), (37, 20000), (130, 16), (67, 48), (300, 12544)]:
            announce("gemv_schedule", ks, t, p, xg, N, K)
            x, w, s = _case(N, K, 7 * N + K, scales="log_uniform")
            y = bits(ops.gemv_fp8(x_to_dev(x), w_to_dev(w), s_to_dev(s)))
            assert_parity(y, oracle_bits(x, w, s), f"ks={ks} t={t} p={p} xg={xg} N={N} K={K}", per_row_scales=True)


# ------------------------------------------------------------------------------- properties
def test_row_slices_match_full_call():
    """Mamba-style in_proj slices (mamba_block.cuh:476-481): offset W/s/y pointers give the
    same rows as the full call, bit for bit (same schedule forced)."""
    N, K = synth.MAMBA_IN, 3136
    announce("row_slices", N, K)
    x, w, s = _case(N, K, 4242, scales="log_uniform")
    xd, wd, sd = x_to_dev(x), w_to_dev(w), s_to_dev(s)
    _lib.tuning_set("gemv.ks", 1)
    full = torch.empty((1, N), dtype=torch.bfloat16, device=DEV)
    L = _lib.lib()
    _lib.check(L.nmi_linear_fp8_w8a16(xd.data_ptr(), K, wd.data_ptr(), K, sd.data_ptr(),
                                      full.data_ptr(), N, 1, N, K, None), "full")
    sliced = torch.full((1, N), float("nan"), dtype=torch.bfloat16, device=DEV)
    for r0, r1 in [(0, 7680), (7680, 14600), (14600, N)]:
        _lib.check(L.nmi_linear_fp8_w8a16(xd.data_ptr(), K, wd.data_ptr() + r0 * K, K,
                                          sd.data_ptr() + 4 * r0, sliced.data_ptr() + 2 * r0, N,
                                          1, r1 - r0, K, None), "slice")
    torch.cuda.synchronize()
    assert np.array_equal(bits(full), bits(sliced))
    assert_parity(bits(full)[0], oracle_bits(x, w, s), "in_proj full", per_row_scales=True)


def test_power_of_two_linearity_full_size():
    """y(2x) == 2 y(x) and y with 4s == 4 y, bit for bit, at config 0's full size."""
    N, K = 12544, 3136
    announce("linearity", N, K)
    x, w, s = _case(N, K, 99)
    xd, wd, sd = x_to_dev(x), w_to_dev(w), s_to_dev(s)
    y = ops.gemv_fp8(xd, wd, sd).float()
    y2 = ops.gemv_fp8((xd.float() * 2).to(torch.bfloat16), wd, sd).float()
    y4 = ops.gemv_fp8(xd, wd, sd * 4).float()
    assert torch.equal(y2, 2 * y) and torch.equal(y4, 4 * y)


def test_deterministic_and_zero_input():
    N, K = 5120, 3136
    announce("determinism", N, K)
    x, w, s = _case(N, K, 5)
    xd, wd, sd = x_to_dev(x), w_to_dev(w), s_to_dev(s)
    a, b = bits(ops.gemv_fp8(xd, wd, sd)), bits(ops.gemv_fp8(xd, wd, sd))
    assert np.array_equal(a, b)
    z = bits(ops.gemv_fp8(torch.zeros_like(xd), wd, sd))
    assert np.all(z == 0)
