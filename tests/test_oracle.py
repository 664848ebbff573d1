"""Pin the CPU oracle (oracle/) against the golden fixtures, torch's own float8 codec and
closed-form facts -- CPU only.

Each check compares the oracle with something computed independently of it: the fixtures
are written by tests/golden/gen_golden.py from torch's float8_e4m3fn cast/decode and float64
brute force, never from oracle/.  The last group plants mistakes in (copies of) the oracle and
shows that the fixtures catch them.
"""
import hashlib
import os

import numpy as np
import pytest
import torch

from oracle import cref, e4m3, linear
from tests.conftest import GOLDEN, load_golden

FIXTURES = ["kat_gemv_n64_k3136", "tiny_m4_n8_k16", "ragged_m3_n37_k208",
            "skinny_m16_n48_k3136", "special_nan_zero"]


def test_fixture_checksums():
    for line in open(os.path.join(GOLDEN, "SHA256SUMS")):
        h, name = line.split()
        assert hashlib.sha256(open(os.path.join(GOLDEN, name), "rb").read()).hexdigest() == h, name


# ---------------------------------------------------------------------------- decode table
def test_lut_matches_fixture_bitwise():
    ref = load_golden("e4m3_lut")["lut_bits"]
    for lut in (e4m3.decode_lut(), cref.e4m3_lut()):
        bits = lut.view(np.uint32)
        nan = np.isnan(lut)
        assert list(np.nonzero(nan)[0]) == [0x7F, 0xFF]
        assert np.array_equal(bits[~nan], ref[~nan])
        assert np.isnan(ref.view(np.float32)[nan]).all()


def test_lut_spec_points():
    lut = e4m3.decode_lut()
    assert lut[0x7E] == 448.0 and lut[0xFE] == -448.0           # max finite
    assert lut[0x01] == 2.0 ** -9 and lut[0x07] == 7 * 2.0 ** -9  # subnormals
    assert lut[0x08] == 2.0 ** -6                                # min normal
    assert lut[0x38] == 1.0 and lut[0x40] == 2.0                 # bias 7
    assert lut[0x80] == 0.0 and np.signbit(lut[0x80])            # -0
    assert np.all(np.diff(lut[:0x7F]) > 0)                       # monotone magnitudes


# ---------------------------------------------------------------------------- quantizer
def _sweep_values():
    rng = np.random.default_rng(7)
    mags = e4m3.decode_lut()[:0x7F].astype(np.float64)
    mids = (mags[:-1] + mags[1:]) / 2                           # exact ties
    vals = np.concatenate([
        mags, mids, np.nextafter(mids.astype(np.float32), np.float32(0)),
        np.nextafter(mids.astype(np.float32), np.float32(1000)),
        rng.uniform(-448, 448, 200_000), rng.standard_normal(50_000) * 1e-2,
        rng.standard_normal(50_000) * 3e-3,
    ]).astype(np.float32)
    vals = np.clip(vals, -448, 448)
    return np.concatenate([vals, -vals])


def test_quantize_rne_matches_torch_cast():
    v = _sweep_values()
    mine = e4m3.quantize_rne(v)
    theirs = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(mine, theirs)


def test_quantize_rejects_unclamped():
    with pytest.raises(ValueError):
        e4m3.quantize_rne(np.array([449.0], np.float32))


def test_perrow_quantizer_reproduces_fixture_codes():
    for name in ("kat_gemv_n64_k3136", "tiny_m4_n8_k16"):
        g = load_golden(name)
        codes, s = e4m3.quant_weight_perrow(g["w_f32"])
        assert np.array_equal(codes, g["w_codes"]), name
        assert np.array_equal(s.view(np.uint32), g["w_scale"].view(np.uint32)), name


# ---------------------------------------------------------------------------- bf16 rounding
def test_bf16_rne_matches_torch_and_c():
    rng = np.random.default_rng(3)
    f = np.concatenate([rng.standard_normal(100_000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 100_000),
                        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1.00390625, 1.01171875, 3.4e38],
                                 np.float32)]).astype(np.float32)
    # exact ties: bf16 values with bit 15 set below them
    ties = ((rng.integers(0, 2**16, 1000, dtype=np.uint32) << 16) | 0x8000).view(np.float32)
    f = np.concatenate([f, ties])
    t = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    mine = linear.bf16_rne(f)
    c = cref.bf16_rne(f)
    nan = np.isnan(f)
    assert np.array_equal(mine[~nan], t[~nan]) and np.array_equal(c[~nan], t[~nan])
    assert np.all((mine[nan] & 0x7FFF) > 0x7F80) and np.all((c[nan] & 0x7FFF) > 0x7F80)


# ---------------------------------------------------------------------------- linear oracles
@pytest.mark.parametrize("name", FIXTURES)
def test_torch_oracle_matches_fp64_fixture(name):
    g = load_golden(name)
    y = linear.linear_fp8_w8a16(g["x_bf16"], g["w_codes"], g["w_scale"])
    ref = linear.bf16_rne(g["y_f64"].astype(np.float32))
    r = linear.parity(y, ref, ulp_tol=1.0, rel_l2_tol=1e-3)
    assert r["ok"], r


@pytest.mark.parametrize("name", FIXTURES)
def test_c_sequential_oracle_matches_fp64_fixture(name):
    g = load_golden(name)
    y32 = cref.gemv_fp8_seq(g["x_bf16"], g["w_codes"], g["w_scale"])
    y64 = g["y_f64"]
    # float32 sequential summation bound: |err| <= K * 2^-24 * sum|w x| * s  (+ final product)
    x = linear.bf16_to_f32(g["x_bf16"]).astype(np.float64)
    w = e4m3.decode_lut().astype(np.float64)[g["w_codes"]]
    absdot = np.abs(x) @ np.abs(np.nan_to_num(w)).T * g["w_scale"].astype(np.float64)[None, :]
    K = g["w_codes"].shape[1]
    bound = (K + 2) * 2.0 ** -24 * absdot + 1e-30
    fin = np.isfinite(y64)
    assert np.array_equal(np.isnan(y32), np.isnan(y64))
    assert np.all(np.abs(y32[fin] - y64[fin]) <= bound[fin])


def test_numpy_sequential_equals_c_sequential():
    g = load_golden("ragged_m3_n37_k208")
    for m in range(g["x_bf16"].shape[0]):
        a = linear.gemv_fp32_sequential(g["x_bf16"][m], g["w_codes"], g["w_scale"])
        b = cref.gemv_fp8_seq(g["x_bf16"][m], g["w_codes"], g["w_scale"])
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_kat_within_reference_tolerance():
    """GemvFP8Test.MatchesReference tolerance (test_gemm.cu:572-576): |y - ref| <= max(0.02, 2%)."""
    g = load_golden("kat_gemv_n64_k3136")
    y = linear.bf16_to_f32(linear.linear_fp8_w8a16(g["x_bf16"], g["w_codes"], g["w_scale"]))[0]
    ref = cref.gemv_fp8_seq(g["x_bf16"], g["w_codes"], g["w_scale"])[0]
    assert np.all(np.abs(y - ref) <= np.maximum(0.02, 0.02 * np.abs(ref)))


def test_special_values():
    g = load_golden("special_nan_zero")
    y = linear.bf16_to_f32(linear.linear_fp8_w8a16(g["x_bf16"], g["w_codes"], g["w_scale"]))
    assert np.isnan(y[:, 1]).all() and np.isnan(y[:, 2]).all()   # NaN codes propagate
    assert np.all(y[1, [0, 3, 4, 5, 6, 7]] == 0.0)                 # zero activation row
    assert np.all(y[:, 3] == 0.0)                                   # -0 weights


# ---------------------------------------------------------------------------- planted mistakes
def _mutants(x, w, s):
    lut = e4m3.decode_lut()
    xf = linear.bf16_to_f32(x).astype(np.float32)
    yield "dropped scale", xf @ lut[w].T
    yield "transposed operand", (xf @ lut[w.reshape(w.shape[1], w.shape[0]).T].T) * s[None, :] \
        if w.shape[0] != w.shape[1] else None
    yield "wrong sign", -(xf @ lut[w].T) * s[None, :]
    yield "scale by column index", (xf @ lut[w].T) * s[::-1][None, :]
    yield "FNUZ decode (bias 8)", (xf @ (lut[w] * 0.5).T) * s[None, :]
    yield "last k dropped", (xf[:, :-16] @ lut[w][:, :-16].T) * s[None, :]
    yield "bf16-truncated activations", ((xf.view(np.uint32) & 0xFFFE0000).view(np.float32)
                                        @ lut[w].T) * s[None, :]


def test_fixtures_catch_planted_mistakes():
    """Every planted mistake must fail at least one fixture (the KAT alone cannot see a
    scale-index mistake: all its per-row scales are equal, which is why the log-uniform-scale
    fixture exists)."""
    caught = {}
    for name in ("ragged_m3_n37_k208", "skinny_m16_n48_k3136", "kat_gemv_n64_k3136"):
        g = load_golden(name)
        ref = linear.bf16_rne(g["y_f64"].astype(np.float32))
        for label, ybad in _mutants(g["x_bf16"], g["w_codes"], g["w_scale"]):
            if ybad is None:
                continue
            r = linear.parity(linear.bf16_rne(ybad.astype(np.float32)), ref)
            caught[label] = caught.get(label, False) or not r["ok"]
    missed = [k for k, v in caught.items() if not v]
    assert len(caught) == 7 and not missed, f"planted mistakes not caught: {missed}"


# ---------------------------------------------------------------------------- parity gate
def test_parity_gate_allows_isolated_rounding_flip_and_rejects_systematic_ones():
    """A one-ulp flip on the element that dominates ||ref|| passes (float32 summation order can
    put an exact value on either side of a bf16 rounding boundary); truncating instead of
    rounding to nearest even, or a sub-ulp scale error, flips many elements and fails; a
    one-element error of three ulp fails."""
    g = load_golden("skinny_m16_n48_k3136")
    yf = (linear.bf16_to_f32(g["x_bf16"]).astype(np.float64)
          @ e4m3.decode_lut().astype(np.float64)[g["w_codes"]].T) * g["w_scale"].astype(np.float64)
    ref = linear.bf16_rne(yf.astype(np.float32))
    big = np.unravel_index(np.argmax(np.abs(linear.bf16_to_f32(ref))), ref.shape)
    flipped = ref.copy()
    flipped[big] = flipped[big] + 1                       # next bf16 value: one ulp away
    r = linear.parity(flipped, ref)
    assert r["ok"] and r["n_flip"] == 1 and r["rel_l2"] == 0.0
    truncated = (yf.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    assert not linear.parity(truncated, ref)["ok"]       # RNE replaced by truncation
    scaled = linear.bf16_rne((yf * (1 + 2.0 ** -10)).astype(np.float32))
    assert not linear.parity(scaled, ref)["ok"]          # sub-ulp systematic scale error
    wrong = ref.copy()
    wrong[big] = wrong[big] + 3
    assert not linear.parity(wrong, ref)["ok"]
