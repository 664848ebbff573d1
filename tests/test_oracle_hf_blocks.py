"""The attention and Mamba-2 oracles against fixtures restated from the reference's own block
dumps (tools/dump_attention_block.py:20-58, seed 777; tools/dump_mamba_block.py:1-40, seed 1234,
at state size 128), whose expectations are the HF formulas in float64 (tests/golden/gen_golden.py,
which imports nothing from oracle/).

Pins: the fp8 blocks' oracles on the per-row quantized weights (test_attention_block.cu:161-194,
test_mamba_block.cu:190-242 quantize the same way) land near the fp32 HF output, stage by stage --
the e4m3 weights alone put the attention block at rel_l2 0.056 and the Mamba block at 0.044 in
exact arithmetic, so the gates are 0.08 and 0.05 (the reference's own gates are 0.3 and 0.35),
while planted misreadings of the semantics (no causal mask, a wrong GQA or group map, k and v
swapped, the gate after the norm, D or dt_bias left out) land at 0.057-1.3; and the chunked SSD of
the fixture equals the oracle's quadratic (semiseparable) form, two independent formulations, to
float32 precision.
"""
import numpy as np
import pytest

from oracle import attention, block, linear, mamba
from tests.conftest import load_golden

ATTN_TOL = 0.08
MAMBA_TOL = 0.05

import numpy as np
import pytest

from oracle import attention, block, linear, mamba
from tests.conftest import load_golden


def rel_l2(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))


def f32(bits):
    return linear.bf16_to_f32(np.asarray(bits, np.uint16))


def test_attention_oracle_matches_the_hf_recipe():
    g = load_golden("attn_block_h256_q4_kv2_s40")
    out, st = attention.attn_forward_block_fp8(g["x_bf16"], g["norm_w"], g["q_codes"], g["q_scale"], g["k_codes"],
                                               g["k_scale"], g["v_codes"], g["v_scale"], g["o_codes"], g["o_scale"],
                                               n_kv=2, return_stages=True)
    assert rel_l2(f32(st["normed"]), g["normed_f32"]) < 4e-3        # bf16 rounding of the input and output
    assert rel_l2(f32(st["o"]), g["attn_f32"]) < ATTN_TOL
    assert rel_l2(f32(st["attn"]), g["o_f32"]) < ATTN_TOL
    r = rel_l2(f32(out), g["expected_f32"])
    assert r < ATTN_TOL, r


def test_attention_decode_continuation_matches_the_hf_recipe():
    """Prefill the first 39 tokens into the caches, decode token 40 against them (the reference's
    BF16_DecodeMatchHF continuation, test_attention_block.cu:197-240, on the fp8 block).  The
    reference's decode attends the cached positions only (sdpa_decode.cuh:57-180), so the gate is
    against that row of the HF formulas (decode_last_f32); HF's own last row also attends the
    token itself and sits further away."""
    g = load_golden("attn_block_h256_q4_kv2_s40")
    S = g["x_bf16"].shape[0]
    w = [g[k] for k in ("q_codes", "q_scale", "k_codes", "k_scale", "v_codes", "v_scale", "o_codes", "o_scale")]
    _, st = attention.attn_forward_block_fp8(g["x_bf16"][:S - 1], g["norm_w"], *w, n_kv=2, return_stages=True)
    cap = 64
    kc = np.zeros((2, cap, 128), np.uint16)
    vc = np.zeros((2, cap, 128), np.uint16)
    kc[:, :S - 1] = st["k"].reshape(S - 1, 2, 128).transpose(1, 0, 2)
    vc[:, :S - 1] = st["v"].reshape(S - 1, 2, 128).transpose(1, 0, 2)
    out = attention.attn_decode_block_fp8(g["x_bf16"][S - 1:], g["norm_w"], *w, kc, vc, S - 1, n_kv=2)[0]
    r = rel_l2(f32(out), g["decode_last_f32"])
    assert r < ATTN_TOL, r
    assert rel_l2(g["decode_last_f32"], g["expected_f32"][S - 1:]) > 0.02   # the self term the decode leaves out


@pytest.mark.parametrize("mistake", ["not_causal", "gqa_head_mod", "k_v_swapped"])
def test_planted_mistakes_fail_the_hf_attention_fixture(mistake):
    g = load_golden("attn_block_h256_q4_kv2_s40")
    xb = g["x_bf16"]
    S = xb.shape[0]
    h = block.rmsnorm_bf16(xb, g["norm_w"], 1e-5)
    q = linear.linear_fp8_w8a16(h, g["q_codes"], g["q_scale"])
    k = linear.linear_fp8_w8a16(h, g["k_codes"], g["k_scale"])
    v = linear.linear_fp8_w8a16(h, g["v_codes"], g["v_scale"])
    if mistake == "not_causal":
        o = linear.f32_to_bf16_bits(attention.sdpa_prefill_f64(q, k, v, 2, causal=False).astype(np.float32))
    elif mistake == "gqa_head_mod":      # query head h reads KV head h % 2 instead of h // 2
        perm = [0, 2, 1, 3]
        o = attention.sdpa_prefill(q.reshape(S, 4, 128)[:, perm].reshape(S, 512), k, v, 2)
        o = o.reshape(S, 4, 128)[:, perm].reshape(S, 512)
    else:
        o = attention.sdpa_prefill(q, v, k, 2)
    out = block.add_bf16(xb, linear.linear_fp8_w8a16(o, g["o_codes"], g["o_scale"]))
    assert rel_l2(f32(out), g["expected_f32"]) > ATTN_TOL


def _mamba_args(g):
    HID, H, P, N, G = (int(v) for v in g["shape"][:5])
    return (g["norm_w"], g["in_codes"], g["in_scale"], g["conv_w"], g["conv_b"], g["A_log"], g["D"], g["dt_bias"],
            g["gnorm_w"], g["out_codes"], g["out_scale"]), (H, P, G, N)


def test_mamba_fixture_ssd_equals_the_quadratic_form():
    """The fixture's chunked SSD (chunks of 8, state passed between them) against the oracle's
    quadratic form on the same float inputs: two formulations of one function."""
    g = load_golden("mamba_block_h64_h4p16_g2_n128_s24")
    HID, H, P, N, G = (int(v) for v in g["shape"][:5])
    inter = H * P
    xc = g["xbc_conv_f32"].astype(np.float64)
    S = xc.shape[0]
    x = xc[:, :inter].reshape(S, H, P)
    Bm = xc[:, inter:inter + G * N].reshape(S, G, N)
    Cm = xc[:, inter + G * N:].reshape(S, G, N)
    y = mamba.ssd_quadratic(x, Bm, Cm, g["dt_f32"].astype(np.float64), g["A_log"], g["D"], G)
    assert rel_l2(y.reshape(S, inter), g["scan_y_f32"]) < 1e-5


def test_mamba_oracle_matches_the_hf_recipe():
    g = load_golden("mamba_block_h64_h4p16_g2_n128_s24")
    args, (H, P, G, N) = _mamba_args(g)
    out, cs, ss, st = mamba.mamba_forward_block_fp8(g["x_bf16"], *args, H, P, G, N, return_stages=True)
    assert rel_l2(f32(st["xconv"]), g["xbc_conv_f32"]) < MAMBA_TOL
    assert rel_l2(f32(st["y"]), g["scan_y_f32"]) < MAMBA_TOL
    assert rel_l2(f32(st["g"]), g["gnormed_f32"]) < 2 * MAMBA_TOL     # the gate's SiLU doubles the relative error
    assert rel_l2(cs[0], g["conv_state_f32"]) < MAMBA_TOL
    assert rel_l2(ss[0], g["ssm_state_f32"]) < MAMBA_TOL
    r = rel_l2(f32(out), g["expected_f32"])
    assert r < MAMBA_TOL, r


def test_mamba_decode_continuation_matches_the_hf_recipe():
    """Prefill 23 tokens (final states), decode token 24 from them: the HF output's last row."""
    g = load_golden("mamba_block_h64_h4p16_g2_n128_s24")
    args, (H, P, G, N) = _mamba_args(g)
    S = g["x_bf16"].shape[0]
    _, cs, ss = mamba.mamba_forward_block_fp8(g["x_bf16"][:S - 1], *args, H, P, G, N)
    out = mamba.mamba_decode_block_fp8(g["x_bf16"][S - 1:], *args, cs, ss, H, P, G, N)[0]
    r = rel_l2(f32(out), g["expected_f32"][S - 1:])
    assert r < MAMBA_TOL, r


@pytest.mark.parametrize("mistake", ["group_of_head_mod", "gate_after_norm", "no_D", "dt_without_bias"])
def test_planted_mistakes_fail_the_hf_mamba_fixture(mistake):
    """Plausible misreadings of the reference's Mamba semantics, planted in a copy of the oracle's
    pipeline, each move the output far outside the gate."""
    g = load_golden("mamba_block_h64_h4p16_g2_n128_s24")
    args, (H, P, G, N) = _mamba_args(g)
    norm_w, in_c, in_s, conv_w, conv_b, A_log, D, dt_bias, gnorm_w, out_c, out_s = args
    xb = g["x_bf16"]
    S = xb.shape[0]
    inter = H * P
    h = block.rmsnorm_bf16(xb, norm_w, 1e-5)
    proj = linear.linear_fp8_w8a16(h, in_c, in_s)
    z, xbc, dt = mamba.split_proj(proj, H, P, G, N)
    cs = np.zeros((1, xbc.shape[1], 3), np.float32)
    ss = np.zeros((1, H, P, N), np.float32)
    Dm = np.zeros_like(D) if mistake == "no_D" else D
    bias = np.zeros_like(dt_bias) if mistake == "dt_without_bias" else dt_bias
    group_of = (lambda h, H_, G_: h % G_) if mistake == "group_of_head_mod" else None
    y = np.zeros((S, inter), np.uint16)
    for t in range(S):
        o, cs = mamba.conv_step(xbc[t:t + 1], conv_w, conv_b, cs)
        yt, ss = mamba.ssm_step(o[:, :inter], o[:, inter:inter + G * N], o[:, inter + G * N:], dt[t:t + 1], A_log, Dm,
                                bias, ss, G, group_of=group_of)
        y[t] = yt[0]
    if mistake == "gate_after_norm":
        yf = f32(y).astype(np.float64).reshape(S, G, inter // G)
        n = yf / np.sqrt((yf * yf).mean(-1, keepdims=True) + 1e-5)
        zf = f32(z).astype(np.float64)
        gv = linear.f32_to_bf16_bits((n.reshape(S, inter) * gnorm_w * zf / (1 + np.exp(-zf))).astype(np.float32))
    else:
        gv = mamba.gated_rmsnorm(y, z, gnorm_w, G, 1e-5)
    out = block.add_bf16(xb, linear.linear_fp8_w8a16(gv, out_c, out_s))
    assert rel_l2(f32(out), g["expected_f32"]) > MAMBA_TOL
