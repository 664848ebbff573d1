"""Pin the Mamba-2 decode oracle (oracle/mamba.py): decode steps from a zero state against the
sequence (semiseparable) form of the SSD, the conv step against torch's F.conv1d with causal
padding, softplus against torch's, the gated norm against a float32 torch restatement of HF's
gated RMSNorm and a closed form; planted mistakes in the oracle are caught by these checks."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import block, linear, mamba

F32 = np.float32


def bf16(v):
    return linear.bf16_rne(np.asarray(v, F32))


def val(b):
    return linear.bf16_to_f32(b).astype(np.float64)


def _seq(T, H, P, G, N, seed):
    rng = np.random.default_rng(seed)
    x = bf16(rng.standard_normal((T, H * P)))
    Bm = bf16(rng.standard_normal((T, G * N)) * 0.5)
    Cm = bf16(rng.standard_normal((T, G * N)) * 0.5)
    dt = bf16(rng.standard_normal((T, H)) - 1.0)
    A_log = rng.uniform(-1.0, 1.5, H).astype(F32)
    D = rng.standard_normal(H).astype(F32)
    dt_bias = (0.1 * rng.standard_normal(H)).astype(F32)
    return x, Bm, Cm, dt, A_log, D, dt_bias


def _run_decode(x, Bm, Cm, dt, A_log, D, dt_bias, H, P, G, N, **kw):
    st = np.zeros((1, H, P, N), F32)
    ys = []
    for t in range(x.shape[0]):
        y, st = mamba.ssm_step(x[t:t + 1], Bm[t:t + 1], Cm[t:t + 1], dt[t:t + 1], A_log, D, dt_bias, st, G, **kw)
        ys.append(y[0])
    return np.stack(ys), st


@pytest.mark.parametrize("H,P,G,N", [(8, 4, 2, 16), (6, 3, 3, 8), (4, 5, 1, 32)])
def test_decode_steps_match_the_sequence_form(H, P, G, N):
    T = 12
    x, Bm, Cm, dt, A_log, D, dt_bias = _seq(T, H, P, G, N, seed=H * 100 + P)
    ys, _ = _run_decode(x, Bm, Cm, dt, A_log, D, dt_bias, H, P, G, N)
    dts = mamba.softplus_ref(val(dt) + dt_bias.astype(np.float64)[None, :])
    ref = mamba.ssd_quadratic(val(x).reshape(T, H, P), val(Bm).reshape(T, G, N), val(Cm).reshape(T, G, N), dts,
                              A_log, D, G)
    ref_bits = block.bf16_round_exact(ref.reshape(T, H * P))
    r = linear.parity(ys, ref_bits)
    assert r["ok"] and r["n_diff"] <= 2, r          # float32 states vs float64: rare one-ulp flips


def test_softplus_matches_torch_and_cutoffs():
    v = np.linspace(-19.99, 19.99, 4001)
    np.testing.assert_allclose(mamba.softplus_ref(v), F.softplus(torch.from_numpy(v)).numpy(), rtol=1e-14, atol=1e-15)
    assert (mamba.softplus_ref(np.array([-20.5, -100.0])) == 0).all()
    assert (mamba.softplus_ref(np.array([20.5, 300.0])) == np.array([20.5, 300.0])).all()


def test_conv_steps_match_causal_conv1d():
    C, T = 24, 9
    rng = np.random.default_rng(3)
    w = rng.standard_normal((C, 4)).astype(F32) * 0.5
    b = rng.standard_normal(C).astype(F32) * 0.1
    xs = bf16(rng.standard_normal((T, C)))
    st = np.zeros((1, C, 3), F32)
    outs = []
    for t in range(T):
        o, st = mamba.conv_step(xs[t:t + 1], w, b, st)
        outs.append(o[0])
    xt = torch.from_numpy(val(xs).T[None])                          # [1, C, T]
    ref = F.conv1d(xt, torch.from_numpy(w.astype(np.float64))[:, None, :], torch.from_numpy(b.astype(np.float64)),
                   padding=3, groups=C)[0, :, :T].T
    ref_bits = block.bf16_round_exact(F.silu(ref).numpy())
    assert (np.stack(outs) != ref_bits).sum() <= 1
    assert np.array_equal(st[0], val(xs[-3:]).T.astype(F32))        # the last three inputs, oldest first


def _hf_gated(y, z, w, G, eps):
    yt, zt = torch.from_numpy(val(y).astype(F32)), torch.from_numpy(val(z).astype(F32))
    u = yt * F.silu(zt)
    ug = u.reshape(*u.shape[:-1], G, -1)
    r = torch.rsqrt(ug.pow(2).mean(-1, keepdim=True) + eps)
    return ((ug * r).reshape(u.shape) * torch.from_numpy(w)).numpy()


def test_gated_norm_matches_hf_and_closed_form():
    rng = np.random.default_rng(4)
    y, z = bf16(rng.standard_normal((2, 96))), bf16(rng.standard_normal((2, 96)))
    w = (1 + 0.1 * rng.standard_normal(96)).astype(F32)
    got = val(mamba.gated_rmsnorm(y, z, w, 4))
    ref = _hf_gated(y, z, w, 4, 1e-5)
    np.testing.assert_allclose(got, ref, rtol=8e-3, atol=1e-6)      # one bf16 rounding
    # closed form: u constant a over a group, eps = 0 -> out = sign(a) w
    yc = bf16(np.full((1, 16), 3.0))
    zc = bf16(np.full((1, 16), 40.0))                                # silu(40) = 40 to float64 precision
    out = val(mamba.gated_rmsnorm(yc, zc, np.full(16, 0.5, F32), 2, eps=0.0))
    assert np.all(out == 0.5)


# --------------------------------------------------------------------------------------
# planted mistakes
# --------------------------------------------------------------------------------------
def test_planted_wrong_group_mapping_is_caught():
    H, P, G, N, T = 8, 4, 2, 16, 6
    x, Bm, Cm, dt, A_log, D, dt_bias = _seq(T, H, P, G, N, seed=5)
    ys, _ = _run_decode(x, Bm, Cm, dt, A_log, D, dt_bias, H, P, G, N, group_of=lambda h, H, G: h % G)
    dts = mamba.softplus_ref(val(dt) + dt_bias.astype(np.float64)[None, :])
    ref = mamba.ssd_quadratic(val(x).reshape(T, H, P), val(Bm).reshape(T, G, N), val(Cm).reshape(T, G, N), dts,
                              A_log, D, G)
    assert not linear.parity(ys, block.bf16_round_exact(ref.reshape(T, H * P)))["ok"]


def test_planted_decay_after_input_is_caught():
    H, P, G, N, T = 4, 4, 2, 8, 8
    x, Bm, Cm, dt, A_log, D, dt_bias = _seq(T, H, P, G, N, seed=6)
    dts = mamba.softplus_ref(val(dt) + dt_bias.astype(np.float64)[None, :])
    ref = mamba.ssd_quadratic(val(x).reshape(T, H, P), val(Bm).reshape(T, G, N), val(Cm).reshape(T, G, N), dts,
                              A_log, D, G)
    # the wrong recurrence S = (S + dt B x) dA, restated here
    A = -np.exp(A_log.astype(np.float64))
    S = np.zeros((H, P, N))
    g = np.arange(H) // (H // G)
    wrong = []
    for t in range(T):
        Bh, Ch = val(Bm[t]).reshape(G, N)[g], val(Cm[t]).reshape(G, N)[g]
        xt = val(x[t]).reshape(H, P)
        S = (S + (dts[t][:, None, None] * Bh[:, None, :]) * xt[:, :, None]) * np.exp(dts[t] * A)[:, None, None]
        wrong.append((S * Ch[:, None, :]).sum(-1) + D[:, None] * xt)
    assert not np.allclose(np.stack(wrong), ref, rtol=1e-3, atol=1e-3)


def test_planted_gate_without_silu_is_caught():
    """u = y * z instead of y * silu(z), restated here: the HF comparison above rejects it."""
    rng = np.random.default_rng(7)
    y, z = bf16(rng.standard_normal((1, 64))), bf16(rng.standard_normal((1, 64)))
    w = np.ones(64, F32)
    u = (val(y) * val(z)).reshape(1, 2, 32)
    wrong = (u / np.sqrt((u ** 2).mean(-1, keepdims=True) + 1e-5)).reshape(1, 64)
    assert not np.allclose(wrong, _hf_gated(y, z, w, 2, 1e-5), rtol=8e-3, atol=1e-6)
    assert np.allclose(val(mamba.gated_rmsnorm(y, z, w, 2)), _hf_gated(y, z, w, 2, 1e-5), rtol=8e-3, atol=1e-6)


# --------------------------------------------------------------------------------------
# the block
# --------------------------------------------------------------------------------------
def test_block_matches_a_float32_torch_step():
    H, P, G, N, hidden = 8, 8, 2, 16, 64
    inter, conv_dim = H * P, H * P + 2 * G * N
    proj_n = inter + conv_dim + H
    rng = np.random.default_rng(8)

    def wq(rows, cols):
        wf = rng.standard_normal((rows, cols)).astype(F32) * 0.1
        s = np.full(rows, np.abs(wf).max() / 448, F32)
        codes = torch.from_numpy(wf / s[:, None]).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        return codes, s

    x = bf16(rng.standard_normal((1, hidden)))
    nw = (1 + 0.1 * rng.standard_normal(hidden)).astype(F32)
    inw, outw = wq(proj_n, hidden), wq(hidden, inter)
    conv_w = rng.standard_normal((conv_dim, 4)).astype(F32) * 0.3
    conv_b = rng.standard_normal(conv_dim).astype(F32) * 0.1
    A_log = rng.uniform(-1, 1, H).astype(F32)
    D = rng.standard_normal(H).astype(F32)
    dt_bias = rng.standard_normal(H).astype(F32) * 0.1
    gw = (1 + 0.1 * rng.standard_normal(inter)).astype(F32)
    cs = rng.standard_normal((1, conv_dim, 3)).astype(F32)
    ss = rng.standard_normal((1, H, P, N)).astype(F32) * 0.1
    out, cs2, ss2 = mamba.mamba_decode_block_fp8(x, nw, *inw, conv_w, conv_b, A_log, D, dt_bias, gw, *outw, cs, ss,
                                                  H, P, G, N)

    t = lambda a: torch.from_numpy(np.asarray(a, F32))  # noqa: E731
    xt = t(val(x))
    h = xt * torch.rsqrt(xt.pow(2).mean(-1, keepdim=True) + 1e-5) * t(nw)
    proj = F.linear(h, t(linear.dequant_f32(*inw)))[0]
    z, xbc, dtr = proj[:inter], proj[inter:inter + conv_dim], proj[inter + conv_dim:]
    conv = t(conv_b) + (t(conv_w)[:, :3] * t(cs[0])).sum(-1) + t(conv_w)[:, 3] * xbc
    xc = F.silu(conv)
    xs, Bv, Cv = xc[:inter].view(H, P), xc[inter:inter + G * N].view(G, N), xc[inter + G * N:].view(G, N)
    dts = F.softplus(dtr + t(dt_bias))
    g = torch.arange(H) // (H // G)
    S = t(ss[0]) * torch.exp(-torch.exp(t(A_log)) * dts)[:, None, None] + (dts[:, None, None] * Bv[g][:, None, :]) * \
        xs[:, :, None]
    y = (S * Cv[g][:, None, :]).sum(-1) + t(D)[:, None] * xs
    u = (y.reshape(-1) * F.silu(z)).view(G, -1)
    gn = (u * torch.rsqrt(u.pow(2).mean(-1, keepdim=True) + 1e-5)).reshape(-1) * t(gw)
    ref = (xt[0] + F.linear(gn, t(linear.dequant_f32(*outw)))).numpy()
    rel = np.linalg.norm(val(out)[0] - ref) / np.linalg.norm(ref)
    assert rel < 2e-2, rel
    np.testing.assert_allclose(ss2[0], S.numpy(), rtol=3e-2, atol=3e-3)
    assert np.array_equal(cs2[0, :, :2], cs[0, :, 1:])


def test_forward_block_continues_like_decode_steps():
    """The prefill block over S tokens leaves the states S decode steps from zero would: its
    final states equal those of the decode oracle run token by token, and its outputs equal the
    decode outputs of each token (the block is per-token at decode, per-sequence at prefill)."""
    H, P, G, N, hidden = 4, 8, 2, 16, 64
    inter, conv_dim = H * P, H * P + 2 * G * N
    rng = np.random.default_rng(9)

    def wq(rows, cols):
        wf = rng.standard_normal((rows, cols)).astype(F32) * 0.1
        s = np.full(rows, np.abs(wf).max() / 448, F32)
        codes = torch.from_numpy(wf / s[:, None]).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        return codes, s

    S = 7
    x = bf16(rng.standard_normal((S, hidden)))
    nw = (1 + 0.1 * rng.standard_normal(hidden)).astype(F32)
    inw, outw = wq(inter + conv_dim + H, hidden), wq(hidden, inter)
    prm = (rng.standard_normal((conv_dim, 4)).astype(F32) * 0.3, rng.standard_normal(conv_dim).astype(F32) * 0.1,
           rng.uniform(-1, 1, H).astype(F32), rng.standard_normal(H).astype(F32),
           rng.standard_normal(H).astype(F32) * 0.1, (1 + 0.1 * rng.standard_normal(inter)).astype(F32))
    out, cs, ss = mamba.mamba_forward_block_fp8(x, nw, *inw, *prm, *outw, H, P, G, N)
    cs_d = np.zeros((1, conv_dim, 3), F32)
    ss_d = np.zeros((1, H, P, N), F32)
    for t in range(S):
        o, cs_d, ss_d = mamba.mamba_decode_block_fp8(x[t:t + 1], nw, *inw, *prm, *outw, cs_d, ss_d, H, P, G, N)
        assert np.array_equal(o[0], out[t]), t
    assert np.array_equal(cs, cs_d) and np.array_equal(ss, ss_d)
