"""CPU oracle for nemotron_infer's Mamba-2 block (decode and prefill) -- TEST INFRASTRUCTURE ONLY.

Restates on the CPU what the reference's Mamba block computes, so that the HIP kernels can be
checked against it.  Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg use it.  bf16 tensors are uint16 bit patterns, as in ``oracle.linear``;
every step is computed in float64 and rounded once where the reference rounds (to bf16 for
activations, float32 for states).

* ``conv_step``   -- ops/mamba2/causal_conv1d.cuh:391-430 (decode, bf16 I/O): for channel c,
  v = b[c] + sum_k w[c, k] s[c, k] + w[c, 3] x[c] over the state [s0, s1, s2], out =
  bf16(silu(v)), the state becomes [s1, s2, x[c]].
* ``ssm_step``    -- ops/mamba2/ssm.cuh:46-101: dt = softplus(dt_raw + dt_bias) with the
  reference's cut-offs (identity above 20, 0 below -20), clamped to [0, FLT_MAX];
  dA = exp(-exp(A_log) dt); S = S dA + dt B x (float32 state); y = bf16(S . C + D x), B and C of
  group h // (H / G).
* ``gated_rmsnorm`` -- ops/reduce.cuh:383-480 (bf16): u = y silu(z); per group of INTER / G
  values r = 1 / sqrt(mean(u^2) + eps); out = bf16(u r w).  (The reference takes r with rsqrtf;
  this oracle and the kernel take the correctly rounded value.)
* ``mamba_decode_block_fp8`` -- model/mamba_block.cuh:436-515: rmsnorm -> in_proj (one linear
  over all rows: [z | xBC | dt]) -> conv_step -> ssm_step on x | B | C -> gated_rmsnorm(y, z) ->
  out_proj -> residual add; returns out and the new states.
* ``mamba_forward_block_fp8`` -- model/mamba_block.cuh:346-425 for one sequence of S tokens on
  bf16 activations (the reference quantizes them to e4m3 into its GEMMs; this build does not):
  rmsnorm -> in_proj -> ``conv_step`` token by token from a zero state (the prefill conv,
  causal_conv1d.cuh:30-90) -> ``ssm_step`` token by token from a zero state (the recurrence the
  chunked scan ssd_scan_chunked.cuh implements) -> gated_rmsnorm -> out_proj -> residual add;
  returns out and the final states.
* ``ssd_quadratic`` -- the definition the recurrence implements (the semiseparable form of
  tools/ref_full_model.py:66-118's chunked SSD, with zero initial state):
  y_t = sum_{s <= t} (C_t . B_s) exp(A sum_{s < r <= t} dt_r) dt_s x_s + D x_t, in float64.

Pinned in tests/test_oracle_mamba.py: t decode steps from zero state against ``ssd_quadratic``
(a different algorithm: no recurrence) and against torch's ``F.conv1d`` with causal padding
for the conv; the gated norm against torch's float32 restatement of HF's gated RMSNorm
(ref_full_model.py:62-66) and closed forms; planted mistakes (a wrong group mapping, the decay
applied after the input, silu missing from the gate) are caught; the prefill block against
token-by-token decode (outputs and final states identical).
"""
from __future__ import annotations

import numpy as np

from . import block, linear

F32 = np.float32
FLT_MAX = float(np.finfo(np.float32).max)


def _f64(bits) -> np.ndarray:
    return linear.bf16_to_f32(np.asarray(bits, np.uint16)).astype(np.float64)


def _silu(v):
    return v / (1.0 + np.exp(-v))


def conv_step(xbc_bits, conv_w, conv_b, conv_state):
    """xbc [B, C] bf16 bits, conv_w [C, 4], conv_b [C], conv_state [B, C, 3] float32 ->
    (out [B, C] bf16 bits, new state [B, C, 3] float32)."""
    x = _f64(np.atleast_2d(xbc_bits))
    w = np.asarray(conv_w, np.float64)
    s = np.asarray(conv_state, np.float64)
    v = np.asarray(conv_b, np.float64)[None, :] + (w[None, :, :3] * s).sum(-1) + w[None, :, 3] * x
    out = block.bf16_round_exact(_silu(v))
    new = np.concatenate([s[:, :, 1:], x[:, :, None]], axis=2).astype(F32)
    return out, new


def softplus_ref(dt):
    """The reference's softplus with cut-offs, then the clamp to [0, FLT_MAX]."""
    dt = np.asarray(dt, np.float64)
    with np.errstate(over="ignore"):
        sp = np.where(dt > 20.0, dt, np.where(dt < -20.0, 0.0, np.log1p(np.exp(np.minimum(dt, 20.0)))))
    return np.clip(sp, 0.0, FLT_MAX)


def ssm_step(x_bits, B_bits, C_bits, dt_bits, A_log, D, dt_bias, ssm_state, G, group_of=None):
    """x [Bt, H*P], B and C [Bt, G*N], dt [Bt, H] (bf16 bits), ssm_state [Bt, H, P, N] float32 ->
    (y [Bt, H*P] bf16 bits, new state float32).  ``group_of(h, H, G)`` maps a head to its group
    (default h // (H / G))."""
    st = np.asarray(ssm_state, np.float64)
    Bt, H, P, N = st.shape
    x = _f64(np.atleast_2d(x_bits)).reshape(Bt, H, P)
    Bm = _f64(np.atleast_2d(B_bits)).reshape(Bt, G, N)
    Cm = _f64(np.atleast_2d(C_bits)).reshape(Bt, G, N)
    dt = softplus_ref(_f64(np.atleast_2d(dt_bits)) + np.asarray(dt_bias, np.float64)[None, :])
    if group_of is None:
        group_of = lambda h, H, G: h // (H // G)  # noqa: E731
    g = np.array([group_of(h, H, G) for h in range(H)])
    dA = np.exp(-np.exp(np.asarray(A_log, np.float64))[None, :] * dt)              # [Bt, H]
    Bh, Ch = Bm[:, g, :], Cm[:, g, :]                                               # [Bt, H, N]
    new = st * dA[:, :, None, None] + (dt[:, :, None, None] * Bh[:, :, None, :]) * x[:, :, :, None]
    y = (new * Ch[:, :, None, :]).sum(-1) + np.asarray(D, np.float64)[None, :, None] * x
    return block.bf16_round_exact(y.reshape(Bt, H * P)), new.astype(F32)


def gated_rmsnorm(y_bits, z_bits, w, G, eps=1e-5):
    """y, z [Bt, INTER] bf16 bits, w [INTER] -> [Bt, INTER] bf16 bits."""
    y = _f64(np.atleast_2d(y_bits))
    z = _f64(np.atleast_2d(z_bits))
    u = y * _silu(z)
    Bt, n = u.shape
    ug = u.reshape(Bt, G, n // G)
    r = 1.0 / np.sqrt((ug ** 2).mean(-1, keepdims=True) + eps)
    return block.bf16_round_exact((ug * r).reshape(Bt, n) * np.asarray(w, np.float64)[None, :])


def split_proj(proj_bits, H, P, G, N):
    inter = H * P
    conv_dim = inter + 2 * G * N
    p = np.atleast_2d(proj_bits)
    return p[:, :inter], p[:, inter:inter + conv_dim], p[:, inter + conv_dim:inter + conv_dim + H]


def mixer_step(proj_bits, conv_w, conv_b, A_log, D, dt_bias, gnorm_w, conv_state, ssm_state, H, P, G, N,
               eps=1e-5):
    """The mixer between the projections: (y, g, new conv state, new ssm state, conv output)."""
    z, xbc, dt = split_proj(proj_bits, H, P, G, N)
    xc, conv_new = conv_step(xbc, conv_w, conv_b, conv_state)
    inter = H * P
    y, ssm_new = ssm_step(xc[:, :inter], xc[:, inter:inter + G * N], xc[:, inter + G * N:], dt, A_log, D,
                          dt_bias, ssm_state, G)
    g = gated_rmsnorm(y, z, gnorm_w, G, eps)
    return y, g, conv_new, ssm_new, xc


def mamba_decode_block_fp8(x_bits, norm_w, in_codes, in_s, conv_w, conv_b, A_log, D, dt_bias, gnorm_w, out_codes,
                           out_s, conv_state, ssm_state, H, P, G, N, eps=1e-5, return_stages=False):
    """The block at decode.  Returns (out, conv_state, ssm_state) (+ the stages)."""
    x_bits = np.atleast_2d(np.asarray(x_bits, np.uint16))
    h = block.rmsnorm_bf16(x_bits, norm_w, eps)
    proj = linear.linear_fp8_w8a16(h, in_codes, in_s)
    y, g, conv_new, ssm_new, xc = mixer_step(proj, conv_w, conv_b, A_log, D, dt_bias, gnorm_w, conv_state,
                                              ssm_state, H, P, G, N, eps)
    mix = linear.linear_fp8_w8a16(g, out_codes, out_s)
    out = block.add_bf16(x_bits, mix)
    if return_stages:
        return out, conv_new, ssm_new, dict(normed=h, proj=proj, xconv=xc, y=y, g=g, mix=mix)
    return out, conv_new, ssm_new


def ssd_quadratic(x, Bm, Cm, dt, A_log, D, G):
    """Sequence form, float64, zero initial state: x [T, H, P], Bm and Cm [T, G, N], dt [T, H]
    (already softplus'ed), A_log, D [H] -> y [T, H, P]."""
    T, H, P = x.shape
    A = -np.exp(np.asarray(A_log, np.float64))
    g = np.arange(H) // (H // G)
    cum = np.cumsum(dt * A[None, :], axis=0)                   # [T, H]: sum_{r <= t} dt_r A
    y = np.zeros((T, H, P))
    for t in range(T):
        for s in range(t + 1):
            decay = np.exp(cum[t] - cum[s])                    # exp(A sum_{s < r <= t} dt_r)
            cb = (Cm[t][g] * Bm[s][g]).sum(-1)                 # [H]
            y[t] += (cb * decay * dt[s])[:, None] * x[s]
        y[t] += np.asarray(D, np.float64)[:, None] * x[t]
    return y


def mamba_forward_block_fp8(x_bits, norm_w, in_codes, in_s, conv_w, conv_b, A_log, D, dt_bias, gnorm_w, out_codes,
                            out_s, H, P, G, N, eps=1e-5, return_stages=False):
    """One sequence x [S, hidden] bf16 bits.  Returns (out, conv_state [1, C, 3], ssm_state
    [1, H, P, N]) (+ the stages)."""
    x_bits = np.atleast_2d(np.asarray(x_bits, np.uint16))
    S = x_bits.shape[0]
    h = block.rmsnorm_bf16(x_bits, norm_w, eps)
    proj = linear.linear_fp8_w8a16(h, in_codes, in_s)
    z, xbc, dt = split_proj(proj, H, P, G, N)
    inter = H * P
    conv_dim = xbc.shape[1]
    cs = np.zeros((1, conv_dim, 3), F32)
    ss = np.zeros((1, H, P, N), F32)
    xc = np.zeros_like(xbc)
    y = np.zeros((S, inter), np.uint16)
    for t in range(S):
        o, cs = conv_step(xbc[t:t + 1], conv_w, conv_b, cs)
        xc[t] = o[0]
        yt, ss = ssm_step(o[:, :inter], o[:, inter:inter + G * N], o[:, inter + G * N:], dt[t:t + 1], A_log, D,
                          dt_bias, ss, G)
        y[t] = yt[0]
    g = gated_rmsnorm(y, z, gnorm_w, G, eps)
    mix = linear.linear_fp8_w8a16(g, out_codes, out_s)
    out = block.add_bf16(x_bits, mix)
    if return_stages:
        return out, cs, ss, dict(normed=h, proj=proj, xconv=xc, y=y, g=g, mix=mix)
    return out, cs, ss
