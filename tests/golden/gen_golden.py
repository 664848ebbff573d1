"""Generate the golden fixtures for the fp8 W8A16 linear path.

Run:  python tests/golden/gen_golden.py      (writes tests/golden/*.npz and SHA256SUMS)

Independence: this script does not import ``oracle/``.  Codes come from torch's own
``float32 -> float8_e4m3fn`` cast, decoded values from torch's own ``float8_e4m3fn ->
float32``, and expected outputs from float64 brute force.  The oracle is then checked
against these files, so a mistake in the oracle's decode table, quantizer or linear shows
up as a mismatch instead of being copied into the expectation.

Inputs follow the reference's known-answer tests where it has them:
* ``kat_gemv_n64_k3136``  -- GemvFP8Test.MatchesReference (tests/ops/test_gemm.cu:538-551):
  x[i] = ((13 i) % 17) * 0.1f - 0.8f -> bf16;  W[i] = ((7 i) % 23) * 0.05f - 0.55f,
  quantized per row (test_gemm.cu:516-529).
* ``tiny_m4_n8_k16``      -- GemmFP8Test.Tiny (test_gemm.cu:310-337): x[i] = (i % 7) * 0.3f
  - 1, W[i] = (i % 11) * 0.2f - 1.1f, per-row weight quant.  The reference quantizes x to
  e4m3 there (W8A8); this build keeps x in bf16 (W8A16), so only the inputs are shared.
Seeded cases cover what those leave open: ragged N and K/16 odd (``ragged_m3_n37_k208``),
skinny M with per-row log-uniform scales (``skinny_m16_n48_k3136``), and special values
(``special_nan_zero``: NaN codes 0x7F/0xFF, -0 codes, subnormal codes, an all-zero x row).

The MLP block fixture ``mlp_block_h64_i256_s8`` follows tools/dump_mlp_block.py:15-53: torch
seed 2024, HIDDEN 64, INTER 256, S 8, EPS 1e-5, the same draws in the same order, and its fp32
HF forward as ``expected_f32`` (the expectation of test_mlp_block.cu:155-185, which quantizes
both weights per row as test_mlp_block.cu:57-70 does and feeds the input as bf16).  It also
holds ``chain_f64``: the block computed in float64 with a bf16 rounding after every step, as
the fp8 block's M == 1 path stores its intermediates (mlp_block.cuh:140-148, 173-175), the
rounding done here on the float64 bit pattern.

The attention block fixture ``attn_block_h256_q4_kv2_s40`` follows
tools/dump_attention_block.py:20-58 exactly: torch seed 777, HIDDEN 256, 4 query heads, 2 KV
heads, head 128, S 40 (more than one KV tile), EPS 1e-5, the same draws in the same order, and
the HF-formula forward (plain RMSNorm, no RoPE, GQA by repeating the KV heads, causal SDPA with
scale 1/sqrt(128), o projection, residual), here in float64, stored as float32 ``expected_f32``
with the intermediates; and ``decode_last_f32``, the last token decoded after a prefill of the
others under the reference's decode contract, whose query attends the cached positions only (its
own k and v are appended after the attention, ops/attention/sdpa_decode.cuh:57-180), unlike the
HF row, which also attends the token itself.  test_attention_block.cu:161-194 quantizes the weights per row
(test_attention_block.cu's up_fp8_perrow) and feeds the input as bf16; the codes and scales of
that quantization are stored too.

The Mamba block fixture ``mamba_block_h64_h4p16_g2_n128_s24`` follows
tools/dump_mamba_block.py:1-40 and its forward: torch seed 1234, HIDDEN 64, 4 heads of 16, 2
groups, conv width 4, chunk 8, S 24 (three chunks), EPS 1e-5, dt limited to (0, inf), the same
draws in the same order and the HF forward -- plain RMSNorm, in_proj split into z | xBC | dt,
depthwise causal conv1d + SiLU, dt = softplus(dt + dt_bias), the chunked SSD (intra-chunk
products with the decay exp(cumA[l] - cumA[s]), chunk states, the state passed from chunk to
chunk, then C against it; head h reads group h // (H / G)), y + D x, the gated RMSNorm with
the gate applied before the norm per group of INTER / G channels, out_proj, residual.  One
change: the SSM state size is 128 (the reference's dump uses 16) because this build's kernels
serve the model's state size only; every draw keeps its recipe (shapes grow with N).  The SSD
is written here from its definition in float64; the final conv and SSM states of the sequence
are stored for the prefill-to-decode continuation.
"""
from __future__ import annotations

import hashlib
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
F32 = np.float32


def torch_decode(codes: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(codes, dtype=np.uint8)).view(torch.float8_e4m3fn)
    return t.float().numpy()


def torch_encode(q: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(q, dtype=np.float32)).to(torch.float8_e4m3fn)
    return t.view(torch.uint8).numpy().copy()


def bf16_bits(f: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(f, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16).copy()


def bf16_value(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def perrow_quant(wf: np.ndarray):
    """test_gemm.cu:516-529 in float32 arithmetic, the cast done by torch."""
    wf = wf.astype(F32)
    rowmax = np.abs(wf).max(axis=1).astype(F32)
    s = (rowmax / F32(448.0)).astype(F32)
    s = np.where(s < F32(1e-10), F32(1.0) / F32(448.0), s).astype(F32)
    inv = (F32(1.0) / s).astype(F32)
    q = np.clip((wf * inv[:, None]).astype(F32), F32(-448.0), F32(448.0))
    return torch_encode(q), s


def fp64_linear(xb: np.ndarray, codes: np.ndarray, s: np.ndarray) -> np.ndarray:
    x = bf16_value(np.atleast_2d(xb)).astype(np.float64)
    w = torch_decode(codes).astype(np.float64)
    return (x @ w.T) * s.astype(np.float64)[None, :]


def bf16_from_f64(v: np.ndarray) -> np.ndarray:
    """float64 -> bf16 bits with one round-to-nearest-even on the float64 bit pattern (keep the
    top 7 explicit mantissa bits).  Normal bf16 range only (checked)."""
    v = np.ascontiguousarray(v, np.float64)
    a = np.abs(v)
    assert np.all(np.isfinite(v)) and np.all((a == 0) | ((a >= 2.0 ** -126) & (a < 2.0 ** 127)))
    u = v.view(np.uint64)
    lsb = (u >> np.uint64(45)) & np.uint64(1)
    r = ((u + np.uint64((1 << 44) - 1) + lsb) >> np.uint64(45)) << np.uint64(45)
    return bf16_bits(r.view(np.float64).astype(F32))    # exact: 8 significant bits


def save(name: str, **arrays):
    path = os.path.join(HERE, name + ".npz")
    np.savez_compressed(path, **arrays)
    return path


def _rmsnorm64(x, w, eps):
    x = x.double()
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w.double()


def attention_fixture():
    """tools/dump_attention_block.py:20-58 (seed 777), forward in float64."""
    HID, HQ, HKV, HEAD, S, EPS = 256, 4, 2, 128, 40, 1e-5
    g = torch.Generator().manual_seed(777)
    norm_w = torch.randn(HID, generator=g, dtype=torch.float32)
    q_w = torch.randn(HQ * HEAD, HID, generator=g, dtype=torch.float32) * 0.1
    k_w = torch.randn(HKV * HEAD, HID, generator=g, dtype=torch.float32) * 0.1
    v_w = torch.randn(HKV * HEAD, HID, generator=g, dtype=torch.float32) * 0.1
    o_w = torch.randn(HID, HQ * HEAD, generator=g, dtype=torch.float32) * 0.1
    x = torch.randn(1, S, HID, generator=g, dtype=torch.float32).reshape(S, HID)
    with torch.no_grad():
        h = _rmsnorm64(x, norm_w, EPS)
        q = (h @ q_w.double().T).reshape(S, HQ, HEAD).transpose(0, 1)
        k = (h @ k_w.double().T).reshape(S, HKV, HEAD).transpose(0, 1)
        v = (h @ v_w.double().T).reshape(S, HKV, HEAD).transpose(0, 1)
        rep = HQ // HKV
        k = k.repeat_interleave(rep, dim=0)
        v = v.repeat_interleave(rep, dim=0)
        att = torch.nn.functional.scaled_dot_product_attention(q[None], k[None], v[None], is_causal=True)[0]
        att = att.transpose(0, 1).reshape(S, HQ * HEAD)
        o = att @ o_w.double().T
        out = x.double() + o
        # the reference's decode of the last token after a prefill of the others: its query
        # attends the cached positions [0, S - 1) only, its own k and v are appended afterwards
        # (ops/attention/sdpa_decode.cuh:57-120 loops over [0, S_cache), :122-180 appends)
        ql, kp, vp = q[:, S - 1:], k[:, :S - 1], v[:, :S - 1]
        p = torch.softmax((ql @ kp.transpose(1, 2)) / np.sqrt(HEAD), dim=-1)
        dec = (p @ vp).transpose(0, 1).reshape(1, HQ * HEAD) @ o_w.double().T + x[S - 1:].double()
    codes = {n: perrow_quant(w.numpy()) for n, w in (("q", q_w), ("k", k_w), ("v", v_w), ("o", o_w))}
    return save("attn_block_h256_q4_kv2_s40", x_f32=x.numpy(), x_bf16=bf16_bits(x.numpy()), norm_w=norm_w.numpy(),
                q_w_f32=q_w.numpy(), k_w_f32=k_w.numpy(), v_w_f32=v_w.numpy(), o_w_f32=o_w.numpy(),
                **{f"{n}_codes": c for n, (c, _) in codes.items()}, **{f"{n}_scale": sc for n, (_, sc) in codes.items()},
                expected_f32=out.float().numpy(), normed_f32=h.float().numpy(), attn_f32=att.float().numpy(),
                o_f32=o.float().numpy(), decode_last_f32=dec.float().numpy(), eps=np.float32(EPS))


def ssd_chunked(xdt, adt, Bh, Ch, chunk):
    """The chunked SSD of Mamba-2 in float64: xdt [S, H, P] (x * dt), adt [S, H] (A * dt), Bh, Ch
    [S, H, N] (per head).  Within a chunk, y[l] = sum_{s <= l} (C[l] . B[s]) exp(cumA[l] - cumA[s])
    xdt[s]; each chunk's state is sum_s B[s] exp(cumA[last] - cumA[s]) xdt[s]; the state entering a
    chunk is the previous one decayed over that chunk plus its state; the chunk's outputs add
    C[l] . state_in exp(cumA[l]).  Returns y [S, H, P] and the final state [H, P, N]."""
    S, H, P = xdt.shape
    N = Bh.shape[-1]
    y = torch.zeros(S, H, P, dtype=torch.float64)
    state = torch.zeros(H, P, N, dtype=torch.float64)
    for c0 in range(0, S, chunk):
        sl = slice(c0, min(S, c0 + chunk))
        cum = torch.cumsum(adt[sl], dim=0)                         # [L, H]
        L = cum.shape[0]
        decay = torch.exp(cum[:, None, :] - cum[None, :, :])       # [l, s, H]
        decay = decay * torch.tril(torch.ones(L, L, dtype=torch.float64))[:, :, None]
        cb = torch.einsum("lhn,shn->lsh", Ch[sl], Bh[sl])          # [l, s, H]
        y[sl] = torch.einsum("lsh,shp->lhp", cb * decay, xdt[sl])
        y[sl] += torch.einsum("lhn,hpn->lhp", Ch[sl], state) * torch.exp(cum)[:, :, None]
        to_end = torch.exp(cum[-1][None, :] - cum)                # [s, H]
        chunk_state = torch.einsum("shn,sh,shp->hpn", Bh[sl], to_end, xdt[sl])
        state = state * torch.exp(cum[-1])[:, None, None] + chunk_state
    return y, state


def mamba_fixture():
    """tools/dump_mamba_block.py:1-40 and its forward (seed 1234) with state size 128."""
    HID, H, P, N, G, CK, CHUNK, S, EPS = 64, 4, 16, 128, 2, 4, 8, 24, 1e-5
    INTER = H * P
    CONV = INTER + 2 * G * N
    PROJ = INTER + CONV + H
    GS = INTER // G
    g = torch.Generator().manual_seed(1234)
    norm_w = torch.randn(HID, generator=g, dtype=torch.float32)
    in_w = torch.randn(PROJ, HID, generator=g, dtype=torch.float32) * 0.1
    conv_w = torch.randn(CONV, 1, CK, generator=g, dtype=torch.float32) * 0.2
    conv_b = torch.randn(CONV, generator=g, dtype=torch.float32) * 0.1
    A_log = torch.randn(H, generator=g, dtype=torch.float32) * 0.5 - 1.0
    D = torch.rand(H, generator=g, dtype=torch.float32) * 0.1
    dt_bias = torch.rand(H, generator=g, dtype=torch.float32) * 0.2
    gnorm_w = torch.randn(INTER, generator=g, dtype=torch.float32)
    out_w = torch.randn(HID, INTER, generator=g, dtype=torch.float32) * 0.1
    x = torch.randn(1, S, HID, generator=g, dtype=torch.float32).reshape(S, HID)
    with torch.no_grad():
        h = _rmsnorm64(x, norm_w, EPS)
        proj = h @ in_w.double().T
        z, xbc, dt = proj[:, :INTER], proj[:, INTER:INTER + CONV], proj[:, INTER + CONV:]
        conv = torch.nn.functional.conv1d(xbc.T[None], conv_w.double(), conv_b.double(), padding=CK - 1,
                                          groups=CONV)[0, :, :S].T
        xc = torch.nn.functional.silu(conv)                        # [S, CONV]
        xs, Bs, Cs = xc[:, :INTER], xc[:, INTER:INTER + G * N], xc[:, INTER + G * N:]
        dts = torch.nn.functional.softplus(dt + dt_bias.double()).clamp(0.0, float("inf"))   # [S, H]
        A = -torch.exp(A_log.double())
        xh = xs.reshape(S, H, P)
        Bh = Bs.reshape(S, G, N).repeat_interleave(H // G, dim=1)
        Ch = Cs.reshape(S, G, N).repeat_interleave(H // G, dim=1)
        y, ssm_state = ssd_chunked(xh * dts[:, :, None], A[None, :] * dts, Bh, Ch, CHUNK)
        y = (y + D.double()[None, :, None] * xh).reshape(S, INTER)
        gated = y * torch.nn.functional.silu(z)
        gg = gated.reshape(S, G, GS)
        gn = (gg * torch.rsqrt(gg.pow(2).mean(-1, keepdim=True) + EPS)).reshape(S, INTER) * gnorm_w.double()
        mix = gn @ out_w.double().T
        out = x.double() + mix
        conv_state = xbc[S - (CK - 1):].T                          # [CONV, 3]: the last three xBC inputs
    in_codes, in_s = perrow_quant(in_w.numpy())
    out_codes, out_s = perrow_quant(out_w.numpy())
    return save("mamba_block_h64_h4p16_g2_n128_s24", x_f32=x.numpy(), x_bf16=bf16_bits(x.numpy()),
                norm_w=norm_w.numpy(), in_w_f32=in_w.numpy(), conv_w=conv_w.reshape(CONV, CK).numpy(),
                conv_b=conv_b.numpy(), A_log=A_log.numpy(), D=D.numpy(), dt_bias=dt_bias.numpy(),
                gnorm_w=gnorm_w.numpy(), out_w_f32=out_w.numpy(), in_codes=in_codes, in_scale=in_s,
                out_codes=out_codes, out_scale=out_s, expected_f32=out.float().numpy(),
                normed_f32=h.float().numpy(), xbc_conv_f32=xc.float().numpy(), scan_y_f32=y.float().numpy(),
                gnormed_f32=gn.float().numpy(), mixer_f32=mix.float().numpy(), dt_f32=dts.float().numpy(),
                conv_state_f32=conv_state.float().numpy(), ssm_state_f32=ssm_state.float().numpy(),
                shape=np.array([HID, H, P, N, G, CK, CHUNK, S], np.int32), eps=np.float32(EPS))


def main():
    written = []

    # 1. 256-entry decode table, as torch decodes float8_e4m3fn
    lut = torch_decode(np.arange(256, dtype=np.uint8))
    assert lut[0x7E] == 448.0 and lut[0x01] == 2.0 ** -9 and np.isnan(lut[0x7F]) and np.isnan(lut[0xFF])
    assert lut[0x80] == 0.0 and np.signbit(lut[0x80]) and lut[0x38] == 1.0 and lut[0xFE] == -448.0
    written.append(save("e4m3_lut", lut_bits=lut.view(np.uint32)))

    # 2. GemvFP8Test.MatchesReference known-answer inputs
    N, K = 64, 3136
    i = np.arange(K, dtype=np.int64)
    x_f = (((i * 13) % 17).astype(F32) * F32(0.1) - F32(0.8)).astype(F32)
    j = np.arange(N * K, dtype=np.int64)
    w_f = (((j * 7) % 23).astype(F32) * F32(0.05) - F32(0.55)).astype(F32).reshape(N, K)
    xb = bf16_bits(x_f)
    codes, s = perrow_quant(w_f)
    written.append(save("kat_gemv_n64_k3136", x_f32=x_f, w_f32=w_f, x_bf16=xb[None, :],
                        w_codes=codes, w_scale=s, y_f64=fp64_linear(xb, codes, s)))

    # 3. GemmFP8Test.Tiny inputs, kept W8A16
    M, N, K = 4, 8, 16
    x_f = ((np.arange(M * K) % 7).astype(F32) * F32(0.3) - F32(1.0)).astype(F32).reshape(M, K)
    w_f = ((np.arange(N * K) % 11).astype(F32) * F32(0.2) - F32(1.1)).astype(F32).reshape(N, K)
    xb = bf16_bits(x_f)
    codes, s = perrow_quant(w_f)
    written.append(save("tiny_m4_n8_k16", x_f32=x_f, w_f32=w_f, x_bf16=xb, w_codes=codes,
                        w_scale=s, y_f64=fp64_linear(xb, codes, s)))

    rng = np.random.default_rng(20241201)

    # 4. ragged N, K/16 odd, per-row quantized N(0, 0.02) weights
    M, N, K = 3, 37, 208
    w_f = (rng.standard_normal((N, K)) * 0.02).astype(F32)
    x_f = rng.standard_normal((M, K)).astype(F32)
    xb = bf16_bits(x_f)
    codes, s = perrow_quant(w_f)
    written.append(save("ragged_m3_n37_k208", x_bf16=xb, w_codes=codes, w_scale=s,
                        y_f64=fp64_linear(xb, codes, s)))

    # 5. skinny M=16, per-row log-uniform scales in [1e-4, 1e-2] (config-2 style)
    M, N, K = 16, 48, 3136
    codes = torch_encode(np.clip(rng.standard_normal((N, K)).astype(F32) * F32(64.0), -448, 448).astype(F32))
    s = np.exp(rng.uniform(np.log(1e-4), np.log(1e-2), N)).astype(F32)
    xb = bf16_bits(rng.standard_normal((M, K)).astype(F32))
    written.append(save("skinny_m16_n48_k3136", x_bf16=xb, w_codes=codes, w_scale=s,
                        y_f64=fp64_linear(xb, codes, s)))

    # 6. special values: NaN codes, -0 codes, subnormals, all-zero activation row
    M, N, K = 2, 8, 64
    codes = torch_encode(np.clip(rng.standard_normal((N, K)).astype(F32) * F32(8.0), -448, 448).astype(F32))
    codes[1, 5] = 0x7F                    # NaN
    codes[2, 63] = 0xFF                   # -NaN
    codes[3, :] = 0x80                    # -0 everywhere
    codes[4, :] = np.arange(K, dtype=np.uint8) % 8   # subnormals 0..7 * 2^-9
    s = np.full(N, 0.0078125, dtype=F32)
    xb = bf16_bits(rng.standard_normal((M, K)).astype(F32))
    xb[1, :] = 0                          # +0 activation row
    written.append(save("special_nan_zero", x_bf16=xb, w_codes=codes, w_scale=s,
                        y_f64=fp64_linear(xb, codes, s)))

    # 7. MLP block (tools/dump_mlp_block.py:15-53)
    H, I, S, EPS = 64, 256, 8, 1e-5
    g = torch.Generator().manual_seed(2024)
    norm_w = torch.randn(H, generator=g, dtype=torch.float32)
    up_w = torch.randn(I, H, generator=g, dtype=torch.float32) * 0.1
    down_w = torch.randn(H, I, generator=g, dtype=torch.float32) * 0.1
    x = torch.randn(1, S, H, generator=g, dtype=torch.float32).reshape(S, H)
    with torch.no_grad():
        var = x.pow(2).mean(-1, keepdim=True)
        hs = (x * torch.rsqrt(var + EPS)) * norm_w
        up = hs @ up_w.T
        act = torch.relu(up).pow(2)
        down = act @ down_w.T
        expected = x + down
    up_codes, up_s = perrow_quant(up_w.numpy())
    down_codes, down_s = perrow_quant(down_w.numpy())
    xb = bf16_bits(x.numpy())
    # float64 chain with bf16 rounding after every step
    xf = bf16_value(xb).astype(np.float64)
    ss = (xf * xf).sum(axis=1, keepdims=True)
    r = 1.0 / np.sqrt(ss / H + EPS)
    hb = bf16_from_f64(xf * r * norm_w.numpy().astype(np.float64)[None, :])
    upb = bf16_from_f64(fp64_linear(hb, up_codes, up_s))
    upv = bf16_value(upb).astype(np.float64)
    actb = bf16_from_f64(np.maximum(upv, 0.0) ** 2)
    downb = bf16_from_f64(fp64_linear(actb, down_codes, down_s))
    outb = bf16_from_f64(xf + bf16_value(downb).astype(np.float64))
    written.append(save("mlp_block_h64_i256_s8", x_f32=x.numpy(), x_bf16=xb, norm_w=norm_w.numpy(),
                        up_w_f32=up_w.numpy(), down_w_f32=down_w.numpy(), up_codes=up_codes, up_scale=up_s,
                        down_codes=down_codes, down_scale=down_s, expected_f32=expected.numpy(),
                        normed_f32=hs.numpy(), up_f32=up.numpy(), act_f32=act.numpy(), down_f32=down.numpy(),
                        chain_normed=hb, chain_up=upb, chain_act=actb, chain_down=downb, chain_f64=outb,
                        eps=np.float32(EPS)))

    written.append(attention_fixture())
    written.append(mamba_fixture())

    with open(os.path.join(HERE, "SHA256SUMS"), "w") as f:
        for p in sorted(written):
            h = hashlib.sha256(open(p, "rb").read()).hexdigest()
            f.write(f"{h}  {os.path.basename(p)}\n")
    print("wrote", [os.path.basename(p) for p in written])


if __name__ == "__main__":
    main()
