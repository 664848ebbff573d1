"""GPU parity of the attention prefill path: nmi_sdpa_prefill_bf16 (causal attention,
ops/attention/sdpa_prefill.cuh:224-395) and the fp8 block nmi_attn_forward_fp8
(model/attention_block.cuh:289-366), through the C ABI (ops.py front ends) and the binding.

Bars:
* SDPA vs oracle.attention.sdpa_prefill (float64, rounded once): the parity gate (max 2 bf16
  ulp; rel_l2 <= 1e-3 beyond isolated one-ulp flips, and over all elements) at every tested S
  (one and several key tiles, partial tiles, many query tiles), GQA ratio and row stride.  The
  kernel's scores are float32 MFMA sums of exact bf16 products and its softmax weights enter the
  value product in two bf16 parts (about 16 bits), so it differs from the float64 value by
  float32-level rounding.
* the block vs the composition of the library's calls (rmsnorm, three linears, sdpa_prefill,
  the o linear, torch's bf16 residual add): bit-identical output and caches; then stage by stage
  vs the oracle and end to end (rel_l2 <= 4e-3 over all elements).
* a decode step after the prefill reads the caches the prefill wrote: its result equals the
  oracle decode on the oracle's k and v of the prompt (parity gate).
"""
import numpy as np
import pytest
import torch

from nemotron_infer_amd import ops, synth
from oracle import attention, block, linear
from tests.gpu_util import DEV, announce, assert_parity, bits, s_to_dev, w_to_dev, x_to_dev

pytestmark = pytest.mark.gpu

HIDDEN, H_Q, H_KV, D, EPS = synth.HIDDEN, 40, 8, 128, 1e-5


def _bf16_np(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("S", [1, 2, 63, 64, 65, 127, 128, 129, 300, 1000])
def test_sdpa_prefill_matches_oracle(S):
    announce("sdpa_prefill", S)
    q = _bf16_np((S, H_Q * D), 100 + S)
    k = _bf16_np((S, H_KV * D), 200 + S)
    v = _bf16_np((S, H_KV * D), 300 + S)
    o = ops.sdpa_prefill_bf16(x_to_dev(q), x_to_dev(k), x_to_dev(v), H_Q, H_KV)
    torch.cuda.synchronize()
    assert_parity(bits(o), attention.sdpa_prefill(q, k, v, H_KV), f"S={S}")


@pytest.mark.parametrize("S", [1537, 2048])
def test_sdpa_prefill_long_prompts(S):
    """Prompts of 1537 and 2048 tokens (8 query heads, 2 KV heads): query tiles up to 32 key tiles
    long, so every stage refill, the partial last key tile and the tile-rank order of the launch
    are exercised at the bench's length."""
    H, n_kv = 8, 2
    announce("sdpa_prefill_long", S)
    q = _bf16_np((S, H * D), 700 + S)
    k = _bf16_np((S, n_kv * D), 800 + S)
    v = _bf16_np((S, n_kv * D), 900 + S)
    o = ops.sdpa_prefill_bf16(x_to_dev(q), x_to_dev(k), x_to_dev(v), H, n_kv)
    torch.cuda.synchronize()
    assert_parity(bits(o), attention.sdpa_prefill(q, k, v, n_kv), f"S={S}")


@pytest.mark.parametrize("H,n_kv", [(8, 8), (12, 4), (6, 1), (16, 2)])
def test_sdpa_prefill_gqa_and_packed_rows(H, n_kv):
    """q, k and v as column slices of one packed [S, (H + 2 n_kv) * 128] buffer (the layout of a
    grouped q|k|v output), larger scores (q x 4) for a peaked softmax."""
    S = 200
    announce("sdpa_prefill_gqa", H, n_kv)
    qkv = _bf16_np((S, (H + 2 * n_kv) * D), 400 + H + n_kv)
    qkv[:, :H * D] = _bf16_np((S, H * D), 500 + H, scale=4.0)
    d = x_to_dev(qkv)
    q, k, v = d[:, :H * D], d[:, H * D:(H + n_kv) * D], d[:, (H + n_kv) * D:]
    o = ops.sdpa_prefill_bf16(q, k, v, H, n_kv)
    torch.cuda.synchronize()
    ref = attention.sdpa_prefill(qkv[:, :H * D], qkv[:, H * D:(H + n_kv) * D], qkv[:, (H + n_kv) * D:], n_kv)
    assert_parity(bits(o), ref, f"H={H} n_kv={n_kv}")


# --------------------------------------------------------------------------------------
# the block at the model's dimensions
# --------------------------------------------------------------------------------------
_W = {}


def _weights():
    if not _W:
        for i, (name, rows, cols) in enumerate([("q", H_Q * D, HIDDEN), ("k", H_KV * D, HIDDEN),
                                                ("v", H_KV * D, HIDDEN), ("o", HIDDEN, H_Q * D)]):
            w, s = synth.make_weight(rows, cols, 7700 + i, "cpu")
            _W[name] = (w.numpy(), s.numpy())
        g = torch.Generator().manual_seed(7710)
        _W["norm"] = (1.0 + 0.1 * torch.randn(HIDDEN, generator=g)).float().numpy()
    return _W


def _dev_weights(W):
    return (torch.from_numpy(W["norm"]).to(DEV),) + tuple(
        t for n in "qkvo" for t in (w_to_dev(W[n][0]), s_to_dev(W[n][1])))


def _composed(xd, dw, S):
    nw, qw, qs, kw, ks, vw, vs, ow, os_ = dw
    ws = True          # as the block: its linears get their split-K / stream-K workspace
    h = ops.rmsnorm_bf16(xd, nw, EPS)
    # q | k | v as the block runs them: one grouped dispatch (one launch at S >= 512)
    q, k, v = ops.linear_fp8_w8a16_grouped(h, [(qw, qs), (kw, ks), (vw, vs)], use_workspace=ws)
    o = ops.sdpa_prefill_bf16(q, k, v, H_Q, H_KV)
    attn = ops.linear_fp8_w8a16(o, ow, os_, use_workspace=ws)
    return xd + attn, (h, q, k, v, o)


@pytest.mark.parametrize("S", [1, 5, 77, 600])
def test_attn_forward_equals_composition_and_matches_oracle(S):
    announce("attn_forward", S)
    W = _weights()
    dw = _dev_weights(W)
    x = _bf16_np((S, HIDDEN), 7800 + S)
    xd = x_to_dev(x)
    cap = S + 3
    kc = torch.full((H_KV, cap, D), 7.0, dtype=torch.bfloat16, device=DEV)
    vc = torch.full_like(kc, 7.0)
    got = ops.attn_forward_fp8(xd, *dw, k_cache=kc, v_cache=vc, eps=EPS)
    ref, (h, q, k, v, o) = _composed(xd, dw, S)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), "block != composition"
    kb, vb = bits(k), bits(v)
    assert np.array_equal(bits(kc[:, :S]), kb.reshape(S, H_KV, D).transpose(1, 0, 2)), "k cache"
    assert np.array_equal(bits(vc[:, :S]), vb.reshape(S, H_KV, D).transpose(1, 0, 2)), "v cache"
    assert torch.all(kc[:, S:] == 7.0) and torch.all(vc[:, S:] == 7.0), "cache past S written"

    hb, qb, ob, gotb = bits(h), bits(q), bits(o), bits(got)
    r = linear.parity(hb, block.rmsnorm_bf16(x, W["norm"], EPS))
    assert r["ok"] and r["n_diff"] <= max(3, 0.001 * hb.size), ("normed", r)
    for name, yb in (("q", qb), ("k", kb), ("v", vb)):
        assert_parity(yb, linear.linear_fp8_w8a16(hb, *W[name]), f"{name}_proj S={S}")
    assert_parity(ob, attention.sdpa_prefill(qb, kb, vb, H_KV), f"sdpa S={S}")
    attn_local = block.bf16_round_exact(linear.linear_fp64(ob, *W["o"]))
    mag = np.maximum(np.abs(linear.bf16_to_f32(x)), np.abs(linear.bf16_to_f32(attn_local)))
    r = linear.parity(gotb, block.add_bf16(x, attn_local), mag=mag)
    assert r["ok"], ("o_proj + residual", r)
    out_ref = attention.attn_forward_block_fp8(x, W["norm"], *W["q"], *W["k"], *W["v"], *W["o"], H_KV, EPS)
    r = linear.parity(gotb, out_ref)
    assert r["nan_ok"] and r["rel_l2_all"] <= 4e-3, ("end to end", r)


def test_attn_forward_binding_then_decode_continues_from_the_caches():
    """The drop-in binding entry (bump-allocated buffers, null stream, in place) equals the C-ABI
    call; a decode step at S_cache = S then attends exactly the positions the prefill stored."""
    from nemotron_infer_amd.csrc import binding as B

    announce("attn_forward_binding_decode")
    W = _weights()
    dw = _dev_weights(W)
    S, cap = 96, 128
    x = x_to_dev(_bf16_np((S, HIDDEN), 7900))
    kc1 = torch.zeros((H_KV, cap, D), dtype=torch.bfloat16, device=DEV)
    vc1, kc2, vc2 = torch.zeros_like(kc1), torch.zeros_like(kc1), torch.zeros_like(kc1)
    want = ops.attn_forward_fp8(x, *dw, k_cache=kc1, v_cache=vc1, eps=EPS)
    torch.cuda.synchronize()
    xi = x.clone()
    B.reset_allocator()
    B.attn_forward_fp8(xi.data_ptr(), *[t.data_ptr() for t in dw], xi.data_ptr(), S, kc2.data_ptr(), vc2.data_ptr(),
                       cap)
    B.sync()
    assert torch.equal(xi.view(torch.int16), want.view(torch.int16))
    assert torch.equal(kc1.view(torch.int16), kc2.view(torch.int16)) and torch.equal(vc1.view(torch.int16),
                                                                                        vc2.view(torch.int16))
    # one decode step on the prefilled caches
    xn = x_to_dev(_bf16_np((1, HIDDEN), 7901))
    kc_before, vc_before = bits(kc1), bits(vc1)
    out = ops.attn_decode_fp8(xn, *dw, kc1, vc1, S, eps=EPS)
    torch.cuda.synchronize()
    ref, _, _ = attention.attn_decode_block_fp8(bits(xn), W["norm"], *W["q"], *W["k"], *W["v"], *W["o"],
                                                kc_before, vc_before, S, H_KV, EPS)
    r = linear.parity(bits(out), ref)
    assert r["nan_ok"] and r["rel_l2_all"] <= 4e-3, r
