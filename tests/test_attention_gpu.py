"""GPU parity of the attention decode path: nmi_sdpa_decode_bf16 (ops/attention/
sdpa_decode.cuh:57-285) and the fp8 attention block nmi_attn_decode_fp8
(model/attention_block.cuh:371-414), through the C ABI (ops.py front ends) and the binding.

Bars:
* SDPA vs oracle.attention.sdpa_decode (float64, rounded once to bf16): the parity gate of
  oracle.linear.parity -- max 2 bf16 ulp, rel_l2 <= 1e-3 beyond isolated 1-ulp flips, and over
  all elements (outputs of >= 2048 values) -- at every tested S, GQA ratio and split count.  The
  kernel works in float32 (scores by v_dot2_f32_bf16, base-2 online softmax), so its values
  differ from the float64 ones by float32 rounding only.
* the caches after the call: position S of every KV head equals k_new / v_new bit for bit and
  every other position is unchanged.
* the block vs the composition of the library's separate calls -- rmsnorm, the three linears,
  sdpa_decode, the o linear and torch's bf16 residual add: bit-identical (the fused forms are
  exact restatements on the same kernels), then stage by stage vs the oracle (q/k/v given the
  GPU's normed input, the SDPA given the GPU's q, o_proj + residual given the GPU's attention
  output), then end to end: rel_l2 <= 4e-3 over all elements (a one-ulp flip of q moves the
  softmax and every output a little, so the element-wise bars are the stage-local ones).
"""
import numpy as np
import pytest
import torch

from nemotron_infer_amd import _lib, ops, synth
from oracle import attention, block, linear
from tests.gpu_util import DEV, announce, assert_parity, bits, s_to_dev, w_to_dev, x_to_dev

pytestmark = pytest.mark.gpu

HIDDEN, H_Q, H_KV, HEAD, EPS = synth.HIDDEN, 40, 8, 128, 1e-5


@pytest.fixture(autouse=True)
def _reset_tuning():
    _lib.tuning_set("sdpa.chunk", 0)
    yield
    _lib.tuning_set("sdpa.chunk", 0)


def _bf16_np(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def _sdpa_case(H, n_kv, S, cap, seed, qscale=1.0):
    q = _bf16_np((H, HEAD), seed, qscale)
    kc = _bf16_np((n_kv, cap, HEAD), seed + 1)
    vc = _bf16_np((n_kv, cap, HEAD), seed + 2)
    kn = _bf16_np((n_kv, HEAD), seed + 3)
    vn = _bf16_np((n_kv, HEAD), seed + 4)
    return q, kc, vc, kn, vn


def _run_sdpa(q, kc, vc, kn, vn, S):
    dq, dk, dv = x_to_dev(q), x_to_dev(kc), x_to_dev(vc)
    o = ops.sdpa_decode_bf16(dq, dk, dv, x_to_dev(kn), x_to_dev(vn), S)
    torch.cuda.synchronize()
    return bits(o), bits(dk), bits(dv)


def _check_sdpa(q, kc, vc, kn, vn, S, label):
    o, k2, v2 = _run_sdpa(q, kc, vc, kn, vn, S)
    ref = attention.sdpa_decode(q, kc, vc, S)
    if S == 0:
        assert not o.any(), label
    else:
        assert_parity(o, ref, label)
    rk, rv = attention.append_kv(kc, vc, kn, vn, S)
    assert np.array_equal(k2, rk) and np.array_equal(v2, rv), f"{label}: caches"
    return o


@pytest.mark.parametrize("S", [0, 1, 2, 5, 16, 17, 63, 64, 65, 127, 200, 1000, 4097])
def test_sdpa_matches_oracle_model_heads(S):
    announce("sdpa", H_Q, H_KV, S)
    _check_sdpa(*_sdpa_case(H_Q, H_KV, S, S + 3, 1000 + S), S, f"S={S}")


@pytest.mark.parametrize("H,n_kv", [(8, 8), (8, 4), (12, 4), (16, 4), (20, 4), (24, 4), (6, 1)])
def test_sdpa_gqa_ratios(H, n_kv):
    announce("sdpa_gqa", H, n_kv)
    for S in (3, 150):
        _check_sdpa(*_sdpa_case(H, n_kv, S, 160, 2000 + H * 10 + n_kv + S), S, f"H={H} n_kv={n_kv} S={S}")


@pytest.mark.parametrize("chunk", [16, 64, 100, 4096])
def test_sdpa_split_counts(chunk):
    """One split (chunk >= S), or many: each within the gate, the same caches."""
    announce("sdpa_chunk", chunk)
    _lib.tuning_set("sdpa.chunk", chunk)
    _check_sdpa(*_sdpa_case(H_Q, H_KV, 777, 800, 3000), 777, f"chunk={chunk}")


def test_sdpa_peaked_scores_and_long_context():
    """Large scores (softmax close to one-hot) stay finite and exact to the gate; 32k positions."""
    announce("sdpa_peaked")
    _check_sdpa(*_sdpa_case(H_Q, H_KV, 300, 301, 4000, qscale=8.0), 300, "peaked")
    announce("sdpa_long", 32768)
    _check_sdpa(*_sdpa_case(H_Q, H_KV, 32768, 32769, 4100), 32768, "S=32768")


def test_sdpa_multi_step_decode():
    """Four decode steps in a row on one cache, as the reference's MultiStep test
    (tests/ops/test_sdpa_decode.cu:125-200): each step attends what the previous steps stored."""
    announce("sdpa_multistep")
    S0, cap = 8, 32
    q, kc, vc, _, _ = _sdpa_case(H_Q, H_KV, S0, cap, 5000)
    dk, dv = x_to_dev(kc), x_to_dev(vc)
    host_k, host_v = kc.copy(), vc.copy()
    for step in range(4):
        S = S0 + step
        q = _bf16_np((H_Q, HEAD), 5100 + step)
        kn = _bf16_np((H_KV, HEAD), 5200 + step)
        vn = _bf16_np((H_KV, HEAD), 5300 + step)
        o = ops.sdpa_decode_bf16(x_to_dev(q), dk, dv, x_to_dev(kn), x_to_dev(vn), S)
        torch.cuda.synchronize()
        assert_parity(bits(o), attention.sdpa_decode(q, host_k, host_v, S), f"step {step}")
        host_k, host_v = attention.append_kv(host_k, host_v, kn, vn, S)
        assert np.array_equal(bits(dk), host_k) and np.array_equal(bits(dv), host_v), f"step {step}: caches"


# --------------------------------------------------------------------------------------
# the block at the model's dimensions (hidden 3136, 40 query heads, 8 KV heads)
# --------------------------------------------------------------------------------------
_W = {}


def _weights():
    if not _W:
        mats = {}
        for i, (name, rows, cols) in enumerate([("q", H_Q * HEAD, HIDDEN), ("k", H_KV * HEAD, HIDDEN),
                                                ("v", H_KV * HEAD, HIDDEN), ("o", HIDDEN, H_Q * HEAD)]):
            w, s = synth.make_weight(rows, cols, 7000 + i, "cpu")
            mats[name] = (w.numpy(), s.numpy())
        g = torch.Generator().manual_seed(7100)
        _W["norm"] = (1.0 + 0.1 * torch.randn(HIDDEN, generator=g)).float().numpy()
        _W.update(mats)
    return _W


def _dev_weights(W):
    return (torch.from_numpy(W["norm"]).to(DEV),) + tuple(
        t for n in "qkvo" for t in (w_to_dev(W[n][0]), s_to_dev(W[n][1])))


def _composed(xd, dw, dk, dv, S):
    nw, qw, qs, kw, ks, vw, vs, ow, os_ = dw
    h = ops.rmsnorm_bf16(xd, nw, EPS)
    q = ops.linear_fp8_w8a16(h, qw, qs, use_workspace=False)
    kn = ops.linear_fp8_w8a16(h, kw, ks, use_workspace=False)
    vn = ops.linear_fp8_w8a16(h, vw, vs, use_workspace=False)
    o = ops.sdpa_decode_bf16(q.view(H_Q, HEAD), dk, dv, kn.view(H_KV, HEAD), vn.view(H_KV, HEAD), S)
    attn = ops.linear_fp8_w8a16(o.view(1, -1), ow, os_, use_workspace=False)
    return xd + attn, (h, q, kn, vn, o)


@pytest.mark.parametrize("S", [0, 1, 77, 1500])
def test_attn_block_equals_composition_and_matches_oracle(S):
    announce("attn_block", S)
    W = _weights()
    dw = _dev_weights(W)
    cap = S + 5
    x = _bf16_np((1, HIDDEN), 7200 + S)
    kc = _bf16_np((H_KV, cap, HEAD), 7300 + S)
    vc = _bf16_np((H_KV, cap, HEAD), 7400 + S)
    xd = x_to_dev(x)
    dk1, dv1 = x_to_dev(kc), x_to_dev(vc)
    got = ops.attn_decode_fp8(xd, *dw, dk1, dv1, S, eps=EPS)
    dk2, dv2 = x_to_dev(kc), x_to_dev(vc)
    ref, (h, q, kn, vn, o) = _composed(xd, dw, dk2, dv2, S)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), "block != composition"
    assert torch.equal(dk1.view(torch.int16), dk2.view(torch.int16))
    assert torch.equal(dv1.view(torch.int16), dv2.view(torch.int16))

    # stage by stage against the oracle
    hb, qb, knb, vnb, ob, gotb = bits(h), bits(q), bits(kn), bits(vn), bits(o), bits(got)
    r = linear.parity(hb, block.rmsnorm_bf16(x, W["norm"], EPS))
    assert r["ok"] and r["n_diff"] <= 3, ("normed", r)
    for name, yb in (("q", qb), ("k", knb), ("v", vnb)):
        assert_parity(yb, linear.linear_fp8_w8a16(hb, *W[name]), f"{name}_proj S={S}")
    if S:
        assert_parity(ob, attention.sdpa_decode(qb.reshape(H_Q, HEAD), kc, vc, S), f"sdpa S={S}")
    else:
        assert not ob.any()
    attn_local = block.bf16_round_exact(linear.linear_fp64(ob.reshape(1, -1), *W["o"]))
    mag = np.maximum(np.abs(linear.bf16_to_f32(x)), np.abs(linear.bf16_to_f32(attn_local)))
    r = linear.parity(gotb, block.add_bf16(x, attn_local), mag=mag)
    assert r["ok"], ("o_proj + residual", r)
    rk, rv = attention.append_kv(kc, vc, knb.reshape(H_KV, HEAD), vnb.reshape(H_KV, HEAD), S)
    assert np.array_equal(bits(dk1), rk) and np.array_equal(bits(dv1), rv)

    # end to end
    out_ref, _, _ = attention.attn_decode_block_fp8(x, W["norm"], *W["q"], *W["k"], *W["v"], *W["o"], kc, vc, S,
                                                    H_KV, EPS)
    r = linear.parity(gotb, out_ref)
    assert r["nan_ok"] and r["rel_l2_all"] <= 4e-3, ("end to end", r)


def test_attn_block_binding_in_place_and_bump_allocator():
    """The drop-in binding entry (bump-allocated buffers, null stream) gives the C-ABI result
    bit for bit, also with out == input."""
    from nemotron_infer_amd.csrc import binding as B

    announce("attn_block_binding")
    W = _weights()
    dw = _dev_weights(W)
    S, cap = 300, 512
    x = x_to_dev(_bf16_np((1, HIDDEN), 7500))
    kc = _bf16_np((H_KV, cap, HEAD), 7501)
    vc = _bf16_np((H_KV, cap, HEAD), 7502)
    dk1, dv1, dk2, dv2 = x_to_dev(kc), x_to_dev(vc), x_to_dev(kc), x_to_dev(vc)
    want = ops.attn_decode_fp8(x, *dw, dk1, dv1, S, eps=EPS)
    torch.cuda.synchronize()
    xi = x.clone()
    B.reset_allocator()
    B.attn_decode_fp8(xi.data_ptr(), *[t.data_ptr() for t in dw], dk2.data_ptr(), dv2.data_ptr(), S, cap,
                      xi.data_ptr())
    B.sync()
    assert torch.equal(xi.view(torch.int16), want.view(torch.int16))
    assert torch.equal(dk1.view(torch.int16), dk2.view(torch.int16))
    assert torch.equal(dv1.view(torch.int16), dv2.view(torch.int16))
