"""Pin the attention-decode oracle (oracle/attention.py): sdpa_decode against torch's own
F.scaled_dot_product_attention in float64 (KV heads repeated for GQA), against closed forms (one
cached position, a zero query, an empty cache), and show that those checks catch plausible
mistakes planted in the oracle (a wrong KV-head mapping, attending the new token, a dropped
1/sqrt(D)).  The block oracle is pinned against an independent float32 torch composition and
the closed forms o_w == 0 and S == 0."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention, block, linear

F32 = np.float32
D = attention.HEAD


def bf16(v):
    return linear.bf16_rne(np.asarray(v, F32))


def val(b):
    return linear.bf16_to_f32(b).astype(np.float64)


def _case(H, H_KV, cap, seed, qscale=1.0):
    rng = np.random.default_rng(seed)
    q = bf16(rng.standard_normal((H, D)) * qscale)
    kc = bf16(rng.standard_normal((H_KV, cap, D)))
    vc = bf16(rng.standard_normal((H_KV, cap, D)))
    return q, kc, vc


def _torch_sdpa(q, kc, vc, S):
    """torch's scaled_dot_product_attention on the first S positions, float64, GQA by repeat."""
    H, H_KV = q.shape[0], kc.shape[0]
    qt = torch.from_numpy(val(q))[None, :, None, :]                       # [1, H, 1, D]
    kt = torch.from_numpy(val(kc[:, :S]))[None].repeat_interleave(H // H_KV, dim=1)
    vt = torch.from_numpy(val(vc[:, :S]))[None].repeat_interleave(H // H_KV, dim=1)
    return F.scaled_dot_product_attention(qt, kt, vt)[0, :, 0, :].numpy()


@pytest.mark.parametrize("H,H_KV,S", [(40, 8, 1), (40, 8, 37), (40, 8, 300), (4, 4, 17), (6, 2, 64), (8, 1, 9)])
def test_sdpa_matches_torch_sdpa(H, H_KV, S):
    q, kc, vc = _case(H, H_KV, S + 3, seed=H * 1000 + S)
    got = attention.sdpa_decode_f64(q, kc, vc, S)
    ref = _torch_sdpa(q, kc, vc, S)
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_one_cached_position_returns_its_value_exactly():
    q, kc, vc = _case(40, 8, 5, seed=3, qscale=4.0)
    o = attention.sdpa_decode(q, kc, vc, 1)
    for h in range(40):
        assert np.array_equal(o[h], vc[h // 5, 0])


def test_zero_query_returns_the_mean_of_v():
    _, kc, vc = _case(10, 2, 50, seed=4)
    q = np.zeros((10, D), np.uint16)
    o = attention.sdpa_decode_f64(q, kc, vc, 50)
    for h in range(10):
        np.testing.assert_allclose(o[h], val(vc[h // 5, :50]).mean(axis=0), rtol=1e-13, atol=1e-14)


def test_empty_cache_gives_zero():
    q, kc, vc = _case(40, 8, 4, seed=5)
    assert not attention.sdpa_decode(q, kc, vc, 0).any()


def test_append_writes_position_s_only():
    _, kc, vc = _case(40, 8, 9, seed=6)
    rng = np.random.default_rng(7)
    kn = bf16(rng.standard_normal((8, D)))
    vn = bf16(rng.standard_normal((8, D)))
    k2, v2 = attention.append_kv(kc, vc, kn, vn, 5)
    assert np.array_equal(k2[:, 5], kn) and np.array_equal(v2[:, 5], vn)
    mask = np.ones(9, bool)
    mask[5] = False
    assert np.array_equal(k2[:, mask], kc[:, mask]) and np.array_equal(v2[:, mask], vc[:, mask])


# --------------------------------------------------------------------------------------
# planted mistakes: each must fail one of the checks above
# --------------------------------------------------------------------------------------
def test_planted_wrong_kv_mapping_is_caught():
    q, kc, vc = _case(40, 8, 40, seed=8)
    wrong = attention.sdpa_decode_f64(q, kc, vc, 37, kv_of=lambda h, H, H_KV: h % H_KV)
    assert not np.allclose(wrong, _torch_sdpa(q, kc, vc, 37), rtol=1e-6, atol=1e-6)


def test_planted_attending_the_new_token_is_caught():
    q, kc, vc = _case(40, 8, 40, seed=9)
    wrong = attention.sdpa_decode_f64(q, kc, vc, 38)      # S + 1 positions
    assert not np.allclose(wrong, _torch_sdpa(q, kc, vc, 37), rtol=1e-6, atol=1e-6)


def test_planted_missing_scale_is_caught():
    q, kc, vc = _case(8, 8, 20, seed=10)
    q_scaled = bf16(val(q) * np.sqrt(D))                  # softmax(q.k) instead of q.k / sqrt(D)
    wrong = attention.sdpa_decode_f64(q_scaled, kc, vc, 20)
    assert not np.allclose(wrong, _torch_sdpa(q, kc, vc, 20), rtol=1e-3, atol=1e-3)


# --------------------------------------------------------------------------------------
# the block (attention_block.cuh:371-414)
# --------------------------------------------------------------------------------------
def _block_case(hidden, H, H_KV, cap, seed):
    rng = np.random.default_rng(seed)

    def w(rows, cols):
        wf = rng.standard_normal((rows, cols)).astype(F32) * 0.05
        s = np.full(rows, np.abs(wf).max() / 448, F32)
        codes = torch.from_numpy(wf / s[:, None]).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        return codes, s

    x = bf16(rng.standard_normal((1, hidden)))
    nw = (1 + 0.1 * rng.standard_normal(hidden)).astype(F32)
    qw, kw, vw, ow = w(H * D, hidden), w(H_KV * D, hidden), w(H_KV * D, hidden), w(hidden, H * D)
    _, kc, vc = _case(H, H_KV, cap, seed + 1)
    return x, nw, qw, kw, vw, ow, kc, vc


def test_block_matches_a_float32_torch_composition():
    hidden, H, H_KV, S = 256, 10, 2, 33
    x, nw, qw, kw, vw, ow, kc, vc = _block_case(hidden, H, H_KV, S + 2, seed=11)
    out, k2, v2 = attention.attn_decode_block_fp8(x, nw, *qw, *kw, *vw, *ow, kc, vc, S, H_KV)

    def deq(cs):
        return torch.from_numpy(linear.dequant_f32(*cs))

    xt = torch.from_numpy(val(x).astype(F32))
    h = xt * torch.rsqrt(xt.pow(2).mean(-1, keepdim=True) + 1e-5) * torch.from_numpy(nw)
    q = F.linear(h, deq(qw)).view(1, H, 1, D)
    kt = torch.from_numpy(val(kc[:, :S]).astype(F32))[None].repeat_interleave(H // H_KV, 1)
    vt = torch.from_numpy(val(vc[:, :S]).astype(F32))[None].repeat_interleave(H // H_KV, 1)
    o = F.scaled_dot_product_attention(q, kt, vt).reshape(1, H * D)
    ref = (xt + F.linear(o, deq(ow))).numpy()
    got = val(out)
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel < 2e-2, rel            # bf16 roundings at every stage against none
    kn = F.linear(h, deq(kw)).numpy().reshape(H_KV, D)
    assert np.allclose(val(k2[:, S]), kn, rtol=2e-2, atol=2e-2)
    assert np.array_equal(np.delete(k2, S, axis=1), np.delete(kc, S, axis=1))
    vn = F.linear(h, deq(vw)).numpy().reshape(H_KV, D)
    assert np.allclose(val(v2[:, S]), vn, rtol=2e-2, atol=2e-2)


def test_block_closed_forms_give_the_input():
    hidden, H, H_KV = 128, 4, 2
    x, nw, qw, kw, vw, ow, kc, vc = _block_case(hidden, H, H_KV, 6, seed=12)
    # S == 0: the attention output is 0, so o_proj gives 0 and out == input
    out, _, _ = attention.attn_decode_block_fp8(x, nw, *qw, *kw, *vw, *ow, kc, vc, 0, H_KV)
    assert np.array_equal(out, x)
    # o_w == 0: out == input whatever the attention gives
    zero = (np.zeros_like(ow[0]), ow[1])
    out, _, _ = attention.attn_decode_block_fp8(x, nw, *qw, *kw, *vw, *zero, kc, vc, 4, H_KV)
    assert np.array_equal(out, x)
    # and with both live the output differs from the input
    out, _, _ = attention.attn_decode_block_fp8(x, nw, *qw, *kw, *vw, *ow, kc, vc, 4, H_KV)
    assert not np.array_equal(out, x)
    assert np.array_equal(block.add_bf16(x, np.zeros_like(x)), x)


# --------------------------------------------------------------------------------------
# prefill (sdpa_prefill.cuh:224-320)
# --------------------------------------------------------------------------------------
def _prefill_case(S, H, H_KV, seed):
    rng = np.random.default_rng(seed)
    return (bf16(rng.standard_normal((S, H * D))), bf16(rng.standard_normal((S, H_KV * D))),
            bf16(rng.standard_normal((S, H_KV * D))))


@pytest.mark.parametrize("S,H,H_KV", [(1, 4, 2), (37, 10, 2), (130, 8, 8), (64, 6, 1)])
def test_prefill_matches_torch_causal_sdpa(S, H, H_KV):
    q, k, v = _prefill_case(S, H, H_KV, seed=S + H)
    got = attention.sdpa_prefill_f64(q, k, v, H_KV)
    qt = torch.from_numpy(val(q)).view(S, H, D).transpose(0, 1)[None]
    kt = torch.from_numpy(val(k)).view(S, H_KV, D).transpose(0, 1)[None].repeat_interleave(H // H_KV, dim=1)
    vt = torch.from_numpy(val(v)).view(S, H_KV, D).transpose(0, 1)[None].repeat_interleave(H // H_KV, dim=1)
    ref = F.scaled_dot_product_attention(qt, kt, vt, is_causal=True)[0].transpose(0, 1).reshape(S, H * D).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_prefill_first_row_is_the_first_value():
    q, k, v = _prefill_case(20, 10, 2, seed=5)
    o = attention.sdpa_prefill(q, k, v, 2)
    for h in range(10):
        assert np.array_equal(o[0, h * D:(h + 1) * D], v[0, (h // 5) * D:(h // 5 + 1) * D])


def test_planted_non_causal_prefill_is_caught():
    q, k, v = _prefill_case(33, 4, 2, seed=6)
    wrong = attention.sdpa_prefill_f64(q, k, v, 2, causal=False)
    assert not np.allclose(wrong, attention.sdpa_prefill_f64(q, k, v, 2), rtol=1e-3, atol=1e-3)
