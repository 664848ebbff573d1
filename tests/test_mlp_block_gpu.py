"""GPU parity of the fp8 MLP block (nmi_mlp_forward_fp8, model/mlp_block.cuh:121-176) and of the
RMSNorm (nmi_rmsnorm_bf16, ops/reduce.cuh:135-244).

Bars:
* RMSNorm vs oracle.block.rmsnorm_bf16: the parity gate (rel_l2 <= 1e-3 beyond isolated 1-ulp
  flips, max 2 bf16 ulp, flips <= 1% of elements), and flips below 0.1%: the kernel's float32
  sum of squares and the oracle's float64 sum differ in the last bit of the factor now and then.
* block vs the composition of separate library calls -- rmsnorm, linear, torch's bf16
  relu^2, linear, torch's bf16 residual add: bit-identical.  The fused forms (RMSNorm while the
  GEMV kernel stages x; relu^2 and the residual add in the projections' stores) are exact
  restatements of the separate steps, on the same kernels and schedules.
* block vs the oracle stage by stage (the block's intermediates are the composition's, which
  is bit-identical): RMSNorm as above; the up projection vs float64 sums rounded once, given the
  GPU's normed activations; the block's output vs the float64 down projection of the GPU's
  relu^2 activations plus the residual -- the parity gate, ulps taken at the larger of |out|,
  |x| and |down| (where x + down cancels, one ulp of down is several ulps of out).
* block end to end vs oracle.block.mlp_block_fp8 (precise: float64 projections rounded once):
  rel_l2 <= 4e-3 over all elements.  A one-ulp flip of an up-projection output (a few per 10^4,
  from float32 summation order) moves that relu^2 activation by about 1/128 of its value, and
  through the down projection every output of its row by up to ~0.2 ulp: one flip can change
  4% of its row and add ~1e-3 to its rel_l2, so the element-wise bars are the stage-local ones
  above.  (The torch fp32 oracle is not the reference here: at K = 12544 its own float32 sum is
  off by up to ~3.5 bf16 ulp on outputs near zero.)
* golden fixture (tools/dump_mlp_block.py:15-53 inputs, per-row fp8 weights): rel_l2 against
  the HF fp32 expectation < 0.05 (the reference's own gate, test_mlp_block.cu:184, is 0.3).
"""
import ctypes

import numpy as np
import pytest
import torch

from nemotron_infer_amd import _lib, ops, synth
from oracle import block, linear
from tests.conftest import load_golden
from tests.gpu_util import DEV, announce, bits, s_to_dev, w_to_dev, x_to_dev

pytestmark = pytest.mark.gpu

KNOBS = ("m1.path", "skinny.path", "s16", "gemv.ks", "gemv.t", "gemv.p", "gemv.xg", "gemm.tile", "s4.ks")
HIDDEN, INTER, EPS = synth.HIDDEN, synth.INTER, 1e-5


@pytest.fixture(autouse=True)
def _reset_tuning():
    for k in KNOBS:
        _lib.tuning_set(k, 0)
    yield
    for k in KNOBS:
        _lib.tuning_set(k, 0)


_WEIGHTS = {}


def _weights(hidden, inter, seed=300):
    key = (hidden, inter, seed)
    if key not in _WEIGHTS:
        up_w, up_s = synth.make_weight(inter, hidden, seed, "cpu")
        dn_w, dn_s = synth.make_weight(hidden, inter, seed + 1, "cpu")
        g = torch.Generator().manual_seed(seed + 2)
        nw = (1.0 + 0.1 * torch.randn(hidden, generator=g)).float()
        _WEIGHTS[key] = (nw.numpy(), up_w.numpy(), up_s.numpy(), dn_w.numpy(), dn_s.numpy())
    return _WEIGHTS[key]


def _act(M, hidden, seed):
    x = synth.make_act(M, hidden, seed, "cpu")
    return x.view(torch.int16).numpy().view(np.uint16)


def _dev(nw, upw, ups, dnw, dns):
    return (torch.from_numpy(nw).to(DEV), w_to_dev(upw), s_to_dev(ups), w_to_dev(dnw), s_to_dev(dns))


def _composed(x, nw, upw, ups, dnw, dns, ws=True):
    # The block hands its linears a workspace -- the short-prompt kernel's K split for
    # 17 <= M < 512, the stream-K form where it is forced (the other kernels ignore it); the
    # composition does the same, so that both run the same kernels in the same form (same
    # float32 summation order).
    h = ops.rmsnorm_bf16(x, nw, EPS)
    up = ops.linear_fp8_w8a16(h, upw, ups, use_workspace=ws)
    r = torch.relu(up)
    act = r * r
    down = ops.linear_fp8_w8a16(act, dnw, dns, use_workspace=ws)
    return x + down


# --------------------------------------------------------------------------------------
# RMSNorm
# --------------------------------------------------------------------------------------
@pytest.mark.parametrize("M,K", [(1, 3136), (2, 3136), (5, 64), (3, 8), (7, 12544), (33, 3136), (4, 4104)])
def test_rmsnorm_matches_oracle(M, K):
    announce("rmsnorm", M, K)
    x = _act(M, K, 40 + M)
    w = (1.0 + 0.1 * np.random.default_rng(K).standard_normal(K)).astype(np.float32)
    y = bits(ops.rmsnorm_bf16(x_to_dev(x), torch.from_numpy(w).to(DEV), EPS))
    ref = block.rmsnorm_bf16(x, w, EPS)
    r = linear.parity(y, ref)
    assert r["ok"] and r["n_diff"] <= max(1, 0.001 * y.size), r


def test_rmsnorm_zero_rows_and_binding():
    from nemotron_infer_amd.csrc import binding as B

    announce("rmsnorm_zero_binding")
    x = x_to_dev(_act(3, HIDDEN, 7))
    x[1].zero_()
    w = torch.from_numpy(_weights(HIDDEN, INTER)[0]).to(DEV)
    y = ops.rmsnorm_bf16(x, w, EPS)
    assert torch.count_nonzero(y[1]) == 0
    yb = torch.empty_like(x)
    B.rmsnorm(x.data_ptr(), yb.data_ptr(), w.data_ptr(), 3)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), yb.view(torch.int16))


# --------------------------------------------------------------------------------------
# The block at the real dimensions (hidden 3136, inter 12544)
# --------------------------------------------------------------------------------------
M_LIST = [1, 2, 3, 8, 16, 17, 64, 520]


@pytest.mark.parametrize("M", M_LIST)
def test_block_equals_composition(M):
    announce("mlp_block_composition", M)
    dev = _dev(*_weights(HIDDEN, INTER))
    x = x_to_dev(_act(M, HIDDEN, 100 + M))
    got = ops.mlp_forward_fp8(x, *dev, eps=EPS)
    ref = _composed(x, *dev)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def _summands(x, stages):
    return np.maximum(np.abs(linear.bf16_to_f32(x)), np.abs(linear.bf16_to_f32(stages["down"])))


def _exact_proj(a_bits, codes, s):
    return block.bf16_round_exact(linear.linear_fp64(a_bits, codes, s))


def check_block(x, got, nw, upw, ups, dnw, dns, eps, label):
    """Stage-local parity, then end-to-end parity; see the module docstring."""
    dev = _dev(nw, upw, ups, dnw, dns)
    xd = x_to_dev(x)
    h = ops.rmsnorm_bf16(xd, dev[0], eps)
    up = ops.linear_fp8_w8a16(h, dev[1], dev[2], use_workspace=True)   # as the block
    r_ = torch.relu(up)
    act = bits(r_ * r_)
    h, up = bits(h), bits(up)
    r = linear.parity(h, block.rmsnorm_bf16(x, nw, eps))
    assert r["ok"] and r["n_diff"] <= max(1, 0.001 * h.size), (label, "normed", r)
    r = linear.parity(up, _exact_proj(h, upw, ups))
    assert r["ok"], (label, "up", r)
    down_local = _exact_proj(act, dnw, dns)
    r = linear.parity(got, block.add_bf16(x, down_local), mag=_summands(x, {"down": down_local}))
    assert r["ok"], (label, "down + residual", r)
    ref = block.mlp_block_fp8(x, nw, upw, ups, dnw, dns, eps, precise=True)
    r = linear.parity(got, ref)
    assert r["nan_ok"] and r["rel_l2_all"] <= 4e-3, (label, "end to end", r)
    return r


@pytest.mark.parametrize("M", M_LIST)
def test_block_matches_oracle(M):
    announce("mlp_block_oracle", M)
    nw, upw, ups, dnw, dns = _weights(HIDDEN, INTER)
    x = _act(M, HIDDEN, 200 + M)
    got = bits(ops.mlp_forward_fp8(x_to_dev(x), *_dev(nw, upw, ups, dnw, dns), eps=EPS))
    check_block(x, got, nw, upw, ups, dnw, dns, EPS, f"M={M}")


@pytest.mark.parametrize("knobs,Ms", [
    ({"m1.path": 3}, [1]),                           # M = 1 on the 4x4x4 kernel: separate RMSNorm
    ({"skinny.path": 3}, [2, 3, 4]),                 # GEMV kernel for M <= 4 (fused only M <= 2)
    ({"s16": 2}, [5, 16]),                           # the 4x4x4 kernel instead of the 16x16x32 one
    ({"gemv.ks": 2, "gemv.t": 2, "gemv.p": 3}, [1, 2]),
    ({"gemv.ks": 4, "gemv.t": 1}, [1]),
    ({"gemv.xg": 1}, [1]),                           # the fused form always stages x in LDS
    ({"gemm.tile": 20}, [600]),
    ({"gemm.tile": 21}, [600]),
    ({"gemm.bm": 128}, [520]),                       # 128 x 256 tiles for both projections
    ({"gemm.sk": 1}, [520]),                         # stream-K form of the 256 x 256 kernel
])
def test_block_equals_composition_under_knobs(knobs, Ms):
    dev = _dev(*_weights(HIDDEN, INTER))
    for k, v in knobs.items():
        _lib.tuning_set(k, v)
    for M in Ms:
        announce("mlp_block_knobs", knobs, M)
        x = x_to_dev(_act(M, HIDDEN, 300 + M))
        got = ops.mlp_forward_fp8(x, *dev, eps=EPS)
        ref = _composed(x, *dev)
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), (knobs, M)


@pytest.mark.parametrize("hidden,Ms", [
    (64, [1, 2]),          # 8 staging pieces per row: XP 2 (smallest)
    (4096, [1, 2]),        # 512 pieces: XP 2 at M = 1, 4 at M = 2
    (4112, [1, 2]),        # 514 pieces: XP 4 / 8
    (8192, [2]),           # largest fused hidden at M = 2
    (8208, [2]),           # one chunk more: separate RMSNorm
    (16384, [1]),          # largest fused hidden at M = 1 (XP 8)
    (16400, [1]),          # one chunk more: separate RMSNorm
])
def test_block_norm_fusion_limits(hidden, Ms):
    inter = 512
    dev = _dev(*_weights(hidden, inter, seed=hidden))
    for M in Ms:
        announce("mlp_block_limits", hidden, M)
        x = x_to_dev(_act(M, hidden, hidden + M))
        got = ops.mlp_forward_fp8(x, *dev, eps=EPS)
        ref = _composed(x, *dev)
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), (hidden, M)


@pytest.mark.parametrize("M", [1, 3, 8, 64, 520])
def test_block_in_place_and_bump_allocator(M):
    announce("mlp_block_inplace_alloc", M)
    dev = _dev(*_weights(HIDDEN, INTER))
    x = x_to_dev(_act(M, HIDDEN, 400 + M))
    ref = ops.mlp_forward_fp8(x, *dev, eps=EPS)
    L = _lib.lib()
    assert L.nmi_alloc_rewind() == 0
    before = ctypes.c_size_t()
    L.nmi_alloc_stats(ctypes.byref(before), None)
    xi = x.clone()
    ops.mlp_forward_fp8(xi, *dev, out=xi, eps=EPS, use_workspace=False)   # in place, bump allocator
    after = ctypes.c_size_t()
    L.nmi_alloc_stats(ctypes.byref(after), None)
    torch.cuda.synchronize()
    assert after.value - before.value >= L.nmi_mlp_workspace_bytes(M, HIDDEN, INTER)
    assert torch.equal(xi.view(torch.int16), ref.view(torch.int16))
    assert L.nmi_alloc_rewind() == 0


def test_binding_mlp_forward_fp8_drop_in():
    """The reference's call (engine.py:198-207): B.mlp_forward_fp8(cur, norm, up_w, up_s, down_w,
    down_s, out, S) after B.reset_allocator(), for decode (S = 1) and a prefill chunk."""
    from nemotron_infer_amd.csrc import binding as B

    dev = _dev(*_weights(HIDDEN, INTER))
    nw, upw, ups, dnw, dns = dev
    for S in (1, 2, 37):
        announce("binding_mlp_forward_fp8", S)
        cur = x_to_dev(_act(S, HIDDEN, 500 + S))
        out = torch.empty_like(cur)
        B.reset_allocator()
        B.mlp_forward_fp8(cur.data_ptr(), nw.data_ptr(), upw.data_ptr(), ups.data_ptr(), dnw.data_ptr(),
                          dns.data_ptr(), out.data_ptr(), S)
        B.sync()
        ref = ops.mlp_forward_fp8(cur, *dev, eps=EPS)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), S


# --------------------------------------------------------------------------------------
# Golden fixture: the reference's MLP block test data
# --------------------------------------------------------------------------------------
def test_block_fixture_hf_and_chain():
    g = load_golden("mlp_block_h64_i256_s8")
    eps = float(g["eps"])
    dev = _dev(g["norm_w"], g["up_codes"], g["up_scale"], g["down_codes"], g["down_scale"])
    exp = g["expected_f32"].astype(np.float64)
    S = g["x_bf16"].shape[0]
    for M in range(1, S + 1):                # GEMV (fused RMSNorm) at M <= 2, 4x4x4 MFMA above
        announce("mlp_block_fixture", M)
        x = g["x_bf16"][:M]
        got = bits(ops.mlp_forward_fp8(x_to_dev(x), *dev, eps=eps))
        check_block(x, got, g["norm_w"], g["up_codes"], g["up_scale"], g["down_codes"], g["down_scale"], eps,
                    f"fixture M={M}")
        r = linear.parity(got, g["chain_f64"][:M])
        assert r["nan_ok"] and r["rel_l2_all"] <= 4e-3, (M, r)
        o = linear.bf16_to_f32(got).astype(np.float64)
        rel = np.linalg.norm(o - exp[:M]) / np.linalg.norm(exp[:M])
        assert rel < 0.05, (M, rel)
