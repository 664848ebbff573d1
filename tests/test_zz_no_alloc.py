"""nmi_mlp_forward_fp8_noalloc (no counterpart in the reference; for callers that cannot
allocate: graph capture, tight serving loops): the fp8 MLP block with its transient buffers in a
library-owned device array instead of a workspace or the bump allocator.  Through the C ABI, on
two calls in a row (the second smaller, so stale contents of the shared array from the first
would show): at M = 40 (the short-prompt GEMM, which runs unsplit here) exactly the bytes
nmi_mlp_forward_fp8 gives with its K split switched off (gemm.splits = 1), and the default
(split) result up to float32 summation order (the block's end-to-end gate, rel_l2 <= 4e-3, since
a one-ulp flip of an up-projection output moves its whole row through relu^2 and the down
projection); at M = 1 exactly the default bytes.  Sizes whose buffers exceed the array are
rejected."""
import ctypes

import pytest
import torch

from nemotron_infer_amd import _lib, synth
from oracle import linear
from tests.gpu_util import DEV, announce, bits

pytestmark = pytest.mark.gpu

HID, INTER = synth.HIDDEN, synth.INTER


def _weights():
    up = synth.make_weight(INTER, HID, 8100, DEV)
    dn = synth.make_weight(HID, INTER, 8101, DEV)
    g = torch.Generator(device=DEV).manual_seed(8102)
    nw = (1.0 + 0.1 * torch.randn(HID, generator=g, device=DEV)).float()
    return up, dn, nw


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _call_noalloc(L, x, nw, up, dn, out, M):
    return L.nmi_mlp_forward_fp8_noalloc(x.data_ptr(), nw.data_ptr(), up[0].data_ptr(), up[1].data_ptr(),
                                         dn[0].data_ptr(), dn[1].data_ptr(), out.data_ptr(), M, HID, INTER,
                                         ctypes.c_float(1e-5), _stream())


def _call_ws(L, x, nw, up, dn, out, M):
    need = L.nmi_mlp_workspace_bytes(M, HID, INTER)
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    rc = L.nmi_mlp_forward_fp8(x.data_ptr(), nw.data_ptr(), up[0].data_ptr(), up[1].data_ptr(),
                               dn[0].data_ptr(), dn[1].data_ptr(), out.data_ptr(), M, HID, INTER,
                               ctypes.c_float(1e-5), ws.data_ptr(), need, _stream())
    torch.cuda.synchronize()
    return rc


@pytest.fixture
def _splits_reset():
    yield
    _lib.tuning_set("gemm.splits", 0)


def test_noalloc_matches_the_workspace_entry_point(_splits_reset):
    L = _lib.lib()
    up, dn, nw = _weights()
    assert L.nmi_mlp_noalloc_scratch_bytes() == 4 << 20
    for M in (40, 1):                              # the second call smaller than the first
        announce("noalloc", M)
        x = synth.make_act(M, HID, 8200 + M, DEV)
        got = torch.full_like(x, float("nan"))
        want = torch.full_like(x, float("nan"))
        unsplit = torch.full_like(x, float("nan"))
        _lib.check(_call_noalloc(L, x, nw, up, dn, got, M), "nmi_mlp_forward_fp8_noalloc")
        torch.cuda.synchronize()
        _lib.check(_call_ws(L, x, nw, up, dn, want, M), "nmi_mlp_forward_fp8")
        _lib.tuning_set("gemm.splits", 1)
        _lib.check(_call_ws(L, x, nw, up, dn, unsplit, M), "nmi_mlp_forward_fp8 (gemm.splits = 1)")
        _lib.tuning_set("gemm.splits", 0)
        assert not torch.isnan(got.float()).any()
        assert torch.equal(got.view(torch.int16), unsplit.view(torch.int16)), f"M={M} vs unsplit"
        if M <= 16:
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"M={M}"
        else:
            r = linear.parity(bits(got), bits(want))
            assert r["nan_ok"] and r["rel_l2_all"] <= 4e-3, (M, r)


def test_noalloc_rejects_sizes_beyond_the_array():
    L = _lib.lib()
    up, dn, nw = _weights()
    limit = L.nmi_mlp_noalloc_scratch_bytes()
    # the block's buffers without the GEMMs' split partials: the workspace query with the split off
    _lib.tuning_set("gemm.splits", 1)
    try:
        M = next(m for m in range(1, 4096) if L.nmi_mlp_workspace_bytes(m, HID, INTER) > limit)
    finally:
        _lib.tuning_set("gemm.splits", 0)
    assert M == 134                                # M <= 133 fit at the model's sizes
    announce("noalloc_fits", 133)
    x = synth.make_act(133, HID, 8301, DEV)
    out = torch.empty_like(x)
    _lib.check(_call_noalloc(L, x, nw, up, dn, out, 133), "nmi_mlp_forward_fp8_noalloc M=133")
    torch.cuda.synchronize()
    announce("noalloc_reject", M)
    x = synth.make_act(M, HID, 8300, DEV)
    out = torch.empty_like(x)
    assert _call_noalloc(L, x, nw, up, dn, out, M) == _lib.NMI_ERR_WORKSPACE
    assert "scratch" in L.nmi_last_error().decode()
    assert _call_noalloc(L, x, nw, up, dn, out, 0) == _lib.NMI_ERR_INVALID_ARG
