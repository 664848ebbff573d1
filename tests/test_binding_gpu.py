"""The pybind drop-in module and the hipMalloc bump allocator on the GPU."""
import ctypes

import numpy as np
import pytest
import torch

from nemotron_infer_amd import _lib, ops, synth
from tests.gpu_util import DEV, announce, assert_parity, bits, oracle_bits, s_to_dev, w_to_dev, x_to_dev

pytestmark = pytest.mark.gpu


def _alloc(n):
    p = ctypes.c_void_p()
    _lib.check(_lib.lib().nmi_alloc(n, ctypes.byref(p)), "nmi_alloc")
    return p.value


def _stats():
    t, s = ctypes.c_size_t(), ctypes.c_size_t()
    _lib.lib().nmi_alloc_stats(ctypes.byref(t), ctypes.byref(s))
    return t.value, s.value


def test_bump_allocator_rewind_replays_without_new_slabs():
    """allocator.cuh:58-175 semantics: 128-byte alignment, rewind keeps slabs and replays the
    same addresses, a request larger than a slab gets its own slab, reset frees them all."""
    announce("allocator")
    from nemotron_infer_amd.csrc import binding as B

    B.free_allocator()
    sizes = [1, 3136 * 2, 12544 * 2, 100, 40 << 20, 30 << 20, 200 << 20, 5]
    first = [_alloc(n) for n in sizes]
    assert all(p % 128 == 0 for p in first)
    total, nslabs = _stats()
    assert total == sum((max(n, 1) + 127) // 128 * 128 for n in sizes)
    B.reset_allocator()
    assert _stats() == (0, nslabs)
    again = [_alloc(n) for n in sizes]
    assert again == first and _stats()[1] == nslabs
    # a block is usable device memory: the GEMV writes its output into one
    N, K = 64, 3136
    w, s = synth.make_weight(N, K, 3, "cpu")
    x = synth.make_act(1, K, 4, "cpu")
    xd, wd, sd = x.to(DEV), w.to(DEV), s.to(DEV)
    ref = ops.gemv_fp8(xd, wd, sd)
    B.gemv_fp8(xd.data_ptr(), wd.data_ptr(), sd.data_ptr(), again[6], N, K)
    out = torch.empty(N, dtype=torch.bfloat16, device=DEV)
    B.gemv_fp8(xd.data_ptr(), wd.data_ptr(), sd.data_ptr(), out.data_ptr(), N, K)
    B.sync()
    assert torch.equal(out, ref)
    B.free_allocator()
    assert _stats() == (0, 0)


def test_binding_linear_and_gemv_match_c_abi():
    from nemotron_infer_amd.csrc import binding as B

    N, K = 3136, 12544
    announce("binding", N, K)
    w, s = synth.make_weight(N, K, 11, "cpu")
    x = synth.make_act(1, K, 12, "cpu", kind="relu2")
    xb = x.view(torch.int16).numpy().view(np.uint16)
    xd, wd, sd = x.to(DEV), w.to(DEV), s.to(DEV)
    y1 = torch.empty((1, N), dtype=torch.bfloat16, device=DEV)
    y2 = torch.empty((N,), dtype=torch.bfloat16, device=DEV)
    B.linear_fp8(xd.data_ptr(), K, wd.data_ptr(), K, sd.data_ptr(), y1.data_ptr(), N, 1, N, K)
    B.gemv_fp8(xd.data_ptr(), wd.data_ptr(), sd.data_ptr(), y2.data_ptr(), N, K)
    B.sync()
    assert torch.equal(y1[0], y2)
    assert_parity(bits(y2), oracle_bits(xb[0], w.numpy(), s.numpy()), "binding gemv")
    y3 = ops.linear_fp8_w8a16(xd, wd, sd)
    assert torch.equal(y3, y1)
