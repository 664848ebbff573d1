"""Host-side argument checks of the torch front end (nemotron_infer_amd/ops.py), no GPU needed.

Every call validates dtypes, shapes and strides before it touches the library, so these run on
CPU tensors: a bad argument raises TypeError / ValueError, and a fully valid call on CPU
tensors raises because the tensors are not on a GPU (nothing reaches the C ABI).  The cases
cover the ways a caller can hand over a buffer the kernels would misread: a strided or
non-contiguous output (written as if contiguous), a wrong-shaped output, strided weight rows,
scales of the wrong dtype, length or layout, and mismatched K.
"""
import pytest
import torch

from nemotron_infer_amd import ops

M, N, K = 3, 32, 64


def _args(m=M):
    x = torch.zeros(m, K, dtype=torch.bfloat16)
    w = torch.zeros(N, K, dtype=torch.uint8)
    s = torch.ones(N, dtype=torch.float32)
    return x, w, s


def test_valid_cpu_call_is_refused_before_the_library():
    x, w, s = _args()
    with pytest.raises(ValueError, match="GPU"):
        ops.linear_fp8_w8a16(x, w, s)
    with pytest.raises(ValueError, match="GPU"):
        ops.gemm_fp8_w8a16(x, w, s)
    with pytest.raises(ValueError, match="GPU"):
        ops.gemv_fp8(x[0], w, s)


@pytest.mark.parametrize("make_out,exc", [
    (lambda: torch.empty(M, 2 * N, dtype=torch.bfloat16)[:, ::2], ValueError),     # strided columns
    (lambda: torch.empty(2 * M, N, dtype=torch.bfloat16)[::2], ValueError),         # strided rows
    (lambda: torch.empty(N, M, dtype=torch.bfloat16).t(), ValueError),              # transposed
    (lambda: torch.empty(M, N + 1, dtype=torch.bfloat16), ValueError),              # wrong shape
    (lambda: torch.empty(M * N, dtype=torch.bfloat16), ValueError),                 # flat
    (lambda: torch.empty(M, N, dtype=torch.float16), TypeError),                    # wrong dtype
])
def test_linear_rejects_bad_outputs(make_out, exc):
    x, w, s = _args()
    with pytest.raises(exc):
        ops.linear_fp8_w8a16(x, w, s, out=make_out())
    with pytest.raises(exc):
        ops.gemm_fp8_w8a16(x, w, s, out=make_out())
    with pytest.raises(exc):
        ops.linear_fp8_w8a16_grouped(x, [(w, s)], outs=[make_out()])


def test_m1_output_may_be_a_vector_but_not_strided():
    x, w, s = _args(1)
    with pytest.raises(ValueError, match="GPU"):                                    # [N] is fine
        ops.linear_fp8_w8a16(x[0], w, s, out=torch.empty(N, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="contiguous"):
        ops.linear_fp8_w8a16(x[0], w, s, out=torch.empty(2 * N, dtype=torch.bfloat16)[::2])
    with pytest.raises(ValueError, match="contiguous"):
        ops.gemv_fp8(x[0], w, s, out=torch.empty(2 * N, dtype=torch.bfloat16)[::2])


@pytest.mark.parametrize("make_w,exc", [
    (lambda: torch.zeros(N, 2 * K, dtype=torch.uint8)[:, ::2], ValueError),         # strided row elements
    (lambda: torch.zeros(K, N, dtype=torch.uint8).t(), ValueError),                 # column-major
    (lambda: torch.zeros(N, K + 16, dtype=torch.uint8), ValueError),                # K mismatch
    (lambda: torch.zeros(N * K, dtype=torch.uint8), ValueError),                    # not 2-D
    (lambda: torch.zeros(N, K, dtype=torch.int8), TypeError),                       # wrong dtype
])
def test_rejects_bad_weights(make_w, exc):
    x, _, s = _args()
    with pytest.raises(exc):
        ops.linear_fp8_w8a16(x, make_w(), s)
    with pytest.raises(exc):
        ops.gemm_fp8_w8a16(x, make_w(), s)


@pytest.mark.parametrize("make_s,exc", [
    (lambda: torch.ones(N, dtype=torch.float64), TypeError),
    (lambda: torch.ones(N, dtype=torch.bfloat16), TypeError),
    (lambda: torch.ones(2 * N, dtype=torch.float32)[::2], ValueError),             # strided
    (lambda: torch.ones(N + 1, dtype=torch.float32), ValueError),                   # wrong length
    (lambda: torch.ones(N, 1, dtype=torch.float32), ValueError),                    # not 1-D
])
def test_rejects_bad_scales(make_s, exc):
    x, w, _ = _args()
    with pytest.raises(exc):
        ops.linear_fp8_w8a16(x, w, make_s())
    with pytest.raises(exc):
        ops.gemm_fp8_w8a16(x, w, make_s())
    with pytest.raises(exc):
        ops.gemv_fp8(x[0], w, make_s())
    with pytest.raises(exc):
        ops.linear_fp8_w8a16_grouped(x, [(w, make_s())])


def test_gemv_checks_x():
    _, w, s = _args()
    with pytest.raises(ValueError, match="x must"):
        ops.gemv_fp8(torch.zeros(K + 16, dtype=torch.bfloat16), w, s)
    with pytest.raises(ValueError, match="x must"):
        ops.gemv_fp8(torch.zeros(2 * K, dtype=torch.bfloat16)[::2], w, s)
    with pytest.raises(ValueError, match="x must"):
        ops.gemv_fp8(torch.zeros(K, dtype=torch.float32), w, s)


def test_chain_rejects_strided_or_short_outputs():
    x = torch.zeros(K, dtype=torch.bfloat16)
    w = torch.zeros(N, K, dtype=torch.uint8)
    s = torch.ones(N, dtype=torch.float32)
    buf = torch.empty(2 * N, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="contiguous"):
        ops.GemvChain([(x, [(w, s, buf[::2])], False)])                             # strided y
    with pytest.raises(ValueError):
        ops.GemvChain([(x, [(w, s, buf[:N - 1])], False)])                          # too short
    with pytest.raises(ValueError, match="x must"):
        ops.GemvChain([(torch.zeros(2 * K, dtype=torch.bfloat16)[::2], [(w, s, buf[:N])], False)])
    with pytest.raises(ValueError, match="K"):
        ops.GemvChain([(x, [(torch.zeros(N, K + 16, dtype=torch.uint8), s, buf[:N])], False)])


def test_mlp_block_checks():
    hid, inter = 64, 128
    x = torch.zeros(2, hid, dtype=torch.bfloat16)
    nw = torch.ones(hid, dtype=torch.float32)
    uw, us = torch.zeros(inter, hid, dtype=torch.uint8), torch.ones(inter, dtype=torch.float32)
    dw, ds = torch.zeros(hid, inter, dtype=torch.uint8), torch.ones(hid, dtype=torch.float32)
    with pytest.raises(ValueError, match="GPU"):
        ops.mlp_forward_fp8(x, nw, uw, us, dw, ds)
    with pytest.raises(ValueError):
        ops.mlp_forward_fp8(x, nw, uw, us, torch.zeros(hid, inter + 16, dtype=torch.uint8), ds)
    with pytest.raises(ValueError):
        ops.mlp_forward_fp8(x, nw, uw, us, dw, ds, out=torch.empty(4, hid, dtype=torch.bfloat16)[::2])
    with pytest.raises(ValueError, match="norm_w"):
        ops.mlp_forward_fp8(x, nw[:hid - 8], uw, us, dw, ds)
