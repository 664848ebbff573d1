"""C ABI and binding checks that need no GPU: the library loads, exports every symbol that
include/*.h declares, rejects bad arguments on the host before launching anything, and the
pybind module mirrors the reference's module surface (names, arities, constants)."""
import ctypes
import glob
import os
import re

import pytest

from nemotron_infer_amd import _lib
from tests.conftest import ROOT


def _declared_symbols():
    syms = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        syms |= set(re.findall(r"\b(nmi_\w+)\s*\(", text))
    return syms


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    declared = _declared_symbols()
    assert len(declared) >= 12
    for name in declared:
        assert hasattr(L, name), f"libnmi.so does not export {name}"
    assert set(_lib.SIGNATURES) == declared, "ctypes signature table out of sync with the header"


def test_abi_version():
    assert _lib.lib().nmi_abi_version() == 10000


FAKE = 0x10000          # 16-byte aligned, never dereferenced: validation fails first


@pytest.mark.parametrize("args,code", [
    # x, ldx, w, ldw, s, y, ldy, M, N, K
    ((0, 64, FAKE, 64, FAKE, FAKE, 8, 1, 8, 64), _lib.NMI_ERR_INVALID_ARG),          # NULL x
    ((FAKE, 64, FAKE, 64, FAKE, FAKE, 8, 0, 8, 64), _lib.NMI_ERR_INVALID_ARG),       # M = 0
    ((FAKE, 64, FAKE, 64, FAKE, FAKE, 8, 1, 0, 64), _lib.NMI_ERR_INVALID_ARG),       # N = 0
    ((FAKE, 72, FAKE, 72, FAKE, FAKE, 8, 1, 8, 72), _lib.NMI_ERR_INVALID_ARG),       # K % 16
    ((FAKE, 64, FAKE, 64, FAKE, FAKE, 8, 1, 8, 0), _lib.NMI_ERR_INVALID_ARG),        # K = 0
    ((FAKE, 32, FAKE, 64, FAKE, FAKE, 8, 2, 8, 64), _lib.NMI_ERR_INVALID_ARG),       # ldx < K
    ((FAKE, 64, FAKE, 64, FAKE, FAKE, 4, 2, 8, 64), _lib.NMI_ERR_INVALID_ARG),       # ldy < N
    ((FAKE, 64, FAKE + 8, 64, FAKE, FAKE, 8, 1, 8, 64), _lib.NMI_ERR_ALIGNMENT),     # W misaligned
    ((FAKE, 64, FAKE, 72, FAKE, FAKE, 8, 1, 8, 64), _lib.NMI_ERR_ALIGNMENT),         # ldw % 16
    ((FAKE + 2, 64, FAKE, 64, FAKE, FAKE, 8, 1, 8, 64), _lib.NMI_ERR_ALIGNMENT),     # x misaligned
    ((FAKE, 68, FAKE, 64, FAKE, FAKE, 8, 2, 8, 64), _lib.NMI_ERR_ALIGNMENT),         # ldx*2 % 16
    ((FAKE, 64, FAKE, 64, FAKE + 2, FAKE, 8, 1, 8, 64), _lib.NMI_ERR_ALIGNMENT),     # s misaligned
    ((FAKE, 64, FAKE, 64, FAKE, FAKE + 1, 8, 1, 8, 64), _lib.NMI_ERR_ALIGNMENT),     # y misaligned
])
def test_linear_rejects_bad_arguments(args, code):
    L = _lib.lib()
    rc = L.nmi_linear_fp8_w8a16(*args, None)
    assert rc == code
    assert L.nmi_last_error().decode().startswith("nmi_linear_fp8_w8a16")
    rc = L.nmi_gemm_fp8_w8a16(*args, None, 0, None)
    assert rc == code


@pytest.mark.parametrize("args,code", [
    ((0, 64, FAKE, 64, FAKE, FAKE, 8, 1, 8, 64), _lib.NMI_ERR_INVALID_ARG),          # NULL x
    ((FAKE, 64, FAKE, 64, FAKE, FAKE, 8, 2, 8, 72), _lib.NMI_ERR_INVALID_ARG),       # K % 16
    ((FAKE, 64, FAKE + 8, 64, FAKE, FAKE, 8, 2, 8, 64), _lib.NMI_ERR_ALIGNMENT),     # W misaligned
    ((FAKE, 64, FAKE, 64, FAKE, FAKE + 1, 8, 2, 8, 64), _lib.NMI_ERR_ALIGNMENT),     # y misaligned
])
def test_batch_rejects_bad_jobs(args, code):
    """nmi_linear_fp8_w8a16_batch validates every job like nmi_linear_fp8_w8a16 (a bad second
    job fails the call, which launches nothing), and the job count."""
    x, ldx, w, ldw, s, y, ldy, M, N, K = args
    good = _lib.LinearJob(FAKE, 64, 64, _lib.LinearGroup(FAKE, 64, FAKE, FAKE, 8, 8))
    bad = _lib.LinearJob(x, ldx, K, _lib.LinearGroup(w, ldw, s, y, ldy, N))
    L = _lib.lib()
    arr = (_lib.LinearJob * 2)(good, bad)
    assert L.nmi_linear_fp8_w8a16_batch(arr, 2, M, None) == code
    assert L.nmi_last_error().decode().startswith("nmi_linear_fp8_w8a16_batch")
    for n in (0, _lib.MAX_BATCH + 1):
        assert L.nmi_linear_fp8_w8a16_batch(arr, n, 2, None) == _lib.NMI_ERR_INVALID_ARG
    assert L.nmi_linear_fp8_w8a16_batch(None, 1, 2, None) == _lib.NMI_ERR_INVALID_ARG


def test_gemv_and_decode_reject_bad_arguments():
    L = _lib.lib()
    assert L.nmi_gemv_fp8(FAKE, FAKE, FAKE, FAKE, 8, 3136 + 8, None) == _lib.NMI_ERR_INVALID_ARG
    assert L.nmi_gemv_fp8(FAKE, FAKE + 4, FAKE, FAKE, 8, 64, None) == _lib.NMI_ERR_ALIGNMENT
    assert L.nmi_gemv_fp8(FAKE, FAKE, FAKE, 0, 8, 64, None) == _lib.NMI_ERR_INVALID_ARG
    assert L.nmi_fp8_e4m3_decode(FAKE, FAKE, FAKE, FAKE, 1.0, 6, None) == _lib.NMI_ERR_INVALID_ARG
    assert L.nmi_fp8_e4m3_decode(FAKE, FAKE + 4, FAKE, FAKE, 1.0, 8, None) == _lib.NMI_ERR_ALIGNMENT
    assert L.nmi_tuning_set(b"no.such.knob", 1) == _lib.NMI_ERR_INVALID_ARG
    assert L.nmi_alloc(16, None) == _lib.NMI_ERR_INVALID_ARG


def test_allocator_stats_without_device():
    total, nslabs = ctypes.c_size_t(123), ctypes.c_size_t(456)
    assert _lib.lib().nmi_alloc_stats(ctypes.byref(total), ctypes.byref(nslabs)) == 0
    assert total.value == 0 and nslabs.value == 0


# Names and argument counts of the reference module (nemotron_infer/csrc/binding.pyi:4-83).
REFERENCE_ARITY = {
    "attn_decode": 11, "attn_decode_fp8": 15, "attn_forward": 11, "attn_forward_fp8": 15,
    "embedding": 4, "free_allocator": 0, "lm_head": 4, "mamba_decode": 14, "mamba_decode_fp8": 16,
    "mamba_forward": 15, "mamba_forward_fp8": 17, "mlp_forward": 6, "mlp_forward_fp8": 8,
    "reset_allocator": 0, "rmsnorm": 4, "sync": 0,
}
REFERENCE_CONSTANTS = {
    "CONV_DIM": 9728, "CONV_K": 4, "G": 8, "H": 96, "HEAD": 128, "HIDDEN": 3136, "H_KV": 8,
    "H_Q": 40, "INTER": 12544, "IN_PROJ": 17504, "N": 128, "P": 80, "VOCAB": 131072,
}


def _arity(fn):
    doc = fn.__doc__.splitlines()[0]
    inner = doc[doc.index("(") + 1: doc.rindex(")")]
    inner = inner[: inner.rindex(")")] if "->" in doc and inner.endswith(")") else inner
    return 0 if not inner.strip() else inner.count(":")


def test_binding_mirrors_reference_module():
    from nemotron_infer_amd.csrc import binding as B

    for name, val in REFERENCE_CONSTANTS.items():
        assert getattr(B, name) == val, name
    for name, n in REFERENCE_ARITY.items():
        fn = getattr(B, name)
        assert _arity(fn) == n, f"{name}: arity {_arity(fn)} != {n}"
    assert _arity(B.linear_fp8) == 10 and _arity(B.gemv_fp8) == 6


def test_out_of_scope_entries_fail_loudly():
    from nemotron_infer_amd.csrc import binding as B

    with pytest.raises(NotImplementedError, match="not part of this build"):
        B.attn_forward(*([0] * 11))
    with pytest.raises(NotImplementedError):
        B.mlp_forward(*([0] * 6))
    with pytest.raises(NotImplementedError):
        B.mamba_forward(*([0] * 15))


def test_binding_reports_validation_errors():
    from nemotron_infer_amd.csrc import binding as B

    with pytest.raises(RuntimeError, match="K=72 must be a positive multiple of 16"):
        B.linear_fp8(FAKE, 72, FAKE, 80, FAKE, FAKE, 8, 1, 8, 72)


def test_rmsnorm_rejects_bad_arguments():
    L = _lib.lib()
    assert L.nmi_rmsnorm_bf16(0, FAKE, FAKE, 1, 64, 1e-5, None) == _lib.NMI_ERR_INVALID_ARG
    assert L.nmi_rmsnorm_bf16(FAKE, FAKE, FAKE, 0, 64, 1e-5, None) == _lib.NMI_ERR_INVALID_ARG
    assert L.nmi_rmsnorm_bf16(FAKE, FAKE, FAKE, 1, 12, 1e-5, None) == _lib.NMI_ERR_INVALID_ARG
    assert L.nmi_rmsnorm_bf16(FAKE + 2, FAKE, FAKE, 1, 64, 1e-5, None) == _lib.NMI_ERR_ALIGNMENT
    assert L.nmi_rmsnorm_bf16(FAKE, FAKE + 4, FAKE, 1, 64, 1e-5, None) == _lib.NMI_ERR_ALIGNMENT
    assert L.nmi_last_error().decode().startswith("nmi_rmsnorm_bf16")


def test_mlp_workspace_bytes():
    L = _lib.lib()
    # RMSNorm fused into the up projection (M = 1; M = 2 where the 16x16x32 skinny kernel does
    # not take the up projection, e.g. hidden not a multiple of 64): only act [M, inter] bf16;
    # otherwise also normed [M, hidden]
    assert L.nmi_mlp_workspace_bytes(1, 3136, 12544) == 12544 * 2
    assert L.nmi_mlp_workspace_bytes(2, 3136, 12544) == 2 * 12544 * 2 + ((2 * 3136 * 2 + 255) // 256) * 256
    assert L.nmi_mlp_workspace_bytes(2, 3136 + 16, 12544) == 2 * 12544 * 2
    assert L.nmi_mlp_workspace_bytes(3, 3136, 12544) == 3 * 12544 * 2 + ((3 * 3136 * 2 + 255) // 256) * 256
    assert L.nmi_mlp_workspace_bytes(64, 64, 256) == 64 * 256 * 2 + 64 * 64 * 2
    assert L.nmi_mlp_workspace_bytes(0, 3136, 12544) == 0


@pytest.mark.parametrize("M,hidden,inter,offs,code", [
    (0, 64, 256, {}, _lib.NMI_ERR_INVALID_ARG),
    (1, 72, 256, {}, _lib.NMI_ERR_INVALID_ARG),          # hidden % 16
    (1, 64, 264, {}, _lib.NMI_ERR_INVALID_ARG),          # inter % 16
    (1, 64, 256, {0: 2}, _lib.NMI_ERR_ALIGNMENT),        # input
    (1, 64, 256, {1: 4}, _lib.NMI_ERR_ALIGNMENT),        # norm_w
    (1, 64, 256, {2: 8}, _lib.NMI_ERR_ALIGNMENT),        # up_w
    (1, 64, 256, {4: 8}, _lib.NMI_ERR_ALIGNMENT),        # down_w
    (1, 64, 256, {5: 2}, _lib.NMI_ERR_ALIGNMENT),        # down_s
    (1, 64, 256, {6: 1}, _lib.NMI_ERR_ALIGNMENT),        # out
    (1, 64, 256, {"ws": 8}, _lib.NMI_ERR_ALIGNMENT),     # workspace
    (1, 64, 256, {"ws_bytes": 16}, _lib.NMI_ERR_WORKSPACE),
])
def test_mlp_rejects_bad_arguments(M, hidden, inter, offs, code):
    L = _lib.lib()
    ptrs = [FAKE + offs.get(i, 0) for i in range(7)]
    ws = FAKE + offs.get("ws", 0)
    ws_bytes = offs.get("ws_bytes", 1 << 20)
    rc = L.nmi_mlp_forward_fp8(*ptrs, M, hidden, inter, 1e-5, ws, ws_bytes, None)
    assert rc == code
    assert L.nmi_last_error().decode().startswith("nmi_mlp_forward_fp8")
    ptrs[3] = 0
    assert L.nmi_mlp_forward_fp8(*ptrs, 1, 64, 256, 1e-5, FAKE, 1 << 20, None) == _lib.NMI_ERR_INVALID_ARG


def test_binding_block_entries_validate():
    from nemotron_infer_amd.csrc import binding as B

    with pytest.raises(RuntimeError, match="16-byte aligned"):
        B.rmsnorm(FAKE + 2, FAKE, FAKE, 1)
    with pytest.raises(RuntimeError, match="M=0"):
        B.mlp_forward_fp8(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 0)


def test_sdpa_and_attention_workspace_bytes():
    L = _lib.lib()
    # one split (no partials) up to 64 positions; fp32 (m, l, o[128]) per (head, split) beyond
    assert L.nmi_sdpa_decode_workspace_bytes(40, 8, 0) == 0
    assert L.nmi_sdpa_decode_workspace_bytes(40, 8, 64) == 0
    assert L.nmi_sdpa_decode_workspace_bytes(40, 8, 65) == 40 * 2 * 130 * 4
    assert L.nmi_sdpa_decode_workspace_bytes(40, 8, 4096) == 40 * 32 * 130 * 4
    assert L.nmi_sdpa_decode_workspace_bytes(40, 0, 10) == 0
    base = 2 * 10240 + 2 * 2048 + ((3136 * 2 + 255) // 256) * 256
    assert L.nmi_attn_decode_workspace_bytes(3136, 40, 8, 10) == base
    assert L.nmi_attn_decode_workspace_bytes(3136, 40, 8, 4096) == base + 40 * 32 * 130 * 4
    assert L.nmi_attn_decode_workspace_bytes(8, 40, 8, 10) == 0


@pytest.mark.parametrize("S,cap,H,H_KV,offs,code", [
    (-1, 8, 40, 8, {}, _lib.NMI_ERR_INVALID_ARG),
    (8, 8, 40, 8, {}, _lib.NMI_ERR_INVALID_ARG),          # no room for the new token
    (0, 8, 40, 6, {}, _lib.NMI_ERR_INVALID_ARG),          # 40 % 6
    (0, 8, 56, 8, {}, _lib.NMI_ERR_INVALID_ARG),          # 7 query heads per KV head
    (0, 8, 40, 0, {}, _lib.NMI_ERR_INVALID_ARG),
    (0, 8, 40, 8, {0: 8}, _lib.NMI_ERR_ALIGNMENT),        # q
    (0, 8, 40, 8, {1: 8}, _lib.NMI_ERR_ALIGNMENT),        # k_cache
    (0, 8, 40, 8, {5: 2}, _lib.NMI_ERR_ALIGNMENT),        # v_new
    (0, 8, 40, 8, {3: 1}, _lib.NMI_ERR_ALIGNMENT),        # o
    (100, 128, 40, 8, {"ws_bytes": 16}, _lib.NMI_ERR_WORKSPACE),
])
def test_sdpa_rejects_bad_arguments(S, cap, H, H_KV, offs, code):
    L = _lib.lib()
    ptrs = [FAKE + offs.get(i, 0) for i in range(6)]
    rc = L.nmi_sdpa_decode_bf16(*ptrs, S, cap, H, H_KV, FAKE, offs.get("ws_bytes", 1 << 20), None)
    assert rc == code
    assert L.nmi_last_error().decode().startswith("nmi_sdpa_decode_bf16")
    ptrs[2] = 0
    assert L.nmi_sdpa_decode_bf16(*ptrs, 0, 8, 40, 8, None, 0, None) == _lib.NMI_ERR_INVALID_ARG


@pytest.mark.parametrize("hidden,S,cap,offs,code", [
    (3136, 0, 0, {}, _lib.NMI_ERR_INVALID_ARG),
    (3144, 0, 8, {}, _lib.NMI_ERR_INVALID_ARG),            # hidden % 16
    (3136, 0, 8, {0: 2}, _lib.NMI_ERR_ALIGNMENT),          # input
    (3136, 0, 8, {8: 8}, _lib.NMI_ERR_ALIGNMENT),          # o_w
    (3136, 0, 8, {10: 8}, _lib.NMI_ERR_ALIGNMENT),         # k_cache
    (3136, 0, 8, {9: 2}, _lib.NMI_ERR_ALIGNMENT),          # o_s
    (3136, 0, 8, {"ws": 8}, _lib.NMI_ERR_ALIGNMENT),
    (3136, 0, 8, {"ws_bytes": 64}, _lib.NMI_ERR_WORKSPACE),
])
def test_attn_decode_rejects_bad_arguments(hidden, S, cap, offs, code):
    L = _lib.lib()
    ptrs = [FAKE + offs.get(i, 0) for i in range(12)]
    out = FAKE + offs.get(12, 0)
    rc = L.nmi_attn_decode_fp8(*ptrs, S, cap, out, hidden, 40, 8, 1e-5, FAKE + offs.get("ws", 0),
                               offs.get("ws_bytes", 1 << 20), None)
    assert rc == code
    assert L.nmi_last_error().decode().startswith("nmi_attn_decode_fp8")


def test_binding_attn_decode_validates():
    from nemotron_infer_amd.csrc import binding as B

    with pytest.raises(RuntimeError, match="S_cache=5 cache_cap=5"):
        B.attn_decode_fp8(*([FAKE] * 12), 5, 5, FAKE)


def test_mamba_decode_workspace_bytes_and_rejections():
    L = _lib.lib()
    proj_ld = 17504                                   # already a multiple of 8
    r256 = lambda b: (b + 255) // 256 * 256  # noqa: E731
    want = r256(2 * proj_ld) + 2 * r256(2 * 7680) + r256(3136 * 2)
    assert L.nmi_mamba_decode_workspace_bytes(1, 3136, 96, 80, 8, 128) == want
    assert L.nmi_mamba_decode_workspace_bytes(0, 3136, 96, 80, 8, 128) == 0
    ptrs = [FAKE] * 15

    def call(*dims, ptrs=ptrs, ws=FAKE, ws_bytes=1 << 24):
        return L.nmi_mamba_decode_fp8(*ptrs, *dims, 1e-5, ws, ws_bytes, None)

    assert call(0, 3136, 96, 80, 8, 128, 4) == _lib.NMI_ERR_INVALID_ARG
    assert call(1, 3136, 96, 80, 8, 64, 4) == _lib.NMI_ERR_INVALID_ARG     # d_state
    assert call(1, 3136, 96, 80, 8, 128, 3) == _lib.NMI_ERR_INVALID_ARG    # conv_k
    assert call(1, 3136, 96, 80, 7, 128, 4) == _lib.NMI_ERR_INVALID_ARG    # groups do not divide heads
    assert call(1, 3136, 96, 136, 8, 128, 4) == _lib.NMI_ERR_INVALID_ARG   # head_dim > 128
    assert call(1, 3136, 96, 80, 8, 128, 4, ws_bytes=64) == _lib.NMI_ERR_WORKSPACE
    bad = list(ptrs)
    bad[13] = FAKE + 4                                                     # ssm_state
    assert call(1, 3136, 96, 80, 8, 128, 4, ptrs=bad) == _lib.NMI_ERR_ALIGNMENT
    bad[13] = 0
    assert call(1, 3136, 96, 80, 8, 128, 4, ptrs=bad) == _lib.NMI_ERR_INVALID_ARG
    assert L.nmi_last_error().decode().startswith("nmi_mamba_decode_fp8")
    # the mixer op
    assert L.nmi_mamba_mixer_decode(FAKE, 17500, *([FAKE] * 10), 1, 96, 80, 8, 128, 4, 1e-5,
                                    None) == _lib.NMI_ERR_INVALID_ARG          # proj_ld < PROJ
    assert L.nmi_mamba_mixer_decode(FAKE + 8, 17504, *([FAKE] * 10), 1, 96, 80, 8, 128, 4, 1e-5,
                                    None) == _lib.NMI_ERR_ALIGNMENT


def test_binding_mamba_decode_validates():
    from nemotron_infer_amd.csrc import binding as B

    with pytest.raises(RuntimeError, match="batch=0"):
        B.mamba_decode_fp8(*([FAKE] * 15), 0)


def test_gemv_chain_workspace_bytes():
    """Chains synchronise through launch order only: no launch needs a workspace."""
    L = _lib.lib()
    for n in (0, 1, 4, 84, 4096, 4097):
        assert L.nmi_gemv_chain_workspace_bytes(n) == 0


def _phase(x=FAKE, K=64, group=(FAKE, 64, FAKE, FAKE, 8, 8), ngroups=1, wait=0):
    """A phase of ngroups copies of one group (ngroups may exceed the array to test the bound)."""
    ph = _lib.GemvPhase()
    ph.x_bf16, ph.K, ph.ngroups, ph.wait_prev = x, K, ngroups, wait
    for i in range(min(ngroups, _lib.MAX_GROUPS)):
        ph.groups[i] = _lib.LinearGroup(*group)
    return ph


@pytest.mark.parametrize("phase,code", [
    (dict(x=0), _lib.NMI_ERR_INVALID_ARG),                                       # NULL x
    (dict(K=72), _lib.NMI_ERR_INVALID_ARG),                                      # K % 16
    (dict(ngroups=0), _lib.NMI_ERR_INVALID_ARG),                                 # no group
    (dict(ngroups=5), _lib.NMI_ERR_INVALID_ARG),                                 # > 4 groups
    (dict(group=(FAKE + 8, 64, FAKE, FAKE, 8, 8)), _lib.NMI_ERR_ALIGNMENT),      # W misaligned
    (dict(group=(FAKE, 64, FAKE, FAKE, 8, 0)), _lib.NMI_ERR_INVALID_ARG),        # N = 0
    (dict(x=FAKE + 2), _lib.NMI_ERR_ALIGNMENT),                                  # x misaligned
])
def test_gemv_chain_rejects_bad_phases(phase, code):
    """A bad second phase is rejected on the host, before any device call."""
    L = _lib.lib()
    arr = (_lib.GemvPhase * 2)(_phase(), _phase(**phase))
    h = ctypes.c_void_p()
    assert L.nmi_gemv_chain_create(arr, 2, ctypes.byref(h)) == code
    assert not h.value
    assert L.nmi_last_error().decode().startswith("nmi_gemv_chain_create")


def test_gemv_chain_handle_errors():
    L = _lib.lib()
    h = ctypes.c_void_p()
    arr = (_lib.GemvPhase * 1)(_phase())
    assert L.nmi_gemv_chain_create(arr, 0, ctypes.byref(h)) == _lib.NMI_ERR_INVALID_ARG
    assert L.nmi_gemv_chain_create(arr, 4097, ctypes.byref(h)) == _lib.NMI_ERR_INVALID_ARG
    assert L.nmi_gemv_chain_create(None, 1, ctypes.byref(h)) == _lib.NMI_ERR_INVALID_ARG
    assert L.nmi_gemv_chain_create(arr, 1, None) == _lib.NMI_ERR_INVALID_ARG
    assert L.nmi_gemv_chain_launch(None, None, 0, None) == _lib.NMI_ERR_INVALID_ARG
    assert L.nmi_gemv_chain_destroy(None) == _lib.NMI_OK


def test_tuning_knobs_from_environment():
    """NMI_TUNING applies knobs when the library is loaded; an unknown knob fails loudly."""
    import subprocess
    import sys

    code = "from nemotron_infer_amd import _lib; _lib.lib(); print('loaded')"
    env = dict(os.environ, NMI_TUNING="s4.ks=2, s4.u=4")
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "loaded" in r.stdout, r.stderr
    env["NMI_TUNING"] = "no.such.knob=1"
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "unknown knob 'no.such.knob'" in r.stderr


def test_workspace_error_offset_matches_the_header():
    import re

    hdr = open(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                            "nmi_fp8_linear.h")).read()
    assert int(re.search(r"#define NMI_WS_ERROR_OFFSET (\d+)", hdr).group(1)) == _lib.NMI_WS_ERROR_OFFSET
    L = _lib.lib()
    for knob in ("gemm.sk_spin", "gemm.sk_lostflag", "gemv.grid", "gemv.balance", "sdpa.chunk"):
        assert L.nmi_tuning_set(knob.encode(), 0) == 0, knob


def test_async_error_is_a_host_side_word():
    """nmi_async_status reads the device's asynchronous error word in host memory without a GPU
    call: before any stream-K launch in the process there is none to report.  NMI_ERR_ASYNC has
    one value in the header and the binding, and reaches Python as an NmiError with its code."""
    L = _lib.lib()
    assert L.nmi_async_status() == _lib.NMI_OK
    header = open(os.path.join(ROOT, "include", "nmi_fp8_linear.h")).read()
    assert re.search(r"NMI_ERR_ASYNC\s*=\s*-6\b", header) and _lib.NMI_ERR_ASYNC == -6
    with pytest.raises(_lib.NmiError) as e:
        _lib.check(_lib.NMI_ERR_ASYNC, "an entry point")
    assert e.value.code == _lib.NMI_ERR_ASYNC
