"""GPU parity of nmi_linear_fp8_w8a16_batch: independent linears, each with its own activations,
in one dispatch (one launch of the 16x16x32 skinny kernel for 2 <= M <= 16), against separate
calls and the torch fp32 dequant-then-F.linear oracle.

Tolerance: rel_l2 <= 1e-3 and max |diff| <= 2 bf16 ulp at max(|ref|, 2^-8 rms(ref)) per job.
Bit-exact properties: with the skinny kernel's wave count fixed (tuning knob s16.w), a job's
output equals its separate call bit for bit (the kernel sums every output over the same k order
whatever else the launch holds); where a job falls back (K not a multiple of 64, M outside 2 ..
16) every job equals its separate call; repeated calls and graph replays are bit-identical.
"""
import numpy as np
import pytest
import torch

from nemotron_infer_amd import _lib, ops, synth
from tests.gpu_util import DEV, announce, assert_parity, bits, oracle_bits, s_to_dev, w_to_dev, x_to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _reset_tuning():
    for k in ("s16.w", "s16"):
        _lib.tuning_set(k, 0)
    yield
    for k in ("s16.w", "s16"):
        _lib.tuning_set(k, 0)


def _jobs(M, shapes, seed):
    """One job per (N, K): its own seeded activations, log-uniform per-row scales."""
    out = []
    for i, (N, K) in enumerate(shapes):
        w, s = synth.make_weight(N, K, seed + 7 * i, "cpu", scales="log_uniform")
        x = synth.make_act(M, K, seed + 7 * i + 1, "cpu")
        out.append((x.view(torch.int16).numpy().view(np.uint16), w.numpy(), s.numpy()))
    return out


def _run(M, shapes, seed, label, nw=2):
    host = _jobs(M, shapes, seed)
    dev = [(x_to_dev(x), w_to_dev(w), s_to_dev(s)) for x, w, s in host]
    _lib.tuning_set("s16.w", nw)
    ys = ops.linear_fp8_w8a16_batch(dev)
    again = ops.linear_fp8_w8a16_batch(dev)
    sep = [ops.linear_fp8_w8a16(x, w, s) for x, w, s in dev]
    torch.cuda.synchronize()
    for i, ((x, w, s), y, y2, ys_) in enumerate(zip(host, ys, again, sep)):
        assert torch.equal(y.view(torch.int16), y2.view(torch.int16)), f"{label} job {i}: not deterministic"
        assert np.array_equal(bits(y), bits(ys_)), f"{label} job {i}: differs from its separate call"
        assert_parity(bits(y), oracle_bits(x, w, s), f"{label} job {i}", per_row_scales=True)
    return dev, ys


@pytest.mark.parametrize("M", synth.SKINNY_M)
@pytest.mark.parametrize("nw", [2, 4])
def test_config2_decode_set_as_one_batch(M, nw):
    """Config 2's decode set as one launch: q, k, v, o, up and down, each on its own
    activations (q, k and v included), at M = 2, 4, 8, 16, with two and four waves per
    workgroup."""
    shapes = [(l.N, l.K) for l in synth.SKINNY_SET]
    announce("batch_config2", M, nw, shapes)
    _run(M, shapes, 900 + M, f"config 2 M={M} nw={nw}", nw=nw)


def test_ragged_and_eight_jobs():
    """Eight jobs (the maximum) with ragged N (not multiples of 16 or 32) and K from 64 to 12544,
    M = 7."""
    shapes = [(40, 64), (1000, 3136), (17, 128), (3136, 12544), (520, 1024), (33, 192), (4096, 256), (8, 640)]
    announce("batch_ragged", shapes)
    _run(7, shapes, 4100, "ragged")


@pytest.mark.parametrize("M", [1, 3, 24])
def test_fallback_runs_each_job_as_its_separate_call(M):
    """A job the skinny kernel cannot take (K = 1040, not a multiple of 64) -- or M outside
    2 .. 16 -- sends every job down its separate call's path: outputs equal the separate calls
    bit for bit."""
    shapes = [(300, 3136), (200, 1040), (64, 512)]
    announce("batch_fallback", M, shapes)
    host = _jobs(M, shapes, 4200 + M)
    dev = [(x_to_dev(x), w_to_dev(w), s_to_dev(s)) for x, w, s in host]
    ys = ops.linear_fp8_w8a16_batch(dev)
    sep = [ops.linear_fp8_w8a16(x, w, s, use_workspace=False) for x, w, s in dev]
    torch.cuda.synchronize()
    for i, ((x, w, s), y, ys_) in enumerate(zip(host, ys, sep)):
        assert np.array_equal(bits(y), bits(ys_)), f"M={M} job {i}"
        assert_parity(bits(y), oracle_bits(x, w, s), f"fallback M={M} job {i}", per_row_scales=True)


def test_graph_replays_and_strided_outputs():
    """A captured batch replays bit-identically to the eager call (eager work between replays).
    Through the C ABI the outputs may be column views of one wider buffer (row stride ldy): the
    values equal the contiguous outputs and the buffer's other columns stay untouched."""
    M = 16
    shapes = [(l.N, l.K) for l in synth.SKINNY_SET[:4]]
    announce("batch_graph_strided", M, shapes)
    host = _jobs(M, shapes, 4300)
    dev = [(x_to_dev(x), w_to_dev(w), s_to_dev(s)) for x, w, s in host]
    ref = [y.clone() for y in ops.linear_fp8_w8a16_batch(dev)]
    outs = [torch.empty((M, n), dtype=torch.bfloat16, device=DEV) for n, _ in shapes]
    stream = torch.cuda.Stream()
    ops.linear_fp8_w8a16_batch(dev, outs=outs)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        ops.linear_fp8_w8a16_batch(dev, outs=outs)
    for rep in range(3):
        for y in outs:
            y.zero_()
        g.replay()
        torch.cuda.synchronize()
        for i, (y, r) in enumerate(zip(outs, ref)):
            assert torch.equal(y.view(torch.int16), r.view(torch.int16)), (rep, i)
        ops.linear_fp8_w8a16_batch(dev)                   # eager work between replays
        torch.cuda.synchronize()
    total = sum(n for n, _ in shapes)
    big = torch.full((M, total + 8), 3.0, dtype=torch.bfloat16, device=DEV)
    offs = np.cumsum([0] + [n for n, _ in shapes])
    arr = (_lib.LinearJob * len(shapes))()
    for i, (x, w, s) in enumerate(dev):
        y = big[:, offs[i]:offs[i + 1]]
        arr[i] = _lib.LinearJob(x.data_ptr(), x.stride(0), x.shape[1],
                                _lib.LinearGroup(w.data_ptr(), w.stride(0), s.data_ptr(), y.data_ptr(), y.stride(0),
                                                 w.shape[0]))
    _lib.check(_lib.lib().nmi_linear_fp8_w8a16_batch(arr, len(shapes), M, None), "batch (column views)")
    torch.cuda.synchronize()
    assert torch.all(big[:, total:] == 3.0)
    for i, r in enumerate(ref):
        assert torch.equal(big[:, offs[i]:offs[i + 1]].contiguous().view(torch.int16), r.view(torch.int16)), i
