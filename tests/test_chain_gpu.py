"""GPU tests of the GEMV chain (nmi_gemv_chain_*: the GEMVs of a decode step in as few launches as
their dependencies allow).

* The config-1 decode set (q|k|v grouped, o, up, down) as a chain gives the same bytes as the
  separate launches, also when o, up and down each wait for the phase before them (four
  launches).
* A dependent chain -- each phase's x is the previous phase's output -- equals the same GEMVs
  launched one after the other, for every phase, also with a 20-phase chain of ragged N and
  small K.
* A phase that does not wait may finish before the phase ahead of it (a few rows after a large
  phase): results stay right over repeated launches.
* The same with one workgroup per CU (tuning knob chain.wgs = 1), so that every wave walks many
  steps of several phases in turn.
* Phases whose K spans several slices; phases of four groups with ragged and single-row groups.
* Graph replays (with eager work between them) equal the eager launch.
* Parity with the oracle (fp32 dequant-then-F.linear, rounded once).
"""
import numpy as np
import pytest
import torch

from nemotron_infer_amd import _lib, ops, synth
from tests.gpu_util import DEV, announce, assert_parity, bits, oracle_bits

pytestmark = pytest.mark.gpu


@pytest.fixture(params=[0, 1], ids=["resident_grid", "one_wg_per_cu"])
def chain_wgs(request):
    """Workgroups per CU of the chain grid (0: as many as are resident), set before the chain is
    created (the grid is planned at creation)."""
    _lib.tuning_set("chain.wgs", request.param)
    yield request.param
    _lib.tuning_set("chain.wgs", 0)


def _w(N, K, seed, scales="per_tensor"):
    return synth.make_weight(N, K, seed, DEV, scales=scales)


def _x(K, seed, kind="normal"):
    return synth.make_act(1, K, seed, DEV, kind=kind).reshape(-1)


def test_decode_set_chain_equals_separate_launches(chain_wgs):
    announce("chain_decode_set", chain_wgs)
    shapes = {lin.name: lin for lin in synth.DECODE_SET}
    qkv = [_w(shapes[n].N, shapes[n].K, 10 + i) for i, n in enumerate(("q_proj", "k_proj", "v_proj"))]
    wo = _w(shapes["o_proj"].N, shapes["o_proj"].K, 20)
    wu = _w(shapes["up_proj"].N, shapes["up_proj"].K, 21)
    wd = _w(shapes["down_proj"].N, shapes["down_proj"].K, 22)
    xa, xo = _x(3136, 1), _x(shapes["o_proj"].K, 2)
    xu, xd = _x(3136, 3), _x(shapes["down_proj"].K, 4, kind="relu2")
    yq = [torch.empty(w.shape[0], dtype=torch.bfloat16, device=DEV) for w, _ in qkv]
    yo = torch.empty(wo[0].shape[0], dtype=torch.bfloat16, device=DEV)
    yu = torch.empty(wu[0].shape[0], dtype=torch.bfloat16, device=DEV)
    yd = torch.empty(wd[0].shape[0], dtype=torch.bfloat16, device=DEV)
    chain = ops.GemvChain([
        (xa, [(w, s, y) for (w, s), y in zip(qkv, yq)], False),
        (xo, [(*wo, yo)], True),
        (xu, [(*wu, yu)], True),
        (xd, [(*wd, yd)], True),
    ])
    for rep in range(3):
        for y in yq + [yo, yu, yd]:
            y.fill_(7.0)
        chain.launch()
        torch.cuda.synchronize()
        ref_q = ops.linear_fp8_w8a16_grouped(xa.view(1, -1), qkv)
        for y, r in zip(yq, ref_q):
            assert torch.equal(y.view(torch.int16), r.view(-1).view(torch.int16))
        for x, (w, s), y in ((xo, wo, yo), (xu, wu, yu), (xd, wd, yd)):
            r = ops.linear_fp8_w8a16(x.view(1, -1), w, s).view(-1)
            assert torch.equal(y.view(torch.int16), r.view(torch.int16)), (rep, w.shape)
    xb = xu.view(torch.int16).cpu().numpy().view(np.uint16)[None]
    assert_parity(bits(yu.view(1, -1)), oracle_bits(xb, wu[0].cpu().numpy(), wu[1].cpu().numpy()), "chain up_proj")


def _dependent_case(dims, seed, scales="log_uniform"):
    """phase i: y_i = W_i x_i with x_0 given and x_{i+1} = y_i (dims[i+1] rows of W_i)."""
    x0 = _x(dims[0], seed)
    ws, ys = [], []
    for i in range(len(dims) - 1):
        ws.append(_w(dims[i + 1], dims[i], seed + 1 + i, scales))
        ys.append(torch.empty(dims[i + 1], dtype=torch.bfloat16, device=DEV))
    phases = [((x0 if i == 0 else ys[i - 1]), [(*ws[i], ys[i])], i > 0) for i in range(len(ws))]
    return x0, ws, ys, phases


@pytest.mark.parametrize("dims", [
    [3136, 5120, 3136, 12544, 3136],             # decode-set shapes, each fed by the previous output
    [64, 48, 112, 16, 96, 32, 208, 80, 1040, 64, 48, 112, 16, 96, 32, 208, 80, 1040, 64, 48, 37],
], ids=["decode_shapes", "twenty_ragged"])
def test_dependent_chain_equals_sequential_launches(dims, chain_wgs):
    announce("chain_dependent", len(dims) - 1, chain_wgs)
    x0, ws, ys, phases = _dependent_case(dims, 300 + len(dims))
    chain = ops.GemvChain(phases)
    chain.launch()
    torch.cuda.synchronize()
    x = x0
    for i, (w, s) in enumerate(ws):
        r = ops.linear_fp8_w8a16(x.view(1, -1), w, s).view(-1)
        assert torch.equal(ys[i].view(torch.int16), r.view(torch.int16)), f"phase {i}"
        x = r
    xb = ys[-2].view(torch.int16).cpu().numpy().view(np.uint16)[None]
    assert_parity(bits(ys[-1].view(1, -1)), oracle_bits(xb, ws[-1][0].cpu().numpy(), ws[-1][1].cpu().numpy()),
                  "last phase vs oracle", per_row_scales=True)


def test_phase_without_wait_finishing_first(chain_wgs):
    """phase 0: a large GEMV; phase 1 (no wait, 8 rows) may complete before it; phase 2 waits on
    phase 1 and reads its output; phase 3 waits on phase 2."""
    announce("chain_nowait_first", chain_wgs)
    big = _w(12544, 3136, 501)
    small = _w(8, 1024, 502)
    w2 = _w(2048, 128, 503)              # K = 128: phase 1's 8 outputs, then zeros
    w3 = _w(64, 2048, 504)
    x0, x1 = _x(3136, 505), _x(1024, 506)
    y0 = torch.empty(12544, dtype=torch.bfloat16, device=DEV)
    y1 = torch.empty(128, dtype=torch.bfloat16, device=DEV)   # rows 8.. stay as written below
    y2 = torch.empty(2048, dtype=torch.bfloat16, device=DEV)
    y3 = torch.empty(64, dtype=torch.bfloat16, device=DEV)
    y1.zero_()
    chain = ops.GemvChain([(x0, [(*big, y0)], False), (x1, [(*small, y1[:8])], False),
                           (y1, [(*w2, y2)], True), (y2, [(*w3, y3)], True)])
    for rep in range(4):
        for y in (y0, y2, y3):
            y.fill_(3.0)
        chain.launch()
        torch.cuda.synchronize()
        r0 = ops.linear_fp8_w8a16(x0.view(1, -1), *big).view(-1)
        r1 = ops.linear_fp8_w8a16(x1.view(1, -1), *small).view(-1)
        x2 = torch.cat([r1, torch.zeros(120, dtype=torch.bfloat16, device=DEV)])
        r2 = ops.linear_fp8_w8a16(x2.view(1, -1), *w2).view(-1)
        r3 = ops.linear_fp8_w8a16(r2.view(1, -1), *w3).view(-1)
        for i, (y, r) in enumerate(((y0, r0), (y1[:8], r1), (y2, r2), (y3, r3))):
            assert torch.equal(y.view(torch.int16), r.view(torch.int16)), (rep, i)


def test_long_k_phases_take_several_windows(chain_wgs):
    """Independent phases whose K exceeds one x window (K = 20480: two windows of 1024 chunks)
    next to short ones, byte-identical to separate launches."""
    announce("chain_long_k", chain_wgs)
    shapes = [(96, 20480), (100, 3136), (40, 16400), (8, 64)]
    ws = [_w(N, K, 600 + i, "log_uniform") for i, (N, K) in enumerate(shapes)]
    xs = [_x(K, 610 + i) for i, (_, K) in enumerate(shapes)]
    ys = [torch.empty(N, dtype=torch.bfloat16, device=DEV) for N, _ in shapes]
    chain = ops.GemvChain([(x, [(*w, y)], False) for x, w, y in zip(xs, ws, ys)])
    for rep in range(2):
        for y in ys:
            y.fill_(5.0)
        chain.launch()
        torch.cuda.synchronize()
        for i, (x, (w, s), y) in enumerate(zip(xs, ws, ys)):
            r = ops.linear_fp8_w8a16(x.view(1, -1), w, s).view(-1)
            assert torch.equal(y.view(torch.int16), r.view(torch.int16)), (rep, shapes[i])
    xb = xs[0].view(torch.int16).cpu().numpy().view(np.uint16)[None]
    assert_parity(bits(ys[0].view(1, -1)), oracle_bits(xb, ws[0][0].cpu().numpy(), ws[0][1].cpu().numpy()),
                  "K = 20480 vs oracle", per_row_scales=True)


def test_four_group_phases_and_single_rows(chain_wgs):
    """Phases of the maximum four groups with ragged N (1, 3, 17, 208 rows), a dependent phase
    reading the first group's output, and a single-row phase: each group byte-identical to its
    own launch."""
    announce("chain_groups", chain_wgs)
    K0 = 256
    g0 = [_w(N, K0, 700 + i, "log_uniform") for i, N in enumerate((1, 3, 17, 208))]
    x0 = _x(K0, 710)
    y0 = [torch.empty(w.shape[0], dtype=torch.bfloat16, device=DEV) for w, _ in g0]
    w1 = _w(64, 208, 711, "log_uniform")        # reads group 3's output (208 values)
    y1 = torch.empty(64, dtype=torch.bfloat16, device=DEV)
    w2 = _w(1, 1024, 712)                       # one row, independent x
    x2 = _x(1024, 713)
    y2 = torch.empty(1, dtype=torch.bfloat16, device=DEV)
    chain = ops.GemvChain([(x0, [(w, s, y) for (w, s), y in zip(g0, y0)], False),
                           (y0[3], [(*w1, y1)], True), (x2, [(*w2, y2)], False)])
    for rep in range(3):
        for y in y0 + [y1, y2]:
            y.fill_(9.0)
        chain.launch()
        torch.cuda.synchronize()
        for i, ((w, s), y) in enumerate(zip(g0, y0)):
            r = ops.linear_fp8_w8a16(x0.view(1, -1), w, s).view(-1)
            assert torch.equal(y.view(torch.int16), r.view(torch.int16)), (rep, i)
        r1 = ops.linear_fp8_w8a16(y0[3].view(1, -1), *w1).view(-1)
        assert torch.equal(y1.view(torch.int16), r1.view(torch.int16)), rep
        r2 = ops.linear_fp8_w8a16(x2.view(1, -1), *w2).view(-1)
        assert torch.equal(y2.view(torch.int16), r2.view(torch.int16)), rep


def test_chain_graph_replays():
    announce("chain_graph")
    x0, ws, ys, phases = _dependent_case([3136, 5120, 3136, 12544, 3136], 77)
    chain = ops.GemvChain(phases)
    chain.launch()
    torch.cuda.synchronize()
    want = [y.clone() for y in ys]
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        chain.launch()
    for rep in range(3):
        for y in ys:
            y.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for i, (y, w) in enumerate(zip(ys, want)):
            assert torch.equal(y.view(torch.int16), w.view(torch.int16)), (rep, i)
        chain.launch()                                  # eager launch between replays
        torch.cuda.synchronize()
