"""The launch config 4's bench number comes from, tested as it is timed: the 42-layer decode
stream (4 attention, 17 MLP, 21 Mamba layers; 92 GEMVs, 2.87 GB of e4m3 weights) as one
84-phase GEMV chain built by synth.decode_stream_chain -- q|k|v grouped, the ragged Mamba
in_proj (N = 14690, the row-slice pattern of mamba_block.cuh:474-481 in one matrix) and
out_proj (K = 6272, two slices), the MLP down_proj (K = 12544, four slices).

* every phase is byte-identical to the same GEMV launched alone (the engine's launches);
* one layer of each kind (first and last Mamba layer, an MLP layer, the last attention layer)
  passes the oracle gate, rel_l2 over all elements included (per-tensor scales);
* the same phases as a dependent chain (every phase waits for its predecessor: 84 launches in
  stream order) give the same bytes, on a second launch too.
"""
import numpy as np
import pytest
import torch

from nemotron_infer_amd import ops, synth
from tests.gpu_util import DEV, announce, assert_parity, bits, oracle_bits

pytestmark = pytest.mark.gpu


def _outs(phases):
    return [y.clone() for _, groups, _ in phases for _, _, y in groups]


def test_config4_chain_as_benched():
    announce("config4_chain", "build")
    phases, calls, total_bytes, weight_bytes, _ = synth.decode_stream_chain(DEV)
    assert len(phases) == 84 and weight_bytes == 2_872_105_600
    ys = [y for _, groups, _ in phases for _, _, y in groups]
    chain = ops.GemvChain(phases)
    announce("config4_chain", "launch")
    for y in ys:
        y.fill_(float("nan"))
    chain.launch()
    torch.cuda.synchronize()
    got = _outs(phases)
    # the same work as separate launches, into the same buffers
    announce("config4_chain", "separate")
    for y in ys:
        y.fill_(float("nan"))
    for c in calls:
        if c[0] == "grouped":
            ops.linear_fp8_w8a16_grouped(c[1], c[2], outs=c[3])
        else:
            ops.linear_fp8_w8a16(c[1], c[2], c[3], out=c[4])
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(got, ys)):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"phase output {i} differs"
    # the oracle on one layer of each kind
    layers = synth.decode_stream_layers()
    pi = 0
    checked = []
    for li, kind, lins in layers:
        nph = 2
        pick = (kind == "mamba" and li in (0, 36)) or (kind == "mlp" and li == 1) or (kind == "attn" and li == 41)
        if pick:
            for x, groups, _ in phases[pi:pi + nph]:
                xb = bits(x.view(1, -1))
                for w, s, y in groups:
                    announce("config4_oracle", li, kind, tuple(w.shape))
                    assert_parity(bits(y.view(1, -1)), oracle_bits(xb, w.cpu().numpy(), s.cpu().numpy()),
                                  f"layer {li} {kind} {tuple(w.shape)}", rel_l2_all_tol=1e-3)
                    checked.append((kind, tuple(w.shape)))
        pi += nph
    assert {k for k, _ in checked} == {"mamba", "mlp", "attn"} and len(checked) == 10
    # the dependent form of the same phases
    dep = ops.GemvChain([(x, groups, i > 0) for i, (x, groups, _) in enumerate(phases)])
    for rep in range(2):
        announce("config4_chain_dependent", rep)
        for y in ys:
            y.fill_(float("nan"))
        dep.launch()
        torch.cuda.synchronize()
        assert dep.launches == 84
        for i, (a, b) in enumerate(zip(got, ys)):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"dependent phase output {i} differs"
    del chain, dep, phases, calls, ys, got
    torch.cuda.empty_cache()
