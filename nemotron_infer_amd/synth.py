"""Seeded synthetic workloads of the benchmark configurations (the reference benchmark's configs 0-4).

Weights: float32 N(0, 0.02) from a seeded generator, per-tensor scale s = amax / 448,
codes = RNE(clamp(W / s, +-448)) as float8_e4m3fn, the scale broadcast to a per-row vector
(nemotron_infer/engine.py:117-121).  Config 2 replaces the scales by per-row draws,
log-uniform in [1e-4, 1e-2].  Activations: bf16 N(0, 1); in config 1 (and the config-4
stream) the MLP down_proj input is relu(z)^2 (sparse, non-negative); config 2 gives every M
row its own N(0, 1) draw on all six shapes; config 3 draws N(0, 1) on all three shapes and
multiplies 0.1% of the activations by 50.

Generation runs on the device the caller names (torch's own generator for that device), so
the same seed gives the same bytes on the same kind of device.  Tests that compare with the
CPU oracle generate on the CPU and copy the bytes to the GPU.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

HIDDEN = 3136
INTER = 12544
Q_OUT = 40 * 128
KV_OUT = 8 * 128
MAMBA_IN = 14690          # ragged N of the synthetic Mamba in_proj (config 4)
MAMBA_OUT_K = 6272


@dataclass(frozen=True)
class Linear:
    name: str
    N: int
    K: int
    act: str = "normal"   # "normal" | "relu2"

    @property
    def weight_bytes(self) -> int:
        return self.N * self.K


# Config 1: one attention block and one MLP block at M = 1.
DECODE_SET = (
    Linear("q_proj", Q_OUT, HIDDEN),
    Linear("k_proj", KV_OUT, HIDDEN),
    Linear("v_proj", KV_OUT, HIDDEN),
    Linear("o_proj", HIDDEN, Q_OUT),
    Linear("up_proj", INTER, HIDDEN),
    Linear("down_proj", HIDDEN, INTER, act="relu2"),
)

# Config 2: the config-1 shapes at M in {2, 4, 8, 16}; every row of every input is N(0, 1)
# (down_proj included) and the scales are per-row log-uniform.
SKINNY_SET = tuple(Linear(l.name, l.N, l.K) for l in DECODE_SET)
SKINNY_M = (2, 4, 8, 16)

# Config 3: prefill GEMMs at M = 2048, every input N(0, 1) with 0.1% x50 outliers.
PREFILL_SET = (
    Linear("up_proj", INTER, HIDDEN),
    Linear("down_proj", HIDDEN, INTER),
    Linear("qkv_proj", Q_OUT + 2 * KV_OUT, HIDDEN),
)
PREFILL_M = 2048


def decode_stream_layers():
    """Config 4: 4 attention + 17 MLP + 21 Mamba layers -> 92 GEMVs, in layer order."""
    attn = [Linear("q_proj", Q_OUT, HIDDEN), Linear("k_proj", KV_OUT, HIDDEN),
            Linear("v_proj", KV_OUT, HIDDEN), Linear("o_proj", HIDDEN, Q_OUT)]
    mlp = [Linear("up_proj", INTER, HIDDEN), Linear("down_proj", HIDDEN, INTER, act="relu2")]
    mamba = [Linear("in_proj", MAMBA_IN, HIDDEN), Linear("out_proj", HIDDEN, MAMBA_OUT_K)]
    kinds = ["mamba", "mlp"] * 17 + ["mamba"] * 4 + ["attn"] * 4   # 21 mamba, 17 mlp, 4 attn
    order = []
    for i, kind in enumerate(kinds):
        order.append((i, kind, {"attn": attn, "mlp": mlp, "mamba": mamba}[kind]))
    return order


def linear_bytes(M: int, N: int, K: int) -> int:
    """Algorithmic bytes of one W8A16 linear: W (1 B) + scales (4 B) + x (2 B) + y (2 B)."""
    return N * K + 4 * N + 2 * M * K + 2 * M * N


def linear_flops(M: int, N: int, K: int) -> int:
    return 2 * M * N * K


def _gen(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def make_weight(N: int, K: int, seed: int, device="cpu", scales: str = "per_tensor",
                chunk_rows: int = 4096):
    """(codes uint8 [N, K], scales float32 [N]) with the generator of ``device``."""
    g = _gen(device, seed)
    codes = torch.empty((N, K), dtype=torch.uint8, device=device)
    # amax over the whole tensor first (two passes over the same seeded draws).
    amax = torch.zeros((), dtype=torch.float32, device=device)
    state = g.get_state()
    for r0 in range(0, N, chunk_rows):
        w = torch.randn((min(chunk_rows, N - r0), K), generator=g, device=device) * 0.02
        amax = torch.maximum(amax, w.abs().max())
    s = amax / 448.0
    if float(s) < 1e-10:
        s = torch.tensor(1.0 / 448.0, device=device)
    g.set_state(state)
    for r0 in range(0, N, chunk_rows):
        rows = min(chunk_rows, N - r0)
        w = torch.randn((rows, K), generator=g, device=device) * 0.02
        q = torch.clamp(w / s, -448.0, 448.0).to(torch.float8_e4m3fn)
        codes[r0:r0 + rows] = q.view(torch.uint8)
    if scales == "per_tensor":
        sv = torch.full((N,), float(s), dtype=torch.float32, device=device)
    elif scales == "log_uniform":
        u = torch.rand((N,), generator=g, device=device, dtype=torch.float64)
        sv = torch.exp(math.log(1e-4) + u * (math.log(1e-2) - math.log(1e-4))).to(torch.float32)
    else:
        raise ValueError(scales)
    return codes, sv


def make_act(M: int, K: int, seed: int, device="cpu", kind: str = "normal",
             outlier_frac: float = 0.0) -> torch.Tensor:
    """bf16 [M, K] activations: N(0,1), or relu(z)^2, with optional x50 outliers."""
    g = _gen(device, seed)
    z = torch.randn((M, K), generator=g, device=device)
    if kind == "relu2":
        z = torch.relu(z) ** 2
    elif kind != "normal":
        raise ValueError(kind)
    if outlier_frac > 0:
        n_out = int(round(outlier_frac * M * K))
        idx = torch.randperm(M * K, generator=g, device=device)[:n_out]
        z.view(-1)[idx] *= 50.0
    return z.to(torch.bfloat16)


def decode_stream_chain(device, wait_prev: bool = False):
    """Config 4 as the GEMV chain the bench times: one phase per launch of the engine's decode
    step -- an attention layer's q|k|v grouped (they share the normed input) then o, an MLP
    layer's up then down, a Mamba layer's in_proj (ragged N = 14690) then out_proj (K = 6272) --
    84 phases in layer order.  Weights are seeded per layer and projection; every phase reads its
    own activation, shared by phases of the same (K, kind).  wait_prev makes every phase after
    the first wait for its predecessor (the dependent form; the activations stay independent).

    Returns (phases, calls, total_bytes, weight_bytes, acts): phases as ops.GemvChain takes them;
    calls the same work as separate launches, ("grouped", x, [(w, s)], [y]) or
    ("single", x, w, s, y); acts the activations by (K, kind)."""
    acts = {}

    def act(K, kind):
        if (K, kind) not in acts:
            acts[(K, kind)] = make_act(1, K, 41000 + K, device, kind=kind)
        return acts[(K, kind)]

    phases, calls = [], []
    total_bytes = weight_bytes = 0
    for li, kind, lins in decode_stream_layers():
        mats = []
        for j, lin in enumerate(lins):
            w, s = make_weight(lin.N, lin.K, 40000 + 10 * li + j, device)
            mats.append((lin, w, s, torch.empty((1, lin.N), dtype=torch.bfloat16, device=device)))
            total_bytes += linear_bytes(1, lin.N, lin.K)
            weight_bytes += lin.N * lin.K
        groups = [mats[:3], mats[3:]] if kind == "attn" else [[m] for m in mats]
        for grp in groups:
            x = act(grp[0][0].K, grp[0][0].act)
            wait = wait_prev and len(phases) > 0
            phases.append((x, [(w, s, y) for _, w, s, y in grp], wait))
            if len(grp) > 1:
                calls.append(("grouped", x, [(w, s) for _, w, s, _ in grp], [y for _, _, _, y in grp]))
            else:
                _, w, s, y = grp[0]
                calls.append(("single", x, w, s, y))
    return phases, calls, total_bytes, weight_bytes, acts
