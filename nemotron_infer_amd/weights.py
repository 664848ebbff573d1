"""Checkpoint loader for the fp8 linear path: modelopt safetensors -> device tensors.

The on-disk format (a modelopt fp8 export of Nemotron-H, read by the reference engine at
nemotron_infer/engine.py:94-159):

* top-level tensors ``backbone.embeddings.weight``, ``backbone.norm_f.weight`` and
  ``lm_head.weight``;
* per layer i, under ``backbone.layers.{i}.``, a ``norm.weight`` and one mixer.  The mixer's
  kind follows from the projection it holds: ``mixer.in_proj`` (Mamba-2), ``mixer.q_proj``
  (attention) or ``mixer.up_proj`` (MLP), checked in that order;
* a quantized projection stores ``<key>.weight`` as float8_e4m3fn [N, K] and
  ``<key>.weight_scale`` as one float32 value (per tensor); an unquantized one stores only a
  bf16 ``<key>.weight``.

Layers are the indices 0, 1, 2, ... whose ``norm.weight`` exists, up to the first missing one.
Tensor roles (``_ROLES``): a projection becomes a ``Linear`` -- e4m3 codes as uint8 [N, K] (the
byte layout every kernel reads; no swizzle is applied, so dequantized values are
e4m3(code) * scale[n], unchanged by loading) plus the per-tensor scale repeated into a float32
[N] vector (engine.py:117-121), or a bf16 matrix; norms and Mamba parameters become float32;
the embeddings and lm_head bf16; the depthwise conv weight float32 [channels, CONV_K].

The per-layer dictionaries keep the key names the reference engine consumes ("type", "norm",
"in_proj", "q", "up", "conv_w", ...).  Errors: a layer with none of the three projections
raises RuntimeError, a missing tensor KeyError (as the reference), and a projection whose
shape does not chain with its neighbours (q/k/v and up on the hidden size, o and down back to
it, down's K = up's N, o's K = q's N) or whose scale is not a single value raises ValueError,
which the reference does not check.
"""
from __future__ import annotations

import glob
import os
import re
from dataclasses import dataclass, field

import torch

# Mamba-2 shape constants of the model (binding.cu:35-46): heads, head dim, state size,
# groups, conv width
H, P, N, G, CONV_K = 96, 80, 128, 8, 4
CONV_DIM = H * P + 2 * G * N

_LAYER = "backbone.layers.{}."


@dataclass
class Linear:
    """One projection: ('fp8', codes, scale) or ('bf16', weight, None), the tuple the reference
    engine keeps per projection."""
    kind: str                      # "fp8" or "bf16"
    weight: torch.Tensor           # fp8: uint8 e4m3 codes [N, K]; bf16: [N, K]
    scale: torch.Tensor | None     # fp8: float32 [N] (the per-tensor value per row)

    def as_tuple(self):
        return (self.kind, self.weight, self.scale)

    @property
    def shape(self):
        return tuple(self.weight.shape)


@dataclass
class Checkpoint:
    embed: torch.Tensor
    norm_f: torch.Tensor
    lm_head: torch.Tensor
    layers: list = field(default_factory=list)

    @property
    def nlayers(self) -> int:
        return len(self.layers)


# Layer kinds in detection order: (type, marker key, [(field, key suffix, role), ...]).
_KINDS = (
    ("mamba", "mixer.in_proj.weight", (
        ("in_proj", "mixer.in_proj", "linear"),
        ("out_proj", "mixer.out_proj", "linear"),
        ("conv_w", "mixer.conv1d.weight", "conv"),
        ("conv_b", "mixer.conv1d.bias", "f32"),
        ("A_log", "mixer.A_log", "f32"),
        ("D", "mixer.D", "f32"),
        ("dt_bias", "mixer.dt_bias", "f32"),
        ("gnorm", "mixer.norm.weight", "f32"),
    )),
    ("attn", "mixer.q_proj.weight", (
        ("q", "mixer.q_proj", "linear"),
        ("k", "mixer.k_proj", "linear"),
        ("v", "mixer.v_proj", "linear"),
        ("o", "mixer.o_proj", "linear"),
    )),
    ("mlp", "mixer.up_proj.weight", (
        ("up", "mixer.up_proj", "linear"),
        ("down", "mixer.down_proj", "linear"),
    )),
)

# Shape links checked per kind: (field, dim, must equal) where the right side is "hidden" or
# (other field, dim).  dim 0 = N (output rows), 1 = K.
_LINKS = {
    "mamba": (("in_proj", 1, "hidden"), ("out_proj", 0, "hidden")),
    "attn": (("q", 1, "hidden"), ("k", 1, "hidden"), ("v", 1, "hidden"), ("o", 0, "hidden"),
             ("o", 1, ("q", 0))),
    "mlp": (("up", 1, "hidden"), ("down", 0, "hidden"), ("down", 1, ("up", 0))),
}


def read_safetensors(model_dir: str) -> dict:
    """Every tensor of every ``*.safetensors`` file in model_dir, on the CPU."""
    from safetensors import safe_open

    files = sorted(glob.glob(os.path.join(model_dir, "*.safetensors")))
    if not files:
        raise FileNotFoundError(f"no *.safetensors in {model_dir}")
    out = {}
    for fn in files:
        with safe_open(fn, "pt") as f:
            out.update({k: f.get_tensor(k) for k in f.keys()})
    return out


def _convert(raw: dict, key: str, role: str, device):
    """The one conversion routine: the tensor(s) under ``key`` in the form ``role`` asks for."""
    if role == "linear":
        w = raw[key + ".weight"]
        if w.dim() != 2:
            raise ValueError(f"{key}.weight: expected a 2-D matrix, got shape {tuple(w.shape)}")
        if w.dtype != torch.float8_e4m3fn:
            return Linear("bf16", w.to(device=device, dtype=torch.bfloat16).contiguous(), None)
        sc = raw[key + ".weight_scale"]
        if sc.numel() != 1:
            raise ValueError(f"{key}.weight_scale: expected one per-tensor value, got {sc.numel()}")
        rows = torch.empty(w.shape[0], dtype=torch.float32).fill_(sc.to(torch.float32).flatten()[0])
        return Linear("fp8", w.contiguous().view(torch.uint8).to(device), rows.to(device))
    t = raw[key]
    if role == "bf16":
        return t.to(dtype=torch.bfloat16).contiguous().to(device)
    t = t.to(dtype=torch.float32).contiguous()
    if role == "conv":                              # [channels, 1, CONV_K] -> [channels, CONV_K]
        t = t.reshape(-1, CONV_K)
    return t.to(device)


def _layer_count(raw: dict) -> int:
    pat = re.compile(r"backbone\.layers\.(\d+)\.norm\.weight$")
    present = {int(m.group(1)) for m in map(pat.match, raw) if m}
    n = 0
    while n in present:
        n += 1
    return n


def _check_links(kind: str, ly: dict, hidden: int, index: int) -> None:
    for name, dim, want in _LINKS[kind]:
        got = ly[name].shape[dim]
        ref = hidden if want == "hidden" else ly[want[0]].shape[want[1]]
        if got != ref:
            what = "the hidden size" if want == "hidden" else f"{want[0]} dim {want[1]}"
            raise ValueError(f"layer {index} ({kind}): {name} dim {dim} is {got}, expected {ref} ({what})")


def load_checkpoint(model_dir: str | None = None, device="cuda", raw: dict | None = None) -> Checkpoint:
    """The model's weights on ``device``, from model_dir or from ``raw`` (key -> CPU tensor)."""
    if raw is None:
        raw = read_safetensors(model_dir)
    ck = Checkpoint(embed=_convert(raw, "backbone.embeddings.weight", "bf16", device),
                    norm_f=_convert(raw, "backbone.norm_f.weight", "f32", device),
                    lm_head=_convert(raw, "lm_head.weight", "bf16", device))
    hidden = ck.embed.shape[1]
    for i in range(_layer_count(raw)):
        prefix = _LAYER.format(i)
        kind = next((k for k in _KINDS if prefix + k[1] in raw), None)
        if kind is None:
            raise RuntimeError(f"layer {i}: unknown layer type (no in_proj, q_proj or up_proj)")
        ly = {"type": kind[0], "norm": _convert(raw, prefix + "norm.weight", "f32", device)}
        for name, suffix, role in kind[2]:
            ly[name] = _convert(raw, prefix + suffix, role, device)
        _check_links(kind[0], ly, hidden, i)
        ck.layers.append(ly)
    return ck


def qkv_groups(layer: dict) -> list:
    """An attention layer's q, k and v as (codes, scale) pairs for one grouped launch
    (``ops.linear_fp8_w8a16_grouped`` / ``nmi_linear_fp8_w8a16_grouped``), which the reference
    runs as three GEMVs on the same normed input (attention_block.cuh:400-402)."""
    out = []
    for name in ("q", "k", "v"):
        lin = layer[name]
        if lin.kind != "fp8":
            raise ValueError(f"{name}_proj is {lin.kind}, not fp8")
        out.append((lin.weight, lin.scale))
    return out
