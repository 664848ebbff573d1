"""Checkpoint loader for the fp8 linear path: modelopt safetensors -> device tensors.

Restates the reference engine's loader (nemotron_infer/engine.py:94-159, ``Engine._load``):
every ``*.safetensors`` file of the model directory is read; the layer count is the number of
consecutive ``backbone.layers.{i}.norm.weight`` keys; a layer is Mamba, attention or MLP by
which projection it holds; an fp8 matrix keeps its e4m3 codes and its scalar
``weight_scale`` becomes a per-row float32 vector (engine.py:117-121), a non-fp8 matrix is
passed as bf16 (the reference's bf16 "exclude" layers); norms and the Mamba parameters are
float32, the embeddings and lm_head bf16.

The e4m3 codes are returned as uint8 [N, K] (the byte layout the kernels read: row n is
W[n, :]). No weight swizzle is applied at load: the GEMV streams rows as stored and the
prefill GEMM DMAs 64-byte row pieces of the stored layout into LDS, so the on-disk order is the
kernel order. Dequantized values are e4m3(code) * scale[n], unchanged by loading.

Errors follow the reference: a layer with none of the three projections raises RuntimeError,
a missing tensor raises KeyError.
"""
from __future__ import annotations

import glob
import os
from dataclasses import dataclass, field

import torch

# engine.py / binding.cu:35-46 model constants used by the loader
H, P, N, G, CONV_K = 96, 80, 128, 8, 4
CONV_DIM = H * P + 2 * G * N


@dataclass
class Linear:
    """One projection as the reference's ``gw`` returns it: ('fp8', codes, scale) or
    ('bf16', weight, None)."""
    kind: str                      # "fp8" or "bf16"
    weight: torch.Tensor           # fp8: uint8 e4m3 codes [N, K]; bf16: [N, K]
    scale: torch.Tensor | None     # fp8: float32 [N] (the scalar broadcast per row)

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


def read_safetensors(model_dir: str) -> dict:
    """All tensors of all ``*.safetensors`` files in model_dir, on the CPU (engine.py:97-103)."""
    from safetensors import safe_open

    raw = {}
    files = sorted(glob.glob(os.path.join(model_dir, "*.safetensors")))
    if not files:
        raise FileNotFoundError(f"no *.safetensors in {model_dir}")
    for fn in files:
        with safe_open(fn, "pt") as f:
            for k in f.keys():
                raw[k] = f.get_tensor(k)
    return raw


def fp8_linear(raw: dict, key: str, device) -> Linear:
    """engine.py:113-121 ``gw``: an e4m3 matrix keeps its codes and gets a per-row float32
    scale filled with its scalar ``weight_scale``; any other dtype is passed as bf16."""
    w = raw[key + ".weight"]
    if w.dtype == torch.float8_e4m3fn:
        n = w.shape[0]
        scale = raw[key + ".weight_scale"].float().reshape(())        # a scalar, as in the reference
        codes = w.contiguous().view(torch.uint8).to(device)
        return Linear("fp8", codes, torch.full((n,), float(scale), dtype=torch.float32, device=device))
    return Linear("bf16", w.to(torch.bfloat16).contiguous().to(device), None)


def load_checkpoint(model_dir: str | None = None, device="cuda", raw: dict | None = None) -> Checkpoint:
    """engine.py:94-159 ``_load``: the model's weights on ``device``.  ``raw`` (key -> CPU
    tensor) may be given instead of a directory."""
    if raw is None:
        raw = read_safetensors(model_dir)

    def g32(k):
        return raw[k].to(torch.float32).contiguous().to(device)

    def gbf(k):
        return raw[k].to(torch.bfloat16).contiguous().to(device)

    nlayers = 0
    while f"backbone.layers.{nlayers}.norm.weight" in raw:
        nlayers += 1
    ck = Checkpoint(embed=gbf("backbone.embeddings.weight"), norm_f=g32("backbone.norm_f.weight"),
                    lm_head=gbf("lm_head.weight"))
    for i in range(nlayers):
        p = f"backbone.layers.{i}."
        ly = {"norm": g32(p + "norm.weight")}
        if p + "mixer.in_proj.weight" in raw:
            ly["type"] = "mamba"
            ly["in_proj"] = fp8_linear(raw, p + "mixer.in_proj", device)
            ly["out_proj"] = fp8_linear(raw, p + "mixer.out_proj", device)
            conv = g32(p + "mixer.conv1d.weight")
            ly["conv_w"] = conv.reshape(conv.numel() // CONV_K, CONV_K)   # [CONV_DIM, CONV_K] for the real model
            ly["conv_b"] = g32(p + "mixer.conv1d.bias")
            ly["A_log"] = g32(p + "mixer.A_log")
            ly["D"] = g32(p + "mixer.D")
            ly["dt_bias"] = g32(p + "mixer.dt_bias")
            ly["gnorm"] = g32(p + "mixer.norm.weight")
        elif p + "mixer.q_proj.weight" in raw:
            ly["type"] = "attn"
            for name, key in (("q", "q_proj"), ("k", "k_proj"), ("v", "v_proj"), ("o", "o_proj")):
                ly[name] = fp8_linear(raw, p + "mixer." + key, device)
        elif p + "mixer.up_proj.weight" in raw:
            ly["type"] = "mlp"
            ly["up"] = fp8_linear(raw, p + "mixer.up_proj", device)
            ly["down"] = fp8_linear(raw, p + "mixer.down_proj", device)
        else:
            raise RuntimeError(f"layer {i}: unknown layer type (no in_proj, q_proj or up_proj)")
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
