"""CPU tests of the checkpoint loader (nemotron_infer_amd/weights.py, restating
nemotron_infer/engine.py:94-159) on small synthetic checkpoints in the modelopt layout: e4m3
``*.weight`` with a scalar ``*.weight_scale``, bf16 norms and embeddings, a Mamba, an attention
and two MLP layers (one with bf16 weights, the reference's non-fp8 branch), split over two
files.

Pins: the loaded codes are the stored e4m3 bytes; each per-row scale is the stored scalar;
e4m3(code) * scale equals torch's own float8_e4m3fn -> float32 conversion times the scalar
(the dequantized values are unchanged by loading); layer types and counts follow the key names;
errors as in the reference (RuntimeError for an unknown layer, KeyError for a missing tensor).
"""
import numpy as np
import pytest
import torch

from nemotron_infer_amd import weights
from oracle import e4m3

HID = 64


def _fp8(shape, seed, scale):
    g = torch.Generator().manual_seed(seed)
    wf = torch.randn(shape, generator=g) * 0.02
    w8 = (wf / scale).clamp(-448, 448).to(torch.float8_e4m3fn)
    return w8, torch.tensor(scale, dtype=torch.float32)


def _checkpoint():
    """key -> tensor, as a modelopt export names them."""
    t = {}
    g = torch.Generator().manual_seed(7)
    t["backbone.embeddings.weight"] = torch.randn(32, HID, generator=g).to(torch.bfloat16)
    t["backbone.norm_f.weight"] = (1 + 0.1 * torch.randn(HID, generator=g)).to(torch.bfloat16)
    t["lm_head.weight"] = torch.randn(32, HID, generator=g).to(torch.bfloat16)
    p = "backbone.layers.0."                       # Mamba
    t[p + "norm.weight"] = torch.ones(HID, dtype=torch.bfloat16)
    t[p + "mixer.in_proj.weight"], t[p + "mixer.in_proj.weight_scale"] = _fp8((96, HID), 1, 1e-4)
    t[p + "mixer.out_proj.weight"], t[p + "mixer.out_proj.weight_scale"] = _fp8((HID, 48), 2, 2e-4)
    t[p + "mixer.conv1d.weight"] = torch.randn(40, 1, weights.CONV_K, generator=g).to(torch.bfloat16)
    t[p + "mixer.conv1d.bias"] = torch.randn(40, generator=g).to(torch.bfloat16)
    t[p + "mixer.A_log"] = torch.randn(8, generator=g)
    t[p + "mixer.D"] = torch.randn(8, generator=g)
    t[p + "mixer.dt_bias"] = torch.randn(8, generator=g)
    t[p + "mixer.norm.weight"] = torch.ones(48, dtype=torch.bfloat16)
    p = "backbone.layers.1."                       # attention
    t[p + "norm.weight"] = torch.ones(HID, dtype=torch.bfloat16)
    for i, (name, n) in enumerate((("q_proj", 80), ("k_proj", 16), ("v_proj", 16))):
        t[p + f"mixer.{name}.weight"], t[p + f"mixer.{name}.weight_scale"] = _fp8((n, HID), 10 + i, 3e-4 * (i + 1))
    t[p + "mixer.o_proj.weight"], t[p + "mixer.o_proj.weight_scale"] = _fp8((HID, 80), 13, 5e-5)
    p = "backbone.layers.2."                       # MLP, fp8
    t[p + "norm.weight"] = torch.ones(HID, dtype=torch.bfloat16)
    t[p + "mixer.up_proj.weight"], t[p + "mixer.up_proj.weight_scale"] = _fp8((256, HID), 20, 1e-4)
    t[p + "mixer.down_proj.weight"], t[p + "mixer.down_proj.weight_scale"] = _fp8((HID, 256), 21, 1e-4)
    p = "backbone.layers.3."                       # MLP kept in bf16 (not quantized)
    t[p + "norm.weight"] = torch.ones(HID, dtype=torch.bfloat16)
    t[p + "mixer.up_proj.weight"] = torch.randn(256, HID, generator=g).to(torch.bfloat16)
    t[p + "mixer.down_proj.weight"] = torch.randn(HID, 256, generator=g).to(torch.bfloat16)
    return t


@pytest.fixture
def ckpt_dir(tmp_path):
    from safetensors.torch import save_file

    t = _checkpoint()
    keys = sorted(t)
    save_file({k: t[k] for k in keys[::2]}, str(tmp_path / "model-00001-of-00002.safetensors"))
    save_file({k: t[k] for k in keys[1::2]}, str(tmp_path / "model-00002-of-00002.safetensors"))
    return tmp_path, t


def test_structure_and_dtypes(ckpt_dir):
    d, _ = ckpt_dir
    ck = weights.load_checkpoint(str(d), device="cpu")
    assert ck.nlayers == 4
    assert [ly["type"] for ly in ck.layers] == ["mamba", "attn", "mlp", "mlp"]
    assert ck.embed.dtype == torch.bfloat16 and ck.lm_head.dtype == torch.bfloat16
    assert ck.norm_f.dtype == torch.float32
    mb, at, ml, mlb = ck.layers
    assert mb["in_proj"].shape == (96, HID) and mb["out_proj"].shape == (HID, 48)
    assert mb["conv_w"].shape == (40, weights.CONV_K) and mb["conv_w"].dtype == torch.float32
    for k in ("conv_b", "A_log", "D", "dt_bias", "gnorm", "norm"):
        assert mb[k].dtype == torch.float32
    for name, n in (("q", 80), ("k", 16), ("v", 16)):
        lin = at[name]
        assert lin.kind == "fp8" and lin.weight.dtype == torch.uint8 and lin.shape == (n, HID)
        assert lin.scale.dtype == torch.float32 and lin.scale.shape == (n,)
    assert ml["up"].kind == "fp8" and ml["down"].kind == "fp8"
    assert mlb["up"].kind == "bf16" and mlb["up"].scale is None and mlb["up"].weight.dtype == torch.bfloat16


def test_codes_and_scales_are_the_stored_ones(ckpt_dir):
    d, t = ckpt_dir
    ck = weights.load_checkpoint(str(d), device="cpu")
    lut = e4m3.decode_lut()
    for i, ly in enumerate(ck.layers[:3]):
        for name, lin in ly.items():
            if not isinstance(lin, weights.Linear):
                continue
            key = f"backbone.layers.{i}.mixer.{name if name in ('in_proj', 'out_proj') else name + '_proj'}"
            w8 = t[key + ".weight"]
            scalar = float(t[key + ".weight_scale"])
            assert torch.equal(lin.weight, w8.view(torch.uint8)), key
            assert torch.all(lin.scale == np.float32(scalar)), key
            # dequantized values: oracle table decode of the codes == torch's own e4m3 decode
            deq = lut[lin.weight.numpy()] * lin.scale.numpy()[:, None]
            ref = w8.to(torch.float32).numpy() * np.float32(scalar)
            np.testing.assert_array_equal(deq, ref)


def test_qkv_groups(ckpt_dir):
    d, _ = ckpt_dir
    ck = weights.load_checkpoint(str(d), device="cpu")
    groups = weights.qkv_groups(ck.layers[1])
    assert [w.shape[0] for w, _ in groups] == [80, 16, 16]
    with pytest.raises(KeyError):
        weights.qkv_groups(ck.layers[2])


def test_raw_dict_matches_directory(ckpt_dir):
    d, t = ckpt_dir
    a = weights.load_checkpoint(str(d), device="cpu")
    b = weights.load_checkpoint(raw=t, device="cpu")
    assert torch.equal(a.layers[2]["up"].weight, b.layers[2]["up"].weight)
    assert torch.equal(a.layers[1]["o"].scale, b.layers[1]["o"].scale)


def test_errors(ckpt_dir, tmp_path_factory):
    _, t = ckpt_dir
    bad = dict(t)
    for k in [k for k in bad if k.startswith("backbone.layers.3.mixer.")]:
        del bad[k]
    bad["backbone.layers.3.mixer.weird.weight"] = torch.zeros(4, 4)
    with pytest.raises(RuntimeError, match="layer 3"):
        weights.load_checkpoint(raw=bad, device="cpu")
    missing = dict(t)
    del missing["backbone.layers.2.mixer.up_proj.weight_scale"]
    with pytest.raises(KeyError):
        weights.load_checkpoint(raw=missing, device="cpu")
    with pytest.raises(FileNotFoundError):
        weights.load_checkpoint(str(tmp_path_factory.mktemp("empty")), device="cpu")


def test_layer_count_stops_at_first_gap(ckpt_dir):
    _, t = ckpt_dir
    gap = {k: v for k, v in t.items() if not k.startswith("backbone.layers.1.")}
    ck = weights.load_checkpoint(raw=gap, device="cpu")
    assert ck.nlayers == 1 and ck.layers[0]["type"] == "mamba"


def test_shape_links_are_checked(ckpt_dir):
    """Projections must chain: q/k/v/up/in_proj read the hidden size, o/down/out_proj write it,
    down reads up's rows, o reads q's rows; a per-tensor scale holds one value."""
    _, t = ckpt_dir
    bad = dict(t)
    bad["backbone.layers.2.mixer.down_proj.weight"], _ = _fp8((HID, 128), 30, 1e-4)   # down K != up N
    with pytest.raises(ValueError, match="layer 2 .*down dim 1"):
        weights.load_checkpoint(raw=bad, device="cpu")
    bad = dict(t)
    bad["backbone.layers.1.mixer.k_proj.weight"], _ = _fp8((16, HID + 16), 31, 1e-4)   # k K != hidden
    with pytest.raises(ValueError, match="layer 1 .*k dim 1"):
        weights.load_checkpoint(raw=bad, device="cpu")
    bad = dict(t)
    bad["backbone.layers.0.mixer.in_proj.weight_scale"] = torch.tensor([1e-4, 2e-4])
    with pytest.raises(ValueError, match="weight_scale"):
        weights.load_checkpoint(raw=bad, device="cpu")
    bad = dict(t)
    bad["backbone.layers.2.mixer.up_proj.weight"] = bad["backbone.layers.2.mixer.up_proj.weight"].reshape(-1)
    with pytest.raises(ValueError, match="2-D"):
        weights.load_checkpoint(raw=bad, device="cpu")
