"""GPU tests of the checkpoint loader (nemotron_infer_amd/weights.py): weights loaded from
modelopt safetensors files feed the library's entry points directly.

* a synthetic four-layer checkpoint (tests/test_weights_cpu.py): the loaded MLP projection
  through the M-dispatching linear vs the oracle, and the loaded q/k/v in one grouped launch
  byte-identical to three separate launches;
* the reference's MLP block fixture (tests/golden/mlp_block_h64_i256_s8.npz, from
  tools/dump_mlp_block.py) exported as a modelopt checkpoint -- fp32 weights quantized per
  tensor (scalar weight_scale, engine.py:117-121) -- loaded and run through the block: parity
  with the oracle block on the loaded codes and scales (end-to-end rel_l2 <= 4e-3, the bar of
  tests/test_mlp_block_gpu.py) and rel_l2 < 0.05 against the HF fp32 expectation (the
  reference's own gate, test_mlp_block.cu:184, is 0.3).
"""
import numpy as np
import pytest
import torch

from nemotron_infer_amd import ops, weights
from oracle import block, e4m3, linear
from tests.conftest import load_golden
from tests.gpu_util import DEV, announce, assert_parity, bits, oracle_bits, x_to_dev
from tests.test_weights_cpu import _checkpoint

pytestmark = pytest.mark.gpu


def _x(M, K, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(M, K, generator=g).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def test_loaded_linears_run_on_the_library():
    ck = weights.load_checkpoint(raw=_checkpoint(), device=DEV)
    up = ck.layers[2]["up"]
    for M in (1, 2, 5, 40):
        announce("weights_linear", M)
        x = _x(M, up.shape[1], 100 + M)
        y = bits(ops.linear_fp8_w8a16(x_to_dev(x), up.weight, up.scale))
        assert_parity(y, oracle_bits(x, up.weight.cpu().numpy(), up.scale.cpu().numpy()), f"loaded up M={M}")
    at = ck.layers[1]
    for M in (1, 3):
        announce("weights_qkv", M)
        xd = x_to_dev(_x(M, 64, 200 + M))
        grouped = ops.linear_fp8_w8a16_grouped(xd, weights.qkv_groups(at))
        for (w, s), yg in zip(weights.qkv_groups(at), grouped):
            y1 = ops.linear_fp8_w8a16(xd, w, s)
            assert torch.equal(yg.view(torch.int16), y1.view(torch.int16))


def test_fixture_exported_as_modelopt_checkpoint(tmp_path):
    from safetensors.torch import save_file

    g = load_golden("mlp_block_h64_i256_s8")
    eps = float(g["eps"])
    up_codes, up_s = e4m3.quant_per_tensor(g["up_w_f32"])
    dn_codes, dn_s = e4m3.quant_per_tensor(g["down_w_f32"])
    p = "backbone.layers.0."
    t = {
        "backbone.embeddings.weight": torch.zeros(4, 64, dtype=torch.bfloat16),
        "backbone.norm_f.weight": torch.ones(64, dtype=torch.bfloat16),
        "lm_head.weight": torch.zeros(4, 64, dtype=torch.bfloat16),
        p + "norm.weight": torch.from_numpy(g["norm_w"].copy()),
        p + "mixer.up_proj.weight": torch.from_numpy(up_codes.copy()).view(torch.float8_e4m3fn),
        p + "mixer.up_proj.weight_scale": torch.tensor(float(up_s[0]), dtype=torch.float32),
        p + "mixer.down_proj.weight": torch.from_numpy(dn_codes.copy()).view(torch.float8_e4m3fn),
        p + "mixer.down_proj.weight_scale": torch.tensor(float(dn_s[0]), dtype=torch.float32),
    }
    save_file(t, str(tmp_path / "model.safetensors"))
    ck = weights.load_checkpoint(str(tmp_path), device=DEV)
    ly = ck.layers[0]
    assert ly["type"] == "mlp"
    assert np.array_equal(ly["up"].weight.cpu().numpy(), up_codes)
    assert np.array_equal(ly["down"].scale.cpu().numpy(), dn_s)
    exp = g["expected_f32"].astype(np.float64)
    for M in (1, 2, 8):
        announce("weights_fixture_block", M)
        x = g["x_bf16"][:M]
        got = bits(ops.mlp_forward_fp8(x_to_dev(x), ly["norm"], ly["up"].weight, ly["up"].scale,
                                       ly["down"].weight, ly["down"].scale, eps=eps))
        ref = block.mlp_block_fp8(x, g["norm_w"], up_codes, up_s, dn_codes, dn_s, eps, precise=True)
        r = linear.parity(got, ref)
        assert r["nan_ok"] and r["rel_l2_all"] <= 4e-3, (M, r)
        o = linear.bf16_to_f32(got).astype(np.float64)
        rel = np.linalg.norm(o - exp[:M]) / np.linalg.norm(exp[:M])
        assert rel < 0.05, (M, rel)
