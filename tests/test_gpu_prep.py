"""The GPU weight packer (minicpm5_mk.gpu_prep, libmk's mk_weight_row_amax / mk_weight_quantize) against
the CPU restatement of prepare_mk_weights, whose calibration and quantisation are pinned against the
reference's own functions (tests/test_calib_fixture.py): every output tensor must be bit-identical,
for every quant base, with and without SmoothQuant, and for the full MiniCPM5-1B auto string."""
import os

import pytest
import torch

pytestmark = pytest.mark.gpu


def _same(a, b):
    if a.dtype == torch.float8_e4m3fn:
        a, b = a.view(torch.uint8), b.view(torch.uint8)
    return a.shape == b.shape and a.dtype == b.dtype and torch.equal(a, b.to(a.device))


QUANTS = ["int8d:qkv+gu|sq|lastbf16|fqkv|fmlp", "int8d:qkv+gu+o+down|sq|fmlp", "int8:qkv+gu+o+down|sq",
          "int8|fqkv|fmlp", "fp8:qkv+gu+o+down|sq", "fp8d:qkv+gu|sq", "int8d:qkv+o", "bf16"]


@pytest.mark.parametrize("name", ["tiny", "tiny-hd96"])
@pytest.mark.parametrize("quant", QUANTS)
def test_gpu_prep_bit_identical(name, quant, monkeypatch):
    from minicpm5_mk.config import preset
    from minicpm5_mk.mk_weights import prepare_mk_weights
    from minicpm5_mk.synth import random_hf_state_dict

    for k in [k for k in os.environ if k.startswith("MINICPM5_MK_")]:
        monkeypatch.delenv(k)
    assert torch.cuda.is_available()
    cfg = preset(name)
    sd = random_hf_state_dict(cfg)
    g = torch.Generator().manual_seed(9)
    for i in range(cfg.num_layers):      # non-unit gammas, so folding and activation factors are exercised
        for n in ("input_layernorm.weight", "post_attention_layernorm.weight"):
            sd[f"model.layers.{i}.{n}"] = (torch.rand(cfg.hidden, generator=g) + 0.5).to(torch.bfloat16)
    cpu = prepare_mk_weights(sd, cfg.as_mk_cfg(), quant, 512, log=lambda *a: None)
    gpu = prepare_mk_weights(sd, cfg.as_mk_cfg(), quant, 512, log=lambda *a: None, device="cuda:0")
    assert set(cpu) == set(gpu)
    bad = [k for k in cpu if not _same(gpu[k], cpu[k])]
    assert not bad, f"{name} {quant}: {bad}"
    assert all(t.is_cuda for t in gpu.values())


def test_gpu_prep_bit_identical_full_1b():
    """MiniCPM5-1B (hd 128), the reference's auto string for one device, weights on the GPU."""
    from minicpm5_mk.config import preset
    from minicpm5_mk.mk_weights import prepare_mk_weights
    from minicpm5_mk.quant import resolve_quant_pair
    from minicpm5_mk.synth import random_hf_state_dict

    cfg = preset("1b")
    quant = resolve_quant_pair("auto", cfg.num_layers, 1, cfg.hidden, cfg.inter)[0]
    sd = random_hf_state_dict(cfg)
    cpu = prepare_mk_weights(sd, cfg.as_mk_cfg(), quant, 8256, log=print)
    sd_dev = {k: v.to("cuda:0") for k, v in sd.items()}
    gpu = prepare_mk_weights(sd_dev, cfg.as_mk_cfg(), quant, 8256, log=print, device="cuda:0")
    bad = [k for k in cpu if not _same(gpu[k], cpu[k])]
    assert not bad, bad
