"""Host weight preparation (minicpm5_mk.mk_weights) and the quant-string grammar (minicpm5_mk.quant).

Pinned by invariants, not by restating the formulas:
  * per-output-channel int8: |dequant - w| <= scale / 2, scale = max(amax / 127, 1e-8), codes in +-127;
  * calibration, SmoothQuant and quantisation against the reference's own outputs live in
    tests/test_calib_fixture.py;
  * interleave_gu is a permutation with the [g_0 | u_0 | g_1 | u_1 ...] chunk order;
  * prepare_mk_weights' layout equals what the runtime (and libmk) expect for each quant string;
  * folding gamma / 1/sqrt(hd) is exact algebra: the bf16 path reproduces the FP32 model's q / k / v;
  * auto resolution: model.py:528-551 for one device.
"""
import math

import pytest
import torch


def test_quantize_w_bounds():
    from minicpm5_mk.mk_weights import quantize_w

    g = torch.Generator().manual_seed(0)
    w = torch.randn(300, 70, generator=g) * 0.02
    w[:, 5] = 0.0
    wq, s = quantize_w(w, "int8d", 1.0)
    assert wq.dtype == torch.int8 and s.shape == (70,)
    assert int(wq.abs().max()) == 127
    scale = torch.clamp(w.abs().amax(0) / 127.0, min=1e-8)
    assert torch.equal(s, scale)
    assert ((wq.float() * s - w).abs() <= s / 2 + 1e-12).all()
    assert (wq[:, 5] == 0).all() and float(s[5]) == float(torch.tensor(1e-8, dtype=torch.float32))


def test_interleave_gu_permutation():
    from minicpm5_mk.mk_weights import interleave_gu, mlp_chunk

    assert [mlp_chunk(i) for i in (4608, 6144, 768, 1024, 1000)] == [1536, 1536, 768, 1024, 1000]
    H, inter, ic = 3, 12, 4
    w = torch.arange(H * 2 * inter).reshape(H, 2, inter)
    s = torch.arange(2 * inter, dtype=torch.float32).reshape(2, inter)
    wi, si = interleave_gu(w, s, ic)
    assert wi.shape == (H, 2 * inter) and si.shape == (1, 2 * inter)
    cols = []
    for c in range(inter // ic):
        cols += [(0, c * ic + j) for j in range(ic)] + [(1, c * ic + j) for j in range(ic)]
    for p, (gu, j) in enumerate(cols):
        assert torch.equal(wi[:, p], w[:, gu, j]) and float(si[0, p]) == float(s[gu, j])
    assert sorted(wi[0].tolist()) == sorted(w[0].reshape(-1).tolist())


@pytest.mark.parametrize("quant", ["auto", "bf16", "int8d", "int8d:qkv+gu+o|sq|lastbf16|fqkv|fmlp",
                                   "int8d:qkv+gu|sq", "int8d:qkv+gu+o+down|sq|fmlp"])
def test_prepare_layout_matches_runtime(quant):
    from minicpm5_mk.config import preset
    from minicpm5_mk.mk_weights import prepare_mk_weights
    from minicpm5_mk.quant import resolve_quant_pair
    from minicpm5_mk.runtime import expected_shapes, shape_ok
    from minicpm5_mk.synth import random_hf_state_dict

    cfg = preset("tiny")
    q = resolve_quant_pair(quant, cfg.num_layers, 1, cfg.hidden, cfg.inter)[0]
    w = prepare_mk_weights(random_hf_state_dict(cfg), cfg.as_mk_cfg(), q, 512, log=lambda *a: None)
    for k, (shape, dtype) in expected_shapes(cfg.num_layers, cfg.hidden, cfg.inter, cfg.n_q, cfg.n_kv,
                                             cfg.head_dim, q).items():
        assert shape_ok(w[k], shape, cfg.num_layers - 1) and w[k].dtype == dtype, (k, w[k].shape, w[k].dtype, shape)
    assert w["cos"].shape == (512, cfg.head_dim) and w["cos"].dtype == torch.bfloat16


def test_bf16_folding_reproduces_fp32_projections():
    """bf16 mode folds gamma into the rows and 1/sqrt(hd) into W_q (mk_weights.py:140-160)."""
    from minicpm5_mk.config import preset
    from minicpm5_mk.mk_weights import prepare_mk_weights
    from minicpm5_mk.synth import random_hf_state_dict

    cfg = preset("tiny")
    sd = random_hf_state_dict(cfg)
    g = torch.Generator().manual_seed(2)
    gamma = (torch.rand(cfg.hidden, generator=g) + 0.5).to(torch.bfloat16)
    sd["model.layers.0.input_layernorm.weight"] = gamma
    w = prepare_mk_weights(sd, cfg.as_mk_cfg(), "bf16", 256, log=lambda *a: None)
    xn = torch.randn(4, cfg.hidden, generator=g)
    got = xn @ w["w_qkv"][0].float()
    q = (xn * gamma.float()) @ sd["model.layers.0.self_attn.q_proj.weight"].float().t() / math.sqrt(cfg.head_dim)
    assert torch.allclose(got[:, :cfg.q_dim], q, atol=0.02 * float(q.abs().max()))


def test_rope_tables_match_golden():
    from minicpm5_mk.mk_weights import rope_tables
    from oracle import golden

    c, s = rope_tables(8192, 128, 5e6)
    cg, sg = golden.rope_tables(8192, 128, 5e6)
    # f32 angles rounded to bf16 vs f64 angles: one bf16 ulp plus the f32 angle error at t ~ 8k
    assert (c.float() - cg).abs().max() < 4e-3 and (s.float() - sg).abs().max() < 4e-3


def test_quant_grammar_and_auto():
    from minicpm5_mk.quant import parse_quant, quant_flags, resolve_quant_pair, validate_quant

    assert parse_quant("int8d:qkv+gu|sq|fmlp") == {"qkv": "int8d", "o": "bf16", "gu": "int8d", "down": "bf16"}
    assert parse_quant("bf16") == {k: "bf16" for k in ("qkv", "o", "gu", "down")}
    assert quant_flags("int8d:qkv+gu|sq|lastbf16") == {"sq", "lastbf16"}
    assert resolve_quant_pair("auto", 24, 1, 1536, 4608)[0] == "int8d:qkv+gu|sq|lastbf16|fqkv|fmlp"
    assert resolve_quant_pair("auto", 42, 1, 2048, 6144)[0] == "int8d:qkv+gu+o|sq|lastbf16|fqkv|fmlp"
    assert resolve_quant_pair("auto", 24, 1, 8192, 8192)[0] == "int8d:qkv+gu|sq|lastbf16|fqkv"   # no fmlp: too big
    assert resolve_quant_pair("auto", 24, 2, 1536, 4608) == ("int8d:qkv+gu|sq|lastbf16|fqkv|fmlp", "bf16")
    assert resolve_quant_pair("bf16", 24) == ("bf16", "bf16")
    for bad in ("int4", "int8d:qkv+mlp", "bf16|fast"):
        with pytest.raises(ValueError):
            validate_quant(bad)
    validate_quant("fp8d:qkv+gu|sq")
