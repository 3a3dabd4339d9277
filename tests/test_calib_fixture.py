"""Weight calibration and quantisation pinned against the reference's own outputs.

tests/golden/calib_fixture.npz holds what plugin/minicpm5_mk/mk_weights.py's `_calibrate` (:29-110),
`_quantize_w` (:113-123) and `rope_tables` (:20-26) return on the `tiny` / `tiny-hd96` random-init
weights with non-unit gammas (tests/golden/make_calib_fixture.py, run against the reference tree in
the build container).  The product's `hf_layers`, `calibrate`, `quantize_w`, `smooth_factors` and
`rope_tables` must reproduce them bit for bit; `prepare_mk_weights` is then checked to compose them:
its SmoothQuant factors come from the pinned per-channel amax, and its codes / scales / activation
factors dequantise back to gamma * W within half a quantisation step.
"""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

from minicpm5_mk.config import preset
from minicpm5_mk.mk_weights import (calibrate, hf_layers, prepare_mk_weights, quantize_w, rope_tables,
                                    smooth_factors)
from minicpm5_mk.synth import random_hf_state_dict

FIX = os.path.join(os.path.dirname(__file__), "golden", "calib_fixture.npz")
LIN = ("qkv", "o", "gu", "down")
F32 = torch.float32


@pytest.fixture(scope="module")
def fx():
    z = np.load(FIX)
    d = {k: z[k] for k in z.files}
    d["meta"] = json.loads(bytes(d["meta"]).decode())
    return d


def _weights(name, fx):
    cfg = preset(name)
    sd = random_hf_state_dict(cfg, seed=0)
    for i in range(cfg.num_layers):
        p = f"model.layers.{i}."
        sd[p + "input_layernorm.weight"] = torch.from_numpy(fx[f"{name}/gamma_in/{i}"]).to(torch.bfloat16)
        sd[p + "post_attention_layernorm.weight"] = torch.from_numpy(fx[f"{name}/gamma_post/{i}"]).to(torch.bfloat16)
    return cfg, sd


def _digest(t):
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


@pytest.mark.parametrize("name", ["tiny", "tiny-hd96"])
def test_rope_tables_bit_exact(fx, name):
    cfg = preset(name)
    c, s = rope_tables(512, cfg.head_dim, cfg.rope_theta)
    assert np.array_equal(c.view(torch.int16).numpy(), fx[f"{name}/rope_cos"])
    assert np.array_equal(s.view(torch.int16).numpy(), fx[f"{name}/rope_sin"])


@pytest.mark.parametrize("base", ["int8d", "int8", "fp8"])
@pytest.mark.parametrize("name", ["tiny", "tiny-hd96"])
def test_calibrate_and_quantize_bit_exact(fx, name, base):
    """Static scales, per-channel amax (all positions / without position 0) and the 8-bit codes and
    scales of every matrix equal the reference's, including a smoothed q/k/v matrix with a static scale."""
    cfg, sd = _weights(name, fx)
    key = f"{name}/{base}"
    nthreads = torch.get_num_threads()
    torch.set_num_threads(1)
    try:
        layers = hf_layers(sd, cfg.as_mk_cfg(), False, False)
        rc, rs = rope_tables(128, cfg.head_dim, cfg.rope_theta)
        scales, chan, nob = calibrate(layers, sd["model.embed_tokens.weight"].to(F32), rc.to(F32), rs.to(F32),
                                      cfg.as_mk_cfg(), base, gamma_in_act={"qkv": True, "gu": True})
    finally:
        torch.set_num_threads(nthreads)
    got = np.array([[sc[n] for n in LIN] for sc in scales], dtype=np.float64)
    assert np.array_equal(got, fx[key + "/scales"]), (got, fx[key + "/scales"])
    for li in range(cfg.num_layers):
        for n in LIN:
            assert np.array_equal(chan[li][n].numpy(), fx[f"{key}/chan/{li}/{n}"]), (li, n)
            assert np.array_equal(nob[li][n].numpy(), fx[f"{key}/nob/{li}/{n}"]), (li, n)
    dig = fx["meta"]["digests"]
    for li, ld in enumerate(layers):
        for n in LIN:
            wq, sw = quantize_w(ld["w_" + n], base, 1.0)
            assert np.array_equal(sw.numpy(), fx[f"{key}/qw_scale/{li}/{n}"]), (li, n)
            assert _digest(wq) == dig[f"{key}/qw_codes/{li}/{n}"], (li, n)
        smooth = smooth_factors(chan[li]["qkv"], ld["w_qkv"], 0.5)
        wq, sw = quantize_w(ld["w_qkv"] * smooth[:, None], base, scales[li]["qkv"])
        assert np.array_equal(sw.numpy(), fx[f"{key}/qw_smooth_scale/{li}"]), li
        assert _digest(wq) == dig[f"{key}/qw_smooth_codes/{li}"], li


def test_calibration_catches_a_planted_mistake(fx):
    """The fixture is sensitive: dropping the gammas from the activations (a plausible slip) changes
    the pinned per-channel amax."""
    cfg, sd = _weights("tiny", fx)
    layers = hf_layers(sd, cfg.as_mk_cfg(), False, False)
    rc, rs = rope_tables(128, cfg.head_dim, cfg.rope_theta)
    _, chan, _ = calibrate(layers, sd["model.embed_tokens.weight"].to(F32), rc.to(F32), rs.to(F32),
                           cfg.as_mk_cfg(), "int8d", gamma_in_act={"qkv": False, "gu": False})
    assert not np.array_equal(chan[0]["qkv"].numpy(), fx["tiny/int8d/chan/0/qkv"])


@pytest.mark.parametrize("quant", ["int8d:qkv+gu+o+down|sq", "int8:qkv+gu+o+down|sq", "fp8d:qkv+gu+o+down|sq"])
def test_prepare_composes_pinned_pieces(fx, quant, monkeypatch):
    """prepare_mk_weights on the fixture's weights: SmoothQuant factors from the pinned amax (alpha 0.5),
    and a_x * dequant(codes) * s_w == gamma * W within half a step per element, for every linear."""
    for k in [k for k in os.environ if k.startswith("MINICPM5_MK_")]:
        monkeypatch.delenv(k)
    base = quant.split(":")[0]
    cfg, sd = _weights("tiny", fx)
    torch.set_num_threads(1)
    try:
        w = prepare_mk_weights(sd, cfg.as_mk_cfg(), quant, 256, log=lambda *a: None)
    finally:
        torch.set_num_threads(os.cpu_count() or 1)
    layers = hf_layers(sd, cfg.as_mk_cfg(), False, False)
    fbase = {"fp8d": "fp8"}.get(base, base)        # fp8 and fp8d calibrate identically
    scales = fx[f"tiny/{fbase}/scales"]
    for li in range(cfg.num_layers - 1):
        ld = layers[li]
        for j, n in enumerate(LIN):
            W = ld["w_" + n].reshape(ld["w_" + n].shape[0], -1)
            gamma = ld["in_norm"] if n == "qkv" else ld["post_norm"] if n == "gu" else torch.ones(W.shape[0])
            smooth = smooth_factors(torch.from_numpy(fx[f"tiny/{fbase}/chan/{li}/{n}"]), W, 0.5)
            dynamic = base in ("int8d", "fp8d") or n == "down"
            a = w["a_" + n][li]
            if dynamic:
                assert torch.equal(a, gamma / smooth), (li, n)
            else:   # a = gamma / (smooth * sx) with sx the static scale re-measured after smoothing
                sx = (gamma / smooth / a)
                assert torch.allclose(sx, sx[0].expand_as(sx), rtol=1e-6), (li, n)
                assert float(sx[0]) != float(scales[li, j])   # re-measured on the smoothed activation
            codes = w["w_" + n][li].reshape(W.shape[0], -1).to(F32)
            s_w = w["s_" + n][li].reshape(-1)
            sxv = 1.0 if dynamic else float(sx[0])
            step = s_w / sxv                                   # quantisation step of W * smooth
            r = W * smooth[:, None] / step[None, :]            # the value the codes round
            # int8: half a step; e4m3: half an ulp (2^-4 relative), 2^-10 absolute in the subnormals
            half = torch.full_like(r, 0.5) if base.startswith("int8") else torch.clamp(r.abs() * 2.0 ** -4, min=2.0 ** -10)
            assert bool(((codes - r).abs() <= half * (1 + 1e-5)).all()), (li, n)
            # the invariant the kernels rely on: (x * a) @ (codes * s_w) == (x * gamma) @ W up to that rounding
            lhs = a[:, None] * codes * s_w[None, :]
            bound = (a.abs()[:, None] * s_w[None, :]) * half * (1 + 1e-4) + 1e-12
            assert bool(((lhs - gamma[:, None] * W).abs() <= bound + 1e-6 * (gamma[:, None] * W).abs()).all()), (li, n)
