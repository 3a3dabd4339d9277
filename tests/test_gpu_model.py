"""Whole-model parity of the libmk prefill path (GPU; through MkModel -> the C ABI).

  * tiny config, every supported quant mode: libmk vs the oracle's emulation of the same quantized
    algebra (oracle/emulate.mk_forward) on identical prepared weights and ids; at S <= 1024 also vs the
    emulation with the reference's own short-sequence attention kernel (its default dispatch).
  * full MiniCPM5 architectures at (1, 8192) with random-init weights (seed 0) and ids (seed 1234),
    auto quant: last-token logits vs the committed FP32 golden (tests/golden/golden_*.npz, written by
    tests/golden/make_golden.py from oracle/golden.py).  The argmax must be identical (tie-aware for the
    one config whose golden top-2 margin is below the W8A8 error); the logits tolerance is stated per
    config below (about 2x the CPU emulator's own W8A8 error vs FP32).
  * full architectures at (1, 1024) (the short-prompt path) vs their FP32 goldens, bounds and argmax
    rules from the CPU emulation of the same numerics.
  * full architectures at (1, 8192): libmk vs full-size fixtures of the CPU emulation of the same W8A8
    numerics (tests/golden/emulate_*.npz, tests/golden/make_emulator_fixture.py), bounded tightly.
  * batch invariance at the reference's batch shapes (B, 8192), B = 4..32 for 1B-hd96 and 2B (the
    reference's batch gate, benchmark/run_benchmark.py:714-727): every row of the batch equals the
    same sequence run alone, bitwise, and row 0 (the golden's sequence) meets the golden checks.
  * batch invariance at tiny size, and hipGraph replay equals eager launches, bitwise.
  * the reference-signature op `runtime.forward` (model.py:749-751): 29 arguments, padded ids,
    bf16 (1,) dummies, bitwise equal to MkModel.forward.
"""
import json
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
BF16 = torch.bfloat16


def _dev():
    assert torch.cuda.is_available(), "GPU test needs a visible MI355X"
    return torch.device("cuda:0")


def _build(cfg, quant, sd, max_seq, dev):
    from minicpm5_mk.mk_weights import prepare_mk_weights
    from minicpm5_mk.runtime import WEIGHT_ORDER, MkModel

    w = prepare_mk_weights(sd, cfg.as_mk_cfg(), quant, max_seq, log=lambda *a: None)
    wd = {k: w[k].to(dev) for k in WEIGHT_ORDER}
    m = MkModel(wd, sd["model.embed_tokens.weight"].to(dev), w["cos"].to(dev), w["sin"].to(dev),
                sd["model.norm.weight"].to(dev), quant, cfg.n_q, cfg.n_kv, cfg.head_dim, cfg.eps,
                lm_head=sd["lm_head.weight"].to(dev))
    return m, w


TINY_QUANTS = ["int8d:qkv+gu|sq|lastbf16|fqkv|fmlp", "int8d:qkv+gu+o|sq|lastbf16|fqkv|fmlp", "bf16",
               "int8d|sq|lastbf16|fqkv|fmlp", "int8d:qkv+gu+o+down|sq", "int8d:qkv+gu|sq",
               "fp8d|sq|lastbf16", "fp8:qkv+gu+o|sq", "fp8", "int8|sq|fqkv|fmlp", "int8:qkv+o+gu+down"]


@pytest.mark.parametrize("name", ["tiny", "tiny-hd96"])
@pytest.mark.parametrize("quant", TINY_QUANTS)
def test_tiny_vs_emulator(name, quant):
    from minicpm5_mk.config import preset
    from minicpm5_mk.synth import random_hf_state_dict, random_token_ids
    from oracle import emulate

    dev = _dev()
    cfg = preset(name)
    print(f"[model] {name} {quant}", flush=True)
    sd = random_hf_state_dict(cfg)
    ids = random_token_ids(2, 512)
    m, w = _build(cfg, quant, sd, 1024, dev)
    hid, lg = m.forward(ids.reshape(-1).to(dev), 2, 512, logits=True)
    hid, lg = hid.float().cpu(), lg.cpu()
    h_ref, lg_ref = emulate.mk_forward(ids, w, sd["model.embed_tokens.weight"], sd["model.norm.weight"], cfg, quant,
                                       sd["lm_head.weight"])
    assert torch.equal(hid[2:], torch.zeros_like(hid[2:])), "pad rows must be zero"
    err = (lg - lg_ref).abs()
    herr = (hid[:2] - h_ref.float()).abs()
    print(f"[model] logits max {err.max():.4g} mean {err.mean():.4g}; hidden max {herr.max():.4g}", flush=True)
    # attention / bf16-GEMM summation order differs from the CPU (and the fp8 MFMA sums its products at
    # reduced internal precision), and a bf16 ulp flip of one hidden element moves logits by
    # ~|lm_head row| * 2^-8; an fp8 code flip moves a GEMM input by 1/16-1/8 of its value.  Observed over
    # the 11 quant strings: max 0.035, mean 6.3e-3 (fp8 on the hd-96 shapes), 4.6e-3 for the int8 modes.
    assert err.max() <= 0.05 and err.mean() <= 1e-2
    # tie-aware top-1 (cf. the reference's gate, benchmark/gate.py:47-56): the GPU's argmax must be a
    # top-1 of the emulator up to the measured logit error (random tiny models have near-ties)
    am = lg.argmax(-1, keepdim=True)
    gap = lg_ref.max(-1).values - lg_ref.gather(-1, am).squeeze(-1)
    assert (gap <= 2 * err.max()).all(), gap
    m.close()


@pytest.mark.parametrize("name,B,S", [("tiny", 1, 1024), ("tiny-hd96", 2, 512), ("tiny", 2, 128)])
def test_short_prompt_vs_reference_dispatch(name, B, S):
    """At S <= 1024 the reference (attn=auto, mk_jax.py:364-365) runs its S <= 1024 attention kernel
    (attn_fused_small: exact row max, P normalised to bf16 before PV); this build runs its one attention
    algorithm (the super_gqa_v2 numerics) at every length.  Whole-model logits vs the emulator with the
    reference's dispatch (emulate.mk_forward(attn="auto")).  On these shapes (tiny configs, 1B W8A8 auto)
    the two dispatches differ on the CPU by max 0.0075-0.0100 / mean 1.4-1.8e-3, and the GPU measured
    max 0.0075-0.0115 / mean 1.4-1.9e-3 against the reference's: bound max 0.025 / mean 4e-3 (about 2x),
    with the tie-aware argmax."""
    from minicpm5_mk.config import preset
    from minicpm5_mk.synth import random_hf_state_dict, random_token_ids
    from oracle import emulate

    dev = _dev()
    cfg = preset(name)
    quant = "int8d:qkv+gu|sq|lastbf16|fqkv|fmlp"
    print(f"[short-ref] {name} ({B}, {S})", flush=True)
    sd = random_hf_state_dict(cfg)
    ids = random_token_ids(B, S)
    m, w = _build(cfg, quant, sd, 1024, dev)
    _, lg = m.forward(ids.reshape(-1).to(dev), B, S, logits=True)
    lg = lg[:B].cpu()
    _, lg_ref = emulate.mk_forward(ids, w, sd["model.embed_tokens.weight"], sd["model.norm.weight"], cfg, quant,
                                   sd["lm_head.weight"], attn="auto")
    err = (lg - lg_ref).abs()
    print(f"[short-ref] logits max {err.max():.4g} mean {err.mean():.4g}", flush=True)
    assert err.max() <= 0.025 and err.mean() <= 4e-3
    am = lg.argmax(-1, keepdim=True)
    gap = lg_ref.max(-1).values - lg_ref.gather(-1, am).squeeze(-1)
    assert (gap <= 2 * err.max()).all(), gap
    m.close()


def test_one_kv_head_hd96_vs_emulator():
    """8 query heads over 1 kv head at head_dim 96: the K and V column blocks of the QKV projection do
    not start at multiples of 64 (768 + 96), so the attention's RoPE'd K / V^T come from the prep kernel
    instead of the projection's epilogue; the model still matches the emulator like the other tiny
    configurations, and switching the fused prep on or off changes nothing."""
    import dataclasses

    from minicpm5_mk.config import preset
    from minicpm5_mk.synth import random_hf_state_dict, random_token_ids
    from oracle import emulate

    dev = _dev()
    cfg = dataclasses.replace(preset("tiny-hd96"), n_q=8, n_kv=1, name="tiny-hd96-kv1")
    quant = "int8d:qkv+gu|sq|lastbf16|fqkv|fmlp"
    sd = random_hf_state_dict(cfg)
    ids = random_token_ids(2, 256, seed=9)
    m, w = _build(cfg, quant, sd, 1024, dev)
    hid, lg = m.forward(ids.reshape(-1).to(dev), 2, 256, logits=True)
    m.set_attn_prep_fused(False)
    hid0, lg0 = m.forward(ids.reshape(-1).to(dev), 2, 256, logits=True)
    assert torch.equal(hid, hid0) and torch.equal(lg, lg0)
    _, lg_ref = emulate.mk_forward(ids, w, sd["model.embed_tokens.weight"], sd["model.norm.weight"], cfg, quant,
                                   sd["lm_head.weight"])
    err = (lg.cpu() - lg_ref).abs()
    print(f"[model] tiny-hd96-kv1 logits max {err.max():.4g} mean {err.mean():.4g}", flush=True)
    assert err.max() <= 0.05 and err.mean() <= 1e-2
    m.close()


@pytest.mark.parametrize("name,B,S", [("tiny", 3, 128), ("tiny-hd96", 2, 384), ("tiny", 1, 896)])
def test_short_seq_vs_emulator(name, B, S):
    """Lengths the reference serves below 1024 (multiples of 128, model.py:131-136): the last chunk of
    the last-token attention is partial at 128 / 384 / 896."""
    from minicpm5_mk.config import preset
    from minicpm5_mk.synth import random_hf_state_dict, random_token_ids
    from oracle import emulate

    dev = _dev()
    cfg = preset(name)
    quant = "int8d:qkv+gu|sq|lastbf16|fqkv|fmlp"
    print(f"[short] {name} B={B} S={S}", flush=True)
    sd = random_hf_state_dict(cfg)
    ids = random_token_ids(B, S, seed=S)
    m, w = _build(cfg, quant, sd, 1024, dev)
    hid, lg = m.forward(ids.reshape(-1).to(dev), B, S, logits=True)
    hid, lg = hid.float().cpu(), lg.cpu()
    h_ref, lg_ref = emulate.mk_forward(ids, w, sd["model.embed_tokens.weight"], sd["model.norm.weight"], cfg, quant,
                                       sd["lm_head.weight"])
    err = (lg - lg_ref).abs()
    print(f"[short] logits max {err.max():.4g} mean {err.mean():.4g}", flush=True)
    assert err.max() <= 0.05 and err.mean() <= 5e-3
    am = lg.argmax(-1, keepdim=True)
    gap = lg_ref.max(-1).values - lg_ref.gather(-1, am).squeeze(-1)
    assert (gap <= 2 * err.max()).all(), gap
    m.close()



@pytest.mark.parametrize("name,hd,S", [("tiny-hd96", 96, 12288), ("tiny", 128, 9216)])
def test_long_seq_vs_emulator(name, hd, S):
    """Sequences past 8192 tokens: the last-token attention merges S / 64 chunk partials, 1024 / hd groups
    of chunks with their first 16 loads issued up front; 192 chunks at hd 96 and 144 at hd 128 also take
    the loop over the chunks beyond those (mk_attn_* serve any multiple of 1024 up to max_seq)."""
    import dataclasses

    from minicpm5_mk.config import preset
    from minicpm5_mk.synth import random_hf_state_dict, random_token_ids
    from oracle import emulate

    dev = _dev()
    cfg = dataclasses.replace(preset(name), head_dim=hd, name=f"{name}-s{S}")
    quant = "int8d:qkv+gu|sq|lastbf16|fqkv|fmlp"
    print(f"[long] {name} hd={hd} S={S}", flush=True)
    sd = random_hf_state_dict(cfg)
    ids = random_token_ids(1, S, seed=S)
    m, w = _build(cfg, quant, sd, S, dev)
    _, lg = m.forward(ids.reshape(-1).to(dev), 1, S, logits=True)
    lg = lg.cpu()
    _, lg_ref = emulate.mk_forward(ids, w, sd["model.embed_tokens.weight"], sd["model.norm.weight"], cfg, quant,
                                   sd["lm_head.weight"])
    err = (lg - lg_ref).abs()
    print(f"[long] logits max {err.max():.4g} mean {err.mean():.4g}", flush=True)
    assert err.max() <= 0.05 and err.mean() <= 5e-3
    m.close()

# (preset, logits max-abs tolerance vs FP32, mean-abs tolerance): 2x the error of the CPU emulation of
# the same W8A8 numerics (oracle/emulate.mk_forward) vs the FP32 golden at (1, 8192):
#   1b       max 0.216  mean 0.0359  mean|dlogprob| top-20 0.050
#   1b-hd96  max 0.262  mean 0.0467                        0.046
#   2b       max 0.519  mean 0.0923                        0.092   (int8 O projection too)
# strict: the argmax must equal the golden's.  1b-hd96's golden top-1 / top-2 margin (0.029) is below the
# W8A8 path's mean logit error, so there the top-1 is judged tie-aware like the reference gate
# (benchmark/gate.py:47-56): the chosen token must be within 0.1 nats of the golden top-1.
FULL = [("1b", 0.45, 0.075, True), ("1b-hd96", 0.55, 0.095, False), ("2b", 1.05, 0.19, True)]
_FULL_MODELS: dict = {}


def _golden(name):
    gold = np.load(os.path.join(HERE, "golden", f"golden_{name}_b1_s8192.npz"))
    return gold, json.loads(str(gold["meta"]))


def _full_model(name, quant="auto"):
    """One libmk model per (preset, quant) for the whole module (weight preparation is the slow part)."""
    from minicpm5_mk.config import preset
    from minicpm5_mk.quant import resolve_quant_pair
    from minicpm5_mk.synth import random_hf_state_dict

    key = (name, quant)
    if key not in _FULL_MODELS:
        _, meta = _golden(name)
        cfg = preset(name)
        print(f"[full] {name} {quant}: weights", flush=True)
        sd = random_hf_state_dict(cfg, seed=meta["weight_seed"])
        q = resolve_quant_pair(quant, cfg.num_layers, 1, cfg.hidden, cfg.inter)[0]
        _FULL_MODELS[key] = _build(cfg, q, sd, 8256, _dev())[0]
        del sd
    return _FULL_MODELS[key]


@pytest.fixture(scope="module", autouse=True)
def _close_full_models():
    yield
    for m in _FULL_MODELS.values():
        m.close()
    _FULL_MODELS.clear()


def _golden_checks(name, lg, g, tol_max, tol_mean, strict):
    err = (lg - g).abs()
    srt = torch.sort(g, descending=True).values
    lp, lpg = torch.log_softmax(lg, -1), torch.log_softmax(g, -1)
    top = torch.topk(lpg, 20).indices
    dlp = (lp[top] - lpg[top]).abs().mean()
    print(f"[full] {name}: logits max {err.max():.4f} mean {err.mean():.4f} rel {err.max() / g.abs().max():.4f}; "
          f"argmax {int(lg.argmax())} vs {int(g.argmax())} (golden margin {float(srt[0] - srt[1]):.4f}); "
          f"mean |dlogprob| top20 {float(dlp):.4f}", flush=True)
    if isinstance(strict, (tuple, frozenset, set)):   # the golden top-1 or these named tokens
        assert int(lg.argmax()) in {int(g.argmax()), *strict}
    elif strict:
        assert int(lg.argmax()) == int(g.argmax())
    else:
        assert float(lpg.max() - lpg[int(lg.argmax())]) <= 0.1
    assert err.max() <= tol_max and err.mean() <= tol_mean
    assert float(dlp) <= 0.15            # the reference gate's FAIL boundary (benchmark/gate.py:115)


@pytest.mark.parametrize("name,tol_max,tol_mean,strict", FULL)
def test_full_model_vs_fp32_golden(name, tol_max, tol_mean, strict):
    from minicpm5_mk.synth import random_token_ids

    gold, meta = _golden(name)
    m = _full_model(name)
    ids = random_token_ids(1, 8192, seed=meta["id_seed"])
    print(f"[full] {name} forward quant={m.quant}", flush=True)
    _, lg = m.forward(ids.reshape(-1).to(_dev()), 1, 8192, logits=True)
    _golden_checks(name, lg.cpu()[0], torch.from_numpy(gold["logits"][0]), tol_max, tol_mean, strict)


# (preset, max, mean, argmax rule) at (1, 1024) against tests/golden/golden_<preset>_b1_s1024.npz.  The CPU
# emulation of the same W8A8 numerics (v2 attention / the reference's own S <= 1024 kernel) errs:
#   1b       max 0.202 / 0.188  mean 0.035 / 0.035   argmax = golden top-1 (margin 0.140)
#   1b-hd96  max 0.218 / 0.205  mean 0.042 / 0.039   top-1, or golden #2 (token 123131, 0.039 nats below),
#                                                    which the v2 emulation picks
#   2b       max 0.594 / 0.528  mean 0.092 / 0.095   golden #2 (token 43840, 0.183 nats below) under both
#                                                    attention kernels: the W8A8 error moves the argmax
# Bounds: 1b and 1b-hd96 those of (1, 8192); 2b max 1.2 (2x the emulation), mean 0.19.
SHORT = [("1b", 0.45, 0.075, True), ("1b-hd96", 0.55, 0.095, (123131,)), ("2b", 1.2, 0.19, (43840,))]


@pytest.mark.parametrize("name,tol_max,tol_mean,rule", SHORT)
def test_full_model_short_prompt_vs_fp32_golden(name, tol_max, tol_mean, rule):
    """Full architectures at (1, 1024) -- the short-prompt path: 64x128 two-stage GEMM tiles, one
    attention workgroup per work item, the attention launch's weight prefetch -- vs their FP32 goldens
    (make_golden.py --seq 1024).  Bounds and argmax rules from the CPU emulation of the same numerics
    (table above): where that emulation itself picks the golden's #2 token, so may the GPU."""
    from minicpm5_mk.synth import random_token_ids

    gold = np.load(os.path.join(HERE, "golden", f"golden_{name}_b1_s1024.npz"))
    meta = json.loads(str(gold["meta"]))
    assert meta["seq"] == 1024 and meta["weight_seed"] == _golden(name)[1]["weight_seed"]
    m = _full_model(name)
    ids = random_token_ids(1, 1024, seed=meta["id_seed"])
    print(f"[full] {name} (1, 1024) forward", flush=True)
    _, lg = m.forward(ids.reshape(-1).to(_dev()), 1, 1024, logits=True)
    _golden_checks(f"{name}-s1024", lg.cpu()[0], torch.from_numpy(gold["logits"][0]), tol_max, tol_mean, rule)


# GPU vs the CPU emulation of the same W8A8 numerics at (1, 8192): (preset, max-abs bound, mean-abs bound).
# The emulator uses the kernels' own rounding points (f32 exp2, K RoPE rounded once); what differs is the
# summation order of the bf16 GEMMs and of attention.  Those bf16-ulp differences flip per-token int8
# codes at the next layer's activation quantisation, and the flips compound over 23 (1B) or 41 (2B)
# layers, so the whole-model difference is about half the W8A8 error itself.  Measured on MI355X (max /
# mean): 1b 0.115 / 0.022, 1b-hd96 0.142 / 0.026, 2b 0.428 / 0.070; the bounds are 1.5x those.  The tight
# full-size kernel check is the two-layer test below, where nothing has time to compound.
EMU = [("1b", 0.17, 0.033), ("1b-hd96", 0.21, 0.039), ("2b", 0.64, 0.105)]


@pytest.mark.parametrize("name,tol_max,tol_mean", EMU)
def test_full_model_vs_emulator(name, tol_max, tol_mean):
    from minicpm5_mk.synth import random_token_ids

    path = os.path.join(HERE, "golden", f"emulate_{name}_auto_b1_s8192.npz")
    fx = np.load(path)
    emeta = json.loads(bytes(fx["meta"]).decode())
    m = _full_model(name)
    assert emeta["quant"] == m.quant
    ids = random_token_ids(1, 8192, seed=emeta["id_seed"])
    _, lg = m.forward(ids.reshape(-1).to(_dev()), 1, 8192, logits=True)
    lg = lg.cpu()[0]
    e = torch.from_numpy(fx["logits"][0])
    err = (lg - e).abs()
    print(f"[emu] {name}: GPU vs emulator max {err.max():.4f} mean {err.mean():.4f}; argmax GPU {int(lg.argmax())} "
          f"emulator {int(e.argmax())} golden {emeta.get('golden_argmax')}; emulator vs golden max "
          f"{emeta.get('vs_golden_max', float('nan')):.4f}", flush=True)
    assert err.max() <= tol_max and err.mean() <= tol_mean


# The quantisation variants (fp8 dynamic on the CDNA4 fp8 MFMA, static int8) at full size: MiniCPM5-1B at
# (1, 8192), GPU vs the CPU emulation of the same numerics (tests/golden/emulate_1b_<tag>_b1_s8192.npz, written
# by make_emulator_fixture.py --quant ...) and vs the FP32 golden.  (quant, fixture tag, max, mean): bounds
# 1.5x the measured GPU-vs-emulator error, as for the W8A8 fixtures above.  The emulations themselves err
# vs FP32: fp8d max 0.628 / mean 0.117, mean |dlogprob| top-20 0.129, argmax the golden's #3 (token 6581,
# 0.166 nats below the top-1: e4m3's 3-bit mantissa moves it); static int8 0.211 / 0.038, 0.050, top-1; int8
# with an int8 O and down projection 0.431 / 0.069, 0.071, top-1; 2B fp8d 1.393 / 0.231, 0.236 -- beyond the
# reference gate's FAIL boundary (0.15) already in the emulation, its argmax the golden's rank 16.
# Argmax rule: the golden top-1 or the token the emulation of the same numerics picks; not applied where
# the emulation itself fails the gate (2B fp8d: the fp8 error, mean 0.23, is ~3x the golden's top-2 margin,
# so the top token is noise on either side -- the GPU picked another one than the emulation).
# Measured on MI355X (max / mean vs the emulation): 1B fp8d 0.329 / 0.058, static int8 0.161 / 0.027,
# int8d with int8 O / down 0.352 / 0.062; 2B fp8d 0.727 / 0.136.
QVARIANTS = [("1b", "fp8d:qkv+gu|sq|lastbf16", "fp8d", 0.5, 0.087),
             ("1b", "int8:qkv+gu|sq|lastbf16", "int8", 0.25, 0.041),
             ("1b", "int8d:qkv+gu+o+down|sq|lastbf16|fqkv|fmlp", "int8d", 0.53, 0.093),
             ("2b", "fp8d:qkv+gu|sq|lastbf16", "fp8d", 1.09, 0.204)]


@pytest.mark.parametrize("name,quant,tag,tol_max,tol_mean", QVARIANTS)
def test_full_model_quant_variants(name, quant, tag, tol_max, tol_mean):
    from minicpm5_mk.synth import random_token_ids

    fx = np.load(os.path.join(HERE, "golden", f"emulate_{name}_{tag}_b1_s8192.npz"))
    emeta = json.loads(bytes(fx["meta"]).decode())
    gold, meta = _golden(name)
    m = _full_model(name, quant)
    assert emeta["quant"] == m.quant == quant
    ids = random_token_ids(1, 8192, seed=emeta["id_seed"])
    _, lg = m.forward(ids.reshape(-1).to(_dev()), 1, 8192, logits=True)
    lg = lg.cpu()[0]
    e = torch.from_numpy(fx["logits"][0])
    g = torch.from_numpy(gold["logits"][0])
    err, gerr = (lg - e).abs(), (lg - g).abs()
    lp, lpg = torch.log_softmax(lg, -1), torch.log_softmax(g, -1)
    top = torch.topk(lpg, 20).indices
    dlp = float((lp[top] - lpg[top]).abs().mean())
    edlp = float((torch.log_softmax(e, -1)[top] - lpg[top]).abs().mean())
    print(f"[variant] {name} {quant}: emulator mean |dlogprob| top20 {edlp:.4f}; GPU vs emulator max {err.max():.4f} mean {err.mean():.4f}; vs golden max "
          f"{gerr.max():.4f} mean {gerr.mean():.4f} (emulator vs golden max {emeta['vs_golden_max']:.4f} mean "
          f"{emeta['vs_golden_mean']:.4f}); mean |dlogprob| top20 {dlp:.4f}; argmax GPU {int(lg.argmax())} "
          f"emulator {int(e.argmax())} golden {int(g.argmax())}", flush=True)
    assert err.max() <= tol_max and err.mean() <= tol_mean
    # against FP32: the reference gate's FAIL boundary (benchmark/gate.py:115) and the argmax rule above or,
    # where the emulation of the same numerics is itself beyond that boundary, no more than 1.2x its error
    if edlp <= 0.15:
        assert int(lg.argmax()) in {int(g.argmax()), int(e.argmax())} and dlp <= 0.15
    else:
        assert dlp <= 1.2 * edlp
    m.release_buffers()


@pytest.mark.parametrize("name", ["1b", "1b-hd96", "2b"])
def test_two_layer_full_size_vs_emulator(name):
    """The architectures truncated to two layers (one full-sequence layer, then the last-token layer) at
    (2, 8192): every kernel runs at its full-size shape, and the emulator of the same numerics (run here
    on the CPU) bounds the result tightly, since no rounding difference compounds over layers."""
    from minicpm5_mk.config import preset
    from minicpm5_mk.quant import resolve_quant_pair
    from minicpm5_mk.synth import random_hf_state_dict, random_token_ids
    from oracle import emulate

    full = preset(name)
    cfg = full.replace(num_layers=2, name=name + "-2l")
    quant = resolve_quant_pair("auto", full.num_layers, 1, full.hidden, full.inter)[0]
    print(f"[2l] {name} {quant}", flush=True)
    sd = random_hf_state_dict(cfg, seed=3)
    ids = random_token_ids(2, 8192, seed=99)
    m, w = _build(cfg, quant, sd, 8192, _dev())
    hid, lg = m.forward(ids.reshape(-1).to(_dev()), 2, 8192, logits=True)
    hid, lg = hid.float().cpu(), lg.cpu()
    m.close()
    nthreads = torch.get_num_threads()
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    try:
        h_ref, lg_ref = emulate.mk_forward(ids, w, sd["model.embed_tokens.weight"], sd["model.norm.weight"], cfg,
                                           quant, sd["lm_head.weight"])
    finally:
        torch.set_num_threads(nthreads)
    err = (lg - lg_ref).abs()
    herr = (hid[:2] - h_ref.float()).abs()
    print(f"[2l] {name}: logits max {err.max():.4f} mean {err.mean():.5f}; hidden max {herr.max():.4f}; "
          f"argmax {lg.argmax(-1).tolist()} vs {lg_ref.argmax(-1).tolist()}", flush=True)
    assert err.max() <= TWO_LAYER[name][0] and err.mean() <= TWO_LAYER[name][1]


# two-layer bounds (max, mean |logit error|), 1.5x what MI355X measured: 1b 0.045 / 0.0075,
# 1b-hd96 0.051 / 0.0076, 2b 0.100 / 0.0151 (a few bf16 ulps of the final-normed hidden state, from
# int8 code flips at the MLP's activation quantisation and the bf16 GEMMs' summation order)
TWO_LAYER = {"1b": (0.07, 0.012), "1b-hd96": (0.08, 0.012), "2b": (0.15, 0.023)}


# (preset, batch sizes): the 1B-hd96 and 2B prefill workloads at B = 4..32, plus the reference's 1B; 2B at
# B = 48 runs in two chunks (42 + 6 sequences: the (T, I) bf16 activation of 48 x 8192 tokens exceeds 4 GiB).
# B = 2 at hd 128: the QKV projection takes two rounds of 256x320 tiles (one round at B = 1)
BATCH = [("1b-hd96", 4), ("1b-hd96", 8), ("1b-hd96", 16), ("1b-hd96", 32), ("1b", 2), ("1b", 4), ("1b", 32), ("2b", 2),
         ("2b", 4), ("2b", 8), ("2b", 16), ("2b", 32), ("2b", 48)]


@pytest.mark.parametrize("name,B", BATCH)
def test_full_batch_invariance_s8192(name, B):
    """(B, 8192): every row equals its sequence scored alone, bitwise (hidden and logits); row 0 is the
    golden's sequence and meets its checks."""
    from minicpm5_mk.synth import random_token_ids

    gold, meta = _golden(name)
    tol = {n: (a, b, c) for n, a, b, c in FULL}[name]
    m = _full_model(name)
    dev = _dev()
    ids = random_token_ids(B, 8192, seed=meta["id_seed"]).to(dev)
    print(f"[batch] {name} B={B}", flush=True)
    hB, lB = m.forward(ids.reshape(-1), B, 8192, logits=True)
    assert torch.equal(hB[B:], torch.zeros_like(hB[B:]))
    for b in range(B):
        h1, l1 = m.forward(ids[b].reshape(-1), 1, 8192, logits=True, copy_out=False)
        assert torch.equal(h1[0], hB[b]) and torch.equal(l1[0], lB[b]), f"row {b} differs from its single run"
    _golden_checks(name, lB[0].cpu(), torch.from_numpy(gold["logits"][0]), *tol)
    m.release_buffers()


@pytest.mark.parametrize("name,B,S", [("tiny", 1, 896), ("tiny", 3, 384), ("tiny", 2, 2048), ("tiny-hd96", 2, 1152)])
def test_last_layer_step_isolated(name, B, S):
    """The last-token layer (mk_jax.py:492-520: K/V projection over all S tokens, q / O / gate-up / down on
    the last token only, chunked single-query attention and its merge, bf16 weights) on its own.  Layer
    0's O and down projections are zero, so the residual stream it passes on is the embedding exactly
    (bf16(x + 0) = x); the GPU's final-normed rows and logits are then compared with
    final_norm(emulate.last_layer_step(embedding)).  Bounds: the two sides differ only in f32 summation
    orders, so a hidden value may differ by a bf16 rounding or two (measured: max 1 ulp, 0.0156 at
    |values| ~3.3; mean 5e-4 .. 2.3e-3; logits max 3e-3 .. 8e-3)."""
    from minicpm5_mk.config import preset
    from minicpm5_mk.synth import random_hf_state_dict, random_token_ids
    from oracle import emulate

    dev = _dev()
    cfg = preset(name).replace(num_layers=2)
    sd = random_hf_state_dict(cfg, seed=7)
    sd["model.layers.0.self_attn.o_proj.weight"].zero_()
    sd["model.layers.0.mlp.down_proj.weight"].zero_()
    quant = "int8d:qkv+gu|sq|lastbf16|fqkv|fmlp"
    m, w = _build(cfg, quant, sd, S + 64, dev)
    ids = random_token_ids(B, S, seed=S + B)
    print(f"[last layer] {name} B={B} S={S}", flush=True)
    h, lg = m.forward(ids.reshape(-1).to(dev), B, S, logits=True)
    h, lg = h[:B].float().cpu(), lg.float().cpu()
    x = sd["model.embed_tokens.weight"][ids.long()].to(BF16)
    x_last = emulate.last_layer_step(x, w, w["cos"], w["sin"], cfg.n_q, cfg.n_kv, cfg.head_dim, cfg.eps)
    ref = (emulate._rms_unit_bf16(x_last, cfg.eps) * sd["model.norm.weight"].float()).to(BF16).float()
    lref = ref @ sd["lm_head.weight"].float().t()
    eh, el = (h - ref).abs(), (lg - lref).abs()
    print(f"[last layer] hidden max {eh.max():.4g} mean {eh.mean():.3g} (|ref| max {ref.abs().max():.3g}); "
          f"logits max {el.max():.4g}; argmax {lg.argmax(-1).tolist()} vs {lref.argmax(-1).tolist()}", flush=True)
    assert eh.max() <= 0.012 * ref.abs().max() and eh.mean() <= 1.5e-3 * ref.abs().max()
    assert el.max() <= 0.02 and torch.equal(lg.argmax(-1), lref.argmax(-1))
    m.close()


@pytest.mark.parametrize("name", ["1b", "2b"])
def test_short_prompt_batch_invariance(name):
    """Short prompts pick GEMM tiles by problem size: at (1, 1024) and (1, 2048) the bf16 O / down
    projections run on the deep-ring 64x128 / 128x128 tiles, inside a (4, 1024) batch on the standard
    ones.  The K summation order is the same on every tile, so each row equals its sequence scored
    alone, bitwise."""
    from minicpm5_mk.synth import random_token_ids

    m = _full_model(name)
    dev = _dev()
    for S, B in ((1024, 4), (2048, 2)):
        ids = random_token_ids(B, S, seed=11).to(dev)
        print(f"[short] {name} ({B}, {S})", flush=True)
        hB, lB = m.forward(ids.reshape(-1), B, S, logits=True)
        for b in range(B):
            h1, l1 = m.forward(ids[b].reshape(-1), 1, S, logits=True, copy_out=False)
            assert torch.equal(h1[0], hB[b]) and torch.equal(l1[0], lB[b]), f"({B}, {S}) row {b} differs"
    m.release_buffers()


def test_full_model_bf16_1b_hd96_argmax():
    """BASELINE config 1 (the FP32 golden forward of MiniCPM5-1B-hd96 at (1, 8192)) on the GPU with every
    linear in bf16 (quant "bf16"): the argmax is the golden's top-1, exactly.  The GPU output is
    deterministic (fixed summation orders), so this is a stable check; it separates the kernels from the
    W8A8 numerics, whose quantisation error (mean |dlogit| 0.048) exceeds this golden's top-1 / top-2
    margin (0.029), so the W8A8 test of this model is tie-aware."""
    from minicpm5_mk.synth import random_token_ids

    gold, meta = _golden("1b-hd96")
    fx = np.load(os.path.join(HERE, "golden", "emulate_1b-hd96_bf16_b1_s8192.npz"))
    m = _full_model("1b-hd96", "bf16")
    ids = random_token_ids(1, 8192, seed=meta["id_seed"])
    _, lg = m.forward(ids.reshape(-1).to(_dev()), 1, 8192, logits=True)
    lg = lg.cpu()[0]
    g = torch.from_numpy(gold["logits"][0])
    e = torch.from_numpy(fx["logits"][0])
    err, eerr = (lg - g).abs(), (lg - e).abs()
    print(f"[bf16] 1b-hd96: vs golden max {err.max():.4f} mean {err.mean():.4f}; vs emulator max {eerr.max():.4f}; "
          f"argmax GPU {int(lg.argmax())} emulator {int(e.argmax())} golden {int(g.argmax())}", flush=True)
    assert err.max() <= 0.25 and eerr.max() <= 0.1
    assert int(lg.argmax()) == int(g.argmax())
    m.release_buffers()


def test_batch_invariance_and_graph_replay():
    from minicpm5_mk.config import preset
    from minicpm5_mk.synth import random_hf_state_dict, random_token_ids

    dev = _dev()
    cfg = preset("tiny")
    sd = random_hf_state_dict(cfg)
    m, _ = _build(cfg, "int8d:qkv+gu+o|sq|lastbf16|fqkv|fmlp", sd, 2048, dev)
    ids = random_token_ids(4, 1024, seed=7).to(dev)
    h4, l4 = m.forward(ids.reshape(-1), 4, 1024, logits=True)
    for b in range(4):
        h1, l1 = m.forward(ids[b].reshape(-1), 1, 1024, logits=True)
        assert torch.equal(h1[0], h4[b]) and torch.equal(l1[0], l4[b])
    # graph replays (cached) and eager launches agree bitwise; replay several times with host work between
    outs = [m.forward(ids.reshape(-1), 4, 1024, logits=True)[1] for _ in range(3)]
    m.set_graph_mode(False)
    eager = m.forward(ids.reshape(-1), 4, 1024, logits=True)[1]
    for o in outs:
        assert torch.equal(o, eager)
    m.close()


@pytest.mark.parametrize("B,chunk", [(5, 2), (3, 2), (9, 4)])
def test_chunked_batches_equal_one_launch(B, chunk):
    """A batch run in chunks of sequences (mk_set_max_chunk; by default only past the 4 GiB operand limit)
    gives the same rows and logits bitwise, padding rows zero, in graph and eager mode."""
    from minicpm5_mk.config import preset
    from minicpm5_mk.synth import random_hf_state_dict, random_token_ids

    dev = _dev()
    cfg = preset("tiny")
    sd = random_hf_state_dict(cfg)
    m, _ = _build(cfg, "int8d:qkv+gu+o|sq|lastbf16|fqkv|fmlp", sd, 1024, dev)
    ids = random_token_ids(B, 512, seed=B).to(dev).reshape(-1)
    h_all, l_all = m.forward(ids, B, 512, logits=True)
    ws_all = m.workspace_bytes(B, 512)
    m.set_max_chunk(chunk)
    assert m.workspace_bytes(B, 512) < ws_all
    for graph in (True, False):
        m.set_graph_mode(graph)
        h_c, l_c = m.forward(ids, B, 512, logits=True)
        assert torch.equal(h_c, h_all) and torch.equal(l_c, l_all)
        assert torch.equal(h_c[B:], torch.zeros_like(h_c[B:]))
    t = m.forward_timed(ids, B, 512, logits=True)
    assert t["attn"][1] == (cfg.num_layers - 1) * ((B + chunk - 1) // chunk)
    m.set_max_chunk(0)
    assert m.workspace_bytes(B, 512) == ws_all
    m.close()


def test_forward_timed_matches_forward():
    """mk_forward_timed: same result as the graph-replayed forward, one launch per layer per kernel kind."""
    from minicpm5_mk.config import preset
    from minicpm5_mk.synth import random_hf_state_dict, random_token_ids

    dev = _dev()
    cfg = preset("tiny")
    sd = random_hf_state_dict(cfg)
    m, _ = _build(cfg, "int8d:qkv+gu|sq|lastbf16|fqkv|fmlp", sd, 1024, dev)
    ids = random_token_ids(2, 512, seed=5).to(dev)
    h, lg = m.forward(ids.reshape(-1), 2, 512, logits=True)
    t = m.forward_timed(ids.reshape(-1), 2, 512, logits=True)
    h2, lg2 = m.forward(ids.reshape(-1), 2, 512, logits=True, copy_out=False)   # buffers the timed run wrote
    L = cfg.num_layers - 1
    # the QKV projection's epilogue does the attention prep: no prep launches
    assert t["attn"][1] == L and t["attn_prep"][1] == 0 and t["gemm_qkv"][1] == L and t["gemm_gu"][1] == L
    assert t["embed"][1] == 1 and t["lm_head"][1] >= 1
    assert all(ms >= 0.0 for ms, _ in t.values()) and t["attn"][0] > 0.0
    assert torch.equal(h, h2) and torch.equal(lg, lg2)
    m.set_attn_prep_fused(False)
    assert m.forward_timed(ids.reshape(-1), 2, 512, logits=True)["attn_prep"][1] == L
    m.close()


@pytest.mark.parametrize("name,quant,B,S", [
    ("tiny", "int8d:qkv+gu|sq|lastbf16|fqkv|fmlp", 2, 512), ("tiny-hd96", "int8d:qkv+gu+o|sq|lastbf16", 3, 256),
    ("tiny", "bf16", 2, 384), ("tiny-hd96", "fp8d|sq|lastbf16", 1, 640), ("tiny", "int8|sq|fqkv|fmlp", 2, 256)])
def test_fused_attn_prep_equals_prep_kernel(name, quant, B, S):
    """The QKV projection's routing epilogue (K RoPE'd into krope, V transposed into vt, pack.hip map 2
    column order) gives the same model output, bitwise, as the projection followed by the separate prep
    kernel, for every QKV epilogue (DQ_BF16, DQ2_BF16, BF16, fp8 DQ2_BF16) and both head dims."""
    from minicpm5_mk.config import preset
    from minicpm5_mk.synth import random_hf_state_dict, random_token_ids

    dev = _dev()
    cfg = preset(name)
    sd = random_hf_state_dict(cfg)
    m, _ = _build(cfg, quant, sd, 1024, dev)
    ids = random_token_ids(B, S, seed=B + S).to(dev).reshape(-1)
    h1, l1 = m.forward(ids, B, S, logits=True)
    m.set_attn_prep_fused(False)
    h0, l0 = m.forward(ids, B, S, logits=True)
    assert torch.equal(h1, h0) and torch.equal(l1, l0)
    m.close()


def test_fused_attn_prep_full_size():
    """Fused vs separate attention prep on the full MiniCPM5-1B at (2, 4096) and (1, 8192): bitwise equal."""
    from minicpm5_mk.synth import random_token_ids

    m = _full_model("1b")
    dev = _dev()
    for B, S in ((2, 4096), (1, 8192)):
        ids = random_token_ids(B, S, seed=3).to(dev).reshape(-1)
        print(f"[fused prep] 1b ({B}, {S})", flush=True)
        h1, l1 = m.forward(ids, B, S, logits=True)
        m.set_attn_prep_fused(False)
        h0, l0 = m.forward(ids, B, S, logits=True)
        m.set_attn_prep_fused(True)
        assert torch.equal(h1, h0) and torch.equal(l1, l0)
    m.release_buffers()


@pytest.mark.parametrize("quant", ["int8d:qkv+gu|sq|lastbf16|fqkv|fmlp", "bf16"])
def test_runtime_forward_reference_signature(quant):
    """runtime.forward takes the reference op's 29 arguments in order (model.py:749-751, weight order
    :40-41): ids padded past bs*seq (only the first bs*seq are used, mk_jax.py:660), the prepared
    tensors as prepare_mk_weights returns them ((1,) dummies for an all-bf16 string), and returns the
    (max(8, bs), H) bf16 rows with zero padding rows, bitwise equal to MkModel.forward."""
    from minicpm5_mk import runtime
    from minicpm5_mk.config import preset
    from minicpm5_mk.mk_weights import prepare_mk_weights
    from minicpm5_mk.runtime import WEIGHT_ORDER, MkError, MkModel
    from minicpm5_mk.synth import random_hf_state_dict, random_token_ids

    dev = _dev()
    cfg = preset("tiny")
    sd = random_hf_state_dict(cfg)
    w = prepare_mk_weights(sd, cfg.as_mk_cfg(), quant, 1024, log=lambda *a: None)
    if quant == "bf16":
        assert w["s_qkv"].shape == (1,)
    wd = [w[k].to(dev) for k in WEIGHT_ORDER]
    embed, fnorm = sd["model.embed_tokens.weight"].to(dev), sd["model.norm.weight"].to(dev)
    cos, sin = w["cos"].to(dev), w["sin"].to(dev)
    runtime.clear_cache()
    for bs, seq in ((3, 256), (9, 128)):
        ids = random_token_ids(bs, seq, seed=bs).reshape(-1)
        ids_pad = torch.cat([ids, torch.randint(0, cfg.vocab, (37,), dtype=torch.int32)]).to(dev)
        out = runtime.forward(ids_pad, embed, cos, sin, fnorm, *wd, bs, seq, quant, cfg.n_q, cfg.n_kv, cfg.head_dim,
                              cfg.eps, "auto")
        assert out.shape == (max(8, bs), cfg.hidden) and out.dtype == BF16
        assert torch.equal(out[bs:], torch.zeros_like(out[bs:]))
        m = MkModel(dict(zip(WEIGHT_ORDER, wd)), embed, cos, sin, fnorm, quant, cfg.n_q, cfg.n_kv, cfg.head_dim,
                    cfg.eps)
        ref = m.forward(ids.to(dev), bs, seq)
        m.close()
        assert torch.equal(out, ref)
    assert len(runtime._MODELS) == 1                      # one model per weight set, reused across shapes
    with pytest.raises(MkError):
        runtime.forward(ids_pad, embed, cos, sin, fnorm, *wd, 9, 128, quant, cfg.n_q, cfg.n_kv, cfg.head_dim,
                        cfg.eps, "mystery")
    runtime.clear_cache()


@pytest.mark.gpu
def test_runtime_forward_repacks_after_in_place_update():
    """runtime.forward re-packs a weight set that the caller updated in place (same storage, new
    values): the reference op reads its weight arguments on every call (model.py:749-751), so the next
    call must return what a model built from the updated tensors returns.  The cache holds at most
    MAX_CACHED_MODELS weight sets."""
    from minicpm5_mk import runtime
    from minicpm5_mk.config import preset
    from minicpm5_mk.mk_weights import prepare_mk_weights
    from minicpm5_mk.runtime import WEIGHT_ORDER, MkModel
    from minicpm5_mk.synth import random_hf_state_dict, random_token_ids

    dev = _dev()
    cfg = preset("tiny")
    quant = "int8d:qkv+gu|sq|lastbf16|fqkv|fmlp"
    sd = random_hf_state_dict(cfg)
    w = prepare_mk_weights(sd, cfg.as_mk_cfg(), quant, 1024, log=lambda *a: None)
    wd = [w[k].to(dev) for k in WEIGHT_ORDER]
    embed, fnorm = sd["model.embed_tokens.weight"].to(dev), sd["model.norm.weight"].to(dev)
    cos, sin = w["cos"].to(dev), w["sin"].to(dev)
    bs, seq = 2, 256
    ids = random_token_ids(bs, seq, seed=3).reshape(-1).to(dev)
    args = (bs, seq, quant, cfg.n_q, cfg.n_kv, cfg.head_dim, cfg.eps, "auto")
    runtime.clear_cache()
    out0 = runtime.forward(ids, embed, cos, sin, fnorm, *wd, *args)
    w_o = wd[WEIGHT_ORDER.index("w_o")]
    assert w_o.dtype == BF16
    w_o.mul_(0.5)                                            # in place: same storage, new values
    out1 = runtime.forward(ids, embed, cos, sin, fnorm, *wd, *args)
    assert not torch.equal(out0, out1)
    m = MkModel(dict(zip(WEIGHT_ORDER, wd)), embed, cos, sin, fnorm, quant, cfg.n_q, cfg.n_kv, cfg.head_dim, cfg.eps)
    ref = m.forward(ids, bs, seq)
    m.close()
    assert torch.equal(out1, ref)
    assert len(runtime._MODELS) == 1                        # the stale packing was replaced, not kept
    assert torch.equal(runtime.forward(ids, embed, cos, sin, fnorm, *wd, *args), out1)   # no update: reused
    for i in range(3):                                       # other weight sets: bounded cache
        runtime.forward(ids, embed, cos, sin, fnorm, *[t.clone() for t in wd], *args)
    assert len(runtime._MODELS) == runtime.MAX_CACHED_MODELS
    runtime.clear_cache()


@pytest.mark.gpu
def test_runtime_forward_inference_tensors():
    """vLLM's model runner works under torch.inference_mode, so the op may get inference tensors, which
    have no version counter: runtime.forward takes them, called in inference mode and then outside it
    (the per-shape buffers made in inference mode stay writable), and returns the bits it returns for
    ordinary tensors."""
    from minicpm5_mk import runtime
    from minicpm5_mk.config import preset
    from minicpm5_mk.mk_weights import prepare_mk_weights
    from minicpm5_mk.runtime import WEIGHT_ORDER
    from minicpm5_mk.synth import random_hf_state_dict, random_token_ids

    dev = _dev()
    cfg = preset("tiny")
    quant = "int8d:qkv+gu|sq|lastbf16|fqkv|fmlp"
    sd = random_hf_state_dict(cfg)
    w = prepare_mk_weights(sd, cfg.as_mk_cfg(), quant, 1024, log=lambda *a: None)
    bs, seq = 1, 384
    args = (bs, seq, quant, cfg.n_q, cfg.n_kv, cfg.head_dim, cfg.eps, "auto")
    ids = random_token_ids(bs, seq, seed=5).reshape(-1).to(dev)
    host = [sd["model.embed_tokens.weight"], w["cos"], w["sin"], sd["model.norm.weight"]] + [w[k] for k in WEIGHT_ORDER]
    runtime.clear_cache()
    ref = runtime.forward(ids, *[t.to(dev) for t in host], *args)
    runtime.clear_cache()
    with torch.inference_mode():
        inf = [t.to(dev) for t in host]
        assert all(t.is_inference() for t in inf)
        out = runtime.forward(ids, *inf, *args)
        again = runtime.forward(ids, *inf, *args)
    outside = runtime.forward(ids, *inf, *args)
    assert len(runtime._MODELS) == 1
    assert torch.equal(out, ref) and torch.equal(again, ref) and torch.equal(outside, ref)
    runtime.clear_cache()


@pytest.mark.gpu
def test_per_shape_buffers_are_bounded():
    """MkModel keeps the buffers of at most MAX_SHAPES shapes (least recently used out); a shape whose
    buffers were dropped allocates new ones on its next call and returns the same bits as before."""
    from minicpm5_mk.config import preset
    from minicpm5_mk.engine import MkEngine
    from minicpm5_mk.synth import random_token_ids

    dev = _dev()
    eng = MkEngine(preset("tiny"), quant="auto", max_model_len=2048, device=str(dev), log=lambda *a: None,
                   precompile="")
    m = eng.model
    shapes = [(b, s) for s in (128, 256, 384, 512, 640) for b in (1, 2)]
    assert len(shapes) > m.MAX_SHAPES
    first = {}
    for b, s in shapes:
        ids = random_token_ids(b, s, seed=b * 1000 + s).reshape(-1).to(dev)
        first[(b, s)] = m.forward(ids, b, s, logits=True)
        assert len(m._bufs) <= m.MAX_SHAPES
    assert (1, 128, True) not in m._bufs                 # the oldest shape was dropped
    for b, s in shapes[:3]:                              # dropped shapes run again, bitwise as before
        ids = random_token_ids(b, s, seed=b * 1000 + s).reshape(-1).to(dev)
        h, lg = m.forward(ids, b, s, logits=True)
        assert torch.equal(h, first[(b, s)][0]) and torch.equal(lg, first[(b, s)][1])
    eng.close()


@pytest.mark.gpu
def test_precompile_captures_without_running():
    """MkModel.precompile (MINICPM5_MK_PRECOMPILE, model.py:690-698) captures one hipGraph per shape
    without running it: the output buffers keep their contents, the graph count grows by one per new
    shape, and the first forward of a precompiled shape replays that graph (no new capture) with output
    bitwise equal to a model that was never precompiled."""
    from minicpm5_mk.config import preset
    from minicpm5_mk.engine import MkEngine
    from minicpm5_mk.synth import random_token_ids

    dev = _dev()
    cfg = preset("tiny")
    eng = MkEngine(cfg, quant="auto", max_model_len=1024, device=str(dev), log=lambda *a: None,
                   precompile="2x256, 1x512")
    m = eng.model
    assert m.graph_count() == 2
    b = m._buffers(2, 256, True)
    b["hidden"].fill_(7.0)
    m.precompile([(2, 256)], logits=True)               # cached: no new graph, nothing launched
    torch.cuda.synchronize()
    assert m.graph_count() == 2 and bool((b["hidden"] == 7.0).all())
    ids = random_token_ids(2, 256, seed=5).to(dev)
    lg = eng.logits(ids).clone()
    assert m.graph_count() == 2                          # the forward replayed the precompiled graph
    plain = MkEngine(cfg, quant="auto", max_model_len=1024, device=str(dev), log=lambda *a: None, precompile="")
    assert plain.model.graph_count() == 0
    assert torch.equal(lg, plain.logits(ids))
    eng.close()
    plain.close()
