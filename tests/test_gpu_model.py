"""Whole-model parity of the libmk prefill path (GPU; through MkModel -> the C ABI).

  * tiny config, every supported quant mode: libmk vs the oracle's emulation of the same quantized
    algebra (oracle/emulate.mk_forward) on identical prepared weights and ids.
  * full MiniCPM5 architectures at (1, 8192) with random-init weights (seed 0) and ids (seed 1234),
    auto quant: last-token logits vs the committed FP32 golden (tests/golden/golden_*.npz, written by
    tests/golden/make_golden.py from oracle/golden.py).  The argmax must be identical (tie-aware for the
    one config whose golden top-2 margin is below the W8A8 error); the logits tolerance is stated per
    config below (about 2x the CPU emulator's own W8A8 error vs FP32).
  * batch invariance: a sequence scored inside a batch of 4 equals the same sequence alone, bitwise.
  * hipGraph replay equals eager launches, bitwise.
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


# (preset, logits max-abs tolerance vs FP32, mean-abs tolerance): 2x the error of the CPU emulation of
# the same W8A8 numerics (oracle/emulate.mk_forward) vs the FP32 golden at (1, 8192):
#   1b       max 0.216  mean 0.0359  mean|dlogprob| top-20 0.050
#   1b-hd96  max 0.262  mean 0.0467                        0.046
#   2b       max 0.519  mean 0.0923                        0.092   (int8 O projection too)
# strict: the argmax must equal the golden's.  1b-hd96's golden top-1 / top-2 margin (0.029) is below the
# W8A8 path's mean logit error, so there the top-1 is judged tie-aware like the reference gate
# (benchmark/gate.py:47-56): the chosen token must be within 0.1 nats of the golden top-1.
FULL = [("1b", 0.45, 0.075, True), ("1b-hd96", 0.55, 0.095, False), ("2b", 1.05, 0.19, True)]


@pytest.mark.parametrize("name,tol_max,tol_mean,strict", FULL)
def test_full_model_vs_fp32_golden(name, tol_max, tol_mean, strict):
    from minicpm5_mk.config import preset
    from minicpm5_mk.quant import resolve_quant_pair
    from minicpm5_mk.synth import random_hf_state_dict, random_token_ids

    path = os.path.join(HERE, "golden", f"golden_{name}_b1_s8192.npz")
    gold = np.load(path)
    meta = json.loads(str(gold["meta"]))
    dev = _dev()
    cfg = preset(name)
    print(f"[full] {name} weights", flush=True)
    sd = random_hf_state_dict(cfg, seed=meta["weight_seed"])
    quant = resolve_quant_pair("auto", cfg.num_layers, 1, cfg.hidden, cfg.inter)[0]
    m, _ = _build(cfg, quant, sd, 8256, dev)
    del sd
    ids = random_token_ids(1, 8192, seed=meta["id_seed"])
    print(f"[full] {name} forward quant={quant}", flush=True)
    _, lg = m.forward(ids.reshape(-1).to(dev), 1, 8192, logits=True)
    lg = lg.cpu()[0]
    g = torch.from_numpy(gold["logits"][0])
    err = (lg - g).abs()
    srt = torch.sort(g, descending=True).values
    lp, lpg = torch.log_softmax(lg, -1), torch.log_softmax(g, -1)
    top = torch.topk(lpg, 20).indices
    dlp = (lp[top] - lpg[top]).abs().mean()
    print(f"[full] {name}: logits max {err.max():.4f} mean {err.mean():.4f} rel {err.max() / g.abs().max():.4f}; "
          f"argmax {int(lg.argmax())} vs {int(g.argmax())} (golden margin {float(srt[0] - srt[1]):.4f}); "
          f"mean |dlogprob| top20 {float(dlp):.4f}", flush=True)
    if strict:
        assert int(lg.argmax()) == int(g.argmax())
    else:
        assert float(lpg.max() - lpg[int(lg.argmax())]) <= 0.1
    assert err.max() <= tol_max and err.mean() <= tol_mean
    assert float(dlp) <= 0.15            # the reference gate's FAIL boundary (benchmark/gate.py:115)
    m.close()


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
    assert t["attn"][1] == L and t["attn_prep"][1] == L and t["gemm_qkv"][1] == L and t["gemm_gu"][1] == L
    assert t["embed"][1] == 1 and t["lm_head"][1] >= 1
    assert all(ms >= 0.0 for ms, _ in t.values()) and t["attn"][0] > 0.0
    assert torch.equal(h, h2) and torch.equal(lg, lg2)
    m.close()
