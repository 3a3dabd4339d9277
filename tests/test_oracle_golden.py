"""Pins the FP32 golden (oracle/golden.py, restating benchmark/f32_golden.py).

  * vs transformers' LlamaForCausalLM (the architecture the MiniCPM5 checkpoints declare,
    results/v6e_minicpm5_1b.json:80-82) on identical weights, across the 1024-query chunk boundary,
    for head_dim 64 and 96;
  * RoPE tables vs the closed form cos / sin(t * theta^(-2i/hd)) and vs transformers' rotary embedding;
  * the chunked causal GQA attention vs a brute-force per-query / per-head softmax loop;
  * the committed tiny golden fixture is reproduced bit-for-bit (determinism of synth + oracle).
"""
import math
import os

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def _llama(cfg, sd):
    from transformers import LlamaConfig, LlamaForCausalLM

    hc = LlamaConfig(vocab_size=cfg.vocab, hidden_size=cfg.hidden, intermediate_size=cfg.inter,
                     num_hidden_layers=cfg.num_layers, num_attention_heads=cfg.n_q, num_key_value_heads=cfg.n_kv,
                     head_dim=cfg.head_dim, rms_norm_eps=cfg.eps, rope_theta=cfg.rope_theta,
                     tie_word_embeddings=False, attention_bias=False, mlp_bias=False, max_position_embeddings=4096)
    m = LlamaForCausalLM(hc).float().eval()
    missing, unexpected = m.load_state_dict({k: v.float() for k, v in sd.items()}, strict=False)
    assert not missing and not unexpected
    return m


@pytest.mark.parametrize("name", ["tiny", "tiny-hd96"])
def test_golden_matches_transformers_llama(name):
    from minicpm5_mk.config import preset
    from minicpm5_mk.synth import random_hf_state_dict, random_token_ids
    from oracle import golden

    cfg = preset(name)
    sd = random_hf_state_dict(cfg)
    ids = random_token_ids(1, 1100)
    with torch.no_grad():
        ref = _llama(cfg, sd)(input_ids=ids.long()).logits[0, -1]
    W = golden.load_f32(sd, cfg)
    cos, sin = golden.rope_tables(1100, cfg.head_dim, cfg.rope_theta)
    lg, tids, tlps = golden.forward_one(ids[0], W, cfg, cos, sin)
    assert (lg - ref).abs().max() < 2e-5
    assert tids[0] == int(ref.argmax())
    assert abs(tlps[0] - float(torch.log_softmax(ref, -1).max())) < 1e-5


def test_rope_tables_closed_form_and_transformers():
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding

    from oracle import golden

    S, hd, theta = 777, 96, 5e6
    cos, sin = golden.rope_tables(S, hd, theta)
    t, i = 321, 17
    ang = t * theta ** (-2 * (i % (hd // 2)) / hd)
    assert math.isclose(float(cos[t, i]), math.cos(ang), abs_tol=1e-6)
    assert math.isclose(float(sin[t, i + hd // 2]), math.sin(ang), abs_tol=1e-6)
    hc = LlamaConfig(hidden_size=hd * 4, num_attention_heads=4, head_dim=hd, rope_theta=theta,
                     max_position_embeddings=S)
    rot = LlamaRotaryEmbedding(hc)
    c2, s2 = rot(torch.zeros(1, S, hd), torch.arange(S)[None])
    assert (c2[0] - cos).abs().max() < 2e-3 and (s2[0] - sin).abs().max() < 2e-3   # f32 vs f64 angles at t ~ 800


def test_attn_chunk_brute_force():
    from oracle import golden

    g = torch.Generator().manual_seed(0)
    S, nq, nkv, hd = 23, 4, 2, 8
    q, k, v = (torch.randn(S, n, hd, generator=g) for n in (nq, nkv, nkv))
    got = torch.cat([golden.attn_chunk(q[q0:q0 + 7], k, v, q0) for q0 in range(0, S, 7)], 0)
    for t in range(S):
        for h in range(nq):
            kh = h // (nq // nkv)
            sc = [float(q[t, h] @ k[j, kh]) / math.sqrt(hd) for j in range(t + 1)]
            mx = max(sc)
            w = [math.exp(x - mx) for x in sc]
            o = sum(wj * v[j, kh] for j, wj in enumerate(w)) / sum(w)
            assert torch.allclose(got[t, h * hd:(h + 1) * hd], o, atol=1e-5)


def test_tiny_golden_fixture_reproduces():
    import json

    from minicpm5_mk.config import preset
    from minicpm5_mk.synth import random_hf_state_dict, random_token_ids
    from oracle import golden

    fx = np.load(os.path.join(HERE, "golden", "golden_tiny_b2_s512.npz"))
    meta = json.loads(str(fx["meta"]))
    cfg = preset(meta["preset"])
    W = golden.load_f32(random_hf_state_dict(cfg, seed=meta["weight_seed"]), cfg)
    ids = random_token_ids(meta["batch"], meta["seq"], seed=meta["id_seed"])
    cos, sin = golden.rope_tables(meta["seq"], cfg.head_dim, cfg.rope_theta)
    for b in range(meta["batch"]):
        lg, _, _ = golden.forward_one(ids[b], W, cfg, cos, sin)
        assert np.abs(lg.numpy() - fx["logits"][b]).max() < 1e-5


def test_full_size_fixtures_are_consistent():
    """The committed full-size golden fixtures: right shapes, finite, logprob top-20 consistent."""
    import json

    for name, hd in (("1b", 128), ("1b-hd96", 96), ("2b", 128)):
        fx = np.load(os.path.join(HERE, "golden", f"golden_{name}_b1_s8192.npz"))
        meta = json.loads(str(fx["meta"]))
        assert meta["config"]["head_dim"] == hd and meta["seq"] == 8192
        lg = torch.from_numpy(fx["logits"][0])
        assert lg.shape == (130560,) and torch.isfinite(lg).all()
        lp = torch.log_softmax(lg, -1)
        top = torch.topk(lp, 20)
        assert top.indices.tolist() == fx["top_ids"][0].tolist()
        assert np.allclose(top.values.numpy(), fx["top_logprobs"][0], atol=1e-5)
