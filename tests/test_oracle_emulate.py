"""Pins the oracle's quantized-numerics emulator (oracle/emulate.py) without trusting its own formulas.

  * row_quant: brute force per element in pure Python (round-half-even, +-127 clamp, 1e-6 floor,
    all-zero rows, the two reciprocal / division variants of mk_mlp.py:73-76 vs mk_jax.py:259-262);
  * int_matmul: exact int64 products;
  * fused_qkv: dequantised result within the quantisation error bound of the f32 product
    rmsnorm(x) a (W_q s_w), and exact on an exactly representable case;
  * attention: the emulation and the FP32 reference vs a brute-force per-query softmax loop;
  * fused_mlp: the chunk-interleaved W_gu layout gives exactly the same result as the stacked one;
  * last_layer_step equals the last row of the same bf16 layer computed for every token;
  * whole quantized model: within a stated bound of the FP32 golden, argmax identical.
"""
import math

import numpy as np
import pytest
import torch

BF16 = torch.bfloat16


def _py_round_half_even(x: float) -> int:
    return int(round(x))   # Python's round() is round-half-even


@pytest.mark.parametrize("recip", [True, False])
@pytest.mark.parametrize("norm", [True, False])
def test_row_quant_brute_force(recip, norm):
    from oracle import emulate

    g = torch.Generator().manual_seed(1)
    x = torch.randn(5, 24, generator=g) * 2
    x[3] = 0.0                                   # all-zero row -> scale floor 1e-6
    x[4, :4] = torch.tensor([127.0, -63.5, 0.5, 1.5])
    a = torch.rand(24, generator=g) + 0.5
    q, sx = emulate.row_quant(x, a, 1e-6, norm, recip)
    for t in range(5):
        row = [float(np.float32(x[t, j]) * np.float32(a[j])) for j in range(24)]
        amax = np.float32(max(abs(v) for v in row))
        s = max(np.float32(amax * np.float32(1.0 / 127.0)) if recip else np.float32(amax / np.float32(127.0)),
                np.float32(1e-6))
        inv = np.float32(1.0) / np.float32(s)
        for j in range(24):
            v = np.float32(row[j]) * inv if recip else np.float32(row[j]) / np.float32(s)
            exp = max(-127, min(127, _py_round_half_even(float(v))))
            assert int(q[t, j]) == exp
        ms = float(np.mean(np.float32(x[t].numpy()) ** 2))
        rstd = 1.0 / math.sqrt(ms + 1e-6) if norm else 1.0
        assert math.isclose(float(sx[t]), float(s) * rstd, rel_tol=1e-6)
    assert (q[3] == 0).all()


def test_int_matmul_exact():
    from oracle import emulate

    g = torch.Generator().manual_seed(2)
    a = torch.randint(-127, 128, (17, 1800), generator=g, dtype=torch.int8)
    b = torch.randint(-127, 128, (1800, 9), generator=g, dtype=torch.int8)
    a[0] = 127
    b[:, 0] = 127                                # the largest possible dot product: 1800 * 127^2 > 2^24
    ref = a.long() @ b.long()
    assert torch.equal(emulate.int_matmul(a, b), ref)
    assert int(ref[0, 0]) == 1800 * 127 * 127


def test_fused_qkv_error_bound_and_exact_case():
    from minicpm5_mk.mk_weights import quantize_w
    from oracle import emulate

    g = torch.Generator().manual_seed(3)
    x = torch.randn(64, 256, generator=g).to(BF16)
    w = torch.randn(256, 96, generator=g) * 0.02
    a = torch.rand(256, generator=g) + 0.5
    wq, sw = quantize_w(w, "int8d", 1.0)
    out = emulate.fused_qkv(x, wq, sw, a, 1e-6).float()
    xf = x.float()
    xn = xf * torch.rsqrt((xf * xf).mean(-1, keepdim=True) + 1e-6)
    ref = (xn * a) @ w
    # per-element error: activation rounding (s_u / 2 per term) + weight rounding (s_w / 2 per term)
    assert ((out - ref).abs() <= 0.05 * ref.abs().max()).all()
    # exact case: power-of-two scales, integer-valued x * a and weights already on the int8 grid
    x2 = torch.full((2, 8), 2.0)
    a2 = torch.ones(8)
    w2 = torch.arange(-4, 4, dtype=torch.float32).reshape(8, 1).repeat(1, 2) * (127.0 / 4)
    wq2, sw2 = quantize_w(w2, "int8d", 1.0)
    out2 = emulate.fused_qkv(x2.to(BF16), wq2, sw2, a2, 0.0).float()
    ref2 = (x2 / 2.0) @ w2                       # rmsnorm of a constant row is 1
    assert torch.allclose(out2, ref2.to(BF16).float(), atol=0, rtol=0)


def test_attention_vs_brute_force():
    from minicpm5_mk.mk_weights import rope_tables
    from oracle import emulate

    g = torch.Generator().manual_seed(4)
    S, nq, nkv, hd = 40, 16, 2, 32
    qkv = torch.randn(1, S, (nq + 2 * nkv) * hd, generator=g).to(BF16)
    cos, sin = rope_tables(S, hd, 1e4)
    sm = 1.0 / math.sqrt(hd)
    ref = emulate.attention_fp32(qkv, cos, sin, nq, nkv, hd, sm, chunk=16)
    emu = emulate.attention(qkv, cos, sin, nq, nkv, hd, sm, chunk=16).float()
    x = qkv[0].float().view(S, nq + 2 * nkv, hd)
    c, s = cos.float(), sin.float()

    def rope(v, t):
        h = hd // 2
        return v * c[t] + torch.cat([-v[h:], v[:h]]) * s[t]

    for t in (0, 1, 17, S - 1):
        for h in (0, 7, 8, 15):
            kh = h // (nq // nkv)
            qv = rope(x[t, h], t)
            sc = torch.tensor([float(qv @ rope(x[j, nq + kh], j)) * sm for j in range(t + 1)])
            p = torch.softmax(sc, 0)
            o = (p[:, None] * x[:t + 1, nq + nkv + kh]).sum(0)
            assert torch.allclose(ref[0, t, h * hd:(h + 1) * hd], o, atol=1e-5)
            assert torch.allclose(emu[0, t, h * hd:(h + 1) * hd], o, atol=3e-2)


def test_fused_mlp_interleave_invariant():
    from minicpm5_mk.mk_weights import interleave_gu, quantize_w
    from oracle import emulate

    g = torch.Generator().manual_seed(5)
    H, inter, ic = 64, 1536, 512
    x = torch.randn(8, H, generator=g).to(BF16)
    wgu = torch.randn(H, 2, inter, generator=g) * 0.02
    wq, s = quantize_w(wgu, "int8d", 1.0)                      # s: (2, I)
    a = torch.rand(H, generator=g) + 0.5
    wd = (torch.randn(inter, H, generator=g) * 0.02).to(BF16)
    w_il, s_il = interleave_gu(wq, s, ic)
    y_il = emulate.fused_mlp(x, w_il, s_il, a, wd, None, None, 1e-6, ic)
    y_one = emulate.fused_mlp(x, wq.reshape(H, 2 * inter), s.reshape(1, -1), a, wd, None, None, 1e-6, inter)
    assert torch.equal(y_il, y_one)


def test_last_layer_step_is_last_row_of_full_layer():
    from minicpm5_mk.mk_weights import rope_tables
    from oracle import emulate

    g = torch.Generator().manual_seed(6)
    B, S, H, nq, nkv, hd, inter = 2, 48, 64, 16, 2, 16, 96
    x = (torch.randn(B, S, H, generator=g)).to(BF16)
    w = {"wl_qkv": (torch.randn(H, (nq + 2 * nkv) * hd, generator=g) * 0.1).to(BF16),
         "wl_o": (torch.randn(nq * hd, H, generator=g) * 0.1).to(BF16),
         "wl_gu": (torch.randn(H, 2, inter, generator=g) * 0.1).to(BF16),
         "wl_down": (torch.randn(inter, H, generator=g) * 0.1).to(BF16)}
    cos, sin = rope_tables(S, hd, 1e4)
    last = emulate.last_layer_step(x, w, cos, sin, nq, nkv, hd, 1e-6).float()
    # the same layer for every token (f32 softmax over the causal prefix), then the last row
    xf = x.float()
    xn = emulate._rms_unit_bf16(x, 1e-6)
    qkv = (xn @ w["wl_qkv"].float()).to(BF16).float().view(B, S, nq + 2 * nkv, hd)
    for b in range(B):
        q = emulate.bf(emulate.rope_f32(qkv[b, :, :nq], cos.float(), sin.float()))
        k = emulate.bf(emulate.rope_f32(qkv[b, :, nq:nq + nkv], cos.float(), sin.float()))
        v = qkv[b, :, nq + nkv:]
        att = torch.stack([torch.softmax(q[-1, h] @ k[:, h // 8].t(), 0) @ v[:, h // 8] for h in range(nq)])
        att = att.reshape(-1).to(BF16).float()
        xl = emulate.bf(xf[b, -1] + emulate.bf(att @ w["wl_o"].float()))
        xn2 = emulate._rms_unit_bf16(xl[None], 1e-6)[0]
        gu = emulate.bf(xn2 @ w["wl_gu"].float().reshape(H, -1)).view(2, -1)
        hid = emulate.bf(emulate.bf(emulate.silu_f32(gu[0])) * gu[1])
        out = emulate.bf(xl + emulate.bf(hid @ w["wl_down"].float()))
        assert torch.allclose(last[b], out, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("quant", ["auto", "bf16", "int8d:qkv+gu+o+down|sq"])
def test_quantized_model_close_to_fp32_golden(quant):
    """Tiny config, 2 x 512 tokens: the emulated plugin numerics stay within 0.05 of the FP32 logits."""
    import os

    from minicpm5_mk.config import preset
    from minicpm5_mk.mk_weights import prepare_mk_weights
    from minicpm5_mk.quant import resolve_quant_pair
    from minicpm5_mk.synth import random_hf_state_dict, random_token_ids
    from oracle import emulate

    cfg = preset("tiny")
    sd = random_hf_state_dict(cfg)
    q = resolve_quant_pair(quant, cfg.num_layers, 1, cfg.hidden, cfg.inter)[0]
    w = prepare_mk_weights(sd, cfg.as_mk_cfg(), q, 1024, log=lambda *a: None)
    ids = random_token_ids(2, 512)
    _, lg = emulate.mk_forward(ids, w, sd["model.embed_tokens.weight"], sd["model.norm.weight"], cfg, q,
                               sd["lm_head.weight"])
    fx = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_tiny_b2_s512.npz"))
    gold = torch.from_numpy(fx["logits"])
    assert (lg - gold).abs().max() < 0.05
    assert torch.equal(lg.argmax(-1), gold.argmax(-1))
