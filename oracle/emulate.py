"""CPU emulator of the plugin's quantized prefill numerics -- the oracle's per-kernel half.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Each function restates one piece of the reference's device program on the CPU (torch, f32 unless
stated), with the reference's rounding points:
  act_quant        activation quantisation of every mode: dynamic int8d / fp8d (mk_mlp.py:161-168,
                   mk_jax.py:244-250, :257-262, :283-297) and static int8 / fp8 (mk_jax.py:252-256,
                   :265-268, the bf16-rounded x * rstd of :298-299); row_quant is its int8d case
  int_matmul       exact int8 x int8 -> int64 (the MXU / MFMA int32 accumulation is exact)
  fp8_matmul       e4m3 x e4m3 products summed exactly (float64), rounded once to f32
  fused_qkv        mk_mlp.py:161-170
  linear           mk_jax.py:233-269 (bf16, int8d, int8, fp8d, fp8)
  linear_rmsnorm   mk_jax.py:272-299 (bf16, int8d, fp8d; int8 / fp8 through the bf16 x * rstd)
  fused_mlp        mk_mlp.py:68-97 (bf16 and int8 W_down)
  attention        mk_attn.py:557-657 numerics: RoPE'd q * log2(e) (and the softmax scale) rounded
                   to bf16, RoPE'd k rounded to bf16, scores f32, p = exp2(s - m) rounded to bf16 for
                   the PV product, row sum accumulated from that bf16 p, output bf16.  The reference
                   rounds s - m to bf16 before a bf16 exp2 and rounds k's RoPE products to bf16
                   separately; `ref_numerics=True` reproduces those two TPU-specific roundings.
  attention_fp32   the FP32 reference attention of the attention-kernel benchmark (RoPE in f32 on
                   the bf16 inputs, f32 softmax).
  attention_small  the reference's S <= 1024 kernel (mk_jax.py:58-175): bf16 RoPE products, exact
                   row max, f32 exp and sum, P normalised to bf16 before the PV product.
  last_layer_step  mk_jax.py:492-520
  mk_forward       mk_jax.py:527-569, 608-665 (+ the inherited LM head in f32)

Pinning: see tests/test_oracle_*.py (closed forms, brute force, exact-algebra invariants, and the
FP32 golden, which is itself checked against transformers' Llama).
"""
from __future__ import annotations

import torch

BF16 = torch.bfloat16
F32 = torch.float32
LOG2E = 1.4426950408889634


def bf(x: torch.Tensor) -> torch.Tensor:
    """Round to bf16 (RNE) and back to f32."""
    return x.to(BF16).to(F32)


# ------------------------------------------------------------------------------------------ quant
FP8 = torch.float8_e4m3fn


def act_quant(x: torch.Tensor, a: torch.Tensor | None, eps: float, mode: str, norm: bool, recip: bool = False,
              smul: bool = False):
    """x (T, H) -> (q (T, H) int8 or float8_e4m3fn, sx f32 (T,)); rstd = rsqrt(mean(x^2) + eps) with norm.

    dynamic (int8d, fp8d): u = x * a; s = max(amax * (1/qmax), 1e-6) (smul) or max(amax / qmax, 1e-6);
      q = u * (1/s) (recip) or u / s; sx = s * rstd.
    static (int8, fp8): t = bf16(x * rstd) with norm, else x; q = t * a; sx = 1.
    int8: clip(round_half_even(q), +-127); fp8: e4m3(clip(q, +-448)) with round-to-nearest-even."""
    x = x.to(F32)
    fp8 = mode in ("fp8", "fp8d")
    qmax = 448.0 if fp8 else 127.0
    rstd = torch.rsqrt((x * x).mean(-1, keepdim=True) + eps) if norm else torch.ones_like(x[:, :1])
    if mode in ("int8d", "fp8d"):
        u = x * a if a is not None else x
        amax = u.abs().amax(-1, keepdim=True)
        if smul:
            s = torch.clamp(amax * torch.tensor(1.0 / qmax, dtype=F32), min=1e-6)
        else:
            s = torch.clamp(amax / qmax, min=1e-6)
        t = u * (1.0 / s) if recip else u / s
        sx = (s * rstd).squeeze(-1)
    elif mode in ("int8", "fp8"):
        t = bf(x * rstd) if norm else x
        t = t * a if a is not None else t
        sx = torch.ones(x.shape[0], dtype=F32)
    else:
        raise ValueError(f"act_quant: unknown mode {mode!r}")
    if fp8:
        q = torch.clamp(t, -448.0, 448.0).to(FP8)
    else:
        q = torch.clamp(torch.round(t), -127, 127).to(torch.int8)
    return q, sx


def row_quant(x: torch.Tensor, a: torch.Tensor | None, eps: float, norm: bool, recip: bool):
    """Dynamic int8 (act_quant's int8d): the fused prologue (recip: s = amax * (1/127), q = u * (1/s),
    mk_mlp.py:161-168) or the XLA linear (s = amax / 127, q = u / s, mk_jax.py:257-262)."""
    return act_quant(x, a, eps, "int8d", norm, recip=recip, smul=recip)


def fp8_matmul(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """e4m3 (M, K) @ e4m3 (K, N) -> f32.  Every product has <= 8 significant bits within 2^-18 .. 2^18,
    so float64 sums them exactly for K < 2^17; the result is rounded once to f32."""
    return (a.to(torch.float64) @ b.to(torch.float64)).to(F32)


def qmatmul(q: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """The 8-bit GEMM of a quantised linear, as f32: exact int32 for int8, fp8_matmul for e4m3."""
    return fp8_matmul(q, w) if q.dtype == FP8 else int_matmul(q, w).to(F32)


def int_matmul(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Exact int8 (M, K) @ int8 (K, N) -> int64, via f32 GEMMs over K-chunks of 512: every partial sum
    is an integer of magnitude <= 512 * 127 * 127 < 2**24, so each chunk product is exact in f32."""
    M, K = a.shape
    out = torch.zeros((M, b.shape[1]), dtype=torch.float64)
    af, bfl = a.to(F32), b.to(F32)
    for k0 in range(0, K, 512):
        out += (af[:, k0:k0 + 512] @ bfl[k0:k0 + 512]).to(torch.float64)
    return out.to(torch.int64)


def fused_qkv(x: torch.Tensor, w: torch.Tensor, s_w: torch.Tensor, a: torch.Tensor, eps: float) -> torch.Tensor:
    """(T, H) bf16 -> (T, D) bf16 = bf16((acc * (s_u * rstd)) * s_w)."""
    q, sx = row_quant(x.to(F32), a, eps, norm=True, recip=True)
    acc = int_matmul(q, w).to(F32)
    return ((acc * sx[:, None]) * s_w.reshape(1, -1)).to(BF16)


def linear(x: torch.Tensor, w: torch.Tensor, s_w, a_x, quant: str, dynamic_act: bool = False) -> torch.Tensor:
    """mk_jax.py:233-269.  bf16: bf16(x @ w);  int8d: bf16((acc * s_x) * s_w) with s = amax / 127, q = u / s;
    fp8d: bf16(acc * (s_x * s_w)) with s = amax * (1/448), q = u * (1/s);  static int8 / fp8: bf16(acc * s_w)
    of q = x * a_x.  dynamic_act turns the static modes dynamic (the down projection, mk_jax.py:422-423)."""
    if quant == "bf16":
        return (x.to(F32) @ w.to(F32)).to(BF16)
    if quant == "int8d" or (quant == "int8" and dynamic_act):
        q, sx = act_quant(x, a_x, 0.0, "int8d", norm=False)
        return ((qmatmul(q, w) * sx[:, None]) * s_w.reshape(1, -1)).to(BF16)
    if quant == "fp8d" or (quant == "fp8" and dynamic_act):
        q, sx = act_quant(x, a_x, 0.0, "fp8d", norm=False, recip=True, smul=True)
        return (qmatmul(q, w) * (sx[:, None] * s_w.reshape(1, -1))).to(BF16)
    if quant in ("int8", "fp8"):
        q, _ = act_quant(x, a_x, 0.0, quant, norm=False)
        return (qmatmul(q, w) * s_w.reshape(1, -1)).to(BF16)
    raise NotImplementedError(quant)


def linear_rmsnorm(x: torch.Tensor, w: torch.Tensor, s_w, a_x, eps: float, quant: str) -> torch.Tensor:
    """mk_jax.py:272-299.  Dynamic modes: s = amax * (1/qmax), q = u / s, bf16(acc * (s * rstd * s_w));
    bf16 / static modes: the linear of bf16(x * rstd)."""
    xf = x.to(F32)
    if quant == "bf16":
        rstd = torch.rsqrt((xf * xf).mean(-1, keepdim=True) + eps)
        return (bf(xf * rstd) @ w.to(F32)).to(BF16)
    if quant in ("int8d", "fp8d"):
        q, sx = act_quant(xf, a_x, eps, quant, norm=True, recip=False, smul=True)
        return (qmatmul(q, w) * (sx[:, None] * s_w.reshape(1, -1))).to(BF16)
    if quant in ("int8", "fp8"):
        q, _ = act_quant(xf, a_x, eps, quant, norm=True)
        return (qmatmul(q, w) * s_w.reshape(1, -1)).to(BF16)
    raise NotImplementedError(quant)


def silu_f32(g: torch.Tensor) -> torch.Tensor:
    return g / (1.0 + torch.exp(-g))


def fused_mlp(x: torch.Tensor, w_gu_il: torch.Tensor, s_gu_il: torch.Tensor, a_gu: torch.Tensor, w_down,
              s_down, a_down, eps: float, ic: int) -> torch.Tensor:
    """x + down(silu(g) * u) with chunk-interleaved W_gu (H, 2I) and bf16 or int8 W_down (mk_mlp.py:68-97)."""
    xf = x.to(F32)
    q, sx = row_quant(xf, a_gu, eps, norm=True, recip=True)
    inter = w_gu_il.shape[1] // 2
    n = inter // ic
    gu = (int_matmul(q, w_gu_il).to(F32) * sx[:, None]) * s_gu_il.reshape(1, -1)
    gu = gu.view(-1, n, 2, ic)
    h = (silu_f32(gu[:, :, 0]) * gu[:, :, 1]).reshape(-1, inter)
    if w_down.dtype == torch.int8:
        hs = h * a_down.reshape(1, -1)
        hq, s_h = row_quant(hs, None, 0.0, norm=False, recip=True)
        acc = int_matmul(hq, w_down).to(F32) * (s_h[:, None] * s_down.reshape(1, -1))
    else:
        acc = bf(h) @ w_down.to(F32)
    return (xf + acc).to(BF16)


# ------------------------------------------------------------------------------------------ RoPE
def rope_f32(x: torch.Tensor, c: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE in f32; x (..., S, N, hd), c / s (S, hd) f32."""
    h = x.shape[-1] // 2
    rot = torch.cat([-x[..., h:], x[..., :h]], dim=-1)
    return x * c[:, None, :] + rot * s[:, None, :]


# ------------------------------------------------------------------------------------------ attention
def attention_fp32(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, n_q: int, n_kv: int, hd: int,
                   sm_scale: float, chunk: int = 512) -> torch.Tensor:
    """Causal GQA attention in f32: qkv (B, S, D) (bf16 values) -> (B, S, n_q hd) f32."""
    B, S, _ = qkv.shape
    g = n_q // n_kv
    c, s = cos[:S].to(F32), sin[:S].to(F32)
    out = torch.empty((B, S, n_q * hd), dtype=F32)
    for b in range(B):
        x = qkv[b].to(F32).view(S, n_q + 2 * n_kv, hd)
        q = rope_f32(x[:, :n_q], c, s)
        k = rope_f32(x[:, n_q:n_q + n_kv], c, s)
        v = x[:, n_q + n_kv:]
        for q0 in range(0, S, chunk):
            q1 = min(S, q0 + chunk)
            qg = q[q0:q1].view(q1 - q0, n_kv, g, hd).permute(1, 2, 0, 3).reshape(n_kv, g * (q1 - q0), hd)
            sc = (qg @ k[:q1].permute(1, 2, 0)).view(n_kv, g, q1 - q0, q1) * sm_scale
            mask = torch.arange(q1)[None, :] > torch.arange(q0, q1)[:, None]
            sc.masked_fill_(mask, float("-inf"))
            p = torch.softmax(sc, -1).view(n_kv, g * (q1 - q0), q1)
            o = (p @ v[:q1].permute(1, 0, 2)).view(n_kv, g, q1 - q0, hd).permute(2, 0, 1, 3)
            out[b, q0:q1] = o.reshape(q1 - q0, n_q * hd)
    return out


def attention(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, n_q: int, n_kv: int, hd: int,
              sm_scale: float = 1.0, ref_numerics: bool = False, chunk: int = 512) -> torch.Tensor:
    """The prefill attention with the plugin's rounding points (module docstring) -> bf16."""
    B, S, _ = qkv.shape
    g = n_q // n_kv
    cb, sb = cos[:S].to(F32), sin[:S].to(F32)
    out = torch.empty((B, S, n_q * hd), dtype=BF16)
    for b in range(B):
        x = qkv[b].to(F32).view(S, n_q + 2 * n_kv, hd)
        q = bf(rope_f32(x[:, :n_q], cb, sb) * (LOG2E * sm_scale))
        kr = x[:, n_q:n_q + n_kv]
        if ref_numerics:   # mk_attn.py:572-575: kr*c + bf16(k_rot)*s with bf16 products and sum
            h = hd // 2
            rot = torch.cat([-kr[..., h:], kr[..., :h]], dim=-1)
            k = bf(bf(kr * cb[:, None]) + bf(rot * sb[:, None]))
        else:
            k = bf(rope_f32(kr, cb, sb))
        v = x[:, n_q + n_kv:]
        for q0 in range(0, S, chunk):
            q1 = min(S, q0 + chunk)
            qg = q[q0:q1].view(q1 - q0, n_kv, g, hd).permute(1, 2, 0, 3).reshape(n_kv, g * (q1 - q0), hd)
            sc = (qg @ k[:q1].permute(1, 2, 0)).view(n_kv, g, q1 - q0, q1)
            mask = torch.arange(q1)[None, :] > torch.arange(q0, q1)[:, None]
            sc.masked_fill_(mask, float("-inf"))
            m = sc.amax(-1, keepdim=True)
            z = sc - m
            p = bf(torch.exp2(bf(z))) if ref_numerics else bf(torch.exp2(z))
            l = p.sum(-1, keepdim=True)
            o = (p.view(n_kv, g * (q1 - q0), q1) @ v[:q1].permute(1, 0, 2)).view(n_kv, g, q1 - q0, hd)
            o = o / l
            out[b, q0:q1] = o.permute(2, 0, 1, 3).reshape(q1 - q0, n_q * hd).to(BF16)
    return out



def attention_small(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, n_q: int, n_kv: int, hd: int,
                    sm_scale: float = 1.0) -> torch.Tensor:
    """The reference's S <= 1024 attention (`attn_fused_small`, mk_jax.py:58-175) -> bf16.

    Rounding points as that kernel writes them: q (carrying the softmax scale, which the reference
    folds into W_q: bf16(q * sm_scale) here) and k RoPE'd with bf16 products and a bf16 sum
    (mk_jax.py:86-89, :110-114; the rotate-half matmul with the +-1 permutation is exact); scores f32;
    masked keys -1e30 (:102-104, :115); the exact row max over all keys (:116); e = exp(s - max) and
    its sum in f32 (:117-118); P = bf16(e * (1 / sum)) normalised before the PV product (:119-122); PV
    accumulated in f32 and rounded to bf16 (:131-133).  The reference takes 1 / sum with the TPU's
    approximate reciprocal (pltpu.reciprocal(approx=True)); this restatement divides exactly.
    """
    B, S, _ = qkv.shape
    g = n_q // n_kv
    cb, sb = cos[:S].to(F32), sin[:S].to(F32)
    out = torch.empty((B, S, n_q * hd), dtype=BF16)
    h2 = hd // 2

    def rope_bf16(x):   # x (S, N, hd) of bf16 values
        rot = torch.cat([-x[..., h2:], x[..., :h2]], dim=-1)
        return bf(bf(x * cb[:, None]) + bf(rot * sb[:, None]))

    mask = torch.arange(S)[None, :] > torch.arange(S)[:, None]   # (query, key): key after query
    for b in range(B):
        x = qkv[b].to(F32).view(S, n_q + 2 * n_kv, hd)
        q = rope_bf16(bf(x[:, :n_q] * sm_scale))
        k = rope_bf16(x[:, n_q:n_q + n_kv])
        v = x[:, n_q + n_kv:]
        for h in range(n_q):
            kh = h // g
            sc = q[:, h] @ k[:, kh].T                      # (query, key) f32
            sc = sc.masked_fill(mask, -1e30)
            e = torch.exp(sc - sc.amax(-1, keepdim=True))
            p = bf(e * (1.0 / e.sum(-1, keepdim=True)))
            out[b, :, h * hd:(h + 1) * hd] = (p @ v[:, kh]).to(BF16)
    return out

# ------------------------------------------------------------------------------------------ model
def _rms_unit_bf16(x: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.to(F32)
    return bf(xf * torch.rsqrt((xf * xf).mean(-1, keepdim=True) + eps))


def last_layer_step(x: torch.Tensor, w: dict, cos, sin, n_q: int, n_kv: int, hd: int, eps: float) -> torch.Tensor:
    """x (B, S, H) bf16 -> (B, H) bf16: last layer for the last token only, bf16 weights (mk_jax.py:492-520).
    RoPE results are rounded to bf16 (apply_rope_4d returns bf16); softmax f32 (p not rounded)."""
    B, S, H = x.shape
    g = n_q // n_kv
    qd, kvd = n_q * hd, n_kv * hd
    xn = _rms_unit_bf16(x, eps)                                            # (B, S, H)
    wqkv = w["wl_qkv"].to(F32)
    q_last = (xn[:, -1] @ wqkv[:, :qd]).to(BF16).to(F32).view(B, 1, n_q, hd)
    kv = (xn.reshape(B * S, H) @ wqkv[:, qd:]).to(BF16).to(F32).view(B, S, 2 * kvd)
    cb, sb = cos[:S].to(F32), sin[:S].to(F32)
    k = bf(rope_f32(kv[:, :, :kvd].reshape(B, S, n_kv, hd), cb, sb))
    v = kv[:, :, kvd:].reshape(B, S, n_kv, hd)
    q = bf(rope_f32(q_last, cb[-1:], sb[-1:])).view(B, n_kv, g, hd)
    sc = torch.einsum("bngd,bsnd->bngs", q, k)
    p = torch.softmax(sc, -1)
    att = torch.einsum("bngs,bsnd->bngd", p, v).reshape(B, qd).to(BF16).to(F32)
    x_last = bf(x[:, -1].to(F32) + bf(att @ w["wl_o"].to(F32)))
    xn2 = _rms_unit_bf16(x_last, eps)
    gu = bf(xn2 @ w["wl_gu"].to(F32).reshape(H, -1)).view(B, 2, -1)
    hid = bf(bf(silu_f32(gu[:, 0])) * gu[:, 1])
    return bf(x_last + bf(hid @ w["wl_down"].to(F32))).to(BF16)


@torch.no_grad()
def mk_forward(ids: torch.Tensor, w: dict, embed: torch.Tensor, final_norm: torch.Tensor, cfg, quant: str,
               lm_head: torch.Tensor | None = None, attn: str = "v2"):
    """ids (B, S) -> (hidden (B, H) bf16, logits (B, V) f32 or None).  `w` is prepare_mk_weights' dict;
    supports every quant base (bf16, int8d, int8, fp8d, fp8) with the fused (fqkv, fmlp) or XLA algebra.
    attn: "v2" runs the super_gqa_v2 numerics at every S; "auto" follows the reference's default dispatch
    (mk_jax.py:341, 364-365): the S <= 1024 kernel (attention_small) at S <= 1024, super_gqa_v2 above."""
    assert attn in ("v2", "auto"), attn
    from minicpm5_mk.mk_weights import mlp_chunk
    from minicpm5_mk.quant import parse_quant, quant_flags

    qm = parse_quant(quant)
    fl = quant_flags(quant)
    fqkv = "fqkv" in fl and qm["qkv"] == "int8d"
    fmlp = "fmlp" in fl and qm["gu"] in ("int8", "int8d")
    B, S = ids.shape
    H, n_q, n_kv, hd, eps = cfg.hidden, cfg.n_q, cfg.n_kv, cfg.head_dim, cfg.eps
    inter = cfg.inter
    x = embed[ids.long()].to(BF16).reshape(B * S, H)
    cos, sin = w["cos"], w["sin"]
    w = {k: (t.expand(cfg.num_layers - 1, 1) if k[:2] in ("s_", "a_") and t.dim() == 1 else t) for k, t in w.items()}
    for l in range(cfg.num_layers - 1):
        if fqkv:
            qkv = fused_qkv(x, w["w_qkv"][l], w["s_qkv"][l], w["a_qkv"][l], eps)
        else:
            qkv = linear_rmsnorm(x, w["w_qkv"][l], w["s_qkv"][l], w["a_qkv"][l], eps, qm["qkv"])
        if attn == "auto" and S <= 1024:
            att = attention_small(qkv.view(B, S, -1), cos, sin, n_q, n_kv, hd).reshape(B * S, -1)
        else:
            att = attention(qkv.view(B, S, -1), cos, sin, n_q, n_kv, hd).reshape(B * S, -1)
        o = linear(att, w["w_o"][l], w["s_o"][l], w["a_o"][l], qm["o"])
        x = bf(x.to(F32) + o.to(F32)).to(BF16)
        if fmlp:
            d8 = w["w_down"].dtype == torch.int8
            x = fused_mlp(x, w["w_gu"][l], w["s_gu"][l], w["a_gu"][l], w["w_down"][l],
                          w["s_down"][l] if d8 else None, w["a_down"][l] if d8 else None, eps, mlp_chunk(inter))
        else:
            wgu = w["w_gu"][l].reshape(H, 2 * inter)
            sgu = w["s_gu"][l].reshape(-1)
            gu = linear_rmsnorm(x, wgu, sgu, w["a_gu"][l], eps, qm["gu"]).to(F32).view(-1, 2, inter)
            hid = bf(bf(silu_f32(gu[:, 0])) * gu[:, 1]).to(BF16)
            dn = linear(hid, w["w_down"][l], w["s_down"][l], w["a_down"][l], qm["down"],
                        dynamic_act=qm["down"] in ("int8", "fp8"))
            x = bf(x.to(F32) + dn.to(F32)).to(BF16)
    x_last = last_layer_step(x.view(B, S, H), w, cos, sin, n_q, n_kv, hd, eps)
    hidden = (_rms_unit_bf16(x_last, eps) * final_norm.to(F32)).to(BF16)
    logits = hidden.to(F32) @ lm_head.to(F32).t() if lm_head is not None else None
    return hidden, logits
