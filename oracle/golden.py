"""FP32 CPU golden forward of MiniCPM5 (Llama) -- the oracle's full-precision half.

TEST INFRASTRUCTURE ONLY.  Nothing in the product imports this module; only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may use it, and only as the
checker / the timed CPU baseline.

Restates benchmark/f32_golden.py (the reference's FP32 golden) in torch CPU float32:
  * `rope_tables`  <- f32_golden.py:45-50 (float64 angles, rounded to f32),
  * `rms`          <- f32_golden.py:53-54,
  * `rot_half`     <- f32_golden.py:57-59,
  * `attn_chunk`   <- f32_golden.py:62-75 (GQA q head h*g+j -> kv head h, -inf causal mask,
                      f32 softmax).  Keys past the chunk's last query are skipped: they are masked
                      with -inf in the reference, so they contribute exactly 0 to the softmax,
  * `load_f32`     <- f32_golden.py:121-132 (bf16 weights upcast to f32, (in, out) layout),
  * `forward_one`  <- f32_golden.py:78-102, returning the full last-position logits as well.
"""
from __future__ import annotations

import math

import numpy as np
import torch

F32 = torch.float32


def rope_tables(S: int, hd: int, theta: float):
    inv = 1.0 / (theta ** (np.arange(0, hd, 2, dtype=np.float64) / hd))
    t = np.arange(S, dtype=np.float64)
    f = np.einsum("i,j->ij", t, inv)
    e = np.concatenate([f, f], -1)
    return torch.from_numpy(np.cos(e).astype(np.float32)), torch.from_numpy(np.sin(e).astype(np.float32))


def rms(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps) * w


def rot_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat([-x[..., h:], x[..., :h]], dim=-1)


def attn_chunk(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q0: int) -> torch.Tensor:
    """q: (Cq, nq, hd) for positions q0..q0+Cq-1; k, v: (S, nkv, hd). Returns (Cq, nq*hd)."""
    cq, nq, hd = q.shape
    nkv = k.shape[1]
    g = nq // nkv
    kend = q0 + cq                                   # keys >= kend are masked for every query here
    kk = k[:kend].permute(1, 2, 0)                   # (nkv, hd, kend)
    vv = v[:kend].permute(1, 0, 2)                   # (nkv, kend, hd)
    qg = q.reshape(cq, nkv, g, hd).permute(1, 2, 0, 3).reshape(nkv, g * cq, hd)
    s = torch.bmm(qg, kk).view(nkv, g, cq, kend) / math.sqrt(hd)
    qi = q0 + torch.arange(cq)[:, None]
    kj = torch.arange(kend)[None, :]
    s.masked_fill_(~(kj <= qi)[None, None], float("-inf"))
    p = torch.softmax(s, dim=-1).view(nkv, g * cq, kend)
    o = torch.bmm(p, vv).view(nkv, g, cq, hd).permute(2, 0, 1, 3)
    return o.reshape(cq, nq * hd)


def load_f32(sd: dict, cfg) -> dict:
    """HF-named tensors -> f32 (in, out) weights (f32_golden.py:121-132)."""
    put = lambda t: t.to(F32)  # noqa: E731
    W = {"embed": put(sd["model.embed_tokens.weight"]), "norm": put(sd["model.norm.weight"]),
         "lm_head": put(sd["lm_head.weight"]).t().contiguous() if "lm_head.weight" in sd
         else put(sd["model.embed_tokens.weight"]).t().contiguous(),
         "layers": []}
    for i in range(cfg.num_layers):
        p = f"model.layers.{i}."
        W["layers"].append({
            "in": put(sd[p + "input_layernorm.weight"]), "post": put(sd[p + "post_attention_layernorm.weight"]),
            "q": put(sd[p + "self_attn.q_proj.weight"]).t().contiguous(),
            "k": put(sd[p + "self_attn.k_proj.weight"]).t().contiguous(),
            "v": put(sd[p + "self_attn.v_proj.weight"]).t().contiguous(),
            "o": put(sd[p + "self_attn.o_proj.weight"]).t().contiguous(),
            "gate": put(sd[p + "mlp.gate_proj.weight"]).t().contiguous(),
            "up": put(sd[p + "mlp.up_proj.weight"]).t().contiguous(),
            "down": put(sd[p + "mlp.down_proj.weight"]).t().contiguous(),
        })
    return W


def decoder_layer(x: torch.Tensor, lw: dict, cfg, c: torch.Tensor, s_: torch.Tensor, chunk: int = 1024):
    """One FP32 decoder layer over a full sequence x (S, H) (the body of f32_golden.py:83-97)."""
    S = x.shape[0]
    nq, nkv, hd, eps = cfg.n_q, cfg.n_kv, cfg.head_dim, cfg.eps
    xn = rms(x, lw["in"], eps)
    q = (xn @ lw["q"]).view(S, nq, hd)
    kk = (xn @ lw["k"]).view(S, nkv, hd)
    v = (xn @ lw["v"]).view(S, nkv, hd)
    q = q * c[:, None, :] + rot_half(q) * s_[:, None, :]
    kk = kk * c[:, None, :] + rot_half(kk) * s_[:, None, :]
    a = torch.cat([attn_chunk(q[q0:q0 + chunk], kk, v, q0) for q0 in range(0, S, chunk)], dim=0)
    x = x + a @ lw["o"]
    xn = rms(x, lw["post"], eps)
    gte = xn @ lw["gate"]
    up = xn @ lw["up"]
    return x + (torch.nn.functional.silu(gte) * up) @ lw["down"]


@torch.no_grad()
def forward_one(ids: torch.Tensor, W: dict, cfg, cos: torch.Tensor, sin: torch.Tensor, k: int = 20,
                n_layers: int | None = None):
    """FP32 forward of ONE sequence (f32_golden.py:78-102).

    Returns (last-position logits (V,) f32, top-k ids, top-k logprobs).  `n_layers` truncates the
    layer loop (used only to time a bounded sample of the CPU baseline)."""
    S = ids.shape[0]
    x = W["embed"][ids.long()]
    c, s_ = cos[:S], sin[:S]
    for lw in W["layers"][: (n_layers if n_layers is not None else len(W["layers"]))]:
        x = decoder_layer(x, lw, cfg, c, s_)
    h = rms(x[-1], W["norm"], cfg.eps)
    logits = h @ W["lm_head"]
    lp = torch.log_softmax(logits, dim=-1)
    top = torch.topk(lp, k)
    return logits, top.indices.tolist(), top.values.tolist()
