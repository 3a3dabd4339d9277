"""Host weight preparation: HF tensors -> the plugin's stacked, quantized megakernel layout.

Restates plugin/minicpm5_mk/mk_weights.py (prepare_mk_weights :126-263, _calibrate :29-110,
_quantize_w :113-123, rope_tables :20-26) and mk_mlp.py (interleave_gu :148-158, mlp_chunk :60-65),
in torch CPU float32.  The output dict is the reference's (keys of model.py:40-41 plus cos / sin);
libmk consumes exactly this layout (include/mk.h, mk_weights) and repacks it on the GPU.

Layout produced (Lm = L - 1 scan layers; D = (n_q + 2 n_kv) hd; "int8" where the quant string
quantizes the linear, bf16 otherwise):
  w_qkv (Lm, H, D)  [q heads * 1/sqrt(hd) | k heads | v heads]     s_qkv (Lm, D)   a_qkv (Lm, H)
  w_o   (Lm, q_dim, H)                                              s_o   (Lm, H)   a_o   (Lm, q_dim)
  w_gu  (Lm, H, 2I) chunk-interleaved when "fmlp", else (Lm, H, 2, I); s_gu (Lm, 1, 2I) | (Lm, 2, I)
  w_down(Lm, I, H)                                                  s_down(Lm, H)   a_down(Lm, I)
  bf16 linears: s_* / a_* are (Lm, 1) zeros (the reference's per-layer (1,) dummies, stacked);
  wl_qkv (H, D), wl_o (q_dim, H), wl_gu (H, 2, I), wl_down (I, H): bf16 last layer, gammas folded;
  cos, sin (max_seq, hd) bf16.
"""
from __future__ import annotations

import math
import os
import time
from typing import Dict

import numpy as np
import torch

from .quant import parse_quant, quant_flags

BF16 = torch.bfloat16
F32 = torch.float32


def rope_tables(max_seq: int, head_dim: int, theta: float):
    """cos / sin (max_seq, head_dim): f32 angles, rotate-half layout [f, f], stored bf16."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=F32) / head_dim))
    ang = torch.outer(torch.arange(max_seq, dtype=F32), inv_freq)
    emb = torch.cat([ang, ang], dim=-1)
    return emb.cos().to(BF16), emb.sin().to(BF16)


def mlp_chunk(inter: int) -> int:
    """Column chunk of the interleaved gate/up layout: first of 1536, 1152, 1024, 768, 512 dividing I."""
    return next((c for c in (1536, 1152, 1024, 768, 512) if inter % c == 0), inter)


def interleave_gu(w_gu: torch.Tensor, s_gu: torch.Tensor, ic: int):
    """(.., H, 2, I) -> (.., H, 2I) as [g_0 | u_0 | g_1 | u_1 | ...] with chunks of ic columns;
    scales (.., 2, I) -> (.., 1, 2I) in the same column order."""
    *lead, H, two, inter = w_gu.shape
    if two != 2 or inter % ic:
        raise ValueError(f"interleave_gu: bad shape {tuple(w_gu.shape)} for chunk {ic}")
    n = inter // ic
    w = w_gu.reshape(*lead, H, 2, n, ic).transpose(-3, -2).reshape(*lead, H, 2 * inter)
    s = s_gu.reshape(*lead, 2, n, ic).transpose(-3, -2).reshape(*lead, 1, 2 * inter)
    return w.contiguous(), s.to(F32).contiguous()


def _rms_unit(x: torch.Tensor, eps: float) -> torch.Tensor:
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)


def _rotate(x: torch.Tensor, c: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return x * c + torch.cat([-x[..., h:], x[..., :h]], dim=-1) * s


@torch.no_grad()
def calibrate(layers, embed, cos_f, sin_f, cfg: dict, quant: str, n_seq: int = 4, s_cal: int = 128, seed: int = 42,
              margin=None, margin_down=None, gamma_in_act=None, first_id: int = 1):
    """Static activation statistics from a short FP32 CPU forward over random-id sequences.

    Token ids: numpy RandomState(seed).randint(1000, min(V, 30000), (n_seq, s_cal)), position 0 set to
    `first_id` (MINICPM5_MK_CAL_FIRST_ID, default 1).  Returns per layer (a) the static scales
    max(amax * margin / q_max, 1e-6) of each linear's input, (b) the per-input-channel amax over all
    positions, (c) the same excluding position 0 (_calibrate, mk_weights.py:29-110)."""
    is_fp8 = quant in ("fp8", "fp8d")
    q_max = 448.0 if is_fp8 else 127.0
    margin = margin if margin is not None else (1.35 if is_fp8 else 1.15)
    margin_down = margin_down if margin_down is not None else 1.50
    if gamma_in_act is None:
        gamma_in_act = {"qkv": quant != "bf16", "gu": quant != "bf16"}
    nh, kh, hd, eps = cfg["n_q"], cfg["n_kv"], cfg["head_dim"], cfg["eps"]
    g = nh // kh
    ids = np.random.RandomState(seed).randint(1000, min(embed.shape[0], 30000), size=(n_seq, s_cal))
    ids[:, 0] = first_id
    x = embed[torch.from_numpy(ids)].to(F32)
    c = cos_f[:s_cal][None, :, None, :]
    s = sin_f[:s_cal][None, :, None, :]
    causal = torch.tril(torch.ones((s_cal, s_cal), dtype=torch.bool))
    tail = slice(1, None)

    def amax_all(t, static_skip_first):
        return float((t[:, tail] if static_skip_first else t).abs().max())

    scales, chan, chan_nob = [], [], []
    skip = quant == "int8"        # static int8 excludes the position-0 sink from its static scale
    for ld in layers:
        xe = _rms_unit(x, eps)
        if gamma_in_act["qkv"]:
            xe = xe * ld["in_norm"]
        qkv = (xe @ ld["w_qkv"]).view(n_seq, s_cal, nh + 2 * kh, hd)
        q = _rotate(qkv[:, :, :nh], c, s)
        k = _rotate(qkv[:, :, nh:nh + kh], c, s)
        v = qkv[:, :, nh + kh:]
        qg = q.view(n_seq, s_cal, kh, g, hd).permute(0, 2, 3, 1, 4)          # (n, kh, g, S, hd)
        kg = k.permute(0, 2, 1, 3).unsqueeze(2)                                # (n, kh, 1, S, hd)
        vg = v.permute(0, 2, 1, 3).unsqueeze(2)
        sc = (qg @ kg.transpose(-1, -2)).masked_fill(~causal, -1e30)
        ao = (torch.softmax(sc, -1) @ vg).permute(0, 3, 1, 2, 4).reshape(n_seq, s_cal, nh * hd)
        x = x + ao @ ld["w_o"]
        xe2 = _rms_unit(x, eps)
        if gamma_in_act["gu"]:
            xe2 = xe2 * ld["post_norm"]
        gu = torch.einsum("bsh,hcm->bscm", xe2, ld["w_gu"])
        hid = torch.nn.functional.silu(gu[:, :, 0]) * gu[:, :, 1]
        x = x + hid @ ld["w_down"]
        scales.append({
            "qkv": max(amax_all(xe, skip) * margin / q_max, 1e-6),
            "o": max(amax_all(ao, skip) * margin / q_max, 1e-6),
            "gu": max(amax_all(xe2, skip) * margin / q_max, 1e-6),
            "down": max(float(hid.abs().max()) * margin_down / q_max, 1e-6),
        })
        acts = {"qkv": xe, "o": ao, "gu": xe2, "down": hid}
        chan.append({k: t.abs().amax(dim=(0, 1)) for k, t in acts.items()})
        chan_nob.append({k: t[:, 1:].abs().amax(dim=(0, 1)) for k, t in acts.items()})
    return scales, chan, chan_nob


def quantize_w(w: torch.Tensor, quant: str, sx: float):
    """Per-output-channel 8-bit weights (amax over the input axis 0): returns (wq, scale * sx)."""
    is_fp8 = quant in ("fp8", "fp8d")
    q_max = 448.0 if is_fp8 else 127.0
    scale = torch.clamp(w.abs().amax(dim=0, keepdim=True) / q_max, min=1e-8)
    if is_fp8:
        wq = torch.clamp(w / scale, -q_max, q_max).to(torch.float8_e4m3fn)
    else:
        wq = torch.clamp(torch.round(w / scale), -q_max, q_max).to(torch.int8)
    return wq, (scale.squeeze(0) * sx).to(F32)


@torch.no_grad()
def prepare_mk_weights(sd: Dict[str, torch.Tensor], cfg: dict, quant: str, max_seq: int, bos_id: int = 0,
                       log=print) -> Dict[str, torch.Tensor]:
    """sd: HF-named CPU tensors; cfg: the _mk_cfg keys (num_layers, hidden, inter, n_q, n_kv, head_dim,
    eps, rope_theta).  Returns CPU tensors in the megakernel layout (module docstring)."""
    del bos_id  # kept for signature parity; calibration uses MINICPM5_MK_CAL_FIRST_ID
    t0 = time.perf_counter()
    L, hd = cfg["num_layers"], cfg["head_dim"]
    qm = parse_quant(quant)
    flags = quant_flags(quant)
    base_q = quant.split("|")[0].split(":", 1)[0]
    sm = 1.0 / math.sqrt(hd)
    layers = []
    for i in range(L):
        p = f"model.layers.{i}."
        f = lambda n: sd[p + n].to(F32)  # noqa: E731
        in_norm, post_norm = f("input_layernorm.weight"), f("post_attention_layernorm.weight")
        wq = f("self_attn.q_proj.weight").t() * sm
        wk, wv = f("self_attn.k_proj.weight").t(), f("self_attn.v_proj.weight").t()
        wg, wu = f("mlp.gate_proj.weight").t(), f("mlp.up_proj.weight").t()
        if qm["qkv"] == "bf16":        # exact algebra: gamma folded into the rows of bf16 linears only
            wq, wk, wv = in_norm[:, None] * wq, in_norm[:, None] * wk, in_norm[:, None] * wv
        if qm["gu"] == "bf16":
            wg, wu = post_norm[:, None] * wg, post_norm[:, None] * wu
        layers.append({
            "w_qkv": torch.cat([wq, wk, wv], dim=1).contiguous(),
            "w_o": f("self_attn.o_proj.weight").t().contiguous(),
            "w_gu": torch.stack([wg, wu], dim=1).contiguous(),
            "w_down": f("mlp.down_proj.weight").t().contiguous(),
            "in_norm": in_norm, "post_norm": post_norm,
        })
    cos, sin = rope_tables(max_seq, hd, cfg["rope_theta"])
    out: Dict[str, torch.Tensor] = {"cos": cos, "sin": sin}
    last = layers[-1]
    wl_qkv = last["w_qkv"] if qm["qkv"] == "bf16" else last["in_norm"][:, None] * last["w_qkv"]
    wl_gu = last["w_gu"] if qm["gu"] == "bf16" else last["post_norm"][:, None, None] * last["w_gu"]
    out.update({"wl_qkv": wl_qkv.to(BF16).contiguous(), "wl_o": last["w_o"].to(BF16).contiguous(),
                "wl_gu": wl_gu.to(BF16).contiguous(), "wl_down": last["w_down"].to(BF16).contiguous()})
    scan = layers[:-1]
    if base_q == "bf16":
        for k in ("w_qkv", "w_o", "w_gu", "w_down"):
            out[k] = torch.stack([ld[k] for ld in scan]).to(BF16).contiguous()
        for k in ("s_qkv", "s_o", "s_gu", "s_down", "a_qkv", "a_o", "a_gu", "a_down"):
            out[k] = torch.zeros((len(scan), 1), dtype=F32)
        log(f"[mk] bf16 weights prepared (L-1={len(scan)} + last) in {time.perf_counter() - t0:.1f}s")
        return out

    env = os.environ.get
    s_cal, n_cal = int(env("MINICPM5_MK_CAL_SEQ", "128")), int(env("MINICPM5_MK_CAL_NSEQ", "4"))
    m, md = env("MINICPM5_MK_CAL_MARGIN"), env("MINICPM5_MK_CAL_MARGIN_DOWN")
    rc, rs = rope_tables(s_cal, hd, cfg["rope_theta"])
    embed = sd["model.embed_tokens.weight"].to(F32)
    scales, chan, chan_nob = calibrate(
        layers, embed, rc.to(F32), rs.to(F32), cfg, base_q, n_seq=n_cal, s_cal=s_cal,
        seed=int(env("MINICPM5_MK_CAL_SEED", "42")), margin=float(m) if m else None,
        margin_down=float(md) if md else None,
        gamma_in_act={"qkv": qm["qkv"] != "bf16", "gu": qm["gu"] != "bf16"},
        first_id=int(env("MINICPM5_MK_CAL_FIRST_ID", "1")))
    use_sq = "sq" in flags
    alpha = float(env("MINICPM5_MK_SQ_ALPHA", "0.5"))
    stats = chan_nob if env("MINICPM5_MK_SQ_STATS", "all") == "nobos" else chan
    margins = {"fp8": 1.35, "fp8d": 1.35, "int8": 1.15, "int8d": 1.15}
    q_maxes = {"fp8": 448.0, "fp8d": 448.0, "int8": 127.0, "int8d": 127.0}
    acc = {k: [] for k in ("w_qkv", "w_o", "w_gu", "w_down", "s_qkv", "s_o", "s_gu", "s_down",
                           "a_qkv", "a_o", "a_gu", "a_down")}
    for li, (ld, sc) in enumerate(zip(scan, scales[:-1])):
        for name in ("qkv", "o", "gu", "down"):
            w = ld["w_" + name]
            k_in = w.shape[0]
            lq = qm[name]
            if lq == "bf16":
                acc["w_" + name].append(w.to(BF16))
                acc["s_" + name].append(torch.zeros((1,), dtype=F32))
                acc["a_" + name].append(torch.zeros((1,), dtype=F32))
                continue
            dynamic = lq in ("int8d", "fp8d") or (lq in ("int8", "fp8") and name == "down")
            gam = ld["in_norm"] if name == "qkv" else ld["post_norm"] if name == "gu" else None
            smooth = torch.ones((k_in,), dtype=F32)
            w_eff = w
            if use_sq:
                # SmoothQuant: X diag(1/s), diag(s) W with s_j = amax_x_j^alpha / amax_w_j^(1-alpha)
                ax = stats[li][name].to(F32).clamp(min=1e-5)
                aw = w.reshape(k_in, -1).abs().amax(dim=1).clamp(min=1e-5)
                smooth = (ax.pow(alpha) / aw.pow(1.0 - alpha)).clamp(1e-4, 1e4)
                w_eff = w * smooth.view(-1, *([1] * (w.dim() - 1)))
                if not dynamic:   # static scale recalibrated on the smoothed activation
                    mg = float(env("MINICPM5_MK_CAL_MARGIN") or margins.get(lq, 1.15))
                    ax_s = chan_nob[li][name].to(F32) if lq == "int8" else ax
                    sc = dict(sc)
                    sc[name] = max(float((ax_s / smooth).max()) * mg / q_maxes[lq], 1e-6)
            sx = 1.0 if dynamic else sc[name]
            wq, sw = quantize_w(w_eff, lq, sx)
            acc["w_" + name].append(wq)
            acc["s_" + name].append(sw)
            ones = torch.ones((k_in,), dtype=F32)
            acc["a_" + name].append(((gam if gam is not None else ones) / (smooth * sx)).to(F32))
    for k, v in acc.items():
        out[k] = torch.stack(v).contiguous()
    if "fmlp" in flags and qm["gu"] in ("int8", "int8d"):
        out["w_gu"], out["s_gu"] = interleave_gu(out["w_gu"], out["s_gu"], mlp_chunk(cfg["inter"]))
    log(f"[mk] {quant} weights prepared (L-1={len(scan)}, calibration {n_cal}x{s_cal}, sq={use_sq}, "
        f"alpha={alpha}) in {time.perf_counter() - t0:.1f}s")
    return out
