"""Host weight preparation: HF tensors -> the plugin's stacked, quantized megakernel layout.

The output is the reference's format (plugin/minicpm5_mk/mk_weights.py:126-263, keys of model.py:40-41
plus cos / sin); libmk consumes exactly this layout (include/mk.h, mk_weights) and repacks it on the
GPU.  The values are pinned against the reference's own `_calibrate`, `_quantize_w` and `rope_tables`
(tests/golden/calib_fixture.npz), so every floating-point step below keeps the reference's operation
order; the structure around it is this package's own:

  1. `hf_layers`         HF (out, in) bf16 tensors -> one f32 dict per decoder layer, (in, out)
                         matrices, 1/sqrt(hd) folded into W_q, gammas folded into bf16 linears only.
  2. `calibrate`         a short FP32 forward over seeded random ids recording, per layer, the input
                         of each linear ("taps") -> static scales and per-input-channel amax.
  3. `LinearQuantizer`   per linear: SmoothQuant factors, static-scale recalibration, per-output-channel
                         8-bit weights (`quantize_w`) and the per-input-channel activation factor.
  4. `prepare_mk_weights` stacks layers 0..L-2, keeps the last layer in bf16 with gammas folded, and
                         interleaves gate/up for the fused MLP (`interleave_gu`).

Layout produced (Lm = L - 1 scan layers; D = (n_q + 2 n_kv) hd; 8-bit where the quant string
quantizes the linear, bf16 otherwise):
  w_qkv (Lm, H, D)  [q heads * 1/sqrt(hd) | k heads | v heads]     s_qkv (Lm, D)   a_qkv (Lm, H)
  w_o   (Lm, q_dim, H)                                              s_o   (Lm, H)   a_o   (Lm, q_dim)
  w_gu  (Lm, H, 2I) chunk-interleaved when "fmlp", else (Lm, H, 2, I); s_gu (Lm, 1, 2I) | (Lm, 2, I)
  w_down(Lm, I, H)                                                  s_down(Lm, H)   a_down(Lm, I)
  bf16 linears: s_* / a_* are unread zeros, (1,) for an all-bf16 string and (Lm, 1) (per-layer (1,)
  dummies, stacked) for a bf16 linear of a mixed string, as the reference returns them;
  wl_qkv (H, D), wl_o (q_dim, H), wl_gu (H, 2, I), wl_down (I, H): bf16 last layer, gammas folded;
  cos, sin (max_seq, hd) bf16.
"""
from __future__ import annotations

import math
import os
import time
from dataclasses import dataclass
from typing import Dict

import numpy as np
import torch

from .quant import parse_quant, quant_flags

BF16 = torch.bfloat16
F32 = torch.float32
LINEARS = ("qkv", "o", "gu", "down")
QMAX = {"int8": 127.0, "int8d": 127.0, "fp8": 448.0, "fp8d": 448.0}
STATIC_MARGIN = {"int8": 1.15, "int8d": 1.15, "fp8": 1.35, "fp8d": 1.35}


def rope_tables(max_seq: int, head_dim: int, theta: float):
    """cos / sin (max_seq, head_dim): f32 angles, rotate-half layout [f, f], stored bf16
    (mk_weights.py:20-26)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=F32) / head_dim))
    ang = torch.outer(torch.arange(max_seq, dtype=F32), inv_freq)
    emb = torch.cat([ang, ang], dim=-1)
    return emb.cos().to(BF16), emb.sin().to(BF16)


def mlp_chunk(inter: int) -> int:
    """Column chunk of the interleaved gate/up layout (mk_mlp.py:60-65)."""
    return next((c for c in (1536, 1152, 1024, 768, 512) if inter % c == 0), inter)


def interleave_gu(w_gu: torch.Tensor, s_gu: torch.Tensor, ic: int):
    """(.., H, 2, I) -> (.., H, 2I) as [g_0 | u_0 | g_1 | u_1 | ...] with chunks of ic columns;
    scales (.., 2, I) -> (.., 1, 2I) in the same column order (mk_mlp.py:148-158)."""
    *lead, H, two, inter = w_gu.shape
    if two != 2 or inter % ic:
        raise ValueError(f"interleave_gu: bad shape {tuple(w_gu.shape)} for chunk {ic}")
    n = inter // ic
    w = w_gu.reshape(*lead, H, 2, n, ic).transpose(-3, -2).reshape(*lead, H, 2 * inter)
    s = s_gu.reshape(*lead, 2, n, ic).transpose(-3, -2).reshape(*lead, 1, 2 * inter)
    return w.contiguous(), s.to(F32).contiguous()


# ---------------------------------------------------------------------------------------------- 1. layers
def hf_layer(sd: Dict[str, torch.Tensor], cfg: dict, i: int, fold_qkv_gamma: bool, fold_gu_gamma: bool) -> dict:
    """Layer i as an f32 dict {w_qkv (H, D), w_o (q_dim, H), w_gu (H, 2, I), w_down (I, H), in_norm,
    post_norm}, on the device of its HF tensors.  Gammas are folded into the rows of bf16 linears only:
    a quantized linear keeps its gamma in the activation factor, so outlier channels do not widen the
    weight's row range."""
    sm = 1.0 / math.sqrt(cfg["head_dim"])
    get = lambda n: sd[f"model.layers.{i}.{n}.weight"].to(F32)  # noqa: E731
    g_in, g_post = get("input_layernorm"), get("post_attention_layernorm")
    q, k, v = get("self_attn.q_proj").t() * sm, get("self_attn.k_proj").t(), get("self_attn.v_proj").t()
    gate, up = get("mlp.gate_proj").t(), get("mlp.up_proj").t()
    if fold_qkv_gamma:
        q, k, v = (g_in[:, None] * t for t in (q, k, v))
    if fold_gu_gamma:
        gate, up = g_post[:, None] * gate, g_post[:, None] * up
    return {"w_qkv": torch.cat([q, k, v], dim=1).contiguous(),
            "w_o": get("self_attn.o_proj").t().contiguous(),
            "w_gu": torch.stack([gate, up], dim=1).contiguous(),
            "w_down": get("mlp.down_proj").t().contiguous(),
            "in_norm": g_in, "post_norm": g_post}


def hf_layers(sd: Dict[str, torch.Tensor], cfg: dict, fold_qkv_gamma: bool, fold_gu_gamma: bool) -> list:
    """Every layer (hf_layer) in a list."""
    return [hf_layer(sd, cfg, i, fold_qkv_gamma, fold_gu_gamma) for i in range(cfg["num_layers"])]


# ---------------------------------------------------------------------------------------------- 2. calibration
def _unit_rms(x: torch.Tensor, eps: float) -> torch.Tensor:
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)


def _rope(x: torch.Tensor, c: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return x * c + torch.cat([-x[..., h:], x[..., :h]], dim=-1) * s


def _layer_taps(x, ld, c, s, causal, dims, gamma_qkv: bool, gamma_gu: bool):
    """One f32 decoder layer over x (n, S, H): (x after the layer, {linear: its input})."""
    n, S, nh, kh, hd, eps = dims
    xe = _unit_rms(x, eps)
    if gamma_qkv:
        xe = xe * ld["in_norm"]
    heads = (xe @ ld["w_qkv"]).view(n, S, nh + 2 * kh, hd)
    q = _rope(heads[:, :, :nh], c, s).view(n, S, kh, nh // kh, hd).permute(0, 2, 3, 1, 4)
    k = _rope(heads[:, :, nh:nh + kh], c, s).permute(0, 2, 1, 3).unsqueeze(2)
    v = heads[:, :, nh + kh:].permute(0, 2, 1, 3).unsqueeze(2)
    p = torch.softmax((q @ k.transpose(-1, -2)).masked_fill(~causal, -1e30), -1)
    ao = (p @ v).permute(0, 3, 1, 2, 4).reshape(n, S, nh * hd)
    x = x + ao @ ld["w_o"]
    xe2 = _unit_rms(x, eps)
    if gamma_gu:
        xe2 = xe2 * ld["post_norm"]
    gu = torch.einsum("bsh,hcm->bscm", xe2, ld["w_gu"])
    hid = torch.nn.functional.silu(gu[:, :, 0]) * gu[:, :, 1]
    return x + hid @ ld["w_down"], {"qkv": xe, "o": ao, "gu": xe2, "down": hid}


@torch.no_grad()
def calibrate(layers, embed, cos_f, sin_f, cfg: dict, quant: str, n_seq: int = 4, s_cal: int = 128, seed: int = 42,
              margin=None, margin_down=None, gamma_in_act=None, first_id: int = 1):
    """Activation statistics of a short FP32 CPU forward (the reference's `_calibrate`,
    mk_weights.py:29-110) over numpy RandomState(seed).randint(1000, min(V, 30000), (n_seq, s_cal))
    ids with position 0 = `first_id`.  Returns three per-layer lists:
      scales[l][lin]  = max(amax * margin / q_max, 1e-6), the static activation scale (static int8
                        leaves position 0 out of the amax of qkv / o / gu; down uses margin_down);
      chan[l][lin]    = per-input-channel amax over every position;
      chan_nob[l][lin] = the same without position 0."""
    base = quant
    q_max = QMAX.get(base, 127.0)
    margin = margin if margin is not None else (1.35 if base in ("fp8", "fp8d") else 1.15)
    margin_down = margin_down if margin_down is not None else 1.50
    gam = gamma_in_act if gamma_in_act is not None else {"qkv": base != "bf16", "gu": base != "bf16"}
    ids = np.random.RandomState(seed).randint(1000, min(embed.shape[0], 30000), size=(n_seq, s_cal))
    ids[:, 0] = first_id
    x = embed[torch.from_numpy(ids)].to(F32)
    c, s = cos_f[:s_cal][None, :, None, :], sin_f[:s_cal][None, :, None, :]
    causal = torch.tril(torch.ones((s_cal, s_cal), dtype=torch.bool))
    dims = (n_seq, s_cal, cfg["n_q"], cfg["n_kv"], cfg["head_dim"], cfg["eps"])
    from_pos = 1 if base == "int8" else 0        # static int8 scales skip the position-0 sink
    scales, chan, chan_nob = [], [], []
    for ld in layers:
        x, taps = _layer_taps(x, ld, c, s, causal, dims, gam["qkv"], gam["gu"])
        sc = {}
        for lin, t in taps.items():
            amax = float(t.abs().max()) if lin == "down" else float(t[:, from_pos:].abs().max())
            sc[lin] = max(amax * (margin_down if lin == "down" else margin) / q_max, 1e-6)
        scales.append(sc)
        chan.append({lin: t.abs().amax(dim=(0, 1)) for lin, t in taps.items()})
        chan_nob.append({lin: t[:, 1:].abs().amax(dim=(0, 1)) for lin, t in taps.items()})
    return scales, chan, chan_nob


# ---------------------------------------------------------------------------------------------- 3. quantisation
def quantize_w(w: torch.Tensor, quant: str, sx: float):
    """Per-output-channel 8-bit weights, amax over the input axis 0 (mk_weights.py:113-123):
    returns (codes, scale * sx) with scale = max(amax / q_max, 1e-8); int8 codes are
    clamp(round_half_even(w / scale), +-127), e4m3 codes the RNE cast of clamp(w / scale, +-448)."""
    q_max = QMAX[quant]
    scale = torch.clamp(w.abs().amax(dim=0, keepdim=True) / q_max, min=1e-8)
    r = w / scale
    if quant in ("fp8", "fp8d"):
        codes = torch.clamp(r, -q_max, q_max).to(torch.float8_e4m3fn)
    else:
        codes = torch.clamp(torch.round(r), -q_max, q_max).to(torch.int8)
    return codes, (scale.squeeze(0) * sx).to(F32)


def smooth_from_amax(act_amax: torch.Tensor, w_row_amax: torch.Tensor, alpha: float) -> torch.Tensor:
    """SmoothQuant factors per input channel j: amax_x[j]^alpha / amax_w[j]^(1 - alpha), both
    floored at 1e-5, clamped to [1e-4, 1e4] (mk_weights.py:229-238)."""
    ax = act_amax.to(F32).clamp(min=1e-5)
    aw = w_row_amax.to(F32).clamp(min=1e-5)
    return (ax.pow(alpha) / aw.pow(1.0 - alpha)).clamp(1e-4, 1e4)


def smooth_factors(act_amax: torch.Tensor, w: torch.Tensor, alpha: float) -> torch.Tensor:
    """smooth_from_amax with the weight's per-input-row amax taken from W (in, ...)."""
    return smooth_from_amax(act_amax, w.reshape(w.shape[0], -1).abs().amax(dim=1), alpha)


@dataclass
class LinearQuantizer:
    """Quantises one linear of one scan layer: W (in, ...) -> (codes, s_w, a_x) with
    y = (x * a_x) @ dequant(codes) * s_w reproducing x_eff @ W, where x_eff is x * gamma for qkv / gu.

    A linear is dynamic (per-token activation scale at run time) for the d-bases and for the down
    projection of every base (mk_jax.py:422-423); otherwise its activation scale is the static one
    from calibration, recalibrated on the smoothed activation when SmoothQuant is on.  `plan` makes
    the per-channel decisions from statistics only, so the GPU packer shares it."""
    base: str
    use_sq: bool
    alpha: float
    margin_override: float | None

    def plan(self, lin: str, k_in: int, gamma, static_scale: float, amax_all, amax_nob, w_row_amax):
        """(smooth (in,) f32 or None, sx, a_x (in,) f32) from the calibration statistics and the
        weight's per-input-row amax (w_row_amax: needed only with SmoothQuant)."""
        dynamic = self.base in ("int8d", "fp8d") or lin == "down"
        smooth = None
        if self.use_sq:
            smooth = smooth_from_amax(amax_all, w_row_amax, self.alpha)
            if not dynamic:
                ax = amax_nob.to(F32) if self.base == "int8" else amax_all.to(F32).clamp(min=1e-5)
                mg = self.margin_override if self.margin_override is not None else STATIC_MARGIN[self.base]
                static_scale = max(float((ax / smooth).max()) * mg / QMAX[self.base], 1e-6)
        sx = 1.0 if dynamic else static_scale
        sm = smooth if smooth is not None else torch.ones((k_in,), dtype=F32)
        a_x = ((gamma if gamma is not None else torch.ones((k_in,), dtype=F32)) / (sm * sx)).to(F32)
        return smooth, sx, a_x

    def __call__(self, lin: str, w: torch.Tensor, gamma, static_scale: float, amax_all, amax_nob):
        k_in = w.shape[0]
        aw = w.reshape(k_in, -1).abs().amax(dim=1) if self.use_sq else None
        smooth, sx, a_x = self.plan(lin, k_in, gamma, static_scale, amax_all, amax_nob, aw)
        if smooth is not None:
            w = w * smooth.view(-1, *([1] * (w.dim() - 1)))
        codes, s_w = quantize_w(w, self.base, sx)
        return codes, s_w, a_x


def run_calibration(sd: Dict[str, torch.Tensor], cfg: dict, quant: str, layers) -> dict:
    """The calibration forward with the reference's environment knobs (mk_weights.py:186-200) over
    `layers` (any iterable of hf_layer dicts, consumed once in order): static scales, per-channel amax,
    and the SmoothQuant settings."""
    qm = parse_quant(quant)
    base = quant.split("|")[0].split(":", 1)[0]
    env = os.environ.get
    s_cal, n_cal = int(env("MINICPM5_MK_CAL_SEQ", "128")), int(env("MINICPM5_MK_CAL_NSEQ", "4"))
    m, md = env("MINICPM5_MK_CAL_MARGIN"), env("MINICPM5_MK_CAL_MARGIN_DOWN")
    rc, rs = rope_tables(s_cal, cfg["head_dim"], cfg["rope_theta"])
    scales, chan, chan_nob = calibrate(
        layers, sd["model.embed_tokens.weight"].to("cpu", F32), rc.to(F32), rs.to(F32), cfg, base, n_seq=n_cal,
        s_cal=s_cal, seed=int(env("MINICPM5_MK_CAL_SEED", "42")), margin=float(m) if m else None,
        margin_down=float(md) if md else None, gamma_in_act={"qkv": qm["qkv"] != "bf16", "gu": qm["gu"] != "bf16"},
        first_id=int(env("MINICPM5_MK_CAL_FIRST_ID", "1")))
    return {"scales": scales, "chan": chan, "chan_nob": chan_nob,
            "sq_stats": chan_nob if env("MINICPM5_MK_SQ_STATS", "all") == "nobos" else chan,
            "alpha": float(env("MINICPM5_MK_SQ_ALPHA", "0.5")), "margin": float(m) if m else None,
            "n_seq": n_cal, "s_cal": s_cal}


# ---------------------------------------------------------------------------------------------- 4. assembly
def _last_layer_bf16(ld: dict, qm: dict) -> dict:
    """The last layer runs in bf16 for the last token only (mk_jax.py:492-520): gammas folded."""
    qkv = ld["w_qkv"] if qm["qkv"] == "bf16" else ld["in_norm"][:, None] * ld["w_qkv"]
    gu = ld["w_gu"] if qm["gu"] == "bf16" else ld["post_norm"][:, None, None] * ld["w_gu"]
    return {"wl_qkv": qkv.to(BF16).contiguous(), "wl_o": ld["w_o"].to(BF16).contiguous(),
            "wl_gu": gu.to(BF16).contiguous(), "wl_down": ld["w_down"].to(BF16).contiguous()}


@torch.no_grad()
def prepare_mk_weights(sd: Dict[str, torch.Tensor], cfg: dict, quant: str, max_seq: int, bos_id: int = 0,
                       log=print, device=None) -> Dict[str, torch.Tensor]:
    """sd: HF-named tensors; cfg: the _mk_cfg keys (num_layers, hidden, inter, n_q, n_kv, head_dim, eps,
    rope_theta).  Returns tensors in the megakernel layout (module docstring): on the CPU, or, with a
    CUDA `device`, prepared on that GPU by libmk's packer (minicpm5_mk.gpu_prep; bit-identical).
    Environment knobs of the reference: MINICPM5_MK_CAL_SEQ / _CAL_NSEQ / _CAL_SEED / _CAL_FIRST_ID /
    _CAL_MARGIN / _CAL_MARGIN_DOWN, MINICPM5_MK_SQ_ALPHA, MINICPM5_MK_SQ_STATS (all | nobos)."""
    del bos_id  # signature parity: the calibration's first id is MINICPM5_MK_CAL_FIRST_ID
    if device is not None and torch.device(device).type == "cuda":
        from .gpu_prep import prepare_on_gpu

        return prepare_on_gpu(sd, cfg, quant, max_seq, log=log, device=device)
    t0 = time.perf_counter()
    qm = parse_quant(quant)
    flags = quant_flags(quant)
    base = quant.split("|")[0].split(":", 1)[0]
    layers = hf_layers(sd, cfg, qm["qkv"] == "bf16", qm["gu"] == "bf16")
    out: Dict[str, torch.Tensor] = dict(zip(("cos", "sin"), rope_tables(max_seq, cfg["head_dim"], cfg["rope_theta"])))
    out.update(_last_layer_bf16(layers[-1], qm))
    scan = layers[:-1]
    if base == "bf16":
        for k in ("w_qkv", "w_o", "w_gu", "w_down"):
            out[k] = torch.stack([ld[k] for ld in scan]).to(BF16).contiguous()
        for k in ("s_qkv", "s_o", "s_gu", "s_down", "a_qkv", "a_o", "a_gu", "a_down"):
            out[k] = torch.zeros((1,), dtype=F32)        # unread dummies, as the reference passes them
        log(f"[mk] bf16 weights prepared (L-1={len(scan)} + last) in {time.perf_counter() - t0:.1f}s")
        return out

    cal = run_calibration(sd, cfg, quant, layers)
    scales, chan_nob, sq_stats = cal["scales"], cal["chan_nob"], cal["sq_stats"]
    alpha, m, n_cal, s_cal = cal["alpha"], cal["margin"], cal["n_seq"], cal["s_cal"]
    stacks = {f"{p}_{lin}": [] for p in ("w", "s", "a") for lin in LINEARS}
    dummy = torch.zeros((1,), dtype=F32)
    for li, ld in enumerate(scan):
        for lin in LINEARS:
            w = ld["w_" + lin]
            if qm[lin] == "bf16":
                parts = (w.to(BF16), dummy, dummy)
            else:
                qz = LinearQuantizer(qm[lin], "sq" in flags, alpha, m)
                gamma = ld["in_norm"] if lin == "qkv" else ld["post_norm"] if lin == "gu" else None
                parts = qz(lin, w, gamma, scales[li][lin], sq_stats[li][lin], chan_nob[li][lin])
            for p, t in zip(("w", "s", "a"), parts):
                stacks[f"{p}_{lin}"].append(t)
    out.update({k: torch.stack(v).contiguous() for k, v in stacks.items()})
    if "fmlp" in flags and qm["gu"] in ("int8", "int8d"):
        out["w_gu"], out["s_gu"] = interleave_gu(out["w_gu"], out["s_gu"], mlp_chunk(cfg["inter"]))
    log(f"[mk] {quant} weights prepared (L-1={len(scan)}, calibration {n_cal}x{s_cal}, sq={'sq' in flags}, "
        f"alpha={alpha}) in {time.perf_counter() - t0:.1f}s")
    return out
