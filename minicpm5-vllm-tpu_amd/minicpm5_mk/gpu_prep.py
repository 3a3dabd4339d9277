"""Weight preparation on the GPU: prepare_mk_weights' output, bit-identical, built by libmk's packer.

The CPU restatement (mk_weights.prepare_mk_weights) materialises every layer in f32 on the host and
quantises it there: ~2.7 G f32 values for MiniCPM5-2B, most of the preparation time.  Here:

  * the calibration forward (4 x 128 tokens, mk_weights.py:29-110) stays on the CPU -- its f32
    summation order is what the reference fixes -- but streams the layers one at a time
    (hf_layer), so the host holds one layer in f32 instead of the model;
  * everything per parameter runs on the GPU on the HF bf16 tensors: SmoothQuant's per-row weight
    amax (mk_weight_row_amax), the smoothing multiply, per-output-channel scales and the
    divide-round-clamp to int8 / e4m3 with the transpose into the reference's (in, out) layout
    (mk_weight_quantize), the bf16 linears and the last layer (torch element-wise ops, the same single
    IEEE roundings as on the CPU), and the gate/up interleave;
  * the per-channel decisions (SmoothQuant factors, static scales, activation factors) are computed
    by the same host code as the CPU path (LinearQuantizer.plan) from small vectors.

Every output tensor equals the CPU path's bit for bit (tests/test_gpu_prep.py).
"""
from __future__ import annotations

import ctypes
import math
import time
from typing import Dict

import numpy as np
import torch

from ._lib import check, load
from .mk_weights import (BF16, F32, LINEARS, LinearQuantizer, _last_layer_bf16, hf_layer, interleave_gu, mlp_chunk,
                         rope_tables, run_calibration)
from .quant import parse_quant, quant_flags


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


class _Packer:
    """ctypes front of mk_weight_row_amax / mk_weight_quantize on one device and stream."""

    def __init__(self, device):
        self.lib = load()
        self.dev = torch.device(device)
        self.stream = ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)

    def row_amax(self, parts, k_in):
        """max over the parts' columns of |w^T * fold| per input row j -> (k_in,) f32 on the host."""
        out = None
        aw = torch.empty(k_in, dtype=F32, device=self.dev)
        for w, fold in parts:
            check(self.lib.mk_weight_row_amax(_ptr(w), w.shape[0], w.shape[1], ctypes.c_float(fold), _ptr(aw),
                                              self.stream), "mk_weight_row_amax")
            out = aw.clone() if out is None else torch.maximum(out, aw)
        return out.cpu()

    def quantize(self, parts, k_in, smooth, base, sx):
        """(codes (k_in, n) int8 / e4m3, s_w (n,) f32) for the parts side by side in column order."""
        n = sum(w.shape[0] for w, _ in parts)
        fp8 = base in ("fp8", "fp8d")
        codes = torch.empty((k_in, n), dtype=torch.uint8, device=self.dev)
        s_w = torch.empty(n, dtype=F32, device=self.dev)
        scale = torch.empty(n, dtype=F32, device=self.dev)
        sm = smooth.to(self.dev) if smooth is not None else None
        col = 0
        for w, fold in parts:
            no = w.shape[0]
            check(self.lib.mk_weight_quantize(_ptr(w), no, k_in, ctypes.c_float(fold), _ptr(sm), int(fp8),
                                              ctypes.c_float(sx), ctypes.c_void_p(codes.data_ptr() + col),
                                              n, ctypes.c_void_p(scale.data_ptr() + 4 * col),
                                              ctypes.c_void_p(s_w.data_ptr() + 4 * col), self.stream),
                  "mk_weight_quantize")
            col += no
        codes = codes.view(torch.float8_e4m3fn) if fp8 else codes.view(torch.int8)
        return codes, s_w


def _hf(sd, name, dev):
    return sd[name].to(dev).contiguous()


def _layer_on_host(sd, cfg, i, fold_qkv_gamma, fold_gu_gamma):
    """hf_layer of layer i built on the CPU (the calibration forward's device), wherever sd lives."""
    pre = f"model.layers.{i}."
    return hf_layer({k: v.to("cpu") for k, v in sd.items() if k.startswith(pre)}, cfg, i, fold_qkv_gamma, fold_gu_gamma)


@torch.no_grad()
def prepare_on_gpu(sd: Dict[str, torch.Tensor], cfg: dict, quant: str, max_seq: int, log=print,
                   device="cuda:0") -> Dict[str, torch.Tensor]:
    """prepare_mk_weights(sd, cfg, quant, max_seq) with the result on `device` (module docstring)."""
    t0 = time.perf_counter()
    dev = torch.device(device)
    linear_names = [k for k in sd if k.startswith("model.layers.") and k.endswith("_proj.weight")]
    if any(sd[k].dtype != BF16 for k in linear_names):
        # the packer reads bf16 weights (the checkpoints' dtype); anything else goes the CPU way
        from .mk_weights import prepare_mk_weights

        w = prepare_mk_weights(sd, cfg, quant, max_seq, log=log)
        return {k: v.to(dev) for k, v in w.items()}
    if dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    qm = parse_quant(quant)
    flags = quant_flags(quant)
    base = quant.split("|")[0].split(":", 1)[0]
    L, hd = cfg["num_layers"], cfg["head_dim"]
    fold_q = float(np.float32(1.0 / math.sqrt(hd)))        # the f32 factor the CPU path multiplies W_q by
    fq, fg = qm["qkv"] == "bf16", qm["gu"] == "bf16"
    cos, sin = rope_tables(max_seq, hd, cfg["rope_theta"])
    out: Dict[str, torch.Tensor] = {"cos": cos.to(dev), "sin": sin.to(dev)}
    last = _layer_on_host(sd, cfg, L - 1, fq, fg)
    out.update({k: v.to(dev) for k, v in _last_layer_bf16(last, qm).items()})
    del last

    def bf16_linear(i, lin):
        """A bf16 scan-layer linear in the (in, out) layout: the CPU path's f32 products (1/sqrt(hd) on
        W_q, gammas folded into the rows), then one rounding to bf16, done on the GPU."""
        p = f"model.layers.{i}."
        if lin == "qkv":
            g = _hf(sd, p + "input_layernorm.weight", dev).float()
            q = _hf(sd, p + "self_attn.q_proj.weight", dev).float().t() * fold_q
            ts = [q, _hf(sd, p + "self_attn.k_proj.weight", dev).float().t(),
                  _hf(sd, p + "self_attn.v_proj.weight", dev).float().t()]
            return torch.cat([g[:, None] * t for t in ts], dim=1).to(BF16)
        if lin == "gu":
            g = _hf(sd, p + "post_attention_layernorm.weight", dev).float()
            ts = [_hf(sd, p + "mlp.gate_proj.weight", dev).float().t(), _hf(sd, p + "mlp.up_proj.weight", dev).float().t()]
            return torch.stack([g[:, None] * t for t in ts], dim=1).to(BF16)
        name = "self_attn.o_proj" if lin == "o" else "mlp.down_proj"
        return _hf(sd, p + name + ".weight", dev).float().t().contiguous().to(BF16)

    scan = range(L - 1)
    if base == "bf16":
        for lin in LINEARS:
            out["w_" + lin] = torch.stack([bf16_linear(i, lin) for i in scan]).contiguous()
        for k in ("s_qkv", "s_o", "s_gu", "s_down", "a_qkv", "a_o", "a_gu", "a_down"):
            out[k] = torch.zeros((1,), dtype=F32, device=dev)
        log(f"[mk] bf16 weights prepared on {dev} (L-1={L - 1} + last) in {time.perf_counter() - t0:.1f}s")
        return out

    t_cal = time.perf_counter()
    cal = run_calibration(sd, cfg, quant, (_layer_on_host(sd, cfg, i, fq, fg) for i in range(L)))
    t_cal = time.perf_counter() - t_cal
    pk = _Packer(dev)
    stacks = {f"{p}_{lin}": [] for p in ("w", "s", "a") for lin in LINEARS}
    dummy = torch.zeros((1,), dtype=F32, device=dev)
    for li in scan:
        p = f"model.layers.{li}."
        g_in = sd[p + "input_layernorm.weight"].to("cpu", F32)
        g_post = sd[p + "post_attention_layernorm.weight"].to("cpu", F32)
        for lin in LINEARS:
            if qm[lin] == "bf16":
                parts = (bf16_linear(li, lin), dummy, dummy)
            else:
                if lin == "qkv":
                    hf = [(_hf(sd, p + "self_attn.q_proj.weight", dev), fold_q),
                          (_hf(sd, p + "self_attn.k_proj.weight", dev), 1.0),
                          (_hf(sd, p + "self_attn.v_proj.weight", dev), 1.0)]
                elif lin == "gu":
                    hf = [(_hf(sd, p + "mlp.gate_proj.weight", dev), 1.0), (_hf(sd, p + "mlp.up_proj.weight", dev), 1.0)]
                else:
                    hf = [(_hf(sd, p + ("self_attn.o_proj.weight" if lin == "o" else "mlp.down_proj.weight"), dev), 1.0)]
                k_in = hf[0][0].shape[1]
                qz = LinearQuantizer(qm[lin], "sq" in flags, cal["alpha"], cal["margin"])
                aw = pk.row_amax(hf, k_in) if qz.use_sq else None
                gamma = g_in if lin == "qkv" else g_post if lin == "gu" else None
                smooth, sx, a_x = qz.plan(lin, k_in, gamma, cal["scales"][li][lin], cal["sq_stats"][li][lin],
                                          cal["chan_nob"][li][lin], aw)
                codes, s_w = pk.quantize(hf, k_in, smooth, qm[lin], sx)
                if lin == "gu":
                    codes, s_w = codes.view(k_in, 2, -1), s_w.view(2, -1)
                parts = (codes, s_w, a_x.to(dev))
            for kind, t in zip(("w", "s", "a"), parts):
                stacks[f"{kind}_{lin}"].append(t)
    out.update({k: torch.stack(v).contiguous() for k, v in stacks.items()})
    if "fmlp" in flags and qm["gu"] in ("int8", "int8d"):
        out["w_gu"], out["s_gu"] = interleave_gu(out["w_gu"], out["s_gu"], mlp_chunk(cfg["inter"]))
    torch.cuda.synchronize(dev)
    log(f"[mk] {quant} weights prepared on {dev} (L-1={L - 1}, calibration {cal['n_seq']}x{cal['s_cal']} on the host "
        f"in {t_cal:.1f}s, sq={'sq' in flags}, alpha={cal['alpha']}) in {time.perf_counter() - t0:.1f}s")
    return out
