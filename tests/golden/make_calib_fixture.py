"""Writes tests/golden/calib_fixture.npz: the reference's own weight calibration / quantisation outputs.

    python tests/golden/make_calib_fixture.py

Runs in the build container only (it reads /root/reference, which the GPU machines do not have).
It loads plugin/minicpm5_mk/mk_weights.py from the reference tree by file path -- that module's top
level imports only numpy and torch (mk_weights.py:6-14) -- and calls three of its functions on
small synthetic inputs:

  * `rope_tables(max_seq, hd, theta)`                         (mk_weights.py:20-26)
  * `_calibrate(layers, embed, cos, sin, cfg, quant, ...)`    (mk_weights.py:29-110)
  * `_quantize_w(w, quant, sx)`                               (mk_weights.py:113-123)

Inputs: the `tiny` and `tiny-hd96` presets' random-init weights (minicpm5_mk.synth, seed 0) with
non-unit RMSNorm gammas (0.5 + U[0,1) from torch.Generator seed 5, rounded to bf16, stored in the
fixture), laid out as the reference's prepare_mk_weights builds its per-layer dicts
(mk_weights.py:143-167): (in, out) matrices, 1/sqrt(hd) folded into W_q, gammas kept apart because
qkv and gu are quantised.  The layer dicts are built here by code of this script, not by the
product's helpers, so the test also pins the product's layout construction.

Stored per (preset, base in int8d / int8 / fp8):
  scales   (L, 4) f32  static scales of qkv, o, gu, down     (_calibrate's first result)
  chan_*   per layer and linear, per-input-channel amax     (second result)
  nob_*    the same excluding position 0                    (third result)
  quantize_w of every layer's four matrices with sx = 1 and of the smoothed q/k/v matrix with the
  static scale: int8 / e4m3 codes as sha256 hex digests plus the f32 scale vectors in full.
"""
import hashlib
import importlib.util
import json
import math
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "minicpm5-vllm-tpu_amd")]
REF = "/root/reference/plugin/minicpm5_mk/mk_weights.py"

import numpy as np  # noqa: E402
import torch  # noqa: E402

from minicpm5_mk.config import preset  # noqa: E402
from minicpm5_mk.synth import random_hf_state_dict  # noqa: E402

F32 = torch.float32
PRESETS = ("tiny", "tiny-hd96")
BASES = ("int8d", "int8", "fp8")
LIN = ("qkv", "o", "gu", "down")


def load_reference():
    spec = importlib.util.spec_from_file_location("ref_mk_weights", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def gammas(cfg):
    g = torch.Generator().manual_seed(5)
    return [((torch.rand(cfg.hidden, generator=g) + 0.5).to(torch.bfloat16),
             (torch.rand(cfg.hidden, generator=g) + 0.5).to(torch.bfloat16)) for _ in range(cfg.num_layers)]


def layer_dicts(sd, cfg, gam):
    """Per-layer f32 dicts in the reference's prepare_mk_weights layout (quantised qkv and gu)."""
    sm = 1.0 / math.sqrt(cfg.head_dim)
    out = []
    for i in range(cfg.num_layers):
        p = f"model.layers.{i}."
        w = {n: sd[p + n + ".weight"].to(F32) for n in (
            "self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
            "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")}
        qkv = torch.cat([w["self_attn.q_proj"].T * sm, w["self_attn.k_proj"].T, w["self_attn.v_proj"].T], 1)
        out.append({"w_qkv": qkv.contiguous(), "w_o": w["self_attn.o_proj"].T.contiguous(),
                    "w_gu": torch.stack([w["mlp.gate_proj"].T, w["mlp.up_proj"].T], 1).contiguous(),
                    "w_down": w["mlp.down_proj"].T.contiguous(),
                    "in_norm": gam[i][0].to(F32), "post_norm": gam[i][1].to(F32)})
    return out


def digest(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def main():
    for k in [k for k in os.environ if k.startswith("MINICPM5_MK_")]:
        del os.environ[k]
    torch.set_num_threads(1)   # one summation order for the f32 calibration forward
    ref = load_reference()
    arrays, meta = {}, {"source": "plugin/minicpm5_mk/mk_weights.py:20-123", "threads": 1, "digests": {}}
    for name in PRESETS:
        cfg = preset(name)
        sd = random_hf_state_dict(cfg, seed=0)
        gam = gammas(cfg)
        for i, (a, b) in enumerate(gam):
            arrays[f"{name}/gamma_in/{i}"] = a.float().numpy()
            arrays[f"{name}/gamma_post/{i}"] = b.float().numpy()
        layers = layer_dicts(sd, cfg, gam)
        embed = sd["model.embed_tokens.weight"].to(F32)
        c, s = ref.rope_tables(512, cfg.head_dim, cfg.rope_theta)
        arrays[f"{name}/rope_cos"] = c.view(torch.int16).numpy()
        arrays[f"{name}/rope_sin"] = s.view(torch.int16).numpy()
        rc, rs = ref.rope_tables(128, cfg.head_dim, cfg.rope_theta)
        for base in BASES:
            key = f"{name}/{base}"
            scales, chan, nob = ref._calibrate(layers, embed, rc.to(F32), rs.to(F32), cfg.as_mk_cfg(), base, 0,
                                               n_seq=4, s_cal=128, seed=42,
                                               gamma_in_act={"qkv": True, "gu": True})
            arrays[key + "/scales"] = np.array([[sc[n] for n in LIN] for sc in scales], dtype=np.float64)
            for li in range(cfg.num_layers):
                for n in LIN:
                    arrays[f"{key}/chan/{li}/{n}"] = chan[li][n].numpy()
                    arrays[f"{key}/nob/{li}/{n}"] = nob[li][n].numpy()
            for li, ld in enumerate(layers):
                for n in LIN:
                    wq, sw = ref._quantize_w(ld["w_" + n], base, 1.0)
                    arrays[f"{key}/qw_scale/{li}/{n}"] = sw.numpy()
                    meta["digests"][f"{key}/qw_codes/{li}/{n}"] = digest(wq)
                # smoothed q/k/v with the static scale: the path of a static base with SmoothQuant
                ax = chan[li]["qkv"].clamp(min=1e-5)
                aw = ld["w_qkv"].abs().amax(dim=1).clamp(min=1e-5)
                smooth = (ax.pow(0.5) / aw.pow(0.5)).clamp(1e-4, 1e4)
                wq, sw = ref._quantize_w(ld["w_qkv"] * smooth[:, None], base, scales[li]["qkv"])
                arrays[f"{key}/qw_smooth_scale/{li}"] = sw.numpy()
                meta["digests"][f"{key}/qw_smooth_codes/{li}"] = digest(wq)
            print(f"[calib] {key}: layer-0 scales {[round(scales[0][n], 6) for n in LIN]}", flush=True)
    arrays["meta"] = np.frombuffer(json.dumps(meta, sort_keys=True).encode(), dtype=np.uint8)
    out = os.path.join(HERE, "calib_fixture.npz")
    np.savez_compressed(out, **arrays)
    print(f"[calib] wrote {out} ({os.path.getsize(out) / 1024:.0f} KiB, {len(arrays)} arrays)")


if __name__ == "__main__":
    main()
