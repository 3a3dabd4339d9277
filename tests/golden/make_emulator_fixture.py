"""Writes full-size fixtures of the CPU emulation of the plugin's numerics (oracle/emulate.py).

    python tests/golden/make_emulator_fixture.py --preset 1b-hd96 [--quant auto] [--batch 1 --seq 8192]

Writes tests/golden/emulate_<preset>_<tag>_b<B>_s<S>.npz with the last-position logits (float32,
all V) of `emulate.mk_forward` -- the plugin's W8A8 / bf16 algebra restated in torch
(mk_jax.py:527-569, mk_mlp.py:68-206, mk_attn.py:557-657) -- on the same random-init weights
(seed 0) and token ids (seed 1234) as the FP32 golden fixtures, and the FP32 golden's comparison
figures for the record (max / mean |logit error|, argmax, top-1/top-2 margin).  <tag> is the quant
string's base ("auto" resolves per architecture, model.py:528-551).  A 1B (1, 8192) run takes a few
minutes on 8 CPU threads, 2B about five.
"""
import argparse
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "minicpm5-vllm-tpu_amd")]

import numpy as np  # noqa: E402
import torch  # noqa: E402

from minicpm5_mk.config import preset  # noqa: E402
from minicpm5_mk.mk_weights import prepare_mk_weights  # noqa: E402
from minicpm5_mk.quant import resolve_quant_pair  # noqa: E402
from minicpm5_mk.synth import random_hf_state_dict, random_token_ids  # noqa: E402
from oracle import emulate  # noqa: E402


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--preset", required=True)
    ap.add_argument("--quant", default="auto")
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--seq", type=int, default=8192)
    args = ap.parse_args()
    for k in [k for k in os.environ if k.startswith("MINICPM5_MK_")]:
        del os.environ[k]
    torch.set_num_threads(os.cpu_count())
    cfg = preset(args.preset)
    t0 = time.time()
    sd = random_hf_state_dict(cfg, seed=0)
    quant = resolve_quant_pair(args.quant, cfg.num_layers, 1, cfg.hidden, cfg.inter)[0]
    w = prepare_mk_weights(sd, cfg.as_mk_cfg(), quant, 8256)
    ids = random_token_ids(args.batch, args.seq, seed=1234)
    _, logits = emulate.mk_forward(ids, w, sd["model.embed_tokens.weight"], sd["model.norm.weight"], cfg, quant,
                                   sd["lm_head.weight"])
    meta = {"preset": args.preset, "quant": quant, "batch": args.batch, "seq": args.seq, "weight_seed": 0,
            "id_seed": 1234, "secs": round(time.time() - t0, 1)}
    gpath = os.path.join(HERE, f"golden_{args.preset}_b{args.batch}_s{args.seq}.npz")
    if os.path.exists(gpath):
        g = torch.from_numpy(np.load(gpath)["logits"])
        err = (logits - g).abs()
        top2 = torch.topk(g, 2, dim=-1).values
        meta.update(vs_golden_max=float(err.max()), vs_golden_mean=float(err.mean()),
                    argmax=logits.argmax(-1).tolist(), golden_argmax=g.argmax(-1).tolist(),
                    golden_margin=(top2[:, 0] - top2[:, 1]).tolist())
    tag = "auto" if args.quant == "auto" else quant.split("|")[0].split(":")[0]
    out = os.path.join(HERE, f"emulate_{args.preset}_{tag}_b{args.batch}_s{args.seq}.npz")
    np.savez_compressed(out, logits=logits.numpy().astype(np.float32),
                        meta=np.frombuffer(json.dumps(meta).encode(), dtype=np.uint8))
    print(json.dumps(meta), flush=True)


if __name__ == "__main__":
    main()
