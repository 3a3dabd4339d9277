"""Writes the FP32-golden fixtures used by the full-model parity tests.

    python tests/golden/make_golden.py --preset 1b --batch 1

For preset P and batch B it writes tests/golden/golden_<P>_b<B>_s<S>.npz holding, per sequence, the
FP32 last-position logits (float32, all V of them) and the top-20 ids / logprobs of the oracle's
FP32 forward (oracle/golden.py, a restatement of benchmark/f32_golden.py), on random-init weights
(seed 0) and token ids uniform in [1000, 30000) (seed 1234) -- both from minicpm5_mk.synth.
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
from minicpm5_mk.synth import random_hf_state_dict, random_token_ids  # noqa: E402
from oracle import golden  # noqa: E402


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--preset", required=True)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--seq", type=int, default=8192)
    ap.add_argument("--wseed", type=int, default=0)
    ap.add_argument("--idseed", type=int, default=1234)
    args = ap.parse_args()
    torch.set_num_threads(os.cpu_count())
    cfg = preset(args.preset)
    t0 = time.time()
    sd = random_hf_state_dict(cfg, seed=args.wseed)
    W = golden.load_f32(sd, cfg)
    del sd
    print(f"[golden] weights {cfg.name} in {time.time() - t0:.1f}s", flush=True)
    ids = random_token_ids(args.batch, args.seq, seed=args.idseed)
    cos, sin = golden.rope_tables(args.seq, cfg.head_dim, cfg.rope_theta)
    logits, tids, tlps = [], [], []
    for b in range(args.batch):
        t1 = time.time()
        lg, ti, tl = golden.forward_one(ids[b], W, cfg, cos, sin)
        logits.append(lg.numpy())
        tids.append(ti)
        tlps.append(tl)
        srt = np.sort(lg.numpy())
        print(f"[golden] seq {b} in {time.time() - t1:.1f}s top1={ti[0]} margin={srt[-1] - srt[-2]:.4f}", flush=True)
    out = os.path.join(HERE, f"golden_{args.preset}_b{args.batch}_s{args.seq}.npz")
    np.savez_compressed(out, logits=np.stack(logits).astype(np.float32), top_ids=np.array(tids, np.int64),
                        top_logprobs=np.array(tlps, np.float32),
                        meta=json.dumps({"preset": args.preset, "config": cfg.as_mk_cfg(), "vocab": cfg.vocab,
                                         "batch": args.batch, "seq": args.seq, "weight_seed": args.wseed,
                                         "id_seed": args.idseed}))
    print(f"[golden] wrote {out}", flush=True)


if __name__ == "__main__":
    main()
