"""Deterministic synthetic inputs: random-init HF-named weights and seeded token ids.

No checkpoint can be fetched here, so every measurement and parity check runs on random-init
weights of the real architecture.  The weights follow the HF initialisation of a Llama model:

  * every Linear / Embedding / lm_head weight is N(0, std) with std 0.02 (HF `initializer_range`),
  * RMSNorm gammas are 1.0, `tie_word_embeddings=False`.

Each tensor is drawn in float32 and rounded ONCE to bfloat16 (the checkpoint dtype); the FP32
golden upcasts exactly those bf16 values, as the reference's golden upcasts the bf16 checkpoint
(benchmark/f32_golden.py:28-42).

Stream layout (the definition of the weights): tensor number `t` in `hf_tensor_order(cfg)` is cut
into chunks of 2**22 elements; chunk `c` is filled with `standard_normal(float32)` from
`numpy.random.PCG64(SeedSequence(seed, spawn_key=(t, c)))`, then scaled by `std`.  Chunks are
independent streams, so generation is parallel and bit-reproducible on any machine with the same
numpy.  Token ids are `torch.randint(lo, hi, (B, S))` from `torch.Generator().manual_seed(seed)`.
"""
from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch

from .config import MkConfig

CHUNK = 1 << 22


def hf_tensor_order(cfg: MkConfig):
    """[(name, shape)] of every random tensor, HF (out, in) shapes, in generation order."""
    H, I, V = cfg.hidden, cfg.inter, cfg.vocab
    out = [("model.embed_tokens.weight", (V, H))]
    for i in range(cfg.num_layers):
        p = f"model.layers.{i}."
        out += [
            (p + "self_attn.q_proj.weight", (cfg.q_dim, H)),
            (p + "self_attn.k_proj.weight", (cfg.kv_dim, H)),
            (p + "self_attn.v_proj.weight", (cfg.kv_dim, H)),
            (p + "self_attn.o_proj.weight", (H, cfg.q_dim)),
            (p + "mlp.gate_proj.weight", (I, H)),
            (p + "mlp.up_proj.weight", (I, H)),
            (p + "mlp.down_proj.weight", (H, I)),
        ]
    out.append(("lm_head.weight", (V, H)))
    return out


def _fill_normal(dst: torch.Tensor, seed: int, t_index: int, std: float, pool: ThreadPoolExecutor) -> None:
    flat = dst.view(-1)
    arr = flat.numpy()
    n = flat.numel()

    def work(c):
        lo, hi = c * CHUNK, min(n, (c + 1) * CHUNK)
        g = np.random.Generator(np.random.PCG64(np.random.SeedSequence(seed, spawn_key=(t_index, c))))
        g.standard_normal(out=arr[lo:hi], dtype=np.float32)

    list(pool.map(work, range((n + CHUNK - 1) // CHUNK)))
    flat.mul_(std)


def random_hf_state_dict(cfg: MkConfig, seed: int = 0, std: float = 0.02, threads: int | None = None,
                         names=None) -> dict:
    """HF-named bf16 CPU tensors of a random-init MiniCPM5 (Llama) model.

    `names` optionally restricts which tensors are materialised (the stream of every other tensor is
    unaffected, since each tensor has its own streams)."""
    threads = threads or min(16, os.cpu_count() or 1)
    sd = {}
    scratch = None
    with ThreadPoolExecutor(threads) as pool:
        for t, (name, shape) in enumerate(hf_tensor_order(cfg)):
            if names is not None and name not in names:
                continue
            n = int(np.prod(shape))
            if scratch is None or scratch.numel() < n:
                scratch = torch.empty(n, dtype=torch.float32)
            buf = scratch[:n]
            _fill_normal(buf, seed, t, std, pool)
            sd[name] = buf.view(shape).to(torch.bfloat16)
    for i in range(cfg.num_layers):
        p = f"model.layers.{i}."
        for nm in ("input_layernorm.weight", "post_attention_layernorm.weight"):
            if names is None or p + nm in names:
                sd[p + nm] = torch.ones(cfg.hidden, dtype=torch.bfloat16)
    if names is None or "model.norm.weight" in names:
        sd["model.norm.weight"] = torch.ones(cfg.hidden, dtype=torch.bfloat16)
    return sd


def random_token_ids(batch: int, seq: int, seed: int = 1234, lo: int = 1000, hi: int = 30000) -> torch.Tensor:
    """(batch, seq) int32 token ids uniform in [lo, hi) from a torch generator seeded with `seed`."""
    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi, (batch, seq), generator=g, dtype=torch.int64).to(torch.int32)
