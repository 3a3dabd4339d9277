"""Local HF checkpoint directory -> (MkConfig, HF-named state dict) for MkEngine / prepare_mk_weights.

The reference gets its weights through vLLM's loader from the model directory (model.py:623-698
consumes the HF-named tensors).  This reads the same directory without vLLM: `config.json` (the
fields of model.py:561-568, via MkConfig.from_hf) and the safetensors shards, either one
`model.safetensors` or the shards listed in `model.safetensors.index.json`.  Only the tensors the
prefill path uses are kept (embedding, the decoder layers' projections and norms, the final norm and
the LM head; a tied LM head falls back to the embedding in MkEngine).  safetensors files hold no
code, so loading them executes nothing from the checkpoint.
"""
from __future__ import annotations

import json
import os

from .config import MkConfig

LAYER_TENSORS = ("input_layernorm.weight", "post_attention_layernorm.weight", "self_attn.q_proj.weight",
                 "self_attn.k_proj.weight", "self_attn.v_proj.weight", "self_attn.o_proj.weight",
                 "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight")


def wanted_names(cfg: MkConfig) -> set:
    names = {"model.embed_tokens.weight", "model.norm.weight", "lm_head.weight"}
    for i in range(cfg.num_layers):
        names |= {f"model.layers.{i}.{n}" for n in LAYER_TENSORS}
    return names


def shard_files(path: str) -> list:
    """The safetensors files of a checkpoint directory, in index order."""
    index = os.path.join(path, "model.safetensors.index.json")
    if os.path.isfile(index):
        with open(index) as f:
            wm = json.load(f)["weight_map"]
        files = []
        for fn in wm.values():
            if fn not in files:
                files.append(fn)
        return [os.path.join(path, fn) for fn in files]
    single = os.path.join(path, "model.safetensors")
    if os.path.isfile(single):
        return [single]
    raise FileNotFoundError(f"{path}: no model.safetensors or model.safetensors.index.json")


def load_local_checkpoint(path: str):
    """(MkConfig, state_dict of CPU tensors) from a local HF checkpoint directory."""
    from safetensors import safe_open

    cfg_path = os.path.join(path, "config.json")
    if not os.path.isfile(cfg_path):
        raise FileNotFoundError(f"{path}: no config.json")
    with open(cfg_path) as f:
        hf = json.load(f)
    cfg = MkConfig.from_hf(hf)
    cfg.validate()
    want = wanted_names(cfg)
    sd = {}
    for fn in shard_files(path):
        with safe_open(fn, framework="pt", device="cpu") as f:
            for k in f.keys():
                if k in want:
                    sd[k] = f.get_tensor(k)
    missing = sorted(n for n in want - set(sd) if n != "lm_head.weight")
    if missing:
        raise KeyError(f"{path}: checkpoint lacks {len(missing)} tensors, e.g. {missing[:3]}")
    return cfg, sd


__all__ = ["load_local_checkpoint", "shard_files", "wanted_names"]
