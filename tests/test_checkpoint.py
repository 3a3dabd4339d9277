"""Local checkpoint directories (minicpm5_mk.checkpoint): config.json + safetensors shards -> the same
config and tensors as the in-memory state dict; single-file and indexed-shard layouts, tied LM head,
and the errors for a missing config or tensor.  The GPU test checks that an engine built from the
directory scores exactly like one built from the state dict."""
import json
import os

import pytest
import torch


def _hf_config(cfg):
    return {"hidden_size": cfg.hidden, "num_attention_heads": cfg.n_q, "num_key_value_heads": cfg.n_kv,
            "num_hidden_layers": cfg.num_layers, "intermediate_size": cfg.inter, "head_dim": cfg.head_dim,
            "vocab_size": cfg.vocab, "rms_norm_eps": cfg.eps, "rope_theta": cfg.rope_theta,
            "bos_token_id": cfg.bos_token_id, "architectures": ["LlamaForCausalLM"]}


def _write(path, cfg, sd, shards):
    from safetensors.torch import save_file

    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(_hf_config(cfg), f)
    names = sorted(sd)
    if shards == 1:
        save_file({k: sd[k].contiguous() for k in names}, os.path.join(path, "model.safetensors"))
        return
    wm = {}
    for i in range(shards):
        part = names[i::shards]
        fn = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
        save_file({k: sd[k].contiguous() for k in part}, os.path.join(path, fn))
        wm.update({k: fn for k in part})
    with open(os.path.join(path, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": wm}, f)


@pytest.mark.parametrize("shards", [1, 3])
def test_checkpoint_roundtrip(tmp_path, shards):
    from minicpm5_mk.checkpoint import load_local_checkpoint
    from minicpm5_mk.config import preset
    from minicpm5_mk.synth import random_hf_state_dict

    cfg = preset("tiny")
    sd = random_hf_state_dict(cfg, seed=5)
    sd["lm_head.weight"] = sd["model.embed_tokens.weight"].clone() * 2
    sd["model.rotary_emb.inv_freq"] = torch.ones(4)          # present in some checkpoints, not used
    path = str(tmp_path / "ckpt")
    _write(path, cfg, sd, shards)
    c2, sd2 = load_local_checkpoint(path)
    assert c2.as_mk_cfg() == cfg.as_mk_cfg() and c2.vocab == cfg.vocab
    assert "model.rotary_emb.inv_freq" not in sd2
    assert set(sd2) == set(sd) - {"model.rotary_emb.inv_freq"}
    for k, v in sd2.items():
        assert v.dtype == sd[k].dtype and torch.equal(v, sd[k]), k


def test_checkpoint_tied_head_and_errors(tmp_path):
    from minicpm5_mk.checkpoint import load_local_checkpoint
    from minicpm5_mk.config import preset
    from minicpm5_mk.synth import random_hf_state_dict

    cfg = preset("tiny")
    sd = random_hf_state_dict(cfg, seed=6)
    sd.pop("lm_head.weight", None)
    path = str(tmp_path / "tied")
    _write(path, cfg, sd, 1)
    _, sd2 = load_local_checkpoint(path)
    assert "lm_head.weight" not in sd2                       # tied: the engine uses the embedding
    with pytest.raises(FileNotFoundError):
        load_local_checkpoint(str(tmp_path / "missing"))
    del sd["model.layers.1.mlp.up_proj.weight"]
    bad = str(tmp_path / "bad")
    _write(bad, cfg, sd, 1)
    with pytest.raises(KeyError, match="lacks 1 tensors"):
        load_local_checkpoint(bad)


@pytest.mark.gpu
def test_engine_from_checkpoint_dir(tmp_path):
    from minicpm5_mk.config import preset
    from minicpm5_mk.engine import MkEngine
    from minicpm5_mk.synth import random_hf_state_dict, random_token_ids

    assert torch.cuda.is_available(), "GPU test needs a visible MI355X"
    cfg = preset("tiny")
    sd = random_hf_state_dict(cfg, seed=7)
    path = str(tmp_path / "ckpt")
    _write(path, cfg, sd, 2)
    quiet = lambda *a: None  # noqa: E731
    a = MkEngine(path, max_model_len=1024, log=quiet)
    b = MkEngine(cfg, state_dict=sd, max_model_len=1024, log=quiet)
    ids = random_token_ids(2, 512, seed=3)
    la, lb = a.logits(ids).cpu(), b.logits(ids).cpu()
    assert torch.equal(la, lb)
    a.close()
    b.close()
