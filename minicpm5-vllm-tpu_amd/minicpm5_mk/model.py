"""vLLM model class: MiniCPM5 (Llama) whose uniform fresh prefill steps run through libmk.

Mirrors plugin/minicpm5_mk/model.py (MiniCPM5MegakernelForCausalLM, :554-795): the stock
LlamaForCausalLM serves every other step (decode, chunked or partial prefills, ragged batches, dummy
runs); `load_weights` tees the HF tensors, prepares the plugin's quantized layout
(prepare_mk_weights) and builds an `MkModel`; `forward` runs the fast path when the host-side
decision of this step says so.

That decision is made before the forward from the scheduler's state, as the reference does
(`_eligible_batch`, model.py:139-169): a hook on vLLM's GPU model runner (`dispatch.install_runner_hook`)
checks that every request is a fresh, whole-prompt prefill of one length with max_tokens == 1 and no
prompt logprobs, and records (bs, seq) or a reason code.  The forward never inspects device tensors.
A fast-path prefill writes no KV cache, which is why max_tokens == 1 is required.  When the hook
cannot be installed the fast path stays off.

Without the reference's hidden-state selection patch (model.py:224-235) the forward returns a (T, H)
tensor with the B final-normed last-token rows at rows b*S + S - 1, the rows the stock logits
selection reads.

Requires vLLM (imported at module import, like the reference).  Environment knobs kept from the
reference (model.py:23-32): MINICPM5_MK_ENABLE, MINICPM5_MK_QUANT, MINICPM5_MK_ATTN,
MINICPM5_MK_REQUIRE_MAX_TOKENS_1, MINICPM5_MK_FREE_STOCK, MINICPM5_MK_STATUS_DIR, MINICPM5_MK_PRECOMPILE; and
MINICPM5_MK_CHECK_POSITIONS=1 cross-checks each fast-path step against the device positions (syncs).
"""
from __future__ import annotations

import json
import logging
import os
import time
import weakref
from collections.abc import Iterable

import torch
from vllm.model_executor.models.llama import LlamaForCausalLM

from .config import MkConfig
from .dispatch import STATE, install_runner_hook, positions_match, scatter_last_rows
from .mk_weights import prepare_mk_weights
from .quant import resolve_quant_pair
from .runtime import WEIGHT_ORDER, MkModel, parse_precompile

logger = logging.getLogger("vllm.minicpm5_mk")

_WEIGHT_SUFFIXES = (
    "input_layernorm.weight", "post_attention_layernorm.weight",
    "self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
    "self_attn.o_proj.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight",
)


def _hook_vllm_runner(model) -> bool:
    """Install the eligibility hook on vLLM's v1 GPU model runner (one class per process)."""
    try:
        from vllm.v1.worker.gpu_model_runner import GPUModelRunner
    except ImportError:
        return False
    ref = weakref.ref(model)
    require_mt1 = os.environ.get("MINICPM5_MK_REQUIRE_MAX_TOKENS_1", "1") != "0"
    return install_runner_hook(GPUModelRunner, lambda runner: ref()._mk_max_seq if ref() else 0, require_mt1)


class MiniCPM5MegakernelForCausalLM(LlamaForCausalLM):
    def __init__(self, *, vllm_config, prefix: str = "", **kwargs):
        super().__init__(vllm_config=vllm_config, prefix=prefix, **kwargs)
        hf = vllm_config.model_config.hf_config
        self._mk_cfg = MkConfig.from_hf(hf)
        self._mk_enabled = os.environ.get("MINICPM5_MK_ENABLE", "1") != "0"
        self._mk_max_seq = int(vllm_config.model_config.max_model_len)
        self._mk_attn = os.environ.get("MINICPM5_MK_ATTN", "auto")
        self._mk_counts = {"mk": 0, "stock": 0}
        self._mk_model = None
        self._mk_status = None
        rope = getattr(hf, "rope_scaling", None) or getattr(hf, "rope_parameters", None)
        if isinstance(rope, dict) and rope.get("rope_type", rope.get("type", "default")) not in (None, "default"):
            logger.warning("minicpm5_mk: rope_scaling=%s unsupported; fast path disabled", rope)
            self._mk_enabled = False
        if vllm_config.parallel_config.pipeline_parallel_size != 1 or vllm_config.parallel_config.tensor_parallel_size != 1:
            logger.warning("minicpm5_mk: one GPU per model only (no PP / TP); fast path disabled")
            self._mk_enabled = False
        try:
            self._mk_cfg.validate()
        except ValueError as e:
            logger.warning("minicpm5_mk: %s; fast path disabled", e)
            self._mk_enabled = False
        if self._mk_enabled and not _hook_vllm_runner(self):
            logger.warning("minicpm5_mk: vLLM GPU model runner not found; fast path disabled")
            self._mk_enabled = False

    def load_weights(self, weights: Iterable[tuple[str, torch.Tensor]]) -> set[str]:
        if not self._mk_enabled:
            return super().load_weights(weights)
        stash: dict[str, torch.Tensor] = {}

        def tee():
            for name, t in weights:
                if (name.startswith("model.layers.") and name.endswith(_WEIGHT_SUFFIXES)) or name in (
                        "model.embed_tokens.weight", "model.norm.weight"):
                    stash[name] = t.detach().to("cpu", copy=True)
                yield name, t

        loaded = super().load_weights(tee())
        try:
            self._mk_build(stash)
        except Exception:
            if os.environ.get("MINICPM5_MK_FREE_STOCK", "0") == "1":
                logger.exception("minicpm5_mk: build failed and MINICPM5_MK_FREE_STOCK=1")
                raise
            logger.exception("minicpm5_mk: build failed; stock path only")
            self._mk_model = None
        return loaded

    def _mk_build(self, stash: dict) -> None:
        t0 = time.perf_counter()
        c = self._mk_cfg
        quant, _ = resolve_quant_pair(os.environ.get("MINICPM5_MK_QUANT", "auto"), c.num_layers, 1, c.hidden, c.inter)
        dev = self.lm_head.weight.device
        w = prepare_mk_weights(stash, c.as_mk_cfg(), quant, self._mk_max_seq, c.bos_token_id, log=logger.info,
                               device=dev if dev.type == "cuda" else None)
        emb = self.model.embed_tokens.weight
        embed = emb.data if emb.dtype == torch.bfloat16 else stash["model.embed_tokens.weight"].to(torch.bfloat16).to(dev)
        self._mk_keep = {k: w[k].to(dev) for k in WEIGHT_ORDER}
        self._mk_model = MkModel(self._mk_keep, embed, w["cos"].to(dev), w["sin"].to(dev),
                                 stash["model.norm.weight"].to(torch.bfloat16).to(dev), quant, c.n_q, c.n_kv,
                                 c.head_dim, c.eps)
        self._mk_status = {"arch": "MiniCPM5MegakernelForCausalLM", "quant": quant, "attn": self._mk_attn,
                           "backend": "libmk (HIP, gfx950)", "shapes": {}}
        self._mk_write_status()
        logger.info("minicpm5_mk: libmk ready (quant=%s) in %.1fs", quant, time.perf_counter() - t0)
        # hipGraphs of the listed shapes captured now instead of at each shape's first step (model.py:690-698)
        self._mk_model.precompile(parse_precompile(os.environ.get("MINICPM5_MK_PRECOMPILE", "")), logits=False,
                                  log=logger.info)

    def _mk_write_status(self) -> None:
        d = os.environ.get("MINICPM5_MK_STATUS_DIR")
        if not d or self._mk_status is None:
            return
        os.makedirs(d, exist_ok=True)
        path = os.path.join(d, "minicpm5_mk_status_rank0.json")
        with open(path + ".tmp", "w") as f:
            json.dump(self._mk_status, f, indent=1)
        os.replace(path + ".tmp", path)

    def forward(self, input_ids, positions, intermediate_tensors=None, inputs_embeds=None):
        batch, reason = STATE.take()
        if (batch is not None and self._mk_model is not None and input_ids is not None and inputs_embeds is None
                and intermediate_tensors is None and batch[0] * batch[1] <= input_ids.numel()):
            B, S = batch
            if os.environ.get("MINICPM5_MK_CHECK_POSITIONS") == "1" and not positions_match(positions, B, S):
                raise RuntimeError(f"minicpm5_mk: host decision {B}x{S} disagrees with the step's positions")
            key = f"mk:{B}x{S}"
            self._mk_counts["mk"] += 1
            if key not in self._mk_counts:
                self._mk_counts[key] = 0
                self._mk_status["shapes"][key] = {"mode": "single", "quant": self._mk_model.quant}
                self._mk_write_status()
            self._mk_counts[key] += 1
            rows = self._mk_model.forward(input_ids.reshape(-1)[: B * S].to(torch.int32), B, S)
            return scatter_last_rows(rows, B, S, input_ids.numel())
        self._mk_counts["stock"] += 1
        rkey = f"stock:{reason}"
        self._mk_counts[rkey] = self._mk_counts.get(rkey, 0) + 1
        return super().forward(input_ids, positions, intermediate_tensors, inputs_embeds)
