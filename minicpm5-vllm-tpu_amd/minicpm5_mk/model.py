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

Megakernel-only mode (MINICPM5_MK_FREE_STOCK=1, model.py:683-705, :787-794): after the build the stock
decoder-layer weights are dropped; a dummy (profiling) run then returns zeros and any other ineligible
step raises instead of running stock attention.  Only in this mode may the engine skip KV-cache
allocation for fast-path requests (the hook in `minicpm5_mk.register`), because no stock forward can
then read the unwritten KV blocks.

Prefix caching: a fast-path prefill writes no KV cache, but vLLM registers the request's full prompt
blocks in its prefix-cache table before the forward runs; a later request sharing that prefix would
hit those blocks and the stock path would attend over KV that was never written.  The fast path is
therefore off when the engine runs with prefix caching (the reference runs only with it off,
benchmark/run_benchmark.py:43), and megakernel-only mode refuses to start with it.

Requires vLLM (imported at module import, like the reference).  Environment knobs kept from the
reference (model.py:23-32): MINICPM5_MK_ENABLE, MINICPM5_MK_QUANT, MINICPM5_MK_ATTN,
MINICPM5_MK_REQUIRE_MAX_TOKENS_1, MINICPM5_MK_FREE_STOCK, MINICPM5_MK_STATUS_DIR, MINICPM5_MK_PRECOMPILE,
MINICPM5_MK_LOG_EVERY (log the path counters every N forwards); and MINICPM5_MK_CHECK_POSITIONS=1
cross-checks each fast-path step against the device positions (syncs).
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
    """Install the eligibility hook on vLLM's v1 GPU model runner (one class per process); a later
    model instance re-points the hook at itself."""
    try:
        from vllm.v1.worker.gpu_model_runner import GPUModelRunner
    except ImportError:
        return False
    ref = weakref.ref(model)
    require_mt1 = os.environ.get("MINICPM5_MK_REQUIRE_MAX_TOKENS_1", "1") != "0"
    return install_runner_hook(GPUModelRunner, lambda runner: ref()._mk_max_seq if ref() else 0, require_mt1)


def _free_stock() -> bool:
    return os.environ.get("MINICPM5_MK_FREE_STOCK", "0") == "1"


class MiniCPM5MegakernelForCausalLM(LlamaForCausalLM):
    def __init__(self, *, vllm_config, prefix: str = "", **kwargs):
        super().__init__(vllm_config=vllm_config, prefix=prefix, **kwargs)
        hf = vllm_config.model_config.hf_config
        self._mk_cfg = MkConfig.from_hf(hf)
        self._mk_enabled = os.environ.get("MINICPM5_MK_ENABLE", "1") != "0"
        self._mk_max_seq = int(vllm_config.model_config.max_model_len)
        self._mk_attn = os.environ.get("MINICPM5_MK_ATTN", "auto")
        self._mk_counts = {"mk": 0, "stock": 0}
        self._mk_log_every = int(os.environ.get("MINICPM5_MK_LOG_EVERY", "0") or 0)
        self._mk_model = None
        self._mk_status = None
        self._mk_stock_freed = False
        off = []   # why the fast path is off

        def disable(reason: str) -> None:
            logger.warning("minicpm5_mk: %s; fast path disabled", reason)
            off.append(reason)
            self._mk_enabled = False

        cache_cfg = getattr(vllm_config, "cache_config", None)
        if self._mk_enabled and getattr(cache_cfg, "enable_prefix_caching", False):
            disable("prefix caching is on (a fast-path prefill writes no KV cache; start the engine with "
                    "enable_prefix_caching=False)")
        rope = getattr(hf, "rope_scaling", None) or getattr(hf, "rope_parameters", None)
        if isinstance(rope, dict) and rope.get("rope_type", rope.get("type", "default")) not in (None, "default"):
            disable(f"rope_scaling={rope} unsupported")
        if vllm_config.parallel_config.pipeline_parallel_size != 1 or vllm_config.parallel_config.tensor_parallel_size != 1:
            disable("one GPU per model only (no PP / TP)")
        try:
            self._mk_cfg.validate()
        except ValueError as e:
            disable(str(e))
        if self._mk_enabled and not _hook_vllm_runner(self):
            disable("vLLM GPU model runner not found")
        # Megakernel-only mode lets the engine skip KV allocation for fast-path requests, which is only
        # correct while this model serves them on the fast path: with the fast path off for any reason
        # other than MINICPM5_MK_ENABLE=0 (which turns the KV skip off too), refuse to start.
        if off and _free_stock() and os.environ.get("MINICPM5_MK_ENABLE", "1") != "0":
            raise RuntimeError("minicpm5_mk: MINICPM5_MK_FREE_STOCK=1 needs the fast path, which is off: " + "; ".join(off))

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
            if _free_stock():
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
        logger.info("minicpm5_mk: libmk ready (quant=%s) in %.1fs", quant, time.perf_counter() - t0)
        if _free_stock():
            self._mk_free_stock_layers()
        # the reference's status keys (model.py:683-689); one GPU per model: tp 1, rank 0, no multicore modes
        self._mk_status = {"arch": "MiniCPM5MegakernelForCausalLM", "tp": 1, "rank": 0, "quant": quant,
                           "quant_tp": quant, "attn": self._mk_attn, "multicore_modes": [],
                           "stock_freed": self._mk_stock_freed, "backend": "libmk (HIP, gfx950)", "shapes": {}}
        self._mk_write_status()
        # hipGraphs of the listed shapes captured now instead of at each shape's first step (model.py:690-698)
        self._mk_model.precompile(parse_precompile(os.environ.get("MINICPM5_MK_PRECOMPILE", "")), logits=False,
                                  log=logger.info)

    def _mk_free_stock_layers(self) -> None:
        """Drop the stock decoder layers' weights (model.py:700-705): megakernel-only from here on."""
        for layer in self.model.layers:
            for p in layer.parameters():
                p.data = torch.empty((0,), dtype=p.dtype, device=p.device)
        self._mk_stock_freed = True
        logger.info("minicpm5_mk: freed stock decoder-layer weights (no stock fallback)")

    def _mk_write_status(self) -> None:
        """The path record (one small JSON; first use of each shape and each stock reason only)."""
        d = os.environ.get("MINICPM5_MK_STATUS_DIR")
        if not d or self._mk_status is None:
            return
        try:
            os.makedirs(d, exist_ok=True)
            path = os.path.join(d, "minicpm5_mk_status_rank0.json")
            with open(path + ".tmp", "w") as f:
                json.dump(self._mk_status, f, indent=1)
            os.replace(path + ".tmp", path)
        except OSError as e:
            logger.warning("minicpm5_mk: could not write status file: %r", e)

    def _mk_maybe_log(self, msg: str, reason: str) -> None:
        """Every MINICPM5_MK_LOG_EVERY forwards: the path counters (model.py:797-801)."""
        n = self._mk_log_every
        if n and (self._mk_counts["mk"] + self._mk_counts["stock"]) % n == 0:
            logger.info("minicpm5_mk: %s counts=%s last_reason=%s", msg, self._mk_counts, reason)

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
            self._mk_maybe_log(f"mk bs={B} seq={S} T={input_ids.numel()}", reason)
            rows = self._mk_model.forward(input_ids.reshape(-1)[: B * S].to(torch.int32), B, S)
            return scatter_last_rows(rows, B, S, input_ids.numel())
        self._mk_counts["stock"] += 1
        rkey = f"stock:{reason}"
        if rkey not in self._mk_counts:
            self._mk_counts[rkey] = 0
            if reason != "dummy":
                logger.info("minicpm5_mk: stock path (reason=%s, T=%d)", reason,
                            input_ids.numel() if input_ids is not None else -1)
                if self._mk_status is not None:
                    self._mk_status.setdefault("stock_reasons", []).append(reason)
                    self._mk_write_status()
        self._mk_counts[rkey] += 1
        self._mk_maybe_log(f"stock T={input_ids.numel() if input_ids is not None else -1}", reason)
        if self._mk_stock_freed:
            if reason == "dummy":
                src = input_ids if input_ids is not None else inputs_embeds
                n = src.numel() if input_ids is not None else src.shape[0]
                return torch.zeros((n, self._mk_cfg.hidden), dtype=torch.bfloat16, device=src.device)
            raise RuntimeError(f"minicpm5_mk: stock path needed ({reason}) but stock weights were freed")
        return super().forward(input_ids, positions, intermediate_tensors, inputs_embeds)
