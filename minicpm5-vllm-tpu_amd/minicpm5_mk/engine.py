"""Offline prefill/scoring engine with the `vllm.LLM(...).generate(..., max_tokens=1)` surface.

vLLM is not part of this image, so `MkEngine` provides the same call shape the reference's users
write (README.md:253-266, examples/minimal_vllm_inference.py:90-124):

    llm = MkEngine("1b")                                   # or an MkConfig / HF config + state dict
    outs = llm.generate([{"prompt_token_ids": ids}], SamplingParams(max_tokens=1, temperature=0.0))
    outs[0].outputs[0].token_ids                            # [next token]

It serves exactly the reference plugin's fast path -- uniform fresh prefills, max_tokens == 1,
sampling features of `sampling_fast_ok` (minicpm5_mk/__init__.py:10-32) -- and refuses anything
else with the reference's reason codes (model.py:139-169): ragged, max_tokens,
unsupported_sampling_feature, seq.  Weights come from an HF-named state dict (a local checkpoint)
or the deterministic random init of `minicpm5_mk.synth`; they are prepared by `prepare_mk_weights`
and run through libmk (`MkModel`).
"""
from __future__ import annotations

import os
import time
from dataclasses import dataclass, field

import torch

from .config import MkConfig, preset
from .dispatch import StepView, eligible_step, mk_seq_ok
from .mk_weights import prepare_mk_weights
from .quant import resolve_quant_pair
from .runtime import WEIGHT_ORDER, MkModel, parse_precompile

BF16 = torch.bfloat16


@dataclass
class SamplingParams:
    """The subset of vllm.SamplingParams the fast path reads (plus the fields it must see unset)."""
    max_tokens: int = 1
    min_tokens: int = 0
    temperature: float = 0.0
    top_p: float = 1.0
    top_k: int = 0
    seed: int | None = None
    logprobs: int | None = None
    detokenize: bool = False
    skip_clone: bool = False
    prompt_logprobs: int | None = None
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0
    repetition_penalty: float = 1.0
    min_p: float = 0.0
    logit_bias: dict | None = None
    allowed_token_ids: list | None = None
    bad_words: list | None = None
    structured_outputs: object = None
    logits_processors: list | None = None


@dataclass
class CompletionOutput:
    index: int
    token_ids: list
    logprobs: list | None = None
    text: str = ""
    finish_reason: str = "length"


@dataclass
class RequestOutput:
    request_id: str
    prompt_token_ids: list
    outputs: list = field(default_factory=list)
    finished: bool = True


class NotEligible(RuntimeError):
    """The request batch needs a path this engine does not serve (reason code in .reason)."""

    def __init__(self, reason: str, msg: str):
        super().__init__(f"{reason}: {msg}")
        self.reason = reason


def eligible_batch(prompts, sps, max_seq: int, require_mt1: bool = True):
    """(bs, seq) iff the batch is one uniform fresh prefill the fast path serves, else NotEligible with
    the reference's reason code.  Every prompt here is a fresh, whole-prompt prefill (no KV cache
    exists), so `continuation` and `partial_prefill` cannot occur; the same decision function serves
    the vLLM runner hook (dispatch.eligible_step)."""
    lens = [len(p) for p in prompts]
    view = StepView(scheduled=lens, num_computed=[0] * len(lens), num_prompt=lens, sampling_params=list(sps),
                    prompt_logprobs=[getattr(sp, "prompt_logprobs", None) is not None for sp in sps])
    batch, reason = eligible_step(view, max_seq, require_mt1)
    if batch is None:
        raise NotEligible(reason, {"ragged": f"prompt lengths {sorted(set(lens))} differ",
                                   "max_tokens": "only max_tokens == 1 requests are served",
                                   "unsupported_sampling_feature": "sampling feature outside the fast path",
                                   "seq": f"seq {lens[0] if lens else 0} not served (multiple of 128, of 1024 above "
                                          f"1024, <= {max_seq})"}.get(reason, reason))
    return batch


class MkEngine:
    def __init__(self, model="1b", quant: str = "auto", state_dict: dict | None = None, weight_seed: int = 0,
                 max_model_len: int = 8256, device: str = "cuda:0", log=print, precompile: str | None = None):
        t0 = time.perf_counter()
        if isinstance(model, str) and os.path.isdir(model):   # local HF checkpoint directory
            from .checkpoint import load_local_checkpoint
            model, state_dict = load_local_checkpoint(model)
        self.cfg = preset(model) if isinstance(model, str) else model
        self.cfg.validate()
        cfg = self.cfg
        self.log = log
        self.device = torch.device(device)
        self.max_seq = max_model_len
        self.quant, _ = resolve_quant_pair(quant, cfg.num_layers, 1, cfg.hidden, cfg.inter)
        if state_dict is None:
            from .synth import random_hf_state_dict
            state_dict = random_hf_state_dict(cfg, seed=weight_seed)
        dev = self.device
        w = prepare_mk_weights(state_dict, cfg.as_mk_cfg(), self.quant, max_model_len, cfg.bos_token_id, log=log,
                               device=dev if dev.type == "cuda" else None)
        self.weights = {k: w[k].to(dev) for k in WEIGHT_ORDER}
        self.cos, self.sin = w["cos"].to(dev), w["sin"].to(dev)
        self.embed = state_dict["model.embed_tokens.weight"].to(BF16).to(dev)
        self.final_norm = state_dict["model.norm.weight"].to(BF16).to(dev)
        lm = state_dict.get("lm_head.weight", state_dict["model.embed_tokens.weight"])
        self.lm_head = lm.to(BF16).to(dev)
        self.model = MkModel(self.weights, self.embed, self.cos, self.sin, self.final_norm, self.quant, cfg.n_q,
                             cfg.n_kv, cfg.head_dim, cfg.eps, lm_head=self.lm_head)
        self.counts = {"mk": 0}
        self.status = {"arch": "MiniCPM5MegakernelForCausalLM", "quant": self.quant, "config": cfg.as_mk_cfg(),
                       "shapes": {}}
        log(f"[mk] engine ready ({cfg.name}, quant={self.quant}) in {time.perf_counter() - t0:.1f}s")
        # per-shape graphs at load time (MINICPM5_MK_PRECOMPILE="1x8192,4x8192", model.py:690-698)
        pre = os.environ.get("MINICPM5_MK_PRECOMPILE", "") if precompile is None else precompile
        shapes = parse_precompile(pre)
        for _, s in shapes:
            if not mk_seq_ok(s, self.max_seq):
                raise NotEligible("seq", f"precompile seq {s} not served")
        self.model.precompile(shapes, logits=True, log=log)

    # ------------------------------------------------------------------ scoring
    @torch.no_grad()
    def logits(self, ids: torch.Tensor) -> torch.Tensor:
        """ids (B, S) -> last-position logits (B, V) f32 (the timed prefill step)."""
        B, S = ids.shape
        if not mk_seq_ok(S, self.max_seq):
            raise NotEligible("seq", f"seq {S} not served")
        ids = ids.to(self.device, non_blocking=True)
        key = f"mk:{B}x{S}"
        self.counts["mk"] += 1
        self.counts[key] = self.counts.get(key, 0) + 1
        self.status["shapes"].setdefault(key, {"mode": "single", "quant": self.quant})
        _, lg = self.model.forward(ids.reshape(-1), B, S, logits=True, copy_out=False)
        return lg

    # ------------------------------------------------------------------ vLLM-like generate
    @torch.no_grad()
    def generate(self, prompts, sampling_params=None, use_tqdm: bool = False):
        ps = [p["prompt_token_ids"] if isinstance(p, dict) else list(p) for p in prompts]
        sps = sampling_params if isinstance(sampling_params, (list, tuple)) else [sampling_params or SamplingParams()] * len(ps)
        bs, seq = eligible_batch(ps, sps, self.max_seq)
        ids = torch.tensor(ps, dtype=torch.int32)
        lg = self.logits(ids).clone()
        outs = []
        for b in range(bs):
            sp = sps[b]
            row = lg[b]
            tok = self._sample(row, sp, b)
            lps = None
            if sp.logprobs:
                lp = torch.log_softmax(row, -1)
                top = torch.topk(lp, int(sp.logprobs))
                lps = [{int(i): float(v) for i, v in zip(top.indices.tolist(), top.values.tolist())}]
                lps[0].setdefault(tok, float(lp[tok]))
            outs.append(RequestOutput(str(b), ps[b], [CompletionOutput(0, [tok], lps)]))
        return outs

    @staticmethod
    def _sample(row: torch.Tensor, sp: SamplingParams, b: int) -> int:
        if not sp.temperature or sp.temperature <= 0:
            return int(torch.argmax(row))
        x = row.float() / sp.temperature
        if sp.top_k and sp.top_k > 0:
            kth = torch.topk(x, min(sp.top_k, x.numel())).values[-1]
            x = torch.where(x < kth, torch.full_like(x, float("-inf")), x)
        p = torch.softmax(x, -1)
        if sp.top_p < 1.0:
            srt, idx = torch.sort(p, descending=True)
            keep = torch.cumsum(srt, 0) - srt < sp.top_p
            p = torch.zeros_like(p).scatter_(0, idx[keep], srt[keep])
            p = p / p.sum()
        g = torch.Generator(device=p.device)
        g.manual_seed(sp.seed if sp.seed is not None else b)
        return int(torch.multinomial(p, 1, generator=g))

    def close(self):
        self.model.close()


__all__ = ["MkEngine", "SamplingParams", "RequestOutput", "CompletionOutput", "NotEligible", "mk_seq_ok",
           "eligible_batch"]
