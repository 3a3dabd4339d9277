"""Fast-path eligibility and row hand-back, decided from host-side scheduler state (no vLLM import).

The reference decides per scheduler step, on the host, whether the step is one uniform fresh prefill
the device program can serve (`_eligible_batch`, plugin/minicpm5_mk/model.py:139-169, evaluated in a
runner hook before the forward, :362-403).  The decision travels to the model's forward in a small
process-global (`STATE`), so the forward never inspects device tensors (no host sync; safe while the
runner captures decode graphs).  Reason codes, checked in the reference's order:

  ragged                        query lengths of the step differ (or the step is empty)
  continuation                  a request already has computed tokens (chunked prefill, decode)
  partial_prefill               a request's scheduled chunk is not its whole prompt
  max_tokens                    a request wants more than one output token (the fast path writes no
                                KV cache, so decode after it would be wrong)
  unsupported_sampling_feature  prompt logprobs or a sampling feature outside `sampling_fast_ok`
  seq                           the length is outside the served set (`mk_seq_ok`, model.py:131-136)
  dummy                         a profiling / warm-up run of the runner
  ok                            served by libmk

`StepView` is the runner-independent input.  `step_view_from_runner` builds it from a vLLM v1 model
runner and its scheduler output; `install_runner_hook` wraps a runner class so every step records
its decision.  Everything here runs on the CPU and is unit-tested without vLLM.
"""
from __future__ import annotations

import functools
import threading
from dataclasses import dataclass, field
from typing import Sequence

from . import sampling_fast_ok

REASONS = ("ok", "ragged", "continuation", "partial_prefill", "max_tokens", "unsupported_sampling_feature", "seq",
           "dummy", "init")


def mk_seq_ok(seq: int, max_seq: int) -> bool:
    """The reference's fast-path length rule (model.py:131-136): <= 1024 -> multiple of 128, else of
    1024 (libmk itself serves every multiple of 128)."""
    if seq <= 0 or seq > max_seq:
        return False
    return seq % 128 == 0 if seq <= 1024 else seq % 1024 == 0


@dataclass
class StepView:
    """Host facts of one scheduler step, requests in batch order."""
    scheduled: Sequence[int]                    # tokens scheduled this step, per request
    num_computed: Sequence[int]                 # tokens already computed before this step
    num_prompt: Sequence[int]                   # prompt length
    sampling_params: Sequence = field(default_factory=list)
    prompt_logprobs: Sequence[bool] = field(default_factory=list)   # the request asked for prompt logprobs


def eligible_step(view: StepView, max_seq: int, require_mt1: bool = True):
    """((bs, seq), "ok") when the step is one uniform fresh prefill the fast path serves, else
    (None, reason)."""
    n = len(view.scheduled)
    if n == 0:
        return None, "ragged"
    seq = int(view.scheduled[0])
    if seq <= 0 or any(int(s) != seq for s in view.scheduled):
        return None, "ragged"
    if any(int(c) != 0 for c in view.num_computed):
        return None, "continuation"
    if any(int(p) != seq for p in view.num_prompt):
        return None, "partial_prefill"
    plp = list(view.prompt_logprobs) or [False] * n
    for sp, wants_plp in zip(view.sampling_params, plp):
        if require_mt1 and (sp is None or getattr(sp, "max_tokens", None) != 1):
            return None, "max_tokens"
        if not sampling_fast_ok(sp) or wants_plp:
            return None, "unsupported_sampling_feature"
    if not mk_seq_ok(seq, max_seq):
        return None, "seq"
    return (n, seq), "ok"


class StepState(threading.local):
    """The decision for the forward that follows the current input preparation (one engine thread)."""

    def __init__(self):
        self.batch = None
        self.reason = "init"

    def set(self, batch, reason: str) -> None:
        self.batch, self.reason = batch, reason

    def take(self):
        """(batch or None, reason); clears the batch so a decision is used by one forward only."""
        b, self.batch = self.batch, None
        return b, self.reason


STATE = StepState()


def _np_list(x):
    return [int(v) for v in (x.tolist() if hasattr(x, "tolist") else x)]


def step_view_from_runner(runner, scheduler_output) -> StepView:
    """StepView of a vLLM v1 model runner's current step.  Reads the runner's input batch (request
    order, computed / prompt token counts), its request states (sampling params) and its prompt-logprob
    map, and the scheduler output's per-request scheduled token counts."""
    ib = runner.input_batch
    n = int(getattr(ib, "num_reqs", len(ib.req_ids)))
    rids = list(ib.req_ids[:n])
    sched = scheduler_output.num_scheduled_tokens
    reqs = getattr(runner, "requests", {}) or {}
    plp = getattr(runner, "num_prompt_logprobs", None)
    if plp is None:
        plp = getattr(ib, "num_prompt_logprobs", {}) or {}
    return StepView(
        scheduled=[int(sched.get(r, 0)) for r in rids],
        num_computed=_np_list(ib.num_computed_tokens_cpu[:n]),
        num_prompt=_np_list(ib.num_prompt_tokens[:n]),
        sampling_params=[getattr(reqs.get(r), "sampling_params", None) for r in rids],
        prompt_logprobs=[r in plp for r in rids],
    )


# What the installed hook checks against: the most recent install's model length and max_tokens rule.
# The wrapper reads this slot on every step, so a model built after an earlier one was freed (same
# process, same runner class) re-points the hook instead of inheriting the first model's length.
_HOOK_CFG = {"max_seq_of": lambda runner: 0, "require_mt1": True}


def install_runner_hook(runner_cls, max_seq_of, require_mt1: bool = True) -> bool:
    """Wrap `runner_cls._prepare_inputs` (and `_dummy_run` when present) so each step records its
    decision in STATE.  `max_seq_of(runner)` gives the model's max length.  The class is wrapped once;
    every call updates what the wrapper checks against.  Returns False when the class has no
    `_prepare_inputs`."""
    if getattr(runner_cls, "_minicpm5_mk_hooked", False):
        _HOOK_CFG.update(max_seq_of=max_seq_of, require_mt1=require_mt1)
        return True
    orig_prepare = getattr(runner_cls, "_prepare_inputs", None)
    if orig_prepare is None:
        return False
    _HOOK_CFG.update(max_seq_of=max_seq_of, require_mt1=require_mt1)

    @functools.wraps(orig_prepare)
    def _prepare_inputs(self, scheduler_output, *args, **kwargs):
        STATE.set(None, "init")
        out = orig_prepare(self, scheduler_output, *args, **kwargs)
        try:
            batch, reason = eligible_step(step_view_from_runner(self, scheduler_output),
                                          _HOOK_CFG["max_seq_of"](self), _HOOK_CFG["require_mt1"])
        except Exception as e:  # noqa: BLE001  (a runner layout this hook does not know: stock path)
            batch, reason = None, f"check_error:{type(e).__name__}"
        STATE.set(batch, reason)
        return out

    runner_cls._prepare_inputs = _prepare_inputs
    orig_dummy = getattr(runner_cls, "_dummy_run", None)
    if orig_dummy is not None:
        @functools.wraps(orig_dummy)
        def _dummy_run(self, *args, **kwargs):
            STATE.set(None, "dummy")
            return orig_dummy(self, *args, **kwargs)

        runner_cls._dummy_run = _dummy_run
    runner_cls._minicpm5_mk_hooked = True
    return True


def scatter_last_rows(rows, bs: int, seq: int, num_tokens: int):
    """(num_tokens, H) tensor, zero except row b*seq + seq - 1 = rows[b]: the token rows the stock
    logits selection reads (the last position of each sequence), for runners that select hidden
    states themselves (the reference patches that selection instead, model.py:224-235)."""
    import torch

    if bs * seq > num_tokens:
        raise ValueError(f"scatter_last_rows: bs*seq = {bs * seq} > {num_tokens} tokens")
    out = torch.zeros((num_tokens, rows.shape[1]), dtype=rows.dtype, device=rows.device)
    out[seq - 1: bs * seq: seq] = rows[:bs]
    return out


def positions_match(positions, bs: int, seq: int) -> bool:
    """Debug cross-check of a host decision against the device positions (syncs the device):
    positions[:bs*seq] are bs copies of arange(seq)."""
    import torch

    pos = positions.reshape(-1)
    if pos.numel() < bs * seq:
        return False
    want = torch.arange(seq, device=pos.device, dtype=pos.dtype).repeat(bs)
    return bool(torch.equal(pos[: bs * seq], want))
