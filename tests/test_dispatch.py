"""Fast-path eligibility and row hand-back (minicpm5_mk.dispatch, minicpm5_mk.model), on the CPU.

The decision mirrors the reference's `_eligible_batch` (plugin/minicpm5_mk/model.py:139-169): reason
codes ragged, continuation, partial_prefill, max_tokens, unsupported_sampling_feature, checked in that
order, plus the length rule `_mk_seq_ok` (:131-136).  The vLLM model class is exercised with test
doubles for vLLM's LlamaForCausalLM and GPU model runner (vLLM is not installed here): a step the
runner hook marks eligible goes to libmk's model object, every other step to the stock forward.
"""
import sys
import types
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from minicpm5_mk.dispatch import (STATE, StepView, eligible_step, install_runner_hook, mk_seq_ok, positions_match,
                                  scatter_last_rows, step_view_from_runner)
from minicpm5_mk.engine import SamplingParams

SP1 = SamplingParams(max_tokens=1)


def view(sched, computed=None, prompt=None, sps=None, plp=None):
    n = len(sched)
    return StepView(sched, computed if computed is not None else [0] * n, prompt if prompt is not None else list(sched),
                    sps if sps is not None else [SP1] * n, plp if plp is not None else [False] * n)


def test_eligible_and_reason_codes():
    assert eligible_step(view([8192] * 4), 8256) == ((4, 8192), "ok")
    assert eligible_step(view([1024]), 8256) == ((1, 1024), "ok")
    assert eligible_step(view([]), 8256) == (None, "ragged")
    assert eligible_step(view([8192, 4096]), 8256) == (None, "ragged")
    assert eligible_step(view([8192, 8192], computed=[0, 5]), 8256) == (None, "continuation")
    # chunked prefill: the first 2048-token chunk of a 10k prompt is not the whole prompt
    assert eligible_step(view([2048], prompt=[10240]), 16384) == (None, "partial_prefill")
    assert eligible_step(view([8192, 8192], sps=[SP1, SamplingParams(max_tokens=16)]), 8256) == (None, "max_tokens")
    assert eligible_step(view([8192], sps=[None]), 8256) == (None, "max_tokens")
    assert eligible_step(view([8192], sps=[SamplingParams(max_tokens=16)]), 8256, require_mt1=False) == ((1, 8192), "ok")
    assert eligible_step(view([8192], sps=[SamplingParams(repetition_penalty=1.1)]), 8256) == \
        (None, "unsupported_sampling_feature")
    assert eligible_step(view([8192], plp=[True]), 8256) == (None, "unsupported_sampling_feature")
    assert eligible_step(view([1000]), 8256) == (None, "seq")            # not a multiple of 128
    assert eligible_step(view([1152]), 8256) == (None, "seq")            # above 1024: multiple of 1024 only
    assert eligible_step(view([9216]), 8256) == (None, "seq")            # above max_seq


def test_reason_order_follows_reference():
    """A step that is both a continuation and max_tokens > 1 (decode) reports continuation first."""
    v = view([1, 1], computed=[8192, 8192], prompt=[8192, 8192], sps=[SamplingParams(max_tokens=16)] * 2)
    assert eligible_step(v, 8256) == (None, "continuation")
    v = view([8192, 8192], computed=[8192, 8192], sps=[SamplingParams(max_tokens=16)] * 2)
    assert eligible_step(v, 8256) == (None, "continuation")


def test_mk_seq_ok_rule():
    assert [mk_seq_ok(s, 8256) for s in (128, 384, 896, 1024, 1152, 2048, 3072, 8192, 9216, 0, -128)] == \
        [True, True, True, True, False, True, True, True, False, False, False]


def _fake_runner(req_ids, computed, prompt, sched, sps, plp=()):
    n = len(req_ids)
    ib = SimpleNamespace(num_reqs=n, req_ids=list(req_ids) + ["stale"],
                         num_computed_tokens_cpu=np.array(list(computed) + [7], dtype=np.int32),
                         num_prompt_tokens=np.array(list(prompt) + [3], dtype=np.int32))
    runner = SimpleNamespace(input_batch=ib, requests={r: SimpleNamespace(sampling_params=sp) for r, sp in zip(req_ids, sps)},
                             num_prompt_logprobs={r: 5 for r in plp})
    so = SimpleNamespace(num_scheduled_tokens=dict(zip(req_ids, sched)))
    return runner, so


def test_step_view_from_runner():
    runner, so = _fake_runner(["a", "b"], [0, 0], [8192, 8192], [8192, 8192], [SP1, SP1], plp=["b"])
    v = step_view_from_runner(runner, so)
    assert v.scheduled == [8192, 8192] and v.num_computed == [0, 0] and v.num_prompt == [8192, 8192]
    assert v.prompt_logprobs == [False, True]
    assert eligible_step(v, 8256) == (None, "unsupported_sampling_feature")
    runner, so = _fake_runner(["a", "b"], [0, 0], [8192, 8192], [8192, 8192], [SP1, SP1])
    assert eligible_step(step_view_from_runner(runner, so), 8256) == ((2, 8192), "ok")


def test_runner_hook_records_decision():
    calls = []

    class Runner:
        def _prepare_inputs(self, scheduler_output):
            calls.append("prep")
            return "prepared"

        def _dummy_run(self, n):
            calls.append("dummy")
            return n

    runner, so = _fake_runner(["a"], [0], [4096], [4096], [SP1])
    r = Runner()
    r.__dict__.update(runner.__dict__)
    assert install_runner_hook(Runner, lambda rr: 8256) and install_runner_hook(Runner, lambda rr: 8256)
    assert r._prepare_inputs(so) == "prepared" and calls == ["prep"]       # wrapped once
    assert STATE.take() == ((1, 4096), "ok")
    assert STATE.take() == (None, "ok")                                    # one forward per decision
    r.input_batch.num_computed_tokens_cpu[0] = 4096
    r._prepare_inputs(so)
    assert STATE.take() == (None, "continuation")
    r._dummy_run(8)
    assert STATE.take() == (None, "dummy")
    # a runner layout the hook cannot read falls back to the stock path with a reason
    bad = Runner()
    bad._prepare_inputs(SimpleNamespace())
    b, reason = STATE.take()
    assert b is None and reason.startswith("check_error")


def test_scatter_last_rows_and_positions():
    rows = torch.arange(8 * 4, dtype=torch.float32).view(8, 4)            # (max(8, B), H) with B = 3
    out = scatter_last_rows(rows, 3, 5, 17)
    assert out.shape == (17, 4)
    want = torch.zeros(17, 4)
    for b in range(3):
        want[b * 5 + 4] = rows[b]
    assert torch.equal(out, want)
    with pytest.raises(ValueError):
        scatter_last_rows(rows, 4, 5, 17)
    pos = torch.arange(5).repeat(3)
    assert positions_match(pos, 3, 5) and not positions_match(pos, 5, 3) and not positions_match(pos, 4, 5)
    assert positions_match(torch.cat([pos, torch.zeros(2, dtype=pos.dtype)]), 3, 5)


@pytest.fixture
def fake_vllm(monkeypatch):
    """Minimal stand-ins for the two vLLM classes minicpm5_mk.model touches (test doubles)."""
    class LlamaForCausalLM(torch.nn.Module):
        def __init__(self, *, vllm_config, prefix=""):
            super().__init__()
            self.stock_calls = 0
            hf = vllm_config.model_config.hf_config
            self.model = torch.nn.Module()
            self.model.embed_tokens = torch.nn.Embedding(8, hf.hidden_size).to(torch.bfloat16)
            self.model.layers = torch.nn.ModuleList([torch.nn.Linear(4, 4) for _ in range(hf.num_hidden_layers)])
            self.lm_head = torch.nn.Linear(4, 4)

        def load_weights(self, weights):
            return {name for name, _ in weights}

        def forward(self, input_ids, positions, intermediate_tensors=None, inputs_embeds=None):
            self.stock_calls += 1
            return "stock"

    class GPUModelRunner:
        def _prepare_inputs(self, scheduler_output):
            return None

    mods = {
        "vllm": types.ModuleType("vllm"),
        "vllm.model_executor": types.ModuleType("vllm.model_executor"),
        "vllm.model_executor.models": types.ModuleType("vllm.model_executor.models"),
        "vllm.model_executor.models.llama": types.ModuleType("vllm.model_executor.models.llama"),
        "vllm.v1": types.ModuleType("vllm.v1"),
        "vllm.v1.worker": types.ModuleType("vllm.v1.worker"),
        "vllm.v1.worker.gpu_model_runner": types.ModuleType("vllm.v1.worker.gpu_model_runner"),
    }
    mods["vllm.model_executor.models.llama"].LlamaForCausalLM = LlamaForCausalLM
    mods["vllm.v1.worker.gpu_model_runner"].GPUModelRunner = GPUModelRunner
    for k, m in mods.items():
        monkeypatch.setitem(sys.modules, k, m)
    monkeypatch.delitem(sys.modules, "minicpm5_mk.model", raising=False)
    import minicpm5_mk.model as model_mod
    yield model_mod, GPUModelRunner
    sys.modules.pop("minicpm5_mk.model", None)


def test_model_class_dispatch(fake_vllm):
    model_mod, Runner = fake_vllm
    hf = dict(hidden_size=256, num_attention_heads=16, num_key_value_heads=2, head_dim=64, num_hidden_layers=3,
              intermediate_size=768, vocab_size=32768, rms_norm_eps=1e-6, rope_theta=1e4)
    cfg = SimpleNamespace(model_config=SimpleNamespace(hf_config=SimpleNamespace(**hf), max_model_len=8256),
                          parallel_config=SimpleNamespace(pipeline_parallel_size=1, tensor_parallel_size=1))
    m = model_mod.MiniCPM5MegakernelForCausalLM(vllm_config=cfg)
    assert m._mk_enabled and getattr(Runner, "_minicpm5_mk_hooked", False)

    class FakeMk:
        quant = "int8d"

        def __init__(self):
            self.calls = []

        def forward(self, ids, bs, seq):
            self.calls.append((ids.dtype, ids.numel(), bs, seq))
            return torch.arange(8 * 4, dtype=torch.float32).view(8, 4) + 1

    m._mk_model, m._mk_status = FakeMk(), {"shapes": {}}
    ids = torch.arange(2 * 128 + 16)                                         # padded: T_pad > bs * seq
    pos = torch.cat([torch.arange(128).repeat(2), torch.zeros(16, dtype=torch.long)])
    STATE.set((2, 128), "ok")
    out = m(ids, pos)
    assert m._mk_model.calls == [(torch.int32, 256, 2, 128)]
    assert out.shape == (272, 4) and torch.equal(out[127], torch.arange(4.0) + 1) and torch.equal(out[255], torch.arange(4.0) + 5)
    assert float(out.abs().sum()) == float(out[127].sum() + out[255].sum())
    STATE.set(None, "continuation")
    assert m(ids, pos) == "stock" and m._mk_counts["stock:continuation"] == 1
    assert m(ids, pos) == "stock"                                            # no decision recorded: stock
    STATE.set((4, 128), "ok")                                                # more tokens than the step holds
    assert m(ids, pos) == "stock"
    assert m._mk_counts["mk"] == 1 and m._mk_counts["mk:2x128"] == 1


HF_TINY = dict(hidden_size=256, num_attention_heads=16, num_key_value_heads=2, head_dim=64, num_hidden_layers=3,
               intermediate_size=768, vocab_size=32768, rms_norm_eps=1e-6, rope_theta=1e4)


def _vllm_cfg(max_len=8256, prefix_caching=False):
    return SimpleNamespace(model_config=SimpleNamespace(hf_config=SimpleNamespace(**HF_TINY), max_model_len=max_len),
                           parallel_config=SimpleNamespace(pipeline_parallel_size=1, tensor_parallel_size=1),
                           cache_config=SimpleNamespace(enable_prefix_caching=prefix_caching))


class _FakeMkModel:
    """Stands in for runtime.MkModel (libmk needs a GPU): records the calls, returns (max(8, B), H) rows."""
    quant = "int8d"

    def __init__(self, *args, **kwargs):
        self.calls = []

    def forward(self, ids, bs, seq):
        self.calls.append((bs, seq))
        return torch.ones(max(8, bs), HF_TINY["hidden_size"], dtype=torch.bfloat16)

    def precompile(self, shapes, logits=False, log=None):
        pass


def _load(m, model_mod, monkeypatch):
    """load_weights with the weight preparation and the device model replaced by doubles."""
    from minicpm5_mk.runtime import WEIGHT_ORDER
    monkeypatch.setattr(model_mod, "MkModel", _FakeMkModel)
    monkeypatch.setattr(model_mod, "prepare_mk_weights",
                        lambda *a, **k: {**{n: torch.zeros(1) for n in WEIGHT_ORDER}, "cos": torch.zeros(1),
                                         "sin": torch.zeros(1)})
    H = HF_TINY["hidden_size"]
    names = [("model.embed_tokens.weight", torch.zeros(8, H)), ("model.norm.weight", torch.ones(H)),
             ("model.layers.0.mlp.down_proj.weight", torch.zeros(H, 4))]
    return m.load_weights(iter(names))


def test_stock_freed_mode_and_status(fake_vllm, monkeypatch, tmp_path):
    """MINICPM5_MK_FREE_STOCK=1 (plugin/minicpm5_mk/model.py:700-705, :787-794): the stock decoder
    weights are dropped after the build, a dummy run returns zeros, any other ineligible step raises;
    the status file carries the reference's keys (:683-689) and the stock reasons (:777-785)."""
    import json
    model_mod, _ = fake_vllm
    monkeypatch.setenv("MINICPM5_MK_FREE_STOCK", "1")
    monkeypatch.setenv("MINICPM5_MK_STATUS_DIR", str(tmp_path))
    m = model_mod.MiniCPM5MegakernelForCausalLM(vllm_config=_vllm_cfg())
    assert m._mk_enabled
    assert _load(m, model_mod, monkeypatch) >= {"model.norm.weight"}
    assert m._mk_stock_freed and all(p.numel() == 0 for p in m.model.layers.parameters())
    st = json.loads((tmp_path / "minicpm5_mk_status_rank0.json").read_text())
    assert st["stock_freed"] is True and st["tp"] == 1 and st["rank"] == 0 and st["multicore_modes"] == []
    assert st["quant"] == st["quant_tp"] and st["shapes"] == {} and "stock_reasons" not in st
    ids, pos = torch.arange(2 * 128), torch.arange(128).repeat(2)
    STATE.set((2, 128), "ok")
    out = m(ids, pos)
    assert out.shape == (256, HF_TINY["hidden_size"]) and m._mk_model.calls == [(2, 128)]
    STATE.set(None, "dummy")
    z = m(ids, pos)
    assert z.dtype == torch.bfloat16 and z.shape == (256, HF_TINY["hidden_size"]) and not z.any()
    STATE.set(None, "continuation")
    with pytest.raises(RuntimeError, match="stock weights were freed"):
        m(ids, pos)
    st = json.loads((tmp_path / "minicpm5_mk_status_rank0.json").read_text())
    assert st["shapes"] == {"mk:2x128": {"mode": "single", "quant": "int8d"}}
    assert st["stock_reasons"] == ["continuation"]                       # dummy runs are not recorded
    assert m._mk_counts["stock:dummy"] == 1 and m._mk_counts["stock:continuation"] == 1


def test_stock_path_kept_without_free_stock(fake_vllm, monkeypatch, tmp_path, caplog):
    import json
    import logging
    model_mod, _ = fake_vllm
    monkeypatch.delenv("MINICPM5_MK_FREE_STOCK", raising=False)
    monkeypatch.setenv("MINICPM5_MK_STATUS_DIR", str(tmp_path))
    monkeypatch.setenv("MINICPM5_MK_LOG_EVERY", "2")
    m = model_mod.MiniCPM5MegakernelForCausalLM(vllm_config=_vllm_cfg())
    _load(m, model_mod, monkeypatch)
    assert not m._mk_stock_freed and all(p.numel() > 0 for p in m.model.layers.parameters())
    ids, pos = torch.arange(256), torch.arange(128).repeat(2)
    with caplog.at_level(logging.INFO, logger="vllm.minicpm5_mk"):
        for reason in ("max_tokens", "max_tokens", "ragged"):
            STATE.set(None, reason)
            assert m(ids, pos) == "stock"
    st = json.loads((tmp_path / "minicpm5_mk_status_rank0.json").read_text())
    assert st["stock_freed"] is False and st["stock_reasons"] == ["max_tokens", "ragged"]
    assert m._mk_counts["stock"] == 3 and m._mk_counts["stock:max_tokens"] == 2
    assert sum("counts=" in r.getMessage() for r in caplog.records) == 1    # every 2nd forward


def test_prefix_caching_turns_fast_path_off(fake_vllm, monkeypatch):
    """A fast-path prefill writes no KV cache, so with prefix caching a later request sharing its
    prefix would read unwritten blocks on the stock path: the fast path is off, and megakernel-only
    mode refuses to start."""
    model_mod, _ = fake_vllm
    monkeypatch.delenv("MINICPM5_MK_FREE_STOCK", raising=False)
    m = model_mod.MiniCPM5MegakernelForCausalLM(vllm_config=_vllm_cfg(prefix_caching=True))
    assert not m._mk_enabled
    monkeypatch.setenv("MINICPM5_MK_FREE_STOCK", "1")
    with pytest.raises(RuntimeError, match="prefix caching"):
        model_mod.MiniCPM5MegakernelForCausalLM(vllm_config=_vllm_cfg(prefix_caching=True))


def test_free_stock_refuses_a_disabled_fast_path(fake_vllm, monkeypatch):
    """Megakernel-only mode lets the engine skip KV allocation, so a model whose fast path is off for
    any reason (here: tensor parallelism, unsupported rope scaling) must not start in that mode; with
    MINICPM5_MK_ENABLE=0 the KV skip is off as well and the stock model starts normally."""
    model_mod, _ = fake_vllm
    monkeypatch.setenv("MINICPM5_MK_FREE_STOCK", "1")
    cfg = _vllm_cfg()
    cfg.parallel_config.tensor_parallel_size = 2
    with pytest.raises(RuntimeError, match="PP / TP"):
        model_mod.MiniCPM5MegakernelForCausalLM(vllm_config=cfg)
    cfg = _vllm_cfg()
    cfg.model_config.hf_config.rope_scaling = {"rope_type": "yarn", "factor": 4.0}
    with pytest.raises(RuntimeError, match="rope_scaling"):
        model_mod.MiniCPM5MegakernelForCausalLM(vllm_config=cfg)
    monkeypatch.setenv("MINICPM5_MK_ENABLE", "0")
    m = model_mod.MiniCPM5MegakernelForCausalLM(vllm_config=cfg)
    assert not m._mk_enabled
    monkeypatch.delenv("MINICPM5_MK_FREE_STOCK")
    monkeypatch.delenv("MINICPM5_MK_ENABLE")
    m = model_mod.MiniCPM5MegakernelForCausalLM(vllm_config=cfg)   # stock-capable: warns, keeps stock
    assert not m._mk_enabled


def test_runner_hook_follows_latest_model(fake_vllm):
    """A model built after an earlier one was freed re-points the runner hook at itself."""
    import gc
    model_mod, Runner = fake_vllm
    a = model_mod.MiniCPM5MegakernelForCausalLM(vllm_config=_vllm_cfg(max_len=8256))
    del a
    gc.collect()
    b = model_mod.MiniCPM5MegakernelForCausalLM(vllm_config=_vllm_cfg(max_len=16384))
    runner, so = _fake_runner(["a"], [0], [16384], [16384], [SP1])
    r = Runner()
    r.__dict__.update(runner.__dict__)
    r._prepare_inputs(so)
    assert STATE.take() == ((1, 16384), "ok")
    assert b._mk_max_seq == 16384


class _FakeEngineCore:
    def __init__(self, vllm_config):
        self.vllm_config = vllm_config


class _FakeKVManager:
    empty_kv_cache_blocks = "EMPTY"

    def allocate_slots(self, request, num_new_tokens, *args, **kwargs):
        return "BLOCKS"


def _req(seq=8192, computed=0, sp=SP1):
    return SimpleNamespace(num_prompt_tokens=seq, num_computed_tokens=computed, sampling_params=sp)


def test_kv_alloc_skip(monkeypatch):
    """KV-allocation skip (plugin/minicpm5_mk/__init__.py:154-206): only in megakernel-only mode, only for
    an engine serving the architecture without prefix caching, only for full fresh max_tokens=1 prefills
    with fast-path sampling and a served length; every other request gets vLLM's allocation."""
    import minicpm5_mk as pkg
    monkeypatch.setattr(pkg, "ENGINE_SERVES_ARCH", {"active": False, "prefix_caching": False, "max_model_len": 0})

    class Core(_FakeEngineCore):
        pass

    class KV(_FakeKVManager):
        pass

    pkg.install_kv_skip(Core, KV)
    pkg.install_kv_skip(Core, KV)                                           # idempotent
    mc = SimpleNamespace(architectures=[pkg.ARCH], hf_config=SimpleNamespace(architectures=[]), max_model_len=8256)
    cfg = SimpleNamespace(model_config=mc, cache_config=SimpleNamespace(enable_prefix_caching=False))
    Core(cfg)
    kv = KV()
    monkeypatch.delenv("MINICPM5_MK_FREE_STOCK", raising=False)
    assert kv.allocate_slots(_req(), 8192) == "BLOCKS"                      # stock path may run: allocate
    monkeypatch.setenv("MINICPM5_MK_FREE_STOCK", "1")
    assert kv.allocate_slots(_req(), 8192) == "EMPTY"
    assert kv.allocate_slots(_req(1024), 1024) == "EMPTY"
    assert kv.allocate_slots(_req(384), 384) == "EMPTY"
    assert kv.allocate_slots(_req(), 2048) == "BLOCKS"                      # chunked prefill
    assert kv.allocate_slots(_req(computed=8192), 1) == "BLOCKS"           # continuation / decode
    assert kv.allocate_slots(_req(sp=SamplingParams(max_tokens=4)), 8192) == "BLOCKS"
    assert kv.allocate_slots(_req(sp=None), 8192) == "BLOCKS"
    assert kv.allocate_slots(_req(sp=SamplingParams(max_tokens=1, repetition_penalty=1.2)), 8192) == "BLOCKS"
    assert kv.allocate_slots(_req(1000), 1000) == "BLOCKS"                 # length not served
    assert kv.allocate_slots(_req(1152), 1152) == "BLOCKS"
    assert kv.allocate_slots(_req(16384), 16384) == "BLOCKS"               # beyond the engine's max length
    monkeypatch.setenv("MINICPM5_MK_ENABLE", "0")
    assert kv.allocate_slots(_req(), 8192) == "BLOCKS"
    monkeypatch.delenv("MINICPM5_MK_ENABLE")
    Core(SimpleNamespace(model_config=mc, cache_config=SimpleNamespace(enable_prefix_caching=True)))
    assert kv.allocate_slots(_req(), 8192) == "BLOCKS"                      # prefix caching: never skip
    other = SimpleNamespace(architectures=["LlamaForCausalLM"], hf_config=SimpleNamespace(architectures=[]),
                            max_model_len=8256)
    Core(SimpleNamespace(model_config=other, cache_config=SimpleNamespace(enable_prefix_caching=False)))
    assert kv.allocate_slots(_req(), 8192) == "BLOCKS"                      # another model's engine
    Core(SimpleNamespace(model_config=SimpleNamespace(architectures=None,
                                                      hf_config=SimpleNamespace(architectures=[pkg.ARCH]),
                                                      max_model_len=8256), cache_config=None))
    assert kv.allocate_slots(_req(), 8192) == "EMPTY"                       # architecture from the HF config


def test_single_step_batch_queue():
    """Scoring batches run as one step when the batch queue is deeper than one
    (plugin/minicpm5_mk/__init__.py:208-245)."""
    import minicpm5_mk as pkg

    class Core:
        def __init__(self, waiting, running=(), bq=(), bq_size=2):
            self.batch_queue = list(bq)
            self.batch_queue_size = bq_size
            self.scheduler = SimpleNamespace(waiting=list(waiting), running=list(running), max_num_running_reqs=4,
                                             max_num_scheduled_tokens=32768)
            self.seen = []

        def step_with_batch_queue(self):
            self.seen.append(self.batch_queue_size)
            return "stepped"

    pkg.install_single_step(Core)
    pkg.install_single_step(Core)
    four = [_req() for _ in range(4)]
    c = Core(four)
    assert c.step_with_batch_queue() == "stepped" and c.seen == [1] and c.batch_queue_size == 2
    for core in (Core(four + [_req()]),                                      # more than max running
                 Core([_req(), _req(sp=SamplingParams(max_tokens=2))]),     # not all scoring
                 Core([_req(16384), _req(16384), _req(16384)]),             # over the token budget
                 Core(four, running=[1]), Core(four, bq=[1]), Core(four, bq_size=1), Core([])):
        core.step_with_batch_queue()
        assert core.seen == [core.batch_queue_size]
