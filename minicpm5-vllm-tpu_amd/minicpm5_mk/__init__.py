"""minicpm5_mk -- MI355X-native MiniCPM5 prefill/scoring fast path (drop-in for the vLLM plugin).

Same package name, architecture name and entry point as the reference plugin
(plugin/minicpm5_mk/__init__.py, plugin/pyproject.toml:16-17):
  [vllm.general_plugins] minicpm5_mk = minicpm5_mk:register
The device program is libmk.so (hand-written HIP for gfx950) behind include/mk.h.
"""

ARCH = "MiniCPM5MegakernelForCausalLM"

# Set in the engine-core (scheduler) process when that engine serves ARCH; read by the KV-skip hook.
# "prefix_caching" and "max_model_len" are that engine's settings.
ENGINE_SERVES_ARCH = {"active": False, "prefix_caching": False, "max_model_len": 0}


def sampling_fast_ok(sp) -> bool:
    """True iff a request's SamplingParams only use features the fast path implements
    (plugin/minicpm5_mk/__init__.py:10-32): temperature / top-p / top-k / seed / logprobs / min_tokens.
    Prompt logprobs, penalties, min_p, logit bias, allowed or bad words, structured output and custom
    logits processors need the stock path."""
    if sp is None:
        return False
    g = getattr
    if g(sp, "prompt_logprobs", None) is not None:
        return False
    if (g(sp, "presence_penalty", 0.0) or 0.0) != 0.0 or (g(sp, "frequency_penalty", 0.0) or 0.0) != 0.0:
        return False
    if (g(sp, "repetition_penalty", 1.0) or 1.0) != 1.0 or (g(sp, "min_p", 0.0) or 0.0) != 0.0:
        return False
    if g(sp, "logit_bias", None) or g(sp, "allowed_token_ids", None) or g(sp, "bad_words", None):
        return False
    if g(sp, "structured_outputs", None) is not None or g(sp, "guided_decoding", None) is not None:
        return False
    if g(sp, "logits_processors", None):
        return False
    return True


def kv_alloc_skippable(request, num_new_tokens: int) -> bool:
    """True iff the scheduler may give `request` no KV-cache blocks (plugin/minicpm5_mk/__init__.py:
    154-206): the engine in this process serves ARCH, megakernel-only mode is on
    (MINICPM5_MK_FREE_STOCK=1: an ineligible step raises instead of running stock attention over KV
    that was never written), prefix caching is off, and the request is a full, fresh, max_tokens == 1
    prefill with fast-path sampling whose length the fast path serves.  A fast-path prefill never reads
    or writes its KV cache, so the blocks would be allocated for nothing."""
    import os

    from .dispatch import mk_seq_ok

    sp = request.sampling_params
    if not (ENGINE_SERVES_ARCH["active"] and os.environ.get("MINICPM5_MK_ENABLE", "1") != "0"
            and os.environ.get("MINICPM5_MK_FREE_STOCK", "0") == "1"):
        return False
    if ENGINE_SERVES_ARCH.get("prefix_caching"):
        return False
    if request.num_computed_tokens != 0 or sp is None or sp.max_tokens != 1:
        return False
    seq = int(request.num_prompt_tokens)
    if num_new_tokens != seq or not sampling_fast_ok(sp):
        return False
    return mk_seq_ok(seq, ENGINE_SERVES_ARCH.get("max_model_len") or seq)


def install_kv_skip(engine_core_cls, kv_cache_manager_cls) -> None:
    """Hook vLLM v1's engine core and KV-cache manager for the KV-allocation skip (idempotent).
    `EngineCore.__init__` records whether this engine serves ARCH (and its prefix-caching and length
    settings); `KVCacheManager.allocate_slots` returns the manager's empty block set for requests that
    `kv_alloc_skippable` admits and defers to vLLM for every other request."""
    import functools

    if not getattr(engine_core_cls, "_minicpm5_arch_hooked", False):
        orig_init = engine_core_cls.__init__

        @functools.wraps(orig_init)
        def _core_init(self, vllm_config, *args, **kwargs):
            try:
                mc = vllm_config.model_config
                archs = list(getattr(mc, "architectures", None) or []) + list(
                    getattr(mc.hf_config, "architectures", None) or [])
                ENGINE_SERVES_ARCH["active"] = ARCH in archs
                cc = getattr(vllm_config, "cache_config", None)
                ENGINE_SERVES_ARCH["prefix_caching"] = bool(getattr(cc, "enable_prefix_caching", False))
                ENGINE_SERVES_ARCH["max_model_len"] = int(getattr(mc, "max_model_len", 0) or 0)
            except Exception:  # noqa: BLE001  (an engine layout this hook does not know: no skip)
                ENGINE_SERVES_ARCH["active"] = False
            return orig_init(self, vllm_config, *args, **kwargs)

        engine_core_cls.__init__ = _core_init
        engine_core_cls._minicpm5_arch_hooked = True

    if not getattr(kv_cache_manager_cls, "_minicpm5_mt1_hooked", False):
        orig_alloc = kv_cache_manager_cls.allocate_slots

        @functools.wraps(orig_alloc)
        def _allocate_slots(self, request, num_new_tokens, *args, **kwargs):
            if kv_alloc_skippable(request, num_new_tokens):
                if not ENGINE_SERVES_ARCH.get("logged"):
                    ENGINE_SERVES_ARCH["logged"] = True
                    print("[minicpm5_mk] KV-cache allocation skipped for fast-path max_tokens=1 requests "
                          "(MINICPM5_MK_FREE_STOCK=1)", flush=True)
                return self.empty_kv_cache_blocks
            return orig_alloc(self, request, num_new_tokens, *args, **kwargs)

        kv_cache_manager_cls.allocate_slots = _allocate_slots
        kv_cache_manager_cls._minicpm5_mt1_hooked = True


def single_step_ok(core) -> bool:
    """True iff `core` (a vLLM v1 EngineCore) should schedule its waiting requests as one step
    (plugin/minicpm5_mk/__init__.py:208-245): the batch queue is empty, nothing is running, every
    waiting request wants one token and all of them fit one step's token budget.  With a batch queue
    deeper than one, the engine would otherwise split such a scoring batch over several steps, and each
    step would be a smaller fast-path batch."""
    bq = core.batch_queue
    sch = core.scheduler
    if bq is None or bq or core.batch_queue_size <= 1 or sch.running or not sch.waiting:
        return False
    if len(sch.waiting) > sch.max_num_running_reqs:
        return False
    tot = 0
    for r in sch.waiting:
        sp = r.sampling_params
        if sp is None or sp.max_tokens != 1:
            return False
        tot += r.num_prompt_tokens
    return 0 < tot <= sch.max_num_scheduled_tokens


def install_single_step(engine_core_cls) -> None:
    """Hook `EngineCore.step_with_batch_queue` so that `single_step_ok` batches run with a batch queue
    of depth one for that step (idempotent)."""
    import functools

    if getattr(engine_core_cls, "_minicpm5_single_step_hooked", False):
        return
    orig = engine_core_cls.step_with_batch_queue

    @functools.wraps(orig)
    def _step_with_batch_queue(self):
        if single_step_ok(self):
            saved = self.batch_queue_size
            self.batch_queue_size = 1
            try:
                return orig(self)
            finally:
                self.batch_queue_size = saved
        return orig(self)

    engine_core_cls.step_with_batch_queue = _step_with_batch_queue
    engine_core_cls._minicpm5_single_step_hooked = True


def register() -> None:
    """Entry point of the `vllm.general_plugins` group (runs in every vLLM process): registers ARCH
    with vLLM's ModelRegistry (plugin/minicpm5_mk/__init__.py:35-42) and, unless
    MINICPM5_MK_ENABLE=0, installs the KV-allocation skip (:154-206; off with TTVLLM_SKIP_KV_ALLOC_MT1=0)
    and the single-step batch queue for scoring batches (:208-245; off with TTVLLM_SINGLE_STEP_MT1=0),
    the reference's knob names.  The reference's remaining patches (:47-152: request cloning, EOS and
    token-id validation caches, prompt preprocessing) target front-end modules of the TorchTPU vLLM
    build (`vllm.entrypoints.common.offline`, `vllm.renderers`) and have no counterpart here."""
    import os

    from vllm import ModelRegistry

    if ARCH not in ModelRegistry.get_supported_archs():
        ModelRegistry.register_model(ARCH, "minicpm5_mk.model:MiniCPM5MegakernelForCausalLM")
    if os.environ.get("MINICPM5_MK_ENABLE", "1") == "0":
        return
    try:
        from vllm.v1.core.kv_cache_manager import KVCacheManager
        from vllm.v1.engine.core import EngineCore
    except ImportError:
        return
    if os.environ.get("TTVLLM_SKIP_KV_ALLOC_MT1", "1") == "1":
        install_kv_skip(EngineCore, KVCacheManager)
    if os.environ.get("TTVLLM_SINGLE_STEP_MT1", "1") == "1" and hasattr(EngineCore, "step_with_batch_queue"):
        install_single_step(EngineCore)
