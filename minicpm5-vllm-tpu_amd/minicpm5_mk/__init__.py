"""minicpm5_mk -- MI355X-native MiniCPM5 prefill/scoring fast path (drop-in for the vLLM plugin).

Same package name, architecture name and entry point as the reference plugin
(plugin/minicpm5_mk/__init__.py, plugin/pyproject.toml:16-17):
  [vllm.general_plugins] minicpm5_mk = minicpm5_mk:register
The device program is libmk.so (hand-written HIP for gfx950) behind include/mk.h.
"""

ARCH = "MiniCPM5MegakernelForCausalLM"

# Set in the engine-core process when that engine serves ARCH (kept for interface parity).
ENGINE_SERVES_ARCH = {"active": False}


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


def register() -> None:
    """Entry point of the `vllm.general_plugins` group: registers ARCH with vLLM's ModelRegistry
    (plugin/minicpm5_mk/__init__.py:35-42).  Needs vLLM; the TPU front-end patches of the reference
    (:47-245) are TorchTPU internals and have no counterpart here."""
    from vllm import ModelRegistry

    if ARCH not in ModelRegistry.get_supported_archs():
        ModelRegistry.register_model(ARCH, "minicpm5_mk.model:MiniCPM5MegakernelForCausalLM")
