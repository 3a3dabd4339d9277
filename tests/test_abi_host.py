"""The C ABI (include/mk.h) and the host-side plugin surface, without a GPU.

  * libmk.so loads and exports every function include/mk.h declares;
  * host-only entry points validate like the reference's trace-time asserts and fast-path rules:
    mk_validate / mk_packed_bytes accept the shapes and quant strings the kernels build and reject the rest
    with a message (no GPU call);
  * the packed-weight size matches the layout's arithmetic;
  * sampling_fast_ok / eligible_batch / mk_seq_ok mirror __init__.py:10-32 and model.py:131-169.
"""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "mk.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(mk_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    from minicpm5_mk import _lib

    lib = _lib.load()
    names = _declared()
    assert len(names) >= 15
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures must cover exactly the header"
    assert lib.mk_abi_version() == 1


def _cfg(**kw):
    from minicpm5_mk import _lib

    d = dict(num_layers=24, hidden=1536, inter=4608, n_q=16, n_kv=2, head_dim=128, vocab=130560, eps=1e-6,
             max_seq=8256)
    d.update(kw)
    return _lib.MkConfig(**d)


@pytest.mark.parametrize("kw,quant,bs,seq,code,msg", [
    ({}, b"int8d:qkv+gu|sq|lastbf16|fqkv|fmlp", 1, 8192, 0, ""),
    ({}, b"bf16", 32, 8192, 0, ""),
    ({"head_dim": 96}, b"int8d", 4, 2048, 0, ""),
    ({}, b"fp8d", 1, 8192, 0, ""),
    ({}, b"int8|fmlp", 1, 8192, 0, ""),
    ({}, b"fp8:qkv+o|sq", 1, 8192, 0, ""),
    ({}, b"int4", 1, 8192, -1, "unknown base"),
    ({}, b"int8d:qkv+mlp", 1, 8192, -1, "unknown linear"),
    ({}, b"int8d|fast", 1, 8192, -1, "unknown flag"),
    ({}, b"bf16", 1, 8000, -1, "multiple of 128"),
    ({}, b"bf16", 1, 64, -1, "multiple of 128"),
    ({}, b"bf16", 1, 16384, -1, "max_seq"),
    ({}, b"bf16", 0, 8192, -1, "bs"),
    ({"n_q": 12}, b"bf16", 1, 8192, -1, "8 * n_kv"),
    ({"head_dim": 80}, b"bf16", 1, 8192, -1, "head_dim"),
    ({"hidden": 1000}, b"bf16", 1, 8192, -1, "hidden"),
    ({"num_layers": 1}, b"bf16", 1, 8192, -1, "num_layers"),
])
def test_validate(kw, quant, bs, seq, code, msg):
    from minicpm5_mk import _lib

    lib = _lib.load()
    cfg = _cfg(**kw)
    rc = lib.mk_validate(ctypes.byref(cfg), quant, bs, seq)
    assert rc == code, lib.mk_last_error()
    if code:
        assert msg in lib.mk_last_error().decode()


def test_packed_bytes_arithmetic():
    from minicpm5_mk import _lib

    lib = _lib.load()
    cfg = _cfg()
    n = ctypes.c_size_t()
    assert lib.mk_packed_bytes(ctypes.byref(cfg), b"int8d:qkv+gu|sq|lastbf16|fqkv|fmlp", ctypes.byref(n)) == 0
    Lm, H, I, D, qd = 23, 1536, 4608, 2560, 2048
    al = lambda v: (v + 255) // 256 * 256  # noqa: E731
    # W_qkv + its column scales in the packed order, W_o, W_gu + scales, W_down, the last layer's bf16 weights
    exp = (al(Lm * D * H) + al(Lm * D * 4) + al(Lm * H * qd * 2) + al(Lm * 2 * I * H) + al(Lm * 2 * I * 4)
           + al(Lm * H * I * 2) + al(D * H * 2) + al(H * qd * 2) + al(2 * I * H * 2) + al(H * I * 2))
    assert n.value == exp


def test_parse_precompile():
    """MINICPM5_MK_PRECOMPILE's "BxS,BxS" list (model.py:28, :690-693)."""
    from minicpm5_mk.runtime import MkError, parse_precompile

    assert parse_precompile("") == [] and parse_precompile(None) == []
    assert parse_precompile("1x8192,4x8192, 32X8192 ,") == [(1, 8192), (4, 8192), (32, 8192)]
    for bad in ("8192", "1x", "x8192", "1x8192x2", "0x8192", "ax8192"):
        with pytest.raises(MkError):
            parse_precompile(bad)


def test_sampling_fast_ok_and_eligibility():
    from minicpm5_mk import sampling_fast_ok
    from minicpm5_mk.engine import NotEligible, SamplingParams, eligible_batch, mk_seq_ok

    assert sampling_fast_ok(SamplingParams())
    assert sampling_fast_ok(SamplingParams(temperature=0.7, top_p=0.9, top_k=5, seed=3, logprobs=20))
    assert not sampling_fast_ok(None)
    for bad in ({"prompt_logprobs": 1}, {"presence_penalty": 0.1}, {"frequency_penalty": 0.1},
                {"repetition_penalty": 1.1}, {"min_p": 0.1}, {"logit_bias": {1: 1.0}}, {"allowed_token_ids": [1]},
                {"bad_words": ["x"]}, {"structured_outputs": object()}, {"logits_processors": [print]}):
        assert not sampling_fast_ok(SamplingParams(**bad)), bad
    # the reference rule: <= 1024 -> % 128, else % 1024
    assert [mk_seq_ok(s, 8256) for s in (128, 384, 896, 1024, 1152, 2048, 3072, 8192, 9216, 0)] == \
        [True, True, True, True, False, True, True, True, False, False]
    sp = SamplingParams()
    assert eligible_batch([[1] * 1024] * 3, [sp] * 3, 8256) == (3, 1024)
    for prompts, sps, reason in (([[1] * 1024, [1] * 2048], [sp, sp], "ragged"),
                                 ([[1] * 1024], [SamplingParams(max_tokens=2)], "max_tokens"),
                                 ([[1] * 1024], [SamplingParams(min_p=0.5)], "unsupported_sampling_feature"),
                                 ([[1] * 1000], [sp], "seq")):
        with pytest.raises(NotEligible) as e:
            eligible_batch(prompts, sps, 8256)
        assert e.value.reason == reason


def test_ops_refuse_cpu_tensors():
    """The product has no CPU path: kernel wrappers reject host tensors before any launch."""
    import torch

    from minicpm5_mk import ops

    with pytest.raises(ops.MkError, match="GPU tensor"):
        ops.attn_prefill(torch.zeros(1, 256, 20 * 64, dtype=torch.bfloat16), torch.zeros(256, 64, dtype=torch.bfloat16),
                         torch.zeros(256, 64, dtype=torch.bfloat16), 16, 2, 64)


@pytest.mark.parametrize("B,S,n_q,n_kv,hd,msg", [
    (1, 8192, 512, 64, 128, "63 kv heads"),
    (1, 8192, 16, 3, 128, "8 * n_kv"),
    (1, 100, 16, 2, 128, "multiple of 64"),
    (1, 8192, 16, 2, 80, "head_dim"),
    (0, 8192, 16, 2, 128, "batch"),
    (1, 8192, 16, 2, 128, "null pointer"),
])
def test_attn_prefill_rejects_before_launch(B, S, n_q, n_kv, hd, msg):
    """mk_attn_prefill checks its shapes and pointers on the host and returns an error, no kernel launched."""
    from minicpm5_mk import _lib

    lib = _lib.load()
    rc = lib.mk_attn_prefill(None, None, None, None, None, 0, B, S, n_q, n_kv, hd, 1.0, None)
    assert rc != 0
    assert msg in lib.mk_last_error().decode()


@pytest.mark.parametrize("bad", ["qkv", "cos", "sin", "out", "scratch"])
def test_attn_prefill_rejects_misaligned_pointers(bad):
    """The attention kernels move 16-byte vectors: a misaligned pointer is MK_EINVAL before any launch
    (the pointers here are never dereferenced)."""
    from minicpm5_mk import _lib

    lib = _lib.load()
    ptr = {k: ctypes.c_void_p(0x10000 * (i + 1)) for i, k in enumerate(("qkv", "cos", "sin", "out", "scratch"))}
    ptr[bad] = ctypes.c_void_p(ptr[bad].value + 8)
    need = lib.mk_attn_scratch_bytes(1, 1024, 2, 128)
    rc = lib.mk_attn_prefill(ptr["qkv"], ptr["cos"], ptr["sin"], ptr["out"], ptr["scratch"], need, 1, 1024, 16, 2,
                             128, ctypes.c_float(1.0), None)
    assert rc == -1 and b"16-byte aligned" in lib.mk_last_error()
    avg = ctypes.c_float()
    rc = lib.mk_bench_attn(ptr["qkv"], ptr["cos"], ptr["sin"], ptr["out"], ptr["scratch"], need, 1, 1024, 16, 2, 128,
                           ctypes.c_float(1.0), 1, None, ctypes.byref(avg))
    assert rc == -1 and b"16-byte aligned" in lib.mk_last_error()


def test_attn_prefill_rejects_oversized_seq():
    from minicpm5_mk import _lib

    lib = _lib.load()
    p = ctypes.c_void_p(0x10000)
    rc = lib.mk_attn_prefill(p, p, p, p, p, 1 << 40, 1, 262144, 16, 2, 128, ctypes.c_float(1.0), None)
    assert rc == -1 and b"131072" in lib.mk_last_error()


def test_gemm_rejects_operands_of_4_gib():
    """mk_gemm addresses its operands with 32-bit offsets: an operand of >= 4 GiB is MK_EINVAL before any
    launch (the pointers here are never dereferenced)."""
    from minicpm5_mk import _lib

    lib = _lib.load()
    p = ctypes.c_void_p(0x10000)
    # A: 40000 rows x 65536 bf16 = 5.2 GB
    rc = lib.mk_gemm(0, 4, p, 65536, p, 65536, 40000, 256, 65536, p, 256, None, 0, None, None, None, None)
    assert rc == -1 and b"4 GiB" in lib.mk_last_error()
    # B: 40000 rows x 65536 bf16
    rc = lib.mk_gemm(0, 4, p, 65536, p, 65536, 256, 40000, 65536, p, 40000, None, 0, None, None, None, None)
    assert rc == -1 and b"4 GiB" in lib.mk_last_error()


def test_gemm_k_alignment_by_path():
    """K bytes: a multiple of 64 on the tiled kernels (M > 32), of 32 on the weight-streaming kernel
    (M <= 32); a 32-byte K at M > 32 is MK_EINVAL before any launch (include/mk.h, mk_gemm)."""
    from minicpm5_mk import _lib

    lib = _lib.load()
    p = ctypes.c_void_p(0x10000)
    # int8, K = 32 bytes, M = 64: tiled path -> rejected
    rc = lib.mk_gemm(1, 3, p, 32, p, 32, 64, 64, 32, p, 64, None, 0, None, None, None, None)
    assert rc == -1 and b"multiple of 64" in lib.mk_last_error()
    # bf16, K = 16 elements = 32 bytes, M = 64: rejected the same way
    rc = lib.mk_gemm(0, 4, p, 16, p, 16, 64, 64, 16, p, 64, None, 0, None, None, None, None)
    assert rc == -1 and b"multiple of 64" in lib.mk_last_error()
    # K = 16 bytes is below either path's granule
    rc = lib.mk_gemm(1, 3, p, 16, p, 16, 8, 64, 16, p, 64, None, 0, None, None, None, None)
    assert rc == -1 and b"multiple of 32" in lib.mk_last_error()
