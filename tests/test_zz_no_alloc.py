"""mk_attn_prefill_noalloc (the allocation-free attention entry point) against mk_attn_prefill, through
the C ABI: identical output on two calls in a row, the second smaller, and MK_ENOMEM past the
file-scope scratch's stated maximum (MK_NOALLOC_SCRATCH_BYTES)."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu
NOALLOC_MAX = 40 << 20


def _noalloc(lib):
    f = lib.mk_attn_prefill_noalloc
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] * 5 + [ctypes.c_float, ctypes.c_void_p]
    return f


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def test_noalloc_attention_matches_attn_prefill():
    from minicpm5_mk import _lib
    from minicpm5_mk.mk_weights import rope_tables

    assert torch.cuda.is_available()
    dev = torch.device("cuda:0")
    lib = _lib.load()
    f = _noalloc(lib)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    # two calls in a row, the second with a smaller input (different head_dim too)
    for B, S, hd, seed in ((2, 4096, 128, 11), (1, 1024, 96, 12)):
        print(f"[noalloc] B={B} S={S} hd={hd}", flush=True)
        n_q, n_kv = 16, 2
        D = (n_q + 2 * n_kv) * hd
        g = torch.Generator().manual_seed(seed)
        qkv = torch.randn(B, S, D, generator=g).to(torch.bfloat16).to(dev)
        cos, sin = (t.to(dev) for t in rope_tables(S, hd, 1e4))
        need = lib.mk_attn_scratch_bytes(B, S, n_kv, hd)
        assert need <= NOALLOC_MAX
        scratch = torch.empty(need, dtype=torch.uint8, device=dev)
        ref = torch.empty(B, S, n_q * hd, dtype=torch.bfloat16, device=dev)
        out = torch.full_like(ref, float("nan"))
        _lib.check(lib.mk_attn_prefill(_p(qkv), _p(cos), _p(sin), _p(ref), _p(scratch), need, B, S, n_q, n_kv, hd,
                                       ctypes.c_float(hd ** -0.5), st), "mk_attn_prefill")
        _lib.check(f(_p(qkv), _p(cos), _p(sin), _p(out), B, S, n_q, n_kv, hd, ctypes.c_float(hd ** -0.5), st),
                   "mk_attn_prefill_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"B={B} S={S} hd={hd}"
    # past the maximum: rejected before any launch
    big = torch.empty(16, dtype=torch.bfloat16, device=dev)
    rc = f(_p(big), _p(big), _p(big), _p(big), 8, 8192, 16, 2, 128, ctypes.c_float(1.0), st)
    assert rc == -4 and b"allocation-free maximum" in lib.mk_last_error()
