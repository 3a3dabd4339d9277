"""mk_attn_prefill_noalloc (the allocation-free attention entry point) against mk_attn_prefill, through
the C ABI: identical output on calls in a row (the second smaller; the third on the work-queue path,
whose counters are the array state that persists between calls), a captured hipGraph replayed between
eager calls that change the array, and MK_ENOMEM past the file-scope scratch's stated maximum
(MK_NOALLOC_SCRATCH_BYTES)."""
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
    n_q, n_kv = 16, 2

    def case(B, S, hd, seed):
        g = torch.Generator().manual_seed(seed)
        qkv = torch.randn(B, S, (n_q + 2 * n_kv) * hd, generator=g).to(torch.bfloat16).to(dev)
        cos, sin = (t.to(dev) for t in rope_tables(S, hd, 1e4))
        need = lib.mk_attn_scratch_bytes(B, S, n_kv, hd)
        assert need <= NOALLOC_MAX
        scratch = torch.empty(need, dtype=torch.uint8, device=dev)
        ref = torch.empty(B, S, n_q * hd, dtype=torch.bfloat16, device=dev)
        _lib.check(lib.mk_attn_prefill(_p(qkv), _p(cos), _p(sin), _p(ref), _p(scratch), need, B, S, n_q, n_kv, hd,
                                       ctypes.c_float(hd ** -0.5), st), "mk_attn_prefill")
        return qkv, cos, sin, ref

    def noalloc(B, S, hd, qkv, cos, sin, out, stream):
        _lib.check(f(_p(qkv), _p(cos), _p(sin), _p(out), B, S, n_q, n_kv, hd, ctypes.c_float(hd ** -0.5), stream),
                   "mk_attn_prefill_noalloc")

    # calls in a row: the second with a smaller input (different head_dim too); the third takes the
    # work-queue path (3 * 2 * 1024 / 32 items on 4-wave workgroups: 384 items, persistent workgroups
    # taking them from the counters in the array)
    shapes = ((2, 4096, 128, 11), (1, 1024, 96, 12), (3, 1024, 128, 13))
    for B, S, hd, seed in shapes:
        print(f"[noalloc] B={B} S={S} hd={hd}", flush=True)
        qkv, cos, sin, ref = case(B, S, hd, seed)
        out = torch.full_like(ref, float("nan"))
        noalloc(B, S, hd, qkv, cos, sin, out, st)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"B={B} S={S} hd={hd}"

    # captured into a graph (no allocation, no memset node: the prep kernel clears the counters) and
    # replayed three times, each after eager calls of other shapes that rewrite the array
    print("[noalloc] graph capture of B=3 S=1024 hd=128", flush=True)
    qkv, cos, sin, ref = case(3, 1024, 128, 14)
    out = torch.full_like(ref, float("nan"))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, capture_error_mode="thread_local"):
        noalloc(3, 1024, 128, qkv, cos, sin, out, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    other = [(B, S, hd, *case(B, S, hd, 20 + i)[:3]) for i, (B, S, hd, _) in enumerate(shapes)]
    for rep in range(3):
        B, S, hd, q2, c2, s2 = other[rep]
        o2 = torch.empty(B, S, n_q * hd, dtype=torch.bfloat16, device=dev)
        noalloc(B, S, hd, q2, c2, s2, o2, st)
        torch.cuda.synchronize()
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"graph replay {rep}"
    del graph
    # past the maximum: rejected before any launch
    big = torch.empty(16, dtype=torch.bfloat16, device=dev)
    rc = f(_p(big), _p(big), _p(big), _p(big), 8, 8192, 16, 2, 128, ctypes.c_float(1.0), st)
    assert rc == -4 and b"allocation-free maximum" in lib.mk_last_error()
