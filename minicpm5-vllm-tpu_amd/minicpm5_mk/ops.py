"""torch-facing wrappers of libmk's kernel-level entry points.

PyTorch provides device memory and the current HIP stream; every computation runs in libmk's HIP
kernels.  Each wrapper checks dtypes, devices, contiguity and shapes on the host before the launch
(the kernels assume them) and raises `MkError` with libmk's message on any failure.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import EPI, MkError, check, load

BF16 = torch.bfloat16


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _need(t: torch.Tensor, name: str, dtype=None, shape=None):
    if not isinstance(t, torch.Tensor):
        raise MkError(f"{name}: expected a torch.Tensor")
    if not t.is_cuda:
        raise MkError(f"{name}: must be a GPU tensor (libmk has no CPU path)")
    if not t.is_contiguous():
        raise MkError(f"{name}: must be contiguous")
    if dtype is not None and t.dtype != dtype:
        raise MkError(f"{name}: dtype {t.dtype}, expected {dtype}")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise MkError(f"{name}: shape {tuple(t.shape)}, expected {tuple(shape)}")
    if t.data_ptr() % 16:
        raise MkError(f"{name}: must be 16-byte aligned")


def attn_scratch_bytes(B: int, S: int, n_kv: int, head_dim: int) -> int:
    return int(load().mk_attn_scratch_bytes(B, S, n_kv, head_dim))


def attn_prefill(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, n_q: int, n_kv: int, head_dim: int,
                 sm_scale: float = 1.0, out: torch.Tensor | None = None) -> torch.Tensor:
    """Causal GQA prefill attention (super_gqa_v2, plugin/minicpm5_mk/mk_attn.py:660-710).

    qkv (B, S, (n_q + 2 n_kv) hd) bf16 -> (B, S, n_q hd) bf16; RoPE from the bf16 tables in-kernel."""
    lib = load()
    B, S, D = qkv.shape
    if D != (n_q + 2 * n_kv) * head_dim:
        raise MkError(f"qkv last dim {D} != (n_q + 2 n_kv) * head_dim")
    _need(qkv, "qkv", BF16)
    _need(cos, "cos", BF16)
    _need(sin, "sin", BF16)
    if cos.shape[0] < S or cos.shape[1] != head_dim or sin.shape != cos.shape:
        raise MkError("cos / sin must be (>= S, head_dim)")
    if out is None:
        out = torch.empty((B, S, n_q * head_dim), dtype=BF16, device=qkv.device)
    _need(out, "out", BF16, (B, S, n_q * head_dim))
    nbytes = attn_scratch_bytes(B, S, n_kv, head_dim)
    scratch = torch.empty(nbytes, dtype=torch.uint8, device=qkv.device)
    check(lib.mk_attn_prefill(_ptr(qkv), _ptr(cos), _ptr(sin), _ptr(out), _ptr(scratch), nbytes, B, S, n_q, n_kv,
                              head_dim, float(sm_scale), _stream()), "mk_attn_prefill")
    return out


def row_quant(x: torch.Tensor, a: torch.Tensor | None, eps: float = 1e-6, norm: bool = True, recip: bool = True):
    """Per-token dynamic int8 quantisation (+ RMSNorm statistics): returns (q int8 (T, H), sx f32 (T,))."""
    lib = load()
    if x.dim() != 2 or x.dtype not in (BF16, torch.float32):
        raise MkError("row_quant: x must be (T, H) bf16 or f32")
    T, H = x.shape
    _need(x, "x")
    if a is not None:
        _need(a, "a", torch.float32, (H,))
    q = torch.empty((T, H), dtype=torch.int8, device=x.device)
    sx = torch.empty((T,), dtype=torch.float32, device=x.device)
    check(lib.mk_row_quant(_ptr(x), int(x.dtype == torch.float32), _ptr(a), T, H, float(eps), int(norm), int(recip),
                           _ptr(q), _ptr(sx), _stream()), "mk_row_quant")
    return q, sx


ACT_MODES = {"int8d": 0, "fp8d": 1, "int8": 2, "fp8": 3}
FP8 = torch.float8_e4m3fn


def act_quant(x: torch.Tensor, a: torch.Tensor | None, mode: str, eps: float = 1e-6, norm: bool = False,
              recip: bool = False, smul: bool = False):
    """Activation quantisation in one of the reference's modes (include/mk.h, mk_act_quant): returns
    (q (T, H) int8 or float8_e4m3fn, sx f32 (T,))."""
    lib = load()
    if mode not in ACT_MODES:
        raise MkError(f"act_quant: unknown mode {mode!r}")
    if x.dim() != 2 or x.dtype not in (BF16, torch.float32):
        raise MkError("act_quant: x must be (T, H) bf16 or f32")
    T, H = x.shape
    _need(x, "x")
    if a is not None:
        _need(a, "a", torch.float32, (H,))
    q = torch.empty((T, H), dtype=FP8 if mode.startswith("fp8") else torch.int8, device=x.device)
    sx = torch.empty((T,), dtype=torch.float32, device=x.device)
    flags = int(norm) | 2 * int(recip) | 4 * int(smul)
    check(lib.mk_act_quant(_ptr(x), int(x.dtype == torch.float32), _ptr(a), T, H, float(eps), ACT_MODES[mode], flags,
                           _ptr(q), _ptr(sx), _stream()), "mk_act_quant")
    return q, sx


def gemm(A: torch.Tensor, B: torch.Tensor, epi: str, out: torch.Tensor | None = None, res: torch.Tensor | None = None,
         rs: torch.Tensor | None = None, cs: torch.Tensor | None = None, aux: torch.Tensor | None = None):
    """C = A (M, K) @ B (N, K)^T with a fused epilogue (see include/mk.h MK_EPI_*).

    int8 operands -> int8 MFMA with int32 accumulation; bf16 / float8_e4m3fn operands -> bf16 / fp8 MFMA,
    f32 accumulation."""
    lib = load()
    if epi not in EPI:
        raise MkError(f"unknown epilogue {epi!r}")
    if A.dim() != 2 or B.dim() != 2 or A.shape[1] != B.shape[1] or A.dtype != B.dtype:
        raise MkError("gemm: A (M, K) and B (N, K) must share K and dtype")
    if A.dtype not in (torch.int8, BF16, FP8):
        raise MkError("gemm: operands must be int8, bf16 or float8_e4m3fn")
    _need(A, "A")
    _need(B, "B")
    M, K = A.shape
    N = B.shape[0]
    silu = epi in ("dq_silu", "dq_silu_f32a", "silu_bf16")
    n_out = N // 2 if silu else N
    residual = epi in ("res_bf16add", "dq_res_bf16add", "res_f32add", "dq2_res_f32add", "dq2_res_bf16add")
    if residual:
        if res is None:
            raise MkError("gemm: residual epilogue needs `res`")
        _need(res, "res", BF16, (M, N))
    elif out is None:
        dt = {"f32": torch.float32, "i32": torch.int32, "dq_silu_f32a": torch.float32}.get(epi, BF16)
        out = torch.empty((M, n_out), dtype=dt, device=A.device)
    if out is not None:
        _need(out, "out", None, (M, n_out))
    for t, nm, n in ((rs, "rs", M), (cs, "cs", N), (aux, "aux", n_out)):
        if t is not None:
            _need(t, nm, torch.float32, (n,))
    in_type = {BF16: 0, torch.int8: 1, FP8: 2}[A.dtype]
    check(lib.mk_gemm(in_type, EPI[epi], _ptr(A), K, _ptr(B), K, M, N, K, _ptr(out),
                      n_out if out is not None else 0, _ptr(res), N if res is not None else 0, _ptr(rs), _ptr(cs),
                      _ptr(aux), _stream()), "mk_gemm")
    return res if residual else out


def lm_head(hidden: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """logits (B, V) f32 = hidden (B, H) bf16 @ weight (V, H)^T."""
    lib = load()
    B, H = hidden.shape
    V = weight.shape[0]
    _need(hidden, "hidden", BF16)
    _need(weight, "lm_head", BF16, (V, H))
    out = torch.empty((B, V), dtype=torch.float32, device=hidden.device)
    check(lib.mk_lm_head(_ptr(hidden), _ptr(weight), B, H, V, _ptr(out), _stream()), "mk_lm_head")
    return out


def pack_weight(w: torch.Tensor, map_gu: bool = False, ic: int = 0, inter: int = 0) -> torch.Tensor:
    """(K, N) -> (N, K) repack (the layout mk_model_create builds); map_gu reorders gate/up columns."""
    lib = load()
    K, N = w.shape
    _need(w, "w")
    out = torch.empty((N, K), dtype=w.dtype, device=w.device)
    check(lib.mk_pack_weight(_ptr(w), N, _ptr(out), K, N, w.element_size(), int(map_gu), ic, inter, _stream()),
          "mk_pack_weight")
    return out


__all__ = ["attn_prefill", "attn_scratch_bytes", "row_quant", "act_quant", "gemm", "lm_head", "pack_weight", "MkError", "_lib"]
