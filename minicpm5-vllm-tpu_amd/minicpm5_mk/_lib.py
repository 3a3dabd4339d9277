"""ctypes binding of libmk.so (the C ABI declared in include/mk.h).

The library is built in-tree by `minicpm5_mk._build`.  There is no fallback: if the library is
missing or fails to load, every op raises -- the product never silently computes on the CPU.
"""
from __future__ import annotations

import ctypes
import os
import threading

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmk.so")
_lock = threading.Lock()
_lib = None

MK_OK = 0
EPI = {
    "dq_bf16": 0, "dq_silu": 1, "dq_silu_f32a": 2, "bf16": 3, "f32": 4, "res_bf16add": 5,
    "dq_res_bf16add": 6, "res_f32add": 7, "dq2_res_f32add": 8, "i32": 9, "silu_bf16": 10, "dq2_bf16": 11,
    "dq2_res_bf16add": 12,
}

# Every symbol of include/mk.h with its (restype, argtypes).
_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t


class MkConfig(ctypes.Structure):
    _fields_ = [("num_layers", ctypes.c_int32), ("hidden", ctypes.c_int32), ("inter", ctypes.c_int32),
                ("n_q", ctypes.c_int32), ("n_kv", ctypes.c_int32), ("head_dim", ctypes.c_int32),
                ("vocab", ctypes.c_int32), ("eps", ctypes.c_float), ("max_seq", ctypes.c_int32)]


WEIGHT_FIELDS = ("embed", "cos", "sin", "final_norm", "w_qkv", "w_o", "w_gu", "w_down", "s_qkv", "s_o", "s_gu",
                 "s_down", "a_qkv", "a_o", "a_gu", "a_down", "wl_qkv", "wl_o", "wl_gu", "wl_down", "lm_head")


class MkWeights(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in WEIGHT_FIELDS]


SIGNATURES = {
    "mk_last_error": (ctypes.c_char_p, []),
    "mk_abi_version": (_I, []),
    "mk_validate": (_I, [ctypes.POINTER(MkConfig), ctypes.c_char_p, _I, _I]),
    "mk_packed_bytes": (_I, [ctypes.POINTER(MkConfig), ctypes.c_char_p, ctypes.POINTER(_SZ)]),
    "mk_model_create": (_I, [ctypes.POINTER(MkConfig), ctypes.c_char_p, ctypes.POINTER(MkWeights), _P, _SZ, _P,
                             ctypes.POINTER(_P)]),
    "mk_model_destroy": (_I, [_P]),
    "mk_workspace_bytes": (_I, [_P, _I, _I, ctypes.POINTER(_SZ)]),
    "mk_forward": (_I, [_P, _P, _I, _I, _P, _P, _P, _SZ, _P]),
    "mk_set_graph_mode": (_I, [_P, _I]),
    "mk_precompile": (_I, [_P, _P, _I, _I, _P, _P, _P, _SZ]),
    "mk_graph_count": (_I, [_P, ctypes.POINTER(_I)]),
    "mk_set_attn_prep_fused": (_I, [_P, _I]),
    "mk_set_max_chunk": (_I, [_P, _I]),
    "mk_forward_timed": (_I, [_P, _P, _I, _I, _P, _P, _P, _SZ, _P, _P, _P]),
    "mk_attn_scratch_bytes": (_SZ, [_I, _I, _I, _I]),
    "mk_attn_prefill": (_I, [_P, _P, _P, _P, _P, _SZ, _I, _I, _I, _I, _I, _F, _P]),
    "mk_attn_prefill_noalloc": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _P]),
    "mk_row_quant": (_I, [_P, _I, _P, _I, _I, _F, _I, _I, _P, _P, _P]),
    "mk_act_quant": (_I, [_P, _I, _P, _I, _I, _F, _I, _I, _P, _P, _P]),
    "mk_mfma_peak_scratch_bytes": (_SZ, [_I]),
    "mk_bench_mfma_peak": (_I, [_I, _I, _I, _P, _SZ, _P, _P, _P]),
    "mk_gemm": (_I, [_I, _I, _P, _I, _P, _I, _I, _I, _I, _P, _I, _P, _I, _P, _P, _P, _P]),
    "mk_lm_head": (_I, [_P, _P, _I, _I, _I, _P, _P]),
    "mk_pack_weight": (_I, [_P, _I, _P, _I, _I, _I, _I, _I, _I, _P]),
    "mk_weight_row_amax": (_I, [_P, _I, _I, _F, _P, _P]),
    "mk_weight_quantize": (_I, [_P, _I, _I, _F, _P, _I, _F, _P, _I, _P, _P, _P]),
    "mk_bench_attn": (_I, [_P, _P, _P, _P, _P, _SZ, _I, _I, _I, _I, _I, _F, _I, _P, ctypes.POINTER(_F)]),
    "mk_bench_gemm": (_I, [_I, _I, _P, _I, _P, _I, _I, _I, _I, _P, _I, _P, _I, _P, _P, _P, _I, _P,
                           ctypes.POINTER(_F)]),
}


class MkError(RuntimeError):
    pass


def lib_path() -> str:
    return _LIB_PATH


def load():
    """Loads libmk.so once (raises MkError if it is missing)."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(_LIB_PATH):
                raise MkError(f"libmk.so not found at {_LIB_PATH}; build it with "
                              "`python -m minicpm5_mk._build` (or __graft_entry__.build())")
            lib = ctypes.CDLL(_LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    if rc != MK_OK:
        msg = load().mk_last_error().decode(errors="replace")
        raise MkError(f"{what} failed (code {rc}): {msg}")
