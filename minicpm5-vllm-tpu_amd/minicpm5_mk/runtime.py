"""The whole-model op: libmk's mk_model_create / mk_forward behind the reference's op signature.

`forward(...)` takes exactly the arguments of the reference's `minicpm5_mk::forward` op
(plugin/minicpm5_mk/model.py:749-751, weight order :40-41) and returns the same (max(8, bs), H) bf16
final-normed last-token hidden states (mk_jax.py:624-665).  One `MkModel` (packed weights + cached
hipGraphs) is kept per weight set, like the reference keeps one compiled program per static
signature (model.py:54-86).
"""
from __future__ import annotations

import collections
import ctypes
import threading
import time

import torch

from ._lib import WEIGHT_FIELDS, MkConfig, MkError, MkWeights, check, load
from .quant import parse_quant, quant_flags, validate_quant

BF16 = torch.bfloat16
F32 = torch.float32

WEIGHT_ORDER = ("w_qkv", "w_o", "w_gu", "w_down", "s_qkv", "s_o", "s_gu", "s_down",
                "a_qkv", "a_o", "a_gu", "a_down", "wl_qkv", "wl_o", "wl_gu", "wl_down")
ATTN_PREFIXES = ("auto", "v2", "super", "flash", "pallas", "splash", "xla")
BF16_DUMMY = "bf16-dummy"      # (1,) or (L-1, 1): the unread scale slots of a bf16 linear


def shape_ok(t: torch.Tensor, shape, Lm: int) -> bool:
    if shape == BF16_DUMMY:
        return tuple(t.shape) in ((1,), (Lm, 1))
    return tuple(t.shape) == tuple(shape)


def parse_precompile(spec: str) -> list:
    """MINICPM5_MK_PRECOMPILE's value, e.g. "1x8192,4x8192" -> [(1, 8192), (4, 8192)] (model.py:28, :690-693);
    empty -> []."""
    shapes = []
    for part in (spec or "").split(","):
        part = part.strip()
        if not part:
            continue
        try:
            b, s = (int(v) for v in part.lower().split("x"))
        except ValueError:
            raise MkError(f"precompile shape {part!r}: expected BxS, e.g. 4x8192") from None
        if b < 1 or s < 1:
            raise MkError(f"precompile shape {part!r}: B and S must be positive")
        shapes.append((b, s))
    return shapes


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def expected_shapes(L: int, H: int, inter: int, n_q: int, n_kv: int, hd: int, quant: str) -> dict:
    """{name: (shape, dtype)} of the reference-layout tensors (mk_weights.py:126-263) for `quant`.

    The scales / activation factors of a bf16 linear are dummies that are never read: the reference
    passes (1,) for an all-bf16 string (mk_weights.py:176-179) and (L-1, 1) for a bf16 linear of a
    mixed string; their shape here is BF16_DUMMY, which accepts both."""
    qm = parse_quant(quant)
    fl = quant_flags(quant)
    Lm, qd = L - 1, n_q * hd
    D = qd + 2 * n_kv * hd
    i8 = {k: v != "bf16" for k, v in qm.items()}      # 8-bit weights (int8 or fp8 e4m3)
    fmlp = "fmlp" in fl and qm["gu"] in ("int8", "int8d")
    wdt = {"bf16": BF16, "int8": torch.int8, "int8d": torch.int8, "fp8": torch.float8_e4m3fn,
           "fp8d": torch.float8_e4m3fn}
    wt = lambda k: wdt[qm[k]]  # noqa: E731
    sc = lambda k, n: (Lm, n) if i8[k] else BF16_DUMMY  # noqa: E731
    return {
        "w_qkv": ((Lm, H, D), wt("qkv")), "w_o": ((Lm, qd, H), wt("o")),
        "w_gu": ((Lm, H, 2 * inter) if fmlp else (Lm, H, 2, inter), wt("gu")),
        "w_down": ((Lm, inter, H), wt("down")),
        "s_qkv": (sc("qkv", D), F32), "s_o": (sc("o", H), F32),
        "s_gu": (((Lm, 1, 2 * inter) if fmlp else (Lm, 2, inter)) if i8["gu"] else BF16_DUMMY, F32),
        "s_down": (sc("down", H), F32),
        "a_qkv": (sc("qkv", H), F32), "a_o": (sc("o", qd), F32), "a_gu": (sc("gu", H), F32),
        "a_down": (sc("down", inter), F32),
        "wl_qkv": ((H, D), BF16), "wl_o": ((qd, H), BF16), "wl_gu": ((H, 2, inter), BF16),
        "wl_down": ((inter, H), BF16),
    }


class MkModel:
    """A libmk model over device tensors in the reference layout (kept alive by this object).

    Each (bs, seq, logits) shape gets persistent device buffers (workspace, ids, outputs) that its
    captured hipGraph is bound to; the buffers of the MAX_SHAPES most recently used shapes are kept (a
    2B workspace at (32, 8192) is several GB).  An evicted shape allocates again on its next call; its
    old graph, cached by libmk under the old buffer addresses, is only replayed if a call brings exactly
    those addresses back, so it never touches memory that is not that call's."""

    MAX_SHAPES = 8

    def __init__(self, weights: dict, embed: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                 final_norm: torch.Tensor, quant: str, n_q: int, n_kv: int, head_dim: int, eps: float,
                 lm_head: torch.Tensor | None = None):
        validate_quant(quant)
        lib = load()
        L = int(weights["w_qkv"].shape[0]) + 1
        V, H = (int(v) for v in embed.shape)
        inter = int(weights["w_down"].shape[-2])
        self.dims = dict(L=L, H=H, I=inter, V=V, n_q=n_q, n_kv=n_kv, hd=head_dim, eps=eps)
        exp = expected_shapes(L, H, inter, n_q, n_kv, head_dim, quant)
        for k, (shape, dtype) in exp.items():
            t = weights[k]
            if not shape_ok(t, shape, L - 1) or t.dtype != dtype:
                raise MkError(f"{k}: got {tuple(t.shape)} {t.dtype}, expected {shape} {dtype} for quant {quant!r}")
        others = {"embed": (embed, (V, H), BF16), "final_norm": (final_norm, (H,), BF16),
                  "cos": (cos, (cos.shape[0], head_dim), BF16), "sin": (sin, (cos.shape[0], head_dim), BF16)}
        if lm_head is not None:
            others["lm_head"] = (lm_head, (V, H), BF16)
        for k, (t, shape, dtype) in others.items():
            if tuple(t.shape) != tuple(shape) or t.dtype != dtype:
                raise MkError(f"{k}: got {tuple(t.shape)} {t.dtype}, expected {shape} {dtype}")
        tensors = dict(weights, embed=embed, cos=cos, sin=sin, final_norm=final_norm, lm_head=lm_head)
        for k, t in tensors.items():
            if t is None:
                continue
            if not t.is_cuda or not t.is_contiguous():
                raise MkError(f"{k}: must be a contiguous GPU tensor")
            if t.data_ptr() % 16:
                raise MkError(f"{k}: must be 16-byte aligned")
        self.device = embed.device
        self.quant = quant
        self._keep = tensors
        self.cfg = MkConfig(L, H, inter, n_q, n_kv, head_dim, V, float(eps), int(cos.shape[0]))
        self._w = MkWeights(*[ctypes.c_void_p(tensors[n].data_ptr()) if tensors.get(n) is not None else None
                              for n in WEIGHT_FIELDS])
        nbytes = ctypes.c_size_t()
        check(lib.mk_packed_bytes(ctypes.byref(self.cfg), quant.encode(), ctypes.byref(nbytes)), "mk_packed_bytes")
        self.packed = torch.empty(nbytes.value, dtype=torch.uint8, device=self.device)
        handle = ctypes.c_void_p()
        check(lib.mk_model_create(ctypes.byref(self.cfg), quant.encode(), ctypes.byref(self._w),
                                  ctypes.c_void_p(self.packed.data_ptr()), nbytes.value, _stream(),
                                  ctypes.byref(handle)), "mk_model_create")
        self._h = handle
        self._bufs = collections.OrderedDict()
        self._lock = threading.Lock()

    @property
    def has_lm_head(self) -> bool:
        return self._keep.get("lm_head") is not None

    def set_graph_mode(self, enable: bool) -> None:
        check(load().mk_set_graph_mode(self._h, int(enable)), "mk_set_graph_mode")

    def set_attn_prep_fused(self, enable: bool) -> None:
        """True (default): K RoPE and V^T come from the QKV projection's epilogue; False: a separate prep
        kernel (same results; for checking the fused path)."""
        check(load().mk_set_attn_prep_fused(self._h, int(enable)), "mk_set_attn_prep_fused")

    def set_max_chunk(self, seqs: int) -> None:
        """Cap the sequences per chunk of a large batch (0 = the default, include/mk.h); drops the cached
        per-shape buffers, whose workspace size depends on it."""
        check(load().mk_set_max_chunk(self._h, int(seqs)), "mk_set_max_chunk")
        self._bufs.clear()

    def workspace_bytes(self, bs: int, seq: int) -> int:
        n = ctypes.c_size_t()
        check(load().mk_workspace_bytes(self._h, bs, seq, ctypes.byref(n)), "mk_workspace_bytes")
        return n.value

    def _buffers(self, bs: int, seq: int, want_logits: bool):
        key = (bs, seq, want_logits)
        b = self._bufs.get(key)
        if b is None:
            while len(self._bufs) >= self.MAX_SHAPES:   # least recently used shape out
                self._bufs.popitem(last=False)
            dev, H, V = self.device, self.dims["H"], self.dims["V"]
            # ordinary tensors even when the first call of a shape runs under torch.inference_mode (vLLM's
            # model runner): `ids` is written in place on every call, also outside inference mode
            with torch.inference_mode(False):
                b = {"ws": torch.empty(self.workspace_bytes(bs, seq), dtype=torch.uint8, device=dev),
                     "ids": torch.empty(bs * seq, dtype=torch.int32, device=dev),
                     "hidden": torch.empty((max(8, bs), H), dtype=BF16, device=dev),
                     "logits": torch.empty((bs, V), dtype=F32, device=dev) if want_logits else None}
            self._bufs[key] = b
        self._bufs.move_to_end(key)
        return b

    def release_buffers(self) -> None:
        self._bufs.clear()

    def precompile(self, shapes, logits: bool = False, log=None) -> dict:
        """Captures the hipGraph of every (bs, seq) in `shapes` ahead of its first forward (the reference's
        MINICPM5_MK_PRECOMPILE, model.py:690-698, which compiles the op per shape at load time).  The
        graphs are bound to this model's persistent per-shape buffers, which `forward` then reuses, so the
        first call of a precompiled shape only replays.  Nothing runs on the GPU.  -> {(bs, seq): seconds}"""
        lib = load()
        out = {}
        for bs, seq in shapes:
            t0 = time.perf_counter()
            check(lib.mk_validate(ctypes.byref(self.cfg), self.quant.encode(), bs, seq), "mk_validate")
            if logits and not self.has_lm_head:
                raise MkError("logits requested but the model was built without lm_head")
            with self._lock:
                b = self._buffers(bs, seq, logits)
                lg = b["logits"]
                check(lib.mk_precompile(self._h, ctypes.c_void_p(b["ids"].data_ptr()), bs, seq,
                                        ctypes.c_void_p(b["hidden"].data_ptr()),
                                        ctypes.c_void_p(lg.data_ptr()) if lg is not None else None,
                                        ctypes.c_void_p(b["ws"].data_ptr()), b["ws"].numel()), "mk_precompile")
            out[(bs, seq)] = time.perf_counter() - t0
            if log:
                log(f"minicpm5_mk: precompiled {bs}x{seq} in {out[(bs, seq)]:.2f}s")
        return out

    def graph_count(self) -> int:
        n = ctypes.c_int()
        check(load().mk_graph_count(self._h, ctypes.byref(n)), "mk_graph_count")
        return n.value

    def forward(self, input_ids: torch.Tensor, bs: int, seq: int, logits: bool = False, copy_out: bool = True):
        """input_ids (>= bs*seq,) int32/int64 on the GPU, sequence-major -> hidden (max(8, bs), H) bf16
        [, logits (bs, V) f32].  With copy_out=False the returned tensors are this model's persistent
        buffers for (bs, seq) (overwritten by the next call of that shape)."""
        if logits and not self.has_lm_head:
            raise MkError("logits requested but the model was built without lm_head")
        if input_ids.numel() < bs * seq:
            raise MkError(f"input_ids has {input_ids.numel()} tokens < bs*seq = {bs * seq}")
        if not input_ids.is_cuda:
            raise MkError("input_ids must be on the GPU")
        check(load().mk_validate(ctypes.byref(self.cfg), self.quant.encode(), bs, seq), "mk_validate")
        with self._lock:
            b = self._buffers(bs, seq, logits)
            b["ids"].copy_(input_ids.reshape(-1)[: bs * seq])
            lg = b["logits"]
            check(load().mk_forward(self._h, ctypes.c_void_p(b["ids"].data_ptr()), bs, seq,
                                    ctypes.c_void_p(b["hidden"].data_ptr()),
                                    ctypes.c_void_p(lg.data_ptr()) if lg is not None else None,
                                    ctypes.c_void_p(b["ws"].data_ptr()), b["ws"].numel(), _stream()), "mk_forward")
            hidden = b["hidden"].clone() if copy_out else b["hidden"]
            if not logits:
                return hidden
            return hidden, (lg.clone() if copy_out else lg)

    KERNEL_KINDS = ("embed", "norm", "gemm_qkv", "attn_prep", "attn", "gemm_o", "gemm_gu", "gemm_down", "last_layer",
                    "lm_head", "other")   # MK_KERNEL_* order (include/mk.h)

    def forward_timed(self, input_ids: torch.Tensor, bs: int, seq: int, logits: bool = False) -> dict:
        """One eager forward with a hipEvent pair around every kernel launch: {kind: (ms, launches)}
        (synchronizes the current stream)."""
        if logits and not self.has_lm_head:
            raise MkError("logits requested but the model was built without lm_head")
        if input_ids.numel() < bs * seq or not input_ids.is_cuda:
            raise MkError("input_ids must be a GPU tensor of >= bs*seq tokens")
        n = len(self.KERNEL_KINDS)
        ms, cnt = (ctypes.c_float * n)(), (ctypes.c_int * n)()
        with self._lock:
            b = self._buffers(bs, seq, logits)
            b["ids"].copy_(input_ids.reshape(-1)[: bs * seq])
            lg = b["logits"]
            check(load().mk_forward_timed(self._h, ctypes.c_void_p(b["ids"].data_ptr()), bs, seq,
                                          ctypes.c_void_p(b["hidden"].data_ptr()),
                                          ctypes.c_void_p(lg.data_ptr()) if lg is not None else None,
                                          ctypes.c_void_p(b["ws"].data_ptr()), b["ws"].numel(), _stream(), ms, cnt),
                  "mk_forward_timed")
        return {k: (ms[i], cnt[i]) for i, k in enumerate(self.KERNEL_KINDS)}

    def close(self) -> None:
        if getattr(self, "_h", None):
            load().mk_model_destroy(self._h)
            self._h = None
        self._bufs = collections.OrderedDict()

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001  (interpreter shutdown)
            pass


# runtime.forward's packed models: key (storage, shapes, quant, shape arguments) -> (version counters of
# the tensors, MkModel), least recently used first.  The packed copy is rebuilt when a caller updated
# any of the tensors in place (torch bumps a tensor's version counter on every in-place write), as the
# reference op reads the tensors it is passed on every call.  The MkModel holds the tensors, so their
# storage cannot be freed and reused under the same key while cached.
_MODELS: "collections.OrderedDict" = collections.OrderedDict()
MAX_CACHED_MODELS = 2


def _version(t: torch.Tensor) -> int:
    """The tensor's version counter; inference tensors (made under torch.inference_mode, as vLLM's model
    runner runs) keep none, so an in-place update of one is not seen: -1."""
    return -1 if t.is_inference() else t._version


def _validate_attn(attn: str) -> None:
    if not any(attn.startswith(p) for p in ATTN_PREFIXES):
        raise MkError(f"attn {attn!r}: unknown (auto | v2[:bq,mc] | super... | flash... | splash... | xla)")


def forward(input_ids, embed, cos, sin, final_norm, w_qkv, w_o, w_gu, w_down, s_qkv, s_o, s_gu, s_down,
            a_qkv, a_o, a_gu, a_down, wl_qkv, wl_o, wl_gu, wl_down, bs: int, seq: int, quant: str, n_q: int,
            n_kv: int, head_dim: int, eps: float, attn: str = "auto") -> torch.Tensor:
    """The reference's `minicpm5_mk::forward` op (model.py:749-751) on MI355X.

    `attn` selects among the reference's TPU attention variants; every variant names the same
    causal GQA attention, which libmk runs with its one HIP kernel (the string is validated only)."""
    _validate_attn(attn)
    tensors = (embed, cos, sin, final_norm, w_qkv, w_o, w_gu, w_down, s_qkv, s_o, s_gu, s_down,
               a_qkv, a_o, a_gu, a_down, wl_qkv, wl_o, wl_gu, wl_down)
    key = (tuple(t.data_ptr() for t in tensors), tuple(tuple(t.shape) for t in tensors), quant, n_q, n_kv,
           head_dim, float(eps))
    versions = tuple(_version(t) for t in tensors)
    hit = _MODELS.get(key)
    if hit is not None and hit[0] != versions:        # updated in place since it was packed: re-pack
        _MODELS.pop(key)[1].close()
        hit = None
    if hit is None:
        while len(_MODELS) >= MAX_CACHED_MODELS:
            _MODELS.popitem(last=False)[1][1].close()
        w = dict(zip(WEIGHT_ORDER, (w_qkv, w_o, w_gu, w_down, s_qkv, s_o, s_gu, s_down,
                                    a_qkv, a_o, a_gu, a_down, wl_qkv, wl_o, wl_gu, wl_down)))
        hit = _MODELS[key] = (versions, MkModel(w, embed, cos, sin, final_norm, quant, n_q, n_kv, head_dim, eps))
    _MODELS.move_to_end(key)
    return hit[1].forward(input_ids, bs, seq)


def clear_cache() -> None:
    for _, m in _MODELS.values():
        m.close()
    _MODELS.clear()
