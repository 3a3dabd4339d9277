"""Quant-string grammar and the `auto` resolution of the plugin.

Grammar (plugin/minicpm5_mk/mk_jax.py:302-318): "<q>" (all four linears) or "<q>:<lin>+<lin>"
(only those, the rest bf16), then optional "|flag" suffixes; q in {bf16, int8, int8d, fp8, fp8d},
lin in {qkv, o, gu, down}, flags in {sq, lastbf16, fqkv, fmlp}.

`resolve_quant_pair` restates model.py:528-551 for one device (TP = 1): 1B (<= 24 layers)
"int8d:qkv+gu|sq|lastbf16|fqkv|fmlp", 2B "int8d:qkv+gu+o|sq|lastbf16|fqkv|fmlp"; fmlp only when the
fused MLP's weights fit (3 * H * I <= 56 MiB).  libmk builds every base: bf16, int8d and fp8d
(per-token dynamic activations), int8 and fp8 (static calibrated activation scales; the down
projection stays dynamic, mk_jax.py:422-423).
"""
from __future__ import annotations

LINEARS = ("qkv", "o", "gu", "down")
BASES = ("bf16", "int8", "int8d", "fp8", "fp8d")
FLAGS = ("sq", "lastbf16", "fqkv", "fmlp")


def quant_flags(quant: str) -> set:
    """Flags after '|', e.g. "int8d:qkv+gu|sq|fmlp" -> {"sq", "fmlp"}."""
    return set(quant.split("|")[1:])


def parse_quant(quant: str) -> dict:
    """{linear: precision} for the four linears."""
    base = quant.split("|")[0]
    if ":" in base:
        q, lins = base.split(":", 1)
        sel = set(lins.split("+"))
        return {k: (q if k in sel else "bf16") for k in LINEARS}
    return {k: base for k in LINEARS}


def validate_quant(quant: str) -> None:
    """Raises ValueError on a string outside the grammar."""
    base = quant.split("|")[0]
    q = base.split(":", 1)[0]
    if q not in BASES:
        raise ValueError(f"quant {quant!r}: unknown base {q!r} (one of {BASES})")
    if ":" in base:
        bad = set(base.split(":", 1)[1].split("+")) - set(LINEARS)
        if bad:
            raise ValueError(f"quant {quant!r}: unknown linears {sorted(bad)}")
    bad = quant_flags(quant) - set(FLAGS)
    if bad:
        raise ValueError(f"quant {quant!r}: unknown flags {sorted(bad)}")


def resolve_quant_pair(requested: str, num_layers: int, tp: int = 1, hidden: int = 0, inter: int = 0):
    """(quant for the single / DP mode, quant for the TP mode) -- model.py:528-551."""
    if requested != "auto":
        return requested, requested
    fmlp_ok = 3 * hidden * inter <= (56 if tp == 1 else 30) * 1024 * 1024
    fused = "|fqkv" + ("|fmlp" if fmlp_ok else "")
    if tp > 1:
        return "int8d:qkv+gu|sq|lastbf16" + fused, "bf16"
    q = ("int8d:qkv+gu|sq|lastbf16" if num_layers <= 24 else "int8d:qkv+gu+o|sq|lastbf16") + fused
    return q, q
