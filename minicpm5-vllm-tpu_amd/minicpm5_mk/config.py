"""Model configuration for the MiniCPM5 prefill/scoring path.

The reference plugin has no built-in config: it reads the HF config at load time into a dict with
the keys num_layers, hidden, inter, n_q, n_kv, head_dim, eps, rope_theta
(plugin/minicpm5_mk/model.py:561-567).  `MkConfig` carries the same fields plus the vocabulary
size (used by the LM head) and the BOS id (`model.py:568`).

Presets:
  * ``1b``      -- MiniCPM5-1B as recorded by the reference's result files
                   (results/v6e_minicpm5_1b.json:79-95): L 24, H 1536, I 4608, 16Q/2KV, head_dim 128,
                   V 130560, rope_theta 5e6, eps 1e-6.
  * ``1b-hd96`` -- the same with head_dim 96 (q_dim 1536 == hidden).
  * ``2b``      -- MiniCPM5-2B (results/v6e_minicpm5_2b.json:79-95): L 42, H 2048, I 6144,
                   16Q/2KV, head_dim 128, V 130560, rope_theta 5e6.
  * ``tiny``    -- a small config with the same head structure for fast tests.
"""
from __future__ import annotations

import dataclasses
from dataclasses import dataclass


@dataclass(frozen=True)
class MkConfig:
    num_layers: int
    hidden: int
    inter: int
    n_q: int
    n_kv: int
    head_dim: int
    vocab: int
    eps: float = 1e-6
    rope_theta: float = 5_000_000.0
    bos_token_id: int = 0
    name: str = "custom"

    @property
    def q_dim(self) -> int:
        return self.n_q * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.n_kv * self.head_dim

    @property
    def qkv_dim(self) -> int:
        return (self.n_q + 2 * self.n_kv) * self.head_dim

    def as_mk_cfg(self) -> dict:
        """The reference's `_mk_cfg` dict (model.py:561-567)."""
        return dict(num_layers=self.num_layers, hidden=self.hidden, inter=self.inter, n_q=self.n_q,
                    n_kv=self.n_kv, head_dim=self.head_dim, eps=self.eps, rope_theta=self.rope_theta)

    def replace(self, **kw) -> "MkConfig":
        return dataclasses.replace(self, **kw)

    def validate(self) -> None:
        if self.n_q % self.n_kv:
            raise ValueError(f"n_q={self.n_q} is not a multiple of n_kv={self.n_kv}")
        if self.head_dim % 32 or self.head_dim > 128:
            raise ValueError(f"head_dim={self.head_dim} unsupported (multiple of 32, <= 128)")
        if self.hidden % 64 or self.inter % 64:
            raise ValueError("hidden and inter must be multiples of 64")
        if self.num_layers < 2:
            raise ValueError("num_layers must be >= 2 (scan layers + last-token-only layer)")

    @staticmethod
    def from_hf(hf) -> "MkConfig":
        """Build from an HF config object or dict (same fields the reference reads)."""
        g = (lambda k, d=None: hf.get(k, d)) if isinstance(hf, dict) else (lambda k, d=None: getattr(hf, k, d))
        hidden = int(g("hidden_size"))
        n_q = int(g("num_attention_heads"))
        theta = float(g("rope_theta", 10000.0) or 10000.0)
        rope = g("rope_scaling") or g("rope_parameters")
        if isinstance(rope, dict) and "rope_theta" in rope:
            theta = float(rope["rope_theta"])
        return MkConfig(
            num_layers=int(g("num_hidden_layers")), hidden=hidden, inter=int(g("intermediate_size")),
            n_q=n_q, n_kv=int(g("num_key_value_heads")),
            head_dim=int(g("head_dim") or hidden // n_q), vocab=int(g("vocab_size")),
            eps=float(g("rms_norm_eps")), rope_theta=theta, bos_token_id=int(g("bos_token_id", 0) or 0),
            name="hf")


PRESETS = {
    "1b": MkConfig(24, 1536, 4608, 16, 2, 128, 130560, 1e-6, 5_000_000.0, 0, "minicpm5-1b"),
    "1b-hd96": MkConfig(24, 1536, 4608, 16, 2, 96, 130560, 1e-6, 5_000_000.0, 0, "minicpm5-1b-hd96"),
    "2b": MkConfig(42, 2048, 6144, 16, 2, 128, 130560, 1e-6, 5_000_000.0, 0, "minicpm5-2b"),
    "tiny": MkConfig(3, 256, 768, 16, 2, 64, 32768, 1e-6, 10_000.0, 0, "tiny"),
    "tiny-hd96": MkConfig(3, 384, 1024, 16, 2, 96, 32768, 1e-6, 10_000.0, 0, "tiny-hd96"),
}


def preset(name: str) -> MkConfig:
    try:
        return PRESETS[name]
    except KeyError:
        raise ValueError(f"unknown preset {name!r}; known: {sorted(PRESETS)}") from None
