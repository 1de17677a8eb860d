"""Dimensions of the token-mixing layers.

Same field names and derivations as the reference config
(reference/config.py:51-52, 80-104, 136-158), restricted to what QSA, Gated
DeltaNet and the hyper-connections around them read, plus the paging
parameters this implementation adds (``page_size``).
``from_reference`` accepts any object carrying the reference's field names
(a ``Qwen4ExpConfig`` or a test double), so the layers drop into the reference
engine with its own config object.
"""

from __future__ import annotations

from dataclasses import dataclass, field, fields


@dataclass
class MixConfig:
    hidden_size: int = 2048
    rms_norm_eps: float = 1e-6
    num_attention_heads: int = 16
    num_kv_heads: int = 2
    head_dim: int = 256
    rope_theta: float = 1e7
    rope_dim: int = 64
    mrope_section: list = field(default_factory=lambda: [11, 11, 10])
    full_attention_interval: int = 4
    indexer_heads: int = 4
    indexer_head_dim: int = 128
    indexer_budget: int = 2048
    indexer_compress_ratio: int = 64
    linear_num_v_heads: int = 32
    linear_num_k_heads: int = 16
    linear_head_dim: int = 128
    conv_kernel: int = 4
    output_gate_type: str = "sigmoid"
    hc_count: int = 4
    hc_lowrank: int = 320
    page_size: int = 64

    @property
    def hc_hidden_size(self) -> int:
        return self.hc_count * self.hidden_size

    @property
    def linear_key_dim(self) -> int:
        return self.linear_num_k_heads * self.linear_head_dim

    @property
    def linear_value_dim(self) -> int:
        return self.linear_num_v_heads * self.linear_head_dim

    @property
    def conv_dim(self) -> int:
        return 2 * self.linear_key_dim + self.linear_value_dim

    @property
    def block_topk(self) -> int:
        return self.indexer_budget // self.indexer_compress_ratio

    def is_full_attention(self, layer_idx: int) -> bool:
        return (layer_idx + 1) % self.full_attention_interval == 0

    @classmethod
    def from_reference(cls, ref, **overrides) -> "MixConfig":
        vals = {}
        for f in fields(cls):
            if hasattr(ref, f.name):
                vals[f.name] = getattr(ref, f.name)
        vals.update(overrides)
        return cls(**vals)
