"""Dimensions of the token-mixing path (oracle side).

Follows the fields and derivations of reference/config.py:80-104 and :136-158
(``linear_key_dim``, ``linear_value_dim``, ``conv_dim``, ``is_full_attention``).
Only the fields the token-mixing layers and the hyper-connections around them
read are kept; the MoE and PLE fields are outside this path.

Pinned by: the derived quantities are closed forms checked in
tests/test_oracle_layers.py (conv_dim = 2*Hk*d + Hv*d, the full-attention
layer rule ``(l + 1) % interval == 0``).
"""

from __future__ import annotations

from dataclasses import dataclass, field


@dataclass
class OracleConfig:
    hidden_size: int = 2048
    rms_norm_eps: float = 1e-6
    # QSA (reference/config.py:81-87)
    num_attention_heads: int = 16
    num_kv_heads: int = 2
    head_dim: int = 256
    rope_theta: float = 1e7
    rope_dim: int = 64
    mrope_section: list = field(default_factory=lambda: [11, 11, 10])
    full_attention_interval: int = 4
    # QSA indexer (reference/config.py:90-93)
    indexer_heads: int = 4
    indexer_head_dim: int = 128
    indexer_budget: int = 2048
    indexer_compress_ratio: int = 64
    # Gated DeltaNet (reference/config.py:96-99)
    linear_num_v_heads: int = 32
    linear_num_k_heads: int = 16
    linear_head_dim: int = 128
    conv_kernel: int = 4
    output_gate_type: str = "sigmoid"
    # hyper-connections (reference/config.py:51-52, 80-81)
    hc_count: int = 4
    hc_lowrank: int = 320

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
