"""Oracle restatement of reference/cache.py:19-57 (per-layer decode state).

The token-mixing state of one layer is: the conv window (B, conv_dim, K-1), the
float32 recurrent state (B, Hv, d_k, d_v), the dense K/V cache
(B, n_kv, S, head_dim), and the indexer's raw (pre-norm, pre-rope) key cache
(B, S, indexer_head_dim). The PLE fields of the reference are outside this path.

Pinned by: it is a container; tests/test_oracle_layers.py checks that
``extend_positions`` concatenates along the last axis and ``seq_len`` follows it.
"""

from __future__ import annotations

import torch


class OracleLayerCache:
    __slots__ = ("conv_state", "recurrent_state", "keys", "values", "indexer_keys")

    def __init__(self) -> None:
        self.conv_state = None
        self.recurrent_state = None
        self.keys = None
        self.values = None
        self.indexer_keys = None


class OracleHybridCache:
    def __init__(self, num_layers: int) -> None:
        self.layers = [OracleLayerCache() for _ in range(num_layers)]
        self.position_ids = None  # (3, B, S_total)

    def __getitem__(self, idx: int) -> OracleLayerCache:
        return self.layers[idx]

    @property
    def seq_len(self) -> int:
        return 0 if self.position_ids is None else self.position_ids.shape[-1]

    def extend_positions(self, position_ids: torch.Tensor) -> torch.Tensor:
        if position_ids.ndim == 2:
            position_ids = position_ids[None].expand(3, -1, -1)
        if self.position_ids is None:
            self.position_ids = position_ids
        else:
            self.position_ids = torch.cat([self.position_ids, position_ids], dim=-1)
        return self.position_ids
