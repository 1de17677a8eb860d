"""Device decode state of the token-mixing layers.

Mirrors ``LayerCache`` / ``HybridCache`` (reference/cache.py:19-57) with the
state held in fixed device buffers that the kernels update in place:

==================  ==============================================================
reference field     device storage here
==================  ==============================================================
conv_state          ``conv_ring`` [B, conv_dim, K] (act); slot p % K = input at p
recurrent_state     ``recurrent_state`` [B, Hv, d, d] float32 (same tensor)
keys / values       ``k_pool`` / ``v_pool`` [n_pages, Hkv, P * d] bf16 under
                    ``page_table`` [B, max_pages] int32; each page of a kv head
                    in the attention kernels' MFMA lane order
                    (``qm_qsa_page_index`` maps (row, channel) to an offset)
indexer_keys        ``raw_keys`` [B, max_ctx, idx_dim] (act) plus ``block_keys``
                    [B, max_blocks, idx_dim] float32 (pooled, normed, roped)
==================  ==============================================================

The reference attribute names are kept as properties: reading one gathers a
reference-layout tensor out of the device buffers (for export, inspection and
tests), assigning one imports a reference-layout tensor into them (for prefix
reuse and tests). The kernels never go through these properties.
"""

from __future__ import annotations

import ctypes

import torch

from . import native


class MixLayerCache:
    def __init__(self, owner: "MixHybridCache"):
        self._owner = owner
        self.n_tokens = 0                 # tokens this layer has consumed
        # DeltaNet
        self.conv_ring = None
        self.recurrent_state = None
        # QSA
        self.k_pool = self.v_pool = None
        self.page_table = None
        self.raw_keys = None
        self.block_keys = None
        self.blocks_valid = 0             # block-cache rows that hold pooled keys
        self.last_ids = self.last_n_sel = self.last_iq = self.last_q = None   # last call's intermediates

    # -- allocation -----------------------------------------------------------

    def ensure_dn(self, batch: int, dtype: torch.dtype):
        o = self._owner
        cfg = o.config
        if self.conv_ring is None:
            self.conv_ring = torch.zeros(batch, cfg.conv_dim, cfg.conv_kernel, dtype=dtype, device=o.device)
        if self.recurrent_state is None:
            d = cfg.linear_head_dim
            self.recurrent_state = torch.zeros(batch, cfg.linear_num_v_heads, d, d, dtype=torch.float32,
                                               device=o.device)

    def ensure_qsa(self, batch: int, dtype: torch.dtype):
        if self.k_pool is not None:
            return
        o = self._owner
        cfg = o.config
        P, d = cfg.page_size, cfg.head_dim
        self.page_table = o.page_table
        n_pages = o.n_pages
        # zero-filled: rows beyond a sequence's end are read (with weight 0) by
        # the tail group, so they must hold finite values
        self.k_pool = torch.zeros(n_pages, cfg.num_kv_heads, P * d, dtype=torch.bfloat16, device=o.device)
        self.v_pool = torch.zeros(n_pages, cfg.num_kv_heads, P * d, dtype=torch.bfloat16, device=o.device)
        self.raw_keys = torch.zeros(batch, o.max_ctx, cfg.indexer_head_dim, dtype=dtype, device=o.device)
        self.block_keys = torch.zeros(batch, o.max_blocks, cfg.indexer_head_dim, dtype=torch.float32,
                                      device=o.device)

    # -- reference-layout views ------------------------------------------------

    def _slot_order(self):
        """Ring slot of each of the K-1 history columns, oldest first."""
        K = self._owner.config.conv_kernel
        p = self.n_tokens
        return [(p - (K - 1) + j) % K for j in range(K - 1)]

    @property
    def conv_state(self):
        if self.conv_ring is None:
            return None
        return self.conv_ring[:, :, self._slot_order()].clone()

    @conv_state.setter
    def conv_state(self, value):
        if value is None:
            self.conv_ring = None
            return
        self.ensure_dn(value.shape[0], value.dtype)
        for j, slot in enumerate(self._slot_order()):
            self.conv_ring[:, :, slot] = value[:, :, j].to(self.conv_ring.device, self.conv_ring.dtype)

    def _token_slots(self, n: int):
        """Physical (page, row) of logical tokens 0..n-1 for every sequence."""
        P = self._owner.config.page_size
        tok = torch.arange(n, device=self.page_table.device)
        pages = self.page_table[:, tok // P].long()          # [B, n]
        return pages, (tok % P).long()

    def _rows(self, pool, index):
        """The pool as [n_pages, Hkv, P, d] rows (a gathered copy)."""
        cfg = self._owner.config
        n, h = pool.shape[:2]
        return pool[:, :, index].view(n, h, cfg.page_size, cfg.head_dim)

    def _store_rows(self, pool, index, rows_view):
        n, h = pool.shape[:2]
        pool[:, :, index] = rows_view.reshape(n, h, -1)

    @property
    def keys(self):
        if self.k_pool is None or self.n_tokens == 0:
            return None
        pages, rows = self._token_slots(self.n_tokens)
        ref = self._rows(self.k_pool, self._owner.k_index)
        # [B, n, Hkv, d] -> [B, Hkv, n, d]
        return ref[pages, :, rows[None].expand_as(pages)].permute(0, 2, 1, 3).float()

    @keys.setter
    def keys(self, value):
        """Import reference-layout keys (B, Hkv, S, d); they are stored as bf16."""
        batch, _, n, _ = value.shape
        self.ensure_qsa(batch, self._owner.dtype)
        pages, rows = self._token_slots(n)
        ref = self._rows(self.k_pool, self._owner.k_index)
        ref[pages, :, rows[None].expand_as(pages)] = value.to(ref.device).permute(0, 2, 1, 3).to(torch.bfloat16)
        self._store_rows(self.k_pool, self._owner.k_index, ref)
        self.n_tokens = n

    @property
    def values(self):
        if self.v_pool is None or self.n_tokens == 0:
            return None
        pages, rows = self._token_slots(self.n_tokens)
        ref = self._rows(self.v_pool, self._owner.v_index)
        # [B, n, Hkv, d] -> [B, Hkv, n, d]
        return ref[pages, :, rows[None].expand_as(pages)].permute(0, 2, 1, 3).to(self._owner.dtype)

    @values.setter
    def values(self, value):
        batch, _, n, _ = value.shape
        self.ensure_qsa(batch, self._owner.dtype)
        pages, rows = self._token_slots(n)
        ref = self._rows(self.v_pool, self._owner.v_index)
        ref[pages, :, rows[None].expand_as(pages)] = value.to(ref.device).permute(0, 2, 1, 3).to(torch.bfloat16)
        self._store_rows(self.v_pool, self._owner.v_index, ref)
        self.n_tokens = n

    def page_row(self, pool: str, page: int, row: int) -> torch.Tensor:
        """Row `row` of physical page `page` of the K or V pool, [Hkv, d]."""
        o = self._owner
        base = self.k_pool if pool == "k" else self.v_pool
        index = (o.k_index if pool == "k" else o.v_index).view(o.config.page_size, -1)[row]
        return base[page][:, index]

    @property
    def indexer_keys(self):
        if self.raw_keys is None or self.n_tokens == 0:
            return None
        return self.raw_keys[:, : self.n_tokens].clone()

    @indexer_keys.setter
    def indexer_keys(self, value):
        """Import raw indexer keys (B, S, idx_dim); their blocks are pooled lazily
        at the next call that has the rope tables (``blocks_valid`` tracks it)."""
        batch, n, _ = value.shape
        self.ensure_qsa(batch, self._owner.dtype)
        self.raw_keys[:, :n] = value.to(self.raw_keys.device, self.raw_keys.dtype)
        self.blocks_valid = 0
        self.n_tokens = n


class MixHybridCache:
    """Per-sequence-batch state for every layer, plus the position history.

    ``page_table`` is ``"identity"``, ``"random"`` (a seeded permutation of the
    whole pool, so no two logical neighbours share a physical neighbour) or an
    int32 tensor [batch, max_pages] of physical page ids.
    """

    def __init__(self, num_layers: int, config, batch: int = 1, max_ctx: int = 8192, device=None,
                 dtype: torch.dtype = torch.bfloat16, page_table="identity", seed: int = 0):
        self.config = config
        self.batch = batch
        self.device = torch.device(device if device is not None else "cuda")
        self.dtype = dtype
        P = config.page_size
        ratio = config.indexer_compress_ratio
        self.max_ctx = ((max_ctx + P - 1) // P) * P
        self.max_pages = self.max_ctx // P
        self.max_blocks = max(1, self.max_ctx // ratio)
        self.n_pages = batch * self.max_pages
        if isinstance(page_table, torch.Tensor):
            pt = page_table.to(torch.int32)
            if pt.shape != (batch, self.max_pages):
                raise ValueError(f"page_table must be [{batch}, {self.max_pages}]")
            if int(pt.min()) < 0 or int(pt.max()) >= self.n_pages:
                raise ValueError("page_table entries outside the pool")
        elif page_table == "random":
            g = torch.Generator().manual_seed(seed)
            pt = torch.randperm(self.n_pages, generator=g).to(torch.int32).reshape(batch, self.max_pages)
        elif page_table == "identity":
            pt = torch.arange(self.n_pages, dtype=torch.int32).reshape(batch, self.max_pages)
        else:
            raise ValueError(f"unknown page_table {page_table!r}")
        self.page_table = pt.to(self.device)
        d = config.head_dim
        k_index = (ctypes.c_int * (P * d))()
        v_index = (ctypes.c_int * (P * d))()
        native.call("qm_qsa_page_index", P, d, k_index, v_index)
        # offset in a page of (row, channel), row-major over [P, d]
        self.k_index = torch.tensor(list(k_index), dtype=torch.long, device=self.device)
        self.v_index = torch.tensor(list(v_index), dtype=torch.long, device=self.device)
        self.layers = [MixLayerCache(self) for _ in range(num_layers)]
        self.position_ids = None

    def __getitem__(self, idx: int) -> MixLayerCache:
        return self.layers[idx]

    @property
    def seq_len(self) -> int:
        return 0 if self.position_ids is None else self.position_ids.shape[-1]

    def extend_positions(self, position_ids: torch.Tensor) -> torch.Tensor:
        """As reference/cache.py:44-52."""
        if position_ids.ndim == 2:
            position_ids = position_ids[None].expand(3, -1, -1)
        if self.position_ids is None:
            self.position_ids = position_ids
        else:
            self.position_ids = torch.cat([self.position_ids, position_ids], dim=-1)
        return self.position_ids

    def reset(self) -> None:
        for i in range(len(self.layers)):
            self.layers[i] = MixLayerCache(self)
        self.position_ids = None
