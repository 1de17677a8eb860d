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
                    [B, max_blocks, idx_dim] float32 (pooled, normed, roped;
                    each row permuted, ``block_keys_ref`` un-permutes)
==================  ==============================================================

The reference attribute names are kept as properties: reading one gathers a
reference-layout tensor out of the device buffers (for export, inspection and
tests), assigning one imports a reference-layout tensor into them (for prefix
reuse and tests). The kernels never go through these properties.

Slots (the rows of the batch) are managed for continuous batching as
tt/model.py:2373-2431 manages them: ``reset_slot`` clears one sequence's
state in place while the others keep decoding. With ``page_table="pooled"``
the slots draw K/V pages from a shared ``PagePool`` as they grow
(``ensure_capacity``), give them back on reset, and ``fork_slot`` lets a slot
continue another's prefix on the same pages. ``slot_view`` is a one-sequence
cache over one slot's rows, for prefilling it through the layer methods.
"""

from __future__ import annotations

import ctypes

import torch

from . import native
from .pages import PagePool, PoolExhausted


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
        n_pages = o.pool_pages
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
    def block_keys_ref(self):
        """The pooled block keys in the reference's element order, [B, max_blocks,
        idx_dim] (a gathered copy: the device rows keep element d at
        (d % 16) * 8 + d // 16, the order the scoring lanes read)."""
        if self.block_keys is None:
            return None
        d = torch.arange(self.block_keys.shape[-1], device=self.block_keys.device)
        return self.block_keys[..., (d % 16) * 8 + d // 16]

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
    whole pool, so no two logical neighbours share a physical neighbour), an
    int32 tensor [batch, max_pages] of physical page ids, or ``"pooled"``: a
    pool of ``n_pages`` pages (default batch * max_pages) that the slots map on
    demand, every unmapped entry pointing at a reserved all-zero page.
    """

    def __init__(self, num_layers: int, config, batch: int = 1, max_ctx: int = 8192, device=None,
                 dtype: torch.dtype = torch.bfloat16, page_table="identity", seed: int = 0,
                 n_pages: int | None = None):
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
        self.pool = None
        self.null_page = None
        if isinstance(page_table, str) and page_table == "pooled":
            self.n_pages = n_pages if n_pages is not None else batch * self.max_pages
            self.pool = PagePool(self.n_pages)
            self.null_page = self.n_pages
            pt = torch.full((batch, self.max_pages), self.null_page, dtype=torch.int32)
        elif isinstance(page_table, torch.Tensor):
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
        self._pt_host = pt.clone()
        self._mapped = [self.max_pages if self.pool is None else 0] * batch   # logical pages mapped per slot
        self.slot_tokens = [0] * batch
        self._slot_of = None              # (parent cache, slot) of a slot view
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

    @property
    def pool_pages(self) -> int:
        """Pages in the K/V pools: the table's pages, plus the null page of a pooled table."""
        return self.n_pages + (1 if self.pool is not None else 0)

    def reset(self) -> None:
        for i in range(len(self.layers)):
            self.layers[i] = MixLayerCache(self)
        self.position_ids = None
        if self.pool is not None:
            self.pool = PagePool(self.n_pages)
            self._pt_host.fill_(self.null_page)
            self.page_table.fill_(self.null_page)
            self._mapped = [0] * self.batch
        self.slot_tokens = [0] * self.batch

    # -- slots (continuous batching) ----------------------------------------------

    def _check_slot(self, slot: int) -> None:
        if not 0 <= slot < self.batch:
            raise IndexError(f"slot {slot} out of range for batch {self.batch}")

    def ensure_allocated(self, dtype: torch.dtype | None = None) -> None:
        """Allocate every layer's buffers (DeltaNet or QSA by the config)."""
        dt = dtype if dtype is not None else self.dtype
        for i, lc in enumerate(self.layers):
            if self.config.is_full_attention(i):
                lc.ensure_qsa(self.batch, dt)
            else:
                lc.ensure_dn(self.batch, dt)

    def ensure_capacity(self, slot: int, n_tokens: int) -> None:
        """Map pages for slot's tokens 0..n_tokens-1 before a step writes them.

        Static tables are mapped whole; a pooled table maps the missing pages
        from the pool (raising ``PoolExhausted``, with nothing taken, when too
        few are free) and writes them into the device table in place, so graphs
        captured against it stay valid."""
        if self._slot_of is not None:
            parent, ps = self._slot_of
            return parent.ensure_capacity(ps, n_tokens)
        self._check_slot(slot)
        if n_tokens > self.max_ctx:
            raise ValueError(f"{n_tokens} tokens exceed the cache's {self.max_ctx}")
        if self.pool is None:
            return
        P = self.config.page_size
        need, have = -(-n_tokens // P), self._mapped[slot]
        if need <= have:
            return
        if need - have > self.pool.n_free:
            raise PoolExhausted(f"slot {slot} needs {need - have} pages, {self.pool.n_free} are free")
        pages = [self.pool.alloc() for _ in range(need - have)]
        self._pt_host[slot, have:need] = torch.tensor(pages, dtype=torch.int32)
        self.page_table[slot, have:need].copy_(self._pt_host[slot, have:need])
        self._mapped[slot] = need

    def reset_slot(self, slot: int) -> None:
        """Clear one sequence's state so that a new one can take the slot while
        the others keep decoding (tt/model.py:2373-2431).

        The DeltaNet state and conv ring of the slot are zeroed in place in
        every layer: they accumulate unconditionally, and a position-0 step
        reads the ring's history slots. K/V, raw and pooled indexer keys are
        not cleared: every read is bounded by the position, and a block's
        pooled key is rewritten by the step that completes it, before it can
        be selected. A pooled table gives the slot's pages back."""
        if self._slot_of is not None:
            parent, ps = self._slot_of
            return parent.reset_slot(ps)
        self._check_slot(slot)
        for lc in self.layers:
            if lc.conv_ring is not None:
                lc.conv_ring[slot].zero_()
            if lc.recurrent_state is not None:
                lc.recurrent_state[slot].zero_()
        if self.pool is not None:
            for page in self._pt_host[slot, : self._mapped[slot]].tolist():
                self.pool.release(page)
            self._pt_host[slot].fill_(self.null_page)
            self.page_table[slot].fill_(self.null_page)
            self._mapped[slot] = 0
        self.slot_tokens[slot] = 0

    def fork_slot(self, src: int, dst: int, n_tokens: int) -> None:
        """Prefix reuse: empty slot ``dst`` continues slot ``src``'s first
        ``n_tokens`` tokens.

        ``src`` must have consumed exactly ``n_tokens`` tokens: its DeltaNet
        state and conv ring are copied, and a recurrence cannot be rewound to an
        earlier point (tt/model.py:2302-2308 snapshots it for the same reason).
        A pooled table maps src's full pages into dst (shared, reference
        counted) and gives dst its own copy of the partial last page, the only
        one either slot writes again; a static table copies the pages. The raw
        and pooled indexer keys of the prefix are copied."""
        self._check_slot(src)
        self._check_slot(dst)
        if src == dst:
            raise ValueError("fork_slot needs two different slots")
        if self.slot_tokens[src] != n_tokens:
            raise ValueError(f"slot {src} holds {self.slot_tokens[src]} tokens, not {n_tokens}")
        if self.slot_tokens[dst] != 0 or (self.pool is not None and self._mapped[dst] != 0):
            raise ValueError(f"slot {dst} is not empty (reset it first)")
        P = self.config.page_size
        n_full, n_used = n_tokens // P, -(-n_tokens // P)
        src_pages = self._pt_host[src, :n_used].tolist()
        if self.pool is not None:
            if n_used > n_full and self.pool.n_free < 1:
                raise PoolExhausted("no free page for the partial page of the fork")
            dst_pages = [self.pool.share(p) for p in src_pages[:n_full]]
            if n_used > n_full:
                dst_pages.append(self.pool.alloc())
            if dst_pages:
                self._pt_host[dst, :n_used] = torch.tensor(dst_pages, dtype=torch.int32)
                self.page_table[dst, :n_used].copy_(self._pt_host[dst, :n_used])
            self._mapped[dst] = n_used
            copy_pages = list(zip(src_pages[n_full:], dst_pages[n_full:]))
        else:
            copy_pages = list(zip(src_pages, self._pt_host[dst, :n_used].tolist()))
        ratio = self.config.indexer_compress_ratio
        for lc in self.layers:
            if lc.k_pool is not None:
                for sp, dp in copy_pages:
                    lc.k_pool[dp].copy_(lc.k_pool[sp])
                    lc.v_pool[dp].copy_(lc.v_pool[sp])
                lc.raw_keys[dst, :n_tokens].copy_(lc.raw_keys[src, :n_tokens])
                lc.block_keys[dst, : n_tokens // ratio].copy_(lc.block_keys[src, : n_tokens // ratio])
            if lc.recurrent_state is not None:
                lc.recurrent_state[dst].copy_(lc.recurrent_state[src])
                lc.conv_ring[dst].copy_(lc.conv_ring[src])
        self.slot_tokens[dst] = n_tokens

    def slot_view(self, slot: int) -> "MixHybridCache":
        """A one-sequence cache over slot ``slot``: its page-table row, conv
        ring, recurrent state, raw and pooled keys are views of this cache's
        rows, and the K/V pools are shared, so a layer method run on the view
        (a prefill of that slot) updates this cache in place. Every layer's
        buffers are allocated first. Each view layer starts at the slot's token
        count; ``commit_slot_view`` records the view's count back."""
        self._check_slot(slot)
        self.ensure_allocated()
        v = object.__new__(MixHybridCache)
        v.__dict__.update({k: getattr(self, k) for k in (
            "config", "device", "dtype", "max_ctx", "max_pages", "max_blocks", "n_pages", "pool", "null_page",
            "k_index", "v_index")})
        v.batch = 1
        v.position_ids = None
        v.page_table = self.page_table[slot:slot + 1]
        v._pt_host = self._pt_host[slot:slot + 1]
        v._mapped = [self._mapped[slot]]
        v.slot_tokens = [self.slot_tokens[slot]]
        v._slot_of = (self, slot)
        v.layers = []
        ratio = self.config.indexer_compress_ratio
        for lc in self.layers:
            vl = MixLayerCache(v)
            vl.n_tokens = self.slot_tokens[slot]
            if lc.conv_ring is not None:
                vl.conv_ring = lc.conv_ring[slot:slot + 1]
                vl.recurrent_state = lc.recurrent_state[slot:slot + 1]
            if lc.k_pool is not None:
                vl.k_pool, vl.v_pool = lc.k_pool, lc.v_pool
                vl.page_table = v.page_table
                vl.raw_keys = lc.raw_keys[slot:slot + 1]
                vl.block_keys = lc.block_keys[slot:slot + 1]
                vl.blocks_valid = self.slot_tokens[slot] // ratio
            v.layers.append(vl)
        return v

    def commit_slot_view(self, view: "MixHybridCache") -> None:
        """Record a slot view's token count (after running layers on it) in this cache."""
        parent, slot = view._slot_of
        if parent is not self:
            raise ValueError("the view belongs to another cache")
        self.slot_tokens[slot] = max(l.n_tokens for l in view.layers)
