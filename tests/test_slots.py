"""Slots for continuous batching, host side: the page pool's counts, on-demand
mapping of a pooled page table, slot reset and prefix forks (tensors on the
CPU; the kernels never see anything but the resulting int32 table)."""

from __future__ import annotations

import pytest
import torch


def _cache(qm, batch=2, max_ctx=512, **kw):
    return qm.MixHybridCache(4, qm.MixConfig(), batch, max_ctx, "cpu", torch.float32, **kw)


def test_page_pool_counts(qm):
    pool = qm.PagePool(3)
    assert [pool.alloc() for _ in range(3)] == [0, 1, 2]
    with pytest.raises(qm.PoolExhausted):
        pool.alloc()
    pool.share(1)
    assert pool.refcount(1) == 2
    pool.release(1)
    assert pool.refcount(1) == 1 and pool.n_free == 0
    pool.release(1)
    assert pool.n_free == 1 and pool.alloc() == 1
    pool.release(2)
    with pytest.raises(ValueError):
        pool.release(2)
    with pytest.raises(ValueError):
        pool.share(2)


def test_pooled_table_maps_pages_on_demand(qm):
    cache = _cache(qm, n_pages=6, page_table="pooled")
    null = cache.null_page
    assert null == 6 and cache.pool_pages == 7
    assert cache.page_table.eq(null).all()
    cache.ensure_capacity(0, 1)
    cache.ensure_capacity(1, 130)                    # 3 pages
    assert cache.page_table[0, :2].tolist() == [0, null]
    assert cache.page_table[1, :4].tolist() == [1, 2, 3, null]
    cache.ensure_capacity(0, 64)                     # still one page
    assert cache.pool.n_free == 2
    cache.ensure_capacity(0, 65)
    assert cache.page_table[0, :2].tolist() == [0, 4]
    with pytest.raises(qm.PoolExhausted):
        cache.ensure_capacity(0, 64 * 4)             # needs 2, 1 is free: nothing is taken
    assert cache.pool.n_free == 1 and cache.page_table[0, 2].item() == null
    with pytest.raises(ValueError):
        cache.ensure_capacity(0, 513)
    cache.reset_slot(1)
    assert cache.pool.n_free == 4 and cache.page_table[1].eq(null).all()


def test_reset_slot_clears_only_that_slots_recurrent_state(qm):
    cache = _cache(qm)
    cache.ensure_allocated()
    dn = cache[0]
    dn.recurrent_state.normal_()
    dn.conv_ring.normal_()
    keep = dn.recurrent_state[0].clone(), dn.conv_ring[0].clone()
    cache.slot_tokens[1] = 7
    cache.reset_slot(1)
    assert dn.recurrent_state[1].eq(0).all() and dn.conv_ring[1].eq(0).all()
    assert torch.equal(dn.recurrent_state[0], keep[0]) and torch.equal(dn.conv_ring[0], keep[1])
    assert cache.slot_tokens == [0, 0]
    with pytest.raises(IndexError):
        cache.reset_slot(2)


def test_fork_shares_full_pages_and_copies_the_partial_page(qm):
    cache = _cache(qm, n_pages=8, page_table="pooled")
    cache.ensure_allocated()
    qsa, dn = cache[3], cache[0]
    cache.ensure_capacity(0, 100)                    # pages 0, 1
    qsa.k_pool.normal_()
    qsa.v_pool.normal_()
    qsa.raw_keys.normal_()
    qsa.block_keys.normal_()
    dn.recurrent_state.normal_()
    dn.conv_ring.normal_()
    cache.slot_tokens[0] = 100
    with pytest.raises(ValueError):
        cache.fork_slot(0, 1, 64)                    # slot 0 is at 100, not 64
    cache.fork_slot(0, 1, 100)
    row = cache.page_table[1, :3].tolist()
    assert row[0] == 0 and row[1] not in (0, 1) and row[2] == cache.null_page
    assert cache.pool.refcount(0) == 2 and cache.pool.refcount(1) == 1 and cache.pool.refcount(row[1]) == 1
    assert torch.equal(qsa.k_pool[row[1]], qsa.k_pool[1]) and torch.equal(qsa.v_pool[row[1]], qsa.v_pool[1])
    assert torch.equal(qsa.raw_keys[1, :100], qsa.raw_keys[0, :100])
    assert torch.equal(qsa.block_keys[1, :1], qsa.block_keys[0, :1])
    assert torch.equal(dn.recurrent_state[1], dn.recurrent_state[0])
    assert torch.equal(dn.conv_ring[1], dn.conv_ring[0])
    assert cache.slot_tokens[1] == 100
    with pytest.raises(ValueError):
        cache.fork_slot(0, 1, 100)                   # slot 1 is not empty
    cache.reset_slot(1)
    assert cache.pool.refcount(0) == 1 and cache.pool.n_free == 6


def test_static_table_fork_copies_pages(qm):
    cache = _cache(qm)                               # identity table: slot 1 owns pages 8..15
    cache.ensure_allocated()
    qsa = cache[3]
    qsa.k_pool.normal_()
    cache.slot_tokens[0] = 70
    cache.fork_slot(0, 1, 70)
    assert torch.equal(qsa.k_pool[8], qsa.k_pool[0]) and torch.equal(qsa.k_pool[9], qsa.k_pool[1])


def test_slot_view_aliases_the_slots_rows(qm):
    cache = _cache(qm, n_pages=8, page_table="pooled")
    view = cache.slot_view(1)
    assert view.batch == 1
    assert view[0].recurrent_state.data_ptr() == cache[0].recurrent_state[1].data_ptr()
    assert view[3].raw_keys.data_ptr() == cache[3].raw_keys[1].data_ptr()
    assert view[3].k_pool is cache[3].k_pool
    view.ensure_capacity(0, 70)                      # maps slot 1 of the parent
    assert cache.page_table[1, :2].tolist() == [0, 1] and view.page_table[0, :2].tolist() == [0, 1]
    view[0].recurrent_state.fill_(1.0)
    assert cache[0].recurrent_state[1].eq(1.0).all() and cache[0].recurrent_state[0].eq(0).all()
    view[3].n_tokens = 70
    cache.commit_slot_view(view)
    assert cache.slot_tokens == [0, 70]
