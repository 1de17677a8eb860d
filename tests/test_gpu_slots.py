"""Slots for continuous batching on the GPU.

Sequences at different positions share one launch: each row of a batched
decode step (QSA and DeltaNet) must equal, bit for bit, the same sequence run
alone in its own cache, with its K/V pages drawn on demand from a pooled page
table. A forked slot continues its source's prefix on shared pages: two rows
given the same token agree bit for bit, and the source's later steps are
unaffected by what the fork writes. The kernels are deterministic per row
(nothing a row computes depends on another row), which is what makes these
comparisons exact.
"""

from __future__ import annotations

import os
import sys

import pytest
import torch

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, HERE)
import inputs as gi  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16
CHUNK = 128


def _model(qm, max_ctx):
    w = dict(gi.qsa_weights(3, 90, BF))
    w.update(gi.dn_weights(0, 91, BF))
    return qm.Qwen4MixModel(qm.MixConfig(), gi.FakeStore(w), device=DEV, max_ctx=max_ctx)


def _cache(qm, model, batch, max_ctx, n_pages=None, scramble=0):
    cache = qm.MixHybridCache(4, model.config, batch, max_ctx, DEV, BF, page_table="pooled", n_pages=n_pages)
    cache.ensure_allocated()
    if scramble:
        # take every page and give them back in a seeded order, so that
        # logical neighbours land on unrelated physical pages
        pages = [cache.pool.alloc() for _ in range(cache.pool.n_pages)]
        g = torch.Generator().manual_seed(scramble)
        for i in torch.randperm(len(pages), generator=g).tolist():
            cache.pool.release(pages[i])
    return cache


def _rand(seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return lambda *s: torch.randn(*s, generator=g, device=DEV).to(BF)  # noqa: E731


def _prefill(model, cache, n, seed):
    """n tokens of seeded projections through the QSA (layer 3) and DeltaNet
    (layer 0) cores of a one-sequence cache, in 128-token chunks."""
    r = _rand(seed)
    cache.ensure_capacity(0, n)
    for off in range(0, n, CHUNK):
        s = min(CHUNK, n - off)
        model.qsa_core(r(1, s, 16 * 512), r(1, s, 512), r(1, s, 512), r(1, s, 512), r(1, s, 128), 3, cache, off)
        model.dn_core(r(1, s, 8192), r(1, s, 4096), r(1, s, 32), r(1, s, 32), 0, cache[0])


def _prefill_slot(model, cache, slot, n, seed):
    view = cache.slot_view(slot)
    _prefill(model, view, n, seed)
    cache.commit_slot_view(view)


def _step_inputs(seed, batch):
    r = _rand(seed)
    return ([r(batch, 1, 16 * 512), r(batch, 1, 512), r(batch, 1, 512), r(batch, 1, 512), r(batch, 1, 128)],
            [r(batch, 1, 8192), r(batch, 1, 4096), r(batch, 1, 32), r(batch, 1, 32)])


def _rows(xs, rows):
    return [x[rows].contiguous() for x in xs]


def _decode(qm, model, cache, positions, qsa_in, dn_in, plan_position=None):
    """One decode step through the preplanned layers; every row at its own
    position. The QSA plan is sized for plan_position (default: the largest
    row position), which also picks its kernel: plans of at most 512 keys take
    the short-context kernel, larger ones the long-context kernel."""
    from importlib import import_module
    plan = import_module(qm.__name__ + ".plan")
    for b, p in enumerate(positions):
        cache.ensure_capacity(b, p + 1)
    qp = plan.QsaDecodePlan(model, cache, 3, max(positions) if plan_position is None else plan_position, BF)
    dp = plan.DnDecodePlan(model, cache, 0, BF)
    pos = torch.tensor(positions, dtype=torch.int32, device=DEV)
    qp.positions.copy_(pos)
    dp.positions.copy_(pos)
    out_q = qp.run(*qsa_in).clone()
    out_d = dp.run(*dn_in).clone()
    for b, p in enumerate(positions):
        cache.slot_tokens[b] = p + 1
    torch.cuda.synchronize()
    return out_q, out_d


@pytest.mark.parametrize("p0, p1", [(2300, 130), (700, 64)])
def test_rows_at_different_positions_match_single_sequences(gpu, p0, p1):
    """Slot 0 at p0 and slot 1 at p1 decode in one launch of each kernel; each
    row equals its sequence decoded alone by a plan of the same size, so by the
    same kernel (pos 2300 scores 35 blocks and picks the top 32; 130 and 64 are
    below the budget)."""
    qm = gpu
    max_ctx = 4096
    model = _model(qm, max_ctx)
    both = _cache(qm, model, 2, max_ctx, scramble=3)
    _prefill_slot(model, both, 0, p0, 11)
    _prefill_slot(model, both, 1, p1, 12)
    alone = []
    for p, seed in ((p0, 11), (p1, 12)):
        c = _cache(qm, model, 1, max_ctx, scramble=4)
        _prefill(model, c, p, seed)
        c.slot_tokens[0] = p
        alone.append(c)
    print(f"rows at {p0} and {p1}", flush=True)
    qsa_in, dn_in = _step_inputs(13, 2)
    got_q, got_d = _decode(qm, model, both, [p0, p1], qsa_in, dn_in)
    for b, (c, p) in enumerate(zip(alone, (p0, p1))):
        want_q, want_d = _decode(qm, model, c, [p], _rows(qsa_in, [b]), _rows(dn_in, [b]), plan_position=p0)
        assert torch.equal(got_q[b], want_q[0]), f"QSA row {b}"
        assert torch.equal(got_d[b], want_d[0]), f"DeltaNet row {b}"
        assert torch.equal(both[0].recurrent_state[b], c[0].recurrent_state[0])
        assert torch.equal(both[0].conv_ring[b], c[0].conv_ring[0])


def test_fork_continues_the_prefix_on_shared_pages(gpu):
    qm = gpu
    max_ctx = 1024
    n = 300                                          # 4 full pages and a partial one
    model = _model(qm, max_ctx)
    cache = _cache(qm, model, 2, max_ctx, n_pages=24, scramble=5)
    _prefill_slot(model, cache, 0, n, 21)
    cache.fork_slot(0, 1, n)
    pt = cache.page_table.cpu()
    assert torch.equal(pt[0, :4], pt[1, :4]) and pt[0, 4] != pt[1, 4]
    assert all(cache.pool.refcount(int(p)) == 2 for p in pt[0, :4])
    print("fork: same token on both rows", flush=True)
    qsa_in, dn_in = _step_inputs(22, 1)
    q, d = _decode(qm, model, cache, [n, n], [x.expand(2, -1, -1).contiguous() for x in qsa_in],
                   [x.expand(2, -1, -1).contiguous() for x in dn_in])
    assert torch.equal(q[0], q[1]) and torch.equal(d[0], d[1])
    assert torch.equal(cache[0].recurrent_state[0], cache[0].recurrent_state[1])
    # the source, continued with other tokens than the fork, equals the
    # sequence run alone: the fork's writes never reach the shared pages
    alone = _cache(qm, model, 1, max_ctx)
    _prefill(model, alone, n, 21)
    alone.slot_tokens[0] = n
    _decode(qm, model, alone, [n], qsa_in, dn_in)
    for t in range(3):
        qsa_in, dn_in = _step_inputs(30 + t, 2)
        q, d = _decode(qm, model, cache, [n + 1 + t] * 2, qsa_in, dn_in)
        wq, wd = _decode(qm, model, alone, [n + 1 + t], _rows(qsa_in, [0]), _rows(dn_in, [0]))
        assert torch.equal(q[0], wq[0]) and torch.equal(d[0], wd[0]), t
    # the fork leaves: its state is cleared, its own pages return, the shared ones stay with slot 0
    keep = cache[0].recurrent_state[0].clone()
    cache.reset_slot(1)
    assert cache[0].recurrent_state[1].eq(0).all() and cache[0].conv_ring[1].eq(0).all()
    assert torch.equal(cache[0].recurrent_state[0], keep)
    assert all(cache.pool.refcount(int(p)) == 1 for p in pt[0, :4])
    assert cache.page_table[1].eq(cache.null_page).all()
