"""The token-mixing halves of a layer stack as one step (MixDecoder): graph
replay against eager launches, the step against the reference-interface layer
methods, and the k-token verify step against k single steps.

Stack: layers 0-2 Gated DeltaNet, layer 3 QSA (full_attention_interval 4),
each wrapped in its hyper-connection mix and reinjection, bf16, batch 1, a
seeded random history of ~1000 tokens in a randomly paged cache.

Bars:
* graph replay == eager launches bit for bit, every replay (with eager work
  and host synchronisations between replays), across a bucket switch (position
  1023 -> 1024) and a block completion, and the caches after the steps
  bit-identical;
* decoder step vs the layer methods (_gated_residual, _linear_attention,
  _full_attention, _reinject): within 2e-2 (the QSA split-K grid is sized for
  the bucket in one and for the position in the other, so partial sums meet
  in another order);
* step_n over k tokens vs k single steps: within 2e-2 (chunk paths vs decode
  paths); the first layer's fp32 state within 1e-3 (both paths see the same
  inputs there), every other cache tensor within 2e-2 (a later layer's inputs
  are the earlier layers' bf16 outputs, which differ by up to that between the
  paths); the conv ring compared as the reference's conv_state (its last K-1
  inputs).
"""

from __future__ import annotations

import ctypes
import os
import sys

import pytest
import torch

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import inputs as gi  # noqa: E402

from margins import rel_err  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16
N_LAYERS = 4
START = 1020


@pytest.fixture(scope="module")
def stack(gpu):
    qm = gpu
    w = {}
    for l in range(N_LAYERS):
        w.update(gi.qsa_weights(l, 100 + l, BF) if (l + 1) % 4 == 0 else gi.dn_weights(l, 100 + l, BF))
        w.update(gi.hc_weights(f"blk.{l}.hc_attn", 200 + l, BF))
    cfg = qm.config.MixConfig()
    model = qm.model.Qwen4MixModel(cfg, gi.FakeStore(w), device=DEV)
    cache = qm.cache.MixHybridCache(N_LAYERS, cfg, batch=1, max_ctx=4096, device=DEV, dtype=BF,
                                    page_table="random", seed=3)
    g = torch.Generator(device=DEV).manual_seed(7)
    for l in range(N_LAYERS):
        lc = cache[l]
        if cfg.is_full_attention(l):
            lc.ensure_qsa(1, BF)
            for t in (lc.k_pool, lc.v_pool, lc.raw_keys):
                t.copy_(torch.randn(t.shape, generator=g, device=DEV).to(t.dtype))
            geom = model.qsa_geom(cache, BF)
            cos, sin = model.rope.get(cache.max_ctx)
            n_blocks = START // cfg.indexer_compress_ratio
            qm.native.call("qm_qsa_pool_blocks", ctypes.byref(geom), lc.raw_keys.data_ptr(),
                           model._dw(l, "indexer.k_norm.weight", torch.float32).data_ptr(), cos.data_ptr(),
                           sin.data_ptr(), 0, n_blocks, lc.block_keys.data_ptr(), qm.native.stream_handle())
            lc.blocks_valid = n_blocks
        else:
            lc.ensure_dn(1, BF)
            lc.recurrent_state.copy_(torch.randn(lc.recurrent_state.shape, generator=g, device=DEV) * 0.02)
            lc.conv_ring.copy_(torch.randn(lc.conv_ring.shape, generator=g, device=DEV).to(BF))
        lc.n_tokens = START
    torch.cuda.synchronize()
    return qm, model, cache


FIELDS = ("conv_ring", "recurrent_state", "k_pool", "v_pool", "raw_keys", "block_keys")


def snapshot(cache):
    snap = []
    for lc in cache.layers:
        t = {f: getattr(lc, f).clone() for f in FIELDS if getattr(lc, f) is not None}
        if lc.conv_ring is not None:
            # the reference's conv_state: the last K-1 inputs (the ring's K-th slot is dead state)
            t["conv_state"] = lc.conv_state.clone()
        snap.append((t, lc.n_tokens, lc.blocks_valid))
    return snap


def restore(cache, snap):
    for lc, (tensors, n, b) in zip(cache.layers, snap):
        for f, t in tensors.items():
            if f in FIELDS:
                getattr(lc, f).copy_(t)
        lc.n_tokens, lc.blocks_valid = n, b
    torch.cuda.synchronize()


def inputs(n, k=1, seed=11):
    r = gi.rng(seed)
    return [gi.normal(r, (1, k, 4 * 2048)).to(BF).to(DEV) for _ in range(n)]


def test_graph_replay_matches_eager_launches(stack):
    qm, model, cache = stack
    snap = snapshot(cache)
    xs = inputs(8)
    print(f"decoder eager, positions {START}..{START + len(xs) - 1}", flush=True)
    dec = qm.decoder.MixDecoder(model, cache)
    eager = [dec.step_eager(x).clone() for x in xs]
    torch.cuda.synchronize()
    after_eager = snapshot(cache)
    assert dec.position == START + len(xs)

    restore(cache, snap)
    print("decoder graph replay", flush=True)
    dec = qm.decoder.MixDecoder(model, cache)
    junk = torch.randn(512, 512, device=DEV)
    for i, x in enumerate(xs):
        out = dec.step(x)
        torch.cuda.synchronize()
        # eager work of the program's own between replays
        junk = torch.tanh(junk @ junk.t() * 1e-3)
        assert torch.equal(out, eager[i]), f"replay {i} (position {START + i}) differs from the eager step"
    assert len(dec._graphs) == 2, "positions 1020..1027 span two buckets"
    torch.cuda.synchronize()
    for l, ((a, na, ba), (b, nb, bb)) in enumerate(zip(after_eager, snapshot(cache))):
        assert (na, ba) == (nb, bb)
        for f in a:
            assert torch.equal(a[f], b[f]), f"layer {l} {f} differs after graph steps"
    restore(cache, snap)


def test_decoder_step_matches_layer_methods(stack):
    qm, model, cache = stack
    snap = snapshot(cache)
    xs = inputs(3, seed=12)
    dec = qm.decoder.MixDecoder(model, cache)
    got = [dec.step(x).clone() for x in xs]
    torch.cuda.synchronize()
    restore(cache, snap)
    print("layer methods, eager", flush=True)
    for i, x in enumerate(xs):
        h = x
        for l in range(N_LAYERS):
            mixed, _, inject = model._gated_residual(h, l, "attn")
            if model.config.is_full_attention(l):
                branch = model._full_attention(mixed, l, None, None, cache, START + i)
            else:
                branch = model._linear_attention(mixed, l, cache)
            h = model._reinject(h, branch, inject)
        torch.cuda.synchronize()
        assert rel_err(got[i], h, 2e-2) < 2e-2, f"step {i}"
    restore(cache, snap)


@pytest.mark.parametrize("k", [3, 6])
def test_step_n_matches_single_steps(stack, k):
    qm, model, cache = stack
    snap = snapshot(cache)
    x = inputs(1, k=k, seed=13)[0]
    print(f"step_n k={k}", flush=True)
    dec = qm.decoder.MixDecoder(model, cache)
    rows = dec.step_n(x).clone()
    torch.cuda.synchronize()
    after_n = snapshot(cache)
    assert dec.position == START + k and int(dec.positions[0]) == START + k
    restore(cache, snap)
    dec = qm.decoder.MixDecoder(model, cache)
    singles = [dec.step_eager(x[:, i:i + 1]).clone() for i in range(k)]
    torch.cuda.synchronize()
    for i in range(k):
        assert rel_err(rows[:, i:i + 1], singles[i], 2e-2) < 2e-2, f"row {i}"
    for l, ((a, na, _), (b, nb, _)) in enumerate(zip(after_n, snapshot(cache))):
        assert na == nb == START + k
        for f in a:
            if f == "conv_ring":
                continue   # compared as conv_state: the chunk path does not write the dead slot
            if f == "recurrent_state" and l == 0:
                # same inputs on both paths: the fp32 state bar
                assert (a[f] - b[f]).abs().max().item() < 1e-3, f"layer {l}"
            else:
                assert rel_err(a[f], b[f], 2e-2) < 2e-2, f"layer {l} {f}"
    restore(cache, snap)


def _export(cache):
    """The device caches as the reference's layer caches (reference/cache.py:19-29), on the CPU."""
    from oracle.cache import OracleHybridCache
    oc = OracleHybridCache(N_LAYERS)
    for l, lc in enumerate(cache.layers):
        if lc.conv_ring is not None:
            oc[l].conv_state = lc.conv_state.cpu()
            oc[l].recurrent_state = lc.recurrent_state.cpu().clone()
        if lc.k_pool is not None:
            oc[l].keys, oc[l].values = lc.keys.cpu(), lc.values.cpu()
            oc[l].indexer_keys = lc.indexer_keys.cpu()
    return oc


def _oracle_chain(model, oc, h, position):
    """reference/model.py:443-452 for the token-mixing halves, every piece the
    oracle's: _gated_residual, the branch, _reinject, for the rows of h at
    position, position + 1, ... (the cores take their chunk paths for k > 1)."""
    from oracle.config import OracleConfig
    from oracle.layers import RotaryEmbedding
    from oracle.mixing import OracleMixer
    om = OracleMixer(OracleConfig(), model.store)
    k = h.shape[1]
    rot = RotaryEmbedding(64, 1e7, [11, 11, 10])
    p = torch.arange(position + k)[None]
    cos, sin = rot(p[None].expand(3, -1, -1))
    for l in range(N_LAYERS):
        mixed, _, inject = om._gated_residual(h, l, "attn")
        if model.config.is_full_attention(l):
            branch = om._full_attention(mixed, l, cos, sin, oc, position)
        else:
            branch = om._linear_attention(mixed, l, oc)
        h = om._reinject(h, branch, inject)
    return h


@pytest.mark.parametrize("k", [1, 3])
def test_decoder_matches_oracle_chain(stack, k):
    """MixDecoder.step (k = 1, from the graph) and step_n (k = 3) against the
    all-oracle chain on the CPU over the same exported history: the residual
    within 2e-2; the first layer's fp32 state within 1e-3 (its inputs differ
    from the oracle's only by the rounding of the mix and the projections), the
    other states, the appended keys/values and the conv windows (which hold the
    bf16 projections each side computed) within 2e-2."""
    qm, model, cache = stack
    snap = snapshot(cache)
    x = inputs(1, k=k, seed=21)[0]
    oc = _export(cache)
    print(f"decoder vs oracle chain k={k}", flush=True)
    want = _oracle_chain(model, oc, x.cpu(), START)
    dec = qm.decoder.MixDecoder(model, cache)
    got = dec.step(x).clone() if k == 1 else dec.step_n(x).clone()
    torch.cuda.synchronize()
    assert rel_err(got, want, 2e-2) < 2e-2, rel_err(got, want)
    got_oc = _export(cache)
    for l in range(N_LAYERS):
        if model.config.is_full_attention(l):
            assert rel_err(got_oc[l].keys[:, :, -k:], oc[l].keys[:, :, -k:], 2e-2) < 2e-2, l
            assert rel_err(got_oc[l].values[:, :, -k:], oc[l].values[:, :, -k:], 2e-2) < 2e-2, l
            assert got_oc[l].indexer_keys.shape == oc[l].indexer_keys.shape
        else:
            bar = 1e-3 if l == 0 else None
            diff = (got_oc[l].recurrent_state - oc[l].recurrent_state).abs().max().item()
            if bar is not None:
                assert diff < bar, (l, diff)
            else:
                assert rel_err(got_oc[l].recurrent_state, oc[l].recurrent_state, 2e-2) < 2e-2, l
            assert rel_err(got_oc[l].conv_state, oc[l].conv_state, 2e-2) < 2e-2, l
    dec.check_handoffs()
    restore(cache, snap)


def test_seek_then_step_n_matches_a_run_at_that_position(stack):
    """After seek(p) the k-token step runs every layer at p: the same residual
    and caches, bit for bit, as a decoder whose layers were already at p."""
    qm, model, cache = stack
    snap = snapshot(cache)
    x = inputs(1, k=3, seed=22)[0]
    target = START + 2
    print("seek then step_n", flush=True)
    dec = qm.decoder.MixDecoder(model, cache)
    dec.seek(target)
    assert all(cache[l].n_tokens == target for l in range(N_LAYERS))
    got = dec.step_n(x).clone()
    torch.cuda.synchronize()
    after_seek = snapshot(cache)
    restore(cache, snap)
    for l in range(N_LAYERS):
        cache[l].n_tokens = target
    dec = qm.decoder.MixDecoder(model, cache)
    want = dec.step_n(x).clone()
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    for l, ((a, na, _), (b, nb, _)) in enumerate(zip(after_seek, snapshot(cache))):
        assert na == nb == target + 3
        for f in a:
            assert torch.equal(a[f], b[f]), f"layer {l} {f}"
    restore(cache, snap)


def test_reset_rewinds_in_place(stack):
    qm, model, cache = stack
    snap = snapshot(cache)
    dec = qm.decoder.MixDecoder(model, cache)
    ptrs = [lc.k_pool.data_ptr() if lc.k_pool is not None else lc.conv_ring.data_ptr() for lc in cache.layers]
    dec.reset()
    assert dec.position == 0 and int(dec.positions[0]) == 0
    for lc, p in zip(cache.layers, ptrs):
        assert lc.n_tokens == 0
        assert (lc.k_pool.data_ptr() if lc.k_pool is not None else lc.conv_ring.data_ptr()) == p
        for f in FIELDS:
            t = getattr(lc, f)
            if t is not None:
                assert not t.any()
    out = dec.step(inputs(1, seed=14)[0])
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all() and dec.position == 1
    restore(cache, snap)


ROWS = (1100, 317)      # row positions: buckets 2047 and 1023 when alone


def _two_row_cache(qm, model, seed):
    """Two sequences with seeded random histories of ROWS tokens, randomly paged."""
    cfg = model.config
    cache = qm.cache.MixHybridCache(N_LAYERS, cfg, batch=2, max_ctx=4096, device=DEV, dtype=BF,
                                    page_table="random", seed=5)
    g = torch.Generator(device=DEV).manual_seed(seed)
    for l in range(N_LAYERS):
        lc = cache[l]
        if cfg.is_full_attention(l):
            lc.ensure_qsa(2, BF)
            for t in (lc.k_pool, lc.v_pool, lc.raw_keys):
                t.copy_(torch.randn(t.shape, generator=g, device=DEV).to(t.dtype))
            geom = model.qsa_geom(cache, BF)
            cos, sin = model.rope.get(cache.max_ctx)
            # blocks past a row's position are pooled too and never read by it
            n_blocks = max(ROWS) // cfg.indexer_compress_ratio
            qm.native.call("qm_qsa_pool_blocks", ctypes.byref(geom), lc.raw_keys.data_ptr(),
                           model._dw(l, "indexer.k_norm.weight", torch.float32).data_ptr(), cos.data_ptr(),
                           sin.data_ptr(), 0, n_blocks, lc.block_keys.data_ptr(), qm.native.stream_handle())
            lc.blocks_valid = n_blocks
        else:
            lc.ensure_dn(2, BF)
            lc.recurrent_state.copy_(torch.randn(lc.recurrent_state.shape, generator=g, device=DEV) * 0.02)
            lc.conv_ring.copy_(torch.randn(lc.conv_ring.shape, generator=g, device=DEV).to(BF))
        lc.n_tokens = max(ROWS)
    cache.slot_tokens[:] = list(ROWS)
    torch.cuda.synchronize()
    return cache


def test_rows_at_different_positions_match_single_rows(stack):
    """A two-row decoder with its rows at positions 1100 and 317 (continuous
    batching: one graph, the larger row's bucket) against one single-row
    decoder per row over a slot view of an identical cache (each row's own
    bucket): the residual of every row bit for bit over three steps, the last
    of which completes row 1's block 4 (position 319); positions advance per
    row, and the k-token step refuses rows at different positions."""
    qm, model, _ = stack
    c = model.config
    batch_cache = _two_row_cache(qm, model, 17)
    single_cache = _two_row_cache(qm, model, 17)
    dec = qm.decoder.MixDecoder(model, batch_cache, positions=ROWS)
    singles = [qm.decoder.MixDecoder(model, single_cache.slot_view(r)) for r in range(2)]
    assert [s.position for s in singles] == list(ROWS)
    g = torch.Generator(device=DEV).manual_seed(11)
    for step in range(3):
        print(f"rows at {dec.row_positions}: step {step}", flush=True)
        h = torch.randn(2, 1, c.hc_count * c.hidden_size, generator=g, device=DEV).to(BF)
        got = dec.step(h).clone()
        for r in range(2):
            want = singles[r].step(h[r:r + 1]).clone()
            assert torch.equal(got[r], want[0]), (step, r, rel_err(got[r], want[0]))
    assert dec.row_positions == [p + 3 for p in ROWS]
    assert batch_cache.slot_tokens == [p + 3 for p in ROWS]
    assert dec.positions.cpu().tolist() == [p + 3 for p in ROWS]
    with pytest.raises(ValueError):
        dec.step_n(torch.zeros(2, 2, c.hc_count * c.hidden_size, device=DEV))
    dec.seek(list(ROWS))
    assert dec.positions.cpu().tolist() == list(ROWS) and dec.position == max(ROWS)
    dec.seek(500)
    assert dec.positions.cpu().tolist() == [500, 500] and dec.row_positions == [500, 500]


def _dn_state(cache):
    return [(lc.recurrent_state.clone(), lc.conv_ring.clone()) for lc in cache.layers if lc.recurrent_state is not None]


def test_captured_step_n_matches_eager_step_n(stack):
    """The verify step replayed from its graph runs the layer methods' kernels:
    the same residual rows and caches, bit for bit, over two replays."""
    qm, model, cache = stack
    snap = snapshot(cache)
    xs = inputs(2, k=3, seed=31)
    print("eager step_n k=3, twice", flush=True)
    dec = qm.decoder.MixDecoder(model, cache)
    eager = [dec.step_n(x).clone() for x in xs]
    torch.cuda.synchronize()
    after_eager = snapshot(cache)
    restore(cache, snap)
    print("captured step_n k=3, twice", flush=True)
    dec = qm.decoder.MixDecoder(model, cache)
    for x, want in zip(xs, eager):
        got = dec.step_n_graph(x).clone()
        torch.cuda.synchronize()
        assert torch.equal(got, want)
    assert dec.position == START + 6 and int(dec.positions.item()) == START + 6
    for l, ((a, na, ba), (b, nb, bb)) in enumerate(zip(after_eager, snapshot(cache))):
        assert na == nb == START + 6 and ba == bb
        for f in a:
            assert torch.equal(a[f], b[f]), f"layer {l} {f}"
    restore(cache, snap)


def test_rewound_verify_step_matches_a_fresh_one(stack):
    """Speculation: snapshot, verify k = 4 drafts from the graph, restore, then
    commit j = 2 of them from the graph of j: the residual rows, the DeltaNet
    states and rings and every K/V page row up to the new position equal, bit
    for bit, a decoder that verified only those 2; a single graph step after
    either agrees bit for bit too. The snapshot reuses its buffers on the
    second call."""
    qm, model, cache = stack
    snap = snapshot(cache)
    x4 = inputs(1, k=4, seed=41)[0]
    x1 = inputs(1, k=1, seed=42)[0]
    print("verify 4, rewind, commit 2", flush=True)
    dec = qm.decoder.MixDecoder(model, cache)
    keep = dec.snapshot()
    ptrs = {n: t.data_ptr() for n, t in keep["tensors"].items()}
    dec.step_n_graph(x4)
    assert dec.position == START + 4
    dec.restore(keep)
    assert dec.position == START and int(dec.positions.item()) == START
    assert all(cache[l].n_tokens == START for l in range(N_LAYERS))
    got2 = dec.step_n_graph(x4[:, :2]).clone()
    got_state = _dn_state(cache)
    got_step = dec.step(x1).clone()
    torch.cuda.synchronize()
    got_after = snapshot(cache)
    got_kv = [(lc.keys.clone(), lc.values.clone()) for lc in cache.layers if lc.k_pool is not None]
    keep2 = dec.snapshot(into=keep)
    assert keep2 is keep and all(t.data_ptr() == ptrs[n] for n, t in keep["tensors"].items())

    restore(cache, snap)
    print("fresh commit 2", flush=True)
    dec = qm.decoder.MixDecoder(model, cache)
    want2 = dec.step_n_graph(x4[:, :2]).clone()
    want_state = _dn_state(cache)
    want_step = dec.step(x1).clone()
    torch.cuda.synchronize()
    want_after = snapshot(cache)
    want_kv = [(lc.keys.clone(), lc.values.clone()) for lc in cache.layers if lc.k_pool is not None]
    assert torch.equal(got2, want2)
    for (a, b), (c, d) in zip(got_state, want_state):
        assert torch.equal(a, c) and torch.equal(b, d)
    assert torch.equal(got_step, want_step)
    # K/V up to the committed position (rows past it hold the rejected drafts', never read)
    for (a, b), (c, d) in zip(got_kv, want_kv):
        assert a.shape[2] == START + 3 and torch.equal(a, c) and torch.equal(b, d)
    n_blocks = (START + 3) // model.config.indexer_compress_ratio
    for l, ((a, na, ba), (b, nb, bb)) in enumerate(zip(got_after, want_after)):
        assert na == nb == START + 3 and ba == bb
        for f in a:
            if f in ("k_pool", "v_pool"):
                continue
            if f == "raw_keys":
                assert torch.equal(a[f][:, :START + 3], b[f][:, :START + 3]), f"layer {l} raw_keys"
            elif f == "block_keys":
                # a block a rejected draft completed is pooled again when a token completes it
                assert torch.equal(a[f][:, :n_blocks], b[f][:, :n_blocks]), f"layer {l} block_keys"
            else:
                assert torch.equal(a[f], b[f]), f"layer {l} {f}"
    dec.check_handoffs()
    restore(cache, snap)
