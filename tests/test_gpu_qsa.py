"""QSA on the GPU against the oracle and the reference's goldens.

Bar (north star): selected block indices and page gathers bit-exact; bf16
outputs within 2e-2 max relative error (max |got - want| / max |want|).
Selection parity is checked with the exact projection bits the reference saw
(stored in the fixtures), so the comparison covers the kernels, not the GEMMs.
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import selection as sel
from oracle.cache import OracleHybridCache
from oracle.config import OracleConfig
from oracle.layers import RotaryEmbedding, apply_rotary, rms_norm
from oracle.mixing import OracleMixer

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, HERE)
import inputs as gi  # noqa: E402

from margins import rel_err  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda"
OUT_TOL = 2e-2
META = json.load(open(os.path.join(HERE, "golden_meta.json")))
ROT = RotaryEmbedding(64, 1e7, [11, 11, 10])


def tables(n):
    p = torch.arange(n)[None]
    return ROT(p[None].expand(3, -1, -1))


def _model_and_cache(gpu, store, dtype, max_ctx, cfg=None, page_table="random", batch=1):
    qm = gpu
    cfg = cfg or qm.MixConfig()
    model = qm.Qwen4MixModel(cfg, store, device=DEV, max_ctx=max_ctx)
    cache = qm.MixHybridCache(4, cfg, batch, max_ctx, DEV, dtype, page_table=page_table, seed=5)
    return model, cache


def _oracle_core(cfg, store, hidden, cos, sin, keys, values, idx_keys, pos, layer=3):
    """The oracle's pre-projection QSA output and per-query selected blocks."""
    m = OracleMixer(cfg, store)
    q, k, v, gate = m.qkv_prep(hidden, layer, cos, sin)
    K = torch.cat([keys, k], 2) if keys is not None else k
    V = torch.cat([values, v], 2) if values is not None else v
    kv_len = K.shape[2]
    oc = OracleHybridCache(layer + 1)
    oc[layer].indexer_keys = idx_keys
    mask = m._indexer_mask(hidden, layer, cos, sin, oc, kv_len, pos)
    n_t = hidden.shape[1]
    kpos = torch.arange(kv_len)
    qpos = torch.arange(n_t)[:, None] + pos
    allowed = (kpos[None, :] <= qpos)[None, None] & mask
    out = m.attention_core(q, K, V, allowed, hidden.dtype)
    out = out.transpose(1, 2).reshape(hidden.shape[0], n_t, -1) * torch.sigmoid(gate)
    chosen = []
    for b in range(hidden.shape[0]):
        rows = []
        for i in range(n_t):
            p = pos + i
            n_el = (p + 1) // cfg.indexer_compress_ratio
            rows.append(sorted(j for j in range(n_el) if bool(mask[b, 0, i, j * cfg.indexer_compress_ratio])))
        chosen.append(rows)
    return out, k, v, chosen


def _projections(store, hidden, layer=3):
    g = lambda s: store.get(f"blk.{layer}.{s}")  # noqa: E731
    return [F.linear(hidden, g(n)).contiguous() for n in
            ("attn_q.weight", "attn_k.weight", "attn_v.weight", "indexer.q_proj.weight", "indexer.k_proj.weight")]


def _got_sets(lc):
    ids, n = lc.last_ids.cpu(), lc.last_n_sel.cpu()
    return [[sorted(ids[b, i, : n[b, i]].tolist()) for i in range(ids.shape[1])] for b in range(ids.shape[0])]


@pytest.mark.parametrize("tag", ["cfg3", "cfg3b", "cfg1"])
def test_indexer_stages_and_selection_match_reference(gpu, tag):
    """Pooled block keys and indexer queries bit-exact vs the oracle, selected
    set bit-exact vs the reference, fed the reference's own projection bits."""
    m = META[tag]
    z = np.load(os.path.join(HERE, f"{tag}.npz"))
    dtype = torch.float32 if m["dtype"] == "torch.float32" else torch.bfloat16
    pos = m["pos"]
    store = gi.FakeStore(gi.qsa_weights(3, m["qsa_seeds"][0], dtype))
    _, _, idx_keys = gi.qsa_past(m["qsa_seeds"][1], pos, dtype)
    if dtype == torch.bfloat16:
        iq = gi.from_bf16_bits(z["idx_q_raw"]).reshape(1, 1, -1)
        ik = gi.from_bf16_bits(z["idx_k_raw"]).reshape(1, 1, -1)
    else:
        iq = torch.from_numpy(z["idx_q_raw"]).reshape(1, 1, -1)
        ik = torch.from_numpy(z["idx_k_raw"]).reshape(1, 1, -1)
    cos, sin = gi.golden_rope(ROT, pos + 1)
    model, cache = _model_and_cache(gpu, store, dtype, pos + 64)
    cache[3].indexer_keys = idx_keys.to(DEV)
    print(f"indexer {tag} pos={pos}", flush=True)
    model.qsa_core(None, None, None, iq.to(DEV), ik.to(DEV), 3, cache, pos, cos.to(DEV), sin.to(DEV), attend=False)
    lc = cache[3]
    # oracle stages on the same bits
    om = OracleMixer(OracleConfig(), store)
    q_want = apply_rotary(rms_norm(iq.reshape(1, 1, 4, 128), store.get("blk.3.indexer.q_norm.weight"), 1e-6),
                          cos[:, -1:], sin[:, -1:], unsqueeze_dim=2)
    assert torch.equal(lc.last_iq.cpu(), q_want.float()), "indexer query not bit-exact"
    n_blocks = (pos + 1) // 64
    pooled = om.indexer_pooled(torch.cat([idx_keys, ik], 1), 3, cos, sin, n_blocks)
    got_pooled = lc.block_keys_ref[:, :n_blocks].cpu()
    assert torch.equal(got_pooled, pooled.float()), \
        f"pooled keys differ in {(got_pooled != pooled).sum().item()} entries"
    got = _got_sets(lc)[0][0]
    assert got == sorted(z["selected"].tolist()), "selected blocks differ from the reference"


@pytest.mark.parametrize("pos,dtype", [(192, torch.float32), (1984, torch.bfloat16), (4032, torch.bfloat16),
                                       (8128, torch.bfloat16), (130, torch.bfloat16), (2047, torch.bfloat16),
                                       (0, torch.bfloat16), (63, torch.bfloat16),
                                       # more than 128 eligible blocks: top-k by radix select
                                       (9000, torch.bfloat16), (20000, torch.bfloat16)])
def test_decode_core_matches_oracle(gpu, pos, dtype):
    cfg = OracleConfig()
    store = gi.FakeStore(gi.qsa_weights(3, 61, dtype))
    keys, values, idx_keys = gi.qsa_past(62, pos, dtype)
    hidden = gi.normal(gi.rng(63), (1, 1, gi.HIDDEN)).to(dtype)
    cos, sin = tables(pos + 1)
    print(f"decode core pos={pos} dtype={dtype}", flush=True)
    want, k_new, v_new, chosen = _oracle_core(cfg, store, hidden, cos, sin, keys if pos else None,
                                              values if pos else None, idx_keys, pos)
    model, cache = _model_and_cache(gpu, store, dtype, pos + 128)
    if pos:
        cache[3].keys, cache[3].values, cache[3].indexer_keys = keys.to(DEV), values.to(DEV), idx_keys.to(DEV)
    qg, k, v, iq, ik = (t.to(DEV) for t in _projections(store, hidden))
    got = model.qsa_core(qg, k, v, iq, ik, 3, cache, pos, cos.to(DEV), sin.to(DEV))
    assert _got_sets(cache[3]) == chosen
    assert rel_err(got, want, OUT_TOL) < OUT_TOL
    # the appended token sits at its page slot, bit-exact (bf16 of the roped key)
    P = 64
    page = int(cache.page_table[0, pos // P])
    assert torch.equal(cache[3].page_row("k", page, pos % P).cpu(), k_new[0, :, 0].to(torch.bfloat16))
    assert torch.equal(cache[3].page_row("v", page, pos % P).cpu(), v_new[0, :, 0].to(torch.bfloat16))


@pytest.mark.parametrize("pos", [8128, 4032, 9000])
def test_decode_selection_ties_go_to_lower_index(gpu, pos):
    """Exactly tied block scores at the top-k boundary, through the one-launch
    decode: the indexer query's roped dims are zero (their projection rows
    zeroed), and the raw indexer keys repeat every 20 blocks, so the repeated
    blocks' pooled keys agree outside the roped dims and score bit-identically;
    of a tied group the lower block indices must be selected (the oracle's
    stable descending sort). 8128 and 4032 take
    the kernel's ballot search over at most 128 blocks, 9000 its radix
    select."""
    cfg = OracleConfig()
    dtype = torch.bfloat16
    store = gi.FakeStore(gi.qsa_weights(3, 71, dtype))
    wq = store.get("blk.3.indexer.q_proj.weight")
    for h in range(wq.shape[0] // 128):
        wq[h * 128: h * 128 + cfg.rope_dim] = 0
    keys, values, idx_keys = gi.qsa_past(72, pos, dtype)
    n_blocks = pos // 64
    for j in range(20, n_blocks):
        idx_keys[:, 64 * j: 64 * j + 64] = idx_keys[:, 64 * (j % 20): 64 * (j % 20) + 64]
    hidden = gi.normal(gi.rng(73), (1, 1, gi.HIDDEN)).to(dtype)
    cos, sin = tables(pos + 1)
    print(f"decode ties pos={pos}", flush=True)
    want, _, _, chosen = _oracle_core(cfg, store, hidden, cos, sin, keys, values, idx_keys, pos)
    model, cache = _model_and_cache(gpu, store, dtype, pos + 128)
    cache[3].keys, cache[3].values, cache[3].indexer_keys = keys.to(DEV), values.to(DEV), idx_keys.to(DEV)
    qg, k, v, iq, ik = (t.to(DEV) for t in _projections(store, hidden))
    got = model.qsa_core(qg, k, v, iq, ik, 3, cache, pos, cos.to(DEV), sin.to(DEV))
    # the tie really sits at the boundary: the k-th and (k+1)-th scores are
    # equal (no block completes at these positions: every eligible block is
    # pooled from the past keys)
    om = OracleMixer(cfg, store)
    q = om.indexer_query(hidden, 3, cos, sin)
    sc = om.indexer_scores(q, om.indexer_pooled(idx_keys, 3, cos, sin, (pos + 1) // 64)).flatten()
    top = torch.sort(sc, descending=True).values
    assert top[31] == top[32], "no tie at the top-k boundary"
    assert _got_sets(cache[3]) == chosen
    assert rel_err(got, want, OUT_TOL) < OUT_TOL


def test_page_gather_round_trip_is_bit_exact(gpu):
    store = gi.FakeStore(gi.qsa_weights(3, 64, torch.bfloat16))
    keys, values, idx = gi.qsa_past(65, 1000, torch.bfloat16)
    model, cache = _model_and_cache(gpu, store, torch.bfloat16, 1024)
    cache[3].keys, cache[3].values, cache[3].indexer_keys = keys.to(DEV), values.to(DEV), idx.to(DEV)
    assert torch.equal(cache[3].keys.cpu(), keys.to(torch.bfloat16).float())
    assert torch.equal(cache[3].values.cpu(), values)
    assert torch.equal(cache[3].indexer_keys.cpu(), idx)
    # the page table really is a permutation: no two logical pages share a page
    pt = cache.page_table[0].cpu()
    assert len(set(pt.tolist())) == pt.numel()


@pytest.mark.parametrize("tag", ["cfg1", "cfg3", "cfg3b"])
def test_decode_layer_matches_golden_reference(gpu, tag):
    m = META[tag]
    z = np.load(os.path.join(HERE, f"{tag}.npz"))
    dtype = torch.float32 if m["dtype"] == "torch.float32" else torch.bfloat16
    pos = m["pos"]
    store = gi.FakeStore(gi.qsa_weights(3, m["qsa_seeds"][0], dtype))
    keys, values, idx_keys = gi.qsa_past(m["qsa_seeds"][1], pos, dtype)
    hidden = gi.hidden_states(m["hidden_seed"], 1, dtype)
    cos, sin = gi.golden_rope(ROT, pos + 1)
    model, cache = _model_and_cache(gpu, store, dtype, pos + 64)
    cache[3].keys, cache[3].values, cache[3].indexer_keys = keys.to(DEV), values.to(DEV), idx_keys.to(DEV)
    print(f"golden layer {tag}", flush=True)
    y = model._full_attention(hidden.to(DEV), 3, cos.to(DEV), sin.to(DEV), cache, pos)
    want = torch.from_numpy(z["qsa_out"])
    flat = y.float().reshape(-1).cpu()
    stride = max(1, flat.numel() // want.numel())
    assert rel_err(flat[::stride][: want.numel()], want, OUT_TOL) < OUT_TOL


def test_prefill_chunk_matches_golden_reference(gpu):
    """Config 5: 128 queries at 32640..32767, per-query top-32 and causal tails."""
    m = META["cfg5"]
    z = np.load(os.path.join(HERE, "cfg5.npz"))
    past, seq = m["past"], m["seq"]
    dtype = torch.bfloat16
    store = gi.FakeStore(gi.qsa_weights(3, m["qsa_seeds"][0], dtype))
    keys, values, idx_keys = gi.qsa_past(m["qsa_seeds"][1], past, dtype)
    hidden = gi.hidden_states(m["hidden_seed"], seq, dtype)
    cos, sin = gi.golden_rope(ROT, past + seq)
    model, cache = _model_and_cache(gpu, store, dtype, past + seq)
    cache[3].keys, cache[3].values, cache[3].indexer_keys = keys.to(DEV), values.to(DEV), idx_keys.to(DEV)
    qg, k, v, _, _ = _projections(store, hidden)
    iq = gi.from_bf16_bits(z["idx_q_raw"]).reshape(1, seq, -1)
    ik = gi.from_bf16_bits(z["idx_k_raw"]).reshape(1, seq, -1)
    print("prefill chunk 32640+128", flush=True)
    got = model.qsa_core(qg.to(DEV), k.to(DEV), v.to(DEV), iq.to(DEV), ik.to(DEV), 3, cache, past, cos.to(DEV),
                         sin.to(DEV))
    sets = _got_sets(cache[3])[0]
    for i in range(seq):
        want_ids = z["selected"][i]
        assert sets[i] == sorted(want_ids[want_ids >= 0].tolist()), f"query {i}"
    want = torch.from_numpy(z["qsa_core"])
    flat = got.float().reshape(-1).cpu()
    stride = max(1, flat.numel() // want.numel())
    assert rel_err(flat[::stride][: want.numel()], want, OUT_TOL) < OUT_TOL
    # every output element against the oracle's attention (reference/model.py:
    # 367-383: fp32 scores and softmax, weights @ v in fp32, the sigmoid gate)
    # on the same projections, over the reference's own selected blocks plus
    # each row's causal tail
    om = OracleMixer(OracleConfig(), store)
    c, s_ = cos[:, -seq:], sin[:, -seq:]
    q_, gate = torch.chunk(qg.view(1, seq, -1, 512), 2, dim=-1)
    q_ = apply_rotary(rms_norm(q_, store.get("blk.3.attn_q_norm.weight"), 1e-6).transpose(1, 2), c, s_)
    k_ = apply_rotary(rms_norm(k.view(1, seq, -1, 256), store.get("blk.3.attn_k_norm.weight"), 1e-6)
                      .transpose(1, 2), c, s_)
    v_ = v.view(1, seq, -1, 256).transpose(1, 2)
    K, V = torch.cat([keys, k_], 2), torch.cat([values, v_], 2)
    kv_len = past + seq
    allowed = torch.zeros(1, 1, seq, kv_len, dtype=torch.bool)
    kpos = torch.arange(kv_len)
    for i in range(seq):
        p = past + i
        for j in z["selected"][i][z["selected"][i] >= 0].tolist():
            allowed[0, 0, i, j * 64:(j + 1) * 64] = True
        allowed[0, 0, i] |= (kpos >= ((p + 1) // 64) * 64) & (kpos <= p)
    full = om.attention_core(q_, K, V, allowed, dtype).transpose(1, 2).reshape(1, seq, -1)
    full = full * torch.sigmoid(gate.reshape(1, seq, -1))
    assert rel_err(got, full, OUT_TOL) < OUT_TOL


@pytest.mark.parametrize("past,seq,batch,dtype,shared", [(0, 37, 1, torch.bfloat16, False),
                                                          (2000, 96, 1, torch.bfloat16, False),
                                                          (4030, 70, 2, torch.float32, False),
                                                          (8100, 128, 1, torch.bfloat16, False),
                                                          (3000, 300, 1, torch.bfloat16, False),
                                                          (2000, 96, 1, torch.bfloat16, True)])
def test_prefill_chunk_attention_matches_oracle(gpu, past, seq, batch, dtype, shared):
    """The block-major chunk attention against the oracle, with the entries
    filed by the selection (qm_qsa_select_chunk + qm_qsa_attend_chunk_filed)
    and by the attention (qm_qsa_select + qm_qsa_attend_chunk), and against
    the per-row item attention (qm_qsa_attend) on the same chunk:
    a ragged last tile, chunks that complete blocks part-way (rows whose tail
    block another row has selected), a batch of two with its own pages, a
    chunk of more rows than one launch takes (300), and rows that all carry the
    same hidden state, so that every row selects (nearly) the same blocks and
    one workgroup holds ~96 entries of a block."""
    cfg = OracleConfig()
    store = gi.FakeStore(gi.qsa_weights(3, 90, dtype))
    pasts = [gi.qsa_past(91 + b, past, dtype) for b in range(batch)]
    keys, values, idx_keys = (torch.cat([p[i] for p in pasts]) for i in range(3))
    hidden = gi.normal(gi.rng(93), (batch, seq, gi.HIDDEN)).to(dtype)
    if shared:
        hidden = hidden[:, :1].expand(batch, seq, gi.HIDDEN).contiguous()
    cos, sin = tables(past + seq)
    print(f"prefill chunk past={past} seq={seq} batch={batch} {dtype} shared={shared}", flush=True)
    want, _, _, chosen = _oracle_core(cfg, store, hidden, cos, sin, keys if past else None,
                                      values if past else None, idx_keys, past)
    outs = []
    for chunked, fused in ((True, True), (True, False), (False, False)):
        model, cache = _model_and_cache(gpu, store, dtype, past + seq + 64, batch=batch)
        model.fuse_chunk_select = fused
        if not chunked:
            model.chunk_attend_fits = lambda cache: False
        if past:
            cache[3].keys, cache[3].values, cache[3].indexer_keys = keys.to(DEV), values.to(DEV), idx_keys.to(DEV)
        qg, k, v, iq, ik = (t.to(DEV) for t in _projections(store, hidden))
        got = model.qsa_core(qg, k, v, iq, ik, 3, cache, past, cos.to(DEV), sin.to(DEV))
        assert _got_sets(cache[3]) == chosen
        assert rel_err(got, want, OUT_TOL) < OUT_TOL, ("chunked" if chunked else "items", fused)
        outs.append(got.float())
    assert torch.equal(outs[0], outs[1])           # the same entries either way
    assert rel_err(outs[0], outs[2], 1e-2) < 1e-2


def test_small_ratio_several_blocks_per_page(gpu):
    """ratio 4 < page 64 (the reference checkpoint's ratio), budget 64 -> top-16."""
    qm = gpu
    cfg = OracleConfig(indexer_compress_ratio=4, indexer_budget=64)
    mcfg = qm.MixConfig(indexer_compress_ratio=4, indexer_budget=64)
    dtype = torch.bfloat16
    store = gi.FakeStore(gi.qsa_weights(3, 66, dtype))
    for pos in (3, 50, 130, 301):
        keys, values, idx_keys = gi.qsa_past(67, pos, dtype)
        hidden = gi.normal(gi.rng(68 + pos), (1, 1, gi.HIDDEN)).to(dtype)
        cos, sin = tables(pos + 1)
        want, _, _, chosen = _oracle_core(cfg, store, hidden, cos, sin, keys, values, idx_keys, pos)
        model, cache = _model_and_cache(gpu, store, dtype, 384, cfg=mcfg)
        cache[3].keys, cache[3].values, cache[3].indexer_keys = keys.to(DEV), values.to(DEV), idx_keys.to(DEV)
        qg, k, v, iq, ik = (t.to(DEV) for t in _projections(store, hidden))
        got = model.qsa_core(qg, k, v, iq, ik, 3, cache, pos, cos.to(DEV), sin.to(DEV))
        assert _got_sets(cache[3]) == chosen, pos
        assert rel_err(got, want, OUT_TOL) < OUT_TOL, pos


def test_batch_of_two_with_own_pages(gpu):
    dtype = torch.bfloat16
    cfg = OracleConfig()
    store = gi.FakeStore(gi.qsa_weights(3, 69, dtype))
    pos = 3000
    k1, v1, i1 = gi.qsa_past(70, pos, dtype)
    k2, v2, i2 = gi.qsa_past(71, pos, dtype)
    keys, values, idx = torch.cat([k1, k2]), torch.cat([v1, v2]), torch.cat([i1, i2])
    hidden = gi.normal(gi.rng(72), (2, 1, gi.HIDDEN)).to(dtype)
    cos, sin = tables(pos + 1)
    want, _, _, chosen = _oracle_core(cfg, store, hidden, cos, sin, keys, values, idx, pos)
    model, cache = _model_and_cache(gpu, store, dtype, pos + 64, batch=2)
    cache[3].keys, cache[3].values, cache[3].indexer_keys = keys.to(DEV), values.to(DEV), idx.to(DEV)
    qg, k, v, iq, ik = (t.to(DEV) for t in _projections(store, hidden))
    got = model.qsa_core(qg, k, v, iq, ik, 3, cache, pos, cos.to(DEV), sin.to(DEV))
    assert _got_sets(cache[3]) == chosen
    assert rel_err(got, want, OUT_TOL) < OUT_TOL


def test_consecutive_decode_steps_cross_a_block_boundary(gpu):
    """Steps 8126..8131 append tokens, complete block 126 at 8127 (pooled in the
    same launch) and move the tail into block 127."""
    dtype = torch.bfloat16
    cfg = OracleConfig()
    store = gi.FakeStore(gi.qsa_weights(3, 73, dtype))
    start = 8126
    keys, values, idx_keys = gi.qsa_past(74, start, dtype)
    model, cache = _model_and_cache(gpu, store, dtype, 8192 + 64)
    cache[3].keys, cache[3].values, cache[3].indexer_keys = keys.to(DEV), values.to(DEV), idx_keys.to(DEV)
    om = OracleMixer(cfg, store)
    ocache = OracleHybridCache(4)
    ocache[3].keys, ocache[3].values, ocache[3].indexer_keys = keys, values, idx_keys
    r = gi.rng(75)
    for pos in range(start, start + 6):
        hidden = gi.normal(r, (1, 1, gi.HIDDEN)).to(dtype)
        cos, sin = tables(pos + 1)
        want = om._full_attention(hidden, 3, cos, sin, ocache, pos)
        got = model._full_attention(hidden.to(DEV), 3, cos.to(DEV), sin.to(DEV), cache, pos)
        assert rel_err(got, want, OUT_TOL) < OUT_TOL, pos
    # the in-launch hand-off of the partials: per (sequence, kv head) a
    # generation word counting the launches, then a count of waits that gave up
    gen = model._ws["qsa_decode_3_1"].view(torch.int32).cpu()[: 2 * 32].reshape(2, 32)
    assert gen[:, 0].tolist() == [6, 6]
    assert gen[:, 1].tolist() == [0, 0]
    assert gen[:, 2].tolist() == [0, 0]      # no position outran the launch's splits
    model.check_handoffs()


@pytest.mark.parametrize("pos", [63, 127, 2047, 4095, 8127, 8128, 300, 9000, 20031])
def test_fused_decode_front_equals_prep_then_select(gpu, pos):
    """The one-launch decode (qm_qsa_decode) == qm_qsa_prep + qm_qsa_select, bit
    for bit: pooled block keys (including the block this token completes), the
    indexer query, the appended key and the selected set (the one-launch
    kernel lists up to 128 eligible blocks' selection in block order, the
    select kernel by rank)."""
    dtype = torch.bfloat16
    store = gi.FakeStore(gi.qsa_weights(3, 80, dtype))
    keys, values, idx_keys = gi.qsa_past(81, pos, dtype)
    hidden = gi.normal(gi.rng(82 + pos), (1, 1, gi.HIDDEN)).to(dtype)
    cos, sin = tables(pos + 1)
    qg, k, v, iq, ik = (t.to(DEV) for t in _projections(store, hidden))
    results = []
    for fused in (True, False):
        model, cache = _model_and_cache(gpu, store, dtype, pos + 128)
        cache[3].keys, cache[3].values, cache[3].indexer_keys = keys.to(DEV), values.to(DEV), idx_keys.to(DEV)
        if fused:
            model.qsa_core(qg, k, v, iq, ik, 3, cache, pos, cos.to(DEV), sin.to(DEV))
        else:
            # the same step through the separate launches (the prefill path with seq 1)
            model.qsa_core(None, k, v, iq, ik, 3, cache, pos, cos.to(DEV), sin.to(DEV), attend=False)
        lc = cache[3]
        results.append((lc.block_keys.cpu().clone(), lc.last_iq.cpu().clone(), lc.last_ids.cpu().clone(),
                        lc.last_n_sel.cpu().clone(), lc.k_pool.cpu().clone()))
    (bk1, iq1, ids1, n1, kp1), (bk2, iq2, ids2, n2, kp2) = results
    assert torch.equal(bk1, bk2) and torch.equal(iq1, iq2)
    assert torch.equal(n1, n2)
    k = int(n1.max())
    assert torch.equal(ids1[..., :k].sort(-1).values, ids2[..., :k].sort(-1).values)
    assert torch.equal(kp1, kp2)


def _decode_both_kernels(gpu, monkeypatch, pos, seed):
    """One decode step at `pos` twice on identical caches: through the plan the
    position asks for (at most 10 attention items: the short-context slice
    kernel) and through a plan sized for position 2000 (the long-context
    kernel, whose grid is sized by the plan). Returns (oracle output, chosen
    sets, [(output, cache) per kernel])."""
    qm = gpu
    cfg = OracleConfig()
    dtype = torch.bfloat16
    store = gi.FakeStore(gi.qsa_weights(3, seed, dtype))
    keys, values, idx_keys = gi.qsa_past(seed + 1, pos, dtype)
    hidden = gi.normal(gi.rng(seed + 2), (1, 1, gi.HIDDEN)).to(dtype)
    cos, sin = tables(pos + 1)
    want, _, _, chosen = _oracle_core(cfg, store, hidden, cos, sin, keys if pos else None,
                                      values if pos else None, idx_keys, pos)
    lib = qm.native.load()
    real_splits = lib.qm_qsa_decode_splits
    runs = []
    for plan_pos in (pos, 2000):
        # the model sizes its decode plan with qm_qsa_decode_splits
        monkeypatch.setattr(lib, "qm_qsa_decode_splits", lambda g, p, pp=plan_pos: real_splits(g, pp))
        model, cache = _model_and_cache(gpu, store, dtype, 2048 + 64)
        if pos:
            cache[3].keys, cache[3].values, cache[3].indexer_keys = keys.to(DEV), values.to(DEV), idx_keys.to(DEV)
        qg, k, v, iq, ik = (t.to(DEV) for t in _projections(store, hidden))
        got = model.qsa_core(qg, k, v, iq, ik, 3, cache, pos, cos.to(DEV), sin.to(DEV))
        torch.cuda.synchronize()
        runs.append((got, cache, model))
    monkeypatch.setattr(lib, "qm_qsa_decode_splits", real_splits)
    return want, chosen, runs


@pytest.mark.parametrize("pos", [0, 31, 63, 64, 191, 192, 300])
def test_short_context_kernel_matches_long_context_kernel(gpu, monkeypatch, pos):
    """Below 320 keys (selection off) the slice kernel scores every key per
    query head in one workgroup (no hand-off); the long-context kernel splits
    the keys into 32-key items and merges their partials. Both are within the
    bar of the oracle; they round the softmax differently (one softmax against
    a merge of per-item ones), so their outputs agree to the bar, while the
    appended key/value bits, the pooled block keys (63 and 191 complete a
    block), the indexer query and the selected set agree bit for bit."""
    print(f"short vs long context kernel pos={pos}", flush=True)
    want, chosen, runs = _decode_both_kernels(gpu, monkeypatch, pos, 90)
    (o_s, c_s, m_s), (o_l, c_l, m_l) = runs
    for o, c in ((o_s, c_s), (o_l, c_l)):
        assert _got_sets(c[3]) == chosen
        assert rel_err(o, want, OUT_TOL) < OUT_TOL
    assert rel_err(o_s, o_l, OUT_TOL) < OUT_TOL
    ls, ll = c_s[3], c_l[3]
    assert torch.equal(ls.k_pool, ll.k_pool) and torch.equal(ls.v_pool, ll.v_pool)
    assert torch.equal(ls.raw_keys, ll.raw_keys)
    assert torch.equal(ls.block_keys, ll.block_keys)
    assert torch.equal(ls.last_iq, ll.last_iq)
    for m in (m_s, m_l):
        m.check_handoffs()


def test_short_context_kernel_poisons_a_position_past_its_range(gpu, monkeypatch):
    """A plan of the slice kernel (sized for position 100) launched at position
    600, past the 512 keys its workgroups hold: every output is NaN, the
    launch is counted in the group's overflow word, and nothing is appended
    (no workgroup reads or writes a page)."""
    qm = gpu
    dtype = torch.bfloat16
    pos = 600
    store = gi.FakeStore(gi.qsa_weights(3, 95, dtype))
    keys, values, idx_keys = gi.qsa_past(96, pos, dtype)
    hidden = gi.normal(gi.rng(97), (1, 1, gi.HIDDEN)).to(dtype)
    cos, sin = tables(pos + 1)
    lib = qm.native.load()
    real_splits = lib.qm_qsa_decode_splits
    monkeypatch.setattr(lib, "qm_qsa_decode_splits", lambda g, p: real_splits(g, 100))
    model, cache = _model_and_cache(gpu, store, dtype, 1024)
    cache[3].keys, cache[3].values, cache[3].indexer_keys = keys.to(DEV), values.to(DEV), idx_keys.to(DEV)
    k_before = cache[3].k_pool.clone()
    qg, k, v, iq, ik = (t.to(DEV) for t in _projections(store, hidden))
    print("short context kernel at pos 600 (past its range)", flush=True)
    got = model.qsa_core(qg, k, v, iq, ik, 3, cache, pos, cos.to(DEV), sin.to(DEV))
    torch.cuda.synchronize()
    monkeypatch.setattr(lib, "qm_qsa_decode_splits", real_splits)
    assert torch.isnan(got.float()).all()
    assert torch.equal(cache[3].k_pool, k_before)
    words = model._ws["qsa_decode_3_1"].view(torch.int32).cpu()[: 2 * 32].reshape(2, 32)
    assert words[:, 2].tolist() == [1, 1]     # counted once per (sequence, kv head) group
