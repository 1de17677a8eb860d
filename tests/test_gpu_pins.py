"""Parity pins on the GPU that the layer tests leave open.

* Block scores, by value: qm_qsa_select's fp32 scores equal the tensor the
  reference handed to ``topk`` (reference/model.py:297-306) bit for bit, at
  config 3 (pos 8128), its pos-4032 twin and all 128 rows of config 5. Equal
  selected sets alone are weak evidence near ties; on failure the test reports
  the largest difference in ulps and the gap between ranks 32 and 33.
* The delta rules under extreme decay (reference tests/test_delta_rule.py:37-48:
  a log-decay near -160..-200 makes exp(cum) underflow to 0, which once
  poisoned the carried state with 0/0): the free functions, the prefill core and
  the decode core against the oracle's recurrence, state finite and within
  1e-3.
* Config 4 against the reference's *sequential* recurrence (``rec_out`` /
  ``rec_state``), the form BASELINE words it in.
* The free conv functions causal_conv1d / causal_conv1d_step
  (reference/layers.py:133-147): outputs within tolerance, the new state bit
  for bit.
* ``_indexer_mask`` (reference/model.py:248-327) through the product method,
  bit for bit against the oracle's mask at config 1, 3 and 5 shapes.
* The decode path of two launches (qm_qsa_decode_front + qm_qsa_attend), which
  runs where the one-launch kernel cannot (its group would not fit the device),
  against the oracle at pos 8128.
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import layers as ol
from oracle.cache import OracleHybridCache
from oracle.config import OracleConfig
from oracle.layers import RotaryEmbedding
from oracle.mixing import OracleMixer

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, HERE)
import inputs as gi  # noqa: E402

from margins import abs_err, record, rel_err  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda"
OUT_TOL, STATE_TOL = 2e-2, 1e-3
META = json.load(open(os.path.join(HERE, "golden_meta.json")))
ROT = RotaryEmbedding(64, 1e7, [11, 11, 10])


def tables(n):
    p = torch.arange(n)[None]
    return ROT(p[None].expand(3, -1, -1))


def _layers(qm):
    import importlib
    return importlib.import_module(qm.__name__ + ".layers")


# -- block scores by value ----------------------------------------------------------


def _ulps(a: np.ndarray, b: np.ndarray) -> int:
    """Largest distance in units in the last place between finite float32s."""
    fin = np.isfinite(a) & np.isfinite(b)
    ia = a[fin].view(np.int32).astype(np.int64)
    ib = b[fin].view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, np.int64(-(2 ** 31)) - ia, ia)
    ib = np.where(ib < 0, np.int64(-(2 ** 31)) - ib, ib)
    return int(np.abs(ia - ib).max()) if ia.size else 0


def _gap_32_33(row: np.ndarray) -> float:
    s = np.sort(row[np.isfinite(row)])[::-1]
    return float(s[31] - s[32]) if s.size > 32 else float("inf")


@pytest.mark.parametrize("tag", ["cfg3", "cfg3b", "cfg5"])
def test_block_scores_bit_exact_vs_reference(gpu, tag):
    qm = gpu
    m = META[tag]
    z = np.load(os.path.join(HERE, f"{tag}.npz"))
    dtype = torch.bfloat16
    if tag == "cfg5":
        past, seq = m["past"], m["seq"]
    else:
        past, seq = m["pos"], 1
    store = gi.FakeStore(gi.qsa_weights(3, m["qsa_seeds"][0], dtype))
    _, _, idx_keys = gi.qsa_past(m["qsa_seeds"][1], past, dtype)
    iq = gi.from_bf16_bits(z["idx_q_raw"]).reshape(1, seq, -1)
    ik = gi.from_bf16_bits(z["idx_k_raw"]).reshape(1, seq, -1)
    cos, sin = gi.golden_rope(ROT, past + seq)       # the golden generator's rows where they matter
    model = qm.Qwen4MixModel(qm.MixConfig(), store, device=DEV, max_ctx=past + seq + 64)
    cache = qm.MixHybridCache(4, model.config, 1, past + seq + 64, DEV, dtype, page_table="random", seed=5)
    cache[3].indexer_keys = idx_keys.to(DEV)
    print(f"scores {tag} past={past} seq={seq}", flush=True)
    model.qsa_core(None, None, None, iq.to(DEV), ik.to(DEV), 3, cache, past, cos.to(DEV), sin.to(DEV), attend=False)
    lc = cache[3]
    g = model.qsa_geom(cache, dtype)
    topk = model.config.block_topk
    pos = torch.tensor([past], dtype=torch.int32, device=DEV)
    ids = torch.empty(seq, topk, dtype=torch.int32, device=DEV)
    n_sel = torch.empty(seq, dtype=torch.int32, device=DEV)
    scores = torch.empty(seq, cache.max_blocks, dtype=torch.float32, device=DEV)
    import ctypes
    qm.native.call("qm_qsa_select", ctypes.byref(g), seq, lc.last_iq.data_ptr(), lc.block_keys.data_ptr(),
                   pos.data_ptr(), None, ids.data_ptr(), n_sel.data_ptr(), None, scores.data_ptr(),
                   qm.native.stream_handle())
    want = z["scores"].reshape(seq, -1).astype(np.float32)
    got = scores.cpu().numpy()[:, : want.shape[1]]
    record("ulps", _ulps(got, want), 0)
    same = got.view(np.int32) == want.view(np.int32)
    if not same.all():
        bad = np.argwhere(~same)
        r = int(bad[0][0])
        # which stage departs: the indexer queries or the pooled block keys
        om = OracleMixer(OracleConfig(), store)
        q_want = ol.apply_rotary(ol.rms_norm(iq.reshape(1, seq, 4, 128), store.get("blk.3.indexer.q_norm.weight"),
                                             1e-6), cos[:, -seq:], sin[:, -seq:], unsqueeze_dim=2).float()
        n_blocks = want.shape[1]
        pooled = om.indexer_pooled(torch.cat([idx_keys, ik], 1), 3, cos, sin, n_blocks).float()
        q_rows = (lc.last_iq.cpu() != q_want).reshape(seq, -1).any(-1).nonzero().flatten().tolist()
        k_rows = (lc.block_keys_ref[:, :n_blocks].cpu() != pooled)[0].any(-1).nonzero().flatten().tolist()
        raise AssertionError(f"{tag}: {len(bad)} scores differ (rows {sorted(set(bad[:, 0].tolist()))[:8]}); "
                             f"max {_ulps(got, want)} ulp; rank-32/33 gap of row {r}: {_gap_32_33(want[r]):.3e}; "
                             f"query rows off {q_rows[:8]}, pooled blocks off {k_rows[:8]}")
    # and the selected set of every row is the top-k of those scores, ties low
    for r in range(seq):
        row = want[r]
        n_el = int(np.isfinite(row).sum())
        top = np.lexsort((np.arange(n_el), -row[:n_el].astype(np.float64)))[:topk]
        assert sorted(ids[r, : int(n_sel[r])].cpu().tolist()) == sorted(top.tolist()), r


# -- extreme decay ------------------------------------------------------------------


def _decay_inputs(seed, seq, heads, scale):
    """reference tests/test_delta_rule.py:15-24 at this path's head dim: q, k, v
    ~ N(0, 1), g = -U(0, 1) * scale, beta ~ U(0, 1)."""
    r = gi.rng(seed)
    q = gi.normal(r, (1, seq, heads, 128))
    k = gi.normal(r, (1, seq, heads, 128))
    v = gi.normal(r, (1, seq, heads, 128))
    g = -torch.from_numpy(r.random((1, seq, heads)).astype(np.float32)) * scale
    beta = torch.from_numpy(r.random((1, seq, heads)).astype(np.float32))
    return q, k, v, g, beta


@pytest.mark.parametrize("scale", [160.0, 200.0])
@pytest.mark.parametrize("seq", [7, 100, 256])
def test_delta_rules_under_extreme_decay(gpu, scale, seq):
    lay = _layers(gpu)
    q, k, v, g, beta = _decay_inputs(int(scale) + seq, seq, 8, scale)
    s0 = gi.normal(gi.rng(3), (1, 8, 128, 128), 0.02)
    want_o, want_s = ol.recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=s0)
    assert torch.isfinite(want_s).all()
    print(f"extreme decay scale={scale} seq={seq}", flush=True)
    for rule in (lay.chunk_gated_delta_rule, lay.recurrent_gated_delta_rule):
        got_o, got_s = rule(q.to(DEV), k.to(DEV), v.to(DEV), g.to(DEV), beta.to(DEV), initial_state=s0.to(DEV))
        assert torch.isfinite(got_o).all() and torch.isfinite(got_s).all(), rule.__name__
        assert abs_err(got_o, want_o, 1e-3) < 1e-3, rule.__name__
        assert abs_err(got_s, want_s, STATE_TOL) < STATE_TOL, rule.__name__


@pytest.mark.parametrize("seq", [1, 128])
def test_layer_cores_under_extreme_decay(gpu, seq):
    """The DeltaNet layer with ssm_a = -200 (a decay of e^-200 at the mean
    gate): the prefill chunk (seq 128) and the decode step (seq 1), then one
    more decode step on the carried state."""
    qm = gpu
    dtype = torch.bfloat16
    w = gi.dn_weights(0, 41, dtype)
    w["blk.0.ssm_a"] = torch.full_like(w["blk.0.ssm_a"], -200.0)
    store = gi.FakeStore(w)
    conv, state = gi.dn_past(42, dtype)
    ocache = OracleHybridCache(1)
    ocache[0].conv_state, ocache[0].recurrent_state = conv.clone(), state.clone()
    model = qm.Qwen4MixModel(qm.MixConfig(), store, device=DEV)
    cache = qm.MixHybridCache(1, model.config, 1, 1024, DEV, dtype)
    cache[0].conv_state = conv.to(DEV)
    cache[0].recurrent_state = state.to(DEV).clone()
    om = OracleMixer(OracleConfig(), store)
    r = gi.rng(43)
    print(f"layer cores ssm_a=-200 seq={seq}", flush=True)
    for s in (seq, 1):
        hidden = gi.normal(r, (1, s, gi.HIDDEN)).to(dtype)
        p = [F.linear(hidden, store.get(f"blk.0.{n}")) for n in
             ("attn_qkv.weight", "attn_gate.weight", "ssm_beta.weight", "ssm_alpha.weight")]
        want = om.dn_core(p[0], p[1], p[2], p[3], 0, ocache)
        got = model.dn_core(p[0].to(DEV), p[1].to(DEV), p[3].to(DEV), p[2].to(DEV), 0, cache[0])
        st = cache[0].recurrent_state
        assert torch.isfinite(got).all() and torch.isfinite(st).all()
        assert rel_err(got, want, OUT_TOL) < OUT_TOL
        assert abs_err(st, ocache[0].recurrent_state, STATE_TOL) < STATE_TOL


# -- config 4 against the sequential recurrence -----------------------------------------


@pytest.mark.parametrize("rule_name", ["chunk_gated_delta_rule", "recurrent_gated_delta_rule"])
def test_config4_against_reference_recurrence(gpu, rule_name):
    lay = _layers(gpu)
    z = np.load(os.path.join(HERE, "cfg4.npz"))
    q, k, v, g, beta = gi.delta_rule_inputs(404, 4096)
    s0 = gi.dn_past(405)[1]
    print(f"config 4 {rule_name} vs rec_out/rec_state", flush=True)
    got_o, got_s = getattr(lay, rule_name)(q.to(DEV), k.to(DEV), v.to(DEV), g.to(DEV), beta.to(DEV),
                                           initial_state=s0.to(DEV))
    o = got_o.reshape(-1).cpu()
    want = torch.from_numpy(z["rec_out"])
    stride = max(1, o.numel() // want.numel())
    assert abs_err(o[::stride][: want.numel()], want, 2e-3) < 2e-3
    s = got_s.reshape(-1).cpu()
    ws = torch.from_numpy(z["rec_state"])
    stride = max(1, s.numel() // ws.numel())
    assert abs_err(s[::stride][: ws.numel()], ws, STATE_TOL) < STATE_TOL


# -- the free conv functions ------------------------------------------------------------


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("seq", [1, 2, 5, 130])
def test_causal_conv1d_free_functions(gpu, dtype, seq):
    lay = _layers(gpu)
    r = gi.rng(60 + seq)
    C, K = 8192, 4
    x = gi.normal(r, (2, C, seq)).to(dtype)
    state = gi.normal(r, (2, C, K - 1)).to(dtype)
    w = gi.normal(r, (C, K), 0.5).to(dtype)
    tol = 1e-5 if dtype == torch.float32 else OUT_TOL
    print(f"causal conv seq={seq} {dtype}", flush=True)
    want_o, want_s = ol.causal_conv1d_step(x, state, w)
    got_o, got_s = lay.causal_conv1d_step(x.to(DEV), state.to(DEV), w.to(DEV))
    assert rel_err(got_o, want_o, tol) < tol
    assert torch.equal(got_s.cpu(), want_s)                  # the window only moves inputs
    want = ol.causal_conv1d(x, w)
    got = lay.causal_conv1d(x.to(DEV), w.to(DEV))
    assert rel_err(got, want, tol) < tol
    got_lin = lay.causal_conv1d(x.to(DEV), w.to(DEV), activation=False)
    assert rel_err(got_lin, ol.causal_conv1d(x, w, activation=False), tol) < tol


# -- _indexer_mask through the product method -------------------------------------------


def _ternary(r, shape, density, dtype):
    """Sparse {-1, 0, 1} entries: products and sums of a few of them are exact
    in float32 (and bfloat16) in any order."""
    vals = r.choice(np.array([-1.0, 0.0, 1.0], np.float32), size=shape, p=[density / 2, 1 - density, density / 2])
    return torch.from_numpy(vals).to(dtype)


@pytest.mark.parametrize("past,seq,dtype", [(192, 1, torch.float32), (8128, 1, torch.bfloat16),
                                            (32640, 128, torch.bfloat16), (4000, 37, torch.bfloat16)])
def test_indexer_mask_matches_oracle(gpu, past, seq, dtype):
    """The method projects on its own (a library GEMM on the GPU, torch's CPU
    GEMM in the oracle), so the indexer projections and the hidden rows are
    sparse ternary: every projection is then an exact small integer whatever
    the summation order, and the comparison covers the method's own work --
    raw-key append, pooling, scores, top-k, tails -- bit for bit."""
    qm = gpu
    cfg = OracleConfig()
    r = gi.rng(79)
    w = gi.qsa_weights(3, 77, dtype)
    w["blk.3.indexer.q_proj.weight"] = _ternary(r, tuple(w["blk.3.indexer.q_proj.weight"].shape), 1 / 16, dtype)
    w["blk.3.indexer.k_proj.weight"] = _ternary(r, tuple(w["blk.3.indexer.k_proj.weight"].shape), 1 / 16, dtype)
    store = gi.FakeStore(w)
    _, _, idx_keys = gi.qsa_past(78, past, dtype)
    hidden = _ternary(r, (1, seq, gi.HIDDEN), 1 / 16, dtype)
    cos, sin = tables(past + seq)
    kv_len = past + seq
    oc = OracleHybridCache(4)
    oc[3].indexer_keys = idx_keys
    print(f"indexer mask past={past} seq={seq}", flush=True)
    want = OracleMixer(cfg, store)._indexer_mask(hidden, 3, cos, sin, oc, kv_len, past)
    model = qm.Qwen4MixModel(qm.MixConfig(), store, device=DEV, max_ctx=kv_len + 64)
    cache = qm.MixHybridCache(4, model.config, 1, kv_len + 64, DEV, dtype, page_table="random", seed=5)
    cache[3].indexer_keys = idx_keys.to(DEV)
    got = model._indexer_mask(hidden.to(DEV), 3, cos.to(DEV), sin.to(DEV), cache, kv_len, past)
    assert got.shape == want.shape
    if not torch.equal(got.cpu(), want):
        diff = (got.cpu() != want).nonzero()
        raise AssertionError(f"mask differs at {diff.shape[0]} entries, first {diff[0].tolist()}")
    # the raw keys were appended as the reference appends them
    assert cache[3].n_tokens == kv_len


# -- the decode path of two launches ---------------------------------------------------


def test_split_decode_matches_oracle(gpu):
    """pos 8128 through qm_qsa_prep, the one-row scores spread over the blocks,
    the ranking (qm_qsa_select with a score buffer) and qm_qsa_attend, forced
    the way a plan too large for one resident group is routed."""
    qm = gpu
    dtype = torch.bfloat16
    pos = 8128
    cfg = OracleConfig()
    store = gi.FakeStore(gi.qsa_weights(3, 61, dtype))
    keys, values, idx_keys = gi.qsa_past(62, pos, dtype)
    hidden = gi.normal(gi.rng(63), (1, 1, gi.HIDDEN)).to(dtype)
    cos, sin = tables(pos + 1)
    om = OracleMixer(cfg, store)
    oc = OracleHybridCache(4)
    oc[3].keys, oc[3].values, oc[3].indexer_keys = keys, values, idx_keys
    want = om._full_attention(hidden, 3, cos, sin, oc, pos)
    model = qm.Qwen4MixModel(qm.MixConfig(), store, device=DEV, max_ctx=pos + 128)
    model.decode_group_fits = lambda splits, dt: False
    cache = qm.MixHybridCache(4, model.config, 1, pos + 128, DEV, dtype, page_table="random", seed=5)
    cache[3].keys, cache[3].values, cache[3].indexer_keys = keys.to(DEV), values.to(DEV), idx_keys.to(DEV)
    print("split decode pos=8128", flush=True)
    got = model._full_attention(hidden.to(DEV), 3, cos.to(DEV), sin.to(DEV), cache, pos)
    assert "qsa_decode_3_1" not in model._ws           # the one-launch kernel never ran
    assert rel_err(got, want, OUT_TOL) < OUT_TOL
    # the selection the two launches made is the oracle's
    ids, n = cache[3].last_ids.cpu()[0, 0], int(cache[3].last_n_sel.cpu()[0, 0])
    oc2 = OracleHybridCache(4)
    oc2[3].indexer_keys = idx_keys
    mask = om._indexer_mask(hidden, 3, cos, sin, oc2, pos + 1, pos)
    chosen = sorted(j for j in range((pos + 1) // 64) if bool(mask[0, 0, 0, j * 64]))
    assert sorted(ids[:n].tolist()) == chosen


def _decode_case(qm, pos, seed):
    dtype = torch.bfloat16
    store = gi.FakeStore(gi.qsa_weights(3, seed, dtype))
    keys, values, idx_keys = gi.qsa_past(seed + 1, pos, dtype)
    hidden = gi.normal(gi.rng(seed + 2), (1, 1, gi.HIDDEN)).to(dtype)
    cos, sin = tables(pos + 1)
    om = OracleMixer(OracleConfig(), store)
    oc = OracleHybridCache(4)
    oc[3].keys, oc[3].values, oc[3].indexer_keys = keys, values, idx_keys
    want = om._full_attention(hidden, 3, cos, sin, oc, pos)
    oc2 = OracleHybridCache(4)
    oc2[3].indexer_keys = idx_keys
    mask = om._indexer_mask(hidden, 3, cos, sin, oc2, pos + 1, pos)
    chosen = sorted(j for j in range((pos + 1) // 64) if bool(mask[0, 0, 0, j * 64]))
    model = qm.Qwen4MixModel(qm.MixConfig(), store, device=DEV, max_ctx=pos + 128)
    cache = qm.MixHybridCache(4, model.config, 1, pos + 128, DEV, dtype, page_table="random", seed=5)
    cache[3].keys, cache[3].values, cache[3].indexer_keys = keys.to(DEV), values.to(DEV), idx_keys.to(DEV)
    return model, cache, hidden, cos, sin, want, chosen


def test_decode_front_entry_point_matches_oracle(gpu):
    """qm_qsa_decode_front (prep and selection in one launch) + qm_qsa_attend
    at pos 8128, called through a decode plan: output and selected blocks
    against the oracle."""
    import ctypes
    from importlib import import_module
    qm = gpu
    plan_mod = import_module(qm.__name__ + ".plan")
    pos = 8128
    model, cache, hidden, cos, sin, want, chosen = _decode_case(qm, pos, 71)
    lc = cache[3]
    g = model.qsa_geom(cache, torch.bfloat16)
    cos_t, sin_t = model._rope(cos.to(DEV), sin.to(DEV), pos + 1)
    model._sync_blocks(lc, g, cos_t, sin_t, pos, 3)
    qg, k, v, iq, ik = (t.contiguous() for t in model.project(hidden.to(DEV), 3, "qsa_in"))
    plan = plan_mod.QsaDecodePlan(model, cache, 3, pos, torch.bfloat16, fused=False)
    plan.cos, plan.sin = cos_t, sin_t
    plan.positions.fill_(pos)
    print("front + attend decode pos=8128", flush=True)
    s = qm.native.stream_handle(torch.device(DEV))
    plan.front(qg, k, v, iq, ik, s)
    plan.attend(qg, s)
    got = model.project(plan.out, 3, "qsa_out")[0]
    assert rel_err(got, want, OUT_TOL) < OUT_TOL
    n = int(plan.n_sel.cpu()[0, 0])
    assert sorted(plan.ids.cpu()[0, 0, :n].tolist()) == chosen


def test_long_context_decode_matches_oracle(gpu):
    """pos 131200 of a 131328-token context (2050 eligible blocks, past the
    one-launch kernel's 2048): the model's decode step takes prep, the scores
    spread over the blocks, the ranking and the attention; output and the
    selected blocks against the oracle."""
    qm = gpu
    pos = 131200
    model, cache, hidden, cos, sin, want, chosen = _decode_case(qm, pos, 81)
    assert not model.fused_decode_fits(cache)
    print("long-context decode pos=131200", flush=True)
    got = model._full_attention(hidden.to(DEV), 3, cos.to(DEV), sin.to(DEV), cache, pos)
    assert rel_err(got, want, OUT_TOL) < OUT_TOL
    lc = cache[3]
    n = int(lc.last_n_sel.cpu()[0, 0])
    assert sorted(lc.last_ids.cpu()[0, 0, :n].tolist()) == chosen
