"""Gated DeltaNet on the GPU against the oracle (and the reference's goldens).

Tolerances (north star): bf16/fp32 layer outputs within 2e-2 max relative error
(max |got - want| / max |want|), the float32 recurrent state within 1e-3
absolute, the conv window bit-exact (it only moves inputs).
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np
import pytest
import torch

from oracle import f64
from oracle.cache import OracleHybridCache
from oracle.config import OracleConfig
from oracle.layers import chunk_gated_delta_rule as o_chunk
from oracle.layers import recurrent_gated_delta_rule as o_rec
from oracle.mixing import OracleMixer

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, HERE)
import inputs as gi  # noqa: E402

from margins import abs_err, rel_err  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda"
OUT_TOL, STATE_TOL = 2e-2, 1e-3


def _setup(gpu, dtype, wseed, sseed, batch=1):
    qm = gpu
    store = gi.FakeStore(gi.dn_weights(0, wseed, dtype))
    conv, state = gi.dn_past(sseed, dtype)
    conv = conv.expand(batch, -1, -1).clone()
    state = state.expand(batch, -1, -1, -1).clone()
    ocache = OracleHybridCache(1)
    ocache[0].conv_state, ocache[0].recurrent_state = conv.clone(), state.clone()
    model = qm.Qwen4MixModel(qm.MixConfig(), store, device=DEV)
    cache = qm.MixHybridCache(1, model.config, batch, 4096, DEV, dtype)
    cache[0].conv_state = conv.to(DEV)
    cache[0].recurrent_state = state.to(DEV).clone()
    return store, ocache, model, cache


def _proj(store, hidden):
    """The four projections, computed once on the CPU and fed to both sides."""
    w = lambda s: store.get(f"blk.0.{s}")  # noqa: E731
    F = torch.nn.functional
    return (F.linear(hidden, w("attn_qkv.weight")), F.linear(hidden, w("attn_gate.weight")),
            F.linear(hidden, w("ssm_beta.weight")), F.linear(hidden, w("ssm_alpha.weight")))


def _core_step(model, cache, omix, ocache, store, hidden):
    mixed, z, b, a = _proj(store, hidden)
    want = omix.dn_core(mixed, z, b, a, 0, ocache)
    got = model.dn_core(mixed.to(DEV), z.to(DEV), a.to(DEV), b.to(DEV), 0, cache[0])
    return got, want


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("batch", [1, 3])
def test_decode_core_matches_oracle(gpu, dtype, batch):
    """Same projection bits on both sides: the conv window moves bit-exactly,
    the state stays within 1e-3, the output within 2e-2."""
    store, ocache, model, cache = _setup(gpu, dtype, 21, 22, batch)
    hidden = gi.normal(gi.rng(23), (batch, 1, gi.HIDDEN)).to(dtype)
    print(f"decode core dtype={dtype} batch={batch}", flush=True)
    got, want = _core_step(model, cache, OracleMixer(OracleConfig(), store), ocache, store, hidden)
    torch.cuda.synchronize()
    assert rel_err(got, want, OUT_TOL) < OUT_TOL
    assert abs_err(cache[0].recurrent_state, ocache[0].recurrent_state, STATE_TOL) < STATE_TOL
    assert torch.equal(cache[0].conv_state.cpu(), ocache[0].conv_state)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_decode_layer_matches_oracle(gpu, dtype):
    """The whole layer, projections on the GPU (hipBLASLt) and on the CPU."""
    store, ocache, model, cache = _setup(gpu, dtype, 24, 25)
    hidden = gi.normal(gi.rng(26), (1, 1, gi.HIDDEN)).to(dtype)
    want = OracleMixer(OracleConfig(), store)._linear_attention(hidden, 0, ocache)
    got = model._linear_attention(hidden.to(DEV), 0, cache)
    assert rel_err(got, want, OUT_TOL) < OUT_TOL
    assert abs_err(cache[0].recurrent_state, ocache[0].recurrent_state, STATE_TOL) < STATE_TOL


def test_decode_core_matches_golden_reference(gpu):
    """cfg1 (fp32) and cfg3 (bf16) DeltaNet layers against the reference's own outputs."""
    meta = json.load(open(os.path.join(HERE, "golden_meta.json")))
    for tag in ("cfg1", "cfg3"):
        m = meta[tag]
        z = np.load(os.path.join(HERE, f"{tag}.npz"))
        dtype = torch.float32 if m["dtype"] == "torch.float32" else torch.bfloat16
        store, _, model, cache = _setup(gpu, dtype, m["dn_seeds"][0], m["dn_seeds"][1])
        hidden = gi.hidden_states(m["hidden_seed"], 1, dtype)
        print(f"golden {tag}", flush=True)
        y = model._linear_attention(hidden.to(DEV), 0, cache)
        flat = y.float().reshape(-1).cpu()
        want = torch.from_numpy(z["dn_out"])
        stride = max(1, flat.numel() // want.numel())
        assert rel_err(flat[::stride][: want.numel()], want, OUT_TOL) < OUT_TOL, tag
        st = cache[0].recurrent_state.reshape(-1).cpu()
        ws = torch.from_numpy(z["dn_state"])
        stride = max(1, st.numel() // ws.numel())
        assert abs_err(st[::stride][: ws.numel()], ws, STATE_TOL) < STATE_TOL, tag


def test_64_compounding_decode_steps_stay_within_tolerance(gpu):
    """A single step proves little for a recurrence: 64 steps on identical inputs."""
    dtype = torch.bfloat16
    store, ocache, model, cache = _setup(gpu, dtype, 31, 32)
    omix = OracleMixer(OracleConfig(), store)
    r = gi.rng(33)
    worst_out = worst_state = 0.0
    for t in range(64):
        hidden = gi.normal(r, (1, 1, gi.HIDDEN)).to(dtype)
        got, want = _core_step(model, cache, omix, ocache, store, hidden)
        worst_out = max(worst_out, rel_err(got, want))
        worst_state = max(worst_state, abs_err(cache[0].recurrent_state, ocache[0].recurrent_state))
    print(f"64 steps: worst out rel {worst_out:.2e}, worst state abs {worst_state:.2e}", flush=True)
    assert worst_out < OUT_TOL and worst_state < STATE_TOL
    assert torch.equal(cache[0].conv_state.cpu(), ocache[0].conv_state)
    # the in-launch hand-off of the gated norm's shares: one 128-byte line per
    # head, whose generation word counts the launches and whose second word
    # counts waits that gave up (never)
    lines = model._ws["dn_decode_1"].view(torch.int32).cpu()[: 32 * 32].reshape(32, 32)
    assert lines[:, 0].tolist() == [64] * 32
    assert lines[:, 1].tolist() == [0] * 32
    model.check_handoffs()          # the same counters through qm_dn_decode_check, then reset
    assert model._ws["dn_decode_1"].view(torch.int32).cpu()[: 32 * 32].abs().sum().item() == 0


@pytest.mark.parametrize("seq", [2, 7, 64, 128])
def test_prefill_core_matches_oracle(gpu, seq):
    dtype = torch.bfloat16
    store, ocache, model, cache = _setup(gpu, dtype, 41, 42)
    omix = OracleMixer(OracleConfig(), store)
    hidden = gi.normal(gi.rng(43), (1, seq, gi.HIDDEN)).to(dtype)
    print(f"prefill core seq={seq}", flush=True)
    got, want = _core_step(model, cache, omix, ocache, store, hidden)
    assert rel_err(got, want, OUT_TOL) < OUT_TOL
    assert abs_err(cache[0].recurrent_state, ocache[0].recurrent_state, STATE_TOL) < STATE_TOL
    assert torch.equal(cache[0].conv_state.cpu(), ocache[0].conv_state)
    # a decode step continues from the prefilled state and ring
    h1 = gi.normal(gi.rng(44), (1, 1, gi.HIDDEN)).to(dtype)
    got, want = _core_step(model, cache, omix, ocache, store, h1)
    assert rel_err(got, want, OUT_TOL) < OUT_TOL
    assert torch.equal(cache[0].conv_state.cpu(), ocache[0].conv_state)


def test_prefill_chunk_matches_golden_reference(gpu):
    """The 128-token chunk of config 5 (DeltaNet half) against the reference."""
    meta = json.load(open(os.path.join(HERE, "golden_meta.json")))["cfg5"]
    z = np.load(os.path.join(HERE, "cfg5.npz"))
    dtype = torch.bfloat16
    store, _, model, cache = _setup(gpu, dtype, meta["dn_seeds"][0], meta["dn_seeds"][1])
    hidden = gi.hidden_states(meta["hidden_seed"], meta["seq"], dtype)
    y = model._linear_attention(hidden.to(DEV), 0, cache).float().reshape(-1).cpu()
    want = torch.from_numpy(z["dn_out"])
    stride = max(1, y.numel() // want.numel())
    assert rel_err(y[::stride][: want.numel()], want, OUT_TOL) < OUT_TOL
    st = cache[0].recurrent_state.reshape(-1).cpu()
    ws = torch.from_numpy(z["dn_state"])
    stride = max(1, st.numel() // ws.numel())
    assert abs_err(st[::stride][: ws.numel()], ws, STATE_TOL) < STATE_TOL


@pytest.mark.parametrize("fn", ["recurrent", "chunked"])
@pytest.mark.parametrize("seq", [1, 33, 100])
def test_free_function_rules_match_oracle(gpu, fn, seq):
    import importlib
    layers = importlib.import_module(gpu.__name__ + ".layers")
    q, k, v, g, beta = gi.delta_rule_inputs(51, seq, heads=8)
    s0 = gi.normal(gi.rng(52), (1, 8, 128, 128), 0.02)
    want_o, want_s = o_rec(q, k, v, g, beta, initial_state=s0)
    rule = layers.recurrent_gated_delta_rule if fn == "recurrent" else layers.chunk_gated_delta_rule
    got_o, got_s = rule(q.to(DEV), k.to(DEV), v.to(DEV), g.to(DEV), beta.to(DEV), initial_state=s0.to(DEV))
    assert abs_err(got_o, want_o, 1e-3) < 1e-3
    assert abs_err(got_s, want_s, STATE_TOL) < STATE_TOL
    # and the float64 twin bounds both
    o64, s64 = f64.delta_rule_f64(q[0], k[0], v[0], g[0], beta[0], s0[0])
    assert np.abs(got_s[0].cpu().numpy() - s64).max() < STATE_TOL


def test_chunked_4096_tokens_against_reference_golden(gpu):
    """Config 4: 4096 tokens through the device rule vs the reference's chunked output."""
    import importlib
    layers = importlib.import_module(gpu.__name__ + ".layers")
    z = np.load(os.path.join(HERE, "cfg4.npz"))
    q, k, v, g, beta = gi.delta_rule_inputs(404, 4096)
    s0 = gi.dn_past(405)[1]
    got_o, got_s = layers.chunk_gated_delta_rule(q.to(DEV), k.to(DEV), v.to(DEV), g.to(DEV), beta.to(DEV),
                                                 initial_state=s0.to(DEV))
    o = got_o.reshape(-1).cpu()
    want = torch.from_numpy(z["chunk_out"])
    stride = max(1, o.numel() // want.numel())
    assert abs_err(o[::stride][: want.numel()], want, 2e-3) < 2e-3
    s = got_s.reshape(-1).cpu()
    ws = torch.from_numpy(z["chunk_state"])
    stride = max(1, s.numel() // ws.numel())
    assert abs_err(s[::stride][: ws.numel()], ws, STATE_TOL) < STATE_TOL
    # every output and state element against the oracle's chunked rule, whose
    # output and state digests equal the reference's (tests/test_golden.py)
    want_o, want_s = o_chunk(q, k, v, g, beta, initial_state=s0)
    assert abs_err(got_o, want_o, 2e-3) < 2e-3
    assert abs_err(got_s, want_s, STATE_TOL) < STATE_TOL


@pytest.mark.parametrize("hk,hv", [(1, 4), (3, 6), (2, 8)])
def test_decode_core_other_key_head_counts(gpu, hk, hv):
    """Value head h reads q/k head h % hk for any key-head count, one key head
    included (the decode kernel's division-free h % hk): decode steps between
    prefills of 5 tokens (the token loop), 20 and 70 tokens (the chunked rule
    with the conv inside its prep) against the oracle, conv window bit-exact."""
    qm = gpu
    dtype = torch.bfloat16
    ocfg = OracleConfig(linear_num_k_heads=hk, linear_num_v_heads=hv)
    cfg = qm.MixConfig(linear_num_k_heads=hk, linear_num_v_heads=hv)
    r = gi.rng(60 + hk)
    d, conv_dim = 128, ocfg.conv_dim
    w = {"blk.0.ssm_conv1d.weight": gi.normal(r, (conv_dim, 4), 0.5, dtype),
         "blk.0.ssm_a": -(gi.normal(r, (hv,)).abs() + 0.5),
         "blk.0.ssm_dt.bias": gi.normal(r, (hv,), 0.1),
         "blk.0.ssm_norm.weight": 1.0 + gi.normal(r, (d,), 0.1)}
    store = gi.FakeStore(w)
    conv = gi.normal(r, (1, conv_dim, 3)).to(dtype)
    state = gi.normal(r, (1, hv, d, d), 0.02)
    ocache = OracleHybridCache(1)
    ocache[0].conv_state, ocache[0].recurrent_state = conv.clone(), state.clone()
    model = qm.Qwen4MixModel(cfg, store, device=DEV)
    cache = qm.MixHybridCache(1, cfg, 1, 256, DEV, dtype)
    cache[0].conv_state = conv.to(DEV)
    cache[0].recurrent_state = state.to(DEV).clone()
    omix = OracleMixer(ocfg, store)
    worst_out = worst_state = 0.0
    for t, seq in enumerate((1, 1, 5, 20, 1, 70, 1)):
        mixed = gi.normal(r, (1, seq, conv_dim)).to(dtype)
        z = gi.normal(r, (1, seq, hv * d)).to(dtype)
        b = gi.normal(r, (1, seq, hv)).to(dtype)
        a = gi.normal(r, (1, seq, hv)).to(dtype)
        want = omix.dn_core(mixed, z, b, a, 0, ocache)
        got = model.dn_core(mixed.to(DEV), z.to(DEV), a.to(DEV), b.to(DEV), 0, cache[0])
        torch.cuda.synchronize()
        worst_out = max(worst_out, rel_err(got, want))
        worst_state = max(worst_state, abs_err(cache[0].recurrent_state, ocache[0].recurrent_state))
        assert torch.equal(cache[0].conv_state.cpu(), ocache[0].conv_state), (hk, hv, t)
    print(f"hk={hk} hv={hv}: worst out rel {worst_out:.2e} (bar {OUT_TOL}), "
          f"worst state abs {worst_state:.2e} (bar {STATE_TOL})", flush=True)
    assert worst_out < OUT_TOL and worst_state < STATE_TOL
    model.check_handoffs()
