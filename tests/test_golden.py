"""The oracle reproduces the reference's golden vectors (CPU only).

tests/golden/make_golden.py ran the reference's own modules on the inputs of
tests/golden/inputs.py and stored sha256 digests of every output, plus the
block scores and selected sets. Here the oracle runs on the same inputs and
must reproduce each digest bit for bit (same torch build and CPU kernels as the
generator, which golden_meta.json records); where the torch build differs the
digest check is skipped and the stored samples are compared to tolerance.
"""

from __future__ import annotations

import json
import math
import os
import sys

import numpy as np
import pytest
import torch

from oracle import selection as sel
from oracle.cache import OracleHybridCache
from oracle.config import OracleConfig
from oracle.layers import RotaryEmbedding, chunk_gated_delta_rule, recurrent_gated_delta_rule
from oracle.mixing import OracleMixer

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, HERE)
import inputs as gi  # noqa: E402

META = json.load(open(os.path.join(HERE, "golden_meta.json")))
SAME_BUILD = (META["torch"] == torch.__version__
              and META["cpu_capability"] == torch.backends.cpu.get_cpu_capability())


def _load(name):
    return np.load(os.path.join(HERE, f"{name}.npz"))


def _check(tensor, fixture, key, sample=None, atol=1e-5):
    want = META["digests"][fixture][key + "_sha"]
    if SAME_BUILD:
        assert gi.digest(tensor) == want, f"{fixture}.{key}: oracle is not bit-identical to the reference"
    if sample is not None:
        flat = tensor.detach().float().reshape(-1)
        stride = max(1, flat.numel() // sample.size)
        got = flat[::stride][: sample.size].numpy()
        assert np.abs(got - sample).max() <= atol * max(1.0, np.abs(sample).max())


@pytest.fixture(scope="module")
def rot():
    return RotaryEmbedding(64, 1e7, [11, 11, 10])


def _tables(rot, total):
    pos = torch.arange(total)[None]
    return rot(pos[None].expand(3, -1, -1))


def test_rope_tables_bit_identical(rot):
    cos, sin = _tables(rot, 32768)
    if not SAME_BUILD:
        pytest.skip("different torch build than the golden generator")
    assert gi.digest(cos) == META["digests"]["rope"]["cos_sha"]
    assert gi.digest(sin) == META["digests"]["rope"]["sin_sha"]


@pytest.mark.parametrize("tag", ["cfg1", "cfg3", "cfg3b"])
def test_decode_layers_match_reference(tag, rot):
    m = META[tag]
    z = _load(tag)
    dtype = torch.float32 if m["dtype"] == "torch.float32" else torch.bfloat16
    pos = m["pos"]
    hidden = gi.hidden_states(m["hidden_seed"], 1, dtype)
    cfg = OracleConfig()

    # Gated DeltaNet
    store = gi.FakeStore(gi.dn_weights(0, m["dn_seeds"][0], dtype))
    mixer = OracleMixer(cfg, store)
    cache = OracleHybridCache(4)
    conv, state = gi.dn_past(m["dn_seeds"][1], dtype)
    cache[0].conv_state, cache[0].recurrent_state = conv.clone(), state.clone()
    y = mixer._linear_attention(hidden, 0, cache)
    _check(y, tag, "dn_out", z["dn_out"])
    _check(cache[0].recurrent_state, tag, "dn_state", z["dn_state"])
    _check(cache[0].conv_state, tag, "dn_conv")

    # QSA
    store = gi.FakeStore(gi.qsa_weights(3, m["qsa_seeds"][0], dtype))
    mixer = OracleMixer(cfg, store)
    cache = OracleHybridCache(4)
    keys, values, idx_keys = gi.qsa_past(m["qsa_seeds"][1], pos, dtype)
    cache[3].keys, cache[3].values, cache[3].indexer_keys = keys, values, idx_keys
    cos, sin = _tables(rot, pos + 1)
    y = mixer._full_attention(hidden, 3, cos, sin, cache, pos)
    _check(y, tag, "qsa_out", z["qsa_out"])
    _check(cache[3].keys[:, :, -1:], tag, "qsa_newk")

    # the stage-wise indexer reproduces the reference's score vector and set
    q = mixer.indexer_query(hidden, 3, cos, sin)
    raw = torch.cat([idx_keys, torch.nn.functional.linear(hidden, store.get("blk.3.indexer.k_proj.weight"))], 1)
    n_blocks = (pos + 1) // gi.RATIO
    pooled = mixer.indexer_pooled(raw, 3, cos, sin, n_blocks)
    scores = mixer.indexer_scores(q, pooled)[0, 0]
    if SAME_BUILD:
        # the restated summation order (oracle/scores.c) and torch's own einsum
        # both give the reference's score vector bit for bit
        assert np.array_equal(scores.numpy(), z["scores"])
        assert np.array_equal(mixer.indexer_scores_torch(q, pooled)[0, 0].numpy(), z["scores"])
    ids = sel.select_blocks(z["scores"], pos, gi.RATIO, gi.BUDGET, n_blocks)
    assert np.array_equal(np.sort(ids), z["selected"])


def test_delta_rules_match_reference():
    z = _load("cfg4")
    q, k, v, g, beta = gi.delta_rule_inputs(404, 4096)
    s0 = gi.dn_past(405)[1]
    o_c, s_c = chunk_gated_delta_rule(q, k, v, g, beta, initial_state=s0)
    _check(o_c, "cfg4", "chunk_out", z["chunk_out"])
    _check(s_c, "cfg4", "chunk_state", z["chunk_state"])
    o_r, s_r = recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=s0)
    _check(o_r, "cfg4", "rec_out", z["rec_out"])
    _check(s_r, "cfg4", "rec_state", z["rec_state"])


def test_prefill_chunk_matches_reference(rot):
    m = META["cfg5"]
    z = _load("cfg5")
    past, seq = m["past"], m["seq"]
    dtype = torch.bfloat16
    cfg = OracleConfig()
    hidden = gi.hidden_states(m["hidden_seed"], seq, dtype)
    store = gi.FakeStore(gi.qsa_weights(3, m["qsa_seeds"][0], dtype))
    mixer = OracleMixer(cfg, store)
    cache = OracleHybridCache(4)
    keys, values, idx_keys = gi.qsa_past(m["qsa_seeds"][1], past, dtype)
    cache[3].keys, cache[3].values, cache[3].indexer_keys = keys, values, idx_keys
    cos, sin = _tables(rot, past + seq)
    y = mixer._full_attention(hidden, 3, cos, sin, cache, past)
    _check(y, "cfg5", "qsa_out", z["qsa_out"])
    # per-query selection from the reference's own scores, ties to the lower index
    n_blocks = (past + seq) // gi.RATIO
    for i in range(seq):
        ids = sel.select_blocks(z["scores"][i], past + i, gi.RATIO, gi.BUDGET, n_blocks)
        want = z["selected"][i]
        assert np.array_equal(np.sort(ids), want[want >= 0]), i

    store = gi.FakeStore(gi.dn_weights(0, m["dn_seeds"][0], dtype))
    mixer = OracleMixer(cfg, store)
    cache = OracleHybridCache(4)
    conv, state = gi.dn_past(m["dn_seeds"][1], dtype)
    cache[0].conv_state, cache[0].recurrent_state = conv.clone(), state.clone()
    y = mixer._linear_attention(hidden, 0, cache)
    _check(y, "cfg5", "dn_out", z["dn_out"])
    _check(cache[0].recurrent_state, "cfg5", "dn_state", z["dn_state"])
    _check(cache[0].conv_state, "cfg5", "dn_conv")


@pytest.mark.parametrize("seq", [1, 2, 3, 8, 128])
def test_restated_score_orders_equal_torch_einsum(seq):
    """oracle/scores.c reproduces torch's CPU einsum of reference/model.py:297
    bit for bit on the golden generator's build, for one query row (its
    16-partial order) and several (one chain per dot product), over block
    counts from 15 to 2048: random float32 inputs, so a wrong order would
    differ in most entries."""
    if not SAME_BUILD:
        pytest.skip("torch's einsum order belongs to the golden generator's build")
    from oracle.cnative import block_scores
    rng = np.random.default_rng(seq)
    for n in (15, 127, 512, 2048):
        q = torch.from_numpy(rng.standard_normal((1, seq, 4, 128)).astype(np.float32))
        k = torch.from_numpy(rng.standard_normal((1, n, 128)).astype(np.float32))
        want = torch.relu(torch.einsum("bqhd,bkd->bqhk", q, k)).sum(dim=2) / math.sqrt(128)
        assert torch.equal(block_scores(q, k), want), (seq, n)


def test_rope_rows_fixture_is_the_golden_builds(rot):
    """tests/golden/rope.npz holds the golden generator's table rows (the
    digests of the full tables pin them on that build)."""
    if not SAME_BUILD:
        pytest.skip("different torch build than the golden generator")
    cos, sin = _tables(rot, 32768)
    z = np.load(os.path.join(HERE, "rope.npz"))
    pos = torch.from_numpy(z["positions"].astype(np.int64))
    assert torch.equal(cos[0, pos], torch.from_numpy(z["cos"]))
    assert torch.equal(sin[0, pos], torch.from_numpy(z["sin"]))
