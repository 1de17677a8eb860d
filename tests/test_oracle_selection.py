"""QSA selection semantics of the oracle (CPU only).

Restates the invariants of reference tests/test_indexer_mask.py:122-167 (same
fake-store pattern, HIDDEN 8, DIM 4, HEADS 2, RATIO 4, BUDGET 16) and the
selection arithmetic of reference tests/test_indexer_selection.py:46-121,
199-226, and checks the integer rules of ``oracle.selection`` against the
boolean mask ``oracle.mixing`` builds, position by position.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import selection as sel
from oracle.mixing import OracleMixer

HIDDEN, DIM, HEADS, RATIO, BUDGET = 8, 4, 2, 4, 16


class _Cfg:
    indexer_head_dim = DIM
    indexer_compress_ratio = RATIO
    indexer_budget = BUDGET
    rms_norm_eps = 1e-6


class _Store:
    def __init__(self, weights):
        self._w = weights

    def get(self, name):
        return self._w[name.split(".", 2)[2]]


def _mixer(seed: int = 0, tie_rule: str = "lower_index") -> OracleMixer:
    g = torch.Generator().manual_seed(seed)
    weights = {
        "indexer.q_proj.weight": torch.randn(HEADS * DIM, HIDDEN, generator=g),
        "indexer.k_proj.weight": torch.randn(DIM, HIDDEN, generator=g),
        "indexer.q_norm.weight": torch.ones(DIM),
        "indexer.k_norm.weight": torch.ones(DIM),
    }
    return OracleMixer(_Cfg(), _Store(weights), tie_rule=tie_rule)


def _mask(m, hidden, kv_len, query_offset):
    rope = torch.zeros(1, max(kv_len, hidden.shape[1]), DIM)
    return m._indexer_mask(hidden, 0, rope + 1.0, rope, None, kv_len, query_offset)


def test_whole_prompt_equals_token_by_token():
    m = _mixer()
    g = torch.Generator().manual_seed(1)
    for total in (4, 5, 8, 12, 16, 23, 40):
        hidden = torch.randn(1, total, HIDDEN, generator=g)
        whole = _mask(m, hidden, total, 0)[0, 0]
        for p in range(total):
            alone = _mask(m, hidden[:, : p + 1], p + 1, 0)[0, 0, -1]
            assert torch.equal(whole[p, : p + 1], alone), (total, p)


def test_every_query_sees_at_least_itself_and_nothing_beyond():
    m = _mixer()
    g = torch.Generator().manual_seed(2)
    for total in (4, 8, 12, 16, 20, 33, 64):
        hidden = torch.randn(1, total, HIDDEN, generator=g)
        mask = _mask(m, hidden, total, 0)[0, 0]
        assert mask.any(dim=-1).all()
        future = torch.triu(torch.ones(total, total, dtype=torch.bool), diagonal=1)
        assert not (mask & future).any()


def test_below_budget_is_exactly_causal():
    m = _mixer()
    hidden = torch.randn(1, BUDGET, HIDDEN, generator=torch.Generator().manual_seed(4))
    mask = _mask(m, hidden, BUDGET, 0)[0, 0]
    causal = ~torch.triu(torch.ones(BUDGET, BUDGET, dtype=torch.bool), diagonal=1)
    assert torch.equal(mask, causal)


def test_integer_rules_reproduce_the_mask_position_by_position():
    """oracle.selection (what the HIP kernels implement) == oracle.mixing's mask."""
    m = _mixer(seed=7)
    g = torch.Generator().manual_seed(8)
    total = 61
    hidden = torch.randn(1, total, HIDDEN, generator=g)
    mask = _mask(m, hidden, total, 0)[0, 0]
    rope = torch.zeros(1, total, DIM)
    q = m.indexer_query(hidden, 0, rope + 1.0, rope)
    import torch.nn.functional as F
    raw = F.linear(hidden, m.bw(0, "indexer.k_proj.weight"))
    n_blocks = total // RATIO
    pooled = m.indexer_pooled(raw, 0, rope + 1.0, rope, n_blocks)
    scores = m.indexer_scores(q, pooled)[0].numpy()
    for p in range(total):
        ids = sel.select_blocks(scores[p], p, RATIO, BUDGET, n_blocks)
        toks = sel.visible_tokens(ids, p, RATIO)
        want = np.nonzero(mask[p].numpy())[0]
        assert np.array_equal(toks, want), p


@pytest.mark.parametrize("p", [0, 1, 2, 3, 4, 7, 8, 100, 2047, 2048, 2599, 2598])
def test_only_complete_blocks_are_eligible(p):
    n = sel.n_eligible(p, RATIO)
    for j in range(0, 1024):
        complete = RATIO * j + RATIO - 1 <= p
        assert (j < n) == complete


@pytest.mark.parametrize("p", [0, 1, 2, 4, 5, 100, 2598, 3, 7, 2047, 2599])
def test_tail_is_the_incomplete_block_prefix(p):
    start, end = sel.tail_range(p, RATIO)
    if p % RATIO == RATIO - 1:
        assert start == end == p + 1          # complete: it competes instead
    else:
        assert start == RATIO * (p // RATIO) and end == p + 1
    # the tail never overlaps a selectable block
    assert start >= RATIO * sel.n_eligible(p, RATIO)


def test_every_position_sees_itself_and_budget_rule():
    topk = 2048 // RATIO
    first_binding = None
    for p in range(0, 2600):
        start, end = sel.tail_range(p, RATIO)
        own_selectable = (p // RATIO) < sel.n_eligible(p, RATIO)
        assert (start <= p < end) or own_selectable
        if first_binding is None and sel.n_eligible(p, RATIO) > topk:
            first_binding = p
    assert first_binding >= 2048


def test_topk_ties_go_to_lower_index():
    s = np.array([1.0, 0.0, 0.0, 2.0, 0.0, 0.0, -np.inf, 0.0], np.float32)
    assert sel.topk_lower_index(s, 4).tolist() == [3, 0, 1, 2]
    assert sel.topk_lower_index(s, 10).tolist() == [3, 0, 1, 2, 4, 5, 7]
    # the torch-tensor form in oracle.mixing uses the same rule
    m = _mixer()
    got = m._topk_blocks(torch.from_numpy(s)[None], 4)[0].tolist()
    assert got == [3, 0, 1, 2]


def test_physical_slots_follow_the_page_table():
    rng = np.random.default_rng(0)
    table = rng.permutation(32)
    toks = np.arange(0, 32 * 64, 37)
    slots = sel.physical_slots(toks, table, 64)
    assert np.array_equal(slots[:, 0], table[toks // 64])
    assert np.array_equal(slots[:, 1], toks % 64)
