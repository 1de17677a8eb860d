"""Integer rules of the QSA block selection, in plain numpy / Python.

Restates reference/model.py:281-326 (``_indexer_mask``) as index arithmetic,
and the paging of the Tenstorrent engine (tt/model.py:117-129, 625-666,
1388-1444) as a logical-token -> physical-slot map.

For a query at absolute position ``p`` with compression ratio ``r``:

* block ``j`` covers tokens ``[j*r, j*r + r)`` and is *eligible* once its last
  token is visible: ``j*r + r - 1 <= p``, so ``n_elig(p) = (p + 1) // r``
  (reference/model.py:300-304);
* ``k = min(budget // r, n_blocks)`` blocks are picked by score, and picks that
  are not eligible are dropped (reference/model.py:306-313);
* the *tail* ``[((p + 1) // r) * r, p]`` is always visible; it is empty when p
  is the last token of a block (reference/model.py:323-326);
* ties in score go to the lower block index. (torch's CPU ``topk``, which the
  reference calls, leaves the order of equal scores unspecified; this build
  fixes it to the lower index. Both agree whenever the k-th and (k+1)-th
  eligible scores differ.)

Pinned by: brute force over every position of small contexts against the mask
built by ``oracle.mixing`` (tests/test_oracle_selection.py), the invariants of
reference tests/test_indexer_mask.py:122-167 and
tests/test_indexer_selection.py:46-121, 199-226 restated, and the golden
selected sets of the reference (tests/golden/).
"""

from __future__ import annotations

import numpy as np


def n_eligible(p: int, ratio: int) -> int:
    return (p + 1) // ratio


def tail_range(p: int, ratio: int) -> tuple[int, int]:
    """Half-open ``[start, end)`` of the always-visible trailing partial block."""
    return ((p + 1) // ratio) * ratio, p + 1


def topk_lower_index(scores: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k largest finite scores, best first; equal scores -> lower index."""
    scores = np.asarray(scores, dtype=np.float32)
    finite = np.nonzero(np.isfinite(scores))[0]
    # lexsort sorts by the last key first: descending score, then ascending index
    order = np.lexsort((finite, -scores[finite].astype(np.float64)))
    return finite[order[:k]].astype(np.int64)


def select_blocks(scores: np.ndarray, p: int, ratio: int, budget: int, n_blocks: int) -> np.ndarray:
    """Selected block ids for one query, in rank order (best first).

    ``scores`` holds one float32 score per block ``0..n_blocks-1``; blocks that
    are not eligible at ``p`` are ignored whatever their score.
    """
    k = min(budget // ratio, n_blocks)
    elig = n_eligible(p, ratio)
    row = np.full(n_blocks, -np.inf, dtype=np.float32)
    m = min(elig, n_blocks)
    row[:m] = np.asarray(scores, dtype=np.float32)[:m]
    return topk_lower_index(row, k)


def visible_tokens(block_ids, p: int, ratio: int) -> np.ndarray:
    """Sorted logical token positions a query at ``p`` attends to."""
    toks = [np.arange(int(b) * ratio, int(b) * ratio + ratio) for b in block_ids]
    start, end = tail_range(p, ratio)
    toks.append(np.arange(start, end))
    out = np.concatenate(toks) if toks else np.zeros(0, np.int64)
    return np.sort(out[out <= p])


def physical_slots(tokens, page_table, page_size: int) -> np.ndarray:
    """(page, row) of each logical token under a page table."""
    tokens = np.asarray(tokens, dtype=np.int64)
    pages = np.asarray(page_table, dtype=np.int64)[tokens // page_size]
    return np.stack([pages, tokens % page_size], axis=-1)
