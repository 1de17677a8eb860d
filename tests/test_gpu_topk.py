"""Top-k of the block selection (qm_qsa_select, reference/model.py:297-326):
the ids the kernel selects must be the reference's top-k of the kernel's own
block scores, ties to the lower block index. The scores themselves are pinned
bit for bit against the reference's score vectors in test_gpu_pins.py; here
the inputs are shaped to drive each ranking path:
counting (up to 128 blocks), the bucket threshold over the scores' range
(typically topk plus a few candidates), and radix select where more than 128
keys crowd the threshold bucket (equal, clustered or mostly-zero scores, one
outlier)."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"
RATIO, BUDGET, IDX_HEADS = 64, 2048, 4
TOPK = BUDGET // RATIO


def _select(qm, block_keys: np.ndarray, iq: np.ndarray, pos0: int):
    """qm_qsa_select over rows at positions pos0, pos0 + 1, ... of one sequence."""
    native = qm.native
    rows = iq.shape[0]
    max_blocks = block_keys.shape[0]
    max_ctx = max_blocks * RATIO
    g = native.QsaGeom(1, 16, 2, 256, 64, IDX_HEADS, 128, RATIO, BUDGET, 64, max_ctx // 64, max_ctx, max_blocks,
                       native.act_code(torch.float32), 1e-6)
    bk = torch.from_numpy(block_keys).to(DEV).reshape(1, max_blocks, 128).contiguous()
    q = torch.from_numpy(iq).to(DEV).contiguous()
    pos = torch.tensor([pos0], dtype=torch.int32, device=DEV)
    ids = torch.full((rows, TOPK), -1, dtype=torch.int32, device=DEV)
    n_sel = torch.empty(rows, dtype=torch.int32, device=DEV)
    scores = torch.empty(rows, max_blocks, dtype=torch.float32, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    native.call("qm_qsa_select", ctypes.byref(g), rows, native.ptr(q), native.ptr(bk), native.ptr(pos), None,
                native.ptr(ids), native.ptr(n_sel), None, native.ptr(scores), stream)
    torch.cuda.synchronize()
    return ids.cpu().numpy(), n_sel.cpu().numpy(), scores.cpu().numpy()


def _check(ids, n_sel, scores, pos0):
    for r in range(ids.shape[0]):
        n_elig = min((pos0 + r + 1) // RATIO, scores.shape[1])
        s = scores[r, :n_elig].astype(np.float64)
        want = np.lexsort((np.arange(n_elig), -s))[:TOPK]      # score down, then index up
        assert n_sel[r] == min(n_elig, TOPK)
        got = ids[r, : n_sel[r]]
        assert np.array_equal(got, want), (r, got[:8], want[:8])


def _case(kind: str, n_blocks: int, rng):
    keys = rng.standard_normal((n_blocks, 128)).astype(np.float32)
    iq = rng.standard_normal((8, IDX_HEADS, 128)).astype(np.float32)
    if kind == "equal":
        keys[:] = keys[0]
    elif kind == "clustered":
        keys = keys[rng.integers(0, 3, n_blocks)]
    elif kind == "zeros":
        iq = np.abs(iq)
        keys = -np.abs(keys)
        hot = rng.choice(n_blocks, 10, replace=False)
        keys[hot] = np.abs(keys[hot])
    elif kind == "outlier":
        iq = np.abs(iq)
        keys = np.abs(keys)
        keys[n_blocks // 3] *= 1e6
    elif kind == "duplicates":
        for a, b in [(5, 300), (7, 400), (11, 12)]:
            keys[b % n_blocks] = keys[a]
    return keys, iq


@pytest.mark.parametrize("kind", ["random", "equal", "clustered", "zeros", "outlier", "duplicates"])
@pytest.mark.parametrize("n_blocks", [100, 511, 1500, 4096])
def test_selected_ids_are_the_top_k_of_the_scores(gpu, kind, n_blocks):
    rng = np.random.default_rng(1000 + n_blocks + len(kind))
    keys, iq = _case(kind, n_blocks, rng)
    pos0 = n_blocks * RATIO - 8          # rows at n_blocks - 1 and n_blocks eligible blocks
    print(f"top-k {kind} blocks={n_blocks}", flush=True)
    ids, n_sel, scores = _select(gpu, keys, iq, pos0)
    _check(ids, n_sel, scores, pos0)
