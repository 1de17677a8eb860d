"""Float64 twins of the delta rule, for tolerance analysis.

Straight per-head, per-column loops in float64 over the recurrence of
reference/layers.py:184-191 (decay first, predict with the decayed state,
output from the updated state). Used to measure how far the float32 oracle and
the HIP kernels each sit from the exact answer, and as the brute force that
pins ``oracle.layers.recurrent_gated_delta_rule``.

Pinned by: the special cases beta = 0 (``S' = exp(g) S``, ``o = S'^T q``) and
g = 0, beta = 1, S = 0 (``S' = k v^T``, ``o = (q.k) v``), asserted in
tests/test_oracle_layers.py.
"""

from __future__ import annotations

import numpy as np


def _np64(x):
    if hasattr(x, "detach"):
        x = x.detach().cpu().double().numpy()
    return np.asarray(x, np.float64)


def delta_rule_f64(q, k, v, g, beta, state=None):
    """q, k: (T, H, dk); v: (T, H, dv); g, beta: (T, H); state: (H, dk, dv).

    q and k are L2-normalised here (eps 1e-6) and q is scaled by 1/sqrt(dk),
    as in the reference. Returns (out (T, H, dv), state (H, dk, dv)).
    """
    q, k, v, g, beta = (_np64(x) for x in (q, k, v, g, beta))
    n_t, n_h, dk = k.shape
    dv = v.shape[-1]
    S = np.zeros((n_h, dk, dv)) if state is None else _np64(state).copy()
    qn = q / np.sqrt((q * q).sum(-1, keepdims=True) + 1e-6) / np.sqrt(dk)
    kn = k / np.sqrt((k * k).sum(-1, keepdims=True) + 1e-6)
    out = np.zeros((n_t, n_h, dv))
    for t in range(n_t):
        for h in range(n_h):
            S[h] *= np.exp(g[t, h])
            pred = kn[t, h] @ S[h]
            delta = (v[t, h] - pred) * beta[t, h]
            S[h] += np.outer(kn[t, h], delta)
            out[t, h] = qn[t, h] @ S[h]
    return out, S
