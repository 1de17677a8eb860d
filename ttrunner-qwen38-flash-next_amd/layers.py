"""Device versions of the reference's delta-rule free functions.

``recurrent_gated_delta_rule`` and ``chunk_gated_delta_rule`` keep the
signatures and return values of reference/layers.py:155-192 and :195-275 for
device tensors: q, k (B, T, H, d_k), v (B, T, H, d_v), g and beta (B, T, H),
optional float32 state (B, H, d_k, d_v); they return ``(out, state)`` with
``out`` in the query's dtype. Both run the HIP kernels of libqwen4mix.so.
"""

from __future__ import annotations

import torch

from . import native


def _rule(query, key, value, g, beta, initial_state, name: str):
    batch, seq, heads, d = key.shape
    if value.shape != key.shape or query.shape != key.shape:
        raise ValueError("q, k and v must share one (B, T, H, d) shape")
    dt = query.dtype
    dev = query.device
    q = query.contiguous()
    k = key.to(dt).contiguous()
    v = value.to(dt).contiguous()
    g32 = g.to(torch.float32).contiguous()
    b32 = beta.to(torch.float32).contiguous()
    if initial_state is None:
        state = torch.zeros(batch, heads, d, d, dtype=torch.float32, device=dev)
    else:
        state = initial_state.to(dev, torch.float32).clone().contiguous()
    out = torch.empty(batch, seq, heads, d, dtype=dt, device=dev)
    args = [native.act_code(dt), batch, seq, heads, d, native.ptr(q), native.ptr(k), native.ptr(v),
            native.ptr(g32), native.ptr(b32), native.ptr(state), native.ptr(out)]
    if name == "qm_dn_chunked":
        n_ws = native.load().qm_dn_chunked_workspace(batch, seq, heads, d)
        ws = torch.empty(max(n_ws, 1), dtype=torch.uint8, device=dev)
        args += [native.ptr(ws), n_ws]
    native.call(name, *args, native.stream_handle(dev))
    return out, state


def recurrent_gated_delta_rule(query, key, value, g, beta, initial_state=None):
    """reference/layers.py:155-192 on the device (token loop kernel)."""
    return _rule(query, key, value, g, beta, initial_state, "qm_dn_recurrent")


def chunk_gated_delta_rule(query, key, value, g, beta, initial_state=None, chunk_size: int = 64):
    """reference/layers.py:195-275 on the device: the chunked WY/UT kernel."""
    if chunk_size != 64:
        raise ValueError("the device kernel implements chunk_size=64")
    return _rule(query, key, value, g, beta, initial_state, "qm_dn_chunked")
