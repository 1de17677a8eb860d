"""Device versions of the reference's free functions of this path.

``causal_conv1d`` and ``causal_conv1d_step`` keep the signatures and return
values of reference/layers.py:133-138 and :141-147 for device tensors of shape
(B, C, T) (depthwise weight (C, K)); ``recurrent_gated_delta_rule`` and
``chunk_gated_delta_rule`` those of :155-192 and :195-275: q, k (B, T, H, d_k),
v (B, T, H, d_v), g and beta (B, T, H), optional float32 state (B, H, d_k,
d_v); they return ``(out, state)`` with ``out`` in the query's dtype. All run
the HIP kernels of libqwen4mix.so; inputs must be float32 or bfloat16 tensors
on the GPU.
"""

from __future__ import annotations

import torch

from . import native


def _conv(x, state, weight, activation: bool, want_state: bool):
    if x.dim() != 3 or weight.dim() != 2 or weight.shape[0] != x.shape[1]:
        raise ValueError(f"causal conv: x must be (B, C, T) and weight (C, K), got {tuple(x.shape)}, "
                         f"{tuple(weight.shape)}")
    batch, channels, seq = x.shape
    taps = int(weight.shape[1])
    dt = x.dtype
    dev = x.device
    xc = x.contiguous()
    w = weight.to(dev, dt).contiguous()
    st = None
    if state is not None:
        if tuple(state.shape) != (batch, channels, taps - 1):
            raise ValueError(f"causal conv: state must be {(batch, channels, taps - 1)}, got {tuple(state.shape)}")
        st = state.to(dev, dt).contiguous()
    out = torch.empty_like(xc)
    new_state = torch.empty(batch, channels, taps - 1, dtype=dt, device=dev) if want_state else None
    native.call("qm_causal_conv1d", native.act_code(dt), batch, channels, seq, taps, native.ptr(xc), native.ptr(st),
                native.ptr(w), int(bool(activation)), native.ptr(out), native.ptr(new_state),
                native.stream_handle(dev))
    return out, new_state


def causal_conv1d(x, weight, activation: bool = True):
    """reference/layers.py:133-138 on the device: depthwise causal conv over
    (B, C, T), zero history, silu when ``activation``."""
    return _conv(x, None, weight, activation, want_state=False)[0]


def causal_conv1d_step(x, state, weight, activation: bool = True):
    """reference/layers.py:141-147 on the device: the conv of x (B, C, T)
    against the rolling window ``state`` (B, C, K-1); returns (out, new_state),
    new_state the last K-1 columns of [state | x]."""
    return _conv(x, state, weight, activation, want_state=True)


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
