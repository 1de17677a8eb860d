"""Oracle restatement of reference/layers.py (the token-mixing primitives).

Every function performs the same torch CPU operations, in the same order and on
tensors of the same shapes and dtypes, as the reference function it cites, so
that its float32/bfloat16 results are bit-identical to the reference's on the
same torch build. Only naming and structure are this file's own.

Pinning (see tests/test_oracle_layers.py and tests/test_golden.py):
* rms_norm / rms_norm_gated / l2norm -- closed forms in float64, and golden
  vectors of the reference's whole-layer outputs.
* RotaryEmbedding / apply_rotary -- identity at position 0, norm preservation of
  each rotated pair, agreement with a float64 cos/sin table, golden vectors.
* causal_conv1d / causal_conv1d_step -- brute-force 4-tap sum + silu; the step
  form equals the last column of the full form.
* recurrent_gated_delta_rule -- float64 brute force (oracle/f64.py), the special
  cases beta=0 (pure decay) and g=0, beta=1, S=0 (S' = k v^T).
* chunk_gated_delta_rule -- equals the recurrent form (reference
  tests/test_delta_rule.py:27-61 restated), finite under extreme decay, and
  golden vectors of the reference's chunked output.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, group_size: int | None = None) -> torch.Tensor:
    """reference/layers.py:31-43.

    Normalises the last axis in float32 -- or, with ``group_size``, each run of
    ``group_size`` consecutive elements of it on its own (one residual stream
    each) -- scales by the weight and returns the input dtype.
    """
    in_dtype = x.dtype
    xf = x.float()
    if group_size is not None:
        groups = xf.unflatten(-1, (-1, group_size))
        scale = torch.rsqrt(groups.pow(2).mean(-1, keepdim=True) + eps)
        xf = (groups * scale).flatten(-2)
    else:
        xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (xf * weight.float()).to(in_dtype)


def rms_norm_gated(x, gate, weight, eps: float, activation: str = "sigmoid"):
    """reference/layers.py:46-61: RMS norm, weight, then a sigmoid (or silu) gate."""
    in_dtype = x.dtype
    h = x.float()
    h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    h = weight.float() * h
    if activation == "sigmoid":
        gate_val = torch.sigmoid(gate.float())
    else:
        gate_val = F.silu(gate.float())
    return (h * gate_val).to(in_dtype)


def l2norm(x: torch.Tensor, dim: int = -1, eps: float = 1e-6) -> torch.Tensor:
    """reference/layers.py:64-65."""
    return x * torch.rsqrt((x * x).sum(dim=dim, keepdim=True) + eps)


class RotaryEmbedding:
    """reference/layers.py:73-108: partial, interleaved multimodal RoPE.

    ``inv_freq[i] = 1 / theta^(2i / rope_dim)``. For text input the three
    position rows are equal, so the interleave is a no-op on the values.
    """

    def __init__(self, rope_dim: int, theta: float, mrope_section: list[int]):
        self.rope_dim = rope_dim
        self.mrope_section = list(mrope_section)
        exponents = torch.arange(0, rope_dim, 2, dtype=torch.float) / rope_dim
        self.inv_freq = 1.0 / (theta ** exponents)

    def _interleave(self, freqs: torch.Tensor) -> torch.Tensor:
        # axis 1 (height) owns columns 1, 4, 7, ... and axis 2 (width) 2, 5, 8, ...
        merged = freqs[0].clone()
        for axis in (1, 2):
            span = self.mrope_section[axis] * 3
            cols = slice(axis, span, 3)
            merged[..., cols] = freqs[axis][..., cols]
        return merged

    def __call__(self, position_ids: torch.Tensor):
        if position_ids.ndim == 2:
            position_ids = position_ids[None].expand(3, -1, -1)
        batch = position_ids.shape[1]
        inv = self.inv_freq[None, None, :, None].float().expand(3, batch, -1, 1)
        pos = position_ids[:, :, None, :].float()
        freqs = (inv @ pos).transpose(2, 3)
        freqs = self._interleave(freqs)
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos(), emb.sin()


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """reference/layers.py:111-113: [x1, x2] -> [-x2, x1] over the last axis."""
    mid = x.shape[-1] // 2
    return torch.cat((-x[..., mid:], x[..., :mid]), dim=-1)


def apply_rotary(x, cos, sin, unsqueeze_dim: int = 1):
    """reference/layers.py:116-125: rotate the first cos.shape[-1] channels.

    ``x_rot * cos`` promotes a bf16 ``x`` to float32, so the result is float32
    whenever the tables are.
    """
    cos = cos.unsqueeze(unsqueeze_dim)
    sin = sin.unsqueeze(unsqueeze_dim)
    n_rot = cos.shape[-1]
    head, rest = x[..., :n_rot], x[..., n_rot:]
    head = head * cos + rotate_half(head) * sin
    return torch.cat([head, rest], dim=-1)


def causal_conv1d(x, weight, activation: bool = True):
    """reference/layers.py:133-138: depthwise causal conv over (B, C, T)."""
    n_ch = x.shape[1]
    taps = weight.shape[-1]
    y = F.conv1d(x, weight.unsqueeze(1), padding=taps - 1, groups=n_ch)[:, :, : x.shape[-1]]
    return F.silu(y) if activation else y


def causal_conv1d_step(x, state, weight, activation: bool = True):
    """reference/layers.py:141-147: one conv step against the rolling window.

    ``state`` holds the previous ``K-1`` inputs, oldest first. Returns
    ``(out, new_state)`` where ``new_state`` is the last ``K-1`` columns of
    ``[state | x]``.
    """
    n_ch = x.shape[1]
    window = torch.cat([state, x], dim=-1)
    new_state = window[:, :, -state.shape[-1]:].clone()
    y = F.conv1d(window, weight.unsqueeze(1), padding=0, groups=n_ch)[:, :, -x.shape[-1]:]
    return (F.silu(y) if activation else y), new_state


def _to_heads_f32(*tensors):
    """(B, T, H, ...) -> (B, H, T, ...) float32 contiguous."""
    return [t.transpose(1, 2).to(torch.float32).contiguous() for t in tensors]


def recurrent_gated_delta_rule(query, key, value, g, beta, initial_state=None):
    """reference/layers.py:155-192: the gated delta rule, one token at a time.

    Per head and token: ``S <- S * exp(g)``; ``pred = S^T k``;
    ``delta = (v - pred) * beta``; ``S <- S + k delta^T``; ``o = S^T q``, with
    q, k L2-normalised (eps 1e-6) and q divided by sqrt(d_k). The state is
    float32 ``(B, H, d_k, d_v)``; the output is cast back to the query dtype.
    """
    out_dtype = query.dtype
    q, k, v, bt, gl = _to_heads_f32(query, key, value, beta, g)
    q = l2norm(q, dim=-1)
    k = l2norm(k, dim=-1)
    q = q / (q.shape[-1] ** 0.5)

    n_b, n_h, n_t, d_k = k.shape
    d_v = v.shape[-1]
    if initial_state is None:
        S = torch.zeros(n_b, n_h, d_k, d_v, dtype=torch.float32, device=v.device)
    else:
        S = initial_state.to(torch.float32)
    out = torch.zeros_like(v)
    for t in range(n_t):
        qt, kt, vt = q[:, :, t], k[:, :, t], v[:, :, t]
        S = S * gl[:, :, t].exp()[..., None, None]
        pred = (S * kt.unsqueeze(-1)).sum(dim=-2)
        delta = (vt - pred) * bt[:, :, t].unsqueeze(-1)
        S = S + kt.unsqueeze(-1) * delta.unsqueeze(-2)
        out[:, :, t] = (S * qt.unsqueeze(-1)).sum(dim=-2)
    return out.transpose(1, 2).contiguous().to(out_dtype), S


def chunk_gated_delta_rule(query, key, value, g, beta, initial_state=None, chunk_size: int = 64):
    """reference/layers.py:195-275: the WY/UT chunked form of the same rule.

    Pads T to a multiple of ``chunk_size`` (zero decay, zero beta), forms the
    within-chunk pairwise decays by subtraction in log space, inverts
    ``I + strictly_lower(k_beta k^T * decay)`` by forward substitution, and
    scans the chunks carrying the float32 state.
    """
    out_dtype = query.dtype
    q, k, v, bt, gl = _to_heads_f32(query, key, value, beta, g)
    q = l2norm(q, dim=-1)
    k = l2norm(k, dim=-1)
    q = q * (q.shape[-1] ** -0.5)

    n_b, n_h, n_t, d_k = k.shape
    d_v = v.shape[-1]
    C = chunk_size
    pad = (C - n_t % C) % C
    if pad:
        q, k, v = (F.pad(t, (0, 0, 0, pad)) for t in (q, k, v))
        bt, gl = (F.pad(t, (0, pad)) for t in (bt, gl))
    n_tot = n_t + pad
    n_c = n_tot // C

    v_beta = v * bt.unsqueeze(-1)
    k_beta = k * bt.unsqueeze(-1)

    def per_chunk(t):
        return t.reshape(n_b, n_h, n_c, C, t.shape[-1])

    q, k, k_beta, v_beta = per_chunk(q), per_chunk(k), per_chunk(k_beta), per_chunk(v_beta)
    gl = gl.reshape(n_b, n_h, n_c, C)

    above = torch.ones(C, C, dtype=torch.bool, device=q.device).triu(1)
    cum = gl.cumsum(dim=3)
    # decay[i, j] = exp(cum_i - cum_j) for j <= i, 0 above the diagonal
    decay = (cum.unsqueeze(4) - cum.unsqueeze(3)).masked_fill(above, float("-inf")).exp()

    T = (k_beta @ k.transpose(-1, -2)) * decay
    qk_in = (q @ k.transpose(-1, -2)) * decay
    k_beta_cum = k_beta * cum.exp().unsqueeze(-1)

    eye_b = torch.eye(C, dtype=torch.bool, device=q.device)
    T = -T.masked_fill(~above.T | eye_b, 0)
    for i in range(1, C):
        T[..., i, :i] = T[..., i, :i] + (T[..., i, :, None].clone() * T[..., :, :i].clone()).sum(-2)
    T = T + torch.eye(C, dtype=T.dtype, device=q.device)

    w = T @ k_beta_cum
    u = T @ v_beta

    if initial_state is None:
        S = torch.zeros(n_b, n_h, d_k, d_v, dtype=torch.float32, device=v.device)
    else:
        S = initial_state.to(torch.float32)

    q_dec = q * cum.exp().unsqueeze(-1)
    k_dec = k * (cum[..., -1:] - cum).exp().unsqueeze(-1)
    end_dec = cum[..., -1].exp()[..., None, None]

    out = torch.zeros_like(v.reshape(n_b, n_h, n_c, C, d_v))
    for c in range(n_c):
        v_new = u[:, :, c] - w[:, :, c] @ S
        from_state = q_dec[:, :, c] @ S
        out[:, :, c] = from_state + qk_in[:, :, c] @ v_new
        S = S * end_dec[:, :, c] + k_dec[:, :, c].transpose(-1, -2) @ v_new

    out = out.reshape(n_b, n_h, n_tot, d_v)[:, :, :n_t]
    return out.transpose(1, 2).contiguous().to(out_dtype), S
