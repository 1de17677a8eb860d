"""The oracle's float primitives, pinned by closed forms, brute force and the
reference's own self-consistency tests (reference tests/test_delta_rule.py,
restated). CPU only."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import f64
from oracle.config import OracleConfig
from oracle.layers import (
    RotaryEmbedding,
    apply_rotary,
    causal_conv1d,
    causal_conv1d_step,
    chunk_gated_delta_rule,
    l2norm,
    recurrent_gated_delta_rule,
    rms_norm,
    rms_norm_gated,
)


def _dr_inputs(seq: int, decay_scale: float, seed: int = 0):
    # the generator of reference tests/test_delta_rule.py:15-24
    torch.manual_seed(seed)
    b, h, dk, dv = 2, 4, 32, 32
    return (
        torch.randn(b, seq, h, dk),
        torch.randn(b, seq, h, dk),
        torch.randn(b, seq, h, dv),
        -torch.rand(b, seq, h) * decay_scale,
        torch.rand(b, seq, h),
    )


@pytest.mark.parametrize("seq", [1, 7, 64, 100])
@pytest.mark.parametrize("decay_scale", [0.5, 160.0])
def test_chunked_matches_recurrent(seq, decay_scale):
    q, k, v, g, beta = _dr_inputs(seq, decay_scale)
    o_r, s_r = recurrent_gated_delta_rule(q, k, v, g, beta)
    o_c, s_c = chunk_gated_delta_rule(q, k, v, g, beta)
    assert torch.allclose(o_r, o_c, atol=1e-4)
    assert torch.allclose(s_r, s_c, atol=1e-4)


def test_extreme_decay_keeps_state_finite():
    q, k, v, g, beta = _dr_inputs(100, 200.0)
    out, state = chunk_gated_delta_rule(q, k, v, g, beta)
    assert torch.isfinite(out).all() and torch.isfinite(state).all()


def test_prefill_then_decode_matches_full_prefill():
    seq = 33
    q, k, v, g, beta = _dr_inputs(seq + 1, 8.0)
    full, _ = chunk_gated_delta_rule(q, k, v, g, beta)
    _, state = chunk_gated_delta_rule(*[x[:, :seq] for x in (q, k, v, g, beta)])
    last, _ = recurrent_gated_delta_rule(*[x[:, seq:seq + 1] for x in (q, k, v, g, beta)], initial_state=state)
    assert torch.allclose(full[:, seq:seq + 1], last, atol=1e-4)


def test_recurrent_matches_float64_brute_force():
    q, k, v, g, beta = _dr_inputs(9, 2.0, seed=3)
    s0 = torch.randn(2, 4, 32, 32) * 0.02
    out, state = recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=s0)
    for b in range(2):
        o64, s64 = f64.delta_rule_f64(q[b], k[b], v[b], g[b], beta[b], s0[b])
        assert np.abs(out[b].numpy() - o64).max() < 1e-5
        assert np.abs(state[b].numpy() - s64).max() < 1e-5


def test_delta_rule_special_cases():
    torch.manual_seed(1)
    q, k, v = torch.randn(1, 1, 2, 8), torch.randn(1, 1, 2, 8), torch.randn(1, 1, 2, 8)
    s0 = torch.randn(1, 2, 8, 8)
    g = torch.full((1, 1, 2), -0.7)
    # beta = 0: pure decay, output read from the decayed state
    out, state = recurrent_gated_delta_rule(q, k, v, g, torch.zeros(1, 1, 2), initial_state=s0)
    assert torch.allclose(state, s0 * math.exp(-0.7), atol=1e-6)
    qn = l2norm(q.float()) / math.sqrt(8)
    assert torch.allclose(out[0, 0], torch.einsum("hi,hij->hj", qn[0, 0], state[0]), atol=1e-6)
    # g = 0, beta = 1, S = 0: S' = k v^T and o = (q.k) v
    out, state = recurrent_gated_delta_rule(q, k, v, torch.zeros(1, 1, 2), torch.ones(1, 1, 2))
    kn = l2norm(k.float())
    assert torch.allclose(state[0], torch.einsum("hi,hj->hij", kn[0, 0], v[0, 0]), atol=1e-6)
    qk = (qn[0, 0] * kn[0, 0]).sum(-1, keepdim=True)
    assert torch.allclose(out[0, 0], qk * v[0, 0], atol=1e-6)


def test_conv_step_is_last_column_of_full_conv_and_a_four_tap_sum():
    torch.manual_seed(2)
    ch, taps, t = 6, 4, 9
    x = torch.randn(1, ch, t)
    w = torch.randn(ch, taps)
    full = causal_conv1d(x, w)
    state = torch.zeros(1, ch, taps - 1)
    for i in range(t):
        y, state = causal_conv1d_step(x[:, :, i:i + 1], state, w)
        assert torch.allclose(y[:, :, 0], full[:, :, i], atol=1e-6)
        # brute force: tap 0 is the oldest sample
        acc = torch.zeros(ch)
        for j in range(taps):
            src = i - (taps - 1) + j
            if src >= 0:
                acc += w[:, j] * x[0, :, src]
        assert torch.allclose(y[0, :, 0], F.silu(acc), atol=1e-5)
    assert torch.equal(state, x[:, :, -(taps - 1):])


def test_norms_match_float64_closed_forms():
    torch.manual_seed(4)
    x = torch.randn(5, 128)
    w = torch.rand(128) + 0.5
    z = torch.randn(5, 128)
    x64, w64, z64 = x.double(), w.double(), z.double()
    r = x64 / torch.sqrt((x64 ** 2).mean(-1, keepdim=True) + 1e-6) * w64
    assert torch.allclose(rms_norm(x, w, 1e-6).double(), r, atol=1e-5)
    gated = r / (1 + torch.exp(-z64))
    assert torch.allclose(rms_norm_gated(x, z, w, 1e-6).double(), gated, atol=1e-5)
    l2 = x64 / torch.sqrt((x64 ** 2).sum(-1, keepdim=True) + 1e-6)
    assert torch.allclose(l2norm(x).double(), l2, atol=1e-6)


def test_rope_identity_at_zero_and_pairwise_norm():
    cfg = OracleConfig()
    rot = RotaryEmbedding(cfg.rope_dim, cfg.rope_theta, cfg.mrope_section)
    pos = torch.arange(0, 300)[None]
    cos, sin = rot(pos)
    assert torch.equal(cos[0, 0], torch.ones(cfg.rope_dim)) and torch.equal(sin[0, 0], torch.zeros(cfg.rope_dim))
    # float64 table: angle = pos * theta^(-2i/d), duplicated halves
    i = torch.arange(cfg.rope_dim // 2, dtype=torch.float64)
    ang = pos[0, :, None].double() * cfg.rope_theta ** (-2 * i / cfg.rope_dim)
    ang = torch.cat([ang, ang], -1)
    assert torch.allclose(cos[0].double(), torch.cos(ang), atol=2e-4)
    x = torch.randn(1, 3, 300, 256)
    y = apply_rotary(x, cos, sin)
    half = cfg.rope_dim // 2
    n_in = x[..., :half] ** 2 + x[..., half:cfg.rope_dim] ** 2
    n_out = y[..., :half] ** 2 + y[..., half:cfg.rope_dim] ** 2
    assert torch.allclose(n_in, n_out, atol=1e-4)
    assert torch.equal(y[..., cfg.rope_dim:], x[..., cfg.rope_dim:])


def test_config_derivations():
    cfg = OracleConfig()
    assert cfg.conv_dim == 2 * 16 * 128 + 32 * 128 == 8192
    assert cfg.block_topk == 32
    assert [l for l in range(8) if cfg.is_full_attention(l)] == [3, 7]
