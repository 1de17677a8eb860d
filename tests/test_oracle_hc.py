"""The oracle's hyper-connection mix and reinjection (reference/model.py:53-81),
pinned by closed forms on structured inputs. CPU only.

rms_norm computes in float32 whatever the input dtype (as the reference's
does), so the closed forms hold to float32 precision. The inputs are built so
that each plausible mistake changes the answer by far more than that:
streams of different magnitudes and signs (a norm over the whole row instead of
per stream), hc_count = 3 (a missing or misplaced division by hc_count, a sum
instead of a mean), up and inject rows that differ from row to row (a stream
or position read from the wrong row, an interleaved instead of a stream-major
layout), a norm weight that varies by element, and silu / sigmoid / 2 sigmoid
applied at their own points.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle.config import OracleConfig
from oracle.layers import rms_norm
from oracle.mixing import OracleMixer
from tests.golden.inputs import FakeStore

HC, H, RANK, EPS = 3, 8, 4, 1e-6
U = [1.0, 1.0, 1.0, -1.0, 1.0, 1.0, 1.0, -1.0]      # mean(u^2) = 1, sum(u) = 4
AMP = [3.0, -0.5, 2.0]                               # stream s of hyper is AMP[s] * U


def _sigmoid(x):
    return 1.0 / (1.0 + math.exp(-x))


def _silu(x):
    return x * _sigmoid(x)


def _mixer(layer):
    cfg = OracleConfig(hidden_size=H, hc_count=HC, hc_lowrank=RANK, rms_norm_eps=EPS)
    prefix = "output_hc" if layer is None else f"blk.{layer}.hc_attn"
    K = HC * H
    norm_w = torch.tensor([1.0 + 0.1 * k for k in range(K)], dtype=torch.float64)
    down = torch.full((RANK, K), 0.05, dtype=torch.float64)
    up_scale = [0.3 - 0.02 * i for i in range(K)]   # row i of up is constant up_scale[i]
    up = torch.tensor(up_scale, dtype=torch.float64)[:, None].expand(K, RANK).contiguous()
    inj_scale = [0.2, -0.1, 0.05]                      # row s of inject is constant inj_scale[s]
    inject = torch.tensor(inj_scale, dtype=torch.float64)[:, None].expand(HC, K).contiguous()
    w = {prefix + "_norm.weight": norm_w, prefix + "_down.weight": down, prefix + "_up.weight": up}
    if layer is not None:
        w[prefix + "_inject.weight"] = inject
    return OracleMixer(cfg, FakeStore(w)), norm_w.tolist(), up_scale, inj_scale


def _hyper():
    return torch.tensor([[a * u for a in AMP for u in U]], dtype=torch.float64)


def _closed_form(norm_w, up_scale, inj_scale):
    # stream s normalises to sign(a_s) * |a_s| / sqrt(a_s^2 + eps) * u * w
    r = [a / math.sqrt(a * a + EPS) for a in AMP]
    normed = [r[s] * U[h] * norm_w[s * H + h] for s in range(HC) for h in range(H)]
    total = sum(normed)
    low = _silu(0.05 * total / HC)                       # every down row is 0.05 everywhere
    gate = [_sigmoid(up_scale[i] * RANK * low) for i in range(HC * H)]
    mixed = [sum(gate[s * H + h] * normed[s * H + h] for s in range(HC)) / HC for h in range(H)]
    inject = [2.0 * _sigmoid(inj_scale[s] * total / HC) for s in range(HC)]
    return normed, mixed, inject


def test_grouped_rms_norm_normalises_each_stream_alone():
    x = _hyper()
    w = torch.ones(HC * H, dtype=torch.float64)
    out = rms_norm(x, w, EPS, group_size=H)[0].tolist()
    for s in range(HC):
        scale = AMP[s] / math.sqrt(AMP[s] ** 2 + EPS)
        for h in range(H):
            assert out[s * H + h] == pytest.approx(scale * U[h], rel=1e-6)
    # a norm over the whole row would give a different answer for these streams
    whole = rms_norm(x, w, EPS)[0].tolist()
    assert abs(whole[0] - out[0]) > 0.1


def test_gated_residual_closed_form():
    mixer, norm_w, up_scale, inj_scale = _mixer(layer=2)
    hyper = _hyper()
    mixed, hyper_out, inject = mixer._gated_residual(hyper, 2, "attn")
    _, want_mixed, want_inject = _closed_form(norm_w, up_scale, inj_scale)
    assert hyper_out is hyper
    assert mixed.shape == (1, H) and inject.shape == (1, HC)
    assert mixed[0].tolist() == pytest.approx(want_mixed, rel=1e-5, abs=1e-7)
    assert inject[0].tolist() == pytest.approx(want_inject, rel=1e-6)


def test_final_mixer_has_no_injection():
    mixer, norm_w, up_scale, inj_scale = _mixer(layer=None)
    mixed, _, inject = mixer._gated_residual(_hyper(), None, "")
    _, want_mixed, _ = _closed_form(norm_w, up_scale, inj_scale)
    assert inject is None
    assert mixed[0].tolist() == pytest.approx(want_mixed, rel=1e-5, abs=1e-7)


def test_reinject_adds_the_branch_to_each_stream_by_its_weight():
    hyper = _hyper()
    branch = torch.tensor([[0.5 * h - 1.0 for h in range(H)]], dtype=torch.float64)
    inject = torch.tensor([[1.0, 2.0, -3.0]], dtype=torch.float64)
    out = OracleMixer._reinject(hyper, branch, inject)[0].tolist()
    for s in range(HC):
        for h in range(H):
            want = AMP[s] * U[h] + inject[0, s].item() * branch[0, h].item()
            assert out[s * H + h] == pytest.approx(want, rel=1e-14)


def test_zero_weights_give_half_the_stream_mean_and_unit_injection():
    # down = 0 -> silu(0) = 0 -> up gate sigmoid(0) = 1/2; inject = 2 sigmoid(0) = 1
    cfg = OracleConfig(hidden_size=H, hc_count=HC, hc_lowrank=RANK, rms_norm_eps=EPS)
    K = HC * H
    p = "blk.0.hc_ffn"
    w = {p + "_norm.weight": torch.ones(K, dtype=torch.float64),
         p + "_down.weight": torch.zeros(RANK, K, dtype=torch.float64),
         p + "_up.weight": torch.randn(K, RANK, dtype=torch.float64),
         p + "_inject.weight": torch.zeros(HC, K, dtype=torch.float64)}
    mixer = OracleMixer(cfg, FakeStore(w))
    torch.manual_seed(0)
    hyper = torch.randn(2, 5, K, dtype=torch.float64)
    mixed, _, inject = mixer._gated_residual(hyper, 0, "ffn")
    normed = rms_norm(hyper, w[p + "_norm.weight"], EPS, group_size=H)
    want = 0.5 * normed.unflatten(-1, (HC, H)).mean(-2)
    assert torch.allclose(mixed, want, rtol=1e-12, atol=1e-14)
    assert torch.equal(inject, torch.ones(2, 5, HC, dtype=torch.float64))
