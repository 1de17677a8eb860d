"""The hyper-connection mix and reinjection (qm_hc_mix, qm_hc_reinject) against
the oracle's _gated_residual / _reinject (reference/model.py:53-81).

Bar: bf16 outputs within 2e-2 (max |got - want| / max |want|) of the oracle run
in bf16 on the CPU, float32 outputs within 1e-4 (the sums run in another
order); reinjection bit-exact (one rounding of each product and sum, as the
reference). Cases: 1 to 6 token rows (one and two row groups), the layer mixers
and the final mixer, streams of 2048 and of 2560, reinjection in place.
"""

from __future__ import annotations

import ctypes
import os
import sys

import pytest
import torch

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import inputs as gi  # noqa: E402

from oracle.config import OracleConfig  # noqa: E402
from oracle.mixing import OracleMixer  # noqa: E402

from margins import rel_err  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda"


def tol(dtype):
    return 2e-2 if dtype == torch.bfloat16 else 1e-4


def _pair(qm, hidden, layer, dtype, seed):
    prefix = "output_hc" if layer is None else f"blk.{layer}.hc_attn"
    w = gi.hc_weights(prefix, seed, dtype, hidden=hidden, with_inject=layer is not None)
    store = gi.FakeStore(w)
    cfg = qm.config.MixConfig(hidden_size=hidden)
    model = qm.model.Qwen4MixModel(cfg, store, device=DEV)
    oracle = OracleMixer(OracleConfig(hidden_size=hidden), store)
    return model, oracle


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("hidden,rows", [(2048, 1), (2048, 2), (2048, 3), (2048, 4), (2048, 6), (2560, 1), (2560, 3)])
def test_gated_residual_matches_oracle(gpu, dtype, hidden, rows):
    qm = gpu
    for layer in (5, None):
        print(f"hc mix {dtype} hidden={hidden} rows={rows} layer={layer}", flush=True)
        model, oracle = _pair(qm, hidden, layer, dtype, seed=hidden + rows)
        hyper = gi.normal(gi.rng(rows), (1, rows, 4 * hidden), 1.0).to(dtype)
        want_mixed, _, want_inject = oracle._gated_residual(hyper, layer, "attn")
        mixed, hyper_out, inject = model._gated_residual(hyper.to(DEV), layer, "attn")
        torch.cuda.synchronize()
        assert mixed.shape == want_mixed.shape and mixed.dtype == dtype
        assert rel_err(mixed, want_mixed, tol(dtype)) < tol(dtype)
        if layer is None:
            assert inject is None
        else:
            assert inject.shape == want_inject.shape
            assert rel_err(inject, want_inject, tol(dtype)) < tol(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rows", [1, 5])
def test_reinject_matches_oracle(gpu, dtype, rows):
    qm = gpu
    print(f"hc reinject {dtype} rows={rows}", flush=True)
    r = gi.rng(40 + rows)
    hyper = gi.normal(r, (1, rows, 4 * 2048)).to(dtype)
    branch = gi.normal(r, (1, rows, 2048)).to(dtype)
    inject = (2 * torch.sigmoid(gi.normal(r, (1, rows, 4)))).to(dtype)
    want = OracleMixer._reinject(hyper, branch, inject)
    Model = qm.model.Qwen4MixModel
    got = Model._reinject(hyper.to(DEV), branch.to(DEV), inject.to(DEV))
    h_dev = hyper.to(DEV)
    same = Model._reinject(h_dev, branch.to(DEV), inject.to(DEV), out=h_dev)
    torch.cuda.synchronize()
    assert same.data_ptr() == h_dev.data_ptr()
    # the same two roundings as the reference, so the same bits
    assert torch.equal(got.cpu(), want)
    assert torch.equal(same.cpu(), want)


def test_hc_rejects_unsupported_shapes_before_a_launch(gpu):
    qm = gpu
    lib = qm.native.load()
    g = qm.native.HcGeom(1, 4, 2048, 320, qm.native.QM_ACT_BF16, 1e-6)
    assert lib.qm_hc_mix_workspace(ctypes.byref(g)) > 0
    for bad in (qm.native.HcGeom(1, 4, 2000, 320, 1, 1e-6),     # streams * hidden not a multiple of 2048
                qm.native.HcGeom(1, 9, 2048, 320, 1, 1e-6),     # more than 8 streams
                qm.native.HcGeom(1, 4, 2048, 1024, 1, 1e-6)):   # rank above 512
        assert lib.qm_hc_mix_workspace(ctypes.byref(bad)) == 0
        with pytest.raises(qm.native.QmError):
            qm.native.call("qm_hc_mix", ctypes.byref(bad), 16, 16, 16, 1, 16, 16, 16, 16, 1 << 20, None)
