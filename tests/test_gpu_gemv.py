"""The small-M layer projections (qm_gemv) against an fp32 torch product.

Bar: bf16 outputs within 1e-2 of the fp32 product (max |got - want| / max |want|,
one bf16 rounding of the result is ~4e-3), f32 outputs within 1e-5; every
segment of the row split lands in its own tensor.
"""

from __future__ import annotations

import ctypes
import os
import sys

import pytest
import torch
import torch.nn.functional as F

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import inputs as gi  # noqa: E402

from margins import rel_err  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda"


def run_gemv(qm, w, x, rows):
    m, k = x.shape
    outs = [torch.empty(m, r, dtype=x.dtype, device=DEV) for r in rows]
    seg_rows = (ctypes.c_int * len(rows))(*rows)
    seg_out = (ctypes.c_void_p * len(rows))(*[o.data_ptr() for o in outs])
    qm.native.call("qm_gemv", qm.native.act_code(x.dtype), m, w.shape[0], k, w.data_ptr(), x.data_ptr(), len(rows),
                   seg_rows, seg_out, qm.native.stream_handle())
    torch.cuda.synchronize()
    return outs


@pytest.mark.parametrize("dtype,k", [(torch.bfloat16, 2048), (torch.bfloat16, 4096), (torch.float32, 1024),
                                     (torch.float32, 2048), (torch.float32, 4096)])
@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_gemv_matches_fp32_product(gpu, dtype, k, m):
    qm = gpu
    g = torch.Generator(device=DEV).manual_seed(m * 7 + k)
    # the DeltaNet input projections' row split, and a ragged split of an odd row count
    for rows in ([8192, 4096, 32, 32], [600, 1, 398]):
        n = sum(rows)
        print(f"gemv {dtype} m={m} k={k} rows={rows}", flush=True)
        w = (torch.randn(n, k, generator=g, device=DEV) * 0.02).to(dtype)
        x = torch.randn(m, k, generator=g, device=DEV).to(dtype)
        want = x.float() @ w.float().t()
        got = run_gemv(qm, w, x, rows)
        tol = 1e-2 if dtype == torch.bfloat16 else 1e-5
        start = 0
        for o, r in zip(got, rows):
            assert rel_err(o, want[:, start:start + r], tol) < tol, (rows, r)
            start += r


def test_layer_projections_take_the_gemv(gpu):
    """At one token the layer's projections run qm_gemv over the concatenated
    weights and equal F.linear with each weight; at 128 tokens they are the
    library GEMM on views of the same concatenation."""
    qm = gpu
    dtype = torch.bfloat16
    store = gi.FakeStore(gi.dn_weights(0, 31, dtype))
    model = qm.Qwen4MixModel(qm.MixConfig(), store, device=DEV, max_ctx=256)
    for seq in (1, 128):
        hidden = gi.normal(gi.rng(32 + seq), (1, seq, gi.HIDDEN)).to(dtype).to(DEV)
        got = model.project(hidden, 0, "dn_in")
        for t, name in zip(got, model.PROJ_GROUPS["dn_in"]):
            want = F.linear(hidden.float(), store.get(f"blk.0.{name}").to(DEV).float())
            assert rel_err(t, want, 1e-2) < 1e-2, (seq, name)


@pytest.mark.parametrize("dtype,k", [(torch.bfloat16, 4096), (torch.float32, 2048)])
@pytest.mark.parametrize("m,streams", [(1, 4), (3, 4), (2, 1), (1, 10)])
def test_gemv_reinject_equals_gemv_then_reinject(gpu, dtype, k, m, streams):
    """qm_gemv_reinject == qm_gemv + qm_hc_reinject, bit for bit (the same two
    roundings of each product and sum); past qm_hc_reinject's 8 streams, the
    same two roundings in torch."""
    qm = gpu
    n = 2048
    g = torch.Generator(device=DEV).manual_seed(31 * m + k + streams)
    print(f"gemv_reinject {dtype} m={m} k={k} streams={streams}", flush=True)
    w = (torch.randn(n, k, generator=g, device=DEV) * k ** -0.5).to(dtype)
    x = torch.randn(m, k, generator=g, device=DEV).to(dtype)
    hyper = torch.randn(m, streams * n, generator=g, device=DEV).to(dtype)
    inject = (2 * torch.sigmoid(torch.randn(m, streams, generator=g, device=DEV))).to(dtype)
    branch = run_gemv(qm, w, x, [n])[0]
    if streams <= 8:
        want = torch.empty_like(hyper)
        geom = qm.native.HcGeom(m, streams, n, 0, qm.native.act_code(dtype), 0.0)
        qm.native.call("qm_hc_reinject", ctypes.byref(geom), hyper.data_ptr(), branch.data_ptr(), inject.data_ptr(),
                       want.data_ptr(), qm.native.stream_handle())
    else:
        scaled = (branch.float()[:, None, :] * inject.float()[:, :, None]).to(dtype).float()
        want = (hyper.float().view(m, streams, n) + scaled).to(dtype).view(m, streams * n)
    got = hyper.clone()
    qm.native.call("qm_gemv_reinject", qm.native.act_code(dtype), m, n, k, w.data_ptr(), x.data_ptr(), streams,
                   inject.data_ptr(), got.data_ptr(), qm.native.stream_handle())
    torch.cuda.synchronize()
    assert torch.equal(got, want)
