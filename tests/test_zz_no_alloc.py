"""The allocation-free DeltaNet prefill entry point (qm_dn_prefill_noalloc).

It has no counterpart in the reference: it is qm_dn_prefill with the library's
own per-device scratch array in place of the caller's workspace, for callers
that cannot allocate (graph capture, serving loops). Checked through the C ABI
against qm_dn_prefill on the same inputs and state, bit for bit (the same
kernels run on the same data), on two calls in a row whose second is smaller,
the state carried from one to the next; and the size guard (more than the
scratch holds is an error, before any launch).
"""

from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"
QM_ERR_UNSUPPORTED = -5


def _bind(lib, DnGeom):
    return lib.qm_dn_prefill_noalloc


def test_noalloc_rejects_chunks_beyond_its_scratch(qm):
    """Host-side guard: nothing is launched (no device needed)."""
    lib = qm.native.load()
    fn = _bind(lib, qm.native.DnGeom)
    g = qm.native.DnGeom(1, 32, 16, 128, 4, qm.native.QM_ACT_BF16, 1e-6)
    assert lib.qm_dn_prefill_workspace(ctypes.byref(g), 4096) > lib.qm_dn_prefill_noalloc_max_bytes()
    rc = fn(ctypes.byref(g), 4096, *([1] * 12), None)
    assert rc == QM_ERR_UNSUPPORTED
    assert b"scratch" in lib.qm_last_error()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_prefill_matches_workspace_entry(gpu, dtype):
    qm = gpu
    native = qm.native
    lib = native.load()
    fn = _bind(lib, native.DnGeom)
    B, Hv, Hk, D, K = 1, 32, 16, 128, 4
    conv_dim = (2 * Hk + Hv) * D
    g = native.DnGeom(B, Hv, Hk, D, K, native.act_code(dtype), 1e-6)
    gen = torch.Generator(device=DEV).manual_seed(1234)

    def rnd(*shape, scale=1.0, dt=dtype):
        return (torch.randn(*shape, generator=gen, device=DEV) * scale).to(dt)

    a_neg = -torch.rand(Hv, generator=gen, device=DEV) - 0.5
    dt_bias = rnd(Hv, dt=torch.float32)
    conv_w = rnd(conv_dim, K, scale=0.5)
    norm_w = 1.0 + rnd(D, scale=0.1, dt=torch.float32)
    ring0 = rnd(B, conv_dim, K)
    state0 = rnd(B, Hv, D, D, scale=0.02, dt=torch.float32)
    ring = [ring0.clone(), ring0.clone()]
    state = [state0.clone(), state0.clone()]
    pos = 1000
    for seq in (128, 40):                      # two calls in a row, the second smaller
        print(f"noalloc prefill {dtype} seq={seq} pos={pos}", flush=True)
        qkv, z = rnd(B, seq, conv_dim), rnd(B, seq, Hv * D)
        a, b = rnd(B, seq, Hv), rnd(B, seq, Hv)
        positions = torch.full((B,), pos, dtype=torch.int32, device=DEV)
        outs = [torch.full((B, seq, Hv * D), float("nan"), dtype=dtype, device=DEV) for _ in range(2)]
        ws = torch.empty(lib.qm_dn_prefill_workspace(ctypes.byref(g), seq), dtype=torch.uint8, device=DEV)
        stream = native.stream_handle()
        common = [qkv.data_ptr(), z.data_ptr(), a.data_ptr(), b.data_ptr(), a_neg.data_ptr(), dt_bias.data_ptr(),
                  conv_w.data_ptr(), norm_w.data_ptr(), positions.data_ptr()]
        native.call("qm_dn_prefill", ctypes.byref(g), seq, *common, ring[0].data_ptr(), state[0].data_ptr(),
                    outs[0].data_ptr(), ws.data_ptr(), ws.numel(), stream)
        rc = fn(ctypes.byref(g), seq, *common, ring[1].data_ptr(), state[1].data_ptr(), outs[1].data_ptr(), stream)
        assert rc == 0, lib.qm_last_error()
        torch.cuda.synchronize()
        assert torch.isfinite(outs[1].float()).all()
        assert torch.equal(outs[0], outs[1])
        assert torch.equal(ring[0], ring[1])
        assert torch.equal(state[0], state[1])
        pos += seq
