"""The C ABI library (CPU-side checks: no kernel is launched here).

* libqwen4mix.so loads and exports every function include/*.h declares, and
  the ctypes binding declares exactly those;
* host-side helpers that need no GPU: the V-page slot permutation is a bijection
  of each 32-row group, the argument checks reject bad geometry before any
  launch, the package's rope tables are bit-identical to the reference's.
"""

from __future__ import annotations

import ctypes
import glob
import json
import os
import re
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(qm_\w+)\s*\(", text))
    return names


def test_library_exports_every_declared_symbol(qm):
    lib = qm.native.load()
    declared = _declared()
    assert declared, "no declarations found"
    for name in sorted(declared):
        assert hasattr(lib, name), f"{name} not exported"
    assert declared == set(qm.native.SIGNATURES), "binding and header disagree"
    assert lib.qm_version() >= 1


def test_binding_argument_counts_match_the_header(qm):
    """Each ctypes argtypes list has as many entries as the C declaration has
    parameters (a miscounted list would shift every later argument)."""
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        for name, params in re.findall(r"\b(qm_\w+)\s*\(([^)]*)\)\s*;", text):
            params = params.strip()
            n = 0 if params in ("", "void") else params.count(",") + 1
            assert len(qm.native.SIGNATURES[name][1]) == n, f"{name}: header {n}, binding differs"


def test_v_slot_is_a_permutation_of_each_group(qm):
    lib = qm.native.load()
    for page in (32, 64, 128):
        cols = [lib.qm_v_slot(r) for r in range(page)]
        assert sorted(cols) == list(range(page))
        assert all(c // 32 == r // 32 for r, c in enumerate(cols))


def test_page_index_is_a_permutation_in_lane_order(qm):
    """Each pool page is a permutation of its [P, d] rows, and every 1 KB tile
    holds one MFMA operand: K tiles 16 tokens x 32 channels, V tiles 32 tokens
    x 16 channels (lane order checked against the operand layout)."""
    import numpy as np
    lib = qm.native.load()
    P, d = 64, 256
    k = (ctypes.c_int * (P * d))()
    v = (ctypes.c_int * (P * d))()
    assert lib.qm_qsa_page_index(P, d, k, v) == 0
    k = np.array(k).reshape(P, d)
    v = np.array(v).reshape(P, d)
    for idx in (k, v):
        assert sorted(idx.ravel().tolist()) == list(range(P * d))
    r, c = np.meshgrid(np.arange(P), np.arange(d), indexing="ij")
    # K: tile (r // 16, c // 32); lane = r % 16 + 16 * ((c % 32) // 8); element c % 8
    assert np.array_equal(k // 512, (r // 16) * 8 + c // 32)
    assert np.array_equal((k % 512) // 8, r % 16 + 16 * ((c % 32) // 8))
    assert np.array_equal(k % 8, c % 8)
    # V: tile (r // 32, c // 16); lane = c % 16 + 16 * (slot // 8); element slot % 8
    slot = np.array([lib.qm_v_slot(int(x)) % 32 for x in range(P)])[r]
    assert np.array_equal(v // 512, (r // 32) * 16 + c // 16)
    assert np.array_equal((v % 512) // 8, c % 16 + 16 * (slot // 8))
    assert np.array_equal(v % 8, slot % 8)
    assert lib.qm_qsa_page_index(48, d, (ctypes.c_int * (48 * d))(), (ctypes.c_int * (48 * d))()) == -1


def test_bad_geometry_is_rejected_without_a_launch(qm):
    n = qm.native
    lib = n.load()
    g = n.DnGeom(1, 32, 16, 64, 4, n.QM_ACT_BF16, 1e-6)       # head_dim 64 unsupported
    rc = lib.qm_dn_decode(ctypes.byref(g), *([None] * 12), None, 0, None)
    assert rc == -5 and b"head_dim" in lib.qm_last_error()
    g = n.DnGeom(1, 32, 16, 128, 4, 7, 1e-6)                  # unknown dtype
    rc = lib.qm_dn_decode(ctypes.byref(g), *([ctypes.c_void_p(8)] * 12), ctypes.c_void_p(8), 1 << 20, None)
    assert rc in (-2, -4)
    q = n.QsaGeom(1, 16, 2, 128, 64, 4, 128, 64, 2048, 64, 4, 256, 4, n.QM_ACT_BF16, 1e-6)
    assert lib.qm_qsa_select(ctypes.byref(q), 1, *([None] * 8), None) == -5
    with pytest.raises(n.QmError, match="head_dim"):
        n.call("qm_qsa_select", ctypes.byref(q), 1, *([None] * 8), None)


def test_gemv_rejects_unsupported_shapes_before_a_launch(qm):
    """qm_gemv checks its sizes on the host: m above 4, k outside the tiled
    widths, segments that do not add up, and null outputs are errors."""
    lib = qm.native.load()
    rows = (ctypes.c_int * 2)(3, 5)
    outs = (ctypes.c_void_p * 2)(16, 32)
    dummy = ctypes.c_void_p(64)
    bf16 = qm.native.QM_ACT_BF16
    assert lib.qm_gemv(bf16, 5, 8, 2048, dummy, dummy, 2, rows, outs, None) < 0      # m > 4
    assert lib.qm_gemv(bf16, 1, 8, 1024, dummy, dummy, 2, rows, outs, None) < 0      # k not 2048/4096 for bf16
    assert lib.qm_gemv(bf16, 1, 9, 2048, dummy, dummy, 2, rows, outs, None) < 0      # 3 + 5 != 9
    bad = (ctypes.c_void_p * 2)(16, None)
    assert lib.qm_gemv(bf16, 1, 8, 2048, dummy, dummy, 2, rows, bad, None) < 0       # null output
    assert b"qm_gemv" in lib.qm_last_error()


def test_workspace_sizes_are_sane(qm):
    n = qm.native
    lib = n.load()
    assert lib.qm_dn_decode_workspace(1, 32, 128) > 0 and lib.qm_dn_decode_workspace(0, 32, 128) == 0
    q = n.QsaGeom(1, 16, 2, 256, 64, 4, 128, 64, 2048, 64, 128, 8192, 128, n.QM_ACT_BF16, 1e-6)
    splits = lib.qm_qsa_attend_splits(ctypes.byref(q), 8128, 8128)
    assert splits == (32 * 2 + 1 + 1) // 2          # 64 block groups + 1 tail group, 2 per workgroup
    assert lib.qm_qsa_attend_workspace(ctypes.byref(q), 1, splits) >= splits * 2 * 8 * 256 * 4
    assert lib.qm_qsa_items_stride(ctypes.byref(q)) == 1 + 64 + 3


def test_rope_tables_bit_identical_to_reference(qm):
    meta = json.load(open(os.path.join(ROOT, "tests", "golden", "golden_meta.json")))
    if meta["torch"] != torch.__version__ or meta["cpu_capability"] != torch.backends.cpu.get_cpu_capability():
        pytest.skip("different torch build than the golden generator")
    from importlib import import_module
    rope = import_module(qm.__name__ + ".rope")
    sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
    import inputs as gi
    cos, sin = rope.rope_tables_cpu(32768, 64, 1e7, [11, 11, 10])
    assert gi.digest(cos) == meta["digests"]["rope"]["cos_sha"]
    assert gi.digest(sin) == meta["digests"]["rope"]["sin_sha"]


def test_decode_group_guard(qm):
    """qm_qsa_decode's workgroups of one (sequence, kv head) group wait for one
    another, so a group must fit the device's resident capacity: the guard is
    pure host arithmetic (no launch), checked here at the sizes that matter --
    66 items at pos 8128, 514 at top-k 256 of 64-token blocks against a device
    of 256 compute units holding two workgroups each."""
    lib = qm.native.load()
    UNSUPPORTED, ARG = -5, -1
    assert lib.qm_qsa_decode_group(7) == 64 and lib.qm_qsa_decode_group(66) == 66
    assert lib.qm_qsa_decode_fits(66, 512) == 0
    assert lib.qm_qsa_decode_fits(512, 512) == 0
    assert lib.qm_qsa_decode_fits(514, 512) == UNSUPPORTED
    assert b"resident" in lib.qm_last_error()
    assert lib.qm_qsa_decode_fits(7, 63) == UNSUPPORTED      # widened to 64 slice holders
    assert lib.qm_qsa_decode_fits(0, 512) == ARG
    assert lib.qm_qsa_decode_fits(1025, 4096) == ARG


def test_causal_conv1d_rejects_bad_arguments_before_launch(qm):
    lib = qm.native.load()
    assert lib.qm_causal_conv1d(1, 1, 8, 4, 9, None, None, None, 1, None, None, None) == -1   # taps > 8
    assert lib.qm_causal_conv1d(1, 1, 8, 4, 4, None, None, None, 1, None, None, None) == -1   # null x
    assert lib.qm_causal_conv1d(7, 1, 8, 0, 4, None, None, 1, 1, None, None, None) == -2      # dtype


def test_noalloc_prefill_refuses_chunks_beyond_its_scratch(qm):
    """qm_dn_prefill_noalloc's size guard is host arithmetic: nothing launches."""
    lib = qm.native.load()
    g = qm.native.DnGeom(1, 32, 16, 128, 4, qm.native.QM_ACT_BF16, 1e-6)
    assert lib.qm_dn_prefill_noalloc_max_bytes() == 32 << 20
    assert lib.qm_dn_prefill_workspace(ctypes.byref(g), 128) <= lib.qm_dn_prefill_noalloc_max_bytes()
    rc = lib.qm_dn_prefill_noalloc(ctypes.byref(g), 4096, *([1] * 12), None)
    assert rc == -5 and b"scratch" in lib.qm_last_error()
