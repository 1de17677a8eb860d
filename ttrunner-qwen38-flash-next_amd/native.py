"""ctypes binding of libqwen4mix.so (declared in include/qwen4mix.h).

There is one code path: if the library is missing or a call fails, this module
raises. Nothing here computes anything itself.
"""

from __future__ import annotations

import ctypes
import os
import threading

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libqwen4mix.so")

QM_ACT_F32 = 0
QM_ACT_BF16 = 1

_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_sz = ctypes.c_size_t


class QmError(RuntimeError):
    """A qwen4mix entry point returned an error code."""


class DnGeom(ctypes.Structure):
    _fields_ = [("batch", _i), ("n_v_heads", _i), ("n_k_heads", _i), ("head_dim", _i),
                ("conv_kernel", _i), ("act_dtype", _i), ("eps", _f)]


class QsaGeom(ctypes.Structure):
    _fields_ = [("batch", _i), ("n_heads", _i), ("n_kv_heads", _i), ("head_dim", _i), ("rope_dim", _i),
                ("idx_heads", _i), ("idx_dim", _i), ("ratio", _i), ("budget", _i), ("page_size", _i),
                ("max_pages", _i), ("max_ctx", _i), ("max_blocks", _i), ("act_dtype", _i), ("eps", _f)]


class HcGeom(ctypes.Structure):
    _fields_ = [("rows", _i), ("streams", _i), ("hidden", _i), ("rank", _i), ("act_dtype", _i), ("eps", _f)]


# name -> (restype, argtypes); every symbol include/qwen4mix.h declares
SIGNATURES = {
    "qm_last_error": (ctypes.c_char_p, []),
    "qm_version": (_i, []),
    "qm_dn_decode_workspace": (_sz, [_i, _i, _i]),
    "qm_dn_decode": (_i, [ctypes.POINTER(DnGeom), _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                          _vp, _sz, _vp]),
    "qm_dn_decode_check": (_i, [_i, _i, _i, _vp, _sz, _i, _vp, _vp]),
    "qm_causal_conv1d": (_i, [_i, _i, _i, _i, _i, _vp, _vp, _vp, _i, _vp, _vp, _vp]),
    "qm_dn_recurrent": (_i, [_i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "qm_dn_chunked_workspace": (_sz, [_i, _i, _i, _i]),
    "qm_dn_chunked": (_i, [_i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "qm_v_slot": (_i, [_i]),
    "qm_qsa_page_index": (_i, [_i, _i, _vp, _vp]),
    "qm_qsa_prep": (_i, [ctypes.POINTER(QsaGeom), _i] + [_vp] * 19 + [_vp]),
    "qm_qsa_items_stride": (_i, [ctypes.POINTER(QsaGeom)]),
    "qm_qsa_decode_splits": (_i, [ctypes.POINTER(QsaGeom), _i]),
    "qm_qsa_decode_workspace": (_sz, [ctypes.POINTER(QsaGeom), _i]),
    "qm_qsa_decode_group": (_i, [_i]),
    "qm_qsa_decode_resident": (_i, [_i, _i]),
    "qm_qsa_decode_fits": (_i, [_i, _i]),
    "qm_qsa_decode_check": (_i, [ctypes.POINTER(QsaGeom), _i, _vp, _sz, _i, _vp, _vp]),
    "qm_qsa_decode": (_i, [ctypes.POINTER(QsaGeom)] + [_vp] * 18 + [_i, _vp, _sz, _vp, _vp, _vp, _vp, _vp]),
    "qm_qsa_decode_front": (_i, [ctypes.POINTER(QsaGeom)] + [_vp] * 22 + [_vp]),
    "qm_qsa_select": (_i, [ctypes.POINTER(QsaGeom), _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "qm_qsa_attend_workspace": (_sz, [ctypes.POINTER(QsaGeom), _i, _i]),
    "qm_qsa_attend_splits": (_i, [ctypes.POINTER(QsaGeom), _i, _i]),
    "qm_qsa_attend": (_i, [ctypes.POINTER(QsaGeom), _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp, _sz, _vp]),
    "qm_qsa_attend_chunk_workspace": (_sz, [ctypes.POINTER(QsaGeom), _i]),
    "qm_qsa_attend_chunk": (_i, [ctypes.POINTER(QsaGeom), _i] + [_vp] * 9 + [_vp, _sz, _vp]),
    "qm_qsa_select_chunk": (_i, [ctypes.POINTER(QsaGeom), _i] + [_vp] * 5 + [_vp, _sz, _vp]),
    "qm_qsa_attend_chunk_filed": (_i, [ctypes.POINTER(QsaGeom), _i] + [_vp] * 7 + [_vp, _sz, _vp]),
    "qm_qsa_pool_blocks": (_i, [ctypes.POINTER(QsaGeom), _vp, _vp, _vp, _vp, _i, _i, _vp, _vp]),
    "qm_gemv": (_i, [_i, _i, _i, _i, _vp, _vp, _i, _vp, _vp, _vp]),
    "qm_gemv_reinject": (_i, [_i, _i, _i, _i, _vp, _vp, _i, _vp, _vp, _vp]),
    "qm_dn_prefill_workspace": (_sz, [ctypes.POINTER(DnGeom), _i]),
    "qm_dn_prefill": (_i, [ctypes.POINTER(DnGeom), _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                           _vp, _vp, _sz, _vp]),
    "qm_dn_prefill_noalloc": (_i, [ctypes.POINTER(DnGeom), _i] + [_vp] * 12 + [_vp]),
    "qm_dn_prefill_noalloc_max_bytes": (_sz, []),
    "qm_hc_mix_workspace": (_sz, [ctypes.POINTER(HcGeom)]),
    "qm_hc_mix": (_i, [ctypes.POINTER(HcGeom), _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _sz, _vp]),
    "qm_hc_reinject": (_i, [ctypes.POINTER(HcGeom), _vp, _vp, _vp, _vp, _vp]),
}

_lib = None
_lock = threading.Lock()


def load(path: str | None = None) -> ctypes.CDLL:
    """Load the library (once) and bind every entry point; raise if absent.
    The path defaults to QM_LIB from the environment, else the in-tree build."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = path or os.environ.get("QM_LIB") or LIB_PATH
        if not os.path.exists(path):
            raise QmError(f"{path} is missing: build it with __graft_entry__.build() "
                          "(there is no fallback implementation)")
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def call(name: str, *args) -> int:
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.qm_last_error().decode(errors="replace")
        raise QmError(f"{name} failed ({rc}): {msg}")
    return rc


def ptr(t) -> int | None:
    """Device pointer of a tensor (None for None)."""
    return None if t is None else t.data_ptr()


def stream_handle(device=None) -> int:
    import torch
    return torch.cuda.current_stream(device).cuda_stream


def act_code(dtype) -> int:
    import torch
    if dtype == torch.float32:
        return QM_ACT_F32
    if dtype == torch.bfloat16:
        return QM_ACT_BF16
    raise QmError(f"unsupported activation dtype {dtype}; use float32 or bfloat16")


def dn_decode_faults(batch: int, n_v_heads: int, head_dim: int, ws, reset: bool, name: str, device=None) -> list:
    """Messages for the give-ups qm_dn_decode_check finds in a decode workspace."""
    n = ctypes.c_uint(0)
    call("qm_dn_decode_check", batch, n_v_heads, head_dim, ws.data_ptr(), ws.numel(), int(reset), ctypes.byref(n),
         stream_handle(device))
    return [f"{name}: {n.value} DeltaNet decode waits gave up"] if n.value else []


def qsa_decode_faults(geom, splits: int, ws, reset: bool, name: str, device=None) -> list:
    """Messages for the give-ups and overflows qm_qsa_decode_check finds."""
    counts = (ctypes.c_uint * 2)()
    call("qm_qsa_decode_check", ctypes.byref(geom), splits, ws.data_ptr(), ws.numel(), int(reset), counts,
         stream_handle(device))
    out = []
    if counts[0]:
        out.append(f"{name}: {counts[0]} QSA decode waits gave up")
    if counts[1]:
        out.append(f"{name}: {counts[1]} QSA decode launches had more attention items than their {splits} splits")
    return out
