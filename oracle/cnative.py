"""Loader of the oracle's C restatements (test infrastructure only).

``scores.c`` is compiled with gcc into ``oracle/_build/liboracle.so`` by
``__graft_entry__.build()``, or here on first use when the built file is
missing or older than its source.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
import threading

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
SOURCES = [os.path.join(HERE, "scores.c")]
LIB = os.path.join(HERE, "_build", "liboracle.so")
_lib = None
_lock = threading.Lock()


def build() -> str:
    os.makedirs(os.path.dirname(LIB), exist_ok=True)
    tmp = LIB + f".tmp{os.getpid()}"
    cmd = ["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-shared", "-fPIC", "-o", tmp, *SOURCES, "-lm"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"gcc failed on the oracle sources:\n{res.stderr[-4000:]}")
    os.replace(tmp, LIB)
    return LIB


def load() -> ctypes.CDLL:
    global _lib
    with _lock:
        if _lib is None:
            stale = not os.path.exists(LIB) or any(os.path.getmtime(s) > os.path.getmtime(LIB) for s in SOURCES)
            if stale:
                build()
            lib = ctypes.CDLL(LIB)
            lib.oracle_block_scores.restype = None
            lib.oracle_block_scores.argtypes = [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int] * 4 + [
                ctypes.c_void_p]
            _lib = lib
        return _lib


def block_scores(q: torch.Tensor, pooled: torch.Tensor) -> torch.Tensor:
    """q [B, S, H, 128], pooled [B, N, 128] -> float32 scores [B, S, N] in the
    reference's summation orders (scores.c)."""
    qn = np.ascontiguousarray(q.detach().float().cpu().numpy())
    kn = np.ascontiguousarray(pooled.detach().float().cpu().numpy())
    B, S, H, d = qn.shape
    N = kn.shape[1]
    if d != 128 or kn.shape[2] != 128 or kn.shape[0] != B:
        raise ValueError("oracle block scores: head dim 128 and matching batch expected")
    out = np.empty((B, S, N), np.float32)
    load().oracle_block_scores(qn.ctypes.data, kn.ctypes.data, B, S, H, N, out.ctypes.data)
    return torch.from_numpy(out)
