"""The parity margins the GPU tests achieve.

Every comparison a GPU test makes through ``rel_err`` / ``abs_err`` /
``max_ulps`` records the error it found (and the bar it is held to, where the
call names it) under the running test's id; ``tests/conftest.py`` prints the
worst value per test and kind in pytest's terminal summary, so a shrinking
margin is visible before a test trips.

* ``rel_err``: max |got - want| / max |want| (the bf16/fp32 output bar);
* ``abs_err``: max |got - want| (the fp32 state bar);
* ``max_ulps``: the largest distance in units in the last place between two
  float32 tensors (0 for the bit-exact score pins).
"""

from __future__ import annotations

import os

RECORDS: list = []


def _test_id() -> str:
    return os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0]


def record(kind: str, value: float, bar=None) -> float:
    RECORDS.append((_test_id(), kind, float(value), bar))
    return value


def rel_err(got, want, bar=None) -> float:
    got, want = got.detach().float().cpu(), want.detach().float().cpu()
    v = ((got - want).abs().max() / want.abs().max().clamp_min(1e-30)).item()
    return record("rel", v, bar)


def abs_err(got, want, bar=None) -> float:
    v = (got.detach().float().cpu() - want.detach().float().cpu()).abs().max().item()
    return record("abs", v, bar)


def max_ulps(got, want) -> int:
    """Largest ulp distance between two float32 tensors of finite values."""
    import torch
    a = got.detach().float().cpu().contiguous().view(torch.int32).long()
    b = want.detach().float().cpu().contiguous().view(torch.int32).long()
    # map the sign-magnitude bit patterns onto one monotone integer line
    a = torch.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = torch.where(b < 0, -(b & 0x7FFFFFFF), b)
    v = int((a - b).abs().max().item()) if a.numel() else 0
    record("ulps", v, 0)
    return v


def summary() -> list:
    """[(test, kind, worst value, bar)], worst = largest value per (test, kind)."""
    worst: dict = {}
    for test, kind, v, bar in RECORDS:
        key = (test, kind)
        prev = worst.get(key)
        if prev is None or v > prev[0]:
            worst[key] = (v, bar if bar is not None else (prev[1] if prev else None))
        elif bar is not None and prev[1] is None:
            worst[key] = (prev[0], bar)
    return [(t, k, v, b) for (t, k), (v, b) in worst.items()]
