"""Deterministic synthetic inputs for the token-mixing configurations.

Shared by tests/golden/make_golden.py (which feeds them to the reference) and
by the tests (which feed them to the oracle and the HIP path). Everything is
drawn from numpy's PCG64 with a fixed seed, in float32, and converted to torch
(then rounded to bfloat16 where the configuration says bf16), so every machine
rebuilds identical bits.

Weights follow the survey's recipe: N(0, fan_in^-1/2) for projections, norm
weights 1, ``ssm_a = -1`` and ``ssm_dt.bias = 0`` (so g = -softplus(a)).
"""

from __future__ import annotations

import hashlib

import numpy as np
import torch

HIDDEN = 2048
QSA_HEADS, QSA_KV, QSA_HD = 16, 2, 256
IDX_HEADS, IDX_DIM = 4, 128
DN_HK, DN_HV, DN_D, DN_K = 16, 32, 128, 4
CONV_DIM = 2 * DN_HK * DN_D + DN_HV * DN_D
RATIO, BUDGET = 64, 2048


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def normal(r: np.random.Generator, shape, scale: float = 1.0, dtype=torch.float32) -> torch.Tensor:
    x = r.standard_normal(size=shape, dtype=np.float32)
    if scale != 1.0:
        x = x * np.float32(scale)
    return torch.from_numpy(x).to(dtype)


def digest(t: torch.Tensor) -> str:
    t = t.detach().contiguous().cpu()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    return hashlib.sha256(t.numpy().tobytes()).hexdigest()


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().to(torch.bfloat16).view(torch.int16).numpy()


def from_bf16_bits(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


class FakeStore:
    """``get("blk.{layer}.{suffix}")`` over a dict, like reference/weights.py:74."""

    def __init__(self, weights: dict):
        self.weights = weights

    def get(self, name: str) -> torch.Tensor:
        return self.weights[name]


def dn_weights(layer: int, seed: int, dtype=torch.float32, hidden: int = HIDDEN) -> dict:
    r = rng(seed)
    p = f"blk.{layer}."
    s = hidden ** -0.5
    return {
        p + "attn_qkv.weight": normal(r, (CONV_DIM, hidden), s, dtype),
        p + "attn_gate.weight": normal(r, (DN_HV * DN_D, hidden), s, dtype),
        p + "ssm_beta.weight": normal(r, (DN_HV, hidden), s, dtype),
        p + "ssm_alpha.weight": normal(r, (DN_HV, hidden), s, dtype),
        p + "ssm_conv1d.weight": normal(r, (CONV_DIM, DN_K), 0.5, dtype),
        p + "ssm_a": torch.full((DN_HV,), -1.0, dtype=torch.float32),
        p + "ssm_dt.bias": torch.zeros(DN_HV, dtype=torch.float32),
        p + "ssm_norm.weight": torch.ones(DN_D, dtype=torch.float32),
        p + "ssm_out.weight": normal(r, (hidden, DN_HV * DN_D), (DN_HV * DN_D) ** -0.5, dtype),
    }


def qsa_weights(layer: int, seed: int, dtype=torch.float32, hidden: int = HIDDEN) -> dict:
    r = rng(seed)
    p = f"blk.{layer}."
    s = hidden ** -0.5
    return {
        p + "attn_q.weight": normal(r, (QSA_HEADS * QSA_HD * 2, hidden), s, dtype),
        p + "attn_k.weight": normal(r, (QSA_KV * QSA_HD, hidden), s, dtype),
        p + "attn_v.weight": normal(r, (QSA_KV * QSA_HD, hidden), s, dtype),
        p + "attn_q_norm.weight": torch.ones(QSA_HD, dtype=torch.float32),
        p + "attn_k_norm.weight": torch.ones(QSA_HD, dtype=torch.float32),
        p + "attn_output.weight": normal(r, (hidden, QSA_HEADS * QSA_HD), (QSA_HEADS * QSA_HD) ** -0.5, dtype),
        p + "indexer.q_proj.weight": normal(r, (IDX_HEADS * IDX_DIM, hidden), s, dtype),
        p + "indexer.k_proj.weight": normal(r, (IDX_DIM, hidden), s, dtype),
        p + "indexer.q_norm.weight": torch.ones(IDX_DIM, dtype=torch.float32),
        p + "indexer.k_norm.weight": torch.ones(IDX_DIM, dtype=torch.float32),
    }


def hc_weights(prefix: str, seed: int, dtype=torch.float32, hidden: int = HIDDEN, streams: int = 4,
               rank: int = 320, with_inject: bool = True) -> dict:
    """One hyper-connection mixer (``blk.{l}.hc_{kind}`` or ``output_hc``):
    norm weight 1 + N(0, 0.1), projections N(0, fan_in^-1/2)."""
    r = rng(seed)
    k = streams * hidden
    w = {
        prefix + "_norm.weight": 1.0 + normal(r, (k,), 0.1),
        prefix + "_down.weight": normal(r, (rank, k), k ** -0.5, dtype),
        prefix + "_up.weight": normal(r, (k, rank), rank ** -0.5, dtype),
    }
    if with_inject:
        w[prefix + "_inject.weight"] = normal(r, (streams, k), k ** -0.5, dtype)
    return w


def qsa_past(seed: int, past: int, dtype=torch.float32):
    """Past K (bf16-valued, float32 as the reference's roped keys are), V and raw
    indexer keys for ``past`` tokens, batch 1."""
    r = rng(seed)
    keys = normal(r, (1, QSA_KV, past, QSA_HD)).to(torch.bfloat16).float()
    values = normal(r, (1, QSA_KV, past, QSA_HD)).to(torch.bfloat16).to(dtype)
    idx_keys = normal(r, (1, past, IDX_DIM)).to(torch.bfloat16).to(dtype)
    return keys, values, idx_keys


def dn_past(seed: int, dtype=torch.float32):
    r = rng(seed)
    conv = normal(r, (1, CONV_DIM, DN_K - 1)).to(dtype)
    state = normal(r, (1, DN_HV, DN_D, DN_D), 0.02)
    return conv, state


def hidden_states(seed: int, seq: int, dtype=torch.float32, hidden: int = HIDDEN) -> torch.Tensor:
    return normal(rng(seed), (1, seq, hidden)).to(dtype)


def delta_rule_inputs(seed: int, seq: int, heads: int = DN_HV, d: int = DN_D):
    """Free-function inputs of the delta rule: (q, k, v, g, beta) float32."""
    r = rng(seed)
    q = normal(r, (1, seq, heads, d))
    k = normal(r, (1, seq, heads, d))
    v = normal(r, (1, seq, heads, d))
    g = -torch.nn.functional.softplus(normal(r, (1, seq, heads)))
    beta = torch.sigmoid(normal(r, (1, seq, heads)))
    return q, k, v, g, beta


def golden_rope(rot, n: int):
    """(cos, sin) [1, n, 64] for positions 0..n-1 from the oracle's rotary
    tables, with the rows tests/golden/rope.npz holds (the golden generator's
    own, at the positions the score fixtures use) patched in: the last bit of a
    few entries depends on the host CPU's math library."""
    import os
    p = torch.arange(n)[None]
    cos, sin = rot(p[None].expand(3, -1, -1))
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "rope.npz"))
    pos = z["positions"]
    keep = pos < n
    idx = torch.from_numpy(pos[keep].astype(np.int64))
    cos, sin = cos.clone(), sin.clone()
    cos[0, idx] = torch.from_numpy(z["cos"][keep])
    sin[0, idx] = torch.from_numpy(z["sin"][keep])
    return cos, sin
