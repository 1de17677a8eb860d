"""Device-resident rope tables.

The reference recomputes ``cos, sin = RotaryEmbedding(positions)`` on every
forward (reference/model.py:434-438, reference/layers.py:73-108). The tables
depend only on the position, so this module builds them once per length on the
CPU with the same torch operations the reference uses -- which makes them
bit-identical to the reference's -- and keeps a float32 ``[n_pos, rope_dim]``
copy on the device that the kernels index by position. Text input only: the
three mrope position rows are equal, so the interleave leaves the values alone.
"""

from __future__ import annotations

import torch


def rope_tables_cpu(n_pos: int, rope_dim: int, theta: float, mrope_section) -> tuple[torch.Tensor, torch.Tensor]:
    """cos, sin of shape (1, n_pos, rope_dim), float32, as reference/layers.py:100-108."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, rope_dim, 2, dtype=torch.float) / rope_dim))
    pos = torch.arange(n_pos)[None]
    pos3 = pos[None].expand(3, -1, -1)
    inv = inv_freq[None, None, :, None].float().expand(3, 1, -1, 1)
    freqs = (inv @ pos3[:, :, None, :].float()).transpose(2, 3)
    merged = freqs[0].clone()
    for axis in (1, 2):
        span = mrope_section[axis] * 3
        merged[..., axis:span:3] = freqs[axis][..., axis:span:3]
    emb = torch.cat((merged, merged), dim=-1)
    return emb.cos(), emb.sin()


class RopeTable:
    """Grows on demand; ``get(n)`` returns device (cos, sin) covering n positions."""

    def __init__(self, rope_dim: int, theta: float, mrope_section, device):
        self.rope_dim, self.theta, self.mrope = rope_dim, theta, list(mrope_section)
        self.device = torch.device(device)
        self.cos = self.sin = None

    def get(self, n_pos: int):
        if self.cos is None or self.cos.shape[0] < n_pos:
            n = max(n_pos, 2 * (0 if self.cos is None else self.cos.shape[0]), 1024)
            c, s = rope_tables_cpu(n, self.rope_dim, self.theta, self.mrope)
            self.cos = c[0].contiguous().to(self.device)
            self.sin = s[0].contiguous().to(self.device)
        return self.cos, self.sin
