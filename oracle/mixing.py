"""Oracle restatement of the token-mixing methods of reference/model.py.

``OracleMixer`` carries the three methods the drop-in boundary replaces, with
the reference's signatures:

* ``_linear_attention(hidden, layer, cache)``            reference/model.py:177-244
* ``_indexer_mask(hidden, layer, cos, sin, cache, kv_len, query_offset)``
                                                          reference/model.py:248-327
* ``_full_attention(hidden, layer, cos, sin, cache, query_offset)``
                                                          reference/model.py:331-383

Weights come through ``bw(layer, suffix) -> store.get(f"blk.{layer}.{suffix}")``
exactly as reference/model.py:45-49, so a fake store (the pattern of reference
tests/test_indexer_mask.py:94-113) drives it without a checkpoint.

The only deliberate departure is the top-k tie rule (``tie_rule``): the default
``"lower_index"`` breaks equal scores toward the lower block index; ``"torch"``
calls ``Tensor.topk`` exactly as the reference does. They select the same set
whenever the k-th and (k+1)-th eligible scores differ.

The intermediates the HIP path exposes (indexer query, pooled block keys, block
scores, selected ids) are available as separate methods so they can be compared
one stage at a time; ``_indexer_mask`` is assembled from them with the same op
sequence as the reference.

Pinned by: golden vectors of the reference's own methods on seeded inputs
(tests/golden/make_golden.py, tests/test_golden.py), the invariants of reference
tests/test_indexer_mask.py restated (tests/test_oracle_selection.py), and the
one-key closed form ``out = sigmoid(gate) * v`` (tests/test_oracle_layers.py).
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from .cnative import block_scores
from .layers import (
    apply_rotary,
    causal_conv1d,
    causal_conv1d_step,
    chunk_gated_delta_rule,
    recurrent_gated_delta_rule,
    rms_norm,
    rms_norm_gated,
)


class OracleMixer:
    def __init__(self, config, store, tie_rule: str = "lower_index"):
        if tie_rule not in ("lower_index", "torch"):
            raise ValueError(f"unknown tie rule {tie_rule!r}")
        self.config = config
        self.store = store
        self.tie_rule = tie_rule

    # reference/model.py:45-49
    def w(self, name: str) -> torch.Tensor:
        return self.store.get(name)

    def bw(self, layer: int, suffix: str) -> torch.Tensor:
        return self.store.get(f"blk.{layer}.{suffix}")

    # ------------------------------------------------------------------
    # Hyper-connections around each branch
    # ------------------------------------------------------------------

    def _gated_residual(self, hyper, layer, kind: str):
        """reference/model.py:53-77: (mixed, hyper, inject or None).

        ``hyper`` holds ``hc_count`` residual streams of ``hidden_size`` side by
        side. Each stream is rms-normalised on its own; a low-rank
        down/silu/up/sigmoid product gates every element, and the gated streams
        are averaged into the branch input. The layer mixers also return the
        per-stream injection weights 2 sigmoid(normed . inject_w^T / hc_count);
        the final mixer (``layer is None``) returns None there.
        """
        cfg = self.config
        hc, width = cfg.hc_count, cfg.hidden_size
        prefix = "output_hc" if layer is None else f"blk.{layer}.hc_{kind}"
        normed = rms_norm(hyper, self.w(f"{prefix}_norm.weight"), cfg.rms_norm_eps, group_size=width)
        low = F.silu(F.linear(normed, self.w(f"{prefix}_down.weight")) / hc)
        gate = torch.sigmoid(F.linear(low, self.w(f"{prefix}_up.weight")))
        gated = gate.unflatten(-1, (hc, width)) * normed.unflatten(-1, (hc, width))
        mixed = gated.mean(dim=-2)
        if layer is None:
            return mixed, hyper, None
        inject = 2 * torch.sigmoid(F.linear(normed, self.w(f"{prefix}_inject.weight")) / hc)
        return mixed, hyper, inject

    @staticmethod
    def _reinject(hyper, branch_out, inject):
        """reference/model.py:79-81: stream s gains branch_out * inject[..., s]."""
        scaled = inject.unsqueeze(-1) * branch_out.unsqueeze(-2)
        return hyper + scaled.flatten(-2)

    # ------------------------------------------------------------------
    # Gated DeltaNet
    # ------------------------------------------------------------------

    def _linear_attention(self, hidden, layer: int, cache):
        """reference/model.py:177-244."""
        mixed = F.linear(hidden, self.bw(layer, "attn_qkv.weight"))
        z = F.linear(hidden, self.bw(layer, "attn_gate.weight"))
        b = F.linear(hidden, self.bw(layer, "ssm_beta.weight"))
        a = F.linear(hidden, self.bw(layer, "ssm_alpha.weight"))
        out = self.dn_core(mixed, z, b, a, layer, cache)
        return F.linear(out, self.bw(layer, "ssm_out.weight"))

    def dn_core(self, mixed, z, b, a, layer: int, cache):
        """reference/model.py:184-243 between the projections and ssm_out.

        ``mixed`` [B, S, conv_dim], ``z`` [B, S, Hv*d], ``b``, ``a`` [B, S, Hv]
        are the projection outputs; returns the gated-normed [B, S, Hv*d].
        """
        cfg = self.config
        n_b, n_t, _ = mixed.shape
        n_v, n_k, d = cfg.linear_num_v_heads, cfg.linear_num_k_heads, cfg.linear_head_dim
        mixed = mixed.transpose(1, 2)
        z = z.reshape(n_b, n_t, -1, d)

        conv_w = self.bw(layer, "ssm_conv1d.weight")
        hist = cfg.conv_kernel - 1
        if cache is not None:
            window = cache[layer].conv_state
            if window is None:
                window = mixed.new_zeros(n_b, cfg.conv_dim, hist)
            if n_t == 1:
                mixed, window = causal_conv1d_step(mixed, window, conv_w)
                cache[layer].conv_state = window
            else:
                joined = torch.cat([window, mixed], dim=-1)
                cache[layer].conv_state = joined[:, :, -hist:].clone()
                mixed = causal_conv1d(joined, conv_w)[:, :, -n_t:]
        else:
            mixed = causal_conv1d(mixed, conv_w)

        mixed = mixed.transpose(1, 2)
        kd = cfg.linear_key_dim
        query, key, value = torch.split(mixed, [kd, kd, cfg.linear_value_dim], dim=-1)
        query = query.reshape(n_b, n_t, n_k, d)
        key = key.reshape(n_b, n_t, n_k, d)
        value = value.reshape(n_b, n_t, n_v, d)

        beta = b.sigmoid()
        a_neg = self.bw(layer, "ssm_a")          # stored as -exp(A_log): no exp here
        dt_bias = self.bw(layer, "ssm_dt.bias")
        g = a_neg.float() * F.softplus(a.float() + dt_bias.float())

        # value head j reads key head j % n_k: tile (repeat), not interleave
        if n_v > n_k:
            reps = n_v // n_k
            query = query.repeat(1, 1, reps, 1)
            key = key.repeat(1, 1, reps, 1)

        prev = cache[layer].recurrent_state if cache is not None else None
        rule = recurrent_gated_delta_rule if n_t == 1 else chunk_gated_delta_rule
        out, new_state = rule(query, key, value, g, beta, initial_state=prev)
        if cache is not None:
            cache[layer].recurrent_state = new_state

        return rms_norm_gated(
            out.reshape(-1, d), z.reshape(-1, d), self.bw(layer, "ssm_norm.weight"),
            cfg.rms_norm_eps, cfg.output_gate_type,
        ).reshape(n_b, n_t, -1)

    # ------------------------------------------------------------------
    # QSA indexer, one stage at a time
    # ------------------------------------------------------------------

    def indexer_query(self, hidden, layer: int, cos, sin):
        """reference/model.py:270-272: rope(rms_norm(x W_iq^T)) at the query positions."""
        cfg = self.config
        n_b, n_t, _ = hidden.shape
        q = F.linear(hidden, self.bw(layer, "indexer.q_proj.weight")).reshape(
            n_b, n_t, -1, cfg.indexer_head_dim)
        q = rms_norm(q, self.bw(layer, "indexer.q_norm.weight"), cfg.rms_norm_eps)
        return apply_rotary(q, cos[:, -n_t:], sin[:, -n_t:], unsqueeze_dim=2)

    def indexer_pooled(self, keys, layer: int, cos, sin, n_blocks: int):
        """reference/model.py:289-294: mean-pool each block of raw keys, norm, rope at its start."""
        cfg = self.config
        ratio, dim = cfg.indexer_compress_ratio, cfg.indexer_head_dim
        n_b = keys.shape[0]
        pooled = keys[:, : n_blocks * ratio].reshape(n_b, n_blocks, ratio, dim).float().mean(dim=2)
        pooled = rms_norm(pooled.to(keys.dtype), self.bw(layer, "indexer.k_norm.weight"), cfg.rms_norm_eps)
        starts = torch.arange(n_blocks, device=keys.device) * ratio
        pooled = apply_rotary(pooled.unsqueeze(2), cos[:, starts], sin[:, starts], unsqueeze_dim=2)
        return pooled.squeeze(2)

    def indexer_scores(self, q, pooled):
        """reference/model.py:297-298: sum over heads of relu(q_h . block) / sqrt(d).

        The reference computes this with torch's einsum; its float32 result
        depends on the summation order the host's BLAS takes. The oracle
        restates the order that produced the golden score vectors (scores.c),
        so its scores do not change with the machine it runs on;
        ``indexer_scores_torch`` is the reference's own expression."""
        if self.config.indexer_head_dim != 128:
            return self.indexer_scores_torch(q, pooled)
        return block_scores(q, pooled).to(q.device)

    def indexer_scores_torch(self, q, pooled):
        """reference/model.py:297-298 as the reference writes it (torch einsum)."""
        dim = self.config.indexer_head_dim
        s = torch.einsum("bqhd,bkd->bqhk", q.float(), pooled.float())
        return torch.relu(s).sum(dim=2) / math.sqrt(dim)

    def _topk_blocks(self, scores, k: int):
        if self.tie_rule == "torch":
            return scores.topk(k, dim=-1).indices
        # stable descending sort keeps equal scores in index order
        return torch.sort(scores, dim=-1, descending=True, stable=True).indices[..., :k]

    def indexer_select(self, scores, query_offset: int):
        """reference/model.py:300-308: eligibility, top-k, and which picks are kept.

        Returns ``(chosen, chosen_valid, eligible)`` shaped like the reference's.
        """
        cfg = self.config
        ratio = cfg.indexer_compress_ratio
        n_t, n_blocks = scores.shape[-2], scores.shape[-1]
        starts = torch.arange(n_blocks, device=scores.device) * ratio
        query_pos = torch.arange(n_t, device=scores.device) + query_offset
        eligible = (starts + ratio - 1)[None, :] <= query_pos[:, None]
        scores = scores.masked_fill(~eligible[None], float("-inf"))
        k = min(cfg.indexer_budget // ratio, n_blocks)
        chosen = self._topk_blocks(scores, k)
        chosen_valid = eligible[None].expand(scores.shape[0], -1, -1).gather(-1, chosen)
        return chosen, chosen_valid, eligible

    def _indexer_mask(self, hidden, layer: int, cos, sin, cache, kv_len: int, query_offset: int):
        """reference/model.py:248-327: boolean (B, 1, S, kv_len) visibility mask."""
        cfg = self.config
        n_b, n_t, _ = hidden.shape
        dim, ratio = cfg.indexer_head_dim, cfg.indexer_compress_ratio

        q = self.indexer_query(hidden, layer, cos, sin)
        raw_k = F.linear(hidden, self.bw(layer, "indexer.k_proj.weight")).reshape(n_b, n_t, dim)
        if cache is not None:
            if cache[layer].indexer_keys is not None:
                raw_k = torch.cat([cache[layer].indexer_keys, raw_k], dim=1)
            cache[layer].indexer_keys = raw_k
        keys = raw_k[:, :kv_len]

        n_blocks = kv_len // ratio
        if n_blocks == 0:
            kpos = torch.arange(kv_len, device=hidden.device)
            qpos = torch.arange(n_t, device=hidden.device)[:, None] + query_offset
            return (kpos[None, None, :] <= qpos[None]).expand(n_b, n_t, kv_len).unsqueeze(1)

        pooled = self.indexer_pooled(keys, layer, cos, sin, n_blocks)
        scores = self.indexer_scores(q, pooled)
        chosen, chosen_valid, _ = self.indexer_select(scores, query_offset)

        mask = torch.zeros(n_b, n_t, kv_len, dtype=torch.bool, device=hidden.device)
        token_idx = (chosen.unsqueeze(-1) * ratio + torch.arange(ratio, device=hidden.device)).flatten(2)
        keep = chosen_valid.unsqueeze(-1).expand(-1, -1, -1, ratio).flatten(2)
        mask.scatter_(2, token_idx, keep)

        query_pos = torch.arange(n_t, device=hidden.device) + query_offset
        tail_start = ((query_pos + 1) // ratio) * ratio
        kpos = torch.arange(kv_len, device=hidden.device)
        tail = (kpos[None, :] >= tail_start[:, None]) & (kpos[None, :] <= query_pos[:, None])
        mask |= tail[None]
        return mask.unsqueeze(1)

    # ------------------------------------------------------------------
    # QSA full attention
    # ------------------------------------------------------------------

    def qkv_prep(self, hidden, layer: int, cos, sin):
        """reference/model.py:345-356: q|gate split, q/k RMS norm, partial rope.

        Returns ``(q, k, v, gate)`` with q, k, v shaped (B, heads, S, head_dim).
        """
        cfg = self.config
        n_b, n_t, _ = hidden.shape
        hd = cfg.head_dim
        qg = F.linear(hidden, self.bw(layer, "attn_q.weight")).view(n_b, n_t, -1, hd * 2)
        q, gate = torch.chunk(qg, 2, dim=-1)
        gate = gate.reshape(n_b, n_t, -1)
        q = rms_norm(q, self.bw(layer, "attn_q_norm.weight"), cfg.rms_norm_eps).transpose(1, 2)
        k = F.linear(hidden, self.bw(layer, "attn_k.weight")).view(n_b, n_t, -1, hd)
        k = rms_norm(k, self.bw(layer, "attn_k_norm.weight"), cfg.rms_norm_eps).transpose(1, 2)
        v = F.linear(hidden, self.bw(layer, "attn_v.weight")).view(n_b, n_t, -1, hd).transpose(1, 2)
        c, s = cos[:, -n_t:], sin[:, -n_t:]
        return apply_rotary(q, c, s), apply_rotary(k, c, s), v, gate

    def attention_core(self, q, k, v, allowed, out_dtype):
        """reference/model.py:372-379: GQA, fp32 masked softmax, weights @ v."""
        cfg = self.config
        groups = cfg.num_attention_heads // cfg.num_kv_heads
        k = k.repeat_interleave(groups, dim=1)
        v = v.repeat_interleave(groups, dim=1)
        scores = (q.float() @ k.float().transpose(-1, -2)) / math.sqrt(cfg.head_dim)
        scores = scores.masked_fill(~allowed, torch.finfo(torch.float32).min)
        probs = torch.softmax(scores, dim=-1)
        return (probs @ v.float()).to(out_dtype)

    def _full_attention(self, hidden, layer: int, cos, sin, cache, query_offset: int):
        """reference/model.py:331-383."""
        n_b, n_t, _ = hidden.shape
        q, k, v, gate = self.qkv_prep(hidden, layer, cos, sin)
        if cache is not None:
            if cache[layer].keys is not None:
                k = torch.cat([cache[layer].keys, k], dim=2)
                v = torch.cat([cache[layer].values, v], dim=2)
            cache[layer].keys, cache[layer].values = k, v
        kv_len = k.shape[2]

        qsa = self._indexer_mask(hidden, layer, cos, sin, cache, kv_len, query_offset)
        kpos = torch.arange(kv_len, device=hidden.device)
        qpos = torch.arange(n_t, device=hidden.device)[:, None] + query_offset
        allowed = (kpos[None, :] <= qpos)[None, None] & qsa

        out = self.attention_core(q, k, v, allowed, hidden.dtype)
        out = out.transpose(1, 2).reshape(n_b, n_t, -1)
        out = out * torch.sigmoid(gate)
        return F.linear(out, self.bw(layer, "attn_output.weight"))
