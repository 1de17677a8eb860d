"""Preplanned decode steps: every buffer fixed up front, ``run()`` only launches.

``QsaDecodePlan`` and ``DnDecodePlan`` bind one layer's cache, its device
weights and all intermediate buffers (indexer query, selected ids, split-K
partials, outputs) at construction, so a decode step issues the library's
kernel launches and nothing else: no allocation, no host synchronisation, no
memset. That is what makes a step capturable in a HIP graph (the analogue of the
reference's traced decoder, tt/traced.py:156-314, with positions as device
data as tt/model.py:402-432 binds them) and what the benchmark times.
"""

from __future__ import annotations

import ctypes

import torch

from . import native


class BoundCall:
    """One entry point with every argument but the trailing stream converted
    to its ctypes type once: a call is one foreign call and an error check,
    for a host loop that launches the same step many times (a plan's buffers
    never move). The referenced geometry and tensors must outlive it."""

    def __init__(self, name: str, *args):
        self.name = name
        self.fn = getattr(native.load(), name)
        types = self.fn.argtypes[:-1]
        if len(args) != len(types):
            raise ValueError(f"{name} takes {len(types)} arguments before the stream, got {len(args)}")
        self.args = tuple(a if not isinstance(a, int) and a is not None else t(a) for a, t in zip(args, types))

    def __call__(self, stream: int) -> None:
        rc = self.fn(*self.args, stream)
        if rc:
            raise native.QmError(f"{self.name} failed ({rc}): {native.load().qm_last_error().decode(errors='replace')}")


class DnDecodePlan:
    """One DeltaNet decode step of ``layer`` for a ``batch``-row cache."""

    def __init__(self, model, cache, layer: int, dtype=torch.bfloat16):
        c = model.config
        self.model, self.layer = model, layer
        self.lc = cache[layer]
        batch = cache.batch
        self.lc.ensure_dn(batch, dtype)
        dev = model.device
        self.geom = model.dn_geom(batch, dtype)
        self.positions = torch.zeros(batch, dtype=torch.int32, device=dev)
        self.out = torch.empty(batch, 1, c.linear_value_dim, dtype=dtype, device=dev)
        nbytes = native.load().qm_dn_decode_workspace(batch, c.linear_num_v_heads, c.linear_head_dim)
        self.ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        self.w = {s: model._dw(layer, s, t) for s, t in (("ssm_a", torch.float32), ("ssm_dt.bias", torch.float32),
                                                          ("ssm_conv1d.weight", dtype),
                                                          ("ssm_norm.weight", torch.float32))}

    def check(self, reset: bool = True) -> list:
        """Hand-off faults of this plan's launches since the last check (a sync)."""
        c = self.model.config
        return native.dn_decode_faults(self.geom.batch, c.linear_num_v_heads, c.linear_head_dim, self.ws, reset,
                                       f"layer {self.layer}", self.model.device)

    def _args(self, qkv, z, a, b):
        w, lc = self.w, self.lc
        return (ctypes.byref(self.geom), qkv.data_ptr(), z.data_ptr(), a.data_ptr(), b.data_ptr(),
                w["ssm_a"].data_ptr(), w["ssm_dt.bias"].data_ptr(), w["ssm_conv1d.weight"].data_ptr(),
                w["ssm_norm.weight"].data_ptr(), self.positions.data_ptr(), lc.conv_ring.data_ptr(),
                lc.recurrent_state.data_ptr(), self.out.data_ptr(), self.ws.data_ptr(), self.ws.numel())

    def run(self, qkv, z, a, b, stream=None):
        native.call("qm_dn_decode", *self._args(qkv, z, a, b),
                    stream if stream is not None else native.stream_handle(self.model.device))
        return self.out

    def bind(self, qkv, z, a, b) -> BoundCall:
        """The step on these inputs as a BoundCall (stream at call time)."""
        return BoundCall("qm_dn_decode", *self._args(qkv, z, a, b))


class QsaDecodePlan:
    """One QSA decode step (prep, select, attend) of ``layer``, sized for
    positions up to ``max_position``."""

    def __init__(self, model, cache, layer: int, max_position: int, dtype=torch.bfloat16, fused=None):
        c = model.config
        self.model, self.layer, self.cache = model, layer, cache
        self.lc = cache[layer]
        batch = cache.batch
        self.lc.ensure_qsa(batch, dtype)
        dev = model.device
        self.geom = model.qsa_geom(cache, dtype)
        lib = native.load()
        self.splits = lib.qm_qsa_attend_splits(ctypes.byref(self.geom), max_position, max_position)
        self.ws = torch.zeros(lib.qm_qsa_attend_workspace(ctypes.byref(self.geom), 1, self.splits),
                              dtype=torch.uint8, device=dev)
        self.dec_splits = lib.qm_qsa_decode_splits(ctypes.byref(self.geom), max_position)
        # one launch when the geometry allows it and a group of dec_splits
        # workgroups fits the device at once; else prep + select + attend
        can_fuse = model.fused_decode_fits(cache) and model.decode_group_fits(self.dec_splits, dtype)
        faster = model.fused_decode_fits(cache, max_position)
        if fused and not can_fuse:
            raise native.QmError(f"layer {layer}: this geometry does not fit one qm_qsa_decode launch")
        self.fused = (can_fuse and faster) if fused is None else bool(fused)
        # the other path: prep, the scores spread over the blocks, the ranking,
        # and the attention (the scores' buffer makes qm_qsa_select split them)
        self.scores = None if self.fused else torch.empty(batch, 1, cache.max_blocks, dtype=torch.float32,
                                                           device=dev)
        self.dec_ws = torch.zeros(lib.qm_qsa_decode_workspace(ctypes.byref(self.geom), self.dec_splits),
                                  dtype=torch.uint8, device=dev)
        self.positions = torch.zeros(batch, dtype=torch.int32, device=dev)
        self.q_out = torch.empty(batch, 1, 2, c.num_attention_heads, c.head_dim, dtype=torch.bfloat16, device=dev)
        self.iq_out = torch.empty(batch, 1, c.indexer_heads, c.indexer_head_dim, dtype=torch.float32, device=dev)
        self.ids = torch.zeros(batch, 1, c.block_topk, dtype=torch.int32, device=dev)
        self.n_sel = torch.zeros(batch, 1, dtype=torch.int32, device=dev)
        self.items = torch.zeros(batch, 1, 2 * lib.qm_qsa_items_stride(ctypes.byref(self.geom)), dtype=torch.int32,
                                 device=dev)
        self.out = torch.empty(batch, 1, c.num_attention_heads * c.head_dim, dtype=dtype, device=dev)
        self.w = {s: model._dw(layer, s, torch.float32) for s in
                  ("attn_q_norm.weight", "attn_k_norm.weight", "indexer.q_norm.weight", "indexer.k_norm.weight")}
        self.cos, self.sin = model.rope.get(max_position + 1)

    def front(self, qg, k, v, iq, ik, stream):
        """prep + select in one launch (qm_qsa_decode_front)."""
        lc, w = self.lc, self.w
        native.call("qm_qsa_decode_front", ctypes.byref(self.geom), qg.data_ptr(), k.data_ptr(), v.data_ptr(),
                    iq.data_ptr(), ik.data_ptr(), w["attn_q_norm.weight"].data_ptr(),
                    w["attn_k_norm.weight"].data_ptr(), w["indexer.q_norm.weight"].data_ptr(),
                    w["indexer.k_norm.weight"].data_ptr(), self.cos.data_ptr(), self.sin.data_ptr(),
                    self.positions.data_ptr(), lc.page_table.data_ptr(), lc.k_pool.data_ptr(),
                    lc.v_pool.data_ptr(), lc.raw_keys.data_ptr(), lc.block_keys.data_ptr(), self.q_out.data_ptr(),
                    self.iq_out.data_ptr(), self.ids.data_ptr(), self.n_sel.data_ptr(), self.items.data_ptr(),
                    stream)

    def prep(self, qg, k, v, iq, ik, stream):
        lc, w = self.lc, self.w
        native.call("qm_qsa_prep", ctypes.byref(self.geom), 1, qg.data_ptr(), k.data_ptr(), v.data_ptr(),
                    iq.data_ptr(), ik.data_ptr(), w["attn_q_norm.weight"].data_ptr(),
                    w["attn_k_norm.weight"].data_ptr(), w["indexer.q_norm.weight"].data_ptr(),
                    w["indexer.k_norm.weight"].data_ptr(), self.cos.data_ptr(), self.sin.data_ptr(),
                    self.positions.data_ptr(), lc.page_table.data_ptr(), lc.k_pool.data_ptr(),
                    lc.v_pool.data_ptr(), lc.raw_keys.data_ptr(), lc.block_keys.data_ptr(), self.q_out.data_ptr(),
                    self.iq_out.data_ptr(), stream)

    def select(self, stream):
        native.call("qm_qsa_select", ctypes.byref(self.geom), 1, self.iq_out.data_ptr(),
                    self.lc.block_keys.data_ptr(), self.positions.data_ptr(), self.lc.page_table.data_ptr(),
                    self.ids.data_ptr(), self.n_sel.data_ptr(), self.items.data_ptr(),
                    None if self.scores is None else self.scores.data_ptr(), stream)

    def attend(self, qg, stream):
        lc = self.lc
        native.call("qm_qsa_attend", ctypes.byref(self.geom), 1, self.q_out.data_ptr(), qg.data_ptr(),
                    lc.k_pool.data_ptr(), lc.v_pool.data_ptr(), self.items.data_ptr(), self.out.data_ptr(),
                    self.splits, self.ws.data_ptr(), self.ws.numel(), stream)

    def _decode_args(self, qg, k, v, iq, ik):
        lc, w = self.lc, self.w
        return (ctypes.byref(self.geom), qg.data_ptr(), k.data_ptr(), v.data_ptr(), iq.data_ptr(), ik.data_ptr(),
                w["attn_q_norm.weight"].data_ptr(), w["attn_k_norm.weight"].data_ptr(),
                w["indexer.q_norm.weight"].data_ptr(), w["indexer.k_norm.weight"].data_ptr(), self.cos.data_ptr(),
                self.sin.data_ptr(), self.positions.data_ptr(), lc.page_table.data_ptr(), lc.k_pool.data_ptr(),
                lc.v_pool.data_ptr(), lc.raw_keys.data_ptr(), lc.block_keys.data_ptr(), self.out.data_ptr(),
                self.dec_splits, self.dec_ws.data_ptr(), self.dec_ws.numel(), None, None, None, None)

    def decode(self, qg, k, v, iq, ik, stream):
        """The whole step in one qm_qsa_decode launch."""
        native.call("qm_qsa_decode", *self._decode_args(qg, k, v, iq, ik), stream)

    def bind(self, qg, k, v, iq, ik) -> BoundCall:
        """The one-launch step on these inputs as a BoundCall (stream at call
        time); plans that do not fit one launch are refused."""
        if not self.fused:
            raise native.QmError(f"layer {self.layer}: this plan runs as prep + select + attend, not one launch")
        return BoundCall("qm_qsa_decode", *self._decode_args(qg, k, v, iq, ik))

    def check(self, reset: bool = True) -> list:
        """Hand-off faults of this plan's fused launches since the last check
        (a sync): waits that gave up, positions beyond the plan's splits."""
        if not self.fused:
            return []
        return native.qsa_decode_faults(self.geom, self.dec_splits, self.dec_ws, reset, f"layer {self.layer}",
                                        self.model.device)

    def run(self, qg, k, v, iq, ik, stream=None):
        s = stream if stream is not None else native.stream_handle(self.model.device)
        if self.fused:
            self.decode(qg, k, v, iq, ik, s)
        else:
            self.prep(qg, k, v, iq, ik, s)
            self.select(s)
            self.attend(qg, s)
        return self.out
