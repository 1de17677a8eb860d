"""The token-mixing layers of qwen4exp on MI355X, behind the reference's methods.

``Qwen4MixModel`` carries the three methods of the reference's
``Qwen4ExpModel`` that this path replaces, with the same names, signatures and
return values, so an engine written against the reference can call them:

* ``_linear_attention(hidden, layer, cache)``            reference/model.py:177-244
* ``_indexer_mask(hidden, layer, cos, sin, cache, kv_len, query_offset)``
                                                          reference/model.py:248-327
* ``_full_attention(hidden, layer, cos, sin, cache, query_offset)``
                                                          reference/model.py:331-383

Weights come from ``store.get(f"blk.{layer}.{suffix}")`` as in
reference/model.py:45-49 and are copied to the device once. The projections
(``F.linear``) run as PyTorch-ROCm GEMMs; everything between them -- conv ring,
gates, delta rule, norms, rope, paging, indexer scoring, top-k, attention,
output gate -- runs in the HIP kernels of libqwen4mix.so. There is no other
implementation to fall back to: a missing library or a failed call raises.

``cache`` is a ``MixHybridCache`` (cache.py). ``hidden`` must be a float32 or
bfloat16 tensor on the model's device.
"""

from __future__ import annotations

import ctypes

import torch
import torch.nn.functional as F

from . import native
from .cache import MixHybridCache
from .config import MixConfig
from .rope import RopeTable


class Qwen4MixModel:
    # a prefill chunk's selection files its entries for the chunk attention
    # (qm_qsa_select_chunk + qm_qsa_attend_chunk_filed) rather than the
    # attention filing them itself (qm_qsa_select + qm_qsa_attend_chunk)
    fuse_chunk_select = True

    def __init__(self, config, store, device=None, max_ctx: int = 8192):
        self.config = config if isinstance(config, MixConfig) else MixConfig.from_reference(config)
        self.store = store
        self.device = torch.device(device if device is not None else "cuda")
        self.max_ctx = max_ctx
        self.rope = RopeTable(self.config.rope_dim, self.config.rope_theta, self.config.mrope_section, self.device)
        self._dev = {}
        self._ws = {}
        self._rope_copy = None  # (key, cos, sin): the device copy of the caller's host rope tables
        self._handoff = {}      # decode workspaces whose hand-off counters check_handoffs() reads
        native.load()

    # -- weights (reference/model.py:45-49) -----------------------------------

    def w(self, name: str) -> torch.Tensor:
        return self.store.get(name)

    def bw(self, layer: int, suffix: str) -> torch.Tensor:
        return self.store.get(f"blk.{layer}.{suffix}")

    def _dw(self, layer: int, suffix: str, dtype=None) -> torch.Tensor:
        key = (layer, suffix, dtype)
        t = self._dev.get(key)
        if t is None:
            src = self.bw(layer, suffix)
            t = src.to(self.device, dtype if dtype is not None else src.dtype).contiguous()
            self._dev[key] = t
        return t

    # projections that read the same input, concatenated row-wise so that the
    # small-M GEMV streams a layer's weights for them in one launch
    PROJ_GROUPS = {
        "dn_in": ("attn_qkv.weight", "attn_gate.weight", "ssm_beta.weight", "ssm_alpha.weight"),
        "dn_out": ("ssm_out.weight",),
        "qsa_in": ("attn_q.weight", "attn_k.weight", "attn_v.weight", "indexer.q_proj.weight",
                   "indexer.k_proj.weight"),
        "qsa_out": ("attn_output.weight",),
    }

    def _wcat(self, layer: int, group: str, dtype):
        """(weights [N, K], rows per projection) of a projection group; the
        layer's single matrices become row views of it."""
        key = (layer, "group:" + group, dtype)
        hit = self._dev.get(key)
        if hit is None:
            names = self.PROJ_GROUPS[group]
            parts = [self.bw(layer, n).to(self.device, dtype) for n in names]
            w = torch.cat(parts, 0).contiguous()
            rows = [int(t.shape[0]) for t in parts]
            start = 0
            for n, r in zip(names, rows):
                self._dev[(layer, n, dtype)] = w[start:start + r]
                start += r
            hit = (w, rows)
            self._dev[key] = hit
        return hit

    @staticmethod
    def _gemv_fits(dtype, m: int, k: int) -> bool:
        ks = (2048, 4096) if dtype == torch.bfloat16 else (1024, 2048, 4096)
        return m <= 4 and k in ks and dtype in (torch.bfloat16, torch.float32)

    def project(self, x: torch.Tensor, layer: int, group: str) -> list:
        """The group's projections of x [B, S, K] (F.linear with each weight), as
        a list of [B, S, rows] tensors. Up to 4 rows of x: one qm_gemv launch over
        the concatenated weights; more: a library GEMM per projection."""
        dt = x.dtype
        w, rows = self._wcat(layer, group, dt)
        batch, seq, k = x.shape
        if self._gemv_fits(dt, batch * seq, k):
            xc = x.contiguous()
            outs = [torch.empty(batch, seq, r, dtype=dt, device=self.device) for r in rows]
            seg_rows = (ctypes.c_int * len(rows))(*rows)
            seg_out = (ctypes.c_void_p * len(rows))(*[o.data_ptr() for o in outs])
            native.call("qm_gemv", native.act_code(dt), batch * seq, int(w.shape[0]), k, native.ptr(w),
                        native.ptr(xc), len(rows), seg_rows, seg_out, native.stream_handle(self.device))
            return outs
        outs, start = [], 0
        for r in rows:
            outs.append(F.linear(x, w[start:start + r]))
            start += r
        return outs

    # -- hyper-connections around each branch (reference/model.py:53-81) --------

    def hc_weights(self, layer, kind: str, dtype):
        """(norm_w f32, down|inject [rank + hc or rank, K], up [K, rank], with_inject)
        of one mixer on the device; ``layer is None`` is the final mixer."""
        prefix = "output_hc" if layer is None else f"blk.{layer}.hc_{kind}"
        key = (prefix, "hc", dtype)
        hit = self._dev.get(key)
        if hit is None:
            norm_w = self.w(f"{prefix}_norm.weight").to(self.device, torch.float32).contiguous()
            rows = [self.w(f"{prefix}_down.weight")]
            if layer is not None:
                rows.append(self.w(f"{prefix}_inject.weight"))
            di = torch.cat([r.to(self.device, dtype) for r in rows], 0).contiguous()
            up = self.w(f"{prefix}_up.weight").to(self.device, dtype).contiguous()
            hit = (norm_w, di, up, layer is not None)
            self._dev[key] = hit
        return hit

    def hc_geom(self, rows: int, dtype) -> native.HcGeom:
        c = self.config
        return native.HcGeom(rows, c.hc_count, c.hidden_size, c.hc_lowrank, native.act_code(dtype), c.rms_norm_eps)

    def _gated_residual(self, hyper: torch.Tensor, layer, kind: str, mixed=None, inject=None):
        """reference/model.py:53-77: (mixed [.., hidden], hyper, inject [.., hc_count] or None).

        One qm_hc_mix call (two launches): the per-stream norm, the down and
        inject products and their gates, the up product and the gated mean.
        ``mixed``/``inject`` may be preallocated outputs."""
        c = self.config
        dt = hyper.dtype
        lead = hyper.shape[:-1]
        rows = hyper.numel() // hyper.shape[-1]
        norm_w, di, up, with_inject = self.hc_weights(layer, kind, dt)
        g = self.hc_geom(rows, dt)
        ws = self._workspace("hc", native.load().qm_hc_mix_workspace(ctypes.byref(g)))
        hyper_c = hyper.contiguous()
        if mixed is None:
            mixed = torch.empty(*lead, c.hidden_size, dtype=dt, device=self.device)
        if with_inject and inject is None:
            inject = torch.empty(*lead, c.hc_count, dtype=dt, device=self.device)
        native.call("qm_hc_mix", ctypes.byref(g), native.ptr(hyper_c), native.ptr(norm_w), native.ptr(di),
                    int(with_inject), native.ptr(up), native.ptr(mixed), native.ptr(inject) if with_inject else None,
                    native.ptr(ws), ws.numel(), native.stream_handle(self.device))
        return mixed, hyper, (inject if with_inject else None)

    @staticmethod
    def _reinject(hyper: torch.Tensor, branch_out: torch.Tensor, inject: torch.Tensor, out=None) -> torch.Tensor:
        """reference/model.py:79-81: hyper + branch_out scaled into every stream
        (one qm_hc_reinject launch; ``out`` may be ``hyper`` itself)."""
        streams, hidden = inject.shape[-1], branch_out.shape[-1]
        rows = branch_out.numel() // hidden
        if hyper.shape[-1] != streams * hidden or hyper.numel() != rows * streams * hidden:
            raise ValueError(f"_reinject: hyper {tuple(hyper.shape)} does not hold {streams} streams of "
                             f"{tuple(branch_out.shape)}")
        hyper_c = hyper.contiguous()
        if out is None:
            out = torch.empty_like(hyper_c)
        g = native.HcGeom(rows, streams, hidden, 0, native.act_code(hyper.dtype), 0.0)
        native.call("qm_hc_reinject", ctypes.byref(g), native.ptr(hyper_c), native.ptr(branch_out.contiguous()),
                    native.ptr(inject.contiguous()), native.ptr(out), native.stream_handle(hyper.device))
        return out

    def _workspace(self, name: str, nbytes: int) -> torch.Tensor:
        buf = self._ws.get(name)
        if buf is None or buf.numel() < nbytes:
            buf = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=self.device)
            self._ws[name] = buf
        return buf

    def _positions(self, batch: int, pos: int) -> torch.Tensor:
        return torch.full((batch,), pos, dtype=torch.int32, device=self.device)

    # -- geometry ----------------------------------------------------------------

    def dn_geom(self, batch: int, dtype) -> native.DnGeom:
        c = self.config
        return native.DnGeom(batch, c.linear_num_v_heads, c.linear_num_k_heads, c.linear_head_dim, c.conv_kernel,
                             native.act_code(dtype), c.rms_norm_eps)

    def qsa_geom(self, cache: MixHybridCache, dtype) -> native.QsaGeom:
        c = self.config
        return native.QsaGeom(cache.batch, c.num_attention_heads, c.num_kv_heads, c.head_dim, c.rope_dim,
                              c.indexer_heads, c.indexer_head_dim, c.indexer_compress_ratio, c.indexer_budget,
                              c.page_size, cache.max_pages, cache.max_ctx, cache.max_blocks, native.act_code(dtype),
                              c.rms_norm_eps)

    # -- Gated DeltaNet ------------------------------------------------------------

    def dn_core(self, qkv, z, a, b, layer: int, lc, out=None):
        """The mixer core between the projections (the HIP part of _linear_attention).

        qkv [B, S, conv_dim], z [B, S, Hv*d], a, b [B, S, Hv] (act) -> [B, S, Hv*d].
        ``lc`` is the layer's ``MixLayerCache``; its ring and state update in place.
        """
        c = self.config
        batch, seq = qkv.shape[0], qkv.shape[1]
        dt = qkv.dtype
        lc.ensure_dn(batch, dt)
        if out is None:
            out = torch.empty(batch, seq, c.linear_value_dim, dtype=dt, device=self.device)
        g = self.dn_geom(batch, dt)
        pos = self._positions(batch, lc.n_tokens)
        a_neg = self._dw(layer, "ssm_a", torch.float32)
        dt_bias = self._dw(layer, "ssm_dt.bias", torch.float32)
        conv_w = self._dw(layer, "ssm_conv1d.weight", dt)
        norm_w = self._dw(layer, "ssm_norm.weight", torch.float32)
        stream = native.stream_handle(self.device)
        args = (native.ptr(qkv), native.ptr(z), native.ptr(a), native.ptr(b), native.ptr(a_neg), native.ptr(dt_bias),
                native.ptr(conv_w), native.ptr(norm_w), native.ptr(pos), native.ptr(lc.conv_ring),
                native.ptr(lc.recurrent_state), native.ptr(out))
        if seq == 1:
            nbytes = native.load().qm_dn_decode_workspace(batch, c.linear_num_v_heads, c.linear_head_dim)
            ws = self._workspace(f"dn_decode_{batch}", nbytes)
            self._handoff[f"dn_decode_{batch}"] = ("dn", batch)
            native.call("qm_dn_decode", ctypes.byref(g), *args, native.ptr(ws), ws.numel(), stream)
        else:
            nbytes = native.load().qm_dn_prefill_workspace(ctypes.byref(g), seq)
            ws = self._workspace("dn_prefill", nbytes)
            native.call("qm_dn_prefill", ctypes.byref(g), seq, *args, native.ptr(ws), ws.numel(), stream)
        lc.n_tokens += seq
        return out

    def _linear_attention(self, hidden: torch.Tensor, layer: int, cache) -> torch.Tensor:
        """reference/model.py:177-244."""
        batch, seq, _ = hidden.shape
        dt = hidden.dtype
        if cache is None:
            cache = MixHybridCache(layer + 1, self.config, batch, max(seq, 64), self.device, dt)
        lc = cache[layer]
        qkv, z, b, a = self.project(hidden, layer, "dn_in")
        out = self.dn_core(qkv.contiguous(), z.contiguous(), a.contiguous(), b.contiguous(), layer, lc)
        return self.project(out, layer, "dn_out")[0]

    # -- QSA -------------------------------------------------------------------

    def _rope(self, cos, sin, n_pos: int):
        """Device (cos, sin) tables [n_pos, rope_dim] from the caller's, or our own."""
        if cos is not None and cos.is_cuda and cos.dtype == torch.float32 and cos.shape[-2] >= n_pos:
            c = cos[0] if cos.ndim == 3 else cos
            s = sin[0] if sin.ndim == 3 else sin
            return c.contiguous(), s.contiguous()
        if cos is not None and not cos.is_cuda:
            # the reference's forward hands the same host tables to every layer of
            # a step: copy them once. The cache holds the tables themselves, so
            # their storage cannot be reused by another tensor while it is kept,
            # and an in-place change bumps their version.
            key = (cos, sin, cos._version, sin._version, n_pos)
            if self._rope_copy is not None:
                k0 = self._rope_copy[0]
                if k0[0] is cos and k0[1] is sin and k0[2:] == key[2:]:
                    return self._rope_copy[1], self._rope_copy[2]
            c = (cos[0] if cos.ndim == 3 else cos)[:n_pos].to(self.device, torch.float32).contiguous()
            s = (sin[0] if sin.ndim == 3 else sin)[:n_pos].to(self.device, torch.float32).contiguous()
            self._rope_copy = (key, c, s)
            return c, s
        return self.rope.get(n_pos)

    def _sync_blocks(self, lc, g, cos_t, sin_t, upto_tokens: int, layer: int):
        """Pool any complete block of an imported history that has no pooled key yet."""
        ratio = self.config.indexer_compress_ratio
        n_complete = min(upto_tokens // ratio, lc.block_keys.shape[1])
        if n_complete > lc.blocks_valid:
            native.call("qm_qsa_pool_blocks", ctypes.byref(g), native.ptr(lc.raw_keys),
                        native.ptr(self._dw(layer, "indexer.k_norm.weight", torch.float32)), native.ptr(cos_t),
                        native.ptr(sin_t), lc.blocks_valid, n_complete - lc.blocks_valid, native.ptr(lc.block_keys),
                        native.stream_handle(self.device))
            lc.blocks_valid = n_complete

    def qsa_core(self, qg, k, v, iq, ik, layer: int, cache, query_offset: int, cos=None, sin=None, out=None,
                 attend: bool = True):
        """The HIP part of _full_attention: prep, select and attend on the projections.

        qg [B, S, Hq*2*d], k, v [B, S, Hkv*d], iq [B, S, idx_heads*idx_dim],
        ik [B, S, idx_dim] (act). Returns out [B, S, Hq*d] (act), or None when
        ``attend`` is False (indexer and cache update only).
        """
        c = self.config
        batch, seq = iq.shape[0], iq.shape[1]
        dt = iq.dtype
        lc = cache[layer]
        lc.ensure_qsa(batch, dt)
        if lc.raw_keys.dtype != dt:
            raise ValueError(f"activations are {dt} but the cache was built for {lc.raw_keys.dtype}")
        if query_offset + seq > cache.max_ctx:
            raise ValueError(f"context {query_offset + seq} exceeds the cache's {cache.max_ctx}")
        g = self.qsa_geom(cache, dt)
        cos_t, sin_t = self._rope(cos, sin, query_offset + seq)
        stream = native.stream_handle(self.device)
        self._sync_blocks(lc, g, cos_t, sin_t, query_offset, layer)
        pos = self._positions(batch, query_offset)
        # the query in the attention MFMA's operand order (hi and lo bf16 parts), per row
        q_out = torch.empty(batch, seq, 2 * c.num_attention_heads * c.head_dim, dtype=torch.bfloat16,
                            device=self.device) if qg is not None else None
        iq_out = torch.empty(batch, seq, c.indexer_heads, c.indexer_head_dim, dtype=torch.float32, device=self.device)
        lib = native.load()
        ids = torch.empty(batch, seq, c.block_topk, dtype=torch.int32, device=self.device)
        n_sel = torch.empty(batch, seq, dtype=torch.int32, device=self.device)
        chunked = seq > 1 and attend and self.chunk_attend_fits(cache)
        items = torch.empty(batch, seq, 2 * lib.qm_qsa_items_stride(ctypes.byref(g)), dtype=torch.int32,
                            device=self.device) if attend and not chunked else None
        norms = [native.ptr(self._dw(layer, n, torch.float32)) for n in
                 ("attn_q_norm.weight", "attn_k_norm.weight", "indexer.q_norm.weight", "indexer.k_norm.weight")]
        splits = lib.qm_qsa_decode_splits(ctypes.byref(g), query_offset) if seq == 1 else 0
        if (seq == 1 and qg is not None and k is not None and attend and self.fused_decode_fits(cache, query_offset)
                and self.decode_group_fits(splits, dt)):
            # decode: the whole QSA step in one qm_qsa_decode launch; its workspace
            # (generation words, flags, partials) is kept per layer and batch
            name = f"qsa_decode_{layer}_{batch}"
            ws = self._workspace(name, lib.qm_qsa_decode_workspace(ctypes.byref(g), splits))
            self._handoff[name] = ("qsa", g, splits)
            if out is None:
                out = torch.empty(batch, seq, c.num_attention_heads * c.head_dim, dtype=dt, device=self.device)
            native.call("qm_qsa_decode", ctypes.byref(g), native.ptr(qg), native.ptr(k), native.ptr(v),
                        native.ptr(iq), native.ptr(ik), *norms, native.ptr(cos_t), native.ptr(sin_t),
                        native.ptr(pos), native.ptr(lc.page_table), native.ptr(lc.k_pool), native.ptr(lc.v_pool),
                        native.ptr(lc.raw_keys), native.ptr(lc.block_keys), native.ptr(out), splits,
                        native.ptr(ws), ws.numel(), native.ptr(ids), native.ptr(n_sel), native.ptr(items),
                        native.ptr(iq_out), stream)
            lc.blocks_valid = max(lc.blocks_valid, (query_offset + seq) // c.indexer_compress_ratio)
            lc.n_tokens = query_offset + seq
            lc.last_ids, lc.last_n_sel, lc.last_iq, lc.last_q = ids, n_sel, iq_out, None
            return out
        # every other case: prep, then the selection, then the attention below
        native.call("qm_qsa_prep", ctypes.byref(g), seq, native.ptr(qg), native.ptr(k), native.ptr(v),
                    native.ptr(iq), native.ptr(ik), *norms, native.ptr(cos_t), native.ptr(sin_t),
                    native.ptr(pos), native.ptr(lc.page_table), native.ptr(lc.k_pool), native.ptr(lc.v_pool),
                    native.ptr(lc.raw_keys), native.ptr(lc.block_keys), native.ptr(q_out), native.ptr(iq_out),
                    stream)
        if chunked:
            # the chunk attention's own workspace per geometry: the entry
            # counts it keeps between calls are laid out by batch and block count
            chunk_ws = self._workspace(f"qsa_attend_chunk_{batch}_{cache.max_blocks}",
                                       lib.qm_qsa_attend_chunk_workspace(ctypes.byref(g), seq))
        if chunked and self.fuse_chunk_select:
            # the selection also files each row's blocks into that workspace
            # (one launch fewer per chunk)
            native.call("qm_qsa_select_chunk", ctypes.byref(g), seq, native.ptr(iq_out),
                        native.ptr(lc.block_keys), native.ptr(pos), native.ptr(ids), native.ptr(n_sel),
                        native.ptr(chunk_ws), chunk_ws.numel(), stream)
        else:
            # one row (a decode step past the one-launch kernel's range): a
            # score buffer makes qm_qsa_select spread the scores over the blocks
            scores = (self._workspace(f"qsa_scores_{batch}_{cache.max_blocks}", batch * cache.max_blocks * 4)
                      if seq == 1 else None)
            native.call("qm_qsa_select", ctypes.byref(g), seq, native.ptr(iq_out), native.ptr(lc.block_keys),
                        native.ptr(pos), native.ptr(lc.page_table), native.ptr(ids), native.ptr(n_sel),
                        native.ptr(items), native.ptr(scores), stream)
        lc.blocks_valid = max(lc.blocks_valid, (query_offset + seq) // c.indexer_compress_ratio)
        if k is not None:
            lc.n_tokens = query_offset + seq
        lc.last_ids, lc.last_n_sel, lc.last_iq, lc.last_q = ids, n_sel, iq_out, q_out
        if not attend:
            return None
        if chunked:
            # a chunk of rows: each selected key block is read once for all rows that attend it
            if out is None:
                out = torch.empty(batch, seq, c.num_attention_heads * c.head_dim, dtype=dt, device=self.device)
            if self.fuse_chunk_select:
                native.call("qm_qsa_attend_chunk_filed", ctypes.byref(g), seq, native.ptr(q_out), native.ptr(qg),
                            native.ptr(lc.k_pool), native.ptr(lc.v_pool), native.ptr(pos),
                            native.ptr(lc.page_table), native.ptr(out), native.ptr(chunk_ws), chunk_ws.numel(), stream)
            else:
                native.call("qm_qsa_attend_chunk", ctypes.byref(g), seq, native.ptr(q_out), native.ptr(qg),
                            native.ptr(lc.k_pool), native.ptr(lc.v_pool), native.ptr(pos),
                            native.ptr(lc.page_table), native.ptr(ids), native.ptr(n_sel), native.ptr(out),
                            native.ptr(chunk_ws), chunk_ws.numel(), stream)
            return out
        splits = lib.qm_qsa_attend_splits(ctypes.byref(g), query_offset, query_offset + seq - 1)
        ws = self._workspace("qsa_attend", lib.qm_qsa_attend_workspace(ctypes.byref(g), seq, splits))
        if out is None:
            out = torch.empty(batch, seq, c.num_attention_heads * c.head_dim, dtype=dt, device=self.device)
        native.call("qm_qsa_attend", ctypes.byref(g), seq, native.ptr(q_out), native.ptr(qg), native.ptr(lc.k_pool),
                    native.ptr(lc.v_pool), native.ptr(items), native.ptr(out), splits, native.ptr(ws), ws.numel(),
                    stream)
        return out

    def chunk_attend_fits(self, cache) -> bool:
        """Whether qm_qsa_attend_chunk covers this cache's geometry."""
        c = self.config
        return (c.indexer_compress_ratio in (32, 64) and cache.max_blocks <= 4096
                and cache.max_ctx <= 4096 * c.indexer_compress_ratio and c.block_topk <= 510)

    # Up to this many eligible blocks the one-launch decode is the faster path:
    # each of its workgroups scores and ranks every eligible block itself, so
    # its time grows with the context (cold, MI355X: 11.0 us at 127 blocks,
    # 25.3 at 511, 36.8 at 1023, 60.6 at 2047), while prep + the scores spread
    # over the blocks + the ranking + the attention stay near 28-35 us.
    FUSED_MAX_BLOCKS = 640

    def fused_decode_fits(self, cache, max_position=None) -> bool:
        """Whether qm_qsa_decode covers this cache's geometry (and, given a
        position, whether it is the faster path there)."""
        c = self.config
        fits = (cache.max_blocks <= 2048 and cache.max_pages <= 2048 and c.block_topk <= 256
                and c.indexer_compress_ratio <= 64)
        if max_position is not None:
            fits = fits and (max_position + 1) // c.indexer_compress_ratio <= self.FUSED_MAX_BLOCKS
        return fits

    def decode_group_fits(self, splits: int, dtype) -> bool:
        """Whether a qm_qsa_decode group of ``splits`` workgroups can be resident
        on the device at once (its workgroups wait for one another); larger
        plans go through prep + select + attend."""
        lib = native.load()
        resident = lib.qm_qsa_decode_resident(native.act_code(dtype), splits)
        if resident < 0:
            raise native.QmError(f"qm_qsa_decode_resident failed ({resident}): "
                                 f"{lib.qm_last_error().decode(errors='replace')}")
        return lib.qm_qsa_decode_fits(splits, resident) == 0

    def check_handoffs(self, reset: bool = True) -> None:
        """Read the hand-off counters of every decode workspace this model has
        used (a sync); raise QmError if a wait gave up or a position outran its
        plan since the last check (the affected outputs are NaN). ``reset``
        clears the counters and the hand-off words either way."""
        c = self.config
        faults = []
        for name, spec in self._handoff.items():
            ws = self._ws[name]
            if spec[0] == "dn":
                faults += native.dn_decode_faults(spec[1], c.linear_num_v_heads, c.linear_head_dim, ws, reset,
                                                  name, self.device)
            else:
                faults += native.qsa_decode_faults(spec[1], spec[2], ws, reset, name, self.device)
        if faults:
            raise native.QmError("decode hand-off failed: " + "; ".join(faults))

    def _full_attention(self, hidden, layer: int, cos, sin, cache, query_offset: int) -> torch.Tensor:
        """reference/model.py:331-383."""
        batch, seq, _ = hidden.shape
        dt = hidden.dtype
        if cache is None:
            cache = MixHybridCache(layer + 1, self.config, batch, max(query_offset + seq, 64), self.device, dt)
        qg, k, v, iq, ik = (t.contiguous() for t in self.project(hidden, layer, "qsa_in"))
        out = self.qsa_core(qg, k, v, iq, ik, layer, cache, query_offset, cos, sin)
        return self.project(out, layer, "qsa_out")[0]

    def selection_mask(self, lc, kv_len: int, query_offset: int) -> torch.Tensor:
        """Boolean (B, 1, S, kv_len) mask of the layer's last selection plus tails."""
        c = self.config
        ratio = c.indexer_compress_ratio
        ids, n_sel = lc.last_ids.long(), lc.last_n_sel.long()
        batch, seq, k = ids.shape
        # one spare column takes the unused ranks' writes, so every write to a
        # real column is True and duplicate indices cannot race
        mask = torch.zeros(batch, seq, kv_len + 1, dtype=torch.bool, device=self.device)
        valid = torch.arange(k, device=self.device)[None, None] < n_sel[..., None]
        tok = (ids[..., None] * ratio + torch.arange(ratio, device=self.device)).flatten(2)
        keep = valid[..., None].expand(-1, -1, -1, ratio).flatten(2)
        tok = torch.where(keep, tok, torch.full_like(tok, kv_len))
        mask.scatter_(2, tok, torch.ones_like(keep))
        mask = mask[..., :kv_len]
        qpos = torch.arange(seq, device=self.device) + query_offset
        tail_start = ((qpos + 1) // ratio) * ratio
        kpos = torch.arange(kv_len, device=self.device)
        tail = (kpos[None] >= tail_start[:, None]) & (kpos[None] <= qpos[:, None])
        return (mask | tail[None]).unsqueeze(1)

    def _indexer_mask(self, hidden, layer: int, cos, sin, cache, kv_len: int, query_offset: int) -> torch.Tensor:
        """reference/model.py:248-327: appends the raw indexer keys of ``hidden``,
        selects, and returns the boolean visibility mask."""
        batch, seq, _ = hidden.shape
        dt = hidden.dtype
        if cache is None:
            cache = MixHybridCache(layer + 1, self.config, batch, max(kv_len, 64), self.device, dt)
        iq = F.linear(hidden, self._dw(layer, "indexer.q_proj.weight", dt)).contiguous()
        ik = F.linear(hidden, self._dw(layer, "indexer.k_proj.weight", dt)).contiguous()
        lc = cache[layer]
        self.qsa_core(None, None, None, iq, ik, layer, cache, query_offset, cos, sin, attend=False)
        lc.n_tokens = max(lc.n_tokens, query_offset + seq)
        return self.selection_mask(lc, kv_len, query_offset)
