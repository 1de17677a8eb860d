"""The token-mixing half of a decode step over a stack of layers, replayable
from one HIP graph.

For one token per sequence, ``MixDecoder`` runs the attention half of every
decoder layer of the reference's forward pass (reference/model.py:443-452):

    mixed, hyper, inject = _gated_residual(hyper, layer, "attn")
    branch = _full_attention(mixed, ...)  or  _linear_attention(mixed, ...)
    hyper = _reinject(hyper, branch, inject)

Every buffer is bound at construction, so a step is a fixed sequence of kernel
launches -- per layer: the hyper-connection mix (two launches), the input
projections (one GEMV launch over the layer's concatenated weights), the mixer
core, and the output projection with the reinjection into the residual as its
epilogue (one launch) -- and it is captured once into a graph and replayed,
the MI355X analogue of the reference's traced decoder (tt/traced.py:156-314). The three things that make
that capture valid there hold here by construction:

* positions are device data: one int32 [B] tensor that every layer's kernels
  read, advanced by one inside the graph (tt/model.py:402-432 binds them as
  inputs for the same reason);
* the DeltaNet conv ring is phase-invariant: the kernels pick slot p % K from
  the device position, so a replay never sees a frozen ring phase (the
  reference needed ``trace_safe_rings``, tt/model.py:739-826);
* eligible-prefix bucketing (tt/model.py:117-129): the QSA decode sizes its
  split-K grid for a maximum position, so one graph is captured per
  power-of-two bucket of positions, on first use, and a step replays the
  graph of its position's bucket.

The host keeps only bookkeeping (each layer cache's token count and pooled
block count), advanced after each replay, so eager calls of the layer methods
can follow graph steps on the same cache. ``step_n`` runs k tokens of one
sequence through the same layers at once (the multi-row verify step of
tt/model.py:2135-2165), every per-token stage over k rows and the cores on
their chunk paths; ``step_n_graph`` replays the same kernels from one graph
per k (tt/traced.py:38-155), and ``snapshot`` / ``restore`` rewind the state
that accumulates unconditionally (the DeltaNet states and conv rings,
tt/model.py:2302-2360) so a verifier can commit only an accepted prefix.

The FFN half of each layer (the MoE) and the PLE injection are not part of
this path; callers run them between the layers' token-mixing halves when they
build a whole model.
"""

from __future__ import annotations

import ctypes

import torch

from . import native
from .plan import DnDecodePlan, QsaDecodePlan


class _LayerStep:
    """One layer's token-mixing half for B rows, every buffer bound."""

    def __init__(self, model, cache, layer: int, max_position: int, positions: torch.Tensor, dtype):
        c = model.config
        B = cache.batch
        dev = model.device
        lib = native.load()
        self.model, self.layer, self.dtype = model, layer, dtype
        self.is_qsa = c.is_full_attention(layer)
        self.act = native.act_code(dtype)
        self.rows = B
        # hyper-connection read gate
        self.norm_w, self.w_di, self.w_up, _ = model.hc_weights(layer, "attn", dtype)
        self.hc_geom = model.hc_geom(B, dtype)
        self.hc_ws = torch.zeros(lib.qm_hc_mix_workspace(ctypes.byref(self.hc_geom)), dtype=torch.uint8,
                                 device=dev)
        self.mixed = torch.empty(B, 1, c.hidden_size, dtype=dtype, device=dev)
        self.inject = torch.empty(B, 1, c.hc_count, dtype=dtype, device=dev)
        self.ri_geom = native.HcGeom(B, c.hc_count, c.hidden_size, 0, self.act, 0.0)
        self.hc = c.hc_count
        # projections
        g_in, g_out = ("qsa_in", "qsa_out") if self.is_qsa else ("dn_in", "dn_out")
        self.w_in, rows_in = model._wcat(layer, g_in, dtype)
        self.w_out, rows_out = model._wcat(layer, g_out, dtype)
        self.ins = [torch.empty(B, 1, r, dtype=dtype, device=dev) for r in rows_in]
        self.branch = torch.empty(B, 1, rows_out[0], dtype=dtype, device=dev)
        self.rows_in, self.rows_out = rows_in, rows_out
        self.gemv_in = model._gemv_fits(dtype, B, c.hidden_size)
        self.gemv_out = model._gemv_fits(dtype, B, int(self.w_out.shape[1]))
        self._seg_in = (ctypes.c_int * len(rows_in))(*rows_in)
        self._out_in = (ctypes.c_void_p * len(rows_in))(*[t.data_ptr() for t in self.ins])
        self._seg_out = (ctypes.c_int * 1)(rows_out[0])
        self._out_out = (ctypes.c_void_p * 1)(self.branch.data_ptr())
        # mixer core, reading the shared device positions
        if self.is_qsa:
            self.core = QsaDecodePlan(model, cache, layer, max_position, dtype)
        else:
            self.core = DnDecodePlan(model, cache, layer, dtype)
        self.core.positions = positions

    def _project(self, x, w, rows, outs, seg_rows, seg_out, use_gemv, stream):
        if use_gemv:
            native.call("qm_gemv", self.act, self.rows, int(w.shape[0]), int(w.shape[1]), w.data_ptr(),
                        x.data_ptr(), len(rows), seg_rows, seg_out, stream)
            return
        x2 = x.view(self.rows, -1)
        start = 0
        for r, o in zip(rows, outs):
            torch.matmul(x2, w[start:start + r].t(), out=o.view(self.rows, r))
            start += r

    def launch(self, hyper: torch.Tensor, stream: int):
        native.call("qm_hc_mix", ctypes.byref(self.hc_geom), hyper.data_ptr(), self.norm_w.data_ptr(),
                    self.w_di.data_ptr(), 1, self.w_up.data_ptr(), self.mixed.data_ptr(), self.inject.data_ptr(),
                    self.hc_ws.data_ptr(), self.hc_ws.numel(), stream)
        self._project(self.mixed, self.w_in, self.rows_in, self.ins, self._seg_in, self._out_in, self.gemv_in, stream)
        if self.is_qsa:
            qg, k, v, iq, ik = self.ins
            out = self.core.run(qg, k, v, iq, ik, stream)
        else:
            qkv, z, b, a = self.ins
            out = self.core.run(qkv, z, a, b, stream)
        if self.gemv_out:
            # the output projection with the reinjection as its epilogue
            native.call("qm_gemv_reinject", self.act, self.rows, self.rows_out[0], int(self.w_out.shape[1]),
                        self.w_out.data_ptr(), out.data_ptr(), self.hc, self.inject.data_ptr(), hyper.data_ptr(),
                        stream)
            return
        self._project(out, self.w_out, self.rows_out, [self.branch], self._seg_out, self._out_out, False, stream)
        native.call("qm_hc_reinject", ctypes.byref(self.ri_geom), hyper.data_ptr(), self.branch.data_ptr(),
                    self.inject.data_ptr(), hyper.data_ptr(), stream)


class _LayerStepN:
    """One layer's token-mixing half for k consecutive tokens of one sequence
    (the captured verify step), every buffer bound: the hyper-connection mix
    over k rows, the input projections (one GEMV launch up to 4 rows), the
    core on its chunk path at the device position (qm_dn_prefill, or
    qm_qsa_prep + qm_qsa_select_chunk + qm_qsa_attend_chunk_filed), and the
    output projection with the reinjection as its epilogue. The same kernels
    as the layer methods that MixDecoder.step_n calls, so a replay equals that
    eager pass bit for bit."""

    def __init__(self, model, cache, layer: int, k: int, positions: torch.Tensor, dtype):
        c = model.config
        dev = model.device
        lib = native.load()
        self.model, self.layer, self.dtype, self.k = model, layer, dtype, k
        self.is_qsa = c.is_full_attention(layer)
        self.act = native.act_code(dtype)
        self.positions = positions
        self.lc = cache[layer]
        # hyper-connection read gate over k rows
        self.norm_w, self.w_di, self.w_up, _ = model.hc_weights(layer, "attn", dtype)
        self.hc_geom = model.hc_geom(k, dtype)
        self.hc_ws = torch.zeros(lib.qm_hc_mix_workspace(ctypes.byref(self.hc_geom)), dtype=torch.uint8,
                                 device=dev)
        self.mixed = torch.empty(1, k, c.hidden_size, dtype=dtype, device=dev)
        self.inject = torch.empty(1, k, c.hc_count, dtype=dtype, device=dev)
        self.ri_geom = native.HcGeom(k, c.hc_count, c.hidden_size, 0, self.act, 0.0)
        self.hc = c.hc_count
        # projections
        g_in, g_out = ("qsa_in", "qsa_out") if self.is_qsa else ("dn_in", "dn_out")
        self.w_in, self.rows_in = model._wcat(layer, g_in, dtype)
        self.w_out, self.rows_out = model._wcat(layer, g_out, dtype)
        self.ins = [torch.empty(1, k, r, dtype=dtype, device=dev) for r in self.rows_in]
        self.branch = torch.empty(1, k, self.rows_out[0], dtype=dtype, device=dev)
        self.gemv_in = model._gemv_fits(dtype, k, c.hidden_size)
        self.gemv_out = model._gemv_fits(dtype, k, int(self.w_out.shape[1]))
        self._seg_in = (ctypes.c_int * len(self.rows_in))(*self.rows_in)
        self._out_in = (ctypes.c_void_p * len(self.rows_in))(*[t.data_ptr() for t in self.ins])
        self._seg_out = (ctypes.c_int * 1)(self.rows_out[0])
        self._out_out = (ctypes.c_void_p * 1)(self.branch.data_ptr())
        # the core on its chunk path, reading the shared device position
        if self.is_qsa:
            if not model.chunk_attend_fits(cache):
                raise native.QmError(f"layer {layer}: the chunk attention does not cover this cache's geometry")
            self.lc.ensure_qsa(1, dtype)
            self.geom = model.qsa_geom(cache, dtype)
            self.cos, self.sin = model.rope.get(cache.max_ctx)
            self.norms = [model._dw(layer, n, torch.float32) for n in
                          ("attn_q_norm.weight", "attn_k_norm.weight", "indexer.q_norm.weight",
                           "indexer.k_norm.weight")]
            self.q_out = torch.empty(1, k, 2 * c.num_attention_heads * c.head_dim, dtype=torch.bfloat16, device=dev)
            self.iq_out = torch.empty(1, k, c.indexer_heads, c.indexer_head_dim, dtype=torch.float32, device=dev)
            self.ids = torch.empty(1, k, c.block_topk, dtype=torch.int32, device=dev)
            self.n_sel = torch.empty(1, k, dtype=torch.int32, device=dev)
            self.chunk_ws = torch.zeros(lib.qm_qsa_attend_chunk_workspace(ctypes.byref(self.geom), k),
                                        dtype=torch.uint8, device=dev)
            self.out = torch.empty(1, k, c.num_attention_heads * c.head_dim, dtype=dtype, device=dev)
        else:
            self.lc.ensure_dn(1, dtype)
            self.geom = model.dn_geom(1, dtype)
            self.ws = torch.zeros(max(lib.qm_dn_prefill_workspace(ctypes.byref(self.geom), k), 256),
                                  dtype=torch.uint8, device=dev)
            self.w = {n: model._dw(layer, n, t) for n, t in (("ssm_a", torch.float32), ("ssm_dt.bias", torch.float32),
                                                              ("ssm_conv1d.weight", dtype),
                                                              ("ssm_norm.weight", torch.float32))}
            self.out = torch.empty(1, k, c.linear_value_dim, dtype=dtype, device=dev)

    def _project(self, x, w, rows, outs, seg_rows, seg_out, use_gemv, stream):
        if use_gemv:
            native.call("qm_gemv", self.act, self.k, int(w.shape[0]), int(w.shape[1]), w.data_ptr(),
                        x.data_ptr(), len(rows), seg_rows, seg_out, stream)
            return
        x2 = x.view(self.k, -1)
        start = 0
        for r, o in zip(rows, outs):
            torch.matmul(x2, w[start:start + r].t(), out=o.view(self.k, r))
            start += r

    def launch(self, hyper: torch.Tensor, stream: int):
        native.call("qm_hc_mix", ctypes.byref(self.hc_geom), hyper.data_ptr(), self.norm_w.data_ptr(),
                    self.w_di.data_ptr(), 1, self.w_up.data_ptr(), self.mixed.data_ptr(), self.inject.data_ptr(),
                    self.hc_ws.data_ptr(), self.hc_ws.numel(), stream)
        self._project(self.mixed, self.w_in, self.rows_in, self.ins, self._seg_in, self._out_in, self.gemv_in, stream)
        lc, k, pos = self.lc, self.k, self.positions.data_ptr()
        if self.is_qsa:
            qg, kk, v, iq, ik = self.ins
            g = ctypes.byref(self.geom)
            native.call("qm_qsa_prep", g, k, qg.data_ptr(), kk.data_ptr(), v.data_ptr(), iq.data_ptr(),
                        ik.data_ptr(), *[t.data_ptr() for t in self.norms], self.cos.data_ptr(), self.sin.data_ptr(),
                        pos, lc.page_table.data_ptr(), lc.k_pool.data_ptr(), lc.v_pool.data_ptr(),
                        lc.raw_keys.data_ptr(), lc.block_keys.data_ptr(), self.q_out.data_ptr(),
                        self.iq_out.data_ptr(), stream)
            native.call("qm_qsa_select_chunk", g, k, self.iq_out.data_ptr(), lc.block_keys.data_ptr(), pos,
                        self.ids.data_ptr(), self.n_sel.data_ptr(), self.chunk_ws.data_ptr(), self.chunk_ws.numel(),
                        stream)
            native.call("qm_qsa_attend_chunk_filed", g, k, self.q_out.data_ptr(), qg.data_ptr(),
                        lc.k_pool.data_ptr(), lc.v_pool.data_ptr(), pos, lc.page_table.data_ptr(),
                        self.out.data_ptr(), self.chunk_ws.data_ptr(), self.chunk_ws.numel(), stream)
        else:
            qkv, z, b, a = self.ins
            w = self.w
            native.call("qm_dn_prefill", ctypes.byref(self.geom), k, qkv.data_ptr(), z.data_ptr(), a.data_ptr(),
                        b.data_ptr(), w["ssm_a"].data_ptr(), w["ssm_dt.bias"].data_ptr(),
                        w["ssm_conv1d.weight"].data_ptr(), w["ssm_norm.weight"].data_ptr(), pos,
                        lc.conv_ring.data_ptr(), lc.recurrent_state.data_ptr(), self.out.data_ptr(),
                        self.ws.data_ptr(), self.ws.numel(), stream)
        if self.gemv_out:
            native.call("qm_gemv_reinject", self.act, self.k, self.rows_out[0], int(self.w_out.shape[1]),
                        self.w_out.data_ptr(), self.out.data_ptr(), self.hc, self.inject.data_ptr(),
                        hyper.data_ptr(), stream)
            return
        self._project(self.out, self.w_out, self.rows_out, [self.branch], self._seg_out, self._out_out, False, stream)
        native.call("qm_hc_reinject", ctypes.byref(self.ri_geom), hyper.data_ptr(), self.branch.data_ptr(),
                    self.inject.data_ptr(), hyper.data_ptr(), stream)


class MixDecoder:
    """The token-mixing halves of ``layers`` (default: every layer of the cache)
    for one token per sequence, eager (``step_eager``) or from a captured graph
    (``step``). ``hyper`` is the bound residual [B, 1, hc_count * hidden]: a
    step reads it and leaves the new residual in it.

    Rows may sit at different positions (continuous batching: ``positions``,
    one per row, default every row at the layers' common position). The
    kernels read each row's position from device memory; a step replays the
    graph of the largest position's bucket, and maps each row's next page
    first when the cache draws its pages from a pool."""

    def __init__(self, model, cache, layers=None, dtype=torch.bfloat16, min_bucket: int = 1024, positions=None,
                 check_every: int = 0):
        c = model.config
        self.model, self.cache, self.dtype = model, cache, dtype
        self.layers = list(range(len(cache.layers))) if layers is None else list(layers)
        if not self.layers:
            raise ValueError("MixDecoder needs at least one layer")
        if positions is None:
            starts = {cache[l].n_tokens for l in self.layers}
            if len(starts) != 1:
                raise ValueError(f"layers of the cache are at different positions: {sorted(starts)}")
            rows = [starts.pop()] * cache.batch
        else:
            rows = [int(p) for p in positions]
            if len(rows) != cache.batch or min(rows) < 0:
                raise ValueError(f"need {cache.batch} non-negative row positions, got {rows}")
        self.row_positions = rows
        self.position = max(rows)
        self.min_bucket = min_bucket
        dev = model.device
        self.hyper = torch.zeros(cache.batch, 1, c.hc_count * c.hidden_size, dtype=dtype, device=dev)
        self.positions = torch.tensor(rows, dtype=torch.int32, device=dev)
        self._steps = {}
        self._graphs = {}
        self._steps_n = {}      # k -> [_LayerStepN]: the captured verify step's layers
        self._graphs_n = {}     # k -> (graph, bound residual rows [1, k, hc_count * hidden])
        # every check_every steps (default 0: only when check_handoffs is
        # called) the decode kernels' hand-off counters are read back, which
        # synchronises the stream, and a fault raises QmError
        self.check_every = check_every
        self._since_check = 0

    # -- buckets of positions (tt/model.py:117-129) ---------------------------

    def bucket(self, position: int) -> int:
        """Largest position the step plans of ``position``'s bucket cover."""
        size = self.min_bucket
        while size <= position:
            size *= 2
        top = min(size, self.cache.max_ctx) - 1
        if position > top:
            raise ValueError(f"position {position} is beyond the cache ({self.cache.max_ctx} tokens)")
        return top

    def _layer_steps(self, bucket: int):
        steps = self._steps.get(bucket)
        if steps is None:
            steps = [_LayerStep(self.model, self.cache, l, bucket, self.positions, self.dtype) for l in self.layers]
            self._steps[bucket] = steps
        return steps

    # -- hand-off health ----------------------------------------------------------

    def check_handoffs(self, reset: bool = True) -> None:
        """Read every plan's hand-off counters (a sync) and raise QmError if a
        wait gave up or a position outran its plan since the last check."""
        faults = []
        for steps in self._steps.values():
            for st in steps:
                faults += st.core.check(reset)
        self._since_check = 0
        if faults:
            raise native.QmError("decode hand-off failed: " + "; ".join(faults))

    def _count_step(self):
        self._since_check += 1
        if self.check_every and self._since_check >= self.check_every:
            self.check_handoffs()

    # -- one step ----------------------------------------------------------------

    def _launch(self, steps, stream: int):
        for st in steps:
            st.launch(self.hyper, stream)
        self.positions.add_(1)

    def seek(self, positions) -> None:
        """Set every row's position (an int, or one per row) on the host, in
        the device tensor the graphs read, and in each layer cache's
        bookkeeping (``n_tokens`` becomes the largest row position, pooled
        blocks past it stop counting, ``slot_tokens`` follows the rows). The
        cache contents (pages, keys, states, rings) are not touched: a replay
        then runs at those positions (the bench repeats one position this way;
        a server rewinds a row it refilled). A rewind is always safe. A seek
        forward past the old ``n_tokens`` declares the history up to the new
        position present: the caller must have filled it (K/V pages, raw
        indexer keys), since the layer methods (``step_n``) then pool blocks
        from those raw keys and attend to those pages."""
        rows = [int(positions)] * len(self.row_positions) if isinstance(positions, int) else [int(p) for p in positions]
        if len(rows) != len(self.row_positions) or min(rows) < 0:
            raise ValueError(f"need {len(self.row_positions)} non-negative row positions, got {rows}")
        self.row_positions = rows
        self.position = max(rows)
        if isinstance(positions, int):
            self.positions.fill_(rows[0])          # a device fill, no host copy on the stream
        else:
            self.positions.copy_(torch.tensor(rows, dtype=torch.int32))
        # the layer caches' bookkeeping follows, so that the layer methods
        # (step_n) run every layer at the new position: the DeltaNet cores take
        # theirs from n_tokens, and no block past the position counts as pooled
        ratio = self.model.config.indexer_compress_ratio
        for l in self.layers:
            lc = self.cache[l]
            lc.n_tokens = self.position
            lc.blocks_valid = min(lc.blocks_valid, self.position // ratio)
        if len(self.cache.slot_tokens) == len(rows):
            self.cache.slot_tokens[:] = rows

    def _map_pages(self, n: int):
        """Pages for every row's next n tokens (a no-op for static tables)."""
        for slot, p in enumerate(self.row_positions):
            self.cache.ensure_capacity(slot, p + n)

    def _advance(self, n: int, host_only: bool):
        ratio = self.model.config.indexer_compress_ratio
        self.row_positions = [p + n for p in self.row_positions]
        self.position = max(self.row_positions)
        if host_only:
            return
        for l in self.layers:
            lc = self.cache[l]
            lc.n_tokens = self.position
            if self.model.config.is_full_attention(l):
                lc.blocks_valid = max(lc.blocks_valid, self.position // ratio)
        if len(self.cache.slot_tokens) == len(self.row_positions):
            for slot, p in enumerate(self.row_positions):
                self.cache.slot_tokens[slot] = p

    def _fill(self, hyper_in):
        if hyper_in is not None:
            self.hyper.copy_(hyper_in.reshape(self.hyper.shape))

    def step_eager(self, hyper_in=None) -> torch.Tensor:
        """One step by direct launches on the current stream."""
        self._fill(hyper_in)
        self._map_pages(1)
        steps = self._layer_steps(self.bucket(self.position))
        self._launch(steps, torch.cuda.current_stream(self.model.device).cuda_stream)
        self._advance(1, host_only=False)
        self._count_step()
        return self.hyper

    def graph(self, bucket: int) -> torch.cuda.CUDAGraph:
        """The captured step of ``bucket`` (captured on first use; capturing
        launches nothing, so the cache is untouched)."""
        g = self._graphs.get(bucket)
        if g is None:
            steps = self._layer_steps(bucket)
            if not all(st.gemv_in and st.gemv_out for st in steps):
                # the library GEMMs initialise their handles on first use: not inside a capture
                for st in steps:
                    st._project(st.mixed, st.w_in, st.rows_in, [torch.empty_like(t) for t in st.ins], None, None,
                                False, 0)
                torch.cuda.synchronize(self.model.device)
            g = torch.cuda.CUDAGraph()
            side = torch.cuda.Stream(self.model.device)
            side.wait_stream(torch.cuda.current_stream(self.model.device))
            with torch.cuda.stream(side):
                with torch.cuda.graph(g, stream=side):
                    self._launch(steps, side.cuda_stream)
            torch.cuda.current_stream(self.model.device).wait_stream(side)
            self._graphs[bucket] = g
        return g

    def step(self, hyper_in=None) -> torch.Tensor:
        """One step replayed from the graph of the largest row position's bucket."""
        self._fill(hyper_in)
        self._map_pages(1)
        self.graph(self.bucket(self.position)).replay()
        self._advance(1, host_only=False)
        self._count_step()
        return self.hyper

    # -- k tokens of one sequence (tt/model.py:2135-2165) ----------------------

    def step_n(self, hyper_rows: torch.Tensor) -> torch.Tensor:
        """k consecutive tokens of each sequence in one pass: hyper_rows
        [B, k, hc_count * hidden] -> the residual after the layers at all k
        positions. The per-token stages run over B*k rows; the cores run their
        chunk paths. The cache consumes all k tokens, and the bound residual
        is left holding the last row's. Every row must be at the same
        position (the layer methods take one)."""
        m = self.model
        h = hyper_rows.to(self.dtype).contiguous()
        k = h.shape[1]
        if len(set(self.row_positions)) != 1:
            raise ValueError(f"step_n needs every row at one position, not {self.row_positions}")
        if self.position + k > self.cache.max_ctx:
            raise ValueError(f"{k} tokens from position {self.position} overrun the cache")
        self._map_pages(k)
        for l in self.layers:
            mixed, _, inject = m._gated_residual(h, l, "attn")
            if m.config.is_full_attention(l):
                branch = m._full_attention(mixed, l, None, None, self.cache, self.position)
            else:
                branch = m._linear_attention(mixed, l, self.cache)
            h = m._reinject(h, branch, inject)
        self.hyper.copy_(h[:, -1:])
        self.positions.add_(k)
        self._advance(k, host_only=True)   # the layer methods advanced the caches
        return h

    # -- the captured k-token verify step (tt/traced.py:38-155) ----------------

    def _layer_steps_n(self, k: int):
        steps = self._steps_n.get(k)
        if steps is None:
            steps = [_LayerStepN(self.model, self.cache, l, k, self.positions, self.dtype) for l in self.layers]
            self._steps_n[k] = steps
        return steps

    def graph_n(self, k: int):
        """(graph, bound residual rows) of the k-token verify step, captured on
        first use. One capture per k: k is a shape (the rows of every
        per-token stage), the position is device data, and the graph advances
        the device position by k."""
        hit = self._graphs_n.get(k)
        if hit is None:
            if self.cache.batch != 1:
                raise ValueError("the verify step is single-sequence")
            steps = self._layer_steps_n(k)
            c = self.model.config
            rows = torch.zeros(1, k, c.hc_count * c.hidden_size, dtype=self.dtype, device=self.model.device)
            if not all(st.gemv_in and st.gemv_out for st in steps):
                # the library GEMMs initialise their handles on first use: not inside a capture
                for st in steps:
                    st._project(st.mixed, st.w_in, st.rows_in, [torch.empty_like(t) for t in st.ins], None, None,
                                False, 0)
                torch.cuda.synchronize(self.model.device)
            g = torch.cuda.CUDAGraph()
            side = torch.cuda.Stream(self.model.device)
            side.wait_stream(torch.cuda.current_stream(self.model.device))
            with torch.cuda.stream(side):
                with torch.cuda.graph(g, stream=side):
                    for st in steps:
                        st.launch(rows, side.cuda_stream)
                    self.positions.add_(k)
            torch.cuda.current_stream(self.model.device).wait_stream(side)
            hit = (g, rows)
            self._graphs_n[k] = hit
        return hit

    def step_n_graph(self, hyper_rows: torch.Tensor) -> torch.Tensor:
        """``step_n`` replayed from its graph: hyper_rows [1, k, hc_count *
        hidden] -> the residual rows after the layers at the k positions (the
        bound buffer of the graph, valid until the next replay of this k). The
        same kernels as ``step_n``, so the same bits. The cache consumes all k
        tokens; to commit a prefix, ``snapshot`` before and ``restore`` after,
        then replay the accepted tokens."""
        k = hyper_rows.shape[1]
        if self.cache.batch != 1 or hyper_rows.shape[0] != 1:
            raise ValueError("the verify step is single-sequence")
        if self.position + k > self.cache.max_ctx:
            raise ValueError(f"{k} tokens from position {self.position} overrun the cache")
        self._map_pages(k)
        g, rows = self.graph_n(k)
        rows.copy_(hyper_rows.reshape(rows.shape))
        g.replay()
        self.hyper.copy_(rows[:, -1:])     # the last row's residual, as step_n leaves it
        self._advance(k, host_only=False)
        return rows

    # -- snapshot and restore for speculation (tt/model.py:2302-2360) ----------

    def snapshot(self, into: dict | None = None) -> dict:
        """Copy everything that accumulates unconditionally, for a later
        rewind: each DeltaNet layer's recurrent state and conv ring, the bound
        residual, the device positions, and the host bookkeeping (row
        positions, each layer's token and pooled-block counts, the slots'
        token counts). Pass a previous snapshot as ``into`` to reuse its
        buffers (no allocation). K/V pages and raw or pooled indexer keys are
        not copied: attention reads only up to the position, and a block a
        rejected token completed is pooled again when a token completes it."""
        snap = into if into is not None else {"tensors": {}}
        held = snap["tensors"]

        def take(name, t):
            dst = held.get(name)
            if dst is None or dst.shape != t.shape or dst.dtype != t.dtype:
                dst = torch.empty_like(t)
                held[name] = dst
            dst.copy_(t)

        for l in self.layers:
            lc = self.cache[l]
            if lc.recurrent_state is not None:
                take(f"{l}.recurrent_state", lc.recurrent_state)
            if lc.conv_ring is not None:
                take(f"{l}.conv_ring", lc.conv_ring)
        take("hyper", self.hyper)
        take("positions", self.positions)
        snap["rows"] = list(self.row_positions)
        snap["layers"] = {l: (self.cache[l].n_tokens, self.cache[l].blocks_valid) for l in self.layers}
        snap["slot_tokens"] = list(self.cache.slot_tokens)
        return snap

    def restore(self, snap: dict) -> None:
        """Rewind to a snapshot, in place: every bound buffer keeps its
        address, so the captured graphs stay valid. Pages mapped from a pool
        for the rejected tokens stay mapped to the slot (the next tokens use
        them)."""
        held = snap["tensors"]
        for l in self.layers:
            lc = self.cache[l]
            for f in ("recurrent_state", "conv_ring"):
                t = getattr(lc, f)
                if t is not None:
                    t.copy_(held[f"{l}.{f}"])
            lc.n_tokens, lc.blocks_valid = snap["layers"][l]
        self.hyper.copy_(held["hyper"])
        self.positions.copy_(held["positions"])
        self.row_positions = list(snap["rows"])
        self.position = max(self.row_positions)
        self.cache.slot_tokens[:] = snap["slot_tokens"]

    # -- rewind ------------------------------------------------------------------

    def reset(self) -> None:
        """Back to position 0 with every buffer at its bound address (the graphs
        stay valid): state, rings, pools and keys cleared in place."""
        for l in self.layers:
            lc = self.cache[l]
            for t in (lc.conv_ring, lc.recurrent_state, lc.k_pool, lc.v_pool, lc.raw_keys, lc.block_keys):
                if t is not None:
                    t.zero_()
            lc.n_tokens = 0
            lc.blocks_valid = 0
        self.hyper.zero_()
        self.positions.zero_()
        self.row_positions = [0] * len(self.row_positions)
        self.position = 0
        if len(self.cache.slot_tokens) == len(self.row_positions):
            self.cache.slot_tokens[:] = self.row_positions
