"""Exclusive fixed-active-set decode with persistent buffers and hipGraph replay.

Drop-in for src/moba_opt/prepared_decode.py:1-204 (same constructor
arguments, ``step`` / ``attend`` / ``capture`` / ``close``, context-manager use,
lifecycle errors and the aliasing rule that outputs are persistent workspaces
overwritten by the next call).

One step is ONE call of decode_fused: a fused kernel (page-table delta,
positions, route, stable top-k, paged attention into split partials, scatter
of the new token, closing-chunk mean) and the split merge (output, LSE,
length advance), when the shape allows (Hq/Hkv <= 16, head_dim a multiple of
8); otherwise the fixed sequence
    decode_step (page-table delta + positions + scatter + closing-chunk mean)
    -> decode_route (scores + stable top-k + slot list + work list)
    -> paged_attention (+ its slot combine).
Either way the work is on the cache's stream and can be captured once as a
graph (``torch.cuda.graph`` records HIP graphs on ROCm).
Host work per step is O(active batch) planning plus, only when a row starts a
new page, one synchronous 2 x B int32 upload of the page-table delta.
Every kernel of the sequence is from libmoba_hip.so; none issues a memset, so
graph replays are self-contained.  Routing is always the deterministic stable
rule (descending score, ties -> lowest chunk), so ``stable_routes`` only
documents the behaviour.
"""
from __future__ import annotations

import contextlib

import torch

from .cache_layout import IncrementalLayout, positive_int
from .kv_cache import DecodeResult, _ints, _mode
from .ops import decode as kernels


class PreparedDecode:
    def __init__(self, cache, sequence_ids, num_q_heads, *, topk=4, mode="moba",
                 check_finite=True, stable_routes=False):
        with cache._lock, torch.cuda.device(cache.device):
            cache._check_stream()
            self.num_q_heads = positive_int(num_q_heads, "num_q_heads")
            if self.num_q_heads % cache.num_kv_heads:
                raise ValueError("Hq must be a multiple of Hkv")
            if not isinstance(check_finite, bool):
                raise ValueError("check_finite must be bool")
            if not isinstance(stable_routes, bool):
                raise ValueError("stable_routes must be bool")
            self.stable_routes = stable_routes
            self.dense = _mode(mode, topk)
            self.cache = cache
            self._dev_index = torch.device(cache.device).index
            if self._dev_index is None:
                self._dev_index = torch.cuda.current_device()
            self._state = IncrementalLayout(cache._layout, _ints(sequence_ids, "sequence_ids"))
            self.ids = self._state.ids
            b, h, d = len(self.ids), self.num_q_heads, cache.head_dim
            C, max_len = cache.chunk_size, cache._layout.max_seq_len
            width = max(1, (max_len - 1) // C)
            if b * h * width >= 2 ** 31:
                raise ValueError("route score grid exceeds int32 capacity")
            self.remote = 0 if self.dense else min(topk - 1, (max_len - 1) // C)
            self.max_chunks = -(-max_len // C)
            self.check_finite = check_finite
            self.closed = False
            self.failed = False
            self._graphs = {}
            self.delta_uploads = 0
            kw = dict(device=cache.device, dtype=cache.dtype)
            dev = cache.device
            self.q = torch.zeros((b, h, d), **kw)
            self.k = torch.zeros((b, cache.num_kv_heads, d), **kw)
            self.v = torch.zeros_like(self.k)
            self.output = torch.empty_like(self.q)
            self.lse = torch.empty((b, h), device=dev, dtype=torch.float32)
            self.scores = torch.empty((b, h, width), device=dev, dtype=torch.float32)
            self._work = kernels.RouteWork(b, h, cache.num_kv_heads, self.remote, dev)
            self.selected = self._work.selected
            nslot = self.max_chunks if self.dense else self.remote + 1
            n = b * h * nslot
            self._part_o = torch.empty((n, d), device=dev, dtype=torch.float32)
            self._part_ml = torch.empty((n, 2), device=dev, dtype=torch.float32)
            # one-launch step (route + attention + append) when the shape allows
            # split counts per row follow each row's expected attended tokens
            self._fused = (kernels.FusedWork(b, h, cache.num_kv_heads, d, dev, scheduled=True)
                           if kernels.fused_supported(h, cache.num_kv_heads, d, width, cache._table.shape[1]) else None)
            self._sched_pos = None
            self._fused_args = None
            self.gpu_ids = torch.tensor(self.ids, device=dev, dtype=torch.int32)
            self.positions = torch.empty(b, device=dev, dtype=torch.int32)
            self.delta = torch.full((2, b), -1, device=dev, dtype=torch.int32)
            self.delta_host = torch.empty((2, b), dtype=torch.int32, pin_memory=True)
            if self._fused is not None:  # every launch reads a valid schedule
                self._schedule([self._state.lengths[s] for s in self.ids])
            table, lengths = cache._table.clone(), cache._lengths.clone()
            # publish the exclusive lease only after every allocation succeeded
            cache._table, cache._lengths = table, lengths
            cache._prepared_owner = self

    @property
    def lengths(self):
        with self.cache._lock:
            return tuple(self._state.lengths)

    @property
    def page_table(self):
        with self.cache._lock:
            return tuple(map(tuple, self._state.tables))

    def _check(self):
        """Lifecycle and stream checks; returns the (current) cache stream."""
        if self.closed or self.cache._prepared_owner is not self:
            raise ValueError("prepared decode is closed or no longer owns cache")
        if self.failed:
            raise RuntimeError("CUDA execution failed; discard prepared decode and cache")
        if torch.cuda.is_current_stream_capturing():
            raise ValueError("use capture(), not external capture")
        stream = torch.cuda.current_stream(self.cache.device).cuda_stream
        if stream != self.cache._stream:
            raise ValueError("cross-stream cache access is unsupported")
        return stream

    def _device(self):
        """The cache's device as the current device (no switch when it is)."""
        if torch.cuda.current_device() == self._dev_index:
            return contextlib.nullcontext()
        return torch.cuda.device(self.cache.device)

    def _input(self, tensor, target, name):
        if tensor is target:  # the persistent workspace itself: shape/dtype/storage hold
            if self.check_finite and not bool(torch.isfinite(tensor).all()):
                raise ValueError(f"{name} contains NaN/Inf")
            return
        if not isinstance(tensor, torch.Tensor) or tensor.shape != target.shape:
            raise ValueError(f"{name} must have fixed shape {tuple(target.shape)}")
        if tensor.device != target.device or tensor.dtype != target.dtype \
                or not tensor.is_contiguous():
            raise ValueError(f"{name} must match device/dtype and be contiguous")
        if tensor.requires_grad:
            raise ValueError("prepared decode is inference-only")
        self.cache._reject_storage_alias(tensor)
        workspaces = {x.untyped_storage().data_ptr() for x in (self.q, self.k, self.v)}
        if tensor is not target and tensor.untyped_storage().data_ptr() in workspaces:
            raise ValueError("input aliases another prepared workspace; clone first")
        if self.check_finite and not bool(torch.isfinite(tensor).all()):
            raise ValueError(f"{name} contains NaN/Inf")

    def _upload(self, plan):
        if not plan.updates:
            return
        self.delta_host.fill_(-1)
        row_of = {sid: i for i, sid in enumerate(self.ids)}
        for sid, logical, physical in plan.updates:
            r = row_of[sid]
            self.delta_host[0, r] = logical
            self.delta_host[1, r] = physical
        # synchronous tiny H2D: the pinned buffer is reused next step
        self.delta.copy_(self.delta_host, non_blocking=False)
        self.delta_uploads += 1

    def _schedule(self, positions):
        """Refreshes the fused launch's split schedule when some row's
        position moved by more than 1/8 since the last upload."""
        if self._fused is None:
            return
        old = self._sched_pos
        if old is not None and all(abs(p - o) * 8 <= max(o, 1) for p, o in zip(positions, old)):
            return
        c = self.cache
        entries, splits, _ = kernels.fused_schedule(
            positions, c.num_kv_heads, self.num_q_heads // c.num_kv_heads, self.remote,
            c.chunk_size, self.dense, max_splits=self._fused.splits)
        if splits != self._fused.sched_splits:
            self._fused.set_schedule(entries, splits)
        self._sched_pos = list(positions)

    def _compute(self, append, stream=None):
        c = self.cache
        if self._fused is not None:
            if self._fused_args is None:  # every pointer is a persistent workspace
                self._fused_args = {
                    mode: kernels.FusedLauncher(kernels.fused_args(
                        self.q, self.k if mode == 2 else None, self.v if mode == 2 else None,
                        c.k_cache, c.v_cache, c._table, c._lengths, self.gpu_ids,
                        self.positions, self.delta, c._means, c.chunk_size,
                        self.scores.shape[-1], self.remote, self.dense, mode,
                        None if self.dense else self.selected, self._fused, self.output,
                        self.lse))
                    for mode in (1, 2)}
            if stream is None:
                stream = torch.cuda.current_stream(c.device).cuda_stream
            self._fused_args[2 if append else 1](stream)
            return
        if append:  # metadata + scatter + closing-chunk mean in one launch
            kernels.step(c._table, c._lengths, self.gpu_ids, self.positions, self.delta, self.k,
                         self.v, c.k_cache, c.v_cache, c.chunk_size, c._means)
        else:
            kernels.metadata(c._table, c._lengths, self.gpu_ids, self.positions, self.delta,
                             False)
        if not self.dense:
            kernels.route(self.q, c._means, self.gpu_ids, self.positions, c.chunk_size,
                          self.scores.shape[-1], self.remote, self.scores, self._work)
        kernels.attention(self.q, c.k_cache, c.v_cache, c._table, c._lengths, self.gpu_ids,
                          self.positions, self._work, self.output, self.lse, c.chunk_size,
                          self.dense, self.max_chunks, self._part_o, self._part_ml)

    def _run(self, kind, use_graph, stream):
        try:
            if use_graph:
                self._graphs[kind].replay()
            else:
                self._compute(kind == "step", stream)
        except Exception:
            self.failed = True
            raise

    def _result(self, positions):
        return DecodeResult(self.output, self.lse, None if self.dense else self.selected,
                            self.ids, positions)

    def attend(self, q, *, use_graph=False):
        # no autograd: inputs that require grad are rejected and every op
        # here is an in-place copy or a library launch
        with self.cache._lock, self._device():
            stream = self._check()
            self._input(q, self.q, "q")
            pos = tuple(self._state.lengths[s] - 1 for s in self.ids)
            if min(pos) < 0:
                raise ValueError("query positions must refer to cached tokens")
            if use_graph and "attend" not in self._graphs:
                raise ValueError("capture('attend') first")
            if q is not self.q:
                self.q.copy_(q)
            self._schedule(pos)
            self._run("attend", use_graph, stream)
            return self._result(pos)

    def step(self, q, k, v, *, use_graph=False):
        """One token per fixed active row; validation/capacity errors change nothing."""
        with self.cache._lock, self._device():
            stream = self._check()
            for tensor, target, name in ((q, self.q, "q"), (k, self.k, "k"), (v, self.v, "v")):
                self._input(tensor, target, name)
            if use_graph and "step" not in self._graphs:
                raise ValueError("capture('step') first")
            plan = self._state.plan()
            for tensor, target in ((q, self.q), (k, self.k), (v, self.v)):
                if tensor is not target:
                    target.copy_(tensor)
            self._upload(plan)
            self._schedule(plan.positions)
            self._run("step", use_graph, stream)
            self._state.commit(plan)
            return self._result(plan.positions)

    @torch.no_grad()
    def capture(self, kind="step"):
        """Capture the device work of one step/attend; visible state is restored."""
        if kind not in ("step", "attend"):
            raise ValueError("kind must be step or attend")
        c = self.cache
        with c._lock, torch.cuda.device(c.device):
            self._check()
            if kind in self._graphs:
                raise ValueError("graph already captured")
            plan = self._state.plan() if kind == "step" else None
            if kind == "attend" and any(self._state.lengths[s] == 0 for s in self.ids):
                raise ValueError("attend capture requires nonempty cached sequences")
            snapshots = [t.clone() for t in (c._table, c._lengths, c._means, self.delta)]
            uploads = self.delta_uploads
            main = torch.cuda.current_stream(c.device)
            side = torch.cuda.Stream(device=c.device)
            side.wait_stream(main)
            try:
                if plan is not None:
                    self._upload(plan)
                self._schedule(plan.positions if plan is not None
                               else [self._state.lengths[s] - 1 for s in self.ids])
                side.wait_stream(main)
                with torch.cuda.stream(side):
                    for _ in range(2):  # warm-up outside the graph
                        self._compute(kind == "step")
                        c._lengths.copy_(snapshots[1])
                main.wait_stream(side)
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=side):
                    self._compute(kind == "step")
                self._graphs[kind] = graph
            finally:
                main.wait_stream(side)
                for target, snap in zip((c._table, c._lengths, c._means, self.delta), snapshots):
                    target.copy_(snap)
                self.delta_uploads = uploads
            return self

    def close(self):
        if self.closed:
            return
        c = self.cache
        with c._lock, torch.cuda.device(c.device):
            if c._prepared_owner is not self:
                raise ValueError("prepared ownership lost")
            if torch.cuda.current_stream(c.device).cuda_stream != c._stream:
                raise ValueError("cross-stream cache access is unsupported")
            if self.failed:
                c._invalid = True
            else:
                self._state.publish(c._layout)
                c._candidate_count = c._count_candidates(self._state.lengths)
            c._prepared_owner = None
            self._graphs.clear()
            self.closed = True

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
