"""Exclusive fixed-active-set decode: persistent device buffers, a native
step driver and hipGraph replay.

API of src/moba_opt/prepared_decode.py:1-204 (constructor arguments,
``step`` / ``attend`` / ``capture`` / ``close``, context-manager use, the
lifecycle errors, and outputs that are persistent buffers overwritten by the
next call).

Division of work:

* this module checks arguments, owns the device buffers (torch tensors) and
  copies caller inputs into the bound input buffers;
* the driver in libmoba_hip.so (``moba_prep_*``) does each call's host work in
  native code: it plans the token on a page-pool lease, stages the page-table
  delta through pinned memory when a row starts a page, keeps the fused
  kernel's split schedule current, launches the step (or replays its
  hipGraph) and commits the plan;
* a step is one ``moba_hip_decode_fused`` call (two launches: route +
  attention + scatter + closing-chunk mean, then the split merge) where the
  shape allows, else the multi-kernel sequence step -> route -> paged
  attention.

Routing is always the stable rule (score descending, ties to the lowest
chunk), so ``stable_routes`` only documents the behaviour.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import decode_contract as contract
from .baseline_adapter import _require
from .cache_layout import IncrementalLayout, positive_int
from .kv_cache import DecodeResult
from .ops import _lib
from .ops import decode as kernels


class _Desc(ctypes.Structure):
    """MobaPrepDesc of include/moba_hip.h."""
    _fields_ = ([(n, ctypes.c_int) for n in
                 ("dtype", "rows", "hq", "hkv", "head_dim", "page_size", "table_width",
                  "max_chunks", "chunk", "width", "remote", "dense", "fused", "splits",
                  "n_sched")]
                + [(n, ctypes.c_void_p) for n in
                   ("lease", "q", "k", "v", "k_cache", "v_cache", "table", "lengths", "ids_dev",
                    "positions", "delta", "means", "selected", "scores", "items",
                    "item_counts", "part_o", "part_ml", "out", "lse", "sched")])


def _raw_stream(index):
    """The current stream's handle on device `index` (the raw query torch's
    own stream object wraps)."""
    return torch._C._cuda_getCurrentRawStream(index)


class _SlotPartials:
    """Per-slot partials of the multi-kernel path (no split schedule)."""
    splits, sched, n_sched = 1, None, 0

    def __init__(self, n, d, device):
        self.part_o = torch.empty((n, d), device=device, dtype=torch.float32)
        self.part_ml = torch.empty((n, 2), device=device, dtype=torch.float32)


class PreparedDecode:
    def __init__(self, cache, sequence_ids, num_q_heads, *, topk=4, mode="moba",
                 check_finite=True, stable_routes=False):
        with cache._lock, torch.cuda.device(cache.device):
            cache._guard()
            self.num_q_heads = positive_int(num_q_heads, "num_q_heads")
            _require([
                (lambda: self.num_q_heads % cache.num_kv_heads == 0,
                 "Hq must be a multiple of Hkv"),
                (lambda: isinstance(check_finite, bool), "check_finite must be bool"),
                (lambda: isinstance(stable_routes, bool), "stable_routes must be bool"),
            ])
            self.dense = contract.decode_mode(mode, topk)
            self.check_finite, self.stable_routes = check_finite, stable_routes
            self.cache = cache
            self._dev = cache.device.index
            self._lease = IncrementalLayout(cache._layout,
                                            contract.int_vector(sequence_ids, "sequence_ids"))
            self.ids = self._lease.ids
            rows, hq, hkv, d = len(self.ids), self.num_q_heads, cache.num_kv_heads, cache.head_dim
            layout, C = cache._layout, cache.chunk_size
            width = max(1, (layout.max_seq_len - 1) // C)   # closed chunks of a full row
            _require([(lambda: rows * hq * width < 2 ** 31,
                       "route score grid exceeds int32 capacity")])
            self.remote = 0 if self.dense else min(topk - 1, width)
            self._buffers(rows, hq, hkv, d, width)
            self._positions = np.empty(rows, np.int32)
            self._handle = None
            self._handle = self._make_driver(rows, hq, hkv, d, width)
            self.closed = self.failed = False
            self._captured = set()
            cache._lessee = self   # the lease starts once everything above succeeded

    # ------------------------------------------------------------ buffers
    def _buffers(self, rows, hq, hkv, d, width):
        c = self.cache
        dev, dt = c.device, c.dtype
        self.q = torch.zeros((rows, hq, d), device=dev, dtype=dt)
        self.k = torch.zeros((rows, hkv, d), device=dev, dtype=dt)
        self.v = torch.zeros_like(self.k)
        self.output = torch.empty_like(self.q)
        self.lse = torch.empty((rows, hq), device=dev, dtype=torch.float32)
        self.scores = torch.empty((rows, hq, width), device=dev, dtype=torch.float32)
        self.gpu_ids = torch.tensor(self.ids, device=dev, dtype=torch.int32)
        self.positions = torch.empty(rows, device=dev, dtype=torch.int32)
        self.delta = torch.full((2, rows), -1, device=dev, dtype=torch.int32)
        self._route = kernels.RouteWork(rows, hq, hkv, self.remote, dev)
        self.selected = self._route.selected
        self.fused = kernels.fused_supported(hq, hkv, d, width, c._table.shape[1])
        if self.fused:  # split partials + device schedule of the fused launch
            self._work = kernels.FusedWork(rows, hq, hkv, d, dev, scheduled=True)
        else:           # slot partials of the multi-kernel path
            nslot = -(-c._layout.max_seq_len // c.chunk_size) if self.dense else self.remote + 1
            self._work = _SlotPartials(rows * hq * nslot, d, dev)

    def _make_driver(self, rows, hq, hkv, d, width):
        c, w = self.cache, self._work
        ptr = _lib.ptr
        desc = _Desc(
            dtype=kernels.DTYPE_CODE[c.dtype], rows=rows, hq=hq, hkv=hkv, head_dim=d,
            page_size=c._layout.page_size, table_width=c._table.shape[1],
            max_chunks=c._means.shape[1], chunk=c.chunk_size, width=width, remote=self.remote,
            dense=int(self.dense), fused=int(self.fused), splits=w.splits, n_sched=w.n_sched,
            lease=self._lease.handle, q=ptr(self.q), k=ptr(self.k), v=ptr(self.v),
            k_cache=ptr(c.k_cache), v_cache=ptr(c.v_cache), table=ptr(c._table),
            lengths=ptr(c._lengths), ids_dev=ptr(self.gpu_ids), positions=ptr(self.positions),
            delta=ptr(self.delta), means=ptr(c._means),
            selected=None if self.dense else ptr(self.selected), scores=ptr(self.scores),
            items=ptr(self._route.items), item_counts=ptr(self._route.counts),
            part_o=ptr(w.part_o), part_ml=ptr(w.part_ml), out=ptr(self.output),
            lse=ptr(self.lse), sched=ptr(w.sched))
        self._desc = desc
        return self._create(desc)

    def _create(self, desc):
        ids = np.asarray(self.ids, np.int32)
        h = ctypes.c_void_p()
        lib = _lib.load()
        if lib.moba_prep_create(ctypes.byref(desc), ids.ctypes.data, ctypes.byref(h)):
            raise _lib.MobaHipError(lib.moba_hip_last_error().decode(errors="replace"))
        return h.value

    # ---------------------------------------------------------- snapshots
    @property
    def lengths(self):
        with self.cache._lock:
            return tuple(self._lease.lengths)

    @property
    def page_table(self):
        with self.cache._lock:
            return tuple(map(tuple, self._lease.tables))

    @property
    def delta_uploads(self):
        return int(_lib.load().moba_prep_delta_uploads(self._handle))

    # ------------------------------------------------------------- checks
    def _usable(self):
        """Lifecycle and stream checks; returns the cache stream.  (Plain
        tests: this runs on every step, whose host time bounds graph
        replays.)"""
        c = self.cache
        if self.closed or c._lessee is not self:
            raise ValueError("prepared decode is closed or no longer owns cache")
        if self.failed:
            raise RuntimeError("CUDA execution failed; discard prepared decode and cache")
        stream = _raw_stream(self._dev)
        if torch.cuda.is_current_stream_capturing():
            raise ValueError("use capture(), not external capture")
        if stream != c._stream:
            raise ValueError("cross-stream cache access is unsupported")
        return stream

    def _bind(self, given, buffer, name):
        """Checks a caller input against its bound buffer; True when it must
        be copied in (it is not the buffer itself)."""
        if given is not buffer:
            _require([
                (lambda: isinstance(given, torch.Tensor) and given.shape == buffer.shape,
                 f"{name} must have fixed shape {tuple(buffer.shape)}"),
                (lambda: given.device == buffer.device and given.dtype == buffer.dtype
                 and given.is_contiguous(), f"{name} must match device/dtype and be contiguous"),
                (lambda: not given.requires_grad, "prepared decode is inference-only"),
            ])
            self.cache._no_pool_alias(given)
            own = {t.untyped_storage().data_ptr() for t in (self.q, self.k, self.v)}
            _require([(lambda: given.untyped_storage().data_ptr() not in own,
                       "input aliases another prepared workspace; clone first")])
        return given is not buffer

    def _bind_all(self, specs):
        """`_bind` for each (given, buffer, name) in order, then the NaN/Inf
        test of all of them through one flag (one host synchronisation, not
        one per input).  Raises what binding and testing each input in turn
        would raise first.  Returns the (given, buffer) pairs to copy."""
        copies = []
        for i, (t, b, n) in enumerate(specs):
            try:
                if self._bind(t, b, n):
                    copies.append((t, b))
            except ValueError:
                if self.check_finite:  # an earlier input's NaN/Inf comes first
                    for t0, _, n0 in specs[:i]:
                        contract.finite(t0, n0)
                raise
        if self.check_finite and (len(specs) == 1 or not bool(
                torch.stack([torch.isfinite(t).all() for t, _, _ in specs]).all())):
            for t, _, n in specs:
                contract.finite(t, n)
        return copies

    # ---------------------------------------------------------------- run
    def _run(self, append, use_graph, stream):
        lib = _lib.load()
        rc = lib.moba_prep_run(self._handle, int(append), int(use_graph), stream,
                               self._positions.ctypes.data)
        if rc == 0:
            return tuple(self._positions.tolist())
        msg = lib.moba_hip_last_error().decode(errors="replace")
        if rc == _lib.MOBA_ERR_ARG:   # input errors change nothing
            raise ValueError(msg)
        self.failed = True
        raise _lib.MobaHipError(msg)

    # parts of a step for a caller that sequences several layers' launches
    # on one stream or in one captured graph (moba_hip.qwen2): plan (host
    # work, before the launches), launch (device work, capturable), commit
    def _plan_step(self, stream):
        lib = _lib.load()
        rc = lib.moba_prep_plan(self._handle, 1, stream, self._positions.ctypes.data)
        if rc:
            msg = lib.moba_hip_last_error().decode(errors="replace")
            if rc == _lib.MOBA_ERR_ARG:
                raise ValueError(msg)
            self.failed = True
            raise _lib.MobaHipError(msg)
        return tuple(self._positions.tolist())

    def _launch_step(self, stream):
        lib = _lib.load()
        if lib.moba_prep_launch(self._handle, 1, 0, stream):
            self.failed = True
            raise _lib.MobaHipError(lib.moba_hip_last_error().decode(errors="replace"))

    def _commit_step(self):
        lib = _lib.load()
        if lib.moba_prep_commit(self._handle):
            self.failed = True
            raise _lib.MobaHipError(lib.moba_hip_last_error().decode(errors="replace"))

    def _result(self, positions):
        return DecodeResult(self.output, self.lse, None if self.dense else self.selected,
                            self.ids, positions)

    @torch.no_grad()
    def attend(self, q, *, use_graph=False):
        with self.cache._lock:
            stream = self._usable()
            copy_q = bool(self._bind_all(((q, self.q, "q"),)))
            if use_graph and "attend" not in self._captured:
                raise ValueError("capture('attend') first")
            if copy_q:
                self.q.copy_(q)
            return self._result(self._run(False, use_graph, stream))

    def step(self, q, k, v, *, use_graph=False):
        """One token per leased row; argument and capacity errors change nothing."""
        with self.cache._lock:
            stream = self._usable()
            if q is self.q and k is self.k and v is self.v and not self.check_finite:
                # the bound buffers are the inputs: plan, launch and commit
                # in one native call
                if use_graph and "step" not in self._captured:
                    raise ValueError("capture('step') first")
                return self._result(self._run(True, use_graph, stream))
            copies = self._bind_all(((q, self.q, "q"), (k, self.k, "k"), (v, self.v, "v")))
            if use_graph and "step" not in self._captured:
                raise ValueError("capture('step') first")
            positions = self._plan_step(stream)  # refuses (ValueError) before any change
            with torch.no_grad():
                for given, buffer in copies:
                    buffer.copy_(given)
            lib = _lib.load()
            if lib.moba_prep_launch(self._handle, 1, int(use_graph), stream) or \
                    lib.moba_prep_commit(self._handle):
                self.failed = True
                raise _lib.MobaHipError(lib.moba_hip_last_error().decode(errors="replace"))
            return self._result(positions)

    def capture(self, kind="step"):
        """Records the device work of one step / attend into a hipGraph.
        Nothing runs and no cache state changes."""
        _require([(lambda: kind in ("step", "attend"), "kind must be step or attend")])
        with self.cache._lock:
            stream = self._usable()
            if kind in self._captured:
                raise ValueError("graph already captured")
            if kind == "attend" and min(self._lease.positions()) == 0:
                raise ValueError("attend capture requires nonempty cached sequences")
            lib = _lib.load()
            if lib.moba_prep_capture(self._handle, int(kind == "step"), stream):
                raise _lib.MobaHipError(lib.moba_hip_last_error().decode(errors="replace"))
            self._captured.add(kind)
            return self

    def close(self):
        if self.closed:
            return
        c = self.cache
        with c._lock:
            _require([
                (lambda: c._lessee is self, "prepared ownership lost"),
                (lambda: torch.cuda.current_stream(c.device).cuda_stream == c._stream,
                 "cross-stream cache access is unsupported"),
            ])
            if self.failed:
                c._broken = True
            else:
                self._lease.publish(c._layout)
            c._lessee = None
            self.closed = True
            lib = _lib.load()
            lib.moba_prep_destroy(self._handle)
            self._handle = None

    def __del__(self):
        if getattr(self, "_handle", None):
            _lib.load().moba_prep_destroy(self._handle)
            self._handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
