"""Host page management of the paged KV cache: Python face of the C++ page
pool in libmoba_hip.so (``moba_pool_*``, host-only code, no device needed).

The classes keep the names and observable behaviour of the reference's
allocator (src/moba_opt/cache_layout.py:23-148), which its callers and tests
see through ``PagedKVCache.page_table``:

* :class:`PageAllocator`: a fixed number of batch slots over a pool of
  physical pages.  ``plan_append`` computes an append without changing the
  pool (ValueError with the reference's messages, nothing changed), ``commit``
  installs it and refuses a plan made before the pool last changed
  (RuntimeError "stale").  Free pages form a stack that hands out page 0
  first; ``reset`` pushes a slot's pages back in logical order, so the page
  freed last is handed out next.
* :class:`IncrementalLayout`: the O(rows) lease a prepared decode holds on a
  fixed set of slots; one token per slot per step; ``publish`` hands its
  state back to the allocator.

All state lives in the C++ pool; the properties return immutable snapshots.
"""
from __future__ import annotations

import ctypes
import numbers
from dataclasses import dataclass, field

import numpy as np

from .ops import _lib

_I32 = np.int32


def positive_int(value, name):
    if isinstance(value, bool) or not isinstance(value, numbers.Integral) or value <= 0:
        raise ValueError(f"{name} must be a positive integer")
    return int(value)


def _cptr(arr):
    return arr.ctypes.data if arr is not None and arr.size else None


def _check(rc):
    """Raises the pool's error: ValueError for bad input, RuntimeError for a
    stale plan."""
    if rc == 0:
        return
    msg = _lib.load().moba_hip_last_error().decode(errors="replace")
    raise (RuntimeError if rc == _lib.MOBA_ERR_STALE else ValueError)(msg)


class _Pool:
    """Owner of one C++ pool handle, with zero-copy numpy views of its
    table, lengths and free stack."""
    __slots__ = ("handle", "lib", "table_view", "length_view", "free_view", "__weakref__")

    def __init__(self, handle):
        self.lib = _lib.load()
        self.handle = handle
        info = self.info()
        batch, width, pages = int(info[0]), int(info[5]), int(info[3])
        self.table_view = np.ctypeslib.as_array(self.lib.moba_pool_table(handle),
                                                shape=(batch, width))
        self.length_view = np.ctypeslib.as_array(self.lib.moba_pool_lengths(handle),
                                                 shape=(batch,))
        self.free_view = np.ctypeslib.as_array(self.lib.moba_pool_free(handle), shape=(pages,))

    @classmethod
    def create(cls, batch, max_len, page, pages, chunk):
        h = ctypes.c_void_p()
        _check(_lib.load().moba_pool_create(batch, max_len, page, pages, chunk, ctypes.byref(h)))
        return cls(h.value)

    def clone(self):
        h = ctypes.c_void_p()
        _check(self.lib.moba_pool_clone(self.handle, ctypes.byref(h)))
        return _Pool(h.value)

    def assign(self, src):
        """Takes src's state (views of this pool stay valid)."""
        _check(self.lib.moba_pool_assign(self.handle, src.handle))

    def info(self):
        out = np.zeros(8, np.int64)
        _check(self.lib.moba_pool_info(self.handle, out.ctypes.data))
        return out

    def free_stack(self):
        return self.free_view[: int(self.info()[7])]

    def ids(self, ids, unique):
        arr = np.asarray(ids, dtype=_I32)
        _check(self.lib.moba_pool_check_ids(self.handle, _cptr(arr), len(arr), int(unique)))
        return arr

    def __del__(self):
        if self.handle:
            self.lib.moba_pool_destroy(self.handle)
            self.handle = None


def _slot_ids(ids):
    """Python-level id checks (type), in the reference's order."""
    out = []
    for sid in ids:
        if isinstance(sid, bool) or not isinstance(sid, numbers.Integral):
            raise ValueError("sequence IDs must be integers")
        out.append(int(sid))
    return out


@dataclass(frozen=True)
class AppendPlan:
    """A planned append.  The tuples are the reference's plan fields; the
    arrays (not compared) carry the same data to the C++ pool and the
    device uploads."""
    version: int
    token_sequences: tuple
    token_positions: tuple
    completed_chunks: tuple  # (sequence_id, chunk) pairs this append closes
    lengths: tuple           # new length of each planned slot, in plan order
    ids: np.ndarray = field(compare=False, repr=False)
    seq_arr: np.ndarray = field(compare=False, repr=False)
    pos_arr: np.ndarray = field(compare=False, repr=False)
    closed_arr: np.ndarray = field(compare=False, repr=False)
    grants: np.ndarray = field(compare=False, repr=False)   # [n, 3] slot, logical, physical
    new_lengths: np.ndarray = field(compare=False, repr=False)


@dataclass(frozen=True)
class StepPlan:
    version: int
    positions: tuple
    updates: tuple  # (sequence_id, logical_page, physical_page)
    delta: np.ndarray = field(compare=False, repr=False)  # [2, rows] logical / physical or -1


class PageAllocator:
    """Batch slots whose logical pages map to any physical pages of the pool."""

    def __init__(self, batch_size, max_seq_len, page_size, num_pages, chunk_size):
        dims = [positive_int(v, n) for v, n in ((batch_size, "batch_size"),
                                               (max_seq_len, "max_seq_len"),
                                               (page_size, "page_size"),
                                               (num_pages, "num_pages"),
                                               (chunk_size, "chunk_size"))]
        (self.batch_size, self.max_seq_len, self.page_size, self.num_pages,
         self.chunk_size) = dims
        self._pool = _Pool.create(*dims)
        self.table_width = int(self._pool.info()[5])

    # snapshots of the C++ state
    @property
    def tables(self):
        return tuple(map(tuple, self._pool.table_view.tolist()))

    @property
    def lengths(self):
        return tuple(self._pool.length_view.tolist())

    @property
    def free_pages(self):
        return tuple(self._pool.free_stack().tolist())

    @free_pages.setter
    def free_pages(self, pages):
        """Reorders the free stack (a permutation of the free pages; the last
        entry is handed out first), as a benchmark's fragmented pool does."""
        arr = np.asarray(list(pages), dtype=_I32)
        _check(self._pool.lib.moba_pool_set_free(self._pool.handle, _cptr(arr), len(arr)))

    @property
    def version(self):
        return int(self._pool.info()[6])

    def validate_ids(self, ids, *, unique=False):
        return tuple(self._pool.ids(_slot_ids(ids), unique).tolist())

    def plan_append(self, sequence_ids, counts):
        ids = self._pool.ids(_slot_ids(sequence_ids), True)
        if len(ids) != len(counts):
            raise ValueError("one token count per sequence required")
        counts = [positive_int(n, "append count") for n in counts]
        # the length bound is checked before any buffer is sized by the counts
        # (the native plan checks it again, together with the pool's capacity)
        lengths = self._pool.length_view
        if any(int(lengths[s]) + n > self.max_seq_len for s, n in zip(ids.tolist(), counts)):
            raise ValueError("append exceeds max_seq_len")
        cnt = np.asarray(counts, dtype=_I32)
        tokens = int(cnt.sum())
        seq = np.empty(tokens, _I32)
        pos = np.empty(tokens, _I32)
        cap_closed = int((cnt // self.chunk_size + 1).sum())
        cap_grants = int((cnt // self.page_size + 2).sum())
        closed = np.empty((cap_closed, 2), _I32)
        grants = np.empty((cap_grants, 3), _I32)
        new_len = np.empty(len(ids), _I32)
        n_closed, n_grants, version = ctypes.c_int(), ctypes.c_int(), ctypes.c_int64()
        _check(self._pool.lib.moba_pool_plan_append(
            self._pool.handle, _cptr(ids), _cptr(cnt), len(ids), _cptr(seq), _cptr(pos),
            _cptr(closed), cap_closed, ctypes.byref(n_closed), _cptr(grants), cap_grants,
            ctypes.byref(n_grants), _cptr(new_len), ctypes.byref(version)))
        closed = closed[: n_closed.value]
        return AppendPlan(version.value, tuple(seq.tolist()), tuple(pos.tolist()),
                          tuple(map(tuple, closed.tolist())), tuple(new_len.tolist()),
                          ids, seq, pos, closed, grants[: n_grants.value], new_len)

    def commit(self, plan: AppendPlan):
        _check(self._pool.lib.moba_pool_commit_append(
            self._pool.handle, _cptr(plan.ids), len(plan.ids), _cptr(plan.new_lengths),
            _cptr(plan.grants), len(plan.grants), plan.version))

    def reset(self, sequence_ids):
        ids = np.asarray(_slot_ids(sequence_ids), dtype=_I32)
        _check(self._pool.lib.moba_pool_reset(self._pool.handle, _cptr(ids), len(ids)))


class IncrementalLayout:
    """Exclusive lease of a fixed set of slots for prepared decode: a private
    copy of the pool that advances one token per slot per step and is
    published back to the allocator when the lease ends."""

    def __init__(self, layout: PageAllocator, sequence_ids):
        self.ids = layout.validate_ids(sequence_ids, unique=True)
        self._ids = np.asarray(self.ids, dtype=_I32)
        self._pool = layout._pool.clone()
        self.page_size, self.max_seq_len = layout.page_size, layout.max_seq_len

    @property
    def handle(self):
        return self._pool.handle

    @property
    def tables(self):
        return self._pool.table_view.tolist()

    @property
    def lengths(self):
        return self._pool.length_view.tolist()

    @property
    def free(self):
        return self._pool.free_stack().tolist()

    @property
    def version(self):
        return int(self._pool.info()[6])

    def positions(self):
        """Current length of each leased slot, in lease order."""
        return self._pool.length_view[self._ids]

    def plan(self):
        n = len(self._ids)
        pos = np.empty(n, _I32)
        delta = np.empty((2, n), _I32)
        grants, version = ctypes.c_int(), ctypes.c_int64()
        _check(self._pool.lib.moba_pool_plan_step(self._pool.handle, _cptr(self._ids), n,
                                                  _cptr(pos), _cptr(delta),
                                                  ctypes.byref(grants), ctypes.byref(version)))
        rows = np.nonzero(delta[1] >= 0)[0]
        updates = tuple((self.ids[r], int(delta[0, r]), int(delta[1, r])) for r in rows)
        return StepPlan(version.value, tuple(pos.tolist()), updates, delta)

    def commit(self, plan: StepPlan):
        _check(self._pool.lib.moba_pool_commit_step(self._pool.handle, _cptr(self._ids),
                                                    len(self._ids), _cptr(plan.delta),
                                                    plan.version))

    def publish(self, layout: PageAllocator):
        layout._pool.assign(self._pool)
