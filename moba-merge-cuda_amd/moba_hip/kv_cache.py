"""Paged / contiguous KV cache with incremental MoBA decode on gfx950.

Public API of src/moba_opt/kv_cache.py:42-300 (constructor, ``append``,
``attend``, ``append_and_attend``, ``reset``, ``materialize``,
``prepare_decode``, the ``lengths`` / ``page_table`` snapshots,
``DecodeResult``), with the reference's errors (:mod:`decode_contract`).
Inputs are projected, position-encoded Q/K/V; the cache is inference-only and
is not a serving scheduler.

State and where it lives:

* host: the page pool (C++, :mod:`moba_hip.cache_layout`) owns page
  allocation; its table and lengths are the truth;
* device: the K/V page pools ``[num_pages, page, Hkv, D]``, a mirror of the
  pool's table ``[B, W]`` and lengths ``[B]`` (persistent tensors, rewritten
  in place by one host-to-device copy after each change), and the chunk means
  ``[B, max_chunks, Hkv, D]`` in the cache dtype (kv_cache.py:80-88).

Operations hold one lock and run on the stream that was current at
construction; calls from another stream or inside an external graph capture
are refused.  While a :class:`~moba_hip.prepared_decode.PreparedDecode`
holds the cache, ordinary operations are refused too.
"""
from __future__ import annotations

import threading
from dataclasses import dataclass

import numpy as np
import torch

from . import decode_contract as contract
from .baseline_adapter import _require
from .cache_layout import PageAllocator
from .ops import decode as kernels

# names of the reference module, kept for callers that import them
_ints = contract.int_vector
_mode = contract.decode_mode


@dataclass(frozen=True)
class AppendResult:
    sequence_ids: tuple
    positions: tuple


@dataclass(frozen=True)
class DecodeResult:
    output: torch.Tensor
    lse: torch.Tensor
    selected_blocks: object  # [Nq,Hq,slots] int32, current chunk first, -1 pad; None if dense
    sequence_ids: tuple
    positions: tuple


class PagedKVCache:
    def __init__(self, batch_size, max_seq_len, num_kv_heads, head_dim, *,
                 page_size=16, num_pages=None, chunk_size=128,
                 dtype=torch.bfloat16, device="cuda"):
        dims, requested = contract.constructor(batch_size, max_seq_len, page_size, num_kv_heads,
                                               head_dim, chunk_size, dtype, device)
        self.num_kv_heads, self.head_dim = dims["num_kv_heads"], dims["head_dim"]
        self.chunk_size, self.dtype = dims["chunk_size"], dtype
        B, L, P = dims["batch_size"], dims["max_seq_len"], dims["page_size"]
        pages = B * -(-L // P) if num_pages is None else num_pages
        self._layout = PageAllocator(B, L, P, pages, self.chunk_size)
        self._lock = threading.RLock()
        self._lessee = None      # the PreparedDecode holding the cache, if any
        self._broken = False     # a device failure happened under a lease
        with torch.cuda.device(requested):
            self.device = torch.device("cuda", torch.cuda.current_device())
            self._stream = torch.cuda.current_stream(self.device).cuda_stream
            dev = dict(device=self.device)
            self.k_cache = torch.empty((pages, P, self.num_kv_heads, self.head_dim), dtype=dtype,
                                       **dev)
            self.v_cache = torch.empty_like(self.k_cache)
            self._table = torch.full((B, self._layout.table_width), -1, dtype=torch.int32, **dev)
            self._lengths = torch.zeros(B, dtype=torch.int32, **dev)
            self._means = torch.empty((B, -(-L // self.chunk_size), self.num_kv_heads,
                                       self.head_dim), dtype=dtype, **dev)

    # -------------------------------------------------------------- snapshots
    @property
    def lengths(self):
        lessee = self._lessee
        return lessee.lengths if lessee is not None else self._layout.lengths

    @property
    def page_table(self):
        """Immutable CPU snapshot of the logical -> physical page table."""
        lessee = self._lessee
        return lessee.page_table if lessee is not None else self._layout.tables

    # ----------------------------------------------------------------- guards
    def _guard(self, *, under_lease=False):
        if self._broken:
            raise RuntimeError("CUDA execution failed; discard this cache")
        _require([
            (lambda: under_lease or self._lessee is None,
             "prepared decode owns cache; close it before ordinary cache operations"),
            (lambda: not torch.cuda.is_current_stream_capturing(),
             "CUDA Graph capture is unsupported for this cache API"),
            (lambda: torch.cuda.current_stream(self.device).cuda_stream == self._stream,
             "cross-stream cache access is unsupported"),
        ])

    def _check_inputs(self, *specs):
        contract.tensors(specs, device=self.device, dtype=self.dtype, head_dim=self.head_dim)

    def _no_pool_alias(self, *tensors):
        pools = (self.k_cache.untyped_storage().data_ptr(),
                 self.v_cache.untyped_storage().data_ptr())
        _require([(lambda: all(t.untyped_storage().data_ptr() not in pools for t in tensors),
                   "append inputs must not alias KV cache storage; clone first")])

    def _candidates(self, lengths=None):
        """Routable chunks summed over the slots: every chunk before each
        slot's current one (the reference's bound on topk - 1)."""
        n = self._layout._pool.length_view if lengths is None else np.asarray(lengths)
        return int(np.maximum(0, -(-n // self.chunk_size) - 1).sum())

    # ----------------------------------------------------------- device sync
    def _publish_layout(self, *extra):
        """One host-to-device copy of [table | lengths | *extra] int32; the
        table and lengths mirrors are rewritten in place and device views of
        the extra vectors are returned."""
        pool = self._layout._pool
        parts = [pool.table_view.ravel(), pool.length_view] + [np.asarray(x, np.int32)
                                                              for x in extra]
        flat = torch.from_numpy(np.concatenate(parts)).to(self.device)
        nt, nl = self._table.numel(), self._lengths.numel()
        self._table.view(-1).copy_(flat[:nt])
        self._lengths.copy_(flat[nt:nt + nl])
        views, at = [], nt + nl
        for x in parts[2:]:
            views.append(flat[at:at + len(x)])
            at += len(x)
        return views

    def prepare_decode(self, sequence_ids, num_q_heads, *, topk=4, mode="moba",
                       check_finite=True, stable_routes=False):
        from .prepared_decode import PreparedDecode
        return PreparedDecode(self, sequence_ids, num_q_heads, topk=topk, mode=mode,
                              check_finite=check_finite, stable_routes=stable_routes)

    # ----------------------------------------------------------------- append
    @torch.no_grad()
    def append(self, k, v, *, sequence_ids, cu_seqlens=None):
        with self._lock, torch.cuda.device(self.device):
            self._guard()
            self._check_inputs((k, "k", {"heads": self.num_kv_heads}),
                               (v, "v", {"heads": self.num_kv_heads, "tokens": lambda: k.shape[0]}))
            self._no_pool_alias(k, v)
            ids = self._layout.validate_ids(_ints(sequence_ids, "sequence_ids"), unique=True)
            counts = contract.append_counts(k.shape[0], ids, cu_seqlens)
            return self._store(k, v, ids, counts)[0]

    def _store(self, k, v, ids, counts):
        """Plans, writes and commits an append whose inputs are checked.
        Returns (AppendResult, device token slots, device token positions)."""
        plan = self._layout.plan_append(ids, counts)
        before = self._layout._pool.clone()
        self._layout.commit(plan)
        try:
            seq, pos, cseq, cchunk = self._publish_layout(plan.seq_arr, plan.pos_arr,
                                                          plan.closed_arr[:, 0],
                                                          plan.closed_arr[:, 1])
            kernels.append_tokens(k.contiguous(), v.contiguous(), self.k_cache, self.v_cache,
                                  self._table, seq, pos)
            kernels.block_means(self.k_cache, self._table, self._means, cseq, cchunk,
                                self.chunk_size)
        except Exception:  # a failed launch leaves the pool as it was
            self._layout._pool.assign(before)
            self._publish_layout()
            raise
        return AppendResult(plan.token_sequences, plan.token_positions), seq, pos

    # ----------------------------------------------------------------- attend
    def _positions(self, q, sequence_ids, positions):
        self._check_inputs((q, "q", {}))
        _require([(lambda: q.shape[1] % self.num_kv_heads == 0, "Hq must be a multiple of Hkv")])
        ids = self._layout.validate_ids(_ints(sequence_ids, "sequence_ids"))
        _require([(lambda: len(ids) == q.shape[0], "one sequence ID per query row required")])
        lengths = self.lengths
        pos = (tuple(lengths[s] - 1 for s in ids) if positions is None
               else _ints(positions, "positions"))
        _require([
            (lambda: len(pos) == len(ids) and all(0 <= p < lengths[s] for s, p in zip(ids, pos)),
             "query positions must refer to cached tokens"),
            (lambda: q.shape[0] * q.shape[1] < 2 ** 31, "query grid exceeds int32 capacity"),
        ])
        return ids, pos

    @torch.no_grad()
    def attend(self, q, *, sequence_ids, positions=None, topk=4, mode="moba"):
        with self._lock, torch.cuda.device(self.device):
            self._guard()
            dense = _mode(mode, topk)
            ids, pos = self._positions(q, sequence_ids, positions)
            dev_ids, dev_pos = torch.tensor([ids, pos], dtype=torch.int32, device=self.device)
            return self._decode(q, ids, pos, dev_ids, dev_pos, topk, dense)

    def _decode(self, q, ids, pos, dev_ids, dev_pos, topk, dense):
        """Route + paged attention of checked queries at cached positions
        (nothing in the cache changes)."""
        q = q.contiguous()
        nq, hq, _ = q.shape
        history = max(pos) // self.chunk_size           # closed chunks of the longest row
        remote = 0 if dense else min(int(topk) - 1, self._candidates())
        out = torch.empty_like(q)
        lse = torch.empty((nq, hq), dtype=torch.float32, device=self.device)
        width = max(1, remote, history)
        if kernels.fused_supported(hq, self.num_kv_heads, self.head_dim, width,
                                   self._table.shape[1]) and nq * hq * width < 2 ** 31:
            work = kernels.FusedWork(nq, hq, self.num_kv_heads, self.head_dim, self.device)
            selected = None if dense else torch.empty((nq, hq, remote + 1), dtype=torch.int32,
                                                      device=self.device)
            kernels.fused(q, None, None, self.k_cache, self.v_cache, self._table, self._lengths,
                          dev_ids, dev_pos, None, self._means, self.chunk_size, width, remote,
                          dense, 0, selected, work, out, lse)
            return DecodeResult(out, lse, selected, ids, pos)
        work = None
        if not dense:
            width = max(remote, history)
            _require([(lambda: not remote or width * hq * nq < 2 ** 31,
                       "route score grid exceeds int32 capacity")])
            work = kernels.RouteWork(nq, hq, self.num_kv_heads, remote, self.device)
            scores = (torch.empty((nq, hq, width), dtype=torch.float32, device=self.device)
                      if remote else None)
            kernels.route(q, self._means, dev_ids, dev_pos, self.chunk_size,
                          width if remote else 0, remote, scores, work)
        kernels.attention(q, self.k_cache, self.v_cache, self._table, self._lengths, dev_ids,
                          dev_pos, work, out, lse, self.chunk_size, dense, history + 1)
        return DecodeResult(out, lse, None if dense else work.selected, ids, pos)

    @torch.no_grad()
    def append_and_attend(self, q, k, v, *, sequence_ids, cu_seqlens=None, topk=4, mode="moba"):
        with self._lock, torch.cuda.device(self.device):
            self._guard()
            dense = _mode(mode, topk)
            self._check_inputs((k, "k", {"heads": self.num_kv_heads}),
                               (v, "v", {"heads": self.num_kv_heads, "tokens": lambda: k.shape[0]}),
                               (q, "q", {"tokens": lambda: k.shape[0]}))
            self._no_pool_alias(q, k, v)
            contract.query_grid(q, self.num_kv_heads)
            ids = self._layout.validate_ids(_ints(sequence_ids, "sequence_ids"), unique=True)
            counts = contract.append_counts(k.shape[0], ids, cu_seqlens)
            done, seq, pos = self._store(k, v, ids, counts)
            return self._decode(q, done.sequence_ids, done.positions, seq, pos, topk, dense)

    # ------------------------------------------------------------------ reset
    @torch.no_grad()
    def reset(self, sequence_ids=None):
        with self._lock, torch.cuda.device(self.device):
            self._guard()
            ids = (tuple(range(self._layout.batch_size)) if sequence_ids is None
                   else _ints(sequence_ids, "sequence_ids"))
            self._layout.reset(ids)   # checks every id before changing anything
            self._publish_layout()

    @torch.no_grad()
    def materialize(self, sequence_id):
        """Logical K/V ``[len, Hkv, D]`` of one sequence (diagnostics, tests)."""
        with self._lock, torch.cuda.device(self.device):
            self._guard(under_lease=True)
            sid = self._layout.validate_ids([sequence_id])[0]
            n = self.lengths[sid]
            tok = torch.arange(n, device=self.device)
            P = self._layout.page_size
            page = self._table[sid].long()[tok // P]
            return self.k_cache[page, tok % P], self.v_cache[page, tok % P]


class ContiguousKVCache(PagedKVCache):
    """One contiguous physical slab per sequence (a page of max_seq_len
    tokens per slot), same semantics."""

    def __init__(self, batch_size, max_seq_len, num_kv_heads, head_dim, **kwargs):
        if "page_size" in kwargs or "num_pages" in kwargs:
            raise ValueError("ContiguousKVCache owns page_size/num_pages")
        super().__init__(batch_size, max_seq_len, num_kv_heads, head_dim,
                         page_size=max_seq_len, num_pages=batch_size, **kwargs)
