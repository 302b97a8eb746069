"""Inference-only paged / contiguous KV cache with incremental MoBA decode.

Drop-in for src/moba_opt/kv_cache.py:1-300: same constructor, methods,
properties, result types, validation order and error messages.  Inputs are
already projected / position-encoded Q/K/V.  The cache owns page allocation
(a host :class:`~moba_hip.cache_layout.PageAllocator`) and is not a serving
scheduler: operations are serialised by one lock and bound to the stream that
was current at construction; cross-stream use and external graph capture are
rejected.

All device work is done by the gfx950 kernels of libmoba_hip.so:
scatter append, closed-chunk means, fused route + stable top-k, and paged
split-K attention that reads physical pages through the page table.
"""
from __future__ import annotations

import threading
from dataclasses import dataclass

import torch

from .cache_layout import PageAllocator, positive_int
from .ops import decode as kernels


def _ints(values, name):
    if isinstance(values, torch.Tensor):
        if values.device.type != "cpu" or values.dtype not in (torch.int32, torch.int64) \
                or values.dim() != 1:
            raise ValueError(f"{name} must be a Python sequence or CPU int32/int64 vector")
        values = values.tolist()
    if not isinstance(values, (tuple, list)):
        raise ValueError(f"{name} must be a Python sequence or CPU integer vector")
    if any(isinstance(x, bool) or not isinstance(x, int) for x in values):
        raise ValueError(f"{name} must contain integers")
    return tuple(values)


def _mode(mode, topk):
    """True when the call is dense (mode='dense' or topk=1)."""
    if mode not in ("moba", "dense"):
        raise ValueError("mode must be moba or dense")
    if positive_int(topk, "topk") > 9:
        raise ValueError("topk must be in [1,9]")
    return bool(mode == "dense" or topk == 1)


@dataclass(frozen=True)
class AppendResult:
    sequence_ids: tuple
    positions: tuple


@dataclass(frozen=True)
class DecodeResult:
    output: torch.Tensor
    lse: torch.Tensor
    selected_blocks: object  # [Nq,Hq,slots] int32, current block first; None for dense
    sequence_ids: tuple
    positions: tuple


class PagedKVCache:
    def __init__(self, batch_size, max_seq_len, num_kv_heads, head_dim, *,
                 page_size=16, num_pages=None, chunk_size=128,
                 dtype=torch.bfloat16, device="cuda"):
        batch_size = positive_int(batch_size, "batch_size")
        max_seq_len = positive_int(max_seq_len, "max_seq_len")
        page_size = positive_int(page_size, "page_size")
        self.num_kv_heads = positive_int(num_kv_heads, "num_kv_heads")
        self.head_dim = positive_int(head_dim, "head_dim")
        if self.head_dim > 256:
            raise ValueError("decode head_dim must be in [1,256]")
        self.chunk_size = positive_int(chunk_size, "chunk_size")
        if self.chunk_size > 1024:
            raise ValueError("cache chunk_size must be <=1024")
        if dtype not in (torch.bfloat16, torch.float16):
            raise ValueError("cache dtype must be BF16 or FP16")
        requested = torch.device(device)
        if requested.type != "cuda":
            raise ValueError("cache device must be CUDA")
        if num_pages is None:
            num_pages = batch_size * (-(-max_seq_len // page_size))
        self._layout = PageAllocator(batch_size, max_seq_len, page_size, num_pages,
                                     self.chunk_size)
        self.dtype = dtype
        self._lock = threading.RLock()
        self._prepared_owner = None
        self._invalid = False
        with torch.cuda.device(requested):
            self.device = torch.device("cuda", torch.cuda.current_device())
            self._stream = torch.cuda.current_stream(self.device).cuda_stream
            shape = (self._layout.num_pages, page_size, self.num_kv_heads, self.head_dim)
            self.k_cache = torch.empty(shape, dtype=dtype, device=self.device)
            self.v_cache = torch.empty_like(self.k_cache)
            self._table = torch.full((batch_size, self._layout.table_width), -1,
                                     dtype=torch.int32, device=self.device)
            self._lengths = torch.zeros(batch_size, dtype=torch.int32, device=self.device)
            max_chunks = -(-max_seq_len // self.chunk_size)
            self._means = torch.empty((batch_size, max_chunks, self.num_kv_heads, self.head_dim),
                                      dtype=dtype, device=self.device)
            self._candidate_count = 0

    # ------------------------------------------------------------ properties
    @property
    def lengths(self):
        if self._prepared_owner is not None:
            return self._prepared_owner.lengths
        return self._layout.lengths

    @property
    def page_table(self):
        """Immutable CPU snapshot; callers cannot edit the internal table."""
        if self._prepared_owner is not None:
            return self._prepared_owner.page_table
        return self._layout.tables

    # ----------------------------------------------------------- validation
    def _check_stream(self, *, allow_prepared=False):
        if self._invalid:
            raise RuntimeError("CUDA execution failed; discard this cache")
        if self._prepared_owner is not None and not allow_prepared:
            raise ValueError("prepared decode owns cache; close it before ordinary cache operations")
        if torch.cuda.is_current_stream_capturing():
            raise ValueError("CUDA Graph capture is unsupported for this cache API")
        if torch.cuda.current_stream(self.device).cuda_stream != self._stream:
            raise ValueError("cross-stream cache access is unsupported")

    def _tensor(self, tensor, name, *, expected_heads=None, expected_tokens=None):
        if not isinstance(tensor, torch.Tensor) or tensor.dim() != 3:
            raise ValueError(f"{name} must be [N,H,D]")
        if tensor.device != self.device or tensor.dtype != self.dtype:
            raise ValueError(f"{name} must match cache device and dtype")
        if tensor.requires_grad:
            raise ValueError("KV cache/decode is inference-only; detach Q/K/V")
        if tensor.shape[0] < 1 or tensor.shape[1] < 1 or tensor.shape[2] != self.head_dim:
            raise ValueError(f"{name} has an invalid shape")
        if tensor.stride(-1) != 1:
            raise ValueError(f"{name} last dimension must be contiguous")
        if expected_heads is not None and tensor.shape[1] != expected_heads:
            raise ValueError(f"{name} KV head count differs from cache")
        if expected_tokens is not None and tensor.shape[0] != expected_tokens:
            raise ValueError(f"{name} token count differs")
        if not bool(torch.isfinite(tensor).all()):
            raise ValueError(f"{name} contains NaN/Inf")

    def _reject_storage_alias(self, *tensors):
        pools = {self.k_cache.untyped_storage().data_ptr(),
                 self.v_cache.untyped_storage().data_ptr()}
        if any(t.untyped_storage().data_ptr() in pools for t in tensors):
            raise ValueError("append inputs must not alias KV cache storage; clone first")

    def _append_counts(self, token_count, sequence_ids, cu_seqlens):
        ids = self._layout.validate_ids(_ints(sequence_ids, "sequence_ids"), unique=True)
        cu = tuple(range(len(ids) + 1)) if cu_seqlens is None else _ints(cu_seqlens, "cu_seqlens")
        if len(cu) != len(ids) + 1 or cu[0] != 0 or cu[-1] != token_count:
            raise ValueError("append cu_seqlens must start at 0 and end at N")
        counts = tuple(b - a for a, b in zip(cu, cu[1:]))
        if any(n <= 0 for n in counts):
            raise ValueError("append sequences must be nonempty")
        return ids, counts

    def _count_candidates(self, lengths):
        C = self.chunk_size
        return sum(max(0, -(-n // C) - 1) for n in lengths)

    def _gpu(self, data):
        return torch.tensor(data, dtype=torch.int32, device=self.device)

    def _metadata(self, *vectors):
        """One H2D copy for several int vectors (views share the storage)."""
        flat, sizes = [], []
        for vec in vectors:
            sizes.append(len(vec))
            flat.extend(vec)
        return self._gpu(flat).split(sizes)

    def prepare_decode(self, sequence_ids, num_q_heads, *, topk=4, mode="moba",
                       check_finite=True, stable_routes=False):
        from .prepared_decode import PreparedDecode
        return PreparedDecode(self, sequence_ids, num_q_heads, topk=topk, mode=mode,
                              check_finite=check_finite, stable_routes=stable_routes)

    # --------------------------------------------------------------- append
    @torch.no_grad()
    def append(self, k, v, *, sequence_ids, cu_seqlens=None):
        with self._lock, torch.cuda.device(self.device):
            self._check_stream()
            self._tensor(k, "k", expected_heads=self.num_kv_heads)
            self._tensor(v, "v", expected_heads=self.num_kv_heads, expected_tokens=k.shape[0])
            self._reject_storage_alias(k, v)
            ids, counts = self._append_counts(k.shape[0], sequence_ids, cu_seqlens)
            return self._append_validated(k, v, ids, counts)[0]

    def _append_validated(self, k, v, ids, counts):
        """Caller holds lock/device/stream and validated all inputs."""
        plan = self._layout.plan_append(ids, counts)
        table = self._gpu(plan.tables)
        lengths, token_ids, positions, closed_ids, closed_chunks = self._metadata(
            plan.lengths, plan.token_sequences, plan.token_positions,
            [c[0] for c in plan.completed_chunks], [c[1] for c in plan.completed_chunks])
        candidate_count = self._count_candidates(plan.lengths)
        kernels.append_tokens(k.contiguous(), v.contiguous(), self.k_cache, self.v_cache, table,
                              token_ids, positions)
        kernels.block_means(self.k_cache, table, self._means, closed_ids, closed_chunks,
                            self.chunk_size)
        self._layout.commit(plan)
        self._table, self._lengths = table, lengths
        self._candidate_count = candidate_count
        return AppendResult(plan.token_sequences, plan.token_positions), token_ids, positions

    # --------------------------------------------------------------- attend
    def _query_metadata(self, q, sequence_ids, positions):
        self._tensor(q, "q")
        if q.shape[1] % self.num_kv_heads:
            raise ValueError("Hq must be a multiple of Hkv")
        ids = self._layout.validate_ids(_ints(sequence_ids, "sequence_ids"))
        if len(ids) != q.shape[0]:
            raise ValueError("one sequence ID per query row required")
        pos = (tuple(self.lengths[s] - 1 for s in ids) if positions is None
               else _ints(positions, "positions"))
        if len(pos) != len(ids) or any(not 0 <= p < self.lengths[s] for s, p in zip(ids, pos)):
            raise ValueError("query positions must refer to cached tokens")
        if q.shape[0] * q.shape[1] >= 2 ** 31:
            raise ValueError("query grid exceeds int32 capacity")
        return ids, pos

    def _route(self, q, ids, positions, topk, max_history):
        nq, hq, _ = q.shape
        remote = min(int(topk) - 1, self._candidate_count)
        width = max(remote, max_history)
        if remote and width * hq * nq >= 2 ** 31:
            raise ValueError("route score grid exceeds int32 capacity")
        work = kernels.RouteWork(nq, hq, self.num_kv_heads, remote, self.device)
        scores = (torch.empty((nq, hq, width), dtype=torch.float32, device=self.device)
                  if remote else None)
        kernels.route(q, self._means, ids, positions, self.chunk_size, width if remote else 0,
                      remote, scores, work)
        return work

    @torch.no_grad()
    def attend(self, q, *, sequence_ids, positions=None, topk=4, mode="moba"):
        with self._lock, torch.cuda.device(self.device):
            self._check_stream()
            dense = _mode(mode, topk)
            ids, pos = self._query_metadata(q, sequence_ids, positions)
            return self._attend_validated(q, ids, pos, topk, dense)

    def _attend_validated(self, q, ids, pos, topk, dense, gpu_metadata=None):
        q = q.contiguous()
        gpu_ids, gpu_pos = self._metadata(ids, pos) if gpu_metadata is None else gpu_metadata
        max_hist = max(pos) // self.chunk_size
        nq, hq, _ = q.shape
        remote = 0 if dense else min(int(topk) - 1, self._candidate_count)
        width = max(1, remote, max_hist)
        if kernels.fused_supported(hq, self.num_kv_heads, self.head_dim, width,
                                  self._table.shape[1]) \
                and nq * hq * width < 2 ** 31:
            # route + attention in one launch (positions given; nothing mutates)
            work = kernels.FusedWork(nq, hq, self.num_kv_heads, self.head_dim, self.device)
            selected = None if dense else torch.empty((nq, hq, remote + 1), dtype=torch.int32,
                                                      device=self.device)
            out = torch.empty_like(q)
            lse = torch.empty(q.shape[:2], device=self.device, dtype=torch.float32)
            kernels.fused(q, None, None, self.k_cache, self.v_cache, self._table, self._lengths,
                          gpu_ids, gpu_pos, None, self._means, self.chunk_size, width, remote,
                          dense, 0, selected, work, out, lse)
            return DecodeResult(out, lse, selected, ids, pos)
        work = None if dense else self._route(q, gpu_ids, gpu_pos, topk, max_hist)
        out = torch.empty_like(q)
        lse = torch.empty(q.shape[:2], device=self.device, dtype=torch.float32)
        kernels.attention(q, self.k_cache, self.v_cache, self._table, self._lengths, gpu_ids,
                          gpu_pos, work, out, lse, self.chunk_size, dense, max_hist + 1)
        return DecodeResult(out, lse, None if dense else work.selected, ids, pos)

    @torch.no_grad()
    def append_and_attend(self, q, k, v, *, sequence_ids, cu_seqlens=None, topk=4, mode="moba"):
        with self._lock, torch.cuda.device(self.device):
            self._check_stream()
            dense = _mode(mode, topk)
            self._tensor(k, "k", expected_heads=self.num_kv_heads)
            self._tensor(v, "v", expected_heads=self.num_kv_heads, expected_tokens=k.shape[0])
            self._tensor(q, "q", expected_tokens=k.shape[0])
            self._reject_storage_alias(q, k, v)
            if q.shape[1] % self.num_kv_heads:
                raise ValueError("Hq must be a multiple of Hkv")
            if q.shape[0] * q.shape[1] >= 2 ** 31:
                raise ValueError("query grid exceeds int32 capacity")
            ids, counts = self._append_counts(k.shape[0], sequence_ids, cu_seqlens)
            info, gpu_ids, gpu_pos = self._append_validated(k, v, ids, counts)
            return self._attend_validated(q, info.sequence_ids, info.positions, topk, dense,
                                          gpu_metadata=(gpu_ids, gpu_pos))

    # ---------------------------------------------------------------- reset
    @torch.no_grad()
    def reset(self, sequence_ids=None):
        with self._lock, torch.cuda.device(self.device):
            self._check_stream()
            ids = (tuple(range(self._layout.batch_size)) if sequence_ids is None
                   else _ints(sequence_ids, "sequence_ids"))
            # stage on a scratch allocator so a failure publishes nothing
            old = self._layout
            staged = PageAllocator(old.batch_size, old.max_seq_len, old.page_size, old.num_pages,
                                   old.chunk_size)
            staged.tables, staged.lengths, staged.free_pages = old.tables, old.lengths, old.free_pages
            staged.version = old.version
            staged.reset(ids)
            table, lengths = self._gpu(staged.tables), self._gpu(staged.lengths)
            candidates = self._count_candidates(staged.lengths)
            self._layout, self._table, self._lengths = staged, table, lengths
            self._candidate_count = candidates

    @torch.no_grad()
    def materialize(self, sequence_id):
        """Logical K/V [len,Hkv,D] of one sequence (diagnostics and tests)."""
        with self._lock, torch.cuda.device(self.device):
            self._check_stream(allow_prepared=True)
            sid = self._layout.validate_ids([sequence_id])[0]
            length = self.lengths[sid]
            pos = torch.arange(length, device=self.device)
            page = self._layout.page_size
            pages = self._table[sid, pos.div(page, rounding_mode="floor")].long()
            return self.k_cache[pages, pos % page], self.v_cache[pages, pos % page]


class ContiguousKVCache(PagedKVCache):
    """One contiguous physical slab per sequence, same semantics."""

    def __init__(self, batch_size, max_seq_len, num_kv_heads, head_dim, **kwargs):
        if "page_size" in kwargs or "num_pages" in kwargs:
            raise ValueError("ContiguousKVCache owns page_size/num_pages")
        super().__init__(batch_size, max_seq_len, num_kv_heads, head_dim,
                         page_size=max_seq_len, num_pages=batch_size, **kwargs)
