"""Host page allocator of the paged KV cache.

Same observable behaviour as src/moba_opt/cache_layout.py:1-148 (the tests of
the reference pin it: tests/test_cache_layout.py, tests/test_prepared_layout.py):

* ``PageAllocator`` is transactional: ``plan_append`` computes the complete new
  state without touching the live one and raises ValueError (pool exhausted,
  over ``max_seq_len``, bad ids/counts) with nothing changed; ``commit``
  installs a plan and refuses a stale one (version check).
* Free pages form a stack whose initial order hands out physical page 0
  first; ``reset`` pushes a sequence's pages back in logical order, so the
  most recently freed page is reused first.
* ``IncrementalLayout`` is the O(active batch) lease used by prepared decode:
  one token per leased sequence per step, pages taken from the same stack.
"""
from __future__ import annotations

import numbers
from dataclasses import dataclass


def positive_int(value, name):
    if isinstance(value, bool) or not isinstance(value, numbers.Integral) or value <= 0:
        raise ValueError(f"{name} must be a positive integer")
    return int(value)


def _pages_for(tokens: int, page_size: int) -> int:
    return -(-tokens // page_size)


@dataclass(frozen=True)
class AppendPlan:
    version: int
    tables: tuple
    lengths: tuple
    free_pages: tuple
    token_sequences: tuple
    token_positions: tuple
    completed_chunks: tuple  # (sequence_id, chunk) pairs closed by this append


@dataclass(frozen=True)
class StepPlan:
    version: int
    positions: tuple
    updates: tuple  # (sequence_id, logical_page, physical_page)


class PageAllocator:
    """Fixed batch slots; logical pages map to arbitrary physical pages."""

    def __init__(self, batch_size, max_seq_len, page_size, num_pages, chunk_size):
        self.batch_size = positive_int(batch_size, "batch_size")
        self.max_seq_len = positive_int(max_seq_len, "max_seq_len")
        self.page_size = positive_int(page_size, "page_size")
        self.num_pages = positive_int(num_pages, "num_pages")
        self.chunk_size = positive_int(chunk_size, "chunk_size")
        if self.max_seq_len >= 2 ** 30 or self.num_pages * self.page_size >= 2 ** 31:
            raise ValueError("cache exceeds int32 indexing capacity")
        self.table_width = _pages_for(self.max_seq_len, self.page_size)
        empty_row = (-1,) * self.table_width
        self.tables = (empty_row,) * self.batch_size
        self.lengths = (0,) * self.batch_size
        # stack: the END is the next page handed out, so page 0 goes first
        self.free_pages = tuple(reversed(range(self.num_pages)))
        self.version = 0

    def validate_ids(self, ids, *, unique=False):
        out = []
        for sid in ids:
            if isinstance(sid, bool) or not isinstance(sid, numbers.Integral):
                raise ValueError("sequence IDs must be integers")
            if not 0 <= int(sid) < self.batch_size:
                raise ValueError("sequence ID outside cache batch slots")
            out.append(int(sid))
        if not out or (unique and len(set(out)) != len(out)):
            raise ValueError("nonempty unique sequence IDs required for append/reset")
        return tuple(out)

    def plan_append(self, sequence_ids, counts):
        ids = self.validate_ids(sequence_ids, unique=True)
        if len(ids) != len(counts):
            raise ValueError("one token count per sequence required")
        counts = [positive_int(n, "append count") for n in counts]
        need = 0
        for sid, n in zip(ids, counts):
            old = self.lengths[sid]
            if old + n > self.max_seq_len:
                raise ValueError("append exceeds max_seq_len")
            need += _pages_for(old + n, self.page_size) - _pages_for(old, self.page_size)
        if need > len(self.free_pages):
            raise ValueError("KV page pool exhausted; cache was not modified")
        tables = [list(r) for r in self.tables]
        lengths = list(self.lengths)
        stack = list(self.free_pages)
        seqs, positions, closed = [], [], []
        C = self.chunk_size
        for sid, n in zip(ids, counts):
            old = lengths[sid]
            new = old + n
            for logical in range(_pages_for(old, self.page_size), _pages_for(new, self.page_size)):
                tables[sid][logical] = stack.pop()
            seqs += [sid] * n
            positions += list(range(old, new))
            closed += [(sid, c) for c in range(old // C, new // C)]
            lengths[sid] = new
        return AppendPlan(self.version, tuple(tuple(r) for r in tables), tuple(lengths),
                          tuple(stack), tuple(seqs), tuple(positions), tuple(closed))

    def commit(self, plan):
        if plan.version != self.version:
            raise RuntimeError("stale append plan")
        self.tables, self.lengths, self.free_pages = plan.tables, plan.lengths, plan.free_pages
        self.version += 1

    def reset(self, sequence_ids):
        ids = self.validate_ids(sequence_ids, unique=True)
        tables = [list(r) for r in self.tables]
        lengths = list(self.lengths)
        stack = list(self.free_pages)
        for sid in ids:
            stack += [p for p in tables[sid] if p >= 0]
            tables[sid] = [-1] * self.table_width
            lengths[sid] = 0
        self.tables = tuple(tuple(r) for r in tables)
        self.lengths, self.free_pages = tuple(lengths), tuple(stack)
        self.version += 1


class IncrementalLayout:
    """Exclusive fixed-active-set lease: O(active batch) planning per step.

    Copies the page table once, mutates only newly allocated entries and
    publishes an immutable snapshot back to the allocator on close.
    """

    def __init__(self, layout, sequence_ids):
        self.ids = layout.validate_ids(sequence_ids, unique=True)
        self.tables = [list(r) for r in layout.tables]
        self.lengths = list(layout.lengths)
        self.free = list(layout.free_pages)
        self.version = layout.version
        self.page_size, self.max_seq_len = layout.page_size, layout.max_seq_len

    def plan(self):
        positions = tuple(self.lengths[s] for s in self.ids)
        if any(p >= self.max_seq_len for p in positions):
            raise ValueError("append exceeds max_seq_len")
        needs = [(s, p // self.page_size) for s, p in zip(self.ids, positions)
                 if p % self.page_size == 0]
        if len(needs) > len(self.free):
            raise ValueError("KV page pool exhausted; cache was not modified")
        updates = tuple((s, logical, self.free[len(self.free) - 1 - i])
                        for i, (s, logical) in enumerate(needs))
        return StepPlan(self.version, positions, updates)

    def commit(self, plan):
        if plan.version != self.version:
            raise RuntimeError("stale decode step plan")
        for sid, logical, physical in plan.updates:
            taken = self.free.pop()
            assert taken == physical
            self.tables[sid][logical] = physical
        for sid in self.ids:
            self.lengths[sid] += 1
        self.version += 1

    def publish(self, layout):
        layout.tables = tuple(tuple(r) for r in self.tables)
        layout.lengths = tuple(self.lengths)
        layout.free_pages = tuple(self.free)
        layout.version = self.version
