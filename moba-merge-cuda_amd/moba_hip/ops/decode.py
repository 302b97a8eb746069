"""Launch wrappers of the decode entry points of libmoba_hip.so."""
from __future__ import annotations

import torch

from . import _lib

DTYPE_CODE = {torch.bfloat16: 0, torch.float16: 1}


def work_items(hq, hkv, nslot) -> int:
    return _lib.load().moba_hip_decode_work_items(hq, hkv, nslot)


class RouteWork:
    """Route outputs consumed by ``attention``: slot lists + the work list."""
    __slots__ = ("selected", "items", "counts")

    def __init__(self, nq, hq, hkv, remote, device):
        nhb = -(-(hq // hkv) // 16)
        self.selected = torch.empty((nq, hq, remote + 1), dtype=torch.int32, device=device)
        self.items = torch.empty((nq * hkv * nhb, work_items(hq, hkv, remote + 1), 4),
                                 dtype=torch.int32, device=device)
        self.counts = torch.empty(nq * hkv * nhb, dtype=torch.int32, device=device)


def append_tokens(k, v, kc, vc, table, token_seq, token_pos):
    n, hk, d = k.shape
    _lib.call("moba_hip_paged_append", k.data_ptr(), v.data_ptr(), DTYPE_CODE[k.dtype], n, hk, d,
              kc.data_ptr(), vc.data_ptr(), kc.shape[1], table.data_ptr(), table.shape[1],
              token_seq.data_ptr(), token_pos.data_ptr(), _lib.stream_of(k.device))


def block_means(kc, table, means, item_seq, item_chunk_or_pos, chunk, mode=0):
    n = item_seq.numel()
    if n == 0:
        return
    hk, d = kc.shape[2:]
    _lib.call("moba_hip_block_means", kc.data_ptr(), DTYPE_CODE[kc.dtype], hk, d, kc.shape[1],
              table.data_ptr(), table.shape[1], item_seq.data_ptr(), item_chunk_or_pos.data_ptr(),
              n, mode, chunk, means.data_ptr(), means.shape[1], _lib.stream_of(kc.device))


def route(q, means, q_seq, q_pos, chunk, width, remote, scores, work: RouteWork):
    nq, hq, d = q.shape
    _lib.call("moba_hip_decode_route", q.data_ptr(), DTYPE_CODE[q.dtype], nq, hq, means.shape[2],
              d, means.data_ptr(), means.shape[1], q_seq.data_ptr(), q_pos.data_ptr(), chunk,
              width, remote, _lib.ptr(scores), work.selected.data_ptr(), work.items.data_ptr(),
              work.counts.data_ptr(), _lib.stream_of(q.device))


def attention(q, kc, vc, table, lengths, q_seq, q_pos, work, out, lse, chunk, dense,
              max_chunks_bound, part_o=None, part_ml=None):
    """Paged MoBA / dense attention.  ``work`` is the RouteWork of the route
    (ignored when dense); workspaces are allocated here unless given."""
    nq, hq, d = q.shape
    nslot = max_chunks_bound if dense else work.selected.shape[-1]
    if part_o is None:
        n = nq * hq * nslot
        part_o = torch.empty((n, d), dtype=torch.float32, device=q.device)
        part_ml = torch.empty((n, 2), dtype=torch.float32, device=q.device)
    _lib.call("moba_hip_paged_attention", q.data_ptr(), DTYPE_CODE[q.dtype], nq, hq, kc.shape[2],
              d, kc.data_ptr(), vc.data_ptr(), kc.shape[1], table.data_ptr(), table.shape[1],
              lengths.data_ptr(), q_seq.data_ptr(), q_pos.data_ptr(),
              None if dense else work.selected.data_ptr(), 0 if dense else nslot,
              None if dense else work.items.data_ptr(), None if dense else work.counts.data_ptr(),
              1 if dense else 0, chunk, max_chunks_bound, part_o.data_ptr(), part_ml.data_ptr(),
              out.data_ptr(), lse.data_ptr(), _lib.stream_of(q.device))


def fused_supported(hq, hkv, d, width, table_width) -> bool:
    return bool(_lib.load().moba_hip_decode_fused_supported(hq, hkv, d, width, table_width))


def fused_heads(hq, hkv) -> int:
    """(Virtual) kv heads per row of a fused launch: each kv head with more
    than 16 q heads is served as equal groups of at most 16."""
    return hkv * _lib.load().moba_hip_decode_fused_groups(hq, hkv)


def fused_splits(nq, hkv) -> int:
    """Workgroups per (row, kv head): about one (8-wave workgroup) per CU
    over the whole launch."""
    return max(1, min(64, -(-SCHED_WORKGROUPS // (nq * hkv))))


# Workgroups of a scheduled decode launch (one 8-wave workgroup per CU) and
# the split cap.
SCHED_WORKGROUPS = 256
SCHED_MAX_SPLITS = 64


def expected_union_tokens(pos, group, remote, chunk, dense=False) -> float:
    """Expected tokens a (row, kv head) attends at position ``pos``: the
    current chunk up to pos, plus the closed chunks that at least one of the
    ``group`` q heads selects when each picks ``remote`` of the closed chunks
    (the expected coverage of independent uniform picks)."""
    if dense:
        return float(pos + 1)
    cur = pos // chunk
    own = pos - cur * chunk + 1
    if cur == 0 or remote == 0:
        return float(own)
    picks = min(remote, cur)
    covered = cur * (1.0 - (1.0 - picks / cur) ** group)
    return own + chunk * covered


def sched_workgroups(nq, hkv, workgroups=SCHED_WORKGROUPS, max_splits=SCHED_MAX_SPLITS) -> int:
    """Grid size of a scheduled launch: fixed for a given batch shape."""
    return _lib.load().moba_prep_sched_workgroups(nq, hkv, workgroups, max_splits)


def fused_schedule(positions, hkv, group, remote, chunk, dense=False,
                   workgroups=SCHED_WORKGROUPS, max_splits=SCHED_MAX_SPLITS):
    """The split schedule the prepared-decode driver uploads (computed by
    ``moba_prep_schedule``): split counts per (row, kv head) by the expected
    attended tokens (``expected_union_tokens``) plus the route every
    workgroup recomputes (0.6 tokens per (q head, closed chunk)); each
    workgroup beyond one per row goes to the row whose workgroups carry the
    most (route + expected tokens per split), each count in [1, max_splits],
    over exactly ``sched_workgroups`` workgroups.  Returns (schedule int32 list: the workgroup entries
    (row * hkv + kv head, split, splits of that row) interleaved across rows,
    then the split counts; the split counts; the number of workgroups)."""
    import numpy as np
    rows = len(positions) * hkv
    total = sched_workgroups(len(positions), hkv, workgroups, max_splits)
    pos = np.asarray(positions, dtype=np.int32)
    entries = np.zeros(3 * total + rows, dtype=np.int32)
    splits = np.zeros(rows, dtype=np.int32)
    _lib.call("moba_prep_schedule", pos.ctypes.data, len(positions), hkv, group, remote, chunk,
              int(dense), workgroups, max_splits, entries.ctypes.data, splits.ctypes.data)
    return entries.tolist(), splits.tolist(), total


class FusedWork:
    """Workspaces of ``fused``: the split partials, and with ``scheduled`` a
    device schedule of ``sched_workgroups`` workgroups (see
    ``fused_schedule``) that the prepared-decode driver keeps current."""
    __slots__ = ("splits", "part_o", "part_ml", "sched", "n_sched")

    def __init__(self, nq, hq, hkv, d, device, splits=None, scheduled=False):
        hv = fused_heads(hq, hkv)
        self.splits = splits or (SCHED_MAX_SPLITS if scheduled else fused_splits(nq, hv))
        n = nq * hq * self.splits
        self.part_o = torch.empty((n, d), dtype=torch.float32, device=device)
        self.part_ml = torch.empty((n, 2), dtype=torch.float32, device=device)
        self.sched, self.n_sched = None, 0
        if scheduled:
            self.n_sched = sched_workgroups(nq, hv, max_splits=self.splits)
            self.sched = torch.zeros(3 * self.n_sched + nq * hv, dtype=torch.int32,
                                     device=device)


def fused_args(q, k, v, kc, vc, table, lengths, ids, positions, delta, means, chunk, width,
               remote, dense, pos_mode, selected, work: FusedWork, out, lse):
    """Argument tuple of one ``moba_hip_decode_fused`` launch, without the
    stream (device pointers of the given tensors)."""
    nq, hq, d = q.shape
    return (q.data_ptr(), _lib.ptr(k), _lib.ptr(v), DTYPE_CODE[q.dtype], nq, hq, kc.shape[2], d,
            kc.data_ptr(), vc.data_ptr(), kc.shape[1], table.data_ptr(), table.shape[1],
            lengths.data_ptr(), ids.data_ptr(), positions.data_ptr(), _lib.ptr(delta),
            means.data_ptr(), means.shape[1], chunk, width, remote, 1 if dense else 0, pos_mode,
            work.splits, _lib.ptr(work.sched), work.n_sched, _lib.ptr(selected),
            work.part_o.data_ptr(), work.part_ml.data_ptr(), out.data_ptr(), lse.data_ptr())


def fused(q, k, v, kc, vc, table, lengths, ids, positions, delta, means, chunk, width, remote,
          dense, pos_mode, selected, work: FusedWork, out, lse):
    """One-launch decode (route + attention; step mode also appends)."""
    _lib.call("moba_hip_decode_fused",
              *fused_args(q, k, v, kc, vc, table, lengths, ids, positions, delta, means, chunk,
                          width, remote, dense, pos_mode, selected, work, out, lse),
              _lib.stream_of(q.device))
