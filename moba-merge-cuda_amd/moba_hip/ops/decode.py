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


def metadata(table, lengths, ids, positions, delta, append):
    _lib.call("moba_hip_decode_metadata", table.data_ptr(), table.shape[1], lengths.data_ptr(),
              ids.data_ptr(), positions.data_ptr(), delta.data_ptr(), ids.numel(),
              1 if append else 0, _lib.stream_of(table.device))


def step(table, lengths, ids, positions, delta, k, v, kc, vc, chunk, means):
    """Fused prepared-decode prologue (metadata + append + closing-chunk mean)."""
    b, hk, d = k.shape
    _lib.call("moba_hip_decode_step", table.data_ptr(), table.shape[1], lengths.data_ptr(),
              ids.data_ptr(), positions.data_ptr(), delta.data_ptr(), b, k.data_ptr(),
              v.data_ptr(), DTYPE_CODE[k.dtype], kc.data_ptr(), vc.data_ptr(), kc.shape[1], hk, d,
              chunk, means.data_ptr(), means.shape[1], _lib.stream_of(k.device))


def fused_supported(hq, hkv, d, width, table_width) -> bool:
    return bool(_lib.load().moba_hip_decode_fused_supported(hq, hkv, d, width, table_width))


def fused_splits(nq, hkv) -> int:
    """Workgroups per (row, kv head): about two per CU over the whole launch."""
    return max(1, min(64, -(-512 // (nq * hkv))))


class FusedWork:
    """Persistent workspaces of ``fused``: the split partials."""
    __slots__ = ("splits", "part_o", "part_ml")

    def __init__(self, nq, hq, hkv, d, device, splits=None):
        self.splits = splits or fused_splits(nq, hkv)
        n = nq * hq * self.splits
        self.part_o = torch.empty((n, d), dtype=torch.float32, device=device)
        self.part_ml = torch.empty((n, 2), dtype=torch.float32, device=device)


def fused_args(q, k, v, kc, vc, table, lengths, ids, positions, delta, means, chunk, width,
               remote, dense, pos_mode, selected, work: FusedWork, out, lse):
    """Argument tuple of one ``moba_hip_decode_fused`` launch, without the
    stream (device pointers of the given tensors)."""
    nq, hq, d = q.shape
    return (q.data_ptr(), _lib.ptr(k), _lib.ptr(v), DTYPE_CODE[q.dtype], nq, hq, kc.shape[2], d,
            kc.data_ptr(), vc.data_ptr(), kc.shape[1], table.data_ptr(), table.shape[1],
            lengths.data_ptr(), ids.data_ptr(), positions.data_ptr(), _lib.ptr(delta),
            means.data_ptr(), means.shape[1], chunk, width, remote, 1 if dense else 0, pos_mode,
            work.splits, _lib.ptr(selected), work.part_o.data_ptr(), work.part_ml.data_ptr(),
            out.data_ptr(), lse.data_ptr())


def launch_fused(args, stream):
    _lib.call("moba_hip_decode_fused", *args, stream)


def fused(q, k, v, kc, vc, table, lengths, ids, positions, delta, means, chunk, width, remote,
          dense, pos_mode, selected, work: FusedWork, out, lse):
    """One-launch decode (route + attention; step mode also appends)."""
    launch_fused(fused_args(q, k, v, kc, vc, table, lengths, ids, positions, delta, means, chunk,
                            width, remote, dense, pos_mode, selected, work, out, lse),
                 _lib.stream_of(q.device))
