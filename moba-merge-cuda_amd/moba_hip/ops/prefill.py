"""Host side of the prefill path: chunk metadata and the kernel launch sequence.

``PrefillPlan`` restates calc_chunks (src/moba_opt/diagnostic.py:30-80) on the
host copy of cu_seqlens that validation already read, adds the tile lists the
kernels need, and uploads everything in one int32 buffer.  Plans are cached by
(cu_seqlens values, chunk, heads, device) -- the reference caches calc_chunks
by tensor object (lru_cache, diagnostic.py:30).
"""
from __future__ import annotations

import threading
from collections import OrderedDict

import torch

from . import _lib

DTYPE_CODE = {torch.bfloat16: 0, torch.float16: 1}


def attn_rows(head_dim):
    """Query rows per prefill tile (self tiles and expert tiles), as the
    library's kernels expect them for this head dim."""
    rows = _lib.load().moba_hip_prefill_rows(head_dim)
    if rows <= 0:
        raise ValueError(f"unsupported head_dim {head_dim}")
    return rows


def dkdv_keys(head_dim):
    """Keys per dK/dV workgroup: 4 wave pairs x 32 keys."""
    return 128


class PrefillPlan:
    """Chunk metadata + tile lists for one (cu_seqlens, chunk, Hq, Hkv) shape."""

    def __init__(self, cu, chunk, hq, hkv, head_dim, topk, device, fallback=False):
        self.cu = list(cu)
        self.head_dim = head_dim
        self.chunk = chunk
        self.hq, self.hkv = hq, hkv
        self.groups = hq // hkv
        self.block_rows = attn_rows(head_dim)
        BLOCK_ROWS = self.block_rows
        cu_chunk, chunk_batch, filtered = [0], [], []
        for b in range(len(cu) - 1):
            length = cu[b + 1] - cu[b]
            n = (length + chunk - 1) // chunk
            for i in range(n):
                if i + 1 < n:
                    filtered.append(len(chunk_batch))
                chunk_batch.append(b)
                cu_chunk.append(cu_chunk[-1] + min(chunk, length - i * chunk))
        self.cu_chunk, self.chunk_batch, self.filtered = cu_chunk, chunk_batch, filtered
        self.num_filtered = len(filtered)
        self.remote = min(topk - 1, self.num_filtered)
        self.fallback = fallback or self.remote == 0
        if self.fallback:
            # k=1 / no-candidate fallback: full causal attention per sequence
            # (grouped_attention.py:41-46) == one "chunk" per sequence, no remote.
            att_chunk = list(cu)
            self.remote = 0
        else:
            att_chunk = cu_chunk
        first = []
        for c, b in enumerate(chunk_batch):
            first.append(c if c == 0 or chunk_batch[c - 1] != b else first[-1])
        tiles = self._self_tile_order(att_chunk, hkv, BLOCK_ROWS)
        self.n_self_tiles = len(tiles)
        self.num_experts = self.num_filtered * hkv
        max_tiles = 0
        for c in filtered:
            ns = cu[chunk_batch[c] + 1] - cu_chunk[c + 1]
            max_tiles += hkv * ((self.groups * ns + BLOCK_ROWS - 1) // BLOCK_ROWS)
        # every (token, q head) row sits in at most `remote` experts, and an
        # expert's last tile may be partial: at most rows / BLOCK_ROWS + E
        # tiles.  (The remote kernels' grids are this bound; workgroups past
        # the actual count, known only on the device, return at once.)
        rows_bound = cu[-1] * hq * self.remote
        max_tiles = min(max_tiles, -(-rows_bound // BLOCK_ROWS) + self.num_experts)
        self.max_remote_tiles = max_tiles
        self.chunk_start = [cu_chunk[c] for c in filtered]
        # key-major backward tiles: (chunk, first key, filtered index or -1)
        self.kv_block = dkdv_keys(head_dim)
        fidx = {c: i for i, c in enumerate(filtered)}
        self.kv_tiles_list = self._kv_tile_order(att_chunk, fidx, cu, chunk_batch, cu_chunk)
        self.n_kv_tiles = len(self.kv_tiles_list) // 4
        # few kv heads leave too few key tiles to fill the chip: split each
        # tile's query rows over several workgroups (fp32 partials + reduce);
        # about 1536 workgroups in all (cfg2: 6 splits, 1.50-1.52 ms per step
        # against 1.53 with 4 and 8, 1.54-1.58 with 12-16)
        self.kv_splits = (max(1, min(8, 1536 // max(1, self.n_kv_tiles)))
                          if head_dim % 8 == 0 else 1)
        kv_flat = self.kv_tiles_list

        parts = OrderedDict(
            att_chunk=att_chunk, cu_chunk=cu_chunk, chunk_batch=chunk_batch, first_chunk=first,
            cu_seqlens=list(cu), filtered=filtered or [0], chunk_start=self.chunk_start or [0],
            self_tiles=[x for t in tiles for x in t] or [-1, 0, 0], kv_tiles=kv_flat or [-1, 0, -1, 0])
        flat, self._views = [], {}
        for name, vals in parts.items():
            self._views[name] = (len(flat), len(vals))
            flat.extend(vals)
        self.meta = torch.tensor(flat, dtype=torch.int32).to(device, non_blocking=False)

    N_XCD = 8  # workgroup L of a 1-D grid runs on XCD L % 8

    @classmethod
    def _self_tile_order(cls, att_chunk, hkv, rows):
        """Causal (self) work list: (chunk, first row, kv head) tiles of
        `rows` query rows; a tile attends min(first row + rows, length) keys.

        The tiles, listed kv head by kv head and chunk by chunk, are cut into
        8 contiguous runs of near-equal work, one per XCD, so the tiles that
        read one (chunk, kv head)'s keys share an L2.  In each run the tiles
        with more than a quarter of the largest tile's keys keep that order
        (largest first within a group); the smaller ones follow, largest
        first, and fill the run's tail.  Runs are padded with empty tiles
        (chunk -1) to a common length and concatenated: the kernels map
        workgroup L to run L % 8 (xcd_contiguous).
        """
        items = []
        for kh in range(hkv):
            for c in range(len(att_chunk) - 1):
                length = att_chunk[c + 1] - att_chunk[c]
                for r0 in sorted(range(0, length, rows), reverse=True):
                    items.append((min(r0 + rows, length), c, r0, kh))
        if not items:
            return []
        total = sum(it[0] for it in items)
        runs = [[] for _ in range(cls.N_XCD)]
        acc = 0
        for it in items:
            # the run this tile's midpoint falls in
            x = min(cls.N_XCD - 1, (2 * acc + it[0]) * cls.N_XCD // (2 * total))
            runs[x].append(it)
            acc += it[0]
        big = max(it[0] for it in items)
        out = []
        n = 0
        for x in range(cls.N_XCD):
            head = [it for it in runs[x] if 4 * it[0] > big]
            tail = sorted((it for it in runs[x] if 4 * it[0] <= big), key=lambda it: -it[0])
            runs[x] = [it[1:] for it in head + tail]
            n = max(n, len(runs[x]))
        for x in range(cls.N_XCD):
            out.extend(runs[x] + [(-1, 0, 0)] * (n - len(runs[x])))
        return out

    def _kv_tile_order(self, att_chunk, fidx, cu, chunk_batch, cu_chunk):
        """dK/dV work list: (chunk, first key, filtered index or -1, kv head).

        All key tiles of one (chunk, kv head) group go to one XCD, so the
        query rows they share are fetched into that XCD's L2 once; groups are
        dealt to XCDs in decreasing order of their query-row count.  Lists are
        padded with empty tiles (chunk -1) to a common length and interleaved
        so that entry L lands on XCD L % 8.
        """
        groups = []
        for c in range(len(att_chunk) - 1):
            length = att_chunk[c + 1] - att_chunk[c]
            f = -1 if self.fallback else fidx.get(c, -1)
            tail = 0 if f < 0 else cu[chunk_batch[c] + 1] - cu_chunk[c + 1]
            cost = self.groups * (length + tail * self.remote / max(1, self.num_filtered))
            tiles = list(range(0, length, self.kv_block))
            for kh in range(self.hkv):
                groups.append((cost, c, f, kh, tiles))
        groups.sort(key=lambda g: (-g[0], g[1], g[3]))
        per = [[] for _ in range(self.N_XCD)]
        load = [0.0] * self.N_XCD
        for cost, c, f, kh, tiles in groups:
            x = min(range(self.N_XCD), key=lambda i: (load[i], i))
            load[x] += cost
            per[x].extend((c, k0, f, kh) for k0 in tiles)
        n = max(len(p) for p in per) if per else 0
        out = []
        for i in range(n):
            for x in range(self.N_XCD):
                out.extend(per[x][i] if i < len(per[x]) else (-1, 0, -1, 0))
        return out

    def dev(self, name):
        off, n = self._views[name]
        return self.meta[off:off + n]

    def ptr(self, name):
        return self.dev(name).data_ptr()


_PLANS: "OrderedDict[tuple, PrefillPlan]" = OrderedDict()
_PLANS_LOCK = threading.Lock()


def get_plan(cu, chunk, hq, hkv, head_dim, topk, device, fallback=False):
    """The cached plan of a shape (16 most recent; safe to call from several
    threads: a plan is immutable once built)."""
    key = (tuple(cu), chunk, hq, hkv, head_dim, topk, str(device), fallback)
    with _PLANS_LOCK:
        plan = _PLANS.get(key)
        if plan is not None:
            _PLANS.move_to_end(key)
            return plan
    plan = PrefillPlan(cu, chunk, hq, hkv, head_dim, topk, device, fallback)
    with _PLANS_LOCK:
        _PLANS[key] = plan
        _PLANS.move_to_end(key)
        while len(_PLANS) > 16:
            _PLANS.popitem(last=False)
    return plan


class RouteResult:
    """Device routing state shared by the forward and the backward."""
    __slots__ = ("sel", "counts", "row_off", "tile_off", "rows", "means")


def route(plan: PrefillPlan, q, k, precision: int, want_gate=False):
    """Chunk means, gate + stable top-k, expert packing.  Returns RouteResult
    (and the masked gate [F,Hq,T] when ``want_gate``)."""
    T, hq, d = q.shape
    dev = q.device
    st = _lib.stream_of(dev)
    code = DTYPE_CODE[q.dtype]
    r = RouteResult()
    F, R, E = plan.num_filtered, plan.remote, plan.num_experts
    r.means = torch.empty((F, plan.hkv, d), dtype=torch.float32, device=dev)
    r.sel = torch.empty((T, hq, R), dtype=torch.int32, device=dev)
    r.counts = torch.empty(E, dtype=torch.int32, device=dev)
    r.row_off = torch.empty(E + 1, dtype=torch.int32, device=dev)
    r.tile_off = torch.empty(E + 1, dtype=torch.int32, device=dev)
    r.rows = torch.empty(max(1, T * hq * R), dtype=torch.int32, device=dev)
    gate = torch.empty((F, hq, T), dtype=torch.float32, device=dev) if want_gate else None
    work = torch.empty(max(1, _lib.load().moba_hip_pack_experts_work(T, hq, plan.hkv, F)),
                       dtype=torch.int32, device=dev)
    _lib.call("moba_hip_chunk_means", k.data_ptr(), code, T, plan.hkv, d,
              plan.ptr("chunk_start"), F, plan.chunk, precision, r.means.data_ptr(), st)
    _lib.call("moba_hip_route_prefill", q.data_ptr(), code, T, hq, plan.hkv, d,
              r.means.data_ptr(), plan.ptr("cu_chunk"), len(plan.chunk_batch),
              plan.ptr("chunk_batch"), plan.ptr("first_chunk"), R, F, r.sel.data_ptr(),
              _lib.ptr(gate), st)
    _lib.call("moba_hip_pack_experts", r.sel.data_ptr(), T, hq, plan.hkv, R,
              plan.ptr("cu_chunk"), plan.ptr("chunk_batch"), plan.ptr("cu_seqlens"),
              plan.ptr("filtered"), F, plan.block_rows, r.counts.data_ptr(), r.row_off.data_ptr(),
              r.tile_off.data_ptr(), r.rows.data_ptr(), work.data_ptr(), st)
    return (r, gate) if want_gate else r


def forward(plan: PrefillPlan, q, k, v, rt: RouteResult | None):
    """Sparse attention + merge.  Returns (out [T,Hq,D], lse [T,Hq] fp32)."""
    T, hq, d = q.shape
    dev = q.device
    R = plan.remote
    out = torch.empty_like(q)
    lse = torch.empty((T, hq), dtype=torch.float32, device=dev)
    part_o = part_ml = None
    if R:
        part_o = torch.empty((T * hq * R, d), dtype=q.dtype, device=dev)
        part_ml = torch.empty((T * hq * R, 2), dtype=torch.float32, device=dev)
    _lib.call("moba_hip_prefill_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(),
              DTYPE_CODE[q.dtype], T, hq, plan.hkv, d, d ** -0.5,
              plan.ptr("att_chunk"), plan.ptr("self_tiles"), plan.n_self_tiles,
              _lib.ptr(rt.sel) if R else None, R, plan.ptr("filtered"), plan.num_experts,
              _lib.ptr(rt.tile_off) if R else None, _lib.ptr(rt.row_off) if R else None,
              _lib.ptr(rt.counts) if R else None, _lib.ptr(rt.rows) if R else None,
              plan.max_remote_tiles if R else 0, _lib.ptr(part_o), _lib.ptr(part_ml),
              out.data_ptr(), lse.data_ptr(), _lib.stream_of(dev))
    return out, lse


# Optional (start, stop) torch.cuda.Event pair recorded around the key-major
# dK/dV launch of every backward (used by bench.py to time that kernel live).
DKDV_EVENTS = None


def backward(plan: PrefillPlan, q, k, v, out, lse, dout, rt: RouteResult | None):
    """Gradients (dq, dk, dv) of ``forward`` for the upstream gradient ``dout``."""
    T, hq, d = q.shape
    dev = q.device
    R = plan.remote
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    delta = torch.empty(2 * T * hq, dtype=torch.float32, device=dev)
    part_dq = torch.empty((T * hq * R, d), dtype=q.dtype, device=dev) if R else None
    args = [q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
            dout.data_ptr(), lse.data_ptr(), DTYPE_CODE[q.dtype], T, hq, plan.hkv, d,
            d ** -0.5, plan.ptr("att_chunk"), plan.ptr("self_tiles"), plan.n_self_tiles,
            plan.ptr("kv_tiles"), plan.n_kv_tiles,
            _lib.ptr(rt.sel) if R else None, R, plan.ptr("filtered"), plan.num_experts,
            _lib.ptr(rt.tile_off) if R else None, _lib.ptr(rt.row_off) if R else None,
            _lib.ptr(rt.counts) if R else None, _lib.ptr(rt.rows) if R else None,
            plan.max_remote_tiles if R else 0, delta.data_ptr(), _lib.ptr(part_dq),
            dq.data_ptr(), dk.data_ptr(), dv.data_ptr()]
    ks = plan.kv_splits
    # row-split workspace: the device-built schedule, then fp32 partial slots
    part_dkv = (torch.empty(_lib.load().moba_hip_prefill_bwd_work(plan.n_kv_tiles, ks, d),
                            dtype=torch.uint8, device=dev) if ks > 1 else None)
    # expert rows of q / dO / lse / delta packed contiguously for the key-major kernel
    pack = (torch.empty(T * hq * R * (4 * d + 8), dtype=torch.uint8, device=dev)
            if R and d <= 128 else None)
    st = _lib.stream_of(dev)
    _lib.call("moba_hip_prefill_bwd", *args, 1, ks, _lib.ptr(part_dkv), _lib.ptr(pack), st)
    events = DKDV_EVENTS
    if events is not None:
        events[0].record()
    _lib.call("moba_hip_prefill_bwd", *args, 2, ks, _lib.ptr(part_dkv), _lib.ptr(pack), st)
    if events is not None:
        events[1].record()
    return dq, dk, dv
