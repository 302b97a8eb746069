"""Argument contract of the decode caches.

The accepted inputs and the ValueError messages are those of the reference's
caches (src/moba_opt/kv_cache.py:16-33,101-126,132-140,193-205), so callers
see the same errors.  As in :mod:`moba_hip.baseline_adapter`, each check is
written as a rule (predicate that must hold, message) and rules are tried in
order; the first that fails raises.
"""
from __future__ import annotations

import torch

from .baseline_adapter import _require
from .cache_layout import positive_int


def int_vector(values, name):
    """A Python sequence or CPU int32/int64 vector of ints -> tuple."""
    if isinstance(values, torch.Tensor):
        _require([(lambda: values.device.type == "cpu"
                   and values.dtype in (torch.int32, torch.int64) and values.dim() == 1,
                   f"{name} must be a Python sequence or CPU int32/int64 vector")])
        values = values.tolist()
    _require([
        (lambda: isinstance(values, (tuple, list)),
         f"{name} must be a Python sequence or CPU integer vector"),
        (lambda: all(isinstance(x, int) and not isinstance(x, bool) for x in values),
         f"{name} must contain integers"),
    ])
    return tuple(values)


def decode_mode(mode, topk):
    """True when the call attends densely (mode 'dense', or topk 1: only the
    current chunk would be routed, which the reference also runs dense)."""
    _require([(lambda: mode in ("moba", "dense"), "mode must be moba or dense")])
    k = positive_int(topk, "topk")
    _require([(lambda: k <= 9, "topk must be in [1,9]")])
    return mode == "dense" or k == 1


def constructor(batch_size, max_seq_len, page_size, num_kv_heads, head_dim, chunk_size, dtype,
                device):
    """Checked constructor arguments (every check runs before any GPU work)."""
    dims = dict(batch_size=positive_int(batch_size, "batch_size"),
                max_seq_len=positive_int(max_seq_len, "max_seq_len"),
                page_size=positive_int(page_size, "page_size"),
                num_kv_heads=positive_int(num_kv_heads, "num_kv_heads"),
                head_dim=positive_int(head_dim, "head_dim"))
    _require([(lambda: dims["head_dim"] <= 256, "decode head_dim must be in [1,256]")])
    dims["chunk_size"] = positive_int(chunk_size, "chunk_size")
    dev = torch.device(device)
    _require([
        (lambda: dims["chunk_size"] <= 1024, "cache chunk_size must be <=1024"),
        (lambda: dtype in (torch.bfloat16, torch.float16), "cache dtype must be BF16 or FP16"),
        (lambda: dev.type == "cuda", "cache device must be CUDA"),
    ])
    return dims, dev


def tensor(t, name, *, device, dtype, head_dim, heads=None, tokens=None, finite=True):
    """An [N,H,D] input of the cache's device and dtype, inference-only, with a
    contiguous last dimension (kv_cache.py:110-126)."""
    _require([
        (lambda: isinstance(t, torch.Tensor) and t.dim() == 3, f"{name} must be [N,H,D]"),
        (lambda: t.device == device and t.dtype == dtype,
         f"{name} must match cache device and dtype"),
        (lambda: not t.requires_grad, "KV cache/decode is inference-only; detach Q/K/V"),
        (lambda: t.shape[0] >= 1 and t.shape[1] >= 1 and t.shape[2] == head_dim,
         f"{name} has an invalid shape"),
        (lambda: t.stride(-1) == 1, f"{name} last dimension must be contiguous"),
        (lambda: heads is None or t.shape[1] == heads, f"{name} KV head count differs from cache"),
        (lambda: tokens is None or t.shape[0] == tokens, f"{name} token count differs"),
        (lambda: not finite or bool(torch.isfinite(t).all()), f"{name} contains NaN/Inf"),
    ])


def finite(t, name):
    _require([(lambda: bool(torch.isfinite(t).all()), f"{name} contains NaN/Inf")])


def tensors(specs, *, device, dtype, head_dim):
    """`tensor` for each (t, name, kwargs) in order, raising what those calls
    in sequence would raise first; the NaN/Inf test of all inputs reads one
    flag (one host synchronisation instead of one per tensor).  A callable
    `tokens` is evaluated only once the inputs before it passed their checks
    (so `lambda: k.shape[0]` never reads an unchecked k)."""
    for i, (t, name, kw) in enumerate(specs):
        if callable(kw.get("tokens")):
            kw = dict(kw, tokens=kw["tokens"]())
        try:
            tensor(t, name, device=device, dtype=dtype, head_dim=head_dim, finite=False, **kw)
        except ValueError:
            for t0, n0, _ in specs[:i]:  # an earlier input's NaN/Inf comes first
                finite(t0, n0)
            raise
    if len(specs) == 1 or not bool(torch.stack([torch.isfinite(t).all() for t, _, _ in specs]).all()):
        for t, name, _ in specs:
            finite(t, name)


def append_counts(token_count, ids, cu_seqlens):
    """Tokens per sequence from cu_seqlens (one token each when None)."""
    cu = tuple(range(len(ids) + 1)) if cu_seqlens is None else int_vector(cu_seqlens, "cu_seqlens")
    _require([(lambda: len(cu) == len(ids) + 1 and cu[0] == 0 and cu[-1] == token_count,
               "append cu_seqlens must start at 0 and end at N")])
    counts = tuple(b - a for a, b in zip(cu, cu[1:]))
    _require([(lambda: all(n > 0 for n in counts), "append sequences must be nonempty")])
    return counts


def query_grid(q, hkv):
    _require([
        (lambda: q.shape[1] % hkv == 0, "Hq must be a multiple of Hkv"),
        (lambda: q.shape[0] * q.shape[1] < 2 ** 31, "query grid exceeds int32 capacity"),
    ])
