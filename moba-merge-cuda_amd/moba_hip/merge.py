"""Standalone global-softmax merge (the reference's only native entry).

Drop-in for ``merge_forward_cuda`` (src/moba_opt/ops/merge_cuda.py:32-60,
binding src/moba_opt/ops/bindings.cpp:6-22): same arguments, same checks and
messages, returns ``(O, LSE)``.  The merge itself is ``moba_hip_merge``: no
atomics, remote partials of a row taken in ascending index order, so the
result is always deterministic (``deterministic`` is accepted and documents
that).  ``check_capacity`` reads two status words after the launch (one small
device-to-host copy, like the reference's overflow check) and raises.

The prefill path does not call this: its merge is fused into the self-branch
forward epilogue.  This entry serves callers that hold (o, lse) partials of
their own.
"""
from __future__ import annotations

import torch

from .ops import _lib

_DTYPES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def merge_forward(self_out, self_lse, remote_out, remote_lse, mapping, kmax=None,
                  check_capacity=True, deterministic=False):
    """self_out [T,H,D] (fp32/bf16/fp16, GPU); self_lse [T,H] fp32;
    remote_out [M,1,D] or [M,D]; remote_lse [M]; mapping [M] int32/int64.
    Returns (O [T,H,D] in the input dtype, LSE [T,H] fp32)."""
    if not isinstance(deterministic, bool):
        raise ValueError("deterministic must be bool")
    if mapping.dim() != 1 or mapping.dtype not in (torch.int32, torch.int64):
        raise ValueError("mapping must be a 1D int32/int64 tensor")
    if not (self_out.is_cuda and self_out.dim() == 3):
        raise RuntimeError("self_out must be CUDA [T,H,D]")
    dev = self_out.device
    for t in (self_lse, remote_out, remote_lse, mapping):
        if not (t.is_cuda and t.device == dev):
            raise RuntimeError("all merge inputs must be CUDA tensors on self_out.device")
    if remote_out.dtype != self_out.dtype:
        raise RuntimeError("remote_out dtype must match self_out")
    if remote_lse.dim() != 1:
        raise RuntimeError("mapping and remote_lse must be 1D")
    if not (remote_out.dim() == 2 or (remote_out.dim() == 3 and remote_out.shape[1] == 1)):
        raise RuntimeError("remote_out must be [M,D] or [M,1,D]")
    if self_out.dtype not in _DTYPES:
        raise RuntimeError("self_out dtype must be fp32/bf16/fp16")
    T, H, D = self_out.shape
    P, M = T * H, mapping.numel()
    if kmax is None:
        kmax = 1
        if M:
            # entries outside [0, P) are counted apart (bin P), so the
            # kernel's range check reports them rather than bincount
            m = mapping.long()
            m = torch.where((m >= 0) & (m < P), m, torch.full_like(m, P))
            kmax = max(1, int(torch.bincount(m, minlength=P + 1)[:P].max().item()))
    kmax = int(kmax)
    if not 1 <= kmax <= 8:
        raise RuntimeError("kmax must be in [1,8]")
    if not (T > 0 and H > 0 and 8 <= D <= 256 and D % 8 == 0):
        raise RuntimeError("nonempty T,H required; head_dim must be a multiple of 8 in [8,256]")
    if tuple(self_lse.shape) != (T, H):
        raise RuntimeError("self_lse must be [T,H]")
    if remote_out.numel() != M * D:
        raise RuntimeError("remote_out shape mismatch")
    if remote_lse.numel() != M:
        raise RuntimeError("remote_lse shape mismatch")
    so = self_out.contiguous()
    sl = self_lse.to(torch.float32).contiguous()
    ro = remote_out.reshape(M, D).contiguous()
    rl = remote_lse.to(torch.float32).contiguous()
    mp = mapping.to(torch.int64).contiguous()
    lib = _lib.load()
    nbytes = lib.moba_hip_merge_work(P, M)
    if nbytes < 0:
        raise RuntimeError("mapping exceeds int32 indexing capacity")
    with torch.cuda.device(dev):
        work = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        status = torch.empty(2, dtype=torch.int32, device=dev)
        out = torch.empty_like(so)
        lse = torch.empty((T, H), dtype=torch.float32, device=dev)
        _lib.call("moba_hip_merge", so.data_ptr(), sl.data_ptr(), ro.data_ptr(), rl.data_ptr(),
                  mp.data_ptr(), _DTYPES[so.dtype], T, H, D, M, kmax, work.data_ptr(),
                  status.data_ptr(), out.data_ptr(), lse.data_ptr(), _lib.stream_of(dev))
        if check_capacity and M:
            bad_range, over = status.tolist()
            if bad_range:
                raise RuntimeError("mapping entries must be in [0,T*H)")
            if over:
                raise RuntimeError(
                    f"capacity exceeded: a query row has more remote contributions than kmax "
                    f"allows (kmax={kmax}); refusing to return a partially merged row")
    return out, lse
