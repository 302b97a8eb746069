"""Input/config contract of the prefill entry points.

The accepted envelope and the ValueError messages follow
src/moba_opt/baseline_adapter.py:13-76 so callers of the reference see the same
errors: q/k/v ``[T,H,D]`` bf16/fp16 on the GPU with a contiguous last
dimension, D a multiple of 8 in [8,256], Hq a multiple of Hkv, ``cu_seqlens``
a strictly increasing int32 vector from 0 to T, ``max_seqlen`` equal to the
longest sequence, ``chunk_size`` > 0, ``topk`` in [1,9], causal only, no dropout.
The checks are table-driven here: each rule is (predicate that must hold, message).
"""
import numbers
import threading
import weakref
from collections import OrderedDict

import torch

SUPPORTED_DTYPES = (torch.bfloat16, torch.float16)
MAINLINE_HEAD_DIMS = tuple(range(8, 257, 8))


def _positive_int(value, name):
    if isinstance(value, bool) or not isinstance(value, numbers.Integral) or value < 1:
        raise ValueError(f"{name} must be a positive integer")
    return int(value)


def _require(rules):
    for ok, message in rules:
        if not ok():
            raise ValueError(message() if callable(message) else message)


def validate_shapes(q_shape, k_shape, v_shape, allow_gqa=False):
    """Pure CPU shape contract; returns the GQA group size Hq // Hkv."""
    shapes = (q_shape, k_shape, v_shape)
    hq, hkv = q_shape[1] if len(q_shape) > 1 else 0, k_shape[1] if len(k_shape) > 1 else 0
    _require([
        (lambda: all(len(s) == 3 and min(s) >= 1 for s in shapes),
         "q/k/v must be nonempty [T,H,D]"),
        (lambda: k_shape == v_shape and q_shape[0] == k_shape[0] and q_shape[2] == k_shape[2],
         "q/k/v must share T,D and k/v must share shape"),
        (lambda: q_shape[2] in MAINLINE_HEAD_DIMS, "head_dim must be a multiple of 8 in [8,256]"),
        (lambda: hq % hkv == 0 and (allow_gqa or hq == hkv),
         "Hq must be divisible by Hkv" if allow_gqa
         else "Hq must be divisible by Hkv; this entry is MHA only"),
    ])
    return hq // hkv


def validate_config(config):
    _positive_int(config.get("chunk_size"), "chunk_size")
    topk = _positive_int(config.get("topk"), "topk")
    _require([
        (lambda: topk <= 9, "topk must be in [1,9] (at most 8 remote contributions)"),
        (lambda: config.get("causal", True) is True and config.get("dropout", 0.0) == 0,
         "only causal=True, dropout=0 are supported"),
    ])


def _check_tensor(name, t, q):
    _require([
        (lambda: isinstance(t, torch.Tensor), f"{name} must be a Tensor"),
        (lambda: t.dim() == 3, lambda: f"{name} must be [T,H,D], got shape {tuple(t.shape)}"),
        (lambda: t.dtype in SUPPORTED_DTYPES,
         lambda: f"{name} dtype {t.dtype} not in {SUPPORTED_DTYPES}"),
        (lambda: t.is_cuda, f"{name} must be on CUDA"),
        (lambda: t.device == q.device and t.dtype == q.dtype, "q/k/v must share device and dtype"),
        (lambda: t.stride(-1) == 1, "q/k/v last dimension must be contiguous"),
    ])


# Host copies of validated cu_seqlens tensors: (weak reference, torch version
# counter, list), keyed by id().  Reading cu_seqlens to the host synchronises
# the stream (about 0.2 ms of idle GPU per prefill step); the same tensor,
# not modified in place since (torch bumps its version counter on every
# in-place write), reuses its copy.  Writes that bypass torch (raw pointers)
# are not seen: pass a new tensor after such a write.  Inference-mode tensors
# have no version counter and are read on every call.
_CU_HOST = OrderedDict()
_CU_HOST_MAX = 16
_CU_LOCK = threading.Lock()


def _host_cu(cu_t):
    if cu_t.is_inference():
        return cu_t.tolist()
    key = id(cu_t)
    with _CU_LOCK:
        hit = _CU_HOST.get(key)
        if hit is not None and hit[0]() is cu_t and hit[1] == cu_t._version:
            _CU_HOST.move_to_end(key)
            return hit[2]
    cu = cu_t.tolist()
    with _CU_LOCK:
        _CU_HOST[key] = (weakref.ref(cu_t), cu_t._version, cu)
        _CU_HOST.move_to_end(key)
        while len(_CU_HOST) > _CU_HOST_MAX:
            _CU_HOST.popitem(last=False)
    return cu


def _validate(q, k, v, cu_seqlens, *, allow_gqa=False, max_seqlen=None, config=None):
    """Full contract; returns the host copy of cu_seqlens (one D2H read, or
    none for a tensor read before and unchanged since)."""
    for name, t in (("q", q), ("k", k), ("v", v)):
        _check_tensor(name, t, q)
    validate_shapes(tuple(q.shape), tuple(k.shape), tuple(v.shape), allow_gqa)
    cu_t = cu_seqlens
    _require([
        (lambda: isinstance(cu_t, torch.Tensor), "cu_seqlens must be a Tensor"),
        (lambda: cu_t.dtype == torch.int32 and cu_t.is_cuda, "cu_seqlens must be CUDA int32"),
        (lambda: cu_t.device == q.device and cu_t.dim() == 1 and cu_t.numel() >= 2,
         "cu_seqlens must be 1D [B+1], B>=1, on q.device"),
        (lambda: cu_t.is_contiguous(), "cu_seqlens must be contiguous"),
    ])
    cu = list(_host_cu(cu_t))
    lengths = [b - a for a, b in zip(cu, cu[1:])]
    _require([(lambda: cu[0] == 0 and cu[-1] == q.shape[0] and min(lengths) > 0,
               f"cu_seqlens must start at 0, end at T, strictly increase (non-empty seqs): {cu}")])
    if max_seqlen is not None and _positive_int(max_seqlen, "max_seqlen") != max(lengths):
        raise ValueError("max_seqlen must equal the maximum length in cu_seqlens")
    if config is not None:
        validate_config(config)
    return cu
