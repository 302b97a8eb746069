"""ctypes/numpy front end of the CPU oracle (``moba_oracle.c``).

TEST INFRASTRUCTURE ONLY.  Imported by ``tests/``, by ``__graft_entry__.smoke()``
(as the checker) and by ``bench.py``'s ``cpu_baseline`` leg; the product package
never imports it.

Host-side metadata helpers restate ``calc_chunks``
(src/moba_opt/diagnostic.py:30-80) on Python lists.  The heavy functions call the
C oracle: canonical FP32 routing (bit-exact target of the HIP routing kernels)
and FP64 fixed-route attention forward/backward, merge and decode attention.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libmoba_oracle.so"
DTYPE_CODE = {"bfloat16": 0, "float16": 1}

_lib = None


def build(force: bool = False) -> Path:
    """Compile the oracle with gcc (no FMA contraction; OpenMP)."""
    src = HERE / "moba_oracle.c"
    if force or not LIB_PATH.exists() or LIB_PATH.stat().st_mtime < src.stat().st_mtime:
        LIB_PATH.parent.mkdir(exist_ok=True)
        tmp = LIB_PATH.with_suffix(f".so.{os.getpid()}")
        subprocess.check_call(["gcc", "-O2", "-ffp-contract=off", "-fopenmp", "-fPIC", "-shared",
                               str(src), "-o", str(tmp), "-lm"])
        os.replace(tmp, LIB_PATH)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        _lib.oracle_round_to_dtype.restype = ctypes.c_float
        _lib.oracle_round_to_dtype.argtypes = [ctypes.c_float, ctypes.c_int]
        _lib.oracle_stable_topk.restype = ctypes.c_int
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def set_threads(n: int) -> None:
    lib().oracle_set_threads(int(n))


# ------------------------------------------------------------------ metadata

def calc_chunks(cu: list[int], chunk: int):
    """calc_chunks (diagnostic.py:30-80) on host lists.

    Returns (cu_chunk, chunk_to_batch, filtered): per-sequence chunks of
    ``chunk`` tokens with a possibly short tail; every chunk except each
    sequence's last is a routing candidate.
    """
    cu_chunk, chunk_batch, filtered = [0], [], []
    for b in range(len(cu) - 1):
        length = cu[b + 1] - cu[b]
        n = (length + chunk - 1) // chunk
        for i in range(n):
            if i + 1 < n:
                filtered.append(len(chunk_batch))
            chunk_batch.append(b)
            cu_chunk.append(cu_chunk[-1] + min(chunk, length - i * chunk))
    return cu_chunk, chunk_batch, filtered


def bits16(t) -> np.ndarray:
    """uint16 bit pattern of a bf16/fp16 torch tensor (CPU copy)."""
    import torch
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


# ------------------------------------------------------------ routing (fp32)

def chunk_means(k_bits: np.ndarray, dtype: int, cu_chunk, filtered, chunk: int, precision: int):
    T, hkv, d = k_bits.shape
    starts = np.ascontiguousarray([cu_chunk[c] for c in filtered], dtype=np.int32)
    out = np.zeros((len(filtered), hkv, d), dtype=np.float32)
    kb = np.ascontiguousarray(k_bits)
    lib().oracle_chunk_means(_p(kb), dtype, T, hkv, d, _p(starts), len(filtered), chunk,
                             precision, _p(out))
    return out


def route_prefill(q_bits, dtype, means, cu_chunk, chunk_batch, remote, want_gate=False):
    T, hq, d = q_bits.shape
    hkv = means.shape[1]
    nchunk = len(chunk_batch)
    F = means.shape[0]
    cc = np.ascontiguousarray(cu_chunk, dtype=np.int32)
    cb = np.ascontiguousarray(chunk_batch, dtype=np.int32)
    sel = np.zeros((T, hq, remote), dtype=np.int32)
    gate = np.zeros((F, hq, T), dtype=np.float32) if want_gate else None
    qb = np.ascontiguousarray(q_bits)
    mb = np.ascontiguousarray(means, dtype=np.float32)
    lib().oracle_route_prefill(_p(qb), dtype, T, hq, hkv, d, _p(mb), _p(cc), nchunk, _p(cb),
                               remote, _p(gate) if gate is not None else None, _p(sel))
    return sel, gate


def stable_topk(scores: np.ndarray, k: int):
    s = np.ascontiguousarray(scores, dtype=np.float32)
    idx = np.zeros(max(k, 1), dtype=np.int32)
    val = np.zeros(max(k, 1), dtype=np.float32)
    lib().oracle_stable_topk(_p(s), s.size, k, _p(idx), _p(val))
    return idx[:k], val[:k]


def round_to_dtype(x: float, dtype: int) -> float:
    return float(lib().oracle_round_to_dtype(ctypes.c_float(x), dtype))


# ---------------------------------------------------------- attention (fp64)

def attention_fwd(q, k, v, cu_chunk, sel, scale=None):
    """FP64 fixed-route forward.  q [T,Hq,D], k/v [T,Hkv,D] float64 arrays;
    sel [T,Hq,R] global chunk ids (-1 pad) or None.  Returns (O, LSE)."""
    q, k, v = (np.ascontiguousarray(x, dtype=np.float64) for x in (q, k, v))
    T, hq, d = q.shape
    hkv = k.shape[1]
    R = 0 if sel is None else sel.shape[-1]
    s = np.ascontiguousarray(sel if sel is not None else np.zeros((1,), np.int32), dtype=np.int32)
    cc = np.ascontiguousarray(cu_chunk, dtype=np.int32)
    out = np.zeros_like(q)
    lse = np.zeros((T, hq), dtype=np.float64)
    scale = d ** -0.5 if scale is None else scale
    lib().oracle_attention_fwd(_p(q), _p(k), _p(v), T, hq, hkv, d, _p(cc), len(cu_chunk) - 1,
                               _p(s), R, ctypes.c_double(scale), _p(out), _p(lse))
    return out, lse


def attention_bwd(q, k, v, dout, cu_chunk, sel, lse, scale=None):
    q, k, v, dout, lse = (np.ascontiguousarray(x, dtype=np.float64) for x in (q, k, v, dout, lse))
    T, hq, d = q.shape
    hkv = k.shape[1]
    R = 0 if sel is None else sel.shape[-1]
    s = np.ascontiguousarray(sel if sel is not None else np.zeros((1,), np.int32), dtype=np.int32)
    cc = np.ascontiguousarray(cu_chunk, dtype=np.int32)
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    scale = d ** -0.5 if scale is None else scale
    lib().oracle_attention_bwd(_p(q), _p(k), _p(v), _p(dout), T, hq, hkv, d, _p(cc),
                               len(cu_chunk) - 1, _p(s), R, ctypes.c_double(scale), _p(lse),
                               _p(dq), _p(dk), _p(dv))
    return dq, dk, dv


def merge(self_out, self_lse, remote_out, remote_lse, mapping):
    so = np.ascontiguousarray(self_out, dtype=np.float64).reshape(len(self_lse), -1)
    sl = np.ascontiguousarray(self_lse, dtype=np.float64).reshape(-1)
    P, d = so.shape
    ro = np.ascontiguousarray(remote_out, dtype=np.float64).reshape(-1, d)
    rl = np.ascontiguousarray(remote_lse, dtype=np.float64).reshape(-1)
    mp = np.ascontiguousarray(mapping, dtype=np.int64).reshape(-1)
    # the C loop indexes rows by mapping: shapes and range are checked here
    if sl.size != P or rl.size != mp.size or ro.shape[0] != mp.size or \
            (mp.size and (mp.min() < 0 or mp.max() >= P)):
        raise ValueError("oracle merge: inconsistent shapes or mapping out of range")
    out = np.zeros((P, d), dtype=np.float64)
    lse = np.zeros(P, dtype=np.float64)
    lib().oracle_merge(_p(so), _p(sl), P, d, _p(ro), _p(rl), _p(mp), mp.size, _p(out), _p(lse))
    return out, lse


# ------------------------------------------------------------------- decode

def decode_means(k_bits, dtype, chunk):
    L, hkv, d = k_bits.shape
    out = np.zeros((L // chunk, hkv, d), dtype=np.uint16)
    kb = np.ascontiguousarray(k_bits)
    if L // chunk:
        lib().oracle_decode_means(_p(kb), dtype, L, hkv, d, chunk, _p(out))
    return out


def decode_route(q_bits_row, means_bits, dtype, chunk, pos, width, remote):
    hq, d = q_bits_row.shape
    hkv = means_bits.shape[1] if means_bits.ndim == 3 else 1
    qb = np.ascontiguousarray(q_bits_row)
    mb = np.ascontiguousarray(means_bits) if means_bits.size else np.zeros((1, hkv, d), np.uint16)
    scores = np.zeros((hq, max(width, 1)), dtype=np.float32)
    sel = np.zeros((hq, 1 + remote), dtype=np.int32)
    lib().oracle_decode_route(_p(qb), _p(mb), dtype, hq, hkv, d, chunk, pos, width, remote,
                              _p(scores), _p(sel))
    return scores[:, :width], sel


def decode_attention(q_row, k_seq, v_seq, chunk, pos, chunks=None):
    """FP64 decode attention of one query row [Hq,D] over logical K/V [L,Hkv,D]."""
    q = np.ascontiguousarray(q_row, dtype=np.float64)
    k = np.ascontiguousarray(k_seq, dtype=np.float64)
    v = np.ascontiguousarray(v_seq, dtype=np.float64)
    hq, d = q.shape
    hkv = k.shape[1]
    out = np.zeros((hq, d), dtype=np.float64)
    lse = np.zeros(hq, dtype=np.float64)
    ch = None if chunks is None else np.ascontiguousarray(chunks, dtype=np.int32)
    lib().oracle_decode_attention(_p(q), _p(k), _p(v), hq, hkv, d, chunk, pos,
                                  _p(ch) if ch is not None else None,
                                  0 if ch is None else ch.shape[-1], _p(out), _p(lse))
    return out, lse
