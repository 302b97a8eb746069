"""ctypes binding of libmoba_hip.so (the C ABI declared in include/moba_hip.h).

The shared library is loaded from the package directory.  There is no fallback:
if the library is missing every op raises, so a GPU run can never silently use
another implementation.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parents[1] / "libmoba_hip.so"

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_L = ctypes.c_int64
_PP = ctypes.POINTER(ctypes.c_void_p)

# name -> argtypes (restype int unless listed in _RESTYPES)
SIGNATURES = {
    "moba_hip_version": [],
    "moba_hip_last_error": [],
    "moba_hip_chunk_means": [_P, _I, _I, _I, _I, _P, _I, _I, _I, _P, _P],
    "moba_hip_route_prefill": [_P, _I, _I, _I, _I, _I, _P, _P, _I, _P, _P, _I, _I, _P, _P, _P],
    "moba_hip_pack_experts": [_P, _I, _I, _I, _I, _P, _P, _P, _P, _I, _I, _P, _P, _P, _P, _P, _P],
    "moba_hip_pack_experts_work": [_I, _I, _I, _I],
    "moba_hip_prefill_rows": [_I],
    "moba_hip_prefill_bwd_work": [_I, _I, _I],
    "moba_hip_prefill_fwd": [_P, _P, _P, _I, _I, _I, _I, _I, _F, _P, _P, _I, _P, _I, _P, _I,
                             _P, _P, _P, _P, _I, _P, _P, _P, _P, _P],
    "moba_hip_prefill_bwd": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _P, _P, _I, _P, _I,
                             _P, _I, _P, _I, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _I, _I, _P,
                             _P, _P],
    "moba_hip_merge": [_P, _P, _P, _P, _P, _I, _L, _I, _I, _L, _I, _P, _P, _P, _P, _P],
    "moba_hip_merge_work": [_L, _L],
    "moba_hip_decode_work_items": [_I, _I, _I],
    "moba_hip_paged_append": [_P, _P, _I, _I, _I, _I, _P, _P, _I, _P, _I, _P, _P, _P],
    "moba_hip_block_means": [_P, _I, _I, _I, _I, _P, _I, _P, _P, _I, _I, _I, _P, _I, _P],
    "moba_hip_decode_route": [_P, _I, _I, _I, _I, _I, _P, _I, _P, _P, _I, _I, _I, _P, _P, _P,
                              _P, _P],
    "moba_hip_paged_attention": [_P, _I, _I, _I, _I, _I, _P, _P, _I, _P, _I, _P, _P, _P, _P, _I,
                                 _P, _P, _I, _I, _I, _P, _P, _P, _P, _P],
    "moba_hip_decode_metadata": [_P, _I, _P, _P, _P, _P, _I, _I, _P],
    "moba_hip_decode_step": [_P, _I, _P, _P, _P, _P, _I, _P, _P, _I, _P, _P, _I, _I, _I, _I, _P,
                             _I, _P],
    "moba_hip_decode_fused_supported": [_I, _I, _I, _I, _I],
    "moba_hip_decode_fused_groups": [_I, _I],
    "moba_hip_decode_fused": [_P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _I, _P, _I, _P, _P, _P, _P,
                              _P, _I, _I, _I, _I, _I, _I, _I, _P, _I, _P, _P, _P, _P, _P, _P],
    "moba_hip_decode_attend_noalloc": [_P, _I, _I, _I, _I, _I, _P, _P, _I, _P, _I, _P, _P, _P,
                                       _P, _I, _I, _I, _I, _I, _P, _P, _P, _P],
    # host page pool (CPU only)
    "moba_pool_create": [_I, _I, _I, _I, _I, _PP],
    "moba_pool_destroy": [_P],
    "moba_pool_clone": [_P, _PP],
    "moba_pool_assign": [_P, _P],
    "moba_pool_info": [_P, _P],
    "moba_pool_table": [_P],
    "moba_pool_lengths": [_P],
    "moba_pool_free": [_P],
    "moba_pool_set_free": [_P, _P, _I],
    "moba_pool_check_ids": [_P, _P, _I, _I],
    "moba_pool_plan_append": [_P, _P, _P, _I, _P, _P, _P, _I, _P, _P, _I, _P, _P, _P],
    "moba_pool_commit_append": [_P, _P, _I, _P, _P, _I, _L],
    "moba_pool_reset": [_P, _P, _I],
    "moba_pool_plan_step": [_P, _P, _I, _P, _P, _P, _P],
    "moba_pool_commit_step": [_P, _P, _I, _P, _L],
    # prepared-decode driver
    "moba_prep_create": [_P, _P, _PP],
    "moba_prep_destroy": [_P],
    "moba_prep_run": [_P, _I, _I, _P, _P],
    "moba_prep_capture": [_P, _I, _P],
    "moba_prep_plan": [_P, _I, _P, _P],
    "moba_prep_launch": [_P, _I, _I, _P],
    "moba_prep_commit": [_P],
    "moba_prep_delta_uploads": [_P],
    "moba_prep_sched_workgroups": [_I, _I, _I, _I],
    "moba_prep_schedule": [_P, _I, _I, _I, _I, _I, _I, _I, _I, _P, _P],
}
_I32P = ctypes.POINTER(ctypes.c_int32)
_RESTYPES = {"moba_hip_merge_work": ctypes.c_int64, "moba_pool_destroy": None, "moba_prep_destroy": None,
             "moba_prep_delta_uploads": ctypes.c_int64, "moba_pool_table": _I32P, "moba_pool_lengths": _I32P,
             "moba_pool_free": _I32P, "moba_hip_last_error": ctypes.c_char_p, "moba_hip_pack_experts_work": ctypes.c_int64,
             "moba_hip_prefill_bwd_work": ctypes.c_int64}

_lib = None
_lock = threading.Lock()


class MobaHipError(RuntimeError):
    pass


MOBA_ERR_ARG = 1
MOBA_ERR_CAPACITY = 3
MOBA_ERR_STALE = 4


def load():
    """Load the library (once).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise MobaHipError(
                    f"{LIB_PATH} is missing: build it with `python moba-merge-cuda_amd/build.py` "
                    "(or __graft_entry__.build()); there is no fallback implementation")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, args in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = args
                fn.restype = _RESTYPES.get(name, ctypes.c_int)
            _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Invoke an entry point and raise MobaHipError on a non-zero status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.moba_hip_last_error().decode(errors="replace")
        raise MobaHipError(f"{name} failed ({rc}): {msg}")


def ptr(t) -> int | None:
    """Device address of a torch tensor (None for None)."""
    return None if t is None else t.data_ptr()


def stream_of(device) -> int:
    import torch
    return torch.cuda.current_stream(device).cuda_stream
