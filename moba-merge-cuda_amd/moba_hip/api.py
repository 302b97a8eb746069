"""Implementation registry and dispatch.

Mirrors the registry contract of src/moba_opt/api.py:11-27: ``register`` refuses
duplicates with KeyError, ``run_impl`` dispatches by name with the positional
signature ``(q, k, v, cu_seqlens, max_seqlen, config)`` and raises KeyError
listing the available names for an unknown one.
"""

_IMPLS = {}


def register(name, fn):
    if name in _IMPLS:
        raise KeyError(f"impl already registered: {name}")
    _IMPLS[name] = fn


def available_impls():
    return sorted(_IMPLS)


def run_impl(name, q, k, v, cu_seqlens, max_seqlen, config):
    if name not in _IMPLS:
        raise KeyError(f"unknown impl {name!r}; available: {available_impls()}")
    return _IMPLS[name](q, k, v, cu_seqlens, max_seqlen, config)
