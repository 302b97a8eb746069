"""Shared test utilities: seeded inputs, oracle comparisons, tolerances."""
import itertools
import os

import numpy as np
import torch

from oracle import oracle as O

# north-star tolerance vs the FP64 fixed-route oracle (same routes forced)
TOL = {torch.bfloat16: (2e-2, 2e-3), torch.float16: (4e-3, 4e-4)}


def prefill_inputs(hq, hkv, dim, lens, dtype=torch.bfloat16, seed=61, device="cuda", scale=1.0):
    gen = torch.Generator().manual_seed(seed)
    total = sum(lens)
    q, k, v = [(torch.randn(total, h, dim, generator=gen) * scale).to(device, dtype)
               for h in (hq, hkv, hkv)]
    g = torch.randn(total, hq, dim, generator=gen).to(device, dtype)
    cu = torch.tensor([0] + list(itertools.accumulate(lens)), device=device, dtype=torch.int32)
    return q, k, v, cu, max(lens), g


def assert_close_stats(actual, expected, dtype, what=""):
    a = actual.detach().double().cpu().numpy() if isinstance(actual, torch.Tensor) else actual
    e = expected
    diff = np.abs(a - e)
    max_tol, mean_tol = TOL[dtype]
    assert np.isfinite(a).all(), f"{what}: non-finite values"
    assert diff.max() <= max_tol, f"{what}: max abs {diff.max():.3e} > {max_tol}"
    assert diff.mean() <= mean_tol, f"{what}: mean abs {diff.mean():.3e} > {mean_tol}"
    _log_errors(what, dtype, diff, 0)
    return float(diff.max()), float(diff.mean())


# mantissa bits of the storage dtype (one ulp of |x| is 2^(floor(log2|x|) - bits))
_MANT = {torch.bfloat16: 7, torch.float16: 10}


def _log_errors(what, dtype, diff, n_big, floor=0.0):
    """Append one line of measured errors to $MOBA_PARITY_LOG (if set)."""
    path = os.environ.get("MOBA_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(f"{os.environ.get('PYTEST_CURRENT_TEST', '?').split(' ')[0]} {what} "
                    f"{str(dtype).split('.')[-1]} max_abs={diff.max():.3e} "
                    f"mean_abs={diff.mean():.3e} storage_mean={floor:.3e} ulp_entries={n_big}\n")


def assert_grad_close(actual, expected, dtype, what="", max_tol=None, mean_tol=None):
    """North-star bounds (max-abs, mean-abs of TOL[dtype]) UNSCALED on every
    entry whose reference magnitude is small enough that one ulp of the
    output dtype is within the max-abs bound (|ref| < 4 for bf16, < 8 for
    fp16).  An entry above that cannot be stored closer than half an ulp, so
    it is held to max-abs + one ulp of |ref| instead; such entries are counted
    in the message.  The mean-abs bound applies, raw, to the small entries
    (a caller may pass its own, with the reason at the call site)."""
    a = actual.detach().double().cpu().numpy() if isinstance(actual, torch.Tensor) else actual
    e = np.asarray(expected, dtype=np.float64)
    max_tol = TOL[dtype][0] if max_tol is None else max_tol
    mean_tol = TOL[dtype][1] if mean_tol is None else mean_tol
    assert np.isfinite(a).all(), f"{what}: non-finite values"
    diff = np.abs(a - e)
    mag = np.abs(e)
    ulp = np.exp2(np.floor(np.log2(np.maximum(mag, 1e-300))) - _MANT[dtype])
    big = ulp > max_tol
    n_big = int(big.sum())
    small = diff[~big]
    stored = torch.from_numpy(e).to(dtype).double().numpy()
    _log_errors(what, dtype, diff, n_big, float(np.abs(stored - e).mean()))
    if small.size:
        assert small.max() <= max_tol, \
            f"{what}: max abs {small.max():.3e} > {max_tol} ({n_big} entries above the ulp bound)"
        assert small.mean() <= mean_tol, \
            (f"{what}: mean abs {small.mean():.3e} > {mean_tol} "
             f"({n_big} entries above the ulp bound)")
    if n_big:
        excess = diff[big] - (max_tol + ulp[big])
        assert excess.max() <= 0, \
            f"{what}: {n_big} entries with |ref| ulp > {max_tol}: worst exceeds by {excess.max():.3e}"
    return float(diff.max()), float(diff.mean()), n_big


def oracle_route(q, k, cu, chunk, topk, precision=0):
    """Canonical CPU routing for bf16/fp16 torch inputs: (sel, means, gate, meta)."""
    code = 0 if q.dtype == torch.bfloat16 else 1
    cu_chunk, chunk_batch, filtered = O.calc_chunks(cu.tolist(), chunk)
    remote = min(topk - 1, len(filtered))
    means = O.chunk_means(O.bits16(k), code, cu_chunk, filtered, chunk, precision)
    sel, gate = O.route_prefill(O.bits16(q), code, means, cu_chunk, chunk_batch, remote,
                                want_gate=True)
    return sel, means, gate, (cu_chunk, chunk_batch, filtered, remote)
