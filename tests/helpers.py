"""Shared test utilities: seeded inputs, oracle comparisons, tolerances."""
import itertools

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
    return float(diff.max()), float(diff.mean())


def oracle_route(q, k, cu, chunk, topk, precision=0):
    """Canonical CPU routing for bf16/fp16 torch inputs: (sel, means, gate, meta)."""
    code = 0 if q.dtype == torch.bfloat16 else 1
    cu_chunk, chunk_batch, filtered = O.calc_chunks(cu.tolist(), chunk)
    remote = min(topk - 1, len(filtered))
    means = O.chunk_means(O.bits16(k), code, cu_chunk, filtered, chunk, precision)
    sel, gate = O.route_prefill(O.bits16(q), code, means, cu_chunk, chunk_batch, remote,
                                want_gate=True)
    return sel, means, gate, (cu_chunk, chunk_batch, filtered, remote)
