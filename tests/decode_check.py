"""Oracle check shared by the decode GPU tests.

Mirrors the reference's check() (tests/test_paged_decode.py:22-60) but pins more:
  * closed-chunk means are BIT-equal to the canonical oracle means;
  * routes are BIT-equal to the canonical oracle route of the stored means;
  * output/LSE vs the FP64 decode oracle on the same routes, with the
    reference's tolerances (bf16 0.02/0.02 + rel-L2 < 0.01, fp16 0.002;
    LSE 5e-4 / 2e-5) and the north-star bound (bf16 max-abs <= 2e-2,
    mean-abs <= 2e-3).
"""
import numpy as np
import torch

from oracle import oracle as O


def rand(shape, dtype, seed):
    return torch.randn(shape, generator=torch.Generator().manual_seed(seed)).to("cuda", dtype)


def assert_payload(cache, sid, k, v):
    ak, av = cache.materialize(sid)
    assert torch.equal(ak, k), "cached K differs from original input"
    assert torch.equal(av, v), "cached V differs from original input"


def check(cache, result, q):
    code = 0 if cache.dtype == torch.bfloat16 else 1
    C = cache.chunk_size
    keys, values, mean_bits = [], [], []
    for sid in range(len(cache.lengths)):
        k, v = cache.materialize(sid)
        keys.append(k)
        values.append(v)
        kb = O.bits16(k) if k.shape[0] else np.zeros((0, cache.num_kv_heads, cache.head_dim), np.uint16)
        ref = O.decode_means(kb, code, C)
        mean_bits.append(ref)
        closed = cache.lengths[sid] // C
        if closed:
            got = O.bits16(cache._means[sid, :closed])
            np.testing.assert_array_equal(got, ref, err_msg=f"means of sequence {sid}")
    qb = O.bits16(q)
    sel = None if result.selected_blocks is None else result.selected_blocks.cpu().numpy()
    outs, lses = [], []
    for row, (sid, pos) in enumerate(zip(result.sequence_ids, result.positions)):
        chunks = None
        if sel is not None:
            R = sel.shape[-1] - 1
            _, want = O.decode_route(qb[row], mean_bits[sid], code, C, pos, pos // C, R)
            np.testing.assert_array_equal(sel[row], want, err_msg=f"route of row {row}")
            chunks = sel[row]
        o, l = O.decode_attention(q[row].double().cpu().numpy(), keys[sid].double().cpu().numpy(),
                                  values[sid].double().cpu().numpy(), C, pos, chunks)
        outs.append(o)
        lses.append(l)
    exp_o, exp_l = np.stack(outs), np.stack(lses)
    out = result.output.double().cpu().numpy()
    assert np.isfinite(out).all() and np.isfinite(result.lse.cpu().numpy()).all()
    tol = 0.02 if cache.dtype == torch.bfloat16 else 0.002
    np.testing.assert_allclose(out, exp_o, atol=tol, rtol=tol)
    diff = np.abs(out - exp_o)
    assert diff.max() <= (2e-2 if code == 0 else 4e-3) and diff.mean() <= (2e-3 if code == 0 else 4e-4), \
        f"max {diff.max():.3e} mean {diff.mean():.3e} at {np.unravel_index(diff.argmax(), diff.shape)}: {out.flat[diff.argmax()]} vs {exp_o.flat[diff.argmax()]}"
    rel = np.linalg.norm(out - exp_o) / max(np.linalg.norm(exp_o), 1e-8)
    assert rel < (0.01 if code == 0 else 0.002)
    np.testing.assert_allclose(result.lse.double().cpu().numpy(), exp_l, atol=5e-4, rtol=2e-5)
