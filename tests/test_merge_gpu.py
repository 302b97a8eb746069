"""GPU parity of the standalone merge (moba_hip_merge, the counterpart of
merge_forward in src/moba_opt/ops/bindings.cpp:6-22) against the FP64 oracle
merge (reference/merge_reference.py:10-26), including the reference's own
cases (tests/test_merge_cuda.py:27-31: no remote rows is the identity) and
the closed-form edge cases pinned on the oracle in tests/test_oracle.py."""
import numpy as np
import pytest
import torch

from helpers import assert_close_stats
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _case(T, H, D, dtype, per_row_max, seed, shuffle=True):
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    so = torch.randn((T, H, D), generator=g)
    sl = torch.randn((T, H), generator=g) * 3
    counts = rng.integers(0, per_row_max + 1, T * H)
    mapping = np.repeat(np.arange(T * H), counts)
    if shuffle:
        rng.shuffle(mapping)
    M = len(mapping)
    ro = torch.randn((M, D), generator=g)
    rl = torch.randn(M, generator=g) * 3
    dev = "cuda"
    return (so.to(dev, dtype), sl.to(dev), ro.to(dev, dtype), rl.to(dev),
            torch.from_numpy(mapping).to(dev))


def _ref(so, sl, ro, rl, mp):
    T, H, D = so.shape
    o, l = O.merge(so.double().cpu().numpy().reshape(T * H, D), sl.double().cpu().numpy().reshape(-1),
                   ro.double().cpu().numpy(), rl.double().cpu().numpy(), mp.cpu().numpy())
    return o.reshape(T, H, D), l.reshape(T, H)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("T,H,D,per_row", [(37, 5, 64, 3), (9, 4, 8, 8), (50, 2, 96, 1),
                                           (11, 3, 256, 5)])
def test_merge_matches_fp64(cuda_device, T, H, D, per_row, dtype):
    from moba_hip.merge import merge_forward
    so, sl, ro, rl, mp = _case(T, H, D, dtype, per_row, seed=T * 7 + D)
    out, lse = merge_forward(so, sl, ro, rl, mp)
    o_ref, l_ref = _ref(so, sl, ro, rl, mp)
    assert out.dtype == dtype and lse.dtype == torch.float32
    if dtype == torch.float32:
        np.testing.assert_allclose(out.double().cpu().numpy(), o_ref, atol=2e-6, rtol=1e-5)
    else:
        assert_close_stats(out, o_ref, dtype, "merged out")
    np.testing.assert_allclose(lse.double().cpu().numpy(), l_ref, atol=2e-6, rtol=1e-6)
    again = merge_forward(so, sl, ro, rl, mp)
    assert torch.equal(out, again[0]) and torch.equal(lse, again[1])


@pytest.mark.parametrize("T,H", [(4096, 8), (70000, 1)])
def test_merge_multi_pass_sort(cuda_device, T, H):
    """P = 32768 (two 8-bit digit passes) and P = 70000 (three), with up to
    7 remote partials per row in shuffled order."""
    from moba_hip.merge import merge_forward
    so, sl, ro, rl, mp = _case(T, H, 64, torch.bfloat16, 7, seed=T)
    out, lse = merge_forward(so, sl, ro, rl, mp, kmax=7)
    o_ref, l_ref = _ref(so, sl, ro, rl, mp)
    assert_close_stats(out, o_ref, torch.bfloat16, "merged out")
    np.testing.assert_allclose(lse.double().cpu().numpy(), l_ref, atol=2e-6, rtol=1e-6)


def test_merge_no_remote_is_identity(cuda_device):
    from moba_hip.merge import merge_forward
    so, sl, _, _, _ = _case(6, 3, 32, torch.bfloat16, 0, seed=3)
    ro = torch.empty((0, 32), device="cuda", dtype=torch.bfloat16)
    rl = torch.empty(0, device="cuda")
    mp = torch.empty(0, device="cuda", dtype=torch.int64)
    out, lse = merge_forward(so, sl, ro, rl, mp)
    assert torch.equal(out, so) and torch.equal(lse, sl)


def test_merge_extreme_lse_gap(cuda_device):
    from moba_hip.merge import merge_forward
    so, sl, ro, rl, _ = _case(5, 1, 16, torch.float32, 0, seed=4)
    ro = torch.randn((5, 16), device="cuda")
    mp = torch.arange(5, device="cuda")
    out, lse = merge_forward(so, torch.full_like(sl, -1e30), ro, torch.full((5,), 1e30,
                             device="cuda"), mp)
    assert torch.isfinite(out).all() and torch.isfinite(lse).all()
    torch.testing.assert_close(out[:, 0], ro, atol=1e-6, rtol=0)


def test_merge_capacity_and_range_errors(cuda_device):
    from moba_hip.merge import merge_forward
    so, sl, ro, rl, _ = _case(4, 2, 16, torch.bfloat16, 0, seed=5)
    ro = torch.randn((5, 16), device="cuda").bfloat16()
    rl = torch.randn(5, device="cuda")
    crowded = torch.tensor([3, 3, 3, 1, 0], device="cuda")
    with pytest.raises(RuntimeError, match="capacity exceeded"):
        merge_forward(so, sl, ro, rl, crowded, kmax=2)
    merge_forward(so, sl, ro, rl, crowded, kmax=2, check_capacity=False)  # no raise
    with pytest.raises(RuntimeError, match=r"\[0,T\*H\)"):
        merge_forward(so, sl, ro, rl, torch.tensor([0, 1, 8, 2, 3], device="cuda"))
    # negative and far-out entries with the derived kmax reach the same native check
    for bad in ([0, -1, 2, 3, 4], [0, 1, 2, 3, 1 << 40], [-5, -5, -5, -5, -5]):
        with pytest.raises(RuntimeError, match=r"\[0,T\*H\)"):
            merge_forward(so, sl, ro, rl, torch.tensor(bad, device="cuda"))
    with pytest.raises(ValueError, match="deterministic"):
        merge_forward(so, sl, ro, rl, crowded, deterministic=1)
