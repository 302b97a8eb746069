"""The allocation-free decode entry (moba_hip_decode_attend_noalloc, static
device scratch) against the existing entry with caller workspaces
(moba_hip_decode_fused, positions given), both through the C-ABI: two calls
in a row on the same device, the second with a smaller input, each
bit-identical to the workspace entry (same kernels, same split count)."""
import ctypes

import pytest
import torch

from decode_check import rand

pytestmark = pytest.mark.gpu


def _filled_cache(batch, hkv, d, lengths, seed):
    from moba_hip import PagedKVCache
    cache = PagedKVCache(batch, max(lengths) + 4, hkv, d, page_size=48, chunk_size=64)
    for sid, n in enumerate(lengths):
        cache.append(rand((n, hkv, d), cache.dtype, seed + sid),
                      rand((n, hkv, d), cache.dtype, seed + 100 + sid),
                      sequence_ids=[sid], cu_seqlens=[0, n])
    return cache


def _both(cache, q, ids, pos, topk):
    from moba_hip.ops import _lib
    from moba_hip.ops import decode as K
    lib = _lib.load()
    fn = lib.moba_hip_decode_attend_noalloc
    nq, hq, d = q.shape
    hkv, C = cache.num_kv_heads, cache.chunk_size
    remote = min(topk - 1, cache._candidates())
    width = max(1, remote, max(pos) // C)
    dev_ids = torch.tensor(ids, dtype=torch.int32, device="cuda")
    dev_pos = torch.tensor(pos, dtype=torch.int32, device="cuda")
    outs = []
    for static in (False, True):
        sel = torch.full((nq, hq, remote + 1), -7, dtype=torch.int32, device="cuda")
        out = torch.full_like(q, 3.0)
        lse = torch.full((nq, hq), 5.0, dtype=torch.float32, device="cuda")
        if static:
            rc = fn(q.data_ptr(), K.DTYPE_CODE[q.dtype], nq, hq, hkv, d, cache.k_cache.data_ptr(),
                    cache.v_cache.data_ptr(), cache.k_cache.shape[1], cache._table.data_ptr(),
                    cache._table.shape[1], cache._lengths.data_ptr(), dev_ids.data_ptr(),
                    dev_pos.data_ptr(), cache._means.data_ptr(), cache._means.shape[1], C, width,
                    remote, 0, sel.data_ptr(), out.data_ptr(), lse.data_ptr(),
                    torch.cuda.current_stream().cuda_stream)
            assert rc == 0, lib.moba_hip_last_error().decode()
        else:
            work = K.FusedWork(nq, hq, hkv, d, q.device)   # splits = the uniform default
            K.fused(q, None, None, cache.k_cache, cache.v_cache, cache._table, cache._lengths,
                    dev_ids, dev_pos, None, cache._means, C, width, remote, False, 0, sel, work,
                    out, lse)
        outs.append((sel, out, lse))
    torch.cuda.synchronize()
    return outs


def test_noalloc_matches_workspace_entry_twice(cuda_device):
    cache = _filled_cache(6, 2, 128, [700, 1900, 64, 3000, 1, 1300], seed=41)
    q1 = rand((6, 12, 128), cache.dtype, 51)
    first = _both(cache, q1, [0, 1, 2, 3, 4, 5], [699, 1899, 63, 2999, 0, 1000], topk=4)
    q2 = rand((3, 12, 128), cache.dtype, 52)   # smaller second call on the same scratch
    second = _both(cache, q2, [3, 1, 5], [2100, 5, 1299], topk=3)
    for (ref, got) in (first, second):
        for a, b in zip(ref, got):
            assert torch.equal(a, b)
    assert (first[0][0] >= -1).all() and second[0][0].shape == (3, 12, 3)


def test_noalloc_rejects_oversize_before_launch(cuda_device):
    from moba_hip.ops import _lib
    lib = _lib.load()
    # 4096 rows x 64 heads x 1 split x 258 floats > 8 MiB: refused, nothing launched
    rc = lib.moba_hip_decode_attend_noalloc(None, 0, 4096, 64, 4, 256, None, None, 16, None, 8,
                                            None, None, None, None, 8, 64, 4, 3, 0, None, None,
                                            None, None)
    assert rc == _lib.MOBA_ERR_CAPACITY
    assert b"static scratch" in lib.moba_hip_last_error()
