"""GPU parity of the paged decode path (cases follow tests/test_paged_decode.py
of the reference: cache kinds x dtypes x head ratios, head dims, unaligned
pages, recycling, causality, routing known answer, partition invariance,
extreme logits, max topk, error paths)."""
import pytest
import torch

from decode_check import assert_payload, check, rand

pytestmark = pytest.mark.gpu


def _caches():
    from moba_hip import ContiguousKVCache, PagedKVCache
    return PagedKVCache, ContiguousKVCache


@pytest.mark.parametrize("paged", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hq,hk", [(1, 1), (8, 1), (8, 2), (28, 4), (32, 8)])
def test_incremental_decode(cuda_device, paged, dtype, hq, hk):
    Paged, Contig = _caches()
    cache = Paged(2, 32, hk, 64, chunk_size=4, dtype=dtype, page_size=3) if paged \
        else Contig(2, 32, hk, 64, chunk_size=4, dtype=dtype)
    k, v = rand((9, hk, 64), dtype, 101), rand((9, hk, 64), dtype, 102)
    cache.append(k, v, sequence_ids=[0, 1], cu_seqlens=[0, 4, 9])
    sk, sv = [k[:4], k[4:]], [v[:4], v[4:]]
    for sid in range(2):
        assert_payload(cache, sid, sk[sid], sv[sid])
    for step in range(3):
        q = rand((2, hq, 64), dtype, 103 + step)
        kn, vn = rand((2, hk, 64), dtype, 113 + step), rand((2, hk, 64), dtype, 123 + step)
        result = cache.append_and_attend(q, kn, vn, sequence_ids=[0, 1], topk=2)
        for sid in range(2):
            sk[sid] = torch.cat((sk[sid], kn[sid:sid + 1]))
            sv[sid] = torch.cat((sv[sid], vn[sid:sid + 1]))
            assert_payload(cache, sid, sk[sid], sv[sid])
        check(cache, result, q)
        check(cache, cache.attend(q, sequence_ids=[0, 1], mode="dense"), q)


@pytest.mark.parametrize("dim", [8, 16, 40, 64, 96, 128, 136, 200, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_head_dimensions(cuda_device, dim, dtype):
    Paged, _ = _caches()
    cache = Paged(2, 64, 2, dim, page_size=7, chunk_size=12, dtype=dtype)
    k, v = rand((68, 2, dim), dtype, 131), rand((68, 2, dim), dtype, 132)
    cache.append(k, v, sequence_ids=[0, 1], cu_seqlens=[0, 27, 68])
    assert_payload(cache, 0, k[:27], v[:27])
    assert_payload(cache, 1, k[27:], v[27:])
    q = rand((3, 4, dim), dtype, 133)
    for mode in ("moba", "dense"):
        check(cache, cache.attend(q, sequence_ids=[0, 1, 1], positions=[26, 40, 5], topk=2,
                                  mode=mode), q)


@pytest.mark.parametrize("dim", [32, 64, 96, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_twelve_wave_launch(cuda_device, dim, dtype):
    """Launches whose workgroups carry at least 16 blocks take the 12-wave,
    single-buffered form of the fused kernel: 32 rows x 4 kv heads leave 2
    splits per (row, kv head) over the 256 workgroups, and top-2 routing at
    chunk 512 gives 2 x 16 blocks per row.  Attend and append-and-attend
    against the oracle at every head dim that form is built for."""
    from moba_hip.ops import decode as DK
    Paged, _ = _caches()
    B, hk, hq, C = 32, 4, 16, 512
    lengths = [1024 + 37 * i for i in range(B)]
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    assert 2 * (C // 32) >= 16 * DK.fused_splits(B, hk)  # the 12-wave condition
    cache = Paged(B, 2304, hk, dim, page_size=48, chunk_size=C, dtype=dtype)
    k, v = rand((cu[-1], hk, dim), dtype, 141), rand((cu[-1], hk, dim), dtype, 142)
    rows = list(range(B))
    cache.append(k, v, sequence_ids=rows, cu_seqlens=cu)
    q = rand((B, hq, dim), dtype, 143)
    check(cache, cache.attend(q, sequence_ids=rows, topk=2), q)
    kn, vn = rand((B, hk, dim), dtype, 144), rand((B, hk, dim), dtype, 145)
    check(cache, cache.append_and_attend(q, kn, vn, sequence_ids=rows, topk=2), q)


@pytest.mark.parametrize("dim", [1, 3, 7, 33, 65, 95, 129, 255])
def test_decode_unaligned_head_dimensions(cuda_device, dim):
    Paged, _ = _caches()
    for dtype in (torch.bfloat16, torch.float16):
        cache = Paged(2, 32, 2, dim, page_size=3, chunk_size=6, dtype=dtype)
        k, v = rand((35, 2, dim), dtype, 251), rand((35, 2, dim), dtype, 252)
        cache.append(k, v, sequence_ids=[1, 0], cu_seqlens=[0, 17, 35])
        assert_payload(cache, 1, k[:17], v[:17])
        assert_payload(cache, 0, k[17:], v[17:])
        q = rand((3, 4, dim), dtype, 253)
        for mode in ("dense", "moba"):
            check(cache, cache.attend(q, sequence_ids=[0, 1, 0], positions=[17, 16, 0], topk=2,
                                      mode=mode), q)


@pytest.mark.parametrize("page", [1, 3, 7, 16, 31, 64])
def test_pages_and_chunks_need_not_align(cuda_device, page):
    Paged, _ = _caches()
    cache = Paged(1, 97, 2, 80, page_size=page, chunk_size=24)
    cache.k_cache.fill_(float("nan"))
    cache.v_cache.fill_(float("nan"))
    k, v = rand((79, 2, 80), cache.dtype, 141), rand((79, 2, 80), cache.dtype, 142)
    cache.append(k, v, sequence_ids=[0], cu_seqlens=[0, 79])
    assert_payload(cache, 0, k, v)
    q = rand((2, 8, 80), cache.dtype, 143)
    for topk in (1, 2, 9):
        check(cache, cache.attend(q, sequence_ids=[0, 0], positions=[0, 78], topk=topk), q)


def test_recycled_pages_and_request_isolation(cuda_device):
    Paged, _ = _caches()
    cache = Paged(3, 12, 1, 16, page_size=3, num_pages=4, chunk_size=4)
    cache.append(rand((9, 1, 16), cache.dtype, 151), rand((9, 1, 16), cache.dtype, 152),
                 sequence_ids=[0, 1], cu_seqlens=[0, 6, 9])
    q = rand((1, 4, 16), cache.dtype, 153)
    before = cache.attend(q, sequence_ids=[1], mode="dense").output
    cache.reset([0])
    cache.append(rand((6, 1, 16), cache.dtype, 154), rand((6, 1, 16), cache.dtype, 155),
                 sequence_ids=[2], cu_seqlens=[0, 6])
    assert cache.page_table[2][:2] == (1, 0)
    torch.testing.assert_close(cache.attend(q, sequence_ids=[1], mode="dense").output, before)
    check(cache, cache.attend(q, sequence_ids=[2], topk=2), q)
    with pytest.raises(ValueError, match="cached tokens"):
        cache.attend(q, sequence_ids=[0])


def test_chunked_append_is_causal(cuda_device):
    Paged, _ = _caches()
    dtype = torch.bfloat16
    k, v = rand((19, 2, 32), dtype, 161), rand((19, 2, 32), dtype, 162)
    q = rand((7, 8, 32), dtype, 163)
    cache = Paged(2, 32, 2, 32, page_size=3, chunk_size=4)
    cache.append(torch.cat((k[:5], k[9:16])), torch.cat((v[:5], v[9:16])),
                 sequence_ids=[0, 1], cu_seqlens=[0, 5, 12])
    result = cache.append_and_attend(q, torch.cat((k[5:9], k[16:])), torch.cat((v[5:9], v[16:])),
                                     sequence_ids=[0, 1], cu_seqlens=[0, 4, 7], topk=2)
    assert_payload(cache, 0, k[:9], v[:9])
    assert_payload(cache, 1, k[9:], v[9:])
    assert result.positions == (5, 6, 7, 8, 7, 8, 9)
    check(cache, result, q)
    other = Paged(2, 32, 2, 32, page_size=3, chunk_size=4)
    k2, v2 = k.clone(), v.clone()
    k2[6:9] = 100
    v2[6:9] = -100
    other.append(k2, v2, sequence_ids=[0, 1], cu_seqlens=[0, 9, 19])
    compare = other.attend(q[:1], sequence_ids=[0], positions=[5], topk=2)
    torch.testing.assert_close(compare.output, result.output[:1], atol=0.02, rtol=0.02)


def test_routing_known_answer_per_query_head(cuda_device):
    """Staircase keys: head 0 prefers late chunks, head 2 (kv head 1) early ones
    (known answer of tests/test_paged_decode.py:146-159)."""
    Paged, _ = _caches()
    cache = Paged(1, 16, 2, 8, page_size=3, chunk_size=4)
    k = torch.zeros(13, 2, 8, device="cuda", dtype=cache.dtype)
    for block in range(4):
        k[block * 4:min((block + 1) * 4, 13), 0, 0] = block + 1
        k[block * 4:min((block + 1) * 4, 13), 1, 0] = 4 - block
    cache.append(k, rand(k.shape, cache.dtype, 171), sequence_ids=[0], cu_seqlens=[0, 13])
    q = torch.zeros(2, 4, 8, device="cuda", dtype=cache.dtype)
    q[:, :, 0] = 1
    result = cache.attend(q, sequence_ids=[0, 0], positions=[12, 7], topk=3)
    route = result.selected_blocks.cpu()
    assert set(route[0, 0].tolist()) == {3, 2, 1}
    assert set(route[0, 2].tolist()) == {3, 0, 1}
    assert set(route[1, 0].tolist()) == {1, 0, -1}
    check(cache, result, q)


def test_append_partition_invariance(cuda_device):
    Paged, _ = _caches()
    k, v = rand((25, 2, 24), torch.bfloat16, 181), rand((25, 2, 24), torch.bfloat16, 182)
    a = Paged(1, 32, 2, 24, page_size=7, chunk_size=6)
    b = Paged(1, 32, 2, 24, page_size=7, chunk_size=6)
    a.append(k, v, sequence_ids=[0], cu_seqlens=[0, 25])
    for lo, hi in [(0, 1), (1, 5), (5, 13), (13, 25)]:
        b.append(k[lo:hi], v[lo:hi], sequence_ids=[0], cu_seqlens=[0, hi - lo])
    assert torch.equal(a._means[:, :4], b._means[:, :4])
    q = rand((1, 8, 24), torch.bfloat16, 183)
    x = a.attend(q, sequence_ids=[0], topk=3)
    y = b.attend(q, sequence_ids=[0], topk=3)
    assert torch.equal(x.output, y.output) and torch.equal(x.selected_blocks, y.selected_blocks)


@pytest.mark.parametrize("hq,hk", [(8, 1), (8, 2), (28, 4)])
def test_decode_matches_last_prefill_row(cuda_device, hq, hk):
    from moba_hip.api import run_impl
    Paged, _ = _caches()
    q, k, v = (rand((97, h, 64), torch.bfloat16, s) for h, s in ((hq, 191), (hk, 192), (hk, 193)))
    cu = torch.tensor([0, 97], device="cuda", dtype=torch.int32)
    ref = run_impl("opt_hip", q, k, v, cu, 97, {"chunk_size": 16, "topk": 3})[-1:]
    cache = Paged(1, 128, hk, 64, page_size=7, chunk_size=16)
    cache.append(k, v, sequence_ids=[0], cu_seqlens=[0, 97])
    result = cache.attend(q[-1:], sequence_ids=[0], topk=3)
    torch.testing.assert_close(result.output, ref, atol=0.02, rtol=0.02)
    check(cache, result, q[-1:])


def test_capacity_and_inference_errors_do_not_mutate(cuda_device):
    Paged, _ = _caches()
    cache = Paged(2, 8, 1, 16, page_size=3, num_pages=1, chunk_size=4)
    q = rand((1, 4, 16), cache.dtype, 201)
    with pytest.raises(ValueError, match="cached tokens"):
        cache.attend(q, sequence_ids=[0])
    k, v = rand((3, 1, 16), cache.dtype, 202), rand((3, 1, 16), cache.dtype, 203)
    cache.append(k, v, sequence_ids=[0], cu_seqlens=[0, 3])
    before = cache.materialize(0)
    with pytest.raises(ValueError, match="pool exhausted"):
        cache.append(k[:1], v[:1], sequence_ids=[1])
    assert cache.lengths == (3, 0)
    for actual, expected in zip(cache.materialize(0), before):
        assert torch.equal(actual, expected)
    with pytest.raises(ValueError, match="inference-only"):
        cache.append_and_attend(q.requires_grad_(True), k[:1], v[:1], sequence_ids=[0])
    assert cache.lengths == (3, 0)
    with pytest.raises(ValueError, match="NaN/Inf"):
        cache.append(k[:1] * float("nan"), v[:1], sequence_ids=[0])
    assert cache.lengths == (3, 0)


def test_cross_stream_is_rejected(cuda_device):
    Paged, _ = _caches()
    cache = Paged(1, 8, 1, 8, page_size=3, chunk_size=4)
    k, v = rand((3, 1, 8), cache.dtype, 211), rand((3, 1, 8), cache.dtype, 212)
    cache.append(k, v, sequence_ids=[0], cu_seqlens=[0, 3])
    q = rand((1, 1, 8), cache.dtype, 213)
    with torch.cuda.stream(torch.cuda.Stream()):
        with pytest.raises(ValueError, match="cross-stream"):
            cache.attend(q, sequence_ids=[0])
    check(cache, cache.attend(q, sequence_ids=[0]), q)


def test_long_context_single_token_decode(cuda_device):
    Paged, _ = _caches()
    cache = Paged(1, 8193, 8, 128, page_size=16, chunk_size=128)
    cache.append(rand((8192, 8, 128), cache.dtype, 221), rand((8192, 8, 128), cache.dtype, 222),
                 sequence_ids=[0], cu_seqlens=[0, 8192])
    q, k, v = (rand((1, h, 128), cache.dtype, s) for h, s in ((32, 223), (8, 224), (8, 225)))
    result = cache.append_and_attend(q, k, v, sequence_ids=[0], topk=4)
    assert cache.lengths == (8193,) and result.positions == (8192,)
    check(cache, result, q)


@pytest.mark.parametrize("chunk,dim,length", [(1, 8, 5), (1024, 256, 1025)])
def test_chunk_size_extremes(cuda_device, chunk, dim, length):
    Paged, _ = _caches()
    cache = Paged(1, length + 1, 1, dim, page_size=3, chunk_size=chunk)
    cache.append(rand((length, 1, dim), cache.dtype, 231), rand((length, 1, dim), cache.dtype, 232),
                 sequence_ids=[0], cu_seqlens=[0, length])
    q = rand((1, 4, dim), cache.dtype, 233)
    check(cache, cache.attend(q, sequence_ids=[0], topk=2), q)


def test_extreme_logits_stable_softmax(cuda_device):
    Paged, _ = _caches()
    cache = Paged(1, 16, 1, 8, page_size=3, chunk_size=4)
    k = torch.full((13, 1, 8), 1000.0, device="cuda", dtype=cache.dtype)
    k[::2] = -1000
    cache.append(k, rand((13, 1, 8), cache.dtype, 241), sequence_ids=[0], cu_seqlens=[0, 13])
    q = torch.full((1, 2, 8), 1000.0, device="cuda", dtype=cache.dtype)
    q[:, 1] = -1000
    check(cache, cache.attend(q, sequence_ids=[0], mode="dense"), q)


def test_maximum_topk_with_ragged_queries(cuda_device):
    Paged, _ = _caches()
    cache = Paged(3, 97, 3, 33, page_size=7, chunk_size=8)
    cache.append(rand((153, 3, 33), cache.dtype, 261), rand((153, 3, 33), cache.dtype, 262),
                 sequence_ids=[0, 1, 2], cu_seqlens=[0, 81, 88, 153])
    q = rand((4, 15, 33), cache.dtype, 263)
    result = cache.attend(q, sequence_ids=[2, 0, 1, 2], positions=[64, 80, 6, 23], topk=9)
    assert result.selected_blocks.shape == (4, 15, 9)
    assert (result.selected_blocks[2, :, 1:] == -1).all()
    check(cache, result, q)


@pytest.mark.parametrize("combined", [False, True])
def test_append_rejects_aliases_before_mutation(cuda_device, combined):
    Paged, _ = _caches()
    cache = Paged(1, 8, 1, 8, page_size=3, chunk_size=4)
    cache.k_cache.zero_()
    cache.v_cache.zero_()
    alias = cache.k_cache.reshape(-1, 1, 8)[:1]
    external = rand((1, 1, 8), cache.dtype, 271)
    with pytest.raises(ValueError, match="must not alias"):
        if combined:
            cache.append_and_attend(alias, external, external, sequence_ids=[0])
        else:
            cache.append(alias, external, sequence_ids=[0])
    assert cache.lengths == (0,)
    cache.append(external, external, sequence_ids=[0])
    assert cache.lengths == (1,)


def test_unmapped_page_is_never_written(cuda_device):
    """Regression: a token whose logical page has no physical page (table
    entry -1) must not be written anywhere in the pool (the append kernel once
    computed a negative address for it)."""
    from moba_hip.ops import decode as kernels
    Paged, _ = _caches()
    cache = Paged(2, 16, 1, 8, page_size=4, chunk_size=4)
    cache.k_cache.zero_()
    cache.v_cache.zero_()
    table = torch.full((2, 4), -1, dtype=torch.int32, device="cuda")
    k = torch.ones((1, 1, 8), device="cuda", dtype=cache.dtype)
    ids = torch.tensor([1], dtype=torch.int32, device="cuda")
    pos = torch.tensor([5], dtype=torch.int32, device="cuda")
    kernels.append_tokens(k, k, cache.k_cache, cache.v_cache, table, ids, pos)
    torch.cuda.synchronize()
    assert int(cache.k_cache.count_nonzero()) == 0 and int(cache.v_cache.count_nonzero()) == 0


@pytest.mark.parametrize("dim", [132, 200, 256])
def test_wide_groups_wide_heads(cuda_device, dim):
    """32 q heads per kv head.  Head dims that are multiples of 8 take the
    fused launch as two virtual kv heads of 16 q heads; 132 takes the
    multi-kernel path, whose attention workgroups run 4 waves above 128 dims.
    Attend and append-and-attend against the oracle, moba and dense."""
    from moba_hip.ops import decode as kernels
    Paged, _ = _caches()
    cache = Paged(3, 200, 1, dim, page_size=9, chunk_size=16, dtype=torch.bfloat16)
    assert kernels.fused_supported(32, 1, dim, 12, cache._table.shape[1]) == (dim % 8 == 0)
    k, v = rand((150, 1, dim), torch.bfloat16, 171), rand((150, 1, dim), torch.bfloat16, 172)
    cache.append(k, v, sequence_ids=[0, 1, 2], cu_seqlens=[0, 61, 100, 150])
    q = rand((3, 32, dim), torch.bfloat16, 173)
    for mode in ("moba", "dense"):
        check(cache, cache.attend(q, sequence_ids=[0, 1, 2], topk=3, mode=mode), q)
    kn, vn = rand((3, 1, dim), torch.bfloat16, 174), rand((3, 1, dim), torch.bfloat16, 175)
    check(cache, cache.append_and_attend(q, kn, vn, sequence_ids=[0, 1, 2], topk=3), q)


def test_input_errors_follow_argument_order(cuda_device):
    """Inputs are checked k, v, q, each fully before the next (the reference's
    per-tensor order), although NaN/Inf is tested for all of them at once:
    the first failing input's error is raised and nothing is written."""
    Paged, _ = _caches()
    cache = Paged(2, 32, 2, 16, page_size=4, chunk_size=8)
    k, v = rand((5, 2, 16), torch.bfloat16, 181), rand((5, 2, 16), torch.bfloat16, 182)
    cache.append(k, v, sequence_ids=[0], cu_seqlens=[0, 5])
    lengths = cache.lengths
    q, kn, vn = (rand((1, h, 16), torch.bfloat16, 183 + h) for h in (4, 2, 2))
    nan = float("nan")
    cases = [
        ((q, kn * nan, vn[:, :1]), "k contains NaN/Inf"),       # before v's shape
        ((q * nan, kn, vn * nan), "v contains NaN/Inf"),        # before q's NaN
        ((q[:, :, :8], kn, vn * nan), "v contains NaN/Inf"),    # before q's shape
        ((q * nan, kn, vn), "q contains NaN/Inf"),
        ((q[:, :, :8], kn, vn), "q has an invalid shape"),
    ]
    for (qq, kk, vv), msg in cases:
        with pytest.raises(ValueError, match=msg):
            cache.append_and_attend(qq, kk, vv, sequence_ids=[0])
    with pytest.raises(ValueError, match="k contains NaN/Inf"):
        cache.append(kn * nan, vn[:, :1], sequence_ids=[0])
    assert cache.lengths == lengths


@pytest.mark.parametrize("graph", [False, True])
@pytest.mark.parametrize("hq,hk,dim,dtype", [
    (32, 1, 128, torch.bfloat16),   # 2 virtual kv heads of 16
    (40, 2, 64, torch.float16),     # 2 of 10 per kv head
    (24, 1, 96, torch.bfloat16),    # 2 of 12
    (17, 1, 64, torch.bfloat16),    # 17 of 1 (a prime group)
])
def test_virtual_kv_heads_prepared(cuda_device, graph, hq, hk, dim, dtype):
    """More than 16 q heads per kv head on the fused launch: prepared steps
    (scatter, closing means and the length advance done once per physical
    kv head) and attends, eager and replayed, against the oracle; rows close
    chunks during the run."""
    from moba_hip.ops import decode as kernels
    Paged, _ = _caches()
    vg = {32: 2, 20: 2, 24: 2, 17: 17}[hq // hk]
    assert kernels.fused_heads(hq, hk) == hk * vg
    cache = Paged(3, 120, hk, dim, page_size=5, chunk_size=8, dtype=dtype)
    k, v = rand((90, hk, dim), dtype, 191), rand((90, hk, dim), dtype, 192)
    cache.append(k, v, sequence_ids=[0, 1, 2], cu_seqlens=[0, 29, 61, 90])
    assert kernels.fused_supported(hq, hk, dim, 14, cache._table.shape[1])
    with cache.prepare_decode([2, 0, 1], hq, topk=4) as p:
        assert p.fused
        if graph:
            p.capture("step").capture("attend")
        for step in range(6):
            q = rand((3, hq, dim), dtype, 200 + step)
            kn, vn = rand((3, hk, dim), dtype, 210 + step), rand((3, hk, dim), dtype, 220 + step)
            check(cache, p.step(q, kn, vn, use_graph=graph), q)
            check(cache, p.attend(q, use_graph=graph), q)
    assert cache.lengths == (35, 38, 35)
    q = rand((3, hq, dim), dtype, 230)
    check(cache, cache.attend(q, sequence_ids=[0, 1, 2], topk=4), q)


@pytest.mark.parametrize("tied", [False, True])
@pytest.mark.parametrize("hq,hk,topk", [(8, 2, 4), (32, 1, 9)])
def test_wide_route_top_k(cuda_device, tied, hq, hk, topk):
    """More than 64 closed chunks per row: the route takes the wave-wide top-k
    path.  Routes are compared bit for bit with the oracle's rank rule,
    including exact ties (identical chunk means, ties to the lowest chunk)."""
    Paged, _ = _caches()
    dim, chunk, n = 64, 4, 600
    cache = Paged(2, 640, hk, dim, page_size=7, chunk_size=chunk, dtype=torch.bfloat16)
    k = rand((n, hk, dim), torch.bfloat16, 241)
    if tied:  # chunks repeat every 8: many exactly equal means and scores
        k = k.view(n // chunk, chunk, hk, dim)
        k = k[torch.arange(n // chunk) % 8].reshape(n, hk, dim).contiguous()
    v = rand((n, hk, dim), torch.bfloat16, 242)
    cache.append(k, v, sequence_ids=[0], cu_seqlens=[0, n])
    cache.append(k[:301], v[:301], sequence_ids=[1], cu_seqlens=[0, 301])
    q = rand((2, hq, dim), torch.bfloat16, 243)
    check(cache, cache.attend(q, sequence_ids=[0, 1], topk=topk), q)
    with cache.prepare_decode([0, 1], hq, topk=topk) as p:
        for step in range(3):
            qs = rand((2, hq, dim), torch.bfloat16, 250 + step)
            kn = rand((2, hk, dim), torch.bfloat16, 260 + step)
            check(cache, p.step(qs, kn, kn), qs)
