"""GPU parity of PreparedDecode with and without hipGraph replay (cases follow
tests/test_prepared_decode.py of the reference)."""
import pytest
import torch

from decode_check import check, rand

pytestmark = pytest.mark.gpu


def _paged():
    from moba_hip import PagedKVCache
    return PagedKVCache


@pytest.mark.parametrize("graph", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("page,chunk,dim,hq,hk", [(3, 4, 33, 15, 3), (7, 6, 64, 8, 1),
                                                   (16, 8, 128, 8, 2), (5, 8, 256, 6, 2)])
def test_prepared_steps_match_fp64(cuda_device, graph, dtype, page, chunk, dim, hq, hk):
    cache = _paged()(3, 40, hk, dim, page_size=page, chunk_size=chunk, dtype=dtype)
    k, v = rand((14, hk, dim), dtype, 501), rand((14, hk, dim), dtype, 502)
    cache.append(k, v, sequence_ids=[2, 0], cu_seqlens=[0, 5, 14])
    sk, sv = {2: k[:5], 0: k[5:]}, {2: v[:5], 0: v[5:]}
    lengths, table = cache.lengths, cache.page_table
    before = [cache.materialize(s) for s in (2, 0)]
    with cache.prepare_decode([2, 0], hq, topk=3) as plan:
        if graph:
            plan.capture("step").capture("attend")
            assert cache.lengths == lengths and cache.page_table == table
            for sid, (bk, bv) in zip((2, 0), before):
                ak, av = cache.materialize(sid)
                assert torch.equal(ak, bk) and torch.equal(av, bv)
        ptrs = [t.data_ptr() for t in (cache._table, cache._lengths, plan.output, plan.scores,
                                       plan.selected)]
        for step in range(10):
            q = rand((2, hq, dim), dtype, 510 + step)
            kn, vn = rand((2, hk, dim), dtype, 530 + step), rand((2, hk, dim), dtype, 550 + step)
            result = plan.step(q, kn, vn, use_graph=graph)
            for i, sid in enumerate((2, 0)):
                sk[sid] = torch.cat((sk[sid], kn[i:i + 1]))
                sv[sid] = torch.cat((sv[sid], vn[i:i + 1]))
                ak, av = cache.materialize(sid)
                assert torch.equal(ak, sk[sid]) and torch.equal(av, sv[sid])
            check(cache, result, q)
            check(cache, plan.attend(q, use_graph=graph), q)
        assert ptrs == [t.data_ptr() for t in (cache._table, cache._lengths, plan.output,
                                               plan.scores, plan.selected)]
        assert plan.delta_uploads <= 10
        with pytest.raises(ValueError, match="owns cache"):
            cache.reset()
    cache.reset([2])
    assert cache.lengths == (19, 0, 0)


@pytest.mark.parametrize("graph", [False, True])
@pytest.mark.parametrize("mode,topk", [("moba", 1), ("dense", 4), ("moba", 9)])
def test_prepared_empty_and_dense_fallback(cuda_device, graph, mode, topk):
    cache = _paged()(1, 17, 1, 8, page_size=3, chunk_size=4)
    with cache.prepare_decode([0], 4, topk=topk, mode=mode) as p:
        if graph:
            p.capture("step")
        for step in range(9):
            q = rand((1, 4, 8), cache.dtype, 601 + step)
            kv = rand((1, 1, 8), cache.dtype, 621 + step)
            check(cache, p.step(q, kv, kv, use_graph=graph), q)


def test_lifecycle_capacity_and_metadata_delta(cuda_device):
    c = _paged()(1, 7, 1, 8, page_size=3, chunk_size=4)
    q = torch.ones((1, 1, 8), device="cuda", dtype=c.dtype)
    with c.prepare_decode([0], 1) as p:
        before = c.lengths
        with pytest.raises(ValueError, match="NaN/Inf"):
            p.step(q * float("nan"), q, q)
        with pytest.raises(ValueError, match="capture"):
            p.step(q, q, q, use_graph=True)
        assert c.lengths == before
        for _ in range(7):
            p.step(q, q, q)
        assert p.delta_uploads == 3
        with pytest.raises(ValueError, match="max_seq_len"):
            p.step(q, q, q)
        assert c.lengths == (7,)
        with torch.cuda.stream(torch.cuda.Stream()):
            with pytest.raises(ValueError, match="cross-stream"):
                p.attend(q)
    with pytest.raises(ValueError, match="closed"):
        p.step(q, q, q)
    assert c.lengths == (7,)


def test_workspace_alias_and_output_reuse(cuda_device):
    c = _paged()(1, 8, 1, 8, page_size=3, chunk_size=4)
    q = torch.ones((1, 1, 8), device="cuda", dtype=c.dtype)
    with c.prepare_decode([0], 1, check_finite=False) as p:
        with pytest.raises(ValueError, match="aliases"):
            p.step(p.v, p.k, p.q)
        a = p.step(q, q, q)
        b = p.step(q, q, q)
        assert a.output.data_ptr() == b.output.data_ptr()


def test_capture_after_live_steps_and_capacity_boundary(cuda_device):
    c = _paged()(1, 4, 1, 8, page_size=1, chunk_size=2)
    q = torch.ones(1, 1, 8, device="cuda", dtype=c.dtype)
    with c.prepare_decode([0], 1) as p:
        for value in (1, 2, 3):
            p.step(q, q, q * value)
        before = c.materialize(0)
        p.capture("step").capture("attend")
        assert c.lengths == (3,)
        after = c.materialize(0)
        assert torch.equal(before[0], after[0]) and torch.equal(before[1], after[1])
        check(c, p.step(q, q, q * 4, use_graph=True), q)
        with pytest.raises(ValueError, match="max_seq_len"):
            p.step(q, q, q, use_graph=True)
        assert c.lengths == (4,)


def test_graph_closes_large_chunk_at_max_head_dim(cuda_device):
    c = _paged()(1, 1026, 1, 256, page_size=7, chunk_size=1024)
    k, v = rand((1023, 1, 256), c.dtype, 801), rand((1023, 1, 256), c.dtype, 802)
    c.append(k, v, sequence_ids=[0], cu_seqlens=[0, 1023])
    q = rand((1, 4, 256), c.dtype, 803)
    with c.prepare_decode([0], 4) as p:
        p.capture("step")
        check(c, p.step(q, k[:1], v[:1], use_graph=True), q)


def test_bound_input_buffers_graph_without_staging(cuda_device):
    c = _paged()(1, 8, 1, 1, page_size=4, chunk_size=2)
    with c.prepare_decode([0], 1, check_finite=False) as p:
        p.q.fill_(1)
        p.k.fill_(1)
        p.v.fill_(2)
        p.capture("step")
        for _ in range(3):
            result = p.step(p.q, p.k, p.v, use_graph=True)
            assert torch.equal(result.output, torch.full_like(result.output, 2))
        assert p.delta_uploads == 1
        with pytest.raises(ValueError, match="owns cache"):
            c.prepare_decode([0], 1)


def test_graph_replays_match_eager(cuda_device):
    """Several replays with eager work and syncs in between; every replay must
    equal the eager result bit-for-bit."""
    dtype = torch.bfloat16
    P = _paged()
    eager = P(2, 200, 2, 64, page_size=5, chunk_size=8, dtype=dtype)
    graphed = P(2, 200, 2, 64, page_size=5, chunk_size=8, dtype=dtype)
    k, v = rand((90, 2, 64), dtype, 901), rand((90, 2, 64), dtype, 902)
    for c in (eager, graphed):
        c.append(k, v, sequence_ids=[0, 1], cu_seqlens=[0, 40, 90])
    with eager.prepare_decode([0, 1], 12, topk=4) as pe, \
            graphed.prepare_decode([0, 1], 12, topk=4) as pg:
        pg.capture("step")
        for step in range(12):
            q = rand((2, 12, 64), dtype, 910 + step)
            kn, vn = rand((2, 2, 64), dtype, 930 + step), rand((2, 2, 64), dtype, 950 + step)
            a = pe.step(q, kn, vn)
            _ = torch.randn(1000, device="cuda").sum().item()  # eager work between replays
            b = pg.step(q, kn, vn, use_graph=True)
            torch.cuda.synchronize()
            assert torch.equal(a.output, b.output) and torch.equal(a.lse, b.lse)
            assert torch.equal(a.selected_blocks, b.selected_blocks)


def test_bound_buffer_steps_match_copied_inputs(cuda_device):
    """step() with the plan's own q / k / v buffers as the inputs takes one
    native call (plan, launch, commit) instead of staging copies; eager and
    graph steps must give the same outputs, routes, positions and cache
    contents as steps whose inputs are separate tensors."""
    dtype = torch.bfloat16
    P = _paged()
    copied = P(2, 200, 2, 64, page_size=5, chunk_size=8, dtype=dtype)
    bound = P(2, 200, 2, 64, page_size=5, chunk_size=8, dtype=dtype)
    k, v = rand((90, 2, 64), dtype, 961), rand((90, 2, 64), dtype, 962)
    for c in (copied, bound):
        c.append(k, v, sequence_ids=[0, 1], cu_seqlens=[0, 40, 90])
    with copied.prepare_decode([1, 0], 12, topk=4, check_finite=False) as pc, \
            bound.prepare_decode([1, 0], 12, topk=4, check_finite=False) as pb:
        with pytest.raises(ValueError, match="capture"):
            pb.step(pb.q, pb.k, pb.v, use_graph=True)
        pc.capture("step")
        pb.capture("step")
        for step in range(10):
            graph = step >= 5
            q = rand((2, 12, 64), dtype, 970 + step)
            kn, vn = rand((2, 2, 64), dtype, 980 + step), rand((2, 2, 64), dtype, 990 + step)
            a = pc.step(q, kn, vn, use_graph=graph)
            pb.q.copy_(q)
            pb.k.copy_(kn)
            pb.v.copy_(vn)
            b = pb.step(pb.q, pb.k, pb.v, use_graph=graph)
            torch.cuda.synchronize()
            assert a.positions == b.positions
            assert torch.equal(a.output, b.output) and torch.equal(a.lse, b.lse)
            assert torch.equal(a.selected_blocks, b.selected_blocks)
        assert pc.lengths == pb.lengths
    for sid in range(2):
        ka, va = copied.materialize(sid)
        kb, vb = bound.materialize(sid)
        assert torch.equal(ka, kb) and torch.equal(va, vb)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prepared_route_ties_pick_lowest_chunks(cuda_device, dtype):
    """Constant keys make every closed chunk's gate score equal: the fused
    route must then pick the lowest chunks, in order, exactly as the oracle's
    (score desc, chunk asc) rule does (kv_cache.py:208-223 top-k semantics)."""
    cache = _paged()(2, 60, 2, 64, page_size=5, chunk_size=4, dtype=dtype)
    k = torch.ones((30, 2, 64), dtype=dtype, device="cuda")
    v = rand((30, 2, 64), dtype, 601)
    cache.append(k, v, sequence_ids=[1, 0], cu_seqlens=[0, 13, 30])
    with cache.prepare_decode([1, 0], 12, topk=4) as plan:
        for step in range(6):
            q = rand((2, 12, 64), dtype, 610 + step)
            kn = torch.ones((2, 2, 64), dtype=dtype, device="cuda")
            vn = rand((2, 2, 64), dtype, 630 + step)
            result = plan.step(q, kn, vn)
            check(cache, result, q)
            sel = result.selected_blocks.cpu()
            for row in range(2):
                cur = int(sel[row, 0, 0])
                want = list(range(min(3, cur)))
                assert sel[row, :, 1:1 + len(want)].tolist() == [want] * 12


@pytest.mark.parametrize("graph", [False, True])
def test_decode_under_inference_mode(cuda_device, graph):
    """A cache built, filled and stepped entirely under torch.inference_mode
    gives the same outputs, routes and lengths as the same calls without it."""
    def run(inference):
        with torch.inference_mode(inference):
            cache = _paged()(2, 64, 2, 64, page_size=5, chunk_size=8)
            k, v = rand((30, 2, 64), torch.bfloat16, 601), rand((30, 2, 64), torch.bfloat16, 602)
            cache.append(k, v, sequence_ids=[1, 0], cu_seqlens=[0, 17, 30])
            outs = [cache.attend(rand((2, 6, 64), torch.bfloat16, 603), sequence_ids=[1, 0],
                                 topk=3).output.clone()]
            with cache.prepare_decode([1, 0], 6, topk=3) as plan:
                if graph:
                    plan.capture("step")
                for step in range(4):
                    r = plan.step(rand((2, 6, 64), torch.bfloat16, 610 + step),
                                  rand((2, 2, 64), torch.bfloat16, 620 + step),
                                  rand((2, 2, 64), torch.bfloat16, 630 + step), use_graph=graph)
                    outs += [r.output.clone(), r.selected_blocks.clone()]
            return outs, cache.lengths

    (a, la), (b, lb) = run(False), run(True)
    assert la == lb
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_step_input_errors_follow_argument_order(cuda_device):
    """q, k, v are checked in that order, each fully before the next, with
    the NaN/Inf test of all three through one flag; nothing changes."""
    cache = _paged()(2, 40, 2, 16, page_size=4, chunk_size=8)
    k, v = rand((9, 2, 16), torch.bfloat16, 701), rand((9, 2, 16), torch.bfloat16, 702)
    cache.append(k, v, sequence_ids=[0, 1], cu_seqlens=[0, 4, 9])
    nan = float("nan")
    with cache.prepare_decode([0, 1], 4, topk=2) as p:
        q, kn, vn = rand((2, 4, 16), torch.bfloat16, 703), *(rand((2, 2, 16), torch.bfloat16, s)
                                                              for s in (704, 705))
        lengths = cache.lengths
        cases = [((q * nan, kn[:1], vn), "q contains NaN/Inf"),
                 ((q, kn * nan, vn * nan), "k contains NaN/Inf"),
                 ((q, kn, vn * nan), "v contains NaN/Inf"),
                 ((q, kn * nan, vn[:1]), "k contains NaN/Inf"),
                 ((q, kn, vn[:1]), "v must have fixed shape")]
        for args, msg in cases:
            with pytest.raises(ValueError, match=msg):
                p.step(*args)
        assert cache.lengths == lengths
        r = p.step(q, kn, vn)
        assert cache.lengths == tuple(n + 1 for n in lengths) and r.output.isfinite().all()


@pytest.mark.parametrize("graph", [False, True])
def test_uncommitted_page_grant_never_reaches_the_table(cuda_device, graph):
    """A step planned at a page boundary whose launch never ran (as after a
    failed launch: the plan uploaded its page grant, nothing committed it)
    must not leave that grant on the device: the next attend and step apply
    a clean delta, so the device page table keeps matching the host pool."""
    from moba_hip.ops import _lib  # noqa: F401
    c = _paged()(1, 12, 1, 8, page_size=3, chunk_size=4)
    k = rand((3, 1, 8), c.dtype, 901)
    c.append(k, k, sequence_ids=[0], cu_seqlens=[0, 3])
    q = rand((1, 2, 8), c.dtype, 902)
    with c.prepare_decode([0], 2) as p:
        if graph:
            p.capture("attend").capture("step")
        stream = torch.cuda.current_stream().cuda_stream
        assert p._plan_step(stream) == (3,)   # token 3 opens logical page 1: a grant
        p.attend(q, use_graph=graph)          # no launch or commit of the step above
        torch.cuda.synchronize()
        host = [list(r) for r in p.page_table]
        assert host[0][1] == -1
        assert c._table[0].tolist()[:len(host[0])] == host[0]
        kn = rand((1, 1, 8), c.dtype, 903)
        check(c, p.step(q, kn, kn, use_graph=graph), q)
        torch.cuda.synchronize()
        assert c._table[0].tolist()[:len(host[0])] == [list(r) for r in p.page_table][0]
