"""Pin the CPU oracle (oracle/moba_oracle.c) before trusting it.

Every oracle function is checked against something it does not share code
with: the reference's known answers (tests/golden/known_answers.json), a
closed form, an independent dense-mask formulation, torch FP64 autograd,
finite differences, or brute force on tiny inputs.
"""
import itertools
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle as O

GOLD = json.loads((Path(__file__).parent / "golden" / "known_answers.json").read_text())


def _f(x):
    return -np.inf if x == "-inf" else float(x)


# ------------------------------------------------------------ dtype helpers

def test_bf16_and_fp16_rounding_match_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(4000).astype(np.float32) * s
                        for s in (1e-6, 1e-3, 1.0, 300.0, 6e4)]
                       + [np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 6.1e-5, 5.96e-8,
                                    2.98e-8, 1e-9], np.float32)])
    for code, tdt in ((0, torch.bfloat16), (1, torch.float16)):
        want = torch.from_numpy(x).to(tdt).float().numpy()
        got = np.array([O.round_to_dtype(float(v), code) for v in x], np.float32)
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


# ------------------------------------------------------------------ top-k

def test_stable_topk_known_answer():
    case = GOLD["stable_topk"]
    scores = np.array([_f(x) for x in case["scores"]], np.float32)
    idx, _ = O.stable_topk(scores, case["k"])
    assert idx.tolist() == case["expected_indices"]
    # the reference derives it from a stable descending argsort
    want = torch.tensor(scores).argsort(descending=True, stable=True)[:4].tolist()
    assert idx.tolist() == want
    idx, _ = O.stable_topk(np.full(5, -np.inf, np.float32), 4)
    assert idx.tolist() == [-1] * 4


@pytest.mark.parametrize("seed", range(20))
def test_stable_topk_brute_force(seed):
    rng = np.random.default_rng(seed)
    n, k = int(rng.integers(0, 12)), int(rng.integers(1, 9))
    s = rng.integers(-3, 3, n).astype(np.float32)  # many exact ties
    s[rng.random(n) < 0.2] = -np.inf
    idx, _ = O.stable_topk(s, k)
    order = sorted([i for i in range(n) if np.isfinite(s[i])], key=lambda i: (-s[i], i))[:k]
    assert idx.tolist() == order + [-1] * (k - len(order))


# --------------------------------------------------------------- chunking

@pytest.mark.parametrize("lens,C", [([9, 5], 4), ([1], 4), ([7], 3), ([4, 4, 1], 4), ([16], 16)])
def test_calc_chunks_closed_form(lens, C):
    cu = [0] + list(itertools.accumulate(lens))
    cu_chunk, chunk_batch, filtered = O.calc_chunks(cu, C)
    # rebuilt independently: chunk boundaries every C tokens inside each sequence
    bounds = sorted(set(x for b in range(len(lens)) for x in range(cu[b], cu[b + 1], C)) | {cu[-1]})
    assert cu_chunk == bounds
    last = {max(i for i, b in enumerate(chunk_batch) if b == s) for s in range(len(lens))}
    assert filtered == [c for c in range(len(chunk_batch)) if c not in last]


# ---------------------------------------------------------------- routing

def _canon_sum(x):
    """Independent numpy restatement of the canonical order: 64 strided fp32
    partial sums, then the fixed pairwise tree (off = 32, 16, ..., 1)."""
    part = np.zeros((64,) + x.shape[1:], np.float32)
    for j in range(64):
        acc = np.zeros(x.shape[1:], np.float32)
        for t in range(j, x.shape[0], 64):
            acc = (acc + x[t]).astype(np.float32)
        part[j] = acc
    off = 32
    while off:
        part[:off] = (part[:off] + part[off:2 * off]).astype(np.float32)
        off //= 2
    return part[0]


@pytest.mark.parametrize("precision", [0, 1])
@pytest.mark.parametrize("C", [8, 70, 200])
def test_chunk_means_canonical_order(precision, C):
    torch.manual_seed(3)
    k = torch.randn(3 * C + 5, 2, 8).bfloat16()
    cu_chunk, _, filtered = O.calc_chunks([0, k.shape[0]], C)
    m = O.chunk_means(O.bits16(k), 0, cu_chunk, filtered, C, precision)
    kf = k.float().numpy()
    for f, c in enumerate(filtered):
        want = (_canon_sum(kf[cu_chunk[c]:cu_chunk[c] + C]) / np.float32(C)).astype(np.float32)
        if precision == 0:
            want = torch.from_numpy(want).bfloat16().float().numpy()
        np.testing.assert_array_equal(m[f].view(np.uint32), want.view(np.uint32))
    # and it is the mean to within about one rounding of the dtype
    exact = kf[:3 * C].reshape(3, C, 2, 8).astype(np.float64).mean(1)
    assert np.abs(m - exact).max() <= 2 ** -7 * np.abs(exact).max() + 1e-5


def test_route_prefill_brute_force():
    torch.manual_seed(5)
    lens, C, hq, hkv, d, topk = [37, 20, 45], 6, 6, 2, 16, 4
    cu = [0] + list(itertools.accumulate(lens))
    q = torch.randn(sum(lens), hq, d).bfloat16()
    k = torch.randn(sum(lens), hkv, d).bfloat16()
    cu_chunk, chunk_batch, filtered = O.calc_chunks(cu, C)
    R = min(topk - 1, len(filtered))
    means = O.chunk_means(O.bits16(k), 0, cu_chunk, filtered, C, 1)
    sel, gate = O.route_prefill(O.bits16(q), 0, means, cu_chunk, chunk_batch, R, want_gate=True)
    qf = q.float().numpy()
    for s in range(sum(lens)):
        b = max(i for i in range(len(lens)) if cu[i] <= s)
        legal = [f for f, c in enumerate(filtered)
                 if chunk_batch[c] == b and cu_chunk[c + 1] <= s]
        for h in range(hq):
            g = {}
            for f in legal:
                acc = np.float32(0)
                for j in range(d):  # fma chain == exact product + one rounding
                    acc = np.float32(np.float64(means[f, h // 3, j]) * np.float64(qf[s, h, j]) + acc)
                g[f] = acc
                assert gate[f, h, s] == acc
            for f in set(range(len(filtered))) - set(legal):
                assert gate[f, h, s] == -np.inf
            best = sorted(legal, key=lambda f: (-g[f], f))[:R]
            want = sorted(filtered[f] for f in best)
            assert sel[s, h].tolist() == want + [-1] * (R - len(want))


# -------------------------------------------------------------- attention

def _dense_mask_attention(q, k, v, cu, cu_chunk, chunk_batch, filtered, sel):
    """Independent formulation (reference/fixed_route_attention.py:66-119 style):
    per sequence and head build the [L,L] boolean mask, masked softmax in FP64."""
    T, hq, d = q.shape
    G = hq // k.shape[1]
    o, lse = np.zeros_like(q), np.zeros((T, hq))
    for b in range(len(cu) - 1):
        s0, s1 = cu[b], cu[b + 1]
        L = s1 - s0
        base = np.zeros((L, L), bool)
        for c, bb in enumerate(chunk_batch):
            if bb == b:
                a0, a1 = cu_chunk[c] - s0, cu_chunk[c + 1] - s0
                base[a0:a1, a0:a1] = np.tril(np.ones((a1 - a0, a1 - a0), bool))
        for h in range(hq):
            mask = base.copy()
            if sel is not None:
                for s in range(s0, s1):
                    for c in sel[s, h]:
                        if c >= 0:
                            mask[s - s0, cu_chunk[c] - s0:cu_chunk[c + 1] - s0] = True
            logits = q[s0:s1, h] @ k[s0:s1, h // G].T / np.sqrt(d)
            logits = np.where(mask, logits, -np.inf)
            m = logits.max(1, keepdims=True)
            p = np.exp(logits - m)
            z = p.sum(1, keepdims=True)
            o[s0:s1, h] = (p / z) @ v[s0:s1, h // G]
            lse[s0:s1, h] = (m + np.log(z))[:, 0]
    return o, lse


def _random_route(cu, cu_chunk, chunk_batch, filtered, hq, R, rng):
    T = cu[-1]
    sel = np.full((T, hq, R), -1, np.int32)
    for s in range(T):
        b = max(i for i in range(len(cu) - 1) if cu[i] <= s)
        legal = [c for c in filtered if chunk_batch[c] == b and cu_chunk[c + 1] <= s]
        for h in range(hq):
            pick = sorted(rng.choice(legal, size=min(R, len(legal)), replace=False).tolist()) \
                if legal else []
            sel[s, h, :len(pick)] = pick
    return sel


@pytest.mark.parametrize("lens,C,hq,hkv,d", [([9, 5], 4, 3, 3, 8), ([13], 3, 4, 2, 8),
                                             ([4, 4, 1], 4, 2, 1, 4), ([30, 17], 5, 6, 3, 16)])
def test_fwd_matches_dense_mask_formulation(lens, C, hq, hkv, d):
    rng = np.random.default_rng(1)
    cu = [0] + list(itertools.accumulate(lens))
    q, k, v = (rng.standard_normal((cu[-1], h, d)) for h in (hq, hkv, hkv))
    cu_chunk, chunk_batch, filtered = O.calc_chunks(cu, C)
    sel = _random_route(cu, cu_chunk, chunk_batch, filtered, hq, 2, rng)
    o, lse = O.attention_fwd(q, k, v, cu_chunk, sel)
    o2, lse2 = _dense_mask_attention(q, k, v, cu, cu_chunk, chunk_batch, filtered, sel)
    np.testing.assert_allclose(o, o2, atol=1e-12)
    np.testing.assert_allclose(lse, lse2, atol=1e-12)


def test_all_legal_route_equals_dense_causal():
    rng = np.random.default_rng(2)
    lens, C, h, d = [9, 5], 4, 3, 8
    cu = [0] + list(itertools.accumulate(lens))
    q, k, v = (rng.standard_normal((cu[-1], h, d)) for _ in range(3))
    cu_chunk, chunk_batch, filtered = O.calc_chunks(cu, C)
    R = len(filtered)
    sel = _random_route(cu, cu_chunk, chunk_batch, filtered, h, R, rng)  # R >= legal: all chosen
    o, lse = O.attention_fwd(q, k, v, cu_chunk, sel)
    od, lsed = O.attention_fwd(q, k, v, cu, None)  # one chunk per sequence == dense causal
    np.testing.assert_allclose(o, od, atol=1e-12)
    np.testing.assert_allclose(lse, lsed, atol=1e-12)


def test_gqa_equals_repeated_mha():
    rng = np.random.default_rng(3)
    cu = [0, 21]
    q = rng.standard_normal((21, 6, 8))
    k, v = rng.standard_normal((21, 2, 8)), rng.standard_normal((21, 2, 8))
    cu_chunk, chunk_batch, filtered = O.calc_chunks(cu, 5)
    sel = _random_route(cu, cu_chunk, chunk_batch, filtered, 6, 2, rng)
    o, _ = O.attention_fwd(q, k, v, cu_chunk, sel)
    o2, _ = O.attention_fwd(q, np.repeat(k, 3, 1), np.repeat(v, 3, 1), cu_chunk, sel)
    np.testing.assert_allclose(o, o2, atol=1e-13)
    g = rng.standard_normal(q.shape)
    _, lse = O.attention_fwd(q, k, v, cu_chunk, sel)
    dq, dk, dv = O.attention_bwd(q, k, v, g, cu_chunk, sel, lse)
    dq2, dk2, dv2 = O.attention_bwd(q, np.repeat(k, 3, 1), np.repeat(v, 3, 1), g, cu_chunk, sel, lse)
    np.testing.assert_allclose(dq, dq2, atol=1e-12)
    np.testing.assert_allclose(dk, dk2.reshape(21, 2, 3, 8).sum(2), atol=1e-12)
    np.testing.assert_allclose(dv, dv2.reshape(21, 2, 3, 8).sum(2), atol=1e-12)


def test_bwd_matches_torch_autograd_and_finite_differences():
    rng = np.random.default_rng(4)
    lens, C, hq, hkv, d = [11, 7], 3, 4, 2, 4
    cu = [0] + list(itertools.accumulate(lens))
    T = cu[-1]
    q, k, v = (rng.standard_normal((T, h, d)) for h in (hq, hkv, hkv))
    g = rng.standard_normal((T, hq, d))
    cu_chunk, chunk_batch, filtered = O.calc_chunks(cu, C)
    sel = _random_route(cu, cu_chunk, chunk_batch, filtered, hq, 2, rng)
    _, lse = O.attention_fwd(q, k, v, cu_chunk, sel)
    dq, dk, dv = O.attention_bwd(q, k, v, g, cu_chunk, sel, lse)

    # torch FP64 autograd of the dense-mask formulation
    qt, kt, vt = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    G = hq // hkv
    outs = []
    for b in range(len(lens)):
        s0, s1 = cu[b], cu[b + 1]
        L = s1 - s0
        heads = []
        for h in range(hq):
            mask = torch.zeros(L, L, dtype=torch.bool)
            for c, bb in enumerate(chunk_batch):
                if bb == b:
                    a0, a1 = cu_chunk[c] - s0, cu_chunk[c + 1] - s0
                    mask[a0:a1, a0:a1] = torch.ones(a1 - a0, a1 - a0, dtype=torch.bool).tril()
            for s in range(s0, s1):
                for c in sel[s, h]:
                    if c >= 0:
                        mask[s - s0, cu_chunk[c] - s0:cu_chunk[c + 1] - s0] = True
            logits = qt[s0:s1, h] @ kt[s0:s1, h // G].T * d ** -0.5
            heads.append(torch.softmax(logits.masked_fill(~mask, -float("inf")), -1)
                         @ vt[s0:s1, h // G])
        outs.append(torch.stack(heads, 1))
    out = torch.cat(outs)
    ref = torch.autograd.grad(out, (qt, kt, vt), grad_outputs=torch.tensor(g))
    for a, r in zip((dq, dk, dv), ref):
        np.testing.assert_allclose(a, r.numpy(), atol=1e-11)

    # central finite differences of <O, g> on a few coordinates of k
    def loss(kk):
        o, _ = O.attention_fwd(q, kk, v, cu_chunk, sel)
        return float((o * g).sum())
    eps = 1e-6
    for idx in [(0, 0, 0), (5, 1, 3), (12, 0, 2), (17, 1, 1)]:
        kp, km = k.copy(), k.copy()
        kp[idx] += eps
        km[idx] -= eps
        assert abs((loss(kp) - loss(km)) / (2 * eps) - dk[idx]) < 1e-6


# ------------------------------------------------------------------ merge

def test_merge_closed_forms():
    rng = np.random.default_rng(6)
    so, sl = rng.standard_normal((5, 4)), rng.standard_normal(5)
    # no remote rows: identity
    o, l = O.merge(so, sl, np.zeros((0, 4)), np.zeros(0), np.zeros(0, np.int64))
    np.testing.assert_array_equal(o, so)
    np.testing.assert_allclose(l, sl, atol=1e-15)
    # manual two-branch case
    ro, rl, mp = rng.standard_normal((5, 4)), rng.standard_normal(5), np.arange(5)
    o, l = O.merge(so, sl, ro, rl, mp)
    m = np.maximum(sl, rl)
    w1, w2 = np.exp(sl - m), np.exp(rl - m)
    np.testing.assert_allclose(o, (w1[:, None] * so + w2[:, None] * ro) / (w1 + w2)[:, None], atol=1e-14)
    np.testing.assert_allclose(l, m + np.log(w1 + w2), atol=1e-14)
    # extreme LSE gap: the dominant branch wins without NaN
    o, l = O.merge(so, np.full(5, -1e30), ro, np.full(5, 1e30), mp)
    assert np.isfinite(o).all() and np.isfinite(l).all()
    np.testing.assert_allclose(o, ro, atol=1e-12)


def test_merge_equals_attention_over_union():
    """Merging the (o, lse) of disjoint key sets equals attention over the union."""
    rng = np.random.default_rng(7)
    q, k, v = rng.standard_normal((1, 1, 8)), rng.standard_normal((10, 1, 8)), rng.standard_normal((10, 1, 8))

    def att(keys):
        lg = k[keys, 0] @ q[0, 0] / np.sqrt(8)
        m = lg.max()
        p = np.exp(lg - m)
        return (p / p.sum()) @ v[keys, 0], m + np.log(p.sum())
    o1, l1 = att([0, 1, 2])
    o2, l2 = att([3, 4])
    o3, l3 = att([5, 6, 7, 8, 9])
    o, l = O.merge(o1[None], np.array([l1]), np.stack([o2, o3]), np.array([l2, l3]), np.array([0, 0]))
    ou, lu = att(list(range(10)))
    np.testing.assert_allclose(o[0], ou, atol=1e-13)
    np.testing.assert_allclose(l[0], lu, atol=1e-13)


# ----------------------------------------------------------------- decode

def test_decode_uniform_known_answer():
    case = GOLD["decode_uniform"]
    hq, hk, d, n = case["num_q_heads"], case["num_kv_heads"], case["head_dim"], case["tokens"]
    v = np.arange(n * hk * d, dtype=np.float64).reshape(n, hk, d)
    k = np.zeros((n, hk, d))
    for pos in case["positions"]:
        out, lse = O.decode_attention(np.zeros((hq, d)), k, v, 2, pos)
        for h in range(hq):
            np.testing.assert_allclose(out[h], v[:pos + 1, h // 2].mean(0), atol=1e-12)
        np.testing.assert_allclose(lse, np.full(hq, np.log(pos + 1)), atol=1e-12)


def test_decode_route_staircase_known_answer():
    case = GOLD["decode_routing_staircase"]
    n, C, hk, d, hq = (case[x] for x in ("num_tokens", "chunk", "num_kv_heads", "head_dim",
                                         "num_q_heads"))
    k = torch.zeros(n, hk, d)
    for blk in range(4):
        k[blk * 4:min((blk + 1) * 4, n), 0, 0] = case["key_dim0_per_block"]["kv0"][blk]
        k[blk * 4:min((blk + 1) * 4, n), 1, 0] = case["key_dim0_per_block"]["kv1"][blk]
    kb = O.bits16(k.bfloat16())
    means = O.decode_means(kb, 0, C)
    q = torch.zeros(hq, d)
    q[:, 0] = 1
    qb = O.bits16(q.bfloat16())
    got = {}
    for row, pos in enumerate(case["positions"]):
        _, sel = O.decode_route(qb, means, 0, C, pos, pos // C, case["topk"] - 1)
        got[row] = sel
    exp = case["expected_sets"]
    assert set(got[0][0].tolist()) == set(exp["row0_head0"])
    assert set(got[0][2].tolist()) == set(exp["row0_head2"])
    assert set(got[1][0].tolist()) == set(exp["row1_head0"])


def test_decode_means_quantised_mean_and_partition_free():
    torch.manual_seed(8)
    for code, tdt in ((0, torch.bfloat16), (1, torch.float16)):
        k = torch.randn(50, 3, 12).to(tdt)
        m = torch.from_numpy(O.decode_means(O.bits16(k), code, 8)).view(tdt).double()
        exact = k.double()[:48].reshape(6, 8, 3, 12).mean(1)
        quant = exact.to(tdt).double()
        ulp = (quant.abs() * (2 ** -7 if code == 0 else 2 ** -10)).clamp_min(1e-7)
        assert ((m - quant).abs() <= ulp).all()


def test_decode_attention_matches_dense_when_routes_cover_history():
    rng = np.random.default_rng(9)
    k, v, q = rng.standard_normal((23, 2, 8)), rng.standard_normal((23, 2, 8)), rng.standard_normal((4, 8))
    pos, C = 22, 5
    chunks = np.array([[pos // C] + list(range(pos // C))] * 4, np.int32)
    o1, l1 = O.decode_attention(q, k, v, C, pos, chunks)
    o2, l2 = O.decode_attention(q, k, v, C, pos, None)
    np.testing.assert_allclose(o1, o2, atol=1e-13)
    np.testing.assert_allclose(l1, l2, atol=1e-13)
