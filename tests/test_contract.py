"""CPU contract tests: validation envelope, registry, cache constructor
errors before any GPU work, and the C-ABI library surface (loads and exports
every symbol include/moba_hip.h declares; argument errors return without
touching a device)."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from moba_hip import api
from moba_hip.baseline_adapter import validate_config, validate_shapes
from moba_hip.kv_cache import PagedKVCache, _mode
from moba_hip.ops import _lib

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.parametrize("hq,hkv", [(1, 1), (28, 4), (32, 8), (16, 2), (8, 1), (14, 2)])
def test_grouped_shapes(hq, hkv):
    assert validate_shapes((11, hq, 128), (11, hkv, 128), (11, hkv, 128), True) == hq // hkv


@pytest.mark.parametrize("dim", range(8, 257, 8))
def test_head_dimensions(dim):
    assert validate_shapes((3, 2, dim), (3, 2, dim), (3, 2, dim)) == 1


@pytest.mark.parametrize("qs,ks,vs", [
    ((0, 2, 64), (0, 2, 64), (0, 2, 64)), ((3, 3, 64), (3, 2, 64), (3, 2, 64)),
    ((3, 2, 7), (3, 2, 7), (3, 2, 7)), ((3, 2, 264), (3, 2, 264), (3, 2, 264)),
    ((3, 2, 64), (4, 2, 64), (4, 2, 64)), ((3, 2, 64), (3, 1, 64), (3, 2, 64)),
])
def test_invalid_shapes(qs, ks, vs):
    with pytest.raises(ValueError):
        validate_shapes(qs, ks, vs, True)


def test_mha_only_entry_rejects_gqa():
    with pytest.raises(ValueError, match="MHA only"):
        validate_shapes((3, 4, 64), (3, 2, 64), (3, 2, 64), False)


@pytest.mark.parametrize("override", [
    {"chunk_size": 0}, {"chunk_size": True}, {"topk": 0}, {"topk": 10},
    {"topk": 2.5}, {"causal": False}, {"dropout": 0.1},
])
def test_invalid_configs(override):
    with pytest.raises(ValueError):
        validate_config({"chunk_size": 32, "topk": 4, **override})


def test_registry_contract():
    assert {"opt_hip", "opt_merge_hip"} <= set(api.available_impls())
    with pytest.raises(KeyError, match="already registered"):
        api.register("opt_hip", lambda *a: None)
    with pytest.raises(KeyError, match="unknown impl"):
        api.run_impl("nope", None, None, None, None, None, None)


def test_prefill_rejects_cpu_tensors():
    q = torch.randn(8, 2, 64).bfloat16()
    cu = torch.tensor([0, 8], dtype=torch.int32)
    with pytest.raises(ValueError, match="CUDA"):
        api.run_impl("opt_hip", q, q, q, cu, 8, {"chunk_size": 4, "topk": 3})


@pytest.mark.parametrize("kwargs", [
    {"head_dim": 0}, {"head_dim": 264}, {"num_kv_heads": 0}, {"page_size": 0},
    {"num_pages": 0}, {"chunk_size": 1025}, {"dtype": torch.float32}, {"device": "cpu"},
])
def test_cache_contract_before_gpu_initialization(kwargs):
    cfg = dict(batch_size=1, max_seq_len=16, num_kv_heads=2, head_dim=64)
    cfg.update(kwargs)
    with pytest.raises(ValueError):
        PagedKVCache(**cfg)


@pytest.mark.parametrize("mode,topk", [("other", 4), ("dense", 0), ("moba", 10), ("moba", True)])
def test_decode_mode_contract(mode, topk):
    with pytest.raises(ValueError):
        _mode(mode, topk)


@pytest.mark.parametrize("bad", [None, torch.zeros(()), torch.zeros(4, 2)])
def test_decode_input_checks_run_in_argument_order(bad):
    """The NaN/Inf-batched checks of append / append_and_attend: a malformed
    k raises the [N,H,D] ValueError (kv_cache.py:166-167 in the reference)
    before the token counts of v and q, which depend on k, are looked at."""
    from moba_hip import decode_contract as contract
    v = torch.zeros(3, 2, 8)
    kw = dict(device=torch.device("cpu"), dtype=torch.float32, head_dim=8)
    for specs in (
        ((bad, "k", {"heads": 2}), (v, "v", {"heads": 2, "tokens": lambda: bad.shape[0]})),
        ((bad, "k", {"heads": 2}), (v, "v", {"heads": 2, "tokens": lambda: bad.shape[0]}),
         (v, "q", {"tokens": lambda: bad.shape[0]})),
    ):
        with pytest.raises(ValueError, match=r"k must be \[N,H,D\]"):
            contract.tensors(specs, **kw)
    k = torch.zeros(2, 2, 8)
    with pytest.raises(ValueError, match="v token count differs"):
        contract.tensors(((k, "k", {"heads": 2}), (v, "v", {"heads": 2, "tokens": lambda: k.shape[0]})),
                         **kw)


def _declared_symbols():
    text = (ROOT / "include" / "moba_hip.h").read_text()
    return sorted(set(re.findall(r"\b(moba_(?:hip|pool|prep)_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    names = _declared_symbols()
    assert len(names) >= 13
    for name in names:
        assert hasattr(lib, name), f"{name} missing from libmoba_hip.so"
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"
    assert _lib.load().moba_hip_version() == 1


def test_argument_errors_are_reported_without_a_device():
    with pytest.raises(_lib.MobaHipError, match="dtype"):
        _lib.call("moba_hip_prefill_fwd", None, None, None, 7, 1, 1, 1, 64, 1.0, None, None, 0,
                  None, 0, None, 0, None, None, None, None, 0, None, None, None, None, None)
    with pytest.raises(_lib.MobaHipError, match="head_dim"):
        _lib.call("moba_hip_prefill_bwd", None, None, None, None, None, None, 0, 1, 1, 1, 12,
                  1.0, None, None, 0, None, 0, None, 0, None, 0, None, None, None, None, 0,
                  None, None, None, None, None, 3, 1, None, None, None)
    with pytest.raises(_lib.MobaHipError, match="kv_splits"):
        _lib.call("moba_hip_prefill_bwd", None, None, None, None, None, None, 0, 1, 1, 1, 64,
                  1.0, None, None, 0, None, 0, None, 0, None, 0, None, None, None, None, 0,
                  None, None, None, None, None, 3, 2, None, None, None)
    with pytest.raises(_lib.MobaHipError, match="n_kv_tiles <= 4096"):
        _lib.call("moba_hip_prefill_bwd", None, None, None, None, None, None, 0, 1, 1, 1, 64,
                  1.0, None, None, 0, None, 4097, None, 0, None, 0, None, None, None, None, 0,
                  None, None, None, None, None, 3, 2, 1, None, None)
    with pytest.raises(_lib.MobaHipError, match="remote count"):
        _lib.call("moba_hip_route_prefill", None, 0, 1, 1, 1, 8, None, None, 1, None, None, 9, 1,
                  None, None, None)
    with pytest.raises(_lib.MobaHipError, match="head_dim"):
        _lib.call("moba_hip_paged_attention", None, 0, 1, 1, 1, 300, None, None, 1, None, 1,
                  None, None, None, None, 1, None, None, 0, 4, 1, None, None, None, None, None)
    with pytest.raises(_lib.MobaHipError, match="work list"):
        _lib.call("moba_hip_paged_attention", None, 0, 1, 1, 1, 64, None, None, 1, None, 1,
                  None, None, None, None, 2, None, None, 0, 4, 1, None, None, None, None, None)


def test_row_split_workspace_size():
    """Schedule head (16 B per workgroup + 8 B per tile, 256-byte aligned),
    then one [dK | dV][128 keys][D] fp32 slot per workgroup."""
    f = _lib.load().moba_hip_prefill_bwd_work
    assert f(256, 4, 64) == -(-(16 * 1024 + 8 * 256) // 256) * 256 + 1024 * 2 * 128 * 64 * 4
    assert f(3, 2, 128) == 256 + 6 * 2 * 128 * 128 * 4
    assert f(256, 1, 64) == 0 and f(0, 4, 64) == 0 and f(8, 17, 64) == 0


@pytest.mark.parametrize("att_chunk,hkv,rows", [
    ([i * 4096 for i in range(9)], 32, 128),      # cfg3: 8 chunks x 32 kv heads
    ([0, 2048, 4096, 6144, 8192], 2, 128),
    ([0, 300, 4396], 1, 128),                     # ragged, fewer tiles than XCDs per run
    ([0, 1, 3, 70], 3, 64),
])
def test_self_tile_order_is_a_partition_in_xcd_runs(att_chunk, hkv, rows):
    """The causal work list holds every (chunk, first row, kv head) tile
    once, in 8 equal-length runs whose attended keys differ by at most two of
    the largest tiles, each run's tiles above a quarter of the largest first."""
    from moba_hip.ops.prefill import PrefillPlan
    order = PrefillPlan._self_tile_order(att_chunk, hkv, rows)
    assert len(order) % 8 == 0
    want = {(c, r0, kh) for kh in range(hkv) for c in range(len(att_chunk) - 1)
            for r0 in range(0, att_chunk[c + 1] - att_chunk[c], rows)}
    got = [t for t in order if t[0] >= 0]
    assert len(got) == len(want) and set(got) == want
    n = len(order) // 8

    def keys(t):
        return min(t[1] + rows, att_chunk[t[0] + 1] - att_chunk[t[0]])
    big = max(keys(t) for t in got)
    loads = []
    for x in range(8):
        run = [t for t in order[x * n:(x + 1) * n] if t[0] >= 0]
        assert all(t[0] < 0 for t in order[x * n + len(run):(x + 1) * n])  # padding last
        loads.append(sum(keys(t) for t in run))
        small = [4 * keys(t) <= big for t in run]
        assert small == sorted(small)                 # small tiles after the others
        tail = [keys(t) for t, s in zip(run, small) if s]
        assert tail == sorted(tail, reverse=True)
    assert max(loads) - min(loads) <= 2 * big


def test_cu_seqlens_host_copy_follows_writes():
    """The host copy of cu_seqlens is reused only while the tensor is
    unchanged; inference-mode tensors (no version counter) are re-read."""
    from moba_hip.baseline_adapter import _host_cu
    cu = torch.tensor([0, 5, 9], dtype=torch.int32)
    assert _host_cu(cu) == [0, 5, 9]
    cu[1] = 4
    assert _host_cu(cu) == [0, 4, 9]
    cu[1:].add_(1)                       # a write through a view
    assert _host_cu(cu) == [0, 5, 10]
    with torch.inference_mode():
        ci = torch.tensor([0, 3], dtype=torch.int32)
        assert _host_cu(ci) == [0, 3]
        ci[1] = 2
        assert _host_cu(ci) == [0, 2]
    assert _host_cu(ci) == [0, 2]


def test_plan_cache_is_thread_safe():
    """Concurrent plan lookups over more shapes than the cache holds (so
    entries are evicted while others are read) neither raise nor mix plans."""
    import threading
    from moba_hip.ops import prefill as P
    errors = []

    def worker(seed):
        try:
            for i in range(60):
                n = 64 + 16 * ((seed * 7 + i) % 24)
                plan = P.get_plan([0, n], 16, 4, 2, 64, 3, "cpu")
                assert plan.cu == [0, n]
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(s,)) for s in range(8)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors[:3]
