#!/usr/bin/env python
"""MoBA on one MI355X: the BASELINE.json headline workloads.

Default run (N=1):
  * headline   : cfg3, 32K MHA prefill fwd+bwd through the `opt_hip` registry
                 entry (T=32768, 32 heads, D=128, chunk 4096, topk 3, bf16,
                 Q/K/V/dO iid N(0,1)/sqrt(128)); ms per step and MFMA%
                 (algorithmic FLOPs: attended pairs x (4D fwd + 10D bwd)).
  * gqa_16k    : cfg2 (Qwen2-0.5B GQA 14/2, D=64, T=16384, chunk 2048).
                 cfg3 and cfg2 run in rounds of alternating order (AB / BA);
                 each step is timed with stream events and a config's figure
                 is the median of its per-round medians, the statistic of
                 benchmarks/benchmark_attention.py:245-256; min / max of the
                 round medians are reported beside it.
  * roofline   : the key-major dK/dV backward kernel of cfg3, timed live with
                 stream events around its launch in every timed step;
                 `traffic` is its HBM bytes per launch from the copy-
                 calibrated rocprofv3 FETCH_SIZE / WRITE_SIZE passes in
                 profiles/dkdv_cfg3_traffic.*.
  * decode     : cfg4, batch-8 paged decode (12q/2kv, D=128, bf16, ctx
                 U[2048,16384], page 48, chunk 512, topk 4, shuffled page
                 pools), PreparedDecode steps replayed from their hipGraph
                 (the headline decode figure) and eager beside it.  Steps
                 rotate over several independent caches whose pools together
                 exceed the 256 MB Infinity Cache, so K/V come from HBM.
                 Bytes per step are the unique K/V bytes the routes need.
  * decode_mqa : cfg5, batch-32 MQA fp16 graph decode (D=96, page 64, chunk
                 1024, topk 8, 256 steps), measured the same way.
  * qwen2_decode: a randomly initialised Qwen2-1.5B-shaped model (cfg4's
                 attention shape) decoding after an 8K MoBA prefill, per-token
                 time eager and as one whole-model hipGraph.
  * reference_c12_prefill / reference_decode_matrix: the reference's own
                 published shapes -- C12 prefill fwd+bwd (T 32768, 8 heads,
                 D 128, chunk 512, top-4) and the P01 / P18 rows of its
                 decode matrix as prepared graph / eager steps -- with its A40
                 figures beside them as context only.
  * cpu_baseline: the FP64 CPU oracle (routing + fixed-route fwd + bwd) on 1 of
                 the 32 heads of cfg3, scaled x32, on this host's cores; and
                 cfg1 measured in full (routing + FP64 forward, 8 heads).
Prints ONE JSON line on stdout; progress goes to stderr.
"""
import argparse
import json
import os
import random
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (ROOT, ROOT / "moba-merge-cuda_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
HBM_PEAK_GBS = 8000.0      # MI355X HBM3E
MALL_BYTES = 256 << 20     # MI355X Infinity Cache
METRIC = ("prefill fwd+bwd ms & MFMA% (32K); paged decode µs/step & HBM GB/s (bs 8)")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _spread(xs):
    return {"median": statistics.median(xs), "min": min(xs), "max": max(xs)}


# ------------------------------------------------------------------ prefill

class PrefillCase:
    """One prefill configuration with its inputs resident in HBM."""

    def __init__(self, name, T, hq, hkv, d, chunk, topk, scale, seed):
        import torch
        import moba_hip  # noqa: F401
        self.name, self.T, self.d = name, T, d
        g = torch.Generator(device="cuda").manual_seed(seed)

        def rnd(h):
            return (torch.randn((T, h, d), generator=g, device="cuda") * scale).to(torch.bfloat16)
        self.q, self.k, self.v, self.do = rnd(hq), rnd(hkv), rnd(hkv), rnd(hq)
        for t in (self.q, self.k, self.v):
            t.requires_grad_(True)
        self.cu = torch.tensor([0, T], device="cuda", dtype=torch.int32)
        self.cfg = {"chunk_size": chunk, "topk": topk}
        self.shape = (hq, hkv, chunk, topk)

    def step(self):
        import torch
        import moba_hip
        out = moba_hip.run_impl("opt_hip", self.q, self.k, self.v, self.cu, self.T, self.cfg)
        return torch.autograd.grad(out, (self.q, self.k, self.v), grad_outputs=self.do)

    def flops(self):
        """Algorithmic FLOPs of one fwd+bwd step: attended (q head, key)
        pairs x 14 D; and the 8 D per pair of the key-major dK/dV kernel."""
        from moba_hip.ops import prefill as P
        hq, hkv, chunk, topk = self.shape
        plan = P.get_plan([0, self.T], chunk, hq, hkv, self.d, topk, self.q.device)
        rt = P.route(plan, self.q.detach(), self.k.detach(), 0)
        self_pairs = sum((b - a) * (b - a + 1) // 2
                         for a, b in zip(plan.cu_chunk[:-1], plan.cu_chunk[1:]))
        pairs = self_pairs * hq + int(rt.counts.sum().item()) * chunk
        return pairs, pairs * 14 * self.d, pairs * 8 * self.d


def time_steps(case, n, dkdv=None):
    """Runs n steps with a stream event before each and after the last;
    returns the per-step GPU times (ms).  dkdv collects the dK/dV launch
    times (ms) when given."""
    import torch
    from moba_hip.ops import prefill as P
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    kev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(n)] if dkdv is not None else None
    ev[0].record()
    for i in range(n):
        if kev is not None:
            P.DKDV_EVENTS = kev[i]
        case.step()
        ev[i + 1].record()
    P.DKDV_EVENTS = None
    torch.cuda.synchronize()
    if kev is not None:
        dkdv.extend(a.elapsed_time(b) for a, b in kev)
    return [ev[i].elapsed_time(ev[i + 1]) for i in range(n)]


def bench_prefill(steps, warmup, seed):
    """cfg3 (headline) and cfg2 in rounds of alternating order; exactly
    `steps` timed steps of each, bracketed by synchronisations."""
    import torch
    cases = [PrefillCase("cfg3", 32768, 32, 32, 128, 4096, 3, 128 ** -0.5, seed),
             PrefillCase("cfg2", 16384, 14, 2, 64, 2048, 3, 1.0, seed + 1)]
    for c in cases:
        for _ in range(warmup):
            c.step()
    # at least 4 steps per round: the first step after a synchronisation also
    # carries the host's launch latency, and the round median passes over it
    rounds = max(1, min(5, steps // 4))
    per = [steps // rounds + (1 if r < steps % rounds else 0) for r in range(rounds)]
    res = {c.name: {"round_medians": [], "steps": [], "wall": 0.0} for c in cases}
    dkdv = []
    for r in range(rounds):
        order = cases if r % 2 == 0 else cases[::-1]
        for c in order:
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            ts = time_steps(c, per[r], dkdv if c.name == "cfg3" else None)
            torch.cuda.synchronize()
            res[c.name]["wall"] += time.perf_counter() - t0
            res[c.name]["round_medians"].append(statistics.median(ts))
            res[c.name]["steps"].extend(ts)
    out = {}
    for c in cases:
        pairs, flops, kflops = c.flops()
        rm = res[c.name]["round_medians"]
        ms = statistics.median(rm)
        out[c.name] = {
            "ms_per_step": ms, "round_medians_ms": rm, "rounds": rounds,
            "spread_ms": {"min_round": min(rm), "max_round": max(rm),
                          "min_step": min(res[c.name]["steps"]),
                          "max_step": max(res[c.name]["steps"])},
            "wall_ms_per_step": res[c.name]["wall"] * 1e3 / steps,
            "attended_pairs": pairs, "algorithmic_tflop": flops / 1e12,
            "tflops": flops / ms / 1e9, "mfma_frac": flops / ms / 1e9 / BF16_PEAK_TFLOPS}
        if c.name == "cfg3":
            out[c.name]["dkdv_ms"] = statistics.median(dkdv)
            out[c.name]["dkdv_ms_spread"] = [min(dkdv), max(dkdv)]
            out[c.name]["dkdv_tflop"] = kflops / 1e12
    del cases
    torch.cuda.empty_cache()
    return out


def bench_prefill_case(case, steps, warmup, rounds=3):
    """Median of per-round medians of per-step stream-event times of one
    prefill case, with its algorithmic FLOPs and MFMA fraction."""
    import torch
    for _ in range(warmup):
        case.step()
    rm = []
    for _ in range(rounds):
        torch.cuda.synchronize()
        rm.append(statistics.median(time_steps(case, max(1, steps // rounds))))
    pairs, flops, _ = case.flops()
    ms = statistics.median(rm)
    return {"ms_per_step": ms, "round_medians_ms": rm, "attended_pairs": pairs,
            "algorithmic_tflop": flops / 1e12, "tflops": flops / ms / 1e9,
            "mfma_frac": flops / ms / 1e9 / BF16_PEAK_TFLOPS}


def bench_c12(steps, warmup, seed):
    """The reference's published C12 (configs/core12.yaml: T=32768, 8 heads,
    D=128, chunk 512, top-4, bf16, N(0,1) Q/K/V/dO; 64 chunks, 63 candidates)
    fwd+bwd through opt_hip.  The A40 figure beside it is context only."""
    import torch
    case = PrefillCase("C12", 32768, 8, 8, 128, 512, 4, 1.0, seed + 5)
    res = bench_prefill_case(case, steps, warmup)
    res["reference_a40_ms"] = 54.15
    res["reference_source"] = "docs/profiling_decision.md:7 (A40, opt baseline wall clock)"
    del case
    torch.cuda.empty_cache()
    return res


# ------------------------------------------------------------------- decode

def decode_bytes(selected, positions, hq, hkv, d, chunk, elem):
    """Unique K+V bytes one step needs: per (request, kv head) the union over
    its q heads of the selected chunks (current chunk clipped to pos+1), plus
    the means of the closed chunks, q/out/lse and the appended token."""
    G = hq // hkv
    total = 0
    for b, pos in enumerate(positions):
        for kh in range(hkv):
            chunks = set(int(c) for c in selected[b, kh * G:(kh + 1) * G].reshape(-1) if c >= 0)
            total += sum(min(chunk, pos + 1 - c * chunk) for c in chunks) * d * elem * 2
        total += hkv * (pos // chunk) * d * elem                # means read by the router
    nq = len(positions)
    total += nq * hq * d * elem * 2 + nq * hq * 4              # q in, out + lse out
    total += nq * hkv * d * elem * 2                           # appended K/V
    return total


def build_cache(batch, lengths, hkv, d, page, chunk, dtype, extra, seed):
    """A cache of `lengths` tokens per sequence with a seeded, shuffled free
    page order (a fragmented physical pool, as benchmark_prepared.py:79-81)."""
    import torch
    import moba_hip
    cache = moba_hip.PagedKVCache(batch, max(lengths) + extra, hkv, d, page_size=page,
                                  chunk_size=chunk, dtype=dtype)
    pages = list(cache._layout.free_pages)
    random.Random(seed).shuffle(pages)
    cache._layout.free_pages = tuple(pages)
    g = torch.Generator(device="cuda").manual_seed(seed)
    for sid, length in enumerate(lengths):
        for lo in range(0, length, 2048):
            n = min(2048, length - lo)
            k = torch.randn((n, hkv, d), generator=g, device="cuda", dtype=dtype)
            v = torch.randn((n, hkv, d), generator=g, device="cuda", dtype=dtype)
            cache.append(k, v, sequence_ids=[sid], cu_seqlens=[0, n])
    return cache


def bench_decode(batch, hq, hkv, d, page, chunk, topk, lo, hi, steps, warmup, dtype_name, seed,
                 rounds=4):
    import numpy as np
    import torch
    dtype = torch.bfloat16 if dtype_name == "bf16" else torch.float16
    rng = random.Random(seed)
    lengths = [rng.randint(lo, hi) for _ in range(batch)]
    g = torch.Generator(device="cuda").manual_seed(seed + 1)
    q = torch.randn((batch, hq, d), generator=g, device="cuda", dtype=dtype)
    kn = torch.randn((batch, hkv, d), generator=g, device="cuda", dtype=dtype)
    vn = torch.randn((batch, hkv, d), generator=g, device="cuda", dtype=dtype)
    extra = 2 * (warmup + steps) + 8

    # pass 1 (untimed): the routes of every step of cache 0, to count bytes
    cache = build_cache(batch, lengths, hkv, d, page, chunk, dtype, extra, seed)
    pool_bytes = cache.k_cache.numel() * cache.k_cache.element_size() * 2
    byte_counts = []
    with cache.prepare_decode(list(range(batch)), hq, topk=topk, check_finite=False) as p:
        for i in range(warmup + steps):
            r = p.step(q, kn, vn)
            if i >= warmup:
                byte_counts.append(decode_bytes(r.selected_blocks.cpu().numpy(), r.positions,
                                                hq, hkv, d, chunk, 2))
    del cache, p
    torch.cuda.empty_cache()

    # pass 2 (timed): n caches rotated per step, pools together > the MALL
    n = max(3, -(-3 * MALL_BYTES // pool_bytes))
    caches = [build_cache(batch, lengths, hkv, d, page, chunk, dtype, extra, seed + i)
              for i in range(n)]
    plans = [c.prepare_decode(list(range(batch)), hq, topk=topk, check_finite=False)
             for c in caches]
    for p in plans:  # the bound input buffers are the inputs (no staging copies)
        p.q.copy_(q)
        p.k.copy_(kn)
        p.v.copy_(vn)
        p.capture("step")
    it = [0]

    def run(m, graph):
        for _ in range(m):
            p = plans[it[0] % n]
            p.step(p.q, p.k, p.v, use_graph=graph)
            it[0] += 1

    for graph in (False, True):
        run(warmup, graph)
    per = max(1, steps // rounds)
    times = {False: [], True: []}
    walls = {False: [], True: []}
    host = {False: [], True: []}   # host time to issue the steps (before the sync)
    for r in range(rounds):
        for graph in ((True, False) if r % 2 == 0 else (False, True)):
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0 = time.perf_counter()
            e0.record()
            run(per, graph)
            e1.record()
            t1 = time.perf_counter()
            torch.cuda.synchronize()
            walls[graph].append((time.perf_counter() - t0) * 1e6 / per)
            host[graph].append((t1 - t0) * 1e6 / per)
            times[graph].append(e0.elapsed_time(e1) * 1e3 / per)
    fused = plans[0].fused
    for p in plans:
        p.close()
    del plans, caches
    torch.cuda.empty_cache()
    mean_bytes = float(np.mean(byte_counts))
    g_us, e_us = statistics.median(walls[True]), statistics.median(walls[False])
    return {"us_per_step": g_us, "graph_step_us": g_us, "eager_step_us": e_us,
            "graph_round_us": walls[True], "eager_round_us": walls[False],
            "graph_gpu_us": statistics.median(times[True]),
            "graph_host_us": statistics.median(host[True]),
            "eager_host_us": statistics.median(host[False]),
            "eager_gpu_us": statistics.median(times[False]),
            "one_launch_path": fused, "caches_rotated": n,
            "pool_bytes_per_cache": pool_bytes,
            "bytes_per_step": mean_bytes,
            "graph_gbs": mean_bytes / (g_us * 1e-6) / 1e9,
            "graph_hbm_frac": mean_bytes / (g_us * 1e-6) / 1e9 / HBM_PEAK_GBS,
            "eager_gbs": mean_bytes / (e_us * 1e-6) / 1e9,
            "eager_hbm_frac": mean_bytes / (e_us * 1e-6) / 1e9 / HBM_PEAK_GBS,
            "batch": batch, "contexts": lengths, "steps": per * rounds, "rounds": rounds}


def bench_qwen2(ctx, steps, seed):
    """Whole-model decode of a randomly initialised Qwen2-1.5B-shaped model
    (28 layers, hidden 1536, 12 q / 2 kv heads, head_dim 128 -- the shape of
    cfg4), batch 1: MoBA prefill of `ctx` prompt tokens, then `steps` decode
    tokens, eager and as one whole-model hipGraph per token."""
    import torch
    from transformers import Qwen2Config, Qwen2ForCausalLM
    from moba_hip.qwen2 import Qwen2Session
    torch.manual_seed(seed)
    cfg = Qwen2Config(vocab_size=151936, hidden_size=1536, intermediate_size=8960,
                      num_hidden_layers=28, num_attention_heads=12, num_key_value_heads=2,
                      max_position_embeddings=32768, attn_implementation="eager")
    with torch.device("cuda"):
        model = Qwen2ForCausalLM(cfg).to(torch.bfloat16).eval()
    for p in model.parameters():
        p.requires_grad_(False)
    ids = torch.randint(0, cfg.vocab_size, (1, ctx), device="cuda")
    toks = torch.randint(0, cfg.vocab_size, (steps + 4,)).tolist()
    res = {"model": "Qwen2-1.5B shape, random init, bf16", "context": ctx, "steps": steps,
           "chunk": 512, "topk": 4}
    for backend in ("eager", "model_graph"):
        with Qwen2Session(model, ctx + steps + 8, mode="moba", chunk=512, topk=4, page=48,
                          backend=backend) as s:
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            s.prefill(ids)
            torch.cuda.synchronize()
            res["prefill_ms"] = (time.perf_counter() - t0) * 1e3
            s.prepare()
            for t in toks[:4]:
                s.step(t)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for t in toks[4:]:
                s.step(t)
            torch.cuda.synchronize()
            res[f"{backend}_ms_per_token"] = (time.perf_counter() - t0) * 1e3 / steps
    del model
    torch.cuda.empty_cache()
    return res


def decode_roofline(res, name):
    """Roofline of the decode step's launches: algorithmic bytes per step over
    the step's GPU time measured live here (HIP events on the cache's stream
    around the eager steps, which are GPU-bound; the time includes the gap
    between the two launches).  HBM bytes by counter and the kernels' rocprof
    time come from the committed rocprofv3 summary, or None without it."""
    f = ROOT / "profiles" / f"decode_{name}_traffic.json"
    if not f.exists():
        return None
    t = json.loads(f.read_text())
    ach = res["bytes_per_step"] / (res["eager_gpu_us"] * 1e-6) / 1e9
    return {"bound": "hbm", "kernel": t["kernel"], "achieved": round(ach, 1),
            "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
            "traffic": t["traffic_bytes"], "live_step_gpu_us": round(res["eager_gpu_us"], 2),
            "profile_kernel_us": round(t["kernel_us"], 2), "counter_gbs": round(t["counter_gbs"], 1),
            "source": f"profiles/decode_{name}_traffic.md"}


# Published prepared-decode figures of the reference (A40, seed 701), context
# only: docs/prepared_decode_20261102.md:61 ("strict" = finite checks on,
# "trusted" = caller guarantees finite inputs, as the bound-buffer steps here).
REFERENCE_PREPARED_US = {
    "P01": {"strict_graph_step_us": 361.0, "trusted_graph_step_us": 161.0},
    "P18": {"strict_graph_step_us": 582.0},
}


def bench_reference_decode(steps, warmup, seed):
    """Prepared graph / eager steps at the reference's decode-matrix rows P01
    (B 1, 2K, D 64, 32q/8kv) and P18 (B 16, 32K, D 128, 32q/8kv): page 16,
    chunk 128, top-4, bf16, max_seq_len = length + extra as
    benchmarks/benchmark_decode.py:105-112 builds the step cache (P18's page
    table is 2049+ entries wide)."""
    out = {}
    for name, batch, length, d in (("P01", 1, 2048, 64), ("P18", 16, 32768, 128)):
        log(f"decode {name} (reference matrix row, graph + eager) ...")
        r = bench_decode(batch, 32, 8, d, 16, 128, 4, length, length, steps, warmup, "bf16",
                         seed + 7)
        r.pop("contexts", None)
        r["reference_a40"] = REFERENCE_PREPARED_US[name]
        out[name] = r
        log(json.dumps(r))
    return out


# -------------------------------------------------------------- CPU baseline

def cpu_baseline(seed):
    """FP64 oracle (routing + forward + backward) on head 0 of cfg3, x32."""
    import torch
    from oracle import oracle as O
    T, d, C, K = 32768, 128, 4096, 3
    threads = min(len(os.sched_getaffinity(0)), 16)
    O.set_threads(threads)
    g = torch.Generator().manual_seed(seed)
    q, k, v, do = ((torch.randn(T, 1, d, generator=g) * d ** -0.5).bfloat16() for _ in range(4))
    t0 = time.perf_counter()
    cu_chunk, chunk_batch, filtered = O.calc_chunks([0, T], C)
    means = O.chunk_means(O.bits16(k), 0, cu_chunk, filtered, C, 0)
    sel, _ = O.route_prefill(O.bits16(q), 0, means, cu_chunk, chunk_batch, K - 1)
    qd, kd, vd, gd = (x.double().numpy() for x in (q, k, v, do))
    _, lse = O.attention_fwd(qd, kd, vd, cu_chunk, sel)
    O.attention_bwd(qd, kd, vd, gd, cu_chunk, sel, lse)
    sec = time.perf_counter() - t0
    return {"value": sec * 32 * 1e3, "unit": "ms per cfg3 fwd+bwd step (1 of 32 heads timed, x32)",
            "cores": threads, "kind": "port",
            "sample": f"cfg3 head 0 (T=32768, D=128, chunk 4096, topk 3): canonical routing + "
                      f"FP64 fixed-route forward + backward, {sec:.1f} s on {threads} threads"}


def cpu_baseline_cfg1(seed):
    """cfg1 measured in full on the host: canonical routing + FP64
    fixed-route forward of all 8 heads (T=4096, D=64, chunk 512, topk 3,
    Q/K/V iid N(0,1) fp32 with bf16 copies), with the same forward on the
    GPU (opt_hip, bf16) timed beside it."""
    import torch
    import moba_hip
    from oracle import oracle as O
    T, H, d, C, K = 4096, 8, 64, 512, 3
    threads = min(len(os.sched_getaffinity(0)), 16)
    O.set_threads(threads)
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(T, H, d, generator=g).bfloat16() for _ in range(3))
    t0 = time.perf_counter()
    cu_chunk, chunk_batch, filtered = O.calc_chunks([0, T], C)
    means = O.chunk_means(O.bits16(k), 0, cu_chunk, filtered, C, 0)
    sel, _ = O.route_prefill(O.bits16(q), 0, means, cu_chunk, chunk_batch, K - 1)
    O.attention_fwd(*(x.double().numpy() for x in (q, k, v)), cu_chunk, sel)
    cpu_ms = (time.perf_counter() - t0) * 1e3
    qg, kg, vg = (x.cuda() for x in (q, k, v))
    cu = torch.tensor([0, T], dtype=torch.int32, device="cuda")
    cfg = {"chunk_size": C, "topk": K}
    with torch.no_grad():
        for _ in range(3):
            moba_hip.run_impl("opt_hip", qg, kg, vg, cu, T, cfg)
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(11)]
        ev[0].record()
        for i in range(10):
            moba_hip.run_impl("opt_hip", qg, kg, vg, cu, T, cfg)
            ev[i + 1].record()
        torch.cuda.synchronize()
    gpu_ms = statistics.median(ev[i].elapsed_time(ev[i + 1]) for i in range(10))
    return {"value": cpu_ms, "unit": "ms per cfg1 forward (all 8 heads, measured)",
            "cores": threads, "kind": "port",
            "sample": "cfg1 in full: canonical routing + FP64 fixed-route forward, T=4096, 8 heads, "
                      "D=64, chunk 512, topk 3",
            "gpu_forward_ms": gpu_ms}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--only", choices=["prefill", "decode", "cfg4", "cfg5", "qwen2", "reference"],
                    default=None)
    ap.add_argument("--calib-copy", action="store_true",
                    help="first run one 1 GiB device-to-device copy (a known-size kernel that "
                         "calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one MI355X: multi-GPU runs are not part of this build "
              "(the path would shard by KV-head group or request, with no collective)",
              file=sys.stderr)
        sys.exit(2)
    import torch
    torch.cuda.set_device(0)

    if args.calib_copy:
        src = torch.ones(1 << 29, dtype=torch.int16, device="cuda")  # 1 GiB
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        torch.cuda.empty_cache()
    out = {"metric": METRIC}
    pre = None
    if args.only in (None, "prefill"):
        log("prefill cfg3 + cfg2 (rounds of alternating order) ...")
        pre = bench_prefill(args.steps, args.warmup, args.seed)
        log(json.dumps(pre))
    dec4 = dec5 = None
    if not args.no_decode and args.only in (None, "decode", "cfg4"):
        log("decode cfg4 (batch 8 paged, graph + eager) ...")
        dec4 = bench_decode(8, 12, 2, 128, 48, 512, 4, 2048, 16384, 128, 8, "bf16", args.seed)
        log(json.dumps({k: v for k, v in dec4.items() if k != "contexts"}))
    if not args.no_decode and args.only in (None, "decode", "cfg5"):
        log("decode cfg5 (batch 32 MQA fp16, graph + eager) ...")
        dec5 = bench_decode(32, 16, 1, 96, 64, 1024, 8, 1024, 32768, 256, 8, "fp16",
                            args.seed + 2)
        log(json.dumps({k: v for k, v in dec5.items() if k != "contexts"}))

    c12 = ref_dec = None
    if args.only in (None, "reference"):
        log("reference C12 prefill fwd+bwd (T 32768, 8 heads, D 128, chunk 512, top-4) ...")
        c12 = bench_c12(args.steps, args.warmup, args.seed)
        log(json.dumps(c12))
        if not args.no_decode:
            ref_dec = bench_reference_decode(32, 4, args.seed)

    qw = None
    if not args.no_decode and args.only in (None, "qwen2"):
        log("qwen2-1.5B-shaped whole-model decode (eager and model graph) ...")
        qw = bench_qwen2(8192, 32, args.seed)
        log(json.dumps(qw))

    if pre is not None:
        r3 = pre["cfg3"]
        ach = r3["dkdv_tflop"] / (r3["dkdv_ms"] * 1e-3)
        traffic = None
        tfile = ROOT / "profiles" / "dkdv_cfg3_traffic.json"
        if tfile.exists():  # rocprofv3 FETCH_SIZE + WRITE_SIZE passes, copy-calibrated
            traffic = json.loads(tfile.read_text())["traffic_bytes"]
        out.update({
            "value": round(r3["ms_per_step"], 3), "unit": "ms per 32K MHA prefill fwd+bwd step",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(r3["wall_ms_per_step"], 3), "higher_is_better": False,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded iid N(0,1) Q/K/V/dO, scaled 1/sqrt(128))",
            "config": {"workload": "cfg3: MoBA MHA prefill fwd+bwd, T=32768, heads=32, D=128, "
                                   "chunk=4096, topk=3, causal, bf16",
                       "entry": "moba_hip.run_impl('opt_hip')", "seq_len": 32768},
            "statistic": "value: median of per-round medians of per-step stream-event times "
                         "(rounds alternate cfg3/cfg2 order); ms_per_step: wall clock of the "
                         "timed steps / steps",
            "mfma_frac": round(r3["mfma_frac"], 4),
            "tflops": round(r3["tflops"], 1),
            "roofline": {"bound": "mfma", "kernel": "dkdv2_kernel<bf16,128>",
                         "achieved": round(ach, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(ach / BF16_PEAK_TFLOPS, 4), "traffic": traffic,
                         "traffic_unit": "bytes per launch (profiles/dkdv_cfg3_traffic.md)",
                         "avg_launch_ms": round(r3["dkdv_ms"], 3),
                         "algorithmic_tflop_per_launch": round(r3["dkdv_tflop"], 3)},
            "prefill_32k": r3, "gqa_16k": pre["cfg2"],
        })
    else:
        out.update({"value": None, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup})
    if dec4 is not None:
        dec4["roofline"] = decode_roofline(dec4, "cfg4")
        out["decode"] = dec4
    if dec5 is not None:
        dec5["roofline"] = decode_roofline(dec5, "cfg5")
        out["decode_mqa"] = dec5
    if qw is not None:
        out["qwen2_decode"] = qw
    if c12 is not None:
        out["reference_c12_prefill"] = c12
    if ref_dec is not None:
        out["reference_decode_matrix"] = ref_dec
    if not args.no_cpu and pre is not None:
        log("cpu baseline (FP64 oracle, 1 of 32 heads) ...")
        out["cpu_baseline"] = cpu_baseline(args.seed)
        log("cpu baseline cfg1 (FP64 oracle forward, all heads, measured) ...")
        out["cpu_baseline"]["cfg1_measured"] = cpu_baseline_cfg1(args.seed)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
