#!/usr/bin/env python
"""MoBA on one MI355X: the BASELINE.json headline workloads.

Default run (N=1):
  * headline  : cfg3, 32K MHA prefill fwd+bwd through the `opt_hip` registry
                entry (T=32768, 32 heads, D=128, chunk 4096, topk 3, bf16,
                Q/K/V/dO iid N(0,1)/sqrt(128)); ms per step and MFMA%
                (algorithmic FLOPs: attended pairs x (4D fwd + 10D bwd)).
  * roofline  : the key-major dK/dV backward kernel, timed live with stream
                events around its launch inside every timed step; `traffic`
                is its HBM bytes per launch from the copy-calibrated rocprofv3
                FETCH_SIZE / WRITE_SIZE passes in profiles/dkdv_cfg3_traffic.*.
  * gqa_16k   : cfg2 (Qwen2-0.5B GQA 14/2, D=64, T=16384, chunk 2048).
  * decode    : cfg4, batch-8 paged decode (12q/2kv, D=128, bf16, ctx
                U[2048,16384], page 48, chunk 512, topk 4, shuffled page pool),
                PreparedDecode step replayed as a hipGraph; us/step and the
                logical K/V bytes the routes require per step.
  * decode_mqa: cfg5, batch-32 MQA fp16 graph decode (D=96, page 64, chunk
                1024, topk 8, 256 steps).
  * cpu_baseline: the FP64 CPU oracle (routing + fixed-route fwd + bwd) on 1 of
                the 32 heads of cfg3, scaled x32, on this host's cores.
Prints ONE JSON line on stdout; progress goes to stderr.
"""
import argparse
import json
import os
import random
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (ROOT, ROOT / "moba-merge-cuda_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
HBM_PEAK_GBS = 8000.0      # MI355X HBM3E
METRIC = BASELINE_METRIC = ("prefill fwd+bwd ms & MFMA% (32K); paged decode µs/step & "
                            "HBM GB/s (bs 8)")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ------------------------------------------------------------------ prefill

def prefill_inputs(T, hq, hkv, d, scale, seed, dtype):
    import torch
    g = torch.Generator(device="cuda").manual_seed(seed)

    def rnd(h):
        return (torch.randn((T, h, d), generator=g, device="cuda") * scale).to(dtype)
    q, k, v = rnd(hq), rnd(hkv), rnd(hkv)
    do = rnd(hq)
    return q, k, v, do


def attended_pairs(plan, rt, chunk):
    self_pairs = 0
    for a, b in zip(plan.cu_chunk[:-1], plan.cu_chunk[1:]):
        n = b - a
        self_pairs += n * (n + 1) // 2
    remote = int(rt.counts.sum().item()) * chunk
    return self_pairs * plan.hq + remote


def bench_prefill(T, hq, hkv, d, chunk, topk, steps, warmup, scale, seed, time_dkdv=False):
    import torch
    import moba_hip
    from moba_hip.ops import prefill as P
    dtype = torch.bfloat16
    q, k, v, do = prefill_inputs(T, hq, hkv, d, scale, seed, dtype)
    q.requires_grad_(True)
    k.requires_grad_(True)
    v.requires_grad_(True)
    cu = torch.tensor([0, T], device="cuda", dtype=torch.int32)
    cfg = {"chunk_size": chunk, "topk": topk}

    def step():
        out = moba_hip.run_impl("opt_hip", q, k, v, cu, T, cfg)
        return torch.autograd.grad(out, (q, k, v), grad_outputs=do)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ev = []
    if time_dkdv:
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(steps)]
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record()
    for i in range(steps):
        if time_dkdv:
            P.DKDV_EVENTS = ev[i]
        step()
    e1.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    P.DKDV_EVENTS = None
    gpu_ms = e0.elapsed_time(e1) / steps
    plan = P.get_plan([0, T], chunk, hq, hkv, d, topk, q.device)
    rt = P.route(plan, q.detach(), k.detach(), 0)
    pairs = attended_pairs(plan, rt, chunk)
    flops = pairs * 14 * d
    res = {"ms_per_step": wall, "gpu_ms_per_step": gpu_ms, "attended_pairs": pairs,
           "algorithmic_tflop": flops / 1e12, "tflops": flops / wall / 1e9,
           "mfma_frac": flops / wall / 1e9 / BF16_PEAK_TFLOPS}
    if time_dkdv:
        dk_ms = sum(a.elapsed_time(b) for a, b in ev) / steps
        res["dkdv_ms"] = dk_ms
        res["dkdv_tflop"] = pairs * 8 * d / 1e12
    del q, k, v, do
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
            toks = sum(min(chunk, pos + 1 - c * chunk) for c in chunks)
            total += toks * d * elem * 2
        total += hkv * (pos // chunk) * d * elem            # means read by the router
    nq = len(positions)
    total += nq * hq * d * elem * 2 + nq * hq * 4            # q in, out + lse out
    total += nq * hkv * d * elem * 2                          # appended K/V
    return total


def build_cache(batch, lengths, hq, hkv, d, page, chunk, dtype, extra, seed):
    import torch
    import moba_hip
    cache = moba_hip.PagedKVCache(batch, max(lengths) + extra, hkv, d, page_size=page,
                                  chunk_size=chunk, dtype=dtype)
    pages = list(cache._layout.free_pages)
    random.Random(seed).shuffle(pages)   # fragmented physical pool
    cache._layout.free_pages = tuple(pages)
    g = torch.Generator(device="cuda").manual_seed(seed)
    for sid, length in enumerate(lengths):
        for lo in range(0, length, 2048):
            n = min(2048, length - lo)
            k = torch.randn((n, hkv, d), generator=g, device="cuda", dtype=dtype)
            v = torch.randn((n, hkv, d), generator=g, device="cuda", dtype=dtype)
            cache.append(k, v, sequence_ids=[sid], cu_seqlens=[0, n])
    return cache


def bench_decode(batch, hq, hkv, d, page, chunk, topk, lo, hi, steps, warmup, dtype_name, seed):
    import numpy as np
    import torch
    dtype = torch.bfloat16 if dtype_name == "bf16" else torch.float16
    elem = 2
    rng = random.Random(seed)
    lengths = [rng.randint(lo, hi) for _ in range(batch)]
    extra = 2 * (warmup + steps) + 4
    g = torch.Generator(device="cuda").manual_seed(seed + 1)
    q = torch.randn((batch, hq, d), generator=g, device="cuda", dtype=dtype)
    kn = torch.randn((batch, hkv, d), generator=g, device="cuda", dtype=dtype)
    vn = torch.randn((batch, hkv, d), generator=g, device="cuda", dtype=dtype)

    # pass 1 (untimed): record the routes of every step to count the bytes
    cache = build_cache(batch, lengths, hq, hkv, d, page, chunk, dtype, extra, seed)
    byte_counts = []
    with cache.prepare_decode(list(range(batch)), hq, topk=topk, check_finite=False) as p:
        for i in range(warmup + steps):
            r = p.step(q, kn, vn)
            if i >= warmup:
                byte_counts.append(decode_bytes(r.selected_blocks.cpu().numpy(), r.positions,
                                                hq, hkv, d, chunk, elem))
    del cache
    torch.cuda.empty_cache()

    # pass 2 (timed): identical state; eager steps, then graph-replayed steps
    cache = build_cache(batch, lengths, hq, hkv, d, page, chunk, dtype, extra, seed)

    def timed(fn, n):
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e6 / n, e0.elapsed_time(e1) * 1e3 / n

    with cache.prepare_decode(list(range(batch)), hq, topk=topk, check_finite=False) as p:
        # the prepared workspaces are the inputs (no staging copies)
        p.q.copy_(q)
        p.k.copy_(kn)
        p.v.copy_(vn)
        for _ in range(warmup):
            p.step(p.q, p.k, p.v)
        eager_wall, eager_gpu = timed(lambda: p.step(p.q, p.k, p.v), steps)
        p.capture("step")
        for _ in range(warmup):
            p.step(p.q, p.k, p.v, use_graph=True)
        graph_wall, graph_gpu = timed(lambda: p.step(p.q, p.k, p.v, use_graph=True), steps)
        # device time of the decode work alone: back-to-back attend launches
        # (they read the cache and mutate nothing)
        _, kernel_us = timed(lambda: p.attend(p.q), 50)
        fused = p.fused
    del cache
    torch.cuda.empty_cache()
    mean_bytes = float(np.mean(byte_counts))
    wall_us = min(eager_wall, graph_wall)
    return {"us_per_step": wall_us, "eager_step_us": eager_wall, "graph_step_us": graph_wall,
            "eager_gpu_us": eager_gpu, "graph_gpu_us": graph_gpu, "kernel_us": kernel_us,
            "one_launch": fused,
            "bytes_per_step": mean_bytes, "logical_gbs": mean_bytes / (wall_us * 1e-6) / 1e9,
            "hbm_frac_logical": mean_bytes / (wall_us * 1e-6) / 1e9 / HBM_PEAK_GBS,
            "kernel_gbs": mean_bytes / (kernel_us * 1e-6) / 1e9,
            "kernel_hbm_frac": mean_bytes / (kernel_us * 1e-6) / 1e9 / HBM_PEAK_GBS,
            "batch": batch, "contexts": lengths, "steps": steps}


# -------------------------------------------------------------- CPU baseline

def cpu_baseline(seed):
    """FP64 oracle (routing + forward + backward) on head 0 of cfg3, x32."""
    import numpy as np
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


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--only", choices=["prefill", "decode"], default=None)
    ap.add_argument("--calib-copy", action="store_true",
                    help="first run one 1 GiB device-to-device copy (a known-size kernel that "
                         "calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one MI355X: multi-GPU runs are not part of this build "
              "(the path shards by KV-head group / request with no collective; see DESIGN.md)",
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
    res3 = None
    if args.only in (None, "prefill"):
        log("prefill cfg3 (32K MHA fwd+bwd) ...")
        res3 = bench_prefill(32768, 32, 32, 128, 4096, 3, args.steps, args.warmup,
                             128 ** -0.5, args.seed, time_dkdv=True)
        log(json.dumps(res3))
        log("prefill cfg2 (16K GQA fwd+bwd) ...")
        res2 = bench_prefill(16384, 14, 2, 64, 2048, 3, args.steps, args.warmup, 1.0,
                             args.seed + 1)
        log(json.dumps(res2))
    dec4 = dec5 = None
    if not args.no_decode and args.only in (None, "decode"):
        log("decode cfg4 (batch 8 paged, graph) ...")
        dec4 = bench_decode(8, 12, 2, 128, 48, 512, 4, 2048, 16384, 128, 8, "bf16", args.seed)
        log(json.dumps({k: v for k, v in dec4.items() if k != "contexts"}))
        log("decode cfg5 (batch 32 MQA fp16, graph) ...")
        dec5 = bench_decode(32, 16, 1, 96, 64, 1024, 8, 1024, 32768, 256, 8, "fp16",
                            args.seed + 2)
        log(json.dumps({k: v for k, v in dec5.items() if k != "contexts"}))

    if res3 is not None:
        ach = res3["dkdv_tflop"] / (res3["dkdv_ms"] * 1e-3)
        traffic = None
        tfile = ROOT / "profiles" / "dkdv_cfg3_traffic.json"
        if tfile.exists():  # rocprofv3 FETCH_SIZE + WRITE_SIZE passes, copy-calibrated
            traffic = json.loads(tfile.read_text())["traffic_bytes"]
        out.update({
            "value": round(res3["ms_per_step"], 3), "unit": "ms per 32K MHA prefill fwd+bwd step",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(res3["ms_per_step"], 3), "higher_is_better": False,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded iid N(0,1) Q/K/V/dO, scaled 1/sqrt(128))",
            "config": {"workload": "cfg3: MoBA MHA prefill fwd+bwd, T=32768, heads=32, D=128, "
                                   "chunk=4096, topk=3, causal, bf16",
                       "entry": "moba_hip.run_impl('opt_hip')", "seq_len": 32768},
            "mfma_frac": round(res3["mfma_frac"], 4),
            "tflops": round(res3["tflops"], 1),
            "roofline": {"bound": "mfma", "kernel": "dkdv2_kernel<bf16,128>",
                         "achieved": round(ach, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(ach / BF16_PEAK_TFLOPS, 4), "traffic": traffic,
                         "traffic_unit": "bytes per launch (profiles/dkdv_cfg3_traffic.md)",
                         "avg_launch_ms": round(res3["dkdv_ms"], 3),
                         "algorithmic_tflop_per_launch": round(res3["dkdv_tflop"], 3)},
            "prefill_32k": res3, "gqa_16k": res2,
        })
    else:
        out.update({"value": None, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup})
    if dec4 is not None:
        out["decode"] = dec4
        out["decode_mqa"] = dec5
    if not args.no_cpu and res3 is not None:
        log("cpu baseline (FP64 oracle, 1 of 32 heads) ...")
        out["cpu_baseline"] = cpu_baseline(args.seed)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
