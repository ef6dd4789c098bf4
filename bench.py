#!/usr/bin/env python
"""bench.py -- CSA decode ms/token at 32K context on one MI355X, with the HBM
roofline of the dominant kernel, the CPU oracle baseline, and DSV4 ms/query.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--sweep] [--no-dsv4]

Workload (the decode-step benchmark at its headline point): one decode step = select the
top-8 of 512 chunks from cached fp32 chunk summaries (score + top-k kernels),
then split-KV sparse attention over the 512 selected tokens of each head plus
the partial merge.  B=1, H=8, D=128, S=32768, chunk 64, bf16 N(0,1) inputs from
the CPU generator (seed 0).  Inputs are resident in HBM before timing.

Caches lie: a step touches ~4 MiB, which L2 (4 MiB per XCD) or the 256 MiB
Infinity Cache would hold, so the timed loop rotates through --copies distinct
copies of (K, V, summaries) -- by default 128, i.e. 512 MiB of touched bytes per
rotation and 16 GiB resident.  The K timed steps are HIP-graph replays (one graph
node per kernel) bracketed by synchronisations; eager timing is reported too.

The roofline entry uses per-dispatch device durations measured live with HIP
events (hipExtLaunchKernel start/stop, via csahca_profile_*) over K eager steps.

Prints ONE JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBPS = 8000.0
METRIC = "CSA decode ms/token @32K ctx (1 GPU) + achieved HBM GB/s vs peak; DSV4 ms/query"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2048)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--copies", type=int, default=128)
    ap.add_argument("--tile", type=int, default=0, help="CSA split size for --route two-pass (0 = library choice)")
    ap.add_argument("--route", choices=["fused", "two-pass"], default="fused",
                    help="fused: one launch per step; two-pass: score, top-k, attend and merge kernels")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-dsv4", action="store_true")
    ap.add_argument("--no-hca", action="store_true")
    ap.add_argument("--no-block", action="store_true")
    ap.add_argument("--no-large-batch", action="store_true")
    ap.add_argument("--sweep", action="store_true", help="also run the batch x context x top-k sweep: B {1,8,32} x S {8K,32K,128K} x k {8,32} "
                         "(rows on stderr; --sweep-out FILE also writes them as JSON)")
    ap.add_argument("--dsv4-case", default=None, metavar="cR_nqN_hH",
                    help="run only this DSV4 case (e.g. c4_nq32_h64), --steps eager calls over 16 rotated caches, "
                         "print its timing and exit (a short program to profile)")
    ap.add_argument("--sweep-out", type=Path, default=None)
    ap.add_argument("--no-graph", action="store_true",
                    help="time eager launches only (for profiler counter passes, which serialise dispatches)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run 8 plain device copies of MIB MiB (the known-size kernel that scales the "
                         "FETCH_SIZE / WRITE_SIZE counters) and exit")
    return ap.parse_args()


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------

def graph_of(fn_list):
    """Capture the callables in order into one HIP graph (after a side-stream warm-up)."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for fn in fn_list[:2]:
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for fn in fn_list:
            fn()
    torch.cuda.synchronize()
    return g


def time_graph_steps(graph, rem_graph, per_graph, steps):
    """Replay so that exactly `steps` steps run; returns elapsed ms (device events)."""
    import torch

    full, rem = divmod(steps, per_graph)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(full):
        graph.replay()
    if rem:
        rem_graph[rem].replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end)


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


# ---------------------------------------------------------------------------
# CSA headline
# ---------------------------------------------------------------------------

def csa_bench(args, B=1, H=8, S=32768, D=128, chunk=64, top_k=8, copies=None, seed=0, planted=None,
              profile=True, eager=True, attend_only=False):
    import torch

    from csahca_amd import native
    from csahca_amd.synthetic import make_synthetic_case, plant_chunks, scattered_chunks

    dev = torch.device("cuda", 0)
    if B * S <= 8 * 32768:
        case = make_synthetic_case(batch=B, heads=H, seq_len=S, head_dim=D, chunk_size=chunk, top_k=top_k,
                                   seed=seed)
        kc = case.k_cache
        if planted == "scattered":
            kc = plant_chunks(case.q, kc, scattered_chunks(B, H, S // chunk, top_k), chunk, alpha=1.0)
        q = case.q.to(dev)
        k0, v0 = kc.to(dev), case.v_cache.to(dev)
        del case, kc
    else:  # large sweep points: draw on the device (timing only, no CPU check)
        g = torch.Generator(device=dev).manual_seed(seed)
        q = torch.randn(B, H, D, dtype=torch.bfloat16, device=dev, generator=g)
        k0 = torch.empty(B, H, S, D, dtype=torch.bfloat16, device=dev).normal_(generator=g)
        v0 = torch.empty(B, H, S, D, dtype=torch.bfloat16, device=dev).normal_(generator=g)
    summ0 = native.csa_chunk_summary(k0, chunk)
    C = S // chunk
    sel_bytes = B * H * top_k * chunk * D * 2 * 2
    summ_bytes = B * H * C * D * 4
    small = B * H * D * 2 * 2 + B * H * top_k * 4  # q + out + indices
    step_bytes = sel_bytes + summ_bytes + small
    if copies is None:
        budget = 48 * 2 ** 30
        per_copy = 2 * k0.numel() * k0.element_size() + summ0.numel() * 4
        want = max(1, math.ceil(1.0 * 2 ** 30 / max(step_bytes, 1)))
        copies = max(1, min(args.copies, want, budget // max(per_copy, 1)))
    ks, vs, ss = [k0], [v0], [summ0]
    for _ in range(copies - 1):
        ks.append(k0.clone())
        vs.append(v0.clone())
        ss.append(summ0.clone())
    tile = (args.tile or native.csa_auto_tile_size(B, H, min(top_k, C), chunk)) if args.route == "two-pass" else 0

    def step(i):
        j = i % copies
        return native.csa_decode_step(q, ks[j], vs[j], ss[j], chunk, top_k, tile)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    graph, rem_graph = None, None
    res = dict(B=B, H=H, S=S, D=D, chunk=chunk, top_k=top_k, tile=tile, copies=copies,
               step_bytes=step_bytes, sel_bytes=sel_bytes, summ_bytes=summ_bytes)
    if not args.no_graph:
        per_graph = copies
        graph = graph_of([lambda i=i: step(i) for i in range(per_graph)])
        rem = args.steps % per_graph
        rem_graph = {rem: graph_of([lambda i=i: step(i) for i in range(rem)])} if rem else {}
        res["ms_per_step_graph"] = time_graph_steps(graph, rem_graph, per_graph, args.steps) / args.steps
    if eager or args.no_graph:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(args.steps):
            step(i)
        torch.cuda.synchronize()
        res["ms_per_step_eager"] = (time.perf_counter() - t0) * 1e3 / args.steps
    if profile:
        with native.profile_launches() as prof:
            for i in range(args.steps):
                step(i)
        res["kernels"] = prof.results
    if attend_only and not args.no_graph:
        # The reference's headline mode: attention over a precomputed selection
        # (cuda-csa-tiled, docs/optimization_report.md:34), same rotated copies.
        idxs = [native.csa_select_topk(q, ss[j], top_k) for j in range(copies)]
        atile = native.csa_auto_tile_size(B, H, min(top_k, C), chunk)

        def attend(i):
            j = i % copies
            return native.csa_decode_forward_tiled(q, ks[j], vs[j], idxs[j], chunk, atile)

        for i in range(args.warmup):
            attend(i)
        ga = graph_of([lambda i=i: attend(i) for i in range(copies)])
        res["attend_only_ms"] = time_graph_steps(ga, {}, copies, (args.steps // copies or 1) * copies) / \
            ((args.steps // copies or 1) * copies)
        res["attend_only_tile"] = atile
        del ga, idxs
    del graph, rem_graph, ks, vs, ss, k0, v0, summ0
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return res


def kernel_bytes(name, r):
    """Algorithmic HBM bytes per launch of each CSA kernel for workload r."""
    B, H, D, C, k, chunk = r["B"], r["H"], r["D"], r["S"] // r["chunk"], r["top_k"], r["chunk"]
    if name.startswith("csa_attend"):
        return r["sel_bytes"] + B * H * D * 2 + B * H * k * 4          # selected K,V + q + chunk ids
    if name.startswith("csa_score"):
        return r["summ_bytes"] + B * H * D * 2                            # summaries + q
    if name == "csa_topk_kernel":
        return B * H * C * 4 + B * H * k * 4                              # scores in, ids out
    if name == "csa_merge_kernel":
        return B * H * D * 2                                              # output row
    if name == "csa_step_kernel":
        # summaries + selected K,V + q + out + chunk ids (the whole decode step)
        return r["summ_bytes"] + r["sel_bytes"] + B * H * D * 2 * 2 + B * H * k * 4
    return 0


def cpu_baseline(seconds: float):
    """Time the oracle's decode step (selection from cached summaries + torch-csa
    attention, bf16-rounded probabilities) on the host on a bounded sample, with
    up to 8 threads (the value) and with 1; and the attention alone over a
    precomputed selection (the reference's attend-only torch-csa mode)."""
    import oracle
    from csahca_amd.synthetic import make_synthetic_case

    case = make_synthetic_case(batch=1, heads=8, seq_len=32768, head_dim=128, chunk_size=64, top_k=8, seed=0)
    summ = oracle.chunk_mean(case.k_cache, 64)
    nthreads = max(1, min(oracle.ncores(), 8))  # the attention parallelises over the 8 heads
    t = oracle.DecodeStepTimer(case.q, case.k_cache, case.v_cache, summ, 64, 8)
    t.step(nthreads)

    def sample(fn, secs):
        n = 0
        t0 = time.perf_counter()
        while True:
            fn()
            n += 1
            el = time.perf_counter() - t0
            if el >= secs and n >= 3:
                return el * 1e3 / n, n, el

    ms, n, el = sample(lambda: t.step(nthreads), seconds)
    side = max(1.0, seconds / 4)
    ms1, n1, _ = sample(lambda: t.step(1), side)
    ms_att, n_att, _ = sample(lambda: t.attend(nthreads), side)
    return {"value": round(ms, 5), "unit": "ms/token", "cores": nthreads, "kind": "port",
            "sample": f"{n} decode steps (B1 H8 S32768 D128 chunk64 k8; top-8 selection from cached fp32 "
                      f"summaries + attention over 512 tokens/head) of the C oracle, {el:.1f} s wall, "
                      f"{nthreads} OpenMP threads on '{cpu_model()}' ({oracle.ncores()} cores visible)",
            "one_thread_ms_per_token": round(ms1, 5),
            "attend_only_ms_per_token": round(ms_att, 5),
            "side_samples": f"{n1} steps on 1 thread; {n_att} attend-only calls (precomputed selection) on "
                            f"{nthreads} threads; ~{side:.1f} s each"}


# ---------------------------------------------------------------------------
# DSV4
# ---------------------------------------------------------------------------

def dsv4_bench(steps=200, copies=64):
    import torch

    from csahca_amd import native
    from csahca_amd.synthetic import make_dsv4_window_case

    dev = torch.device("cuda", 0)
    scale = 1.0 / math.sqrt(512)
    out = {}
    for ratio in (0, 4, 128):
        c = make_dsv4_window_case(compress_ratio=ratio, num_queries=32, heads=64, seed=ratio, device=dev)
        caches = [c.cache] + [c.cache.clone() for _ in range(copies - 1)]
        ecaches = ([c.extra_cache] + [c.extra_cache.clone() for _ in range(copies - 1)]) if ratio else None
        for nq in (1, 32):
            for H in (8, 64):
                q = c.q[:nq, :H].contiguous()
                idx = c.token_indices[:nq].contiguous()
                lens = c.topk_lengths[:nq].contiguous()
                sink = c.attn_sink[:H].contiguous()
                if ratio:
                    eidx = c.extra_token_indices[:nq].contiguous()
                    elens = c.extra_topk_lengths[:nq].contiguous()

                def call(j):
                    if ratio:
                        return native.dsv4_decode_forward_tiled(q, caches[j], idx, lens, ecaches[j], eidx, elens,
                                                                sink, c.page_size, c.extra_page_size, 0, scale)
                    return native.dsv4_decode_forward_tiled(q, caches[j], idx, lens, None, None, None, sink,
                                                            c.page_size, 1, 0, scale)

                for j in range(3):
                    call(j)
                g = graph_of([lambda j=j: call(j) for j in range(copies)])
                reps = max(1, steps // copies)
                ms = time_graph_steps(g, {}, copies, reps * copies) / (reps * copies)
                with native.profile_launches() as prof:
                    for j in range(copies):
                        call(j)
                slots = idx.shape[1] + (eidx.shape[1] if ratio else 0)
                bytes_q = nq * slots * 584 + nq * H * 1024 * 2 + nq * slots * 4 + H * 4
                key = f"c{ratio}_nq{nq}_h{H}"
                kern = {n: round(v["avg_us"], 3) for n, v in prof.results.items()}
                main = "dsv4_mfma_kernel" if "dsv4_mfma_kernel" in kern else "dsv4_tile_kernel"
                out[key] = {"ms_per_call": round(ms, 5), "ms_per_query": round(ms / nq, 5),
                            "query_heads_per_s": round(nq * H / (ms / 1e3), 1),
                            "kernels_avg_us": kern,
                            "algorithmic_bytes": bytes_q,
                            "achieved_gbps_call": round(bytes_q / (ms / 1e3) / 1e9, 1),
                            "main_kernel": main,
                            "main_kernel_gbps": round(bytes_q / (kern.get(main, float("nan")) * 1e-6) / 1e9, 1)}
                log(f"dsv4 {key}: {out[key]}")
                del g
        del caches, ecaches, c
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    # quantize-on-write of the SWA pool's 65536 tokens (1 KiB bf16 in, 584 B out each)
    T, ps = 65536, 64
    tok = torch.randn(T, 512, device=dev).to(torch.bfloat16)
    cache = native.dsv4_pack_tokens(tok, ps)
    for _ in range(3):
        native.dsv4_pack_tokens(tok, ps, cache=cache)
    with native.profile_launches() as prof:
        for _ in range(20):
            native.dsv4_pack_tokens(tok, ps, cache=cache)
    us = prof.results["dsv4_pack_kernel"]["avg_us"]
    nbytes = T * (1024 + 584)
    out["pack_65536_tokens"] = {"kernel_us": round(us, 3), "bytes": nbytes,
                                "achieved_gbps": round(nbytes / (us * 1e-6) / 1e9, 1),
                                "frac_of_hbm_peak": round(nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4)}
    log(f"dsv4 pack: {out['pack_65536_tokens']}")
    del tok, cache
    return out


def dsv4_case_run(key, calls, copies=16):
    """One DSV4 case of the dsv4 leg (same inputs), `calls` eager calls over
    `copies` rotated caches; returns the mean call time from device events."""
    import re

    import torch

    from csahca_amd import native
    from csahca_amd.synthetic import make_dsv4_window_case

    m = re.fullmatch(r"c(0|4|128)_nq(\d+)_h(\d+)", key)
    if not m:
        raise SystemExit(f"bench.py: --dsv4-case wants cR_nqN_hH with R in 0/4/128, got {key!r}")
    ratio, nq, H = (int(x) for x in m.groups())
    if nq > 32 or H > 64:
        raise SystemExit("bench.py: --dsv4-case covers nq <= 32, H <= 64 (the dsv4 leg's inputs)")
    dev = torch.device("cuda", 0)
    c = make_dsv4_window_case(compress_ratio=ratio, num_queries=32, heads=64, seed=ratio, device=dev)
    caches = [c.cache] + [c.cache.clone() for _ in range(copies - 1)]
    ecaches = ([c.extra_cache] + [c.extra_cache.clone() for _ in range(copies - 1)]) if ratio else None
    q = c.q[:nq, :H].contiguous()
    idx, lens = c.token_indices[:nq].contiguous(), c.topk_lengths[:nq].contiguous()
    sink = c.attn_sink[:H].contiguous()
    eidx = c.extra_token_indices[:nq].contiguous() if ratio else None
    elens = c.extra_topk_lengths[:nq].contiguous() if ratio else None
    scale = 1.0 / math.sqrt(512)

    def call(j):
        if ratio:
            return native.dsv4_decode_forward_tiled(q, caches[j], idx, lens, ecaches[j], eidx, elens, sink,
                                                    c.page_size, c.extra_page_size, 0, scale)
        return native.dsv4_decode_forward_tiled(q, caches[j], idx, lens, None, None, None, sink, c.page_size, 1, 0,
                                                scale)

    for j in range(copies):
        call(j)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(calls):
        call(i % copies)
    end.record()
    torch.cuda.synchronize()
    slots = idx.shape[1] + (eidx.shape[1] if ratio else 0)
    return {"dsv4_case": key, "calls": calls, "ms_per_call_eager": round(start.elapsed_time(end) / calls, 5),
            "algorithmic_bytes": nq * slots * 584 + nq * H * 1024 * 2 + nq * slots * 4 + H * 4,
            "flops": 2048 * slots * H * nq}


def large_batch_bench(steps=40, copies=2):
    """The fused step where enough heads are in flight to be bandwidth-bound:
    Sweep point B32 H8 D128 S131072 chunk 64 top-32 (the sweep's largest), two distinct 17 GiB K/V copies alternating (no cache reuse).
    Reports the step time and HBM roofline on the algorithmic bytes (fp32
    summaries + selected K/V rows)."""
    import torch

    from csahca_amd import native

    dev = torch.device("cuda", 0)
    B, H, D, S, chunk, k = 32, 8, 128, 131072, 64, 32
    g = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(B, H, D, dtype=torch.bfloat16, device=dev, generator=g)
    ks = [torch.empty(B, H, S, D, dtype=torch.bfloat16, device=dev).normal_(generator=g) for _ in range(copies)]
    vs = [torch.empty(B, H, S, D, dtype=torch.bfloat16, device=dev).normal_(generator=g) for _ in range(copies)]
    ss = [native.csa_chunk_summary(kk, chunk) for kk in ks]
    for i in range(4):
        native.csa_decode_step(q, ks[i % copies], vs[i % copies], ss[i % copies], chunk, k)
    with native.profile_launches() as prof:
        for i in range(steps):
            native.csa_decode_step(q, ks[i % copies], vs[i % copies], ss[i % copies], chunk, k)
    us = prof.results["csa_step_kernel"]["avg_us"]
    nbytes = B * H * (S // chunk) * D * 4 + B * H * k * chunk * D * 2 * 2 + B * H * D * 2 * 2 + B * H * k * 4
    gbps = nbytes / (us * 1e-6) / 1e9
    out = {"config": f"csa_decode_step B{B} H{H} D{D} S{S} chunk{chunk} top_k{k} bf16, {copies} alternating "
                     f"cache copies", "avg_launch_us": round(us, 3), "tokens_per_s": round(B / (us * 1e-6), 1),
           "roofline": {"bound": "hbm", "kernel": "csa_step_kernel", "bytes_per_launch": nbytes,
                        "achieved": round(gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                        "frac": round(gbps / PEAK_HBM_GBPS, 4)}}
    log(f"large batch: {out}")
    del ks, vs, ss, q
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out


def hca_bench(steps=256, copies=4, hca_chunk=256):
    """HCA and the CSA/HCA hybrid at the headline shape (B1 H8 S32768 D128 bf16,
    hca_chunk 256 as in the reference benchmark, CSA chunk 64 top-8 from cached
    summaries).  HCA reads all of K and V once per call: 128 MiB, HBM-bound.
    `copies` distinct K/V sets (512 MiB) rotate so the 256 MiB MALL cannot hold
    a call's data; inputs are drawn on the device (timing only)."""
    import torch

    from csahca_amd import native

    dev = torch.device("cuda", 0)
    B, H, S, D = 1, 8, 32768, 128
    g = torch.Generator(device=dev).manual_seed(1)
    q = torch.randn(B, H, D, dtype=torch.bfloat16, device=dev, generator=g)
    ks = [torch.empty(B, H, S, D, dtype=torch.bfloat16, device=dev).normal_(generator=g) for _ in range(copies)]
    vs = [torch.empty(B, H, S, D, dtype=torch.bfloat16, device=dev).normal_(generator=g) for _ in range(copies)]
    summs = [native.csa_chunk_summary(k, 64) for k in ks]

    def hca(j):
        return native.hca_decode_forward(q, ks[j], vs[j], hca_chunk)

    def hybrid(j):
        return native.hybrid_decode_forward(q, ks[j], vs[j], csa_chunk_size=64, csa_top_k=8,
                                            hca_chunk_size=hca_chunk, summary=summs[j])

    kv_bytes = 2 * B * H * S * D * 2
    out = {"config": f"B{B} H{H} S{S} D{D} bf16, hca_chunk {hca_chunk}; hybrid adds the CSA step "
                     f"(chunk 64, top-8, cached summaries) and the 0.7/0.3 blend"}
    for name, fn in (("hca", hca), ("hybrid", hybrid)):
        for j in range(copies):
            fn(j)
        gr = graph_of([lambda j=j: fn(j) for j in range(copies)])
        reps = max(1, steps // copies)
        ms = time_graph_steps(gr, {}, copies, reps * copies) / (reps * copies)
        with native.profile_launches() as prof:
            for _ in range(4):
                for j in range(copies):
                    fn(j)
        kern = {n: round(v["avg_us"], 3) for n, v in prof.results.items()}
        row = {"ms_per_token": round(ms, 5), "tokens_per_s": round(B / (ms / 1e3), 1), "kernels_avg_us": kern}
        if name == "hca":
            us = prof.results["hca_chunk_kernel"]["avg_us"]
            gbps = kv_bytes / (us * 1e-6) / 1e9
            row["roofline"] = {"bound": "hbm", "kernel": "hca_chunk_kernel", "bytes_per_launch": kv_bytes,
                               "achieved": round(gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                               "frac": round(gbps / PEAK_HBM_GBPS, 4)}
        out[name] = row
        log(f"{name}: {row}")
        del gr
    del ks, vs, summs
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out


GRAPH_STEPS = 10  # decode steps per captured graph in the block leg (as a 10-layer step graph holds 10 blocks)


def block_bench(steps=200, warmup=20):
    """The decode blocks of csahca_amd.block at S=32768,
    H=8, D=128 (hidden 1024), chunk 64, top-8, bf16, 200 steps after 20 warm-up
    steps, the hidden state fed back each step (the reference harness,
    hybrid_attention/model_inference.py:140-162).  Like that harness it reuses
    one static cache (no rotation).  Reference block: precomputed selection
    (tiled op, tile 8) and dynamic selection (fused step from cached summaries,
    and from summaries rebuilt every step as the reference does), eager and as
    HIP graphs of GRAPH_STEPS consecutive steps (the result written back in
    place as the next input).  Hybrid block (RMSNorm/QKV/SiLU MLP, growing
    cache): eager, and as graphs of GRAPH_STEPS steps whose replays advance the
    cache (position and chunk count live on the device); with the library's
    fused decode-step products, and with torch's products for comparison.
    Graph figures are per step (replay time / GRAPH_STEPS)."""
    import torch

    from csahca_amd import native
    from csahca_amd.block import HybridDecodeBlock, MiniCSADecodeBlock

    dev = torch.device("cuda", 0)
    B, H, D, S, chunk, k = 1, 8, 128, 32768, 64, 8
    g = torch.Generator(device=dev).manual_seed(0)
    hidden0 = torch.randn(B, H * D, dtype=torch.bfloat16, device=dev, generator=g)
    kc = torch.randn(B, H, S, D, dtype=torch.bfloat16, device=dev, generator=g)
    vc = torch.randn(B, H, S, D, dtype=torch.bfloat16, device=dev, generator=g)
    summ = native.csa_chunk_summary(kc, chunk)

    def timed(fn, n):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / n

    out = {"config": f"B{B} H{H} D{D} S{S} chunk{chunk} top{k} bf16, {steps} steps + {warmup} warm-up"}
    for mlp, fused in ((2.0, True), (0.0, True), (2.0, False), (0.0, False)):
        blk = MiniCSADecodeBlock(heads=H, head_dim=D, dtype=torch.bfloat16, device=dev, mlp_ratio=mlp, seed=0,
                                 fused=fused)
        q0 = torch.nn.functional.linear(hidden0, blk.w_q).view(B, H, D)
        sel = native.csa_select_topk(q0, summ, k)
        modes = {"precomputed": dict(selection="precomputed", selected_chunks=sel),
                 "dynamic_cached_summary": dict(selection="dynamic", summary=summ)}
        if mlp == 0.0:
            modes["dynamic_recomputed_summary"] = dict(selection="dynamic", summary=None)
        if not fused:
            modes = {"precomputed": modes["precomputed"]}
        for mode, kw in modes.items():
            hbuf = hidden0.clone()

            def one():  # the step's result becomes the next step's input, in place
                blk(hbuf, kc, vc, chunk_size=chunk, top_k=k, out=hbuf, **kw)

            for _ in range(warmup):
                one()
            ms_eager = timed(one, steps)
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                one()
            torch.cuda.current_stream().wait_stream(s)
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                for _ in range(GRAPH_STEPS):
                    one()
            gr.replay()
            ms_graph = timed(gr.replay, max(1, steps // GRAPH_STEPS)) / GRAPH_STEPS
            row = {"ms_per_token_eager": round(ms_eager, 5), "ms_per_token_graph": round(ms_graph, 5),
                   "tokens_per_s_graph": round(B / (ms_graph / 1e3), 1)}
            name = f"mini_mlp{mlp:g}_{mode}" + ("" if fused else "_torch_products")
            out[name] = row
            log(f"block {name}: {row}")
            del gr
    for mlp, fused in ((2.0, True), (0.0, True), (2.0, False), (0.0, False)):
        reps = max(1, steps // GRAPH_STEPS)
        hb = HybridDecodeBlock(batch=B, heads=H, head_dim=D, chunk_size=chunk, top_k=k, mlp_ratio=mlp, device=dev,
                               seed=0, fused=fused,
                               capacity=S + warmup + steps + 16 + 1 + GRAPH_STEPS * (reps + 2) + 64)
        hb.prefill(kc, vc)
        hbuf = hidden0.clone()

        def one_h():  # the step's result becomes the next step's input, in place
            hb(hbuf, out=hbuf)

        for _ in range(warmup):
            one_h()
        ms = timed(one_h, steps)
        replay, _ = hb.capture(hbuf, steps=GRAPH_STEPS, feedback=True)
        replay()
        replay()
        ms_graph = timed(replay, reps) / GRAPH_STEPS
        row = {"ms_per_token_eager": round(ms, 5), "ms_per_token_graph": round(ms_graph, 5),
               "tokens_per_s_graph": round(B / (ms_graph / 1e3), 1), "final_length": hb.length}
        if fused:
            # library kernels of eager steps (start/stop events per dispatch)
            nprof = 16
            with native.profile_launches() as prof:
                for _ in range(nprof):
                    one_h()
            row["library_kernels_us_per_step"] = {n_: round(v["avg_us"] * v["launches"] / nprof, 3)
                                                  for n_, v in prof.results.items()}
            g = prof.results.get("block_gemv_kernel")
            if g:
                wbytes = sum(t.numel() * t.element_size() for t in (hb.w_qkv, hb.w_out)
                             + ((hb.w_up, hb.w_down) if hb.use_mlp else ()))
                us = g["avg_us"] * g["launches"] / nprof
                row["block_gemv"] = {"weight_bytes_per_step": wbytes, "us_per_step": round(us, 3),
                                     "launches_per_step": g["launches"] // nprof,
                                     "achieved_gbps": round(wbytes / (us * 1e-6) / 1e9, 1),
                                     "frac_of_hbm_peak": round(wbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4)}
        name = f"baseline_block_mlp{mlp:g}_growing_cache" + ("" if fused else "_torch_products")
        out[name] = row
        log(f"block {name}: {row}")
        del hb, replay
    del kc, vc, summ
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out


def sweep(args):
    rows = []
    for B in (1, 8, 32):
        for S in (8192, 32768, 131072):
            for k in (8, 32):
                for variant in ("iid", "scattered"):
                    if variant == "scattered" and B * S > 8 * 32768:
                        continue  # planting is a CPU loop; keep it to the small points
                    r = csa_bench(args, B=B, S=S, top_k=k, copies=None, planted=None if variant == "iid" else
                                     "scattered", eager=False)
                    kern = {n: v["avg_us"] for n, v in r["kernels"].items()}
                    row = dict(B=B, S=S, top_k=k, variant=variant, tile=r["tile"], copies=r["copies"],
                               ms_per_step=round(r["ms_per_step_graph"], 5),
                               step_gbps=round(r["step_bytes"] / (r["ms_per_step_graph"] / 1e3) / 1e9, 1),
                               kernels_us={n: round(v, 3) for n, v in kern.items()})
                    att = [n for n in kern if n.startswith("csa_attend")]
                    if att:
                        row["attend_gbps"] = round(kernel_bytes(att[0], r) / (kern[att[0]] * 1e-6) / 1e9, 1)
                    log("sweep", json.dumps(row))
                    rows.append(row)
    return rows


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE={world}); "
              "the decode path has no cross-GPU exchange to time here", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        sys.exit(1)
    from csahca_amd import native

    native.lib()
    log(f"device: {torch.cuda.get_device_name(0)}")
    if args.calibrate_copy > 0:
        n = args.calibrate_copy * 2 ** 20
        src = torch.empty(n // 4, dtype=torch.float32, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(8):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy": {"bytes_read_per_launch": n, "bytes_written_per_launch": n,
                                             "launches": 8}}), flush=True)
        return
    if args.dsv4_case:
        print(json.dumps(dsv4_case_run(args.dsv4_case, args.steps)), flush=True)
        return
    r = csa_bench(args, copies=args.copies, attend_only=True)
    ms = r["ms_per_step_eager"] if args.no_graph else r["ms_per_step_graph"]
    kern = r["kernels"]
    log("csa kernels:", json.dumps(kern))
    # dominant kernel = largest total device time
    dom = max(kern, key=lambda n: kern[n]["total_ms"])
    dom_bytes = kernel_bytes(dom, r)
    dom_us = kern[dom]["avg_us"]
    achieved = dom_bytes / (dom_us * 1e-6) / 1e9
    traffic = None
    tfile = ROOT / "profiles" / "traffic.json"
    if tfile.exists():
        try:
            traffic = json.loads(tfile.read_text()).get(dom, {}).get("hbm_bytes_per_launch")
        except (ValueError, AttributeError):
            traffic = None
    line = {
        "metric": METRIC,
        "value": round(ms, 6),
        "unit": "ms/token",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "csa_decode_step B1 H8 D128 S32768 chunk64 top_k8 (select from cached fp32 "
                               "summaries + split-KV attend + merge)",
                   "batch": 1, "heads": 8, "head_dim": 128, "seq_len": 32768, "chunk_size": 64, "top_k": 8,
                   "route": args.route, "tile": r["tile"] or None, "cache_copies_rotated": r["copies"],
                   "timing": "eager launches" if args.no_graph else "hip graph replay",
                   "parallelism": "single GPU"},
        "tokens_per_s": round(1e3 / ms, 1),
        "attend_only_ms": round(r["attend_only_ms"], 6) if "attend_only_ms" in r else None,
        "attend_only_note": "precomputed selection, split-KV op (tile %s) + merge; the reference's "
                            "cuda-csa-tiled headline mode (H100: 0.0232 ms)" % r.get("attend_only_tile"),
        "ms_per_step_eager": round(r["ms_per_step_eager"], 6),
        "step_bytes": r["step_bytes"],
        "step_hbm_gbps": round(r["step_bytes"] / (ms / 1e3) / 1e9, 1),
        "kernels_avg_us": {n: round(v["avg_us"], 3) for n, v in kern.items()},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": PEAK_HBM_GBPS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBPS, 4), "traffic": traffic,
                     "bytes_per_launch": dom_bytes, "avg_launch_us": round(dom_us, 3)},
    }
    if not args.no_large_batch:
        line["large_batch"] = large_batch_bench()
    if not args.no_hca:
        line["hca"] = hca_bench()
    if not args.no_block:
        line["block"] = block_bench()
    if not args.no_dsv4:
        line["dsv4"] = dsv4_bench()
    if args.sweep:
        rows = sweep(args)
        if args.sweep_out is not None:
            args.sweep_out.parent.mkdir(parents=True, exist_ok=True)
            args.sweep_out.write_text(json.dumps(rows, indent=1) + "\n")
    bad = {str(k): v for k, v in native.csa_step_status().items() if v}
    if bad:
        print(f"bench.py: a decode-step exchange timed out (status words {bad}); results are invalid",
              file=sys.stderr)
        sys.exit(3)
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
