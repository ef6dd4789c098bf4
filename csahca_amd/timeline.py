"""Phase timeline of the fused CSA decode step (a diagnostic, not part of the op path).

    python -m csahca_amd.timeline [--batch 1] [--heads 8] [--seq 32768] [--head-dim 128]
                                  [--chunk 64] [--top-k 8] [--steps 200] [--copies 32]

Loads libcsahca_timeline.so -- the library built with the decode step's phase
stamps (csahca_amd/build.py builds it beside libcsahca.so; the product library
has none) -- and runs csa_decode_step (selection from cached summaries, split
attention, merge) on cuda:0 over `copies` rotated copies of K, V and the
summaries, so no measured step reads a copy an earlier step left in cache.
Thread 0 of every workgroup stamps the device wall clock at each phase
boundary; per launch, each boundary's time is the latest workgroup's stamp
minus the first workgroup's entry stamp.  Prints the medians over the measured
steps as a markdown table.
"""
from __future__ import annotations

import argparse
import ctypes
import statistics

import numpy as np
import torch

from . import build as _build
from . import native

# Stamp order in the kernel (csa_step.hip): entry, A done, keys gathered,
# top-k done, attention done, partial published, output written.
PHASES = [
    (1, "A: chunk scores from the summaries, keys published"),
    (2, "B: the head's keys gathered"),
    (3, "B: top-k done"),
    (4, "C: attention over the selected rows"),
    (5, "D: partial published"),
    (6, "D: output written (merging workgroup)"),
]


def _timeline_lib():
    if native._LIB is not None and native._LIB_PATH != _build.LIB_TIMELINE:
        raise RuntimeError("libcsahca.so is already loaded in this process; run the timeline in a fresh one")
    native._LIB_PATH = _build.LIB_TIMELINE
    lib = native.lib()
    lib.csahca_step_timeline_read.argtypes = [ctypes.c_void_p, ctypes.c_int64]
    lib.csahca_step_timeline_read.restype = ctypes.c_int
    lib.csahca_step_timeline_clear.argtypes = []
    lib.csahca_step_timeline_clear.restype = ctypes.c_int
    lib.csahca_step_timeline_rate_khz.argtypes = []
    lib.csahca_step_timeline_rate_khz.restype = ctypes.c_int64
    return lib


def run(batch=1, heads=8, seq=32768, head_dim=128, chunk=64, top_k=8, steps=200, copies=32, warmup=20):
    lib = _timeline_lib()
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(batch, heads, head_dim, device=dev, generator=g).to(torch.bfloat16)
    k0 = torch.randn(batch, heads, seq, head_dim, device=dev, generator=g, dtype=torch.bfloat16)
    v0 = torch.randn(batch, heads, seq, head_dim, device=dev, generator=g, dtype=torch.bfloat16)
    s0 = native.csa_chunk_summary(k0, chunk)
    ks, vs, ss = [k0], [v0], [s0]
    for _ in range(copies - 1):
        ks.append(k0.clone())
        vs.append(v0.clone())
        ss.append(s0.clone())
    khz = lib.csahca_step_timeline_rate_khz()
    if khz <= 0:
        raise RuntimeError("the wall clock rate query failed")
    us_per_tick = 1e3 / khz
    nblk = 4096
    host = np.zeros((nblk, 8), dtype=np.uint64)
    stream = torch.cuda.Stream()
    per_phase = {i: [] for i, _ in PHASES}
    spread, grids = [], set()
    for j in range(warmup + steps):
        c = j % copies
        torch.cuda.synchronize()
        if lib.csahca_step_timeline_clear() != 0:
            raise RuntimeError("clearing the stamps failed")
        with torch.cuda.stream(stream):
            native.csa_decode_step(q, ks[c], vs[c], ss[c], chunk, top_k)
        torch.cuda.synchronize()
        if lib.csahca_step_timeline_read(host.ctypes.data, nblk) != 0:
            raise RuntimeError("reading the stamps failed")
        if j < warmup:
            continue
        live = host[:, 0] != 0
        t = host[live].astype(np.int64)
        grids.add(int(live.sum()))
        t0 = t[:, 0].min()
        spread.append((t[:, 0].max() - t0) * us_per_tick)
        for i, _ in PHASES:
            col = t[:, i]
            col = col[col != 0]
            if col.size:
                per_phase[i].append((col.max() - t0) * us_per_tick)
    med = {i: statistics.median(v) for i, v in per_phase.items() if v}
    lines = [f"csa_decode_step B{batch} H{heads} D{head_dim} S{seq} chunk {chunk} top-{top_k} bf16, "
             f"{steps} steps after {warmup} warm-up over {copies} rotated copies; "
             f"{sorted(grids)} workgroups per launch; clock {khz} kHz", "",
             "| boundary (latest workgroup) | µs after the first workgroup starts | phase µs |", "|---|---:|---:|",
             f"| last workgroup starts | {statistics.median(spread):.2f} | |"]
    prev = 0.0
    for i, name in PHASES:
        if i in med:
            lines.append(f"| {name} | {med[i]:.2f} | {med[i] - prev:.2f} |")
            prev = med[i]
    return "\n".join(lines) + "\n"


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--heads", type=int, default=8)
    ap.add_argument("--seq", type=int, default=32768)
    ap.add_argument("--head-dim", type=int, default=128)
    ap.add_argument("--chunk", type=int, default=64)
    ap.add_argument("--top-k", type=int, default=8)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--copies", type=int, default=32)
    a = ap.parse_args()
    if not torch.cuda.is_available():
        raise SystemExit("the phase timeline needs a GPU")
    print(run(a.batch, a.heads, a.seq, a.head_dim, a.chunk, a.top_k, a.steps, a.copies), end="")


if __name__ == "__main__":
    main()
