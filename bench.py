#!/usr/bin/env python3
"""Projection-GEMM benchmark on one MI355X.

One step = the whole projection stack of the model (every layer's
projections, fused epilogues included) over one packed ragged batch whose
inputs are already resident in HBM.  Default workload: ModernBERT-base
shapes (22 layers, hidden 768, intermediate 1152) in bf16, sequence lengths
U[16,512] packed to an 8192-token budget, a fresh batch (and so a fresh M)
every step from a cycle of pre-drawn batches.  Weights N(0, 0.02) and
activations N(0, 1), seeded, synthetic.

Prints ONE JSON line.  `value` is the projection throughput in TFLOP/s
(algorithmic 2*M*N*K per projection); tokens/s and the fraction of the bf16
dense MFMA peak ride along.  `roofline` is the dominant kernel (largest total
time) timed with HIP events on the stream the projections run on, in a pass
identical to the timed one.  `cpu_baseline` is the CPU oracle's f32
projection stack (ModernBERT-base, M = 8 x 128 = 1024) on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA (published)
CHAIN_KERNEL = "chain_kernel<128,192,4,2,3,4>"  # the projection-chain kernel's tile shape (csrc/chain.hip)
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E (published)
RIDGE = PEAK_BF16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)

WORKLOADS = {
    # name: (stack config, length range, budget, exact packing)
    "modernbert-base": ("modernbert-base", (16, 512), 8192, False),
    "modernbert-large": ("modernbert-large", None, None, False),
    "qwen35-small": ("qwen35-small", (64, 2048), 8192, True),
    "qwen35-27b": ("qwen35-27b", (32, 1024), 4096, True),
    # images of 64..1024 patches (multiples of the 2x2 merge do not matter
    # to the projections) packed to 8192 patch rows
    "qwen35-vision": ("qwen35-vision", (64, 1024), 8192, False),
}


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="modernbert-base", choices=sorted(WORKLOADS))
    ap.add_argument("--tokens", type=int, default=None,
                    help="fixed packed M instead of ragged draws (e.g. the large-config sweep)")
    ap.add_argument("--batches", type=int, default=8, help="distinct ragged batches cycled")
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-roofline", action="store_true")
    ap.add_argument("--no-small-m", action="store_true",
                    help="skip the small-M (ModernBERT-large at M = 64 and 256) object of the line")
    ap.add_argument("--norms", action="store_true",
                    help="fuse each projection's pre-norm (LayerNorm / RMSNorm) into it; the "
                         "row-statistics pass then sits inside the timed step")
    ap.add_argument("--conv", action="store_true",
                    help="fuse the DeltaNet causal conv + SiLU into each in_proj (Qwen3.5 stacks; "
                         "positions from the packed batch's sequence lengths)")
    ap.add_argument("--row-major", action="store_true",
                    help="keep the weights row-major [out, in] (candle's layout) instead of the blocked "
                         "layout packed at load (contiguous 4 KB per 32 rows and k-step; "
                         "sys1hip_pack_blocked_weight), which the default uses: same results bit for bit, "
                         "measured 0-5%% faster, most at small M")
    ap.add_argument("--chain", choices=("on", "off"), default="off",
                    help="on: each row-local run of projections (between two attention calls) is one "
                         "persistent launch (sys1hip_linear_chain_bf16)")
    ap.add_argument("--graph", action="store_true",
                    help="replay one HIP graph per prepared batch instead of enqueueing every "
                         "projection from the host (measured: no difference on one MI355X)")
    ap.add_argument("--kernel", default=None, metavar="NAME",
                    help="force one tile kernel (a sys1hip_kernel_name) for every projection, "
                         "for tuning the kernel choice; the line then records it in config")
    ap.add_argument("--calibration-copy", type=int, default=0, metavar="MIB",
                    help="after the run, 8 bf16 negations of MIB MiB (read MIB, write MIB): the "
                         "known-size kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE")
    ap.add_argument("--vs-torch", action="store_true",
                    help="with --workload and --tokens: time each distinct projection shape of the stack (no "
                         "epilogue) on this library and on torch's matmul (hipBLASLt) over rotated weight "
                         "copies larger than the MALL, print a table and exit")
    ap.add_argument("--trace-summary", metavar="CSV",
                    help="reduce a rocprofv3 kernel_trace.csv of a bench run (with --workload, --tokens) "
                         "to per-projection kernel durations and their HBM / MFMA rates, and exit")
    ap.add_argument("--chain-timeline", action="store_true",
                    help="with --chain on: after the warm-up, record the in-kernel timeline of one chain "
                         "launch (the middle layer's; sys1hip_set_chain_trace), print its per-projection "
                         "summary as markdown and exit")
    ap.add_argument("--pmc-summary", nargs="+", metavar="CSV",
                    help="reduce rocprofv3 counter_collection.csv files to per-kernel averages "
                         "per dispatch and exit (no GPU use)")
    return ap.parse_args()


def pmc_summary(paths: list[str]) -> None:
    """Average counter value per dispatch, per kernel name, over the given
    rocprofv3 --pmc CSV files (rows are one counter of one dispatch; a
    counter collected per XCD/SE instance is summed within the dispatch)."""
    import csv
    import collections
    per = collections.defaultdict(lambda: collections.defaultdict(float))
    for path in paths:
        for r in csv.DictReader(open(path)):
            per[(r["Kernel_Name"], r["Dispatch_Id"])][r["Counter_Name"]] += float(r["Counter_Value"])
    by_kernel = collections.defaultdict(lambda: collections.defaultdict(list))
    for (name, _), counters in per.items():
        for c, v in counters.items():
            by_kernel[name][c].append(v)
    for name in sorted(by_kernel):
        cs = by_kernel[name]
        n = max(len(v) for v in cs.values())
        vals = ", ".join(f"{c}={sum(v) / len(v):.6g}" for c, v in sorted(cs.items()))
        print(f"{n:6d} dispatches | {vals} | {name[:160]}")


def chain_timeline(dev, launches, M: int) -> None:
    """One chain launch with the in-kernel trace on: every workgroup's
    wave 0 records each item or tile it runs (100 MHz constant clock).
    Prints per projection the start / dependency / end windows (weight-
    streaming chain, M <= 64) or the tile, k-loop and epilogue times (tile
    chain), as markdown."""
    import ctypes
    import collections
    import numpy as np
    import torch
    from sys1_amd import _lib
    from sys1_amd.stacks import STREAM_CHAIN_MAX_M, STREAM_CHAIN_MAX_K
    chains = [c for c in launches if isinstance(c[0], tuple)]
    if not chains:
        raise SystemExit("--chain-timeline: no chain launch in this stack (use --chain on)")
    projs, fn, a = chains[len(chains) // 2]
    names = [p.name for p in projs]
    stream = M <= STREAM_CHAIN_MAX_M and all(p.K <= STREAM_CHAIN_MAX_K for p in projs)
    slots, per = 1024, 64
    buf = torch.zeros(slots * per * 4, dtype=torch.int64, device="cuda:0")
    L = dev._L
    _lib.check(L.sys1hip_set_chain_trace(dev.ctx, ctypes.c_void_p(buf.data_ptr()), buf.numel() * 8), dev.ctx)
    try:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        dev.follow_torch_stream()
        e0.record()
        if fn(*a):
            raise RuntimeError("chain launch failed")
        e1.record()
        torch.cuda.synchronize()
        flags = dev.chain_status()
    finally:
        _lib.check(L.sys1hip_set_chain_trace(dev.ctx, None, 0), dev.ctx)
    t = buf.view(slots, per, 4).cpu().numpy().astype(np.uint64)
    us = lambda ticks: ticks / 100.0
    q = lambda v: f"{np.min(v):.1f} / {np.median(v):.1f} / {np.max(v):.1f}"
    print(f"chain {' -> '.join(names)}, M = {M}, "
          f"{'weight-streaming chain' if stream else 'tile chain'}: launch {e0.elapsed_time(e1) * 1e3:.1f} us "
          f"(HIP events), status {flags}")
    if stream:
        recs = [(wg, k, int(r[0]) >> 32, int(r[1]), int(r[2]), int(r[3]))
                for wg in range(slots) for k in range(per) for r in [t[wg, k]] if r[3]]
        t0 = min(r[3] for r in recs)
        print(f"items {len(recs)}, workgroups {len(set(r[0] for r in recs))}, "
              f"span {us(max(r[5] for r in recs) - t0):.1f} us, second-round items {sum(r[1] > 0 for r in recs)}")
        print()
        print("| projection | items | start (min / median / max, us) | dependency met | end | "
              "work after the wait |")
        print("|---|---:|---|---|---|---|")
        for p in range(len(names)):
            rs = [r for r in recs if r[2] == p]
            st = [us(r[3] - t0) for r in rs]
            dp = [us(r[4] - t0) for r in rs]
            en = [us(r[5] - t0) for r in rs]
            wk = [us(r[5] - r[4]) for r in rs]
            print(f"| {names[p]} | {len(rs)} | {q(st)} | {q(dp)} | {q(en)} | {q(wk)} |")
        return
    recs, entries = [], []
    for wg in range(slots):
        for k in range(per):
            r = t[wg, k]
            if r[1] == 0 and r[2] == 0:
                continue
            if int(r[0]) == 0xffffffff:
                entries.append((int(r[1]), int(r[2])))
                continue
            recs.append((wg, int(r[0]) >> 40 & 1, int(r[1]), int(r[2]), int(r[3]) & 0xff, us(int(r[3]) >> 8)))
    t0 = min(e[0] for e in entries)
    print(f"tiles {len(recs)}, workgroups {len(entries)}, span {us(max(r[3] for r in recs) - t0):.1f} us, "
          f"tiles that waited for their dependency {sum(r[1] for r in recs)}, "
          f"entry to first k-tile in LDS {q([us(e[1] - e[0]) for e in entries])} us")
    print()
    print("| projection | tiles | tile (mean, us) | k-loop (min / median / max) | epilogue (mean) | "
          "first start / last end |")
    print("|---|---:|---:|---|---:|---|")
    for p in range(len(names)):
        rs = [r for r in recs if r[4] == p]
        d = [us(r[3] - r[2]) for r in rs]
        kl = [r[5] for r in rs]
        print(f"| {names[p]} | {len(rs)} | {np.mean(d):.1f} | {q(kl)} | {np.mean(d) - np.mean(kl):.1f} | "
              f"{us(min(r[2] for r in rs) - t0):.1f} / {us(max(r[3] for r in rs) - t0):.1f} |")


def trace_summary(path: str, workload: str, tokens: int | None) -> None:
    """Per-projection kernel durations from a rocprofv3 kernel trace of a
    bench run: the projection kernels (sys1 GEMM kernels, in dispatch order)
    map onto the stack's projection sequence, layer after layer; the last
    whole steps are averaged.  With --tokens, each projection's algorithmic
    bytes and FLOP give its HBM and MFMA rates."""
    import csv
    import collections
    from sys1_amd.stacks import CONFIGS
    cfg = CONFIGS[WORKLOADS[workload][0]]()
    seq = [p for layer in cfg.layers for p in layer]
    rows = [r for r in csv.DictReader(open(path))
            if "gemm_tile_kernel" in r["Kernel_Name"] or "skinny_kernel" in r["Kernel_Name"]]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    steps = len(rows) // len(seq)
    rows = rows[len(rows) - steps * len(seq):]
    per = collections.defaultdict(list)
    names = {}
    for i, r in enumerate(rows):
        p = seq[i % len(seq)]
        per[p.name].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
        names.setdefault(p.name, r["Kernel_Name"].split("(")[0].replace("void sys1::", ""))
    total = sum(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in rows) / steps / 1e3
    span = (int(rows[-1]["End_Timestamp"]) - int(rows[0]["Start_Timestamp"])) / steps / 1e3
    print(f"{workload} M={tokens}: {steps} steps; kernel time per step {total:.1f} us, "
          f"first start to last end per step {span:.1f} us")
    first = {p.name: p for p in seq}
    for name, d in per.items():
        us = sum(d) / len(d) / 1e3
        line = f"  {name:16s} {names[name]:48s} {len(d):5d} launches  {us:8.2f} us"
        if tokens:
            p = first[name]
            line += (f"  {p.bytes(tokens) / us / 1e3:8.1f} GB/s ({p.bytes(tokens) / us / 1e3 / PEAK_HBM_GBS:.3f})"
                     f"  {p.flops(tokens) / us / 1e6:7.1f} TFLOP/s")
        print(line)


def vs_torch(workload: str, tokens: int, reps: int = 30) -> None:
    """Each distinct (N, K) projection shape of the stack at M = tokens, as
    a plain GEMM: this library (its automatic plan, blocked weights) and
    torch.matmul(x, w.T) (hipBLASLt), each over enough rotated weight copies
    to exceed the 256 MB MALL, so every call streams its weight from HBM as
    in a deep stack.  Times are HIP events over back-to-back calls (launch
    gaps included); a rocprofv3 kernel trace of the same run gives the
    kernel durations."""
    import torch
    from sys1_amd.device import HipDevice
    from sys1_amd.linear import Linear
    from sys1_amd.stacks import CONFIGS
    cfg = CONFIGS[WORKLOADS[workload][0]]()
    dev = HipDevice(0)
    shapes = []
    for p in cfg.layers[0]:
        if (p.N, p.K) not in shapes:
            shapes.append((p.N, p.K))
    x = torch.randn(tokens, max(k for _, k in shapes), device="cuda:0").to(torch.bfloat16)
    print(f"{workload} M={tokens}: plain GEMMs over rotated weights (HIP events, launch gaps included)")
    for N, K in shapes:
        copies = max(2, (300 << 20) // (2 * N * K) + 1)
        ws = [(torch.randn(N, K, device="cuda:0") * 0.02).to(torch.bfloat16) for _ in range(copies)]
        ours = [Linear(w, device=dev, blocked=True) for w in ws]
        xk = x[:, :K].contiguous()
        y = torch.empty(tokens, N, dtype=torch.bfloat16, device="cuda:0")
        res = {}
        for tag, fn in (("sys1hip", lambda i: ours[i % copies].forward_into(xk, y)),
                        ("torch", lambda i: torch.matmul(xk, ws[i % copies].t(), out=y))):
            for i in range(copies):
                fn(i)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for i in range(reps * copies // max(1, copies // 4) if copies < 8 else reps):
                fn(i)
            e1.record()
            torch.cuda.synchronize()
            n = reps * copies // max(1, copies // 4) if copies < 8 else reps
            res[tag] = e0.elapsed_time(e1) * 1e3 / n
        kname = dev.query_kernel(tokens, N, K, 0)[1]
        print(f"  N={N:6d} K={K:6d}  sys1hip {res['sys1hip']:8.2f} us ({kname})  torch {res['torch']:8.2f} us")
        del ws, ours
        torch.cuda.empty_cache()


def load_traffic(workload: str, kernel: str) -> dict | None:
    """HBM bytes per launch of the dominant kernel, measured by rocprofv3
    FETCH_SIZE / WRITE_SIZE passes and committed as profiles/traffic.json
    (per workload and kernel, already scaled by the copy calibration)."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        table = json.load(open(path))
    except (OSError, ValueError):
        return None
    return table.get(workload, {}).get(kernel)


def cpu_baseline(seconds: float) -> dict:
    """The CPU oracle's f32 projection stack, ModernBERT-base shapes at
    M = 8 x 128 = 1024 tokens (the reference's CPU configuration), run
    layer after layer until `seconds` have passed."""
    import numpy as np
    from oracle import oracle as orc
    from sys1_amd.stacks import CONFIGS
    cfg = CONFIGS["modernbert-base"]()
    M = 1024
    H, I = 768, 1152
    x = orc.fill_normal((M, H), 1)
    ws = [orc.fill_normal((p.N, p.K), 100 + i, 0.02) for i, p in enumerate(cfg.layers[0])]
    orc.linear_f32(x[:64], ws[0])  # load + thread start-up outside the clock
    flops = 0
    layers = 0
    h = x
    t0 = time.perf_counter()
    while True:
        qkv = orc.linear_f32(h, ws[0])
        h1 = orc.linear_f32(np.ascontiguousarray(qkv[:, 2 * H:]), ws[1]) + h
        g = orc.geglu(orc.linear_f32(h1, ws[2]))
        h = orc.linear_f32(g, ws[3]) + h1
        layers += 1
        flops += sum(p.flops(M) for p in cfg.layers[0])
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    threads = int(os.environ.get("OMP_NUM_THREADS", 0)) or len(os.sched_getaffinity(0))
    return {"value": round(flops / el / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": f"ModernBERT-base projection layers (Wqkv, Wo, Wi+GeGLU, Wo) f32 at "
                      f"M=1024 (8x128), {layers} layers in {el:.1f} s; "
                      f"{layers * M / el:.0f} layer-tokens/s = {layers * M / el / 22:.0f} "
                      f"22-layer tokens/s"}


def small_m_pass(dev, seed: int, blocked: bool, steps: int = 20) -> dict:
    """BASELINE config 3 at the skinny end: the ModernBERT-large projection
    stack (28 layers, hidden 1024, GeGLU 2x2624) at M = 64 and M = 256
    packed tokens.  Per projection: the kernel the plan picks, its average
    time from HIP events around each launch (each step queued behind a spin
    kernel longer than the host's enqueue, so the events bracket the GPU
    work; they include the launch's dispatch gap, so they run a little above
    rocprofv3's kernel durations), the algorithmic HBM bytes per launch and
    their rate as a fraction of the 8 TB/s peak."""
    import numpy as np
    import torch
    from sys1_amd.stacks import CONFIGS, ProjectionStack
    cfg = CONFIGS["modernbert-large"]()
    stack = ProjectionStack(cfg, dev, 256, seed=seed, blocked=blocked)
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(seed + 2000)
    x = torch.randn(256, cfg.hidden, generator=gen, device="cuda:0").to(torch.bfloat16)
    out = {}
    for M in (64, 256):
        prep = stack.prepare(x, M)
        for _ in range(3):
            stack.run_prepared(prep)
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(steps):
            stack.run_prepared(prep)
        t1.record()
        torch.cuda.synchronize()
        step_ms = t0.elapsed_time(t1) / steps
        tq = time.perf_counter()
        stack.run_prepared(prep)
        host_s = time.perf_counter() - tq
        torch.cuda.synchronize()
        c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        c0.record()
        torch.cuda._sleep(1 << 20)
        c1.record()
        torch.cuda.synchronize()
        spin = int((1 << 20) * 2.0 * host_s / (c0.elapsed_time(c1) * 1e-3)) + 1
        recs = []
        for _ in range(steps):
            torch.cuda._sleep(spin)
            for p, fn, a in prep:
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                if fn(*a):
                    raise RuntimeError("launch failed")
                e1.record()
                recs.append((p, e0, e1))
        torch.cuda.synchronize()
        in_step = step_ms * steps / sum(e0.elapsed_time(e1) for _, e0, e1 in recs)
        per = {}
        for p, e0, e1 in recs:
            d = per.setdefault(p.name, {"ms": 0.0, "n": 0, "bytes": p.bytes(M), "N": p.N, "K": p.K,
                                        "epi": p.epi})
            d["ms"] += e0.elapsed_time(e1)
            d["n"] += 1
        res = {}
        for name, d in per.items():
            us = d["ms"] / d["n"] * 1e3
            gbs = d["bytes"] / (us * 1e-6) / 1e9
            res[name] = {"kernel": dev.query_kernel(M, d["N"], d["K"], d["epi"])[1], "avg_us": round(us, 2),
                         "bytes": d["bytes"], "gbs": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4),
                         "avg_us_in_step": round(us * in_step, 2),
                         "frac_in_step": round(gbs / in_step / PEAK_HBM_GBS, 4)}
        dom = max(res, key=lambda k: res[k]["avg_us"])
        total_bytes = sum(p.bytes(M) for layer in cfg.layers for p in layer)
        out[f"M{M}"] = {
            "step_ms": round(step_ms, 4),
            "stack_gbs": round(total_bytes / (step_ms * 1e-3) / 1e9, 1),
            "stack_frac": round(total_bytes / (step_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "tflops": round(cfg.flops_per_token() * M / (step_ms * 1e-3) / 1e12, 2),
            "dominant": {"projection": dom, **res[dom]},
            "per_projection": res,
        }
    out["note"] = ("ModernBERT-large (config 3) projection stack, 28 layers; per-projection times from "
                   "HIP events (each pair adds its own gap); *_in_step: a projection's share of the event "
                   "time applied to the uninterrupted step (they sum to step_ms); bytes are algorithmic "
                   "per launch")
    return out


def main():
    args = parse()
    if args.pmc_summary:
        pmc_summary(args.pmc_summary)
        return
    if args.trace_summary:
        trace_summary(args.trace_summary, args.workload, args.tokens)
        return
    if args.vs_torch:
        if not args.tokens:
            raise SystemExit("--vs-torch needs --tokens")
        vs_torch(args.workload, args.tokens)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported in this build "
              "(the projection path runs on a single MI355X; multi-GPU sharding is a design "
              "note only).", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch
    from sys1_amd import batching
    from sys1_amd.device import HipDevice
    from sys1_amd.stacks import CONFIGS, ProjectionStack

    cfg_name, lens, budget, exact = WORKLOADS[args.workload]
    cfg = CONFIGS[cfg_name]()
    if args.tokens:
        Ms = [args.tokens]
        seqs = [np.array([args.tokens])]
        batch_desc = f"fixed M={args.tokens}"
    else:
        if lens is None:
            raise SystemExit(f"--workload {args.workload} needs --tokens")
        seqs = [batching.draw_lengths(args.seed + b, lens[0], lens[1], budget, exact)
                for b in range(args.batches)]
        Ms = [int(l.sum()) for l in seqs]
        batch_desc = (f"lengths U[{lens[0]},{lens[1]}] packed to {budget}"
                      f"{' exactly' if exact else ''}, {args.batches} batches cycled")
    max_m = max(Ms)

    torch.cuda.set_device(0)
    dev = HipDevice(0)
    if args.kernel:
        from sys1_amd import kernel_names
        dev.set_kernel(kernel_names().index(args.kernel))
    stack = ProjectionStack(cfg, dev, max_m, seed=args.seed, norms=args.norms, conv=args.conv,
                            blocked=not args.row_major, chain=args.chain == "on")
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(args.seed + 1000)
    x = torch.randn(max_m, cfg.hidden, generator=gen, device="cuda:0").to(torch.bfloat16)
    positions = [torch.from_numpy(batching.positions(l)).to("cuda:0") for l in seqs]
    prepared = [stack.prepare(x, M, positions[b]) for b, M in enumerate(Ms)]
    torch.cuda.synchronize()

    for s in range(args.warmup):
        stack.run_prepared(prepared[s % len(Ms)])
    torch.cuda.synchronize()
    if args.chain_timeline:
        chain_timeline(dev, prepared[0], Ms[0])
        return

    # Optionally one HIP graph per prepared batch: the same kernel launches,
    # with the host's enqueue cost taken out of the step.  Every launch reads
    # only the inputs and the stack's own buffers, so a replay recomputes the
    # step from x; the first batch's replay is checked bit for bit (as int16
    # patterns: deep norm-free stand-in chains overflow to inf/nan) against
    # eager.
    graphs = None
    if args.graph:
        out = stack.buffers["h"]
        stack.run_prepared(prepared[0])
        torch.cuda.synchronize()
        ref = out[:Ms[0]].clone()
        graphs = []
        for b in range(len(Ms)):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                dev.follow_torch_stream()
                stack.run_prepared(prepared[b])
            graphs.append(g)
        dev.follow_torch_stream()
        for b in range(len(Ms)):
            graphs[b].replay()
        graphs[0].replay()
        torch.cuda.synchronize()
        if not torch.equal(out[:Ms[0]].view(torch.int16), ref.view(torch.int16)):
            raise SystemExit("graph replay differs from the eager step")
        for s in range(args.warmup):
            graphs[s % len(Ms)].replay()
        torch.cuda.synchronize()

    def step(s):
        if graphs is not None:
            graphs[s % len(Ms)].replay()
        else:
            stack.run_prepared(prepared[s % len(Ms)])

    # Timed region: exactly `steps` steps, synchronised on both sides.
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_wall = time.perf_counter()
    start.record()
    for s in range(args.steps):
        step(s)
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    ms = start.elapsed_time(end)
    tokens = sum(Ms[s % len(Ms)] for s in range(args.steps))
    flops = tokens * cfg.flops_per_token()
    tflops = flops / (ms * 1e-3) / 1e12

    # Roofline pass: same steps, HIP events around every launch, grouped by
    # projection kind (each kind is one kernel instantiation per shape).
    # Each step's launches queue behind a spin kernel that outlasts the
    # host's enqueue of that step, so the GPU runs behind the host and the
    # events around a launch bracket the kernel, not the host call (small-M
    # kernels are shorter than one call's host time).
    roofline = None
    per_proj = {}
    if not args.no_roofline:
        def enqueue_events(s, recs):
            for p, fn, a in prepared[s % len(Ms)]:
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                rc = fn(*a)
                e1.record()
                if rc:
                    raise RuntimeError(f"launch failed: {rc}")
                recs.append((p, Ms[s % len(Ms)], e0, e1))
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        enqueue_events(0, [])
        host_s = time.perf_counter() - t0
        torch.cuda.synchronize()
        c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        c0.record()
        torch.cuda._sleep(1 << 20)
        c1.record()
        torch.cuda.synchronize()
        spin_cycles = int((1 << 20) * 2.0 * host_s / (c0.elapsed_time(c1) * 1e-3)) + 1
        recs = []
        for s in range(args.steps):
            torch.cuda._sleep(spin_cycles)
            enqueue_events(s, recs)
        torch.cuda.synchronize()
        # The timed region runs the same steps without events between the
        # launches; each event pair adds its own gap, so the events sum to
        # more than the timed region.  A launch's share of the event time,
        # applied to the timed region, is its time inside the step.
        in_step = ms / sum(e0.elapsed_time(e1) for _, _, e0, e1 in recs)
        for p, M, e0, e1 in recs:
            # (a chain launch carries the tuple of its projections: its work
            # is theirs summed)
            ps = p if isinstance(p, tuple) else (p,)
            key = "+".join(q.name for q in ps)
            d = per_proj.setdefault(key, {"n": 0, "ms": 0.0, "flop": 0, "bytes": 0, "K": ps[0].K,
                                          "N": ps[0].N, "epi": ps[0].epi, "chain": len(ps) > 1})
            d["n"] += 1
            d["ms"] += e0.elapsed_time(e1)
            d["flop"] += sum(q.flops(M) for q in ps)
            d["bytes"] += sum(q.bytes(M) for q in ps)
        name = max(per_proj, key=lambda k: per_proj[k]["ms"])
        d = per_proj[name]
        avg_s = d["ms"] / d["n"] * 1e-3
        flop_per = d["flop"] / d["n"]
        byte_per = d["bytes"] / d["n"]
        ai = flop_per / byte_per
        if d["chain"]:
            kname = CHAIN_KERNEL
        else:
            kid, kname = dev.query_kernel(int(np.mean(Ms)), d["N"], d["K"], d["epi"])
        if ai >= RIDGE:
            achieved = flop_per / avg_s / 1e12
            roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                        "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                        "traffic": None}
        else:
            achieved = byte_per / avg_s / 1e9
            roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                        "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                        "traffic": None}
        roofline.update({"kernel": f"{name} ({kname})", "avg_us": round(avg_s * 1e6, 2),
                         "algorithmic_per_launch": {"flop": int(flop_per), "bytes": int(byte_per)},
                         # the same kernel's time inside the uninterrupted step
                         # (event share x timed region), the same rate from it
                         "in_step": {"avg_us": round(avg_s * in_step * 1e6, 2),
                                     "frac": round(roofline["frac"] / in_step, 4)}})
        for k, v in per_proj.items():
            v["avg_us"] = round(v["ms"] / v["n"] * 1e3, 2)
            v["avg_us_in_step"] = round(v["ms"] / v["n"] * 1e3 * in_step, 2)
            v["tflops"] = round(v["flop"] / (v["ms"] * 1e-3) / 1e12, 1)
            v["gbs"] = round(v["bytes"] / (v["ms"] * 1e-3) / 1e9, 1)
            for key in ("ms", "flop", "bytes", "n", "chain"):
                v.pop(key)

    if roofline is not None:
        kernel_id = roofline["kernel"]
        t = load_traffic(args.workload, kernel_id)
        if t is not None:
            roofline["traffic"] = int(t["bytes_per_launch"])
            roofline["traffic_source"] = t["source"]

    if args.calibration_copy:
        n = args.calibration_copy * (1 << 20) // 2
        src = torch.ones(n, dtype=torch.bfloat16, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(8):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()

    small_m = None
    if not args.no_small_m and args.workload == "modernbert-base" and not args.tokens:
        small_m = small_m_pass(dev, args.seed, not args.row_major)

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(args.cpu_seconds)

    line = {
        "metric": "projection TFLOP/s (% bf16 MFMA peak) + encoder tokens/s @ 8192-token batch",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) random-init weights)",
        "config": {"workload": f"{cfg.name} projection stack: {cfg.description}; {batch_desc}",
                   "launch": "one HIP graph per prepared batch" if args.graph else "eager",
                   "chains": "one launch per row-local run of projections" if args.chain == "on"
                   else "one launch per projection",
                   **({"forced_kernel": args.kernel} if args.kernel else {}),
                   "pre_norms": "fused (row statistics + folded norm weights)" if args.norms
                   else "none (projections only)",
                   "deltanet_conv": "fused into in_proj" if args.conv else "none",
                   "weight_layout": "row-major [out, in]" if args.row_major
                   else "blocked at load (4 KB per 32 rows x 64 k)",
                   "layers": len(cfg.layers), "hidden": cfg.hidden,
                   "packed_M": Ms, "flop_per_token": cfg.flops_per_token(),
                   "weight_bytes": cfg.weight_bytes(), "parallelism": "single GPU"},
        "tokens_per_s": round(tokens / (ms * 1e-3), 1),
        "pct_bf16_peak": round(100 * tflops / PEAK_BF16_TFLOPS, 2),
        "wall_s_timed": round(wall, 4),
        "roofline": roofline,
        "per_projection": per_proj,
        "small_m": small_m,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
