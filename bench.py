"""Benchmark of the MI355X decode hot path (one JSON line on stdout).

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Workload (the isolated quantized GEMV sweep): weights
[N,K] in {4096x4096, 14336x4096, 4096x14336, 128256x4096}, INT8 and FP8 E4M3
per-row scaled, drawn N(0, 0.02) and quantized by the library's own codec,
fp32 activations N(0, 1) at batch 1, 4 and 16.  One step runs every one of the
24 GEMVs once; each GEMV reads a different copy of its weights from a pool of
>= 1 GiB per shape, so the 256 MB Infinity Cache cannot serve repeats.

value = algorithmic bytes of a step / step time (GB/s), with the algorithmic
bytes of one GEMV N*K + 4N (row scales) + 4BK (x) + 4BN (y).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "42-berlin-engine_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

HBM_PEAK_GBS = 8000.0
SHAPES = [(4096, 4096), (14336, 4096), (4096, 14336), (128256, 4096)]
BATCHES = [1, 4, 16]
KINDS = ["int8", "fp8"]
POOL_BYTES = 1 << 30


def gemv_bytes(n, k, b):
    return n * k + 4 * n + 4 * b * k + 4 * b * n


def host_cores():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_baseline(seconds=10.0):
    """The oracle's OpenMP GEMV (a port of the reference GEMV structure with
    the reference dequantisation) on a bounded sample: INT8 14336x4096, B=1."""
    import numpy as np
    from oracle_bind import Oracle

    orc = Oracle()
    cores = min(16, host_cores())
    rng = np.random.default_rng(1)
    n, k = 14336, 4096
    wq = rng.integers(-127, 128, (n, k), dtype=np.int8)
    ws = rng.uniform(0.005, 0.02, n).astype(np.float32)
    x = rng.standard_normal((1, k)).astype(np.float32)
    orc.gemv(wq, ws, x, "int8", threads=cores)       # warm-up
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end and len(times) < 500:
        t0 = time.perf_counter()
        orc.gemv(wq, ws, x, "int8", threads=cores)
        times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
    return {"value": round(gemv_bytes(n, k, 1) / med / 1e9, 2), "unit": "GB/s", "cores": cores,
            "kind": "port",
            "sample": f"oracle or_gemv_q8 INT8 {n}x{k} batch 1, OpenMP {cores} threads, "
                      f"median of {len(times)} runs over {seconds:.0f} s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              f"(the multi-GPU design is described in DESIGN.md)", file=sys.stderr)
        sys.exit(2)

    import torch
    import be42

    lib = be42.load()
    lib.init(0)
    dev = torch.device("cuda:0")
    torch.manual_seed(0)

    # ---- data: rotated weight pools per (kind, shape) -------------------------
    configs = []
    for kind in KINDS:
        for (n, k) in SHAPES:
            copies = max(2, min(64, -(-POOL_BYTES // (n * k))))
            w32 = torch.randn(n, k, device=dev) * 0.02
            q0, s0 = lib.quant_rows_int8(w32) if kind == "int8" else lib.quant_rows_fp8(w32)
            del w32
            pool = [q0] + [q0.roll(shifts=i * 7, dims=1).contiguous() for i in range(1, copies)]
            for b in BATCHES:
                x = torch.randn(b, k, device=dev)
                xdig = lib.gemv_prepare(x, kind)
                y = torch.empty(b, n, device=dev)
                configs.append(dict(kind=kind, n=n, k=k, b=b, pool=pool, s=s0, x=x, xdig=xdig, y=y, i=0))
    torch.cuda.synchronize()

    def run_step(ev=None):
        for ci, c in enumerate(configs):
            w = c["pool"][c["i"] % len(c["pool"])]
            c["i"] += 1
            if ev is not None:
                ev[ci][0].record()
            lib.gemv_prepare(c["x"], c["kind"], buf=c["xdig"])
            if ev is not None:
                ev[ci][1].record()
            lib.gemv_prepared(w, c["s"], c["xdig"], c["b"], c["kind"], c["y"])
            if ev is not None:
                ev[ci][2].record()

    for _ in range(args.warmup):
        run_step()
    torch.cuda.synchronize()

    evs = [[[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in configs]
           for _ in range(args.steps)]
    t0 = time.perf_counter()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for s in range(args.steps):
        run_step(evs[s])
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    total_ms = start.elapsed_time(stop)

    step_bytes = sum(gemv_bytes(c["n"], c["k"], c["b"]) for c in configs)
    ms_per_step = total_ms / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    sweep = []
    dominant = None
    for ci, c in enumerate(configs):
        op_ms = sum(evs[s][ci][0].elapsed_time(evs[s][ci][2]) for s in range(args.steps)) / args.steps
        main_ms = sum(evs[s][ci][1].elapsed_time(evs[s][ci][2]) for s in range(args.steps)) / args.steps
        nb = gemv_bytes(c["n"], c["k"], c["b"])
        row = {"dtype": c["kind"], "n": c["n"], "k": c["k"], "batch": c["b"],
               "op_us": round(op_ms * 1e3, 2), "kernel_us": round(main_ms * 1e3, 2),
               "op_GBps": round(nb / (op_ms * 1e-3) / 1e9, 1),
               "kernel_GBps": round(nb / (main_ms * 1e-3) / 1e9, 1)}
        sweep.append(row)
        if dominant is None or main_ms > dominant[0]:
            dominant = (main_ms, c, nb)

    dm, dc, dnb = dominant
    achieved = dnb / (dm * 1e-3) / 1e9
    kname = "be42::k_gemv<%s, RT=%d>" % ("fp8" if dc["kind"] == "fp8" else "int8", 1 if dc["b"] <= 4 else 2)
    out = {
        "metric": "decode tokens/s; quant GEMV HBM GB/s (% of peak); LSH attn µs/token @32k",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8/fp8 weights, fp32 activations",
        "data": "synthetic",
        "config": {"workload": "configs[1]: quantized GEMV sweep, INT8+FP8 per-row weights, "
                               "shapes 4096x4096/14336x4096/4096x14336/128256x4096, batch 1/4/16",
                   "pool_bytes_per_shape": POOL_BYTES, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": kname,
                     "workload": f"{dc['kind']} {dc['n']}x{dc['k']} batch {dc['b']}",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "bytes_per_launch": dnb},
        "gemv_sweep": sweep,
        "wall_s": round(wall, 2),
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
