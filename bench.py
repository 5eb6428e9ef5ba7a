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


# ---- LSH sparse attention ------------------------
LSH = dict(heads=32, kv_heads=8, head_dim=128, page=16, ctx=32768, k_sel=64, cap=64, planted=0.05)
LSH_BATCHES = [1, 16, 64, 128]


def lsh_bytes(n_sel, n_cand, cfg=LSH):
    """Algorithmic bytes of one query step, all heads: selected pages' bf16
    K+V, candidate centroids, projection, q, out, bucket/chain metadata."""
    page_kv = cfg["page"] * cfg["kv_heads"] * cfg["head_dim"] * 2 * 2
    hd = cfg["head_dim"]
    return (n_sel * page_kv + n_cand * hd * 4 + hd * 16 * 4 + cfg["heads"] * hd * 4 * 2
            + 4 * (17 + n_cand))


def plant_keys(K, q, rng, cfg=LSH):
    """5% of the pages (never the first or last) get keys 6*unit(q_mean) +
    N(0, 0.05^2) on every KV head."""
    import numpy as np
    hd, P = cfg["head_dim"], cfg["page"]
    npg = K.shape[0] // P
    qm = q.reshape(cfg["heads"], hd).astype(np.float64).mean(0)
    u = (6.0 * qm / np.linalg.norm(qm)).astype(np.float32)
    pages = rng.choice(np.arange(1, npg - 1), size=int(round(cfg["planted"] * npg)), replace=False)
    for pg in pages:
        for h in range(cfg["kv_heads"]):
            K[pg * P:(pg + 1) * P, h * hd:(h + 1) * hd] = u + 0.05 * rng.standard_normal((P, hd)).astype(np.float32)
    return pages


def plant_keys_gpu(K, q, gen, cfg=LSH):
    """plant_keys on the device: K is a (T, kv_heads * head_dim) cuda tensor."""
    import numpy as np
    import torch
    hd, P, KVH = cfg["head_dim"], cfg["page"], cfg["kv_heads"]
    T = K.shape[0]
    npg = T // P
    qm = q.reshape(cfg["heads"], hd).astype(np.float64).mean(0)
    u = torch.from_numpy((6.0 * qm / np.linalg.norm(qm)).astype(np.float32)).to(K.device)
    n = int(round(cfg["planted"] * npg))
    pages = torch.randperm(npg - 2, generator=gen, device=K.device)[:n] + 1
    rows = (pages[:, None] * P + torch.arange(P, device=K.device)).reshape(-1)
    noise = torch.randn(rows.numel(), KVH, hd, generator=gen, device=K.device) * 0.05
    K.view(T, KVH, hd)[rows] = u + noise


def lsh_bench(lib, steps, warmup, batches=LSH_BATCHES):
    """Route + sparse attention over the first B sequences of one pool, for
    each B in `batches`; every sequence is a 32k-token bf16 context."""
    import numpy as np
    import torch
    cfg = LSH
    H, KVH, hd, T = cfg["heads"], cfg["kv_heads"], cfg["head_dim"], cfg["ctx"]
    BM = max(batches)
    _, hpT = lib.lsh_projection(hd, 42)
    pool = lib.kv_pool(1, BM, KVH, hd, T // cfg["page"] + 1, hpT)
    rng = np.random.default_rng(4)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(4)
    q = rng.standard_normal((BM, H, hd)).astype(np.float32)
    for b in range(BM):
        K = torch.randn(T, KVH * hd, generator=gen, device="cuda")
        plant_keys_gpu(K, q[b], gen)
        V = torch.randn(T, KVH * hd, generator=gen, device="cuda")
        pool.append(b, K, V, 0)
        del K, V
    torch.cuda.synchronize()
    qall = torch.from_numpy(q).cuda()
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    sel_stride = 64
    n_split = 1        # <= 64 pages: the single fused kernel
    rows = []
    for B in batches:
        qd = qall[:B].contiguous()
        sel = torch.empty((B, sel_stride), dtype=torch.int32, device="cuda")
        nsel = torch.empty(B, dtype=torch.int32, device="cuda")
        cand = torch.empty((B, cfg["cap"]), dtype=torch.int32, device="cuda")
        ncand = torch.empty(B, dtype=torch.int32, device="cuda")
        out = torch.empty((B, H, hd), device="cuda")
        ws = torch.empty(max(1, lib.lib.be42_attn_workspace_bytes(B, H, hd, cfg["k_sel"], n_split)),
                         dtype=torch.uint8, device="cuda")

        def step(ev=None):
            if ev is not None:
                ev[0].record()
            lib._call("be42_lsh_route", pool.handle, lib.p(qd), None, B, H, cfg["k_sel"], cfg["cap"], lib.p(sel),
                      lib.p(nsel), sel_stride, lib.p(cand), lib.p(ncand), None, lib.stream())
            if ev is not None:
                ev[1].record()
            lib.paged_attention(pool, qd, sel, nsel, cfg["k_sel"], scale, n_split=n_split, out=out, workspace=ws)
            if ev is not None:
                ev[2].record()

        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
        for i in range(steps):
            step(evs[i])
        torch.cuda.synchronize()
        route_ms = sum(e[0].elapsed_time(e[1]) for e in evs) / steps
        attn_ms = sum(e[1].elapsed_time(e[2]) for e in evs) / steps
        tot_ms = sum(e[0].elapsed_time(e[2]) for e in evs) / steps
        ns = nsel.cpu().numpy()
        nc = ncand.cpu().numpy()
        nbytes = sum(lsh_bytes(int(a), int(c)) for a, c in zip(ns, nc))
        kv_bytes = sum(int(a) * cfg["page"] * KVH * hd * 2 * 2 for a in ns)
        rows.append({"batch": B, "us_per_token": round(tot_ms * 1e3 / B, 3), "step_us": round(tot_ms * 1e3, 2),
                     "route_us": round(route_ms * 1e3, 2), "attention_us": round(attn_ms * 1e3, 2),
                     "n_sel_mean": float(ns.mean()), "n_cand_mean": float(nc.mean()),
                     "bytes_per_step": nbytes, "GBps": round(nbytes / (tot_ms * 1e-3) / 1e9, 1),
                     "frac_of_hbm_peak": round(nbytes / (tot_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "attention_GBps": round(kv_bytes / (attn_ms * 1e-3) / 1e9, 1)})
    pool.close()
    head = max(rows, key=lambda r: r["batch"])
    return {"workload": f"configs[3]: B sequences x {T}-token bf16 paged KV (page 16), {H} heads / {KVH} KV heads, "
                        f"head_dim {hd}, top-K {cfg['k_sel']} pages, candidate cap {cfg['cap']}, 5% planted pages; "
                        f"one step = route + sparse attention of one decode token per sequence",
            "us_per_token": head["us_per_token"], "batch": head["batch"],
            "frac_of_hbm_peak": head["frac_of_hbm_peak"], "by_batch": rows}


# ---- prefill GEMM ---------------------------------
GEMM_M = [512, 2048, 8192]
MFMA_PEAK_TOPS = {"int8": 5000.0, "fp8": 5000.0}     # dense, MI355X datasheet


def gemm_bench(lib, steps, warmup):
    """M tokens in {512, 2048, 8192} x the GEMV (N, K) shapes,
    INT8 x INT8 (per-token activations, per-row weights, int32 accumulate)
    and FP8 x FP8 (fp32 accumulate); inputs N(0,1) with 1% outliers at +-8."""
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    rows = []
    for kind in KINDS:
        qf = lib.quant_rows_int8 if kind == "int8" else lib.quant_rows_fp8
        for (n, k) in SHAPES:
            wq, sw = qf(torch.randn(n, k, generator=g, device="cuda") * 0.02)
            for m in GEMM_M:
                x = torch.randn(m, k, generator=g, device="cuda")
                mask = torch.rand(m, k, generator=g, device="cuda") < 0.01
                x[mask] = torch.where(torch.rand(int(mask.sum()), generator=g, device="cuda") < 0.5, -8.0, 8.0)
                xq, sx = qf(x)
                del x, mask
                y = torch.empty(m, n, device="cuda")
                for _ in range(warmup):
                    lib.gemm(xq, sx, wq, sw, kind, out=y)
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(steps):
                    lib.gemm(xq, sx, wq, sw, kind, out=y)
                e1.record()
                torch.cuda.synchronize()
                ms = e0.elapsed_time(e1) / steps
                tops = 2.0 * m * n * k / (ms * 1e-3) / 1e12
                rows.append({"kind": kind, "m": m, "n": n, "k": k, "us": round(ms * 1e3, 1),
                             "TOPS": round(tops, 1), "frac_of_mfma_peak": round(tops / MFMA_PEAK_TOPS[kind], 4)})
                del xq, sx, y
            del wq, sw
            torch.cuda.empty_cache()
    tot_ops = sum(2.0 * r["m"] * r["n"] * r["k"] for r in rows)
    tot_s = sum(r["us"] for r in rows) * 1e-6
    best = max(rows, key=lambda r: r["TOPS"])
    return {"workload": "configs[2]: M in {512,2048,8192} x (N,K) in {4096x4096, 14336x4096, 4096x14336, "
                        "128256x4096}, INT8xINT8 and FP8xFP8 per-token x per-row scaled",
            "TOPS_aggregate": round(tot_ops / tot_s / 1e12, 1), "best": best, "by_shape": rows}


def lsh_cpu_baseline(seconds=10.0):
    """The oracle (port of the reference route + paged sparse attention, bf16
    pages) on one 32k-token sequence of the configs[3] workload."""
    import numpy as np
    from oracle_bind import OR_KV_BF16, Oracle, OracleIndex, OraclePaged
    cfg = LSH
    orc = Oracle()
    cores = min(16, host_cores())
    H, KVH, hd, T, P = cfg["heads"], cfg["kv_heads"], cfg["head_dim"], cfg["ctx"], cfg["page"]
    rng = np.random.default_rng(5)
    _, hpT = orc.lsh_init(hd, 42)
    q = rng.standard_normal((H, hd)).astype(np.float32)
    K = rng.standard_normal((T, KVH * hd)).astype(np.float32)
    V = rng.standard_normal((T, KVH * hd)).astype(np.float32)
    plant_keys(K, q, rng)
    pk = OraclePaged(orc, 1, KVH, hd, T // P + 1, OR_KV_BF16)
    ix = OracleIndex(orc, T // P + 1)
    for t in range(T):
        pk.append(0, K[t], V[t], t)
        if t % P == P - 1:
            ix.insert(orc.lsh_hash(hpT, pk.page_arrays(pk.phys(0, t // P))[4]), t - P + 1, P)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end and len(times) < 2000:
        t0 = time.perf_counter()
        sel, _ = pk.route(0, q, H, hpT, ix, cfg["cap"], cfg["k_sel"])
        pk.attention_pages(q, sel, H, scale, threads=cores)
        times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
    return {"value": round(med * 1e6, 1), "unit": "us/token", "cores": cores, "kind": "port",
            "sample": f"oracle or_route_pages + or_paged_attention_pages (bf16 pages), one {T}-token sequence, "
                      f"OpenMP {cores} threads over heads, median of {len(times)} runs"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-lsh", action="store_true", help="skip the LSH attention leg")
    ap.add_argument("--no-gemm", action="store_true", help="skip the prefill GEMM leg")
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
    if not args.no_gemm:
        configs.clear()
        torch.cuda.empty_cache()
        out["prefill_gemm"] = gemm_bench(lib, 5, 1)
    if not args.no_lsh:
        # free the GEMV pools first
        configs.clear()
        torch.cuda.empty_cache()
        out["lsh_attention"] = lsh_bench(lib, max(args.steps, 10), max(args.warmup, 2))
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline()
        if not args.no_lsh:
            out["lsh_attention"]["cpu_baseline"] = lsh_cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
