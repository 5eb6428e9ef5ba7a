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


def cpu_threads():
    """Threads for the CPU baselines: every CPU this job is granted.  A GPU
    box grants each GPU's job a share of the host and states it in
    OMP_NUM_THREADS (16 per GPU); without it, every CPU the process may run
    on."""
    avail = host_cores()
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        return min(int(env), avail)
    return avail


def host_info():
    """The host the CPU baselines ran on: model, sockets, logical CPUs, and
    the job's CPU grant (cgroup cpu.max, OMP_NUM_THREADS)."""
    model, sockets = None, set()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name") and model is None:
                model = line.split(":", 1)[1].strip()
            elif line.startswith("physical id"):
                sockets.add(line.split(":", 1)[1].strip())
    except OSError:
        pass
    quota = None
    try:
        quota = open("/sys/fs/cgroup/cpu.max").read().strip()
    except OSError:
        pass
    return {"cpu_model": model, "sockets": len(sockets) or None, "logical_cpus": os.cpu_count(),
            "affinity_cpus": host_cores(), "cgroup_cpu_max": quota,
            "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS")}


def cpu_baseline(seconds=10.0):
    """The oracle's OpenMP GEMV (a port of the reference GEMV structure with
    the reference dequantisation) on a bounded sample: INT8 14336x4096, B=1."""
    import numpy as np
    from oracle_bind import Oracle

    orc = Oracle()
    cores = cpu_threads()
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


def cpu_baseline_reference(seconds=10.0):
    """The reference's own decode GEMV: op_matmul (ops_matmul.c:366) with BF16
    weights and an fp32 column, i.e. matvec_bf16_f32_blocked (:57-153, AVX2
    + OpenMP), compiled from the reference sources by oracle/Makefile into
    oracle/_ref/libref42.so; 14336x4096 at batch 1 on a bounded sample.  The
    reference has no INT8/FP8 GEMV, so its bytes are 2 per weight."""
    import ctypes as C
    import numpy as np
    from oracle_bind import REF_SO, RefLib

    if not os.path.exists(REF_SO):
        return None
    ref = RefLib()
    cores = cpu_threads()
    rng = np.random.default_rng(2)
    n, k = 14336, 4096
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    wb = (w.view(np.uint32) >> 16).astype(np.uint16)          # bf16 codes (truncated)
    x = rng.standard_normal((k, 1)).astype(np.float32)
    y = np.zeros((n, 1), np.float32)
    call = lambda: ref.lib.ref_matmul(y.ctypes.data, 0, wb.ctypes.data, 1, n, k, x.ctypes.data, 0, 1)  # noqa: E731
    os.environ.setdefault("OMP_NUM_THREADS", str(cores))
    if call() != 0:
        return None
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end and len(times) < 500:
        t0 = time.perf_counter()
        call()
        times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
    nbytes = 2 * n * k + 4 * k + 4 * n
    return {"value": round(nbytes / med / 1e9, 2), "unit": "GB/s", "cores": cores, "kind": "reference",
            "sample": f"reference op_matmul BF16 {n}x{k} x fp32 column (matvec_bf16_f32_blocked, AVX2 + OpenMP, "
                      f"{cores} threads, built -O3 -march=x86-64-v3), median of {len(times)} runs over "
                      f"{seconds:.0f} s; GB/s of bf16 weight bytes"}


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
    return pages


def lsh_bench(lib, steps, warmup, batches=LSH_BATCHES, ctx=None):
    """Route + sparse attention over the first B sequences of one pool, for
    each B in `batches`; every sequence is a ctx-token bf16 context (32k
    unless given)."""
    import numpy as np
    import torch
    cfg = dict(LSH, ctx=ctx or LSH["ctx"])
    H, KVH, hd, T = cfg["heads"], cfg["kv_heads"], cfg["head_dim"], cfg["ctx"]
    BM = max(batches)
    _, hpT = lib.lsh_projection(hd, 42)
    pool = lib.kv_pool(1, BM, KVH, hd, T // cfg["page"] + 1, hpT)
    rng = np.random.default_rng(4)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(4)
    q = rng.standard_normal((BM, H, hd)).astype(np.float32)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    P, G, npg = cfg["page"], H // KVH, T // cfg["page"]
    exact_top, planted, page_mass = [], [], []
    for b in range(BM):
        K = torch.randn(T, KVH * hd, generator=gen, device="cuda")
        planted.append(set(plant_keys_gpu(K, q[b], gen, cfg).tolist()))
        V = torch.randn(T, KVH * hd, generator=gen, device="cuda")
        pool.append(b, K, V, 0)
        # the selection over every page: the anchors (first, last) and the
        # k-2 best middle pages by q head 0 . head-0 centroid (what
        # score_blocks + select_top_k_blocks rank, over all pages)
        cs = K.view(npg, P, KVH, hd)[:, :, 0, :].bfloat16().float().mean(1) @ torch.from_numpy(q[b, 0]).cuda()
        mid = torch.topk(cs[1:npg - 1], cfg["k_sel"] - 2).indices + 1
        exact_top.append(set(mid.tolist()) | {0, npg - 1})
        # dense softmax mass per page, averaged over heads
        qb = torch.from_numpy(q[b]).cuda().view(KVH, G, hd).transpose(1, 2).contiguous()
        lg = torch.bmm(K.view(T, KVH, hd).transpose(0, 1).contiguous(), qb) * scale
        page_mass.append(torch.softmax(lg, dim=1).view(KVH, npg, P, G).sum(2).mean(dim=(0, 2)).cpu().numpy())
        del K, V, lg
    torch.cuda.synchronize()
    phys_to_logical = []
    for b in range(BM):
        m = {}
        for j, ph in enumerate(pool.layer_pages(b)):
            m[int(ph)] = j
        phys_to_logical.append(m)
    qall = torch.from_numpy(q).cuda()
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

        def step_split(ev=None):
            if ev is not None:
                ev[0].record()
            lib._call("be42_lsh_route", pool.handle, lib.p(qd), None, B, H, cfg["k_sel"], cfg["cap"], lib.p(sel),
                      lib.p(nsel), sel_stride, lib.p(cand), lib.p(ncand), None, lib.stream())
            if ev is not None:
                ev[1].record()
            lib.paged_attention(pool, qd, sel, nsel, cfg["k_sel"], scale, n_split=n_split, out=out, workspace=ws)
            if ev is not None:
                ev[2].record()

        fsel = torch.empty((B, sel_stride), dtype=torch.int32, device="cuda")
        fnsel = torch.empty(B, dtype=torch.int32, device="cuda")
        fout = torch.empty((B, H, hd), device="cuda")

        def step_fused():
            lib._call("be42_lsh_attention", pool.handle, lib.p(qd), None, B, H, cfg["k_sel"], cfg["cap"], scale,
                      lib.p(fout), lib.p(fsel), lib.p(fnsel), sel_stride, lib.stream())

        for _ in range(warmup):
            step_split()
            step_fused()
        torch.cuda.synchronize()
        # the decode path: route + attention in one launch
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(steps):
            step_fused()
        e1.record()
        torch.cuda.synchronize()
        tot_ms = e0.elapsed_time(e1) / steps
        # breakdown: the same work as two launches (router, then attention)
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
        for i in range(steps):
            step_split(evs[i])
        torch.cuda.synchronize()
        route_ms = sum(e[0].elapsed_time(e[1]) for e in evs) / steps
        attn_ms = sum(e[1].elapsed_time(e[2]) for e in evs) / steps
        split_ms = sum(e[0].elapsed_time(e[2]) for e in evs) / steps
        ns = fnsel.cpu().numpy()
        assert torch.equal(fnsel, nsel) and all(
            torch.equal(fsel[b, :ns[b]], sel[b, :ns[b]]) for b in range(B)), "fused and two-launch selections differ"
        nc = ncand.cpu().numpy()
        # recall of the LSH route against the same selection over every
        # page (lsh_validate_recall's hits / k, ops_lsh.c:587, with the
        # paged path's own ranking), the planted pages it found, and the
        # share of the dense softmax mass the selected pages hold
        fs = fsel.cpu().numpy()
        rec, found, held = [], [], []
        for b in range(B):
            got = {phys_to_logical[b][int(x)] for x in fs[b, :ns[b]]}
            rec.append(len(got & exact_top[b]) / cfg["k_sel"])
            found.append(len(got & planted[b]) / min(cfg["k_sel"] - 2, len(planted[b])))
            held.append(float(page_mass[b][sorted(got)].sum()))
        nbytes = sum(lsh_bytes(int(a), int(c), cfg) for a, c in zip(ns, nc))
        kv_bytes = sum(int(a) * cfg["page"] * KVH * hd * 2 * 2 for a in ns)
        rows.append({"batch": B, "us_per_token": round(tot_ms * 1e3 / B, 3), "step_us": round(tot_ms * 1e3, 2),
                     "two_launch_us": round(split_ms * 1e3, 2), "route_us": round(route_ms * 1e3, 2),
                     "attention_us": round(attn_ms * 1e3, 2),
                     "n_sel_mean": float(ns.mean()), "n_cand_mean": float(nc.mean()),
                     "bytes_per_step": nbytes, "GBps": round(nbytes / (tot_ms * 1e-3) / 1e9, 1),
                     "frac_of_hbm_peak": round(nbytes / (tot_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "attention_GBps": round(kv_bytes / (attn_ms * 1e-3) / 1e9, 1),
                     "recall_at_k": round(float(np.mean(rec)), 4), "planted_found": round(float(np.mean(found)), 4),
                     "attention_mass_held": round(float(np.mean(held)), 4)})
    pool.close()
    head = max(rows, key=lambda r: r["frac_of_hbm_peak"])
    launch_bytes = head["bytes_per_step"]
    achieved = launch_bytes / (head["step_us"] * 1e-6) / 1e9
    # be42_lsh_attention's dispatch: up to 64 (query, KV head) pairs the split
    # launch, below 1024 the fused route + attention, from 1024 the router's
    # own launch and then the fused attention
    pairs = head["batch"] * KVH
    kname = ("be42::k_lsh_attn_split (route + sparse attention, one launch)" if pairs <= 64 else
             "be42::k_lsh_attn (route + sparse attention, one launch)" if pairs < 1024 else
             "be42::k_route + be42::k_attn_fused (route, then sparse attention: two launches)")
    roof = {"bound": "hbm", "kernel": kname,
            "workload": f"batch {head['batch']}, {T}-token bf16 context",
            "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": lsh_traffic(head["batch"]) if T == LSH["ctx"] else None,
            "bytes_per_launch": launch_bytes, "launch_us": head["step_us"]}
    return {"roofline": roof,
            "recall_definition": "recall_at_k: share of the k pages the same ranking selects over every page "
                                 "(anchors + best middle pages by q head 0 . head-0 centroid) that the LSH route "
                                 "selects; planted_found: planted pages selected / min(k-2, planted); "
                                 "attention_mass_held: dense softmax mass of the selected pages, averaged over heads",
            "workload": f"configs[3]: B sequences x {T}-token bf16 paged KV (page 16), {H} heads / {KVH} KV heads, "
                        f"head_dim {hd}, top-K {cfg['k_sel']} pages, candidate cap {cfg['cap']}, 5% planted pages; "
                        f"one step = route + sparse attention of one decode token per sequence "
                        f"(be42_lsh_attention: one launch below 1024 query x KV-head pairs, from 1024 the "
                        f"router's own launch then the attention; route_us / attention_us time the work as "
                        f"be42_lsh_route + be42_paged_attention)",
            "us_per_token": head["us_per_token"], "batch": head["batch"], "recall_at_k": head["recall_at_k"],
            "frac_of_hbm_peak": head["frac_of_hbm_peak"], "by_batch": rows}


# ---- prefill GEMM ---------------------------------
GEMM_M = [512, 2048, 8192]
MFMA_PEAK_TOPS = {"int8": 5000.0, "fp8": 5000.0}     # dense, MI355X datasheet


def vendor_gemm_us(xq, wq, kind, steps, warmup):
    """The same product through ROCm's hipBLASLt, as torch exposes it, for
    comparison: FP8 codes (E4M3) by torch._scaled_mm with unit scalar scales
    and an fp32 output, INT8 by torch._int_mm with an int32 output (neither
    applies the per-token / per-row scales this library's epilogue does).
    Microseconds per call, or None where torch refuses the call."""
    import torch
    try:
        if kind == "fp8":
            a, b = xq.view(torch.float8_e4m3fn), wq.view(torch.float8_e4m3fn).t()
            one = torch.ones((), device="cuda")
            fn = lambda: torch._scaled_mm(a, b, scale_a=one, scale_b=one, out_dtype=torch.float32)
        else:
            a, b = xq, wq.t()
            fn = lambda: torch._int_mm(a, b)
        for _ in range(warmup):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return round(e0.elapsed_time(e1) / steps * 1e3, 1)
    except Exception:
        torch.cuda.synchronize()
        return None


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
                vend = vendor_gemm_us(xq, wq, kind, steps, warmup)
                rows.append({"kind": kind, "m": m, "n": n, "k": k, "us": round(ms * 1e3, 1),
                             "TOPS": round(tops, 1), "frac_of_mfma_peak": round(tops / MFMA_PEAK_TOPS[kind], 4),
                             "hipblaslt_us": vend, "hipblaslt_over_ours": round(vend / (ms * 1e3), 3) if vend else None})
                del xq, sx, y
            del wq, sw
            torch.cuda.empty_cache()
    tot_ops = sum(2.0 * r["m"] * r["n"] * r["k"] for r in rows)
    tot_s = sum(r["us"] for r in rows) * 1e-6
    best = max(rows, key=lambda r: r["TOPS"])
    traffic = None
    summ = os.path.join(ROOT, "profiles", "gemm_fp8_8192x4096x14336_and_int8_512x4096x4096_counters.txt")
    tag = f"traffic_bytes_per_launch[{best['kind']} {best['m']}x{best['n']}x{best['k']}]"
    if os.path.exists(summ):
        for line in open(summ):
            if line.startswith(tag):
                traffic = int(line.split("=")[1].split()[0])
    roof = {"bound": "mfma", "kernel": "be42::k_gemm_dma", "workload": f"{best['kind']} M={best['m']} "
            f"N={best['n']} K={best['k']}", "achieved": best["TOPS"], "peak": MFMA_PEAK_TOPS[best["kind"]],
            "unit": "TFLOP/s", "frac": best["frac_of_mfma_peak"], "traffic": traffic,
            "ops_per_launch": 2 * best["m"] * best["n"] * best["k"], "launch_us": best["us"]}
    return {"roofline": roof, "workload": "configs[2]: M in {512,2048,8192} x (N,K) in {4096x4096, 14336x4096, 4096x14336, "
                        "128256x4096}, INT8xINT8 and FP8xFP8 per-token x per-row scaled",
            "TOPS_aggregate": round(tot_ops / tot_s / 1e12, 1), "best": best, "by_shape": rows,
            "hipblaslt_note": "hipblaslt_us: the same codes through torch._scaled_mm (FP8, unit scales, fp32 out) "
                              "and torch._int_mm (INT8, int32 out) on the same GPU; hipblaslt_over_ours > 1: this "
                              "library is faster",
            "digit_gemm": digit_gemm_bench(lib, steps, warmup)}


def digit_gemm_bench(lib, steps, warmup):
    """The prefill's projections: fp32 activations (N(0,1)) as digit planes
    against per-row INT8 / FP8 weights, at the 3B model's layer shapes for a
    1024-token pass (q/k/v and gate/up as one multi-segment launch).  The
    matrix cores run nd = 3 (INT8) or 4 (FP8) digit products per logical
    multiply-add: 'TOPS' counts 2 M N K nd, 'logical_TOPS' 2 M N K."""
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(12)
    m = 1024
    d, F, kvd = B3["dim"], B3["hidden_dim"], B3["n_kv_heads"] * B3["head_dim"]
    shapes = [("qkv", [d, kvd, kvd], d), ("o", [d], d), ("gate_up", [F, F], d), ("down", [d], F)]
    rows = []
    for kind in KINDS:
        nd = 3 if kind == "int8" else 4
        qf = lib.quant_rows_int8 if kind == "int8" else lib.quant_rows_fp8
        for name, ns, k in shapes:
            segs = [qf(torch.randn(n, k, generator=g, device="cuda") * 0.02) for n in ns]
            x = torch.randn(m, k, generator=g, device="cuda")
            for _ in range(warmup):
                lib.gemm_f32_multi(x, segs, kind)
            torch.cuda.synchronize()
            # the digit split once, then the timed GEMM launches
            fp8 = 0 if kind == "int8" else 1
            buf = torch.empty(lib.lib.be42_gemm_xdig_bytes(k, m, fp8), dtype=torch.uint8, device="cuda")
            lib._call("be42_gemm_prepare", lib.p(buf), lib.p(x), k, m, fp8, lib.stream())
            import ctypes as C
            import be42
            outs = [torch.empty((m, w.shape[0]), device="cuda") for w, _ in segs]
            arr = (be42.GemvSeg * len(segs))()
            for i, ((w, sw), y) in enumerate(zip(segs, outs)):
                arr[i] = be42.GemvSeg(lib.p(w), lib.p(sw), lib.p(y), w.shape[0])
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(steps):
                lib._call("be42_gemm_prepared_multi", C.addressof(arr), len(segs), lib.p(buf), k, m, fp8,
                          lib.stream())
            e1.record()
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / steps
            n = sum(ns)
            ops = 2.0 * m * n * k
            rows.append({"kind": kind, "proj": name, "m": m, "n": n, "k": k, "us": round(ms * 1e3, 1),
                         "TOPS": round(ops * nd / (ms * 1e-3) / 1e12, 1),
                         "logical_TOPS": round(ops / (ms * 1e-3) / 1e12, 1),
                         "frac_of_mfma_peak": round(ops * nd / (ms * 1e-3) / 1e12 / MFMA_PEAK_TOPS[kind], 4)})
            del segs, x, buf, outs
            torch.cuda.empty_cache()
    return {"workload": "prefill projections of configs[4] for a 1024-token pass: fp32 activations as digit planes "
                        "(INT8 3, FP8 4) x per-row INT8/FP8 weights, be42_gemm_prepared_multi",
            "by_shape": rows}


# ---- the drop-in boundary with host arrays (PCIe-inclusive) -----------------------
def dropin_bench(lib, calls=50):
    """op_matmul (ops_matmul.c:366) called the way the reference's forward
    pass calls it: t_tensor operands in host memory, b = x as [k][1].  The
    library mirrors a host weight once (the first call, timed apart as
    `first_call_ms`: the weight's PCIe upload); every later call stages x in
    and y out over PCIe and waits for the result, so `us_per_call` is the
    caller's wall time per GEMV and `GBps` counts the algorithmic weight bytes
    over it.  Reported beside the device-resident sweep; never `value`."""
    import ctypes as C
    import numpy as np

    class TTensor(C.Structure):           # be42_engine.h t_tensor (tensor.h:19-39)
        _fields_ = [("data", C.c_void_p), ("shape", C.c_int * 4), ("stride", C.c_int * 4), ("ndim", C.c_int),
                    ("size", C.c_size_t), ("dtype", C.c_int), ("row_scale", C.c_void_p)]

    def tt(a, dtype, rows, cols, scale=None):
        t = TTensor()
        t.data, t.ndim, t.size, t.dtype = a.ctypes.data, 2, rows * cols, dtype
        t.shape[0], t.shape[1], t.stride[0], t.stride[1] = rows, cols, cols, 1
        t.row_scale = scale.ctypes.data if scale is not None else None
        return t

    fn = lib.lib.op_matmul
    fn.restype = C.c_int
    fn.argtypes = [C.POINTER(TTensor)] * 3
    rng = np.random.default_rng(17)
    rows = []
    for kind, dt in (("int8", 2), ("fp8", 3)):
        for n, k in ((4096, 4096), (14336, 4096)):
            if kind == "int8":
                w = rng.integers(-127, 128, (n, k), dtype=np.int8)
            else:   # E4M3 codes without the NaN patterns (0x7F / 0xFF)
                w = rng.integers(0, 0x7F, (n, k), dtype=np.uint8) | (rng.integers(0, 2, (n, k), dtype=np.uint8) << 7)
            s = (rng.random(n, dtype=np.float32) * 0.015 + 0.005).astype(np.float32)
            x = rng.standard_normal((k, 1)).astype(np.float32)
            y = np.zeros((n, 1), np.float32)
            ta, tb, to = tt(w, dt, n, k, s), tt(x, 0, k, 1), tt(y, 0, n, 1)
            t0 = time.perf_counter()
            if fn(C.byref(to), C.byref(ta), C.byref(tb)) != 0:
                raise RuntimeError(f"op_matmul {kind} {n}x{k} failed")
            first = time.perf_counter() - t0
            for _ in range(3):
                fn(C.byref(to), C.byref(ta), C.byref(tb))
            t0 = time.perf_counter()
            for _ in range(calls):
                fn(C.byref(to), C.byref(ta), C.byref(tb))
            per = (time.perf_counter() - t0) / calls
            nb = gemv_bytes(n, k, 1)
            rows.append({"dtype": kind, "n": n, "k": k, "batch": 1, "first_call_ms": round(first * 1e3, 2),
                         "us_per_call": round(per * 1e6, 2), "GBps": round(nb / per / 1e9, 1)})
            del w, s, x, y
    return {"workload": "op_matmul with host t_tensor operands (weights mirrored once, x / y staged over PCIe "
                        "each call), configs[1] shapes 4096x4096 and 14336x4096, batch 1",
            "calls": calls, "by_shape": rows}


# ---- decode step -----------------------
TINY = dict(n_layers=4, dim=512, n_heads=8, n_kv_heads=8, head_dim=64, hidden_dim=1408, vocab=4096)
B3 = dict(n_layers=28, dim=3072, n_heads=24, n_kv_heads=8, head_dim=128, hidden_dim=8192, vocab=128256)
B3_CTX = 32768


def decoder_weights(lib, arch, kind, gen):
    """Random-init weights on the device: INT8 codes U{-127..127} with row
    scales U[0.005, 0.02], or N(0, 0.02) weights quantized to FP8
    E4M3 per row; RMSNorm weights 1.0 (bf16)."""
    import torch
    dev = "cuda"

    def mat(r, c):
        if kind == "int8":
            q = torch.randint(-127, 128, (r, c), dtype=torch.int8, device=dev, generator=gen)
            return q, torch.rand(r, device=dev, generator=gen) * 0.015 + 0.005
        w = torch.randn(r, c, device=dev, generator=gen) * 0.02
        q, sc = lib.quant_rows_fp8(w)
        del w
        return q, sc
    d, H, KV, hd, F, V = (arch[k] for k in ("dim", "n_heads", "n_kv_heads", "head_dim", "hidden_dim", "vocab"))
    one = torch.full((d,), 0x3F80, dtype=torch.int16, device=dev)
    layers = []
    for _ in range(arch["n_layers"]):
        L = {}
        for name, (r, c) in {"wq": (H * hd, d), "wk": (KV * hd, d), "wv": (KV * hd, d), "wo": (d, H * hd),
                             "w1": (F, d), "w3": (F, d), "w2": (d, F)}.items():
            L[name], L["s" + name[1:]] = mat(r, c)
        L["attn_norm"], L["ffn_norm"] = one, one
        layers.append(L)
    emb, emb_s = mat(V, d)
    out, out_s = mat(V, d)
    return dict(emb=emb, emb_s=emb_s, final_norm=one, out=out, out_s=out_s, layers=layers)


def weight_bytes(arch):
    """Weight bytes one decode step streams: every layer's 7 matrices and the
    lm_head (1 B per code + 4 B per row scale), plus one embedding row."""
    d, H, KV, hd, F, V = (arch[k] for k in ("dim", "n_heads", "n_kv_heads", "head_dim", "hidden_dim", "vocab"))
    rows_cols = [(H * hd, d), (KV * hd, d), (KV * hd, d), (d, H * hd), (F, d), (F, d), (d, F)]
    per_layer = sum(r * c + 4 * r for r, c in rows_cols)
    return arch["n_layers"] * per_layer + V * d + 4 * V + d


def decoder_cfg(arch, max_seq, max_batch, wkind, kv_kind, sparse_k=64, cand_cap=64):
    c = dict(arch)
    c.update(max_seq=max_seq, max_batch=max_batch, wkind=wkind, kv_kind=kv_kind, sparse_k=sparse_k,
             cand_cap=cand_cap, rope_len=0, rope_theta=1e4, norm_eps=1e-5)
    return c


def decode_tiny_bench(lib, n_gen=64, reps=3):
    """128-token prompt, then 64 greedy tokens, each step fed the
    previous step's device argmax (no host round trip); tokens/s over the 64."""
    import numpy as np
    import torch
    import be42
    gen = torch.Generator(device="cuda")
    gen.manual_seed(31)
    w = decoder_weights(lib, TINY, "int8", gen)
    _, hpT = lib.lsh_projection(TINY["head_dim"], 42)
    dec = be42.Decoder(lib, decoder_cfg(TINY, 256, 1, 0, be42.KV_INT8), w, hpT)
    prompt = np.random.default_rng(3).integers(0, TINY["vocab"], 128)
    best = best_pf = None
    for _ in range(reps):
        for l in range(TINY["n_layers"]):
            dec.pool.reset(l)
        torch.cuda.synchronize()
        # the prompt in one batched prefill call, then the greedy steps fed
        # from the device argmax the prefill left
        p0, p1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        p0.record()
        dec.prefill(prompt)
        p1.record()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for pos in range(128, 128 + n_gen):
            dec.step(None, pos, sync=False, batch=1)
        e1.record()
        torch.cuda.synchronize()
        ms, pf = e0.elapsed_time(e1), p0.elapsed_time(p1)
        best = ms if best is None else min(best, ms)
        best_pf = pf if best_pf is None else min(best_pf, pf)
    dec.close()
    wb = weight_bytes(TINY)
    return {"workload": "configs[0]: tiny Llama (4 layers, d 512, 8/8 heads, FFN 1408, vocab 4096), INT8 row-scaled "
                        "weights, 128-token prompt (one be42_decoder_prefill call), 64 greedy tokens, dense paged "
                        "INT8 attention, batch 1",
            "tokens_per_s": round(n_gen / (best * 1e-3), 1), "ms_per_token": round(best / n_gen, 4),
            "weight_bytes_per_token": wb, "weight_GBps": round(wb * n_gen / (best * 1e-3) / 1e9, 1),
            "prefill_ms": round(best_pf, 3), "prefill_tokens_per_s": round(128 / (best_pf * 1e-3), 1)}


def decode_3b_bench(lib, batches=(1, 8), steps=10):
    """3B-class model, FP8 weights, LSH sparse attention (top-K 64
    pages, candidate cap 64) over a 32k-token bf16 paged KV prefix per
    sequence.  The prefix is N(0,1) K/V with the configs[3] planting: layer by
    layer, a probe step at position 32768 captures the layer's queries and the
    layer's prefix is rebuilt with 5% of its pages planted along their mean.
    A timed step is one full decode step at position 32768 (re-running the
    position overwrites its K/V), so every step routes to the planted pages."""
    import numpy as np
    import torch
    import be42
    gen = torch.Generator(device="cuda")
    gen.manual_seed(41)
    A = B3
    BM = max(batches)
    L, H, KVH, hd = A["n_layers"], A["n_heads"], A["n_kv_heads"], A["head_dim"]
    w = decoder_weights(lib, A, "fp8", gen)
    _, hpT = lib.lsh_projection(hd, 42)
    cfg = decoder_cfg(A, B3_CTX + 64, BM, 1, be42.KV_BF16)
    dec = be42.Decoder(lib, cfg, w, hpT)
    T = B3_CTX
    tok0 = np.random.default_rng(5).integers(0, A["vocab"], BM)
    lsh_cfg = dict(LSH, heads=H, kv_heads=KVH, head_dim=hd)

    def build(slot, q=None):
        dec.pool.reset(slot)
        for t0 in range(0, T, 8192):
            n = min(8192, T - t0)
            K = torch.randn(n, KVH * hd, generator=gen, device="cuda")
            V = torch.randn(n, KVH * hd, generator=gen, device="cuda")
            if q is not None:
                plant_keys_gpu(K, q, gen, lsh_cfg)
            dec.pool.append(slot, K, V, t0)
            del K, V
    for l in range(L):
        for b in range(BM):
            build(l * BM + b)
    torch.cuda.synchronize()
    cq = torch.zeros((L, BM, H * hd), device="cuda")
    cn = torch.zeros((L, BM), dtype=torch.int32, device="cuda")
    dec.capture(cq, cn)
    for l in range(L):
        dec.step(tok0, T, sync=True)
        qs = cq[l].cpu().numpy()
        for b in range(BM):
            build(l * BM + b, qs[b])
    torch.cuda.synchronize()
    rows = []
    for B in batches:
        toks = tok0[:B]
        # one step that records the attended page counts, then the timed
        # steps without the inspection copies
        dec.capture(cq, cn)
        dec.step(toks, T, sync=True)
        nsel = cn[:, :B].cpu().numpy()
        dec.capture(None, None)
        for _ in range(2):
            dec.step(toks, T, sync=False)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            dec.step(toks, T, sync=False)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        kv_bytes = int(nsel.sum()) * 16 * KVH * hd * 2 * 2
        wb = weight_bytes(A)
        rows.append({"batch": B, "tokens_per_s": round(B / (ms * 1e-3), 1), "ms_per_step": round(ms, 3),
                     "pages_attended_mean": round(float(nsel.mean()), 2),
                     "step_bytes": wb + kv_bytes, "GBps": round((wb + kv_bytes) / (ms * 1e-3) / 1e9, 1),
                     "frac_of_hbm_peak": round((wb + kv_bytes) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
    dec.capture(None, None)
    # batched prefill of a fresh 4096-token prompt into sequence 0 (its
    # slots reset first): 4 passes of 1024 tokens, dense attention up to 64
    # pages and LSH-routed after
    n_pf = 4096
    prompt = np.random.default_rng(6).integers(0, A["vocab"], n_pf)
    pf_ms = []
    for _ in range(3):
        for l in range(L):
            dec.pool.reset(l * BM)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        dec.prefill(prompt)
        e1.record()
        torch.cuda.synchronize()
        pf_ms.append(e0.elapsed_time(e1))
    dec.close()
    pf = min(pf_ms)
    return {"workload": "configs[4]: 3B-class Llama (28 layers, d 3072, 24/8 heads, hd 128, FFN 8192, vocab "
                        "128256), FP8 E4M3 per-row weights, 32k-token bf16 paged KV prefix per sequence with "
                        "configs[3] planting, LSH sparse attention top-K 64 pages / candidate cap 64",
            "by_batch": rows,
            "prefill": {"tokens": n_pf, "ms": round(pf, 2), "tokens_per_s": round(n_pf / (pf * 1e-3), 1),
                        "us_per_token": round(pf * 1e3 / n_pf, 2),
                        "note": "be42_decoder_prefill: digit-plane MFMA GEMMs over 1024-token passes, each "
                                "token attending to the cache as of its position (bit-identical to token-by-"
                                "token decode for INT8 weights)"}}


def decode_cpu_baseline(seconds=10.0):
    """The oracle's transformer_forward (OpenMP GEMVs, paged INT8 attention)
    on configs[0]: tokens/s of greedy steps after a 128-token prompt."""
    import numpy as np
    from oracle_bind import OR_KV_INT8, Oracle, OracleDecoder
    orc = Oracle()
    cores = cpu_threads()
    rng = np.random.default_rng(31)
    A = TINY
    d, H, KV, hd, F, V = (A[k] for k in ("dim", "n_heads", "n_kv_heads", "head_dim", "hidden_dim", "vocab"))

    def q(r, c):
        return rng.integers(-127, 128, (r, c), dtype=np.int8), rng.uniform(0.005, 0.02, r).astype(np.float32)
    one = np.full(d, 0x3F80, np.uint16)
    layers = []
    for _ in range(A["n_layers"]):
        Lw = {}
        for name, (r, c) in {"wq": (H * hd, d), "wk": (KV * hd, d), "wv": (KV * hd, d), "wo": (d, H * hd),
                             "w1": (F, d), "w3": (F, d), "w2": (d, F)}.items():
            Lw[name], Lw["s" + name[1:]] = q(r, c)
        Lw["attn_norm"], Lw["ffn_norm"] = one, one
        layers.append(Lw)
    emb, emb_s = q(V, d)
    out, out_s = q(V, d)
    w = dict(emb=emb, emb_s=emb_s, final_norm=one, out=out, out_s=out_s, layers=layers)
    cfg = dict(n_layers=A["n_layers"], dim=d, n_heads=H, n_kv=KV, hd=hd, hidden=F, vocab=V, max_seq=4096, wkind=0,
               kv_kind=OR_KV_INT8, sparse_k=64, cand_cap=64, theta=1e4, eps=1e-5)
    _, hpT = orc.lsh_init(hd, 42)
    dec = OracleDecoder(orc, cfg, w, hpT)
    prompt = rng.integers(0, V, 128)
    for pos in range(128):
        nxt, _ = dec.step(prompt[pos], pos, threads=cores)
    times = []
    pos = 128
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end and pos < 1024:
        t0 = time.perf_counter()
        nxt, _ = dec.step(nxt, pos, threads=cores)
        times.append(time.perf_counter() - t0)
        pos += 1
    med = sorted(times)[len(times) // 2]
    return {"value": round(1.0 / med, 1), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"oracle or_decoder_step on configs[0] after a 128-token prompt, greedy, batch 1, OpenMP "
                      f"{cores} threads, median of {len(times)} steps"}


def lsh_cpu_baseline(seconds=10.0):
    """The oracle (port of the reference route + paged sparse attention, bf16
    pages) on one 32k-token sequence of the configs[3] workload."""
    import numpy as np
    from oracle_bind import OR_KV_BF16, Oracle, OracleIndex, OraclePaged
    cfg = LSH
    orc = Oracle()
    cores = cpu_threads()
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


def decode_3b_cpu_baseline(seconds=12.0):
    """The oracle's transformer_forward (OpenMP GEMVs, LSH page route and bf16
    paged attention) on the configs[4] model dimensions at batch 1 after a
    32k-token prefix per layer.  A 28-layer step does not fit a bounded
    sample, so models of 1 and 2 layers of the same dimensions are timed and
    the step is extrapolated: t28 = t1 + 27 (t2 - t1)."""
    import numpy as np
    from oracle_bind import OR_KV_BF16, Oracle, OracleDecoder
    orc = Oracle()
    cores = cpu_threads()
    rng = np.random.default_rng(43)
    A = B3
    d, H, KV, hd, F, V = (A[k] for k in ("dim", "n_heads", "n_kv_heads", "head_dim", "hidden_dim", "vocab"))
    # E4M3 codes without the NaN code (|c| <= 0x7E), tiled from one random block
    block = (rng.integers(0, 0x7F, 1 << 24, dtype=np.uint8) | (rng.integers(0, 2, 1 << 24, dtype=np.uint8) << 7))

    def fp8(r, c):
        return np.resize(block, (r, c)), (rng.uniform(0.5, 1.0, r) * (0.02 / 448.0)).astype(np.float32)
    one = np.full(d, 0x3F80, np.uint16)

    def layer():
        Lw = {}
        for name, (r, c) in {"wq": (H * hd, d), "wk": (KV * hd, d), "wv": (KV * hd, d), "wo": (d, H * hd),
                             "w1": (F, d), "w3": (F, d), "w2": (d, F)}.items():
            Lw[name], Lw["s" + name[1:]] = fp8(r, c)
        Lw["attn_norm"], Lw["ffn_norm"] = one, one
        return Lw
    layers = [layer(), layer()]
    emb, emb_s = fp8(V, d)
    out, out_s = fp8(V, d)
    _, hpT = orc.lsh_init(hd, 42)
    T = B3_CTX
    times = {}
    for n_layers in (1, 2):
        w = dict(emb=emb, emb_s=emb_s, final_norm=one, out=out, out_s=out_s, layers=layers[:n_layers])
        cfg = dict(n_layers=n_layers, dim=d, n_heads=H, n_kv=KV, hd=hd, hidden=F, vocab=V, max_seq=T + 256,
                   wkind=1, kv_kind=OR_KV_BF16, sparse_k=64, cand_cap=64, theta=1e4, eps=1e-5)
        dec = OracleDecoder(orc, cfg, w, hpT)
        for l in range(n_layers):
            dec.kv_append_n(l, rng.standard_normal((T, KV * hd)).astype(np.float32),
                            rng.standard_normal((T, KV * hd)).astype(np.float32), 0)
        tok = 1
        tok, _ = dec.step(tok, T, threads=cores)            # warm-up
        ts = []
        t_end = time.perf_counter() + seconds / 2
        pos = T + 1
        while time.perf_counter() < t_end and pos < T + 200:
            t0 = time.perf_counter()
            tok, _ = dec.step(tok, pos, threads=cores)
            ts.append(time.perf_counter() - t0)
            pos += 1
        times[n_layers] = (sorted(ts)[len(ts) // 2], len(ts))
        del dec
    t1, t2 = times[1][0], times[2][0]
    t28 = t1 + (A["n_layers"] - 1) * (t2 - t1)
    return {"value": round(1.0 / t28, 2), "unit": "tokens/s", "cores": cores, "kind": "port",
            "t_1layer_ms": round(t1 * 1e3, 2), "t_2layer_ms": round(t2 * 1e3, 2), "host": host_info(),
            "sample": f"oracle or_decoder_step on the configs[4] dimensions (FP8 weights, bf16 pages, LSH route "
                      f"top-64 pages) at position {T} after a random {T}-token prefix, batch 1, OpenMP {cores} "
                      f"threads: 1- and 2-layer models timed ({times[1][1]} and {times[2][1]} steps, medians), "
                      f"28-layer step extrapolated as t1 + 27 (t2 - t1)"}


def gemm_cpu_baseline(seconds=10.0):
    """The oracle's OpenMP GEMM (per-token x per-row scaled FP8, the
    reference's dequantised dot order) on a bounded sample of configs[2]:
    FP8 M=512 x 4096x4096."""
    import numpy as np
    from oracle_bind import Oracle
    orc = Oracle()
    cores = cpu_threads()
    rng = np.random.default_rng(12)
    m, n, k = 512, 4096, 4096
    xq, sx = orc.quantize_rows(rng.standard_normal((m, k)).astype(np.float32), "fp8")
    wq, sw = orc.quantize_rows((rng.standard_normal((n, k)) * 0.02).astype(np.float32), "fp8")
    orc.gemm(xq[:16], sx[:16], wq, sw, "fp8", threads=cores)     # warm-up
    ts = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end and len(ts) < 50:
        t0 = time.perf_counter()
        orc.gemm(xq, sx, wq, sw, "fp8", threads=cores)
        ts.append(time.perf_counter() - t0)
    med = sorted(ts)[len(ts) // 2]
    return {"value": round(2.0 * m * n * k / med / 1e12, 4), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "host": host_info(),
            "sample": f"oracle or_gemm_fp8 M={m} N={n} K={k}, OpenMP {cores} threads, median of {len(ts)} runs"}


LSH_PMC_SUMMARY = os.path.join(ROOT, "profiles", "lsh_attn_32k_pmc.txt")


def lsh_traffic(batch):
    """HBM bytes per step of the route + attention at this batch (its one or
    two launches), from the committed rocprofv3 --pmc summary (scaled like
    the GEMV's)."""
    if not os.path.exists(LSH_PMC_SUMMARY):
        return None
    for line in open(LSH_PMC_SUMMARY):
        if line.startswith(f"traffic_bytes_per_launch[b={batch}]"):
            return int(line.split("=")[-1].split()[0])
    return None


def lsh_probe():
    """For rocprofv3 runs: the configs[3] pool for 128 sequences (as
    lsh_bench builds it), then 10 fused route + attention launches at each of
    batch 1, 64 and 128, then 10 copies of 1 GiB as the counters' byte
    reference."""
    import numpy as np
    import torch
    import be42
    lib = be42.load()
    lib.init(0)
    cfg = LSH
    H, KVH, hd, T = cfg["heads"], cfg["kv_heads"], cfg["head_dim"], cfg["ctx"]
    BM = 128
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
    print("lsh probe: pool built", flush=True)
    qall = torch.from_numpy(q).cuda()
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    for B in (1, 64, 128):
        qd = qall[:B].contiguous()
        out = torch.empty((B, H, hd), device="cuda")
        sel = torch.empty((B, 64), dtype=torch.int32, device="cuda")
        nsel = torch.empty(B, dtype=torch.int32, device="cuda")
        for _ in range(10):
            lib._call("be42_lsh_attention", pool.handle, lib.p(qd), None, B, H, cfg["k_sel"], cfg["cap"], scale,
                      lib.p(out), lib.p(sel), lib.p(nsel), 64, lib.stream())
        torch.cuda.synchronize()
        print(f"lsh probe: batch {B} done, n_sel mean {nsel.float().mean().item():.1f}", flush=True)
    src = torch.empty(1 << 28, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    pool.close()
    print("lsh probe done", flush=True)


def gemm_probe():
    """For rocprofv3 runs: 5 launches each of the prefill GEMM at FP8
    8192x4096x14336 (the best shape), INT8 2048x4096x14336 and INT8
    512x4096x4096."""
    import torch
    import be42
    lib = be42.load()
    lib.init(0)
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    for kind, m, n, k in (("fp8", 8192, 4096, 14336), ("int8", 2048, 4096, 14336), ("int8", 512, 4096, 4096)):
        qf = lib.quant_rows_int8 if kind == "int8" else lib.quant_rows_fp8
        wq, sw = qf(torch.randn(n, k, generator=g, device="cuda") * 0.02)
        xq, sx = qf(torch.randn(m, k, generator=g, device="cuda"))
        y = torch.empty(m, n, device="cuda")
        for _ in range(5):
            lib.gemm(xq, sx, wq, sw, kind, out=y)
        torch.cuda.synchronize()
        print(f"gemm probe: {kind} {m}x{n}x{k} done", flush=True)
        del wq, sw, xq, sx, y


def decode_probe():
    """For rocprofv3 runs (--pmc counters or --kernel-trace): the configs[4]
    3B model (FP8 weights, bf16 pages) at batch 1 after a 1088-token prompt
    (68 pages: the steps route, as at 32k), 10 decode steps (each a
    fused-layer launch per layer over 100.8 MB of weights: 2.8 GB per step,
    so the 256 MB Infinity Cache serves no weight of the next step), then 10
    copies of 1 GiB as the byte reference of the FETCH_SIZE / WRITE_SIZE
    counters."""
    import numpy as np
    import torch
    import be42
    lib = be42.load()
    lib.init(0)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(41)
    A = B3
    w = decoder_weights(lib, A, "fp8", gen)
    _, hpT = lib.lsh_projection(A["head_dim"], 42)
    dec = be42.Decoder(lib, decoder_cfg(A, 2048, 1, 1, be42.KV_BF16), w, hpT)
    n_prompt = 1088
    prompt = np.random.default_rng(6).integers(0, A["vocab"], n_prompt)
    tok = dec.prefill(prompt)
    for i in range(10):
        tok = dec.step([int(tok)] if i == 0 else None, n_prompt + i, sync=False, batch=1)
    torch.cuda.synchronize()
    dec.status()
    dec.close()
    src = torch.empty(1 << 28, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print("decode probe done", flush=True)


PMC_CONFIG = ("fp8", 128256, 4096, 16)
PMC_SUMMARY = os.path.join(ROOT, "profiles", "gemv_fp8_128256x4096_b16_pmc.txt")


def pmc_probe():
    """For rocprofv3 runs (--pmc counters or --kernel-trace): 10 launches of
    the FP8 128256x4096 batch-16 GEMV, rotating over 3 weight copies (1.6 GB,
    so the 256 MB Infinity Cache cannot serve a repeat), then 10 copies of
    1 GiB (runtime copy kernel) as the byte-count reference of the
    FETCH_SIZE / WRITE_SIZE counters."""
    import torch
    import be42
    lib = be42.load()
    lib.init(0)
    kind, n, k, b = PMC_CONFIG
    w = torch.randn(n, k, device="cuda") * 0.02
    q, sc = lib.quant_rows_fp8(w)
    del w
    qs = [q] + [q.roll(shifts=7 * i, dims=1).contiguous() for i in (1, 2)]
    x = torch.randn(b, k, device="cuda")
    xdig = lib.gemv_prepare(x, kind)
    y = torch.empty(b, n, device="cuda")
    for i in range(10):
        lib.gemv_prepared(qs[i % 3], sc, xdig, b, kind, y)
    src = torch.empty(1 << 28, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print("pmc probe done", flush=True)


def measured_traffic(dc):
    """HBM bytes per launch of the dominant GEMV from the committed
    rocprofv3 --pmc summary (FETCH_SIZE + WRITE_SIZE, scaled by the copy
    kernel's reading of a known byte count), when it covers this workload."""
    if (dc["kind"], dc["n"], dc["k"], dc["b"]) != PMC_CONFIG or not os.path.exists(PMC_SUMMARY):
        return None
    for line in open(PMC_SUMMARY):
        if line.startswith("traffic_bytes_per_launch"):
            return int(line.split("=")[1].split()[0])
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-gemv", action="store_true",
                    help="skip the GEMV sweep (value is then null; for profiling the other legs)")
    ap.add_argument("--no-lsh", action="store_true", help="skip the LSH attention leg")
    ap.add_argument("--no-gemm", action="store_true", help="skip the prefill GEMM leg")
    ap.add_argument("--no-decode", action="store_true", help="skip the decode-step leg")
    ap.add_argument("--no-dropin", action="store_true", help="skip the host-array op_matmul (PCIe) leg")
    ap.add_argument("--no-3b", action="store_true", help="skip the 3B-model decode (its setup takes ~1 minute)")
    ap.add_argument("--pmc-probe", action="store_true", help="only run the kernels profiled for HBM traffic")
    ap.add_argument("--lsh-probe", action="store_true", help="only run the LSH launches profiled for HBM traffic")
    ap.add_argument("--gemm-probe", action="store_true", help="only run the GEMM launches profiled for counters")
    ap.add_argument("--decode-probe", action="store_true",
                    help="only run 3B batch-1 decode steps (fused layers) profiled for HBM traffic")
    args = ap.parse_args()
    if args.pmc_probe:
        pmc_probe()
        return
    if args.lsh_probe:
        lsh_probe()
        return
    if args.gemm_probe:
        gemm_probe()
        return
    if args.decode_probe:
        decode_probe()
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              f"(the hot path is built and measured on one GPU's share: GEMV rows, KV heads and "
              f"queries would shard across GPUs, but no multi-GPU path is built)", file=sys.stderr)
        sys.exit(2)

    import torch
    import be42

    lib = be42.load()
    lib.init(0)
    dev = torch.device("cuda:0")
    torch.manual_seed(0)

    def gemv_sweep():
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

        # one step: the 24 GEMVs y = W x through the library's x -> y entry
        # point (be42_gemv_q8 / be42_gemv_fp8: a prepare launch forming the
        # digit planes of x, then the GEMV launch).  With prepared=True
        # (breakdown only) the GEMV launch alone, on digits prepared
        # beforehand.
        def run_step(ev=None, prepared=False):
            for ci, c in enumerate(configs):
                w = c["pool"][c["i"] % len(c["pool"])]
                c["i"] += 1
                if ev is not None:
                    ev[ci][0].record()
                if prepared:
                    lib.gemv_prepared(w, c["s"], c["xdig"], c["b"], c["kind"], c["y"])
                else:
                    lib.gemv(w, c["s"], c["x"], c["kind"], out=c["y"])
                if ev is not None:
                    ev[ci][1].record()

        for _ in range(args.warmup):
            run_step()
        torch.cuda.synchronize()

        # the timed steps: nothing but the 24 x -> y GEMVs
        t0 = time.perf_counter()
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        start.record()
        for s in range(args.steps):
            run_step()
        stop.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        total_ms = start.elapsed_time(stop)

        step_bytes = sum(gemv_bytes(c["n"], c["k"], c["b"]) for c in configs)
        ms_per_step = total_ms / args.steps
        value = step_bytes / (ms_per_step * 1e-3) / 1e9

        # breakdown, in further steps: an event pair around each x -> y call
        # (op_us), and around each GEMV launch on prepared digits (kernel_us)
        evs = [[[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in configs]
               for _ in range(args.steps)]
        evk = [[[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in configs]
               for _ in range(args.steps)]
        for s in range(args.steps):
            run_step(evs[s])
        for s in range(args.steps):
            run_step(evk[s], prepared=True)
        torch.cuda.synchronize()
        sweep = []
        for ci, c in enumerate(configs):
            op_ms = sum(evs[s][ci][0].elapsed_time(evs[s][ci][1]) for s in range(args.steps)) / args.steps
            main_ms = sum(evk[s][ci][0].elapsed_time(evk[s][ci][1]) for s in range(args.steps)) / args.steps
            nb = gemv_bytes(c["n"], c["k"], c["b"])
            row = {"dtype": c["kind"], "n": c["n"], "k": c["k"], "batch": c["b"],
                   "op_us": round(op_ms * 1e3, 2), "kernel_us": round(main_ms * 1e3, 2),
                   "op_GBps": round(nb / (op_ms * 1e-3) / 1e9, 1),
                   "kernel_GBps": round(nb / (main_ms * 1e-3) / 1e9, 1)}
            sweep.append(row)

        # The roofline kernel: the step's largest launch (FP8 128256 x 4096,
        # batch 16: 534 MB), timed over back-to-back launches on the launch
        # stream (each on the next weight copy of its pool) between one
        # event pair, so the average is the launch duration in a stream.
        dc = next(c for c in configs if (c["kind"], c["n"], c["k"], c["b"]) == PMC_CONFIG)
        dnb = gemv_bytes(dc["n"], dc["k"], dc["b"])
        reps = max(args.steps, 20)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(reps):
            lib.gemv_prepared(dc["pool"][i % len(dc["pool"])], dc["s"], dc["xdig"], dc["b"], dc["kind"], dc["y"])
        e1.record()
        torch.cuda.synchronize()
        dm = e0.elapsed_time(e1) / reps
        achieved = dnb / (dm * 1e-3) / 1e9
        kname = "be42::k_gemv_coop (%s)" % dc["kind"]
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
                         "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(dc),
                         "bytes_per_launch": dnb, "launch_us": round(dm * 1e3, 2)},
            "gemv_sweep": sweep,
            "wall_s": round(wall, 2),
        }
        return out, configs

    if args.no_gemv:
        configs = []
        out = {"metric": "decode tokens/s; quant GEMV HBM GB/s (% of peak); LSH attn µs/token @32k",
               "value": None, "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
               "ms_per_step": None, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
               "dtype": "int8/fp8 weights, fp32 activations", "data": "synthetic",
               "config": {"workload": "GEMV sweep skipped (--no-gemv)", "parallelism": "single GPU"}}
    else:
        out, configs = gemv_sweep()
    if not args.no_dropin:
        out["dropin_pcie"] = dropin_bench(lib)
    if not args.no_decode:
        configs.clear()
        torch.cuda.empty_cache()
        out["decode"] = {"tiny": decode_tiny_bench(lib)}
        if not args.no_3b:
            out["decode"]["3b"] = decode_3b_bench(lib)
        torch.cuda.empty_cache()
    if not args.no_gemm:
        configs.clear()
        torch.cuda.empty_cache()
        out["prefill_gemm"] = gemm_bench(lib, 5, 1)
    if not args.no_lsh:
        # free the GEMV pools first
        configs.clear()
        torch.cuda.empty_cache()
        out["lsh_attention"] = lsh_bench(lib, max(args.steps, 10), max(args.warmup, 2))
        torch.cuda.empty_cache()
        # configs[3]'s other contexts: 8k (512 pages per sequence) and 128k
        # (8192 pages: twice the reference index's LSH_MAX_BLOCKS)
        out["lsh_attention_8k"] = lsh_bench(lib, max(args.steps, 10), max(args.warmup, 2), ctx=8192)
        torch.cuda.empty_cache()
        out["lsh_attention_128k"] = lsh_bench(lib, max(args.steps, 10), max(args.warmup, 2), batches=[1, 16, 64],
                                              ctx=131072)
        torch.cuda.empty_cache()
    if not args.no_cpu:
        # the reference's own GEMV (BF16 weights) when its compiled sources
        # are here; the oracle's INT8 port of its structure beside it
        port = cpu_baseline()
        port["host"] = host_info()
        ref_gemv = cpu_baseline_reference()
        if ref_gemv is not None:
            ref_gemv["host"] = port["host"]
            out["cpu_baseline"] = ref_gemv
            out["cpu_baseline_port"] = port
        else:
            out["cpu_baseline"] = port
        if not args.no_lsh:
            out["lsh_attention"]["cpu_baseline"] = lsh_cpu_baseline()
        if not args.no_gemm:
            out["prefill_gemm"]["cpu_baseline"] = gemm_cpu_baseline()
        if not args.no_decode:
            out["decode"]["tiny"]["cpu_baseline"] = decode_cpu_baseline()
            if not args.no_3b:
                out["decode"]["3b"]["cpu_baseline"] = decode_3b_cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
