"""Temperature and top-p sampling on the GPU (be42_sample_temperature /
be42_sample_top_p, and the drop-in sample_temperature / sample_top_p) against
the oracle (tests/test_oracle_sample.py pins it to the compiled reference).
The GPU sums probabilities 64 at a time with a carried sum (temperature)
or exactly in 62-bit fixed point (top-p), the oracle (and the reference) sequentially in
fp32, which over 128k terms drifts from the exact running
sum by up to ~1e-4 -- more than the mean probability of a 128k vocabulary, so
near most draws the reference's own pick is set by its rounding.  Every GPU
pick is checked to be the exact (float64) pick to within that drift (the
draw lies in the picked index's cumulative interval widened by it); where
the draw is farther than the drift from every boundary the pick must equal
the oracle's, and each test requires that a quarter of the cases got that
exact comparison (top-p over 128k entries, whose cut moves with the drift
too and whose set then holds ~1e5 entries: at least two)."""
import ctypes as C

import numpy as np
import pytest
import torch

import dropin_bind as D
from test_oracle_sample import probs64, rand_u, libc

pytestmark = pytest.mark.gpu

def logits_batch(rng, B, n, spread):
    return (rng.standard_normal((B, n)) * spread).astype(np.float32)


def drift(p):
    """max |sequential fp32 running sum - float64 running sum| of p, + 2e-6."""
    c64 = np.cumsum(p)
    c32 = np.cumsum(p.astype(np.float32), dtype=np.float32).astype(np.float64)
    return float(np.abs(c32 - c64).max()) + 2e-6


def consistent(cum, i, r, m):
    """index i is the first running sum above r, to within m"""
    lo = cum[i - 1] if i > 0 else 0.0
    return lo - m <= r < cum[i] + m


def temperature_case(x, temp, r):
    """(drawn index is consistent) checker, and whether r is near a boundary"""
    p = probs64(x, temp, False)
    cum = np.cumsum(p)
    m = drift(p)
    return (lambda i: consistent(cum, i, r, m)), abs(cum - r).min() < m


def top_p_case(x, temp, top_p, u):
    """as temperature_case; the cut itself may move within the drift, which
    moves r = u * (the set's sum) by at most the drift again"""
    p = probs64(x, temp, True)
    order = np.lexsort((np.arange(len(p)), -p))
    ps = p[order]
    cum = np.cumsum(ps)
    m = drift(ps)
    n = len(p)
    c_lo = min(int(np.searchsorted(cum, top_p - m, side="right")) + 1, n)
    c_hi = min(int(np.searchsorted(cum, top_p + m, side="right")) + 1, n)
    r_lo, r_hi = u * cum[c_lo - 1] - m, u * cum[c_hi - 1] + m
    pos = np.empty(n, np.int64)
    pos[order] = np.arange(n)

    def ok(i):
        k = int(pos[i])
        lo = cum[k - 1] if k > 0 else 0.0
        return k < c_hi and lo - m <= r_hi and r_lo < cum[k] + m

    b = cum[:c_hi]
    near = bool(((b >= r_lo - m) & (b <= r_hi + m)).any())
    return ok, near


def near_top_p_boundary(x, temp, top_p, u):
    return top_p_case(x, temp, top_p, u)[1]


@pytest.mark.parametrize("n,spread", [(4096, 2.0), (128256, 3.0), (1000, 0.3)])
@pytest.mark.parametrize("temp", [0.7, 1.0])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_temperature_matches_oracle(be, orc, n, spread, temp, dtype):
    rng = np.random.default_rng(n + int(temp * 10))
    B = 8
    x = logits_batch(rng, B, n, spread)
    xt = torch.from_numpy(x).cuda()
    if dtype == "bf16":
        xt = xt.bfloat16()
        x = xt.float().cpu().numpy()
    compared = 0
    reps = 8 if n > 100000 else 4
    for rep in range(reps):
        r = rng.uniform(0, 1, B).astype(np.float32)
        got = be.sample_temperature(xt, temp, torch.from_numpy(r).cuda()).cpu().numpy()
        for b in range(B):
            ok, near = temperature_case(x[b], temp, float(r[b]))
            assert ok(int(got[b])), (rep, b)
            if near:
                continue
            assert got[b] == orc.sample_temperature(x[b], temp, float(r[b])), (rep, b)
            compared += 1
    assert compared >= reps * B // 4


@pytest.mark.parametrize("n,spread", [(4096, 2.0), (128256, 3.0), (1000, 0.3)])
@pytest.mark.parametrize("temp,top_p", [(1.0, 0.9), (0.7, 0.5), (1.2, 0.995)])
def test_top_p_matches_oracle(be, orc, n, spread, temp, top_p):
    rng = np.random.default_rng(n + int(top_p * 1000))
    B = 6
    x = logits_batch(rng, B, n, spread)
    xt = torch.from_numpy(x).cuda()
    compared = 0
    reps = 8 if n > 100000 else 3
    for rep in range(reps):
        u = rng.uniform(0, 1, B).astype(np.float32)
        got = be.sample_top_p(xt, temp, top_p, torch.from_numpy(u).cuda()).cpu().numpy()
        for b in range(B):
            ok, near = top_p_case(x[b], temp, top_p, float(u[b]))
            assert ok(int(got[b])), (rep, b)
            if near:
                continue
            assert got[b] == orc.sample_top_p(x[b], temp, top_p, float(u[b])), (rep, b)
            compared += 1
    assert compared >= (2 if n > 100000 else reps * B // 4)


def test_top_p_ties_keep_index_order(be, orc):
    """Equal logits: the sorted order is ascending index (the oracle's
    deterministic tie rule), so every draw maps to the oracle's index."""
    x = np.repeat(np.float32([2.0, 1.0, 0.5]), 40)[None, :].copy()
    for u in (0.0, 0.1, 0.33, 0.5, 0.77, 0.999):
        got = be.sample_top_p(torch.from_numpy(x).cuda(), 1.0, 0.8,
                              torch.tensor([u], dtype=torch.float32, device="cuda")).item()
        assert got == orc.sample_top_p(x[0], 1.0, 0.8, u), u


def test_top_p_edges(be, orc):
    """A draw of u = 1 exceeds no running sum of the set: the set's last
    entry.  top_p >= 1 cuts nothing: the set is every entry, and its last one
    is the smallest probability.  top_p = 0: the set is the largest entry."""
    rng = np.random.default_rng(17)
    x = logits_batch(rng, 1, 3000, 2.0)
    xt = torch.from_numpy(x).cuda()
    for top_p, u in ((0.9, 1.0), (1.5, 1.0), (1.5, 0.5), (0.0, 0.3), (0.0, 1.0)):
        got = be.sample_top_p(xt, 1.0, top_p, torch.tensor([u], dtype=torch.float32, device="cuda")).item()
        ok, near = top_p_case(x[0], 1.0, top_p, u)
        assert ok(got), (top_p, u, got)
        if top_p != 0.9 or not near:
            assert got == orc.sample_top_p(x[0], 1.0, top_p, u), (top_p, u, got)
    p = probs64(x[0], 1.0, True)
    assert be.sample_top_p(xt, 1.0, 1.5, torch.tensor([1.0], device="cuda")).item() == int(np.argmin(p))
    assert be.sample_top_p(xt, 1.0, 0.0, torch.tensor([0.7], device="cuda")).item() == int(np.argmax(p))


@pytest.mark.parametrize("n", [1, 2, 5, 63, 65])
def test_samplers_short_rows(be, orc, n):
    """Rows shorter than a wave or a block: the per-wave ranges of the
    temperature walk and of the top-p tie pass are mostly empty, and one
    entry is its own set; every pick equals the oracle's (short rows keep
    the fp32 drift far below the gaps between their running sums)."""
    rng = np.random.default_rng(500 + n)
    B = 4
    x = logits_batch(rng, B, n, 2.0)
    xt = torch.from_numpy(x).cuda()
    for rep in range(3):
        u = rng.uniform(0, 1, B).astype(np.float32)
        ut = torch.from_numpy(u).cuda()
        gt = be.sample_temperature(xt, 1.0, ut).cpu().numpy()
        gp = be.sample_top_p(xt, 1.0, 0.9, ut).cpu().numpy()
        for b in range(B):
            ok, near = temperature_case(x[b], 1.0, float(u[b]))
            assert ok(int(gt[b])), (n, rep, b)
            if not near:
                assert gt[b] == orc.sample_temperature(x[b], 1.0, float(u[b])), (n, rep, b)
            ok, near = top_p_case(x[b], 1.0, 0.9, float(u[b]))
            assert ok(int(gp[b])), (n, rep, b)
            if not near:
                assert gp[b] == orc.sample_top_p(x[b], 1.0, 0.9, float(u[b])), (n, rep, b)
            if n == 1:
                assert gt[b] == 0 and gp[b] == 0


def test_dropin_samplers(be, orc):
    dl = D.bind(be.lib)
    rng = np.random.default_rng(9)
    arena = D.Arena()
    for seed in range(6):
        x = (rng.standard_normal(5000) * 2).astype(np.float32)
        libc.srand(C.c_uint(seed))
        got = dl.sample_top_p(C.byref(D.tensor(x, D.DTYPE_F32, 1, 5000)), 1.0, 0.9, C.byref(arena))
        u = rand_u(seed)
        if not near_top_p_boundary(x, 1.0, 0.9, u):
            assert got == orc.sample_top_p(x, 1.0, 0.9, u), seed
    # the temperature sampler's draw is its own LCG: one-hot logits give the argmax
    x = np.zeros(300, np.float32)
    x[123] = 200.0
    # (a draw of exactly 1.0, one in 32768, exceeds no running sum: the last index)
    got = [dl.sample_temperature(C.byref(D.tensor(x, D.DTYPE_F32, 1, 300)), 1.0, C.byref(arena)) for _ in range(3)]
    assert all(g in (123, 299) for g in got) and 123 in got
