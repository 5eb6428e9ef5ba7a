"""GPU decode GEMV (INT8 / FP8 per-row weights, fp32 activations) vs the oracle.

Tolerance (north star): max-rel-err <= 1e-3 with fp32 accumulation, written
here as max|y - y_ref| / max|y_ref|; the digit-split MFMA path is expected at
~1e-6.  Element-wise relative error is also bounded where |y_ref| is not tiny.
"""
import numpy as np
import pytest
import torch

from conftest import rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _check(y, want):
    err = rel_err(y, want)
    assert err <= TOL, err
    big = np.abs(want) > 1e-2 * np.abs(want).max()
    el = np.abs(y[big] - want[big]) / np.abs(want[big])
    assert el.max() <= 1e-2, el.max()
    return err


SHAPES = [(37, 4096, 1), (64, 1024, 4), (100, 4096, 16), (16, 16, 1), (300, 512, 3),
          (1408, 512, 1), (512, 1408, 2), (129, 4096, 8)]
GENERIC = [(33, 7, 1), (20, 1000, 2), (5, 4099, 1), (40, 256, 17)]


@pytest.mark.parametrize("kind", ["int8", "fp8"])
@pytest.mark.parametrize("n,k,b", SHAPES + GENERIC)
def test_gemv_small(be, orc, kind, n, k, b):
    rng = np.random.default_rng(n * 1000 + k + b)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((b, k)).astype(np.float32)
    wq, ws = orc.quantize_rows(w, kind)
    want = orc.gemv(wq, ws, x, kind)
    # quantize on the GPU too: identical codes, then the GPU GEMV
    wt = torch.from_numpy(w).cuda()
    q, s = be.quant_rows_int8(wt) if kind == "int8" else be.quant_rows_fp8(wt)
    np.testing.assert_array_equal(q.cpu().numpy(), wq)
    y = be.gemv(q, s, torch.from_numpy(x).cuda(), kind).cpu().numpy()
    _check(y, want)


@pytest.mark.parametrize("kind", ["int8", "fp8"])
@pytest.mark.parametrize("n,k", [(4096, 4096), (14336, 4096), (4096, 14336)])
@pytest.mark.parametrize("b", [1, 4, 16])
def test_gemv_config_shapes(be, orc, kind, n, k, b):
    """BASELINE config 2 shapes; codes drawn directly to keep host time short."""
    rng = np.random.default_rng(n + k + b)
    if kind == "int8":
        wq = rng.integers(-127, 128, (n, k), dtype=np.int8)
    else:
        wq = rng.integers(0, 256, (n, k), dtype=np.uint8)
        wq[(wq & 0x7F) == 0x7F] = 0x7E       # the reference encoder never emits 0x7F
    ws = rng.uniform(0.005, 0.02, n).astype(np.float32) / (1.0 if kind == "int8" else 200.0)
    x = rng.standard_normal((b, k)).astype(np.float32)
    want = orc.gemv(wq, ws, x, kind)
    y = be.gemv(torch.from_numpy(wq).cuda(), torch.from_numpy(ws).cuda(),
                torch.from_numpy(x).cuda(), kind).cpu().numpy()
    _check(y, want)


@pytest.mark.parametrize("kind", ["int8", "fp8"])
@pytest.mark.parametrize("b", [1, 4, 16])
def test_gemv_lm_head(be, orc, kind, b):
    """The largest config-2 shape (128256 x 4096) at every batch; FP8 at
    batch 16 is the benchmark's roofline launch (the block-cooperative kernel
    with 32 row tiles per block)."""
    rng = np.random.default_rng(7 + b)
    n, k = 128256, 4096
    if kind == "int8":
        wq = rng.integers(-127, 128, (n, k), dtype=np.int8)
        ws = rng.uniform(0.005, 0.02, n).astype(np.float32)
    else:
        wq = rng.integers(0, 256, (n, k), dtype=np.uint8)
        wq[(wq & 0x7F) == 0x7F] = 0x7E
        ws = rng.uniform(0.005, 0.02, n).astype(np.float32) / 200.0
    x = rng.standard_normal((b, k)).astype(np.float32)
    want = orc.gemv(wq, ws, x, kind)
    y = be.gemv(torch.from_numpy(wq).cuda(), torch.from_numpy(ws).cuda(),
                torch.from_numpy(x).cuda(), kind).cpu().numpy()
    _check(y, want)
    assert rel_err(y, want) <= (1e-5 if kind == "int8" else 1e-4)


def test_gemv_outliers_and_zero(be, orc):
    """Activations with 8-sigma outliers, an all-zero batch row, ragged n."""
    rng = np.random.default_rng(8)
    n, k, b = 77, 2048, 3
    x = rng.standard_normal((b, k)).astype(np.float32)
    x[0, rng.integers(0, k, 20)] = 8.0
    x[1] = 0.0
    for kind in ("int8", "fp8"):
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        wq, ws = orc.quantize_rows(w, kind)
        want = orc.gemv(wq, ws, x, kind)
        y = be.gemv(torch.from_numpy(wq).cuda(), torch.from_numpy(ws).cuda(),
                    torch.from_numpy(x).cuda(), kind).cpu().numpy()
        assert np.all(y[1] == 0.0)
        _check(y, want)


@pytest.mark.parametrize("kind", ["int8", "fp8"])
@pytest.mark.parametrize("b", [1, 5, 16])
def test_gemv_multi_segments(be, orc, kind, b):
    """Three matrices sharing one prepared input in one launch (ragged row
    counts, so row tiles straddle segments) against the oracle per segment
    and against one launch per matrix."""
    rng = np.random.default_rng(31 + b)
    k = 1024
    ns = (300, 64, 77)
    x = rng.standard_normal((b, k)).astype(np.float32)
    xt = torch.from_numpy(x).cuda()
    xdig = be.gemv_prepare(xt, kind)
    segs, wants, singles = [], [], []
    for n in ns:
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        wq, ws = orc.quantize_rows(w, kind)
        wants.append(orc.gemv(wq, ws, x, kind))
        wt, st = torch.from_numpy(wq).cuda(), torch.from_numpy(ws).cuda()
        segs.append((wt, st, torch.full((b, n), float("nan"), device="cuda")))
        singles.append(be.gemv_prepared(wt, st, xdig, b, kind, torch.empty((b, n), device="cuda")))
    outs = be.gemv_prepared_multi(segs, xdig, b, kind)
    for y, want, one in zip(outs, wants, singles):
        y = y.cpu().numpy()
        _check(y, want)
        # the digit-split path is far inside the north-star tolerance (FP8:
        # four digit planes, each element to ~1.2e-6 of max|x|)
        assert rel_err(y, one.cpu().numpy()) <= 1e-6
        assert rel_err(y, want) <= (1e-5 if kind == "int8" else 4e-5)


@pytest.mark.parametrize("kind", ["int8", "fp8"])
@pytest.mark.parametrize("b", [4, 8, 16])
def test_gemv_lds_stream_shapes(be, orc, kind, b):
    """Row counts past 8192 at batch >= 4 take the LDS-staged streaming
    kernel: a ragged row count (not a multiple of any tile), k not a multiple
    of the 128-byte stage, and three segments whose row tiles straddle."""
    rng = np.random.default_rng(400 + b)
    k = 1040
    ns = (20011, 5000, 8002)
    x = rng.standard_normal((b, k)).astype(np.float32)
    xt = torch.from_numpy(x).cuda()
    xdig = be.gemv_prepare(xt, kind)
    segs, wants = [], []
    for n in ns:
        if kind == "int8":
            wq = rng.integers(-127, 128, (n, k), dtype=np.int8)
            ws = rng.uniform(0.005, 0.02, n).astype(np.float32)
        else:
            wq = rng.integers(0, 256, (n, k), dtype=np.uint8)
            wq[(wq & 0x7F) == 0x7F] = 0x7E
            ws = rng.uniform(0.005, 0.02, n).astype(np.float32) / 200.0
        wants.append(orc.gemv(wq, ws, x, kind))
        segs.append((torch.from_numpy(wq).cuda(), torch.from_numpy(ws).cuda(),
                     torch.full((b, n), float("nan"), device="cuda")))
    # INT8 digit sums are exact int32; FP8 sums accumulate in fp32 inside the
    # MFMA, and codes drawn uniformly over all 256 (|w| up to 448) put that
    # rounding at ~1e-5 relative -- inside the north-star 1e-3, bounded at 1e-4
    tight = 1e-5 if kind == "int8" else 1e-4
    outs = be.gemv_prepared_multi(segs, xdig, b, kind)
    for y, want in zip(outs, wants):
        y = y.cpu().numpy()
        _check(y, want)
        assert rel_err(y, want) <= tight
    # one matrix alone (33013 rows)
    w_all = torch.cat([s[0] for s in segs]).contiguous()
    s_all = torch.cat([s[1] for s in segs]).contiguous()
    y1 = be.gemv_prepared(w_all, s_all, xdig, b, kind, torch.empty((b, sum(ns)), device="cuda")).cpu().numpy()
    assert rel_err(y1, np.concatenate(wants, axis=1)) <= tight


# Launch shapes forced through BE42_GEMV_TILE ("kind,rt,u,ks,waves,pf"):
# every slab configuration the dispatcher can name, and the direct-to-LDS
# ones at their column-group count, each run several times on one input.
FORCED = [
    ("slab", "3,4,2,4,8,4", None), ("slab", "3,2,2,4,8,4", None), ("slab", "3,1,2,2,8,4", None),
    ("slab", "3,4,4,1,8,4", None), ("slab", "3,2,4,1,8,4", None), ("slab", "3,1,4,1,8,4", None),
    ("slab split", "3,1,2,2,8,4,2", None), ("slab split", "3,2,2,4,8,4,2", None),
    ("slab split", "3,1,4,1,8,4,2", None), ("slab split", "3,1,2,2,8,4,4", ("fp8", 5)),
    ("coop", "4,0,6,0,8,0", None), ("coop", "4,0,6,0,8,1", None), ("coop split", "4,0,6,0,8,0,2", None),
    ("dma", "1,2,3,0,4,0", ("fp8", 16)), ("dma", "1,1,4,0,4,0", ("fp8", 16)),
    ("dma", "1,1,5,0,4,0", ("int8", 16)), ("dma", "1,1,3,0,8,0", ("int8", 16)),
]


# every shape at batch 1, 5 and 16, INT8 and FP8; a shape instantiated for
# one column-group count only at that (dtype, batch)
FORCED_CASES = [(kind, b, name, tile) for name, tile, only in FORCED for b in (1, 5, 16)
                for kind in ("int8", "fp8") if only is None or only == (kind, b)]


@pytest.mark.parametrize("kind,b,name,tile", FORCED_CASES)
def test_gemv_forced_tiles(be, orc, monkeypatch, kind, b, name, tile):
    """Each launch shape against the oracle on a ragged row count with k not
    a multiple of the 128-byte stage, five times in a row: the results must
    be identical every time (the direct-to-LDS rings and their barriers
    leave no read of a slot in flight when it is refilled)."""
    rng = np.random.default_rng(900 + b)
    n, k = 20011, 1040
    if kind == "int8":
        wq = rng.integers(-127, 128, (n, k), dtype=np.int8)
        ws = rng.uniform(0.005, 0.02, n).astype(np.float32)
    else:
        wq = rng.integers(0, 256, (n, k), dtype=np.uint8)
        wq[(wq & 0x7F) == 0x7F] = 0x7E
        ws = rng.uniform(0.005, 0.02, n).astype(np.float32) / 200.0
    x = rng.standard_normal((b, k)).astype(np.float32)
    want = orc.gemv(wq, ws, x, kind)
    wt, st = torch.from_numpy(wq).cuda(), torch.from_numpy(ws).cuda()
    xdig = be.gemv_prepare(torch.from_numpy(x).cuda(), kind)
    monkeypatch.setenv("BE42_GEMV_TILE", tile)
    first = None
    for _ in range(5):
        y = be.gemv_prepared(wt, st, xdig, b, kind, torch.full((b, n), float("nan"), device="cuda"))
        y = y.cpu().numpy()
        if first is None:
            first = y
            _check(y, want)
            assert rel_err(y, want) <= (1e-5 if kind == "int8" else 1e-4)
        else:
            assert np.array_equal(y, first)


@pytest.mark.parametrize("kind", ["int8", "fp8"])
@pytest.mark.parametrize("b", [8, 16])
def test_gemv_split_k_segments(be, orc, kind, b):
    """The split-K slab path (partials added by a second launch) on the
    decode projections of configs[4] at batch 8 / 16: q/k/v as three
    segments (5120 rows over k = 3072) and the down projection (3072 rows
    over k = 8192), against the oracle and one launch per matrix."""
    rng = np.random.default_rng(1200 + b)
    for ns, k in (((3072, 1024, 1024), 3072), ((3072,), 8192)):
        x = rng.standard_normal((b, k)).astype(np.float32)
        xdig = be.gemv_prepare(torch.from_numpy(x).cuda(), kind)
        segs, wants = [], []
        for n in ns:
            w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
            wq, ws = orc.quantize_rows(w, kind)
            wants.append(orc.gemv(wq, ws, x, kind))
            segs.append((torch.from_numpy(wq).cuda(), torch.from_numpy(ws).cuda(),
                         torch.full((b, n), float("nan"), device="cuda")))
        outs = be.gemv_prepared_multi(segs, xdig, b, kind)
        for (wt, st, _), y, want in zip(segs, outs, wants):
            y = y.cpu().numpy()
            _check(y, want)
            assert rel_err(y, want) <= 1e-5
            one = be.gemv_prepared(wt, st, xdig, b, kind, torch.empty((b, wt.shape[0]), device="cuda"))
            assert rel_err(one.cpu().numpy(), want) <= 1e-5


@pytest.mark.parametrize("kind", ["int8", "fp8"])
@pytest.mark.parametrize("b", [7, 16])
def test_gemv_coop_segments(be, orc, monkeypatch, kind, b):
    """The block-cooperative kernel over three segments whose boundaries fall
    inside 16-row tiles (rows 3000 / 1000 / 1100 over k = 3072, three steps of
    k per wave) and, split in two k ranges, over k = 8192 (four steps per
    wave), against the oracle; then a row count that is not a multiple of 16
    with forced tiles per block."""
    rng = np.random.default_rng(1300 + b)
    cases = (((3000, 1000, 1100), 3072, "4,0,6,0,8,0"), ((3000,), 8192, "4,0,6,0,8,0,2"),
             ((4099,), 4096, "4,0,6,0,8,3"))
    for ns, k, tile in cases:
        monkeypatch.setenv("BE42_GEMV_TILE", tile)
        x = rng.standard_normal((b, k)).astype(np.float32)
        xdig = be.gemv_prepare(torch.from_numpy(x).cuda(), kind)
        segs, wants = [], []
        for n in ns:
            w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
            wq, ws = orc.quantize_rows(w, kind)
            wants.append(orc.gemv(wq, ws, x, kind))
            segs.append((torch.from_numpy(wq).cuda(), torch.from_numpy(ws).cuda(),
                         torch.full((b, n), float("nan"), device="cuda")))
        outs = be.gemv_prepared_multi(segs, xdig, b, kind)
        for y, want in zip(outs, wants):
            y = y.cpu().numpy()
            _check(y, want)
            assert rel_err(y, want) <= (1e-5 if kind == "int8" else 1e-4)
