"""GPU prefill GEMM: per-token-quantized activations against
per-row-quantized weights on the matrix cores, vs the oracle.

INT8: the int32 accumulators are exact, so Y = ((float)acc * sx) * sw must be
bit-identical to the oracle (or_gemm_i8) and to an int64 numpy evaluation.
FP8: products of E4M3 values are exact, the sums are not: the oracle runs a
sequential fmaf chain and the f8f6f4 matrix core reduces each 128-product
block in its own adder tree (measured ~3e-5 of max|y| from the float64 sum of
the same codes), so the bound is the north star's max-rel-err 1e-3 (fp32
accumulate), written as max|y - y_ref| / max|y_ref|, against the oracle, and
2e-4 against the float64 sum.
"""
import numpy as np
import pytest
import torch

from conftest import rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _inputs(rng, m, n, k, outliers=True):
    """X ~ N(0,1) with 1% of entries replaced by +-8; W ~ N(0, 0.02^2)."""
    x = rng.standard_normal((m, k)).astype(np.float32)
    if outliers:
        mask = rng.random((m, k)) < 0.01
        x[mask] = np.where(rng.random(mask.sum()) < 0.5, -8.0, 8.0).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    return x, w


def _gpu_quant(be, a, kind):
    t = torch.from_numpy(a).cuda()
    return be.quant_rows_int8(t) if kind == "int8" else be.quant_rows_fp8(t)


def _exact_int8(xq, sx, wq, sw):
    acc = xq.astype(np.int64) @ wq.astype(np.int64).T
    return (acc.astype(np.float32) * sx[:, None]).astype(np.float32) * sw[None, :]


def _exact_fp8(orc, xq, sx, wq, sw):
    lut = orc.fp8_lut().astype(np.float64)
    s = lut[xq] @ lut[wq].T
    return s * sx[:, None].astype(np.float64) * sw[None, :].astype(np.float64)


SMALL = [(1, 1, 16), (17, 33, 48), (64, 128, 128), (130, 257, 4096), (5, 300, 144), (128, 128, 14336),
         (200, 1000, 1040)]


@pytest.mark.parametrize("kind", ["int8", "fp8"])
@pytest.mark.parametrize("m,n,k", SMALL)
def test_gemm_vs_oracle(be, orc, kind, m, n, k):
    rng = np.random.default_rng(m * 7 + n * 13 + k)
    x, w = _inputs(rng, m, n, k)
    xq_g, sx_g = _gpu_quant(be, x, kind)
    wq_g, sw_g = _gpu_quant(be, w, kind)
    xq, sx = orc.quantize_rows(x, kind)
    wq, sw = orc.quantize_rows(w, kind)
    # the GPU quantizers give the oracle's codes and scales
    np.testing.assert_array_equal(xq_g.cpu().numpy(), xq)
    np.testing.assert_array_equal(sx_g.cpu().numpy(), sx)
    y = be.gemm(xq_g, sx_g, wq_g, sw_g, kind).cpu().numpy()
    want = orc.gemm(xq, sx, wq, sw, kind)
    if kind == "int8":
        np.testing.assert_array_equal(y, want)
        np.testing.assert_array_equal(y, _exact_int8(xq, sx, wq, sw))
    else:
        assert rel_err(y, want) <= TOL
        assert rel_err(y.astype(np.float64), _exact_fp8(orc, xq, sx, wq, sw)) <= 2e-4


@pytest.mark.parametrize("kind", ["int8", "fp8"])
@pytest.mark.parametrize("m,n,k", [(512, 4096, 4096), (2048, 14336, 4096), (512, 4096, 14336),
                                   (8192, 4096, 14336), (2048, 128256, 4096), (8192, 128256, 4096)])
def test_gemm_config_shapes_sampled(be, orc, kind, m, n, k):
    """configs[2] shapes up to M = 8192 and N = 128256: the full product on
    the GPU, checked on 64 sampled rows x 96 sampled columns (the last row
    and column always among them) against exact host arithmetic of the same
    codes."""
    g = torch.Generator(device="cuda")
    g.manual_seed(m + n + k)
    x = torch.randn(m, k, generator=g, device="cuda")
    mask = torch.rand(m, k, generator=g, device="cuda") < 0.01
    x[mask] = torch.where(torch.rand(int(mask.sum()), generator=g, device="cuda") < 0.5, -8.0, 8.0)
    w = torch.randn(n, k, generator=g, device="cuda") * 0.02
    qf = be.quant_rows_int8 if kind == "int8" else be.quant_rows_fp8
    xq, sx = qf(x)
    wq, sw = qf(w)
    y = be.gemm(xq, sx, wq, sw, kind)
    rng = np.random.default_rng(m ^ n ^ k)
    rows = np.sort(rng.choice(m, 64, replace=False))
    cols = np.sort(rng.choice(n, 96, replace=False))
    rows[-1], cols[-1] = m - 1, n - 1
    r, c = torch.from_numpy(rows).cuda(), torch.from_numpy(cols).cuda()
    xs, sxs = xq[r].cpu().numpy(), sx[r].cpu().numpy()
    ws, sws = wq[c].cpu().numpy(), sw[c].cpu().numpy()
    got = y[r][:, c].cpu().numpy()
    if kind == "int8":
        np.testing.assert_array_equal(got, _exact_int8(xs, sxs, ws, sws))
    else:
        assert rel_err(got.astype(np.float64), _exact_fp8(orc, xs, sxs, ws, sws)) <= 2e-4


def test_gemm_int8_extremes(be, orc):
    """All +-127 codes at the largest configs[2] K: |acc| = 127^2 * 14336,
    within int32; zero rows give zero scale 1 rows."""
    m, n, k = 32, 48, 14336
    xq = np.full((m, k), 127, np.int8)
    xq[1::2] = -127
    wq = np.full((n, k), -127, np.int8)
    wq[:, ::3] = 127
    xq[5] = 0
    sx = np.linspace(0.5, 2.0, m).astype(np.float32)
    sw = np.linspace(0.001, 0.02, n).astype(np.float32)
    t = lambda a: torch.from_numpy(a).cuda()
    y = be.gemm(t(xq), t(sx), t(wq), t(sw), "int8").cpu().numpy()
    np.testing.assert_array_equal(y, orc.gemm(xq, sx, wq, sw, "int8"))
    np.testing.assert_array_equal(y, _exact_int8(xq, sx, wq, sw))


def test_gemm_rejects_bad_shapes(be):
    t = torch.zeros(64, dtype=torch.int8, device="cuda")
    f = torch.zeros(64, dtype=torch.float32, device="cuda")
    y = torch.zeros(64, dtype=torch.float32, device="cuda")
    rc = be.lib.be42_gemm_i8(be.p(y), be.p(t), be.p(f), be.p(t), be.p(f), 2, 2, 24, None)
    assert rc != 0 and "multiple of 16" in be.last_error()


@pytest.mark.parametrize("kind", ["int8", "fp8"])
@pytest.mark.parametrize("tile", ["1", "2", "3", "4", "5"])
def test_gemm_every_tile(be, orc, kind, tile, monkeypatch):
    """Each kernel and workgroup tiling (BE42_GEMM_TILE: 1 = 256x256,
    2 = 128x128 and 5 = 64x128 on the direct-to-LDS 32x32 kernel, which needs
    k a multiple of 128; 3 = 128x128 and 4 = 64x128 on the 16x16 kernel, here
    with k not a multiple of the 128-byte stage) on a ragged shape whose
    edges cut every tile."""
    monkeypatch.setenv("BE42_GEMM_TILE", tile)
    rng = np.random.default_rng(77 + int(tile))
    m, n, k = (300, 520, 1152) if tile in ("1", "2", "5") else (300, 520, 1040)
    x, w = _inputs(rng, m, n, k)
    xq, sx = orc.quantize_rows(x, kind)
    wq, sw = orc.quantize_rows(w, kind)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    y = be.gemm(t(xq), t(sx), t(wq), t(sw), kind).cpu().numpy()
    want = orc.gemm(xq, sx, wq, sw, kind)
    if kind == "int8":
        np.testing.assert_array_equal(y, want)
    else:
        assert rel_err(y, want) <= TOL
        assert rel_err(y.astype(np.float64), _exact_fp8(orc, xq, sx, wq, sw)) <= 2e-4


# ---- fp32 activations through the digit planes (the prefill projections) ----

def _weights(rng, n, k, kind, be):
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    wt = torch.from_numpy(w).cuda()
    return be.quant_rows_int8(wt) if kind == "int8" else be.quant_rows_fp8(wt)


@pytest.mark.parametrize("variant", ["0", "1", "3"])
@pytest.mark.parametrize("kind", ["int8", "fp8"])
@pytest.mark.parametrize("m,n,k", [(1, 64, 512), (17, 1000, 1424), (64, 3072, 512), (200, 1408, 4096),
                                   (300, 96, 8192)])
def test_gemm_f32_equals_gemv_rows(be, kind, m, n, k, variant, monkeypatch):
    """Every row of the digit-plane GEMM against the decode GEMV of the same
    row (batches of up to 16 rows, and single rows): INT8 bit-identical
    (exact int32 digit sums, one fp64 scaling), FP8 to fp32 accumulation
    order; within the GEMV tests' bounds of the float64 product of the
    codes: 1e-5 (INT8: digits to 2^-24 of max|x|) and 1e-4 (FP8: the matrix
    core's own fp32 reduction of each block of digit products).  Kernels:
    the direct-to-LDS one at its two tile shapes (BE42_GEMM_DIG 0, 3; K a
    multiple of 128) and the register-staged one (1, any K)."""
    monkeypatch.setenv("BE42_GEMM_DIG", variant)
    rng = np.random.default_rng(m * 7 + n + k)
    wq, sw = _weights(rng, n, k, kind, be)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[rng.random((m, k)) < 0.01] *= 50.0
    xt = torch.from_numpy(x).cuda()
    y = be.gemm_f32(xt, wq, sw, kind)
    ref = torch.empty_like(y)
    for r0 in range(0, m, 16):
        r1 = min(m, r0 + 16)
        ref[r0:r1] = be.gemv(wq, sw, xt[r0:r1].contiguous(), kind)
    single = [0, m - 1, m // 2]
    for r in single:
        ref1 = be.gemv(wq, sw, xt[r:r + 1].contiguous(), kind)
        if kind == "int8":
            assert torch.equal(ref1[0], ref[r]), r
    yh, rh = y.cpu().numpy(), ref.cpu().numpy()
    if kind == "int8":
        np.testing.assert_array_equal(yh, rh)
        wd = wq.cpu().numpy().astype(np.float64)
    else:
        from oracle_bind import Oracle
        wd = Oracle().fp8_lut()[wq.cpu().numpy()].astype(np.float64)
        assert rel_err(yh, rh) <= 1e-4
    exact = (x.astype(np.float64) @ wd.T) * sw.cpu().numpy().astype(np.float64)
    assert rel_err(yh, exact) <= (1e-5 if kind == "int8" else 1e-4)


@pytest.mark.parametrize("variant", ["0", "1", "3"])
@pytest.mark.parametrize("kind", ["int8", "fp8"])
def test_gemm_f32_segments_equal_single(be, kind, variant, monkeypatch):
    """q/k/v-shaped segments (3072, 1024, 1000 rows) in one launch equal
    three single-matrix launches bit for bit."""
    monkeypatch.setenv("BE42_GEMM_DIG", variant)
    rng = np.random.default_rng(11)
    k, m = 1024, 333
    segs = [_weights(rng, n, k, kind, be) for n in (3072, 1024, 1000)]
    xt = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).cuda()
    outs = be.gemm_f32_multi(xt, segs, kind)
    for (w, sw), y in zip(segs, outs):
        assert torch.equal(y, be.gemm_f32(xt, w, sw, kind))


def test_gemm_f32_rejects_bad_shapes(be):
    import be42
    w = torch.zeros((16, 24), dtype=torch.int8, device="cuda")
    s = torch.ones(16, device="cuda")
    with pytest.raises(be42.Be42Error, match="k % 16 == 0"):
        be.gemm_f32(torch.zeros((4, 24), device="cuda"), w, s, "int8")
