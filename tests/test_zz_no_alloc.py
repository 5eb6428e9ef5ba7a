"""be42_gemv_noalloc: the GEMV with its digit planes in the library's fixed
device scratch (no allocation), called through the C ABI, against the
allocating entry point (be42_gemv_q8 / be42_gemv_fp8) on the same inputs --
the same kernels, so the outputs must be bit-identical -- and against the
oracle within the north star's 1e-3.  Two calls in a row share the scratch,
the second with a smaller input; a shape past the scratch is refused."""
import ctypes as C

import numpy as np
import pytest
import torch

from conftest import rel_err

pytestmark = pytest.mark.gpu


def _weights(rng, kind, n, k):
    if kind == "int8":
        return (rng.integers(-127, 128, (n, k), dtype=np.int8),
                rng.uniform(0.005, 0.02, n).astype(np.float32))
    wq = rng.integers(0, 256, (n, k), dtype=np.uint8)
    wq[(wq & 0x7F) == 0x7F] = 0x7E
    return wq, rng.uniform(0.005, 0.02, n).astype(np.float32) / 200.0


def _noalloc(be, y, w, s, x, n, k, b, kind):
    return be.lib.be42_gemv_noalloc(be.p(y), be.p(w), be.p(s), be.p(x), n, k, b, int(kind == "fp8"), None)


@pytest.mark.parametrize("kind", ["int8", "fp8"])
def test_gemv_noalloc_matches_gemv(be, orc, kind):
    rng = np.random.default_rng(77 if kind == "int8" else 78)
    # a split-K launch (4096 x 14336 at batch 16), then a smaller one
    for n, k, b in ((4096, 14336, 16), (300, 1024, 3)):
        wq, ws = _weights(rng, kind, n, k)
        x = rng.standard_normal((b, k)).astype(np.float32)
        wt, st, xt = torch.from_numpy(wq).cuda(), torch.from_numpy(ws).cuda(), torch.from_numpy(x).cuda()
        y = torch.full((b, n), float("nan"), device="cuda")
        assert _noalloc(be, y, wt, st, xt, n, k, b, kind) == 0, be.last_error()
        ref = be.gemv(wt, st, xt, kind)
        torch.cuda.synchronize()
        assert torch.equal(y, ref), (n, k, b)
        assert rel_err(y.cpu().numpy(), orc.gemv(wq, ws, x, kind)) <= 1e-3


def test_gemv_noalloc_refuses_oversize(be):
    k, b = 131072, 16                     # 8 MiB of FP8 digit planes and the scales
    y = torch.zeros((b, 16), device="cuda")
    w = torch.zeros((16, k), dtype=torch.uint8, device="cuda")
    s = torch.ones(16, device="cuda")
    x = torch.zeros((b, k), device="cuda")
    rc = be.lib.be42_gemv_noalloc(be.p(y), be.p(w), be.p(s), be.p(x), 16, k, b, 1, None)
    assert rc != 0 and "scratch" in be.last_error()
