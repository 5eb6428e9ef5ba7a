"""GPU quant codecs vs the oracle: codes and scales bit-identical."""
import numpy as np
import pytest
import torch

from conftest import golden

pytestmark = pytest.mark.gpu


def _rows(rng):
    yield rng.standard_normal((7, 128)).astype(np.float32)
    yield (rng.standard_normal((33, 4096)) * 0.02).astype(np.float32)
    yield rng.standard_normal((3, 1)).astype(np.float32)
    z = np.zeros((2, 64), np.float32)
    z[1, 5] = -3.0
    yield z
    x = rng.standard_normal((5, 1000)).astype(np.float32) * 50
    x[2, 7] = 1e-30
    yield x
    # exact .5 points after scaling (roundf half away from zero)
    yield np.array([[127.0, 0.5, -0.5, 1.5, -2.5, 63.5, -63.5, 0.0]], np.float32)


def test_quant_int8_rows(be, orc):
    rng = np.random.default_rng(100)
    for x in _rows(rng):
        q, s = be.quant_rows_int8(torch.from_numpy(x).cuda())
        for r in range(x.shape[0]):
            wq, ws = orc.quant_int8(x[r])
            np.testing.assert_array_equal(q[r].cpu().numpy(), wq)
            assert s[r].item() == ws or (np.isnan(ws) and np.isnan(s[r].item()))
            assert np.float32(s[r].item()).view(np.uint32) == np.float32(ws).view(np.uint32)


def test_quant_fp8_rows(be, orc):
    rng = np.random.default_rng(101)
    g = golden("fp8_codec")
    cases = list(_rows(rng)) + [g["direct_in"][None, :]]
    i = 0
    while f"vec{i}_in" in g:
        cases.append(g[f"vec{i}_in"][None, :])
        i += 1
    for x in cases:
        x = np.ascontiguousarray(x, np.float32)
        q, s = be.quant_rows_fp8(torch.from_numpy(x).cuda())
        for r in range(x.shape[0]):
            wq, ws = orc.quant_fp8(x[r])
            np.testing.assert_array_equal(q[r].cpu().numpy(), wq)
            assert np.float32(s[r].item()).view(np.uint32) == np.float32(ws).view(np.uint32)
    # the reference's direct encoder codes (scale == 1 for this vector)
    q, s = be.quant_rows_fp8(torch.from_numpy(np.ascontiguousarray(g["direct_in"][None, :])).cuda())
    np.testing.assert_array_equal(q[0].cpu().numpy(), g["direct_codes"])


def test_fp8_encoder_binade_edges(be, orc):
    """Values a few ulps below every power of two, where log2f rounds up."""
    vals = []
    for e in range(-9, 8):
        p = np.float32(2.0 ** e)
        v = p
        for _ in range(8):
            v = np.nextafter(v, np.float32(0))
            vals.append(v)
        vals.append(p)
    vals = np.array(vals + [224.0], np.float32)     # absmax 224: scale == 1
    q, s = be.quant_rows_fp8(torch.from_numpy(vals[None, :]).cuda())
    assert s.item() == 1.0
    want, _ = orc.quant_fp8(vals)
    np.testing.assert_array_equal(q[0].cpu().numpy(), want)
    # (x * (224 / amax) never exceeds 224, so quant_f32_to_fp8 cannot reach the
    # binades above 2^7.)


def test_fp8_decode_all_codes(be, orc):
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8).cuda()
    out = be.fp8_decode(codes).cpu().numpy()
    np.testing.assert_array_equal(out.view(np.uint32), orc.fp8_lut().view(np.uint32))


def test_dequant_rows_int8(be, orc):
    rng = np.random.default_rng(102)
    x = rng.standard_normal((9, 130)).astype(np.float32)
    q, s = be.quant_rows_int8(torch.from_numpy(x).cuda())
    out = be.dequant_rows_int8(q, s).cpu().numpy()
    want = q.cpu().numpy().astype(np.float32) * s.cpu().numpy()[:, None]
    np.testing.assert_array_equal(out, want)
