"""The oracle's samplers (or_sample_temperature / or_sample_top_p) pinned:
top-p against the compiled reference's sample_top_p (sampler_topp.c:113-158)
on the same glibc rand() draw (srand(seed), then the first rand()); the
temperature sampler against a float64 restatement of sampler_temp.c:96-114
for given draws, and the compiled reference's sample_temperature (whose draw
is its own time-seeded LCG) on one-hot logits."""
import ctypes

import numpy as np
import pytest

RAND_MAX = np.float32(2147483647)
libc = ctypes.CDLL("libc.so.6")


def rand_u(seed):
    libc.srand(ctypes.c_uint(seed))
    return float(np.float32(np.float32(libc.rand()) / RAND_MAX))


def probs64(x, temp, max_from_first):
    m = x[0] if max_from_first else max(np.float32(-1e9), x.max())
    e = np.exp((x.astype(np.float64) - m) / temp)
    return e / e.sum()


@pytest.mark.parametrize("n", [10, 1000, 4096])
@pytest.mark.parametrize("temp,top_p", [(1.0, 0.9), (0.7, 0.5), (1.3, 0.99), (1.0, 1.0)])
def test_top_p_matches_reference(orc, ref, n, temp, top_p):
    rng = np.random.default_rng(n + int(temp * 10))
    for seed in range(8):
        x = (rng.standard_normal(n) * 2.5).astype(np.float32)
        want = ref.lib.ref_sample_top_p(x, n, temp, top_p, seed)
        assert orc.sample_top_p(x, temp, top_p, rand_u(seed)) == want, seed


def test_top_p_closed_form(orc):
    """Independent float64 restatement: the cut set and the draw position."""
    rng = np.random.default_rng(5)
    for trial in range(200):
        n = int(rng.integers(2, 300))
        x = (rng.standard_normal(n) * 3).astype(np.float32)
        temp, top_p, u = float(rng.uniform(0.5, 1.5)), float(rng.uniform(0.2, 0.99)), float(rng.uniform(0, 1))
        p = probs64(x, temp, True)
        order = sorted(range(n), key=lambda i: (-p[i], i))
        cum = np.cumsum(p[order])
        count = int(np.argmax(cum > top_p)) + 1 if (cum > top_p).any() else n
        r = u * cum[count - 1]
        j = int(np.argmax(cum[:count] > r)) if (cum[:count] > r).any() else count - 1
        # skip draws within float32 rounding of a boundary
        if min(abs(cum[:count] - r).min(), abs(cum - top_p).min()) < 1e-5:
            continue
        assert orc.sample_top_p(x, temp, top_p, u) == order[j], trial


def test_temperature_closed_form(orc):
    rng = np.random.default_rng(6)
    checked = 0
    for trial in range(300):
        n = int(rng.integers(1, 500))
        x = (rng.standard_normal(n) * 2).astype(np.float32)
        temp, r = float(rng.uniform(0.3, 2.0)), float(np.float32(rng.uniform(0, 1)))
        cum = np.cumsum(probs64(x, temp, False))
        if abs(cum - r).min() < 1e-5:
            continue
        want = int(np.argmax(cum > r)) if (cum > r).any() else n
        assert orc.sample_temperature(x, temp, r) == want, trial
        checked += 1
    assert checked > 250


def test_temperature_reference_one_hot(orc, ref):
    """The reference's own draw: with one logit far above the rest its
    probability is 1, so every draw below 1.0 gives that index (a draw of
    exactly 1.0, one in 32768, runs past the end: n)."""
    x = np.zeros(100, np.float32)
    x[37] = 200.0
    got = [ref.lib.ref_sample_temperature(x, 100, 1.0) for _ in range(6)]
    assert all(g in (37, 100) for g in got) and 37 in got
    assert orc.sample_temperature(x, 1.0, 0.999) == 37 and orc.sample_temperature(x, 1.0, 1.0) == 100
