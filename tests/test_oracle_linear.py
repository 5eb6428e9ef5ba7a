"""Oracle of the linear KV cache path, pinned without a GPU:
  - or_attention_linear against the compiled reference's op_attention_dense,
    op_attention_sparse and op_multihead_attention (ops_attention.c:84-245),
    bit-exact, and against a float64 two-pass softmax with the same exponent;
  - the linear cache's bf16 rows (kv_cache_append, kv_cache.c:55-80) against
    the reference and the closed-form round-to-nearest-even;
  - or_kv_evict against the reference's kv_cache_evict (incl. tied zero
    scores) and a float64 selection on untied data;
  - or_route_tokens (inference.c:268-423, no reference function: inline
    glue) against an independent numpy restatement whose parts are the
    reference's own heap (through the compiled reference) and the pinned
    bf16 dot."""
import numpy as np
import pytest

from oracle_bind import OracleIndex


def _bf16(orc, x):
    return orc.f32_to_bf16(np.asarray(x, np.float32))


def _f(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("T,n_kv,hd,H", [(300, 2, 64, 4), (77, 1, 128, 3), (1030, 8, 128, 32)])
def test_attention_linear_vs_reference(orc, ref, T, n_kv, hd, H):
    rng = np.random.default_rng(T + hd)
    k = _bf16(orc, rng.standard_normal((T, n_kv, hd)))
    v = _bf16(orc, rng.standard_normal((T, n_kv, hd)))
    q = rng.standard_normal(H * hd).astype(np.float32)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    idx = rng.permutation(T)[: min(64, T - 1)].astype(np.int32)
    for sel, multi in ((None, 0), (idx, 0), (idx, 1), (None, 1)):
        got = orc.attention_linear(q, k, v, sel, H, scale)
        want = np.zeros(H * hd, np.float32)
        ref.lib.ref_attention_linear(want.ctypes.data, q.ctypes.data, k.ctypes.data, v.ctypes.data, T,
                                     None if sel is None else sel.ctypes.data, 0 if sel is None else len(sel),
                                     H, n_kv, hd, scale, multi)
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    # structure: a two-pass softmax with the sequential running maxima
    kf, vf = _f(k), _f(v)
    for h in (0, H - 1):
        kvh = h // (H // n_kv)
        toks = idx
        s = (kf[toks, kvh].astype(np.float64) @ q[h * hd:(h + 1) * hd].astype(np.float64)) * float(scale)
        m = np.maximum.accumulate(s)
        prev = np.concatenate([[-np.inf], m[:-1]])
        a = orc.fast_expf(prev - m).astype(np.float64)
        p = orc.fast_expf(s - m).astype(np.float64)
        suffix = np.concatenate([np.cumprod(a[::-1])[::-1][1:], [1.0]])
        w = p * suffix
        want = (w @ vf[toks, kvh].astype(np.float64)) / w.sum()
        got = orc.attention_linear(q, k, v, idx, H, scale)[h * hd:(h + 1) * hd]
        np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5)


def test_linear_cache_rows(orc, ref):
    rng = np.random.default_rng(3)
    n, heads, dim = 37, 4, 64
    kf = (rng.standard_normal((n, heads * dim)) * 10).astype(np.float32)
    vf = rng.standard_normal((n, heads * dim)).astype(np.float32)
    ko = np.zeros((n, heads * dim), np.uint16)
    vo = np.zeros_like(ko)
    ref.lib.ref_kv_fill(ko.ctypes.data, vo.ctypes.data, kf.ctypes.data, vf.ctypes.data, n, 64, heads, dim)
    np.testing.assert_array_equal(ko, orc.f32_to_bf16(kf))
    np.testing.assert_array_equal(vo, orc.f32_to_bf16(vf))


@pytest.mark.parametrize("n,keep", [(200, 64), (100, 99), (50, 1)])
def test_kv_evict_vs_reference(orc, ref, n, keep):
    rng = np.random.default_rng(n + keep)
    heads, dim = 4, 32
    k = _bf16(orc, rng.standard_normal((n, heads, dim)))
    v = _bf16(orc, rng.standard_normal((n, heads, dim)))
    q = _bf16(orc, rng.standard_normal((heads, dim)))
    w = _bf16(orc, rng.uniform(0.5, 1.5, heads))
    # a third of the rows score exactly 0 (every head's dot clamped): ties
    k[::3] = _bf16(orc, -np.sign(_f(q))[None] * np.abs(_f(k[::3])))
    gk, gv, m = orc.kv_evict(k, v, q, w, keep)
    rk, rv = k.copy(), v.copy()
    rm = ref.lib.ref_kv_evict(rk.ctypes.data, rv.ctypes.data, n, heads, dim, q.ctypes.data, w.ctypes.data, keep)
    assert m == rm == keep
    np.testing.assert_array_equal(gk[:m], rk[:m])
    np.testing.assert_array_equal(gv[:m], rv[:m])
    # float64: keep the `keep` best (score desc, position asc), in position order
    kf, qf, wf = _f(k).astype(np.float64), _f(q).astype(np.float64), _f(w).astype(np.float64)
    score = (np.maximum(np.einsum("shd,hd->sh", kf, qf), 0.0) * wf).sum(1)
    order = sorted(range(n), key=lambda s: (-score[s], s))[:keep]
    np.testing.assert_array_equal(gk[:m], k[sorted(order)])


def _py_heap(scores, payload, cap):
    """ops_heap.h:33-100 (heap_push with strict root replacement) in Python."""
    h = []
    for s, e in zip(scores, payload):
        if len(h) < cap:
            h.append((s, e))
            i = len(h) - 1
            while i > 0:
                p = (i - 1) // 2
                if h[p][0] <= h[i][0]:
                    break
                h[i], h[p] = h[p], h[i]
                i = p
        elif s > h[0][0]:
            h[0] = (s, e)
            i = 0
            while True:
                sm, l, r = i, 2 * i + 1, 2 * i + 2
                if l < len(h) and h[l][0] < h[sm][0]:
                    sm = l
                if r < len(h) and h[r][0] < h[sm][0]:
                    sm = r
                if sm == i:
                    break
                h[i], h[sm] = h[sm], h[i]
                i = sm
    return [e for _, e in h]


def _route_tokens_numpy(orc, k, kv_len, q, H, hpT, hashes, starts, lens, window, sparse_k):
    n_kv, hd = k.shape[1], k.shape[2]
    ws = max(0, kv_len - window)
    cand = list(range(ws, kv_len))
    if ws > 0 and len(hashes):
        qh = orc.lsh_hash(hpT, orc.q_mean(q, H, hd))
        ids = []
        for p in range(17):
            ph = qh if p == 0 else qh ^ (1 << (p - 1))
            ids += [i for i in range(len(hashes) - 1, -1, -1) if hashes[i] == ph]
        for b in ids[:64]:
            if starts[b] + lens[b] <= ws:
                cand += [starts[b] + p for p in range(lens[b]) if starts[b] + p < ws]
    cand.sort()
    G = H // n_kv
    scores = []
    for t in cand:
        s = np.float32(0.0)
        for kv in range(n_kv):
            s = np.float32(s + np.float32(orc.lib.or_dot_bf16_f32(k[t, kv].copy(), q[kv * G * hd:(kv * G + 1) * hd].copy(), hd)))
        scores.append(s)
    return _py_heap(scores, cand, min(len(cand), sparse_k))


@pytest.mark.parametrize("kv_len,window,sparse_k", [(1000, 128, 64), (300, 128, 200), (60, 128, 64), (2000, 64, 32)])
def test_route_tokens_restated(orc, kv_len, window, sparse_k):
    rng = np.random.default_rng(kv_len + sparse_k)
    n_kv, hd, H = 2, 64, 8
    k = _bf16(orc, rng.standard_normal((kv_len, n_kv, hd)))
    q = rng.standard_normal(H * hd).astype(np.float32)
    _, hpT = orc.lsh_init(hd, 42)
    qh = orc.lsh_hash(hpT, orc.q_mean(q, H, hd))
    # 64-token blocks as lsh_update makes them; half the blocks hash near qh
    nb = kv_len // 64
    hashes = [int(qh ^ (1 << int(rng.integers(0, 16))) if rng.random() < 0.3 else (qh if rng.random() < 0.3
                   else rng.integers(0, 65536))) for _ in range(nb)]
    ix = OracleIndex(orc, 4096)
    for b, hb in enumerate(hashes):
        ix.insert(hb, 64 * b, 64)
    got = orc.route_tokens(k, kv_len, q, H, hpT, ix, window, sparse_k)
    if not (sparse_k > 0 and kv_len > sparse_k):
        assert got is None
        return
    want = _route_tokens_numpy(orc, k, kv_len, q, H, hpT, hashes, [64 * b for b in range(nb)], [64] * nb,
                               window, sparse_k)
    np.testing.assert_array_equal(got, want)
    assert len(got) == min(sparse_k, len(set(want)) if len(want) < sparse_k else sparse_k)
