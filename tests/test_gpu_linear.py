"""The linear KV cache path on the GPU against the oracle: the device API
(be42_kv_linear_append, be42_linear_attention, be42_lsh_route_tokens,
be42_kv_linear_evict) and the reference-named drop-in (kv_cache_init /
kv_cache_append / kv_cache_evict, op_multihead_attention, op_attention_dense,
op_attention_sparse, flash_attention_head) called with host arrays as
src/inference calls them.

Bars: bf16 rows, evictions and token routes (positions in the heap's array
order) bit-exact; attention within 2e-5 normwise (the online softmax is
split across workgroups and merged, so the summation order differs from the
sequential reference)."""
import ctypes as C

import numpy as np
import pytest
import torch

import dropin_bind as D
from conftest import rel_err
from oracle_bind import OracleIndex

pytestmark = pytest.mark.gpu
ATTN_TOL = 2e-5


def _bf16(orc, x):
    return orc.f32_to_bf16(np.asarray(x, np.float32))


def _f(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _u16(a):
    return _dev(np.ascontiguousarray(a, np.uint16).view(np.int16))


@pytest.fixture(scope="module")
def dl(be):
    return D.bind(be.lib)


# ---- device API ---------------------------------------------------------------

def test_linear_append_rows(be, orc):
    rng = np.random.default_rng(5)
    T, n_kv, hd = 9, 4, 64
    kc = torch.zeros((T, n_kv, hd), dtype=torch.int16, device="cuda")
    vc = torch.zeros_like(kc)
    rows_k, rows_v = [], []
    for pos in range(T):
        k = (rng.standard_normal(n_kv * hd) * 10 ** rng.uniform(-30, 30, n_kv * hd)).astype(np.float32)
        v = rng.standard_normal(n_kv * hd).astype(np.float32)
        # round-half-to-even ties and the edges of the range
        k[:4] = np.array([0x3F808000, 0x3F818000, 0x7F7FFFFF, 0x80000001], np.uint32).view(np.float32)
        rows_k.append(k)
        rows_v.append(v)
        be.kv_linear_append(kc, vc, pos, _dev(k), _dev(v))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(kc.cpu().numpy().view(np.uint16).reshape(T, -1), orc.f32_to_bf16(np.stack(rows_k)))
    np.testing.assert_array_equal(vc.cpu().numpy().view(np.uint16).reshape(T, -1), orc.f32_to_bf16(np.stack(rows_v)))


@pytest.mark.parametrize("T,n_kv,hd,H", [(1, 1, 64, 1), (77, 1, 128, 3), (300, 2, 64, 4), (1030, 8, 128, 32),
                                         (5000, 8, 128, 32), (32768, 8, 128, 32)])
def test_linear_attention(be, orc, T, n_kv, hd, H):
    rng = np.random.default_rng(T + hd + H)
    k = _bf16(orc, rng.standard_normal((T, n_kv, hd)))
    v = _bf16(orc, rng.standard_normal((T, n_kv, hd)))
    q = (rng.standard_normal(H * hd) * 2).astype(np.float32)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    kd, vd, qd = _u16(k), _u16(v), _dev(q)
    # dense, a scattered selection, and a selection that repeats positions
    sels = [None, rng.permutation(T)[: min(64, T)].astype(np.int32),
            rng.integers(0, T, size=min(200, 3 * T)).astype(np.int32)]
    for sel in sels:
        n = T if sel is None else len(sel)
        got = be.linear_attention(qd, kd, vd, n, H, scale, idx=None if sel is None else _dev(sel)).cpu().numpy()
        want = orc.attention_linear(q, k, v, sel, H, scale)
        assert rel_err(got, want) <= ATTN_TOL, (T, None if sel is None else len(sel))


def test_linear_attention_empty(be):
    q = torch.ones(2 * 64, dtype=torch.float32, device="cuda")
    kc = torch.zeros((4, 1, 64), dtype=torch.int16, device="cuda")
    out = torch.full((2 * 64,), 7.0, device="cuda")
    be.linear_attention(q, kc, kc, 0, 2, 0.125, out=out)
    assert torch.count_nonzero(out).item() == 0


def _index(orc, rng, qh, nb):
    hashes = [int(qh ^ (1 << int(rng.integers(0, 16))) if rng.random() < 0.3 else (qh if rng.random() < 0.3
                   else rng.integers(0, 65536))) for _ in range(nb)]
    ix = OracleIndex(orc, 4096)
    for b, hb in enumerate(hashes):
        ix.insert(hb, 64 * b, 64)
    return hashes, ix


@pytest.mark.parametrize("kv_len,window,sparse_k,n_kv,H", [(1000, 128, 64, 2, 8), (300, 128, 64, 2, 8),
                                                          (65, 128, 64, 8, 32), (2000, 64, 32, 8, 32),
                                                          (32768, 128, 64, 8, 32), (4096, 4096, 64, 8, 32)])
def test_route_tokens(be, orc, kv_len, window, sparse_k, n_kv, H):
    rng = np.random.default_rng(kv_len + window)
    hd = 128 if H == 32 else 64
    k = _bf16(orc, rng.standard_normal((kv_len, n_kv, hd)))
    q = rng.standard_normal(H * hd).astype(np.float32)
    _, hpT = orc.lsh_init(hd, 42)
    qh = orc.lsh_hash(hpT, orc.q_mean(q, H, hd))
    nb = kv_len // 64
    hashes, ix = _index(orc, rng, qh, nb)
    # plant high-scoring keys in the newest exactly-matching blocks before
    # the window (the first candidates found), so that the route has to
    # reach past the window for them
    match = [b for b in range(nb) if hashes[b] == qh and 64 * (b + 1) <= kv_len - window][-3:]
    for b in match:
        k[64 * b + 5] = _bf16(orc, np.tile(q[:hd], (n_kv, 1)) * 3)
    want = orc.route_tokens(k, kv_len, q, H, hpT, ix, window, sparse_k)
    hh = np.asarray(hashes, np.uint16)
    topk, n = be.lsh_route_tokens(_u16(k), kv_len, _dev(q), H, _dev(hpT.astype(np.float32)),
                                  _u16(hh) if nb else None, _dev(np.arange(nb, dtype=np.int32) * 64),
                                  _dev(np.full(nb, 64, np.int32)), window, sparse_k)
    n = int(n.item())
    assert n == len(want)
    np.testing.assert_array_equal(topk.cpu().numpy()[:n], want)
    for b in match:
        assert 64 * b + 5 in want


@pytest.mark.parametrize("n,keep,heads,dim", [(200, 64, 4, 32), (100, 99, 8, 128), (50, 1, 2, 64),
                                              (4096, 1024, 8, 128)])
def test_kv_evict(be, orc, n, keep, heads, dim):
    rng = np.random.default_rng(n + keep)
    k = _bf16(orc, rng.standard_normal((n, heads, dim)))
    v = _bf16(orc, rng.standard_normal((n, heads, dim)))
    q = _bf16(orc, rng.standard_normal((heads, dim)))
    w = _bf16(orc, rng.uniform(0.5, 1.5, heads))
    k[::3] = _bf16(orc, -np.sign(_f(q))[None] * np.abs(_f(k[::3])))     # ties at score 0
    gk, gv, m = orc.kv_evict(k, v, q, w, keep)
    kd, vd = _u16(k), _u16(v)
    got = be.kv_linear_evict(kd, vd, n, _u16(q), _u16(w), keep)
    assert got == m == keep
    np.testing.assert_array_equal(kd.cpu().numpy().view(np.uint16)[:m], gk[:m])
    np.testing.assert_array_equal(vd.cpu().numpy().view(np.uint16)[:m], gv[:m])


# ---- drop-in ------------------------------------------------------------------

class _Cache:
    def __init__(self, dl, max_seq, heads, dim, arena_bytes=None):
        need = 2 * max_seq * heads * dim * 2 + 256
        self.buf = np.zeros(arena_bytes or need, np.uint8)
        self.arena = D.Arena(self.buf.ctypes.data, self.buf.nbytes, 0)
        self.c = D.KvCache()
        self.params = D.KvInitParams(max_seq, heads, dim)
        dl.kv_cache_init(C.byref(self.c), C.byref(self.arena), C.byref(self.params))
        self.heads, self.dim = heads, dim

    def host_rows(self, which):
        t = self.c.k if which == "k" else self.c.v
        n = self.c.current_seq_len * self.heads * self.dim
        return np.ctypeslib.as_array(C.cast(t.data, C.POINTER(C.c_uint16)), (max(n, 1),))[:n].reshape(
            -1, self.heads, self.dim).copy()


def _vec(a, dtype):
    t = D.Tensor()
    t.data = a.ctypes.data
    t.shape[0] = a.size
    t.stride[0] = 1
    t.ndim = 1
    t.size = a.size
    t.dtype = dtype
    return t


def test_dropin_cache_attention_evict(dl, orc, capfd):
    rng = np.random.default_rng(11)
    max_seq, n_kv, hd, H = 300, 2, 64, 8
    cache = _Cache(dl, max_seq, n_kv, hd)
    c = cache.c
    assert c.max_seq_len == max_seq and c.current_seq_len == 0 and c.k.ndim == 3
    assert c.k.shape[0] == max_seq and c.k.shape[1] == n_kv and c.k.shape[2] == hd
    assert cache.arena.offset >= 2 * max_seq * n_kv * hd * 2
    ks, vs = [], []
    for t in range(260):
        if t % 2:   # F32 rows are rounded; BF16 rows copied
            k = rng.standard_normal(n_kv * hd).astype(np.float32)
            v = rng.standard_normal(n_kv * hd).astype(np.float32)
            dl.kv_cache_append(C.byref(c), C.byref(_vec(k, D.DTYPE_F32)), C.byref(_vec(v, D.DTYPE_F32)))
            ks.append(orc.f32_to_bf16(k))
            vs.append(orc.f32_to_bf16(v))
        else:
            k = _bf16(orc, rng.standard_normal(n_kv * hd))
            v = _bf16(orc, rng.standard_normal(n_kv * hd))
            dl.kv_cache_append(C.byref(c), C.byref(_vec(k, D.DTYPE_BF16)), C.byref(_vec(v, D.DTYPE_BF16)))
            ks.append(k)
            vs.append(v)
    assert c.current_seq_len == 260
    K = np.stack(ks).reshape(-1, n_kv, hd)
    V = np.stack(vs).reshape(-1, n_kv, hd)
    np.testing.assert_array_equal(cache.host_rows("k"), K)
    np.testing.assert_array_equal(cache.host_rows("v"), V)

    q = rng.standard_normal(H * hd).astype(np.float32)
    out = np.zeros(H * hd, np.float32)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    p = D.AttentionParams(q.ctypes.data, C.pointer(c), out.ctypes.data, H, n_kv, hd, scale, None, 0)
    dl.op_multihead_attention(C.byref(p))
    assert rel_err(out, orc.attention_linear(q, K, V, None, H, scale)) <= ATTN_TOL
    dl.op_attention_dense(C.byref(p), 100)
    assert rel_err(out, orc.attention_linear(q, K[:100], V[:100], None, H, scale)) <= ATTN_TOL
    idx = rng.permutation(260)[:64].astype(np.int32)
    p.topk_idx, p.attend_k = idx.ctypes.data, 64
    dl.op_multihead_attention(C.byref(p))
    assert rel_err(out, orc.attention_linear(q, K, V, idx, H, scale)) <= ATTN_TOL
    # attend_k >= kv_len: the dispatcher falls back to dense
    p.attend_k = 260
    big = np.concatenate([idx, np.zeros(260 - 64, np.int32)])
    p.topk_idx = big.ctypes.data
    dl.op_multihead_attention(C.byref(p))
    assert rel_err(out, orc.attention_linear(q, K, V, None, H, scale)) <= ATTN_TOL

    # one head over contiguous rows (kv heads = 1)
    K1 = np.ascontiguousarray(K[:, 1])
    V1 = np.ascontiguousarray(V[:, 1])
    o1 = np.zeros(hd, np.float32)
    q1 = q[:hd].copy()
    dl.flash_attention_head(o1.ctypes.data, q1.ctypes.data, K1.ctypes.data, V1.ctypes.data, 260, hd, scale)
    want1 = orc.attention_linear(q1, K1[:, None], V1[:, None], None, 1, scale)
    assert rel_err(o1, want1) <= ATTN_TOL

    # eviction keeps the best 100 rows in position order; the mirror follows
    qe = _bf16(orc, rng.standard_normal((n_kv, hd)))
    we = _bf16(orc, rng.uniform(0.5, 1.5, n_kv))
    scratch = np.zeros(1 << 16, np.uint8)
    sa = D.Arena(scratch.ctypes.data, scratch.nbytes, 0)
    ep = D.EvictParams(C.pointer(_vec(qe, D.DTYPE_BF16)), C.pointer(_vec(we, D.DTYPE_BF16)), 100, C.pointer(sa))
    dl.kv_cache_evict(C.byref(c), C.byref(ep))
    gk, gv, m = orc.kv_evict(K, V, qe, we, 100)
    assert c.current_seq_len == m == 100 and sa.offset == 0
    np.testing.assert_array_equal(cache.host_rows("k"), gk[:m])
    np.testing.assert_array_equal(cache.host_rows("v"), gv[:m])
    p.topk_idx, p.attend_k = None, 0
    dl.op_multihead_attention(C.byref(p))
    assert rel_err(out, orc.attention_linear(q, gk[:m], gv[:m], None, H, scale)) <= ATTN_TOL
    # keep_k <= 0 warns and does nothing; keep_k >= length does nothing
    capfd.readouterr()
    ep.keep_k = 0
    dl.kv_cache_evict(C.byref(c), C.byref(ep))
    assert "keep_k=0 invalid" in capfd.readouterr().err and c.current_seq_len == 100
    ep.keep_k = 500
    dl.kv_cache_evict(C.byref(c), C.byref(ep))
    assert c.current_seq_len == 100


def test_dropin_cache_full(dl, orc, capfd):
    cache = _Cache(dl, 3, 1, 64)
    c = cache.c
    row = np.ones(64, np.float32)
    for _ in range(3):
        dl.kv_cache_append(C.byref(c), C.byref(_vec(row, D.DTYPE_F32)), C.byref(_vec(row, D.DTYPE_F32)))
    capfd.readouterr()
    dl.kv_cache_append(C.byref(c), C.byref(_vec(row, D.DTYPE_F32)), C.byref(_vec(row, D.DTYPE_F32)))
    assert "KV Cache Full!" in capfd.readouterr().err and c.current_seq_len == 3
    np.testing.assert_array_equal(cache.host_rows("k"), np.full((3, 1, 64), 0x3F80, np.uint16))


def test_dropin_attention_on_foreign_cache(dl, orc):
    """A t_kv_cache filled by the caller (not by kv_cache_init) is read from
    its host rows."""
    rng = np.random.default_rng(2)
    T, n_kv, hd, H = 150, 4, 128, 16
    K = _bf16(orc, rng.standard_normal((T, n_kv, hd)))
    V = _bf16(orc, rng.standard_normal((T, n_kv, hd)))
    c = D.KvCache()
    c.k.data, c.v.data = K.ctypes.data, V.ctypes.data
    c.max_seq_len, c.num_heads, c.head_dim, c.current_seq_len = T, n_kv, hd, T
    q = rng.standard_normal(H * hd).astype(np.float32)
    out = np.zeros(H * hd, np.float32)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    idx = rng.permutation(T)[:40].astype(np.int32)
    p = D.AttentionParams(q.ctypes.data, C.pointer(c), out.ctypes.data, H, n_kv, hd, scale, idx.ctypes.data, 40)
    dl.op_attention_sparse(C.byref(p))
    assert rel_err(out, orc.attention_linear(q, K, V, idx, H, scale)) <= ATTN_TOL


def test_dropin_cache_struct_address_reused(dl, orc):
    """One t_kv_cache address (a reused ctypes buffer) holds first a cache
    made by kv_cache_init, then caller-filled caches of other shapes, then
    library caches again: every call must read the rows of the cache the
    struct holds at that moment (kv_cache.c:18-80, kv_cache_evict.c:34-70,
    ops_attention.c:175-245), never a device mirror made for an earlier
    struct at the same address."""
    rng = np.random.default_rng(21)
    raw = (C.c_uint8 * C.sizeof(D.KvCache))()
    c = D.KvCache.from_buffer(raw)
    scale_of = lambda hd: np.float32(1.0) / np.sqrt(np.float32(hd))  # noqa: E731
    keep = []

    def library_cache(max_seq, n_kv, hd, n_rows):
        C.memset(raw, 0, C.sizeof(raw))
        buf = np.zeros(2 * max_seq * n_kv * hd * 2 + 256, np.uint8)
        arena = D.Arena(buf.ctypes.data, buf.nbytes, 0)
        params = D.KvInitParams(max_seq, n_kv, hd)
        dl.kv_cache_init(C.byref(c), C.byref(arena), C.byref(params))
        keep.append(buf)
        K = _bf16(orc, rng.standard_normal((n_rows, n_kv, hd)))
        V = _bf16(orc, rng.standard_normal((n_rows, n_kv, hd)))
        for t in range(n_rows):
            dl.kv_cache_append(C.byref(c), C.byref(_vec(K[t], D.DTYPE_BF16)), C.byref(_vec(V[t], D.DTYPE_BF16)))
        return K, V

    def foreign_cache(T, n_kv, hd):
        C.memset(raw, 0, C.sizeof(raw))
        K = _bf16(orc, rng.standard_normal((T, n_kv, hd)))
        V = _bf16(orc, rng.standard_normal((T, n_kv, hd)))
        keep.extend([K, V])
        c.k.data, c.v.data = K.ctypes.data, V.ctypes.data
        c.max_seq_len, c.num_heads, c.head_dim, c.current_seq_len = T, n_kv, hd, T
        return K, V

    def check_attention(K, V, n_kv, hd, H):
        T = K.shape[0]
        q = rng.standard_normal(H * hd).astype(np.float32)
        out = np.zeros(H * hd, np.float32)
        sc = scale_of(hd)
        idx = rng.permutation(T)[:min(40, T - 1)].astype(np.int32)
        p = D.AttentionParams(q.ctypes.data, C.pointer(c), out.ctypes.data, H, n_kv, hd, sc, idx.ctypes.data,
                              len(idx))
        dl.op_attention_sparse(C.byref(p))
        assert rel_err(out, orc.attention_linear(q, K, V, idx, H, sc)) <= ATTN_TOL
        dl.op_multihead_attention(C.byref(p))
        assert rel_err(out, orc.attention_linear(q, K, V, idx, H, sc)) <= ATTN_TOL
        dl.op_attention_dense(C.byref(p), T)
        assert rel_err(out, orc.attention_linear(q, K, V, None, H, sc)) <= ATTN_TOL
        p.topk_idx, p.attend_k = None, 0
        dl.op_multihead_attention(C.byref(p))
        assert rel_err(out, orc.attention_linear(q, K, V, None, H, sc)) <= ATTN_TOL

    def check_evict(K, V, n_kv, hd, keep_k, host):
        K, V = K.copy(), V.copy()      # a foreign cache's rows are compacted in place
        qe = _bf16(orc, rng.standard_normal((n_kv, hd)))
        we = _bf16(orc, rng.uniform(0.5, 1.5, n_kv))
        scratch = np.zeros(1 << 16, np.uint8)
        sa = D.Arena(scratch.ctypes.data, scratch.nbytes, 0)
        ep = D.EvictParams(C.pointer(_vec(qe, D.DTYPE_BF16)), C.pointer(_vec(we, D.DTYPE_BF16)), keep_k,
                           C.pointer(sa))
        dl.kv_cache_evict(C.byref(c), C.byref(ep))
        gk, gv, m = orc.kv_evict(K, V, qe, we, keep_k)
        assert c.current_seq_len == m == keep_k
        np.testing.assert_array_equal(host("k")[:m], gk[:m])
        np.testing.assert_array_equal(host("v")[:m], gv[:m])
        return gk[:m], gv[:m]

    def host_rows(which, n_kv, hd):
        t = c.k if which == "k" else c.v
        n = c.current_seq_len * n_kv * hd
        return np.ctypeslib.as_array(C.cast(t.data, C.POINTER(C.c_uint16)), (n,)).reshape(-1, n_kv, hd).copy()

    # a 3-row library cache, then a 150-row foreign cache of 4 x 128 at the
    # same address (the sequence that once made op_attention_sparse refuse
    # positions >= 3)
    K, V = library_cache(3, 1, 64, 3)
    check_attention(K, V, 1, 64, 2)
    K, V = foreign_cache(150, 4, 128)
    check_attention(K, V, 4, 128, 16)
    K2, V2 = check_evict(K, V, 4, 128, 60, lambda w: host_rows(w, 4, 128))
    check_attention(K2, V2, 4, 128, 16)
    # a 400-row library cache of 1 x 64 (400 x 64 rows of mirror), then a
    # foreign cache of fewer but 8x wider rows: read through the old mirror
    # this would run past it
    K, V = library_cache(400, 1, 64, 300)
    check_attention(K, V, 1, 64, 4)
    K, V = foreign_cache(100, 4, 128)
    check_attention(K, V, 4, 128, 8)
    # appending to a foreign cache writes its host rows (F32 rounded to bf16)
    T = 100
    big_k = np.zeros((T + 5, 4, 128), np.uint16)
    big_v = np.zeros_like(big_k)
    big_k[:T], big_v[:T] = K, V
    keep.extend([big_k, big_v])
    c.k.data, c.v.data, c.max_seq_len = big_k.ctypes.data, big_v.ctypes.data, T + 5
    for t in range(5):
        if t % 2:
            nk = rng.standard_normal(4 * 128).astype(np.float32)
            nv = rng.standard_normal(4 * 128).astype(np.float32)
            dl.kv_cache_append(C.byref(c), C.byref(_vec(nk, D.DTYPE_F32)), C.byref(_vec(nv, D.DTYPE_F32)))
            want_k, want_v = orc.f32_to_bf16(nk), orc.f32_to_bf16(nv)
        else:
            want_k = _bf16(orc, rng.standard_normal(4 * 128))
            want_v = _bf16(orc, rng.standard_normal(4 * 128))
            dl.kv_cache_append(C.byref(c), C.byref(_vec(want_k, D.DTYPE_BF16)), C.byref(_vec(want_v, D.DTYPE_BF16)))
        np.testing.assert_array_equal(big_k[T + t].ravel(), want_k)
        np.testing.assert_array_equal(big_v[T + t].ravel(), want_v)
    assert c.current_seq_len == T + 5
    check_attention(big_k, big_v, 4, 128, 8)
    # a library cache again, released explicitly; the struct then reads as
    # a foreign cache of its own arena rows
    K, V = library_cache(64, 2, 64, 50)
    check_attention(K, V, 2, 64, 4)
    dl.kv_cache_release(C.byref(c))
    check_attention(K, V, 2, 64, 4)
