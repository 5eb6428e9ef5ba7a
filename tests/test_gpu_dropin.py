"""The reference-named drop-in ABI (include/be42_engine.h) on the GPU, called
the way src/inference calls it, with host arrays, against the oracle.

op_matmul: the reference's own known answers (tests/unit/test_ops.c:179-233:
identity, [[1,2,3],[4,5,6]] x [[1,2],[3,4],[5,6]] = [[22,28],[49,64]]) and the
quantized GEMV within 1e-3.  Codecs, hashes, candidate lists, page tables,
block scores and selections are bit-exact; paged attention within 2e-5."""
import ctypes as C

import numpy as np
import pytest
import torch

import dropin_bind as D
from conftest import golden, rel_err
from oracle_bind import OR_KV_INT8, OracleIndex, OraclePaged

pytestmark = pytest.mark.gpu
PAGE = 16


@pytest.fixture(scope="module")
def dl(be):
    return D.bind(be.lib)


def _mm(dl, a, adt, b, out_dt=D.DTYPE_F32, scale=None, out=None):
    m, k = a.shape
    n = b.shape[1]
    if out is None:
        out = np.zeros((m, n), np.float32 if out_dt == D.DTYPE_F32 else np.uint16)
    ta = D.tensor(a, adt, m, k, scale)
    tb = D.tensor(b, D.DTYPE_BF16 if b.dtype == np.uint16 else D.DTYPE_F32, b.shape[0], n)
    to = D.tensor(out, out_dt, m, n)
    rc = dl.op_matmul(C.byref(to), C.byref(ta), C.byref(tb))
    return rc, out


def test_op_matmul_reference_kats(dl):
    ident = np.eye(2, dtype=np.float32)
    x = np.array([[3.0], [7.0]], np.float32)
    rc, y = _mm(dl, ident, D.DTYPE_F32, x)
    assert rc == 0 and y.ravel().tolist() == [3.0, 7.0]
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[1, 2], [3, 4], [5, 6]], np.float32)
    rc, y = _mm(dl, a, D.DTYPE_F32, b)
    assert rc == 0 and y.tolist() == [[22.0, 28.0], [49.0, 64.0]]
    # the same with BF16 weights (all values exact in bf16)
    rc, y = _mm(dl, (a.view(np.uint32) >> 16).astype(np.uint16), D.DTYPE_BF16, b)
    assert rc == 0 and y.tolist() == [[22.0, 28.0], [49.0, 64.0]]


def test_op_matmul_errors(dl, capfd):
    a = np.zeros((4, 8), np.float32)
    rc, _ = _mm(dl, a, D.DTYPE_F32, np.zeros((7, 1), np.float32))
    assert rc == -1 and "dim mismatch" in capfd.readouterr().err
    rc, _ = _mm(dl, np.zeros((4, 8), np.int8), D.DTYPE_I8, np.zeros((8, 1), np.float32))
    assert rc == -1 and "row_scale" in capfd.readouterr().err
    rc, _ = _mm(dl, a, D.DTYPE_F32, np.zeros((8, 1), np.float32), out_dt=D.DTYPE_BF16)
    assert rc == -1 and "unsupported dtypes" in capfd.readouterr().err


@pytest.mark.parametrize("kind", ["int8", "fp8"])
@pytest.mark.parametrize("m,k,n", [(64, 512, 1), (300, 1024, 1), (96, 256, 5), (40, 512, 37), (300, 1024, 200),
                                   (64, 1424, 70)])
def test_op_matmul_quantized(dl, orc, kind, m, k, n):
    rng = np.random.default_rng(m + k + n)
    w = (rng.standard_normal((m, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((k, n)).astype(np.float32)           # op_matmul's b is [k][n]
    wq, ws = orc.quantize_rows(w, kind)
    rc, y = _mm(dl, wq, D.DTYPE_I8 if kind == "int8" else D.DTYPE_FP8, x, scale=ws)
    assert rc == 0
    want = orc.gemv(wq, ws, x.T.copy(), kind).T                   # [n][m] -> [m][n]
    assert rel_err(y, want) <= 1e-3


def test_op_matmul_bf16_gemv(dl, orc):
    rng = np.random.default_rng(3)
    m, k = 200, 768
    w = rng.standard_normal((m, k)).astype(np.float32)
    wb = orc.f32_to_bf16(w)
    x = rng.standard_normal((k, 1)).astype(np.float32)
    rc, y = _mm(dl, wb, D.DTYPE_BF16, x)
    assert rc == 0
    want = orc.gemv_bf16(wb, x.ravel())
    assert rel_err(y.ravel(), want) <= 1e-5


def test_quant_codecs(dl, orc):
    rng = np.random.default_rng(9)
    x = (rng.standard_normal(128) * 3).astype(np.float32)
    q = np.zeros(128, np.int8)
    s = dl.quant_f32_to_int8(D.ptr(q), D.ptr(x), 128)
    wq, ws = orc.quant_int8(x)
    assert np.array_equal(q, wq) and np.float32(s) == ws
    f = np.zeros(128, np.uint8)
    sc = C.c_float()
    dl.quant_f32_to_fp8(D.ptr(f), D.ptr(x), 128, C.byref(sc))
    fq, fs = orc.quant_fp8(x)
    assert np.array_equal(f, fq) and np.float32(sc.value) == fs
    out = np.zeros(128, np.float32)
    dl.dequant_int8_to_f32_avx2(D.ptr(out), D.ptr(q), C.c_float(s), 128)
    assert np.array_equal(out, q.astype(np.float32) * np.float32(s))
    dl.quant_init_fp8_lut()
    lut = np.ctypeslib.as_array((C.c_float * 256).in_dll(dl, "g_fp8_lut"))
    assert np.array_equal(lut, orc.fp8_lut())
    # lightning score: 8 lane sums of relu(lut[q]*lut[k]) in order, then the tail
    kq = rng.integers(0, 256, 100, dtype=np.uint8) & 0x7E | (rng.integers(0, 2, 100, dtype=np.uint8) << 7)
    qq = rng.integers(0, 256, 100, dtype=np.uint8) & 0x7E
    L = orc.fp8_lut()
    p = (L[qq] * L[kq]).astype(np.float32)
    lanes = np.zeros(8, np.float32)
    for i in range(96):
        lanes[i % 8] = np.float32(lanes[i % 8] + max(p[i], np.float32(0)))
    r = np.float32(0)
    for j in range(8):
        r = np.float32(r + lanes[j])
    for i in range(96, 100):
        if p[i] > 0:
            r = np.float32(r + p[i])
    got = dl.compute_lightning_score_fp8(D.ptr(qq), D.ptr(kq), C.c_float(0.5), 100)
    assert np.float32(got) == np.float32(r * np.float32(0.5))


def test_lsh_drop_in(dl, orc):
    g = golden("lsh")
    ctx = D.LshCtx()
    dl.lsh_init(C.byref(ctx), 128, 42)
    hpT = np.ctypeslib.as_array(ctx.hp_transposed)[:128].copy()
    assert np.array_equal(hpT, g["hpT_128_42"])
    assert ctx.dim == 128 and ctx.initialized == 1
    rng = np.random.default_rng(5)
    v = rng.standard_normal(128).astype(np.float32)
    assert dl.lsh_hash(C.byref(ctx), D.ptr(v)) == orc.lsh_hash(hpT, v)
    assert dl.lsh_hamming_distance(0b1011, 0b0110) == 3
    # lsh_update over 300 keys: 4 committed 64-key blocks + an active one
    idx = D.LshIndex()
    dl.lsh_index_init(C.byref(idx))
    keys = rng.standard_normal((300, 128)).astype(np.float32)
    keys[64:128] += 2.0
    for t in range(300):
        dl.lsh_update(C.byref(idx), C.byref(ctx), D.ptr(keys[t]), 128, t)
    assert idx.n_blocks == 4
    want = OracleIndex(orc, 4096)
    for b in range(4):
        s = np.zeros(128, np.float32)
        for t in range(64 * b, 64 * b + 64):
            s = (s + keys[t]).astype(np.float32)
        c = (s * np.float32(1.0 / 64)).astype(np.float32)
        h = orc.lsh_hash(hpT, c)
        assert idx.block_hashes[b] == h and idx.block_starts[b] == 64 * b and idx.block_lens[b] == 64
        want.insert(h, 64 * b, 64)
    st, ln = C.c_int(), C.c_int()
    assert dl.lsh_get_active_block(C.byref(idx), C.byref(st), C.byref(ln)) == 1 and (st.value, ln.value) == (256, 44)
    # skewed hashes so that candidates span several probes
    for i in range(600):
        dl.lsh_insert_block(C.byref(idx), int(rng.choice([0x1234, 0x1235, 0x1236, 0x9234, 0x0F0F])), 256 + i, 1)
        want.insert(int(idx.block_hashes[idx.n_blocks - 1]), 256 + i, 1)
    for qh, cap in [(0x1234, 64), (0x1234, 500), (0x0F0F, 17), (int(idx.block_hashes[1]), 64)]:
        ids = np.zeros(cap, np.int32)
        n = dl.lsh_find_candidates(C.byref(idx), qh, D.ptr(ids), cap)
        np.testing.assert_array_equal(ids[:n], want.candidates(qh, cap))
    dl.lsh_index_reset(C.byref(idx))
    assert idx.n_blocks == 0 and dl.lsh_find_candidates(C.byref(idx), 0x1234, D.ptr(np.zeros(4, np.int32)), 4) == 0
    dl.lsh_index_release(C.byref(idx))
    dl.lsh_ctx_release(C.byref(ctx))


def test_lsh_structs_at_reused_addresses(dl, orc):
    """A t_lsh_ctx / t_lsh_index address that later holds another context or
    index (a struct freed and reused, or overwritten by the caller): hashes,
    candidates and block sums follow the struct's current contents
    (ops_lsh.c:138-242, :256-430), not the device copies made for the earlier
    struct."""
    rng = np.random.default_rng(31)
    ctx, other = D.LshCtx(), D.LshCtx()
    dl.lsh_init(C.byref(ctx), 128, 42)
    dl.lsh_init(C.byref(other), 128, 7)
    hp42 = np.ctypeslib.as_array(ctx.hp_transposed)[:128].copy()
    hp7 = np.ctypeslib.as_array(other.hp_transposed)[:128].copy()
    v = rng.standard_normal(128).astype(np.float32)
    assert dl.lsh_hash(C.byref(ctx), D.ptr(v)) == orc.lsh_hash(hp42, v)
    C.memmove(C.addressof(ctx), C.addressof(other), C.sizeof(D.LshCtx))
    for _ in range(4):
        w = rng.standard_normal(128).astype(np.float32)
        assert dl.lsh_hash(C.byref(ctx), D.ptr(w)) == orc.lsh_hash(hp7, w)
    # lsh_init again in place: back to seed 42
    dl.lsh_init(C.byref(ctx), 128, 42)
    assert dl.lsh_hash(C.byref(ctx), D.ptr(v)) == orc.lsh_hash(hp42, v)

    # an index searched once (its hashes uploaded), then replaced in place by
    # another index with as many blocks but other hashes
    idx, repl = D.LshIndex(), D.LshIndex()
    dl.lsh_index_init(C.byref(idx))
    dl.lsh_index_init(C.byref(repl))
    want = OracleIndex(orc, 4096)
    for i in range(300):
        dl.lsh_insert_block(C.byref(idx), int(rng.choice([0x1234, 0x1235, 0x9234])), i, 1)
        h = int(rng.choice([0x1234, 0x0F0F, 0x1236, 0x5234]))
        dl.lsh_insert_block(C.byref(repl), h, i, 1)
        want.insert(h, i, 1)
    ids = np.zeros(64, np.int32)
    dl.lsh_find_candidates(C.byref(idx), 0x1234, D.ptr(ids), 64)
    C.memmove(C.addressof(idx), C.addressof(repl), C.sizeof(D.LshIndex))
    for qh in (0x1234, 0x0F0F, 0x5234):
        n = dl.lsh_find_candidates(C.byref(idx), qh, D.ptr(ids), 64)
        np.testing.assert_array_equal(ids[:n], want.candidates(qh, 64))

    # an index with a half-summed active block, replaced in place by a fresh
    # index: the next block's hash is that of its own 64 keys only
    acc = D.LshIndex()
    dl.lsh_index_init(C.byref(acc))
    for t in range(10):
        dl.lsh_update(C.byref(acc), C.byref(ctx), D.ptr(rng.standard_normal(128).astype(np.float32)), 128, t)
    fresh = D.LshIndex()
    dl.lsh_index_init(C.byref(fresh))
    C.memmove(C.addressof(acc), C.addressof(fresh), C.sizeof(D.LshIndex))
    keys = rng.standard_normal((64, 128)).astype(np.float32)
    for t in range(64):
        dl.lsh_update(C.byref(acc), C.byref(ctx), D.ptr(keys[t]), 128, 100 + t)
    s_ = np.zeros(128, np.float32)
    for t in range(64):
        s_ = (s_ + keys[t]).astype(np.float32)
    assert acc.n_blocks == 1 and acc.block_starts[0] == 100
    assert acc.block_hashes[0] == orc.lsh_hash(hp42, (s_ * np.float32(1.0 / 64)).astype(np.float32))
    for x in (idx, repl, acc, fresh):
        dl.lsh_index_release(C.byref(x))
    dl.lsh_ctx_release(C.byref(ctx))
    dl.lsh_ctx_release(C.byref(other))


def test_block_manager_reinitialised_in_place(be, dl, orc):
    """block_manager_init twice on one struct (other shapes the second time):
    the second pool serves every call (paged.c:29-110, :195-272)."""
    bm = D.BlockManager()
    assert dl.block_manager_init(C.byref(bm), 2, 2, 64, 8) == 0
    assert dl.block_manager_init(C.byref(bm), 1, 4, 128, 4) == 0
    assert (bm.n_layers, bm.n_kv_heads, bm.head_dim, bm.max_logical) == (1, 4, 128, 4)
    pkv = D.PagedKv(C.pointer(bm), 0, 0, 0)
    rng = np.random.default_rng(3)
    op = OraclePaged(orc, 1, 4, 128, 4, OR_KV_INT8)
    for t in range(20):
        k = rng.standard_normal(4 * 128).astype(np.float32)
        v = rng.standard_normal(4 * 128).astype(np.float32)
        dl.paged_kv_append(C.byref(pkv), D.ptr(k), D.ptr(v), t)
        op.append(0, k, v, t)
    assert pkv.n_blocks == 2 and bm.logical_len[0] == 2
    for pos in (0, 7, 16, 19):
        kp, vp_, ks, vs = C.c_void_p(), C.c_void_p(), C.c_float(), C.c_float()
        dl.paged_kv_get_int8(C.byref(pkv), pos, 3, C.byref(kp), C.byref(vp_), C.byref(ks), C.byref(vs))
        got = np.zeros(128, np.int8)
        be.lib.be42_memcpy_d2h(got.ctypes.data, kp, 128, None)
        arr = op.page_arrays(op.phys(0, pos // PAGE))
        kq, kscale = arr[0].reshape(4, PAGE, 128), arr[2].reshape(4, PAGE)
        assert np.array_equal(got, kq[3, pos % PAGE]) and np.float32(ks.value) == kscale[3, pos % PAGE]
    dl.block_manager_free(C.byref(bm))


def _manager(dl, n_layers, n_kv, hd, max_pages):
    bm = D.BlockManager()
    assert dl.block_manager_init(C.byref(bm), n_layers, n_kv, hd, max_pages) == 0
    pkvs = [D.PagedKv(C.pointer(bm), i, 0, 0) for i in range(n_layers)]
    return bm, pkvs


def test_paged_pipeline_drop_in(be, dl, orc):
    """inference.c's paged decode sequence: paged_kv_append per token and
    layer, then score_blocks -> select_top_k_blocks ->
    op_paged_attention_sparse, and the dense op_paged_attention."""
    rng = np.random.default_rng(77)
    n_layers, n_kv, hd, H, max_pages = 2, 4, 64, 8, 40
    bm, pkvs = _manager(dl, n_layers, n_kv, hd, max_pages)
    op = OraclePaged(orc, n_layers, n_kv, hd, max_pages, OR_KV_INT8)
    lens = (37 * PAGE + 5, 3 * PAGE + 1)
    for layer, T in enumerate(lens):
        K = rng.standard_normal((T, n_kv * hd)).astype(np.float32)
        V = rng.standard_normal((T, n_kv * hd)).astype(np.float32)
        for t in range(T):
            dl.paged_kv_append(C.byref(pkvs[layer]), D.ptr(K[t]), D.ptr(V[t]), t)
            op.append(layer, K[t], V[t], t)
    for layer, T in enumerate(lens):
        nb = op.n_blocks(layer)
        assert pkvs[layer].n_blocks == nb and pkvs[layer].n_tokens == T and bm.logical_len[layer] == nb
        for i in range(nb):
            assert bm.page_table[layer * max_pages + i] == op.phys(layer, i)
    # codes and scales of one token through paged_kv_get_int8 (device pointers)
    kp, vp, ks, vs = C.c_void_p(), C.c_void_p(), C.c_float(), C.c_float()
    dl.paged_kv_get_int8(C.byref(pkvs[0]), 21, 2, C.byref(kp), C.byref(vp), C.byref(ks), C.byref(vs))
    got = np.zeros(hd, np.int8)
    be.lib.be42_memcpy_d2h(got.ctypes.data, kp, hd, None)
    arr = op.page_arrays(op.phys(0, 1))
    kq, kscale = arr[0].reshape(n_kv, PAGE, hd), arr[2].reshape(n_kv, PAGE)
    assert np.array_equal(got, kq[2, 21 - PAGE]) and np.float32(ks.value) == kscale[2, 21 - PAGE]
    # scores and selection, bit-exact (selection order included)
    q = rng.standard_normal(H * hd).astype(np.float32)
    for layer in range(n_layers):
        nb = pkvs[layer].n_blocks
        sc = (D.BlockScore * nb)()
        dl.score_blocks(C.cast(sc, C.c_void_p), D.ptr(q), C.byref(pkvs[layer]), nb)
        want = op.score_blocks(layer, q, nb)
        got = np.array([(s.block_idx, s.phys_idx, s.score) for s in sc], dtype=object)
        assert [int(x) for x in got[:, 0]] == list(want["block_idx"])
        assert [int(x) for x in got[:, 1]] == list(want["phys_idx"])
        assert np.array_equal(np.array([s.score for s in sc], np.float32), want["score"])
        for k in (8, 64, 3):
            sel = np.zeros(k + 2, np.int32)
            n = dl.select_top_k_blocks(D.ptr(sel), C.cast(sc, C.c_void_p), nb, k)
            np.testing.assert_array_equal(sel[:n], orc.select_top_k(want, k))
        # sparse attention over the top-8 selection, dense over all pages
        sel = np.zeros(10, np.int32)
        n = dl.select_top_k_blocks(D.ptr(sel), C.cast(sc, C.c_void_p), nb, 8)
        scale = np.float32(1.0) / np.sqrt(np.float32(hd))
        out = np.zeros(H * hd, np.float32)
        dl.op_paged_attention_sparse(D.ptr(out), D.ptr(q), C.byref(bm), D.ptr(sel), n, H, n_kv, hd, C.c_float(scale))
        assert rel_err(out, op.attention_pages(q.reshape(H, hd), list(sel[:n]), H, scale)) <= 2e-5
        dl.op_paged_attention(D.ptr(out), D.ptr(q), C.byref(pkvs[layer]), H, n_kv, hd, C.c_float(scale))
        assert rel_err(out, op.attention_dense(q.reshape(H, hd), layer, H, scale)) <= 2e-5
    # centroid of a full page recomputed from its codes equals the stored one
    phys = op.phys(0, 4)
    blk = bm.blocks[phys]
    before = np.zeros(hd, np.float32)
    be.lib.be42_memcpy_d2h(before.ctypes.data, C.c_void_p(blk.centroid), hd * 4, None)
    dl.calc_block_centroid_int8(C.byref(bm.blocks[phys]), hd, n_kv)
    after = np.zeros(hd, np.float32)
    be.lib.be42_memcpy_d2h(after.ctypes.data, C.c_void_p(blk.centroid), hd * 4, None)
    assert np.array_equal(before, after) and np.array_equal(after, op.page_arrays(phys)[4])
    # reset returns the pages LIFO; block_alloc / block_free follow the same stack
    dl.paged_kv_reset(C.byref(pkvs[1]))
    op.reset(1)
    assert pkvs[1].n_blocks == 0 and bm.logical_len[1] == 0
    p = dl.block_alloc(C.byref(bm))
    assert p == op.alloc() and bm.blocks[p].start_pos == -1
    dl.block_free(C.byref(bm), p)
    op.free(p)
    assert bm.free_top == op.free_top() and bm.free_stack[bm.free_top] == p
    dl.block_manager_free(C.byref(bm))
    assert bm.capacity == 0


def test_sparse_attention_skips_unmapped_ids(be, dl, orc):
    """attention_head_paged_sparse (ops_attention.c:403-411) skips selection
    entries < 0: score_blocks marks unmapped pages -1 and
    select_top_k_blocks keeps its anchors even then.  The drop-in drops them
    on the host; an all -1 selection gives zeros, as the reference's
    memset output with sum_exp == 0."""
    rng = np.random.default_rng(5)
    n_kv, hd, H, max_pages = 2, 64, 4, 8
    bm, pkvs = _manager(dl, 1, n_kv, hd, max_pages)
    op = OraclePaged(orc, 1, n_kv, hd, max_pages, OR_KV_INT8)
    T = 5 * PAGE + 3
    K = rng.standard_normal((T, n_kv * hd)).astype(np.float32)
    V = rng.standard_normal((T, n_kv * hd)).astype(np.float32)
    for t in range(T):
        dl.paged_kv_append(C.byref(pkvs[0]), D.ptr(K[t]), D.ptr(V[t]), t)
        op.append(0, K[t], V[t], t)
    q = rng.standard_normal(H * hd).astype(np.float32)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    phys = [op.phys(0, i) for i in range(op.n_blocks(0))]
    sel = np.array([-1, phys[3], -1, phys[0], phys[5], -1], np.int32)
    out = np.zeros(H * hd, np.float32)
    dl.op_paged_attention_sparse(D.ptr(out), D.ptr(q), C.byref(bm), D.ptr(sel), len(sel), H, n_kv, hd,
                                 C.c_float(scale))
    want = op.attention_pages(q.reshape(H, hd), [phys[3], phys[0], phys[5]], H, scale)
    assert rel_err(out, want) <= 2e-5
    # the same selection from device memory
    dsel = torch.from_numpy(sel).cuda()
    out2 = np.zeros(H * hd, np.float32)
    dl.op_paged_attention_sparse(D.ptr(out2), D.ptr(q), C.byref(bm), C.c_void_p(dsel.data_ptr()), len(sel), H,
                                 n_kv, hd, C.c_float(scale))
    assert np.array_equal(out, out2)
    none = np.full(3, -1, np.int32)
    out3 = np.full(H * hd, 7.0, np.float32)
    dl.op_paged_attention_sparse(D.ptr(out3), D.ptr(q), C.byref(bm), D.ptr(none), 3, H, n_kv, hd,
                                 C.c_float(scale))
    assert not out3.any()
    dl.block_manager_free(C.byref(bm))


def test_adjacent_ops(dl, orc):
    """op_rmsnorm, op_silu_mul (F32 and BF16), rope_apply_multihead_cached and
    sample_argmax through the drop-in ABI, bit-exact against the oracle (whose
    functions are pinned to the compiled reference)."""
    rng = np.random.default_rng(31)
    # RMSNorm over 3 rows of 3072 and one column vector of 509
    for rows, dim in ((3, 3072), (1, 509)):
        x = (rng.standard_normal((rows, dim)) * 2).astype(np.float32)
        w = orc.f32_to_bf16(rng.uniform(0.5, 1.5, dim).astype(np.float32))
        out = np.zeros_like(x)
        tx = D.tensor(x, D.DTYPE_F32, rows, dim) if rows > 1 else D.tensor(x, D.DTYPE_F32, dim, 1)
        to = D.tensor(out, D.DTYPE_F32, rows, dim) if rows > 1 else D.tensor(out, D.DTYPE_F32, dim, 1)
        tw = D.tensor(w, D.DTYPE_BF16, 1, dim)
        dl.op_rmsnorm(C.byref(to), C.byref(tx), C.byref(tw), C.c_float(1e-5))
        for r in range(rows):
            np.testing.assert_array_equal(out[r], orc.rmsnorm(x[r], w, 1e-5))
    # SiLU * up, F32 and BF16 (n not a multiple of 8: the scalar remainder)
    n = 8195
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    out = np.zeros(n, np.float32)
    dl.op_silu_mul(C.byref(D.tensor(out, D.DTYPE_F32, 1, n)), C.byref(D.tensor(g, D.DTYPE_F32, 1, n)),
                   C.byref(D.tensor(u, D.DTYPE_F32, 1, n)))
    np.testing.assert_array_equal(out, orc.silu_mul(g, u))
    gb, ub = orc.f32_to_bf16(g), orc.f32_to_bf16(u)
    ob = np.zeros(n, np.uint16)
    dl.op_silu_mul(C.byref(D.tensor(ob, D.DTYPE_BF16, 1, n)), C.byref(D.tensor(gb, D.DTYPE_BF16, 1, n)),
                   C.byref(D.tensor(ub, D.DTYPE_BF16, 1, n)))
    np.testing.assert_array_equal(ob, orc.silu_mul_bf16(gb, ub))
    # RoPE over 8 heads of 128 at a position inside and one past the table
    hd, n_pos = 128, 300
    cos_t, sin_t = orc.rope_table(hd, n_pos, 1e4)
    cache = D.RopeCache(cos_t.ctypes.data, sin_t.ctypes.data, hd, n_pos)
    for pos in (257, 300):
        q = rng.standard_normal(8 * hd).astype(np.float32)
        want = orc.rope_apply(q.copy(), 8, hd, pos, cos_t, sin_t)
        dl.rope_apply_multihead_cached(D.ptr(q), 8, pos, C.byref(cache))
        np.testing.assert_array_equal(q, want)
    # argmax: F32 with equal maxima in different lanes and in the tail, BF16
    x = rng.standard_normal(4099).astype(np.float32)
    for idx in (17, 9, 4096, 3):
        x[idx] = 5.0
    tx = D.tensor(x, D.DTYPE_F32, 1, 4099)
    assert dl.sample_argmax(C.byref(tx)) == orc.argmax(x) == 9
    x[8] = 5.0
    assert dl.sample_argmax(C.byref(tx)) == orc.argmax(x) == 8
    xb = orc.f32_to_bf16(rng.standard_normal(1000).astype(np.float32))
    assert dl.sample_argmax(C.byref(D.tensor(xb, D.DTYPE_BF16, 1, 1000))) == orc.argmax_bf16(xb)


@pytest.mark.parametrize("hd,theta,factor,mscale,bf16,cache", [
    (64, 1e4, 1.0, 1.0, False, False),
    (128, 5e5, 8.0, 1.2079, False, False),      # YaRN ramp and mscale
    (128, 1e4, 4.0, 1.0, True, False),
    (96, 1e4, 1.0, 1.0, True, True),            # thetas cache, BF16
])
def test_op_rope_ctx(dl, orc, hd, theta, factor, mscale, bf16, cache):
    """op_rope with a t_rope_ctx (transformer_forward without a RoPE cache)
    through the drop-in, host and device data, bit-exact against the oracle
    (pinned to the compiled reference); ctx->pos is ignored, the tail past the
    last whole vector is untouched."""
    rng = np.random.default_rng(hd + int(factor))
    mscale = float(np.float32(mscale))
    thetas = (1.0 / (theta ** (np.arange(0, hd, 2) / hd))).astype(np.float32) if cache else None
    ctx = D.RopeCtx(hd, 999, theta, 32.0, 1.0, factor, mscale, 4096, None if thetas is None else thetas.ctypes.data)
    dt = D.DTYPE_BF16 if bf16 else D.DTYPE_F32
    for pos in (0, 1, 77, 5000, 131071):
        x = rng.standard_normal(7 * hd + 5).astype(np.float32)
        if bf16:
            x = orc.f32_to_bf16(x)
        want = orc.op_rope(x, pos, hd, theta_base=theta, factor=factor, mscale=mscale, thetas=thetas)
        got = x.copy()
        dl.op_rope(C.byref(D.tensor(got, dt, 1, got.size)), pos, C.byref(ctx))
        np.testing.assert_array_equal(got, want)
        xd = torch.from_numpy(x.view(np.int16) if bf16 else x).cuda()
        dl.op_rope(C.byref(D.tensor(xd.data_ptr(), dt, 1, x.size)), pos, C.byref(ctx))
        torch.cuda.synchronize()
        gd = xd.cpu().numpy()
        np.testing.assert_array_equal(gd.view(np.uint16) if bf16 else gd, want)


def test_lsh_diagnostics(dl, orc, capfd):
    """lsh_validate_recall and adaptive_k_cutoff (ops_lsh.c:513-668) against
    the oracle (pinned to the compiled reference); the stats counters reset
    and print as the reference."""
    rng = np.random.default_rng(44)
    for n, dim, k in ((300, 128, 32), (9000, 64, 64), (50, 128, 80)):
        q = rng.standard_normal(dim).astype(np.float32)
        keys = orc.f32_to_bf16(rng.standard_normal((n, dim)).astype(np.float32))
        lsh = rng.integers(0, n, 2 * k).astype(np.int32)
        kf = (keys.astype(np.uint32) << 16).view(np.float32)
        lsh[: k // 2] = np.argsort(-(kf @ q))[: k // 2]
        got = dl.lsh_validate_recall(D.ptr(q), D.ptr(keys), n, dim, D.ptr(lsh), len(lsh), k)
        assert got == orc.validate_recall(q, keys, lsh, k)
    p = np.sort(rng.random(200).astype(np.float32))[::-1].copy()
    p /= p.sum()
    for thr in (0.3, 0.95, 5.0):
        assert dl.adaptive_k_cutoff(D.ptr(p), None, len(p), C.c_float(thr)) == orc.adaptive_k(p, thr)
    st = D.LshStats(5, 2, 30, 40, 0, 2, 96, 2)
    dl.lsh_stats_print_atomic(C.byref(st), 64)
    out = capfd.readouterr().out
    assert "Queries: 5 (validated: 2)" in out and "Recall: 75.0%" in out and "Avg Dynamic K: 48.0" in out
    dl.lsh_stats_reset_atomic(C.byref(st))
    assert st.total_queries == 0 and st.k_samples == 0
    dl.lsh_stats_print_atomic(C.byref(st), 64)
    assert "No validation data" in capfd.readouterr().out

