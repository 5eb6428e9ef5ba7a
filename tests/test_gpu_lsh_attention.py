"""GPU LSH routing, paged KV cache and sparse attention vs the oracle.

Bit-exact: projection, hashes, candidate ids and order, page tables, INT8
codes and scales, bf16 rows, centroids, page hashes, selected pages and their
order.  Floating point: attention outputs within max-rel-err 1e-3 (fp32
accumulate) as max|out - ref| / max|ref|.
"""
import numpy as np
import pytest
import torch

from conftest import golden, rel_err
from oracle_bind import OR_KV_BF16, OR_KV_INT8, PAGE, OracleIndex, OraclePaged

pytestmark = pytest.mark.gpu

TOL = 1e-3


def bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


def test_projection_host_matches_reference(be):
    g = golden("lsh")
    for dim, seed in ((128, 42), (64, 42), (128, 7)):
        hp, hpT = be.lsh_projection(dim, seed)
        np.testing.assert_array_equal(bits(hp), bits(g[f"hp_{dim}_{seed}"]))
        np.testing.assert_array_equal(bits(hpT), bits(g[f"hpT_{dim}_{seed}"]))


def test_lsh_hash_gpu(be, orc):
    g = golden("lsh")
    rng = np.random.default_rng(200)
    for dim, seed in ((128, 42), (64, 42), (128, 7)):
        hpT = g[f"hpT_{dim}_{seed}"]
        vs = np.concatenate([g[f"vec_{dim}_{seed}"], rng.standard_normal((333, dim)).astype(np.float32)])
        out = be.lsh_hash(torch.from_numpy(vs).cuda(), torch.from_numpy(hpT).cuda()).cpu().numpy().view(np.uint16)
        want = np.array([orc.lsh_hash(hpT, v) for v in vs], np.uint16)
        np.testing.assert_array_equal(out, want)
        np.testing.assert_array_equal(out[:len(g[f"hash_{dim}_{seed}"])], g[f"hash_{dim}_{seed}"])


def _closed_form_candidates(hashes, qh, cap):
    ids = []
    for p in range(17):
        ph = qh if p == 0 else qh ^ (1 << (p - 1))
        ids += [i for i in range(len(hashes) - 1, -1, -1) if hashes[i] == ph]
    return np.array(ids[:cap], np.int32)


def test_lsh_candidates_gpu(be):
    g = golden("lsh_candidates")
    hashes = g["hashes"][:4096]         # the reference index keeps the first 4096 blocks
    qs = g["queries"]
    ht = torch.from_numpy(hashes.view(np.int16).copy()).cuda()
    qt = torch.from_numpy(qs.view(np.int16).copy()).cuda()
    for cap in (1, 64):
        ids, n = be.lsh_candidates(ht, qt, cap)
        ids, n = ids.cpu().numpy(), n.cpu().numpy()
        lens, flat = g[f"cand_{cap}_len"], g[f"cand_{cap}_ids"]
        off = 0
        for i in range(len(qs)):
            np.testing.assert_array_equal(ids[i, :n[i]], flat[off:off + lens[i]])
            off += lens[i]
    ids, n = be.lsh_candidates(ht, qt, 256)
    ids, n = ids.cpu().numpy(), n.cpu().numpy()
    for i, q in enumerate(qs):
        np.testing.assert_array_equal(ids[i, :n[i]], _closed_form_candidates(hashes, int(q), 256))


def _build(be, orc, kind, n_layers, n_kv, hd, max_pages, lens, rng, hpT, planted=None, chunks=(1, 7, 64, 100),
           kgen=None, poison=False):
    """The same appends on the GPU pool and the oracle; returns both plus the
    per-layer oracle LSH indexes (page hashes inserted as pages fill).
    poison: fill the pool's K/V rows and scales with 0xFF bytes first (NaN
    bf16 and fp32 patterns), so token slots past a page's count hold NaNs."""
    gp = be.kv_pool(be42_kind(kind), n_layers, n_kv, hd, max_pages, hpT)
    if poison:
        cap = gp.s.capacity
        row = 2 if kind == OR_KV_BF16 else 1
        for field, nbytes in (("k", cap * n_kv * PAGE * hd * row), ("v", cap * n_kv * PAGE * hd * row),
                              ("k_scale", cap * n_kv * PAGE * 4), ("v_scale", cap * n_kv * PAGE * 4)):
            ptr = getattr(gp.s, field)
            if ptr:
                be._call("be42_memset", ptr, 0xFF, nbytes, be.stream())
        torch.cuda.synchronize()
    op = OraclePaged(orc, n_layers, n_kv, hd, max_pages, kind)
    idx = [OracleIndex(orc, max_pages) for _ in range(n_layers)]
    for layer, T in enumerate(lens):
        K = rng.standard_normal((T, n_kv * hd)).astype(np.float32) if kgen is None else kgen(layer, T)
        V = rng.standard_normal((T, n_kv * hd)).astype(np.float32)
        if planted is not None:
            for pg, vec in planted(layer, T):
                K[pg * PAGE:(pg + 1) * PAGE, :hd] = vec + 0.05 * rng.standard_normal((PAGE, hd))
        pos = 0
        ci = 0
        while pos < T:
            n = min(chunks[ci % len(chunks)], T - pos)
            ci += 1
            gp.append(layer, torch.from_numpy(K[pos:pos + n]).cuda(), torch.from_numpy(V[pos:pos + n]).cuda(), pos)
            for t in range(pos, pos + n):
                op.append(layer, K[t], V[t], t)
                if t % PAGE == PAGE - 1:
                    c = op.page_arrays(op.phys(layer, t // PAGE))[4]
                    idx[layer].insert(orc.lsh_hash(hpT, c), t - PAGE + 1, PAGE)
            pos += n
    torch.cuda.synchronize()
    return gp, op, idx


def be42_kind(kind):
    return 0 if kind == OR_KV_INT8 else 1


@pytest.mark.parametrize("kind", [OR_KV_INT8, OR_KV_BF16])
def test_kv_append_matches_oracle(be, orc, kind):
    rng = np.random.default_rng(300 + kind)
    n_layers, n_kv, hd, max_pages = 3, 2, 64, 12
    _, hpT = orc.lsh_init(hd, 42)
    gp, op, _ = _build(be, orc, kind, n_layers, n_kv, hd, max_pages, (150, 37, 16), rng, hpT)
    cap = n_layers * max_pages
    pe = n_kv * PAGE * hd
    if kind == OR_KV_INT8:
        gk = gp.fetch("k", cap * pe, np.int8).reshape(cap, pe)
        gv = gp.fetch("v", cap * pe, np.int8).reshape(cap, pe)
        gks = gp.fetch("k_scale", cap * n_kv * PAGE, np.float32).reshape(cap, n_kv * PAGE)
        gvs = gp.fetch("v_scale", cap * n_kv * PAGE, np.float32).reshape(cap, n_kv * PAGE)
    else:
        gk = gp.fetch("k", cap * pe, np.uint16).reshape(cap, pe)
        # bf16 V pages are stored [kv head][dim][16 tokens]
        gv = gp.fetch("v", cap * pe, np.uint16).reshape(cap, n_kv, hd, PAGE).transpose(0, 1, 3, 2).reshape(cap, pe)
    gc = gp.fetch("centroid", cap * hd, np.float32).reshape(cap, hd)
    gnt = gp.fetch("ntok", cap, np.int32)
    gh = gp.fetch("page_hash", cap, np.uint16).reshape(n_layers, max_pages)
    gnl = gp.fetch("n_logical", n_layers, np.int32)
    gni = gp.fetch("n_indexed", n_layers, np.int32)
    gpt = gp.fetch("page_table", cap, np.int32).reshape(n_layers, max_pages)
    for layer in range(n_layers):
        nb = op.n_blocks(layer)
        assert gnl[layer] == nb
        phys = [op.phys(layer, i) for i in range(nb)]
        np.testing.assert_array_equal(gp.layer_pages(layer), phys)
        np.testing.assert_array_equal(gpt[layer, :nb], phys)
        for i, p in enumerate(phys):
            kq, vq, ks, vs, cen = op.page_arrays(p)
            nt = op.ntok(p)
            assert gnt[p] == nt
            rows = (np.arange(n_kv * PAGE) % PAGE) < nt
            np.testing.assert_array_equal(gk[p].reshape(n_kv * PAGE, hd)[rows], kq.reshape(n_kv * PAGE, hd)[rows])
            np.testing.assert_array_equal(gv[p].reshape(n_kv * PAGE, hd)[rows], vq.reshape(n_kv * PAGE, hd)[rows])
            if kind == OR_KV_INT8:
                np.testing.assert_array_equal(bits(gks[p])[rows], bits(ks)[rows])
                np.testing.assert_array_equal(bits(gvs[p])[rows], bits(vs)[rows])
            if nt == PAGE:
                np.testing.assert_array_equal(bits(gc[p]), bits(cen))
                assert gh[layer, i] == orc.lsh_hash(hpT, cen)
        assert gni[layer] == sum(1 for p in phys if op.ntok(p) == PAGE)
    # reset returns pages LIFO; re-appending reuses them in the reference order
    gp.reset(0)
    op.reset(0)
    K = rng.standard_normal((40, n_kv * hd)).astype(np.float32)
    gp.append(0, torch.from_numpy(K).cuda(), torch.from_numpy(K).cuda(), 0)
    for t in range(40):
        op.append(0, K[t], K[t], t)
    np.testing.assert_array_equal(gp.layer_pages(0), [op.phys(0, i) for i in range(op.n_blocks(0))])
    gp.close()


def _planter(orc, hpT, hd, n_heads, q_by_layer, frac, rng):
    def plant(layer, T):
        npg = T // PAGE
        qm = orc.q_mean(q_by_layer[layer], n_heads, hd)
        u = qm / np.linalg.norm(qm)
        k = max(1, int(round(frac * npg)))
        pages = rng.choice(np.arange(1, max(2, npg - 1)), size=min(k, max(1, npg - 2)), replace=False)
        return [(int(p), (6.0 * u).astype(np.float32)) for p in pages]
    return plant


@pytest.mark.parametrize("kind", [OR_KV_INT8, OR_KV_BF16])
@pytest.mark.parametrize("cap,k_sel,max_pages", [(64, 64, 140), (16, 8, 140), (256, 64, 140), (256, 40, 20000)])
def test_route_matches_oracle(be, orc, kind, cap, k_sel, max_pages):
    """With 20000 pages per layer the page table and hashes (6 bytes a page)
    do not fit in LDS next to the candidate lists and are read from HBM."""
    rng = np.random.default_rng(400 + cap + kind)
    n_layers, n_kv, hd, H = 4, 4, 64, 8
    lens = (70 * PAGE + 5, 130 * PAGE, 40 * PAGE + 3, 5 * PAGE)
    _, hpT = orc.lsh_init(hd, 42)
    q = rng.standard_normal((n_layers, H, hd)).astype(np.float32)
    gp, op, idx = _build(be, orc, kind, n_layers, n_kv, hd, max_pages, lens, rng, hpT,
                         planted=_planter(orc, hpT, hd, H, q, 0.1, rng), chunks=(64, 3, 17))
    sel, nsel, cand, ncand, qh = be.route(gp, torch.from_numpy(q).cuda(), k_sel, cap)
    sel, nsel, cand, ncand, qh = (x.cpu().numpy() for x in (sel, nsel, cand, ncand, qh))
    for layer in range(n_layers):
        want_sel, want_cand = op.route(layer, q[layer], H, hpT, idx[layer], cap, k_sel)
        np.testing.assert_array_equal(sel[layer, :nsel[layer]], want_sel)
        if op.n_blocks(layer) > k_sel:
            assert qh.view(np.uint16)[layer] == orc.lsh_hash(hpT, orc.q_mean(q[layer], H, hd))
            np.testing.assert_array_equal(cand[layer, :ncand[layer]], want_cand)
    gp.close()


@pytest.mark.parametrize("k_sel,cap", [(64, 256), (8, 64)])
def test_route_tied_scores(be, orc, k_sel, cap):
    """Pages built from three repeated patterns: equal hashes, equal centroids,
    equal scores -- the heap's strict comparisons decide the order."""
    rng = np.random.default_rng(450 + k_sel)
    n_kv, hd, H = 2, 64, 4
    pats = rng.standard_normal((3, PAGE, n_kv * hd)).astype(np.float32)

    def kgen(layer, T):
        K = np.empty((T, n_kv * hd), np.float32)
        for pg in range((T + PAGE - 1) // PAGE):
            rows = K[pg * PAGE:(pg + 1) * PAGE]
            rows[:] = pats[(pg * 7) % 3][:len(rows)]
        return K
    _, hpT = orc.lsh_init(hd, 42)
    q = np.repeat(pats[0, :, :hd].mean(axis=0)[None, None], H, axis=1).astype(np.float32)   # ~ pattern 0's centroid
    gp, op, idx = _build(be, orc, OR_KV_BF16, 1, n_kv, hd, 300, (290 * PAGE,), rng, hpT, chunks=(64,), kgen=kgen)
    sel, nsel, cand, ncand, qh = be.route(gp, torch.from_numpy(q).cuda(), k_sel, cap)
    want_sel, want_cand = op.route(0, q[0], H, hpT, idx[0], cap, k_sel)
    np.testing.assert_array_equal(cand.cpu().numpy()[0, :ncand.item()], want_cand)
    np.testing.assert_array_equal(sel.cpu().numpy()[0, :nsel.item()], want_sel)
    assert len(want_cand) > k_sel
    gp.close()


@pytest.mark.parametrize("kind", [OR_KV_INT8, OR_KV_BF16])
@pytest.mark.parametrize("n_split", [1, 3, 8])
def test_attention_matches_oracle(be, orc, kind, n_split):
    rng = np.random.default_rng(500 + kind + n_split)
    n_layers, n_kv, hd, H = 3, 2, 128, 8
    lens = (33 * PAGE + 7, 3 * PAGE, 1)
    _, hpT = orc.lsh_init(hd, 42)
    gp, op, _ = _build(be, orc, kind, n_layers, n_kv, hd, 40, lens, rng, hpT, chunks=(64,))
    q = rng.standard_normal((n_layers, H, hd)).astype(np.float32)
    scale = np.float32(1.0 / np.sqrt(np.float32(hd)))
    # dense (all pages, logical order), and an arbitrary sparse order incl. a partial page
    sels = []
    for layer in range(n_layers):
        sels.append([op.phys(layer, i) for i in range(op.n_blocks(layer))])
    p0 = sels[0]
    sels2 = [[p0[0], p0[-1]] + [p0[i] for i in (17, 3, 30, 9, 22)], [sels[1][2], sels[1][0]], sels[2]]
    for sl in (sels, sels2):
        max_sel = max(len(x) for x in sl)
        st = max(max_sel, 64)
        sel = np.full((n_layers, st), -1, np.int32)
        nsel = np.array([len(x) for x in sl], np.int32)
        for i, x in enumerate(sl):
            sel[i, :len(x)] = x
        out = be.paged_attention(gp, torch.from_numpy(q).cuda(), torch.from_numpy(sel).cuda(),
                                 torch.from_numpy(nsel).cuda(), max_sel, scale, n_split=n_split).cpu().numpy()
        for layer in range(n_layers):
            want = op.attention_pages(q[layer], sl[layer], H, scale)
            err = rel_err(out[layer].ravel(), want)
            assert err <= TOL, (layer, err)
            assert err <= 2e-5, (layer, err)      # the closed form keeps every fast_expf argument
    gp.close()


@pytest.mark.parametrize("kind", [OR_KV_INT8, OR_KV_BF16])
@pytest.mark.parametrize("n_kv,H,hd", [(8, 8, 64), (8, 24, 128), (2, 6, 64), (1, 2, 128)])
def test_attention_fused_group_shapes(be, orc, kind, n_kv, H, hd):
    """Single-kernel path (n_split 1, <= 64 pages) for every GQA group size it
    instantiates and both head dims: the tiny model (8/8, hd 64), the 3B
    model (24/8, hd 128)."""
    rng = np.random.default_rng(700 + kind + H + hd)
    lens = (64 * PAGE, 20 * PAGE + 5, 9)
    _, hpT = orc.lsh_init(hd, 42)
    gp, op, _ = _build(be, orc, kind, 3, n_kv, hd, 70, lens, rng, hpT, chunks=(64,))
    q = rng.standard_normal((3, H, hd)).astype(np.float32)
    scale = np.float32(1.0 / np.sqrt(np.float32(hd)))
    sl = [[op.phys(layer, i) for i in range(op.n_blocks(layer))] for layer in range(3)]
    sl[1] = sl[1][::-1]
    sel = np.full((3, 64), -1, np.int32)
    nsel = np.array([len(x) for x in sl], np.int32)
    for i, x in enumerate(sl):
        sel[i, :len(x)] = x
    out = be.paged_attention(gp, torch.from_numpy(q).cuda(), torch.from_numpy(sel).cuda(),
                             torch.from_numpy(nsel).cuda(), 64, scale, n_split=1).cpu().numpy()
    for layer in range(3):
        want = op.attention_pages(q[layer], sl[layer], H, scale)
        assert rel_err(out[layer].ravel(), want) <= 2e-5, layer
    gp.close()


@pytest.mark.parametrize("kind", [OR_KV_INT8, OR_KV_BF16])
def test_attention_ignores_unwritten_token_slots(be, orc, kind):
    """Pages whose last token slots were never written (a partial last page)
    hold whatever the memory held: here NaN patterns.  The dense, split and
    routed attention read those slots (whole 16-token tiles on the matrix
    cores) and must give them no weight and no value."""
    rng = np.random.default_rng(1200 + kind)
    n_kv, hd, H = 2, 128, 6
    lens = (20 * PAGE + 5, 70 * PAGE + 3)
    _, hpT = orc.lsh_init(hd, 42)
    q = rng.standard_normal((2, H, hd)).astype(np.float32)
    gp, op, idx = _build(be, orc, kind, 2, n_kv, hd, 72, lens, rng, hpT,
                         planted=_planter(orc, hpT, hd, H, q, 0.1, rng), chunks=(64, 3), poison=True)
    scale = np.float32(1.0 / np.sqrt(np.float32(hd)))
    qd = torch.from_numpy(q).cuda()
    sl = [[op.phys(layer, i) for i in range(op.n_blocks(layer))][:64] for layer in range(2)]
    sl[1][-1] = op.phys(1, op.n_blocks(1) - 1)      # the partial last page of layer 1
    sel = np.full((2, 64), -1, np.int32)
    nsel = np.array([len(x) for x in sl], np.int32)
    for i, x in enumerate(sl):
        sel[i, :len(x)] = x
    for n_split in (1, 3):
        out = be.paged_attention(gp, qd, torch.from_numpy(sel).cuda(), torch.from_numpy(nsel).cuda(), 64, scale,
                                 n_split=n_split).cpu().numpy()
        for layer in range(2):
            assert np.isfinite(out[layer]).all(), (n_split, layer)
            assert rel_err(out[layer].ravel(), op.attention_pages(q[layer], sl[layer], H, scale)) <= 2e-5
    fo, fsel, fn = be.lsh_attention(gp, qd, 64, 64, scale)
    fo, fsel, fn = fo.cpu().numpy(), fsel.cpu().numpy(), fn.cpu().numpy()
    for layer in range(2):
        want_sel, _ = op.route(layer, q[layer], H, hpT, idx[layer], 64, 64) if layer == 1 else (sl[0], None)
        np.testing.assert_array_equal(fsel[layer, :fn[layer]], want_sel)
        assert np.isfinite(fo[layer]).all(), layer
        assert rel_err(fo[layer].ravel(), op.attention_pages(q[layer], list(want_sel), H, scale)) <= 2e-5
    gp.close()


@pytest.mark.parametrize("T", [8192, 32768, 131072])
def test_lsh_attention_pipeline_c4_shape(be, orc, T):
    """configs[3] at each of its contexts (8k, 32k, 128k = 512 / 2048 / 8192
    pages): 32 query heads, 8 KV heads, head_dim 128, bf16 pages, 5% planted
    pages, top-K 64 pages, candidate cap 64.  The router (two launches) and
    the fused route + attention launch both give the oracle's candidates and
    selection bit for bit and its attention within 1e-3 (measured ~1e-6)."""
    rng = np.random.default_rng(600 + T // 8192)
    n_kv, hd, H = 8, 128, 32
    _, hpT = orc.lsh_init(hd, 42)
    q = rng.standard_normal((1, H, hd)).astype(np.float32)
    gp, op, idx = _build(be, orc, OR_KV_BF16, 1, n_kv, hd, T // PAGE + 1, (T,), rng, hpT,
                         planted=_planter(orc, hpT, hd, H, q, 0.05, rng), chunks=(64,))
    print(f"c4 T={T}: built", flush=True)
    sel, nsel, cand, ncand, qh = be.route(gp, torch.from_numpy(q).cuda(), 64, 64)
    want_sel, want_cand = op.route(0, q[0], H, hpT, idx[0], 64, 64)
    s = sel.cpu().numpy()[0, :nsel.item()]
    np.testing.assert_array_equal(s, want_sel)
    np.testing.assert_array_equal(cand.cpu().numpy()[0, :ncand.item()], want_cand)
    # 5% planted: 26 pages at 8k (all selected with the anchors), 102 / 410 at 32k / 128k (cap and top-K full)
    n_planted = int(round(0.05 * (T // PAGE)))
    assert len(want_sel) == min(64, n_planted + 2) or (T == 8192 and len(want_sel) >= n_planted)
    scale = np.float32(1.0 / np.sqrt(np.float32(hd)))
    out = be.paged_attention(gp, torch.from_numpy(q).cuda(), sel, nsel, 64, scale, n_split=1).cpu().numpy()
    want = op.attention_pages(q[0], want_sel, H, scale)
    assert rel_err(out.ravel(), want) <= TOL
    assert rel_err(out.ravel(), want) <= 2e-5
    fo, fsel, fn = be.lsh_attention(gp, torch.from_numpy(q).cuda(), 64, 64, scale)
    np.testing.assert_array_equal(fsel.cpu().numpy()[0, :fn.item()], want_sel)
    assert rel_err(fo.cpu().numpy().ravel(), want) <= 2e-5
    gp.close()


@pytest.mark.parametrize("kind", [OR_KV_INT8, OR_KV_BF16])
@pytest.mark.parametrize("cap,k_sel", [(64, 64), (16, 8), (64, 40)])
@pytest.mark.parametrize("n_kv,H,hd", [(4, 8, 64), (2, 8, 128)])
def test_lsh_attention_fused_matches_oracle(be, orc, kind, cap, k_sel, n_kv, H, hd):
    """Route + attention in one launch: the selection is the oracle's route
    (bit-exact) and the output its attention over that selection.  k 64 with
    cap 64 selects every middle candidate (the scores start while the heap
    orders them); k 8 / cap 16 and k 40 / cap 64 replace heap entries (the
    scores wait for the heap); the 3-page layers take the dense path."""
    rng = np.random.default_rng(900 + cap + k_sel + kind + hd)
    n_layers = 4
    lens = (70 * PAGE + 5, 130 * PAGE, 3 * PAGE, 2 * PAGE + 1)
    _, hpT = orc.lsh_init(hd, 42)
    q = rng.standard_normal((n_layers, H, hd)).astype(np.float32)
    gp, op, idx = _build(be, orc, kind, n_layers, n_kv, hd, 140, lens, rng, hpT,
                         planted=_planter(orc, hpT, hd, H, q, 0.1, rng), chunks=(64, 3, 17))
    scale = np.float32(1.0 / np.sqrt(np.float32(hd)))
    out, sel, nsel = be.lsh_attention(gp, torch.from_numpy(q).cuda(), k_sel, cap, scale)
    out, sel, nsel = out.cpu().numpy(), sel.cpu().numpy(), nsel.cpu().numpy()
    for layer in range(n_layers):
        want_sel, _ = op.route(layer, q[layer], H, hpT, idx[layer], cap, k_sel)
        np.testing.assert_array_equal(sel[layer, :nsel[layer]], want_sel)
        want = op.attention_pages(q[layer], list(want_sel), H, scale)
        assert rel_err(out[layer].ravel(), want) <= 2e-5, layer
    # the same as the two-launch path
    s2, n2, _, _, _ = be.route(gp, torch.from_numpy(q).cuda(), k_sel, cap)
    o2 = be.paged_attention(gp, torch.from_numpy(q).cuda(), s2, n2, k_sel, scale, n_split=1).cpu().numpy()
    assert rel_err(out.ravel(), o2.ravel()) <= 1e-6
    gp.close()


@pytest.mark.parametrize("k_sel,cap,frac", [(64, 64, 0.1), (40, 128, 0.7)])
def test_lsh_attention_split_bit_identical(be, orc, k_sel, cap, frac):
    """A launch of at most 128 (query, KV head) pairs splits each pair over
    2-16 workgroups (bf16 pages): every score, weight and 16-wave partial is
    computed as in one workgroup, so 1, 8 and 16 queries give the bits of
    the same queries inside a 24-query launch (192 pairs, one workgroup
    each).  frac 0.7 plants ~90 pages, more candidates than the slots
    scored while the heap runs (the scores then follow the heap) and more
    than the heap holds (root replacements)."""
    rng = np.random.default_rng(1300 + cap)
    n_kv, hd, H = 8, 128, 24
    lens = (70 * PAGE + 5, 130 * PAGE + 9, 3 * PAGE + 2, 90 * PAGE)
    _, hpT = orc.lsh_init(hd, 42)
    q4 = rng.standard_normal((4, H, hd)).astype(np.float32)
    gp, op, idx = _build(be, orc, OR_KV_BF16, 4, n_kv, hd, 140, lens, rng, hpT,
                         planted=_planter(orc, hpT, hd, H, q4, frac, rng), chunks=(64,))
    B = 24
    slots_np = np.array([b % 4 for b in range(B)], np.int32)
    qn = q4[slots_np] + 0.01 * rng.standard_normal((B, H, hd)).astype(np.float32)
    scale = np.float32(1.0 / np.sqrt(np.float32(hd)))
    full, fsel, fn = be.lsh_attention(gp, torch.from_numpy(qn).cuda(), k_sel, cap, scale,
                                      slots=torch.from_numpy(slots_np).cuda())
    full, fsel, fn = full.cpu().numpy(), fsel.cpu().numpy(), fn.cpu().numpy()
    for b in range(4):
        want_sel, _ = op.route(b, qn[b], H, hpT, idx[b], cap, k_sel)
        np.testing.assert_array_equal(fsel[b, :fn[b]], want_sel)
        assert rel_err(full[b].ravel(), op.attention_pages(qn[b], list(want_sel), H, scale)) <= 2e-5
    for lo, hi in ((5, 6), (8, 16), (0, 16), (1, 3)):
        o, s_, n_ = be.lsh_attention(gp, torch.from_numpy(qn[lo:hi]).cuda(), k_sel, cap, scale,
                                     slots=torch.from_numpy(slots_np[lo:hi]).cuda())
        np.testing.assert_array_equal(n_.cpu().numpy(), fn[lo:hi])
        np.testing.assert_array_equal(s_.cpu().numpy(), fsel[lo:hi])
        np.testing.assert_array_equal(bits(o.cpu().numpy()), bits(full[lo:hi]), err_msg=f"queries {lo}:{hi}")
    gp.close()


def test_lsh_attention_split_without_waiting(be, orc, monkeypatch):
    """BE42_ATTN_SPLIT_SPIN=0: a workgroup of a split pair that finds the
    others not yet arrived stops waiting at once and scores every page
    itself (the path taken when a pair's workgroups are not resident
    together); the output keeps the same bits."""
    rng = np.random.default_rng(1400)
    n_kv, hd, H = 8, 128, 24
    lens = (130 * PAGE + 9, 70 * PAGE + 5)
    _, hpT = orc.lsh_init(hd, 42)
    q2 = rng.standard_normal((2, H, hd)).astype(np.float32)
    gp, op, idx = _build(be, orc, OR_KV_BF16, 2, n_kv, hd, 140, lens, rng, hpT,
                         planted=_planter(orc, hpT, hd, H, q2, 0.1, rng), chunks=(64,))
    scale = np.float32(1.0 / np.sqrt(np.float32(hd)))
    for B in (1, 8):
        slots = torch.tensor([b % 2 for b in range(B)], dtype=torch.int32, device="cuda")
        q = torch.from_numpy(q2[[b % 2 for b in range(B)]] + 0.01 * rng.standard_normal((B, H, hd)).astype(np.float32)).cuda()
        o1, s1, n1 = be.lsh_attention(gp, q, 64, 64, scale, slots=slots)
        monkeypatch.setenv("BE42_ATTN_SPLIT_SPIN", "0")
        o2, s2, n2 = be.lsh_attention(gp, q, 64, 64, scale, slots=slots)
        monkeypatch.delenv("BE42_ATTN_SPLIT_SPIN")
        assert torch.equal(n1, n2) and torch.equal(s1, s2)
        np.testing.assert_array_equal(bits(o1.cpu().numpy()), bits(o2.cpu().numpy()), err_msg=f"batch {B}")
    gp.close()


def test_lsh_attention_many_queries(be, orc):
    """65 queries x 8 KV heads (> 512 pairs): be42_lsh_attention runs the
    router and the attention as two launches; the result equals those two
    calls, with and without a selection output."""
    rng = np.random.default_rng(990)
    n_kv, hd, H = 8, 64, 16
    lens = (70 * PAGE + 5, 130 * PAGE, 3 * PAGE, 90 * PAGE)
    _, hpT = orc.lsh_init(hd, 42)
    q4 = rng.standard_normal((4, H, hd)).astype(np.float32)
    gp, op, idx = _build(be, orc, OR_KV_BF16, 4, n_kv, hd, 140, lens, rng, hpT,
                         planted=_planter(orc, hpT, hd, H, q4, 0.1, rng), chunks=(64,))
    B = 65
    slots = torch.tensor([b % 4 for b in range(B)], dtype=torch.int32, device="cuda")
    q = torch.from_numpy(rng.standard_normal((B, H, hd)).astype(np.float32)).cuda()
    scale = np.float32(1.0 / np.sqrt(np.float32(hd)))
    out, sel, nsel = be.lsh_attention(gp, q, 64, 64, scale, slots=slots)
    out2, _, _ = be.lsh_attention(gp, q, 64, 64, scale, slots=slots, want_sel=False)
    s2, n2, _, _, _ = be.route(gp, q, 64, 64, slots=slots)
    o2 = be.paged_attention(gp, q, s2, n2, 64, scale, n_split=1)
    assert torch.equal(sel[:, :64], s2[:, :64]) and torch.equal(nsel, n2)
    assert torch.equal(out, o2) and torch.equal(out2, o2)
    for b in (0, 1, 3, 64):
        want_sel, _ = op.route(b % 4, q[b].cpu().numpy(), H, hpT, idx[b % 4], 64, 64)
        np.testing.assert_array_equal(sel[b, :nsel[b]].cpu().numpy(), want_sel)
    gp.close()
