"""Write the golden fixtures of the decode hot path from the compiled reference.

Run where the reference tree exists (it needs oracle/_ref/libref42.so, built by
``make -C oracle ref``):

    python tests/golden/make_golden.py

Every fixture is data: seeded inputs and the reference's outputs for them.
The reference's functions are called through oracle/ref_shim.c; nothing of the
reference's source is stored here.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from oracle_bind import PAGE, RefLib  # noqa: E402


def fp8_codec(ref, rng):
    lut = ref.fp8_lut()
    # float_to_fp8 directly: a vector whose absmax is 224 has scale 1.0 exactly
    edges = []
    for e in range(-10, 10):
        b = np.float32(2.0 ** e)
        for d in (-3, -2, -1, 0, 1, 2, 3):
            edges.append(np.nextafter(b, np.float32(np.inf if d > 0 else -np.inf)) if d else b)
            if abs(d) > 1:
                v = b
                for _ in range(abs(d) * 4):
                    v = np.nextafter(v, np.float32(np.inf if d > 0 else -np.inf))
                edges.append(v)
    for base in np.arange(1.0, 2.0, 1.0 / 16, dtype=np.float32):  # half-up and no-carry points
        edges += [base, np.nextafter(base, np.float32(0)), np.nextafter(base, np.float32(4))]
    edges = np.array(edges, np.float32)
    edges = edges[(edges > 0) & (edges < 224)]
    edges = np.concatenate([edges, -edges, [224.0, 0.0, -0.0, 1e-9, 3e-4]]).astype(np.float32)
    direct_codes, direct_scale = ref.quant_fp8(edges)
    assert direct_scale == 1.0
    vecs = [rng.standard_normal(128).astype(np.float32) * s for s in (1e-3, 0.02, 1.0, 50.0)]
    vecs.append(np.zeros(32, np.float32))
    v = rng.standard_normal(257).astype(np.float32)
    v[17] = 9.0
    vecs.append(v)
    out = {"lut": lut, "direct_in": edges, "direct_codes": direct_codes}
    for i, x in enumerate(vecs):
        q, s = ref.quant_fp8(x)
        out[f"vec{i}_in"], out[f"vec{i}_codes"], out[f"vec{i}_scale"] = x, q, np.float32(s)
    return out


def int8_quant(ref, rng):
    out = {}
    cases = [rng.standard_normal(n).astype(np.float32) for n in (1, 7, 64, 128, 4096)]
    cases.append(np.zeros(16, np.float32))
    x = rng.standard_normal(128).astype(np.float32)
    x[5] = -40.0
    cases.append(x)
    half = np.array([0.5, -0.5, 1.5, -2.5, 127.0, 63.5, -63.5, 0.0], np.float32)  # exact .5 after scaling
    cases.append(half)
    for i, x in enumerate(cases):
        q, s = ref.quant_int8(x)
        out[f"c{i}_in"], out[f"c{i}_codes"], out[f"c{i}_scale"] = x, q, np.float32(s)
    return out


def lsh(ref, rng):
    out = {}
    for dim, seed in ((128, 42), (64, 42), (128, 7)):
        ctx, hp, hpT = ref.lsh_init(dim, seed)
        out[f"hp_{dim}_{seed}"] = hp
        out[f"hpT_{dim}_{seed}"] = hpT
        vs = rng.standard_normal((64, dim)).astype(np.float32)
        vs[0] = 0.0
        vs[1] = hp[3] * 1e-3           # on a hyperplane direction
        vs[2] = -hp[0]
        h = np.array([ref.lib.ref_lsh_hash(ctx, np.ascontiguousarray(v)) for v in vs], np.uint16)
        out[f"vec_{dim}_{seed}"] = vs
        out[f"hash_{dim}_{seed}"] = h
        ref.lib.ref_lsh_ctx_free(ctx)
    return out


def lsh_candidates(ref, rng):
    """A skewed hash stream (many blocks in few buckets) and several queries."""
    ix = ref.lib.ref_lsh_index_new()
    centers = rng.integers(0, 65536, 6).astype(np.uint16)
    hashes = []
    for i in range(4200):   # past LSH_MAX_BLOCKS=4096: the tail is dropped
        c = centers[rng.integers(0, len(centers))]
        r = rng.random()
        if r < 0.5:
            h = c
        elif r < 0.8:
            h = c ^ (1 << int(rng.integers(0, 16)))
        else:
            h = rng.integers(0, 65536)
        hashes.append(int(h))
        ref.lib.ref_lsh_insert(ix, int(h), i * 64, 64)
    hashes = np.array(hashes, np.uint16)
    queries = np.concatenate([centers, rng.integers(0, 65536, 6).astype(np.uint16),
                              centers ^ np.uint16(1 << 3)]).astype(np.uint16)
    out = {"hashes": hashes, "queries": queries}
    for cap in (1, 64, 300, 5000):
        rows = []
        for qh in queries:
            ids = np.zeros(cap, np.int32)
            n = ref.lib.ref_lsh_candidates(ix, int(qh), ids, cap)
            rows.append(ids[:n])
        out[f"cand_{cap}_len"] = np.array([len(r) for r in rows], np.int32)
        out[f"cand_{cap}_ids"] = np.concatenate(rows).astype(np.int32) if rows else np.zeros(0, np.int32)
    ref.lib.ref_lsh_index_free(ix)
    return out


def numerics(ref, rng):
    xs = np.concatenate([np.linspace(-100, 100, 4001, dtype=np.float32),
                         rng.uniform(-90, 5, 4000).astype(np.float32),
                         np.array([-87.0, -87.00001, 87.0, 87.00001, 0.0, -0.0, -1e-30, 1e-30], np.float32)])
    fe = np.array([ref.lib.ref_fast_expf(float(x)) for x in xs], np.float32)
    out = {"fexp_in": xs, "fexp_out": fe}
    dl, dbf, dargs_a, dargs_b, dlen = [], [], [], [], []
    for n in list(range(1, 40)) + [64, 127, 128, 129, 255, 256, 300]:
        a = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        ab = np.array([ref.lib.ref_f32_to_bf16(float(v)) for v in a], np.uint16)
        dl.append(ref.lib.ref_dot_f32_f32(a, b, n))
        dbf.append(ref.lib.ref_dot_bf16_f32(ab, b, n))
        dargs_a.append(a)
        dargs_b.append(b)
        dlen.append(n)
    out.update({"dot_len": np.array(dlen, np.int32), "dot_a": np.concatenate(dargs_a),
                "dot_b": np.concatenate(dargs_b), "dot_f32": np.array(dl, np.float32),
                "dot_bf16": np.array(dbf, np.float32)})
    bfx = np.concatenate([rng.standard_normal(500).astype(np.float32),
                          np.array([1.0, 0.0, -0.0, np.inf, -np.inf, 1.00390625, 1.01171875, 3.4e38], np.float32)])
    out["bf16_in"] = bfx
    out["bf16_out"] = np.array([ref.lib.ref_f32_to_bf16(float(v)) for v in bfx], np.uint16)
    # heap
    hs_in, hs_len, hs_cap, hs_sc, hs_ix, hs_n = [], [], [], [], [], []
    for n, cap in ((5, 2), (10, 10), (64, 62), (100, 62), (300, 62), (40, 7)):
        s = rng.standard_normal(n).astype(np.float32)
        if n == 100:
            s[::7] = 0.25   # ties
        so = np.zeros(256, np.float32)
        io = np.zeros(256, np.int32)
        m = ref.lib.ref_heap_run(s, n, cap, so, io)
        hs_in.append(s)
        hs_len.append(n)
        hs_cap.append(cap)
        hs_sc.append(so[:m])
        hs_ix.append(io[:m])
        hs_n.append(m)
    out.update({"heap_in": np.concatenate(hs_in), "heap_len": np.array(hs_len, np.int32),
                "heap_cap": np.array(hs_cap, np.int32), "heap_scores": np.concatenate(hs_sc),
                "heap_idx": np.concatenate(hs_ix), "heap_n": np.array(hs_n, np.int32)})
    return out


def matmul(ref, rng):
    out = {}
    # test_ops.c KATs through the f32 path
    a = np.array([1, 2, 3, 4, 5, 6], np.float32)
    b = np.array([1, 2, 3, 4, 5, 6], np.float32)
    o = np.zeros(4, np.float32)
    ref.lib.ref_matmul(o.ctypes.data, 0, a.ctypes.data, 0, 2, 3, b.ctypes.data, 0, 2)
    out["kat_general"] = o
    # BF16 weight x F32 vector GEMV (matvec_bf16_f32_blocked)
    for n, k in ((33, 1), (17, 7), (40, 8), (13, 31), (9, 32), (21, 100), (6, 4096), (3, 4099)):
        w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
        wb = np.array([ref.lib.ref_f32_to_bf16(float(v)) for v in w.ravel()], np.uint16).reshape(n, k)
        x = rng.standard_normal(k).astype(np.float32)
        y = np.zeros(n, np.float32)
        rc = ref.lib.ref_matmul(y.ctypes.data, 0, wb.ctypes.data, 1, n, k, x.ctypes.data, 0, 1)
        assert rc == 0
        out[f"gemv_{n}x{k}_w"] = wb
        out[f"gemv_{n}x{k}_x"] = x
        out[f"gemv_{n}x{k}_y"] = y
    return out


def paged(ref, rng):
    """INT8 paged KV: appends over two layers, scores, selection, attention."""
    n_layers, n_kv, hd, max_blocks, n_heads = 2, 2, 64, 12, 4
    r = ref.lib.ref_paged_new(n_layers, n_kv, hd, max_blocks)
    lens = (150, 37)
    ks = [rng.standard_normal((lens[l], n_kv * hd)).astype(np.float32) for l in range(n_layers)]
    vs = [rng.standard_normal((lens[l], n_kv * hd)).astype(np.float32) for l in range(n_layers)]
    ks[0][40:56] *= 4.0
    for l in range(n_layers):
        for pos in range(lens[l]):
            ref.lib.ref_paged_append(r, l, ks[l][pos], vs[l][pos], pos)
    out = {"cfg": np.array([n_layers, n_kv, hd, max_blocks, n_heads], np.int32)}
    for l in range(n_layers):
        out[f"k{l}"], out[f"v{l}"] = ks[l], vs[l]
        nb = ref.lib.ref_paged_n_blocks(r, l)
        phys = np.array([ref.lib.ref_paged_phys(r, l, i) for i in range(nb)], np.int32)
        out[f"phys{l}"] = phys
        pe = n_kv * PAGE * hd
        kq = np.zeros((nb, pe), np.int8)
        vq = np.zeros((nb, pe), np.int8)
        kss = np.zeros((nb, n_kv * PAGE), np.float32)
        vss = np.zeros((nb, n_kv * PAGE), np.float32)
        cen = np.zeros((nb, hd), np.float32)
        ntok = np.zeros(nb, np.int32)
        for i, p in enumerate(phys):
            ntok[i] = ref.lib.ref_paged_page(r, int(p), kq[i], vq[i], kss[i], vss[i], cen[i])
        out[f"kq{l}"], out[f"vq{l}"], out[f"ks{l}"], out[f"vs{l}"] = kq, vq, kss, vss
        out[f"cen{l}"], out[f"ntok{l}"] = cen, ntok
        q = rng.standard_normal(n_heads * hd).astype(np.float32)
        scale = np.float32(1.0 / np.sqrt(np.float32(hd)))
        o = np.zeros(n_heads * hd, np.float32)
        ref.lib.ref_paged_attention(r, l, o, q, n_heads, scale)
        out[f"q{l}"], out[f"dense{l}"] = q, o
        sphys = np.zeros(nb, np.int32)
        ssc = np.zeros(nb, np.float32)
        ref.lib.ref_score_blocks(r, l, q, nb, sphys, ssc)
        out[f"score{l}"] = ssc
        for kk in (3, 6):
            sel = np.zeros(nb + 2, np.int32)
            ns = ref.lib.ref_select_top_k(np.arange(nb, dtype=np.int32), sphys, ssc, nb, kk, sel)
            out[f"sel{l}_{kk}"] = sel[:ns].copy()
            o2 = np.zeros(n_heads * hd, np.float32)
            ref.lib.ref_paged_attention_sparse(r, o2, q, sel[:ns].copy(), ns, n_heads, scale)
            out[f"sparse{l}_{kk}"] = o2
    ref.lib.ref_paged_free(r)
    return out


def bf16_attention(ref, rng):
    """Linear-cache BF16 attention (flash_attention_head), the math of bf16 pages."""
    out = {}
    for i, (T, hd) in enumerate(((1, 64), (16, 64), (48, 128), (200, 128))):
        q = rng.standard_normal(hd).astype(np.float32)
        k = rng.standard_normal((T, hd)).astype(np.float32)
        v = rng.standard_normal((T, hd)).astype(np.float32)
        kb = np.array([ref.lib.ref_f32_to_bf16(float(x)) for x in k.ravel()], np.uint16)
        vb = np.array([ref.lib.ref_f32_to_bf16(float(x)) for x in v.ravel()], np.uint16)
        o = np.zeros(hd, np.float32)
        scale = np.float32(1.0 / np.sqrt(np.float32(hd)))
        ref.lib.ref_flash_attention_head(o, q, kb, vb, T, hd, scale)
        out.update({f"c{i}_q": q, f"c{i}_k": kb.reshape(T, hd), f"c{i}_v": vb.reshape(T, hd), f"c{i}_o": o})
    return out


def main():
    ref = RefLib()
    rng = np.random.default_rng(20251205)
    fixtures = {
        "fp8_codec": fp8_codec, "int8_quant": int8_quant, "lsh": lsh,
        "lsh_candidates": lsh_candidates, "numerics": numerics, "matmul": matmul,
        "paged_int8": paged, "bf16_attention": bf16_attention,
    }
    for name, fn in fixtures.items():
        data = fn(ref, rng)
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **data)
        print(f"{name}: {len(data)} arrays, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
