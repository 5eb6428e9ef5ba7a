"""Pin the CPU oracle before trusting it.

Each oracle function is checked three ways where possible:
  * against golden fixtures written from the compiled reference
    (tests/golden/make_golden.py) -- bit-exact;
  * against the compiled reference itself on fresh seeded inputs, when
    oracle/_ref is built here;
  * against what the mathematics fixes independently of the reference
    (closed forms, brute force in float64, an independent E4M3 decoder,
    invariants), chosen so a dropped term, wrong index or transposed operand
    fails.
"""
import numpy as np
import pytest
import torch

from conftest import golden
from oracle_bind import OR_KV_BF16, OR_KV_INT8, PAGE, OracleIndex, OraclePaged


def bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


# --------------------------------------------------------------------------- numerics
def test_fast_expf_golden(orc):
    g = golden("numerics")
    out = orc.fast_expf(g["fexp_in"])
    np.testing.assert_array_equal(bits(out), bits(g["fexp_out"]))


def test_fast_expf_closed_form(orc):
    # Schraudolph: exact at 0, zero below -87, saturates at 87, overestimates
    # exp by at most ~6.2% (2^f vs 1+f).
    assert orc.fast_expf([0.0])[0] == 1.0
    assert orc.fast_expf([-87.5])[0] == 0.0
    assert orc.fast_expf([300.0])[0] == orc.fast_expf([87.0])[0]
    xs = np.linspace(-80, 80, 20001, dtype=np.float32)
    r = orc.fast_expf(xs).astype(np.float64) / np.exp(xs.astype(np.float64))
    assert r.min() > 0.999 and r.max() < 1.0625


def test_bf16_golden(orc):
    g = golden("numerics")
    out = np.array([orc.lib.or_f32_to_bf16(float(v)) for v in g["bf16_in"]], np.uint16)
    np.testing.assert_array_equal(out, g["bf16_out"])
    assert orc.lib.or_f32_to_bf16(1.0) == 0x3F80          # test_tensor.c:252-253
    # RNE independent check against torch's bfloat16 cast for finite values
    x = np.random.default_rng(1).standard_normal(4096).astype(np.float32)
    t = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(orc.f32_to_bf16(x), t)


def test_dot_golden(orc):
    g = golden("numerics")
    off = 0
    for n, want, want_bf in zip(g["dot_len"], g["dot_f32"], g["dot_bf16"]):
        a = np.ascontiguousarray(g["dot_a"][off:off + n])
        b = np.ascontiguousarray(g["dot_b"][off:off + n])
        off += n
        assert bits([orc.lib.or_dot_f32_f32(a, b, int(n))])[0] == bits([want])[0], n
        ab = orc.f32_to_bf16(a)
        assert bits([orc.lib.or_dot_bf16_f32(ab, b, int(n))])[0] == bits([want_bf])[0], n


def test_dot_brute_force(orc):
    rng = np.random.default_rng(2)
    for n in (1, 8, 13, 128, 1000):
        a = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        exact = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
        got = orc.lib.or_dot_f32_f32(a, b, n)
        assert abs(got - exact) <= 1e-5 * max(1.0, np.abs(a * b).sum())


# --------------------------------------------------------------------------- quant codecs
def test_int8_quant_golden(orc):
    g = golden("int8_quant")
    i = 0
    while f"c{i}_in" in g:
        q, s = orc.quant_int8(g[f"c{i}_in"])
        np.testing.assert_array_equal(q, g[f"c{i}_codes"])
        assert bits([s])[0] == bits([g[f"c{i}_scale"]])[0]
        i += 1
    assert i >= 8


def test_int8_quant_properties(orc):
    rng = np.random.default_rng(3)
    for n in (1, 5, 128, 4096):
        x = rng.standard_normal(n).astype(np.float32) * 3
        q, s = orc.quant_int8(x)
        amax = np.abs(x).max()
        assert s == np.float32(amax / np.float32(127))
        assert np.abs(q).max() == 127 and q[np.argmax(np.abs(x))] == np.sign(x[np.argmax(np.abs(x))]) * 127
        deq = q.astype(np.float32) * s
        assert np.all(np.abs(deq - x) <= s * 0.5 + 1e-6 * amax)
    q, s = orc.quant_int8(np.zeros(9, np.float32))
    assert s == 1.0 and not q.any()
    # roundf is half away from zero: 0.5 * (127/127) -> 1, -2.5 -> -3
    q, s = orc.quant_int8(np.array([127.0, 0.5, -2.5, 1.5], np.float32))
    assert s == 1.0 and list(q) == [127, 1, -3, 2]


def test_fp8_lut_golden_and_independent(orc):
    g = golden("fp8_codec")
    lut = orc.fp8_lut()
    np.testing.assert_array_equal(bits(lut), bits(g["lut"]))
    # independent decoder: torch's OCP E4M3FN; the reference has no NaN so 0x7F/0xFF differ
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    dec = codes.view(torch.float8_e4m3fn).float().numpy()
    mask = np.ones(256, bool)
    mask[[0x7F, 0xFF]] = False
    np.testing.assert_array_equal(lut[mask], dec[mask])
    assert lut[0x7F] == 480.0 and lut[0xFF] == -480.0


def test_fp8_encode_golden(orc):
    g = golden("fp8_codec")
    codes = np.array([orc.lib.or_float_to_fp8(float(v)) for v in g["direct_in"]], np.uint8)
    np.testing.assert_array_equal(codes, g["direct_codes"])
    i = 0
    while f"vec{i}_in" in g:
        q, s = orc.quant_fp8(g[f"vec{i}_in"])
        np.testing.assert_array_equal(q, g[f"vec{i}_codes"])
        assert bits([s])[0] == bits([g[f"vec{i}_scale"]])[0]
        i += 1


def test_fp8_encode_properties(orc):
    lut = orc.fp8_lut()
    enc = lambda v: orc.lib.or_float_to_fp8(float(v))  # noqa: E731
    # half-up mantissa: 1 + 1/16 (exactly between 1 and 1.125) -> 1.125
    assert lut[enc(1.0625)] == 1.125
    # no carry into the exponent: 1.99 would round to 2.0, stays 1.875
    assert lut[enc(1.99)] == 1.875
    # saturation at 448, never the 0x7F code
    assert enc(1e6) == 0x7E and lut[0x7E] == 448.0
    assert enc(-1e6) == 0xFE
    # subnormals: m/8 * 2^-6
    assert lut[enc(3.0 / 8 * 2 ** -6)] == np.float32(3.0 / 8 * 2 ** -6)
    # every representable E4M3 value (except NaN) encodes to itself
    for c in range(256):
        if c in (0x7F, 0xFF, 0x80):
            continue
        assert enc(lut[c]) == c, hex(c)


# --------------------------------------------------------------------------- LSH
def test_lsh_init_golden(orc):
    g = golden("lsh")
    for dim, seed in ((128, 42), (64, 42), (128, 7)):
        hp, hpT = orc.lsh_init(dim, seed)
        np.testing.assert_array_equal(bits(hp), bits(g[f"hp_{dim}_{seed}"]))
        np.testing.assert_array_equal(bits(hpT), bits(g[f"hpT_{dim}_{seed}"]))
        np.testing.assert_allclose(np.linalg.norm(hp.astype(np.float64), axis=1), 1.0, atol=1e-6)


def test_lsh_hash_golden_and_brute_force(orc):
    g = golden("lsh")
    for dim, seed in ((128, 42), (64, 42), (128, 7)):
        hpT = g[f"hpT_{dim}_{seed}"]
        vs = g[f"vec_{dim}_{seed}"]
        got = np.array([orc.lsh_hash(hpT, v) for v in vs], np.uint16)
        np.testing.assert_array_equal(got, g[f"hash_{dim}_{seed}"])
        # independent: sign of the float64 projection wherever it is not razor-thin
        proj = vs.astype(np.float64) @ hpT.astype(np.float64)
        want = ((proj > 0) * (1 << np.arange(16))).sum(1)
        clear = np.all(np.abs(proj) > 1e-5, axis=1)
        np.testing.assert_array_equal(got[clear], want[clear].astype(np.uint16))
        assert got[0] == 0   # zero vector: no strictly positive sum


def _brute_candidates(hashes, qh, cap):
    """Closed form of the chain walk: probes in order (exact, then bit 0..15),
    each bucket newest block first; radius 4 never rejects a distance <= 1."""
    ids = []
    for p in range(17):
        ph = qh if p == 0 else qh ^ (1 << (p - 1))
        ids += [i for i in range(len(hashes) - 1, -1, -1) if hashes[i] == ph]
    return np.array(ids[:cap], np.int32)


def test_lsh_candidates_golden_and_closed_form(orc):
    g = golden("lsh_candidates")
    hashes = g["hashes"]
    ix = OracleIndex(orc, 4096)
    for i, h in enumerate(hashes):
        ix.insert(int(h), i * 64, 64)
    assert ix.ix.n_blocks == 4096        # LSH_MAX_BLOCKS drops the tail
    for cap in (1, 64, 300, 5000):
        lens = g[f"cand_{cap}_len"]
        flat = g[f"cand_{cap}_ids"]
        off = 0
        for qh, n in zip(g["queries"], lens):
            got = ix.candidates(int(qh), cap)
            np.testing.assert_array_equal(got, flat[off:off + n])
            np.testing.assert_array_equal(got, _brute_candidates(hashes[:4096], int(qh), cap))
            off += n


def test_q_mean(orc):
    rng = np.random.default_rng(4)
    q = rng.standard_normal((32, 128)).astype(np.float32)
    want = np.zeros(128, np.float32)
    for h in range(32):
        want = (want + q[h]).astype(np.float32)
    want = (want / np.float32(32)).astype(np.float32)
    np.testing.assert_array_equal(orc.q_mean(q, 32, 128), want)


# --------------------------------------------------------------------------- heap / selection
def test_heap_golden(orc):
    g = golden("numerics")
    off = off_out = 0
    for n, cap, m in zip(g["heap_len"], g["heap_cap"], g["heap_n"]):
        s = g["heap_in"][off:off + n]
        off += n
        hs = np.zeros(256, np.float32)
        hi = np.zeros(256, np.int32)
        size = __import__("ctypes").c_int(0)
        for i, v in enumerate(s):
            orc.lib.or_heap_push(hs, hi, __import__("ctypes").byref(size), int(cap), float(v), i)
        assert size.value == m
        np.testing.assert_array_equal(hi[:m], g["heap_idx"][off_out:off_out + m])
        np.testing.assert_array_equal(bits(hs[:m]), bits(g["heap_scores"][off_out:off_out + m]))
        # independent: without ties the kept set is the top-cap by score
        if len(np.unique(s)) == len(s):
            assert set(hi[:m]) == set(np.argsort(-s, kind="stable")[:m])
        off_out += m


# --------------------------------------------------------------------------- GEMV / GEMM
def test_gemv_structure_golden(orc):
    """The GEMV row macro reproduces the reference BF16 GEMV bit for bit."""
    g = golden("matmul")
    keys = sorted({k.rsplit("_", 1)[0] for k in g.files if k.startswith("gemv_")})
    for key in keys:
        w, x, y = g[key + "_w"], g[key + "_x"], g[key + "_y"]
        n, k = w.shape
        out = np.zeros(n, np.float32)
        orc.lib.or_gemv_bf16(out, np.ascontiguousarray(w), x, n, k, 1)
        np.testing.assert_array_equal(bits(out), bits(y), err_msg=key)


def test_matmul_kat(orc):
    # test_ops.c:208-233: [[1,2,3],[4,5,6]] x [[1,2],[3,4],[5,6]] = [[22,28],[49,64]]
    g = golden("matmul")
    np.testing.assert_array_equal(g["kat_general"], [22, 28, 49, 64])
    xq = np.array([[1, 2, 3], [4, 5, 6]], np.int8)
    wq = np.array([[1, 3, 5], [2, 4, 6]], np.int8)      # W rows = output features
    one = np.ones(2, np.float32)
    np.testing.assert_array_equal(orc.gemm_i8_acc(xq, wq), [[22, 28], [49, 64]])
    np.testing.assert_array_equal(orc.gemm(xq, one, wq, one, "int8"), [[22, 28], [49, 64]])
    lut = orc.fp8_lut()
    enc = np.array([[orc.lib.or_float_to_fp8(float(v)) for v in r] for r in xq], np.uint8)
    wenc = np.array([[orc.lib.or_float_to_fp8(float(v)) for v in r] for r in wq], np.uint8)
    assert np.all(lut[enc] == xq)
    np.testing.assert_array_equal(orc.gemm(enc, one, wenc, one, "fp8"), [[22, 28], [49, 64]])


@pytest.mark.parametrize("kind", ["int8", "fp8"])
def test_gemv_quant_brute_force(orc, kind):
    rng = np.random.default_rng(5)
    lut = orc.fp8_lut()
    for n, k, b in ((37, 4096, 1), (16, 1000, 4), (8, 4099, 16), (3, 5, 2)):
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        q, sc = orc.quantize_rows(w, kind)
        x = rng.standard_normal((b, k)).astype(np.float32)
        y = orc.gemv(q, sc, x, kind)
        deq = (q.astype(np.float64) if kind == "int8" else lut[q].astype(np.float64)) * sc[:, None]
        exact = x.astype(np.float64) @ deq.T
        err = np.abs(y - exact).max() / np.abs(exact).max()
        assert err < 1e-5, (n, k, b, err)
        # transposing the operands must fail this check
        if n == k:
            assert np.abs(x.astype(np.float64) @ deq - exact).max() / np.abs(exact).max() > 1e-2


def test_gemm_brute_force(orc):
    rng = np.random.default_rng(6)
    m, n, k = 9, 13, 300
    xq = rng.integers(-127, 128, (m, k)).astype(np.int8)
    wq = rng.integers(-127, 128, (n, k)).astype(np.int8)
    acc = orc.gemm_i8_acc(xq, wq)
    np.testing.assert_array_equal(acc, xq.astype(np.int64) @ wq.astype(np.int64).T)
    sx = rng.uniform(0.01, 0.1, m).astype(np.float32)
    sw = rng.uniform(0.01, 0.1, n).astype(np.float32)
    y = orc.gemm(xq, sx, wq, sw, "int8")
    np.testing.assert_array_equal(y, (acc.astype(np.float32) * sx[:, None]).astype(np.float32) * sw[None, :])


# --------------------------------------------------------------------------- paged KV + attention
def _replay_paged(orc, g):
    n_layers, n_kv, hd, max_blocks, n_heads = [int(v) for v in g["cfg"]]
    pk = OraclePaged(orc, n_layers, n_kv, hd, max_blocks, OR_KV_INT8)
    for l in range(n_layers):
        for pos, (k, v) in enumerate(zip(g[f"k{l}"], g[f"v{l}"])):
            pk.append(l, k, v, pos)
    return pk, n_layers, n_kv, hd, n_heads


def test_paged_int8_golden(orc):
    g = golden("paged_int8")
    pk, n_layers, n_kv, hd, n_heads = _replay_paged(orc, g)
    scale = np.float32(1.0 / np.sqrt(np.float32(hd)))
    for l in range(n_layers):
        nb = pk.n_blocks(l)
        phys = np.array([pk.phys(l, i) for i in range(nb)], np.int32)
        np.testing.assert_array_equal(phys, g[f"phys{l}"])
        for i, p in enumerate(phys):
            kq, vq, ks, vs, cen = pk.page_arrays(p)
            np.testing.assert_array_equal(kq, g[f"kq{l}"][i])
            np.testing.assert_array_equal(vq, g[f"vq{l}"][i])
            assert pk.ntok(p) == g[f"ntok{l}"][i]
            # the reference mallocs the scale arrays: only written slots are defined
            valid = (np.arange(n_kv * PAGE) % PAGE) < pk.ntok(p)
            np.testing.assert_array_equal(bits(ks)[valid], bits(g[f"ks{l}"][i])[valid])
            np.testing.assert_array_equal(bits(vs)[valid], bits(g[f"vs{l}"][i])[valid])
            if pk.ntok(p) == PAGE:
                np.testing.assert_array_equal(bits(cen), bits(g[f"cen{l}"][i]))
        q = g[f"q{l}"]
        np.testing.assert_array_equal(bits(pk.attention_dense(q, l, n_heads, scale)), bits(g[f"dense{l}"]))
        for kk in (3, 6):
            sel = g[f"sel{l}_{kk}"]
            out = pk.attention_pages(q, sel, n_heads, scale)
            np.testing.assert_array_equal(bits(out), bits(g[f"sparse{l}_{kk}"]))


def test_paged_centroid_closed_form(orc):
    g = golden("paged_int8")
    hd = int(g["cfg"][2])
    for i, n in enumerate(g["ntok0"]):
        if n != PAGE:
            continue
        kq = g["kq0"][i][:PAGE * hd].reshape(PAGE, hd)   # head 0 rows
        ks = g["ks0"][i][:PAGE]
        c = np.zeros(hd, np.float32)
        for t in range(PAGE):
            c = (c + (kq[t].astype(np.float32) * ks[t]).astype(np.float32)).astype(np.float32)
        c = (c * np.float32(1.0 / 16)).astype(np.float32)
        np.testing.assert_array_equal(bits(c), bits(g["cen0"][i]))


def test_paged_centroid_bf16_closed_form(orc):
    """or_centroid_bf16: the bf16-page centroid (calc_block_centroid_int8,
    paged.c:350-393, on bf16 rows) through the append path.  Closed form:
    head 0's rows rounded to bf16 by an independent round-to-nearest-even
    (torch), summed per dimension token by token in float32, then x (1/16);
    bit-exact.  Page 1 holds +-2^20 around small values on head 0, where a
    float32 sum in any other order (pairwise, reversed) rounds differently,
    and head 1 differs from head 0, so a wrong head, a wrong token order or
    a wrong divisor fails."""
    rng = np.random.default_rng(11)
    n_kv, hd = 2, 64
    pk = OraclePaged(orc, 1, n_kv, hd, 4, OR_KV_BF16)
    T = 3 * PAGE + 5
    K = (rng.standard_normal((T, n_kv * hd)) * 3).astype(np.float32)
    K[PAGE:2 * PAGE, :hd] = rng.uniform(0.1, 0.9, (PAGE, hd)).astype(np.float32)
    K[PAGE, :hd] = 2.0 ** 20
    K[2 * PAGE - 1, :hd] = -(2.0 ** 20)
    V = rng.standard_normal((T, n_kv * hd)).astype(np.float32)
    for t in range(T):
        pk.append(0, K[t], V[t], t)
    bf = torch.from_numpy(K).to(torch.bfloat16).to(torch.float32).numpy()
    for pg in range(pk.n_blocks(0)):
        phys = pk.phys(0, pg)
        kb = pk.page_arrays(phys)[0].reshape(n_kv, PAGE, hd)
        n = min(PAGE, T - pg * PAGE)
        # the stored rows are the independent bf16 rounding of the inputs
        np.testing.assert_array_equal((kb[0, :n].astype(np.uint32) << 16).view(np.float32), bf[pg * PAGE:pg * PAGE + n, :hd])
        if n < PAGE:
            continue
        c = np.zeros(hd, np.float32)
        for t in range(PAGE):
            c = (c + bf[pg * PAGE + t, :hd]).astype(np.float32)
        c = (c * np.float32(1.0 / 16)).astype(np.float32)
        np.testing.assert_array_equal(bits(pk.page_arrays(phys)[4]), bits(c))
        if pg == 1:
            rows = bf[PAGE:2 * PAGE, :hd]
            pair = (rows.reshape(8, 2, hd).sum(1, dtype=np.float32))
            while len(pair) > 1:
                pair = pair.reshape(-1, 2, hd).sum(1, dtype=np.float32)
            assert not np.array_equal(bits(pair[0] * np.float32(1.0 / 16)), bits(c))


def _two_pass_attention(orc, q, K, V, scale):
    """Sequential-max softmax written as prefix max + suffix products of the
    rescale factors (the formulation the GPU kernel uses), in float64 sums."""
    s = (K.astype(np.float32) @ q.astype(np.float32)).astype(np.float32) * np.float32(scale)
    m = np.maximum.accumulate(s)
    prev = np.concatenate([[-np.inf], m[:-1]])
    a = orc.fast_expf(prev - m).astype(np.float64)
    r = orc.fast_expf(s - m).astype(np.float64)
    suffix = np.concatenate([np.cumprod(a[::-1])[::-1][1:], [1.0]])
    w = r * suffix
    return (w @ V.astype(np.float64)) / w.sum()


def test_attention_invariants(orc):
    """Dense == all-pages sparse; sequential online softmax == suffix-product form."""
    rng = np.random.default_rng(7)
    n_kv, hd, n_heads = 2, 64, 4
    pk = OraclePaged(orc, 1, n_kv, hd, 8, OR_KV_INT8)
    T = 100
    K = rng.standard_normal((T, n_kv * hd)).astype(np.float32)
    V = rng.standard_normal((T, n_kv * hd)).astype(np.float32)
    for t in range(T):
        pk.append(0, K[t], V[t], t)
    q = rng.standard_normal(n_heads * hd).astype(np.float32)
    scale = np.float32(1 / 8)
    dense = pk.attention_dense(q, 0, n_heads, scale)
    pages = [pk.phys(0, i) for i in range(pk.n_blocks(0))]
    np.testing.assert_array_equal(dense, pk.attention_pages(q, pages, n_heads, scale))
    for h in range(n_heads):
        kvh = h // (n_heads // n_kv)
        Kd = np.concatenate([pk.page_arrays(p)[0].reshape(n_kv, PAGE, hd)[kvh][:pk.ntok(p)].astype(np.float32)
                             * pk.page_arrays(p)[2].reshape(n_kv, PAGE)[kvh][:pk.ntok(p), None] for p in pages])
        Vd = np.concatenate([pk.page_arrays(p)[1].reshape(n_kv, PAGE, hd)[kvh][:pk.ntok(p)].astype(np.float32)
                             * pk.page_arrays(p)[3].reshape(n_kv, PAGE)[kvh][:pk.ntok(p), None] for p in pages])
        want = _two_pass_attention(orc, q[h * hd:(h + 1) * hd], Kd, Vd, scale)
        np.testing.assert_allclose(dense[h * hd:(h + 1) * hd], want, rtol=2e-5, atol=2e-6)


def test_bf16_pages_golden(orc):
    """BF16 pages follow the reference's linear-cache BF16 attention exactly."""
    g = golden("bf16_attention")
    i = 0
    while f"c{i}_q" in g:
        q, kb, vb, o = g[f"c{i}_q"], g[f"c{i}_k"], g[f"c{i}_v"], g[f"c{i}_o"]
        T, hd = kb.shape
        pk = OraclePaged(orc, 1, 1, hd, (T + PAGE - 1) // PAGE, OR_KV_BF16)
        kf = (kb.astype(np.uint32) << 16).view(np.float32)
        vf = (vb.astype(np.uint32) << 16).view(np.float32)
        for t in range(T):
            pk.append(0, kf[t], vf[t], t)
        scale = np.float32(1.0 / np.sqrt(np.float32(hd)))
        out = pk.attention_dense(q, 0, 1, scale)
        np.testing.assert_array_equal(bits(out), bits(o))
        i += 1


def test_route_closed_form(orc):
    """or_route_pages == anchors + brute-force top-k over the candidate list."""
    rng = np.random.default_rng(8)
    n_kv, hd, n_heads, n_pages = 2, 64, 4, 90
    hp, hpT = orc.lsh_init(hd, 42)
    pk = OraclePaged(orc, 1, n_kv, hd, n_pages + 1, OR_KV_INT8)
    ix = OracleIndex(orc, 8192)
    q = rng.standard_normal(n_heads * hd).astype(np.float32)
    qm = orc.q_mean(q, n_heads, hd)
    qh = orc.lsh_hash(hpT, qm)
    planted = set(rng.choice(np.arange(1, n_pages - 1), 20, replace=False).tolist())
    T = n_pages * PAGE - 5
    for t in range(T):
        page = t // PAGE
        k = rng.standard_normal(n_kv * hd).astype(np.float32)
        if page in planted:
            k[:hd] = 6 * qm / np.linalg.norm(qm) + 0.05 * rng.standard_normal(hd)
        pk.append(0, k, rng.standard_normal(n_kv * hd).astype(np.float32), t)
        if t % PAGE == PAGE - 1:
            p = pk.phys(0, page)
            ix.insert(orc.lsh_hash(hpT, pk.page_arrays(p)[4]), page * PAGE, PAGE)
    nb = pk.n_blocks(0)
    for cap, k in ((64, 64), (16, 8), (300, 64)):
        sel, cand = pk.route(0, q, n_heads, hpT, ix, cap, k)
        hashes = np.array([orc.lsh_hash(hpT, pk.page_arrays(pk.phys(0, i))[4]) for i in range(nb - 1)], np.uint16)
        np.testing.assert_array_equal(cand, _brute_candidates(hashes, qh, cap))
        assert planted & set(cand.tolist())
        if nb <= k:
            assert list(sel) == [pk.phys(0, i) for i in range(nb)]
            continue
        mid = [c for c in cand if c not in (0, nb - 1)]
        sc = np.array([orc.lib.or_dot_f32_f32(np.ascontiguousarray(q[:hd]), pk.page_arrays(pk.phys(0, c))[4], hd)
                       for c in mid], np.float32)
        keep = min(k - 2, len(mid), 62)
        order = sorted(range(len(mid)), key=lambda i: (-sc[i], i))[:keep]
        assert sel[0] == pk.phys(0, 0) and sel[1] == pk.phys(0, nb - 1)
        assert set(sel[2:].tolist()) == {pk.phys(0, mid[i]) for i in order}


# --------------------------------------------------------------------------- live reference
def test_live_reference_random(orc, ref):
    rng = np.random.default_rng(9)
    for n in (3, 64, 128, 1000):
        x = (rng.standard_normal(n) * rng.uniform(0.01, 100)).astype(np.float32)
        q1, s1 = orc.quant_int8(x)
        q2, s2 = ref.quant_int8(x)
        np.testing.assert_array_equal(q1, q2)
        assert bits([s1])[0] == bits([s2])[0]
        f1, t1 = orc.quant_fp8(x)
        f2, t2 = ref.quant_fp8(x)
        np.testing.assert_array_equal(f1, f2)
        assert bits([t1])[0] == bits([t2])[0]
    ctx, hp, hpT = ref.lsh_init(128, 42)
    for _ in range(200):
        v = rng.standard_normal(128).astype(np.float32)
        assert orc.lsh_hash(hpT, v) == ref.lib.ref_lsh_hash(ctx, v)
    ref.lib.ref_lsh_ctx_free(ctx)
    xs = rng.uniform(-88, 88, 20000).astype(np.float32)
    np.testing.assert_array_equal(bits(orc.fast_expf(xs)),
                                  bits(np.array([ref.lib.ref_fast_expf(float(v)) for v in xs], np.float32)))


def test_live_reference_paged(orc, ref):
    rng = np.random.default_rng(10)
    n_kv, hd, n_heads, nb_max = 8, 128, 32, 80
    r = ref.lib.ref_paged_new(1, n_kv, hd, nb_max)
    pk = OraclePaged(orc, 1, n_kv, hd, nb_max, OR_KV_INT8)
    T = 70 * PAGE + 9
    for t in range(T):
        k = rng.standard_normal(n_kv * hd).astype(np.float32)
        v = rng.standard_normal(n_kv * hd).astype(np.float32)
        ref.lib.ref_paged_append(r, 0, k, v, t)
        pk.append(0, k, v, t)
    q = rng.standard_normal(n_heads * hd).astype(np.float32)
    scale = np.float32(1 / np.sqrt(128.0))
    o1 = np.zeros(n_heads * hd, np.float32)
    ref.lib.ref_paged_attention(r, 0, o1, q, n_heads, scale)
    np.testing.assert_array_equal(bits(pk.attention_dense(q, 0, n_heads, scale)), bits(o1))
    nb = pk.n_blocks(0)
    sphys = np.zeros(nb, np.int32)
    ssc = np.zeros(nb, np.float32)
    ref.lib.ref_score_blocks(r, 0, q, nb, sphys, ssc)
    sel = np.zeros(nb + 2, np.int32)
    ns = ref.lib.ref_select_top_k(np.arange(nb, dtype=np.int32), sphys, ssc, nb, 64, sel)
    sel = sel[:ns].copy()
    o2 = np.zeros(n_heads * hd, np.float32)
    ref.lib.ref_paged_attention_sparse(r, o2, q, sel, ns, n_heads, scale)
    np.testing.assert_array_equal(bits(pk.attention_pages(q, sel, n_heads, scale)), bits(o2))
    ref.lib.ref_paged_free(r)


# --------------------------------------------------------------------------- LSH diagnostics
def _recall_closed_form(q, keys_f, lsh, actual_k):
    """Brute force in float64 on untied data: the top actual_k by q . key
    (every stride-th key past 4096), recall = |lsh[:min(len, k)] & top| / k."""
    n = keys_f.shape[0]
    actual_k = min(actual_k, n)
    lk = min(len(lsh), actual_k)
    actual_k = min(actual_k, 64)
    stride = n // 4096 if n > 4096 else 1
    idx = np.arange(min(n, 4096)) * stride
    sc = keys_f[idx].astype(np.float64) @ q.astype(np.float64)
    top = set(idx[np.argsort(-sc, kind="stable")[:actual_k]].tolist())
    return sum(1 for x in lsh[:lk] if int(x) in top) / actual_k


@pytest.mark.parametrize("n,dim,k", [(300, 128, 32), (9000, 64, 64), (50, 128, 80)])
def test_validate_recall(orc, ref, n, dim, k):
    rng = np.random.default_rng(n + k)
    q = rng.standard_normal(dim).astype(np.float32)
    keys = orc.f32_to_bf16(rng.standard_normal((n, dim)).astype(np.float32))
    kf = (keys.astype(np.uint32) << 16).view(np.float32)
    sc = kf @ q
    stride = n // 4096 if n > 4096 else 1
    good = np.argsort(-sc[::stride][:4096])[:k] * stride
    lsh = np.concatenate([good[: k // 2], rng.integers(0, n, k)]).astype(np.int32)
    got = orc.validate_recall(q, keys, lsh, k)
    want = ref.lib.ref_validate_recall(q.ctypes.data, keys.ctypes.data, n, dim, lsh.ctypes.data, len(lsh), k)
    assert got == want
    assert got == pytest.approx(_recall_closed_form(q, kf, lsh, k), abs=1e-7)
    assert 0.0 < got <= 1.0


def test_adaptive_k(orc, ref):
    rng = np.random.default_rng(5)
    p = rng.random(100).astype(np.float32)
    p /= p.sum()
    p = np.sort(p)[::-1].copy()
    for thr in (0.0, 0.5, 0.95, 2.0):
        got = orc.adaptive_k(p, thr)
        assert got == ref.lib.ref_adaptive_k(p.ctypes.data, len(p), thr)
        c = np.cumsum(p.astype(np.float32), dtype=np.float32)
        want = max(1, int(np.argmax(c >= thr)) + 1) if (c >= thr).any() else len(p)
        assert got == want

