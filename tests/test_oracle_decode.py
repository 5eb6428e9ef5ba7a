"""Oracle of the decode-step adjacents (RMSNorm, RoPE, SiLU*up, argmax) and
of the decoder loop, pinned without a GPU:
  - bit-exact against the compiled reference (oracle/_ref) where it builds;
  - against closed forms (float64 RMSNorm, rotation, sigmoid) within the
    rounding they allow, and np.argmax on untied data;
  - the decoder against an independent float64 numpy forward of the same
    weights (catches a missing residual, a swapped gate/up, a wrong norm)."""
import numpy as np
import pytest

from oracle_bind import OR_KV_INT8, OracleDecoder


def _bf16(orc, x):
    return orc.f32_to_bf16(np.asarray(x, np.float32))


@pytest.mark.parametrize("dim", [512, 3072, 13, 64])
def test_rmsnorm(orc, ref, dim):
    rng = np.random.default_rng(dim)
    x = (rng.standard_normal(dim) * 3).astype(np.float32)
    w = _bf16(orc, rng.uniform(0.5, 1.5, dim))
    got = orc.rmsnorm(x, w)
    want = np.zeros(dim, np.float32)
    ref.lib.ref_rmsnorm(want, x, w, dim, 1e-5)
    assert np.array_equal(got, want)
    x64 = x.astype(np.float64)
    wf = (w.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    exact = x64 / np.sqrt((x64 ** 2).mean() + 1e-5) * wf
    assert np.max(np.abs(got - exact)) <= 4e-7 * np.max(np.abs(exact))


@pytest.mark.parametrize("hd,theta", [(64, 1e4), (128, 5e5)])
def test_rope(orc, ref, hd, theta):
    n_pos = 300
    c, s = orc.rope_table(hd, n_pos, theta)
    rc_, rs_ = np.zeros_like(c), np.zeros_like(s)
    assert ref.lib.ref_rope_table(rc_, rs_, hd, n_pos, theta) == 0
    assert np.array_equal(c, rc_) and np.array_equal(s, rs_)
    rng = np.random.default_rng(hd)
    for pos in (0, 1, 77, 299, 300, 5000):
        x = rng.standard_normal(4 * hd).astype(np.float32)
        got = orc.rope_apply(x, 4, hd, pos, c, s)
        want = x.copy()
        ref.lib.ref_rope_apply(want, 4, hd, pos, n_pos, c, s)
        assert np.array_equal(got, want), pos
        if pos >= n_pos:
            assert np.array_equal(got, x)     # no rotation past the table
        else:
            # a rotation keeps each (i, i + hd/2) pair's norm
            h = hd // 2
            for hh in range(4):
                a, b = x[hh * hd:hh * hd + h], x[hh * hd + h:(hh + 1) * hd]
                ga, gb = got[hh * hd:hh * hd + h], got[hh * hd + h:(hh + 1) * hd]
                np.testing.assert_allclose(ga ** 2 + gb ** 2, a ** 2 + b ** 2, rtol=2e-5, atol=1e-6)


@pytest.mark.parametrize("n", [1408, 8192, 13])
def test_silu_mul(orc, ref, n):
    rng = np.random.default_rng(n)
    g = (rng.standard_normal(n) * 6).astype(np.float32)
    g[:4] = [100.0, -100.0, 0.0, -0.0]
    u = rng.standard_normal(n).astype(np.float32)
    got = orc.silu_mul(g, u)
    want = np.zeros(n, np.float32)
    ref.lib.ref_silu_mul(want, g, u, n)
    assert np.array_equal(got, want)
    # Schraudolph exp is within ~6% of exp; the sigmoid inherits less
    exact = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.max(np.abs(got - exact)) <= 0.1 * np.max(np.abs(exact))


def test_argmax(orc, ref):
    rng = np.random.default_rng(1)
    for n in (4096, 128256, 13, 5, 8, 9):
        x = rng.standard_normal(n).astype(np.float32)
        assert orc.argmax(x) == np.argmax(x) == ref.lib.ref_argmax(x.copy(), n)
    # ties: lane order decides in the vector part, the tail loses ties
    x = np.zeros(4099, np.float32)
    for idx in (17, 9, 4096, 3):   # lanes 1, 1, tail, 3
        x[idx] = 5.0
    assert orc.argmax(x) == ref.lib.ref_argmax(x.copy(), 4099) == 9
    x[8] = 5.0                     # lane 0 wins over lane 1
    assert orc.argmax(x) == ref.lib.ref_argmax(x.copy(), 4099) == 8


def tiny_model(rng, n_layers=2, dim=64, n_heads=4, n_kv=2, hd=16, hidden=96, vocab=300, kind="int8"):
    """Random-init weights in the configs[0] recipe (codes U{-127..127},
    row scales U[0.005, 0.02], norms 1.0)."""
    def q(rows, cols):
        return rng.integers(-127, 128, (rows, cols), dtype=np.int8), rng.uniform(0.005, 0.02, rows).astype(np.float32)
    one = np.full(dim, 0x3F80, np.uint16)
    layers = []
    for _ in range(n_layers):
        L = {}
        for name, (r, c) in {"wq": (n_heads * hd, dim), "wk": (n_kv * hd, dim), "wv": (n_kv * hd, dim),
                             "wo": (dim, n_heads * hd), "w1": (hidden, dim), "w3": (hidden, dim),
                             "w2": (dim, hidden)}.items():
            L[name], L["s" + name[1:]] = q(r, c)
        L["attn_norm"], L["ffn_norm"] = one, one
        layers.append(L)
    emb, emb_s = q(vocab, dim)
    out, out_s = q(vocab, dim)
    cfg = dict(n_layers=n_layers, dim=dim, n_heads=n_heads, n_kv=n_kv, hd=hd, hidden=hidden, vocab=vocab,
               max_seq=256, wkind=0, kv_kind=OR_KV_INT8, sparse_k=64, cand_cap=64, theta=1e4, eps=1e-5)
    return cfg, dict(emb=emb, emb_s=emb_s, final_norm=one, out=out, out_s=out_s, layers=layers)


def _fexp_vec(x):
    """fast_expf_avx2 (ops_math_fast.h:105-126) in numpy: clamp, fused
    12102203*x + 1065353216 (exact in float64, then rounded once), RNE."""
    x = np.clip(np.asarray(x, np.float32), -87.0, 87.0).astype(np.float64)
    f = (x * 12102203.0 + 1065353216.0).astype(np.float32)
    return np.rint(f).astype(np.int32).view(np.float32)


def numpy_forward(orc, cfg, w, tokens, cos_t, sin_t):
    """float64 restatement of the decode loop with the same quantization and
    exponential as the engine (INT8 K/V rows, online softmax over tokens with
    the scalar fast_expf, SiLU with the vector one) but no fp32 rounding of
    the linear algebra: a structural check of the composition."""
    dim, hd, H, KV = cfg["dim"], cfg["hd"], cfg["n_heads"], cfg["n_kv"]
    G = H // KV
    deq = lambda q, s: q.astype(np.float64) * s.astype(np.float64)[:, None]
    Ks = [[] for _ in w["layers"]]
    Vs = [[] for _ in w["layers"]]
    half = hd // 2

    def rope(x, pos, n):
        x = x.reshape(n, hd).copy()
        c = cos_t[pos * half:(pos + 1) * half].astype(np.float64)
        s = sin_t[pos * half:(pos + 1) * half].astype(np.float64)
        a, b = x[:, :half].copy(), x[:, half:].copy()
        x[:, :half], x[:, half:] = a * c - b * s, a * s + b * c
        return x.ravel()

    def norm(x):
        return x / np.sqrt((x ** 2).mean() + cfg["eps"])

    def kvq(x):
        rows = []
        for h in range(KV):
            q, sc = orc.quant_int8(x[h * hd:(h + 1) * hd].astype(np.float32))
            rows.append(q.astype(np.float64) * np.float64(sc))
        return np.stack(rows)
    outs = []
    for pos, tok in enumerate(tokens):
        x = w["emb"][tok].astype(np.float64) * np.float64(w["emb_s"][tok])
        for li, L in enumerate(w["layers"]):
            xb = norm(x)
            q = rope(deq(L["wq"], L["sq"]) @ xb, pos, H)
            k = rope(deq(L["wk"], L["sk"]) @ xb, pos, KV)
            v = deq(L["wv"], L["sv"]) @ xb
            Ks[li].append(kvq(k))
            Vs[li].append(kvq(v))
            K, V = np.stack(Ks[li]), np.stack(Vs[li])
            att = np.zeros((H, hd))
            for h in range(H):
                s = (K[:, h // G] @ q[h * hd:(h + 1) * hd]) / np.sqrt(hd)
                m, l, o = -np.inf, 0.0, np.zeros(hd)
                for t in range(len(s)):
                    mn = max(m, s[t])
                    a = float(orc.fast_expf(np.float32(m - mn))[0]) if m > -np.inf else 1.0
                    p_ = float(orc.fast_expf(np.float32(s[t] - mn))[0])
                    l, o, m = l * a + p_, o * a + p_ * V[t, h // G], mn
                att[h] = o / l
            x = x + deq(L["wo"], L["so"]) @ att.ravel()
            xb = norm(x)
            g, u = deq(L["w1"], L["s1"]) @ xb, deq(L["w3"], L["s3"]) @ xb
            sig = 1.0 / (1.0 + _fexp_vec(-g).astype(np.float64))
            x = x + deq(L["w2"], L["s2"]) @ (g * sig * u)
        outs.append(deq(w["out"], w["out_s"]) @ norm(x))
    return outs


def test_decoder_matches_float64_forward(orc):
    rng = np.random.default_rng(21)
    cfg, w = tiny_model(rng)
    # small weights so that the softmax and SiLU stay in their accurate range
    for L in w["layers"]:
        for k in ("sq", "sk", "sv", "so", "s1", "s2", "s3"):
            L[k] = (L[k] * 0.1).astype(np.float32)
    _, hpT = orc.lsh_init(cfg["hd"], 42)
    dec = OracleDecoder(orc, cfg, w, hpT)
    tokens = rng.integers(0, cfg["vocab"], 40)
    cos_t, sin_t = orc.rope_table(cfg["hd"], cfg["max_seq"], cfg["theta"])
    want = numpy_forward(orc, cfg, w, tokens, cos_t, sin_t)
    for pos, tok in enumerate(tokens):
        nxt, logits = dec.step(tok, pos)
        assert nxt == orc.argmax(logits)
        err = np.max(np.abs(logits - want[pos])) / np.max(np.abs(want[pos]))
        assert err < 2e-3, (pos, err)
