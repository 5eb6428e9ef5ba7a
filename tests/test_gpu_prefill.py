"""Batched prefill (be42_decoder_prefill) against the decode step run token by
token over the same prompt, on configs[0]-shaped models.

The prefill's projections are GEMMs over the GEMV's activation digit planes,
its row kernels and attention are the decode step's, and each token's
attention sees the cache as the decode step at its position saw it.  With
INT8 weights every step of that is bit-identical, so the tests require exact
equality: the KV pages of every layer (codes, scales, bf16 values,
centroids, token counts), the LSH page hashes and index counts, the last
token's logits and its argmax, and the greedy tokens generated afterwards.
With FP8 weights the matrix cores accumulate fp32 digit sums in a different
order (GEMM vs GEMV), so the logits agree to ~1e-6 relative until a K/V
element rounds to a different code; the bound there is the decode tests'
free-running one (2e-2 relative) and identical argmax outside near ties.

The token-by-token side is itself pinned to the oracle's transformer_forward
by tests/test_gpu_decode.py."""
import numpy as np
import pytest
import torch

import be42
from oracle_bind import OR_KV_BF16, OR_KV_INT8
from test_gpu_decode import configs, make_model, near_tie, to_device

pytestmark = pytest.mark.gpu


def snapshot(dec, gc):
    """Per layer slot, in logical page order: the page contents and index."""
    pool = dec.pool
    s = pool.s
    cap = s.capacity
    n_kv, hd = gc["n_kv_heads"], gc["head_dim"]
    per_page = n_kv * 16 * hd
    bf16 = gc["kv_kind"] == be42.KV_BF16
    kdt = np.uint16 if bf16 else np.int8
    k = pool.fetch("k", cap * per_page, kdt).reshape(cap, -1)
    v = pool.fetch("v", cap * per_page, kdt).reshape(cap, -1)
    ks = vs = None
    if not bf16:
        ks = pool.fetch("k_scale", cap * n_kv * 16, np.float32).reshape(cap, -1)
        vs = pool.fetch("v_scale", cap * n_kv * 16, np.float32).reshape(cap, -1)
    cen = pool.fetch("centroid", cap * hd, np.float32).reshape(cap, hd)
    ntok = pool.fetch("ntok", cap, np.int32)
    nslot = gc["n_layers"] * gc["max_batch"]
    ml = pool.max_logical
    ph = pool.fetch("page_hash", nslot * ml, np.uint16).reshape(nslot, ml)
    nidx = pool.fetch("n_indexed", nslot, np.int32)
    nlog = pool.fetch("n_logical", nslot, np.int32)
    # token slots at or past a page's count hold whatever the memory held
    # before (the pool is not cleared): compare written slots only
    tok = np.arange(16)
    out = []
    for slot in range(nslot):
        pages = pool.layer_pages(slot)
        sealed = pages[: nidx[slot]]
        nt = ntok[pages]
        live = tok[None, :] < nt[:, None]                                   # [page][token]
        kk = np.where(live[:, None, :, None], k[pages].reshape(-1, n_kv, 16, hd), 0)
        if bf16:   # V pages [kv head][dim][token]
            vv = np.where(live[:, None, None, :], v[pages].reshape(-1, n_kv, hd, 16), 0)
        else:
            vv = np.where(live[:, None, :, None], v[pages].reshape(-1, n_kv, 16, hd), 0)
        sc = lambda a: None if a is None else np.where(live[:, None, :], a[pages].reshape(-1, n_kv, 16), 0)
        out.append(dict(n_logical=int(nlog[slot]), n_indexed=int(nidx[slot]), ntok=nt, k=kk, v=vv, ks=sc(ks),
                        vs=sc(vs), centroid=cen[sealed], hash=ph[slot, : nidx[slot]].copy()))
    return out


def assert_same_cache(a, b, exact=True):
    assert len(a) == len(b)
    for slot, (x, y) in enumerate(zip(a, b)):
        assert x["n_logical"] == y["n_logical"] and x["n_indexed"] == y["n_indexed"], slot
        np.testing.assert_array_equal(x["ntok"], y["ntok"], err_msg=f"slot {slot}")
        if exact:
            for f in ("k", "v", "ks", "vs", "centroid", "hash"):
                if x[f] is not None:
                    np.testing.assert_array_equal(x[f], y[f], err_msg=f"slot {slot} {f}")


def build(be, orc, kind, kv_kind, sparse_k, cap, max_seq, max_batch=1, seed=2024, dims=(4, 512, 8, 8, 64, 1408, 4096)):
    rng = np.random.default_rng(seed)
    L, dim, H, KV, hd, hidden, vocab = dims
    w = make_model(rng, L, dim, H, KV, hd, hidden, vocab, kind)
    oc, gc = configs(L, dim, H, KV, hd, hidden, vocab, max_seq, max_batch, kind, kv_kind, sparse_k, cap)
    _, hpT = orc.lsh_init(hd, 42)
    wd = to_device(w)
    return rng, gc, wd, hpT


def token_by_token(be, gc, wd, hpT, prompt, n_gen):
    dec = be42.Decoder(be, gc, wd, hpT)
    vocab = gc["vocab"]
    lg = torch.empty((1, vocab), device="cuda")
    nxt = None
    for pos, t in enumerate(prompt):
        nxt = int(dec.step([int(t)], pos, logits=lg)[0])
    last = lg[0].cpu().numpy().copy()
    snap = snapshot(dec, gc)
    gen = [nxt]
    for i in range(n_gen - 1):
        gen.append(int(dec.step([gen[-1]], len(prompt) + i)[0]))
    dec.close()
    return last, snap, gen


def prefilled(be, gc, wd, hpT, prompt, n_gen, splits=None):
    dec = be42.Decoder(be, gc, wd, hpT)
    lg = torch.empty(gc["vocab"], device="cuda")
    cuts = [0] + list(splits or []) + [len(prompt)]
    nxt = None
    for a, b in zip(cuts[:-1], cuts[1:]):
        nxt = dec.prefill(prompt[a:b], pos0=a, logits=lg)
    last = lg.cpu().numpy().copy()
    snap = snapshot(dec, gc)
    gen = [nxt]
    for i in range(n_gen - 1):
        gen.append(int(dec.step([gen[-1]], len(prompt) + i)[0]))
    dec.close()
    return last, snap, gen


@pytest.mark.parametrize("kv_kind", [OR_KV_INT8, OR_KV_BF16])
@pytest.mark.parametrize("sparse_k,n,splits", [(64, 128, None), (8, 200, None), (8, 300, None), (8, 333, [100, 117])])
def test_prefill_int8_bit_identical(be, orc, kv_kind, sparse_k, n, splits):
    """Dense (128 tokens, 8 pages <= 64) and LSH-routed (sparse_k 8: from page
    9 on each token routes) prompts, one pass, two passes (300 > 256) and
    three calls at pos0 = 0, 100, 117."""
    rng, gc, wd, hpT = build(be, orc, "int8", kv_kind, sparse_k, 64, 512)
    prompt = rng.integers(0, gc["vocab"], n)
    l1, s1, g1 = token_by_token(be, gc, wd, hpT, prompt, 8)
    l2, s2, g2 = prefilled(be, gc, wd, hpT, prompt, 8, splits)
    assert_same_cache(s1, s2)
    np.testing.assert_array_equal(l1, l2)
    assert g1 == g2


@pytest.mark.parametrize("kv_kind", [OR_KV_INT8, OR_KV_BF16])
def test_prefill_fp8_close(be, orc, kv_kind):
    rng, gc, wd, hpT = build(be, orc, "fp8", kv_kind, 8, 64, 512)
    prompt = rng.integers(0, gc["vocab"], 270)
    l1, s1, g1 = token_by_token(be, gc, wd, hpT, prompt, 1)
    l2, s2, g2 = prefilled(be, gc, wd, hpT, prompt, 1)
    assert_same_cache(s1, s2, exact=False)
    err = np.max(np.abs(l1 - l2)) / np.max(np.abs(l1))
    assert err <= 2e-2, err
    assert g1[0] == g2[0] or near_tie(l1), (g1[0], g2[0])


def test_prefill_two_sequences_then_batched_steps(be, orc):
    """Sequences 0 and 1 prefilled separately, then batched greedy steps fed
    from the device argmax (tokens == NULL), against the batch-2 decode step
    run over both prompts token by token."""
    rng, gc, wd, hpT = build(be, orc, "int8", OR_KV_INT8, 8, 64, 512, max_batch=2)
    prompts = [rng.integers(0, gc["vocab"], 180) for _ in range(2)]
    n = len(prompts[0])
    ref = be42.Decoder(be, gc, wd, hpT)
    lg = torch.empty((2, gc["vocab"]), device="cuda")
    for pos in range(n):
        nxt = ref.step([int(prompts[0][pos]), int(prompts[1][pos])], pos, logits=lg)
    ref_first = [int(x) for x in nxt]
    ref_snap = snapshot(ref, gc)
    ref_gen = [ref_first]
    for i in range(5):
        ref_gen.append([int(x) for x in ref.step(None, n + i, batch=2)])
    ref.close()

    dec = be42.Decoder(be, gc, wd, hpT)
    firsts = [dec.prefill(prompts[b], seq=b) for b in range(2)]
    assert firsts == ref_first
    assert_same_cache(ref_snap, snapshot(dec, gc))
    gen = [firsts]
    for i in range(5):
        gen.append([int(x) for x in dec.step(None, n + i, batch=2)])
    dec.close()
    assert gen == ref_gen


def test_prefill_rejects_bad_arguments(be, orc):
    rng, gc, wd, hpT = build(be, orc, "int8", OR_KV_INT8, 8, 64, 64)
    dec = be42.Decoder(be, gc, wd, hpT)
    with pytest.raises(be42.Be42Error, match="positions"):
        dec.prefill(np.zeros(65, np.int32))
    with pytest.raises(be42.Be42Error, match="sequence"):
        dec.prefill(np.zeros(4, np.int32), seq=1)
    with pytest.raises(be42.Be42Error, match="out of range"):
        dec.prefill(np.array([gc["vocab"]], np.int32))
    dec.close()


@pytest.mark.parametrize("splits", [None, [100]])
def test_prefill_fp8_forced_kv_against_oracle(be, orc, splits):
    """FP8 weights and bf16 pages, against the oracle's transformer_forward
    (not the GPU's own decode step): the prompt through be42_decoder_prefill
    (one call, or two at pos0 = 0 and 100), then 8 greedy decode steps.  The
    oracle runs the same tokens one at a time, fed the K/V rows the GPU wrote
    (for the prompt: read back from the bf16 pages, values the oracle's own
    bf16 rounding keeps; for the decode steps: captured per layer), so both
    caches hold the same values.  The last prompt token's logits and every
    decode step's must agree within the north star's 1e-3 (max|dl| / max|l|),
    and the tokens must be identical outside near ties."""
    from oracle_bind import OracleDecoder
    rng = np.random.default_rng(808)
    dims = (4, 512, 8, 8, 64, 1408, 4096)
    L, dim, H, KV, hd, hidden, vocab = dims
    w = make_model(rng, *dims, "fp8")
    oc, gc = configs(*dims, 512, 1, "fp8", OR_KV_BF16, 8, 64)
    _, hpT = orc.lsh_init(hd, 42)
    dec = be42.Decoder(be, gc, to_device(w), hpT)
    prompt = rng.integers(0, vocab, 270)
    lg = torch.empty(vocab, device="cuda")
    cuts = [0] + list(splits or []) + [len(prompt)]
    nxt = None
    for a, b in zip(cuts[:-1], cuts[1:]):
        nxt = dec.prefill(prompt[a:b], pos0=a, logits=lg)
    gl = lg.cpu().numpy().copy()
    snap = snapshot(dec, gc)
    f32 = lambda u: (np.asarray(u, np.uint16).astype(np.uint32) << 16).view(np.float32)  # noqa: E731
    n = len(prompt)
    fk = np.zeros((n, L, KV * hd), np.float32)
    fv = np.zeros_like(fk)
    for layer in range(L):
        k, v = snap[layer]["k"], snap[layer]["v"]        # [page][kv][16][hd], [page][kv][hd][16]
        for t in range(n):
            fk[t, layer] = f32(k[t // 16][:, t % 16, :]).ravel()
            fv[t, layer] = f32(v[t // 16][:, :, t % 16]).ravel()
    od = OracleDecoder(orc, oc, w, hpT)
    ol = None
    for t in range(n):
        on, ol = od.step(int(prompt[t]), t, force_k=fk[t], force_v=fv[t])
    err = np.max(np.abs(gl - ol)) / np.max(np.abs(ol))
    assert err <= 1e-3, err
    assert nxt == on or near_tie(ol), (nxt, on)
    if nxt != on:
        dec.close()
        return
    ck = torch.zeros((L, 1, KV * hd), device="cuda")
    cv = torch.zeros_like(ck)
    dec.capture_kv(ck, cv)
    lg2 = torch.empty((1, vocab), device="cuda")
    cur = nxt
    for i in range(8):
        g = int(dec.step([cur], n + i, logits=lg2)[0])
        on, ol = od.step(cur, n + i, force_k=ck[:, 0].cpu().numpy(), force_v=cv[:, 0].cpu().numpy())
        err = np.max(np.abs(lg2[0].cpu().numpy() - ol)) / np.max(np.abs(ol))
        assert err <= 1e-3, (i, err)
        if g != on:
            assert near_tie(ol), (i, g, on)
            break
        cur = g
    dec.close()
