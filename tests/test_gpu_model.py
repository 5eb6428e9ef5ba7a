"""Checkpoint loader on the GPU: a decoder loaded from a safetensors file
(be42_model_load) gives the same logits, bit for bit, as a decoder built
directly from the same weight codes -- for INT8 and FP8 codes stored as
such (I8 / F8_E4M3 + per-row F32 scales), and for BF16 / F32 weights that the
loader quantizes on load (compared with the library's codecs applied to the
same values, which test_gpu_quant pins to the oracle)."""
import numpy as np
import pytest
import torch

import be42
from checkpoint import fp8_values, write_checkpoint, write_config
from test_gpu_decode import configs, make_model, to_device
from oracle_bind import OR_KV_INT8, OR_KV_BF16

pytestmark = pytest.mark.gpu

TINY = dict(n_layers=4, dim=512, n_heads=8, n_kv=8, hd=64, hidden=1408, vocab=4096)


def run(dec, tokens, n_gen, vocab):
    logits = torch.empty((1, vocab), device="cuda")
    out, cur = [], int(tokens[0])
    for pos in range(len(tokens) + n_gen - 1):
        nxt = dec.step([cur], pos, logits=logits)
        out.append(logits.cpu().numpy().copy())
        cur = int(tokens[pos + 1]) if pos + 1 < len(tokens) else int(nxt[0])
    return np.array(out)


def requantized(be, w, kind, fmt, quant):
    """The codes the loader makes of a bf16 / f32 file: the stored values
    (code * scale, rounded to bf16 for BF16 files) quantized per row."""
    def one(codes, scale):
        vals = (codes.astype(np.float32) if kind == "int8" else fp8_values(codes)) * scale[:, None]
        t = torch.from_numpy(vals.astype(np.float32))
        if fmt == "bf16":
            t = t.to(torch.bfloat16).float()
        q, s = (be.quant_rows_fp8 if quant == "fp8" else be.quant_rows_int8)(t.cuda())
        return q.cpu().numpy(), s.cpu().numpy()
    out = {k: v for k, v in w.items() if k not in ("layers",)}
    out["emb"], out["emb_s"] = one(w["emb"], w["emb_s"])
    out["out"], out["out_s"] = one(w["out"], w["out_s"])
    out["layers"] = []
    for L in w["layers"]:
        M = dict(L)
        for k in ("wq", "wk", "wv", "wo", "w1", "w2", "w3"):
            M[k], M["s" + k[1:]] = one(L[k], L["s" + k[1:]])
        out["layers"].append(M)
    return out


@pytest.mark.parametrize("kind,names,fmt,quant,kv", [
    ("int8", "hf", "codes", "int8", OR_KV_INT8),
    ("fp8", "llama", "codes", "fp8", OR_KV_BF16),
    ("fp8", "hf", "bf16", "fp8", OR_KV_BF16),
    ("int8", "llama", "f32", "int8", OR_KV_INT8),
])
def test_loaded_model_matches_direct_decoder(be, orc, tmp_path, kind, names, fmt, quant, kv):
    rng = np.random.default_rng(77)
    w = make_model(rng, TINY["n_layers"], TINY["dim"], TINY["n_heads"], TINY["n_kv"], TINY["hd"],
                   TINY["hidden"], TINY["vocab"], kind)
    m, c = str(tmp_path / "m.safetensors"), str(tmp_path / "config.json")
    write_checkpoint(m, w, kind, names=names, fmt=fmt)
    write_config(c, **TINY, theta=10000.0)
    qkind = 0 if quant == "int8" else 1
    model = be42.Model(be, m, c, max_seq=256, max_batch=1, kv_kind=be42.KV_INT8 if kv == OR_KV_INT8 else be42.KV_BF16,
                       quant_kind=qkind)
    assert model.cfg["wkind"] == qkind and model.cfg["norm_eps"] == np.float32(1e-5)
    direct_w = w if fmt == "codes" else requantized(be, w, kind, fmt, quant)
    _, gc = configs(*(TINY[k] for k in ("n_layers", "dim", "n_heads", "n_kv", "hd", "hidden", "vocab")),
                    256, 1, quant, kv, 64, 64)
    _, hpT = orc.lsh_init(TINY["hd"], 42)
    direct = be42.Decoder(be, gc, to_device(direct_w), hpT)
    tokens = rng.integers(0, TINY["vocab"], 24)
    a = run(model, tokens, 8, TINY["vocab"])
    b = run(direct, tokens, 8, TINY["vocab"])
    model.close()
    direct.close()
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("kind,kv", [("int8", OR_KV_INT8), ("fp8", OR_KV_BF16)])
def test_loaded_model_against_oracle(be, orc, tmp_path, kind, kv):
    """A checkpoint of stored codes (I8 / F8_E4M3 + F32 row scales), loaded by
    be42_model_load, against the oracle's transformer_forward on the same
    numpy weights (not against another GPU decoder): 24 prompt tokens, then
    greedy steps, the oracle fed the K/V rows the loaded decoder appended
    (captured per layer), so both caches hold the same codes.  Every step's
    logits within the north star's 1e-3 (max|dl| / max|l|), tokens
    identical outside near ties."""
    from oracle_bind import OracleDecoder
    from test_gpu_decode import near_tie
    rng = np.random.default_rng(91)
    dims = tuple(TINY[k] for k in ("n_layers", "dim", "n_heads", "n_kv", "hd", "hidden", "vocab"))
    w = make_model(rng, *dims, kind)
    m, c = str(tmp_path / "m.safetensors"), str(tmp_path / "config.json")
    write_checkpoint(m, w, kind, names="hf", fmt="codes")
    write_config(c, **TINY, theta=10000.0)
    model = be42.Model(be, m, c, max_seq=256, max_batch=1, kv_kind=be42.KV_INT8 if kv == OR_KV_INT8 else be42.KV_BF16,
                       quant_kind=0 if kind == "int8" else 1)
    oc, _ = configs(*dims, 256, 1, kind, kv, 64, 64)
    _, hpT = orc.lsh_init(TINY["hd"], 42)                 # the loader's default projection seed
    od = OracleDecoder(orc, oc, w, hpT)
    L, kd, V = TINY["n_layers"], TINY["n_kv"] * TINY["hd"], TINY["vocab"]
    ck = torch.zeros((L, 1, kd), device="cuda")
    cv = torch.zeros_like(ck)
    model.capture_kv(ck, cv)
    logits = torch.empty((1, V), device="cuda")
    tokens = rng.integers(0, V, 24)
    cur = int(tokens[0])
    for pos in range(24 + 8 - 1):
        nxt = int(model.step([cur], pos, logits=logits)[0])
        on, ol = od.step(cur, pos, force_k=ck[:, 0].cpu().numpy(), force_v=cv[:, 0].cpu().numpy())
        gl = logits[0].cpu().numpy()
        err = np.max(np.abs(gl - ol)) / np.max(np.abs(ol))
        assert err <= 1e-3, (pos, err)
        if pos >= 23 and nxt != on:
            assert near_tie(ol), (pos, nxt, on)
            break
        cur = int(tokens[pos + 1]) if pos + 1 < 24 else nxt
    model.close()
