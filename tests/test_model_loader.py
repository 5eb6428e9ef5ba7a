"""Checkpoint loader, host side (no GPU): safetensors header parsing, the
reference's name mapping (src/inference/model.c:194-255) and config keys
(model.c:32-143), dtype handling and error messages, through
be42_model_check."""
import os

import numpy as np
import pytest

import be42
from checkpoint import write_checkpoint, write_config

ARCH = dict(n_layers=2, dim=64, n_heads=4, n_kv=2, hd=16, hidden=96, vocab=128)


def weights(rng, kind):
    d, H, KV, hd, F, V = (ARCH[k] for k in ("dim", "n_heads", "n_kv", "hd", "hidden", "vocab"))

    def q(r, c):
        if kind == "int8":
            return rng.integers(-127, 128, (r, c), dtype=np.int8), rng.uniform(0.005, 0.02, r).astype(np.float32)
        codes = rng.integers(0, 256, (r, c), dtype=np.uint8)
        codes[(codes & 0x7F) == 0x7F] = 0x7E
        return codes, rng.uniform(0.005, 0.02, r).astype(np.float32)
    one = np.full(d, 0x3F80, np.uint16)
    layers = []
    for _ in range(ARCH["n_layers"]):
        L = {}
        for name, (r, c) in {"wq": (H * hd, d), "wk": (KV * hd, d), "wv": (KV * hd, d), "wo": (d, H * hd),
                             "w1": (F, d), "w3": (F, d), "w2": (d, F)}.items():
            L[name], L["s" + name[1:]] = q(r, c)
        L["attn_norm"], L["ffn_norm"] = one, one
        layers.append(L)
    emb, emb_s = q(V, d)
    out, out_s = q(V, d)
    return dict(emb=emb, emb_s=emb_s, final_norm=one, out=out, out_s=out_s, layers=layers)


@pytest.fixture(scope="module")
def lib():
    return be42.load()


def paths(tmp_path, name="m"):
    return str(tmp_path / f"{name}.safetensors"), str(tmp_path / f"{name}.json")


def arch_of(cfg):
    return dict(n_layers=cfg["n_layers"], dim=cfg["dim"], n_heads=cfg["n_heads"], n_kv=cfg["n_kv_heads"],
                hd=cfg["head_dim"], hidden=cfg["hidden_dim"], vocab=cfg["vocab"])


@pytest.mark.parametrize("kind,names,fmt,style,quant,want_kind", [
    ("int8", "hf", "codes", "hf", 1, 0),
    ("fp8", "llama", "codes", "params", 0, 1),
    ("fp8", "hf", "bf16", "vlm", 1, 1),
    ("int8", "llama", "f32", "hf", 0, 0),
])
def test_check_maps_names_and_config(lib, tmp_path, kind, names, fmt, style, quant, want_kind):
    m, c = paths(tmp_path)
    write_checkpoint(m, weights(np.random.default_rng(1), kind), kind, names=names, fmt=fmt)
    write_config(c, **ARCH, theta=5000.0, style=style)
    cfg, wkind = be42.model_check(lib, m, c, quant)
    assert wkind == want_kind == cfg["wkind"]
    if style == "params":
        # params.json has no head_dim: dim / n_heads (model.c:128-134)
        assert cfg["head_dim"] == ARCH["dim"] // ARCH["n_heads"]
    assert arch_of(cfg) == ARCH
    assert cfg["rope_theta"] == 5000.0
    assert cfg["norm_eps"] == np.float32(1e-5)          # forced (model.c:139)


def test_check_tied_output_and_defaults(lib, tmp_path):
    m, c = paths(tmp_path)
    write_checkpoint(m, weights(np.random.default_rng(2), "int8"), "int8", tie_output=True)
    write_config(c, **ARCH)
    cfg, _ = be42.model_check(lib, m, c)
    assert cfg["vocab"] == ARCH["vocab"]
    # a config without dimensions gets the reference's defaults (model.c:112-127):
    # dim 3072, 32 heads of 3072 / 32 = 96, so q_proj must be [3072, 3072]
    with open(c, "w") as f:
        f.write('{\n  "model_type": "llama"\n}\n')
    with pytest.raises(be42.Be42Error, match=r"q_proj.weight.: shape must be \[3072, 3072\]"):
        be42.model_check(lib, m, c)


@pytest.mark.parametrize("case,pattern", [
    ("no_scale", r"need a scale tensor '.*q_proj\.weight_scale'"),
    ("missing", r"missing tensor: layers\.1\.w3"),
    ("shape", r"shape must be \[96, 64\]"),
    ("mixed", r"INT8 and FP8 weights mixed"),
    ("no_norm", r"missing tensor: final norm"),
    ("not_st", r"safetensors"),
])
def test_check_errors(lib, tmp_path, case, pattern):
    m, c = paths(tmp_path)
    rng = np.random.default_rng(3)
    w = weights(rng, "int8")
    write_config(c, **ARCH)
    if case == "no_scale":
        write_checkpoint(m, w, "int8", drop=("model.layers.0.self_attn.q_proj.weight_scale",))
    elif case == "missing":
        write_checkpoint(m, w, "int8", drop=("model.layers.1.mlp.up_proj.weight",
                                            "model.layers.1.mlp.up_proj.weight_scale"))
    elif case == "shape":
        w["layers"][0]["w1"] = w["layers"][0]["w1"][:, :32]
        write_checkpoint(m, w, "int8")
    elif case == "mixed":
        # FP8 codes in the file, everything else INT8
        write_checkpoint(m, w, "int8")
        m2 = m + ".fp8"
        write_checkpoint(m2, weights(rng, "fp8"), "fp8")
        from safetensors.torch import load_file, save_file
        a, b = load_file(m), load_file(m2)
        for k in ("model.layers.0.mlp.down_proj.weight", "model.layers.0.mlp.down_proj.weight_scale"):
            a[k] = b[k]
        save_file(a, m)
    elif case == "no_norm":
        write_checkpoint(m, w, "int8", drop=("model.norm.weight",))
    else:
        with open(m, "wb") as f:
            f.write(b"\x05\x00\x00\x00\x00\x00\x00\x00{\"a\"")
    with pytest.raises(be42.Be42Error, match=pattern):
        be42.model_check(lib, m, c)


def test_check_header_offsets_validated(lib, tmp_path):
    """A header whose data offsets disagree with shape x dtype is refused
    before any tensor is read."""
    m, c = paths(tmp_path)
    write_checkpoint(m, weights(np.random.default_rng(4), "int8"), "int8")
    write_config(c, **ARCH)
    raw = bytearray(open(m, "rb").read())
    n = int.from_bytes(raw[:8], "little")
    head = raw[8:8 + n].decode()
    i = head.index('"model.norm.weight"')
    j = head.index("[64]", i)
    head = head[:j] + "[65]" + head[j + 4:]
    raw[8:8 + n] = head.encode()
    open(m, "wb").write(bytes(raw))
    with pytest.raises(be42.Be42Error, match="data offsets do not match"):
        be42.model_check(lib, m, c)


def test_check_header_numbers_stop_at_header_end(lib, tmp_path):
    """The header is parsed within its own bytes: a number at its end does not
    run on into the tensor data (here '2' + data '99]}}' would read as 299
    and close the header)."""
    m, c = paths(tmp_path)
    write_config(c, **ARCH)
    head = b'{"x":{"dtype":"I8","shape":[299],"data_offsets":[0,2'
    with open(m, "wb") as f:
        f.write(len(head).to_bytes(8, "little") + head + b"99]}}" + bytes(400))
    with pytest.raises(be42.Be42Error, match="malformed safetensors header"):
        be42.model_check(lib, m, c)


@pytest.mark.parametrize("shape,offsets,pattern", [
    # 2^32 x 2^32 x 16 elements wrap to 0 bytes in 64 bits
    ("[4294967296,4294967296,16]", "[0,0]", "data offsets do not match"),
    ("[1,99999999999999999999]", "[0,0]", "malformed safetensors header"),
])
def test_check_header_shape_overflow(lib, tmp_path, shape, offsets, pattern):
    m, c = paths(tmp_path)
    write_config(c, **ARCH)
    head = ('{"x":{"dtype":"I8","shape":%s,"data_offsets":%s}}' % (shape, offsets)).encode()
    with open(m, "wb") as f:
        f.write(len(head).to_bytes(8, "little") + head + bytes(16))
    with pytest.raises(be42.Be42Error, match=pattern):
        be42.model_check(lib, m, c)
