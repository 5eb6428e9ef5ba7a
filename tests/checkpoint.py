"""Writes decoder weights (the dict layout of be42.Decoder / test_gpu_decode
make_model) as a safetensors checkpoint and an HF-style config.json, for the
checkpoint loader's tests.

names: "hf" (model.layers.N.self_attn.q_proj.weight ...) or "llama"
(layers.N.attention.wq.weight ...), the two families the reference maps
(src/inference/model.c:194-255).  fmt: "codes" stores I8 / F8_E4M3 codes with
"<name>_scale" F32 row scales; "bf16" / "f32" store the dequantized values
(code * scale) for the loader to quantize."""
import json

import numpy as np
import torch
from safetensors.torch import save_file

HF = {"wq": "self_attn.q_proj", "wk": "self_attn.k_proj", "wv": "self_attn.v_proj", "wo": "self_attn.o_proj",
      "w1": "mlp.gate_proj", "w3": "mlp.up_proj", "w2": "mlp.down_proj",
      "attn_norm": "input_layernorm", "ffn_norm": "post_attention_layernorm"}
LLAMA = {"wq": "attention.wq", "wk": "attention.wk", "wv": "attention.wv", "wo": "attention.wo",
         "w1": "feed_forward.w1", "w3": "feed_forward.w3", "w2": "feed_forward.w2",
         "attn_norm": "attention_norm", "ffn_norm": "ffn_norm"}
GLOBAL = {"hf": ("model.embed_tokens.weight", "model.norm.weight", "lm_head.weight"),
          "llama": ("tok_embeddings.weight", "norm.weight", "output.weight")}


def fp8_values(codes):
    """E4M3 codes (bias 7, no NaN case: the reference's LUT) -> float32."""
    c = codes.astype(np.int32)
    e, m = (c >> 3) & 0xF, c & 7
    v = np.where(e == 0, m / 512.0, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    return np.where(c & 0x80, -v, v).astype(np.float32)


def _tensor(codes, scale, kind, fmt):
    # np.array copies: every tensor owns its storage (tied inputs share none)
    if fmt == "codes":
        if kind == "int8":
            return {"": torch.from_numpy(np.array(codes, np.int8)),
                    "_scale": torch.from_numpy(np.array(scale, np.float32))}
        return {"": torch.from_numpy(np.array(codes, np.uint8)).view(torch.float8_e4m3fn),
                "_scale": torch.from_numpy(np.array(scale, np.float32))}
    vals = (codes.astype(np.float32) if kind == "int8" else fp8_values(codes)) * scale[:, None]
    t = torch.from_numpy(vals.astype(np.float32))
    return {"": t.to(torch.bfloat16) if fmt == "bf16" else t}


def _norm(bits):
    return torch.from_numpy(np.array(bits, np.uint16).view(np.int16)).view(torch.bfloat16)


def write_checkpoint(path, w, kind, names="hf", fmt="codes", tie_output=False, drop=(), rename=None):
    """drop: tensor names to leave out; rename: {old: new} applied last."""
    table = HF if names == "hf" else LLAMA
    prefix = "model.layers." if names == "hf" else "layers."
    out = {}

    def put(name, codes, scale):
        for suffix, t in _tensor(codes, scale, kind, fmt).items():
            out[name + suffix] = t
    for l, L in enumerate(w["layers"]):
        for k in ("wq", "wk", "wv", "wo", "w1", "w2", "w3"):
            put(f"{prefix}{l}.{table[k]}.weight", L[k], L["s" + k[1:]])
        out[f"{prefix}{l}.{table['attn_norm']}.weight"] = _norm(L["attn_norm"])
        out[f"{prefix}{l}.{table['ffn_norm']}.weight"] = _norm(L["ffn_norm"])
    emb, norm, outn = GLOBAL[names]
    put(emb, w["emb"], w["emb_s"])
    out[norm] = _norm(w["final_norm"])
    if not tie_output:
        put(outn, w["out"], w["out_s"])
    for n in drop:
        out.pop(n)
    for a, b in (rename or {}).items():
        out[b] = out.pop(a)
    save_file(out, path)


def write_config(path, n_layers, dim, n_heads, n_kv, hd, hidden, vocab, theta=10000.0, style="hf"):
    if style == "hf":
        c = {"hidden_size": dim, "intermediate_size": hidden, "num_hidden_layers": n_layers,
             "num_attention_heads": n_heads, "num_key_value_heads": n_kv, "vocab_size": vocab, "head_dim": hd,
             "rope_theta": theta, "rms_norm_eps": 1e-6}
    elif style == "vlm":
        c = {"text_config": {"hidden_size": dim, "intermediate_size": hidden, "num_hidden_layers": n_layers,
                             "num_attention_heads": n_heads, "num_key_value_heads": n_kv, "vocab_size": vocab,
                             "head_dim": hd, "rope_parameters": {"rope_theta": theta, "factor": 1.0}},
             "vision_config": {"hidden_size": 7, "num_hidden_layers": 99, "num_attention_heads": 3}}
    else:   # params.json style
        c = {"dim": dim, "n_layers": n_layers, "n_heads": n_heads, "n_kv_heads": n_kv, "vocab_size": vocab,
             "intermediate_size": hidden, "rope_theta": theta}
    with open(path, "w") as f:
        json.dump(c, f, indent=2)
        f.write("\n")
