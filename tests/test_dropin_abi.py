"""The drop-in ABI (include/be42_engine.h) without a GPU: struct layouts are
the reference's (paged.h, ops_lsh.h, tensor.h) field for field, the ctypes
mirror used by the GPU tests agrees with the C compiler, and the library
exports every declared function and the g_fp8_lut table."""
import ctypes
import os
import subprocess

import pytest

import dropin_bind as D

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROBE = os.path.join(ROOT, "tests", "layout_probe.c")
REF_SRC = "/root/reference/src"


def _probe(tmp_path, extra):
    exe = tmp_path / ("probe_ref" if "-DUSE_REF" in extra else "probe")
    subprocess.run(["gcc", "-O0", "-o", str(exe), PROBE] + extra, check=True, capture_output=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    return dict(line.rsplit(" ", 1) for line in out.splitlines() if not line.startswith("DTYPE")), out


def test_layouts_match_ctypes_mirror(tmp_path):
    lay, _ = _probe(tmp_path, ["-I", os.path.join(ROOT, "include")])
    mirror = {"t_lsh_ctx": D.LshCtx, "t_block_acc": D.BlockAcc, "t_lsh_index": D.LshIndex, "t_kv_block": D.KvBlock,
              "t_block_manager": D.BlockManager, "t_paged_kv_cache": D.PagedKv, "t_block_score": D.BlockScore,
              "t_tensor": D.Tensor, "t_arena": D.Arena, "t_kv_cache": D.KvCache, "t_kv_init_params": D.KvInitParams,
              "t_evict_params": D.EvictParams, "t_attention_params": D.AttentionParams, "t_rope_ctx": D.RopeCtx,
              "t_rope_cache": D.RopeCache}
    for key, val in lay.items():
        if "." in key:
            t, f = key.split(".")
            assert getattr(mirror[t], f).offset == int(val), key
        else:
            assert ctypes.sizeof(mirror[key]) == int(val), key


@pytest.mark.skipif(not os.path.isdir(REF_SRC), reason="reference sources not present")
def test_layouts_match_reference_headers(tmp_path):
    mine, _ = _probe(tmp_path, ["-I", os.path.join(ROOT, "include")])
    ref, _ = _probe(tmp_path, ["-DUSE_REF", "-I", REF_SRC])
    assert mine.keys() == ref.keys()
    # t_kv_cache holds two t_tensor by value, each one pointer (row_scale)
    # longer than the reference's; every other layout is identical
    grow = ctypes.sizeof(ctypes.c_void_p)
    for key in mine:
        if key.startswith("t_kv_cache."):
            n_before = 1 if key == "t_kv_cache.v" else 2
            assert int(mine[key]) == int(ref[key]) + n_before * grow, key
        else:
            assert mine[key] == ref[key], key


def test_library_exports_lut_table():
    lib = ctypes.CDLL(os.path.join(ROOT, "42-berlin-engine_amd", "lib42be_hip.so"))
    assert ctypes.c_float.in_dll(lib, "g_fp8_lut") is not None
    D.bind(lib)
