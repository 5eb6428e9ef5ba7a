"""Host-side mirror of the gfx950 decode hot-path library (lib42be_hip.so).

Loads the C-ABI shared library through ctypes and exposes its entry points on
torch device tensors.  torch is imported before the library is loaded so that
the process holds exactly one HIP runtime (torch ships its own
libamdhip64.so.7; the library then binds to the already-loaded copy).

There is no CPU path here: when the library or a GPU is missing, calls raise.
"""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib42be_hip.so")

BE42_OK = 0
ERRORS = {-1: "EINVAL", -2: "EHIP", -3: "ENOMEM", -4: "ENODEV"}

vp, i32, sz, f32 = C.c_void_p, C.c_int, C.c_size_t, C.c_float

# name -> (restype, argtypes); keep in sync with include/*.h
SIGNATURES = {
    "be42_init": (i32, [i32]),
    "be42_last_error": (C.c_char_p, []),
    "be42_device_count": (i32, []),
    "be42_sync": (i32, [vp]),
    "be42_malloc": (vp, [sz]),
    "be42_free": (i32, [vp]),
    "be42_memcpy_h2d": (i32, [vp, vp, sz, vp]),
    "be42_memcpy_d2h": (i32, [vp, vp, sz, vp]),
    "be42_memset": (i32, [vp, i32, sz, vp]),
    "be42_quant_rows_int8": (i32, [vp, vp, vp, i32, i32, vp]),
    "be42_quant_rows_fp8": (i32, [vp, vp, vp, i32, i32, vp]),
    "be42_dequant_rows_int8": (i32, [vp, vp, vp, i32, i32, vp]),
    "be42_fp8_decode": (i32, [vp, vp, sz, vp]),
    "be42_gemv_q8": (i32, [vp, vp, vp, vp, i32, i32, i32, vp]),
    "be42_gemv_fp8": (i32, [vp, vp, vp, vp, i32, i32, i32, vp]),
    "be42_gemv_xdig_bytes": (sz, [i32, i32, i32]),
    "be42_gemv_prepare": (i32, [vp, vp, i32, i32, i32, vp]),
    "be42_gemv_q8_prepared": (i32, [vp, vp, vp, vp, i32, i32, i32, vp]),
    "be42_gemv_fp8_prepared": (i32, [vp, vp, vp, vp, i32, i32, i32, vp]),
    "be42_gemv_prepared_multi": (i32, [vp, i32, vp, i32, i32, i32, vp]),
    "be42_gemv_noalloc": (i32, [vp, vp, vp, vp, i32, i32, i32, i32, vp]),
    "be42_lsh_attention": (i32, [vp, vp, vp, i32, i32, i32, i32, f32, vp, vp, vp, i32, vp]),
    "be42_gemm_i8": (i32, [vp, vp, vp, vp, vp, i32, i32, i32, vp]),
    "be42_gemm_xdig_bytes": (C.c_size_t, [i32, i32, i32]),
    "be42_gemm_prepare": (i32, [vp, vp, i32, i32, i32, vp]),
    "be42_gemm_q8_prepared": (i32, [vp, vp, vp, vp, i32, i32, i32, vp]),
    "be42_gemm_fp8_prepared": (i32, [vp, vp, vp, vp, i32, i32, i32, vp]),
    "be42_gemm_prepared_multi": (i32, [vp, i32, vp, i32, i32, i32, vp]),
    "be42_gemm_fp8": (i32, [vp, vp, vp, vp, vp, i32, i32, i32, vp]),
    "be42_decoder_create": (i32, [vp, vp, vp, vp]),
    "be42_sample_temperature": (i32, [vp, vp, i32, i32, C.c_float, vp, vp]),
    "be42_sample_top_p": (i32, [vp, vp, i32, i32, C.c_float, C.c_float, vp, vp]),
    "be42_sample_temperature_dt": (i32, [vp, vp, i32, i32, i32, C.c_float, vp, vp]),
    "be42_sample_top_p_dt": (i32, [vp, vp, i32, i32, i32, C.c_float, C.c_float, vp, vp]),
    "be42_model_load": (i32, [vp, C.c_char_p, C.c_char_p, vp]),
    "be42_model_check": (i32, [C.c_char_p, C.c_char_p, i32, vp, vp]),
    "be42_model_decoder": (vp, [vp]),
    "be42_model_config": (i32, [vp, vp]),
    "be42_model_free": (None, [vp]),
    "be42_decoder_destroy": (None, [vp]),
    "be42_decoder_pool": (vp, [vp]),
    "be42_decoder_step": (i32, [vp, vp, i32, i32, vp, vp, vp]),
    "be42_decoder_prefill": (i32, [vp, i32, vp, i32, i32, vp, vp, vp]),
    "be42_decoder_next_tokens": (i32, [vp, vp]),
    "be42_decoder_status": (i32, [vp]),
    "be42_lsh_attention_status": (i32, [vp]),
    "be42_decoder_capture": (i32, [vp, vp, vp]),
    "be42_decoder_capture_kv": (i32, [vp, vp, vp]),
    "be42_decoder_capture_sel": (i32, [vp, vp]),
    "be42_kv_create": (i32, [vp, i32, i32, i32, i32, i32, vp]),
    "be42_kv_destroy": (None, [vp]),
    "be42_kv_set_projection": (i32, [vp, vp]),
    "be42_kv_append": (i32, [vp, i32, vp, vp, i32, i32, vp]),
    "be42_kv_reset": (i32, [vp, i32, vp]),
    "be42_kv_layer_pages": (i32, [vp, i32, vp, i32]),
    "be42_kv_append_step": (i32, [vp, vp, vp, i32, vp, vp, vp]),
    "be42_kv_page_alloc": (i32, [vp]),
    "be42_kv_page_free": (i32, [vp, i32]),
    "be42_kv_export": (i32, [vp, vp, vp, vp, vp]),
    "be42_lsh_projection": (None, [vp, vp, i32, C.c_uint]),
    "be42_lsh_hash": (i32, [vp, vp, i32, vp, i32, vp]),
    "be42_lsh_candidates": (i32, [vp, vp, vp, i32, vp, i32, i32, vp]),
    "be42_lsh_route": (i32, [vp, vp, vp, i32, i32, i32, i32, vp, vp, i32, vp, vp, vp, vp]),
    "be42_attn_workspace_bytes": (sz, [i32, i32, i32, i32, i32]),
    "be42_paged_attention": (i32, [vp, vp, i32, i32, vp, vp, i32, i32, f32, vp, i32, vp, sz, vp]),
    "be42_kv_linear_append": (i32, [vp, vp, i32, vp, vp, i32, vp]),
    "be42_linear_attention_workspace_bytes": (sz, [i32, i32, i32, i32]),
    "be42_linear_attention": (i32, [vp, vp, vp, vp, vp, i32, i32, i32, i32, f32, vp, sz, vp]),
    "be42_lsh_route_tokens": (i32, [vp, i32, vp, i32, i32, i32, vp, vp, vp, vp, i32, i32, i32, vp, vp, vp]),
    "be42_kv_linear_evict": (i32, [vp, vp, i32, i32, i32, vp, vp, i32, vp, vp]),
}

KV_INT8, KV_BF16 = 0, 1


class GemvSeg(C.Structure):
    _fields_ = [("w", C.c_void_p), ("w_scale", C.c_void_p), ("y", C.c_void_p), ("n", C.c_int)]


class DecoderConfig(C.Structure):
    """Layout of be42_decoder_config (include/be42_hip.h)."""
    _fields_ = [(n, C.c_int) for n in ("n_layers", "dim", "n_heads", "n_kv_heads", "head_dim", "hidden_dim", "vocab",
                                       "max_seq", "max_batch", "wkind", "kv_kind", "sparse_k", "cand_cap",
                                       "rope_len")] + [("rope_theta", C.c_float), ("norm_eps", C.c_float)]


class ModelOptions(C.Structure):
    """Layout of be42_model_options (include/be42_hip.h)."""
    _fields_ = [(n, C.c_int) for n in ("max_seq", "max_batch", "kv_kind", "sparse_k", "cand_cap", "rope_len",
                                       "quant_kind", "lsh_seed")]


class DecoderLayer(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("wq", "wk", "wv", "wo", "w1", "w2", "w3", "sq", "sk", "sv", "so", "s1",
                                          "s2", "s3", "attn_norm", "ffn_norm")]


class DecoderWeights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("emb", "emb_s", "final_norm", "out", "out_s", "layers")]


class KVPoolStruct(C.Structure):
    """Layout of be42_kv_pool (include/be42_hip.h)."""
    _fields_ = [("kind", C.c_int), ("n_layers", C.c_int), ("n_kv", C.c_int), ("head_dim", C.c_int),
                ("max_logical", C.c_int), ("capacity", C.c_int),
                ("k", C.c_void_p), ("v", C.c_void_p), ("k_scale", C.c_void_p), ("v_scale", C.c_void_p),
                ("centroid", C.c_void_p), ("ntok", C.c_void_p), ("page_table", C.c_void_p),
                ("n_logical", C.c_void_p), ("page_hash", C.c_void_p), ("n_indexed", C.c_void_p),
                ("hpT", C.c_void_p)]


class Be42Error(RuntimeError):
    pass


def _torch():
    import torch  # noqa: F401  (must precede the library load, see module doc)
    return torch


class Lib:
    def __init__(self, path=LIB_PATH):
        self.torch = _torch()
        if not os.path.exists(path):
            raise Be42Error(f"{path} is not built: run __graft_entry__.build()")
        self.lib = C.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(self.lib, name)
            fn.restype = res
            fn.argtypes = args
        self._inited = False

    # -- plumbing -------------------------------------------------------------
    def device_available(self):
        return self.lib.be42_device_count() > 0

    def init(self, device=0):
        if not self._inited:
            self.check(self.lib.be42_init(device), "be42_init")
            self._inited = True

    def last_error(self):
        return (self.lib.be42_last_error() or b"").decode()

    def check(self, rc, what):
        if rc != BE42_OK:
            raise Be42Error(f"{what}: {ERRORS.get(rc, rc)}: {self.last_error()}")

    def stream(self, s=None):
        t = self.torch
        s = s if s is not None else t.cuda.current_stream()
        return C.c_void_p(s.cuda_stream)

    @staticmethod
    def p(t):
        return C.c_void_p(t.data_ptr()) if t is not None else None

    def _call(self, name, *args):
        self.init()
        self.check(getattr(self.lib, name)(*args), name)

    # -- quant codecs ---------------------------------------------------------
    def quant_rows_int8(self, x):
        t = self.torch
        rows, cols = x.shape
        q = t.empty((rows, cols), dtype=t.int8, device=x.device)
        s = t.empty(rows, dtype=t.float32, device=x.device)
        self._call("be42_quant_rows_int8", self.p(q), self.p(s), self.p(x), rows, cols, self.stream())
        return q, s

    def quant_rows_fp8(self, x):
        t = self.torch
        rows, cols = x.shape
        q = t.empty((rows, cols), dtype=t.uint8, device=x.device)
        s = t.empty(rows, dtype=t.float32, device=x.device)
        self._call("be42_quant_rows_fp8", self.p(q), self.p(s), self.p(x), rows, cols, self.stream())
        return q, s

    def dequant_rows_int8(self, q, s):
        t = self.torch
        rows, cols = q.shape
        out = t.empty((rows, cols), dtype=t.float32, device=q.device)
        self._call("be42_dequant_rows_int8", self.p(out), self.p(q), self.p(s), rows, cols, self.stream())
        return out

    def fp8_decode(self, q):
        t = self.torch
        out = t.empty(q.shape, dtype=t.float32, device=q.device)
        self._call("be42_fp8_decode", self.p(out), self.p(q), q.numel(), self.stream())
        return out

    # -- GEMV -----------------------------------------------------------------
    def gemv(self, w, sw, x, kind, out=None, stream=None):
        t = self.torch
        n, k = w.shape
        batch = x.shape[0] if x.dim() == 2 else 1
        y = out if out is not None else t.empty((batch, n), dtype=t.float32, device=x.device)
        name = "be42_gemv_q8" if kind == "int8" else "be42_gemv_fp8"
        self._call(name, self.p(y), self.p(w), self.p(sw), self.p(x), n, k, batch, self.stream(stream))
        return y


    def gemv_prepare(self, x, kind, buf=None, stream=None):
        """Split activations x [batch][k] into MFMA digit planes (device buffer)."""
        t = self.torch
        batch, k = x.shape
        fp8 = 1 if kind == "fp8" else 0
        nbytes = self.lib.be42_gemv_xdig_bytes(k, batch, fp8)
        if nbytes == 0:
            raise Be42Error("gemv_prepare: unsupported shape")
        if buf is None:
            buf = t.empty(nbytes, dtype=t.uint8, device=x.device)
        self._call("be42_gemv_prepare", self.p(buf), self.p(x), k, batch, fp8, self.stream(stream))
        return buf

    def gemv_prepared(self, w, sw, xdig, batch, kind, out, stream=None):
        n, k = w.shape
        name = "be42_gemv_q8_prepared" if kind == "int8" else "be42_gemv_fp8_prepared"
        self._call(name, self.p(out), self.p(w), self.p(sw), self.p(xdig), n, k, batch, self.stream(stream))
        return out

    def gemv_prepared_multi(self, segs, xdig, batch, kind, stream=None):
        """segs: [(w [n][k], w_scale [n], out [batch][n])], up to 3, one launch."""
        k = segs[0][0].shape[1]
        arr = (GemvSeg * len(segs))()
        for i, (w, sw, out) in enumerate(segs):
            assert w.shape[1] == k
            arr[i] = GemvSeg(self.p(w), self.p(sw), self.p(out), w.shape[0])
        self._call("be42_gemv_prepared_multi", C.addressof(arr), len(segs), self.p(xdig), k, batch,
                   1 if kind == "fp8" else 0, self.stream(stream))
        return [s[2] for s in segs]


    # -- prefill GEMM -----------------------------------------------------------
    def gemm(self, xq, sx, wq, sw, kind, out=None, stream=None):
        """Y [M][N] = per-token-quantized xq [M][K] x per-row-quantized wq [N][K]."""
        t = self.torch
        m, k = xq.shape
        n = wq.shape[0]
        y = out if out is not None else t.empty((m, n), dtype=t.float32, device=xq.device)
        name = "be42_gemm_i8" if kind == "int8" else "be42_gemm_fp8"
        self._call(name, self.p(y), self.p(xq), self.p(sx), self.p(wq), self.p(sw), m, n, k, self.stream(stream))
        return y

    def gemm_f32(self, x, w, sw, kind, out=None, stream=None):
        """Y [M][N] = sw[n] * w [N][K] . x [M][K] for fp32 x, through the
        GEMV's digit planes (be42_gemm_prepare + be42_gemm_*_prepared)."""
        t = self.torch
        m, k = x.shape
        n = w.shape[0]
        fp8 = 0 if kind == "int8" else 1
        buf = t.empty(self.lib.be42_gemm_xdig_bytes(k, m, fp8), dtype=t.uint8, device=x.device)
        self._call("be42_gemm_prepare", self.p(buf), self.p(x), k, m, fp8, self.stream(stream))
        y = out if out is not None else t.empty((m, n), dtype=t.float32, device=x.device)
        name = "be42_gemm_q8_prepared" if kind == "int8" else "be42_gemm_fp8_prepared"
        self._call(name, self.p(y), self.p(w), self.p(sw), self.p(buf), n, k, m, self.stream(stream))
        return y

    def gemm_f32_multi(self, x, segs, kind, stream=None):
        """segs: [(w [n][k], w_scale [n])], up to 3, sharing x [M][K]: one
        launch (be42_gemm_prepared_multi); returns the outputs [M][n]."""
        t = self.torch
        m, k = x.shape
        fp8 = 0 if kind == "int8" else 1
        buf = t.empty(self.lib.be42_gemm_xdig_bytes(k, m, fp8), dtype=t.uint8, device=x.device)
        self._call("be42_gemm_prepare", self.p(buf), self.p(x), k, m, fp8, self.stream(stream))
        outs = [t.empty((m, w.shape[0]), dtype=t.float32, device=x.device) for w, _ in segs]
        arr = (GemvSeg * len(segs))()
        for i, ((w, sw), y) in enumerate(zip(segs, outs)):
            assert w.shape[1] == k
            arr[i] = GemvSeg(self.p(w), self.p(sw), self.p(y), w.shape[0])
        self._call("be42_gemm_prepared_multi", C.addressof(arr), len(segs), self.p(buf), k, m, fp8,
                   self.stream(stream))
        return outs

    # -- LSH / paged KV / attention --------------------------------------------
    def lsh_projection(self, dim, seed):
        import numpy as np
        hp = np.zeros(16 * dim, np.float32)
        hpT = np.zeros(dim * 16, np.float32)
        self.lib.be42_lsh_projection(hp.ctypes.data, hpT.ctypes.data, dim, seed)
        return hp.reshape(16, dim), hpT.reshape(dim, 16)

    def lsh_hash(self, vecs, hpT):
        t = self.torch
        n, dim = vecs.shape
        out = t.empty(n, dtype=t.int16, device=vecs.device)
        self._call("be42_lsh_hash", self.p(out), self.p(vecs), n, self.p(hpT), dim, self.stream())
        return out

    def lsh_candidates(self, hashes, qh, cap):
        t = self.torch
        n_q = qh.numel()
        ids = t.full((n_q, cap), -1, dtype=t.int32, device=qh.device)
        n = t.zeros(n_q, dtype=t.int32, device=qh.device)
        self._call("be42_lsh_candidates", self.p(ids), self.p(n), self.p(hashes), hashes.numel(), self.p(qh),
                   n_q, cap, self.stream())
        return ids, n

    def sample_temperature(self, logits, temp, r):
        """logits [batch][n] (float32 or bfloat16), r [batch] uniforms -> [batch] int32."""
        t = self.torch
        B, n = logits.shape
        out = t.empty(B, dtype=t.int32, device=logits.device)
        self._call("be42_sample_temperature_dt", self.p(out), self.p(logits), int(logits.dtype == t.bfloat16), n, B,
                   float(temp), self.p(r), self.stream())
        return out

    def sample_top_p(self, logits, temp, top_p, u):
        t = self.torch
        B, n = logits.shape
        out = t.empty(B, dtype=t.int32, device=logits.device)
        self._call("be42_sample_top_p_dt", self.p(out), self.p(logits), int(logits.dtype == t.bfloat16), n, B,
                   float(temp), float(top_p), self.p(u), self.stream())
        return out

    def kv_pool(self, kind, n_layers, n_kv, head_dim, max_logical, hpT=None):
        return KVPool(self, kind, n_layers, n_kv, head_dim, max_logical, hpT)

    def route(self, pool, q, k_sel, cap, slots=None, sel_stride=None):
        t = self.torch
        B, H, hd = q.shape
        sel_stride = sel_stride or max(k_sel, 64, pool.max_logical if k_sel >= pool.max_logical else 0)
        sel = t.full((B, sel_stride), -1, dtype=t.int32, device=q.device)
        nsel = t.zeros(B, dtype=t.int32, device=q.device)
        cand = t.full((B, cap), -1, dtype=t.int32, device=q.device)
        ncand = t.zeros(B, dtype=t.int32, device=q.device)
        qh = t.zeros(B, dtype=t.int16, device=q.device)
        self._call("be42_lsh_route", pool.handle, self.p(q), self.p(slots), B, H, k_sel, cap, self.p(sel),
                   self.p(nsel), sel_stride, self.p(cand), self.p(ncand), self.p(qh), self.stream())
        return sel, nsel, cand, ncand, qh

    def lsh_attention(self, pool, q, k_sel, cap, scale, slots=None, out=None, want_sel=True):
        """Route + sparse attention in one launch; returns (out, sel, nsel)
        (sel, nsel None when want_sel is False)."""
        t = self.torch
        B, H, hd = q.shape
        out = out if out is not None else t.empty((B, H, hd), dtype=t.float32, device=q.device)
        sel = nsel = None
        stride = max(k_sel, 64)
        if want_sel:
            sel = t.full((B, stride), -1, dtype=t.int32, device=q.device)
            nsel = t.zeros(B, dtype=t.int32, device=q.device)
        self._call("be42_lsh_attention", pool.handle, self.p(q), self.p(slots), B, H, k_sel, cap, float(scale),
                   self.p(out), self.p(sel), self.p(nsel), stride, self.stream())
        return out, sel, nsel

    def paged_attention(self, pool, q, sel, nsel, max_sel, scale, n_split=1, out=None, workspace=None):
        t = self.torch
        B, H, hd = q.shape
        out = out if out is not None else t.empty((B, H, hd), dtype=t.float32, device=q.device)
        ws, wsb = (self.p(workspace), workspace.numel()) if workspace is not None else (None, 0)
        self._call("be42_paged_attention", pool.handle, self.p(q), B, H, self.p(sel), self.p(nsel),
                   sel.shape[1], max_sel, float(scale), self.p(out), n_split, ws, wsb, self.stream())
        return out

    # -- linear KV cache [T][n_kv][head_dim] bf16 (kv_cache.c) ------------------
    def kv_linear_append(self, k_cache, v_cache, pos, k, v, stream=None):
        """Row `pos` of the bf16 caches from fp32 k, v [n_kv * head_dim]."""
        row = k.numel()
        self._call("be42_kv_linear_append", self.p(k_cache), self.p(v_cache), pos, self.p(k), self.p(v), row,
                   self.stream(stream))

    def linear_attention(self, q, k_cache, v_cache, n_tok, n_heads, scale, idx=None, out=None, stream=None):
        """Online-softmax attention of q [n_heads * head_dim] over tokens idx
        (or 0 .. n_tok-1) of the caches [T][n_kv][head_dim]."""
        t = self.torch
        n_kv, hd = k_cache.shape[1], k_cache.shape[2]
        out = out if out is not None else t.empty(n_heads * hd, dtype=t.float32, device=q.device)
        self._call("be42_linear_attention", self.p(out), self.p(q), self.p(k_cache), self.p(v_cache), self.p(idx),
                   n_tok, n_heads, n_kv, hd, float(scale), None, 0, self.stream(stream))
        return out

    def lsh_route_tokens(self, k_cache, kv_len, q, n_heads, hpT, hashes, starts, lens, window, sparse_k,
                         stream=None):
        """Token route (window + LSH candidate blocks, top sparse_k by the
        bf16 dot); returns (positions [sparse_k] device, count)."""
        t = self.torch
        n_kv, hd = k_cache.shape[1], k_cache.shape[2]
        topk = t.full((max(sparse_k, 1),), -1, dtype=t.int32, device=q.device)
        n = t.zeros(1, dtype=t.int32, device=q.device)
        self._call("be42_lsh_route_tokens", self.p(k_cache), kv_len, self.p(q), n_heads, n_kv, hd, self.p(hpT),
                   self.p(hashes), self.p(starts), self.p(lens), 0 if hashes is None else hashes.numel(), window,
                   sparse_k, self.p(topk), self.p(n), self.stream(stream))
        return topk, n

    def kv_linear_evict(self, k_cache, v_cache, n, q, w, keep_k, stream=None):
        """kv_cache_evict in place on the device caches; returns the new length."""
        heads, dim = k_cache.shape[1], k_cache.shape[2]
        new_len = C.c_int(n)
        self._call("be42_kv_linear_evict", self.p(k_cache), self.p(v_cache), n, heads, dim, self.p(q), self.p(w),
                   keep_k, C.byref(new_len), self.stream(stream))
        return new_len.value


class KVPool:
    """Owner of a be42_kv_pool (device page pool + host page allocator)."""

    def __init__(self, lib, kind, n_layers, n_kv, head_dim, max_logical, hpT=None, handle=None):
        import numpy as np
        self.lib = lib
        lib.init()
        self.owned = handle is None
        if handle is None:
            h = C.c_void_p()
            hp = None if hpT is None else np.ascontiguousarray(hpT, np.float32)
            lib.check(lib.lib.be42_kv_create(C.byref(h), kind, n_layers, n_kv, head_dim, max_logical,
                                             None if hp is None else hp.ctypes.data), "be42_kv_create")
        else:
            h = handle
        self.handle = h
        self.s = C.cast(h, C.POINTER(KVPoolStruct)).contents
        self.kind, self.n_layers, self.n_kv, self.head_dim = kind, n_layers, n_kv, head_dim
        self.max_logical = max_logical

    def append(self, layer, k, v, pos0):
        n = k.shape[0]
        self.lib._call("be42_kv_append", self.handle, layer, self.lib.p(k), self.lib.p(v), pos0, n,
                       self.lib.stream())

    def reset(self, layer):
        self.lib._call("be42_kv_reset", self.handle, layer, self.lib.stream())

    def export(self):
        """Host bookkeeping: (page_table [n_layers*max_logical], free_stack,
        free_top, logical_len)."""
        import numpy as np
        cap = self.s.capacity
        pt = np.zeros(self.n_layers * self.max_logical, np.int32)
        fs = np.zeros(max(cap, 1), np.int32)
        top = C.c_int()
        ll = np.zeros(self.n_layers, np.int32)
        self.lib.check(self.lib.lib.be42_kv_export(self.handle, pt.ctypes.data, fs.ctypes.data, C.byref(top),
                                                   ll.ctypes.data), "be42_kv_export")
        return pt, fs[:cap], top.value, ll

    def page_alloc(self):
        return self.lib.lib.be42_kv_page_alloc(self.handle)

    def page_free(self, phys):
        self.lib.check(self.lib.lib.be42_kv_page_free(self.handle, phys), "be42_kv_page_free")

    def layer_pages(self, layer):
        import numpy as np
        out = np.zeros(self.max_logical, np.int32)
        n = self.lib.lib.be42_kv_layer_pages(self.handle, layer, out.ctypes.data, self.max_logical)
        return out[:n].copy()

    def fetch(self, field, count, dtype):
        """Copy `count` elements of a device array of the pool to the host."""
        import numpy as np
        arr = np.empty(count, dtype)
        self.lib.torch.cuda.synchronize()
        self.lib.check(self.lib.lib.be42_memcpy_d2h(arr.ctypes.data, getattr(self.s, field), arr.nbytes, None),
                       "be42_memcpy_d2h")
        return arr

    def close(self):
        if self.handle and self.owned:
            self.lib.torch.cuda.synchronize()
            self.lib.lib.be42_kv_destroy(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


_LIB = None



class Decoder:
    """A decode-step engine over device weights (dict of torch tensors, see
    be42_decoder_weights): cfg is a dict of be42_decoder_config fields."""

    def __init__(self, lib, cfg, w, hpT):
        import numpy as np
        self.lib = lib
        self.cfg = cfg
        self.w = w                      # keeps the device tensors alive
        self.c = DecoderConfig(**cfg)
        self.layers = (DecoderLayer * cfg["n_layers"])()
        for i, L in enumerate(w["layers"]):
            for k in ("wq", "wk", "wv", "wo", "w1", "w2", "w3", "sq", "sk", "sv", "so", "s1", "s2", "s3",
                      "attn_norm", "ffn_norm"):
                setattr(self.layers[i], k, L[k].data_ptr())
        self.weights = DecoderWeights(w["emb"].data_ptr(), w["emb_s"].data_ptr(), w["final_norm"].data_ptr(),
                                      w["out"].data_ptr(), w["out_s"].data_ptr(), C.cast(self.layers, C.c_void_p))
        self.handle = C.c_void_p()
        hpT = np.ascontiguousarray(hpT, np.float32)
        lib._call("be42_decoder_create", C.byref(self.handle), C.byref(self.c), C.byref(self.weights),
                  hpT.ctypes.data)
        self.pool = KVPool(lib, cfg["kv_kind"], cfg["n_layers"] * cfg["max_batch"], cfg["n_kv_heads"],
                           cfg["head_dim"], (cfg["max_seq"] + 15) // 16,
                           handle=C.c_void_p(lib.lib.be42_decoder_pool(self.handle)))

    def step(self, tokens, pos, logits=None, sync=True, batch=None):
        """tokens: host ints, or None to feed back the previous argmax (then
        give batch); sync=False leaves the argmax on the device."""
        import numpy as np
        if tokens is None:
            t, n = None, batch
        else:
            t = np.ascontiguousarray(tokens, np.int32)
            n = len(t)
        nxt = np.zeros(n, np.int32)
        self.lib._call("be42_decoder_step", self.handle, None if t is None else t.ctypes.data, n, int(pos),
                       nxt.ctypes.data if sync else None, self.lib.p(logits), self.lib.stream())
        return nxt

    def prefill(self, tokens, pos0=0, seq=0, logits=None):
        """The prompt tokens of sequence seq at positions pos0.. in batched
        passes; returns the argmax after the last one."""
        import numpy as np
        t = np.ascontiguousarray(tokens, np.int32)
        nxt = np.zeros(1, np.int32)
        self.lib._call("be42_decoder_prefill", self.handle, int(seq), t.ctypes.data, len(t), int(pos0),
                       nxt.ctypes.data, self.lib.p(logits), self.lib.stream())
        return int(nxt[0])

    def status(self):
        """Waits for the queued steps; raises if a grid barrier timed out."""
        self.lib._call("be42_decoder_status", self.handle)

    def capture(self, q=None, nsel=None):
        self.lib._call("be42_decoder_capture", self.handle, self.lib.p(q), self.lib.p(nsel))

    def capture_kv(self, k=None, v=None):
        self.lib._call("be42_decoder_capture_kv", self.handle, self.lib.p(k), self.lib.p(v))

    def capture_sel(self, sel=None):
        self.lib._call("be42_decoder_capture_sel", self.handle, self.lib.p(sel))

    def close(self):
        if self.handle:
            self.lib.torch.cuda.synchronize()
            self.pool.close()
            self.lib.lib.be42_decoder_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

class Model:
    """A decoder loaded from a safetensors checkpoint (be42_model_load); the
    library owns its device weights.  step() as Decoder.step()."""

    def __init__(self, lib, model_path, config_path, **opts):
        self.lib = lib
        lib.init()
        o = ModelOptions(**opts)
        self.handle = C.c_void_p()
        lib._call("be42_model_load", C.byref(self.handle), os.fsencode(model_path), os.fsencode(config_path),
                  C.byref(o))
        self.c = DecoderConfig()
        lib._call("be42_model_config", self.handle, C.byref(self.c))
        self.cfg = {n: getattr(self.c, n) for n, _ in DecoderConfig._fields_}
        self.dec = C.c_void_p(lib.lib.be42_model_decoder(self.handle))

    def step(self, tokens, pos, logits=None, sync=True, batch=None):
        import numpy as np
        if tokens is None:
            t, n = None, batch
        else:
            t = np.ascontiguousarray(tokens, np.int32)
            n = len(t)
        nxt = np.zeros(n, np.int32)
        self.lib._call("be42_decoder_step", self.dec, None if t is None else t.ctypes.data, n, int(pos),
                       nxt.ctypes.data if sync else None, self.lib.p(logits), self.lib.stream())
        return nxt

    def capture_kv(self, k=None, v=None):
        self.lib._call("be42_decoder_capture_kv", self.dec, self.lib.p(k), self.lib.p(v))

    def close(self):
        if self.handle:
            self.lib.torch.cuda.synchronize()
            self.lib.lib.be42_model_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def model_check(lib, model_path, config_path, quant_kind=1):
    """Parse, map and validate a checkpoint without device work: (config
    dict, weight kind) or raises Be42Error with the library's message."""
    c = DecoderConfig()
    kind = C.c_int(-1)
    lib.check(lib.lib.be42_model_check(os.fsencode(model_path), os.fsencode(config_path), quant_kind, C.byref(c),
                                       C.byref(kind)), "be42_model_check")
    return {n: getattr(c, n) for n, _ in DecoderConfig._fields_}, kind.value


def load():
    """The process-wide library handle (raises if the .so is not built)."""
    global _LIB
    if _LIB is None:
        _LIB = Lib()
    return _LIB
