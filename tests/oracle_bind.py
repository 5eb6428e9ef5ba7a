"""ctypes bindings for the CPU checkers (test infrastructure only).

* ``Oracle``  -- oracle/liboracle42.so, the C restatement of the reference path.
* ``RefLib``  -- oracle/_ref/libref42.so, the reference's own sources compiled in
  place (present only where oracle/Makefile could build it).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module.
"""
import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle42.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libref42.so")

f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")

PAGE = 16
OR_KV_INT8, OR_KV_BF16 = 0, 1


def _sig(lib, name, res, *args):
    fn = getattr(lib, name)
    fn.restype = res
    fn.argtypes = list(args)
    return fn


BLOCK_SCORE = np.dtype([("block_idx", np.int32), ("phys_idx", np.int32), ("score", np.float32)])


class OrLshIndex(C.Structure):
    _fields_ = [("cap", C.c_int), ("n_blocks", C.c_int), ("hash", C.POINTER(C.c_uint16)),
                ("start", C.POINTER(C.c_int)), ("len", C.POINTER(C.c_int)),
                ("next", C.POINTER(C.c_int)), ("heads", C.POINTER(C.c_int))]


class OrPaged(C.Structure):
    _fields_ = [("n_layers", C.c_int), ("n_kv", C.c_int), ("hd", C.c_int),
                ("max_logical", C.c_int), ("cap", C.c_int), ("kind", C.c_int),
                ("kq", C.POINTER(C.c_int8)), ("vq", C.POINTER(C.c_int8)),
                ("kb", C.POINTER(C.c_uint16)), ("vb", C.POINTER(C.c_uint16)),
                ("ks", C.POINTER(C.c_float)), ("vs", C.POINTER(C.c_float)),
                ("centroid", C.POINTER(C.c_float)), ("ntok", C.POINTER(C.c_int)),
                ("start_pos", C.POINTER(C.c_int)), ("registered", C.POINTER(C.c_int)),
                ("page_table", C.POINTER(C.c_int)), ("free_stack", C.POINTER(C.c_int)),
                ("free_top", C.c_int), ("logical_len", C.POINTER(C.c_int))]


class OrDecoderCfg(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_layers", "dim", "n_heads", "n_kv", "hd", "hidden", "vocab", "max_seq",
                                       "wkind", "kv_kind", "sparse_k", "cand_cap")] + \
               [("theta", C.c_float), ("eps", C.c_float)]


class OrLayerW(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("wq", "wk", "wv", "wo", "w1", "w2", "w3", "sq", "sk", "sv", "so", "s1",
                                          "s2", "s3", "attn_norm", "ffn_norm")]


class OrModelW(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("emb", "emb_s", "final_norm", "out", "out_s", "layers")]


DECODER_CFG_KEYS = ("n_layers", "dim", "n_heads", "n_kv", "hd", "hidden", "vocab", "max_seq", "wkind", "kv_kind",
                    "sparse_k", "cand_cap", "theta", "eps")
LAYER_KEYS = ("wq", "wk", "wv", "wo", "w1", "w2", "w3")


class OracleDecoder:
    """The oracle's transformer_forward on the paged path over numpy weights
    (dict: emb, emb_s, final_norm, out, out_s, layers=[{wq.., sq.., attn_norm,
    ffn_norm}]); the arrays are kept alive by this object."""

    def __init__(self, orc, cfg, w, hpT):
        self.o = orc
        self.cfg = OrDecoderCfg(*[cfg[k] for k in DECODER_CFG_KEYS])
        self.keep = []

        def ptr(a):
            a = np.ascontiguousarray(a)
            self.keep.append(a)
            return a.ctypes.data
        self.layers = (OrLayerW * cfg["n_layers"])()
        for i, L in enumerate(w["layers"]):
            for k in LAYER_KEYS:
                setattr(self.layers[i], k, ptr(L[k]))
                setattr(self.layers[i], "s" + k[1:], ptr(L["s" + k[1:]]))
            self.layers[i].attn_norm = ptr(L["attn_norm"])
            self.layers[i].ffn_norm = ptr(L["ffn_norm"])
        self.mw = OrModelW(ptr(w["emb"]), ptr(w["emb_s"]), ptr(w["final_norm"]), ptr(w["out"]), ptr(w["out_s"]),
                           C.cast(self.layers, C.c_void_p))
        self.buf = C.create_string_buffer(4096)
        hpT = np.ascontiguousarray(hpT, np.float32)
        if orc.lib.or_decoder_init(self.buf, C.byref(self.cfg), C.byref(self.mw), hpT.ravel()) != 0:
            raise MemoryError("or_decoder_init")
        self.vocab = cfg["vocab"]

    def kv_append(self, layer, k, v, pos):
        return self.o.lib.or_decoder_kv_append(self.buf, layer, np.ascontiguousarray(k, np.float32),
                                               np.ascontiguousarray(v, np.float32), pos)

    def log_selection(self, on=True):
        """Record each step's attended logical pages per layer (last_selection)."""
        c = self.cfg
        if on:
            self.sel_log = np.zeros((c.n_layers, c.sparse_k), np.int32)
            self.nsel_log = np.zeros(c.n_layers, np.int32)
            self.o.lib.or_decoder_log_selection(self.buf, self.sel_log.ctypes.data, self.nsel_log.ctypes.data)
        else:
            self.o.lib.or_decoder_log_selection(self.buf, None, None)

    def last_selection(self, layer):
        return self.sel_log[layer, :self.nsel_log[layer]].copy()

    def route(self, layer, q):
        """The decoder's route for `layer` and rotated query q over its current
        cache: logical pages in attention order."""
        out = np.zeros(max(self.cfg.sparse_k, 64) + 2, np.int32)
        n = self.o.lib.or_decoder_route(self.buf, layer, np.ascontiguousarray(q, np.float32).ctypes.data,
                                        out.ctypes.data)
        return out[:n].copy()

    def kv_append_n(self, layer, k, v, pos0):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        return self.o.lib.or_decoder_kv_append_n(self.buf, layer, k.ctypes.data, v.ctypes.data, pos0, k.shape[0])

    def step(self, token, pos, threads=0, force_k=None, force_v=None):
        """One step; force_k / force_v ([n_layers][n_kv*hd] fp32) replace the
        K and V rows the step appends (or_decoder_force_kv)."""
        logits = np.zeros(self.vocab, np.float32)
        if force_k is not None:
            fk = np.ascontiguousarray(force_k, np.float32)
            fv = np.ascontiguousarray(force_v, np.float32)
            self.o.lib.or_decoder_force_kv(self.buf, fk.ctypes.data, fv.ctypes.data)
        nxt = self.o.lib.or_decoder_step(self.buf, int(token), int(pos), logits, threads)
        return nxt, logits

    def __del__(self):
        try:
            self.o.lib.or_decoder_free(self.buf)
        except Exception:
            pass


class Oracle:
    def __init__(self, path=ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run __graft_entry__.build()")
        L = self.lib = C.CDLL(path)
        _sig(L, "or_fast_expf", C.c_float, C.c_float)
        _sig(L, "or_f32_to_bf16", C.c_uint16, C.c_float)
        _sig(L, "or_bf16_to_f32", C.c_float, C.c_uint16)
        _sig(L, "or_dot_f32_f32", C.c_float, f32p, f32p, C.c_int)
        _sig(L, "or_dot_bf16_f32", C.c_float, u16p, f32p, C.c_int)
        _sig(L, "or_quant_f32_to_int8", C.c_float, i8p, f32p, C.c_int)
        _sig(L, "or_fp8_lut", None, f32p)
        _sig(L, "or_float_to_fp8", C.c_uint8, C.c_float)
        _sig(L, "or_quant_f32_to_fp8", None, u8p, f32p, C.c_int, C.POINTER(C.c_float))
        _sig(L, "or_quantize_rows_int8", None, i8p, f32p, f32p, C.c_int, C.c_int)
        _sig(L, "or_quantize_rows_fp8", None, u8p, f32p, f32p, C.c_int, C.c_int)
        _sig(L, "or_gemv_q8", None, f32p, i8p, f32p, f32p, C.c_int, C.c_int, C.c_int, C.c_int)
        _sig(L, "or_gemv_fp8", None, f32p, u8p, f32p, f32p, C.c_int, C.c_int, C.c_int, C.c_int)
        _sig(L, "or_gemv_bf16", None, f32p, u16p, f32p, C.c_int, C.c_int, C.c_int)
        _sig(L, "or_gemm_i8_acc", None, i32p, i8p, i8p, C.c_int, C.c_int, C.c_int, C.c_int)
        _sig(L, "or_gemm_i8", None, f32p, i8p, f32p, i8p, f32p, C.c_int, C.c_int, C.c_int, C.c_int)
        _sig(L, "or_gemm_fp8", None, f32p, u8p, f32p, u8p, f32p, C.c_int, C.c_int, C.c_int, C.c_int)
        _sig(L, "or_lsh_init", None, f32p, f32p, C.c_int, C.c_uint)
        _sig(L, "or_lsh_hash", C.c_uint16, f32p, C.c_int, f32p)
        _sig(L, "or_hamming", C.c_int, C.c_uint16, C.c_uint16)
        _sig(L, "or_lsh_index_create", C.c_int, C.POINTER(OrLshIndex), C.c_int)
        _sig(L, "or_lsh_index_destroy", None, C.POINTER(OrLshIndex))
        _sig(L, "or_lsh_index_reset", None, C.POINTER(OrLshIndex))
        _sig(L, "or_lsh_insert_block", None, C.POINTER(OrLshIndex), C.c_uint16, C.c_int, C.c_int)
        _sig(L, "or_lsh_find_candidates", C.c_int, C.POINTER(OrLshIndex), C.c_uint16, i32p, C.c_int)
        _sig(L, "or_heap_push", None, f32p, i32p, C.POINTER(C.c_int), C.c_int, C.c_float, C.c_int)
        _sig(L, "or_paged_init", C.c_int, C.POINTER(OrPaged), C.c_int, C.c_int, C.c_int, C.c_int, C.c_int)
        _sig(L, "or_paged_free", None, C.POINTER(OrPaged))
        _sig(L, "or_paged_append", C.c_int, C.POINTER(OrPaged), C.c_int, f32p, f32p, C.c_int)
        _sig(L, "or_paged_reset", None, C.POINTER(OrPaged), C.c_int)
        _sig(L, "or_centroid_int8", None, f32p, i8p, f32p, C.c_int, C.c_int)
        _sig(L, "or_centroid_bf16", None, f32p, u16p, C.c_int, C.c_int)
        _sig(L, "or_paged_attention_pages", None, f32p, f32p, C.POINTER(OrPaged), i32p, C.c_int,
             C.c_int, C.c_float, C.c_int)
        _sig(L, "or_paged_attention_dense", None, f32p, f32p, C.POINTER(OrPaged), C.c_int, C.c_int,
             C.c_float, C.c_int)
        _sig(L, "or_route_pages", C.c_int, i32p, C.POINTER(C.c_int), i32p, C.POINTER(OrPaged), C.c_int,
             f32p, C.c_int, f32p, C.POINTER(OrLshIndex), C.c_int, C.c_int)
        _sig(L, "or_q_mean", None, f32p, f32p, C.c_int, C.c_int)
        _sig(L, "or_rmsnorm", None, f32p, f32p, u16p, C.c_int, C.c_float)
        _sig(L, "or_rope_table", None, f32p, f32p, C.c_int, C.c_int, C.c_float)
        _sig(L, "or_rope_apply", None, f32p, C.c_int, C.c_int, C.c_int, C.c_int, f32p, f32p)
        _sig(L, "or_op_rope", None, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, C.c_float,
             C.c_float, C.c_float, C.c_float, C.c_void_p)
        _sig(L, "or_silu_mul", None, f32p, f32p, f32p, C.c_int)
        _sig(L, "or_argmax", C.c_int, f32p, C.c_int)
        _sig(L, "or_sample_temperature", C.c_int, f32p, C.c_int, C.c_float, C.c_float)
        _sig(L, "or_sample_top_p", C.c_int, f32p, C.c_int, C.c_float, C.c_float, C.c_float)
        _sig(L, "or_decoder_init", C.c_int, C.c_void_p, C.POINTER(OrDecoderCfg), C.POINTER(OrModelW), f32p)
        _sig(L, "or_decoder_free", None, C.c_void_p)
        _sig(L, "or_decoder_kv_append", C.c_int, C.c_void_p, C.c_int, f32p, f32p, C.c_int)
        _sig(L, "or_decoder_step", C.c_int, C.c_void_p, C.c_int, C.c_int, f32p, C.c_int)
        _sig(L, "or_decoder_force_kv", None, C.c_void_p, C.c_void_p, C.c_void_p)
        _sig(L, "or_silu_mul_bf16", None, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int)
        _sig(L, "or_argmax_bf16", C.c_int, C.c_void_p, C.c_int)
        _sig(L, "or_lsh_validate_recall", C.c_float, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_int,
             C.c_int)
        _sig(L, "or_adaptive_k_cutoff", C.c_int, C.c_void_p, C.c_int, C.c_float)
        _sig(L, "or_attention_linear", None, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int,
             C.c_int, C.c_int, C.c_int, C.c_float, C.c_int)
        _sig(L, "or_kv_evict", C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
             C.c_int)
        _sig(L, "or_route_tokens", C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_int,
             C.c_void_p, C.c_void_p, C.c_int, C.c_int)
        _sig(L, "or_decoder_kv_append_n", C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_int)
        _sig(L, "or_decoder_log_selection", None, C.c_void_p, C.c_void_p, C.c_void_p)
        _sig(L, "or_decoder_route", C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p)
        _sig(L, "or_paged_alloc", C.c_int, C.POINTER(OrPaged))
        _sig(L, "or_paged_release", None, C.POINTER(OrPaged), C.c_int)
        _sig(L, "or_score_blocks", None, C.c_void_p, f32p, C.POINTER(OrPaged), C.c_int, C.c_int)
        _sig(L, "or_select_top_k_blocks", C.c_int, i32p, C.c_void_p, C.c_int, C.c_int)

    # -- scalar helpers -----------------------------------------------------
    def rmsnorm(self, x, w, eps=1e-5):
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros_like(x)
        self.lib.or_rmsnorm(out, x, np.ascontiguousarray(w, np.uint16), len(x), eps)
        return out

    def rope_table(self, hd, n_pos, theta):
        c = np.zeros(n_pos * (hd // 2), np.float32)
        s = np.zeros_like(c)
        self.lib.or_rope_table(c, s, hd, n_pos, theta)
        return c, s

    def rope_apply(self, data, n_heads, hd, pos, cos_t, sin_t):
        d = np.ascontiguousarray(data, np.float32).copy()
        self.lib.or_rope_apply(d, n_heads, hd, pos, len(cos_t) // (hd // 2), cos_t, sin_t)
        return d

    def op_rope(self, data, pos, hd, theta_base=1e4, beta_fast=32.0, beta_slow=1.0, factor=1.0, mscale=1.0,
                thetas=None):
        """op_rope with a t_rope_ctx on a copy of data (float32, or uint16 as BF16)."""
        d = np.ascontiguousarray(data).copy()
        th = None if thetas is None else np.ascontiguousarray(thetas, np.float32)
        self.lib.or_op_rope(d.ctypes.data, int(d.dtype == np.uint16), d.size, pos, hd, theta_base, beta_fast,
                            beta_slow, factor, mscale, None if th is None else th.ctypes.data)
        return d

    def silu_mul(self, g, u):
        out = np.zeros(len(g), np.float32)
        self.lib.or_silu_mul(out, np.ascontiguousarray(g, np.float32), np.ascontiguousarray(u, np.float32), len(g))
        return out

    def silu_mul_bf16(self, g, u):
        g = np.ascontiguousarray(g, np.uint16)
        u = np.ascontiguousarray(u, np.uint16)
        out = np.zeros_like(g)
        self.lib.or_silu_mul_bf16(out.ctypes.data, g.ctypes.data, u.ctypes.data, len(g))
        return out

    def argmax_bf16(self, x):
        x = np.ascontiguousarray(x, np.uint16)
        return self.lib.or_argmax_bf16(x.ctypes.data, len(x))

    def validate_recall(self, q, keys, lsh, actual_k):
        q = np.ascontiguousarray(q, np.float32)
        keys = np.ascontiguousarray(keys, np.uint16)
        lsh = np.ascontiguousarray(lsh, np.int32)
        return self.lib.or_lsh_validate_recall(q.ctypes.data, keys.ctypes.data, keys.shape[0], keys.shape[1],
                                               lsh.ctypes.data, len(lsh), actual_k)

    def adaptive_k(self, scores, threshold):
        scores = np.ascontiguousarray(scores, np.float32)
        return self.lib.or_adaptive_k_cutoff(scores.ctypes.data, len(scores), threshold)

    def attention_linear(self, q, k, v, idx, n_heads, scale, threads=0):
        """or_attention_linear: k, v [T][n_kv][hd] bf16; idx None = dense over T."""
        T, n_kv, hd = k.shape
        out = np.zeros(n_heads * hd, np.float32)
        q = np.ascontiguousarray(q, np.float32)
        k = np.ascontiguousarray(k, np.uint16)
        v = np.ascontiguousarray(v, np.uint16)
        ia = None if idx is None else np.ascontiguousarray(idx, np.int32)
        self.lib.or_attention_linear(out.ctypes.data, q.ctypes.data, k.ctypes.data, v.ctypes.data,
                                     None if ia is None else ia.ctypes.data, T if ia is None else len(ia),
                                     n_heads, n_kv, hd, scale, threads)
        return out

    def kv_evict(self, k, v, q, w, keep_k):
        """or_kv_evict on copies; returns (k, v, new length)."""
        k = np.ascontiguousarray(k, np.uint16).copy()
        v = np.ascontiguousarray(v, np.uint16).copy()
        n, heads, dim = k.shape
        q = np.ascontiguousarray(q, np.uint16)
        w = np.ascontiguousarray(w, np.uint16)
        m = self.lib.or_kv_evict(k.ctypes.data, v.ctypes.data, n, heads, dim, q.ctypes.data, w.ctypes.data, keep_k)
        return k, v, m

    def route_tokens(self, k, kv_len, q, n_heads, hpT, index, window, sparse_k):
        """or_route_tokens over the first kv_len rows of k [T][n_kv][hd]."""
        T, n_kv, hd = k.shape
        out = np.zeros(max(sparse_k, 1) + 1, np.int32)
        k = np.ascontiguousarray(k, np.uint16)
        q = np.ascontiguousarray(q, np.float32)
        hpT = np.ascontiguousarray(hpT, np.float32)
        n = self.lib.or_route_tokens(out.ctypes.data, k.ctypes.data, kv_len, n_kv, hd, q.ctypes.data, n_heads,
                                     hpT.ctypes.data, C.byref(index.ix) if index is not None else None, window,
                                     sparse_k)
        return out[:n].copy() if n <= sparse_k and kv_len > sparse_k else None

    def argmax(self, x):
        return self.lib.or_argmax(np.ascontiguousarray(x, np.float32), len(x))

    def sample_temperature(self, x, temp, r):
        return self.lib.or_sample_temperature(np.ascontiguousarray(x, np.float32), len(x), temp, r)

    def sample_top_p(self, x, temp, top_p, u):
        return self.lib.or_sample_top_p(np.ascontiguousarray(x, np.float32), len(x), temp, top_p, u)

    def gemv_bf16(self, wb, x, threads=0):
        n, k = wb.shape
        y = np.zeros(n, np.float32)
        self.lib.or_gemv_bf16(y, np.ascontiguousarray(wb, np.uint16), np.ascontiguousarray(x, np.float32).ravel(),
                              n, k, threads)
        return y

    def select_top_k(self, scores, k):
        """select_top_k_blocks over a BLOCK_SCORE structured array."""
        scores = np.ascontiguousarray(scores, BLOCK_SCORE)
        sel = np.zeros(max(k, 2) + 2, np.int32)
        n = self.lib.or_select_top_k_blocks(sel, scores.ctypes.data, len(scores), k)
        return sel[:n].copy()

    def fast_expf(self, x):
        return np.array([self.lib.or_fast_expf(float(v)) for v in np.ravel(x)], np.float32)

    def f32_to_bf16(self, x):
        x = np.ascontiguousarray(x, np.float32)
        u = x.view(np.uint32).astype(np.uint64)
        return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)

    def fp8_lut(self):
        lut = np.zeros(256, np.float32)
        self.lib.or_fp8_lut(lut)
        return lut

    def quant_int8(self, x):
        x = np.ascontiguousarray(x, np.float32)
        q = np.zeros(x.shape[-1], np.int8)
        s = self.lib.or_quant_f32_to_int8(q, x, x.shape[-1])
        return q, np.float32(s)

    def quant_fp8(self, x):
        x = np.ascontiguousarray(x, np.float32)
        q = np.zeros(x.shape[-1], np.uint8)
        s = C.c_float()
        self.lib.or_quant_f32_to_fp8(q, x, x.shape[-1], C.byref(s))
        return q, np.float32(s.value)

    def quantize_rows(self, w, kind):
        w = np.ascontiguousarray(w, np.float32)
        n, k = w.shape
        sc = np.zeros(n, np.float32)
        if kind == "int8":
            q = np.zeros((n, k), np.int8)
            self.lib.or_quantize_rows_int8(q, sc, w, n, k)
        else:
            q = np.zeros((n, k), np.uint8)
            self.lib.or_quantize_rows_fp8(q, sc, w, n, k)
        return q, sc

    def gemv(self, wq, sc, x, kind, threads=0):
        n, k = wq.shape
        x = np.ascontiguousarray(x, np.float32).reshape(-1, k)
        y = np.zeros((x.shape[0], n), np.float32)
        fn = self.lib.or_gemv_q8 if kind == "int8" else self.lib.or_gemv_fp8
        fn(y, np.ascontiguousarray(wq), np.ascontiguousarray(sc, np.float32), x, n, k, x.shape[0], threads)
        return y

    def gemm_i8_acc(self, xq, wq, threads=0):
        m, k = xq.shape
        n = wq.shape[0]
        acc = np.zeros((m, n), np.int32)
        self.lib.or_gemm_i8_acc(acc, np.ascontiguousarray(xq), np.ascontiguousarray(wq), m, n, k, threads)
        return acc

    def gemm(self, xq, sx, wq, sw, kind, threads=0):
        m, k = xq.shape
        n = wq.shape[0]
        y = np.zeros((m, n), np.float32)
        fn = self.lib.or_gemm_i8 if kind == "int8" else self.lib.or_gemm_fp8
        fn(y, np.ascontiguousarray(xq), np.ascontiguousarray(sx, np.float32), np.ascontiguousarray(wq),
           np.ascontiguousarray(sw, np.float32), m, n, k, threads)
        return y

    def lsh_init(self, dim, seed):
        hp = np.zeros(16 * dim, np.float32)
        hpT = np.zeros(dim * 16, np.float32)
        self.lib.or_lsh_init(hp, hpT, dim, seed)
        return hp.reshape(16, dim), hpT.reshape(dim, 16)

    def lsh_hash(self, hpT, v):
        return int(self.lib.or_lsh_hash(np.ascontiguousarray(hpT, np.float32).ravel(), hpT.shape[0],
                                        np.ascontiguousarray(v, np.float32)))

    def q_mean(self, q, n_heads, hd):
        out = np.zeros(hd, np.float32)
        self.lib.or_q_mean(out, np.ascontiguousarray(q, np.float32).ravel(), n_heads, hd)
        return out


class OracleIndex:
    """The reference LSH index (heads + LIFO chains) restated in the oracle."""

    def __init__(self, orc, cap):
        self.o = orc
        self.ix = OrLshIndex()
        if orc.lib.or_lsh_index_create(C.byref(self.ix), cap) != 0:
            raise MemoryError("or_lsh_index_create")

    def insert(self, h, start, length):
        self.o.lib.or_lsh_insert_block(C.byref(self.ix), h, start, length)

    def candidates(self, qh, cap):
        ids = np.zeros(max(cap, 1), np.int32)
        n = self.o.lib.or_lsh_find_candidates(C.byref(self.ix), qh, ids, cap)
        return ids[:n].copy()

    def __del__(self):
        try:
            self.o.lib.or_lsh_index_destroy(C.byref(self.ix))
        except Exception:
            pass


class OraclePaged:
    """The reference paged KV block manager restated in the oracle."""

    def __init__(self, orc, n_layers, n_kv, hd, max_logical, kind):
        self.o = orc
        self.p = OrPaged()
        if orc.lib.or_paged_init(C.byref(self.p), n_layers, n_kv, hd, max_logical, kind) != 0:
            raise MemoryError("or_paged_init")
        self.n_kv, self.hd, self.kind = n_kv, hd, kind

    def append(self, layer, k, v, pos):
        return self.o.lib.or_paged_append(C.byref(self.p), layer, np.ascontiguousarray(k, np.float32),
                                          np.ascontiguousarray(v, np.float32), pos)

    def reset(self, layer):
        self.o.lib.or_paged_reset(C.byref(self.p), layer)

    def n_blocks(self, layer):
        return self.p.logical_len[layer]

    def alloc(self):
        return self.o.lib.or_paged_alloc(C.byref(self.p))

    def free(self, phys):
        self.o.lib.or_paged_release(C.byref(self.p), phys)

    def free_top(self):
        return self.p.free_top

    def score_blocks(self, layer, q, n_blocks):
        out = np.zeros(n_blocks, BLOCK_SCORE)
        self.o.lib.or_score_blocks(out.ctypes.data, np.ascontiguousarray(q, np.float32).ravel(), C.byref(self.p),
                                   layer, n_blocks)
        return out

    def phys(self, layer, logical):
        return self.p.page_table[layer * self.p.max_logical + logical]

    def ntok(self, phys):
        return self.p.ntok[phys]

    def page_arrays(self, phys):
        """(K, V, k_scales, v_scales, centroid) of one physical page as numpy copies."""
        pe = self.n_kv * PAGE * self.hd
        cen = np.ctypeslib.as_array(self.p.centroid, shape=(self.p.cap * self.hd,))[phys * self.hd:(phys + 1) * self.hd].copy()
        if self.kind == OR_KV_INT8:
            kq = np.ctypeslib.as_array(self.p.kq, shape=(self.p.cap * pe,))[phys * pe:(phys + 1) * pe]
            vq = np.ctypeslib.as_array(self.p.vq, shape=(self.p.cap * pe,))[phys * pe:(phys + 1) * pe]
            ns = self.n_kv * PAGE
            ks = np.ctypeslib.as_array(self.p.ks, shape=(self.p.cap * ns,))[phys * ns:(phys + 1) * ns]
            vs = np.ctypeslib.as_array(self.p.vs, shape=(self.p.cap * ns,))[phys * ns:(phys + 1) * ns]
            return kq.copy(), vq.copy(), ks.copy(), vs.copy(), cen
        kb = np.ctypeslib.as_array(self.p.kb, shape=(self.p.cap * pe,))[phys * pe:(phys + 1) * pe]
        vb = np.ctypeslib.as_array(self.p.vb, shape=(self.p.cap * pe,))[phys * pe:(phys + 1) * pe]
        return kb.copy(), vb.copy(), None, None, cen

    def attention_pages(self, q, pages, n_heads, scale, threads=0):
        out = np.zeros(n_heads * self.hd, np.float32)
        pages = np.ascontiguousarray(pages, np.int32)
        self.o.lib.or_paged_attention_pages(out, np.ascontiguousarray(q, np.float32).ravel(), C.byref(self.p),
                                            pages, len(pages), n_heads, scale, threads)
        return out

    def attention_dense(self, q, layer, n_heads, scale, threads=0):
        out = np.zeros(n_heads * self.hd, np.float32)
        self.o.lib.or_paged_attention_dense(out, np.ascontiguousarray(q, np.float32).ravel(), C.byref(self.p),
                                            layer, n_heads, scale, threads)
        return out

    def route(self, layer, q, n_heads, hpT, index, cand_cap, k):
        sel = np.zeros(max(k, self.n_blocks(layer)) + 2, np.int32)
        cand = np.zeros(max(cand_cap, 1), np.int32)
        nc = C.c_int()
        ns = self.o.lib.or_route_pages(sel, C.byref(nc), cand, C.byref(self.p), layer,
                                       np.ascontiguousarray(q, np.float32).ravel(), n_heads,
                                       np.ascontiguousarray(hpT, np.float32).ravel(), C.byref(index.ix),
                                       cand_cap, k)
        return sel[:ns].copy(), cand[:nc.value].copy()

    def __del__(self):
        try:
            self.o.lib.or_paged_free(C.byref(self.p))
        except Exception:
            pass


class RefLib:
    """The compiled reference (oracle/_ref/libref42.so) through ref_shim.c."""

    def __init__(self, path=REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        L = self.lib = C.CDLL(path)
        _sig(L, "ref_fast_expf", C.c_float, C.c_float)
        _sig(L, "ref_dot_f32_f32", C.c_float, f32p, f32p, C.c_int)
        _sig(L, "ref_dot_bf16_f32", C.c_float, u16p, f32p, C.c_int)
        _sig(L, "ref_f32_to_bf16", C.c_uint16, C.c_float)
        _sig(L, "ref_heap_run", C.c_int, f32p, C.c_int, C.c_int, f32p, i32p)
        _sig(L, "ref_fp8_lut", None, f32p)
        _sig(L, "quant_f32_to_fp8", None, u8p, f32p, C.c_int, C.POINTER(C.c_float))
        _sig(L, "quant_f32_to_int8", C.c_float, i8p, f32p, C.c_int)
        _sig(L, "ref_lsh_ctx_new", C.c_void_p, C.c_int, C.c_uint)
        _sig(L, "ref_lsh_ctx_free", None, C.c_void_p)
        _sig(L, "ref_lsh_ctx_get", None, C.c_void_p, f32p, f32p)
        _sig(L, "ref_lsh_hash", C.c_uint16, C.c_void_p, f32p)
        _sig(L, "ref_lsh_index_new", C.c_void_p)
        _sig(L, "ref_lsh_index_free", None, C.c_void_p)
        _sig(L, "ref_lsh_insert", None, C.c_void_p, C.c_uint16, C.c_int, C.c_int)
        _sig(L, "ref_lsh_candidates", C.c_int, C.c_void_p, C.c_uint16, i32p, C.c_int)
        _sig(L, "ref_paged_new", C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int)
        _sig(L, "ref_paged_free", None, C.c_void_p)
        _sig(L, "ref_paged_append", None, C.c_void_p, C.c_int, f32p, f32p, C.c_int)
        _sig(L, "ref_paged_reset", None, C.c_void_p, C.c_int)
        _sig(L, "ref_paged_n_blocks", C.c_int, C.c_void_p, C.c_int)
        _sig(L, "ref_paged_phys", C.c_int, C.c_void_p, C.c_int, C.c_int)
        _sig(L, "ref_paged_page", C.c_int, C.c_void_p, C.c_int, i8p, i8p, f32p, f32p, f32p)
        _sig(L, "ref_score_blocks", None, C.c_void_p, C.c_int, f32p, C.c_int, i32p, f32p)
        _sig(L, "ref_select_top_k", C.c_int, i32p, i32p, f32p, C.c_int, C.c_int, i32p)
        _sig(L, "ref_paged_attention", None, C.c_void_p, C.c_int, f32p, f32p, C.c_int, C.c_float)
        _sig(L, "ref_paged_attention_sparse", None, C.c_void_p, f32p, f32p, i32p, C.c_int, C.c_int,
             C.c_float)
        _sig(L, "ref_flash_attention_head", None, f32p, f32p, u16p, u16p, C.c_int, C.c_int, C.c_float)
        _sig(L, "ref_matmul", C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_int,
             C.c_void_p, C.c_int, C.c_int)
        _sig(L, "lsh_hamming_distance", C.c_int, C.c_uint16, C.c_uint16)
        _sig(L, "ref_rmsnorm", None, f32p, f32p, u16p, C.c_int, C.c_float)
        _sig(L, "ref_rope_table", C.c_int, f32p, f32p, C.c_int, C.c_int, C.c_float)
        _sig(L, "ref_rope_apply", None, f32p, C.c_int, C.c_int, C.c_int, C.c_int, f32p, f32p)
        _sig(L, "ref_silu_mul", None, f32p, f32p, f32p, C.c_int)
        _sig(L, "ref_argmax", C.c_int, f32p, C.c_int)
        _sig(L, "ref_sample_top_p", C.c_int, f32p, C.c_int, C.c_float, C.c_float, C.c_uint)
        _sig(L, "ref_sample_temperature", C.c_int, f32p, C.c_int, C.c_float)
        _sig(L, "ref_silu_mul_bf16", None, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int)
        _sig(L, "ref_argmax_bf16", C.c_int, C.c_void_p, C.c_int)
        _sig(L, "ref_op_rope", None, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, C.c_float,
             C.c_float, C.c_float, C.c_float, C.c_void_p)
        _sig(L, "ref_validate_recall", C.c_float, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_int,
             C.c_int)
        _sig(L, "ref_adaptive_k", C.c_int, C.c_void_p, C.c_int, C.c_float)
        _sig(L, "ref_attention_linear", None, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p,
             C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, C.c_int)
        _sig(L, "ref_kv_fill", None, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int,
             C.c_int)
        _sig(L, "ref_kv_evict", C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p,
             C.c_void_p, C.c_int)
        # the reference's block_manager_init prints a banner on stdout; silence nothing,
        # tests capture it.

    def fp8_lut(self):
        lut = np.zeros(256, np.float32)
        self.lib.ref_fp8_lut(lut)
        return lut

    def quant_int8(self, x):
        x = np.ascontiguousarray(x, np.float32)
        q = np.zeros(x.shape[-1], np.int8)
        s = self.lib.quant_f32_to_int8(q, x, x.shape[-1])
        return q, np.float32(s)

    def quant_fp8(self, x):
        x = np.ascontiguousarray(x, np.float32)
        q = np.zeros(x.shape[-1], np.uint8)
        s = C.c_float()
        self.lib.quant_f32_to_fp8(q, x, x.shape[-1], C.byref(s))
        return q, np.float32(s.value)

    def lsh_init(self, dim, seed):
        ctx = self.lib.ref_lsh_ctx_new(dim, seed)
        hp = np.zeros(16 * dim, np.float32)
        hpT = np.zeros(dim * 16, np.float32)
        self.lib.ref_lsh_ctx_get(ctx, hp, hpT)
        return ctx, hp.reshape(16, dim), hpT.reshape(dim, 16)


def ref_available():
    return os.path.exists(REF_SO)
