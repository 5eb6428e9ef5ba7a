"""ctypes mirror of include/be42_engine.h (the reference-named drop-in ABI)
for the tests: struct layouts and function signatures."""
import ctypes as C

import numpy as np

DTYPE_F32, DTYPE_BF16, DTYPE_I8, DTYPE_FP8 = 0, 1, 2, 3
LSH_MAX_DIM, LSH_MAX_BLOCKS, LSH_NUM_BUCKETS = 256, 4096, 65536
KV_BLOCK_SIZE = 16


class Tensor(C.Structure):
    _fields_ = [("data", C.c_void_p), ("shape", C.c_int * 4), ("stride", C.c_int * 4), ("ndim", C.c_int),
                ("size", C.c_size_t), ("dtype", C.c_int), ("row_scale", C.c_void_p)]


class LshCtx(C.Structure):
    _fields_ = [("hyperplanes", (C.c_float * LSH_MAX_DIM) * 16), ("hp_transposed", (C.c_float * 16) * LSH_MAX_DIM),
                ("dim", C.c_int), ("initialized", C.c_int)]


class BlockAcc(C.Structure):
    _fields_ = [("sum_buffer", C.c_float * LSH_MAX_DIM), ("count", C.c_int), ("start_pos", C.c_int)]


class LshIndex(C.Structure):
    _fields_ = [("block_hashes", C.c_uint16 * LSH_MAX_BLOCKS), ("block_starts", C.c_int * LSH_MAX_BLOCKS),
                ("block_lens", C.c_int * LSH_MAX_BLOCKS), ("n_blocks", C.c_int),
                ("bucket_heads", C.c_int * LSH_NUM_BUCKETS), ("chain_next", C.c_int * LSH_MAX_BLOCKS),
                ("active", BlockAcc), ("block_size", C.c_int)]


class KvBlock(C.Structure):
    _fields_ = [("k_quant", C.c_void_p), ("v_quant", C.c_void_p), ("k_scales", C.c_void_p),
                ("v_scales", C.c_void_p), ("centroid", C.c_void_p), ("n_tokens", C.c_int), ("start_pos", C.c_int),
                ("layer_idx", C.c_int), ("lsh_registered", C.c_int), ("lsh_hash", C.c_uint32)]


class BlockManager(C.Structure):
    _fields_ = [("blocks", C.POINTER(KvBlock)), ("page_table", C.POINTER(C.c_int)),
                ("free_stack", C.POINTER(C.c_int)), ("free_top", C.c_int), ("capacity", C.c_int),
                ("n_layers", C.c_int), ("n_kv_heads", C.c_int), ("head_dim", C.c_int), ("max_logical", C.c_int),
                ("logical_len", C.POINTER(C.c_int))]


class PagedKv(C.Structure):
    _fields_ = [("bm", C.POINTER(BlockManager)), ("layer_idx", C.c_int), ("n_blocks", C.c_int),
                ("n_tokens", C.c_int)]


class RopeCache(C.Structure):
    _fields_ = [("cos_table", C.c_void_p), ("sin_table", C.c_void_p), ("head_dim", C.c_int),
                ("max_seq_len", C.c_int)]


class RopeCtx(C.Structure):
    _fields_ = [("head_dim", C.c_int), ("pos", C.c_int), ("theta_base", C.c_float), ("beta_fast", C.c_float),
                ("beta_slow", C.c_float), ("factor", C.c_float), ("mscale", C.c_float), ("orig_ctx", C.c_int),
                ("thetas_cache", C.c_void_p)]


class LshStats(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("total_queries", "validated_queries", "topk_hits", "topk_total",
                                          "recall_scaled", "validation_count", "total_used_k", "k_samples")]


class Arena(C.Structure):
    _fields_ = [("base", C.c_void_p), ("size", C.c_size_t), ("offset", C.c_size_t)]


class KvCache(C.Structure):
    _fields_ = [("k", Tensor), ("v", Tensor), ("max_seq_len", C.c_int), ("num_heads", C.c_int),
                ("head_dim", C.c_int), ("current_seq_len", C.c_int)]


class KvInitParams(C.Structure):
    _fields_ = [("max_seq", C.c_int), ("num_heads", C.c_int), ("head_dim", C.c_int)]


class EvictParams(C.Structure):
    _fields_ = [("q", C.POINTER(Tensor)), ("w", C.POINTER(Tensor)), ("keep_k", C.c_int),
                ("scratch", C.POINTER(Arena))]


class AttentionParams(C.Structure):
    _fields_ = [("q", C.c_void_p), ("kv_cache", C.POINTER(KvCache)), ("output", C.c_void_p),
                ("n_heads", C.c_int), ("n_kv_heads", C.c_int), ("head_dim", C.c_int), ("scale", C.c_float),
                ("topk_idx", C.c_void_p), ("attend_k", C.c_int)]


class BlockScore(C.Structure):
    _fields_ = [("block_idx", C.c_int), ("phys_idx", C.c_int), ("score", C.c_float)]


def bind(lib):
    """Declare the drop-in signatures on a loaded lib42be_hip.so handle."""
    vp, i32, f32 = C.c_void_p, C.c_int, C.c_float
    P = C.POINTER
    sig = {
        "op_matmul": (i32, [P(Tensor), P(Tensor), P(Tensor)]),
        "quant_init_fp8_lut": (None, []),
        "quant_f32_to_fp8": (None, [vp, vp, i32, P(C.c_float)]),
        "quant_f32_to_int8": (f32, [vp, vp, i32]),
        "dequant_int8_to_f32_avx2": (None, [vp, vp, f32, i32]),
        "compute_lightning_score_fp8": (f32, [vp, vp, f32, i32]),
        "compute_lightning_score_fp8_avx2": (f32, [vp, vp, f32, i32]),
        "lsh_init": (None, [P(LshCtx), i32, C.c_uint]),
        "lsh_index_init": (None, [P(LshIndex)]),
        "lsh_index_reset": (None, [P(LshIndex)]),
        "lsh_hash": (C.c_uint16, [P(LshCtx), vp]),
        "lsh_hamming_distance": (i32, [C.c_uint16, C.c_uint16]),
        "lsh_insert_block": (None, [P(LshIndex), C.c_uint16, i32, i32]),
        "lsh_update": (None, [P(LshIndex), P(LshCtx), vp, i32, i32]),
        "lsh_find_candidates": (i32, [P(LshIndex), C.c_uint16, vp, i32]),
        "lsh_get_active_block": (i32, [P(LshIndex), P(C.c_int), P(C.c_int)]),
        "lsh_ctx_release": (None, [P(LshCtx)]),
        "lsh_index_release": (None, [P(LshIndex)]),
        "block_manager_init": (i32, [P(BlockManager), i32, i32, i32, i32]),
        "block_manager_free": (None, [P(BlockManager)]),
        "block_alloc": (i32, [P(BlockManager)]),
        "block_free": (None, [P(BlockManager), i32]),
        "paged_kv_append": (None, [P(PagedKv), vp, vp, i32]),
        "paged_kv_get_int8": (None, [P(PagedKv), i32, i32, P(C.c_void_p), P(C.c_void_p), P(C.c_float),
                                     P(C.c_float)]),
        "paged_kv_reset": (None, [P(PagedKv)]),
        "calc_block_centroid_int8": (None, [P(KvBlock), i32, i32]),
        "score_blocks": (None, [vp, vp, P(PagedKv), i32]),
        "select_top_k_blocks": (i32, [vp, vp, i32, i32]),
        "op_paged_attention": (None, [vp, vp, P(PagedKv), i32, i32, i32, f32]),
        "op_paged_attention_sparse": (None, [vp, vp, P(BlockManager), vp, i32, i32, i32, i32, f32]),
        "op_rmsnorm": (None, [P(Tensor), P(Tensor), P(Tensor), f32]),
        "op_silu_mul": (None, [P(Tensor), P(Tensor), P(Tensor)]),
        "rope_apply_multihead_cached": (None, [vp, i32, i32, P(RopeCache)]),
        "op_rope": (None, [P(Tensor), i32, P(RopeCtx)]),
        "sample_argmax": (i32, [P(Tensor)]),
        "sample_temperature": (i32, [P(Tensor), f32, P(Arena)]),
        "sample_top_p": (i32, [P(Tensor), f32, f32, P(Arena)]),
        "lsh_stats_reset_atomic": (None, [P(LshStats)]),
        "lsh_stats_print_atomic": (None, [P(LshStats), i32]),
        "lsh_validate_recall": (f32, [vp, vp, i32, i32, vp, i32, i32]),
        "adaptive_k_cutoff": (i32, [vp, vp, i32, f32]),
        "kv_cache_init": (None, [P(KvCache), P(Arena), P(KvInitParams)]),
        "kv_cache_append": (None, [P(KvCache), P(Tensor), P(Tensor)]),
        "kv_cache_evict": (None, [P(KvCache), P(EvictParams)]),
        "kv_cache_release": (None, [P(KvCache)]),
        "flash_attention_head": (None, [vp, vp, vp, vp, i32, i32, f32]),
        "op_multihead_attention": (None, [P(AttentionParams)]),
        "op_attention_dense": (None, [P(AttentionParams), i32]),
        "op_attention_sparse": (None, [P(AttentionParams)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def ptr(a):
    """Host address of a contiguous numpy array."""
    return C.c_void_p(a.ctypes.data)


def tensor(a, dtype, rows, cols, row_scale=None):
    t = Tensor()
    t.data = a.ctypes.data if isinstance(a, np.ndarray) else a
    t.shape[0], t.shape[1] = rows, cols
    t.stride[0], t.stride[1] = cols, 1
    t.ndim = 2
    t.size = rows * cols
    t.dtype = dtype
    t.row_scale = row_scale.ctypes.data if isinstance(row_scale, np.ndarray) else row_scale
    return t
