/* be42_engine.h -- the drop-in C ABI of the decode hot path.
 *
 * These are the entry points that src/inference of the reference engine calls
 * on the decode path (quantized linear layers, LSH routing, paged KV cache,
 * paged sparse attention), with the reference's names, argument meaning,
 * struct layouts and error conventions, implemented in lib42be_hip.so on
 * gfx950.  Every prototype names the reference declaration it replaces.
 *
 * Types.  The reference types are restated here with identical layouts; the
 * only change is the tensor extension for quantized weights:
 *   t_dtype gains DTYPE_I8 and DTYPE_FP8 (after the reference's two values),
 *   t_tensor gains a trailing `row_scale` (one fp32 scale per row of a
 *   quantized weight; ignored for F32/BF16), so t_kv_cache, which holds two
 *   t_tensor by value, grows by two pointers.
 * A build of the reference that links this library compiles its sources
 * against these definitions (the layouts of every other field are unchanged).
 *
 * Pointers.  Arguments documented as host memory may also be device memory
 * (hipMalloc): the library detects device pointers and then reads/writes
 * them in place, with no copy.  Host inputs are copied to the device per
 * call; host outputs are complete when the call returns (synchronous, as the
 * reference).  Weights passed as host pointers are mirrored to HBM on first
 * use, keyed by (pointer, size), and never written back; a weight is expected
 * not to change while it stays at one address (a few sampled words are
 * compared on each use, which catches a freed array whose address is reused).
 * All work runs on one HIP stream of the calling process.
 *
 * Device-resident state.  The page pool of a t_block_manager (K/V codes,
 * scales, centroids) lives in HBM: the k_quant / v_quant / k_scales /
 * v_scales / centroid members of t_kv_block, and the pointers returned by
 * paged_kv_get_int8, are DEVICE addresses.  page_table, free_stack,
 * logical_len and the per-block counters are host arrays kept equal to the
 * device copies.  An LSH index keeps a device copy of its block hashes.
 *
 * Errors follow the reference: op_matmul prints to stderr and returns -1;
 * block_manager_init / block_alloc return -1; paged_kv_append prints and
 * calls exit(1) when the pool is exhausted.  A HIP failure (or a missing GPU)
 * prints the library's message and aborts: there is no CPU fallback.
 */
#ifndef BE42_ENGINE_H
#define BE42_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- tensor (src/tensor/tensor.h:19-39) ------------------------------------ */
typedef uint16_t t_bf16;

typedef enum e_dtype {
    DTYPE_F32,  /* tensor.h:23 */
    DTYPE_BF16, /* tensor.h:24 */
    DTYPE_I8,   /* extension: int8 codes, per-row fp32 scale in row_scale */
    DTYPE_FP8   /* extension: E4M3 codes (ops_quant.c:27-48), per-row scale in row_scale */
} t_dtype;

typedef struct s_tensor {
    void *data;
    int shape[4];
    int stride[4];
    int ndim;
    size_t size;
    t_dtype dtype;
    const float *row_scale; /* extension: [shape[0]] scales of a DTYPE_I8/FP8 weight */
} t_tensor;

/* ---- linear layers (src/compute/ops.h:33, ops_matmul.c:366-477) -------------
 * out[m][n] = a[m][k] . b[k][n] (row-major; for n == 1, b and out are
 * vectors).  a may be DTYPE_I8 / DTYPE_FP8 (per-row scaled weights,
 * dequantized on the fly: (float)q * row_scale[i], g_fp8_lut[q] *
 * row_scale[i]), DTYPE_BF16 or DTYPE_F32; b and out DTYPE_F32 (or all three
 * DTYPE_BF16, ops_matmul.c:411).  Returns 0, or -1 with a message on stderr
 * (shape mismatch, unsupported dtypes, missing row_scale). */
int op_matmul(t_tensor *out, const t_tensor *a, const t_tensor *b);

/* ---- decode-step adjacents (src/compute/ops.h:34-41, ops_rope.h:33-81,
 * sampler.h:19) ---------------------------------------------------------------
 * op_rmsnorm: out = (x * 1/sqrtf(mean(x^2) + eps)) * w per row of x's last
 * dimension (a [dim][1] column is one row), F32 x/out with BF16 w, the
 * reference's summation order; other dtypes print and do nothing.
 * op_silu_mul: out = (g * sigmoid(g)) * u element-wise, all F32 or all BF16
 * (the reference's vector/scalar exp split and bf16 truncation); size
 * mismatch: no-op.
 * rope_apply_multihead_cached: rotates n_heads contiguous [head_dim] vectors
 * in place with the cache's tables (host tables, mirrored to HBM once);
 * positions at or past max_seq_len are left unchanged.
 * op_rope: the same rotation for transformer_forward's path without a RoPE
 * cache: x->size / head_dim vectors of F32 or BF16 x (other dtypes, a null x
 * or data: nothing), thetas from ctx->thetas_cache (host, head_dim / 2
 * floats) or the YaRN formula, angle pos * theta (ctx->pos is ignored),
 * inputs scaled by mscale when it is not 1.
 * sample_argmax: index of the largest logit (F32: argmax_simd_f32's lane tie
 * rule; BF16: first maximum above -1e9). */
typedef struct s_rope_ctx {                                        /* ops.h:19-31 */
    int head_dim;
    int pos;
    float theta_base;
    float beta_fast;    /* YaRN */
    float beta_slow;
    float factor;
    float mscale;
    int orig_ctx;
    float *thetas_cache;  /* [head_dim / 2] or NULL */
} t_rope_ctx;

typedef struct s_rope_cache {                                      /* ops_rope.h:33-38 */
    float *cos_table;   /* [max_seq_len][head_dim / 2] */
    float *sin_table;
    int head_dim;
    int max_seq_len;
} t_rope_cache;

void op_rmsnorm(t_tensor *out, const t_tensor *x, const t_tensor *w,  /* ops.h:34 */
                float epsilon);
void op_silu_mul(t_tensor *out, const t_tensor *gate,                /* ops.h:41 */
                 const t_tensor *val);
void rope_apply_multihead_cached(float *data, int n_heads, int pos,   /* ops_rope.h:80 */
                                 const t_rope_cache *cache);
void op_rope(t_tensor *x, int pos, const t_rope_ctx *ctx);          /* ops.h:36 */
int sample_argmax(const t_tensor *logits);                         /* sampler.h:19 */

/* ---- quant codecs (src/compute/ops_quant.h:22-117) ------------------------- */
typedef uint8_t t_fp8_e4m3;
typedef int8_t t_qint8;

extern float g_fp8_lut[256];                                      /* ops_quant.h:61 */
void quant_init_fp8_lut(void);                                    /* ops_quant.h:66 */
void quant_f32_to_fp8(t_fp8_e4m3 *out, const float *in, int n,     /* ops_quant.h:75 */
                      float *scale);
float quant_f32_to_int8(t_qint8 *out, const float *in, int n);     /* ops_quant.h:99 */
void dequant_int8_to_f32_avx2(float *out, const t_qint8 *in,       /* ops_quant.h:116 */
                              float scale, int n);
float compute_lightning_score_fp8(const t_fp8_e4m3 *q_fp8,         /* ops_quant.h:83 */
                                  const t_fp8_e4m3 *k_fp8, float scale, int head_dim);
float compute_lightning_score_fp8_avx2(const t_fp8_e4m3 *q_fp8,    /* ops_quant.h:89 */
                                       const t_fp8_e4m3 *k_fp8, float scale, int head_dim);

/* ---- LSH (src/compute/ops_lsh.h:33-117) ------------------------------------ */
#define LSH_NUM_HASHES 16
#define LSH_MAX_DIM 256
#define LSH_BLOCK_SIZE 64
#define LSH_MAX_BLOCKS 4096
#define LSH_HAMMING_RADIUS 4
#define LSH_NUM_BUCKETS 65536

typedef struct s_lsh_ctx {                                         /* ops_lsh.h:47-53 */
    float hyperplanes[LSH_NUM_HASHES][LSH_MAX_DIM];
    float hp_transposed[LSH_MAX_DIM][LSH_NUM_HASHES];
    int dim;
    int initialized;
} t_lsh_ctx;

typedef struct s_block_acc {                                       /* ops_lsh.h:59-64 */
    float sum_buffer[LSH_MAX_DIM]; /* kept on the device by this library: stays 0 here */
    int count;
    int start_pos;
} t_block_acc;

typedef struct s_lsh_index {                                       /* ops_lsh.h:70-85 */
    uint16_t block_hashes[LSH_MAX_BLOCKS];
    int block_starts[LSH_MAX_BLOCKS];
    int block_lens[LSH_MAX_BLOCKS];
    int n_blocks;
    int bucket_heads[LSH_NUM_BUCKETS];
    int chain_next[LSH_MAX_BLOCKS];
    t_block_acc active;
    int block_size;
} t_lsh_index;

void lsh_init(t_lsh_ctx *ctx, int dim, unsigned int seed);        /* ops_lsh.h:88 */
void lsh_index_init(t_lsh_index *idx);                            /* ops_lsh.h:91 */
void lsh_index_reset(t_lsh_index *idx);                           /* ops_lsh.h:94 */
uint16_t lsh_hash(const t_lsh_ctx *ctx, const float *vec);        /* ops_lsh.h:97 */
int lsh_hamming_distance(uint16_t h1, uint16_t h2);               /* ops_lsh.h:100 */
void lsh_insert_block(t_lsh_index *idx, uint16_t hash,            /* ops_lsh.h:103 */
                      int start_pos, int len);
void lsh_update(t_lsh_index *idx, const t_lsh_ctx *ctx,           /* ops_lsh.h:107 */
                const float *key, int dim, int pos);
int lsh_find_candidates(const t_lsh_index *idx, uint16_t query_hash, /* ops_lsh.h:111 */
                        int *block_ids, int max_blocks);
int lsh_get_active_block(const t_lsh_index *idx, int *start_pos,  /* ops_lsh.h:115 */
                         int *len);
/* LSH diagnostics (ops_lsh.h:118-216, ops_lsh.c:447-668).  The reference's
 * counters are atomic_uint_fast64_t (8 bytes each on the reference's
 * platform); this library updates them with atomic built-ins. */
typedef struct s_lsh_stats_atomic {                                /* ops_lsh.h:128-138 */
    uint64_t total_queries;
    uint64_t validated_queries;
    uint64_t topk_hits;
    uint64_t topk_total;
    uint64_t recall_scaled;
    uint64_t validation_count;
    uint64_t total_used_k;
    uint64_t k_samples;
} t_lsh_stats_atomic;

void lsh_stats_reset_atomic(t_lsh_stats_atomic *s);               /* ops_lsh.h:177 */
void lsh_stats_print_atomic(const t_lsh_stats_atomic *s,          /* ops_lsh.h:178 */
                            int sparse_k);
/* fraction of the brute-force top-actual_k keys (q . bf16 key, every
 * stride-th key above 4096, actual_k capped at 64) found among
 * lsh_indices[0 .. min(lsh_k, actual_k)) */
float lsh_validate_recall(const float *query, const uint16_t *keys,  /* ops_lsh.h:195 */
                          int n_keys, int dim, const int *lsh_indices, int lsh_k, int actual_k);
int adaptive_k_cutoff(const float *scores, const int *indices,     /* ops_lsh.h:212 */
                      int n_cand, float threshold);
/* Release the device copies this library keeps for a context / an index
 * (no counterpart in the reference, whose structs own no device memory). */
void lsh_ctx_release(const t_lsh_ctx *ctx);
void lsh_index_release(const t_lsh_index *idx);

/* ---- paged KV cache (src/memory/paged.h:30-212) ---------------------------- */
#define KV_BLOCK_SIZE 16
#define KV_MAX_BLOCKS 4096

typedef struct s_kv_block {                                        /* paged.h:53-70 */
    int8_t *k_quant;   /* device: [n_kv_heads][16][head_dim] */
    int8_t *v_quant;   /* device */
    float *k_scales;   /* device: [n_kv_heads][16] */
    float *v_scales;   /* device */
    float *centroid;   /* device: [head_dim] */
    int n_tokens;
    int start_pos;
    int layer_idx;
    int lsh_registered;
    uint32_t lsh_hash;
} t_kv_block;

typedef struct s_block_manager {                                   /* paged.h:76-88 */
    t_kv_block *blocks;
    int *page_table;
    int *free_stack;
    int free_top;
    int capacity;
    int n_layers;
    int n_kv_heads;
    int head_dim;
    int max_logical;
    int *logical_len;
} t_block_manager;

typedef struct s_paged_kv_cache {                                  /* paged.h:93-99 */
    t_block_manager *bm;
    int layer_idx;
    int n_blocks;
    int n_tokens;
} t_paged_kv_cache;

typedef struct s_block_score {                                     /* paged.h:186-191 */
    int block_idx;
    int phys_idx;
    float score;
} t_block_score;

int block_manager_init(t_block_manager *bm, int n_layers, int n_kv_heads, /* paged.h:115 */
                       int head_dim, int max_blocks_per_layer);
void block_manager_free(t_block_manager *bm);                     /* paged.h:121 */
int block_alloc(t_block_manager *bm);                             /* paged.h:127 */
void block_free(t_block_manager *bm, int phys_idx);               /* paged.h:133 */
void paged_kv_append(t_paged_kv_cache *pkv, const float *k,       /* paged.h:143 */
                     const float *v, int pos);
void paged_kv_get_int8(t_paged_kv_cache *pkv, int pos, int kv_head, /* paged.h:156 */
                       int8_t **out_k, int8_t **out_v, float *out_k_scale, float *out_v_scale);
void paged_kv_reset(t_paged_kv_cache *pkv);                       /* paged.h:162 */
void calc_block_centroid_int8(t_kv_block *block, int head_dim,    /* paged.h:178 */
                              int n_kv_heads);
void score_blocks(t_block_score *scores, const float *q,          /* paged.h:200 */
                  t_paged_kv_cache *pkv, int n_blocks);
int select_top_k_blocks(int *selected, t_block_score *scores,     /* paged.h:211 */
                        int n_blocks, int k);

/* ---- linear KV cache (src/memory/kv_cache.h:19-46, arena.h) ---------------
 * The cache rows live where the reference keeps them -- in the caller's arena
 * (host memory, [max_seq][num_heads][head_dim] bf16), which inference.c reads
 * directly -- and in a device mirror this library keeps per t_kv_cache
 * (created by kv_cache_init, updated by kv_cache_append / kv_cache_evict,
 * read by the attention functions below).  A cache that did not come from
 * kv_cache_init is uploaded on each attention call, and kv_cache_append
 * writes only its host rows. */
typedef struct s_arena {                                           /* arena.h:18-23 */
    char *base;
    size_t size;
    size_t offset;
} t_arena;

/* sample_temperature: p = expf((x - max) / temperature) / sum (max from -1e9),
 * the first index whose running sum of p exceeds a draw of the reference's
 * sampler_random_float LCG (time-seeded per thread).  sample_top_p: the same
 * probabilities (max from x[0]) sorted descending -- equal probabilities in
 * ascending index order, which the reference's qsort leaves unspecified -- cut
 * after the first running sum above top_p, and the first entry whose running
 * sum exceeds (rand() / RAND_MAX) * that sum.  F32 or BF16 logits; the
 * scratch arena is not used.  The sums are block scans on the GPU (fp32
 * rounding apart from the reference's sequential sums); where rounding leaves
 * no sum above the draw the last index is returned (the reference returns n). */
int sample_temperature(const t_tensor *logits, float temperature,  /* sampler.h:20 */
                       t_arena *scratch);
int sample_top_p(const t_tensor *logits, float temperature,        /* sampler.h:22 */
                 float top_p, t_arena *scratch);

typedef struct s_kv_cache {                                        /* kv_cache.h:19-27 */
    t_tensor k;
    t_tensor v;
    int max_seq_len;
    int num_heads;
    int head_dim;
    int current_seq_len;
} t_kv_cache;

typedef struct s_kv_init_params {                                  /* kv_cache.h:29-34 */
    int max_seq;
    int num_heads;
    int head_dim;
} t_kv_init_params;

typedef struct s_evict_params {                                    /* kv_cache.h:36-42 */
    const t_tensor *q;
    const t_tensor *w;
    int keep_k;
    t_arena *scratch;
} t_evict_params;

/* allocates K and V from the arena (exit(1) when it is too small, as
 * arena_alloc_or_die) and the device mirror */
void kv_cache_init(t_kv_cache *c, t_arena *a, t_kv_init_params *p); /* kv_cache.h:44 */
/* appends one token's rows (F32 rounded to bf16, or BF16 copied); prints
 * "KV Cache Full!" and does nothing when full */
void kv_cache_append(t_kv_cache *c, const t_tensor *k,            /* kv_cache.h:45 */
                     const t_tensor *v);
/* keeps the keep_k positions with the highest sum_h bf16(w[h]) *
 * relu(bf16(q[h]) . k[h]) (q->data and w->data read as bf16; ties: lower
 * position first), compacted to the front in position order */
void kv_cache_evict(t_kv_cache *c, t_evict_params *p);            /* kv_cache.h:46 */
/* Release the device mirror kv_cache_init made for the struct at c (no
 * counterpart in the reference, whose caches own only arena memory).  A
 * mirror is also released by the next call that finds the struct at its
 * address naming other arena rows or another shape than kv_cache_init gave
 * it: a struct freed and reused for another cache is never read through the
 * old mirror. */
void kv_cache_release(const t_kv_cache *c);

/* ---- linear-cache attention (src/compute/ops_attention.h:29-68) ------------ */
typedef struct s_attention_params {                                /* ops_attention.h:29-40 */
    const float *q;         /* [n_heads * head_dim] */
    t_kv_cache *kv_cache;
    float *output;          /* [n_heads * head_dim] */
    int n_heads;
    int n_kv_heads;
    int head_dim;
    float scale;            /* 1/sqrt(head_dim) */
    int *topk_idx;          /* optional: positions for sparse attention */
    int attend_k;
} t_attention_params;

/* one head over seq_len contiguous [head_dim] bf16 K and V rows */
void flash_attention_head(float *out, const float *q,              /* ops_attention.h:46 */
                          const t_bf16 *k_cache, const t_bf16 *v_cache, int seq_len, int head_dim, float scale);
void op_multihead_attention(t_attention_params *p);                /* ops_attention.h:54 */
void op_attention_dense(t_attention_params *p, int kv_len);        /* ops_attention.h:59 */
void op_attention_sparse(t_attention_params *p);                   /* ops_attention.h:64 */

/* ---- paged attention (src/compute/ops_attention.h:75-84) ------------------- */
void op_paged_attention(float *output, const float *q,            /* ops_attention.h:75 */
                        t_paged_kv_cache *pkv, int n_heads, int n_kv_heads,
                        int head_dim, float scale);
void op_paged_attention_sparse(float *output, const float *q,     /* ops_attention.h:82 */
                               t_block_manager *bm, const int *selected_blocks, int n_selected,
                               int n_heads, int n_kv_heads, int head_dim, float scale);

#ifdef __cplusplus
}
#endif

#endif /* BE42_ENGINE_H */
