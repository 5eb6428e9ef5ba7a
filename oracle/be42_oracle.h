/*
 * be42_oracle.h -- CPU restatement of 42-Berlin-Engine's decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP product
 * is compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product library (lib42be_hip.so) never
 * links, loads or calls anything in oracle/.
 *
 * Every function follows one reference function (file:line under the
 * reference tree, src/...).  The reference is compiled by gcc in GNU C mode,
 * where -ffp-contract=fast fuses scalar a*b+c into an FMA whenever -mfma is
 * on; this file is compiled with -ffp-contract=off and writes every fused
 * operation of the reference as an explicit fmaf(), so the rounding sequence
 * is fixed by the source rather than by compiler choices.
 *
 * Pinning status of each function (which check fails if the restatement has a
 * dropped term, a wrong index or a transposed operand) is listed in
 * tests/test_oracle.py; functions without such a check say "parity unpinned"
 * in their comment below.
 */
#ifndef BE42_ORACLE_H
#define BE42_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OR_PAGE_TOKENS   16     /* KV_BLOCK_SIZE, src/memory/paged.h:35 */
#define OR_LSH_BITS      16     /* LSH_NUM_HASHES, src/compute/ops_lsh.h:33 */
#define OR_LSH_BUCKETS   65536  /* LSH_NUM_BUCKETS, src/compute/ops_lsh.h:38 */
#define OR_LSH_RADIUS    4      /* LSH_HAMMING_RADIUS, src/compute/ops_lsh.h:37 */
#define OR_HEAP_MAX      62     /* cap in select_top_k_blocks, src/memory/paged.c:473 */

/* ---- numerics primitives ------------------------------------------------ */
float    or_fast_expf(float x);                                   /* ops_math_fast.h:48-64 */
uint16_t or_f32_to_bf16(float f);                                 /* tensor.c:67-76 */
float    or_bf16_to_f32(uint16_t b);                              /* tensor.c:78-85 */
float    or_dot_f32_f32(const float *a, const float *b, int n);   /* simd_kernels.h:162-191 */
float    or_dot_bf16_f32(const uint16_t *a, const float *b, int n); /* simd_kernels.h:97-156 (AVX2 build) */

/* ---- quant codecs ------------------------------------------------------- */
float    or_quant_f32_to_int8(int8_t *out, const float *in, int n);           /* ops_quant.c:229-270 */
void     or_dequant_int8(float *out, const int8_t *in, float scale, int n);   /* ops_quant.c:275-305 */
void     or_fp8_lut(float *lut256);                                           /* ops_quant.c:27-63 */
uint8_t  or_float_to_fp8(float v);                                            /* ops_quant.c:68-98 */
void     or_quant_f32_to_fp8(uint8_t *out, const float *in, int n, float *scale); /* ops_quant.c:103-136 */

/* per-output-row weight quantization (quant codecs applied row by row) */
void or_quantize_rows_int8(int8_t *q, float *scales, const float *w, int rows, int k);
void or_quantize_rows_fp8(uint8_t *q, float *scales, const float *w, int rows, int k);

/* ---- quantized linear layers -------------------------------------------- */
/* y[b*n + i] = sum_j dequant(w[i*k + j]) * x[b*k + j], with the accumulation
 * structure of matvec_bf16_f32_blocked (ops_matmul.c:57-153). */
void or_gemv_q8(float *y, const int8_t *w, const float *scales, const float *x,
                int n, int k, int batch, int n_threads);
void or_gemv_fp8(float *y, const uint8_t *w, const float *scales, const float *x,
                 int n, int k, int batch, int n_threads);
/* the reference's own BF16 x F32 GEMV (op_matmul n == 1 path), through the same
 * row macro: pins the shared accumulation structure bit-exactly */
void or_gemv_bf16(float *y, const uint16_t *w, const float *x, int n, int k, int n_threads);
/* prefill GEMM: acc[m*n + i] = sum_j xq[m*k + j] * wq[i*k + j] (exact int32) */
void or_gemm_i8_acc(int32_t *acc, const int8_t *xq, const int8_t *wq,
                    int m, int n, int k, int n_threads);
/* y = (float)acc * sx[m] * sw[i] */
void or_gemm_i8(float *y, const int8_t *xq, const float *sx, const int8_t *wq,
                const float *sw, int m, int n, int k, int n_threads);
/* y = (sum_j lut[xq]*lut[wq], fp32 fma in ascending j) * sx[m] * sw[i] */
void or_gemm_fp8(float *y, const uint8_t *xq, const float *sx, const uint8_t *wq,
                 const float *sw, int m, int n, int k, int n_threads);

/* ---- LSH ----------------------------------------------------------------- */
void     or_lsh_init(float *hp, float *hpT, int dim, unsigned int seed); /* ops_lsh.c:22-85; hp [16][dim], hpT [dim][16] */
uint16_t or_lsh_hash(const float *hpT, int dim, const float *v);         /* ops_lsh.c:138-242 */
int      or_hamming(uint16_t a, uint16_t b);                             /* ops_lsh.c:248-251 */

typedef struct or_lsh_index {
    int       cap;       /* LSH_MAX_BLOCKS of the reference is 4096 (ops_lsh.h:36) */
    int       n_blocks;
    uint16_t *hash;      /* [cap] */
    int      *start;     /* [cap] */
    int      *len;       /* [cap] */
    int      *next;      /* [cap] */
    int      *heads;     /* [65536] */
} or_lsh_index;

int  or_lsh_index_create(or_lsh_index *ix, int cap);                          /* ops_lsh.c:90-107 */
void or_lsh_index_destroy(or_lsh_index *ix);
void or_lsh_index_reset(or_lsh_index *ix);                                    /* ops_lsh.c:114-118 */
void or_lsh_insert_block(or_lsh_index *ix, uint16_t h, int start, int len);   /* ops_lsh.c:256-272 */
int  or_lsh_find_candidates(const or_lsh_index *ix, uint16_t qh, int *ids, int max_ids); /* ops_lsh.c:361-418 */

/* ---- LSH diagnostics (ops_lsh.c:513-668) ---------------------------------- */
float or_lsh_validate_recall(const float *q, const uint16_t *keys, int n_keys, int dim,
                             const int *lsh, int lsh_k, int actual_k);
int   or_adaptive_k_cutoff(const float *scores, int n, float threshold);

/* ---- selection ------------------------------------------------------------ */
typedef struct or_block_score { int block_idx; int phys_idx; float score; } or_block_score; /* paged.h:186-191 */
/* min-heap push, ops_heap.h:33-100 */
void or_heap_push(float *hs, int *hi, int *size, int cap, float score, int index);
int  or_select_top_k_blocks(int *selected, const or_block_score *scores, int n_blocks, int k); /* paged.c:439-495 */

/* ---- paged KV cache ------------------------------------------------------- */
enum { OR_KV_INT8 = 0, OR_KV_BF16 = 1 };

typedef struct or_paged {
    int n_layers, n_kv, hd, max_logical, cap, kind;
    int8_t   *kq, *vq;        /* INT8: [cap][n_kv][16][hd] */
    uint16_t *kb, *vb;        /* BF16: [cap][n_kv][16][hd] */
    float    *ks, *vs;        /* INT8 scales: [cap][n_kv][16] */
    float    *centroid;       /* [cap][hd] */
    int      *ntok;           /* [cap] */
    int      *start_pos;      /* [cap] */
    int      *registered;     /* [cap] */
    int      *page_table;     /* [n_layers][max_logical] */
    int      *free_stack;     /* [cap] */
    int       free_top;
    int      *logical_len;    /* [n_layers] */
} or_paged;

int  or_paged_init(or_paged *p, int n_layers, int n_kv, int hd, int max_logical, int kind); /* paged.c:29-131 */
void or_paged_free(or_paged *p);                                               /* paged.c:133-157 */
int  or_paged_alloc(or_paged *p);                                              /* paged.c:159-179 */
void or_paged_release(or_paged *p, int phys);                                  /* paged.c:181-187 */
/* returns the physical page written, -1 when the pool is exhausted (the reference exits) */
int  or_paged_append(or_paged *p, int layer, const float *k, const float *v, int pos); /* paged.c:195-272 */
void or_paged_reset(or_paged *p, int layer);                                   /* paged.c:312-336 */
void or_centroid_int8(float *c, const int8_t *kq, const float *ks, int ntok, int hd); /* paged.c:350-393 */
void or_centroid_bf16(float *c, const uint16_t *kb, int ntok, int hd);         /* extension: paged.c:350-393 on bf16 rows */
void or_score_blocks(or_block_score *s, const float *q, const or_paged *p, int layer, int n_blocks); /* paged.c:401-431 */

/* attention over pages in the given order (physical ids), all query heads.
 * INT8 pages follow attention_block_int8 + attention_head_paged_sparse
 * (ops_attention.c:292-348, :391-416); BF16 pages follow attention_head_sparse
 * (ops_attention.c:131-170) applied to the page tokens in page order. */
void or_paged_attention_pages(float *out, const float *q, const or_paged *p,
                              const int *pages, int n_pages, int n_heads,
                              float scale, int n_threads);
/* dense: all mapped pages of a layer in logical order, ops_attention.c:353-438 */
void or_paged_attention_dense(float *out, const float *q, const or_paged *p, int layer,
                              int n_heads, float scale, int n_threads);

/* ---- routing composition (hash -> candidates -> score -> top-K) ------------
 * q_mean = (sum over heads ascending of q[h]) / n_heads     inference.c:291-295
 * qh = lsh_hash(q_mean)                                      inference.c:297
 * cand = lsh_find_candidates over the page hashes            inference.c:300-302
 * list = [page 0] ++ [cand \ {0, n-1} in candidate order] ++ [page n-1]
 * scores = score_blocks semantics (q head 0 . centroid)      paged.c:401-431
 * selected = select_top_k_blocks(list, k)                    paged.c:439-495
 * When n_blocks <= k the dense path is taken (inference.c:447) and every page
 * is selected in logical order.  The index ids are logical page numbers: page
 * j is inserted when it fills, so insertion order equals logical order.
 * Returns n_selected; selected[] holds physical ids; n_cand_out the candidate
 * count; cand_out (optional, >= cand_cap entries) the candidate logical ids. */
int or_route_pages(int *selected, int *n_cand_out, int *cand_out,
                   const or_paged *p, int layer, const float *q, int n_heads,
                   const float *hpT, const or_lsh_index *ix, int cand_cap, int k);
void or_q_mean(float *qm, const float *q, int n_heads, int hd);

/* ---- linear KV cache path (kv_cache.c, ops_attention.c:41-245, inference.c:268-423) ----
 * The linear cache is [T][n_kv][hd] bf16 rows (kv_cache.h:19-27). */
/* attention_head_sparse / attention_head_dense over tokens idx[0..n) of the
 * cache (idx NULL: 0 .. n-1) in that order, all query heads */
void or_attention_linear(float *out, const float *q, const uint16_t *k, const uint16_t *v, const int *idx,
                         int n, int n_heads, int n_kv, int hd, float scale, int n_threads);
/* kv_cache_evict (kv_cache_evict.c:34-70, kv_cache_score.c): keeps keep_k of
 * n rows, compacting them to the front in position order; q and w are read
 * as bf16 ([heads][dim], [heads]); returns the new length */
int  or_kv_evict(uint16_t *k, uint16_t *v, int n, int heads, int dim, const uint16_t *q, const uint16_t *w,
                 int keep_k);
/* the token route of transformer_forward (inference.c:268-423): a window of
 * the last `window` positions, plus the positions of the LSH candidate
 * blocks (lsh_find_candidates, max 64) that end before the window, sorted
 * ascending; score = sum over KV heads of dot_bf16(K[t][kv], q head kv*G);
 * the min-heap keeps min(#candidates, sparse_k).  Writes the heap's
 * positions in its array order and returns their count; with kv_len <=
 * sparse_k returns kv_len and writes nothing (dense). */
int  or_route_tokens(int *topk, const uint16_t *k, int kv_len, int n_kv, int hd, const float *q, int n_heads,
                     const float *hpT, const or_lsh_index *ix, int window, int sparse_k);

/* ---- decode-step adjacents (E rows) and the decoder loop ----------------- */
void or_rmsnorm(float *out, const float *x, const uint16_t *w, int dim, float eps);      /* ops_norm.c:27-138 */
void or_rope_table(float *cos_t, float *sin_t, int hd, int n_pos, float theta);          /* ops_rope.c:30-95 */
void or_rope_apply(float *data, int n_heads, int hd, int pos, int n_pos,
                   const float *cos_t, const float *sin_t);                              /* ops_rope.c:192-228 */
/* op_rope (legacy t_rope_ctx path): n elements of F32 (bf16 = 0) or BF16 data
 * rotated in place as n / hd vectors; thetas_cache NULL = YaRN thetas. */
void or_op_rope(void *data, int bf16, int n, int pos, int hd, float theta_base, float beta_fast,
                float beta_slow, float factor, float mscale, const float *thetas_cache);  /* ops_rope.c:243-353 */
void or_silu_mul(float *dst, const float *gate, const float *up, int n);                 /* ops_activation.c:48-105 */
int  or_argmax(const float *x, int n);                                                   /* sampler.c:42-117 */
int  or_sample_temperature(const float *x, int n, float temp, float r);                         /* sampler_temp.c:96-114 */
int  or_sample_top_p(const float *x, int n, float temp, float top_p, float u);                  /* sampler_topp.c:113-158 */
void or_silu_mul_bf16(uint16_t *dst, const uint16_t *gate, const uint16_t *up, int n);  /* ops_activation.c:143-230 */
int  or_argmax_bf16(const uint16_t *x, int n);                                          /* sampler.c:122-140 */

typedef struct or_decoder_cfg {
    int n_layers, dim, n_heads, n_kv, hd, hidden, vocab, max_seq;
    int wkind;      /* 0: INT8 codes, 1: FP8 E4M3 codes; per-row fp32 scales */
    int kv_kind;    /* OR_KV_INT8 / OR_KV_BF16 */
    int sparse_k;   /* pages; dense attention while n_pages <= sparse_k */
    int cand_cap;
    float theta, eps;
} or_decoder_cfg;

typedef struct or_layer_w {
    const void *wq, *wk, *wv, *wo, *w1, *w2, *w3;
    const float *sq, *sk, *sv, *so, *s1, *s2, *s3;
    const uint16_t *attn_norm, *ffn_norm;
} or_layer_w;

typedef struct or_model_w {
    const void *emb;           /* [vocab][dim] codes */
    const float *emb_s;        /* [vocab] */
    const uint16_t *final_norm;
    const void *out;           /* [vocab][dim] codes */
    const float *out_s;
    const or_layer_w *layers;  /* [n_layers] */
} or_model_w;

typedef struct or_decoder {
    or_decoder_cfg c;
    or_model_w w;
    or_paged kv;
    or_lsh_index *ix;
    float *hpT, *cos_t, *sin_t;
    float *x, *xb, *q, *k, *v, *att, *hb, *hb2;
    const float *kv_force_k, *kv_force_v;   /* [n_layers][n_kv*hd] rows for the next step's appends, or NULL */
    int *sel_log, *nsel_log;                 /* optional [n_layers][sparse_k], [n_layers]: logical pages attended */
} or_decoder;

int  or_decoder_init(or_decoder *d, const or_decoder_cfg *c, const or_model_w *w, const float *hpT);
void or_decoder_free(or_decoder *d);
int  or_decoder_kv_append(or_decoder *d, int layer, const float *k, const float *v, int pos);
/* n consecutive positions pos0.. of one layer, k and v [n][n_kv*hd] */
int  or_decoder_kv_append_n(or_decoder *d, int layer, const float *k, const float *v, int pos0, int n);
/* transformer_forward (inference.c:60-696), paged path; returns the argmax */
int  or_decoder_step(or_decoder *d, int token, int pos, float *logits, int n_threads);
/* Test hook (no reference counterpart): the next or_decoder_step appends the
 * given post-RoPE K and V rows ([n_layers][n_kv*hd] each, kept by the caller
 * until that step returns) instead of its own, so a checker can give the
 * oracle exactly the K/V values another implementation stored and compare the
 * rest of the step without code flips of the KV quantization. */
void or_decoder_force_kv(or_decoder *d, const float *k, const float *v);
/* Test hook: every step records, per layer, the logical ids of the pages it
 * attended in attention order (sel [n_layers][sparse_k]) and their count
 * (nsel [n_layers]); NULL stops it. */
void or_decoder_log_selection(or_decoder *d, int *sel, int *nsel);
/* Test hook: the page selection the decoder's route makes for layer `layer`
 * and the given rotated query q [n_heads*hd] over its current cache, as
 * logical page ids in attention order; returns their count. */
int  or_decoder_route(or_decoder *d, int layer, const float *q, int *sel_logical);

#ifdef __cplusplus
}
#endif
#endif
