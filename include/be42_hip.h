/*
 * be42_hip.h -- device-level C ABI of the gfx950 decode hot-path library
 * (lib42be_hip.so).
 *
 * Every pointer argument is device memory (HBM) unless stated otherwise and
 * every entry point enqueues its work on `stream` (a hipStream_t, NULL for
 * the default stream) and returns without synchronising.  Return value:
 * BE42_OK or a negative BE42_E* code; be42_last_error() then holds a message.
 *
 * One stream at a time per device: the library keeps one grow-only workspace,
 * one split-K partial-sum buffer and the exchange buffers of the split route +
 * attention per process (used by the GEMVs, by be42_paged_attention /
 * be42_lsh_attention without a caller workspace, by be42_lsh_attention and the
 * decoder when at most 64 (query, KV head) pairs are split over several
 * workgroups each, and by the decoder's fallback paths), so calls that use
 * them must not run concurrently on two streams.  Calls on one stream are
 * always safe.
 *
 * The reference-signature entry points built on top of these (op_matmul,
 * paged_kv_append, lsh_hash, op_paged_attention_sparse, ...) are declared in
 * be42_engine.h.
 */
#ifndef BE42_HIP_H
#define BE42_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BE42_OK        0
#define BE42_EINVAL   (-1)
#define BE42_EHIP     (-2)
#define BE42_ENOMEM   (-3)
#define BE42_ENODEV   (-4)

/* ---- runtime plumbing ----------------------------------------------------- */
/* Select `device` for the calling thread and upload the constant tables. */
int         be42_init(int device);
const char *be42_last_error(void);
int         be42_device_count(void);
int         be42_sync(void *stream);
void       *be42_malloc(size_t bytes);
int         be42_free(void *ptr);
int         be42_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream);
int         be42_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream);
int         be42_memset(void *dst, int value, size_t bytes, void *stream);

/* ---- quant codecs ------------------------------------------------------------
 * Row-wise versions of quant_f32_to_int8 (src/compute/ops_quant.c:229-270) and
 * quant_f32_to_fp8 (ops_quant.c:103-136): one scale per row of `cols` values.
 * Codes and scales are bit-identical to the reference. */
int be42_quant_rows_int8(int8_t *q, float *scales, const float *x, int rows, int cols, void *stream);
int be42_quant_rows_fp8(uint8_t *q, float *scales, const float *x, int rows, int cols, void *stream);
/* (float)q * scale[row], dequant_int8_to_f32_avx2 (ops_quant.c:275-305) row-wise */
int be42_dequant_rows_int8(float *out, const int8_t *q, const float *scales, int rows, int cols,
                           void *stream);
/* g_fp8_lut[q] (ops_quant.c:18-63): E4M3 with bias 7 and no NaN (0x7F -> 480) */
int be42_fp8_decode(float *out, const uint8_t *q, size_t n, void *stream);

/* ---- decode GEMV ---------------------------------------------------------------
 * y[b*n + i] = w_scale[i] * sum_j w[i*k + j] * x[b*k + j] for b < batch <= 16:
 * per-output-row scaled INT8 or FP8 E4M3 weights [n][k] against fp32
 * activations [batch][k], fp32 output [batch][n].  Replaces the n == 1 GEMV of
 * op_matmul (src/compute/ops_matmul.c:366-417, matvec_bf16_f32_blocked :57)
 * for the quantized weight dtypes. */
int be42_gemv_q8(float *y, const int8_t *w, const float *w_scale, const float *x,
                 int n, int k, int batch, void *stream);
int be42_gemv_fp8(float *y, const uint8_t *w, const float *w_scale, const float *x,
                  int n, int k, int batch, void *stream);

/* The same GEMV in two steps, for callers that reuse one activation for
 * several weight matrices (q/k/v, gate/up) or time the weight stream alone:
 * be42_gemv_prepare splits x [batch][k] (k % 16 == 0, batch <= 16) into the
 * MFMA digit planes held in `xdig` (be42_gemv_xdig_bytes(k, batch, fp8) bytes
 * of device memory); be42_gemv_{q8,fp8}_prepared then stream the weights. */
size_t be42_gemv_xdig_bytes(int k, int batch, int fp8);
int be42_gemv_prepare(void *xdig, const float *x, int k, int batch, int fp8, void *stream);
int be42_gemv_q8_prepared(float *y, const int8_t *w, const float *w_scale, const void *xdig,
                          int n, int k, int batch, void *stream);
int be42_gemv_fp8_prepared(float *y, const uint8_t *w, const float *w_scale, const void *xdig,
                           int n, int k, int batch, void *stream);
/* be42_gemv_q8 / be42_gemv_fp8 (fp8 = 0 / 1) without any allocation.  No
 * counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc).  The digit planes live in a fixed 8 MiB device array per GPU,
 * held until the process ends, so k * batch is limited to what fits:
 * be42_gemv_xdig_bytes(k, batch, fp8) <= 8 MiB (k <= 130,048 at batch 16
 * for FP8, 174,080 for INT8), else BE42_EINVAL.  Same kernels and results as
 * the allocating entry points.  Every call on one GPU shares that array:
 * calls that overlap on one GPU (two streams, two threads) race. */
int be42_gemv_noalloc(float *y, const void *w, const float *w_scale, const float *x, int n, int k, int batch,
                      int fp8, void *stream);

/* Several weight matrices of one kind and one k that share a prepared input
 * (the q/k/v or gate/up projections of a decode step), streamed in one
 * launch: up to 3 segments, segment i writes y [batch][n]. */
typedef struct be42_gemv_seg {
    const void  *w;        /* [n][k] INT8 or E4M3 codes, 16-byte aligned */
    const float *w_scale;  /* [n] */
    float       *y;        /* [batch][n] */
    int          n;
} be42_gemv_seg;
int be42_gemv_prepared_multi(const be42_gemv_seg *segs, int nseg, const void *xdig, int k, int batch, int fp8,
                             void *stream);

/* ---- prefill GEMM ---------------------------------------------------------------
 * Y[m][n] for m < M tokens, n < N features, both operands K-contiguous
 * ([M][K] activations, [N][K] weights), fp32 output [M][N].  Replaces the
 * n > 1 tiled-GEMM branch of op_matmul (src/compute/ops_matmul.c:366-477,
 * gemm_bf16_f32_tiled :231) for quantized operands.
 *   INT8: xq/sx from per-token quant_f32_to_int8 (be42_quant_rows_int8),
 *         Y = ((float)sum_k xq*wq * sx[m]) * sw[n]; the int32 sum is exact, so
 *         Y is bit-identical to any exact evaluation (k < 133144).
 *   FP8:  xq/sx from per-token E4M3 (be42_quant_rows_fp8),
 *         Y = (sum_k e4m3(xq)*e4m3(wq) * sx[m]) * sw[n], fp32 accumulation.
 * k % 16 == 0, operands 16-byte aligned. */
int be42_gemm_i8(float *y, const int8_t *xq, const float *sx, const int8_t *wq, const float *sw,
                 int m, int n, int k, void *stream);
int be42_gemm_fp8(float *y, const uint8_t *xq, const float *sx, const uint8_t *wq, const float *sw,
                  int m, int n, int k, void *stream);
/* The same GEMM for fp32 activations, as the decode GEMV computes them: x
 * [m][k] is split once into the GEMV's digit planes (be42_gemm_prepare, one
 * "batch row" per token, m <= 65535, buffer of be42_gemm_xdig_bytes), then
 * Y[m][n] = sw[n] * sum_k w[n][k] * x[m][k] through the matrix cores.  INT8:
 * bit-identical to be42_gemv_q8_prepared on each row; FP8: equal to
 * be42_gemv_fp8_prepared up to the order of the fp32 accumulations.  This is
 * the projection step of the batched prefill (op_matmul with n > 1,
 * src/inference/inference.c:841-843, :1033-1036, :1087). */
size_t be42_gemm_xdig_bytes(int k, int m, int fp8);
int    be42_gemm_prepare(void *xdig, const float *x, int k, int m, int fp8, void *stream);
int    be42_gemm_q8_prepared(float *y, const int8_t *w, const float *w_scale, const void *xdig, int n, int k,
                             int m, void *stream);
int    be42_gemm_fp8_prepared(float *y, const uint8_t *w, const float *w_scale, const void *xdig, int n, int k,
                              int m, void *stream);
/* Up to three weight matrices that share the activations (q/k/v, gate/up) in
 * one launch; y of each segment is [m][n]. */
int    be42_gemm_prepared_multi(const be42_gemv_seg *segs, int nseg, const void *xdig, int k, int m, int fp8,
                                void *stream);

/* ---- paged KV cache in HBM ------------------------------------------------------
 * Mirrors t_block_manager / t_paged_kv_cache (src/memory/paged.h:53-99): pages
 * of 16 tokens, [n_kv][16][head_dim] per page, INT8 codes with a per-(token,
 * head) scale (quant_f32_to_int8) or bf16 (float_to_bf16, tensor.c:67-76).
 * Page allocation is the reference's LIFO free stack (paged.c:159-187), kept
 * on the host.  A page that fills gets its head-0 centroid
 * (calc_block_centroid_int8, paged.c:350-393) and the 16-bit lsh_hash of that
 * centroid (ops_lsh.c:138-242) under the projection `hpT` [head_dim][16];
 * logical page j is LSH index id j.  "Layers" are independent page tables,
 * usable as (sequence, layer) slots. */
#define BE42_KV_INT8 0
#define BE42_KV_BF16 1

typedef struct be42_kv_pool {
    int       kind;            /* BE42_KV_INT8 or BE42_KV_BF16 */
    int       n_layers, n_kv, head_dim, max_logical, capacity;
    void     *k, *v;           /* [capacity][n_kv][16][head_dim] int8 or bf16 */
    float    *k_scale, *v_scale; /* [capacity][n_kv][16], INT8 pages only */
    float    *centroid;        /* [capacity][head_dim] */
    int      *ntok;            /* [capacity] tokens written per page */
    int      *page_table;      /* [n_layers][max_logical] -> physical page, -1 unmapped */
    int      *n_logical;       /* [n_layers] pages in use */
    uint16_t *page_hash;       /* [n_layers][max_logical] hash of logical page j */
    int      *n_indexed;       /* [n_layers] pages sealed (hashed) */
    const float *hpT;          /* [head_dim][16] LSH projection */
} be42_kv_pool;

/* block_manager_init (paged.c:29-131) for n_layers page tables of
 * max_logical pages each; hpT_host (may be NULL) is uploaded. */
int  be42_kv_create(be42_kv_pool **pool, int kind, int n_layers, int n_kv, int head_dim,
                    int max_logical, const float *hpT_host);
void be42_kv_destroy(be42_kv_pool *pool);
int  be42_kv_set_projection(be42_kv_pool *pool, const float *hpT_host);
/* paged_kv_append (paged.c:195-272) for n_tokens consecutive positions
 * pos0.. of one layer; k, v are device [n_tokens][n_kv*head_dim] fp32.
 * Returns BE42_ENOMEM when the pool is exhausted (the reference exits). */
int  be42_kv_append(be42_kv_pool *pool, int layer, const float *k, const float *v, int pos0,
                    int n_tokens, void *stream);
/* paged_kv_reset (paged.c:312-336) */
int  be42_kv_reset(be42_kv_pool *pool, int layer, void *stream);
/* host copy of a layer's page table; returns the number of logical pages */
int  be42_kv_layer_pages(const be42_kv_pool *pool, int layer, int *phys_out, int max_out);

/* Host bookkeeping of the pool: block_alloc / block_free (paged.c:159-187) on
 * the pool's free stack (page_free ignores ids outside [0, capacity), as
 * block_free does), and a copy of the host page table
 * [n_layers * max_logical], free stack [capacity], its top and the logical
 * lengths [n_layers] (any output may be NULL). */
/* One token for each of n (<= 64) distinct layer slots, K and V device rows
 * [n][n_kv * head_dim]: the per-step append of a decode batch in one launch. */
int  be42_kv_append_step(be42_kv_pool *pool, const int *slots, const int *pos, int n, const float *k,
                         const float *v, void *stream);
int  be42_kv_page_alloc(be42_kv_pool *pool);
int  be42_kv_page_free(be42_kv_pool *pool, int phys);
int  be42_kv_export(const be42_kv_pool *pool, int *page_table, int *free_stack, int *free_top,
                    int *logical_len);

/* ---- LSH routing ------------------------------------------------------------------ */
/* lsh_init (src/compute/ops_lsh.c:22-85) on the host: hp [16][dim] and its
 * transpose hpT [dim][16] (hpT may be NULL). */
void be42_lsh_projection(float *hp, float *hpT, int dim, unsigned int seed);
/* lsh_hash (ops_lsh.c:138-242) of n device vectors [n][dim] -> out[n] */
int  be42_lsh_hash(uint16_t *out, const float *vecs, int n, const float *hpT, int dim, void *stream);
/* lsh_find_candidates (ops_lsh.c:361-418) for n_q query hashes over an index
 * whose block id i has hash hashes[i] (ids inserted in order, i < n_ids):
 * ids[q*cap + 0..n_out[q]) in the reference's probe-then-chain order. */
int  be42_lsh_candidates(int *ids, int *n_out, const uint16_t *hashes, int n_ids, const uint16_t *qh,
                         int n_q, int cap, void *stream);
/* Page selection for n_queries queries q [n_queries][n_heads][head_dim]
 * (fp32), query b reading page table slots[b] (slots NULL: b):
 *   pages <= k_sel: every page in logical order (inference.c:447-494, dense);
 *   else q_mean -> lsh_hash -> lsh_find_candidates(cap) over the page hashes
 *   -> score_blocks(q head 0) -> select_top_k_blocks(k_sel), in the
 *   reference's output order (anchors, then the min-heap array).
 * sel[b*sel_stride ..] receives physical page ids, n_sel[b] their count
 * (sel_stride >= max(k_sel, 64)); cand/n_cand (optional) the candidate logical
 * ids [b*cand_cap ..]; qhash (optional) the query hash. */
int  be42_lsh_route(const be42_kv_pool *pool, const float *q, const int *slots, int n_queries,
                    int n_heads, int k_sel, int cand_cap, int *sel, int *n_sel, int sel_stride,
                    int *cand, int *n_cand, uint16_t *qhash, void *stream);

/* ---- attention over selected pages --------------------------------------------------
 * op_paged_attention_sparse (src/compute/ops_attention.c:443-461) for
 * n_queries queries: query head h reads KV head h / (n_heads / n_kv) of the
 * pages sel[b*sel_stride + 0..n_sel[b]) in that order, with the reference's
 * online softmax (fast_expf) evaluated in closed form.  out [n_queries]
 * [n_heads][head_dim] fp32.  max_sel bounds n_sel[b]; n_split splits the
 * pages of a query over workgroups.  workspace may be NULL (library-owned,
 * grow-only) or a device buffer of be42_attn_workspace_bytes() bytes. */
size_t be42_attn_workspace_bytes(int n_queries, int n_heads, int head_dim, int max_sel, int n_split);
int  be42_paged_attention(const be42_kv_pool *pool, const float *q, int n_queries, int n_heads,
                          const int *sel, const int *n_sel, int sel_stride, int max_sel, float scale,
                          float *out, int n_split, void *workspace, size_t workspace_bytes, void *stream);
/* be42_lsh_route followed by be42_paged_attention over its selection, in one
 * launch (the decode step's sparse path, inference.c:447-494 with
 * op_paged_attention_sparse, ops_attention.c:443-461): the same selection,
 * bit for bit, and the same attention up to the order of the V sum.
 * k_sel <= 64, cand_cap <= 256, n_heads / n_kv <= 4, head_dim 64 or 128.
 * sel / n_sel (both or neither) receive the selection as be42_lsh_route
 * writes it (sel_stride >= 64).  From 1024 (query, KV head) pairs on it runs
 * as the two launches (the library workspace holds the selection when sel is
 * NULL). */
int  be42_lsh_attention(const be42_kv_pool *pool, const float *q, const int *slots, int n_queries,
                        int n_heads, int k_sel, int cand_cap, float scale, float *out, int *sel, int *n_sel,
                        int sel_stride, void *stream);
/* Waits for `stream`; an error if a bounded wait inside a be42_lsh_attention
 * launch gave up since the last call (that launch's output is invalid).  The
 * word it reads is the device's, shared by every stream, and is cleared. */
int  be42_lsh_attention_status(void *stream);

/* ---- linear (non-paged) bf16 KV cache -----------------------------------------------
 * The cache layout of kv_cache.h:19-27: rows [T][n_kv][head_dim] bf16.
 *   be42_kv_linear_append: row `pos` of K and V from fp32 [row] (float_to_bf16,
 *     kv_cache.c:55-80; row = n_kv * head_dim).
 *   be42_linear_attention: op_attention_sparse / op_attention_dense
 *     (ops_attention.c:84-245) for one query [n_heads][head_dim]: the online
 *     softmax over tokens idx[0 .. n_tok) in that order (idx NULL: 0 ..
 *     n_tok-1), query head h reading KV head h / (n_heads / n_kv); out
 *     [n_heads][head_dim].  workspace NULL: the library's (grow-only), else
 *     be42_linear_attention_workspace_bytes() bytes.
 *   be42_lsh_route_tokens: the token route of transformer_forward
 *     (inference.c:268-423) for kv_len > sparse_k: the last `window`
 *     positions, plus every position of the LSH candidate blocks
 *     (lsh_find_candidates over block_hashes, at most 64 blocks) that end
 *     before the window, sorted; score = sum over KV heads of
 *     simd_dot_bf16_f32(K[t][kv], q head kv * G); the reference min-heap keeps
 *     min(#candidates, sparse_k <= 64) of them.  topk (device, >= sparse_k)
 *     receives the positions in the heap's array order, *n_topk their count.
 *     hpT [head_dim][16]; block arrays of the 64-token index (lsh_update).
 *   be42_kv_linear_evict: kv_cache_evict (kv_cache_evict.c:34-70): keeps the
 *     keep_k positions with the highest sum_h bf16(w[h]) * relu(q[h] . k[h])
 *     (ties: lower position first), compacted to the front in position order;
 *     q [heads][dim] and w [heads] bf16; *new_len (host) gets the length. */
int    be42_kv_linear_append(uint16_t *k_cache, uint16_t *v_cache, int pos, const float *k, const float *v, int row,
                             void *stream);
size_t be42_linear_attention_workspace_bytes(int n_tok, int n_heads, int n_kv, int head_dim);
int    be42_linear_attention(float *out, const float *q, const uint16_t *k, const uint16_t *v, const int *idx,
                             int n_tok, int n_heads, int n_kv, int head_dim, float scale, void *workspace,
                             size_t workspace_bytes, void *stream);
int    be42_lsh_route_tokens(const uint16_t *k, int kv_len, const float *q, int n_heads, int n_kv, int head_dim,
                             const float *hpT, const uint16_t *block_hashes, const int *block_starts,
                             const int *block_lens, int n_blocks, int window, int sparse_k, int *topk, int *n_topk,
                             void *stream);
int    be42_kv_linear_evict(uint16_t *k, uint16_t *v, int n, int heads, int dim, const uint16_t *q, const uint16_t *w,
                            int keep_k, int *new_len, void *stream);

/* ---- decode step ------------------------------------------------------------------
 * transformer_forward (src/inference/inference.c:60-696) on the paged path for a
 * batch of independent sequences at one position: embedding (row-scaled codes),
 * then per layer RMSNorm (ops_norm.c:126) -> q/k/v GEMV -> RoPE
 * (ops_rope.c:192) -> paged append -> attention (dense over all pages while a
 * layer has <= sparse_k pages, inference.c:447-494; else the LSH route and sparse
 * attention) -> o GEMV -> residual -> RMSNorm -> gate/up GEMV -> SiLU*up
 * (ops_activation.c:48) -> down GEMV -> residual; final RMSNorm, lm_head GEMV and
 * argmax (sampler.c:42).  Weights are device arrays owned by the caller: codes
 * [rows][cols] (INT8 or E4M3) with per-row fp32 scales, bf16 norm weights.  The
 * KV pool has n_layers * max_batch slots: slot = layer * max_batch + b. */
typedef struct be42_decoder_config {
    int n_layers, dim, n_heads, n_kv_heads, head_dim, hidden_dim, vocab, max_seq, max_batch;
    int wkind;      /* 0: INT8 codes, 1: FP8 E4M3 codes */
    int kv_kind;    /* BE42_KV_INT8 / BE42_KV_BF16 */
    int sparse_k;   /* pages attended per token once a layer has more */
    int cand_cap;   /* LSH candidate cap of the router (<= 256) */
    int rope_len;   /* RoPE table positions (0: max_seq); later positions are not rotated */
    float rope_theta, norm_eps;
} be42_decoder_config;

typedef struct be42_decoder_layer {
    const void *wq, *wk, *wv, *wo, *w1, *w2, *w3;   /* [out][in] codes */
    const float *sq, *sk, *sv, *so, *s1, *s2, *s3; /* [out] scales */
    const uint16_t *attn_norm, *ffn_norm;          /* [dim] bf16 */
} be42_decoder_layer;

typedef struct be42_decoder_weights {
    const void *emb;             /* [vocab][dim] codes */
    const float *emb_s;          /* [vocab] */
    const uint16_t *final_norm;  /* [dim] bf16 */
    const void *out;             /* [vocab][dim] codes */
    const float *out_s;          /* [vocab] */
    const be42_decoder_layer *layers;  /* [n_layers], copied at create */
} be42_decoder_weights;

typedef struct be42_decoder be42_decoder;

int  be42_decoder_create(be42_decoder **out, const be42_decoder_config *cfg, const be42_decoder_weights *w,
                         const float *hpT_host);
void be42_decoder_destroy(be42_decoder *d);
be42_kv_pool *be42_decoder_pool(be42_decoder *d);
/* One token for each of `batch` sequences at position pos: tokens and
 * next_tokens are host arrays.  tokens == NULL feeds back the previous step's
 * device argmax (greedy decoding with no host round trip); next_tokens may be
 * NULL (the argmax stays on the device, be42_decoder_next_tokens);
 * logits_out (device, [batch][vocab]) may be NULL.  Re-running a position
 * overwrites that position's K/V.
 * The step's kernels run on the decoder's own stream, after the work already
 * queued on `stream`, and `stream` waits for them; they are captured once per
 * (batch, dense or routed attention, token source, output buffers) and replayed
 * as a HIP graph (environment BE42_DECODE_NO_GRAPH=1 launches them one by one).
 * The call returns once the host side of the step is queued; it blocks only
 * for next_tokens, or when the step before the last still runs.
 * One-sequence steps run each layer as one launch whose blocks meet at grid
 * barriers; a barrier wait that does not complete within its bound sets a
 * device flag.  The step that sets it is reported by itself when next_tokens
 * is given, else by the next be42_decoder_step / be42_decoder_prefill that
 * finds it finished, or by be42_decoder_status; from then on the decoder
 * refuses every step (its cache and results are invalid: destroy it). */
int  be42_decoder_step(be42_decoder *d, const int *tokens, int batch, int pos, int *next_tokens,
                       float *logits_out, void *stream);
int  be42_decoder_next_tokens(be42_decoder *d, const int **dev_ptr);
/* Waits for the decoder's queued work; BE42_OK, or an error when a grid
 * barrier of any step so far timed out. */
int  be42_decoder_status(be42_decoder *d);
/* Batched prefill (forward_prefill_batch, src/inference/inference.c:718-1112,
 * with its token-major / feature-major layout fixed): the n prompt tokens of
 * sequence seq at positions pos0 .. pos0+n-1, in passes of up to 256 tokens
 * whose projections are GEMMs (be42_gemm_*_prepared) and whose attention lets
 * each token see the cache as of its own position.  The argmax of the last
 * token goes to *next_token (host, may be NULL) and to the sequence's device
 * feedback slot (a following be42_decoder_step with tokens == NULL continues
 * from it); logits_out (device [vocab], may be NULL) takes its logits.  INT8
 * weights: bit-identical to n one-sequence decode steps (KV pages, LSH index,
 * logits); FP8: equal up to fp32 accumulation order.  Needs sparse_k <= 64,
 * cand_cap <= 256, <= 4 heads per KV head, head_dim 64 or 128.  Ordered on
 * `stream` like be42_decoder_step; on error the sequence's cache may hold
 * part of the prompt (reset its slots with be42_kv_reset). */
int  be42_decoder_prefill(be42_decoder *d, int seq, const int *tokens, int n, int pos0, int *next_token,
                          float *logits_out, void *stream);
/* Inspection: each step copies every layer's rotated queries into q_dst
 * ([n_layers][max_batch][n_heads * head_dim], device) and the number of pages
 * each layer attended into nsel_dst ([n_layers][max_batch], device); NULL
 * stops either. */
int  be42_decoder_capture(be42_decoder *d, float *q_dst, int *nsel_dst);
/* Inspection: each step copies every layer's post-RoPE K and V rows (the
 * values it appends to the page pool) into k_dst / v_dst ([n_layers]
 * [max_batch][n_kv_heads * head_dim], device); NULL stops either. */
int  be42_decoder_capture_kv(be42_decoder *d, float *k_dst, float *v_dst);
/* Inspection: on routed steps (a layer past sparse_k pages) each step copies
 * every layer's page selection (physical ids in attention order) into
 * sel_dst ([n_layers][max_batch][max(sparse_k, 64)], device); NULL stops it. */
int  be42_decoder_capture_sel(be42_decoder *d, int *sel_dst);

/* ---- sampling ------------------------------------------------------------------
 * sample_temperature (src/compute/sampler_temp.c:96-114) and sample_top_p
 * (sampler_topp.c:113-158) for `batch` rows of n device logits [batch][n]:
 * p = expf((x - max) / temp) / sum; temperature: the first index whose running sum
 * of p exceeds r[b]; top-p: p sorted descending (stable: equal p in ascending index
 * order), cut after the first running sum above top_p, then the first sorted entry
 * whose running sum exceeds u[b] * the cut's sum.  r, u: device [batch] uniforms
 * (the reference's sampler_random_float and rand() / RAND_MAX draws); out: device
 * [batch].  The _dt forms take bf16 logits when logits_bf16 != 0.  Both use the
 * library workspace (one stream at a time). */
int be42_sample_temperature(int *out, const float *logits, int n, int batch, float temp, const float *r,
                            void *stream);
int be42_sample_top_p(int *out, const float *logits, int n, int batch, float temp, float top_p, const float *u,
                      void *stream);
int be42_sample_temperature_dt(int *out, const void *logits, int logits_bf16, int n, int batch, float temp,
                               const float *r, void *stream);
int be42_sample_top_p_dt(int *out, const void *logits, int logits_bf16, int n, int batch, float temp, float top_p,
                         const float *u, void *stream);

/* ---- checkpoints --------------------------------------------------------------
 * A decoder from a safetensors checkpoint and an HF config.json: load_config
 * (src/inference/model.c:32-143), load_model / parse_header (src/loader/loader_io.c:44,
 * loader_parse.c:28-110) and the weight mapping by name (model.c:180-265, LLaMA and
 * HF names, output tied to the embedding when absent).  Unlike the reference, which
 * maps every tensor as BF16 (loader_parse.c:48), the dtype is honoured: I8 and F8_E4M3
 * weights with a per-row F32 scale tensor "<name>_scale" ([rows] or [rows, 1]) are
 * streamed as stored; BF16 / F16 / F32 weights are quantized per row on load to
 * quant_kind (0: INT8, 1: FP8 E4M3); norm weights become bf16.  One model holds one
 * weight kind.  Errors: BE42_EINVAL with a message naming the tensor. */
typedef struct be42_model_options {
    int max_seq;     /* 0: 8192 (seq_len, model.c:140) */
    int max_batch;   /* 0: 1 */
    int kv_kind;     /* BE42_KV_INT8 / BE42_KV_BF16 */
    int sparse_k;    /* 0: 64 (SPARSE_BLOCKS_K) */
    int cand_cap;    /* 0: 64 */
    int rope_len;    /* 0: max_seq */
    int quant_kind;  /* kind BF16 / F16 / F32 weights are quantized to */
    int lsh_seed;    /* 0: 42 (model.c:620) */
} be42_model_options;
typedef struct be42_model be42_model;
int  be42_model_load(be42_model **out, const char *model_path, const char *config_path,
                     const be42_model_options *opt);
/* parse, map and validate only (no device work): the config it would use and
 * the weight kind */
int  be42_model_check(const char *model_path, const char *config_path, int quant_kind,
                      be42_decoder_config *cfg_out, int *wkind_out);
be42_decoder *be42_model_decoder(be42_model *m);
int  be42_model_config(const be42_model *m, be42_decoder_config *cfg);
void be42_model_free(be42_model *m);

#ifdef __cplusplus
}
#endif
#endif
