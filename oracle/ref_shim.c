/*
 * ref_shim.c -- flat C wrappers around the compiled reference, so tests can
 * drive it through ctypes.  TEST INFRASTRUCTURE ONLY: compiled together with
 * the reference's own sources (read in place under the reference tree) into
 * oracle/_ref/libref42.so by oracle/Makefile.  It contains no reference code;
 * it includes the reference headers and calls the reference functions.
 */
#include "compute/ops_math_fast.h"
#include "compute/simd_kernels.h"
#include "compute/ops_heap.h"
#include "compute/ops_quant.h"
#include "compute/ops_lsh.h"
#include "compute/ops_attention.h"
#include "compute/ops.h"
#include "memory/paged.h"
#include "tensor/tensor.h"
#include "compute/ops_rope.h"
#include "compute/ops_activation.h"
#include "compute/sampler.h"
#include "memory/kv_cache.h"
#include "memory/arena.h"

#include <stdlib.h>
#include <string.h>

/* header-only helpers */
float ref_fast_expf(float x) { return fast_expf(x); }
float ref_dot_f32_f32(const float *a, const float *b, int n) { return simd_dot_f32_f32(a, b, n); }
float ref_dot_bf16_f32(const uint16_t *a, const float *b, int n) { return simd_dot_bf16_f32(a, b, n); }
uint16_t ref_f32_to_bf16(float f) { return float_to_bf16(f); }

/* heap: push a sequence, return the heap array (scores and indices) */
int ref_heap_run(const float *scores, int n, int cap, float *out_scores, int *out_idx)
{
    t_heap_item heap[256];
    int size = 0;
    if (cap > 256)
        cap = 256;
    for (int i = 0; i < n; i++)
        heap_push(heap, &size, cap, scores[i], i);
    for (int i = 0; i < size; i++) {
        out_scores[i] = heap[i].score;
        out_idx[i] = heap[i].index;
    }
    return size;
}

/* quant */
void ref_fp8_lut(float *out)
{
    quant_init_fp8_lut();
    memcpy(out, g_fp8_lut, sizeof(float) * 256);
}

/* LSH context */
void *ref_lsh_ctx_new(int dim, unsigned int seed)
{
    t_lsh_ctx *c = calloc(1, sizeof(t_lsh_ctx));
    lsh_init(c, dim, seed);
    return c;
}
void ref_lsh_ctx_free(void *c) { free(c); }
void ref_lsh_ctx_get(const void *c, float *hp, float *hpT)
{
    const t_lsh_ctx *x = c;
    for (int h = 0; h < LSH_NUM_HASHES; h++)
        for (int d = 0; d < x->dim; d++) {
            hp[h * x->dim + d] = x->hyperplanes[h][d];
            hpT[d * LSH_NUM_HASHES + h] = x->hp_transposed[d][h];
        }
}
uint16_t ref_lsh_hash(const void *c, const float *v) { return lsh_hash(c, v); }

/* LSH index */
void *ref_lsh_index_new(void)
{
    t_lsh_index *ix = calloc(1, sizeof(t_lsh_index));
    lsh_index_init(ix);
    return ix;
}
void ref_lsh_index_free(void *ix) { free(ix); }
void ref_lsh_insert(void *ix, uint16_t h, int start, int len) { lsh_insert_block(ix, h, start, len); }
int ref_lsh_candidates(const void *ix, uint16_t qh, int *ids, int max_ids)
{
    return lsh_find_candidates(ix, qh, ids, max_ids);
}
int ref_lsh_n_blocks(const void *ix) { return ((const t_lsh_index *)ix)->n_blocks; }

/* paged KV: one block manager plus one per-layer view array */
typedef struct {
    t_block_manager   bm;
    t_paged_kv_cache *pkv;
} ref_paged;

void *ref_paged_new(int n_layers, int n_kv, int hd, int max_blocks)
{
    ref_paged *r = calloc(1, sizeof(ref_paged));
    if (block_manager_init(&r->bm, n_layers, n_kv, hd, max_blocks) != 0) {
        free(r);
        return NULL;
    }
    r->pkv = calloc((size_t)n_layers, sizeof(t_paged_kv_cache));
    for (int l = 0; l < n_layers; l++) {
        r->pkv[l].bm = &r->bm;
        r->pkv[l].layer_idx = l;
    }
    return r;
}
void ref_paged_free(void *p)
{
    ref_paged *r = p;
    block_manager_free(&r->bm);
    free(r->pkv);
    free(r);
}
void ref_paged_append(void *p, int layer, const float *k, const float *v, int pos)
{
    ref_paged *r = p;
    paged_kv_append(&r->pkv[layer], k, v, pos);
}
void ref_paged_reset(void *p, int layer) { ref_paged *r = p; paged_kv_reset(&r->pkv[layer]); }
int ref_paged_n_blocks(void *p, int layer) { return ((ref_paged *)p)->pkv[layer].n_blocks; }
int ref_paged_phys(void *p, int layer, int logical)
{
    ref_paged *r = p;
    return r->bm.page_table[layer * r->bm.max_logical + logical];
}
/* copy one physical page out: codes [n_kv][16][hd], scales [n_kv][16], centroid [hd] */
int ref_paged_page(void *p, int phys, int8_t *kq, int8_t *vq, float *ks, float *vs, float *cen)
{
    ref_paged *r = p;
    t_kv_block *b = &r->bm.blocks[phys];
    int nq = r->bm.n_kv_heads * KV_BLOCK_SIZE * r->bm.head_dim;
    int ns = r->bm.n_kv_heads * KV_BLOCK_SIZE;
    memcpy(kq, b->k_quant, (size_t)nq);
    memcpy(vq, b->v_quant, (size_t)nq);
    memcpy(ks, b->k_scales, sizeof(float) * ns);
    memcpy(vs, b->v_scales, sizeof(float) * ns);
    memcpy(cen, b->centroid, sizeof(float) * r->bm.head_dim);
    return b->n_tokens;
}
void ref_score_blocks(void *p, int layer, const float *q, int n_blocks, int *phys, float *score)
{
    ref_paged *r = p;
    t_block_score *s = malloc(sizeof(t_block_score) * (n_blocks > 0 ? n_blocks : 1));
    score_blocks(s, q, &r->pkv[layer], n_blocks);
    for (int i = 0; i < n_blocks; i++) {
        phys[i] = s[i].phys_idx;
        score[i] = s[i].score;
    }
    free(s);
}
int ref_select_top_k(const int *block_idx, const int *phys, const float *score, int n, int k, int *selected)
{
    t_block_score *s = malloc(sizeof(t_block_score) * (n > 0 ? n : 1));
    for (int i = 0; i < n; i++) {
        s[i].block_idx = block_idx[i];
        s[i].phys_idx = phys[i];
        s[i].score = score[i];
    }
    int cnt = select_top_k_blocks(selected, s, n, k);
    free(s);
    return cnt;
}
void ref_paged_attention(void *p, int layer, float *out, const float *q, int n_heads, float scale)
{
    ref_paged *r = p;
    op_paged_attention(out, q, &r->pkv[layer], n_heads, r->bm.n_kv_heads, r->bm.head_dim, scale);
}
void ref_paged_attention_sparse(void *p, float *out, const float *q, const int *sel, int n_sel,
                                int n_heads, float scale)
{
    ref_paged *r = p;
    op_paged_attention_sparse(out, q, &r->bm, sel, n_sel, n_heads, r->bm.n_kv_heads,
                              r->bm.head_dim, scale);
}

/* linear BF16 token attention (ops_attention.c:41-79) on one head */
void ref_flash_attention_head(float *out, const float *q, const uint16_t *k, const uint16_t *v,
                              int seq_len, int hd, float scale)
{
    flash_attention_head(out, q, k, v, seq_len, hd, scale);
}

/* op_matmul on raw buffers */
int ref_matmul(void *out, int out_dtype, const void *a, int a_dtype, int m, int k,
               const void *b, int b_dtype, int n)
{
    int sa[2] = {m, k}, sb[2] = {k, n}, so[2] = {m, n};
    t_tensor ta = tensor_view((void *)a, sa, 2), tb = tensor_view((void *)b, sb, 2);
    t_tensor to = tensor_view(out, so, 2);
    ta.dtype = a_dtype;
    tb.dtype = b_dtype;
    to.dtype = out_dtype;
    return op_matmul(&to, &ta, &tb);
}

/* decode-step adjacents */
void ref_rmsnorm(float *out, const float *x, const uint16_t *w, int dim, float eps)
{
    int sx[2] = {dim, 1}, sw[1] = {dim};
    t_tensor tx = tensor_view((void *)x, sx, 2), to = tensor_view(out, sx, 2);
    t_tensor tw = tensor_view((void *)w, sw, 1);
    tx.dtype = DTYPE_F32;
    to.dtype = DTYPE_F32;
    tw.dtype = DTYPE_BF16;
    op_rmsnorm(&to, &tx, &tw, eps);
}

int ref_rope_table(float *cos_t, float *sin_t, int hd, int n_pos, float theta)
{
    t_rope_cache *c = rope_cache_init(hd, n_pos, theta);
    if (!c)
        return -1;
    memcpy(cos_t, c->cos_table, sizeof(float) * (size_t)n_pos * (hd / 2));
    memcpy(sin_t, c->sin_table, sizeof(float) * (size_t)n_pos * (hd / 2));
    rope_cache_free(c);
    return 0;
}

void ref_rope_apply(float *data, int n_heads, int hd, int pos, int n_pos, float *cos_t, float *sin_t)
{
    t_rope_cache c;
    c.cos_table = cos_t;
    c.sin_table = sin_t;
    c.head_dim = hd;
    c.max_seq_len = n_pos;
    rope_apply_multihead_cached(data, n_heads, pos, &c);
}

void ref_silu_mul(float *dst, const float *gate, const float *up, int n)
{
    op_silu_mul_fused_f32(dst, gate, up, (size_t)n);
}

int ref_argmax(float *x, int n)
{
    int s[1] = {n};
    t_tensor t = tensor_view(x, s, 1);
    t.dtype = DTYPE_F32;
    return sample_argmax(&t);
}

/* sample_top_p after srand(seed): its draw is the first rand() of that seed */
int ref_sample_top_p(float *x, int n, float temp, float top_p, unsigned int seed)
{
    int s[1] = {n};
    t_tensor t = tensor_view(x, s, 1);
    t.dtype = DTYPE_F32;
    t_arena a;
    arena_init(&a, (size_t)n * 8 + 4096);
    srand(seed);
    const int r = sample_top_p(&t, temp, top_p, &a);
    arena_free(&a);
    return r;
}

/* sample_temperature (its draw comes from the reference's own time-seeded LCG) */
int ref_sample_temperature(float *x, int n, float temp)
{
    int s[1] = {n};
    t_tensor t = tensor_view(x, s, 1);
    t.dtype = DTYPE_F32;
    t_arena a;
    arena_init(&a, (size_t)n * 4 + 4096);
    const int r = sample_temperature(&t, temp, &a);
    arena_free(&a);
    return r;
}

void ref_silu_mul_bf16(uint16_t *dst, const uint16_t *gate, const uint16_t *up, int n)
{
    op_silu_mul_fused_bf16(dst, gate, up, (size_t)n);
}

/* op_rope through a t_rope_ctx: n elements (F32, or BF16 when bf16) */
void ref_op_rope(void *data, int bf16, int n, int pos, int hd, float theta_base, float beta_fast,
                 float beta_slow, float factor, float mscale, float *thetas)
{
    int s[1] = {n};
    t_tensor t = tensor_view(data, s, 1);
    t.dtype = bf16 ? DTYPE_BF16 : DTYPE_F32;
    t_rope_ctx c;
    memset(&c, 0, sizeof c);
    c.head_dim = hd;
    c.theta_base = theta_base;
    c.beta_fast = beta_fast;
    c.beta_slow = beta_slow;
    c.factor = factor;
    c.mscale = mscale;
    c.thetas_cache = thetas;
    op_rope(&t, pos, &c);
}

int ref_argmax_bf16(uint16_t *x, int n)
{
    int s[1] = {n};
    t_tensor t = tensor_view(x, s, 1);
    t.dtype = DTYPE_BF16;
    return sample_argmax(&t);
}

float ref_validate_recall(const float *q, const uint16_t *keys, int n_keys, int dim, const int *lsh, int lsh_k,
                          int actual_k)
{
    return lsh_validate_recall(q, keys, n_keys, dim, lsh, lsh_k, actual_k);
}

int ref_adaptive_k(const float *scores, int n, float threshold)
{
    return adaptive_k_cutoff(scores, NULL, n, threshold);
}

/* linear KV cache path */
static t_kv_cache ref_linear_cache(const uint16_t *k, const uint16_t *v, int n, int n_kv, int hd)
{
    t_kv_cache c;
    int shape[3] = {n, n_kv, hd};
    memset(&c, 0, sizeof c);
    c.k = tensor_view((void *)k, shape, 3);
    c.v = tensor_view((void *)v, shape, 3);
    c.k.dtype = DTYPE_BF16;
    c.v.dtype = DTYPE_BF16;
    c.max_seq_len = n;
    c.num_heads = n_kv;
    c.head_dim = hd;
    c.current_seq_len = n;
    return c;
}

/* idx NULL: op_attention_dense over all n; else op_attention_sparse over
 * n_idx listed tokens; multi != 0: op_multihead_attention */
void ref_attention_linear(float *out, const float *q, const uint16_t *k, const uint16_t *v, int n, const int *idx,
                          int n_idx, int n_heads, int n_kv, int hd, float scale, int multi)
{
    t_kv_cache c = ref_linear_cache(k, v, n, n_kv, hd);
    t_attention_params p;
    p.q = q;
    p.kv_cache = &c;
    p.output = out;
    p.n_heads = n_heads;
    p.n_kv_heads = n_kv;
    p.head_dim = hd;
    p.scale = scale;
    p.topk_idx = (int *)idx;
    p.attend_k = idx ? n_idx : n;
    if (multi)
        op_multihead_attention(&p);
    else if (idx)
        op_attention_sparse(&p);
    else
        op_attention_dense(&p, n);
}

/* kv_cache_init + kv_cache_append of n_tok f32 rows, bf16 rows copied out */
void ref_kv_fill(uint16_t *k_out, uint16_t *v_out, const float *kf, const float *vf, int n_tok, int max_seq,
                 int heads, int dim)
{
    t_arena a;
    t_kv_cache c;
    t_kv_init_params ip = {max_seq, heads, dim};
    arena_init(&a, (size_t)max_seq * heads * dim * 4 + 4096);
    kv_cache_init(&c, &a, &ip);
    for (int t = 0; t < n_tok; t++) {
        int shape[1] = {heads * dim};
        t_tensor tk = tensor_view((void *)(kf + (size_t)t * heads * dim), shape, 1);
        t_tensor tv = tensor_view((void *)(vf + (size_t)t * heads * dim), shape, 1);
        tk.dtype = DTYPE_F32;
        tv.dtype = DTYPE_F32;
        kv_cache_append(&c, &tk, &tv);
    }
    memcpy(k_out, c.k.data, (size_t)c.current_seq_len * heads * dim * 2);
    memcpy(v_out, c.v.data, (size_t)c.current_seq_len * heads * dim * 2);
    arena_free(&a);
}

/* kv_cache_evict over n filled rows (in place); returns the new length */
int ref_kv_evict(uint16_t *k, uint16_t *v, int n, int heads, int dim, const uint16_t *q, const uint16_t *w,
                 int keep_k)
{
    t_arena scratch;
    t_kv_cache c = ref_linear_cache(k, v, n, heads, dim);
    int sq[2] = {heads, dim}, sw[1] = {heads};
    t_tensor tq = tensor_view((void *)q, sq, 2), tw = tensor_view((void *)w, sw, 1);
    t_evict_params ep;
    tq.dtype = DTYPE_BF16;
    tw.dtype = DTYPE_BF16;
    arena_init(&scratch, (size_t)n * 8 + 4096);
    ep.q = &tq;
    ep.w = &tw;
    ep.keep_k = keep_k;
    ep.scratch = &scratch;
    kv_cache_evict(&c, &ep);
    arena_free(&scratch);
    return c.current_seq_len;
}

