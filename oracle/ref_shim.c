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
