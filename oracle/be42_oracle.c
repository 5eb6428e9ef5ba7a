/*
 * be42_oracle.c -- CPU restatement of 42-Berlin-Engine's decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see be42_oracle.h).  Compiled with
 * -ffp-contract=off: every fused multiply-add of the reference is an explicit
 * fmaf() below, every unfused one is a separate multiply and add.
 */
#include "be42_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ======================================================================== */
/* numerics primitives                                                      */
/* ======================================================================== */

/* Schraudolph exponential, src/compute/ops_math_fast.h:48-64.  The reference
 * expression 12102203.0f * x + 1065353216.0f is fused by gcc (GNU C, -mfma);
 * the cast truncates toward zero. */
float or_fast_expf(float x)
{
    if (x < -87.0f)
        return 0.0f;
    if (x > 87.0f)
        x = 87.0f;
    int32_t bits = (int32_t)fmaf(12102203.0f, x, 1065353216.0f);
    float r;
    memcpy(&r, &bits, sizeof r);
    return r;
}

/* round-to-nearest-even on the upper half, no NaN case: tensor.c:67-76 */
uint16_t or_f32_to_bf16(float f)
{
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* tensor.c:78-85 */
float or_bf16_to_f32(uint16_t b)
{
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* Horizontal sum of 8 lanes, simd_hsum_ps (simd_kernels.h:57-68):
 * lo[i] = v[i] + v[i+4]; hadd; hadd  ==  (lo0 + lo1) + (lo2 + lo3). */
static float hsum8(const float v[8])
{
    float l0 = v[0] + v[4], l1 = v[1] + v[5], l2 = v[2] + v[6], l3 = v[3] + v[7];
    return (l0 + l1) + (l2 + l3);
}

/* simd_dot_f32_f32, simd_kernels.h:162-191: 8 lanes, lane l accumulates
 * indices i = l (mod 8) with FMA in ascending order, then hsum8.  The scalar
 * tail loop (:185-189) is itself vectorized by gcc -O3: when 4 or more
 * elements remain, 4 products are formed unfused and added in order, and the
 * last (< 4) elements are fused.  head_dim 64/128 has no tail. */
float or_dot_f32_f32(const float *a, const float *b, int n)
{
    float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 7 < n; i += 8)
        for (int l = 0; l < 8; l++)
            lane[l] = fmaf(a[i + l], b[i + l], lane[l]);
    float sum = hsum8(lane);
    if (n - i >= 4) {
        for (int l = 0; l < 4; l++)
            sum = sum + a[i + l] * b[i + l];
        i += 4;
    }
    for (; i < n; i++)
        sum = fmaf(a[i], b[i], sum);
    return sum;
}

/* simd_dot_bf16_f32, simd_kernels.h:97-156, as compiled without AVX-512
 * (the AVX2 loop, then 0.0f + hsum, then a fused scalar tail). */
float or_dot_bf16_f32(const uint16_t *a, const float *b, int n)
{
    float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 7 < n; i += 8)
        for (int l = 0; l < 8; l++)
            lane[l] = fmaf(or_bf16_to_f32(a[i + l]), b[i + l], lane[l]);
    float sum = 0.0f;
    sum = sum + hsum8(lane);
    for (; i < n; i++)
        sum = fmaf(or_bf16_to_f32(a[i]), b[i], sum);
    return sum;
}

/* ======================================================================== */
/* quant codecs                                                             */
/* ======================================================================== */

/* ops_quant.c:229-270: absmax, scale = amax/127 and inv = 127/amax (both 1
 * when amax == 0), code = clamp((int)roundf(x * inv), -127, 127). */
float or_quant_f32_to_int8(int8_t *out, const float *in, int n)
{
    float amax = 0.0f;
    for (int i = 0; i < n; i++)
        if (fabsf(in[i]) > amax)
            amax = fabsf(in[i]);
    float scale = 1.0f, inv = 1.0f;
    if (amax > 0.0f) {
        scale = amax / 127.0f;
        inv = 127.0f / amax;
    }
    for (int i = 0; i < n; i++) {
        int v = (int)roundf(in[i] * inv);
        if (v > 127) v = 127;
        if (v < -127) v = -127;
        out[i] = (int8_t)v;
    }
    return scale;
}

/* ops_quant.c:275-305 (and dequant_int8, ops_quant.h:104-107) */
void or_dequant_int8(float *out, const int8_t *in, float scale, int n)
{
    for (int i = 0; i < n; i++)
        out[i] = (float)in[i] * scale;
}

/* E4M3 decode, bias 7, no NaN: ops_quant.c:27-48, table built at :53-63. */
void or_fp8_lut(float *lut)
{
    for (int c = 0; c < 256; c++) {
        int e = (c >> 3) & 0xF, m = c & 7;
        float v = (e == 0) ? ldexpf((float)m / 8.0f, -6)
                           : ldexpf(1.0f + (float)m / 8.0f, e - 7);
        lut[c] = (c & 0x80) ? -v : v;
    }
}

/* E4M3 encode, ops_quant.c:68-98: clamp to 448, exponent from floorf(log2f),
 * mantissa rounded half-up and clamped to 7 (no carry into the exponent). */
uint8_t or_float_to_fp8(float v)
{
    if (v == 0.0f)
        return 0;
    int sign = v < 0.0f;
    float a = fabsf(v);
    if (a > 448.0f)
        a = 448.0f;
    int e = (int)floorf(log2f(a)) + 7;
    if (e < 0) e = 0;
    if (e > 15) e = 15;
    float frac = (e == 0) ? a * 64.0f : a / ldexpf(1.0f, e - 7) - 1.0f;
    int m = (int)fmaf(frac, 8.0f, 0.5f);
    if (m > 7) m = 7;
    return (uint8_t)((sign << 7) | (e << 3) | m);
}

/* ops_quant.c:103-136: scale = amax/224, inv = 1/scale, codes of x*inv. */
void or_quant_f32_to_fp8(uint8_t *out, const float *in, int n, float *scale)
{
    float amax = 0.0f;
    for (int i = 0; i < n; i++)
        if (fabsf(in[i]) > amax)
            amax = fabsf(in[i]);
    float inv;
    if (amax > 0.0f) {
        *scale = amax / 224.0f;
        inv = 1.0f / *scale;
    } else {
        *scale = 1.0f;
        inv = 1.0f;
    }
    for (int i = 0; i < n; i++)
        out[i] = or_float_to_fp8(in[i] * inv);
}

void or_quantize_rows_int8(int8_t *q, float *scales, const float *w, int rows, int k)
{
    for (int r = 0; r < rows; r++)
        scales[r] = or_quant_f32_to_int8(q + (size_t)r * k, w + (size_t)r * k, k);
}

void or_quantize_rows_fp8(uint8_t *q, float *scales, const float *w, int rows, int k)
{
    for (int r = 0; r < rows; r++)
        or_quant_f32_to_fp8(q + (size_t)r * k, w + (size_t)r * k, k, &scales[r]);
}

/* ======================================================================== */
/* quantized linear layers                                                  */
/* ======================================================================== */

static void set_threads(int n_threads)
{
#ifdef _OPENMP
    if (n_threads > 0)
        omp_set_num_threads(n_threads);
#else
    (void)n_threads;
#endif
}

/* One output row in the structure of matvec_bf16_f32_blocked
 * (ops_matmul.c:57-153): four 8-lane FMA accumulators over j step 32, an
 * 8-lane cleanup into the first, (s0+s1)+(s2+s3), hsum8, fused scalar tail.
 * The weight element is dequantized first: (float)q * scale (ops_quant.h:104)
 * or lut[q] * scale. */
#define GEMV_ROW(DEQ)                                                            \
    do {                                                                         \
        float acc[4][8];                                                         \
        memset(acc, 0, sizeof acc);                                              \
        int j = 0;                                                               \
        for (; j + 31 < k; j += 32)                                              \
            for (int a = 0; a < 4; a++)                                          \
                for (int l = 0; l < 8; l++) {                                    \
                    int jj = j + 8 * a + l;                                      \
                    acc[a][l] = fmaf(DEQ(row[jj]), xv[jj], acc[a][l]);           \
                }                                                                \
        for (; j + 7 < k; j += 8)                                                \
            for (int l = 0; l < 8; l++)                                          \
                acc[0][l] = fmaf(DEQ(row[j + l]), xv[j + l], acc[0][l]);         \
        float s[8];                                                              \
        for (int l = 0; l < 8; l++)                                              \
            s[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);            \
        float sum = hsum8(s);                                                    \
        for (; j < k; j++)                                                       \
            sum = fmaf(DEQ(row[j]), xv[j], sum);                                 \
        yv[i] = sum;                                                             \
    } while (0)

void or_gemv_q8(float *y, const int8_t *w, const float *scales, const float *x,
                int n, int k, int batch, int n_threads)
{
    set_threads(n_threads);
    for (int b = 0; b < batch; b++) {
        const float *xv = x + (size_t)b * k;
        float *yv = y + (size_t)b * n;
        #pragma omp parallel for schedule(static)
        for (int i = 0; i < n; i++) {
            const int8_t *row = w + (size_t)i * k;
            const float sc = scales[i];
#define DEQ_I8(q) ((float)(q) * sc)
            GEMV_ROW(DEQ_I8);
#undef DEQ_I8
        }
    }
}

void or_gemv_fp8(float *y, const uint8_t *w, const float *scales, const float *x,
                 int n, int k, int batch, int n_threads)
{
    float lut[256];
    or_fp8_lut(lut);
    set_threads(n_threads);
    for (int b = 0; b < batch; b++) {
        const float *xv = x + (size_t)b * k;
        float *yv = y + (size_t)b * n;
        #pragma omp parallel for schedule(static)
        for (int i = 0; i < n; i++) {
            const uint8_t *row = w + (size_t)i * k;
            const float sc = scales[i];
#define DEQ_F8(q) (lut[(q)] * sc)
            GEMV_ROW(DEQ_F8);
#undef DEQ_F8
        }
    }
}

void or_gemv_bf16(float *y, const uint16_t *w, const float *x, int n, int k, int n_threads)
{
    set_threads(n_threads);
    const float *xv = x;
    float *yv = y;
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < n; i++) {
        const uint16_t *row = w + (size_t)i * k;
#define DEQ_BF(q) or_bf16_to_f32(q)
        GEMV_ROW(DEQ_BF);
#undef DEQ_BF
    }
}

void or_gemm_i8_acc(int32_t *acc, const int8_t *xq, const int8_t *wq,
                    int m, int n, int k, int n_threads)
{
    set_threads(n_threads);
    #pragma omp parallel for collapse(2) schedule(static)
    for (int r = 0; r < m; r++)
        for (int i = 0; i < n; i++) {
            const int8_t *a = xq + (size_t)r * k, *b = wq + (size_t)i * k;
            int32_t s = 0;
            for (int j = 0; j < k; j++)
                s += (int32_t)a[j] * (int32_t)b[j];
            acc[(size_t)r * n + i] = s;
        }
}

void or_gemm_i8(float *y, const int8_t *xq, const float *sx, const int8_t *wq,
                const float *sw, int m, int n, int k, int n_threads)
{
    set_threads(n_threads);
    #pragma omp parallel for collapse(2) schedule(static)
    for (int r = 0; r < m; r++)
        for (int i = 0; i < n; i++) {
            const int8_t *a = xq + (size_t)r * k, *b = wq + (size_t)i * k;
            int32_t s = 0;
            for (int j = 0; j < k; j++)
                s += (int32_t)a[j] * (int32_t)b[j];
            y[(size_t)r * n + i] = ((float)s * sx[r]) * sw[i];
        }
}

void or_gemm_fp8(float *y, const uint8_t *xq, const float *sx, const uint8_t *wq,
                 const float *sw, int m, int n, int k, int n_threads)
{
    float lut[256];
    or_fp8_lut(lut);
    set_threads(n_threads);
    #pragma omp parallel for collapse(2) schedule(static)
    for (int r = 0; r < m; r++)
        for (int i = 0; i < n; i++) {
            const uint8_t *a = xq + (size_t)r * k, *b = wq + (size_t)i * k;
            float s = 0.0f;
            for (int j = 0; j < k; j++)
                s = fmaf(lut[a[j]], lut[b[j]], s);
            y[(size_t)r * n + i] = (s * sx[r]) * sw[i];
        }
}

/* ======================================================================== */
/* LSH                                                                      */
/* ======================================================================== */

/* ops_lsh.c:22-34: LCG, 15-bit uniforms, Box-Muller with libm. */
static float lcg_gaussian(unsigned int *s)
{
    *s = *s * 1103515245u + 12345u;
    float u1 = (float)((*s >> 16) & 0x7FFF) / 32767.0f;
    *s = *s * 1103515245u + 12345u;
    float u2 = (float)((*s >> 16) & 0x7FFF) / 32767.0f;
    if (u1 < 1e-6f)
        u1 = 1e-6f;
    return sqrtf(-2.0f * logf(u1)) * cosf(2.0f * 3.14159265f * u2);
}

/* ops_lsh.c:40-85: 16 Gaussian rows, each L2-normalised (the squared norm is
 * accumulated with a fused multiply-add), then transposed to [dim][16]. */
void or_lsh_init(float *hp, float *hpT, int dim, unsigned int seed)
{
    if (dim > 256)
        dim = 256;
    for (int h = 0; h < OR_LSH_BITS; h++) {
        float nrm = 0.0f;
        for (int d = 0; d < dim; d++) {
            float g = lcg_gaussian(&seed);
            hp[h * dim + d] = g;
            nrm = fmaf(g, g, nrm);
        }
        nrm = sqrtf(nrm);
        if (nrm > 1e-6f)
            for (int d = 0; d < dim; d++)
                hp[h * dim + d] /= nrm;
    }
    for (int d = 0; d < dim; d++)
        for (int h = 0; h < OR_LSH_BITS; h++)
            hpT[d * OR_LSH_BITS + h] = hp[h * dim + d];
}

/* ops_lsh.c:138-242: bit h is set when the FMA chain over d ascending,
 * s_h = fma(v[d], hpT[d][h], s_h) from +0, ends strictly above zero. */
uint16_t or_lsh_hash(const float *hpT, int dim, const float *v)
{
    if (dim > 256) dim = 256;
    if (dim <= 0) return 0;
    float s[OR_LSH_BITS];
    for (int h = 0; h < OR_LSH_BITS; h++)
        s[h] = 0.0f;
    for (int d = 0; d < dim; d++)
        for (int h = 0; h < OR_LSH_BITS; h++)
            s[h] = fmaf(v[d], hpT[d * OR_LSH_BITS + h], s[h]);
    uint16_t hash = 0;
    for (int h = 0; h < OR_LSH_BITS; h++)
        if (s[h] > 0.0f)
            hash |= (uint16_t)(1u << h);
    return hash;
}

int or_hamming(uint16_t a, uint16_t b)
{
    return __builtin_popcount((unsigned)(a ^ b));
}

int or_lsh_index_create(or_lsh_index *ix, int cap)
{
    memset(ix, 0, sizeof *ix);
    ix->cap = cap;
    ix->hash = calloc((size_t)cap, sizeof *ix->hash);
    ix->start = calloc((size_t)cap, sizeof *ix->start);
    ix->len = calloc((size_t)cap, sizeof *ix->len);
    ix->next = calloc((size_t)cap, sizeof *ix->next);
    ix->heads = malloc(sizeof(int) * OR_LSH_BUCKETS);
    if (!ix->hash || !ix->start || !ix->len || !ix->next || !ix->heads) {
        or_lsh_index_destroy(ix);
        return -1;
    }
    or_lsh_index_reset(ix);
    return 0;
}

void or_lsh_index_destroy(or_lsh_index *ix)
{
    free(ix->hash); free(ix->start); free(ix->len); free(ix->next); free(ix->heads);
    memset(ix, 0, sizeof *ix);
}

/* ops_lsh.c:90-118 */
void or_lsh_index_reset(or_lsh_index *ix)
{
    ix->n_blocks = 0;
    for (int b = 0; b < OR_LSH_BUCKETS; b++)
        ix->heads[b] = -1;
}

/* ops_lsh.c:256-272: append, then push on the bucket's chain (LIFO);
 * silently dropped once the index is full. */
void or_lsh_insert_block(or_lsh_index *ix, uint16_t h, int start, int len)
{
    if (ix->n_blocks >= ix->cap)
        return;
    int id = ix->n_blocks;
    ix->hash[id] = h;
    ix->start[id] = start;
    ix->len[id] = len;
    int bucket = h % OR_LSH_BUCKETS;
    ix->next[id] = ix->heads[bucket];
    ix->heads[bucket] = id;
    ix->n_blocks++;
}

/* ops_lsh.c:361-418: probe 0 is the query hash, probe p>0 flips bit p-1;
 * each probed bucket's chain is walked newest first, filtered by Hamming
 * radius 4 and de-duplicated with a bitmap; stops at max_ids. */
int or_lsh_find_candidates(const or_lsh_index *ix, uint16_t qh, int *ids, int max_ids)
{
    int words = (ix->cap + 63) / 64;
    uint64_t *seen = calloc((size_t)(words ? words : 1), sizeof(uint64_t));
    int n = 0;
    for (int probe = 0; probe <= OR_LSH_BITS && n < max_ids; probe++) {
        uint16_t ph = probe == 0 ? qh : (uint16_t)(qh ^ (1u << (probe - 1)));
        int id = ix->heads[ph % OR_LSH_BUCKETS];
        while (id != -1 && n < max_ids) {
            if (or_hamming(qh, ix->hash[id]) <= OR_LSH_RADIUS) {
                uint64_t bit = 1ull << (id % 64);
                if (!(seen[id / 64] & bit)) {
                    seen[id / 64] |= bit;
                    ids[n++] = id;
                }
            }
            id = ix->next[id];
        }
    }
    free(seen);
    return n;
}

void or_q_mean(float *qm, const float *q, int n_heads, int hd)
{
    for (int d = 0; d < hd; d++)
        qm[d] = 0.0f;
    for (int h = 0; h < n_heads; h++)
        for (int d = 0; d < hd; d++)
            qm[d] += q[h * hd + d];
    for (int d = 0; d < hd; d++)
        qm[d] /= (float)n_heads;
}

/* ======================================================================== */
/* selection                                                                */
/* ======================================================================== */

/* ops_heap.h:33-100: min-heap on score; a full heap replaces its root only
 * for a strictly larger score. */
static void heap_down(float *hs, int *hi, int size, int i)
{
    for (;;) {
        int sm = i, l = 2 * i + 1, r = 2 * i + 2;
        if (l < size && hs[l] < hs[sm]) sm = l;
        if (r < size && hs[r] < hs[sm]) sm = r;
        if (sm == i) break;
        float ts = hs[i]; hs[i] = hs[sm]; hs[sm] = ts;
        int ti = hi[i]; hi[i] = hi[sm]; hi[sm] = ti;
        i = sm;
    }
}

static void heap_up(float *hs, int *hi, int i)
{
    while (i > 0) {
        int p = (i - 1) / 2;
        if (hs[p] <= hs[i]) break;
        float ts = hs[i]; hs[i] = hs[p]; hs[p] = ts;
        int ti = hi[i]; hi[i] = hi[p]; hi[p] = ti;
        i = p;
    }
}

void or_heap_push(float *hs, int *hi, int *size, int cap, float score, int index)
{
    if (*size < cap) {
        hs[*size] = score;
        hi[*size] = index;
        heap_up(hs, hi, *size);
        (*size)++;
    } else if (score > hs[0]) {
        hs[0] = score;
        hi[0] = index;
        heap_down(hs, hi, *size, 0);
    }
}

/* paged.c:439-495: first and last entries are anchors; the heap keeps the
 * best min(k-2, n-2, 62) of entries 1..n-2; output is the heap array order. */
int or_select_top_k_blocks(int *selected, const or_block_score *s, int n_blocks, int k)
{
    if (n_blocks <= 0)
        return 0;
    int first = s[0].phys_idx, cnt = 0;
    selected[cnt++] = first;
    int last = s[n_blocks - 1].phys_idx;
    if (last != first && n_blocks > 1)
        selected[cnt++] = last;
    if (n_blocks <= 2 || k <= 2)
        return cnt;
    int ak = k - 2;
    if (ak > n_blocks - 2) ak = n_blocks - 2;
    if (ak > OR_HEAP_MAX) ak = OR_HEAP_MAX;
    float hs[OR_HEAP_MAX];
    int hi[OR_HEAP_MAX], hsize = 0;
    for (int i = 1; i < n_blocks - 1; i++)
        or_heap_push(hs, hi, &hsize, ak, s[i].score, i);
    for (int i = 0; i < hsize; i++)
        selected[cnt++] = s[hi[i]].phys_idx;
    return cnt;
}

/* ======================================================================== */
/* paged KV cache                                                           */
/* ======================================================================== */

static size_t page_elems(const or_paged *p) { return (size_t)p->n_kv * OR_PAGE_TOKENS * p->hd; }

int or_paged_init(or_paged *p, int n_layers, int n_kv, int hd, int max_logical, int kind)
{
    memset(p, 0, sizeof *p);
    p->n_layers = n_layers; p->n_kv = n_kv; p->hd = hd;
    p->max_logical = max_logical; p->kind = kind;
    p->cap = n_layers * max_logical;
    size_t pe = page_elems(p), cap = (size_t)p->cap;
    if (kind == OR_KV_INT8) {
        p->kq = calloc(cap * pe, 1);
        p->vq = calloc(cap * pe, 1);
        p->ks = calloc(cap * n_kv * OR_PAGE_TOKENS, sizeof(float));
        p->vs = calloc(cap * n_kv * OR_PAGE_TOKENS, sizeof(float));
    } else {
        p->kb = calloc(cap * pe, sizeof(uint16_t));
        p->vb = calloc(cap * pe, sizeof(uint16_t));
    }
    p->centroid = calloc(cap * hd, sizeof(float));
    p->ntok = calloc(cap, sizeof(int));
    p->start_pos = malloc(cap * sizeof(int));
    p->registered = calloc(cap, sizeof(int));
    p->page_table = malloc(cap * sizeof(int));
    p->free_stack = malloc(cap * sizeof(int));
    p->logical_len = calloc((size_t)n_layers, sizeof(int));
    if (!p->centroid || !p->ntok || !p->start_pos || !p->registered || !p->page_table ||
        !p->free_stack || !p->logical_len || (kind == OR_KV_INT8 ? (!p->kq || !p->vq || !p->ks || !p->vs)
                                                                 : (!p->kb || !p->vb))) {
        or_paged_free(p);
        return -1;
    }
    for (int i = 0; i < p->cap; i++) {
        p->start_pos[i] = -1;
        p->page_table[i] = -1;
        p->free_stack[i] = i;
    }
    p->free_top = p->cap - 1;
    return 0;
}

void or_paged_free(or_paged *p)
{
    free(p->kq); free(p->vq); free(p->kb); free(p->vb); free(p->ks); free(p->vs);
    free(p->centroid); free(p->ntok); free(p->start_pos); free(p->registered);
    free(p->page_table); free(p->free_stack); free(p->logical_len);
    memset(p, 0, sizeof *p);
}

/* paged.c:159-179: pop the free stack (first allocation is cap-1); the page
 * keeps its old centroid and codes. */
int or_paged_alloc(or_paged *p)
{
    if (p->free_top < 0)
        return -1;
    int phys = p->free_stack[p->free_top--];
    p->ntok[phys] = 0;
    p->start_pos[phys] = -1;
    p->registered[phys] = 0;
    return phys;
}

void or_paged_release(or_paged *p, int phys)
{
    if (phys < 0 || phys >= p->cap)
        return;
    p->free_stack[++p->free_top] = phys;
}

/* paged.c:350-393: per dimension, the head-0 keys of the page are dequantized
 * and summed token by token, then multiplied by 1.0f/n. */
void or_centroid_int8(float *c, const int8_t *kq, const float *ks, int ntok, int hd)
{
    if (ntok <= 0)
        return;
    for (int d = 0; d < hd; d++)
        c[d] = 0.0f;
    for (int t = 0; t < ntok; t++)
        for (int d = 0; d < hd; d++)
            c[d] = c[d] + (float)kq[t * hd + d] * ks[t];
    float inv = 1.0f / (float)ntok;
    for (int d = 0; d < hd; d++)
        c[d] = c[d] * inv;
}

/* The same centroid on bf16 rows (storage extension, same summation order). */
void or_centroid_bf16(float *c, const uint16_t *kb, int ntok, int hd)
{
    if (ntok <= 0)
        return;
    for (int d = 0; d < hd; d++)
        c[d] = 0.0f;
    for (int t = 0; t < ntok; t++)
        for (int d = 0; d < hd; d++)
            c[d] = c[d] + or_bf16_to_f32(kb[t * hd + d]);
    float inv = 1.0f / (float)ntok;
    for (int d = 0; d < hd; d++)
        c[d] = c[d] * inv;
}

/* paged.c:195-272: page = pos/16, slot = pos%16; a new logical page takes
 * the top of the free stack; every KV head's K and V row is quantized
 * (INT8: quant_f32_to_int8; BF16: tensor.c:67-76); a page that becomes full
 * gets its head-0 centroid. */
int or_paged_append(or_paged *p, int layer, const float *k, const float *v, int pos)
{
    int blk = pos / OR_PAGE_TOKENS, off = pos % OR_PAGE_TOKENS;
    int base = layer * p->max_logical;
    if (blk >= p->logical_len[layer]) {
        int phys = or_paged_alloc(p);
        if (phys < 0)
            return -1;
        p->page_table[base + blk] = phys;
        p->logical_len[layer] = blk + 1;
        p->start_pos[phys] = blk * OR_PAGE_TOKENS;
    }
    int phys = p->page_table[base + blk];
    int hd = p->hd;
    for (int h = 0; h < p->n_kv; h++) {
        size_t row = (size_t)phys * page_elems(p) + ((size_t)h * OR_PAGE_TOKENS + off) * hd;
        size_t sidx = ((size_t)phys * p->n_kv + h) * OR_PAGE_TOKENS + off;
        if (p->kind == OR_KV_INT8) {
            p->ks[sidx] = or_quant_f32_to_int8(p->kq + row, k + h * hd, hd);
            p->vs[sidx] = or_quant_f32_to_int8(p->vq + row, v + h * hd, hd);
        } else {
            for (int d = 0; d < hd; d++) {
                p->kb[row + d] = or_f32_to_bf16(k[h * hd + d]);
                p->vb[row + d] = or_f32_to_bf16(v[h * hd + d]);
            }
        }
    }
    p->ntok[phys] = off + 1;
    if (p->ntok[phys] == OR_PAGE_TOKENS && !p->registered[phys]) {
        size_t head0 = (size_t)phys * page_elems(p);
        if (p->kind == OR_KV_INT8)
            or_centroid_int8(p->centroid + (size_t)phys * hd, p->kq + head0,
                             p->ks + (size_t)phys * p->n_kv * OR_PAGE_TOKENS, OR_PAGE_TOKENS, hd);
        else
            or_centroid_bf16(p->centroid + (size_t)phys * hd, p->kb + head0, OR_PAGE_TOKENS, hd);
        p->registered[phys] = 1;
    }
    return phys;
}

/* paged.c:312-336 */
void or_paged_reset(or_paged *p, int layer)
{
    int base = layer * p->max_logical;
    for (int i = 0; i < p->logical_len[layer]; i++) {
        int phys = p->page_table[base + i];
        if (phys >= 0)
            or_paged_release(p, phys);
        p->page_table[base + i] = -1;
    }
    p->logical_len[layer] = 0;
}

/* paged.c:401-431 */
void or_score_blocks(or_block_score *s, const float *q, const or_paged *p, int layer, int n_blocks)
{
    int base = layer * p->max_logical;
    for (int i = 0; i < n_blocks; i++) {
        int phys = p->page_table[base + i];
        s[i].block_idx = i;
        s[i].phys_idx = phys;
        s[i].score = phys < 0 ? -1e9f : or_dot_f32_f32(q, p->centroid + (size_t)phys * p->hd, p->hd);
    }
}

/* ======================================================================== */
/* attention                                                                */
/* ======================================================================== */

/* One online-softmax step of the INT8 block kernel (ops_attention.c:330-346):
 *   m' = max(m, s); a = fast_expf(m - m'); p = fast_expf(s - m');
 *   l = l * a + p (fused); out = out * a; out = fma(p, v, out). */
static void attend_page_int8(float *o, float *m, float *l, const float *qh, const int8_t *kq,
                             const float *ks, const int8_t *vq, const float *vs, int ntok,
                             int hd, float scale, float *kbuf, float *vbuf)
{
    for (int t = 0; t < ntok; t++) {
        or_dequant_int8(kbuf + t * hd, kq + t * hd, ks[t], hd);
        or_dequant_int8(vbuf + t * hd, vq + t * hd, vs[t], hd);
    }
    for (int t = 0; t < ntok; t++) {
        float s = or_dot_f32_f32(qh, kbuf + t * hd, hd) * scale;
        float prev = *m;
        if (s > prev)
            *m = s;
        float a = or_fast_expf(prev - *m);
        float pr = or_fast_expf(s - *m);
        *l = fmaf(*l, a, pr);
        for (int d = 0; d < hd; d++)
            o[d] = o[d] * a;
        for (int d = 0; d < hd; d++)
            o[d] = fmaf(pr, vbuf[t * hd + d], o[d]);
    }
}

/* One step of the BF16 token kernel (ops_attention.c:131-170): score from
 * simd_dot_bf16_f32, out = out * a then fma(p, bf16(v), out)
 * (simd_rescale_fma_bf16, simd_kernels.h:264-301). */
static void attend_page_bf16(float *o, float *m, float *l, const float *qh, const uint16_t *kb,
                             const uint16_t *vb, int ntok, int hd, float scale)
{
    for (int t = 0; t < ntok; t++) {
        float s = or_dot_bf16_f32(kb + t * hd, qh, hd) * scale;
        float prev = *m;
        if (s > prev)
            *m = s;
        float a = or_fast_expf(prev - *m);
        float pr = or_fast_expf(s - *m);
        *l = fmaf(*l, a, pr);
        for (int d = 0; d < hd; d++)
            o[d] = fmaf(pr, or_bf16_to_f32(vb[t * hd + d]), o[d] * a);
    }
}

static void attend_head(float *o, const float *qh, const or_paged *p, const int *pages,
                        int n_pages, int kvh, float scale)
{
    int hd = p->hd;
    float m = -INFINITY, l = 0.0f;
    float *kbuf = malloc(sizeof(float) * OR_PAGE_TOKENS * hd);
    float *vbuf = malloc(sizeof(float) * OR_PAGE_TOKENS * hd);
    for (int d = 0; d < hd; d++)
        o[d] = 0.0f;
    for (int i = 0; i < n_pages; i++) {
        int phys = pages[i];
        if (phys < 0 || p->ntok[phys] <= 0)
            continue;
        size_t row = (size_t)phys * page_elems(p) + (size_t)kvh * OR_PAGE_TOKENS * hd;
        if (p->kind == OR_KV_INT8) {
            size_t sidx = ((size_t)phys * p->n_kv + kvh) * OR_PAGE_TOKENS;
            attend_page_int8(o, &m, &l, qh, p->kq + row, p->ks + sidx, p->vq + row, p->vs + sidx,
                             p->ntok[phys], hd, scale, kbuf, vbuf);
        } else {
            attend_page_bf16(o, &m, &l, qh, p->kb + row, p->vb + row, p->ntok[phys], hd, scale);
        }
    }
    if (l > 0.0f) {
        float inv = 1.0f / l;
        for (int d = 0; d < hd; d++)
            o[d] = o[d] * inv;
    }
    free(kbuf);
    free(vbuf);
}

/* ops_attention.c:443-461: query head h reads KV head h / (n_heads / n_kv). */
void or_paged_attention_pages(float *out, const float *q, const or_paged *p,
                              const int *pages, int n_pages, int n_heads,
                              float scale, int n_threads)
{
    set_threads(n_threads);
    int group = n_heads / p->n_kv;
    #pragma omp parallel for schedule(static)
    for (int h = 0; h < n_heads; h++)
        attend_head(out + (size_t)h * p->hd, q + (size_t)h * p->hd, p, pages, n_pages,
                    h / group, scale);
}

void or_paged_attention_dense(float *out, const float *q, const or_paged *p, int layer,
                              int n_heads, float scale, int n_threads)
{
    int n = p->logical_len[layer];
    int *pages = malloc(sizeof(int) * (n > 0 ? n : 1));
    for (int i = 0; i < n; i++)
        pages[i] = p->page_table[layer * p->max_logical + i];
    or_paged_attention_pages(out, q, p, pages, n, n_heads, scale, n_threads);
    free(pages);
}

/* ======================================================================== */
/* linear KV cache path                                                     */
/* ======================================================================== */

/* ops_attention.c:84-245: per query head, the online softmax of
 * flash_attention_head over the listed tokens of its KV head (the token
 * step of attend_page_bf16), then o *= 1 / l. */
void or_attention_linear(float *out, const float *q, const uint16_t *k, const uint16_t *v, const int *idx,
                         int n, int n_heads, int n_kv, int hd, float scale, int n_threads)
{
    set_threads(n_threads);
    const int group = n_heads / n_kv;
    #pragma omp parallel for schedule(static)
    for (int h = 0; h < n_heads; h++) {
        const int kvh = h / group;
        float *o = out + (size_t)h * hd;
        const float *qh = q + (size_t)h * hd;
        float m = -INFINITY, l = 0.0f;
        for (int d = 0; d < hd; d++)
            o[d] = 0.0f;
        for (int i = 0; i < n; i++) {
            const int t = idx ? idx[i] : i;
            const size_t row = ((size_t)t * n_kv + kvh) * hd;
            attend_page_bf16(o, &m, &l, qh, k + row, v + row, 1, hd, scale);
        }
        if (l > 0.0f) {
            float inv = 1.0f / l;
            for (int d = 0; d < hd; d++)
                o[d] = o[d] * inv;
        }
    }
}

typedef struct { float val; int idx; } or_score_index;

/* qsort in glibc sorts with a stable merge sort: equal scores keep their
 * position order */
static int or_cmp_evict(const void *a, const void *b)
{
    const or_score_index *x = a, *y = b;
    if (x->val != y->val)
        return x->val < y->val ? 1 : -1;
    return (x->idx > y->idx) - (x->idx < y->idx);
}

static int or_cmp_idx(const void *a, const void *b)
{
    return ((const or_score_index *)a)->idx - ((const or_score_index *)b)->idx;
}

int or_kv_evict(uint16_t *k, uint16_t *v, int n, int heads, int dim, const uint16_t *q, const uint16_t *w,
                int keep_k)
{
    if (keep_k <= 0)
        return n;
    if (keep_k > n)
        keep_k = n;
    if (n <= keep_k)
        return n;
    or_score_index *si = malloc(sizeof(or_score_index) * (size_t)n);
    for (int s = 0; s < n; s++) {
        float total = 0.0f;
        for (int h = 0; h < heads; h++) {
            float dot = 0.0f;
            const size_t off = ((size_t)s * heads + h) * dim;
            for (int d = 0; d < dim; d++)
                dot = fmaf(or_bf16_to_f32(q[h * dim + d]), or_bf16_to_f32(k[off + d]), dot);
            if (dot < 0)
                dot = 0.0f;
            total = fmaf(or_bf16_to_f32(w[h]), dot, total);
        }
        si[s].val = total;
        si[s].idx = s;
    }
    qsort(si, (size_t)n, sizeof *si, or_cmp_evict);
    qsort(si, (size_t)keep_k, sizeof *si, or_cmp_idx);
    const size_t blk = (size_t)heads * dim;
    for (int i = 0; i < keep_k; i++)
        if (si[i].idx != i) {
            memcpy(k + i * blk, k + (size_t)si[i].idx * blk, blk * 2);
            memcpy(v + i * blk, v + (size_t)si[i].idx * blk, blk * 2);
        }
    free(si);
    return keep_k;
}

static int or_cmp_int(const void *a, const void *b)
{
    const int x = *(const int *)a, y = *(const int *)b;
    return (x > y) - (x < y);
}

int or_route_tokens(int *topk, const uint16_t *k, int kv_len, int n_kv, int hd, const float *q, int n_heads,
                    const float *hpT, const or_lsh_index *ix, int window, int sparse_k)
{
    if (!(sparse_k > 0 && kv_len > sparse_k))
        return kv_len;
    int *cand = malloc(sizeof(int) * (size_t)kv_len);
    int nc = 0;
    const int ws = kv_len > window ? kv_len - window : 0;
    for (int t = ws; t < kv_len; t++)
        cand[nc++] = t;
    if (ws > 0 && ix && ix->n_blocks > 0) {
        float *qm = malloc(sizeof(float) * (size_t)hd);
        or_q_mean(qm, q, n_heads, hd);
        uint16_t qh = or_lsh_hash(hpT, hd, qm);
        free(qm);
        int ids[64];
        int nb = or_lsh_find_candidates(ix, qh, ids, 64);
        for (int b = 0; b < nb && nc < kv_len; b++) {
            int st = ix->start[ids[b]], ln = ix->len[ids[b]];
            if (st + ln <= ws)
                for (int p = 0; p < ln && nc < kv_len; p++)
                    if (st + p < ws)
                        cand[nc++] = st + p;
        }
    }
    if (nc > 1)
        qsort(cand, (size_t)nc, sizeof(int), or_cmp_int);
    const int group = n_heads / n_kv;
    int size = 0, cap = nc < sparse_k ? nc : sparse_k;
    float *hs = malloc(sizeof(float) * (size_t)(cap > 0 ? cap : 1));
    int *hi = malloc(sizeof(int) * (size_t)(cap > 0 ? cap : 1));
    for (int c = 0; c < nc; c++) {
        const int t = cand[c];
        float score = 0.0f;
        for (int kv = 0; kv < n_kv; kv++)
            score += or_dot_bf16_f32(k + ((size_t)t * n_kv + kv) * hd, q + (size_t)kv * group * hd, hd);
        or_heap_push(hs, hi, &size, cap, score, t);
    }
    for (int i = 0; i < size; i++)
        topk[i] = hi[i];
    free(hs);
    free(hi);
    free(cand);
    return size;
}

/* ======================================================================== */
/* routing composition                                                      */
/* ======================================================================== */

int or_route_pages(int *selected, int *n_cand_out, int *cand_out,
                   const or_paged *p, int layer, const float *q, int n_heads,
                   const float *hpT, const or_lsh_index *ix, int cand_cap, int k)
{
    int n = p->logical_len[layer], base = layer * p->max_logical;
    if (n_cand_out)
        *n_cand_out = 0;
    if (n <= 0)
        return 0;
    if (n <= k) {
        for (int i = 0; i < n; i++)
            selected[i] = p->page_table[base + i];
        return n;
    }
    float *qm = malloc(sizeof(float) * p->hd);
    or_q_mean(qm, q, n_heads, p->hd);
    uint16_t qh = or_lsh_hash(hpT, p->hd, qm);
    free(qm);
    int *cand = malloc(sizeof(int) * (cand_cap > 0 ? cand_cap : 1));
    int nc = or_lsh_find_candidates(ix, qh, cand, cand_cap);
    if (n_cand_out)
        *n_cand_out = nc;
    if (cand_out)
        memcpy(cand_out, cand, sizeof(int) * nc);
    or_block_score *list = malloc(sizeof(or_block_score) * (nc + 2));
    int m = 0;
    list[m].block_idx = 0;
    list[m].phys_idx = p->page_table[base];
    m++;
    for (int i = 0; i < nc; i++) {
        int lg = cand[i];
        if (lg == 0 || lg == n - 1 || lg >= n)
            continue;
        list[m].block_idx = lg;
        list[m].phys_idx = p->page_table[base + lg];
        m++;
    }
    list[m].block_idx = n - 1;
    list[m].phys_idx = p->page_table[base + n - 1];
    m++;
    for (int i = 0; i < m; i++) {
        int phys = list[i].phys_idx;
        list[i].score = phys < 0 ? -1e9f : or_dot_f32_f32(q, p->centroid + (size_t)phys * p->hd, p->hd);
    }
    int ns = or_select_top_k_blocks(selected, list, m, k);
    free(list);
    free(cand);
    return ns;
}

/* ======================================================================== */
/* decode-step adjacents and the decoder loop                               */
/* ======================================================================== */

/* op_rmsnorm, ops_norm.c:27-124: sum of squares in 8 FMA lanes (lane l over
 * i = l (mod 8)), hsum tree, fused scalar remainder; ss / dim;
 * inv = 1 / sqrtf(ss + eps); out = (x * inv) * bf16(w). */
void or_rmsnorm(float *out, const float *x, const uint16_t *w, int dim, float eps)
{
    float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int j = 0;
    for (; j + 7 < dim; j += 8)
        for (int l = 0; l < 8; l++)
            lane[l] = fmaf(x[j + l], x[j + l], lane[l]);
    float ss = hsum8(lane);
    for (; j < dim; j++)
        ss = fmaf(x[j], x[j], ss);
    ss = ss / (float)dim;
    const float inv = 1.0f / sqrtf(ss + eps);
    for (int i = 0; i < dim; i++)
        out[i] = (x[i] * inv) * or_bf16_to_f32(w[i]);
}

/* rope_cache_init, ops_rope.c:30-95 (libm): inv_freq[i] = 1 / powf(theta,
 * (2i) / hd); angle = (float)p * inv_freq[i]; tables [pos][hd/2]. */
void or_rope_table(float *cos_t, float *sin_t, int hd, int n_pos, float theta)
{
    int half = hd / 2;
    float *inv = malloc(sizeof(float) * (size_t)half);
    for (int i = 0; i < half; i++)
        inv[i] = 1.0f / powf(theta, (float)(i * 2) / (float)hd);
    for (int p = 0; p < n_pos; p++)
        for (int i = 0; i < half; i++) {
            float a = (float)p * inv[i];
            cos_t[(size_t)p * half + i] = cosf(a);
            sin_t[(size_t)p * half + i] = sinf(a);
        }
    free(inv);
}

/* rope_apply_multihead_cached, ops_rope.c:192-228, as the compiled loop
 * evaluates it: x0' = fma(x0, c, -(x1 * s)), x1' = fma(x0, s, x1 * c);
 * positions at or past the table are left unrotated. */
void or_rope_apply(float *data, int n_heads, int hd, int pos, int n_pos, const float *cos_t, const float *sin_t)
{
    if (pos >= n_pos)
        return;
    int half = hd / 2;
    const float *cr = cos_t + (size_t)pos * half, *sr = sin_t + (size_t)pos * half;
    for (int h = 0; h < n_heads; h++) {
        float *x = data + (size_t)h * hd;
        for (int i = 0; i < half; i++) {
            float c = cr[i], s = sr[i], x0 = x[i], x1 = x[i + half];
            x[i] = fmaf(x0, c, -(x1 * s));
            x[i + half] = fmaf(x0, s, x1 * c);
        }
    }
}

/* theta of pair index j2 = 2j for op_rope without a thetas cache
 * (get_yarn_theta / compute_yarn_ramp, ops_rope.c:243-276): frequency index
 * j2 / hd in float, powers in double, YaRN ramp between beta_slow / hd and
 * beta_fast / hd when factor > 1.  The ramp's (1 - a) * t + a * ts is fused
 * by gcc (GNU C, -mfma) on its first product. */
static float or_yarn_theta(int j2, int hd, float theta_base, float beta_fast, float beta_slow, float factor)
{
    const float f = (float)j2 / (float)hd;
    const double td = 1.0 / pow(theta_base, f);
    if (factor <= 1.0f)
        return (float)td;
    const float lo = beta_slow / (float)hd, hi = beta_fast / (float)hd;
    if (f < lo)
        return (float)td;
    const double ts = 1.0 / pow(theta_base * factor, f);
    if (f > hi)
        return (float)ts;
    const float a = (f - lo) / (hi - lo);
    return (float)fma(1.0 - a, td, a * ts);
}

/* op_rope with t_rope_ctx, ops_rope.c:278-353: angle = (float)pos * theta[j],
 * optional mscale on both inputs, x0' = fma(x0, cos, -(x1 * sin)),
 * x1' = fma(x0, sin, x1 * cos) (gcc fuses each expression's first product);
 * BF16 in (bits << 16) and out (round to nearest even).  Trailing elements
 * beyond the last whole vector are left alone. */
void or_op_rope(void *data, int bf16, int n, int pos, int hd, float theta_base, float beta_fast,
                float beta_slow, float factor, float mscale, const float *thetas_cache)
{
    const int half = hd / 2;
    if (hd <= 0 || half == 0)
        return;
    float *th = malloc(sizeof(float) * (size_t)half);
    for (int j = 0; j < half; j++)
        th[j] = thetas_cache ? thetas_cache[j] : or_yarn_theta(2 * j, hd, theta_base, beta_fast, beta_slow, factor);
    const int nv = n / hd;
    for (int v = 0; v < nv; v++)
        for (int j = 0; j < half; j++) {
            const float ang = (float)pos * th[j];
            const float c = cosf(ang), s = sinf(ang);
            const size_t i0 = (size_t)v * hd + j, i1 = i0 + half;
            float x0, x1;
            if (bf16) {
                x0 = or_bf16_to_f32(((uint16_t *)data)[i0]);
                x1 = or_bf16_to_f32(((uint16_t *)data)[i1]);
            } else {
                x0 = ((float *)data)[i0];
                x1 = ((float *)data)[i1];
            }
            if (mscale != 1.0f) {
                x0 = x0 * mscale;
                x1 = x1 * mscale;
            }
            const float y0 = fmaf(x0, c, -(x1 * s)), y1 = fmaf(x0, s, x1 * c);
            if (bf16) {
                ((uint16_t *)data)[i0] = or_f32_to_bf16(y0);
                ((uint16_t *)data)[i1] = or_f32_to_bf16(y1);
            } else {
                ((float *)data)[i0] = y0;
                ((float *)data)[i1] = y1;
            }
        }
    free(th);
}

/* fast_expf_avx2, ops_math_fast.h:105-126: clamp to [-87, 87], fused
 * 12102203 * x + 1065353216, convert with round-to-nearest-even. */
static float fast_expf_vec(float x)
{
    x = x > -87.0f ? x : -87.0f;
    x = x < 87.0f ? x : 87.0f;
    float f = fmaf(x, 12102203.0f, 1065353216.0f);
    int32_t i = (int32_t)lrintf(f);
    float r;
    memcpy(&r, &i, sizeof r);
    return r;
}

/* op_silu_mul_fused_f32, ops_activation.c:48-105: in blocks of 8,
 * sig = 1 / (1 + fast_expf_avx2(0 - g)); out = (g * sig) * u; the scalar
 * remainder uses the truncating fast_expf. */
void or_silu_mul(float *dst, const float *gate, const float *up, int n)
{
    int i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) {
            float g = gate[i + l];
            float sig = 1.0f / (1.0f + fast_expf_vec(0.0f - g));
            dst[i + l] = (g * sig) * up[i + l];
        }
    for (; i < n; i++) {
        float g = gate[i];
        float sig = 1.0f / (1.0f + or_fast_expf(-g));
        dst[i] = g * sig * up[i];
    }
}

/* op_silu_mul_fused_bf16, ops_activation.c:143-230: bf16 in (bits << 16),
 * the f32 arithmetic of the f32 kernel (vector exp for blocks of 8, scalar
 * exp for the remainder), the result truncated to its high 16 bits. */
void or_silu_mul_bf16(uint16_t *dst, const uint16_t *gate, const uint16_t *up, int n)
{
    int i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) {
            float g = or_bf16_to_f32(gate[i + l]), u = or_bf16_to_f32(up[i + l]);
            float sig = 1.0f / (1.0f + fast_expf_vec(0.0f - g));
            float r = (g * sig) * u;
            uint32_t b;
            memcpy(&b, &r, 4);
            dst[i + l] = (uint16_t)(b >> 16);
        }
    for (; i < n; i++) {
        float g = or_bf16_to_f32(gate[i]), u = or_bf16_to_f32(up[i]);
        float sig = 1.0f / (1.0f + or_fast_expf(-g));
        float r = g * sig * u;
        uint32_t b;
        memcpy(&b, &r, 4);
        dst[i] = (uint16_t)(b >> 16);
    }
}

/* sample_temperature, sampler_temp.c:17-114, with the uniform draw r given
 * (the reference draws it from sampler_random_float): max from -1e9 (strict
 * >), p_i = expf((x_i - max) / temp) summed in index order, p_i /= sum, the
 * first index whose running sum exceeds r -- n when none does, as the
 * reference. */
int or_sample_temperature(const float *x, int n, float temp, float r)
{
    float m = -1e9f;
    for (int i = 0; i < n; i++)
        if (x[i] > m)
            m = x[i];
    float *p = (float *)malloc((size_t)n * sizeof(float));
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        p[i] = expf((x[i] - m) / temp);
        sum += p[i];
    }
    for (int i = 0; i < n; i++)
        p[i] /= sum;
    float cum = 0.0f;
    int idx = 0;
    while (idx < n) {
        cum += p[idx];
        if (r < cum)
            break;
        idx++;
    }
    free(p);
    return idx;
}

typedef struct {
    float prob;
    int idx;
} or_prob_idx;

/* probability descending; equal probabilities by ascending index (the
 * reference's qsort comparator returns 0 for them: unspecified order) */
static int or_cmp_prob(const void *a, const void *b)
{
    const or_prob_idx *pa = (const or_prob_idx *)a, *pb = (const or_prob_idx *)b;
    if (pa->prob > pb->prob)
        return -1;
    if (pa->prob < pb->prob)
        return 1;
    return (pa->idx > pb->idx) - (pa->idx < pb->idx);
}

/* sample_top_p, sampler_topp.c:17-158, with u = rand() / RAND_MAX given: max
 * from x[0], p_i = expf((x_i - max) / temp) / sum, sorted as above, cut after
 * the first running sum above top_p (that entry included), r = u * that sum,
 * the first entry whose running sum exceeds r, else the last of the cut. */
int or_sample_top_p(const float *x, int n, float temp, float top_p, float u)
{
    float m = x[0];
    for (int i = 1; i < n; i++)
        if (x[i] > m)
            m = x[i];
    or_prob_idx *pi = (or_prob_idx *)malloc((size_t)n * sizeof(or_prob_idx));
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        pi[i].prob = expf((x[i] - m) / temp);
        pi[i].idx = i;
        sum += pi[i].prob;
    }
    for (int i = 0; i < n; i++)
        pi[i].prob /= sum;
    qsort(pi, (size_t)n, sizeof(or_prob_idx), or_cmp_prob);
    float cum = 0.0f;
    int i = 0;
    while (i < n) {
        cum += pi[i].prob;
        if (cum > top_p) {
            i++;
            break;
        }
        i++;
    }
    const float r = u * cum;
    float running = 0.0f;
    int res = pi[i - 1].idx;
    for (int j = 0; j < i; j++) {
        running += pi[j].prob;
        if (running > r) {
            res = pi[j].idx;
            break;
        }
    }
    free(pi);
    return res;
}

/* argmax_loop_bf16, sampler.c:122-140: best starts at -1e9 (index 0), the
 * first strictly larger value wins. */
int or_argmax_bf16(const uint16_t *x, int n)
{
    int best = 0;
    float bv = -1e9f;
    for (int i = 0; i < n; i++) {
        float v = or_bf16_to_f32(x[i]);
        if (v > bv) {
            bv = v;
            best = i;
        }
    }
    return best;
}

/* argmax_simd_f32, sampler.c:42-117: 8 lanes keep the first strict maximum
 * of i = l (mod 8); lanes are reduced in order with strict >, then the
 * scalar tail with strict >. */
int or_argmax(const float *x, int n)
{
    if (n < 8) {
        int b = 0;
        for (int i = 1; i < n; i++)
            if (x[i] > x[b])
                b = i;
        return b;
    }
    float mv[8];
    int mi[8];
    for (int l = 0; l < 8; l++) {
        mv[l] = x[l];
        mi[l] = l;
    }
    int i = 8;
    for (; i + 7 < n; i += 8)
        for (int l = 0; l < 8; l++)
            if (x[i + l] > mv[l]) {
                mv[l] = x[i + l];
                mi[l] = i + l;
            }
    float bv = mv[0];
    int bi = mi[0];
    for (int l = 1; l < 8; l++)
        if (mv[l] > bv) {
            bv = mv[l];
            bi = mi[l];
        }
    for (; i < n; i++)
        if (x[i] > bv) {
            bv = x[i];
            bi = i;
        }
    return bi;
}

static void gemv_kind(float *y, int wkind, const void *w, const float *s, const float *x, int n, int k, int th)
{
    if (wkind == 0)
        or_gemv_q8(y, (const int8_t *)w, s, x, n, k, 1, th);
    else
        or_gemv_fp8(y, (const uint8_t *)w, s, x, n, k, 1, th);
}

int or_decoder_init(or_decoder *d, const or_decoder_cfg *c, const or_model_w *w, const float *hpT)
{
    memset(d, 0, sizeof *d);
    d->c = *c;
    d->w = *w;
    int max_pages = (c->max_seq + OR_PAGE_TOKENS - 1) / OR_PAGE_TOKENS;
    if (or_paged_init(&d->kv, c->n_layers, c->n_kv, c->hd, max_pages, c->kv_kind))
        return -1;
    d->ix = calloc((size_t)c->n_layers, sizeof(or_lsh_index));
    for (int l = 0; l < c->n_layers; l++)
        if (or_lsh_index_create(&d->ix[l], max_pages))
            return -1;
    d->hpT = malloc(sizeof(float) * (size_t)c->hd * 16);
    memcpy(d->hpT, hpT, sizeof(float) * (size_t)c->hd * 16);
    size_t half = (size_t)c->hd / 2;
    d->cos_t = malloc(sizeof(float) * (size_t)c->max_seq * half);
    d->sin_t = malloc(sizeof(float) * (size_t)c->max_seq * half);
    or_rope_table(d->cos_t, d->sin_t, c->hd, c->max_seq, c->theta);
    int qd = c->n_heads * c->hd, kd = c->n_kv * c->hd;
    d->x = calloc((size_t)c->dim, sizeof(float));
    d->xb = calloc((size_t)(c->dim > qd ? c->dim : qd), sizeof(float));
    d->q = calloc((size_t)qd, sizeof(float));
    d->k = calloc((size_t)kd, sizeof(float));
    d->v = calloc((size_t)kd, sizeof(float));
    d->att = calloc((size_t)qd, sizeof(float));
    d->hb = calloc((size_t)c->hidden, sizeof(float));
    d->hb2 = calloc((size_t)c->hidden, sizeof(float));
    return 0;
}

void or_decoder_free(or_decoder *d)
{
    or_paged_free(&d->kv);
    for (int l = 0; l < d->c.n_layers && d->ix; l++)
        or_lsh_index_destroy(&d->ix[l]);
    free(d->ix);
    free(d->hpT);
    free(d->cos_t);
    free(d->sin_t);
    free(d->x);
    free(d->xb);
    free(d->q);
    free(d->k);
    free(d->v);
    free(d->att);
    free(d->hb);
    free(d->hb2);
    memset(d, 0, sizeof *d);
}

void or_decoder_force_kv(or_decoder *d, const float *k, const float *v)
{
    d->kv_force_k = k;
    d->kv_force_v = v;
}

void or_decoder_log_selection(or_decoder *d, int *sel, int *nsel)
{
    d->sel_log = sel;
    d->nsel_log = nsel;
}

int or_decoder_route(or_decoder *d, int layer, const float *q, int *sel_logical)
{
    const or_decoder_cfg *c = &d->c;
    int *sel = malloc(sizeof(int) * (size_t)(d->kv.max_logical + 2));
    int nc = 0;
    int ns = or_route_pages(sel, &nc, NULL, &d->kv, layer, q, c->n_heads, d->hpT, &d->ix[layer], c->cand_cap,
                            c->sparse_k);
    for (int i = 0; i < ns; i++)
        sel_logical[i] = d->kv.start_pos[sel[i]] / OR_PAGE_TOKENS;
    free(sel);
    return ns;
}

/* paged_kv_append plus the page index: a page that fills is hashed (its
 * centroid under the projection) and inserted as logical page id. */
int or_decoder_kv_append(or_decoder *d, int layer, const float *k, const float *v, int pos)
{
    int phys = or_paged_append(&d->kv, layer, k, v, pos);
    if (phys < 0)
        return -1;
    if (pos % OR_PAGE_TOKENS == OR_PAGE_TOKENS - 1) {
        uint16_t h = or_lsh_hash(d->hpT, d->c.hd, d->kv.centroid + (size_t)phys * d->c.hd);
        or_lsh_insert_block(&d->ix[layer], h, pos - OR_PAGE_TOKENS + 1, OR_PAGE_TOKENS);
    }
    return 0;
}

int or_decoder_kv_append_n(or_decoder *d, int layer, const float *k, const float *v, int pos0, int n)
{
    const size_t kd = (size_t)d->c.n_kv * d->c.hd;
    for (int t = 0; t < n; t++)
        if (or_decoder_kv_append(d, layer, k + t * kd, v + t * kd, pos0 + t))
            return -1;
    return 0;
}

/* transformer_forward, inference.c:60-696, on the paged path: embedding
 * (row-scaled codes, dequantized), per layer RMSNorm -> q/k/v GEMV -> RoPE ->
 * paged append -> attention (dense when n_pages <= sparse_k, else the LSH
 * route + sparse attention) -> o GEMV -> residual -> RMSNorm -> gate/up GEMV
 * -> SiLU*up -> down GEMV -> residual; final RMSNorm -> lm_head GEMV.  The
 * zero-initialised adapter and bias stages are numerically no-ops. */
int or_decoder_step(or_decoder *d, int token, int pos, float *logits, int th)
{
    const or_decoder_cfg *c = &d->c;
    const int dim = c->dim, hd = c->hd, qd = c->n_heads * hd, kd = c->n_kv * hd;
    const float scale = 1.0f / sqrtf((float)hd);
    if (c->wkind == 0) {
        const int8_t *e = (const int8_t *)d->w.emb + (size_t)token * dim;
        for (int i = 0; i < dim; i++)
            d->x[i] = (float)e[i] * d->w.emb_s[token];
    } else {
        float lut[256];
        or_fp8_lut(lut);
        const uint8_t *e = (const uint8_t *)d->w.emb + (size_t)token * dim;
        for (int i = 0; i < dim; i++)
            d->x[i] = lut[e[i]] * d->w.emb_s[token];
    }
    int *sel = malloc(sizeof(int) * (size_t)(d->kv.max_logical + 2));
    for (int l = 0; l < c->n_layers; l++) {
        const or_layer_w *L = &d->w.layers[l];
        or_rmsnorm(d->xb, d->x, L->attn_norm, dim, c->eps);
        gemv_kind(d->q, c->wkind, L->wq, L->sq, d->xb, qd, dim, th);
        gemv_kind(d->k, c->wkind, L->wk, L->sk, d->xb, kd, dim, th);
        gemv_kind(d->v, c->wkind, L->wv, L->sv, d->xb, kd, dim, th);
        or_rope_apply(d->q, c->n_heads, hd, pos, c->max_seq, d->cos_t, d->sin_t);
        or_rope_apply(d->k, c->n_kv, hd, pos, c->max_seq, d->cos_t, d->sin_t);
        const float *kr = d->kv_force_k ? d->kv_force_k + (size_t)l * kd : d->k;
        const float *vr = d->kv_force_v ? d->kv_force_v + (size_t)l * kd : d->v;
        if (or_decoder_kv_append(d, l, kr, vr, pos)) {
            free(sel);
            return -1;
        }
        int nb = d->kv.logical_len[l];
        if (nb <= c->sparse_k) {
            or_paged_attention_dense(d->att, d->q, &d->kv, l, c->n_heads, scale, th);
            if (d->sel_log) {
                for (int i = 0; i < nb; i++)
                    d->sel_log[(size_t)l * c->sparse_k + i] = i;
                d->nsel_log[l] = nb;
            }
        } else {
            int nc = 0;
            int ns = or_route_pages(sel, &nc, NULL, &d->kv, l, d->q, c->n_heads, d->hpT, &d->ix[l], c->cand_cap,
                                    c->sparse_k);
            or_paged_attention_pages(d->att, d->q, &d->kv, sel, ns, c->n_heads, scale, th);
            if (d->sel_log) {
                for (int i = 0; i < ns; i++)
                    d->sel_log[(size_t)l * c->sparse_k + i] = d->kv.start_pos[sel[i]] / OR_PAGE_TOKENS;
                d->nsel_log[l] = ns;
            }
        }
        gemv_kind(d->xb, c->wkind, L->wo, L->so, d->att, dim, qd, th);
        for (int i = 0; i < dim; i++)
            d->x[i] = d->x[i] + d->xb[i];
        or_rmsnorm(d->xb, d->x, L->ffn_norm, dim, c->eps);
        gemv_kind(d->hb, c->wkind, L->w1, L->s1, d->xb, c->hidden, dim, th);
        gemv_kind(d->hb2, c->wkind, L->w3, L->s3, d->xb, c->hidden, dim, th);
        or_silu_mul(d->hb, d->hb, d->hb2, c->hidden);
        gemv_kind(d->xb, c->wkind, L->w2, L->s2, d->hb, dim, c->hidden, th);
        for (int i = 0; i < dim; i++)
            d->x[i] = d->x[i] + d->xb[i];
    }
    free(sel);
    d->kv_force_k = d->kv_force_v = NULL;
    or_rmsnorm(d->x, d->x, d->w.final_norm, dim, c->eps);
    gemv_kind(logits, c->wkind, d->w.out, d->w.out_s, d->x, c->vocab, dim, th);
    return or_argmax(logits, c->vocab);
}

/* ======================================================================== */
/* LSH diagnostics                                                          */
/* ======================================================================== */

/* bf_compute_topk + lsh_validate_recall, ops_lsh.c:513-640: above 4096 keys
 * every (n / 4096)-th key is scored; score = fused chain over d of
 * q[d] * bf16(key[d]); the top k by repeated strict-> argmax from -1e30
 * (index 0 if nothing is larger), chosen scores set to -1e30; recall =
 * hits / actual_k, hits = entries of lsh[0 .. min(lsh_k, actual_k)) among
 * the top k (actual_k clamped to n_keys, then lsh_k to it, then it to 64). */
float or_lsh_validate_recall(const float *q, const uint16_t *keys, int n_keys, int dim,
                             const int *lsh, int lsh_k, int actual_k)
{
    if (actual_k > n_keys)
        actual_k = n_keys;
    if (lsh_k > actual_k)
        lsh_k = actual_k;
    if (actual_k > 64)
        actual_k = 64;
    int stride = 1, nn = n_keys;
    if (n_keys > 4096) {
        stride = n_keys / 4096;
        nn = 4096;
    }
    float *sc = malloc(sizeof(float) * (size_t)(nn > 0 ? nn : 1));
    int top[64];
    for (int i = 0; i < nn; i++) {
        float dot = 0.0f;
        for (int d = 0; d < dim; d++)
            dot = fmaf(q[d], or_bf16_to_f32(keys[(size_t)i * stride * dim + d]), dot);
        sc[i] = dot;
    }
    int nk = 0;
    for (int j = 0; j < actual_k && j < nn; j++) {
        float mv = -1e30f;
        int mi = 0;
        for (int i = 0; i < nn; i++)
            if (sc[i] > mv) {
                mv = sc[i];
                mi = i;
            }
        top[j] = mi * stride;
        sc[mi] = -1e30f;
        nk++;
    }
    int hits = 0;
    for (int i = 0; i < lsh_k; i++)
        for (int j = 0; j < actual_k && j < nk; j++)
            if (lsh[i] == top[j]) {
                hits++;
                break;
            }
    free(sc);
    return (float)hits / (float)actual_k;
}

/* adaptive_k_cutoff, ops_lsh.c:645-668 */
int or_adaptive_k_cutoff(const float *scores, int n, float threshold)
{
    float cum = 0.0f;
    int k = 0;
    while (k < n) {
        cum += scores[k];
        k++;
        if (cum >= threshold)
            break;
    }
    return k < 1 ? 1 : k;
}

