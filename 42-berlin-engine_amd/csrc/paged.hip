// paged.hip -- paged KV cache in HBM: page pool, quantizing append, page
// centroids and their LSH hashes.
//
// block_manager_init / block_alloc / block_free   src/memory/paged.c:29-187
// paged_kv_append                                 src/memory/paged.c:195-272
// paged_kv_reset                                  src/memory/paged.c:312-336
// calc_block_centroid_int8                        src/memory/paged.c:350-393
// quant_f32_to_int8                               src/compute/ops_quant.c:229-270
// float_to_bf16                                   src/tensor/tensor.c:67-76
// lsh_hash                                        src/compute/ops_lsh.c:138-242
//
// Layout in HBM (one allocation per array, pages indexed by physical id):
//   k, v        [cap][n_kv][16][hd]   int8 codes or bf16
//   k_scale...  [cap][n_kv][16]       fp32 (INT8 pages)
//   centroid    [cap][hd]             fp32, head 0 of the page
//   ntok        [cap]                 tokens written in the page
//   page_table  [n_layers][max_logical] -> physical id
//   page_hash   [n_layers][max_logical]   16-bit hash of logical page j's
//               centroid; page j is the j-th page to fill, so the index id of
//               lsh_insert_block (ops_lsh.c:256-272) is the logical page.
// The page allocator (free stack, page table, logical lengths) is host
// bookkeeping exactly as in the reference; the device copies of the page
// table and per-layer counts are updated with each append.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "be42_common.h"
#include "paged_dev.h"
#include "paged_step.h"

namespace be42 {


// Bookkeeping of one append of up to kArgTok tokens, passed by value as a
// kernel argument so that a decode step needs no host-to-device copy.
constexpr int kArgPages = kArgTok / 16 + 2;
struct AppendArgs {
    int pos0, n_tok, layer_base;
    int tok_phys[kArgTok];
    int n_new, new_first;              // page-table entries to publish
    int new_phys[kArgPages];
    int n_logical;                     // value of n_logical[layer] after the append
    int n_seal, n_indexed;             // pages to seal, n_indexed[layer] after
    int seal_phys[kArgPages], seal_logical[kArgPages];
    int layer;
};

struct PoolImpl {
    be42_kv_pool pub;
    std::vector<int> page_table;   // host shadow [n_layers * max_logical]
    std::vector<int> free_stack;
    int free_top = -1;
    std::vector<int> logical_len;  // [n_layers]
    std::vector<int> registered;   // [cap]
    std::vector<int> n_indexed;    // [n_layers]
    // page lists of a bulk append (device copy, and the host array it is
    // copied from, which stays untouched until the next bulk append has
    // waited for the stream)
    int *d_lists = nullptr;
    std::vector<int> h_lists;
};

static PoolImpl *impl(be42_kv_pool *p) { return reinterpret_cast<PoolImpl *>(p); }

// One wave per (token, kv head) of a run of consecutive positions of one
// layer.
template <bool BF16>
__global__ __launch_bounds__(64) void k_kv_append(void *__restrict__ kdst, void *__restrict__ vdst,
                                                  float *__restrict__ kscale, float *__restrict__ vscale,
                                                  int *__restrict__ ntok, int *__restrict__ page_table,
                                                  int *__restrict__ n_logical, const AppendArgs a,
                                                  const float *__restrict__ k, const float *__restrict__ v,
                                                  int n_kv, int hd)
{
    const int tok = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const int pos = a.pos0 + tok, off = pos % kPage;
    const int phys = a.tok_phys[tok];
    if (tok == 0 && h == 0) {
        if (lane < a.n_new)
            page_table[a.layer_base + a.new_first + lane] = a.new_phys[lane];
        if (lane == 0)
            n_logical[a.layer] = a.n_logical;
    }
    const size_t slot = ((size_t)phys * n_kv + h) * kPage + off;
    store_kv_row<BF16>(kdst, vdst, kscale, vscale, slot, k + (size_t)tok * n_kv * hd + (size_t)h * hd,
                       v + (size_t)tok * n_kv * hd + (size_t)h * hd, hd, lane);
    // the page's last token in this append publishes the count (blocks of
    // one page run concurrently)
    if (h == 0 && lane == 0 && (off == kPage - 1 || tok == a.n_tok - 1))
        ntok[phys] = off + 1;
}

// One token for each of n layer slots (a decode step of a batch): the same
// store, with per-token slot, position and page bookkeeping.

template <bool BF16>
__device__ __forceinline__ void append_step_body(void *__restrict__ kdst, void *__restrict__ vdst,
                                                 float *__restrict__ kscale, float *__restrict__ vscale,
                                                 int *__restrict__ ntok, int *__restrict__ page_table,
                                                 int *__restrict__ n_logical, const AppendStepArgs &a,
                                                 const float *__restrict__ k, const float *__restrict__ v, int n_kv,
                                                 int hd)
{
    const int tok = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    if (tok >= a.n)
        return;
    const int pos = a.pos[tok], off = pos % kPage, blk = pos / kPage, phys = a.phys[tok];
    if (h == 0 && lane == 0) {
        if (a.publish[tok]) {
            page_table[(size_t)a.slot[tok] * a.max_logical + blk] = phys;
            n_logical[a.slot[tok]] = blk + 1;
        }
        ntok[phys] = off + 1;
    }
    const size_t slot = ((size_t)phys * n_kv + h) * kPage + off;
    store_kv_row<BF16>(kdst, vdst, kscale, vscale, slot, k + (size_t)tok * n_kv * hd + (size_t)h * hd,
                       v + (size_t)tok * n_kv * hd + (size_t)h * hd, hd, lane);
}

template <bool BF16>
__global__ __launch_bounds__(64) void k_kv_append_step(void *__restrict__ kdst, void *__restrict__ vdst,
                                                       float *__restrict__ kscale, float *__restrict__ vscale,
                                                       int *__restrict__ ntok, int *__restrict__ page_table,
                                                       int *__restrict__ n_logical, const AppendStepArgs a,
                                                       const float *__restrict__ k, const float *__restrict__ v,
                                                       int n_kv, int hd)
{
    append_step_body<BF16>(kdst, vdst, kscale, vscale, ntok, page_table, n_logical, a, k, v, n_kv, hd);
}

// A bulk append: one wave per (token, kv head) of n_tok consecutive
// positions, the physical page of each touched logical page read from a list
// (page_phys[blk - first_blk]); block (0, 0) publishes the new page-table
// entries.
template <bool BF16>
__global__ __launch_bounds__(64) void k_kv_append_bulk(void *__restrict__ kdst, void *__restrict__ vdst,
                                                       float *__restrict__ kscale, float *__restrict__ vscale,
                                                       int *__restrict__ ntok, int *__restrict__ page_table,
                                                       int *__restrict__ n_logical, const int *__restrict__ lists,
                                                       int pos0, int n_tok, int first_blk, int n_pages, int n_new,
                                                       int new_first, int layer_base, int layer, int n_log,
                                                       const float *__restrict__ k, const float *__restrict__ v,
                                                       int n_kv, int hd)
{
    const int tok = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const int pos = pos0 + tok, off = pos % kPage;
    const int phys = lists[pos / kPage - first_blk];
    if (tok == 0 && h == 0) {
        for (int i = lane; i < n_new; i += kWave)
            page_table[layer_base + new_first + i] = lists[n_pages + i];
        if (lane == 0)
            n_logical[layer] = n_log;
    }
    const size_t slot = ((size_t)phys * n_kv + h) * kPage + off;
    store_kv_row<BF16>(kdst, vdst, kscale, vscale, slot, k + (size_t)tok * n_kv * hd + (size_t)h * hd,
                       v + (size_t)tok * n_kv * hd + (size_t)h * hd, hd, lane);
    if (h == 0 && lane == 0 && (off == kPage - 1 || tok == n_tok - 1))
        ntok[phys] = off + 1;
}

// One block per page a bulk append filled: seal list (physical, logical) at
// lists[0 .. n_seal), lists[n_seal .. 2 n_seal).
template <bool BF16>
__global__ __launch_bounds__(256) void k_kv_seal_bulk(const void *__restrict__ kpool, const float *__restrict__ kscale,
                                                      float *__restrict__ centroid, uint16_t *__restrict__ page_hash,
                                                      int *__restrict__ n_indexed, const int *__restrict__ lists,
                                                      int n_seal, int layer_base, int layer, int n_idx,
                                                      const float *__restrict__ hpT, int n_kv, int hd)
{
    __shared__ float c[256];
    if (blockIdx.x == 0 && threadIdx.x == 0)
        n_indexed[layer] = n_idx;
    seal_page<BF16>(kpool, kscale, centroid, page_hash + layer_base + lists[n_seal + blockIdx.x],
                    lists[blockIdx.x], hpT, n_kv, hd, c);
}

template <bool BF16>
__global__ __launch_bounds__(256) void k_kv_seal(const void *__restrict__ kpool, const float *__restrict__ kscale,
                                                 float *__restrict__ centroid, uint16_t *__restrict__ page_hash,
                                                 int *__restrict__ n_indexed, const AppendArgs a,
                                                 const float *__restrict__ hpT, int n_kv, int hd)
{
    __shared__ float c[256];
    if (blockIdx.x == 0 && threadIdx.x == 0)
        n_indexed[a.layer] = a.n_indexed;
    seal_page<BF16>(kpool, kscale, centroid, page_hash + a.layer_base + a.seal_logical[blockIdx.x],
                    a.seal_phys[blockIdx.x], hpT, n_kv, hd, c);
}

template <bool BF16>
__device__ __forceinline__ void seal_step_body(const void *__restrict__ kpool, const float *__restrict__ kscale,
                                               float *__restrict__ centroid, uint16_t *__restrict__ page_hash,
                                               int *__restrict__ n_indexed, const AppendStepArgs &a,
                                               const float *__restrict__ hpT, int n_kv, int hd)
{
    __shared__ float c[256];
    const int i = blockIdx.x;
    if (i >= a.n_seal)
        return;
    const int slot = a.seal_slot[i];
    if (threadIdx.x == 0)
        n_indexed[slot] = a.seal_nidx[i];
    seal_page<BF16>(kpool, kscale, centroid, page_hash + (size_t)slot * a.max_logical + a.seal_logical[i],
                    a.seal_phys[i], hpT, n_kv, hd, c);
}

template <bool BF16>
__global__ __launch_bounds__(256) void k_kv_seal_step(const void *__restrict__ kpool, const float *__restrict__ kscale,
                                                      float *__restrict__ centroid, uint16_t *__restrict__ page_hash,
                                                      int *__restrict__ n_indexed, const AppendStepArgs a,
                                                      const float *__restrict__ hpT, int n_kv, int hd)
{
    seal_step_body<BF16>(kpool, kscale, centroid, page_hash, n_indexed, a, hpT, n_kv, hd);
}

// RoPE + append + seal of one decode token of one layer slot, for KV head h
// (block (token, h), 256 threads): the q heads of h's group and k head h are
// rotated in place (the RoPE of inference.c / ops_rope.c:192 as k_rope does
// it), the rotated k row and the v row are stored into the page, and block
// h == 0 seals the page when this token fills it.
template <bool BF16>
__global__ __launch_bounds__(256) void k_rope_append_dev(const be42_kv_pool P, const AppendStepArgs *__restrict__ ap,
                                                         float *__restrict__ q, float *__restrict__ k,
                                                         const float *__restrict__ v,
                                                         const float *__restrict__ cos_t,
                                                         const float *__restrict__ sin_t,
                                                         const int *__restrict__ pos_p, int rope_len, int H)
{
    __shared__ float ks[256];
    __shared__ float c[256];
    rope_append_body<BF16>(P, ap, q, k, v, cos_t, sin_t, pos_p, rope_len, H, blockIdx.x, blockIdx.y, ks, c);
}

}  // namespace be42

using namespace be42;

extern "C" int be42_kv_create(be42_kv_pool **out, int kind, int n_layers, int n_kv, int head_dim,
                              int max_logical, const float *hpT_host)
{
    BE42_CHECK(out, "be42_kv_create: null out");
    *out = nullptr;
    BE42_CHECK(kind == BE42_KV_INT8 || kind == BE42_KV_BF16, "be42_kv_create: bad kind %d", kind);
    BE42_CHECK(n_layers > 0 && n_kv > 0 && max_logical > 0 && head_dim > 0 && head_dim <= 256 &&
                   head_dim % 8 == 0,
               "be42_kv_create: bad shape (layers %d, kv heads %d, head_dim %d, pages %d)", n_layers, n_kv,
               head_dim, max_logical);
    PoolImpl *p = new PoolImpl();
    be42_kv_pool &P = p->pub;
    memset(&P, 0, sizeof P);
    P.kind = kind;
    P.n_layers = n_layers;
    P.n_kv = n_kv;
    P.head_dim = head_dim;
    P.max_logical = max_logical;
    P.capacity = n_layers * max_logical;
    const size_t cap = (size_t)P.capacity;
    const size_t elem = kind == BE42_KV_INT8 ? 1 : 2;
    const size_t kvbytes = cap * n_kv * kPage * head_dim * elem;
    hipError_t e = hipSuccess;
    auto alloc = [&](void **ptr, size_t bytes) {
        if (e == hipSuccess)
            e = hipMalloc(ptr, bytes ? bytes : 1);
    };
    alloc(&P.k, kvbytes);
    alloc(&P.v, kvbytes);
    if (kind == BE42_KV_INT8) {
        alloc((void **)&P.k_scale, cap * n_kv * kPage * sizeof(float));
        alloc((void **)&P.v_scale, cap * n_kv * kPage * sizeof(float));
    }
    alloc((void **)&P.centroid, cap * head_dim * sizeof(float));
    alloc((void **)&P.ntok, cap * sizeof(int));
    alloc((void **)&P.page_table, cap * sizeof(int));
    alloc((void **)&P.n_logical, n_layers * sizeof(int));
    alloc((void **)&P.page_hash, cap * sizeof(uint16_t));
    alloc((void **)&P.n_indexed, n_layers * sizeof(int));
    alloc((void **)&P.hpT, head_dim * 16 * sizeof(float));
    if (e == hipSuccess) e = hipMemset(P.k, 0, kvbytes);
    if (e == hipSuccess) e = hipMemset(P.v, 0, kvbytes);
    if (e == hipSuccess) e = hipMemset(P.ntok, 0, cap * sizeof(int));
    if (e == hipSuccess) e = hipMemset(P.centroid, 0, cap * head_dim * sizeof(float));
    if (e == hipSuccess) e = hipMemset(P.page_table, 0xFF, cap * sizeof(int));
    if (e == hipSuccess) e = hipMemset(P.n_logical, 0, n_layers * sizeof(int));
    if (e == hipSuccess) e = hipMemset(P.n_indexed, 0, n_layers * sizeof(int));
    if (e == hipSuccess) e = hipMemset(P.page_hash, 0, cap * sizeof(uint16_t));
    if (e == hipSuccess && hpT_host)
        e = hipMemcpy((void *)P.hpT, hpT_host, head_dim * 16 * sizeof(float), hipMemcpyHostToDevice);
    else if (e == hipSuccess)
        e = hipMemset((void *)P.hpT, 0, head_dim * 16 * sizeof(float));
    if (e != hipSuccess) {
        be42_kv_destroy(&P);
        return hip_fail(e, "be42_kv_create", __FILE__, __LINE__);
    }
    p->page_table.assign(cap, -1);
    p->free_stack.resize(cap);
    for (size_t i = 0; i < cap; i++)
        p->free_stack[i] = (int)i;
    p->free_top = (int)cap - 1;
    p->logical_len.assign(n_layers, 0);
    p->registered.assign(cap, 0);
    p->n_indexed.assign(n_layers, 0);
    *out = &P;
    return BE42_OK;
}

extern "C" void be42_kv_destroy(be42_kv_pool *pool)
{
    if (!pool)
        return;
    void *ptrs[] = {pool->k, pool->v, pool->k_scale, pool->v_scale, pool->centroid, pool->ntok,
                    pool->page_table, pool->n_logical, pool->page_hash, pool->n_indexed, (void *)pool->hpT,
                    impl(pool)->d_lists};
    if (impl(pool)->d_lists)
        (void)hipDeviceSynchronize();   // a bulk append may still read its lists
    for (void *q : ptrs)
        if (q)
            (void)hipFree(q);
    delete impl(pool);
}

extern "C" int be42_kv_set_projection(be42_kv_pool *pool, const float *hpT_host)
{
    BE42_CHECK(pool && hpT_host, "be42_kv_set_projection: null pointer");
    BE42_HIP(hipMemcpy((void *)pool->hpT, hpT_host, pool->head_dim * 16 * sizeof(float), hipMemcpyHostToDevice));
    return BE42_OK;
}

// Host page allocator, paged.c:159-179 (pop the free stack).
static int pool_alloc(PoolImpl *p)
{
    if (p->free_top < 0)
        return -1;
    const int phys = p->free_stack[p->free_top--];
    p->registered[phys] = 0;
    return phys;
}

// One chunk of <= kArgTok tokens: host bookkeeping of paged.c:195-272, then
// the quantizing store and, for pages that fill, centroid + hash.
static int append_chunk(PoolImpl *p, int layer, const float *k, const float *v, int pos0, int n, hipStream_t s)
{
    be42_kv_pool &P = p->pub;
    AppendArgs a;
    memset(&a, 0, sizeof a);
    a.pos0 = pos0;
    a.n_tok = n;
    a.layer = layer;
    a.layer_base = layer * P.max_logical;
    a.new_first = p->logical_len[layer];
    const int last_blk = (pos0 + n - 1) / kPage;
    for (int blk = pos0 / kPage; blk <= last_blk; blk++) {
        if (blk >= p->logical_len[layer]) {
            // pages are appended in order: a gap would leave unmapped pages
            if (blk != p->logical_len[layer]) {
                set_error("be42_kv_append: position %d skips page %d", blk * kPage, p->logical_len[layer]);
                return BE42_EINVAL;
            }
            const int phys = pool_alloc(p);
            if (phys < 0) {
                set_error("be42_kv_append: page pool exhausted at pos %d", blk * kPage);
                return BE42_ENOMEM;
            }
            p->page_table[a.layer_base + blk] = phys;
            p->logical_len[layer] = blk + 1;
            a.new_phys[a.n_new++] = phys;
        }
    }
    a.n_logical = p->logical_len[layer];
    for (int t = 0; t < n; t++) {
        const int pos = pos0 + t, blk = pos / kPage;
        const int phys = p->page_table[a.layer_base + blk];
        a.tok_phys[t] = phys;
        if (pos % kPage == kPage - 1 && !p->registered[phys]) {
            p->registered[phys] = 1;
            a.seal_phys[a.n_seal] = phys;
            a.seal_logical[a.n_seal] = blk;
            a.n_seal++;
            if (blk + 1 > p->n_indexed[layer])
                p->n_indexed[layer] = blk + 1;
        }
    }
    a.n_indexed = p->n_indexed[layer];
    const dim3 grid(n, P.n_kv);
    if (P.kind == BE42_KV_BF16)
        hipLaunchKernelGGL(k_kv_append<true>, grid, dim3(64), 0, s, P.k, P.v, P.k_scale, P.v_scale, P.ntok,
                           P.page_table, P.n_logical, a, k, v, P.n_kv, P.head_dim);
    else
        hipLaunchKernelGGL(k_kv_append<false>, grid, dim3(64), 0, s, P.k, P.v, P.k_scale, P.v_scale, P.ntok,
                           P.page_table, P.n_logical, a, k, v, P.n_kv, P.head_dim);
    BE42_LAUNCH_CHECK();
    if (a.n_seal) {
        if (P.kind == BE42_KV_BF16)
            hipLaunchKernelGGL(k_kv_seal<true>, dim3(a.n_seal), dim3(256), 0, s, P.k, P.k_scale, P.centroid,
                               P.page_hash, P.n_indexed, a, P.hpT, P.n_kv, P.head_dim);
        else
            hipLaunchKernelGGL(k_kv_seal<false>, dim3(a.n_seal), dim3(256), 0, s, P.k, P.k_scale, P.centroid,
                               P.page_hash, P.n_indexed, a, P.hpT, P.n_kv, P.head_dim);
        BE42_LAUNCH_CHECK();
    }
    return BE42_OK;
}

namespace be42 {

// Host bookkeeping of a run of n consecutive positions of one layer slot
// (paged.c:195-272 for each): pages allocated in logical order, and the page
// lists of the run written to L: the physical page of each logical page the
// run touches [n_pages], the new ones [n_new], then the pages it fills
// (physical [n_seal], logical [n_seal]).  L holds 4 * (n / 16 + 2) ints.
int plan_append_run(be42_kv_pool *pool, int layer, int pos0, int n, int *L, AppendRun *out)
{
    PoolImpl *p = impl(pool);
    be42_kv_pool &P = p->pub;
    AppendRun &r = *out;
    r.layer = layer;
    r.layer_base = layer * P.max_logical;
    r.pos0 = pos0;
    r.n = n;
    r.first_blk = pos0 / kPage;
    const int last_blk = (pos0 + n - 1) / kPage;
    r.n_pages = last_blk - r.first_blk + 1;
    r.new_first = p->logical_len[layer];
    int *fresh = L + r.n_pages;
    r.n_new = 0;
    for (int blk = r.first_blk; blk <= last_blk; blk++) {
        if (blk >= p->logical_len[layer]) {
            // pages are appended in order: a gap would leave unmapped pages
            if (blk != p->logical_len[layer]) {
                set_error("be42_kv_append: position %d skips page %d", blk * kPage, p->logical_len[layer]);
                return BE42_EINVAL;
            }
            const int phys = pool_alloc(p);
            if (phys < 0) {
                set_error("be42_kv_append: page pool exhausted at pos %d", blk * kPage);
                return BE42_ENOMEM;
            }
            p->page_table[r.layer_base + blk] = phys;
            p->logical_len[layer] = blk + 1;
            fresh[r.n_new++] = phys;
        }
        L[blk - r.first_blk] = p->page_table[r.layer_base + blk];
    }
    int *seal = L + r.n_pages + r.n_new;
    int ns = 0;
    for (int blk = r.first_blk; blk <= last_blk; blk++) {
        const int phys = p->page_table[r.layer_base + blk];
        const int end = (blk + 1) * kPage - 1;          // the page's last position
        if (end >= pos0 && end < pos0 + n && !p->registered[phys]) {
            p->registered[phys] = 1;
            seal[ns++] = phys;
            if (blk + 1 > p->n_indexed[layer])
                p->n_indexed[layer] = blk + 1;
        }
    }
    // logical ids of the sealed pages, after the physical ones
    int ls = 0;
    for (int blk = r.first_blk; blk <= last_blk && ls < ns; blk++)
        if (p->page_table[r.layer_base + blk] == seal[ls])
            seal[ns + ls++] = blk;
    r.n_seal = ns;
    r.n_log = p->logical_len[layer];
    r.n_idx = p->n_indexed[layer];
    r.list_len = r.n_pages + r.n_new + 2 * ns;
    return BE42_OK;
}

// The run's store and seal launches, with its lists at d_lists (device).
int launch_append_run(const be42_kv_pool &P, const AppendRun &r, const int *d_lists, const float *k, const float *v,
                      hipStream_t s)
{
    const dim3 grid(r.n, P.n_kv);
    if (P.kind == BE42_KV_BF16)
        hipLaunchKernelGGL(k_kv_append_bulk<true>, grid, dim3(64), 0, s, P.k, P.v, P.k_scale, P.v_scale, P.ntok,
                           P.page_table, P.n_logical, d_lists, r.pos0, r.n, r.first_blk, r.n_pages, r.n_new,
                           r.new_first, r.layer_base, r.layer, r.n_log, k, v, P.n_kv, P.head_dim);
    else
        hipLaunchKernelGGL(k_kv_append_bulk<false>, grid, dim3(64), 0, s, P.k, P.v, P.k_scale, P.v_scale, P.ntok,
                           P.page_table, P.n_logical, d_lists, r.pos0, r.n, r.first_blk, r.n_pages, r.n_new,
                           r.new_first, r.layer_base, r.layer, r.n_log, k, v, P.n_kv, P.head_dim);
    BE42_LAUNCH_CHECK();
    if (r.n_seal) {
        const int *sl = d_lists + r.n_pages + r.n_new;
        if (P.kind == BE42_KV_BF16)
            hipLaunchKernelGGL(k_kv_seal_bulk<true>, dim3(r.n_seal), dim3(256), 0, s, P.k, P.k_scale, P.centroid,
                               P.page_hash, P.n_indexed, sl, r.n_seal, r.layer_base, r.layer, r.n_idx, P.hpT, P.n_kv,
                               P.head_dim);
        else
            hipLaunchKernelGGL(k_kv_seal_bulk<false>, dim3(r.n_seal), dim3(256), 0, s, P.k, P.k_scale, P.centroid,
                               P.page_hash, P.n_indexed, sl, r.n_seal, r.layer_base, r.layer, r.n_idx, P.hpT, P.n_kv,
                               P.head_dim);
        BE42_LAUNCH_CHECK();
    }
    return BE42_OK;
}

}  // namespace be42

// More than kArgTok tokens: the bookkeeping of the whole run, its page lists
// copied to the device, then one append launch and one seal launch.
static int append_bulk(PoolImpl *p, int layer, const float *k, const float *v, int pos0, int n, hipStream_t s)
{
    be42_kv_pool &P = p->pub;
    // the previous bulk append's lists (host and device) may still be in use
    BE42_HIP(hipStreamSynchronize(s));
    if (!p->d_lists) {
        p->h_lists.assign((size_t)4 * P.max_logical + 8, 0);
        BE42_HIP(hipMalloc((void **)&p->d_lists, p->h_lists.size() * sizeof(int)));
    }
    AppendRun r;
    const int rc = plan_append_run(&p->pub, layer, pos0, n, p->h_lists.data(), &r);
    if (rc)
        return rc;
    BE42_HIP(hipMemcpyAsync(p->d_lists, p->h_lists.data(), (size_t)r.list_len * sizeof(int), hipMemcpyHostToDevice,
                            s));
    return launch_append_run(P, r, p->d_lists, k, v, s);
}

extern "C" int be42_kv_append(be42_kv_pool *pool, int layer, const float *k, const float *v, int pos0,
                              int n_tokens, void *stream)
{
    BE42_CHECK(pool && k && v, "be42_kv_append: null pointer");
    PoolImpl *p = impl(pool);
    be42_kv_pool &P = p->pub;
    BE42_CHECK(layer >= 0 && layer < P.n_layers, "be42_kv_append: layer %d out of range", layer);
    BE42_CHECK(pos0 >= 0 && n_tokens >= 0, "be42_kv_append: bad positions");
    if (n_tokens == 0)
        return BE42_OK;
    BE42_CHECK((pos0 + n_tokens - 1) / kPage < P.max_logical, "be42_kv_append: position %d beyond %d pages",
               pos0 + n_tokens - 1, P.max_logical);
    hipStream_t s = as_stream(stream);
    if (n_tokens > kArgTok)
        return append_bulk(p, layer, k, v, pos0, n_tokens, s);
    const size_t row = (size_t)P.n_kv * P.head_dim;
    for (int t = 0; t < n_tokens; t += kArgTok) {
        const int n = n_tokens - t < kArgTok ? n_tokens - t : kArgTok;
        const int rc = append_chunk(p, layer, k + t * row, v + t * row, pos0 + t, n, s);
        if (rc)
            return rc;
    }
    return BE42_OK;
}

extern "C" int be42_kv_reset(be42_kv_pool *pool, int layer, void *stream)
{
    BE42_CHECK(pool, "be42_kv_reset: null pool");
    PoolImpl *p = impl(pool);
    be42_kv_pool &P = p->pub;
    BE42_CHECK(layer >= 0 && layer < P.n_layers, "be42_kv_reset: layer %d out of range", layer);
    const int base = layer * P.max_logical;
    // paged.c:312-336: return pages to the free stack, unmap
    for (int i = 0; i < p->logical_len[layer]; i++) {
        const int phys = p->page_table[base + i];
        if (phys >= 0)
            p->free_stack[++p->free_top] = phys;
        p->page_table[base + i] = -1;
    }
    const int n = p->logical_len[layer];
    p->logical_len[layer] = 0;
    p->n_indexed[layer] = 0;
    hipStream_t s = as_stream(stream);
    if (n > 0)
        BE42_HIP(hipMemsetAsync(P.page_table + base, 0xFF, n * sizeof(int), s));
    BE42_HIP(hipMemsetAsync(P.n_logical + layer, 0, sizeof(int), s));
    BE42_HIP(hipMemsetAsync(P.n_indexed + layer, 0, sizeof(int), s));
    return BE42_OK;
}

extern "C" int be42_kv_layer_pages(const be42_kv_pool *pool, int layer, int *phys_out, int max_out)
{
    BE42_CHECK(pool, "be42_kv_layer_pages: null pool");
    const PoolImpl *p = reinterpret_cast<const PoolImpl *>(pool);
    BE42_CHECK(layer >= 0 && layer < pool->n_layers, "be42_kv_layer_pages: layer out of range");
    const int n = p->logical_len[layer];
    if (phys_out)
        for (int i = 0; i < n && i < max_out; i++)
            phys_out[i] = p->page_table[layer * pool->max_logical + i];
    return n;
}

// block_alloc / block_free (paged.c:159-187) on the pool's own free stack.
extern "C" int be42_kv_page_alloc(be42_kv_pool *pool)
{
    BE42_CHECK(pool, "be42_kv_page_alloc: null pool");
    const int phys = pool_alloc(impl(pool));
    if (phys < 0)
        set_error("be42_kv_page_alloc: page pool exhausted");
    return phys;
}

extern "C" int be42_kv_page_free(be42_kv_pool *pool, int phys)
{
    BE42_CHECK(pool, "be42_kv_page_free: null pool");
    PoolImpl *p = impl(pool);
    if (phys < 0 || phys >= pool->capacity)
        return BE42_OK;    // ignored, as block_free does
    p->free_stack[++p->free_top] = phys;
    return BE42_OK;
}

extern "C" int be42_kv_export(const be42_kv_pool *pool, int *page_table, int *free_stack, int *free_top,
                              int *logical_len)
{
    BE42_CHECK(pool, "be42_kv_export: null pool");
    const PoolImpl *p = reinterpret_cast<const PoolImpl *>(pool);
    if (page_table)
        memcpy(page_table, p->page_table.data(), p->page_table.size() * sizeof(int));
    if (free_stack)
        memcpy(free_stack, p->free_stack.data(), p->free_stack.size() * sizeof(int));
    if (free_top)
        *free_top = p->free_top;
    if (logical_len)
        memcpy(logical_len, p->logical_len.data(), p->logical_len.size() * sizeof(int));
    return BE42_OK;
}

namespace be42 {

// Host bookkeeping of one decode token for each of n distinct layer slots
// (paged.c:195-272 per slot): page allocation, page table, seal list.
int plan_append_step(be42_kv_pool *pool, const int *slots, const int *pos, int n, AppendStepArgs *out,
                     PlanUndo *undo)
{
    BE42_CHECK(n >= 0 && n <= kArgTok, "be42_kv_append_step: %d slots (at most %d)", n, kArgTok);
    PoolImpl *p = impl(pool);
    be42_kv_pool &P = p->pub;
    AppendStepArgs &a = *out;
    memset(&a, 0, sizeof a);
    a.n = n;
    a.max_logical = P.max_logical;
    if (undo && undo->free_top == -2)
        undo->free_top = p->free_top;
    for (int t = 0; t < n; t++) {
        const int s = slots[t], ps = pos[t];
        BE42_CHECK(s >= 0 && s < P.n_layers, "be42_kv_append_step: slot %d out of range", s);
        BE42_CHECK(ps >= 0 && ps / kPage < P.max_logical, "be42_kv_append_step: position %d out of range", ps);
        for (int u = 0; u < t; u++)
            BE42_CHECK(slots[u] != s, "be42_kv_append_step: slot %d given twice", s);
        if (undo) {
            undo->slot.push_back(s);
            undo->len.push_back(p->logical_len[s]);
            undo->nidx.push_back(p->n_indexed[s]);
        }
        const int blk = ps / kPage, base = s * P.max_logical;
        if (blk >= p->logical_len[s]) {
            if (blk != p->logical_len[s]) {
                set_error("be42_kv_append_step: position %d skips page %d", ps, p->logical_len[s]);
                return BE42_EINVAL;
            }
            const int phys = pool_alloc(p);
            if (phys < 0) {
                set_error("be42_kv_append_step: page pool exhausted at pos %d", ps);
                return BE42_ENOMEM;
            }
            p->page_table[base + blk] = phys;
            p->logical_len[s] = blk + 1;
            a.publish[t] = 1;
        }
        const int phys = p->page_table[base + blk];
        a.pos[t] = ps;
        a.phys[t] = phys;
        a.slot[t] = s;
        a.seal_of[t] = -1;
        if (ps % kPage == kPage - 1 && !p->registered[phys]) {
            a.seal_of[t] = a.n_seal;
            p->registered[phys] = 1;
            if (undo)
                undo->sealed.push_back(phys);
            if (blk + 1 > p->n_indexed[s])
                p->n_indexed[s] = blk + 1;
            a.seal_phys[a.n_seal] = phys;
            a.seal_slot[a.n_seal] = s;
            a.seal_logical[a.n_seal] = blk;
            a.seal_nidx[a.n_seal] = p->n_indexed[s];
            a.n_seal++;
        }
    }
    return BE42_OK;
}

void undo_append_plans(be42_kv_pool *pool, const PlanUndo &u)
{
    if (u.free_top == -2)
        return;
    PoolImpl *p = impl(pool);
    const int ml = p->pub.max_logical;
    for (int phys : u.sealed)
        p->registered[phys] = 0;
    // newest entry first: a slot logged twice ends at its oldest values
    for (size_t i = u.slot.size(); i-- > 0;) {
        const int s = u.slot[i];
        for (int blk = u.len[i]; blk < p->logical_len[s]; blk++)
            p->page_table[(size_t)s * ml + blk] = -1;
        p->logical_len[s] = u.len[i];
        p->n_indexed[s] = u.nidx[i];
    }
    // pops only move the top, so the stack's contents above it are intact
    p->free_top = u.free_top;
}

int launch_rope_append_step_dev(const be42_kv_pool &P, const AppendStepArgs *a_dev, int n, float *q, float *k,
                                const float *v, const float *cos_t, const float *sin_t, const int *pos_p,
                                int rope_len, int n_heads, hipStream_t st)
{
    BE42_CHECK(P.head_dim <= 256 && n_heads % P.n_kv == 0, "rope+append: head_dim %d, %d heads over %d kv heads",
               P.head_dim, n_heads, P.n_kv);
    const dim3 grid(n, P.n_kv);
    if (P.kind == BE42_KV_BF16)
        hipLaunchKernelGGL(k_rope_append_dev<true>, grid, dim3(256), 0, st, P, a_dev, q, k, v, cos_t, sin_t, pos_p,
                           rope_len, n_heads);
    else
        hipLaunchKernelGGL(k_rope_append_dev<false>, grid, dim3(256), 0, st, P, a_dev, q, k, v, cos_t, sin_t, pos_p,
                           rope_len, n_heads);
    BE42_LAUNCH_CHECK();
    return BE42_OK;
}

}  // namespace be42

// One decode token for each of n layer slots (paged.c:195-272 per slot).
extern "C" int be42_kv_append_step(be42_kv_pool *pool, const int *slots, const int *pos, int n, const float *k,
                                   const float *v, void *stream)
{
    BE42_CHECK(pool && slots && pos && k && v, "be42_kv_append_step: null pointer");
    if (n == 0)
        return BE42_OK;
    AppendStepArgs a;
    const int rc = plan_append_step(pool, slots, pos, n, &a);
    if (rc)
        return rc;
    const be42_kv_pool &P = *pool;
    hipStream_t st = as_stream(stream);
    const dim3 grid(n, P.n_kv);
    if (P.kind == BE42_KV_BF16)
        hipLaunchKernelGGL(k_kv_append_step<true>, grid, dim3(64), 0, st, P.k, P.v, P.k_scale, P.v_scale, P.ntok,
                           P.page_table, P.n_logical, a, k, v, P.n_kv, P.head_dim);
    else
        hipLaunchKernelGGL(k_kv_append_step<false>, grid, dim3(64), 0, st, P.k, P.v, P.k_scale, P.v_scale, P.ntok,
                           P.page_table, P.n_logical, a, k, v, P.n_kv, P.head_dim);
    BE42_LAUNCH_CHECK();
    if (a.n_seal) {
        if (P.kind == BE42_KV_BF16)
            hipLaunchKernelGGL(k_kv_seal_step<true>, dim3(a.n_seal), dim3(256), 0, st, P.k, P.k_scale, P.centroid,
                               P.page_hash, P.n_indexed, a, P.hpT, P.n_kv, P.head_dim);
        else
            hipLaunchKernelGGL(k_kv_seal_step<false>, dim3(a.n_seal), dim3(256), 0, st, P.k, P.k_scale,
                               P.centroid, P.page_hash, P.n_indexed, a, P.hpT, P.n_kv, P.head_dim);
        BE42_LAUNCH_CHECK();
    }
    return BE42_OK;
}
