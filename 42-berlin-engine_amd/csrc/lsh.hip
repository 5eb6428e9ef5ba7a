// lsh.hip -- LSH-routed page selection on gfx950.
//
// lsh_init (projection)         src/compute/ops_lsh.c:22-85     (host, at init)
// lsh_hash                      src/compute/ops_lsh.c:138-242
// lsh_find_candidates           src/compute/ops_lsh.c:361-418
// q_mean routing glue           src/inference/inference.c:291-302
// score_blocks                  src/memory/paged.c:401-431 (simd_dot_f32_f32,
//                               src/compute/simd_kernels.h:162-191)
// select_top_k_blocks + heap    src/memory/paged.c:439-495, src/compute/ops_heap.h:33-100
//
// One workgroup (4 waves) routes one query:
//  1. q_mean over the heads (sum in head order, then / n_heads) and its hash:
//     16 lanes each run the FMA chain over d, the sign bits are packed with a
//     ballot.
//  2. Candidates.  The reference walks, for probes p = 0..16 (p = 0: the query
//     hash, p > 0: bit p-1 flipped), the bucket's LIFO chain.  A bucket holds
//     exactly the blocks whose hash equals the probed hash, newest first, and
//     the Hamming filter (radius 4) never rejects them, so the candidate list
//     is: for p ascending, the indexed pages with hash == qh ^ flip(p) in
//     descending id order, truncated at `cap`.  The waves scan the page-hash
//     array in descending id order (wave 0 the highest ids) and file each hit
//     under its probe with a ballot; per-probe lists are concatenated.
//  3. Middle entries = candidates other than the first and last page; each is
//     scored q[head 0] . centroid with the reference's 8-lane reduction tree.
//  4. Selection = [first page, last page] + the exact min-heap of the
//     reference (capacity min(k-2, #middle, 62), strict replacement), run in
//     wave 0 with heap slot i held by lane i; the heap array order is the
//     output order, as in the reference.
// With n_pages <= k every page is selected in logical order (the dense path
// of inference.c:447-494).
#include <cmath>

#include "be42_common.h"
#include "paged_step.h"
#include "route.h"

namespace be42 {

// With lim, query b sees only the first lim[b] positions of its slot (the
// pages and LSH index it saw when position lim[b] - 1 was the newest), as in
// k_lsh_attn.
template <bool STAGE>
__global__ __launch_bounds__(256) void k_route(const be42_kv_pool P, const float *__restrict__ q,
                                               const int *__restrict__ slots, const int *__restrict__ lim, int H,
                                               int k_sel, int cap,
                                               int *__restrict__ sel, int *__restrict__ nsel, int sel_stride,
                                               int *__restrict__ cand_out, int *__restrict__ ncand_out,
                                               uint16_t *__restrict__ qhash_out)
{
    extern __shared__ __align__(16) unsigned char smem[];
    const RouteView V = route_view(smem, route_smem(P.head_dim, cap, P.max_logical));
    const int b = blockIdx.x, tid = threadIdx.x;
    const int layer = slots ? slots[b] : b;
    const int base = layer * P.max_logical;
    const int lim_b = lim ? lim[b] : 0;
    const int n = lim ? (lim_b + kPg - 1) / kPg : P.n_logical[layer];
    int *selb = sel + (size_t)b * sel_stride;

    if (n <= 0 || n <= k_sel) {
        // dense: every page, logical order
        for (int i = tid; i < n; i += blockDim.x)
            selb[i] = P.page_table[base + i];
        if (tid == 0) {
            nsel[b] = n > 0 ? n : 0;
            if (ncand_out)
                ncand_out[b] = 0;
        }
        return;
    }
    const int nidx = min(lim ? min(P.n_indexed[layer], lim_b / kPg) : P.n_indexed[layer], P.max_logical);
    route_prepare<STAGE>(P, q + (size_t)b * H * P.head_dim, base, n, nidx, H, cap, V,
                         qhash_out ? qhash_out + b : nullptr, cand_out ? cand_out + (size_t)b * cap : nullptr,
                         ncand_out ? ncand_out + b : nullptr);
    if ((tid >> 6) != 0)
        return;
    const int ns = route_select(k_sel, cap, V, selb, nullptr);
    if ((tid & 63) == 0)
        nsel[b] = ns;
}

// Hash of n vectors: each wave hashes 4 vectors, 16 lanes per vector, one
// ballot packs the 4 sign masks.
__global__ __launch_bounds__(256) void k_lsh_hash(uint16_t *__restrict__ out, const float *__restrict__ vecs,
                                                  int n, const float *__restrict__ hpT, int dim)
{
    const int lane = threadIdx.x & 63, wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int vi = wave * 4 + (lane >> 4), h = lane & 15;
    float s = 0.0f;
    if (vi < n) {
        const float *v = vecs + (size_t)vi * dim;
        for (int d = 0; d < dim; d++)
            s = __fmaf_rn(v[d], hpT[d * 16 + h], s);
    }
    const unsigned long long m = __ballot(vi < n && s > 0.0f);
    if (h == 0 && vi < n)
        out[vi] = (uint16_t)((m >> (lane & 48)) & 0xFFFFu);
}

// Candidate lookup over a flat array of index hashes (index id = position):
// the chain-walk order restated as probe order, then descending id.  One
// block per query, same ballot scan as the router.
__global__ __launch_bounds__(256) void k_lsh_candidates(const uint16_t *__restrict__ hashes, int n_ids,
                                                        const uint16_t *__restrict__ qh, int n_q, int cap,
                                                        int *__restrict__ ids, int *__restrict__ n_out)
{
    extern __shared__ __align__(16) unsigned char smem[];
    int *list = (int *)smem;                          // [4][17][cap]
    int *cnt = list + 4 * kProbes * cap;              // [4][17]
    const int b = blockIdx.x, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int q = qh[b];
    const int part = (n_ids + 3) / 4;
    const int hi = max(n_ids - wave * part, 0), lo = max(n_ids - (wave + 1) * part, 0);
    int cntv = 0;
    int *mylist = list + wave * kProbes * cap;
    for (int top = hi - 1; top >= lo; top -= kWave) {
        const int id = top - lane;
        int p = kProbes;
        if (id >= lo) {
            const int dd = (int)hashes[id] ^ q;
            p = dd == 0 ? 0 : (((dd & (dd - 1)) == 0) ? __ffs(dd) : kProbes);
        }
        unsigned long long hits = __ballot(p < kProbes);
        while (hits) {
            const int l0 = __ffsll((long long)hits) - 1;
            const int pp = rl(p, l0);
            const unsigned long long m = __ballot(p == pp);
            const int basec = rl(cntv, pp);
            if (p == pp) {
                const int rank = __popcll(m & ((1ull << lane) - 1ull));
                if (basec + rank < cap)
                    mylist[pp * cap + basec + rank] = id;
            }
            if (lane == pp)
                cntv += __popcll(m);
            hits &= ~m;
        }
    }
    if (lane < kProbes)
        cnt[wave * kProbes + lane] = cntv;
    __syncthreads();
    if (wave != 0)
        return;
    int total = 0;
    for (int p = 0; p < kProbes && total < cap; p++)
        for (int w = 0; w < 4 && total < cap; w++) {
            const int c = min(cnt[w * kProbes + p], cap);
            const int take = min(c, cap - total);
            for (int i = lane; i < take; i += kWave)
                ids[(size_t)b * cap + total + i] = list[(w * kProbes + p) * cap + i];
            total += take;
        }
    if (lane == 0)
        n_out[b] = total;
}

int launch_route(const be42_kv_pool &P, const float *q, const int *slots, const int *lim, int n_queries, int H,
                 int k_sel, int cap, int *sel, int *nsel, int sel_stride, int *cand, int *ncand, uint16_t *qhash,
                 hipStream_t s)
{
    const RouteSmem L = route_smem(P.head_dim, cap, P.max_logical);
    const void *fn = L.stage ? (const void *)k_route<true> : (const void *)k_route<false>;
    if (L.bytes > 65536)
        BE42_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, L.bytes));
    if (L.stage)
        hipLaunchKernelGGL(k_route<true>, dim3(n_queries), dim3(256), (size_t)L.bytes, s, P, q, slots, lim, H, k_sel,
                           cap, sel, nsel, sel_stride, cand, ncand, qhash);
    else
        hipLaunchKernelGGL(k_route<false>, dim3(n_queries), dim3(256), (size_t)L.bytes, s, P, q, slots, lim, H,
                           k_sel, cap, sel, nsel, sel_stride, cand, ncand, qhash);
    BE42_LAUNCH_CHECK();
    return BE42_OK;
}

}  // namespace be42

using namespace be42;

// lsh_init (ops_lsh.c:22-85): LCG uniforms, Box-Muller with libm, rows
// L2-normalised (squared norm accumulated with fused multiply-add, as the
// reference's compiled loop does), transposed.  Host code: it runs once at
// model load and its libm-dependent output is uploaded.
extern "C" void be42_lsh_projection(float *hp, float *hpT, int dim, unsigned int seed)
{
    if (dim > 256)
        dim = 256;
    for (int h = 0; h < 16; h++) {
        float nrm = 0.0f;
        for (int d = 0; d < dim; d++) {
            seed = seed * 1103515245u + 12345u;
            float u1 = (float)((seed >> 16) & 0x7FFF) / 32767.0f;
            seed = seed * 1103515245u + 12345u;
            const float u2 = (float)((seed >> 16) & 0x7FFF) / 32767.0f;
            if (u1 < 1e-6f)
                u1 = 1e-6f;
            const float g = sqrtf(-2.0f * logf(u1)) * cosf(2.0f * 3.14159265f * u2);
            hp[h * dim + d] = g;
            nrm = fmaf(g, g, nrm);
        }
        nrm = sqrtf(nrm);
        if (nrm > 1e-6f)
            for (int d = 0; d < dim; d++)
                hp[h * dim + d] /= nrm;
    }
    if (hpT)
        for (int d = 0; d < dim; d++)
            for (int h = 0; h < 16; h++)
                hpT[d * 16 + h] = hp[h * dim + d];
}

extern "C" int be42_lsh_hash(uint16_t *out, const float *vecs, int n, const float *hpT, int dim, void *stream)
{
    BE42_CHECK(out && vecs && hpT, "be42_lsh_hash: null pointer");
    BE42_CHECK(n >= 0 && dim > 0 && dim <= 256, "be42_lsh_hash: bad shape n=%d dim=%d", n, dim);
    if (n == 0)
        return BE42_OK;
    const int waves = (n + 3) / 4;
    const int blocks = (waves + 3) / 4;
    hipLaunchKernelGGL(k_lsh_hash, dim3(blocks), dim3(256), 0, as_stream(stream), out, vecs, n, hpT, dim);
    BE42_LAUNCH_CHECK();
    return BE42_OK;
}

extern "C" int be42_lsh_candidates(int *ids, int *n_out, const uint16_t *hashes, int n_ids, const uint16_t *qh,
                                   int n_q, int cap, void *stream)
{
    BE42_CHECK(ids && n_out && hashes && qh, "be42_lsh_candidates: null pointer");
    BE42_CHECK(n_ids >= 0 && n_q >= 0 && cap > 0 && cap <= kMaxCandList, "be42_lsh_candidates: bad sizes (cap %d)",
               cap);
    if (n_q == 0)
        return BE42_OK;
    const size_t smem = (size_t)(4 * kProbes * cap + 4 * kProbes) * sizeof(int);
    if (smem > 65536)
        BE42_HIP(hipFuncSetAttribute((const void *)k_lsh_candidates, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)smem));
    hipLaunchKernelGGL(k_lsh_candidates, dim3(n_q), dim3(256), smem, as_stream(stream), hashes, n_ids, qh, n_q,
                       cap, ids, n_out);
    BE42_LAUNCH_CHECK();
    return BE42_OK;
}

extern "C" int be42_lsh_route(const be42_kv_pool *pool, const float *q, const int *slots, int n_queries,
                              int n_heads, int k_sel, int cand_cap, int *sel, int *n_sel, int sel_stride,
                              int *cand, int *n_cand, uint16_t *qhash, void *stream)
{
    BE42_CHECK(pool && q && sel && n_sel, "be42_lsh_route: null pointer");
    BE42_CHECK(n_queries >= 0 && n_heads > 0 && k_sel > 0 && cand_cap > 0 && cand_cap <= kMaxCand,
               "be42_lsh_route: bad sizes (heads %d, k %d, cap %d)", n_heads, k_sel, cand_cap);
    BE42_CHECK(sel_stride >= k_sel && sel_stride >= kHeapMax + 2,
               "be42_lsh_route: sel_stride %d must be >= max(k, 64)", sel_stride);
    if (n_queries == 0)
        return BE42_OK;
    return be42::launch_route(*pool, q, slots, nullptr, n_queries, n_heads, k_sel, cand_cap, sel, n_sel, sel_stride,
                              cand, n_cand, qhash, as_stream(stream));
}
