// linear.hip -- the linear (non-paged) bf16 KV cache path on gfx950.
//
// kv_cache_append / kv_cache_evict      src/memory/kv_cache.c:55-80,
//                                       kv_cache_evict.c:34-70, kv_cache_score.c
// flash_attention_head / op_attention_dense / op_attention_sparse /
// op_multihead_attention                src/compute/ops_attention.c:41-245
// token routing glue                    src/inference/inference.c:268-423
//
// The cache is [T][n_kv][hd] bf16 rows (kv_cache.h:19-27).
//  * Attention over a list of tokens (or all of them) gathers the listed rows
//    into 16-token pages ([page][n_kv][16][hd], the page pool's layout) and
//    runs the paged attention kernels over them in list order: the same
//    online softmax, evaluated in the same closed form.
//  * The token route runs in one workgroup: window positions, the LSH
//    candidate blocks (probe order, newest first, as lsh_find_candidates)
//    that end before the window, the union sorted (blocks are disjoint
//    position ranges, so sorting the ranges by start sorts the positions),
//    per-candidate scores sum_kv dot_bf16 in the reference's reduction order,
//    and the reference min-heap over the candidates in position order.  The
//    heap's root only rises once the heap is full, so a candidate scoring <=
//    the root when its group of 64 starts cannot change the heap and is not
//    pushed.
//  * Eviction scores every position, ranks it by (score desc, position asc)
//    -- the order of the reference's stable sort -- and compacts the kept
//    rows in position order through a staging buffer.
#include <algorithm>

#include "be42_common.h"
#include "heap_wave.h"

namespace be42 {

constexpr int kLinPage = 16;

// rows idx[i] (i < n; idx NULL: i) of K and V into page i / 16, slot i % 16
__global__ __launch_bounds__(64) void k_linear_gather(uint16_t *__restrict__ kp, uint16_t *__restrict__ vp,
                                                      int *__restrict__ ntok, const uint16_t *__restrict__ k,
                                                      const uint16_t *__restrict__ v, const int *__restrict__ idx,
                                                      int n, int n_kv, int hd)
{
    const int i = blockIdx.x, h = blockIdx.y;
    const int t = idx ? idx[i] : i;
    const size_t src = ((size_t)t * n_kv + h) * hd;
    const size_t dst = (((size_t)(i / kLinPage) * n_kv + h) * kLinPage + i % kLinPage) * hd;
    // V pages [kv head][dim][16 tokens], as the page pool's bf16 pages
    const size_t vdst = ((size_t)(i / kLinPage) * n_kv + h) * hd * kLinPage + i % kLinPage;
    for (int d = threadIdx.x; d < hd; d += 64) {
        kp[dst + d] = k[src + d];
        vp[vdst + (size_t)d * kLinPage] = v[src + d];
    }
    if (h == 0 && threadIdx.x == 0 && i % kLinPage == 0)
        ntok[i / kLinPage] = min(kLinPage, n - i);
}

__global__ void k_iota(int *__restrict__ sel, int *__restrict__ nsel, int n)
{
    for (int i = threadIdx.x; i < n; i += blockDim.x)
        sel[i] = i;
    if (threadIdx.x == 0)
        *nsel = n;
}

// f32 K and V rows of one token -> bf16 (float_to_bf16, tensor.c:67-76)
__global__ __launch_bounds__(256) void k_linear_append(uint16_t *__restrict__ kd, uint16_t *__restrict__ vd,
                                                       const float *__restrict__ k, const float *__restrict__ v,
                                                       int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        kd[i] = f32_to_bf16(k[i]);
        vd[i] = f32_to_bf16(v[i]);
    }
}

// simd_dot_bf16_f32 as the reference build evaluates it (simd_kernels.h:97-156,
// 8 lanes): lane l accumulates i = l (mod 8) with fused multiply-adds, then
// 0 + ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)), then the fused scalar tail.
__device__ __forceinline__ float dot_bf16_ref(const uint16_t *__restrict__ a, const float *__restrict__ b, int n)
{
    float l[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int i = 0;
    for (; i + 7 < n; i += 8)
#pragma unroll
        for (int j = 0; j < 8; j++)
            l[j] = __fmaf_rn(bf16_to_f32(a[i + j]), b[i + j], l[j]);
    float sum = 0.0f;
    sum = sum + (((l[0] + l[4]) + (l[1] + l[5])) + ((l[2] + l[6]) + (l[3] + l[7])));
    for (; i < n; i++)
        sum = __fmaf_rn(bf16_to_f32(a[i]), b[i], sum);
    return sum;
}

// kv_cache_score.c: score_s = sum_h bf16(w[h]) * max(0, sum_d bf16(q[h][d]) *
// bf16(k[s][h][d])), each sum a fused chain in order
__global__ __launch_bounds__(256) void k_evict_scores(float *__restrict__ score, const uint16_t *__restrict__ k,
                                                      const uint16_t *__restrict__ q,
                                                      const uint16_t *__restrict__ w, int n, int heads, int dim)
{
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= n)
        return;
    float total = 0.0f;
    for (int h = 0; h < heads; h++) {
        const uint16_t *kr = k + ((size_t)s * heads + h) * dim;
        float dot = 0.0f;
        for (int d = 0; d < dim; d++)
            dot = __fmaf_rn(bf16_to_f32(q[h * dim + d]), bf16_to_f32(kr[d]), dot);
        if (dot < 0.0f)
            dot = 0.0f;
        total = __fmaf_rn(bf16_to_f32(w[h]), dot, total);
    }
    score[s] = total;
}

// keep[s] = rank of s by (score desc, position asc) < keep_k
__global__ __launch_bounds__(256) void k_evict_keep(int *__restrict__ keep, const float *__restrict__ score, int n,
                                                    int keep_k)
{
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= n)
        return;
    const float v = score[s];
    int rank = 0;
    for (int t = 0; t < n && rank < keep_k; t++) {
        const float u = score[t];
        rank += (u > v || (u == v && t < s)) ? 1 : 0;
    }
    keep[s] = rank < keep_k;
}

// dst[s] = number of kept positions before s (one block: each thread
// counts a contiguous range, the counts are scanned in LDS)
__global__ __launch_bounds__(1024) void k_evict_dst(int *__restrict__ dst, const int *__restrict__ keep, int n)
{
    __shared__ int cnt[1024];
    const int t = threadIdx.x, per = (n + 1023) / 1024;
    const int lo = min(n, t * per), hi = min(n, lo + per);
    int c = 0;
    for (int s = lo; s < hi; s++)
        c += keep[s];
    cnt[t] = c;
    __syncthreads();
    if (t == 0) {
        int run = 0;
        for (int i = 0; i < 1024; i++) {
            const int x = cnt[i];
            cnt[i] = run;
            run += x;
        }
    }
    __syncthreads();
    int run = cnt[t];
    for (int s = lo; s < hi; s++) {
        dst[s] = run;
        run += keep[s];
    }
}

// the kept rows, in position order, into the staging buffer (row dst[s] of
// the staging buffer); one block per position
__global__ __launch_bounds__(64) void k_evict_stage(uint16_t *__restrict__ ks, uint16_t *__restrict__ vs,
                                                    const uint16_t *__restrict__ k, const uint16_t *__restrict__ v,
                                                    const int *__restrict__ keep, const int *__restrict__ dst,
                                                    int row)
{
    const int s = blockIdx.x;
    if (!keep[s])
        return;
    const size_t o = (size_t)dst[s] * row, i = (size_t)s * row;
    for (int d = threadIdx.x; d < row; d += 64) {
        ks[o + d] = k[i + d];
        vs[o + d] = v[i + d];
    }
}

// ---- token route (inference.c:268-423) -------------------------------------------
constexpr int kTokMaxBlocks = 64;           // lsh_find_candidates(.., 64)
constexpr int kTokThreads = 256;

struct TokRouteArgs {
    const uint16_t *k;              // [T][n_kv][hd]
    const float *q;                 // [n_heads][hd]
    const float *hpT;               // [hd][16]
    const uint16_t *bhash;          // [n_blocks]
    const int *bstart, *blen;       // [n_blocks]
    int *cand;                      // [kv_len] candidate positions (work)
    float *score;                   // [kv_len] their scores (work)
    int *topk, *n_topk;
    int kv_len, n_blocks, n_heads, n_kv, hd, window, sparse_k;
};

__global__ __launch_bounds__(kTokThreads) void k_route_tokens(const TokRouteArgs A)
{
    __shared__ float qm[256];
    __shared__ int sh_qh, sh_nb, sh_nc;
    __shared__ int bids[kTokMaxBlocks], bst[kTokMaxBlocks], bln[kTokMaxBlocks], boff[kTokMaxBlocks + 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int hd = A.hd, kv_len = A.kv_len;
    const int ws = kv_len > A.window ? kv_len - A.window : 0;
    const bool lsh = ws > 0 && A.n_blocks > 0;
    if (tid == 0) {
        sh_nb = 0;
        sh_qh = 0;
    }
    // q_mean (head order, then / n_heads) and its hash
    if (lsh) {
        for (int d = tid; d < hd; d += kTokThreads) {
            float s = 0.0f;
            for (int h = 0; h < A.n_heads; h++)
                s = s + A.q[(size_t)h * hd + d];
            qm[d] = s / (float)A.n_heads;
        }
        __syncthreads();
        if (wave == 0) {
            float s = 0.0f;
            if (lane < 16)
                for (int d = 0; d < hd; d++)
                    s = __fmaf_rn(qm[d], A.hpT[d * 16 + lane], s);
            const unsigned long long m = __ballot(lane < 16 && s > 0.0f);
            if (lane == 0)
                sh_qh = (int)(m & 0xFFFFu);
        }
        __syncthreads();
        // candidate blocks: probe p (0: the hash, p: bit p-1 flipped), ids
        // newest first within a probe, at most 64
        if (wave == 0) {
            const int qh = sh_qh;
            int nb = 0;
            for (int p = 0; p < 17 && nb < kTokMaxBlocks; p++) {
                const int ph = p == 0 ? qh : (qh ^ (1 << (p - 1)));
                for (int top = A.n_blocks - 1; top >= 0 && nb < kTokMaxBlocks; top -= 64) {
                    const int id = top - lane;
                    const bool hit = id >= 0 && (int)A.bhash[id] == ph;
                    const unsigned long long m = __ballot(hit);
                    const int r = __popcll(m & ((1ull << lane) - 1ull));
                    if (hit && nb + r < kTokMaxBlocks)
                        bids[nb + r] = id;
                    nb = min(nb + __popcll(m), kTokMaxBlocks);
                }
            }
            if (lane == 0)
                sh_nb = nb;
        }
        __syncthreads();
    }
    // qualifying blocks (end before the window), ordered by start: every
    // position before the window comes from exactly one of them
    const int nb = sh_nb;
    if (wave == 0) {
        int st = 0, ln = 0, ok = 0;
        if (lane < nb) {
            st = A.bstart[bids[lane]];
            ln = A.blen[bids[lane]];
            ok = st >= 0 && ln > 0 && (long long)st + ln <= ws;
        }
        int rank = 0;
        for (int j = 0; j < nb; j++) {
            const int sj = __shfl(st, j), oj = __shfl(ok, j);
            rank += (oj && (sj < st || (sj == st && j < lane))) ? 1 : 0;
        }
        const unsigned long long mo = __ballot(ok);
        const int nq = __popcll(mo);
        if (ok) {
            bst[rank] = st;
            bln[rank] = ln;
        }
        __builtin_amdgcn_wave_barrier();
        // exclusive prefix of the lengths in start order
        int len_r = lane < nq ? bln[lane] : 0;
        int inc = len_r;
        for (int o = 1; o < 64; o <<= 1) {
            const int v = __shfl_up(inc, o);
            if (lane >= o)
                inc += v;
        }
        if (lane < nq)
            boff[lane] = inc - len_r;
        const int tot = __shfl(inc, 63);
        if (lane == 0) {
            boff[nq] = tot;
            sh_nb = nq;
            // blocks from lsh_update are disjoint, so tot <= ws; overlapping
            // caller-made blocks are cut here to keep within the buffers
            sh_nc = min(tot, ws) + (kv_len - ws);
        }
    }
    __syncthreads();
    const int nq = sh_nb, nc = sh_nc, nblk_pos = boff[nq];
    // positions (sorted), then their scores in the reference's order
    for (int i = tid; i < nc; i += kTokThreads) {
        int t;
        if (i >= nblk_pos) {
            t = ws + (i - nblk_pos);
        } else {
            int lo = 0, hi = nq - 1;
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (boff[mid] <= i)
                    lo = mid;
                else
                    hi = mid - 1;
            }
            t = bst[lo] + (i - boff[lo]);
        }
        A.cand[i] = t;
        const int G = A.n_heads / A.n_kv;
        float s = 0.0f;
        for (int kv = 0; kv < A.n_kv; kv++)
            s = s + dot_bf16_ref(A.k + ((size_t)t * A.n_kv + kv) * hd, A.q + (size_t)kv * G * hd, hd);
        A.score[i] = s;
    }
    __syncthreads();
    __threadfence_block();
    if (wave != 0)
        return;
    const int cap = min(nc, A.sparse_k);
    WaveHeap heap(cap);
    for (int c0 = 0; c0 < nc; c0 += 64) {
        const int c = c0 + lane;
        const float sv = c < nc ? A.score[c] : 0.0f;
        const int tv = c < nc ? A.cand[c] : 0;
        // a full heap's root only rises: scores <= it now change nothing
        const bool full = heap.size >= cap;
        const float root = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(heap.hs), 0));
        unsigned long long act = __ballot(c < nc && (!full || sv > root));
        while (act) {
            const int u = __ffsll((long long)act) - 1;
            act &= act - 1;
            heap.push(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(sv), u)),
                      __builtin_amdgcn_readlane(tv, u));
        }
    }
    if (lane < heap.size)
        A.topk[lane] = heap.hi;
    if (lane == 0)
        *A.n_topk = heap.size;
}

}  // namespace be42

using namespace be42;

extern "C" int be42_kv_linear_append(uint16_t *k_cache, uint16_t *v_cache, int pos, const float *k, const float *v,
                                     int row, void *stream)
{
    BE42_CHECK(k_cache && v_cache && k && v && pos >= 0 && row > 0, "be42_kv_linear_append: bad arguments");
    const size_t off = (size_t)pos * row;
    hipLaunchKernelGGL(k_linear_append, dim3((row + 255) / 256), dim3(256), 0, as_stream(stream), k_cache + off,
                       v_cache + off, k, v, row);
    BE42_LAUNCH_CHECK();
    return BE42_OK;
}

extern "C" size_t be42_linear_attention_workspace_bytes(int n_tok, int n_heads, int n_kv, int head_dim)
{
    if (n_tok <= 0)
        return 0;
    const size_t np = (size_t)(n_tok + kLinPage - 1) / kLinPage;
    const size_t pages = np * n_kv * kLinPage * head_dim * 2;
    const int split = np <= 64 ? 1 : (int)((np + 63) / 64);
    const size_t attn = be42_attn_workspace_bytes(1, n_heads, head_dim, (int)np, split);
    return 2 * pages + ((np + 1) * 4 + 255) / 256 * 256 * 2 + attn + 1024;
}

extern "C" int be42_linear_attention(float *out, const float *q, const uint16_t *k, const uint16_t *v,
                                     const int *idx, int n_tok, int n_heads, int n_kv, int head_dim, float scale,
                                     void *workspace_ptr, size_t workspace_bytes, void *stream)
{
    BE42_CHECK(out && q && k && v, "be42_linear_attention: null pointer");
    BE42_CHECK(n_heads > 0 && n_kv > 0 && n_heads % n_kv == 0 && (head_dim == 64 || head_dim == 128 || head_dim == 256),
               "be42_linear_attention: %d heads over %d kv heads, head_dim %d", n_heads, n_kv, head_dim);
    hipStream_t s = as_stream(stream);
    if (n_tok <= 0) {
        BE42_HIP(hipMemsetAsync(out, 0, (size_t)n_heads * head_dim * 4, s));
        return BE42_OK;
    }
    const size_t need = be42_linear_attention_workspace_bytes(n_tok, n_heads, n_kv, head_dim);
    void *ws = workspace_ptr;
    if (!ws) {
        ws = workspace(need, s);
        if (!ws)
            return BE42_ENOMEM;
    } else {
        BE42_CHECK(workspace_bytes >= need, "be42_linear_attention: workspace %zu < %zu bytes", workspace_bytes, need);
    }
    const int np = (n_tok + kLinPage - 1) / kLinPage;
    const size_t pages = (size_t)np * n_kv * kLinPage * head_dim * 2;
    uint8_t *base = (uint8_t *)ws;
    uint16_t *kp = (uint16_t *)base;
    uint16_t *vp = (uint16_t *)(base + pages);
    const size_t ib = ((size_t)(np + 1) * 4 + 255) / 256 * 256;
    int *ntok = (int *)(base + 2 * pages);
    int *sel = (int *)(base + 2 * pages + ib);
    void *attn_ws = base + 2 * pages + 2 * ib;
    const size_t attn_bytes = need - 2 * pages - 2 * ib;
    hipLaunchKernelGGL(k_linear_gather, dim3(n_tok, n_kv), dim3(64), 0, s, kp, vp, ntok, k, v, idx, n_tok, n_kv,
                       head_dim);
    BE42_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_iota, dim3(1), dim3(256), 0, s, sel, sel + np, np);
    BE42_LAUNCH_CHECK();
    be42_kv_pool P{};
    P.kind = BE42_KV_BF16;
    P.n_layers = 1;
    P.n_kv = n_kv;
    P.head_dim = head_dim;
    P.max_logical = np;
    P.capacity = np;
    P.k = kp;
    P.v = vp;
    P.ntok = ntok;
    const int split = np <= 64 ? 1 : (np + 63) / 64;
    return be42_paged_attention(&P, q, 1, n_heads, sel, sel + np, np, np, scale, out, split, attn_ws, attn_bytes,
                                stream);
}

extern "C" int be42_lsh_route_tokens(const uint16_t *k, int kv_len, const float *q, int n_heads, int n_kv,
                                     int head_dim, const float *hpT, const uint16_t *block_hashes,
                                     const int *block_starts, const int *block_lens, int n_blocks, int window,
                                     int sparse_k, int *topk, int *n_topk, void *stream)
{
    BE42_CHECK(k && q && topk && n_topk, "be42_lsh_route_tokens: null pointer");
    BE42_CHECK(sparse_k > 0 && sparse_k <= 64, "be42_lsh_route_tokens: sparse_k %d (1..64)", sparse_k);
    BE42_CHECK(head_dim > 0 && head_dim <= 256 && n_kv > 0 && n_heads % n_kv == 0 && window >= 0 && kv_len > sparse_k,
               "be42_lsh_route_tokens: needs kv_len > sparse_k (else attention is dense), head_dim <= 256");
    BE42_CHECK(n_blocks <= 0 || (hpT && block_hashes && block_starts && block_lens),
               "be42_lsh_route_tokens: an index needs hpT and its block arrays");
    hipStream_t s = as_stream(stream);
    int *cand = (int *)workspace((size_t)kv_len * 8, s);
    if (!cand)
        return BE42_ENOMEM;
    TokRouteArgs A{};
    A.k = k;
    A.q = q;
    A.hpT = hpT;
    A.bhash = block_hashes;
    A.bstart = block_starts;
    A.blen = block_lens;
    A.cand = cand;
    A.score = (float *)(cand + kv_len);
    A.topk = topk;
    A.n_topk = n_topk;
    A.kv_len = kv_len;
    A.n_blocks = n_blocks > 0 ? n_blocks : 0;
    A.n_heads = n_heads;
    A.n_kv = n_kv;
    A.hd = head_dim;
    A.window = window;
    A.sparse_k = sparse_k;
    hipLaunchKernelGGL(k_route_tokens, dim3(1), dim3(kTokThreads), 0, s, A);
    BE42_LAUNCH_CHECK();
    return BE42_OK;
}

extern "C" int be42_kv_linear_evict(uint16_t *k, uint16_t *v, int n, int heads, int dim, const uint16_t *q,
                                    const uint16_t *w, int keep_k, int *new_len, void *stream)
{
    BE42_CHECK(k && v && q && w && new_len && heads > 0 && dim > 0, "be42_kv_linear_evict: bad arguments");
    if (keep_k <= 0 || keep_k >= n) {
        *new_len = n;
        return BE42_OK;
    }
    hipStream_t s = as_stream(stream);
    const size_t row = (size_t)heads * dim;
    const size_t nb = ((size_t)n * 4 + 255) / 256 * 256;
    uint8_t *ws = (uint8_t *)workspace(3 * nb + 2 * (size_t)keep_k * row * 2, s);
    if (!ws)
        return BE42_ENOMEM;
    float *score = (float *)ws;
    int *keep = (int *)(ws + nb);
    int *dst = (int *)(ws + 2 * nb);
    uint16_t *ks = (uint16_t *)(ws + 3 * nb);
    uint16_t *vs = ks + (size_t)keep_k * row;
    const dim3 g((n + 255) / 256);
    hipLaunchKernelGGL(k_evict_scores, g, dim3(256), 0, s, score, k, q, w, n, heads, dim);
    hipLaunchKernelGGL(k_evict_keep, g, dim3(256), 0, s, keep, score, n, keep_k);
    hipLaunchKernelGGL(k_evict_dst, dim3(1), dim3(1024), 0, s, dst, keep, n);
    hipLaunchKernelGGL(k_evict_stage, dim3(n), dim3(64), 0, s, ks, vs, k, v, keep, dst, (int)row);
    BE42_LAUNCH_CHECK();
    BE42_HIP(hipMemcpyAsync(k, ks, (size_t)keep_k * row * 2, hipMemcpyDeviceToDevice, s));
    BE42_HIP(hipMemcpyAsync(v, vs, (size_t)keep_k * row * 2, hipMemcpyDeviceToDevice, s));
    *new_len = keep_k;
    return BE42_OK;
}
