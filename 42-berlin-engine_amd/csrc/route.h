// route.h -- the LSH router's phases as device functions, shared by the
// router kernel (lsh.hip) and the fused route + attention kernel
// (attention.hip).  Reference: lsh_hash ops_lsh.c:138-242,
// lsh_find_candidates ops_lsh.c:361-418, the q_mean glue inference.c:291-302,
// score_blocks paged.c:401-431, select_top_k_blocks paged.c:439-495 and the
// heap of ops_heap.h:33-100; the algorithm is described in lsh.hip.
#pragma once

#include "be42_common.h"
#include "heap_wave.h"

namespace be42 {

constexpr int kPg = 16;             // tokens per KV page
constexpr int kProbes = 17;
constexpr int kMaxCand = 256;       // router candidate cap
constexpr int kMaxCandList = 512;   // be42_lsh_candidates cap

constexpr int kLdsBytes = 160 * 1024;   // LDS of one gfx950 workgroup
// Waves the candidate scan can use (a block's waves, at most 16); the
// router's counters after them: query hash, candidates, middle entries.
constexpr int kScanWaves = 16;
constexpr int kCntHash = kScanWaves * kProbes, kCntTotal = kCntHash + 1, kCntMid = kCntHash + 2;

struct RouteSmem {
    int off_qm, off_q0, off_hp, off_cnt, off_offs, off_cand, off_mid, off_sc, off_rk, off_mpt, off_ph,
        off_pt, stage, stage_pt, bytes;
};

// LDS the router's own layout may take (dynamic shared memory), leaving room
// for the static LDS of the kernels that embed it.
constexpr int kRouteLdsBudget = 96 * 1024;
// The page table is staged too only while the layout stays within this, so
// that two route + attention workgroups (~25 KB of static LDS each) still
// share a CU: at 128k context (8192 pages) staging it would take 32 KB more
// and leave one workgroup per CU.  Unstaged, the router reads the ~66
// entries it needs (the anchors and the middle entries) from HBM.
constexpr int kRouteLdsStagePt = 40 * 1024;

// LDS layout of the router.  When they fit in the budget, the layer's page
// hashes (stage = max_logical) and page table (stage_pt) are staged there,
// else read from HBM.
__host__ __device__ inline RouteSmem route_smem(int hd, int cap, int max_logical)
{
    RouteSmem r;
    int o = 0;
    r.off_qm = o;   o += 256 * 4;
    r.off_q0 = o;   o += 256 * 4;
    r.off_hp = o;   o += 16 * (hd + 4) * 4;   // projection, bit-major, rows padded by 16 bytes
    r.off_cnt = o;  o += kScanWaves * kProbes * 4 + 4 * 4;
    r.off_offs = o; o += kScanWaves * kProbes * 4 + 4 * 4;
    r.off_cand = o; o += cap * 4;
    r.off_mid = o;  o += cap * 4;
    o = (o + 15) & ~15;                          // route_select reads sc four at a time
    r.off_sc = o;   o += (cap * 4 + 15) & ~15;
    r.off_rk = o;   o += 4 * cap * 4;             // partial ranks, [4][cap]
    r.off_mpt = o;  o += cap * 4 + 4 * 4;
    r.stage = o + max_logical * 2 + 16 <= kRouteLdsBudget ? max_logical : 0;
    r.stage_pt = r.stage && o + max_logical * 6 + 32 <= kRouteLdsStagePt ? 1 : 0;
    r.off_pt = o;   o += r.stage_pt ? (r.stage * 4 + 15) & ~15 : 0;
    r.off_ph = o;   o += (r.stage * 2 + 15) & ~15;
    r.bytes = o;
    return r;
}

// Threads that do router work; a larger block's other threads only take part
// in the barriers.
constexpr int kRouteThreads = 256;

// Pointers into the router's LDS.
struct RouteView {
    float *qm, *q0, *hp, *sc;
    int *cnt, *offs, *cand, *mid, *mpt, *pt_s, *rk;
    uint16_t *ph_s;
};

__device__ __forceinline__ RouteView route_view(unsigned char *smem, const RouteSmem &L)
{
    RouteView V;
    V.qm = (float *)(smem + L.off_qm);
    V.q0 = (float *)(smem + L.off_q0);
    V.hp = (float *)(smem + L.off_hp);
    V.cnt = (int *)(smem + L.off_cnt);
    V.offs = (int *)(smem + L.off_offs);
    V.cand = (int *)(smem + L.off_cand);
    V.mid = (int *)(smem + L.off_mid);
    V.sc = (float *)(smem + L.off_sc);
    V.mpt = (int *)(smem + L.off_mpt);   // [cap] physical page of mid[e]; [cap], [cap+1]: first, last page
    V.ph_s = (uint16_t *)(smem + L.off_ph);
    V.pt_s = L.stage_pt ? (int *)(smem + L.off_pt) : nullptr;   // page table staged
    V.rk = (int *)(smem + L.off_rk);
    return V;
}

__device__ __forceinline__ int rl(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }

// Phases 0-4 for one query over n > k pages of a layer (page table row
// `base`): staging, q_mean and its hash, the candidate scan, concatenation
// and middle entries, and the middle entries' scores.  Called by every thread
// of the block (>= kRouteThreads threads).  Leaves in LDS: mid[e] (logical
// page), mpt[e] (physical page), sc[e] for e < cnt[kCntMid], and the
// first and last physical page in mpt[cap], mpt[cap + 1]; qhash_b, cand_b
// and ncand_b (optional) receive the query hash and the candidate list.
template <bool STAGE, class Idle>
__device__ __forceinline__ void route_prepare(const be42_kv_pool &P, const float *__restrict__ qb, int base, int n,
                                              int nidx, int H, int cap, const RouteView &V, uint16_t *qhash_b,
                                              int *cand_b, int *ncand_b, Idle &&idle)
{
    const int hd = P.head_dim;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    float *qm = V.qm, *q0 = V.q0, *hp = V.hp, *sc = V.sc;
    int *cnt = V.cnt, *offs = V.offs, *cand = V.cand, *mid = V.mid, *mpt = V.mpt;
    uint16_t *ph_s = V.ph_s;
    // 0./1. loads that do not depend on the query hash, issued before any is
    //    used: page hashes and page table (staged), projection, the query's
    //    heads for q_mean; then q_mean (inference.c:291-295: sum in head
    //    order, then / n_heads)
    const uint16_t *ph = STAGE ? ph_s : P.page_hash + base;
    const bool spt = STAGE && V.pt_s;
    // entry i of the layer's page table, from LDS when staged
    auto ptab = [&](int i) -> int { return spt ? V.pt_s[i] : P.page_table[base + i]; };
    if (tid < kRouteThreads) {
        // unconditional loads at clamped indices (a conditional load is a
        // branch, and the compiler then waits for each load on its own);
        // the values past the ends are never used
        uint16_t hv[8];
        int pv[8];
        float wv[8], qv[32];
        const int ih = max(nidx - 1, 0), ip = max(n - 1, 0), iw = hd * 16 - 1;
        const int d = tid, dc = min(d, hd - 1);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int i = j * kRouteThreads + tid;
            if (STAGE)
                hv[j] = P.page_hash[base + min(i, ih)];
            if (spt)
                pv[j] = P.page_table[base + min(i, ip)];
            wv[j] = P.hpT[min(i, iw)];
        }
#pragma unroll
        for (int j = 0; j < 32; j++)
            qv[j] = qb[min(j, H - 1) * hd + dc];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int i = j * kRouteThreads + tid;
            if (STAGE && i < nidx)
                ph_s[i] = hv[j];
            if (spt && i < n)
                V.pt_s[i] = pv[j];
            if (i < hd * 16)
                hp[(i & 15) * (hd + 4) + (i >> 4)] = wv[j];   // hpT[d][bit] -> hp[bit][d]
        }
        // the rest (more than 2048 pages, head_dim > 128, more than 32 heads)
        for (int i = 8 * kRouteThreads + tid; STAGE && i < max(nidx, n); i += kRouteThreads) {
            if (i < nidx)
                ph_s[i] = P.page_hash[base + i];
            if (spt && i < n)
                V.pt_s[i] = P.page_table[base + i];
        }
        for (int i = 8 * kRouteThreads + tid; i < hd * 16; i += kRouteThreads)
            hp[(i & 15) * (hd + 4) + (i >> 4)] = P.hpT[i];
        if (d < hd) {
            float sum = 0.0f;
#pragma unroll
            for (int j = 0; j < 32; j++)
                sum = j < H ? sum + qv[j] : sum;
            for (int h = 32; h < H; h++)
                sum = sum + qb[h * hd + d];
            qm[d] = sum / (float)H;
            q0[d] = qv[0];
        }
    }
    __syncthreads();
    if (tid >= kRouteThreads)
        idle();
    if (tid == 0) {
        mpt[cap] = ptab(0);
        mpt[cap + 1] = ptab(n - 1);
    }
    if (wave == 0) {
        float s = 0.0f;
        if (lane < 16) {
            // the reference's order (d ascending, one fused multiply-add
            // each), four terms per 16-byte LDS read: qm broadcast, the
            // lane's projection row padded so the 16 rows hit different banks
            const float4 *qm4 = (const float4 *)qm;
            const float4 *hp4 = (const float4 *)(hp + lane * (hd + 4));
#pragma unroll 8
            for (int i4 = 0; i4 < hd / 4; i4++) {
                const float4 a = qm4[i4], w = hp4[i4];
                s = __fmaf_rn(a.x, w.x, s);
                s = __fmaf_rn(a.y, w.y, s);
                s = __fmaf_rn(a.z, w.z, s);
                s = __fmaf_rn(a.w, w.w, s);
            }
        }
        const unsigned long long m = __ballot(lane < 16 && s > 0.0f);
        if (lane == 0)
            cnt[kCntHash] = (int)(m & 0xFFFFu);
    }
    __syncthreads();
    const int qh = cnt[kCntHash];
    if (tid == 0 && qhash_b)
        *qhash_b = (uint16_t)qh;

    // 2. candidate scan in two passes over the ids, wave w of the nw waves
    //    owning ids [lo, hi) scanned from hi-1 down (wave 0 the highest):
    //    (a) every wave counts its hits per probe; (b) the counts give each
    //    (probe, wave) run its place in the concatenation (probe order, then
    //    descending id), and the second pass writes the hits there, up to
    //    cap.  Lane p < 17 keeps the running count of probe p.
    const int nw = min((int)(blockDim.x >> 6), kScanWaves);
    const int part = (nidx + nw - 1) / nw;
    const int shi = max(nidx - wave * part, 0), slo = max(nidx - (wave + 1) * part, 0);
    auto scan = [&](auto &&hit) {
        int cntv = 0;
        for (int top0 = shi - 1; top0 >= slo; top0 -= 4 * kWave) {
            // four chunks of 64 ids: their hash reads are issued together
            int pv[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int id = top0 - u * kWave - lane;
                const int dd = (int)ph[max(id, slo)] ^ qh;
                pv[u] = id < slo ? kProbes : (dd == 0 ? 0 : (((dd & (dd - 1)) == 0) ? __ffs(dd) : kProbes));
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int id = top0 - u * kWave - lane;
                const int p = pv[u];
                unsigned long long hits = __ballot(p < kProbes);
                while (hits) {
                    const int l0 = __ffsll((long long)hits) - 1;
                    const int pp = rl(p, l0);
                    const unsigned long long m = __ballot(p == pp);
                    const int basec = rl(cntv, pp);
                    if (p == pp)
                        hit(pp, basec + __popcll(m & ((1ull << lane) - 1ull)), id);
                    if (lane == pp)
                        cntv += __popcll(m);
                    hits &= ~m;
                }
            }
        }
        return cntv;
    };
    if (wave < nw) {
        const int c = scan([](int, int, int) {});
        if (lane < kProbes)
            cnt[wave * kProbes + lane] = c;
    }
    __syncthreads();
    // run j = probe * nw + w starts at offs[j]; lane l of wave 0 owns runs
    // 5l .. 5l + 4 (at most 16 * 17 = 272 runs)
    if (wave == 0) {
        constexpr int RPL = (kScanWaves * kProbes + kWave - 1) / kWave;
        const int nj = nw * kProbes;
        int c[RPL], sum = 0;
#pragma unroll
        for (int i = 0; i < RPL; i++) {
            const int j = lane * RPL + i;
            c[i] = j < nj ? cnt[(j % nw) * kProbes + j / nw] : 0;
            sum += c[i];
        }
        int inc = sum;
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) {
            const int v = __shfl_up(inc, o, kWave);
            if (lane >= o)
                inc += v;
        }
        int run = inc - sum;
#pragma unroll
        for (int i = 0; i < RPL; i++) {
            const int j = lane * RPL + i;
            if (j < nj)
                offs[j] = run;
            run += c[i];
        }
        if (lane == kWave - 1)
            cnt[kCntTotal] = min(inc, cap);
    }
    __syncthreads();
    if (wave < nw)
        scan([&](int pp, int rank, int id) {
            const int at = offs[pp * nw + wave] + rank;
            if (at < cap)
                cand[at] = id;
        });
    __syncthreads();
    const int total = cnt[kCntTotal];
    if (cand_b)
        for (int i = tid; i < total; i += kRouteThreads)
            cand_b[i] = cand[i];
    if (tid == 0 && ncand_b)
        *ncand_b = total;
    // middle entries: candidates other than the first and last page
    if (wave == 0) {
        int nm = 0;
        for (int i0 = 0; i0 < total; i0 += kWave) {
            const int i = i0 + lane;
            const int id = i < total ? cand[i] : -1;
            const bool keep = i < total && id != 0 && id != n - 1 && id < n;
            const unsigned long long m = __ballot(keep);
            if (keep)
                mid[nm + __popcll(m & ((1ull << lane) - 1ull))] = id;
            nm += __popcll(m);
        }
        if (lane == 0)
            cnt[kCntMid] = nm;
    }
    __syncthreads();
    const int nm = cnt[kCntMid];

    // 4. scores of the middle entries (score_blocks semantics), a lane pair each
    for (int e0 = 0; tid < kRouteThreads && e0 < nm; e0 += 128) {
        const int e = e0 + (tid >> 1), half = tid & 1;
        const int ee = e < nm ? e : nm - 1;
        const int phys = ptab(mid[ee]);
        const float s = dot_ref8x2(q0, P.centroid + (size_t)phys * hd, hd, half);
        if (half == 0 && e < nm) {
            sc[e] = s;
            mpt[e] = phys;
        }
    }
    __syncthreads();
    // 5a. ranks of the middle scores for the heap's integer keys (the number
    //     of strictly smaller ones), for more than 64 entries: wave w counts,
    //     for entries lane + 64 j, the smaller ones among its quarter of the
    //     entries (every lane reads the same score: an LDS broadcast).  Up to
    //     64 entries route_select ranks them itself on wave 0, so the other
    //     waves go on to the attention's scores without this phase.
    if (wave < 4 && nm > kWave) {
        const int q0i = wave * nm / 4, q1i = (wave + 1) * nm / 4;
        float own[4];
        int r[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            own[j] = sc[min(lane + 64 * j, nm - 1)];
            r[j] = 0;
        }
        for (int i0 = q0i; i0 < q1i; i0 += 8) {
            float x[8];
#pragma unroll
            for (int u = 0; u < 8; u++)
                x[u] = sc[min(i0 + u, q1i - 1)];
#pragma unroll
            for (int u = 0; u < 8; u++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    r[j] += i0 + u < q1i && x[u] < own[j] ? 1 : 0;
        }
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (lane + 64 * j < nm)
                V.rk[wave * cap + lane + 64 * j] = r[j];
    }
    __syncthreads();

}

template <bool STAGE>
__device__ __forceinline__ void route_prepare(const be42_kv_pool &P, const float *__restrict__ qb, int base, int n,
                                              int nidx, int H, int cap, const RouteView &V, uint16_t *qhash_b,
                                              int *cand_b, int *ncand_b)
{
    route_prepare<STAGE>(P, qb, base, n, nidx, H, cap, V, qhash_b, cand_b, ncand_b, [] {});
}

__device__ __forceinline__ int route_middles(const RouteView &V) { return V.cnt[kCntMid]; }

// Phase 5 on wave 0: selection = [first page, last page] + the reference
// min-heap over the middle entries (capacity min(k-2, #middle, 62), strict
// replacement) in heap array order.  Writes the physical pages to selb (if
// not NULL) and, if `order` is not NULL, the selection in "set slots":
// slot 0 the first page, slot 1 the last (when it differs), slot ns0 + e
// middle entry e.  Returns the number selected (uniform).
__device__ __forceinline__ int route_select(int k_sel, int cap, const RouteView &V, int *selb, int *order)
{
    const int lane = threadIdx.x & 63;
    const int nm = route_middles(V);
    const int first = V.mpt[cap], last = V.mpt[cap + 1];
    const int ns = last != first ? 2 : 1;
    if (lane == 0) {
        if (selb) {
            selb[0] = first;
            if (ns == 2)
                selb[1] = last;
        }
        if (order) {
            order[0] = 0;
            if (ns == 2)
                order[1] = 1;
        }
    }
    int ak = min(k_sel - 2, min(nm, kHeapMax));
    if (k_sel <= 2 || nm == 0)
        ak = 0;
    // every middle score is known before the first push: the heap runs on
    // (rank, entry) keys, which order exactly as the scores
    int rk[4];
    if (nm <= kWave) {
        // entry lane's rank: the scores four at a time as LDS broadcasts
        // (every lane reads one address; sc is 16-byte aligned, its entries
        // rounded up to four).  Reading lanes' scores across the wave one
        // at a time (a readlane per entry) took twice as long next to the
        // waves that score the pages meanwhile.
        const float own = V.sc[min(lane, max(nm - 1, 0))];
        const float4 *sc4 = (const float4 *)V.sc;
        int r = 0;
        for (int j0 = 0; j0 < nm; j0 += 16) {
            float4 x[4];
#pragma unroll
            for (int u = 0; u < 4; u++)
                x[u] = sc4[min(j0 / 4 + u, (nm - 1) / 4)];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int j = j0 + 4 * u;
                r += j < nm && x[u].x < own ? 1 : 0;
                r += j + 1 < nm && x[u].y < own ? 1 : 0;
                r += j + 2 < nm && x[u].z < own ? 1 : 0;
                r += j + 3 < nm && x[u].w < own ? 1 : 0;
            }
        }
        rk[0] = r;
        rk[1] = rk[2] = rk[3] = 0;
    } else {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int e = min(lane + 64 * j, max(nm - 1, 0));
            rk[j] = V.rk[e] + V.rk[cap + e] + V.rk[2 * cap + e] + V.rk[3 * cap + e];
        }
    }
    WaveHeapKey heap(ak);
    // the pushes that fill the heap on the scalar unit, then the ones that
    // may replace its root
    heap.fill(ak, rk);
    for (int e0 = ak & ~(kWave - 1); e0 < nm && ak > 0; e0 += kWave) {
        const int j = e0 >> 6;
        const int rv = j == 0 ? rk[0] : (j == 1 ? rk[1] : (j == 2 ? rk[2] : rk[3]));
        const int ecnt = min(kWave, nm - e0);
        for (int u = max(ak - e0, 0); u < ecnt; u++)
            heap.push(rl(rv, u), e0 + u);
    }
    const int size = heap.size, hi = heap.payload();
    if (lane < size) {
        if (selb)
            selb[ns + lane] = V.mpt[hi];
        if (order)
            order[ns + lane] = ns + hi;
    }
    return ns + size;
}

}  // namespace be42
