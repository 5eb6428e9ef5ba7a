// attention.hip -- attention over selected KV pages on gfx950.
//
// op_paged_attention_sparse / attention_head_paged_sparse /
// attention_block_int8        src/compute/ops_attention.c:292-348, :391-461
// op_paged_attention          src/compute/ops_attention.c:353-438
// attention_head_sparse (BF16 rows) src/compute/ops_attention.c:131-170
// fast_expf                   src/compute/ops_math_fast.h:48-64
//
// The reference runs, per query head, one online-softmax recurrence over the
// tokens of the selected pages in selection order:
//     m_t = max(m_{t-1}, s_t);  a_t = fast_expf(m_{t-1} - m_t);
//     p_t = fast_expf(s_t - m_t);  l_t = l_{t-1} a_t + p_t;  o_t = o_{t-1} a_t + p_t v_t
//     out = o_T * (1 / l_T)
// fast_expf (Schraudolph) is not multiplicative, so the result depends on the
// exact sequence of running maxima.  Here the same recurrence is evaluated in
// closed form, o_T = sum_t w_t v_t and l_T = sum_t w_t with
// w_t = p_t * prod_{t'>t} a_{t'}: running maxima from a prefix-max scan,
// products from a suffix-product scan.  Every fast_expf argument is the
// reference's; only the rounding of the sums differs.
//
// Kernels, for queries b, KV head h_kv (serving the G = H / n_kv query heads
// of its group) and splits of the selected pages:
//   k_attn_scores   s_t = (q_h . k_t) * scale, INT8 keys dequantized per
//                   element as (float)code * scale_t like the reference's
//                   JIT dequant;
//   k_attn_weights  one wave per head: the scan above, w_t over s_t in place,
//                   l = sum w_t;
//   k_attn_apply    partial o = sum_t w_t v_t over the split's pages;
//   k_attn_combine  out = (sum over splits) * (1 / l).
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "be42_common.h"
#include "paged_step.h"
#include "attn_dev.h"
#include "route.h"
#include "xdigits.h"

namespace be42 {

__device__ __forceinline__ void load_row_f32(float *dst, const void *base, size_t elem_off, int n, bool bf16,
                                             float scale)
{
    // n is a multiple of 8; 16-byte loads
    if (bf16) {
        const uint4 *p = (const uint4 *)((const uint16_t *)base + elem_off);
        for (int i = 0; i < n / 8; i++) {
            const uint4 u = p[i];
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                dst[8 * i + 2 * j] = __uint_as_float(w[j] << 16);
                dst[8 * i + 2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
            }
        }
    } else {
        const uint2 *p = (const uint2 *)((const int8_t *)base + elem_off);
        for (int i = 0; i < n / 8; i++) {
            const uint2 u = p[i];
            const uint32_t w[2] = {u.x, u.y};
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int e = 0; e < 4; e++)
                    dst[8 * i + 4 * j + e] = (float)(int8_t)((w[j] >> (8 * e)) & 0xFF) * scale;
        }
    }
}

// lane = (token t of the page: lane / 4, quarter of head_dim: lane % 4)
template <bool BF16, int HD>
__global__ __launch_bounds__(256) void k_attn_scores(const be42_kv_pool P, const float *__restrict__ q,
                                                     const int *__restrict__ sel, const int *__restrict__ nsel,
                                                     int sel_stride, int H, float scale, int pages_per_split,
                                                     float *__restrict__ scores, int t_stride)
{
    constexpr int DQ = HD / 4;
    const int b = blockIdx.x, kvh = blockIdx.y, split = blockIdx.z;
    const int n_kv = P.n_kv, G = H / n_kv;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int ns = nsel[b];
    const int i0 = split * pages_per_split, i1 = min(ns, i0 + pages_per_split);
    const int t = lane >> 2, part = lane & 3;
    for (int g = wave; g < G; g += 4) {
        const int h = kvh * G + g;
        const float *qh = q + ((size_t)b * H + h) * HD + part * DQ;
        float qv[DQ];
#pragma unroll
        for (int j = 0; j < DQ; j++)
            qv[j] = qh[j];
        float *sh = scores + ((size_t)b * H + h) * t_stride;
        for (int i = i0; i < i1; i++) {
            const int phys = sel[(size_t)b * sel_stride + i];
            const size_t slot = ((size_t)phys * n_kv + kvh) * kPg + t;
            float kv[DQ];
            load_row_f32(kv, P.k, slot * HD + part * DQ, DQ, BF16, BF16 ? 1.0f : P.k_scale[slot]);
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < DQ; j++)
                acc = __fmaf_rn(qv[j], kv[j], acc);
            acc += __shfl_xor(acc, 1, 4);
            acc += __shfl_xor(acc, 2, 4);
            if (part == 0)
                sh[i * kPg + t] = acc * scale;
        }
    }
}

// One wave per query head.  Lane l owns slots [l*C, (l+1)*C) of the
// T = 16 * n_sel slots; slots at or past a page's ntok are skipped, exactly as
// the reference never visits them.  aux holds a_t between the passes.
__global__ __launch_bounds__(256) void k_attn_weights(const be42_kv_pool P, const int *__restrict__ sel,
                                                      const int *__restrict__ nsel, int sel_stride, int H, int BH,
                                                      float *__restrict__ sw, float *__restrict__ aux,
                                                      int t_stride, float *__restrict__ lsum)
{
    const int gw = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;   // global wave = (b, h)
    const int lane = threadIdx.x & 63;
    if (gw >= BH)
        return;
    const int b = gw / H;
    const int ns = nsel[b];
    const int T = ns * kPg, C = (T + kWave - 1) / kWave;
    const int *selb = sel + (size_t)b * sel_stride;
    float *s = sw + (size_t)gw * t_stride;
    float *a = aux + (size_t)gw * t_stride;
    const int t0 = min(T, lane * C), t1 = min(T, t0 + C);
    auto valid = [&](int tt) { return (tt % kPg) < P.ntok[selb[tt / kPg]]; };

    float lm = -INFINITY;
    for (int tt = t0; tt < t1; tt++)
        if (valid(tt))
            lm = fmaxf(lm, s[tt]);
    float inc = lm;                                   // inclusive prefix max over lanes
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const float v = __shfl_up(inc, o, kWave);
        if (lane >= o)
            inc = fmaxf(inc, v);
    }
    float m = __shfl_up(inc, 1, kWave);               // max of all earlier lanes' tokens
    if (lane == 0)
        m = -INFINITY;
    float lprod = 1.0f;
    for (int tt = t0; tt < t1; tt++) {
        if (!valid(tt))
            continue;
        const float st = s[tt];
        const float mprev = m;
        m = fmaxf(m, st);
        // the first token's rescale multiplies an empty state; it never enters a product
        const float at = mprev == -INFINITY ? 1.0f : fast_expf(mprev - m);
        s[tt] = fast_expf(st - m);
        a[tt] = at;
        lprod *= at;
    }
    float suf = lprod;                                 // inclusive suffix product over lanes
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const float v = __shfl_down(suf, o, kWave);
        if (lane + o < kWave)
            suf *= v;
    }
    float pr = __shfl_down(suf, 1, kWave);
    if (lane == kWave - 1)
        pr = 1.0f;
    float ls = 0.0f;
    for (int tt = t1 - 1; tt >= t0; tt--) {
        if (!valid(tt)) {
            s[tt] = 0.0f;
            continue;
        }
        const float w = s[tt] * pr;
        s[tt] = w;
        ls += w;
        pr *= a[tt];
    }
    ls = wave_sum(ls);
    if (lane == 0)
        lsum[gw] = ls;
}

// lane = (token group tq, dim lane dl): 8 dims per lane, HD/8 dim lanes,
// 64/(HD/8) token groups; group tq takes tokens tq, tq+TG, ...
template <bool BF16, int HD>
__global__ __launch_bounds__(256) void k_attn_apply(const be42_kv_pool P, const int *__restrict__ sel,
                                                    const int *__restrict__ nsel, int sel_stride, int H,
                                                    int pages_per_split, const float *__restrict__ w,
                                                    int t_stride, float *__restrict__ part_o, int n_split)
{
    constexpr int D = 8, DL = HD / D, TG = kWave / DL;
    const int b = blockIdx.x, kvh = blockIdx.y, split = blockIdx.z;
    const int n_kv = P.n_kv, G = H / n_kv;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int ns = nsel[b];
    const int i0 = split * pages_per_split, i1 = min(ns, i0 + pages_per_split);
    const int tq = lane / DL, dl = lane % DL;
    const int *selb = sel + (size_t)b * sel_stride;
    for (int g = wave; g < G; g += 4) {
        const int h = kvh * G + g;
        const float *wh = w + ((size_t)b * H + h) * t_stride;
        float o[D];
#pragma unroll
        for (int j = 0; j < D; j++)
            o[j] = 0.0f;
        for (int i = i0; i < i1; i++) {
            const int phys = selb[i];
            const int nt = P.ntok[phys];
            for (int tk = tq; tk < nt; tk += TG) {
                const float wt = wh[i * kPg + tk];
                const size_t slot = ((size_t)phys * n_kv + kvh) * kPg + tk;
                float v[D];
                if constexpr (BF16) {
                    // V pages [kv head][dim][16 tokens]
                    const uint16_t *vc = (const uint16_t *)P.v + (slot / kPg) * (size_t)HD * kPg + slot % kPg;
#pragma unroll
                    for (int j = 0; j < D; j++)
                        v[j] = bf16_to_f32(vc[(size_t)(dl * D + j) * kPg]);
                } else {
                    load_row_f32(v, P.v, slot * HD + dl * D, D, false, P.v_scale[slot]);
                }
#pragma unroll
                for (int j = 0; j < D; j++)
                    o[j] = __fmaf_rn(wt, v[j], o[j]);
            }
        }
#pragma unroll
        for (int j = 0; j < D; j++) {
            float v = o[j];
#pragma unroll
            for (int x = DL; x < kWave; x <<= 1)
                v += __shfl_xor(v, x, kWave);
            o[j] = v;
        }
        if (tq == 0) {
            float *po = part_o + (((size_t)b * H + h) * n_split + split) * HD + dl * D;
#pragma unroll
            for (int j = 0; j < D; j++)
                po[j] = o[j];
        }
    }
}

__global__ void k_attn_combine(float *__restrict__ out, const float *__restrict__ part_o,
                               const float *__restrict__ lsum, int BH, int hd, int n_split)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)BH * hd)
        return;
    const size_t bh = i / hd, d = i % hd;
    float s = 0.0f;
    for (int sp = 0; sp < n_split; sp++)
        s += part_o[(bh * n_split + sp) * hd + d];
    const float l = lsum[bh];
    out[i] = l > 0.0f ? s * (1.0f / l) : s;
}

template <bool BF16, int HD>
static void launch_scores_apply(const be42_kv_pool &P, const float *q, const int *sel, const int *nsel,
                                int sel_stride, int B, int H, float scale, int pps, int n_split, float *scores,
                                float *aux, float *lsum, float *part, int t_stride, hipStream_t s)
{
    const dim3 grid(B, P.n_kv, n_split);
    hipLaunchKernelGGL((k_attn_scores<BF16, HD>), grid, dim3(256), 0, s, P, q, sel, nsel, sel_stride, H, scale,
                       pps, scores, t_stride);
    const int waves = B * H;
    hipLaunchKernelGGL(k_attn_weights, dim3((waves + 3) / 4), dim3(256), 0, s, P, sel, nsel, sel_stride, H, waves,
                       scores, aux, t_stride, lsum);
    hipLaunchKernelGGL((k_attn_apply<BF16, HD>), grid, dim3(256), 0, s, P, sel, nsel, sel_stride, H, pps, scores,
                       t_stride, part, n_split);
}


// Attention of routed queries: query b's selection is sel[b * sel_stride ..]
// (nsel[b] pages, in the router's output order).  With lim (and slots), query
// b sees the first lim[b] positions of slot slots[b]: its last visible page
// holds lim[b] - 16 (pages - 1) tokens.  The phases and the order of every
// sum are those of k_lsh_attn's selection-order path, so at the same WAVES
// an output equals k_lsh_attn's.  VW > WAVES: the values are summed in the
// layout of VW waves (attn_values_layout), so that the output equals that of
// a VW-wave launch (and of the split decode kernel) with fewer waves per
// workgroup.
template <bool BF16, int HD, int G, int WAVES, int UNR, int VW = WAVES>
__global__ __launch_bounds__(WAVES * 64) void k_attn_fused(const be42_kv_pool P, const float *__restrict__ q,
                                                           const int *__restrict__ sel,
                                                           const int *__restrict__ nsel, int sel_stride,
                                                           const int *__restrict__ slots,
                                                           const int *__restrict__ lim, int H, float scale,
                                                           float *__restrict__ out)
{
    static_assert(VW % WAVES == 0, "value layout");
    __shared__ AttnShared<HD, G, WAVES> S;
    __shared__ float red[VW * G * HD];
    S.red = red;
    const int b = blockIdx.x, kvh = blockIdx.y;
    const int ns = min(nsel[b], kFusedMaxPages);
    const int *selb = sel + (size_t)b * sel_stride;
    int last_ph = -1, last_nt = 0;
    if (lim) {
        const int lim_b = lim[b], n = (lim_b + kPg - 1) / kPg;
        last_ph = n > 0 ? P.page_table[(size_t)slots[b] * P.max_logical + n - 1] : -1;
        last_nt = lim_b - kPg * (n - 1);
    }
    attn_load_q(S, q, b, kvh, H);
    for (int i = threadIdx.x; i < ns; i += blockDim.x) {
        const int ph = selb[i];
        S.pphys[i] = ph;
        S.pnt[i] = ph == last_ph ? last_nt : P.ntok[ph];
    }
    __syncthreads();
    if (ns <= 0) {
        for (int i = threadIdx.x; i < G * HD; i += blockDim.x)
            out[((size_t)b * H + kvh * G) * HD + i] = 0.0f;
        return;
    }
    attn_scores<BF16, HD, G, WAVES, UNR>(P, S, kvh, ns, scale, 0, WAVES);
    __syncthreads();
    attn_weights(S, ns, nullptr);
    __syncthreads();
    if constexpr (VW == WAVES)
        attn_values<BF16, HD, G, WAVES, UNR>(P, S, b, kvh, ns, H, out, nullptr);
    else
        attn_values_layout<BF16, HD, G, WAVES, VW, UNR>(P, S, b, kvh, ns, H, out, nullptr);
}

// LSH route + sparse attention of one query in one kernel: workgroup
// (query b, KV head kvh) runs the router's phases 0-4 itself (every KV head
// of a query repeats them: a few KiB of hashes and centroids from L2), so
// the attention needs no second launch.  The selection is a subset of the
// anchors and the middle candidates, so while wave 0 runs the heap the
// other waves already compute the scores of all of them (up to kSetMax
// "set slots": at cap 64 two candidates more than the 62 heap slots); the
// weights and V then follow the heap's order through S.order.  With more
// candidates the scores wait for the heap.  The workgroup of KV head 0
// writes the selection to sel / nsel (when given).
// With lim, query b sees only the first lim[b] positions of its slot: the
// pages, the LSH index and the last page's token count it would have seen
// when position lim[b] - 1 was the newest (a prefill runs the queries of many
// positions after appending all of their K/V).
template <bool BF16, int HD, int G, int WAVES, int UNR, bool STAGE>
__global__ __launch_bounds__(WAVES * 64, 4) void k_lsh_attn(const be42_kv_pool P, const float *__restrict__ q,
                                                         const int *__restrict__ slots, const int *__restrict__ lim,
                                                         int H, int k_sel, int cap, float scale,
                                                         float *__restrict__ out, int *__restrict__ sel,
                                                         int *__restrict__ nsel, int sel_stride)
{
    static_assert(WAVES * 64 >= kRouteThreads, "the router needs 4 waves");
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ AttnShared<HD, G, WAVES> S;
    __shared__ int set_n;
    const RouteView V = route_view(smem, route_smem(HD, cap, P.max_logical));
    S.red = (float *)smem;   // the router's LDS, unused once the weights are computed
    const int b = blockIdx.x, kvh = blockIdx.y;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int layer = slots ? slots[b] : b;
    const int base = layer * P.max_logical;
    const int lim_b = lim ? lim[b] : 0;
    const int n = lim ? (lim_b + kPg - 1) / kPg : P.n_logical[layer];
    // tokens of a page: the view's last page holds lim - 16 (n - 1)
    const int last_ph = lim && n > 0 ? P.page_table[base + n - 1] : -1;
    const int last_nt = lim_b - kPg * (n - 1);
    auto page_nt = [&](int ph) { return ph == last_ph ? last_nt : P.ntok[ph]; };
    int *selb = sel && kvh == 0 ? sel + (size_t)b * sel_stride : nullptr;
    attn_load_q(S, q, b, kvh, H);

    if (n <= k_sel) {
        // dense: every page in logical order
        const int ns = n > 0 ? n : 0;
        for (int i = tid; i < ns; i += blockDim.x) {
            const int ph = P.page_table[base + i];
            S.pphys[i] = ph;
            S.pnt[i] = page_nt(ph);
            if (selb)
                selb[i] = ph;
        }
        if (tid == 0 && selb)
            nsel[b] = ns;
        __syncthreads();
        if (ns == 0) {
            for (int i = tid; i < G * HD; i += blockDim.x)
                out[((size_t)b * H + kvh * G) * HD + i] = 0.0f;
            return;
        }
        attn_scores<BF16, HD, G, WAVES, UNR>(P, S, kvh, ns, scale, 0, WAVES);
        __syncthreads();
        attn_weights(S, ns, nullptr);
        __syncthreads();
        attn_values<BF16, HD, G, WAVES, UNR>(P, S, b, kvh, ns, H, out, nullptr);
        return;
    }
    const int nidx = min(lim ? min(P.n_indexed[layer], lim_b / kPg) : P.n_indexed[layer], P.max_logical);
    // the waves the router leaves idle form the q split meanwhile
    route_prepare<STAGE>(P, q + (size_t)b * H * HD, base, n, nidx, H, cap, V, nullptr, nullptr, nullptr,
                         [&] { attn_q_store(S, tid - kRouteThreads, blockDim.x - kRouteThreads); });
    const int nm = route_middles(V);
    const int ns0 = V.mpt[cap + 1] != V.mpt[cap] ? 2 : 1;
    const int nset = ns0 + nm;
    const bool early = nset <= kSetMax;      // score every candidate while the heap runs
    if (early) {
        for (int i = tid; i < nset; i += blockDim.x) {
            const int ph = i == 0 ? V.mpt[cap] : (i < ns0 ? V.mpt[cap + 1] : V.mpt[i - ns0]);
            S.pphys[i] = ph;
            S.pnt[i] = page_nt(ph);
        }
    }
    __syncthreads();
    if (wave == 0) {
        const int ns = route_select(k_sel, cap, V, selb, S.order);
        if (lane == 0) {
            set_n = ns;
            if (selb)
                nsel[b] = ns;
        }
    } else if (early) {
        attn_scores<BF16, HD, G, WAVES, UNR, true>(P, S, kvh, nset, scale, 1, WAVES - 1);
    }
    __syncthreads();
    const int ns = set_n;
    if (!early) {
        // too many candidates: score only the selection, in selection order
        for (int i = tid; i < ns; i += blockDim.x) {
            const int slot = S.order[i];
            const int ph = slot == 0 ? V.mpt[cap] : (slot < ns0 ? V.mpt[cap + 1] : V.mpt[slot - ns0]);
            S.pphys[i] = ph;
            S.pnt[i] = page_nt(ph);
        }
        __syncthreads();
        attn_scores<BF16, HD, G, WAVES, UNR, true>(P, S, kvh, ns, scale, 0, WAVES);
        __syncthreads();
    }
    attn_weights(S, ns, early ? S.order : nullptr);
    __syncthreads();
    attn_values<BF16, HD, G, WAVES, UNR>(P, S, b, kvh, ns, H, out, early ? S.order : nullptr);
}

// Route + attention of few queries over more CUs: the NS workgroups
// (blockIdx.z) of a (query, KV head) pair each run the router and the heap
// (as k_lsh_attn does), score 1/NS of the pages, exchange the scores, compute
// every weight, and take 16/NS of the 16 value waves of k_lsh_attn's 16-wave
// layout; the last workgroup to finish adds the 16 wave partials in wave
// order.  Every page's scores, every weight and every wave partial are
// computed exactly as in that layout, so the output is the same to the bit.
// The exchange goes through device-scope loads and stores; the NS workgroups
// meet at one counter barrier (the last to arrive resets the count and flips
// a flag the others wait on, so nothing is reset between launches).  A wait
// that does not end within ~kSplitSpinMax polls (workgroups of a pair not
// resident together) gives up and scores every page itself, so the result
// never depends on the others.
constexpr int kSplitMaxPairs = 128;           // (query, KV head) pairs of a split launch
constexpr int kSplitWaves = 16;                // the value layout a split launch reproduces
constexpr unsigned kSplitSpinMax = 1u << 14;
constexpr unsigned kSplitSpinCap = 1u << 20;   // largest poll limit a caller may set
struct SplitSync {
    unsigned arrive, flag, done, pad[13];      // one 64-byte line per pair
};
__device__ SplitSync g_split_sync[kSplitMaxPairs];
__device__ float g_split_sc[kSplitMaxPairs][4][kSetMax * 17];          // scores, AttnShared::sc layout
__device__ float g_split_o[kSplitMaxPairs][kSplitWaves][4 * 128];       // wave partials [g][dim]
__device__ unsigned g_split_seq[kSplitMaxPairs];                         // pairs of a query done (digit output)
// error word of split launches whose caller gave none (be42_lsh_attention):
// 4 = a wait among a workgroup's own waves gave up (its output is invalid);
// read and cleared by be42_lsh_attention_status
__device__ int g_attn_err;

__device__ __forceinline__ unsigned ld_dev_u(const unsigned *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev_u(unsigned *p, unsigned v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev_f(const float *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev_f(float *p, float v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int HD, int G, bool STAGE>
__global__ __launch_bounds__(kSplitWaves * 64) void k_lsh_attn_split(const be42_kv_pool P, const float *__restrict__ q,
                                                                    const int *__restrict__ slots,
                                                                    const int *__restrict__ lim, int H, int k_sel,
                                                                    int cap, float scale, float *__restrict__ out,
                                                                    int *__restrict__ sel, int *__restrict__ nsel,
                                                                    int sel_stride, unsigned spin_max,
                                                                    uint8_t *__restrict__ dig, int Kp, int dig_fp8,
                                                                    int *__restrict__ err)
{
    constexpr int WAVES = kSplitWaves;
    static_assert(G <= 4 && HD <= 128, "exchange buffers");
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ AttnShared<HD, G, WAVES> S;
    __shared__ int set_n, last, alone, xcnt;
    __shared__ unsigned sense;
    const RouteView V = route_view(smem, route_smem(HD, cap, P.max_logical));
    S.red = (float *)smem;
    const int b = blockIdx.x, kvh = blockIdx.y, z = blockIdx.z, NS = gridDim.z;
    const int pair = b * gridDim.y + kvh;
    SplitSync *sy = &g_split_sync[pair];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // the flag flips only once every workgroup of the pair has arrived, so
    // each reads it before that
    if (tid == 0) {
        sense = ld_dev_u(&sy->flag);
        xcnt = 0;
    }
    const int layer = slots ? slots[b] : b;
    const int base = layer * P.max_logical;
    const int lim_b = lim ? lim[b] : 0;
    const int n = lim ? (lim_b + kPg - 1) / kPg : P.n_logical[layer];
    const int last_ph = lim && n > 0 ? P.page_table[base + n - 1] : -1;
    const int last_nt = lim_b - kPg * (n - 1);
    auto page_nt = [&](int ph) { return ph == last_ph ? last_nt : P.ntok[ph]; };
    int *selb = sel && kvh == 0 && z == 0 ? sel + (size_t)b * sel_stride : nullptr;
    if (n <= k_sel) {
        // dense: the first workgroup of the pair alone, as k_lsh_attn
        if (z != 0)
            return;
        attn_load_q(S, q, b, kvh, H);
        const int ns = n > 0 ? n : 0;
        for (int i = tid; i < ns; i += blockDim.x) {
            const int ph = P.page_table[base + i];
            S.pphys[i] = ph;
            S.pnt[i] = page_nt(ph);
            if (selb)
                selb[i] = ph;
        }
        if (tid == 0 && selb)
            nsel[b] = ns;
        __syncthreads();
        if (ns == 0) {
            for (int i = tid; i < G * HD; i += blockDim.x)
                out[((size_t)b * H + kvh * G) * HD + i] = 0.0f;
            return;
        }
        attn_scores<true, HD, G, WAVES, 8>(P, S, kvh, ns, scale, 0, WAVES);
        __syncthreads();
        attn_weights(S, ns, nullptr);
        __syncthreads();
        attn_values<true, HD, G, WAVES, 8>(P, S, b, kvh, ns, H, out, nullptr);
        return;
    }
    attn_load_q(S, q, b, kvh, H);
    const int nidx = min(lim ? min(P.n_indexed[layer], lim_b / kPg) : P.n_indexed[layer], P.max_logical);
    // the waves the router leaves idle form the q split meanwhile
    route_prepare<STAGE>(P, q + (size_t)b * H * HD, base, n, nidx, H, cap, V, nullptr, nullptr, nullptr,
                         [&] { attn_q_store(S, tid - kRouteThreads, blockDim.x - kRouteThreads); });
    const int nm = route_middles(V);
    const int ns0 = V.mpt[cap + 1] != V.mpt[cap] ? 2 : 1;
    const int nset = ns0 + nm;
    const bool early = nset <= kSetMax;
    if (early) {
        for (int i = tid; i < nset; i += blockDim.x) {
            const int ph = i == 0 ? V.mpt[cap] : (i < ns0 ? V.mpt[cap + 1] : V.mpt[i - ns0]);
            S.pphys[i] = ph;
            S.pnt[i] = page_nt(ph);
        }
    }
    __syncthreads();
    // this workgroup's share of the scored slots: [lo, hi) of the set slots
    // (early) or of the selection (after the heap)
    int lo = z * nset / NS, hi = (z + 1) * nset / NS;
    float *xs = &g_split_sc[pair][0][0];
    // Publish the scores of [lo, hi), meet the pair's other workgroups and
    // take their scores of [0, E) (or, after a wait that did not end, score
    // every page here): run by waves w0 .. WAVES-1, which sync() joins.
    auto exchange = [&](int w0, int E, auto &&sync) {
        const int t = tid - w0 * kWave, nt = (WAVES - w0) * kWave;
        const int nsh = (hi - lo) * kPg;
        for (int i = t; i < G * nsh; i += nt) {
            const int g = i / nsh, r = lo * kPg + i % nsh;
            const int at = (r / kPg) * 17 + r % kPg;
            st_dev_f(xs + g * (kSetMax * 17) + at, S.sc[g][at]);
        }
        wait_vmcnt<0>();
        sync();
        if (t == 0) {
            const unsigned s0 = sense;
            int gave_up = 0;
            if (__hip_atomic_fetch_add(&sy->arrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                (unsigned)NS - 1) {
                st_dev_u(&sy->arrive, 0u);
                st_dev_u(&sy->flag, s0 ^ 1u);
            } else {
                unsigned spins = 0;
                while (ld_dev_u(&sy->flag) == s0) {
                    __builtin_amdgcn_s_sleep(1);
                    if (++spins > spin_max) {
                        gave_up = 1;
                        break;
                    }
                }
            }
            alone = gave_up;
        }
        sync();
        if (alone) {
            attn_scores_mfma<HD, G, WAVES, 1, true>(P, S, kvh, E, scale, w0, WAVES - w0, 0);
        } else {
            for (int i = t; i < G * E * kPg; i += nt) {
                const int g = i / (E * kPg), r = i % (E * kPg), sl = r / kPg;
                const int at = sl * 17 + r % kPg;
                if (sl < lo || sl >= hi)
                    S.sc[g][at] = ld_dev_f(xs + g * (kSetMax * 17) + at);
            }
        }
    };
    if (wave == 0) {
        const int ns = route_select(k_sel, cap, V, selb, S.order);
        if (lane == 0) {
            set_n = ns;
            if (selb)
                nsel[b] = ns;
        }
    } else if (early) {
        // the set's scores do not depend on the heap: waves 1.. score this
        // share, exchange it and take the others' while wave 0 runs the heap,
        // joined by a counter in LDS (a block barrier would wait for wave 0)
        int target = 0;
        auto sync15 = [&] {
            target += WAVES - 1;
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (lane == 0)
                __hip_atomic_fetch_add(&xcnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            // every wave of the group gets here within its own bounded work
            // (wave 1's cross-workgroup wait polls at most kSplitSpinCap
            // times), so this bound is only a guard: reaching it means the
            // scores may be incomplete, which the error word reports
            unsigned spins = 0;
            while (__hip_atomic_load(&xcnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target) {
                __builtin_amdgcn_s_sleep(1);
                if (++spins > (kSplitSpinCap << 2)) {
                    if (lane == 0)
                        __hip_atomic_store(err, 4, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
            }
            asm volatile("" ::: "memory");
        };
        attn_scores_mfma<HD, G, WAVES, 1, true>(P, S, kvh, hi, scale, 1, WAVES - 1, lo);
        sync15();      // every wave's scores are in LDS before any is published
        exchange(1, nset, sync15);
    }
    __syncthreads();
    const int ns = set_n;
    if (!early) {
        for (int i = tid; i < ns; i += blockDim.x) {
            const int slot = S.order[i];
            const int ph = slot == 0 ? V.mpt[cap] : (slot < ns0 ? V.mpt[cap + 1] : V.mpt[slot - ns0]);
            S.pphys[i] = ph;
            S.pnt[i] = page_nt(ph);
        }
        __syncthreads();
        lo = z * ns / NS;
        hi = (z + 1) * ns / NS;
        attn_scores_mfma<HD, G, WAVES, 1, true>(P, S, kvh, hi, scale, 0, WAVES, lo);
        __syncthreads();
        exchange(0, ns, [] { __syncthreads(); });
        __syncthreads();
    }
    attn_weights(S, ns, early ? S.order : nullptr);
    __syncthreads();
    // value waves z * per .. z * per + per - 1 of the 16-wave layout
    const int per = WAVES / NS;
    if (wave < per) {
        float *dst = &g_split_o[pair][z * per + wave][0];
        attn_values_mfma_wave<HD, G, WAVES, 4>(P, S, kvh, ns, early ? S.order : nullptr, z * per + wave,
                                               [dst](int i, float v) { st_dev_f(dst + i, v); });
    }
    wait_vmcnt<0>();
    __syncthreads();
    if (tid == 0) {
        const unsigned old = __hip_atomic_fetch_add(&sy->done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = old == (unsigned)NS - 1;
        if (last)
            st_dev_u(&sy->done, 0u);
    }
    __syncthreads();
    if (!last)
        return;
    // out = (sum of the 16 wave partials in wave order) * (1 / l)
    for (int i = tid; i < G * HD; i += blockDim.x) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; w++)
            v += ld_dev_f(&g_split_o[pair][w][i]);
        const float l = S.lsh[i / HD];
        const float o = l > 0.0f ? v * (1.0f / l) : v;
        if (dig)
            st_dev_f(out + ((size_t)b * H + kvh * G) * HD + i, o);
        else
            out[((size_t)b * H + kvh * G) * HD + i] = o;
    }
    if (!dig)
        return;
    // the last of the query's KV-head pairs to finish writes the query's
    // output row as the next GEMV's digit planes, as xdig_prepare does
    wait_vmcnt<0>();
    __syncthreads();
    if (tid == 0) {
        const unsigned old = __hip_atomic_fetch_add(&g_split_seq[b], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = old == (unsigned)gridDim.y - 1;
        if (last)
            __hip_atomic_store(&g_split_seq[b], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last)
        return;
    const int K = H * HD, B = gridDim.x;
    const float *row = out + (size_t)b * K;
    float m = 0.0f;
    for (int i4 = tid; 4 * i4 < K; i4 += blockDim.x)
#pragma unroll
        for (int e = 0; e < 4; e++)
            m = fmaxf(m, fabsf(ld_dev_f(row + 4 * i4 + e)));
    m = wave_max(m);
    __syncthreads();
    if (lane == 0)
        S.red[wave] = m;
    __syncthreads();
    float amax = 0.0f;
#pragma unroll
    for (int w = 0; w < WAVES; w++)
        amax = fmaxf(amax, S.red[w]);
    auto put = [&](auto f8) {
        constexpr bool F8 = decltype(f8)::value;
        const float sc = digit_scale<F8>(amax);
        if (tid == 0)
            xdig_scales(dig, K, B, F8)[b] = sc;
        for (int i4 = tid; 4 * i4 < Kp; i4 += blockDim.x) {
            const int k0 = 4 * i4;
            float xe[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (k0 < K)
#pragma unroll
                for (int e = 0; e < 4; e++)
                    xe[e] = ld_dev_f(row + k0 + e);
            store_digit_words<F8>(xe, sc, dig, B, Kp, b, k0);
        }
    };
    if (dig_fp8)
        put(std::true_type());
    else
        put(std::false_type());
}

// 16 waves when the grid is small (more loads in flight per workgroup), 8
// waves once there are enough workgroups to fill the chip.
// slots / lim: as k_attn_fused (lim null: every slot's whole cache).
// wide16 keeps the 16-wave layout for any grid (k_lsh_attn's wide16), from
// 8-wave workgroups that sum the values in that layout.
struct FusedOpt {
    const int *slots = nullptr, *lim = nullptr;
    bool wide16 = false;
};

template <bool BF16, int HD, int G>
static void launch_fused_g(const be42_kv_pool &P, const float *q, const int *sel, const int *nsel, int sel_stride,
                           int B, int H, float scale, float *out, const FusedOpt &o, hipStream_t s)
{
    const dim3 grid(B, P.n_kv);
    if (o.wide16) {
        // the 16-wave value layout from 8-wave workgroups (two per CU)
        hipLaunchKernelGGL((k_attn_fused<BF16, HD, G, 8, 8, 16>), grid, dim3(512), 0, s, P, q, sel, nsel, sel_stride,
                           o.slots, o.lim, H, scale, out);
        return;
    }
    if ((long)B * P.n_kv < 512)
        hipLaunchKernelGGL((k_attn_fused<BF16, HD, G, 16, 8>), grid, dim3(1024), 0, s, P, q, sel, nsel, sel_stride,
                           o.slots, o.lim, H, scale, out);
    else
        hipLaunchKernelGGL((k_attn_fused<BF16, HD, G, 8, 8>), grid, dim3(512), 0, s, P, q, sel, nsel, sel_stride,
                           o.slots, o.lim, H, scale, out);
}

template <bool BF16, int HD>
static bool launch_fused_hd(const be42_kv_pool &P, const float *q, const int *sel, const int *nsel, int sel_stride,
                            int B, int H, float scale, float *out, const FusedOpt &o, hipStream_t s)
{
    switch (H / P.n_kv) {
    case 1: launch_fused_g<BF16, HD, 1>(P, q, sel, nsel, sel_stride, B, H, scale, out, o, s); return true;
    case 2: launch_fused_g<BF16, HD, 2>(P, q, sel, nsel, sel_stride, B, H, scale, out, o, s); return true;
    case 3: launch_fused_g<BF16, HD, 3>(P, q, sel, nsel, sel_stride, B, H, scale, out, o, s); return true;
    case 4: launch_fused_g<BF16, HD, 4>(P, q, sel, nsel, sel_stride, B, H, scale, out, o, s); return true;
    default: return false;
    }
}

static bool launch_fused(const be42_kv_pool &P, const float *q, const int *sel, const int *nsel, int sel_stride, int B,
                         int H, float scale, float *out, hipStream_t s, const FusedOpt &o = FusedOpt())
{
    const bool bf16 = P.kind == BE42_KV_BF16;
    if (P.head_dim == 128)
        return bf16 ? launch_fused_hd<true, 128>(P, q, sel, nsel, sel_stride, B, H, scale, out, o, s)
                    : launch_fused_hd<false, 128>(P, q, sel, nsel, sel_stride, B, H, scale, out, o, s);
    if (P.head_dim == 64)
        return bf16 ? launch_fused_hd<true, 64>(P, q, sel, nsel, sel_stride, B, H, scale, out, o, s)
                    : launch_fused_hd<false, 64>(P, q, sel, nsel, sel_stride, B, H, scale, out, o, s);
    return false;
}

// Dynamic LDS of k_lsh_attn: the router's layout, which the cross-wave
// reduction of o reuses afterwards.
template <int HD, int G, int WAVES>
static size_t lsh_attn_lds(const RouteSmem &L)
{
    return std::max((size_t)L.bytes, (size_t)WAVES * G * HD * sizeof(float));
}

// lim: per-query visible positions (NULL: the slot's whole cache).  The
// grid shape picks 16 or 8 waves; wide16 keeps 16 for any grid, so that a
// query is computed exactly as it is in a small (decode-sized) launch.
struct LshAttnOpt {
    const int *lim = nullptr;
    bool wide16 = false;
    // optional: the output rows as GEMV digit planes (xdig_prepare's layout
    // for k = H * head_dim), written by split launches; dig_done tells
    // whether this launch wrote them
    void *dig = nullptr;
    bool dig_fp8 = false;
    bool *dig_done = nullptr;
    int *err = nullptr;   // device error word of split launches (else g_attn_err)
};

// BE42_ATTN_SPLIT=0 keeps every launch at one workgroup per (query, KV head)
static bool split_enabled()
{
    static const bool on = [] {
        const char *e = getenv("BE42_ATTN_SPLIT");
        return !(e && e[0] == '0');
    }();
    return on;
}

// polls before a workgroup of a split pair stops waiting for the others and
// scores every page itself; BE42_ATTN_SPLIT_SPIN overrides it (read at every
// launch: the tests set 0 to run that path)
static unsigned split_spin_max()
{
    const char *e = getenv("BE42_ATTN_SPLIT_SPIN");
    const unsigned long v = e ? strtoul(e, nullptr, 10) : kSplitSpinMax;
    return v < kSplitSpinCap ? (unsigned)v : kSplitSpinCap;
}

// device address of g_attn_err (the current device's copy)
static int *attn_err_default()
{
    static int *p[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return nullptr;
    if (!p[dev] && hipGetSymbolAddress((void **)&p[dev], HIP_SYMBOL(g_attn_err)) != hipSuccess)
        p[dev] = nullptr;
    return p[dev];
}

template <bool BF16, int HD, int G, bool STAGE>
static int launch_lsh_attn_s(const be42_kv_pool &P, const float *q, const int *slots, int B, int H, int k_sel,
                             int cap, float scale, float *out, int *sel, int *nsel, int sel_stride,
                             const RouteSmem &L, const LshAttnOpt &o, hipStream_t s)
{
    if constexpr (BF16 && (HD == 64 || HD == 128)) {
        // few pairs: NS workgroups per pair, NS * pairs <= 256 (one per CU);
        // at 2 per pair the exchange costs more than it saves (measured)
        const long pairs = (long)B * P.n_kv;
        if (pairs <= 64 && split_enabled()) {
            int ns = kSplitWaves;
            while (ns > 4 && pairs * ns > 256)
                ns >>= 1;
            const size_t lds = lsh_attn_lds<HD, G, kSplitWaves>(L);
            if (lds > 65536)
                BE42_HIP(hipFuncSetAttribute((const void *)k_lsh_attn_split<HD, G, STAGE>,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
            const int Kp = o.dig ? (int)xdig_kp(H * HD, o.dig_fp8) : 0;
            int *err = o.err ? o.err : attn_err_default();
            BE42_CHECK(err, "lsh attention: no address for the error word");
            hipLaunchKernelGGL((k_lsh_attn_split<HD, G, STAGE>), dim3(B, P.n_kv, ns), dim3(kSplitWaves * 64), lds, s,
                               P, q, slots, o.lim, H, k_sel, cap, scale, out, sel, nsel, sel_stride, split_spin_max(),
                               (uint8_t *)o.dig, Kp, (int)o.dig_fp8, err);
            if (o.dig_done)
                *o.dig_done = o.dig != nullptr;
            BE42_LAUNCH_CHECK();
            return BE42_OK;
        }
    }
    const dim3 grid(B, P.n_kv);
    if ((long)B * P.n_kv < 512 || o.wide16) {
        const size_t lds = lsh_attn_lds<HD, G, 16>(L);
        if (lds > 65536)
            BE42_HIP(hipFuncSetAttribute((const void *)k_lsh_attn<BF16, HD, G, 16, 8, STAGE>,
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        hipLaunchKernelGGL((k_lsh_attn<BF16, HD, G, 16, 8, STAGE>), grid, dim3(1024), lds, s, P, q, slots, o.lim, H,
                           k_sel, cap, scale, out, sel, nsel, sel_stride);
    } else {
        const size_t lds = lsh_attn_lds<HD, G, 8>(L);
        if (lds > 65536)
            BE42_HIP(hipFuncSetAttribute((const void *)k_lsh_attn<BF16, HD, G, 8, 8, STAGE>,
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        hipLaunchKernelGGL((k_lsh_attn<BF16, HD, G, 8, 8, STAGE>), grid, dim3(512), lds, s, P, q, slots, o.lim, H,
                           k_sel, cap, scale, out, sel, nsel, sel_stride);
    }
    BE42_LAUNCH_CHECK();
    return BE42_OK;
}

template <bool BF16, int HD, int G>
static int launch_lsh_attn_g(const be42_kv_pool &P, const float *q, const int *slots, int B, int H, int k_sel,
                             int cap, float scale, float *out, int *sel, int *nsel, int sel_stride,
                             const LshAttnOpt &o, hipStream_t s)
{
    const RouteSmem L = route_smem(HD, cap, P.max_logical);
    if (L.stage)
        return launch_lsh_attn_s<BF16, HD, G, true>(P, q, slots, B, H, k_sel, cap, scale, out, sel, nsel, sel_stride,
                                                    L, o, s);
    return launch_lsh_attn_s<BF16, HD, G, false>(P, q, slots, B, H, k_sel, cap, scale, out, sel, nsel, sel_stride, L,
                                                 o, s);
}

template <bool BF16, int HD>
static int launch_lsh_attn_hd(const be42_kv_pool &P, const float *q, const int *slots, int B, int H, int k_sel,
                              int cap, float scale, float *out, int *sel, int *nsel, int sel_stride,
                              const LshAttnOpt &o, hipStream_t s)
{
    switch (H / P.n_kv) {
    case 1: return launch_lsh_attn_g<BF16, HD, 1>(P, q, slots, B, H, k_sel, cap, scale, out, sel, nsel, sel_stride, o, s);
    case 2: return launch_lsh_attn_g<BF16, HD, 2>(P, q, slots, B, H, k_sel, cap, scale, out, sel, nsel, sel_stride, o, s);
    case 3: return launch_lsh_attn_g<BF16, HD, 3>(P, q, slots, B, H, k_sel, cap, scale, out, sel, nsel, sel_stride, o, s);
    default: return launch_lsh_attn_g<BF16, HD, 4>(P, q, slots, B, H, k_sel, cap, scale, out, sel, nsel, sel_stride, o, s);
    }
}

static int launch_lsh_attn(const be42_kv_pool &P, const float *q, const int *slots, int B, int H, int k_sel, int cap,
                           float scale, float *out, int *sel, int *nsel, int sel_stride, const LshAttnOpt &o,
                           hipStream_t s)
{
    const bool bf16 = P.kind == BE42_KV_BF16;
    if (P.head_dim == 128)
        return bf16 ? launch_lsh_attn_hd<true, 128>(P, q, slots, B, H, k_sel, cap, scale, out, sel, nsel, sel_stride,
                                                    o, s)
                    : launch_lsh_attn_hd<false, 128>(P, q, slots, B, H, k_sel, cap, scale, out, sel, nsel,
                                                     sel_stride, o, s);
    return bf16 ? launch_lsh_attn_hd<true, 64>(P, q, slots, B, H, k_sel, cap, scale, out, sel, nsel, sel_stride, o, s)
                : launch_lsh_attn_hd<false, 64>(P, q, slots, B, H, k_sel, cap, scale, out, sel, nsel, sel_stride, o,
                                                s);
}

}  // namespace be42

using namespace be42;

// Workspace: scores/weights and a_t [B][H][t_stride], l [B][H], partial o
// [B][H][n_split][hd].
extern "C" size_t be42_attn_workspace_bytes(int n_queries, int n_heads, int head_dim, int max_sel, int n_split)
{
    const size_t bh = (size_t)n_queries * n_heads;
    const size_t t_stride = (size_t)max_sel * kPg;
    return bh * t_stride * 4 * 2 + bh * 4 + bh * (size_t)n_split * head_dim * 4 + 1024;
}

extern "C" int be42_paged_attention(const be42_kv_pool *pool, const float *q, int n_queries, int n_heads,
                                    const int *sel, const int *n_sel, int sel_stride, int max_sel, float scale,
                                    float *out, int n_split, void *workspace_ptr, size_t workspace_bytes,
                                    void *stream)
{
    BE42_CHECK(pool && q && sel && n_sel && out, "be42_paged_attention: null pointer");
    const be42_kv_pool &P = *pool;
    BE42_CHECK(n_heads > 0 && n_heads % P.n_kv == 0, "be42_paged_attention: %d heads not a multiple of %d kv heads",
               n_heads, P.n_kv);
    BE42_CHECK(P.head_dim == 64 || P.head_dim == 128 || P.head_dim == 256,
               "be42_paged_attention: head_dim %d not supported (64, 128, 256)", P.head_dim);
    BE42_CHECK(max_sel > 0 && max_sel <= sel_stride, "be42_paged_attention: bad max_sel %d", max_sel);
    if (n_queries <= 0)
        return BE42_OK;
    hipStream_t s0 = as_stream(stream);
    // up to 64 pages per query and no split requested: one fused kernel
    if (max_sel <= kFusedMaxPages && n_split <= 1 &&
        launch_fused(P, q, sel, n_sel, sel_stride, n_queries, n_heads, scale, out, s0)) {
        BE42_LAUNCH_CHECK();
        return BE42_OK;
    }
    if (n_split < 1)
        n_split = 1;
    if (n_split > max_sel)
        n_split = max_sel;
    hipStream_t s = as_stream(stream);
    const size_t need = be42_attn_workspace_bytes(n_queries, n_heads, P.head_dim, max_sel, n_split);
    void *ws = workspace_ptr;
    if (!ws) {
        ws = workspace(need, s);
        if (!ws)
            return BE42_ENOMEM;
    } else {
        BE42_CHECK(workspace_bytes >= need, "be42_paged_attention: workspace %zu < %zu bytes", workspace_bytes, need);
    }
    const size_t bh = (size_t)n_queries * n_heads;
    const int t_stride = max_sel * kPg;
    float *scores = (float *)ws;
    float *aux = scores + bh * t_stride;
    float *lsum = aux + bh * t_stride;
    float *part = lsum + bh;
    const int pps = (max_sel + n_split - 1) / n_split;
    const bool bf16 = P.kind == BE42_KV_BF16;
    switch (P.head_dim) {
    case 64:
        if (bf16) launch_scores_apply<true, 64>(P, q, sel, n_sel, sel_stride, n_queries, n_heads, scale, pps, n_split, scores, aux, lsum, part, t_stride, s);
        else launch_scores_apply<false, 64>(P, q, sel, n_sel, sel_stride, n_queries, n_heads, scale, pps, n_split, scores, aux, lsum, part, t_stride, s);
        break;
    case 128:
        if (bf16) launch_scores_apply<true, 128>(P, q, sel, n_sel, sel_stride, n_queries, n_heads, scale, pps, n_split, scores, aux, lsum, part, t_stride, s);
        else launch_scores_apply<false, 128>(P, q, sel, n_sel, sel_stride, n_queries, n_heads, scale, pps, n_split, scores, aux, lsum, part, t_stride, s);
        break;
    default:
        if (bf16) launch_scores_apply<true, 256>(P, q, sel, n_sel, sel_stride, n_queries, n_heads, scale, pps, n_split, scores, aux, lsum, part, t_stride, s);
        else launch_scores_apply<false, 256>(P, q, sel, n_sel, sel_stride, n_queries, n_heads, scale, pps, n_split, scores, aux, lsum, part, t_stride, s);
        break;
    }
    BE42_LAUNCH_CHECK();
    const size_t tot = bh * P.head_dim;
    hipLaunchKernelGGL(k_attn_combine, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, s, out, part, lsum,
                       (int)bh, P.head_dim, n_split);
    BE42_LAUNCH_CHECK();
    return BE42_OK;
}

extern "C" int be42_lsh_attention_status(void *stream)
{
    BE42_HIP(hipStreamSynchronize(as_stream(stream)));
    int *p = attn_err_default();
    BE42_CHECK(p, "be42_lsh_attention_status: no address for the error word");
    int v = 0;
    BE42_HIP(hipMemcpy(&v, p, sizeof v, hipMemcpyDeviceToHost));
    if (v) {
        const int zero = 0;
        BE42_HIP(hipMemcpy(p, &zero, sizeof zero, hipMemcpyHostToDevice));
    }
    BE42_CHECK(v == 0, "be42_lsh_attention: a wait inside a split launch gave up (code %d); the output of a launch "
                       "since the last check is invalid", v);
    return BE42_OK;
}

extern "C" int be42_lsh_attention(const be42_kv_pool *pool, const float *q, const int *slots, int n_queries,
                                  int n_heads, int k_sel, int cand_cap, float scale, float *out, int *sel,
                                  int *n_sel, int sel_stride, void *stream)
{
    BE42_CHECK(pool && q && out, "be42_lsh_attention: null pointer");
    const be42_kv_pool &P = *pool;
    BE42_CHECK(k_sel > 0 && k_sel <= kFusedMaxPages && cand_cap > 0 && cand_cap <= kMaxCand,
               "be42_lsh_attention: k %d (1..%d), cap %d (1..%d)", k_sel, kFusedMaxPages, cand_cap, kMaxCand);
    BE42_CHECK(n_heads > 0 && n_heads % P.n_kv == 0 && n_heads / P.n_kv <= 4,
               "be42_lsh_attention: %d heads over %d kv heads (groups of 1..4)", n_heads, P.n_kv);
    BE42_CHECK(P.head_dim == 64 || P.head_dim == 128, "be42_lsh_attention: head_dim %d (64 or 128)", P.head_dim);
    BE42_CHECK((sel == nullptr) == (n_sel == nullptr), "be42_lsh_attention: sel and n_sel go together");
    BE42_CHECK(!sel || (sel_stride >= k_sel && sel_stride >= kHeapMax + 2),
               "be42_lsh_attention: sel_stride %d must be >= max(k, 64)", sel_stride);
    if (n_queries <= 0)
        return BE42_OK;
    hipStream_t s = as_stream(stream);
    if ((long)n_queries * P.n_kv >= 1024) {
        // Enough workgroups to fill the chip: the router's latency is better
        // spent once per query in its own launch than once per KV head in
        // the attention's workgroups (measured on MI355X: at 1024 (query, KV
        // head) pairs 2% faster, at 512 15% slower).  The selection
        // goes through the library workspace when the caller wants none.
        int *ws_sel = sel, *ws_n = n_sel, stride = sel_stride;
        if (!sel) {
            stride = std::max(k_sel, kHeapMax + 2);
            int *w = (int *)workspace((size_t)n_queries * (stride + 1) * sizeof(int), s);
            if (!w)
                return BE42_ENOMEM;
            ws_sel = w;
            ws_n = w + (size_t)n_queries * stride;
        }
        const int rc = be42_lsh_route(pool, q, slots, n_queries, n_heads, k_sel, cand_cap, ws_sel, ws_n, stride,
                                      nullptr, nullptr, nullptr, stream);
        if (rc)
            return rc;
        // <= 64 pages, no split: the fused attention kernel, which takes no workspace
        return be42_paged_attention(pool, q, n_queries, n_heads, ws_sel, ws_n, stride, k_sel, scale, out, 1, nullptr,
                                    0, stream);
    }
    return launch_lsh_attn(P, q, slots, n_queries, n_heads, k_sel, cand_cap, scale, out, sel, n_sel, sel_stride,
                           LshAttnOpt(), s);
}

namespace be42 {

// Prefill attention: query b of slot slots[b] sees the first lim[b]
// positions, computed exactly as a one-query decode launch computes it.
// be42_lsh_attention for the decoder's unfused steps: when the launch is a
// split one, it also writes the output rows as the o projection's digit
// planes (xdig, xdig_prepare's layout) and sets *done.
int lsh_attention_digits(const be42_kv_pool &P, const float *q, const int *slots, int n_queries, int n_heads,
                         int k_sel, int cand_cap, float scale, float *out, int *sel, int *n_sel, int sel_stride,
                         void *xdig, bool fp8, bool *done, int *err, hipStream_t s)
{
    *done = false;
    if ((long)n_queries * P.n_kv >= 1024)
        return be42_lsh_attention(&P, q, slots, n_queries, n_heads, k_sel, cand_cap, scale, out, sel, n_sel,
                                  sel_stride, s);
    BE42_CHECK(k_sel > 0 && k_sel <= kFusedMaxPages && cand_cap > 0 && cand_cap <= kMaxCand &&
                   n_heads % P.n_kv == 0 && n_heads / P.n_kv <= 4 && (P.head_dim == 64 || P.head_dim == 128),
               "lsh_attention_digits: unsupported shape");
    if (n_queries <= 0)
        return BE42_OK;
    LshAttnOpt o;
    o.dig = xdig;
    o.dig_fp8 = fp8;
    o.dig_done = done;
    o.err = err;
    return launch_lsh_attn(P, q, slots, n_queries, n_heads, k_sel, cand_cap, scale, out, sel, n_sel, sel_stride, o,
                           s);
}

// The router runs once per query (k_route), then the attention of every
// (query, KV head) pair over that selection (k_attn_fused at 16 waves, the
// layout a one-query decode launch sums in); k_lsh_attn would repeat the
// router in each KV head's workgroup.
int lsh_attention_prefix(const be42_kv_pool &P, const float *q, const int *slots, const int *lim, int n_queries,
                         int n_heads, int k_sel, int cand_cap, float scale, float *out, int *sel, int *nsel,
                         int sel_stride, hipStream_t s)
{
    BE42_CHECK(k_sel > 0 && k_sel <= kFusedMaxPages && cand_cap > 0 && cand_cap <= kMaxCand &&
                   n_heads % P.n_kv == 0 && n_heads / P.n_kv <= 4 && (P.head_dim == 64 || P.head_dim == 128),
               "prefill attention: unsupported shape (k %d, cap %d, %d heads / %d kv, head_dim %d)", k_sel, cand_cap,
               n_heads, P.n_kv, P.head_dim);
    BE42_CHECK(slots && lim && sel && nsel && sel_stride >= prefix_sel_stride(k_sel),
               "prefill attention: needs slots, lim and a selection workspace of stride >= %d (got %d)",
               prefix_sel_stride(k_sel), sel_stride);
    if (n_queries <= 0)
        return BE42_OK;
    const int rc = launch_route(P, q, slots, lim, n_queries, n_heads, k_sel, cand_cap, sel, nsel, sel_stride, nullptr,
                                nullptr, nullptr, s);
    if (rc != BE42_OK)
        return rc;
    FusedOpt o;
    o.slots = slots;
    o.lim = lim;
    o.wide16 = true;
    BE42_CHECK(launch_fused(P, q, sel, nsel, sel_stride, n_queries, n_heads, scale, out, s, o),
               "prefill attention: unsupported head grouping");
    BE42_LAUNCH_CHECK();
    return BE42_OK;
}

}  // namespace be42
