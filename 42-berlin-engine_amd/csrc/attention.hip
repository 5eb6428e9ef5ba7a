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
#include <type_traits>

#include "be42_common.h"

namespace be42 {

constexpr int kPg = 16;

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
                load_row_f32(v, P.v, slot * HD + dl * D, D, BF16, BF16 ? 1.0f : P.v_scale[slot]);
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


// ---------------------------------------------------------------------------
// Fused attention for up to 64 selected pages: one workgroup of WAVES waves
// per (query, KV head) serves the G query heads of the group.
//  A. scores: a row (token) of K is read by RL = HD/8 lanes (16 bytes bf16 or
//     8 bytes INT8 each), RPW = 64/RL rows per wave per step, UNR steps in
//     flight as raw registers (16 waves x 8 steps = the 512 rows of 32 pages
//     per pass); each lane forms the G partial dots of its 8 elements, the
//     RL lanes of a row reduce them; s = dot * scale goes to LDS.
//  B. weights: wave g scans head g's scores, lane = selected page (LDS padded
//     to 17 floats per page against bank conflicts), the closed-form online
//     softmax of the file header, l = sum w.
//  C. V: the same row mapping accumulates o[g][8 dims] for all G heads, summed
//     over the row groups of a wave and then over the waves through LDS;
//     out = o * (1 / l).
// Every K and V row of the selected pages is read once per KV head.
constexpr int kFusedMaxPages = 64;

template <bool BF16>
struct RawRow {
    using T = typename std::conditional<BF16, uint4, uint2>::type;
};

template <bool BF16>
__device__ __forceinline__ void raw_to_f32(float *dst, const typename RawRow<BF16>::T &u, float scale)
{
    if constexpr (BF16) {
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            dst[2 * j] = __uint_as_float(w[j] << 16);
            dst[2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
        }
    } else {
        const uint32_t w[2] = {u.x, u.y};
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int e = 0; e < 4; e++)
                dst[4 * j + e] = (float)(int8_t)((w[j] >> (8 * e)) & 0xFF) * scale;
    }
}

// Sum over aligned groups of RL (4, 8 or 16) lanes with DPP lane moves:
// quad swaps (xor 1, xor 2), then the half-row and row mirrors, which pair
// the remaining quads / halves.  Every lane of a group ends with the sum.
template <int RL>
__device__ __forceinline__ float group_sum(float a)
{
    auto mv = [](float v, int ctrl) -> float {
        const int i = __float_as_int(v);
        int r;
        switch (ctrl) {
        case 0: r = __builtin_amdgcn_update_dpp(0, i, 0xB1, 0xF, 0xF, false); break;   // quad_perm [1,0,3,2]
        case 1: r = __builtin_amdgcn_update_dpp(0, i, 0x4E, 0xF, 0xF, false); break;   // quad_perm [2,3,0,1]
        case 2: r = __builtin_amdgcn_update_dpp(0, i, 0x141, 0xF, 0xF, false); break;  // row_half_mirror
        default: r = __builtin_amdgcn_update_dpp(0, i, 0x140, 0xF, 0xF, false); break; // row_mirror
        }
        return __int_as_float(r);
    };
    a = a + mv(a, 0);
    a = a + mv(a, 1);
    if constexpr (RL >= 8)
        a = a + mv(a, 2);
    if constexpr (RL >= 16)
        a = a + mv(a, 3);
    return a;
}

template <bool BF16, int HD, int G, int WAVES, int UNR>
__global__ __launch_bounds__(WAVES * 64) void k_attn_fused(const be42_kv_pool P, const float *__restrict__ q,
                                                           const int *__restrict__ sel,
                                                           const int *__restrict__ nsel, int sel_stride, int H,
                                                           float scale, float *__restrict__ out)
{
    constexpr int RL = HD / 8;                 // lanes per row
    constexpr int RPW = kWave / RL;            // rows per wave per step
    using Raw = typename RawRow<BF16>::T;
    __shared__ float qs[G][HD];
    __shared__ float sc[G][kFusedMaxPages * 17];
    __shared__ float red[WAVES][G][HD];
    __shared__ float lsh[G];
    __shared__ int pphys[kFusedMaxPages], pnt[kFusedMaxPages];

    const int b = blockIdx.x, kvh = blockIdx.y;
    const int n_kv = P.n_kv;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int ns = min(nsel[b], kFusedMaxPages);
    const int *selb = sel + (size_t)b * sel_stride;
    for (int i = tid; i < G * HD; i += blockDim.x)
        qs[i / HD][i % HD] = q[((size_t)b * H + kvh * G + i / HD) * HD + i % HD];
    for (int i = tid; i < ns; i += blockDim.x) {
        const int ph = selb[i];
        pphys[i] = ph;
        pnt[i] = P.ntok[ph];
    }
    __syncthreads();

    const int rsub = lane / RL, rl = lane % RL;   // row within the step, lane within the row
    const int T = ns * kPg;
    constexpr int rows_per_iter = WAVES * RPW;

    auto load_raw = [&](const void *base, int r, float &sc_out) -> Raw {
        const int rr = r < T ? r : T - 1;
        const int pg = rr / kPg, t = rr % kPg;
        const size_t slot = ((size_t)pphys[pg] * n_kv + kvh) * kPg + t;
        if constexpr (BF16) {
            sc_out = 1.0f;
            return *(const Raw *)((const uint16_t *)base + slot * HD + rl * 8);
        } else {
            sc_out = (base == P.k ? P.k_scale : P.v_scale)[slot];
            return *(const Raw *)((const int8_t *)base + slot * HD + rl * 8);
        }
    };

    // A. scores
    float qv[G][8];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int j = 0; j < 8; j++)
            qv[g][j] = qs[g][rl * 8 + j];
    for (int r0 = wave * RPW; r0 < T; r0 += rows_per_iter * UNR) {
        Raw kr[UNR];
        float ks[UNR];
#pragma unroll
        for (int u = 0; u < UNR; u++)
            kr[u] = load_raw(P.k, r0 + u * rows_per_iter + rsub, ks[u]);
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            const int r = r0 + u * rows_per_iter + rsub;
            float kv[8];
            raw_to_f32<BF16>(kv, kr[u], ks[u]);
            float acc[G];
#pragma unroll
            for (int g = 0; g < G; g++) {
                float a = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; j++)
                    a = __fmaf_rn(qv[g][j], kv[j], a);
                acc[g] = group_sum<RL>(a);
            }
            if (rl == 0 && r < T) {
                const int pg = r / kPg, t = r % kPg;
#pragma unroll
                for (int g = 0; g < G; g++)
                    sc[g][pg * 17 + t] = acc[g] * scale;
            }
        }
    }
    __syncthreads();

    // B. weights, wave g <-> head g, lane <-> page
    for (int g = wave; g < G; g += WAVES) {
        float *s = sc[g];
        const int nt = lane < ns ? pnt[lane] : 0;
        float lm = -INFINITY;
        for (int t = 0; t < nt; t++)
            lm = fmaxf(lm, s[lane * 17 + t]);
        float inc = lm;
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) {
            const float v = __shfl_up(inc, o, kWave);
            if (lane >= o)
                inc = fmaxf(inc, v);
        }
        float m = __shfl_up(inc, 1, kWave);
        if (lane == 0)
            m = -INFINITY;
        float av[kPg], lprod = 1.0f;
#pragma unroll
        for (int t = 0; t < kPg; t++) {
            av[t] = 1.0f;
            if (t < nt) {
                const float st = s[lane * 17 + t];
                const float mprev = m;
                m = fmaxf(m, st);
                const float at = mprev == -INFINITY ? 1.0f : fast_expf(mprev - m);
                s[lane * 17 + t] = fast_expf(st - m);
                av[t] = at;
                lprod *= at;
            }
        }
        float suf = lprod;
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
#pragma unroll
        for (int t = kPg - 1; t >= 0; t--) {
            if (t < nt) {
                const float w = s[lane * 17 + t] * pr;
                s[lane * 17 + t] = w;
                ls += w;
                pr *= av[t];
            }
        }
        ls = wave_sum(ls);
        if (lane == 0)
            lsh[g] = ls;
    }
    __syncthreads();

    // C. o = sum_t w_t v_t
    float o[G][8];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int j = 0; j < 8; j++)
            o[g][j] = 0.0f;
    for (int r0 = wave * RPW; r0 < T; r0 += rows_per_iter * UNR) {
        Raw vr[UNR];
        float vsc[UNR];
#pragma unroll
        for (int u = 0; u < UNR; u++)
            vr[u] = load_raw(P.v, r0 + u * rows_per_iter + rsub, vsc[u]);
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            const int r = r0 + u * rows_per_iter + rsub;
            if (r < T) {
                const int pg = r / kPg, t = r % kPg;
                if (t < pnt[pg]) {
                    float vv[8];
                    raw_to_f32<BF16>(vv, vr[u], vsc[u]);
#pragma unroll
                    for (int g = 0; g < G; g++) {
                        const float w = sc[g][pg * 17 + t];
#pragma unroll
                        for (int j = 0; j < 8; j++)
                            o[g][j] = __fmaf_rn(w, vv[j], o[g][j]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int j = 0; j < 8; j++) {
            float v = o[g][j];
#pragma unroll
            for (int x = RL; x < kWave; x <<= 1)
                v += __shfl_xor(v, x, kWave);
            o[g][j] = v;
        }
    if (rsub == 0)
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int j = 0; j < 8; j++)
                red[wave][g][rl * 8 + j] = o[g][j];
    __syncthreads();
    for (int i = tid; i < G * HD; i += blockDim.x) {
        const int g = i / HD, d = i % HD;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; w++)
            v += red[w][g][d];
        const float l = lsh[g];
        out[((size_t)b * H + kvh * G + g) * HD + d] = l > 0.0f ? v * (1.0f / l) : v;
    }
}

// 16 waves when the grid is small (more loads in flight per workgroup), 8
// waves once there are enough workgroups to fill the chip.
template <bool BF16, int HD, int G>
static void launch_fused_g(const be42_kv_pool &P, const float *q, const int *sel, const int *nsel, int sel_stride,
                           int B, int H, float scale, float *out, hipStream_t s)
{
    const dim3 grid(B, P.n_kv);
    if ((long)B * P.n_kv < 512)
        hipLaunchKernelGGL((k_attn_fused<BF16, HD, G, 16, 8>), grid, dim3(1024), 0, s, P, q, sel, nsel, sel_stride,
                           H, scale, out);
    else
        hipLaunchKernelGGL((k_attn_fused<BF16, HD, G, 8, 8>), grid, dim3(512), 0, s, P, q, sel, nsel, sel_stride, H,
                           scale, out);
}

template <bool BF16, int HD>
static bool launch_fused_hd(const be42_kv_pool &P, const float *q, const int *sel, const int *nsel, int sel_stride,
                            int B, int H, float scale, float *out, hipStream_t s)
{
    switch (H / P.n_kv) {
    case 1: launch_fused_g<BF16, HD, 1>(P, q, sel, nsel, sel_stride, B, H, scale, out, s); return true;
    case 2: launch_fused_g<BF16, HD, 2>(P, q, sel, nsel, sel_stride, B, H, scale, out, s); return true;
    case 3: launch_fused_g<BF16, HD, 3>(P, q, sel, nsel, sel_stride, B, H, scale, out, s); return true;
    case 4: launch_fused_g<BF16, HD, 4>(P, q, sel, nsel, sel_stride, B, H, scale, out, s); return true;
    default: return false;
    }
}

static bool launch_fused(const be42_kv_pool &P, const float *q, const int *sel, const int *nsel, int sel_stride, int B,
                         int H, float scale, float *out, hipStream_t s)
{
    const bool bf16 = P.kind == BE42_KV_BF16;
    if (P.head_dim == 128)
        return bf16 ? launch_fused_hd<true, 128>(P, q, sel, nsel, sel_stride, B, H, scale, out, s)
                    : launch_fused_hd<false, 128>(P, q, sel, nsel, sel_stride, B, H, scale, out, s);
    if (P.head_dim == 64)
        return bf16 ? launch_fused_hd<true, 64>(P, q, sel, nsel, sel_stride, B, H, scale, out, s)
                    : launch_fused_hd<false, 64>(P, q, sel, nsel, sel_stride, B, H, scale, out, s);
    return false;
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
