// attn_dev.h -- the phases of attention over up to 64 selected KV pages as
// device functions (scores, closed-form online-softmax weights, values, the
// cross-wave sum), shared by the attention kernels (attention.hip) and the
// fused decode layer (decode.hip), which runs the next layer's dense
// attention after its K/V append.  Reference: ops_attention.c:292-461 and
// fast_expf ops_math_fast.h:48-64; the closed form is described in
// attention.hip.
#pragma once

#include <type_traits>

#include "be42_common.h"
#include "route.h"

namespace be42 {

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
// Slots whose scores the fused route + attention computes while the heap
// orders them: the two anchors and every middle candidate, when they number
// at most this many.
constexpr int kSetMax = 80;

template <bool BF16>
struct RawRow {
    using T = typename std::conditional<BF16, uint4, uint2>::type;
};

// K / V rows are read once per step: non-temporal loads (each wave
// instruction covers whole 128-byte lines of 4 consecutive rows)
__device__ __forceinline__ uint4 ld_row_nt(const uint16_t *p)
{
    const v4i v = __builtin_nontemporal_load((const v4i *)p);
    return make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
}
__device__ __forceinline__ uint2 ld_row_nt(const int8_t *p)
{
    typedef int v2i __attribute__((ext_vector_type(2)));
    const v2i v = __builtin_nontemporal_load((const v2i *)p);
    return make_uint2((uint32_t)v[0], (uint32_t)v[1]);
}

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

// LDS of the fused attention: per selected page ("slot") its physical page
// and token count, the scores / weights of the G heads per slot, and the
// cross-wave reduction of o.
template <int HD, int G, int WAVES>
struct AttnShared {
    float qs[G][HD];
    // the q split of the matrix-core scores, per lane and 32-dim block
    // (attn_q_store), for kernels that form it once for all their waves
    uint4 qp[kWave][HD / 32];
    float sc[G][kSetMax * 17];
    float lsh[G];
    int pphys[kSetMax], pnt[kSetMax], order[kFusedMaxPages];
    // cross-wave reduction of o ([WAVES][G][HD]): a static array of the
    // kernel, or LDS of a phase that has ended (the router's)
    float *red;
};

template <int HD, int G, int WAVES>
__device__ __forceinline__ void attn_load_q(AttnShared<HD, G, WAVES> &S, const float *__restrict__ q, int b, int kvh,
                                            int H)
{
    for (int i = threadIdx.x; i < G * HD; i += blockDim.x)
        S.qs[i / HD][i % HD] = q[((size_t)b * H + kvh * G + i / HD) * HD + i % HD];
}

// A on the matrix cores (bf16 pages): S[g][t] = q_g . k_t for the 16 tokens of
// a page in one v_mfma_f32_16x16x32_bf16 chain.  Each fp32 q_g is written as
// three bf16 parts hi + mid + lo (exact to 2^-27 |q|; bf16 products are exact
// in fp32), and A row r = 4 g + part (part 3 and heads past G are zero), so
// the C value of lane (token t = lane % 16, row group lane / 16 = g) holds the
// three partial sums of head g: s = ((hi + mid) + lo) * scale, no lane
// exchange.  The head dimension is permuted the same way in A and B: MFMA j
// takes dims [32 j, 32 j + 32), lane group gi the 8 at 32 j + 8 gi, so the
// load of one MFMA's operand reads 64 contiguous bytes of each of 16 rows
// and two consecutive loads complete the rows' 128-byte lines.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

template <int HD>
struct QParts {
    bf16x8_t a[HD / 32];
};

// lane `lane`'s A operand of 32-dim block j: its part of the 8 dims it holds
template <int HD, int G, int WAVES>
__device__ __forceinline__ uint4 attn_q_word(const AttnShared<HD, G, WAVES> &S, int lane, int j)
{
    const int r = lane & 15, gi = lane >> 4;
    const int g = r >> 2, part = r & 3;
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
        uint16_t h[2];
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const float q = g < G ? S.qs[g < G ? g : 0][32 * j + 8 * gi + i + e] : 0.0f;
            const uint16_t hi = f32_to_bf16(q);
            const float r1 = q - bf16_to_f32(hi);
            const uint16_t mid = f32_to_bf16(r1);
            const float r2 = r1 - bf16_to_f32(mid);
            const uint16_t lo = f32_to_bf16(r2);
            h[e] = part == 0 ? hi : (part == 1 ? mid : (part == 2 ? lo : (uint16_t)0));
        }
        w[i / 2] = (uint32_t)h[0] | ((uint32_t)h[1] << 16);
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
}

template <int HD, int G, int WAVES>
__device__ __forceinline__ QParts<HD> attn_q_parts(const AttnShared<HD, G, WAVES> &S)
{
    QParts<HD> Q;
#pragma unroll
    for (int j = 0; j < HD / 32; j++)
        Q.a[j] = __builtin_bit_cast(bf16x8_t, attn_q_word(S, threadIdx.x & 63, j));
    return Q;
}

// S.qp from S.qs by threads t0, t0 + nt, ... (one (lane, block) word each)
template <int HD, int G, int WAVES>
__device__ __forceinline__ void attn_q_store(AttnShared<HD, G, WAVES> &S, int t, int nt)
{
    for (int i = t; i < kWave * (HD / 32); i += nt)
        S.qp[i / (HD / 32)][i % (HD / 32)] = attn_q_word(S, i / (HD / 32), i % (HD / 32));
}

// scores of the pages at slots [lo, ns) of S.pphys, UNR pages per wave step,
// by waves w0 .. w0+nw-1
template <int HD, int G, int WAVES, int UNR, bool QLDS = false>
__device__ __forceinline__ void attn_scores_mfma(const be42_kv_pool &P, AttnShared<HD, G, WAVES> &S, int kvh, int ns,
                                                 float scale, int w0, int nw, int lo = 0)
{
    constexpr int NJ = HD / 32;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t = lane & 15, gi = lane >> 4;
    // a wave with no page to score skips the q split too (with few pages
    // most waves have none, and their vector work would only slow the ones
    // that do, and the heap replay, on the same SIMDs)
    if (lo + (wave - w0) * UNR >= ns)
        return;
    QParts<HD> Q;
    if constexpr (QLDS) {
        // formed once for the workgroup (attn_q_store)
#pragma unroll
        for (int j = 0; j < NJ; j++)
            Q.a[j] = __builtin_bit_cast(bf16x8_t, S.qp[lane][j]);
    } else {
        Q = attn_q_parts<HD, G, WAVES>(S);
    }
    const int n_kv = P.n_kv;
    for (int s0 = lo + (wave - w0) * UNR; s0 < ns; s0 += nw * UNR) {
        uint4 kb[UNR][NJ];
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            const int sl = min(s0 + u, ns - 1);
            const uint16_t *row = (const uint16_t *)P.k + (((size_t)S.pphys[sl] * n_kv + kvh) * kPg + t) * HD + 8 * gi;
#pragma unroll
            for (int j = 0; j < NJ; j++)
                kb[u][j] = *(const uint4 *)(row + 32 * j);
        }
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < NJ; j++)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Q.a[j], __builtin_bit_cast(bf16x8_t, kb[u][j]), acc, 0,
                                                              0, 0);
            if (gi < G && s0 + u < ns)
                S.sc[gi < G ? gi : 0][(s0 + u) * 17 + t] = ((acc[0] + acc[1]) + acc[2]) * scale;
        }
    }
}

// A. scores of the ns pages of S.pphys (slot order) for the G heads, by
// waves w0 .. w0+nw-1.
template <bool BF16, int HD, int G, int WAVES, int UNR, bool QLDS = false>
__device__ __forceinline__ void attn_scores(const be42_kv_pool &P, AttnShared<HD, G, WAVES> &S, int kvh, int ns,
                                            float scale, int w0, int nw)
{
    if constexpr (BF16 && (HD == 64 || HD == 128)) {
        attn_scores_mfma<HD, G, WAVES, 4, QLDS>(P, S, kvh, ns, scale, w0, nw);
        return;
    }
    constexpr int RL = HD / 8;                 // lanes per row
    constexpr int RPW = kWave / RL;            // rows per wave per step
    using Raw = typename RawRow<BF16>::T;
    const int n_kv = P.n_kv;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rsub = lane / RL, rl = lane % RL;
    const int T = ns * kPg;
    const int rows_per_iter = nw * RPW;
    auto load_raw = [&](const void *base, int r, float &sc_out) -> Raw {
        const int rr = r < T ? r : T - 1;
        const int pg = rr / kPg, t = rr % kPg;
        const size_t slot = ((size_t)S.pphys[pg] * n_kv + kvh) * kPg + t;
        if constexpr (BF16) {
            sc_out = 1.0f;
            return ld_row_nt((const uint16_t *)base + slot * HD + rl * 8);
        } else {
            sc_out = P.k_scale[slot];
            return ld_row_nt((const int8_t *)base + slot * HD + rl * 8);
        }
    };
    float qv[G][8];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int j = 0; j < 8; j++)
            qv[g][j] = S.qs[g][rl * 8 + j];
    for (int r0 = (wave - w0) * RPW; r0 < T; r0 += rows_per_iter * UNR) {
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
                    S.sc[g][pg * 17 + t] = acc[g] * scale;
            }
        }
    }
}

// B. weights: wave g <-> head g, lane <-> selection position p (slot
// order[p], or p when order is NULL), the closed-form online softmax of the
// file header over the selection order; l = sum w.
template <int HD, int G, int WAVES>
__device__ __forceinline__ void attn_weights(AttnShared<HD, G, WAVES> &S, int ns, const int *order)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int g = wave; g < G; g += WAVES) {
        float *s = S.sc[g];
        const int slot = lane < ns ? (order ? order[lane] : lane) : 0;
        const int nt = lane < ns ? S.pnt[slot] : 0;
        // the slot's 16 scores in registers (one LDS round trip)
        float sv[kPg];
#pragma unroll
        for (int t = 0; t < kPg; t++)
            sv[t] = s[slot * 17 + t];
        float lm = -INFINITY;
#pragma unroll
        for (int t = 0; t < kPg; t++)
            if (t < nt)
                lm = fmaxf(lm, sv[t]);
        // running max before this slot: exclusive prefix max over the lanes
        float m = wave_shift_up1(wave_prefix_max(lm), -INFINITY);
        // the token steps without branches: every step is computed and
        // selected (tokens past the page's count keep their state), which
        // does the same operations for the valid tokens as the reference's
        // loop; per-token branches cost more than the arithmetic
        float av[kPg], lprod = 1.0f;
#pragma unroll
        for (int t = 0; t < kPg; t++) {
            const bool v = t < nt;
            const float st = sv[t];
            const float mprev = m;
            const float mn = fmaxf(m, st);
            const float ex = fast_expf(mprev - mn);
            const float at = mprev == -INFINITY ? 1.0f : ex;
            const float e = fast_expf(st - mn);
            m = v ? mn : m;
            sv[t] = v ? e : st;
            av[t] = v ? at : 1.0f;
            lprod = v ? lprod * at : lprod;
        }
        // rescales of all later slots: exclusive suffix product over the lanes
        float pr = wave_shift_down1(wave_suffix_prod(lprod), 1.0f);
        float ls = 0.0f;
#pragma unroll
        for (int t = kPg - 1; t >= 0; t--) {
            const bool v = t < nt;
            const float w = sv[t] * pr;
            if (v)
                s[slot * 17 + t] = w;
            ls = v ? ls + w : ls;
            pr *= av[t];   // av = 1 past the count
        }
        ls = wave_sum_dpp(ls);
        if (lane == 0)
            S.lsh[g] = ls;
    }
}

// A batch of V rows of a wave (UNR row steps).
template <bool BF16, int UNR>
struct VBatch {
    typename RawRow<BF16>::T vr[UNR];
    float vsc[UNR];
};

template <bool BF16, int HD, int G, int WAVES, int UNR, int SW>
__device__ __forceinline__ void attn_values_load(const be42_kv_pool &P, const AttnShared<HD, G, SW> &S, int kvh, int ns,
                                                 const int *order, int r0, VBatch<BF16, UNR> &vb)
{
    constexpr int RL = HD / 8;
    constexpr int RPW = kWave / RL;
    constexpr int rows_per_iter = WAVES * RPW;
    const int lane = threadIdx.x & 63, rsub = lane / RL, rl = lane % RL;
    const int T = ns * kPg;
#pragma unroll
    for (int u = 0; u < UNR; u++) {
        const int r = r0 + u * rows_per_iter + rsub;
        const int rr = r < T ? r : T - 1;
        const int pg = rr / kPg, t = rr % kPg;
        const size_t slot = ((size_t)S.pphys[order ? order[pg] : pg] * P.n_kv + kvh) * kPg + t;
        if constexpr (BF16) {
            vb.vsc[u] = 1.0f;
            vb.vr[u] = ld_row_nt((const uint16_t *)P.v + slot * HD + rl * 8);
        } else {
            vb.vsc[u] = P.v_scale[slot];
            vb.vr[u] = ld_row_nt((const int8_t *)P.v + slot * HD + rl * 8);
        }
    }
}

// out = (sum over the waves' partial o) * (1 / l)
template <int HD, int G, int WAVES, int SW>
__device__ __forceinline__ void attn_values_finish(const AttnShared<HD, G, SW> &S, int b, int kvh, int H,
                                                   float *__restrict__ out)
{
    const int tid = threadIdx.x;
    for (int i = tid; i < G * HD; i += blockDim.x) {
        const int g = i / HD, d = i % HD;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; w++)
            v += S.red[(w * G + g) * HD + d];
        const float l = S.lsh[g];
        out[((size_t)b * H + kvh * G + g) * HD + d] = l > 0.0f ? v * (1.0f / l) : v;
    }
}

// C on the matrix cores (bf16 pages, V stored [kv head][dim][16 tokens]):
// o[g][d] = sum_t w[g][t] v[t][d] with one v_mfma_f32_16x16x16bf16_1k per
// page and 16-dim tile.  A row r = 4 g + part holds the bf16 parts of the
// weights w[g][t] (zero past the page's token count, for part 3 and for heads
// past G); B is 4 consecutive tokens of one dim (8 bytes, a tile's 16 dims x
// 16 tokens = 512 contiguous bytes per load; zero past the page's token
// count); the C value of lane (dim of the
// tile, row group g) adds up to the three parts of head g.  Pages go round
// robin over the waves, UNR in flight per wave.
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef int v2i_t __attribute__((ext_vector_type(2)));

// The pages of wave `wave` of a WAVES-wave layout (positions wave * UNR +
// WAVES * UNR * i + u) into put(index, value), index = g * HD + dim: the
// partial o of that wave.
template <int HD, int G, int WAVES, int UNR, int SW, class Put>
__device__ __forceinline__ void attn_values_mfma_wave(const be42_kv_pool &P, const AttnShared<HD, G, SW> &S,
                                                      int kvh, int ns, const int *order, int wave, Put &&put)
{
    constexpr int NT = HD / 16;
    const int lane = threadIdx.x & 63;
    const int n = lane & 15, gi = lane >> 4;
    const int ag = n >> 2, apart = n & 3;
    v4f acc[NT];
#pragma unroll
    for (int i = 0; i < NT; i++)
        acc[i] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    for (int p0 = wave * UNR; p0 < ns; p0 += WAVES * UNR) {
        v2i_t vb[UNR][NT];
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            const int p = min(p0 + u, ns - 1);
            const int sl = order ? order[p] : p;
            const uint16_t *vp = (const uint16_t *)P.v + ((size_t)S.pphys[sl] * P.n_kv + kvh) * HD * kPg + 4 * gi;
#pragma unroll
            for (int tile = 0; tile < NT; tile++)
                vb[u][tile] = __builtin_nontemporal_load((const v2i_t *)(vp + (tile * 16 + n) * kPg));
        }
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            if (p0 + u < ns) {
                const int sl = order ? order[p0 + u] : p0 + u;
                const int nt = S.pnt[sl];
                uint16_t h[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int t = 4 * gi + i;
                    const float w = ag < G && t < nt ? S.sc[ag < G ? ag : 0][sl * 17 + t] : 0.0f;
                    const uint16_t hi = f32_to_bf16(w);
                    const float r1 = w - bf16_to_f32(hi);
                    const uint16_t mid = f32_to_bf16(r1);
                    const float r2 = r1 - bf16_to_f32(mid);
                    const uint16_t lo = f32_to_bf16(r2);
                    h[i] = apart == 0 ? hi : (apart == 1 ? mid : (apart == 2 ? lo : (uint16_t)0));
                }
                const s16x4_t a = {(short)h[0], (short)h[1], (short)h[2], (short)h[3]};
                // token slots past the count hold whatever the page held
                // before: zero them (a zero weight times a NaN or infinite
                // bf16 pattern would still be NaN)
                const int t0 = 4 * gi;
                const v2i_t keep = {(int)((t0 < nt ? 0xFFFFu : 0u) | (t0 + 1 < nt ? 0xFFFF0000u : 0u)),
                                    (int)((t0 + 2 < nt ? 0xFFFFu : 0u) | (t0 + 3 < nt ? 0xFFFF0000u : 0u))};
#pragma unroll
                for (int tile = 0; tile < NT; tile++)
                    acc[tile] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
                        a, __builtin_bit_cast(s16x4_t, vb[u][tile] & keep), acc[tile], 0, 0, 0);
            }
        }
    }
    if (gi < G)
#pragma unroll
        for (int tile = 0; tile < NT; tile++)
            put(gi * HD + tile * 16 + n, (acc[tile][0] + acc[tile][1]) + acc[tile][2]);
}

template <int HD, int G, int WAVES, int UNR>
__device__ __forceinline__ void attn_values_mfma(const be42_kv_pool &P, AttnShared<HD, G, WAVES> &S, int kvh, int ns,
                                                 const int *order)
{
    const int wave = threadIdx.x >> 6;
    float *red = S.red + wave * G * HD;
    attn_values_mfma_wave<HD, G, WAVES, UNR>(P, S, kvh, ns, order, wave, [red](int i, float v) { red[i] = v; });
}

// C (rows): the rows of wave `wave` of a WAVES-wave layout (rows wave * RPW
// + WAVES * RPW * i, UNR steps in flight) accumulate o[g][8 dims] per lane,
// summed over the row groups of the wave; put(index, value) receives the
// wave's partial o (index = g * HD + dim).
template <bool BF16, int HD, int G, int WAVES, int UNR, int SW, class Put>
__device__ __forceinline__ void attn_values_rows_wave(const be42_kv_pool &P, const AttnShared<HD, G, SW> &S, int kvh,
                                                      int ns, const int *order, int wave, Put &&put)
{
    constexpr int RL = HD / 8;
    constexpr int RPW = kWave / RL;
    const int lane = threadIdx.x & 63;
    const int rsub = lane / RL, rl = lane % RL;
    const int T = ns * kPg;
    constexpr int rows_per_iter = WAVES * RPW;
    float o[G][8];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int j = 0; j < 8; j++)
            o[g][j] = 0.0f;
    for (int r0 = wave * RPW; r0 < T; r0 += rows_per_iter * UNR) {
        VBatch<BF16, UNR> vb;
        attn_values_load<BF16, HD, G, WAVES, UNR>(P, S, kvh, ns, order, r0, vb);
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            const int r = r0 + u * rows_per_iter + rsub;
            if (r < T) {
                const int pg = r / kPg, t = r % kPg;
                const int sl = order ? order[pg] : pg;
                if (t < S.pnt[sl]) {
                    float vv[8];
                    raw_to_f32<BF16>(vv, vb.vr[u], vb.vsc[u]);
#pragma unroll
                    for (int g = 0; g < G; g++) {
                        const float w = S.sc[g][sl * 17 + t];
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
                put(g * HD + rl * 8 + j, o[g][j]);
}

// C. o = sum_t w_t v_t over the slots (the order of the sum is free), then
// out = o * (1 / l).
template <bool BF16, int HD, int G, int WAVES, int UNR>
__device__ __forceinline__ void attn_values(const be42_kv_pool &P, AttnShared<HD, G, WAVES> &S, int b, int kvh,
                                            int ns, int H, float *__restrict__ out, const int *order)
{
    const int wave = threadIdx.x >> 6;
    if constexpr (BF16 && (HD == 64 || HD == 128)) {
        attn_values_mfma<HD, G, WAVES, 4>(P, S, kvh, ns, order);
    } else {
        float *red = S.red + wave * G * HD;
        attn_values_rows_wave<BF16, HD, G, WAVES, UNR>(P, S, kvh, ns, order, wave,
                                                       [red](int i, float v) { red[i] = v; });
    }
    __syncthreads();
    attn_values_finish<HD, G, WAVES>(S, b, kvh, H, out);
}

// C in the layout of VW waves from the block's WAVES waves (VW a multiple of
// WAVES): wave w forms the partials of layout waves w, w + WAVES, ..., which
// are then added in layout order -- the output of a VW-wave workgroup, bit
// for bit.  S.red holds VW partials.
template <bool BF16, int HD, int G, int WAVES, int VW, int UNR, int SW>
__device__ __forceinline__ void attn_values_layout(const be42_kv_pool &P, const AttnShared<HD, G, SW> &S, int b,
                                                   int kvh, int ns, int H, float *__restrict__ out, const int *order)
{
    static_assert(VW % WAVES == 0, "layout");
    for (int vw = threadIdx.x >> 6; vw < VW; vw += WAVES) {
        float *dst = S.red + vw * G * HD;
        if constexpr (BF16 && (HD == 64 || HD == 128))
            attn_values_mfma_wave<HD, G, VW, 4>(P, S, kvh, ns, order, vw, [dst](int i, float v) { dst[i] = v; });
        else
            attn_values_rows_wave<BF16, HD, G, VW, UNR>(P, S, kvh, ns, order, vw,
                                                        [dst](int i, float v) { dst[i] = v; });
    }
    __syncthreads();
    attn_values_finish<HD, G, VW>(S, b, kvh, H, out);
}

}  // namespace be42
