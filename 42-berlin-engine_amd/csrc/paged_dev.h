// paged_dev.h -- device code of the page pool shared by the pool's own
// kernels (paged.hip) and the decode step's fused layer kernel (decode.hip):
// the quantizing row store, the page seal (centroid + hash) and the decode
// step's RoPE + append + seal of one token.
#pragma once

#include "be42_common.h"
#include "paged_step.h"

namespace be42 {

constexpr int kPage = 16;

// Quantize (INT8) or round (BF16) one K row and one V row of a kv head into
// page slot `slot` (= (phys * n_kv + head) * 16 + offset), one wave.  INT8
// follows quant_f32_to_int8: exact absmax, IEEE scale = amax/127 and
// inv = 127/amax, roundf, clamp.
template <bool BF16>
__device__ __forceinline__ void store_kv_row(void *__restrict__ kdst, void *__restrict__ vdst,
                                             float *__restrict__ kscale, float *__restrict__ vscale, size_t slot,
                                             const float *__restrict__ ks, const float *__restrict__ vs, int hd,
                                             int lane)
{
    if constexpr (BF16) {
        // bf16 V pages are stored [kv head][dim][16 tokens]: the attention's
        // matrix cores read 4 consecutive tokens of one dim as one operand
        uint16_t *kd = (uint16_t *)kdst + slot * hd;
        uint16_t *vd = (uint16_t *)vdst + (slot / kPage) * (size_t)hd * kPage + slot % kPage;
        for (int d = lane; d < hd; d += kWave) {
            kd[d] = f32_to_bf16(ks[d]);
            vd[(size_t)d * kPage] = f32_to_bf16(vs[d]);
        }
    } else {
        float km = 0.0f, vm = 0.0f;
        for (int d = lane; d < hd; d += kWave) {
            km = fmaxf(km, fabsf(ks[d]));
            vm = fmaxf(vm, fabsf(vs[d]));
        }
        km = wave_max(km);
        vm = wave_max(vm);
        float ksc = 1.0f, kinv = 1.0f, vsc = 1.0f, vinv = 1.0f;
        if (km > 0.0f) {
            ksc = km / 127.0f;
            kinv = 127.0f / km;
        }
        if (vm > 0.0f) {
            vsc = vm / 127.0f;
            vinv = 127.0f / vm;
        }
        int8_t *kd = (int8_t *)kdst + slot * hd, *vd = (int8_t *)vdst + slot * hd;
        for (int d = lane; d < hd; d += kWave) {
            const int kc = (int)roundf(ks[d] * kinv), vc = (int)roundf(vs[d] * vinv);
            kd[d] = (int8_t)(kc > 127 ? 127 : (kc < -127 ? -127 : kc));
            vd[d] = (int8_t)(vc > 127 ? 127 : (vc < -127 ? -127 : vc));
        }
        if (lane == 0) {
            kscale[slot] = ksc;
            vscale[slot] = vsc;
        }
    }
}

// One block per page that became full: centroid of the head-0 keys (per
// dimension, tokens summed in order, then * (1.0f/16)), then its hash: 16
// lanes each run the FMA chain over d ascending from +0 (bit h = sum > 0).
template <bool BF16>
__device__ __forceinline__ void seal_page(const void *__restrict__ kpool, const float *__restrict__ kscale,
                                          float *__restrict__ centroid, uint16_t *__restrict__ hash_out, int phys,
                                          const float *__restrict__ hpT, int n_kv, int hd, float *c)
{
    const size_t head0 = (size_t)phys * n_kv * kPage;      // slot of (phys, head 0, token 0)
    const int d = threadIdx.x;
    if (d < hd) {
        float acc = 0.0f;
        for (int t = 0; t < kPage; t++) {
            float val;
            if constexpr (BF16)
                val = bf16_to_f32(((const uint16_t *)kpool)[(head0 + t) * hd + d]);
            else
                val = (float)((const int8_t *)kpool)[(head0 + t) * hd + d] * kscale[head0 + t];
            acc = acc + val;
        }
        acc = acc * (1.0f / (float)kPage);
        c[d] = acc;
        centroid[(size_t)phys * hd + d] = acc;
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        const int h = threadIdx.x;
        float s = 0.0f;
        if (h < 16)
            for (int i = 0; i < hd; i++)
                s = __fmaf_rn(c[i], hpT[i * 16 + h], s);
        const unsigned long long m = __ballot(h < 16 && s > 0.0f);
        if (h == 0)
            *hash_out = (uint16_t)(m & 0xFFFFu);
    }
}

// The store of token tok's rotated k row (ks) and v row (vs, any address
// space) for KV head h, the page-table publish, and for h == 0 the seal of the
// page it fills (AppendStepArgs bookkeeping).  Run by a whole block.
template <bool BF16>
__device__ __forceinline__ void append_seal_tail(const be42_kv_pool &P, const AppendStepArgs &a, int tok, int h,
                                                 const float *ks, const float *vs, float *c)
{
    const int tid = threadIdx.x, n_kv = P.n_kv, hd = P.head_dim;
    const int off = a.pos[tok] % kPage, blk = a.pos[tok] / kPage, phys = a.phys[tok];
    if (tid < kWave) {
        if (h == 0 && tid == 0) {
            if (a.publish[tok]) {
                P.page_table[(size_t)a.slot[tok] * a.max_logical + blk] = phys;
                P.n_logical[a.slot[tok]] = blk + 1;
            }
            P.ntok[phys] = off + 1;
        }
        const size_t slot = ((size_t)phys * n_kv + h) * kPage + off;
        store_kv_row<BF16>(P.k, P.v, P.k_scale, P.v_scale, slot, ks, vs, hd, tid);
    }
    const int si = a.seal_of[tok];
    if (h != 0 || si < 0)
        return;
    __syncthreads();                       // the page's last row is in memory
    if (tid == 0)
        P.n_indexed[a.seal_slot[si]] = a.seal_nidx[si];
    seal_page<BF16>(P.k, P.k_scale, P.centroid,
                    P.page_hash + (size_t)a.seal_slot[si] * a.max_logical + a.seal_logical[si], a.seal_phys[si],
                    P.hpT, n_kv, hd, c);
}

// RoPE + append + seal of token `tok` of a decode step for KV head h, run by
// one whole block (any size >= 64): the q heads of h's group and k head h are
// rotated in place (the RoPE of inference.c / ops_rope.c:192 as k_rope does
// it), the rotated k row and the v row are stored into the page, and the
// block of h == 0 seals the page when this token fills it.  ks and c are
// block-shared scratch of 256 floats each.
template <bool BF16>
__device__ __forceinline__ void rope_append_body(const be42_kv_pool &P, const AppendStepArgs *__restrict__ ap,
                                                 float *__restrict__ q, float *__restrict__ k,
                                                 const float *__restrict__ v, const float *__restrict__ cos_t,
                                                 const float *__restrict__ sin_t, const int *__restrict__ pos_p,
                                                 int rope_len, int H, int tok, int h, float *ks, float *c)
{
    const AppendStepArgs &a = *ap;
    const int tid = threadIdx.x;
    if (tok >= a.n)
        return;
    const int n_kv = P.n_kv, hd = P.head_dim, half = hd / 2, G = H / n_kv;
    const int pos = *pos_p;
    float *krow = k + ((size_t)tok * n_kv + h) * hd;
    if (pos < rope_len) {
        for (int i = tid; i < (G + 1) * half; i += blockDim.x) {
            const int j = i / half, pr = i % half;
            float *base = j < G ? q + ((size_t)tok * H + h * G + j) * hd : krow;
            const float cs = cos_t[(size_t)pos * half + pr], sn = sin_t[(size_t)pos * half + pr];
            const float x0 = base[pr], x1 = base[pr + half];
            const float y0 = __fmaf_rn(x0, cs, -(x1 * sn)), y1 = __fmaf_rn(x0, sn, x1 * cs);
            base[pr] = y0;
            base[pr + half] = y1;
            if (j == G) {
                ks[pr] = y0;
                ks[pr + half] = y1;
            }
        }
    } else {
        for (int i = tid; i < hd; i += blockDim.x)
            ks[i] = krow[i];
    }
    __syncthreads();
    append_seal_tail<BF16>(P, a, tok, h, ks, v + ((size_t)tok * n_kv + h) * hd, c);
}

}  // namespace be42
