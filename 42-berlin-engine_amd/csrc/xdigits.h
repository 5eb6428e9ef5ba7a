// xdigits.h -- activation digit planes of the MFMA GEMV.
//
// The GEMV feeds raw INT8 / E4M3 weight codes to the matrix cores; the fp32
// activations are split once per call into exact fixed-point digits of the
// MFMA input type:
//     x[b][k] = s_b * sum_d digit_d[b][k] * R^-d
//   INT8: 3 digits in [-127, 127], R = 254, s_b = max|x_b| / 127
//   FP8:  4 integer digits in [-15, 15] stored as exact E4M3 codes, R = 30,
//         s_b = max|x_b| / 15
// INT8 to ~2^-24 of max|x_b|; FP8 to 0.5 * 30^-3 * s_b, ~1.2e-6 of max|x_b|
// (a fifth FP8 plane would take the split to ~4e-8 for a quarter more
// matrix-core work and digit bytes; with four the GEMV's error stays near
// 1e-5, a hundredth of the 1e-3 bound).  Buffer layout: digit planes
// dig[d][b][0..Kp) bytes (zero past K), then, on a 256-byte boundary, the
// floats s_b (room for max(16, batch)).  Kp is K rounded up to the largest
// burst a GEMV tile uses.  The prefill GEMM reads the same layout with one
// "batch row" per token.
#pragma once

#include "be42_common.h"

namespace be42 {

constexpr int kI8Digits = 3;
constexpr int kI8Base = 254;
constexpr int kF8Digits = 4;
constexpr int kF8Base = 30;
// weight of FP8 digit d in the recombination, 30^-d
__device__ constexpr double kF8DigitW[kF8Digits] = {1.0, 1.0 / 30, 1.0 / 900, 1.0 / 27000};

template <bool FP8>
__device__ __forceinline__ float digit_scale(float amax)
{
    return amax > 0.0f ? amax / (FP8 ? 15.0f : 127.0f) : 1.0f;
}

// digits of four consecutive elements xe at scale s, one 32-bit word (four
// digit bytes) per plane.  FP8 digits (integers in [-15, 15], exact in E4M3)
// are encoded by the hardware conversion, two per instruction; + 0.0f turns
// a -0 digit into +0, so the code of 0 is 0x00 (the conversion gives -0 the
// code 0x80).
template <bool FP8>
__device__ __forceinline__ void digit_words(const float xe[4], float s, uint32_t (&word)[FP8 ? kF8Digits : kI8Digits])
{
    constexpr int R0 = FP8 ? 15 : 127;
    constexpr int ND = FP8 ? kF8Digits : kI8Digits;
    constexpr float BASE = FP8 ? (float)kF8Base : (float)kI8Base;
    const float rs = 1.0f / s;
    float dv[4][ND];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        float v = xe[e] * rs;
#pragma unroll
        for (int d = 0; d < ND; d++) {
            float t = rintf(v);
            t = fminf(fmaxf(t, -(float)R0), (float)R0);
            v = (v - t) * BASE;
            dv[e][d] = t + 0.0f;
        }
    }
#pragma unroll
    for (int d = 0; d < ND; d++) {
        if constexpr (FP8) {
            int w = __builtin_amdgcn_cvt_pk_fp8_f32(dv[0][d], dv[1][d], 0, false);
            w = __builtin_amdgcn_cvt_pk_fp8_f32(dv[2][d], dv[3][d], w, true);
            word[d] = (uint32_t)w;
        } else {
            word[d] = (uint32_t)(uint8_t)(int8_t)(int)dv[0][d] | ((uint32_t)(uint8_t)(int8_t)(int)dv[1][d] << 8) |
                      ((uint32_t)(uint8_t)(int8_t)(int)dv[2][d] << 16) |
                      ((uint32_t)(uint8_t)(int8_t)(int)dv[3][d] << 24);
        }
    }
}

// digits of x[b][k0 .. k0+4) (xe), one 32-bit word per plane
template <bool FP8>
__device__ __forceinline__ void store_digit_words(const float xe[4], float s, uint8_t *__restrict__ dig, int B,
                                                  int Kp, int b, int k0)
{
    constexpr int ND = FP8 ? kF8Digits : kI8Digits;
    uint32_t word[ND];
    digit_words<FP8>(xe, s, word);
#pragma unroll
    for (int d = 0; d < ND; d++)
        *(uint32_t *)(dig + ((size_t)d * B + b) * Kp + k0) = word[d];
}

struct XDigits {
    int nd, step, burst;
};
__host__ __device__ inline XDigits xdig_layout(bool fp8)
{
    return fp8 ? XDigits{kF8Digits, 128, 128 * 8} : XDigits{kI8Digits, 64, 64 * 16};
}
__host__ __device__ inline size_t xdig_kp(int k, bool fp8)
{
    const XDigits L = xdig_layout(fp8);
    return ((size_t)(k + L.burst - 1) / L.burst) * L.burst;
}
// digits first, then the float scales on a 256-byte boundary
__host__ __device__ inline size_t xdig_bytes(int k, int batch, bool fp8)
{
    const size_t dig = (size_t)xdig_layout(fp8).nd * batch * xdig_kp(k, fp8);
    return ((dig + 255) & ~(size_t)255) + (size_t)(batch > 16 ? batch : 16) * sizeof(float);
}
__host__ __device__ inline float *xdig_scales(void *buf, int k, int batch, bool fp8)
{
    const size_t dig = (size_t)xdig_layout(fp8).nd * batch * xdig_kp(k, fp8);
    return (float *)((uint8_t *)buf + ((dig + 255) & ~(size_t)255));
}

// host: the digit planes (and scales) of x [batch][k] into buf (gemv.hip);
// any batch, k % 16 == 0
int xdig_prepare(void *buf, const float *x, int k, int batch, bool fp8, hipStream_t s);

}  // namespace be42
