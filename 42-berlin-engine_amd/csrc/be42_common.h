// be42_common.h -- shared definitions of the gfx950 decode hot-path library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "be42_hip.h"

// --------------------------------------------------------------------------
// error handling: every entry point returns BE42_OK or a negative code and
// records a message readable through be42_last_error().
// --------------------------------------------------------------------------
namespace be42 {

void set_error(const char *fmt, ...);
int hip_fail(hipError_t e, const char *what, const char *file, int line);

// Grow-only device workspace, one per device, owned by the library.
void *workspace(size_t bytes, hipStream_t s);

// FP8 encoder exponent thresholds (see quant.hip): thr[i] is the smallest
// float a in [2^(i+e0-1), 2^(i+e0)) for which glibc's floorf(log2f(a)) returns
// i+e0.  Uploaded once per device by be42_init().
constexpr int kFp8ThrE0 = -10;   // exponent of thr[0]
constexpr int kFp8ThrN = 21;     // exponents -10 .. 10
int fp8_thresholds_ready(int device);

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace be42

#define BE42_HIP(call)                                                          \
    do {                                                                        \
        hipError_t be42_e_ = (call);                                            \
        if (be42_e_ != hipSuccess)                                              \
            return be42::hip_fail(be42_e_, #call, __FILE__, __LINE__);          \
    } while (0)

#define BE42_CHECK(cond, ...)                                                   \
    do {                                                                        \
        if (!(cond)) {                                                          \
            be42::set_error(__VA_ARGS__);                                       \
            return BE42_EINVAL;                                                 \
        }                                                                       \
    } while (0)

#define BE42_LAUNCH_CHECK()                                                     \
    do {                                                                        \
        hipError_t be42_e_ = hipGetLastError();                                 \
        if (be42_e_ != hipSuccess)                                              \
            return be42::hip_fail(be42_e_, "kernel launch", __FILE__, __LINE__); \
    } while (0)

// --------------------------------------------------------------------------
// device helpers
// --------------------------------------------------------------------------
namespace be42 {

constexpr int kWave = 64;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef int v16i __attribute__((ext_vector_type(16)));

// s_waitcnt immediate that waits until at most N vector-memory operations of
// this wave are outstanding (expcnt and lgkmcnt left unconstrained).  The
// direct-to-LDS loads (global_load_lds_dwordx4) count here until their bytes
// are in LDS; the compiler does not order LDS reads after them by itself.
template <int N>
__device__ __forceinline__ void wait_vmcnt()
{
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Stage boundary of a direct-to-LDS ring shared by the waves of a block:
// wait until at most N vector-memory operations of this wave are outstanding
// and until every LDS read this wave issued has returned, then s_barrier.
// After it, every wave's loads older than its N newest are in LDS, and no
// wave still has a read of a ring slot in flight, so the slot the previous
// stage used may be refilled.  (A raw s_barrier, unlike __syncthreads, does
// not drain the loads still in flight for later stages.)  The empty asm
// statements keep the compiler from moving memory operations across it.
template <int N>
__device__ __forceinline__ void stage_barrier()
{
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (0 << 8));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
        v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
        v += __shfl_xor(v, o, kWave);
    return v;
}

// Wave-wide scans with DPP lane moves (no LDS crossbar round trips):
// row_shr / row_shl steps within each 16-lane row, then row_bcast:15 / :31
// (or readlane of the row totals) across rows.
template <int CTRL, int ROWMASK = 0xF>
__device__ __forceinline__ float dpp_mov(float old, float v)
{
    return __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROWMASK, 0xF, false));
}

// inclusive prefix max over lanes 0 .. lane
__device__ __forceinline__ float wave_prefix_max(float v)
{
    const float ninf = -INFINITY;
    v = fmaxf(v, dpp_mov<0x111>(ninf, v));          // row_shr:1
    v = fmaxf(v, dpp_mov<0x112>(ninf, v));          // row_shr:2
    v = fmaxf(v, dpp_mov<0x114>(ninf, v));          // row_shr:4
    v = fmaxf(v, dpp_mov<0x118>(ninf, v));          // row_shr:8
    v = fmaxf(v, dpp_mov<0x142, 0xA>(ninf, v));     // row_bcast:15 into rows 1, 3
    v = fmaxf(v, dpp_mov<0x143, 0xC>(ninf, v));     // row_bcast:31 into rows 2, 3
    return v;
}

// inclusive suffix product over lanes lane .. 63
__device__ __forceinline__ float wave_suffix_prod(float v)
{
    v = v * dpp_mov<0x101>(1.0f, v);                // row_shl:1
    v = v * dpp_mov<0x102>(1.0f, v);                // row_shl:2
    v = v * dpp_mov<0x104>(1.0f, v);                // row_shl:4
    v = v * dpp_mov<0x108>(1.0f, v);                // row_shl:8
    // lane 16 r now holds the product of row r
    const float t1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float t2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float t3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    const int row = (threadIdx.x & 63) >> 4;
    const float t23 = t2 * t3;
    return row == 0 ? v * (t1 * t23) : row == 1 ? v * t23 : row == 2 ? v * t3 : v;
}

// the value of lane - 1 (fill in lane 0) / of lane + 1 (fill in lane 63)
__device__ __forceinline__ float wave_shift_up1(float v, float fill) { return dpp_mov<0x138>(fill, v); }
__device__ __forceinline__ float wave_shift_down1(float v, float fill) { return dpp_mov<0x130>(fill, v); }

// sum over the wave (any order), in every lane
__device__ __forceinline__ float wave_sum_dpp(float v)
{
    v = v + dpp_mov<0x111>(0.0f, v);
    v = v + dpp_mov<0x112>(0.0f, v);
    v = v + dpp_mov<0x114>(0.0f, v);
    v = v + dpp_mov<0x118>(0.0f, v);
    v = v + dpp_mov<0x142, 0xA>(0.0f, v);
    v = v + dpp_mov<0x143, 0xC>(0.0f, v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ int wave_sum_i(int v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
        v += __shfl_xor(v, o, kWave);
    return v;
}

// Schraudolph exponential with the reference's clamps; the product and the
// bias are fused exactly as gcc fuses the reference expression.
__device__ __forceinline__ float fast_expf(float x)
{
    if (x < -87.0f)
        return 0.0f;
    if (x > 87.0f)
        x = 87.0f;
    return __int_as_float((int)__fmaf_rn(12102203.0f, x, 1065353216.0f));
}

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// round-to-nearest-even on the upper half, without a NaN case
__device__ __forceinline__ uint16_t f32_to_bf16(float f)
{
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// simd_dot_f32_f32 (simd_kernels.h:162-191) of q0 and c with the reference's
// reduction tree, computed by a lane pair (half = lane % 2): the eight
// accumulator chains i = k (mod 8) run with FMA in order, chains 0-3 in half 0
// and 4-7 in half 1 (one 16-byte load per lane per 8 elements); then
// t_k = s_k + s_{k+4}, ((t0+t1)+(t2+t3)), and the compiled scalar tail (4
// unfused products added in order when >= 4 remain, the rest fused).  hd is a
// multiple of 8, so the tail is empty for every pool; it is kept for parity
// with the reference routine.  The result is valid in half 0.
__device__ __forceinline__ float dot_ref8x2(const float *q0, const float *c, int hd, int half)
{
    const int main = hd & ~7;
    const float4 *c4 = (const float4 *)c;
    const float4 *q4 = (const float4 *)q0;
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll 8
    for (int j = 0; j < main / 8; j++) {
        const float4 cv = c4[2 * j + half], qv = q4[2 * j + half];
        s0 = __fmaf_rn(qv.x, cv.x, s0);
        s1 = __fmaf_rn(qv.y, cv.y, s1);
        s2 = __fmaf_rn(qv.z, cv.z, s2);
        s3 = __fmaf_rn(qv.w, cv.w, s3);
    }
    const float t0 = s0 + __shfl_down(s0, 1, 2);
    const float t1 = s1 + __shfl_down(s1, 1, 2);
    const float t2 = s2 + __shfl_down(s2, 1, 2);
    const float t3 = s3 + __shfl_down(s3, 1, 2);
    float sum = (t0 + t1) + (t2 + t3);
    if (half == 0) {
        int i = main;
        if (hd - i >= 4) {
            for (int j = 0; j < 4; j++)
                sum = sum + q0[i + j] * c[i + j];
            i += 4;
        }
        for (; i < hd; i++)
            sum = __fmaf_rn(q0[i], c[i], sum);
    }
    return sum;
}

// g_fp8_lut entry (ops_quant.c:27-48): E4M3, bias 7, no NaN (0x7F -> 480)
__device__ __forceinline__ float fp8_to_f32(uint8_t c)
{
    const int e = (c >> 3) & 0xF, m = c & 7;
    float v = (e == 0) ? (float)m * (1.0f / 512.0f)
                       : __uint_as_float((uint32_t)(e + 120) << 23) * (1.0f + (float)m * 0.125f);
    return (c & 0x80) ? -v : v;
}

}  // namespace be42
