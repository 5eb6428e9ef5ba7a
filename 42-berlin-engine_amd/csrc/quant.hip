// quant.hip -- INT8 / FP8 E4M3 codecs of the reference, row-wise, on gfx950.
//
// quant_f32_to_int8  src/compute/ops_quant.c:229-270
// quant_f32_to_fp8   src/compute/ops_quant.c:103-136 (float_to_fp8 :68-98)
// g_fp8_lut          src/compute/ops_quant.c:18-63
//
// Codes and scales are bit-identical to the reference: the absmax is an exact
// max reduction, the divisions are IEEE divisions, roundf rounds half away
// from zero, and the FP8 exponent reproduces glibc's floorf(log2f(a)) through
// a per-binade threshold table measured on the host at init.
#include <cmath>
#include <cstring>

#include "be42_common.h"

namespace be42 {

__constant__ float c_fp8_thr[kFp8ThrN];

// Reference E4M3 encoder (ops_quant.c:68-98) on the device.
__device__ __forceinline__ uint8_t f32_to_fp8(float v)
{
    if (v == 0.0f)
        return 0;
    const uint32_t sign = v < 0.0f ? 0x80u : 0u;
    float a = fabsf(v);
    if (a > 448.0f)
        a = 448.0f;
    int ex = (int)((__float_as_uint(a) >> 23) & 0xFF) - 127;   // floor(log2 a), a normal
    if ((__float_as_uint(a) >> 23) == 0)
        ex = -127;                                            // subnormal: far below e = 0
    const int up = ex + 1;
    if (up >= kFp8ThrE0 && up < kFp8ThrE0 + kFp8ThrN && a >= c_fp8_thr[up - kFp8ThrE0])
        ex = up;                                              // log2f rounded up to an integer
    int e = ex + 7;
    e = e < 0 ? 0 : (e > 15 ? 15 : e);
    const float frac = (e == 0) ? a * 64.0f
                                : a * __uint_as_float((uint32_t)(127 + 7 - e) << 23) - 1.0f;
    int m = (int)__fmaf_rn(frac, 8.0f, 0.5f);
    if (m > 7)
        m = 7;
    return (uint8_t)(sign | ((uint32_t)e << 3) | (uint32_t)m);
}


// block-wide absmax of one row (256 threads)
__device__ __forceinline__ float row_absmax(const float *x, int cols, float *red)
{
    float m = 0.0f;
    for (int i = threadIdx.x; i < cols; i += blockDim.x)
        m = fmaxf(m, fabsf(x[i]));
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = m;
    __syncthreads();
    float r = red[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); w++)
        r = fmaxf(r, red[w]);
    return r;
}

__global__ __launch_bounds__(256) void k_quant_rows_int8(int8_t *q, float *scales, const float *x,
                                                         int cols)
{
    __shared__ float red[4];
    const size_t row = blockIdx.x;
    const float *xr = x + row * cols;
    const float amax = row_absmax(xr, cols, red);
    float scale = 1.0f, inv = 1.0f;
    if (amax > 0.0f) {
        scale = amax / 127.0f;
        inv = 127.0f / amax;
    }
    if (threadIdx.x == 0)
        scales[row] = scale;
    for (int i = threadIdx.x; i < cols; i += blockDim.x) {
        int v = (int)roundf(xr[i] * inv);
        v = v > 127 ? 127 : (v < -127 ? -127 : v);
        q[row * cols + i] = (int8_t)v;
    }
}

__global__ __launch_bounds__(256) void k_quant_rows_fp8(uint8_t *q, float *scales, const float *x,
                                                        int cols)
{
    __shared__ float red[4];
    const size_t row = blockIdx.x;
    const float *xr = x + row * cols;
    const float amax = row_absmax(xr, cols, red);
    float scale = 1.0f, inv = 1.0f;
    if (amax > 0.0f) {
        scale = amax / 224.0f;
        inv = 1.0f / scale;
    }
    if (threadIdx.x == 0)
        scales[row] = scale;
    for (int i = threadIdx.x; i < cols; i += blockDim.x)
        q[row * cols + i] = f32_to_fp8(xr[i] * inv);
}

__global__ void k_dequant_rows_int8(float *out, const int8_t *q, const float *scales, int cols,
                                    size_t total)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x)
        out[i] = (float)q[i] * scales[i / cols];
}

__global__ void k_fp8_decode(float *out, const uint8_t *q, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        out[i] = fp8_to_f32(q[i]);
}

// Threshold table of glibc's log2f: smallest float in [2^(E-1), 2^E) whose
// floorf(log2f()) is E (log2f rounds up within a few ulps of 2^E).
static void host_fp8_thresholds(float *thr)
{
    for (int i = 0; i < kFp8ThrN; i++) {
        const int E = kFp8ThrE0 + i;
        float a = ldexpf(1.0f, E);
        for (int step = 0; step < 64; step++) {
            const float b = nextafterf(a, 0.0f);
            if ((int)floorf(log2f(b)) != E)
                break;
            a = b;
        }
        thr[i] = a;
    }
}

static int g_thr_ready[64];

int upload_fp8_thresholds(int device)
{
    if (device < 0 || device >= 64)
        return BE42_EINVAL;
    if (g_thr_ready[device])
        return BE42_OK;
    float thr[kFp8ThrN];
    host_fp8_thresholds(thr);
    BE42_HIP(hipMemcpyToSymbol(HIP_SYMBOL(c_fp8_thr), thr, sizeof thr));
    g_thr_ready[device] = 1;
    return BE42_OK;
}

int fp8_thresholds_ready(int device) { return device >= 0 && device < 64 && g_thr_ready[device]; }

}  // namespace be42

using namespace be42;

static int ensure_thresholds()
{
    int dev = 0;
    BE42_HIP(hipGetDevice(&dev));
    if (!fp8_thresholds_ready(dev))
        return upload_fp8_thresholds(dev);
    return BE42_OK;
}

extern "C" int be42_quant_rows_int8(int8_t *q, float *scales, const float *x, int rows, int cols,
                                    void *stream)
{
    BE42_CHECK(q && scales && x, "be42_quant_rows_int8: null pointer");
    BE42_CHECK(rows >= 0 && cols > 0, "be42_quant_rows_int8: bad shape %d x %d", rows, cols);
    if (rows == 0)
        return BE42_OK;
    hipLaunchKernelGGL(k_quant_rows_int8, dim3(rows), dim3(256), 0, as_stream(stream), q, scales, x, cols);
    BE42_LAUNCH_CHECK();
    return BE42_OK;
}

extern "C" int be42_quant_rows_fp8(uint8_t *q, float *scales, const float *x, int rows, int cols,
                                   void *stream)
{
    BE42_CHECK(q && scales && x, "be42_quant_rows_fp8: null pointer");
    BE42_CHECK(rows >= 0 && cols > 0, "be42_quant_rows_fp8: bad shape %d x %d", rows, cols);
    int rc = ensure_thresholds();
    if (rc)
        return rc;
    if (rows == 0)
        return BE42_OK;
    hipLaunchKernelGGL(k_quant_rows_fp8, dim3(rows), dim3(256), 0, as_stream(stream), q, scales, x, cols);
    BE42_LAUNCH_CHECK();
    return BE42_OK;
}

extern "C" int be42_dequant_rows_int8(float *out, const int8_t *q, const float *scales, int rows,
                                      int cols, void *stream)
{
    BE42_CHECK(out && q && scales, "be42_dequant_rows_int8: null pointer");
    BE42_CHECK(rows >= 0 && cols > 0, "be42_dequant_rows_int8: bad shape");
    size_t total = (size_t)rows * cols;
    if (total == 0)
        return BE42_OK;
    int blocks = (int)((total + 255) / 256);
    if (blocks > 8192)
        blocks = 8192;
    hipLaunchKernelGGL(k_dequant_rows_int8, dim3(blocks), dim3(256), 0, as_stream(stream), out, q, scales,
                       cols, total);
    BE42_LAUNCH_CHECK();
    return BE42_OK;
}

extern "C" int be42_fp8_decode(float *out, const uint8_t *q, size_t n, void *stream)
{
    BE42_CHECK(out && q, "be42_fp8_decode: null pointer");
    if (n == 0)
        return BE42_OK;
    int blocks = (int)((n + 255) / 256);
    if (blocks > 8192)
        blocks = 8192;
    hipLaunchKernelGGL(k_fp8_decode, dim3(blocks), dim3(256), 0, as_stream(stream), out, q, n);
    BE42_LAUNCH_CHECK();
    return BE42_OK;
}
