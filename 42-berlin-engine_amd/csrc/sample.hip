// sample.hip -- temperature and top-p sampling of logits on gfx950.
//
// sample_temperature  src/compute/sampler_temp.c:57-114
// sample_top_p        src/compute/sampler_topp.c:17-158
//
// Both turn logits into probabilities p_i = expf((x_i - max) / temp) / sum
// (the temperature sampler starts its max at -1e9, top-p at x_0), then draw
// one index with a uniform number the caller supplies:
//   temperature: the first index whose running sum of p exceeds r
//                (sampler_random_float's draw);
//   top-p:       p sorted descending (a stable radix sort: equal
//                probabilities keep ascending index order, where the
//                reference's qsort leaves them unspecified), the shortest
//                prefix whose running sum exceeds top_p, r = u * that sum
//                (u = rand() / RAND_MAX), the first sorted entry whose
//                running sum exceeds r.
// The sums run as block-wide scans: equal to the reference's sequential sums
// to fp32 rounding, so the drawn index is the reference's unless r lies within
// that rounding of a boundary.  Where no running sum exceeds r (possible only
// through rounding) the reference returns n, an index past the vocabulary;
// here the last index is returned.
#include <cstring>

#include <rocprim/device/device_radix_sort.hpp>

#include "be42_common.h"

namespace be42 {

constexpr int kSampT = 1024;

__device__ __forceinline__ float block_reduce(float v, float *red, bool is_max)
{
    v = is_max ? wave_max(v) : wave_sum(v);
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0)
        red[wave] = v;
    __syncthreads();
    float r = red[0];
    for (int w = 1; w < kSampT / 64; w++)
        r = is_max ? fmaxf(r, red[w]) : r + red[w];
    return r;
}

// p[b][i] = expf((x - m) / temp) / sum for row b (one block per row)
template <bool BF16>
__global__ __launch_bounds__(kSampT) void k_probs(float *__restrict__ p, const void *__restrict__ logits, int n,
                                                  float temp, bool max_from_first)
{
    __shared__ float red[kSampT / 64];
    const int b = blockIdx.x;
    auto x = [&](int i) {
        return BF16 ? bf16_to_f32(((const uint16_t *)logits)[(size_t)b * n + i])
                    : ((const float *)logits)[(size_t)b * n + i];
    };
    float m = max_from_first ? x(0) : -1e9f;
    for (int i = threadIdx.x; i < n; i += kSampT)
        m = fmaxf(m, x(i));
    m = block_reduce(m, red, true);
    float *pb = p + (size_t)b * n;
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += kSampT) {
        const float e = expf(__fdiv_rn(x(i) - m, temp));
        pb[i] = e;
        s += e;
    }
    s = block_reduce(s, red, false);
    for (int i = threadIdx.x; i < n; i += kSampT)
        pb[i] = __fdiv_rn(pb[i], s);
}

// Exclusive block scan of one float per thread (thread order).
__device__ __forceinline__ float block_excl_scan(float v, float *sh)
{
    sh[threadIdx.x] = v;
    __syncthreads();
    for (int o = 1; o < kSampT; o <<= 1) {
        const float a = threadIdx.x >= (unsigned)o ? sh[threadIdx.x - o] : 0.0f;
        __syncthreads();
        sh[threadIdx.x] += a;
        __syncthreads();
    }
    const float incl = sh[threadIdx.x];
    return incl - v;
}

// The first position i < lim (thread t walks the contiguous chunk
// [t C, (t + 1) C)) whose running sum of q exceeds thr, or -1; with thr_rel the
// threshold is thr times the running sum at position lim - 1.
__device__ int block_first_exceeding(const float *__restrict__ q, int lim, float thr, bool thr_rel, float *sh,
                                     int *found, float *total)
{
    const int C = (lim + kSampT - 1) / kSampT;
    const int i0 = min(lim, (int)threadIdx.x * C), i1 = min(lim, i0 + C);
    float cs = 0.0f;
    for (int i = i0; i < i1; i++)
        cs += q[i];
    const float pre = block_excl_scan(cs, sh);
    if (threadIdx.x == kSampT - 1)
        *total = pre + cs;
    if (threadIdx.x == 0)
        *found = INT32_MAX;
    __syncthreads();
    const float r = thr_rel ? thr * *total : thr;
    float cum = pre;
    for (int i = i0; i < i1; i++) {
        cum += q[i];
        if (cum > r) {
            atomicMin(found, i);
            break;
        }
    }
    __syncthreads();
    const int f = *found;
    __syncthreads();
    return f == INT32_MAX ? -1 : f;
}

__global__ __launch_bounds__(kSampT) void k_pick_temperature(int *__restrict__ out, const float *__restrict__ p, int n,
                                                             const float *__restrict__ r)
{
    __shared__ float sh[kSampT];
    __shared__ int found;
    __shared__ float total;
    const int b = blockIdx.x;
    const int i = block_first_exceeding(p + (size_t)b * n, n, r[b], false, sh, &found, &total);
    if (threadIdx.x == 0)
        out[b] = i < 0 ? n - 1 : i;
}

// sorted probabilities ps and their indices: cut at top_p, then draw
__global__ __launch_bounds__(kSampT) void k_pick_top_p(int *__restrict__ out, const float *__restrict__ ps,
                                                       const int *__restrict__ idx, int n, float top_p,
                                                       const float *__restrict__ u)
{
    __shared__ float sh[kSampT];
    __shared__ int found;
    __shared__ float total;
    const int b = blockIdx.x;
    const float *pb = ps + (size_t)b * n;
    const int *ib = idx + (size_t)b * n;
    // the set: the prefix through the first running sum above top_p
    const int c = block_first_exceeding(pb, n, top_p, false, sh, &found, &total);
    const int count = c < 0 ? n : c + 1;
    // r = u * (the set's running sum); the first entry whose running sum exceeds it
    const int j = block_first_exceeding(pb, count, u[b], true, sh, &found, &total);
    if (threadIdx.x == 0)
        out[b] = ib[j < 0 ? count - 1 : j];
}

__global__ void k_iota_rows(int *__restrict__ v, int n, int batch)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < (size_t)n * batch)
        v[i] = (int)(i % n);
}

int probs_launch(float *p, const void *logits, bool bf16, int n, int batch, float temp, bool max_first,
                 hipStream_t s)
{
    if (bf16)
        hipLaunchKernelGGL(k_probs<true>, dim3(batch), dim3(kSampT), 0, s, p, logits, n, temp, max_first);
    else
        hipLaunchKernelGGL(k_probs<false>, dim3(batch), dim3(kSampT), 0, s, p, logits, n, temp, max_first);
    BE42_LAUNCH_CHECK();
    return BE42_OK;
}

}  // namespace be42

using namespace be42;

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// logits_bf16: logits are bf16 (the reference's DTYPE_BF16 tensors)
extern "C" int be42_sample_temperature_dt(int *out, const void *logits, int logits_bf16, int n, int batch, float temp,
                                          const float *r, void *stream)
{
    BE42_CHECK(out && logits && r, "be42_sample_temperature: null pointer");
    BE42_CHECK(n > 0 && batch > 0, "be42_sample_temperature: n %d, batch %d", n, batch);
    hipStream_t s = as_stream(stream);
    float *p = (float *)workspace((size_t)n * batch * 4, s);
    if (!p)
        return BE42_ENOMEM;
    const int rc = probs_launch(p, logits, logits_bf16 != 0, n, batch, temp, false, s);
    if (rc)
        return rc;
    hipLaunchKernelGGL(k_pick_temperature, dim3(batch), dim3(kSampT), 0, s, out, p, n, r);
    BE42_LAUNCH_CHECK();
    return BE42_OK;
}

extern "C" int be42_sample_temperature(int *out, const float *logits, int n, int batch, float temp, const float *r,
                                       void *stream)
{
    return be42_sample_temperature_dt(out, logits, 0, n, batch, temp, r, stream);
}

extern "C" int be42_sample_top_p_dt(int *out, const void *logits, int logits_bf16, int n, int batch, float temp,
                                    float top_p, const float *u, void *stream)
{
    BE42_CHECK(out && logits && u, "be42_sample_top_p: null pointer");
    BE42_CHECK(n > 0 && batch > 0, "be42_sample_top_p: n %d, batch %d", n, batch);
    hipStream_t s = as_stream(stream);
    const size_t rowsz = (size_t)n * batch;
    size_t sort_bytes = 0;
    BE42_HIP(rocprim::radix_sort_pairs_desc(nullptr, sort_bytes, (const float *)nullptr, (float *)nullptr,
                                            (const int *)nullptr, (int *)nullptr, (unsigned)n, 0, 32, s));
    const size_t fb = align256(rowsz * 4);
    uint8_t *ws = (uint8_t *)workspace(4 * fb + align256(sort_bytes), s);
    if (!ws)
        return BE42_ENOMEM;
    float *p = (float *)ws, *ps = (float *)(ws + fb);
    int *iv = (int *)(ws + 2 * fb), *is = (int *)(ws + 3 * fb);
    void *tmp = ws + 4 * fb;
    int rc = probs_launch(p, logits, logits_bf16 != 0, n, batch, temp, true, s);
    if (rc)
        return rc;
    hipLaunchKernelGGL(k_iota_rows, dim3((unsigned)((rowsz + 255) / 256)), dim3(256), 0, s, iv, n, batch);
    BE42_LAUNCH_CHECK();
    for (int b = 0; b < batch; b++) {
        size_t bytes = sort_bytes;
        BE42_HIP(rocprim::radix_sort_pairs_desc(tmp, bytes, p + (size_t)b * n, ps + (size_t)b * n, iv + (size_t)b * n,
                                                is + (size_t)b * n, (unsigned)n, 0, 32, s));
    }
    hipLaunchKernelGGL(k_pick_top_p, dim3(batch), dim3(kSampT), 0, s, out, ps, is, n, top_p, u);
    BE42_LAUNCH_CHECK();
    return BE42_OK;
}

extern "C" int be42_sample_top_p(int *out, const float *logits, int n, int batch, float temp, float top_p,
                                 const float *u, void *stream)
{
    return be42_sample_top_p_dt(out, logits, 0, n, batch, temp, top_p, u, stream);
}
