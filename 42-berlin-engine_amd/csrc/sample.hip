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
//   top-p:       in the order of p descending (equal probabilities in
//                ascending index order, where the reference's qsort leaves
//                them unspecified), the shortest prefix whose running sum
//                exceeds top_p, r = u * that sum (u = rand() / RAND_MAX),
//                the first entry of the prefix whose running sum exceeds r.
// The temperature sampler's running sums are formed 64 entries at a time
// (lane prefix sums plus a carried sum), equal to the reference's
// sequential fp32 sums to rounding.  Where no running sum exceeds
// r (possible only through rounding) the reference returns n, an index past
// the vocabulary; here the last index is returned.
//
// Top-p never sorts: both cuts are weighted selections.  The entry at which
// the descending-order running sum first exceeds a threshold is found by a
// most-significant-byte-first radix select over the bit patterns of the
// (non-negative) probabilities, where each pass sums the probabilities of the
// remaining candidates per byte value and keeps the byte whose bucket holds
// the crossing; after four passes the crossing entry's value is known, and
// among the entries of that value (ascending index) the crossing is the
// (T - sum above) / value-th.  The sums are exact: probabilities as 62-bit
// fixed point (p * 2^62, truncated) in 64-bit integer additions, so they do
// not depend on the order of the atomic additions, and they are the float64
// running sums to ~n * 2^-62 -- closer than the reference's fp32 sums.
#include <cstring>

#include "be42_common.h"

namespace be42 {

constexpr int kSampT = 1024;

// The loops below read a row with their loads issued U at a time (the
// values into registers first, then used in the same order as one at a
// time): a loop that uses each value as it arrives waits a full memory
// round trip per element, and one block walks a whole 128k-entry row.
//   strided: i = t, t + kSampT, ... (thread t), f(i, v)
template <int U, class Ld, class F>
__device__ __forceinline__ void strided_batches(int n, Ld &&ld, F &&f)
{
    for (int i0 = threadIdx.x; i0 < n; i0 += U * kSampT) {
        decltype(ld(0)) v[U];
#pragma unroll
        for (int j = 0; j < U; j++) {
            const int i = i0 + j * kSampT;
            v[j] = ld(i < n ? i : i0);
        }
#pragma unroll
        for (int j = 0; j < U; j++)
            if (i0 + j * kSampT < n)
                f(i0 + j * kSampT, v[j]);
    }
}
//   wave:    entries c0 .. c1 - 1 of one wave, 64 a step (lane l: entry
//            a + l, T(0) past c1), f(a, v) returns true (wave-uniform) to stop
template <int U, class T, class F>
__device__ __forceinline__ void wave_steps(const T *__restrict__ q, int c0, int c1, F &&f)
{
    const int lane = threadIdx.x & (kWave - 1);
    for (int a0 = c0; a0 < c1; a0 += kWave * U) {
        T v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = a0 + kWave * u + lane;
            v[u] = i < c1 ? q[i] : T(0);
        }
#pragma unroll
        for (int u = 0; u < U; u++)
            if (a0 + kWave * u < c1 && f(a0 + kWave * u, v[u]))
                return;
    }
}

// the block's row split into one contiguous range per wave, whole steps of 64
__device__ __forceinline__ void wave_range(int n, int &c0, int &c1)
{
    constexpr int NW = kSampT / kWave;
    const int cw = (((n + NW - 1) / NW) + kWave - 1) & ~(kWave - 1);
    c0 = min(n, (int)(threadIdx.x / kWave) * cw);
    c1 = min(n, c0 + cw);
}

// inclusive prefix sum over the lanes (DPP row shifts, then row broadcasts)
__device__ __forceinline__ float wave_prefix_sum(float v)
{
    v = v + dpp_mov<0x111>(0.0f, v);         // row_shr:1
    v = v + dpp_mov<0x112>(0.0f, v);         // row_shr:2
    v = v + dpp_mov<0x114>(0.0f, v);         // row_shr:4
    v = v + dpp_mov<0x118>(0.0f, v);         // row_shr:8
    v = v + dpp_mov<0x142, 0xA>(0.0f, v);    // row_bcast:15 into rows 1, 3
    v = v + dpp_mov<0x143, 0xC>(0.0f, v);    // row_bcast:31 into rows 2, 3
    return v;
}
__device__ __forceinline__ float lane63(float v) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63)); }

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
    strided_batches<16>(n, x, [&](int, float v) { m = fmaxf(m, v); });
    m = block_reduce(m, red, true);
    float *pb = p + (size_t)b * n;
    float s = 0.0f;
    strided_batches<16>(n, x, [&](int i, float v) {
        const float e = expf(__fdiv_rn(v - m, temp));
        pb[i] = e;
        s += e;
    });
    s = block_reduce(s, red, false);
    strided_batches<16>(n, [&](int i) { return pb[i]; }, [&](int i, float v) { pb[i] = __fdiv_rn(v, s); });
}

// The first position i < lim whose running sum of q exceeds thr, or -1.
// Each wave walks its own contiguous range 64 entries a step; a step's
// running sums are the lanes' prefix sums plus the sum carried from the
// steps before (the range's first step carries the sum of the ranges before).
// sh: 2 * (kSampT / 64) floats.
__device__ int block_first_exceeding(const float *__restrict__ q, int lim, float thr, float *sh, int *found)
{
    constexpr int NW = kSampT / kWave;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
    int c0, c1;
    wave_range(lim, c0, c1);
    float carry = 0.0f;
    wave_steps<8>(q, c0, c1, [&](int, float v) {
        carry += lane63(wave_prefix_sum(v));
        return false;
    });
    if (lane == 0)
        sh[wave] = carry;
    if (threadIdx.x == 0)
        *found = INT32_MAX;
    __syncthreads();
    if (threadIdx.x == 0) {
        float o = 0.0f;
        for (int w = 0; w < NW; w++) {
            const float t = sh[w];
            sh[NW + w] = o;
            o += t;
        }
    }
    __syncthreads();
    carry = sh[NW + wave];
    wave_steps<8>(q, c0, c1, [&](int a, float v) {
        const float ps = wave_prefix_sum(v);
        const unsigned long long m = __ballot(carry + ps > thr);
        if (m) {
            if (lane == 0)
                atomicMin(found, a + __ffsll((unsigned long long)m) - 1);
            return true;
        }
        carry += lane63(ps);
        return false;
    });
    __syncthreads();
    const int f = *found;
    __syncthreads();
    return f == INT32_MAX ? -1 : f;
}

__global__ __launch_bounds__(kSampT) void k_pick_temperature(int *__restrict__ out, const float *__restrict__ p, int n,
                                                             const float *__restrict__ r)
{
    __shared__ float sh[2 * (kSampT / kWave)];
    __shared__ int found;
    const int b = blockIdx.x;
    const int i = block_first_exceeding(p + (size_t)b * n, n, r[b], sh, &found);
    if (threadIdx.x == 0)
        out[b] = i < 0 ? n - 1 : i;
}

// the bit fields of a probability's pattern the three passes resolve
// (12, 12 and 8 bits: the first pass spreads over exponent and 4 mantissa
// bits, so the atomic additions of one wave rarely meet in one bucket)
constexpr int kSelPasses = 3;
constexpr int kSelShift[kSelPasses] = {20, 8, 0};
constexpr int kSelBits[kSelPasses] = {12, 12, 8};
constexpr int kSelBins = 1 << 12;

// p as 62-bit fixed point, floor(p * 2^62), from the bits of p in [0, 1]:
// mantissa (with its leading 1) shifted by exponent - 88 (0 for zero,
// subnormal, negative or NaN patterns; those above 1 do not occur)
__device__ __forceinline__ unsigned long long fixp_bits(unsigned k)
{
    const int e = (int)(k >> 23);   // the sign bit makes negative patterns > 255
    if (e == 0 || e > 127)
        return 0ull;
    const unsigned long long m = (unsigned long long)((k & 0x7FFFFFu) | 0x800000u);
    const int sh = e - 88;
    return sh >= 0 ? m << sh : (sh > -64 ? m >> -sh : 0ull);
}
__device__ __forceinline__ unsigned long long fixp(float p) { return fixp_bits(__float_as_uint(p)); }

struct TopPShared {
    unsigned long long hist[kSelBins];   // bucket sums of a pass
    unsigned long long scan[kSampT];
    int isum[kSampT / kWave];
    unsigned long long total, above;
    int pos, bin, idx;
};

// Exclusive block scan of one value per thread (thread order).
template <class T>
__device__ __forceinline__ T block_excl_scan_t(T v, T *sh)
{
    sh[threadIdx.x] = v;
    __syncthreads();
    for (int o = 1; o < kSampT; o <<= 1) {
        const T a = threadIdx.x >= (unsigned)o ? sh[threadIdx.x - o] : T(0);
        __syncthreads();
        sh[threadIdx.x] += a;
        __syncthreads();
    }
    const T incl = sh[threadIdx.x];
    __syncthreads();
    return incl - v;
}

// The entry of p[0 .. n) at which the running sum of fixp(p), taken in
// descending order of p with equal values in ascending index order, first
// exceeds T; -1 if none does.  *above: the running sum before that entry;
// *all: the sum of every entry.  Called by the whole block.
__device__ int weighted_select(const float *__restrict__ p, int n, unsigned long long T, TopPShared &S,
                               unsigned long long *above, unsigned long long *all)
{
    const int tid = threadIdx.x;
    unsigned prefix = 0, pmask = 0;
    unsigned long long base = 0;   // the sum of the entries above the current bucket
    for (int pass = 0; pass < kSelPasses; pass++) {
        const int shift = kSelShift[pass], nb = 1 << kSelBits[pass];
        for (int i = tid; i < nb; i += kSampT)
            S.hist[i] = 0ull;
        if (tid == 0)
            S.pos = INT32_MAX;
        __syncthreads();
        strided_batches<16>(n, [&](int i) { return __float_as_uint(p[i]); }, [&](int, unsigned k) {
            if ((k & pmask) == prefix) {
                const unsigned long long f = fixp_bits(k);
                if (f)
                    atomicAdd(&S.hist[(k >> shift) & (nb - 1)], f);
            }
        });
        __syncthreads();
        // thread t takes the buckets at descending positions 4t .. 4t + 3
        unsigned long long h[4], ts = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int d = 4 * tid + j;
            h[j] = d < nb ? S.hist[nb - 1 - d] : 0ull;
            ts += h[j];
        }
        const unsigned long long ex = block_excl_scan_t<unsigned long long>(ts, S.scan);
        if (pass == 0 && tid == kSampT - 1)
            S.total = ex + ts;
        unsigned long long acc = base + ex;
        int hit = -1;
        unsigned long long hit_above = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (hit < 0 && h[j] && acc + h[j] > T) {
                hit = 4 * tid + j;
                hit_above = acc;
            }
            acc += h[j];
        }
        if (hit >= 0)
            atomicMin(&S.pos, hit);
        __syncthreads();
        const int pos = S.pos;
        if (hit >= 0 && hit == pos) {
            S.bin = nb - 1 - pos;
            S.above = hit_above;
        }
        __syncthreads();
        if (pass == 0)
            *all = S.total;
        const int bin = S.bin;
        base = S.above;
        __syncthreads();   // S is rewritten by the next pass
        if (pos == INT32_MAX)
            return -1;
        prefix |= (unsigned)bin << shift;
        pmask |= (unsigned)(nb - 1) << shift;
    }
    // the crossing entry has the value whose bits are `prefix`; among the
    // entries of that value (ascending index) it is the k-th
    const unsigned long long fv = fixp(__uint_as_float(prefix));   // > 0: its bucket's sum is positive
    const unsigned long long k = (T - base) / fv;
    const int wave = tid / kWave, lane = tid & (kWave - 1);
    int c0, c1;
    wave_range(n, c0, c1);
    auto match = [&](int a, float v) { return __ballot(a + lane < c1 && __float_as_uint(v) == prefix); };
    int cnt = 0;   // entries of that value in this wave's range
    wave_steps<8>(p, c0, c1, [&](int a, float v) {
        cnt += __popcll(match(a, v));
        return false;
    });
    if (lane == 0)
        S.isum[wave] = cnt;
    if (tid == 0)
        S.idx = -1;
    __syncthreads();
    int off = 0;
    for (int w = 0; w < wave; w++)
        off += S.isum[w];
    if ((unsigned long long)off <= k && k < (unsigned long long)(off + cnt)) {
        int rem = (int)(k - (unsigned long long)off);
        wave_steps<8>(p, c0, c1, [&](int a, float v) {
            unsigned long long m = match(a, v);
            const int c = __popcll(m);
            if (rem < c) {
                for (int j = 0; j < rem; j++)
                    m &= m - 1;
                if (lane == 0)
                    S.idx = a + __ffsll(m) - 1;
                return true;
            }
            rem -= c;
            return false;
        });
    }
    __syncthreads();
    *above = base + k * fv;
    const int idx = S.idx;
    __syncthreads();
    return idx;
}

// The last entry in descending order: the smallest value, the largest index
// among equal ones.
__device__ int last_entry(const float *__restrict__ p, int n, TopPShared &S)
{
    const int tid = threadIdx.x;
    unsigned long long best = 0;   // (~key << 32 | index): the largest is the last entry
    strided_batches<16>(n, [&](int i) { return __float_as_uint(p[i]); }, [&](int i, unsigned k) {
        const unsigned long long c = ((unsigned long long)~k << 32) | (unsigned)i;
        best = c > best ? c : best;
    });
    unsigned long long *words = S.scan;
    words[tid] = best;
    __syncthreads();
    if (tid == 0) {
        unsigned long long t = 0;
        for (int i = 0; i < kSampT; i++)
            t = words[i] > t ? words[i] : t;
        S.idx = (int)(unsigned)t;
    }
    __syncthreads();
    const int idx = S.idx;
    __syncthreads();
    return idx;
}

// probabilities p (one row per block): cut at top_p, then draw with u
__global__ __launch_bounds__(kSampT) void k_top_p(int *__restrict__ out, const float *__restrict__ p, int n,
                                                  float top_p, const float *__restrict__ u)
{
    __shared__ TopPShared S;
    const float *pb = p + (size_t)blockIdx.x * n;
    // the set: through the first entry whose running sum exceeds top_p
    // (the sums stay near 2^62: a threshold of 2 or more is never exceeded)
    const unsigned long long T1 =
        top_p >= 2.0f ? ~0ull : (top_p > 0.0f ? (unsigned long long)((double)top_p * 0x1p62) : 0ull);
    unsigned long long above, all;
    const int c = weighted_select(pb, n, T1, S, &above, &all);
    const unsigned long long total = c >= 0 ? above + fixp(pb[c]) : all;
    // r = u * (the set's sum); the first entry whose running sum exceeds it,
    // or the set's last entry when none does
    const float uu = u[blockIdx.x];
    const unsigned long long R = uu > 0.0f ? (unsigned long long)fmin((double)uu * (double)total, 1.8e19) : 0ull;
    int pick = -1;
    if (R < total) {
        unsigned long long a2, all2;
        pick = weighted_select(pb, n, R, S, &a2, &all2);
    }
    if (pick < 0)
        pick = c >= 0 ? c : last_entry(pb, n, S);
    if (threadIdx.x == 0)
        out[blockIdx.x] = pick;
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
    float *p = (float *)workspace((size_t)n * batch * 4, s);
    if (!p)
        return BE42_ENOMEM;
    const int rc = probs_launch(p, logits, logits_bf16 != 0, n, batch, temp, true, s);
    if (rc)
        return rc;
    hipLaunchKernelGGL(k_top_p, dim3(batch), dim3(kSampT), 0, s, out, p, n, top_p, u);
    BE42_LAUNCH_CHECK();
    return BE42_OK;
}

extern "C" int be42_sample_top_p(int *out, const float *logits, int n, int batch, float temp, float top_p,
                                 const float *u, void *stream)
{
    return be42_sample_top_p_dt(out, logits, 0, n, batch, temp, top_p, u, stream);
}
