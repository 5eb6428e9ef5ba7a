// dropin.hip -- the reference-named C ABI of the decode hot path
// (include/be42_engine.h) on top of the be42 device library.
//
// Each entry point keeps the reference's name, arguments, struct contents and
// error behaviour and runs its arithmetic on the GPU:
//   op_matmul                 src/compute/ops_matmul.c:366-477
//   quant codecs              src/compute/ops_quant.c:18-305
//   lsh_*                     src/compute/ops_lsh.c:40-430
//   block manager, paged KV   src/memory/paged.c:29-495
//   paged attention           src/compute/ops_attention.c:353-470
// Host arrays in and out are staged through device buffers on the legacy
// null stream, so each call is ordered after the previous one and complete
// on return; device pointers are used in place.  Only bookkeeping (the
// page allocator mirror, the LSH bucket chains, argument checks) runs on the
// host.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <ctime>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "be42_common.h"
#include "be42_engine.h"
#include "heap_wave.h"

namespace be42 {
namespace {

// ---- kernels ----------------------------------------------------------------

// out[c][r] = in[r][c] for an R x C fp32 matrix, 32 x 32 tiles through LDS.
__global__ __launch_bounds__(256) void k_transpose(float *__restrict__ out, const float *__restrict__ in, int R,
                                                   int C)
{
    __shared__ float t[32][33];
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int i = ty; i < 32; i += 8)
        if (r0 + i < R && c0 + tx < C)
            t[i][tx] = in[(size_t)(r0 + i) * C + c0 + tx];
    __syncthreads();
    for (int i = ty; i < 32; i += 8)
        if (c0 + i < C && r0 + tx < R)
            out[(size_t)(c0 + i) * R + r0 + tx] = t[tx][i];
}

// Dense op_matmul cases (ops_matmul.c:383-470): out[i][c] = sum_j a[i][j] *
// b[j][c] with a BF16 or F32 [m][k], b F32 or BF16 [k][n], fp32 accumulation,
// output F32 or BF16 (float_to_bf16, tensor.c:67-76).  One wave per output
// row i and column chunk of up to 8 columns.
template <typename WT, typename XT, bool OBF16>
__global__ __launch_bounds__(256) void k_dense_mm(void *__restrict__ out, const WT *__restrict__ a,
                                                  const XT *__restrict__ b, int m, int k, int n)
{
    const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6, lane = threadIdx.x & 63;
    const int chunks = (n + 7) / 8;
    if (wave >= m * chunks)
        return;
    const int i = wave / chunks, c0 = (wave % chunks) * 8, nc = min(8, n - c0);
    auto ld = [](auto v) -> float {
        if constexpr (sizeof(v) == 2)
            return bf16_to_f32(v);
        else
            return (float)v;
    };
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const WT *ar = a + (size_t)i * k;
    for (int j = lane; j < k; j += 64) {
        const float w = ld(ar[j]);
        const XT *br = b + (size_t)j * n + c0;
#pragma unroll
        for (int c = 0; c < 8; c++)
            if (c < nc)
                acc[c] = __fmaf_rn(w, ld(br[c]), acc[c]);
    }
#pragma unroll
    for (int c = 0; c < 8; c++)
        acc[c] = wave_sum(acc[c]);
    if (lane < nc) {
        float v = acc[0];
#pragma unroll
        for (int c = 1; c < 8; c++)
            if (lane == c)
                v = acc[c];
        if (OBF16)
            ((uint16_t *)out)[(size_t)i * n + c0 + lane] = f32_to_bf16(v);
        else
            ((float *)out)[(size_t)i * n + c0 + lane] = v;
    }
}

// calc_block_centroid_int8 (paged.c:350-393): per-dim sequential sum of the
// dequantized head-0 keys of the n tokens, then * (1.0f / n).
__global__ void k_centroid_one(float *__restrict__ centroid, const int8_t *__restrict__ kq,
                               const float *__restrict__ ks, int n_tok, int hd)
{
    const int d = blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= hd)
        return;
    float c = 0.0f;
    for (int t = 0; t < n_tok; t++)
        c = c + (float)kq[t * hd + d] * ks[t];
    centroid[d] = c * (1.0f / (float)n_tok);
}

// score_blocks (paged.c:401-431): score = simd_dot_f32_f32(q[0:hd], centroid)
// of mapped pages, -1e9 for unmapped ones; a lane pair per page.
__global__ __launch_bounds__(256) void k_score_pages(t_block_score *__restrict__ out, const float *__restrict__ q,
                                                     const float *__restrict__ centroid,
                                                     const int *__restrict__ page_table, int n_blocks, int hd)
{
    __shared__ __align__(16) float qs[256];
    for (int d = threadIdx.x; d < hd; d += blockDim.x)
        qs[d] = q[d];
    __syncthreads();
    const int i = (blockIdx.x * blockDim.x + threadIdx.x) >> 1, half = threadIdx.x & 1;
    const int ii = i < n_blocks ? i : n_blocks - 1;
    const int phys = page_table[ii];
    const float s = dot_ref8x2(qs, centroid + (size_t)(phys < 0 ? 0 : phys) * hd, hd, half);
    if (half == 0 && i < n_blocks) {
        t_block_score r;
        r.block_idx = i;
        r.phys_idx = phys;
        r.score = phys < 0 ? -1e9f : s;
        out[i] = r;
    }
}

// select_top_k_blocks (paged.c:439-495) over n_blocks scores.  A middle entry
// t (1 <= t <= n-2, push number m = t-1) changes the heap only while the heap
// is filling (m < cap) or when its score beats the root, i.e. when fewer than
// cap earlier middle entries score >= it; the others are skipped, and wave 0
// pushes the rest in order.
constexpr int kSelMax = 16384;

__global__ __launch_bounds__(256) void k_select_top_k(int *__restrict__ selected, int *__restrict__ n_out,
                                                      const t_block_score *__restrict__ scores, int n, int k)
{
    extern __shared__ __align__(16) unsigned char smem[];
    float *sc = (float *)smem;                 // [n] middle scores by push number
    int *act = (int *)(sc + n);                // [n] pushes that reach the heap
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int first = scores[0].phys_idx, last = scores[n - 1].phys_idx;
    int cnt = 1;
    if (last != first && n > 1)
        cnt = 2;
    if (n <= 2 || k <= 2) {
        if (tid == 0) {
            selected[0] = first;
            if (cnt == 2)
                selected[1] = last;
            *n_out = cnt;
        }
        return;
    }
    int cap = min(k - 2, n - 2);
    cap = min(cap, kHeapMax);
    const int nm = n - 2;
    for (int m = tid; m < nm; m += blockDim.x)
        sc[m] = scores[m + 1].score;
    __syncthreads();
    // activity flags, compacted in push order by wave 0 afterwards
    for (int m = tid; m < nm; m += blockDim.x) {
        int a = 1;
        if (m >= cap) {
            const float s = sc[m];
            int c = 0;
            for (int u = 0; u < m && c < cap; u++)
                c += sc[u] >= s;
            a = c < cap;
        }
        act[m] = a;
    }
    __syncthreads();
    if (wave != 0)
        return;
    int na = 0;
    for (int m0 = 0; m0 < nm; m0 += 64) {
        const int m = m0 + lane;
        const bool a = m < nm && act[m];
        const unsigned long long msk = __ballot(a);
        const int pos = na + __popcll(msk & ((1ull << lane) - 1ull));
        __builtin_amdgcn_wave_barrier();
        if (a)
            act[pos] = m;      // pos <= m: entries not yet read by this wave
        na += __popcll(msk);
    }
    __builtin_amdgcn_s_waitcnt(0);
    WaveHeap heap(cap);
    for (int a0 = 0; a0 < na; a0 += 64) {
        const int mv = a0 + lane < na ? act[a0 + lane] : 0;
        const int c = min(64, na - a0);
        for (int u = 0; u < c; u++) {
            const int m = __builtin_amdgcn_readlane(mv, u);
            heap.push(sc[m], m + 1);
        }
    }
    if (lane == 0) {
        selected[0] = first;
        if (cnt == 2)
            selected[1] = last;
        *n_out = cnt + heap.size;
    }
    if (lane < heap.size)
        selected[cnt + lane] = scores[heap.hi].phys_idx;
}

// lsh_update (ops_lsh.c:296-360): sum[d] += key[d]; on the block's last key
// the centroid sum[d] * (1.0f / count) is hashed (sequential FMA chain per
// bit, lsh_hash ops_lsh.c:138-242) and the sum cleared.
__global__ void k_lsh_accumulate(float *__restrict__ sum, const float *__restrict__ key, int dim)
{
    const int d = blockIdx.x * blockDim.x + threadIdx.x;
    if (d < dim)
        sum[d] = sum[d] + key[d];
}

// The sum buffer is zero past `dim`, so hashing over the context's hdim
// entries matches lsh_hash(ctx, sum_buffer).
__global__ __launch_bounds__(256) void k_lsh_commit(uint16_t *__restrict__ hash_out, float *__restrict__ sum,
                                                    const float *__restrict__ hpT, int dim, int hdim, int count)
{
    __shared__ float c[256];
    const float scale = 1.0f / (float)count;
    const int nd = dim > hdim ? dim : hdim;
    for (int d = threadIdx.x; d < nd; d += blockDim.x) {
        c[d] = sum[d] * scale;
        sum[d] = 0.0f;
    }
    __syncthreads();
    if (threadIdx.x >= 64)
        return;
    const int lane = threadIdx.x;
    float s = 0.0f;
    if (lane < 16)
        for (int d = 0; d < hdim; d++)
            s = __fmaf_rn(c[d], hpT[d * 16 + lane], s);
    const unsigned long long m = __ballot(lane < 16 && s > 0.0f);
    if (lane == 0)
        *hash_out = (uint16_t)(m & 0xFFFFu);
}

// compute_lightning_score_fp8_avx2 (ops_quant.c:150-222): 8 lanes accumulate
// max(lut[q]*lut[k], 0) over i = lane (mod 8), the lane sums are added in
// order, then the scalar tail, then * scale.
__global__ void k_lightning(float *__restrict__ out, const uint8_t *__restrict__ q, const uint8_t *__restrict__ k,
                            float scale, int hd)
{
    __shared__ float part[8];
    const int lane = threadIdx.x;
    const int main = hd & ~7;
    if (lane < 8) {
        float s = 0.0f;
        for (int i = lane; i < main; i += 8) {
            const float p = fp8_to_f32(q[i]) * fp8_to_f32(k[i]);
            s = s + fmaxf(p, 0.0f);
        }
        part[lane] = s;
    }
    __syncthreads();
    if (lane == 0) {
        float r = 0.0f;
        for (int j = 0; j < 8; j++)
            r = r + part[j];
        for (int i = main; i < hd; i++) {
            const float p = fp8_to_f32(q[i]) * fp8_to_f32(k[i]);
            if (p > 0.0f)
                r = r + p;
        }
        *out = r * scale;
    }
}


// ---- decode-step adjacents ---------------------------------------------------------

// op_rmsnorm row by row (ops_norm.c:27-138), one wave per row, the
// reference's arithmetic: 8 FMA chains (chain l over j = l mod 8 below
// 8 * floor(dim / 8)), ((s0+s4)+(s1+s5)) + ((s2+s6)+(s3+s7)), fused scalar
// remainder, ss / dim, 1 / sqrtf(ss + eps), out = (x * inv) * w.
__global__ __launch_bounds__(64) void k_rmsnorm_rows(float *__restrict__ out, const float *__restrict__ x,
                                                     const uint16_t *__restrict__ w, int dim, float eps)
{
    const int lane = threadIdx.x;
    const float *r = x + (size_t)blockIdx.x * dim;
    float *o = out + (size_t)blockIdx.x * dim;
    const int d8 = dim & ~7;
    float s = 0.0f;
    if (lane < 8)
        for (int j = lane; j < d8; j += 8)
            s = __fmaf_rn(r[j], r[j], s);
    const float a = s + __shfl_down(s, 4, 8);          // lanes 0-3: s_l + s_(l+4)
    const float b = a + __shfl_down(a, 1, 8);          // lanes 0, 2: (a0+a1), (a2+a3)
    float ss = b + __shfl_down(b, 2, 8);               // lane 0
    ss = __shfl(ss, 0, 64);
    if (lane == 0)
        for (int j = d8; j < dim; j++)
            ss = __fmaf_rn(r[j], r[j], ss);
    ss = __shfl(ss, 0, 64);
    ss = __fdiv_rn(ss, (float)dim);
    const float inv = __fdiv_rn(1.0f, sqrtf(ss + eps));   // sqrtf rounds correctly; __fsqrt_rn is the native one
    for (int j = lane; j < dim; j += 64)
        o[j] = (r[j] * inv) * bf16_to_f32(w[j]);
}

// op_silu_mul_fused_f32 / _bf16 (ops_activation.c:48-105, :143-230): blocks of
// 8 use the vector Schraudolph exp (round to nearest), the n % 8 remainder
// the scalar one (truncating); sig = 1 / (1 + e); out = (g * sig) * u; bf16
// in and out, the result's low 16 bits dropped.
__device__ __forceinline__ float silu_ref(float g, float u, bool vec)
{
    float e;
    if (vec) {
        float xv = fminf(fmaxf(0.0f - g, -87.0f), 87.0f);
        e = __int_as_float(__float2int_rn(__fmaf_rn(xv, 12102203.0f, 1065353216.0f)));
    } else {
        e = fast_expf(-g);
    }
    const float sig = __fdiv_rn(1.0f, 1.0f + e);
    return (g * sig) * u;
}

template <bool BF16>
__global__ __launch_bounds__(256) void k_silu_mul_ref(void *__restrict__ out, const void *__restrict__ gate,
                                                      const void *__restrict__ up, size_t n)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n)
        return;
    const bool vec = i < (n & ~(size_t)7);
    if constexpr (BF16) {
        const float g = bf16_to_f32(((const uint16_t *)gate)[i]), u = bf16_to_f32(((const uint16_t *)up)[i]);
        ((uint16_t *)out)[i] = (uint16_t)(__float_as_uint(silu_ref(g, u, vec)) >> 16);
    } else {
        ((float *)out)[i] = silu_ref(((const float *)gate)[i], ((const float *)up)[i], vec);
    }
}

// rope_apply_multihead_cached (ops_rope.c:192-228) as the compiled loop
// evaluates it: x0' = fma(x0, c, -(x1 * s)), x1' = fma(x0, s, x1 * c).
__global__ __launch_bounds__(256) void k_rope_heads(float *__restrict__ data, int n_heads, int hd,
                                                    const float *__restrict__ cos_row,
                                                    const float *__restrict__ sin_row)
{
    const int half = hd / 2;
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n_heads * half)
        return;
    const int h = t / half, i = t % half;
    float *x = data + (size_t)h * hd;
    const float c = cos_row[i], s = sin_row[i], x0 = x[i], x1 = x[i + half];
    x[i] = __fmaf_rn(x0, c, -(x1 * s));
    x[i + half] = __fmaf_rn(x0, s, x1 * c);
}

// op_rope (ops_rope.c:278-353) on nvec [hd] vectors of F32 or BF16 data:
// cs holds cos then sin of the hd / 2 angles (computed on the host with the
// C library, as the reference does); inputs scaled by mscale when it is not
// 1, then x0' = fma(x0, c, -(x1 * s)), x1' = fma(x0, s, x1 * c), the
// compiled loop's contraction.
template <bool BF16>
__global__ __launch_bounds__(256) void k_rope_ctx(void *__restrict__ data, int nvec, int hd,
                                                  const float *__restrict__ cs, float mscale)
{
    const int half = hd / 2;
    const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (long long)nvec * half)
        return;
    const int v = (int)(t / half), j = (int)(t % half);
    const size_t i0 = (size_t)v * hd + j, i1 = i0 + half;
    float x0, x1;
    if constexpr (BF16) {
        x0 = bf16_to_f32(((const uint16_t *)data)[i0]);
        x1 = bf16_to_f32(((const uint16_t *)data)[i1]);
    } else {
        x0 = ((const float *)data)[i0];
        x1 = ((const float *)data)[i1];
    }
    if (mscale != 1.0f) {
        x0 = x0 * mscale;
        x1 = x1 * mscale;
    }
    const float c = cs[j], s = cs[half + j];
    const float y0 = __fmaf_rn(x0, c, -(x1 * s)), y1 = __fmaf_rn(x0, s, x1 * c);
    if constexpr (BF16) {
        ((uint16_t *)data)[i0] = f32_to_bf16(y0);
        ((uint16_t *)data)[i1] = f32_to_bf16(y1);
    } else {
        ((float *)data)[i0] = y0;
        ((float *)data)[i1] = y1;
    }
}

// sample_argmax (sampler.c:42-148) in one block.  F32: argmax_simd_f32 --
// the maximum wins; equal maxima in the 8-lane part (indices below
// 8 * floor(n / 8), n >= 8) go to the lowest lane (i % 8), then the first
// index; tail entries win only with a strictly larger value; n < 8 scans
// with strict >.  BF16: argmax_loop_bf16 -- the first index with the largest
// value above -1e9, else 0.
__device__ __forceinline__ void amax_merge(float &vm, unsigned long long &key, float v2, unsigned long long k2)
{
    if (v2 > vm || (v2 == vm && k2 < key)) {
        vm = v2;
        key = k2;
    }
}

template <bool BF16>
__global__ __launch_bounds__(256) void k_argmax_ref(int *__restrict__ out, const void *__restrict__ data, int n)
{
    __shared__ float rv[4];
    __shared__ unsigned long long rk[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int main = BF16 ? n : (n < 8 ? 0 : (n & ~7));
    float vm = -INFINITY;
    unsigned long long key = ~0ull;
    for (int i = threadIdx.x; i < main; i += blockDim.x) {
        const float v = BF16 ? bf16_to_f32(((const uint16_t *)data)[i]) : ((const float *)data)[i];
        const unsigned long long k = BF16 ? (unsigned)i : (((unsigned long long)(i & 7) << 32) | (unsigned)i);
        amax_merge(vm, key, v, k);
    }
    for (int o = 32; o > 0; o >>= 1)
        amax_merge(vm, key, __shfl_xor(vm, o), __shfl_xor(key, o));
    if (lane == 0) {
        rv[wave] = vm;
        rk[wave] = key;
    }
    __syncthreads();
    if (threadIdx.x != 0)
        return;
    for (int w = 1; w < 4; w++)
        amax_merge(vm, key, rv[w], rk[w]);
    if (BF16) {
        *out = (key != ~0ull && vm > -1e9f) ? (int)(key & 0xFFFFFFFFu) : 0;
        return;
    }
    const float *x = (const float *)data;
    float tm = -INFINITY;
    int ti = -1;
    for (int i = main; i < n; i++)
        if (ti < 0 || x[i] > tm) {
            tm = x[i];
            ti = i;
        }
    int res;
    if (main == 0 || (ti >= 0 && tm > vm))
        res = ti >= 0 ? ti : 0;
    else
        res = key == ~0ull ? 0 : (int)(key & 0xFFFFFFFFu);
    *out = res;
}


// ---- LSH diagnostics ----------------------------------------------------------------

// bf_compute_topk + hit count of lsh_validate_recall (ops_lsh.c:513-640): one
// block.  Above 4096 keys every stride-th key is scored (stride = n / 4096);
// score_i = fused multiply-add chain over d of q[d] * bf16(k_i[d]); the top k
// by repeated argmax (strict >, first index; chosen entries set to -1e30);
// hits = how many of lsh[0 .. lsh_k) are among them.
constexpr int kValMaxKeys = 4096;
constexpr int kValMaxTopK = 64;

__global__ __launch_bounds__(256) void k_validate_recall(int *__restrict__ hits_out, const float *__restrict__ q,
                                                         const uint16_t *__restrict__ keys, int actual_n,
                                                         int stride, int dim, const int *__restrict__ lsh,
                                                         int lsh_k, int actual_k)
{
    __shared__ float sc[kValMaxKeys];
    __shared__ float rv[4];
    __shared__ int ri[4];
    __shared__ int top[kValMaxTopK];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i < actual_n; i += blockDim.x) {
        const uint16_t *k = keys + (size_t)i * stride * dim;
        float dot = 0.0f;
        for (int d = 0; d < dim; d++)
            dot = __fmaf_rn(q[d], bf16_to_f32(k[d]), dot);
        sc[i] = dot;
    }
    __syncthreads();
    for (int j = 0; j < actual_k && j < actual_n; j++) {
        float bv = -1e30f;
        int bi = 0x7FFFFFFF;
        for (int i = tid; i < actual_n; i += blockDim.x)
            if (sc[i] > bv) {
                bv = sc[i];
                bi = i;
            }
        for (int o = 32; o > 0; o >>= 1) {
            const float v2 = __shfl_xor(bv, o);
            const int i2 = __shfl_xor(bi, o);
            if (v2 > bv || (v2 == bv && i2 < bi)) {
                bv = v2;
                bi = i2;
            }
        }
        if (lane == 0) {
            rv[wave] = bv;
            ri[wave] = bi;
        }
        __syncthreads();
        if (tid == 0) {
            for (int w = 1; w < 4; w++)
                if (rv[w] > bv || (rv[w] == bv && ri[w] < bi)) {
                    bv = rv[w];
                    bi = ri[w];
                }
            // nothing above -1e30 left: the reference keeps max_idx = 0
            if (bi == 0x7FFFFFFF)
                bi = 0;
            top[j] = bi * stride;
            sc[bi] = -1e30f;
        }
        __syncthreads();
    }
    if (tid == 0) {
        int hits = 0;
        const int nk = actual_k < actual_n ? actual_k : actual_n;
        for (int i = 0; i < lsh_k; i++)
            for (int j = 0; j < nk; j++)
                if (lsh[i] == top[j]) {
                    hits++;
                    break;
                }
        *hits_out = hits;
    }
}

// adaptive_k_cutoff (ops_lsh.c:645-668): the sequential running sum of the
// scores until it reaches the threshold; at least 1.
__global__ void k_adaptive_k(int *__restrict__ out, const float *__restrict__ scores, int n, float threshold)
{
    float cum = 0.0f;
    int k = 0;
    while (k < n) {
        cum = cum + scores[k];
        k++;
        if (cum >= threshold)
            break;
    }
    *out = k < 1 ? 1 : k;
}

// ---- host runtime -------------------------------------------------------------

[[noreturn]] void die(const char *what, const char *msg)
{
    fprintf(stderr, "[be42] %s: %s\n", what, msg);
    abort();
}

void ok(int rc, const char *what)
{
    if (rc != BE42_OK)
        die(what, be42_last_error());
}

void hip_ok(hipError_t e, const char *what)
{
    if (e != hipSuccess)
        die(what, hipGetErrorString(e));
}

// Words of a host weight compared on each use: the mirror is reloaded when
// any of them changed (a freed host array whose address is reused with other
// contents); weights that stay at one address are expected not to change.
constexpr int kSampleWords = 32;

void sample_words(const void *host, size_t bytes, uint64_t *out)
{
    const unsigned char *p = (const unsigned char *)host;
    for (int i = 0; i < kSampleWords; i++) {
        uint64_t w = 0;
        if (bytes >= 8) {
            const size_t off = (bytes - 8) * (size_t)i / (kSampleWords - 1);
            memcpy(&w, p + off, 8);
        } else if (i == 0) {
            memcpy(&w, p, bytes);
        }
        out[i] = w;
    }
}

struct Runtime {
    std::mutex mu;
    bool ready = false;
    struct Buf {
        void *p = nullptr;
        size_t n = 0;
    } buf[8];
    struct Mirror {
        size_t bytes = 0;
        void *dev = nullptr;
        uint64_t sample[kSampleWords];
    };
    std::unordered_map<const void *, Mirror> mirrors;   // host weight -> device copy
    // Every map below is keyed by the address of a caller's struct, which the
    // caller may free and reuse for another struct: an entry is used only
    // while the struct still holds what the entry recorded, and is dropped
    // (its device memory freed) as soon as it does not.
    struct Pool {
        be42_kv_pool *pool = nullptr;
        const t_kv_block *blocks = nullptr;   // block_manager_init's host arrays and shape
        const int *page_table = nullptr;
        int capacity = 0, n_layers = 0, n_kv_heads = 0, head_dim = 0, max_logical = 0;
    };
    std::unordered_map<const t_block_manager *, Pool> pools;
    struct Ctx {
        float *dev = nullptr;               // hp_transposed on the device
        std::vector<float> host;            // what was uploaded (dim x 16)
    };
    std::unordered_map<const t_lsh_ctx *, Ctx> ctx_hpT;
    struct Index {
        uint16_t *hash = nullptr;   // [LSH_MAX_BLOCKS]
        float *sum = nullptr;       // [LSH_MAX_DIM]
        int uploaded = 0;           // block hashes already on the device ...
        std::vector<uint16_t> sent; // ... and their values
        int count = 0;              // keys summed in `sum` since the last commit
    };
    std::unordered_map<const t_lsh_index *, Index> indexes;
    struct Linear {
        uint16_t *k = nullptr, *v = nullptr;   // device mirror [max_seq][heads][dim]
        size_t rows = 0, row = 0;
        const void *hk = nullptr, *hv = nullptr;   // the arena rows kv_cache_init gave the struct
        int max_seq = 0, heads = 0, dim = 0;
    };
    std::unordered_map<const t_kv_cache *, Linear> linear;
};

Runtime &rt()
{
    static Runtime r;
    if (!r.ready) {
        ok(be42_init(0), "be42_init");
        r.ready = true;
    }
    return r;
}

// staging slots
enum { kS0, kS1, kS2, kS3, kS4, kS5, kS6, kS7 };

void *scratch(int slot, size_t bytes)
{
    Runtime &r = rt();
    Runtime::Buf &b = r.buf[slot];
    if (b.n < bytes) {
        if (b.p) {
            hip_ok(hipDeviceSynchronize(), "staging resize");
            hip_ok(hipFree(b.p), "staging free");
        }
        size_t n = 1 << 16;
        while (n < bytes)
            n <<= 1;
        hip_ok(hipMalloc(&b.p, n), "staging alloc");
        b.n = n;
    }
    return b.p;
}

bool is_device(const void *p)
{
    if (!p)
        return false;
    hipPointerAttribute_t a;
    if (hipPointerGetAttributes(&a, p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return a.type == hipMemoryTypeDevice;
}

// input: device pointer as is, or a copy of the host bytes in a staging slot
const void *in_dev(const void *host, size_t bytes, int slot)
{
    if (is_device(host) || bytes == 0)
        return host;
    void *d = scratch(slot, bytes);
    hip_ok(hipMemcpy(d, host, bytes, hipMemcpyHostToDevice), "stage in");
    return d;
}

// output: device pointer as is, or a staging slot copied back by out_done
void *out_dev(void *host, size_t bytes, int slot, bool *staged)
{
    *staged = !is_device(host);
    return *staged ? scratch(slot, bytes) : host;
}

void out_done(void *host, const void *dev, size_t bytes, bool staged)
{
    if (staged)
        hip_ok(hipMemcpy(host, dev, bytes, hipMemcpyDeviceToHost), "stage out");
}

// weights: mirrored once per (host pointer, size)
const void *weight_dev(const void *host, size_t bytes)
{
    if (is_device(host))
        return host;
    Runtime &r = rt();
    uint64_t smp[kSampleWords];
    sample_words(host, bytes, smp);
    auto it = r.mirrors.find(host);
    if (it != r.mirrors.end() && it->second.bytes == bytes && !memcmp(it->second.sample, smp, sizeof smp))
        return it->second.dev;
    if (it != r.mirrors.end()) {
        hip_ok(hipDeviceSynchronize(), "mirror replace");
        hip_ok(hipFree(it->second.dev), "mirror free");
        r.mirrors.erase(it);
    }
    Runtime::Mirror m;
    m.bytes = bytes;
    memcpy(m.sample, smp, sizeof smp);
    hip_ok(hipMalloc(&m.dev, bytes ? bytes : 1), "weight mirror");
    hip_ok(hipMemcpy(m.dev, host, bytes, hipMemcpyHostToDevice), "weight upload");
    r.mirrors[host] = m;
    return m.dev;
}

bool pool_matches(const Runtime::Pool &p, const t_block_manager *bm)
{
    return p.blocks == bm->blocks && p.page_table == bm->page_table && p.capacity == bm->capacity &&
           p.n_layers == bm->n_layers && p.n_kv_heads == bm->n_kv_heads && p.head_dim == bm->head_dim &&
           p.max_logical == bm->max_logical;
}

void pool_drop(Runtime &r, std::unordered_map<const t_block_manager *, Runtime::Pool>::iterator it)
{
    hip_ok(hipDeviceSynchronize(), "block manager release");
    be42_kv_destroy(it->second.pool);
    r.pools.erase(it);
}

be42_kv_pool *pool_of(const t_block_manager *bm, const char *what)
{
    Runtime &r = rt();
    auto it = r.pools.find(bm);
    if (it != r.pools.end() && !pool_matches(it->second, bm))
        pool_drop(r, it), it = r.pools.end();
    if (it == r.pools.end())
        die(what, "block manager was not created by block_manager_init of this library");
    return it->second.pool;
}

// host mirror of the pool's allocator state
void sync_manager(t_block_manager *bm, be42_kv_pool *pool)
{
    ok(be42_kv_export(pool, bm->page_table, bm->free_stack, &bm->free_top, bm->logical_len), "be42_kv_export");
}

// The device copy of a context's transposed projection, uploaded again
// whenever the struct's values differ from the ones last uploaded (a context
// re-initialised, or another context at a reused address).
const float *ctx_hpT(const t_lsh_ctx *ctx)
{
    Runtime &r = rt();
    const size_t n = (size_t)LSH_MAX_DIM * 16;
    const float *h = &ctx->hp_transposed[0][0];
    Runtime::Ctx &c = r.ctx_hpT[ctx];
    if (!c.dev)
        hip_ok(hipMalloc((void **)&c.dev, n * sizeof(float)), "lsh ctx");
    else if (c.host.size() == n && !memcmp(c.host.data(), h, n * sizeof(float)))
        return c.dev;
    c.host.assign(h, h + n);
    hip_ok(hipMemcpy(c.dev, h, n * sizeof(float), hipMemcpyHostToDevice), "lsh ctx upload");
    return c.dev;
}

Runtime::Index &index_of(const t_lsh_index *idx)
{
    Runtime &r = rt();
    Runtime::Index &x = r.indexes[idx];
    if (!x.hash) {
        hip_ok(hipMalloc((void **)&x.hash, LSH_MAX_BLOCKS * sizeof(uint16_t)), "lsh index");
        hip_ok(hipMalloc((void **)&x.sum, LSH_MAX_DIM * sizeof(float)), "lsh index");
        hip_ok(hipMemset(x.sum, 0, LSH_MAX_DIM * sizeof(float)), "lsh index");
        x.uploaded = 0;
        x.count = 0;
        x.sent.assign(LSH_MAX_BLOCKS, 0);
    }
    return x;
}

// Bring the device copy of the index's block hashes to [0, nb): hashes
// uploaded before are trusted only while the struct still holds them (an
// index rebuilt in place, or another index at a reused address, differs).
void index_sync_hashes(Runtime::Index &x, const t_lsh_index *idx, int nb)
{
    int from = x.uploaded < nb ? x.uploaded : nb;
    for (int i = 0; i < from; i++)
        if (x.sent[i] != idx->block_hashes[i]) {
            from = i;
            break;
        }
    if (from < nb) {
        hip_ok(hipMemcpy(x.hash + from, idx->block_hashes + from, (size_t)(nb - from) * 2, hipMemcpyHostToDevice),
               "lsh index upload");
        memcpy(x.sent.data() + from, idx->block_hashes + from, (size_t)(nb - from) * 2);
    }
    x.uploaded = nb;
}

// column chunks of the quantized GEMV
constexpr int kGemvBatch = 16;

int matmul_quant(t_tensor *out, const t_tensor *a, const t_tensor *b, int m, int k, int n)
{
    const bool fp8 = a->dtype == DTYPE_FP8;
    if (!a->row_scale) {
        fprintf(stderr, "MatMul: quantized weight without row_scale\n");
        return -1;
    }
    const void *w = weight_dev(a->data, (size_t)m * k);
    const float *ws = (const float *)weight_dev(a->row_scale, (size_t)m * sizeof(float));
    if (n == 1) {
        const float *x = (const float *)in_dev(b->data, (size_t)k * 4, kS0);
        bool st;
        float *y = (float *)out_dev(out->data, (size_t)m * 4, kS1, &st);
        ok(fp8 ? be42_gemv_fp8(y, (const uint8_t *)w, ws, x, m, k, 1, nullptr)
               : be42_gemv_q8(y, (const int8_t *)w, ws, x, m, k, 1, nullptr),
           "op_matmul");
        out_done(out->data, y, (size_t)m * 4, st);
        return 0;
    }
    // b [k][n] -> x [n][k]; y [n][m]: up to 16 tokens as one GEMV, more as
    // the prefill GEMM over the same digit planes (INT8: identical values);
    // out = y^T [m][n]
    const float *bd = (const float *)in_dev(b->data, (size_t)k * n * 4, kS0);
    float *x = (float *)scratch(kS2, (size_t)n * k * 4);
    float *y = (float *)scratch(kS3, (size_t)n * m * 4);
    hipLaunchKernelGGL(k_transpose, dim3((n + 31) / 32, (k + 31) / 32), dim3(256), 0, nullptr, x, bd, k, n);
    hip_ok(hipGetLastError(), "op_matmul transpose");
    if (n <= kGemvBatch || k % 16 != 0 || n > 65535) {
        for (int c0 = 0; c0 < n; c0 += kGemvBatch) {
            const int bc = n - c0 < kGemvBatch ? n - c0 : kGemvBatch;
            ok(fp8 ? be42_gemv_fp8(y + (size_t)c0 * m, (const uint8_t *)w, ws, x + (size_t)c0 * k, m, k, bc, nullptr)
                   : be42_gemv_q8(y + (size_t)c0 * m, (const int8_t *)w, ws, x + (size_t)c0 * k, m, k, bc, nullptr),
               "op_matmul");
        }
    } else {
        void *dig = scratch(kS4, be42_gemm_xdig_bytes(k, n, fp8));
        ok(be42_gemm_prepare(dig, x, k, n, fp8, nullptr), "op_matmul");
        ok(fp8 ? be42_gemm_fp8_prepared(y, (const uint8_t *)w, ws, dig, m, k, n, nullptr)
               : be42_gemm_q8_prepared(y, (const int8_t *)w, ws, dig, m, k, n, nullptr),
           "op_matmul");
    }
    bool st;
    float *o = (float *)out_dev(out->data, (size_t)m * n * 4, kS1, &st);
    hipLaunchKernelGGL(k_transpose, dim3((m + 31) / 32, (n + 31) / 32), dim3(256), 0, nullptr, o, y, n, m);
    hip_ok(hipGetLastError(), "op_matmul transpose");
    out_done(out->data, o, (size_t)m * n * 4, st);
    return 0;
}

int matmul_dense(t_tensor *out, const t_tensor *a, const t_tensor *b, int m, int k, int n)
{
    const bool wbf = a->dtype == DTYPE_BF16, xbf = b->dtype == DTYPE_BF16, obf = out->dtype == DTYPE_BF16;
    const void *w = weight_dev(a->data, (size_t)m * k * (wbf ? 2 : 4));
    const void *x = in_dev(b->data, (size_t)k * n * (xbf ? 2 : 4), kS0);
    const size_t ob = (size_t)m * n * (obf ? 2 : 4);
    bool st;
    void *o = out_dev(out->data, ob, kS1, &st);
    const long waves = (long)m * ((n + 7) / 8);
    const dim3 grid((unsigned)((waves + 3) / 4));
    if (wbf && !xbf && !obf)
        hipLaunchKernelGGL((k_dense_mm<uint16_t, float, false>), grid, dim3(256), 0, nullptr, o,
                           (const uint16_t *)w, (const float *)x, m, k, n);
    else if (wbf && xbf && obf)
        hipLaunchKernelGGL((k_dense_mm<uint16_t, uint16_t, true>), grid, dim3(256), 0, nullptr, o,
                           (const uint16_t *)w, (const uint16_t *)x, m, k, n);
    else
        hipLaunchKernelGGL((k_dense_mm<float, float, false>), grid, dim3(256), 0, nullptr, o, (const float *)w,
                           (const float *)x, m, k, n);
    hip_ok(hipGetLastError(), "op_matmul");
    out_done(out->data, o, ob, st);
    return 0;
}

void paged_attention(float *output, const float *q, be42_kv_pool *pool, const int *sel_host, int n_sel,
                     int n_heads, int n_kv_heads, int head_dim, float scale, const char *what)
{
    if (pool->n_kv != n_kv_heads || pool->head_dim != head_dim) {
        char msg[160];
        snprintf(msg, sizeof msg, "pool has %d kv heads x %d dims, call passes %d x %d", pool->n_kv,
                 pool->head_dim, n_kv_heads, head_dim);
        die(what, msg);
    }
    const size_t qb = (size_t)n_heads * head_dim * 4;
    const float *dq = (const float *)in_dev(q, qb, kS0);
    // attention_head_paged_sparse (ops_attention.c:403-411) skips entries < 0
    // (score_blocks marks unmapped pages -1 and select_top_k_blocks keeps its
    // anchors even then); an id past the pool is a caller error
    std::vector<int> ids;
    if (n_sel > 0) {
        std::vector<int> raw((size_t)n_sel);
        hip_ok(hipMemcpy(raw.data(), sel_host, (size_t)n_sel * 4,
                         is_device(sel_host) ? hipMemcpyDeviceToHost : hipMemcpyHostToHost),
               "stage selection");
        ids.reserve(raw.size());
        for (int id : raw) {
            if (id < 0)
                continue;
            if (id >= pool->capacity) {
                char msg[96];
                snprintf(msg, sizeof msg, "page id %d outside the pool (capacity %d)", id, pool->capacity);
                die(what, msg);
            }
            ids.push_back(id);
        }
    }
    const int ns = (int)ids.size();
    int *dsel = (int *)scratch(kS4, (size_t)(ns + 1) * 4);
    if (ns)
        hip_ok(hipMemcpy(dsel, ids.data(), (size_t)ns * 4, hipMemcpyHostToDevice), "stage selection");
    hip_ok(hipMemcpy(dsel + ns, &ns, 4, hipMemcpyHostToDevice), "stage selection");
    bool st;
    float *o = (float *)out_dev(output, qb, kS1, &st);
    const int stride = ns > 0 ? ns : 1;
    const int n_split = ns <= 64 ? 1 : (ns + 63) / 64;
    const size_t wsb = be42_attn_workspace_bytes(1, n_heads, head_dim, stride, n_split);
    void *ws = scratch(kS5, wsb ? wsb : 16);
    ok(be42_paged_attention(pool, dq, 1, n_heads, dsel, dsel + ns, stride, stride, scale, o, n_split, ws, wsb,
                            nullptr),
       what);
    out_done(output, o, qb, st);
}

}  // namespace
}  // namespace be42

using namespace be42;

// ---- linear layers ----------------------------------------------------------------

extern "C" int op_matmul(t_tensor *out, const t_tensor *a, const t_tensor *b)
{
    const int m = a->shape[0], k = a->shape[1], n = b->shape[1];
    if (a->shape[1] != b->shape[0]) {
        fprintf(stderr, "MatMul dim mismatch: [%d,%d] x [%d,%d] (A.k=%d != B.m=%d)\n", a->shape[0], a->shape[1],
                b->shape[0], b->shape[1], a->shape[1], b->shape[0]);
        return -1;
    }
    std::lock_guard<std::mutex> g(rt().mu);
    if (m <= 0 || n <= 0)
        return 0;
    if ((a->dtype == DTYPE_I8 || a->dtype == DTYPE_FP8) && b->dtype == DTYPE_F32 && out->dtype == DTYPE_F32)
        return matmul_quant(out, a, b, m, k, n);
    if ((a->dtype == DTYPE_BF16 && b->dtype == DTYPE_F32 && out->dtype == DTYPE_F32) ||
        (a->dtype == DTYPE_BF16 && b->dtype == DTYPE_BF16 && out->dtype == DTYPE_BF16) ||
        (a->dtype == DTYPE_F32 && b->dtype == DTYPE_F32 && out->dtype == DTYPE_F32))
        return matmul_dense(out, a, b, m, k, n);
    fprintf(stderr, "MatMul unsupported dtypes: A=%d B=%d Out=%d\n", a->dtype, b->dtype, out->dtype);
    return -1;
}

// ---- decode-step adjacents ------------------------------------------------------------

static int norm_dim(const t_tensor *x)
{
    if (x->ndim == 2 && x->shape[1] == 1)
        return x->shape[0];
    return x->shape[x->ndim > 0 ? x->ndim - 1 : 0];
}

extern "C" void op_rmsnorm(t_tensor *out, const t_tensor *x, const t_tensor *w, float epsilon)
{
    if (!(x->dtype == DTYPE_F32 && out->dtype == DTYPE_F32 && w->dtype == DTYPE_BF16)) {
        fprintf(stderr, "RMSNorm unsupported dtypes\n");
        return;
    }
    const int dim = norm_dim(x);
    if (dim <= 0 || x->size == 0)
        return;
    const int rows = (int)(x->size / (size_t)dim);
    std::lock_guard<std::mutex> g(rt().mu);
    const size_t bytes = (size_t)rows * dim * 4;
    const float *dx = (const float *)in_dev(x->data, bytes, kS0);
    const uint16_t *dw = (const uint16_t *)weight_dev(w->data, (size_t)dim * 2);
    bool st;
    float *o = (float *)out_dev(out->data, bytes, kS1, &st);
    hipLaunchKernelGGL(k_rmsnorm_rows, dim3(rows), dim3(64), 0, nullptr, o, dx, dw, dim, epsilon);
    hip_ok(hipGetLastError(), "op_rmsnorm");
    out_done(out->data, o, bytes, st);
}

extern "C" void op_silu_mul(t_tensor *out, const t_tensor *gate, const t_tensor *val)
{
    if (gate->size != out->size || val->size != out->size)
        return;
    const bool f32 = out->dtype == DTYPE_F32 && gate->dtype == DTYPE_F32 && val->dtype == DTYPE_F32;
    const bool bf = out->dtype == DTYPE_BF16 && gate->dtype == DTYPE_BF16 && val->dtype == DTYPE_BF16;
    if (!f32 && !bf) {
        fprintf(stderr, "SiLU unsupported dtypes\n");
        return;
    }
    const size_t n = out->size;
    if (n == 0)
        return;
    std::lock_guard<std::mutex> g(rt().mu);
    const size_t bytes = n * (f32 ? 4 : 2);
    const void *dg = in_dev(gate->data, bytes, kS0);
    const void *du = in_dev(val->data, bytes, kS2);
    bool st;
    void *o = out_dev(out->data, bytes, kS1, &st);
    const dim3 grid((unsigned)((n + 255) / 256));
    if (f32)
        hipLaunchKernelGGL(k_silu_mul_ref<false>, grid, dim3(256), 0, nullptr, o, dg, du, n);
    else
        hipLaunchKernelGGL(k_silu_mul_ref<true>, grid, dim3(256), 0, nullptr, o, dg, du, n);
    hip_ok(hipGetLastError(), "op_silu_mul");
    out_done(out->data, o, bytes, st);
}

extern "C" void rope_apply_multihead_cached(float *data, int n_heads, int pos, const t_rope_cache *cache)
{
    if (pos >= cache->max_seq_len || n_heads <= 0)
        return;
    const int hd = cache->head_dim, half = hd / 2;
    std::lock_guard<std::mutex> g(rt().mu);
    // the tables are read-only model state: mirrored once, like weights
    const size_t tb = (size_t)cache->max_seq_len * half * 4;
    const float *ct = (const float *)weight_dev(cache->cos_table, tb);
    const float *sn = (const float *)weight_dev(cache->sin_table, tb);
    const size_t bytes = (size_t)n_heads * hd * 4;
    bool st;
    float *d = (float *)out_dev(data, bytes, kS1, &st);
    if (st)
        hip_ok(hipMemcpy(d, data, bytes, hipMemcpyHostToDevice), "rope_apply_multihead_cached");
    const int n = n_heads * half;
    hipLaunchKernelGGL(k_rope_heads, dim3((n + 255) / 256), dim3(256), 0, nullptr, d, n_heads, hd,
                       ct + (size_t)pos * half, sn + (size_t)pos * half);
    hip_ok(hipGetLastError(), "rope_apply_multihead_cached");
    out_done(data, d, bytes, st);
}

// theta of pair index j2 = 2j without a thetas cache (get_yarn_theta and
// compute_yarn_ramp, ops_rope.c:243-276): frequency index j2 / hd in float,
// powers in double, the YaRN ramp between beta_slow / hd and beta_fast / hd
// when factor > 1, its (1 - a) * t + a * ts fused on the first product as
// the compiled reference evaluates it.
static float yarn_theta(int j2, const t_rope_ctx *c)
{
    const float f = (float)j2 / (float)c->head_dim;
    const double td = 1.0 / ::pow((double)c->theta_base, (double)f);
    if (c->factor <= 1.0f)
        return (float)td;
    const float lo = c->beta_slow / (float)c->head_dim, hi = c->beta_fast / (float)c->head_dim;
    if (f < lo)
        return (float)td;
    const double ts = 1.0 / ::pow((double)(c->theta_base * c->factor), (double)f);
    if (f > hi)
        return (float)ts;
    const float a = (f - lo) / (hi - lo);
    return (float)::fma(1.0 - (double)a, td, (double)a * ts);
}

extern "C" void op_rope(t_tensor *x, int pos, const t_rope_ctx *ctx)
{
    if (!x || !x->data || !ctx)
        return;
    const bool bf = x->dtype == DTYPE_BF16;
    if (!bf && x->dtype != DTYPE_F32)
        return;
    const int hd = ctx->head_dim, half = hd / 2;
    if (hd <= 0 || half == 0)
        return;
    const size_t nvec = x->size / (size_t)hd;
    if (nvec == 0)
        return;
    const size_t n = nvec * (size_t)half;
    if (nvec > (size_t)INT32_MAX || (n + 255) / 256 > (size_t)INT32_MAX)
        die("op_rope", "tensor too large");
    // angles and their cosine / sine on the host: cosf and sinf of the C
    // library, the reference's own
    std::vector<float> cs(2 * (size_t)half);
    for (int j = 0; j < half; j++) {
        const float th = ctx->thetas_cache ? ctx->thetas_cache[j] : yarn_theta(2 * j, ctx);
        const float ang = (float)pos * th;
        cs[j] = ::cosf(ang);
        cs[half + j] = ::sinf(ang);
    }
    std::lock_guard<std::mutex> g(rt().mu);
    const size_t bytes = x->size * (bf ? 2 : 4);
    const float *dcs = (const float *)in_dev(cs.data(), cs.size() * 4, kS0);
    bool st;
    void *d = out_dev(x->data, bytes, kS1, &st);
    if (st)
        hip_ok(hipMemcpy(d, x->data, bytes, hipMemcpyHostToDevice), "op_rope");
    const dim3 grid((unsigned)((n + 255) / 256));
    if (bf)
        hipLaunchKernelGGL(k_rope_ctx<true>, grid, dim3(256), 0, nullptr, d, (int)nvec, hd, dcs, ctx->mscale);
    else
        hipLaunchKernelGGL(k_rope_ctx<false>, grid, dim3(256), 0, nullptr, d, (int)nvec, hd, dcs, ctx->mscale);
    hip_ok(hipGetLastError(), "op_rope");
    out_done(x->data, d, bytes, st);
}

extern "C" int sample_argmax(const t_tensor *logits)
{
    const bool f32 = logits->dtype == DTYPE_F32;
    const size_t n = logits->size;
    if (n == 0)
        return 0;
    if (n > (size_t)INT32_MAX)
        die("sample_argmax", "more than 2^31 logits");
    std::lock_guard<std::mutex> g(rt().mu);
    const void *d = in_dev(logits->data, n * (f32 ? 4 : 2), kS0);
    int *dres = (int *)scratch(kS1, 4);
    if (f32)
        hipLaunchKernelGGL(k_argmax_ref<false>, dim3(1), dim3(256), 0, nullptr, dres, d, (int)n);
    else
        hipLaunchKernelGGL(k_argmax_ref<true>, dim3(1), dim3(256), 0, nullptr, dres, d, (int)n);
    hip_ok(hipGetLastError(), "sample_argmax");
    int res = 0;
    hip_ok(hipMemcpy(&res, dres, 4, hipMemcpyDeviceToHost), "sample_argmax");
    return res;
}

// sampler_random_float (sampler.c:33-45): a per-thread LCG seeded from the
// time and a thread-local address, 15 bits per draw
static float sampler_draw(void)
{
    static thread_local int init = 0;
    static thread_local unsigned int seed;
    if (!init) {
        seed = (unsigned int)time(nullptr) ^ (unsigned int)(size_t)&init;
        init = 1;
    }
    seed = seed * 1103515245u + 12345u;
    return (float)((seed >> 16) & 0x7FFF) / 32767.0f;
}

// sample_temperature (sampler_temp.c:96-114) and sample_top_p
// (sampler_topp.c:113-158) on the GPU; the uniform draws are the reference's
// (sampler_random_float; rand() / RAND_MAX), made on the host.  The scratch
// arena is not used (the probabilities live in device memory).
static int sample_dropin(const t_tensor *logits, float temp, float top_p, bool topp, const char *what)
{
    const bool f32 = logits->dtype == DTYPE_F32;
    const size_t n = logits->size;
    if (n == 0)
        return 0;
    if (n > (size_t)INT32_MAX)
        die(what, "more than 2^31 logits");
    const float u = topp ? (float)rand() / (float)RAND_MAX : sampler_draw();
    std::lock_guard<std::mutex> g(rt().mu);
    const void *d = in_dev(logits->data, n * (f32 ? 4 : 2), kS0);
    int *dres = (int *)scratch(kS1, 8);
    float *du = (float *)(dres + 1);
    hip_ok(hipMemcpy(du, &u, 4, hipMemcpyHostToDevice), what);
    const int rc = topp ? be42_sample_top_p_dt(dres, d, f32 ? 0 : 1, (int)n, 1, temp, top_p, du, nullptr)
                        : be42_sample_temperature_dt(dres, d, f32 ? 0 : 1, (int)n, 1, temp, du, nullptr);
    if (rc != BE42_OK)
        die(what, be42_last_error());
    int res = 0;
    hip_ok(hipMemcpy(&res, dres, 4, hipMemcpyDeviceToHost), what);
    return res;
}

extern "C" int sample_temperature(const t_tensor *logits, float temperature, t_arena *scratch)
{
    (void)scratch;
    return sample_dropin(logits, temperature, 0.0f, false, "sample_temperature");
}

extern "C" int sample_top_p(const t_tensor *logits, float temperature, float top_p, t_arena *scratch)
{
    (void)scratch;
    return sample_dropin(logits, temperature, top_p, true, "sample_top_p");
}

// ---- quant codecs ------------------------------------------------------------------

extern "C" {
float g_fp8_lut[256];
}

extern "C" void quant_init_fp8_lut(void)
{
    std::lock_guard<std::mutex> g(rt().mu);
    uint8_t codes[256];
    for (int i = 0; i < 256; i++)
        codes[i] = (uint8_t)i;
    const uint8_t *dc = (const uint8_t *)in_dev(codes, sizeof codes, kS0);
    float *d = (float *)scratch(kS1, sizeof g_fp8_lut);
    ok(be42_fp8_decode(d, dc, 256, nullptr), "quant_init_fp8_lut");
    hip_ok(hipMemcpy(g_fp8_lut, d, sizeof g_fp8_lut, hipMemcpyDeviceToHost), "quant_init_fp8_lut");
}

static float quant_vec(bool fp8, void *out, const float *in, int n)
{
    std::lock_guard<std::mutex> g(rt().mu);
    const float *din = (const float *)in_dev(in, (size_t)n * 4, kS0);
    bool st;
    void *dq = out_dev(out, (size_t)n, kS1, &st);
    float *ds = (float *)scratch(kS2, 4);
    ok(fp8 ? be42_quant_rows_fp8((uint8_t *)dq, ds, din, 1, n, nullptr)
           : be42_quant_rows_int8((int8_t *)dq, ds, din, 1, n, nullptr),
       fp8 ? "quant_f32_to_fp8" : "quant_f32_to_int8");
    out_done(out, dq, (size_t)n, st);
    float s = 0.0f;
    hip_ok(hipMemcpy(&s, ds, 4, hipMemcpyDeviceToHost), "quant scale");
    return s;
}

extern "C" float quant_f32_to_int8(t_qint8 *out, const float *in, int n)
{
    if (n <= 0)
        return 1.0f;     // amax = 0 over an empty vector
    return quant_vec(false, out, in, n);
}

extern "C" void quant_f32_to_fp8(t_fp8_e4m3 *out, const float *in, int n, float *scale)
{
    const float s = n <= 0 ? 1.0f : quant_vec(true, out, in, n);
    if (scale)
        *scale = s;
}

extern "C" void dequant_int8_to_f32_avx2(float *out, const t_qint8 *in, float scale, int n)
{
    if (n <= 0)
        return;
    std::lock_guard<std::mutex> g(rt().mu);
    const int8_t *din = (const int8_t *)in_dev(in, (size_t)n, kS0);
    const float *ds = (const float *)in_dev(&scale, 4, kS2);
    bool st;
    float *dout = (float *)out_dev(out, (size_t)n * 4, kS1, &st);
    ok(be42_dequant_rows_int8(dout, din, ds, 1, n, nullptr), "dequant_int8_to_f32_avx2");
    out_done(out, dout, (size_t)n * 4, st);
}

extern "C" float compute_lightning_score_fp8_avx2(const t_fp8_e4m3 *q_fp8, const t_fp8_e4m3 *k_fp8, float scale,
                                                  int head_dim)
{
    if (head_dim <= 0)
        return 0.0f * scale;
    std::lock_guard<std::mutex> g(rt().mu);
    const uint8_t *dq = (const uint8_t *)in_dev(q_fp8, (size_t)head_dim, kS0);
    const uint8_t *dk = (const uint8_t *)in_dev(k_fp8, (size_t)head_dim, kS1);
    float *d = (float *)scratch(kS2, 4);
    hipLaunchKernelGGL(k_lightning, dim3(1), dim3(64), 0, nullptr, d, dq, dk, scale, head_dim);
    hip_ok(hipGetLastError(), "compute_lightning_score_fp8");
    float r = 0.0f;
    hip_ok(hipMemcpy(&r, d, 4, hipMemcpyDeviceToHost), "compute_lightning_score_fp8");
    return r;
}

extern "C" float compute_lightning_score_fp8(const t_fp8_e4m3 *q_fp8, const t_fp8_e4m3 *k_fp8, float scale,
                                             int head_dim)
{
    return compute_lightning_score_fp8_avx2(q_fp8, k_fp8, scale, head_dim);
}

// ---- LSH ---------------------------------------------------------------------------

extern "C" void lsh_init(t_lsh_ctx *ctx, int dim, unsigned int seed)
{
    if (dim > LSH_MAX_DIM)
        dim = LSH_MAX_DIM;
    std::vector<float> hp((size_t)16 * dim), hpT((size_t)dim * 16);
    be42_lsh_projection(hp.data(), hpT.data(), dim, seed);
    ctx->dim = dim;
    for (int h = 0; h < 16; h++)
        for (int d = 0; d < dim; d++)
            ctx->hyperplanes[h][d] = hp[(size_t)h * dim + d];
    for (int d = 0; d < dim; d++)
        for (int h = 0; h < 16; h++)
            ctx->hp_transposed[d][h] = hpT[(size_t)d * 16 + h];
    ctx->initialized = 1;
    // the device copy (if any) is refreshed by its next use, which compares it
    // with these values
}

extern "C" void lsh_ctx_release(const t_lsh_ctx *ctx)
{
    std::lock_guard<std::mutex> g(rt().mu);
    Runtime &r = rt();
    auto it = r.ctx_hpT.find(ctx);
    if (it != r.ctx_hpT.end()) {
        hip_ok(hipDeviceSynchronize(), "lsh_ctx_release");
        hip_ok(hipFree(it->second.dev), "lsh_ctx_release");
        r.ctx_hpT.erase(it);
    }
}

extern "C" void lsh_index_init(t_lsh_index *idx)
{
    idx->n_blocks = 0;
    idx->block_size = LSH_BLOCK_SIZE;
    for (int i = 0; i < LSH_NUM_BUCKETS; i++)
        idx->bucket_heads[i] = -1;
    memset(idx->active.sum_buffer, 0, sizeof(idx->active.sum_buffer));
    idx->active.count = 0;
    idx->active.start_pos = 0;
    std::lock_guard<std::mutex> g(rt().mu);
    Runtime::Index &x = index_of(idx);
    x.uploaded = 0;
    x.count = 0;
    hip_ok(hipMemset(x.sum, 0, LSH_MAX_DIM * sizeof(float)), "lsh_index_init");
}

extern "C" void lsh_index_reset(t_lsh_index *idx)
{
    lsh_index_init(idx);
}

extern "C" void lsh_index_release(const t_lsh_index *idx)
{
    std::lock_guard<std::mutex> g(rt().mu);
    Runtime &r = rt();
    auto it = r.indexes.find(idx);
    if (it != r.indexes.end()) {
        hip_ok(hipDeviceSynchronize(), "lsh_index_release");
        hip_ok(hipFree(it->second.hash), "lsh_index_release");
        hip_ok(hipFree(it->second.sum), "lsh_index_release");
        r.indexes.erase(it);
    }
}

extern "C" uint16_t lsh_hash(const t_lsh_ctx *ctx, const float *vec)
{
    std::lock_guard<std::mutex> g(rt().mu);
    const float *hpT = ctx_hpT(ctx);
    const float *dv = (const float *)in_dev(vec, (size_t)ctx->dim * 4, kS0);
    uint16_t *d = (uint16_t *)scratch(kS1, 2);
    ok(be42_lsh_hash(d, dv, 1, hpT, ctx->dim, nullptr), "lsh_hash");
    uint16_t h = 0;
    hip_ok(hipMemcpy(&h, d, 2, hipMemcpyDeviceToHost), "lsh_hash");
    return h;
}

extern "C" int lsh_hamming_distance(uint16_t h1, uint16_t h2)
{
    return __builtin_popcount((unsigned)(h1 ^ h2));
}

extern "C" void lsh_insert_block(t_lsh_index *idx, uint16_t hash, int start_pos, int len)
{
    // ops_lsh.c:256-272: append, LIFO chain per bucket, drop beyond the cap
    if (idx->n_blocks >= LSH_MAX_BLOCKS)
        return;
    const int id = idx->n_blocks;
    idx->block_hashes[id] = hash;
    idx->block_starts[id] = start_pos;
    idx->block_lens[id] = len;
    const int bucket = hash % LSH_NUM_BUCKETS;
    idx->chain_next[id] = idx->bucket_heads[bucket];
    idx->bucket_heads[bucket] = id;
    idx->n_blocks++;
}

extern "C" void lsh_update(t_lsh_index *idx, const t_lsh_ctx *ctx, const float *key, int dim, int pos)
{
    std::lock_guard<std::mutex> g(rt().mu);
    if (dim > LSH_MAX_DIM)
        dim = LSH_MAX_DIM;
    Runtime::Index &x = index_of(idx);
    t_block_acc *acc = &idx->active;
    // the running key sum lives on the device: it must hold the struct's
    // `count` keys (an index at a reused address, or one the caller changed,
    // starts again from zero when its block is empty and is refused otherwise)
    if (acc->count != x.count) {
        if (acc->count != 0)
            die("lsh_update", "the index's active block was not accumulated by this library's lsh_update");
        hip_ok(hipMemset(x.sum, 0, LSH_MAX_DIM * sizeof(float)), "lsh_update");
        x.count = 0;
    }
    if (acc->count == 0)
        acc->start_pos = pos;
    const float *dk = (const float *)in_dev(key, (size_t)dim * 4, kS0);
    hipLaunchKernelGGL(k_lsh_accumulate, dim3((dim + 255) / 256), dim3(256), 0, nullptr, x.sum, dk, dim);
    hip_ok(hipGetLastError(), "lsh_update");
    acc->count++;
    x.count = acc->count;
    if (acc->count >= LSH_BLOCK_SIZE) {
        uint16_t *dh = (uint16_t *)scratch(kS1, 2);
        hipLaunchKernelGGL(k_lsh_commit, dim3(1), dim3(256), 0, nullptr, dh, x.sum, ctx_hpT(ctx), dim, ctx->dim,
                           acc->count);
        hip_ok(hipGetLastError(), "lsh_update");
        uint16_t h = 0;
        hip_ok(hipMemcpy(&h, dh, 2, hipMemcpyDeviceToHost), "lsh_update");
        lsh_insert_block(idx, h, acc->start_pos, acc->count);
        acc->count = 0;
        x.count = 0;
    }
}

constexpr int kCandCapMax = 512;

extern "C" int lsh_find_candidates(const t_lsh_index *idx, uint16_t query_hash, int *block_ids, int max_blocks)
{
    if (max_blocks <= 0 || idx->n_blocks <= 0)
        return 0;
    std::lock_guard<std::mutex> g(rt().mu);
    Runtime::Index &x = index_of(idx);
    const int nb = idx->n_blocks < LSH_MAX_BLOCKS ? idx->n_blocks : LSH_MAX_BLOCKS;
    index_sync_hashes(x, idx, nb);
    int cap = max_blocks < nb ? max_blocks : nb;
    if (cap > kCandCapMax) {
        char msg[96];
        snprintf(msg, sizeof msg, "max_blocks %d with %d blocks exceeds %d", max_blocks, nb, kCandCapMax);
        die("lsh_find_candidates", msg);
    }
    uint16_t *dq = (uint16_t *)scratch(kS0, 2);
    hip_ok(hipMemcpy(dq, &query_hash, 2, hipMemcpyHostToDevice), "lsh_find_candidates");
    int *dn = (int *)scratch(kS1, 4);
    bool st;
    int *dids = (int *)out_dev(block_ids, (size_t)cap * 4, kS2, &st);
    ok(be42_lsh_candidates(dids, dn, x.hash, nb, dq, 1, cap, nullptr), "lsh_find_candidates");
    int n = 0;
    hip_ok(hipMemcpy(&n, dn, 4, hipMemcpyDeviceToHost), "lsh_find_candidates");
    out_done(block_ids, dids, (size_t)n * 4, st);
    return n;
}

extern "C" int lsh_get_active_block(const t_lsh_index *idx, int *start_pos, int *len)
{
    if (idx->active.count == 0)
        return 0;
    *start_pos = idx->active.start_pos;
    *len = idx->active.count;
    return 1;
}

// ---- block manager / paged KV ---------------------------------------------------------

extern "C" int block_manager_init(t_block_manager *bm, int n_layers, int n_kv_heads, int head_dim,
                                  int max_blocks_per_layer)
{
    std::lock_guard<std::mutex> g(rt().mu);
    {
        // a manager initialised again in place abandons its previous pool
        Runtime &r = rt();
        auto it = r.pools.find(bm);
        if (it != r.pools.end())
            pool_drop(r, it);
    }
    memset(bm, 0, sizeof *bm);
    be42_kv_pool *pool = nullptr;
    if (be42_kv_create(&pool, BE42_KV_INT8, n_layers, n_kv_heads, head_dim, max_blocks_per_layer, nullptr)) {
        fprintf(stderr, "[PagedKV] ERROR: %s\n", be42_last_error());
        return -1;
    }
    const int cap = pool->capacity;
    bm->capacity = cap;
    bm->n_layers = n_layers;
    bm->n_kv_heads = n_kv_heads;
    bm->head_dim = head_dim;
    bm->max_logical = max_blocks_per_layer;
    bm->blocks = (t_kv_block *)calloc((size_t)cap, sizeof(t_kv_block));
    bm->page_table = (int *)malloc((size_t)cap * sizeof(int));
    bm->free_stack = (int *)malloc((size_t)cap * sizeof(int));
    bm->logical_len = (int *)calloc((size_t)n_layers, sizeof(int));
    if (!bm->blocks || !bm->page_table || !bm->free_stack || !bm->logical_len) {
        fprintf(stderr, "[PagedKV] ERROR: host allocation failed\n");
        free(bm->blocks);
        free(bm->page_table);
        free(bm->free_stack);
        free(bm->logical_len);
        be42_kv_destroy(pool);
        memset(bm, 0, sizeof *bm);
        return -1;
    }
    const size_t kv = (size_t)n_kv_heads * KV_BLOCK_SIZE * head_dim;
    const size_t sc = (size_t)n_kv_heads * KV_BLOCK_SIZE;
    for (int i = 0; i < cap; i++) {
        t_kv_block &b = bm->blocks[i];
        b.k_quant = (int8_t *)pool->k + i * kv;
        b.v_quant = (int8_t *)pool->v + i * kv;
        b.k_scales = pool->k_scale + i * sc;
        b.v_scales = pool->v_scale + i * sc;
        b.centroid = pool->centroid + (size_t)i * head_dim;
        b.n_tokens = 0;
        b.start_pos = -1;
        b.layer_idx = -1;
        b.lsh_registered = 0;
        b.lsh_hash = 0;
    }
    sync_manager(bm, pool);
    Runtime::Pool &e = rt().pools[bm];
    e.pool = pool;
    e.blocks = bm->blocks;
    e.page_table = bm->page_table;
    e.capacity = bm->capacity;
    e.n_layers = bm->n_layers;
    e.n_kv_heads = bm->n_kv_heads;
    e.head_dim = bm->head_dim;
    e.max_logical = bm->max_logical;
    return 0;
}

extern "C" void block_manager_free(t_block_manager *bm)
{
    std::lock_guard<std::mutex> g(rt().mu);
    Runtime &r = rt();
    auto it = r.pools.find(bm);
    if (it != r.pools.end())
        pool_drop(r, it);
    free(bm->blocks);
    free(bm->page_table);
    free(bm->free_stack);
    free(bm->logical_len);
    memset(bm, 0, sizeof *bm);
}

extern "C" int block_alloc(t_block_manager *bm)
{
    std::lock_guard<std::mutex> g(rt().mu);
    be42_kv_pool *pool = pool_of(bm, "block_alloc");
    const int phys = be42_kv_page_alloc(pool);
    if (phys < 0) {
        fprintf(stderr, "[PagedKV] ERROR: Block pool exhausted!\n");
        return -1;
    }
    t_kv_block &b = bm->blocks[phys];
    b.n_tokens = 0;
    b.start_pos = -1;
    b.layer_idx = -1;
    b.lsh_registered = 0;
    b.lsh_hash = 0;
    sync_manager(bm, pool);
    return phys;
}

extern "C" void block_free(t_block_manager *bm, int phys_idx)
{
    std::lock_guard<std::mutex> g(rt().mu);
    be42_kv_pool *pool = pool_of(bm, "block_free");
    ok(be42_kv_page_free(pool, phys_idx), "block_free");
    sync_manager(bm, pool);
}

extern "C" void paged_kv_append(t_paged_kv_cache *pkv, const float *k, const float *v, int pos)
{
    std::lock_guard<std::mutex> g(rt().mu);
    t_block_manager *bm = pkv->bm;
    be42_kv_pool *pool = pool_of(bm, "paged_kv_append");
    const int layer = pkv->layer_idx;
    const int blk = pos / KV_BLOCK_SIZE, off = pos % KV_BLOCK_SIZE;
    const int base = layer * bm->max_logical;
    const bool fresh = blk >= bm->logical_len[layer];
    const size_t row = (size_t)bm->n_kv_heads * bm->head_dim * 4;
    const float *dk = (const float *)in_dev(k, row, kS0);
    const float *dv = (const float *)in_dev(v, row, kS1);
    const int rc = be42_kv_append(pool, layer, dk, dv, pos, 1, nullptr);
    if (rc == BE42_ENOMEM) {
        fprintf(stderr, "[PagedKV] FATAL: Block pool exhausted at pos=%d\n", pos);
        exit(1);
    }
    ok(rc, "paged_kv_append");
    sync_manager(bm, pool);
    const int phys = bm->page_table[base + blk];
    t_kv_block &b = bm->blocks[phys];
    if (fresh) {
        b.n_tokens = 0;
        b.layer_idx = -1;
        b.lsh_registered = 0;
        b.lsh_hash = 0;
        b.start_pos = blk * KV_BLOCK_SIZE;
        pkv->n_blocks = blk + 1;
    }
    b.n_tokens = off + 1;
    b.layer_idx = layer;
    pkv->n_tokens = pos + 1;
    if (b.n_tokens == KV_BLOCK_SIZE && !b.lsh_registered)
        b.lsh_registered = 1;   // the pool computed the centroid when the page filled
}

extern "C" void paged_kv_get_int8(t_paged_kv_cache *pkv, int pos, int kv_head, int8_t **out_k, int8_t **out_v,
                                  float *out_k_scale, float *out_v_scale)
{
    std::lock_guard<std::mutex> g(rt().mu);
    t_block_manager *bm = pkv->bm;
    const int blk = pos / KV_BLOCK_SIZE, off = pos % KV_BLOCK_SIZE;
    const int phys = bm->page_table[pkv->layer_idx * bm->max_logical + blk];
    if (phys < 0) {
        *out_k = nullptr;
        *out_v = nullptr;
        *out_k_scale = 0.0f;
        *out_v_scale = 0.0f;
        return;
    }
    const t_kv_block &b = bm->blocks[phys];
    const int data = kv_head * KV_BLOCK_SIZE * bm->head_dim + off * bm->head_dim;
    const int si = kv_head * KV_BLOCK_SIZE + off;
    *out_k = b.k_quant + data;
    *out_v = b.v_quant + data;
    hip_ok(hipMemcpy(out_k_scale, b.k_scales + si, 4, hipMemcpyDeviceToHost), "paged_kv_get_int8");
    hip_ok(hipMemcpy(out_v_scale, b.v_scales + si, 4, hipMemcpyDeviceToHost), "paged_kv_get_int8");
}

extern "C" void paged_kv_reset(t_paged_kv_cache *pkv)
{
    std::lock_guard<std::mutex> g(rt().mu);
    t_block_manager *bm = pkv->bm;
    be42_kv_pool *pool = pool_of(bm, "paged_kv_reset");
    ok(be42_kv_reset(pool, pkv->layer_idx, nullptr), "paged_kv_reset");
    sync_manager(bm, pool);
    pkv->n_blocks = 0;
    pkv->n_tokens = 0;
}

extern "C" void calc_block_centroid_int8(t_kv_block *block, int head_dim, int n_kv_heads)
{
    (void)n_kv_heads;   // head 0
    if (block->n_tokens <= 0)
        return;
    std::lock_guard<std::mutex> g(rt().mu);
    hipLaunchKernelGGL(k_centroid_one, dim3((head_dim + 255) / 256), dim3(256), 0, nullptr, block->centroid,
                       block->k_quant, block->k_scales, block->n_tokens, head_dim);
    hip_ok(hipGetLastError(), "calc_block_centroid_int8");
    hip_ok(hipStreamSynchronize(nullptr), "calc_block_centroid_int8");
}

extern "C" void score_blocks(t_block_score *scores, const float *q, t_paged_kv_cache *pkv, int n_blocks)
{
    if (n_blocks <= 0)
        return;
    std::lock_guard<std::mutex> g(rt().mu);
    t_block_manager *bm = pkv->bm;
    be42_kv_pool *pool = pool_of(bm, "score_blocks");
    const int hd = bm->head_dim;
    const float *dq = (const float *)in_dev(q, (size_t)hd * 4, kS0);
    // page-table entries past max_logical do not exist: map them to -1
    int *pt = (int *)scratch(kS2, (size_t)n_blocks * 4);
    const int base = pkv->layer_idx * bm->max_logical;
    std::vector<int> host((size_t)n_blocks, -1);
    for (int i = 0; i < n_blocks && i < bm->max_logical; i++)
        host[i] = bm->page_table[base + i];
    hip_ok(hipMemcpy(pt, host.data(), (size_t)n_blocks * 4, hipMemcpyHostToDevice), "score_blocks");
    bool st;
    t_block_score *d = (t_block_score *)out_dev(scores, (size_t)n_blocks * sizeof(t_block_score), kS1, &st);
    const int blocks = (2 * n_blocks + 255) / 256;
    hipLaunchKernelGGL(k_score_pages, dim3(blocks), dim3(256), 0, nullptr, d, dq, pool->centroid, pt, n_blocks, hd);
    hip_ok(hipGetLastError(), "score_blocks");
    out_done(scores, d, (size_t)n_blocks * sizeof(t_block_score), st);
}

extern "C" int select_top_k_blocks(int *selected, t_block_score *scores, int n_blocks, int k)
{
    if (n_blocks <= 0)
        return 0;
    if (n_blocks > kSelMax) {
        char msg[64];
        snprintf(msg, sizeof msg, "%d blocks exceed %d", n_blocks, kSelMax);
        die("select_top_k_blocks", msg);
    }
    std::lock_guard<std::mutex> g(rt().mu);
    const t_block_score *ds =
        (const t_block_score *)in_dev(scores, (size_t)n_blocks * sizeof(t_block_score), kS0);
    int *dsel = (int *)scratch(kS1, 64 * 4 + 4);
    int *dn = dsel + 64;
    const size_t smem = (size_t)n_blocks * 8;
    if (smem > 65536)
        hip_ok(hipFuncSetAttribute((const void *)k_select_top_k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                   (int)smem),
               "select_top_k_blocks");
    hipLaunchKernelGGL(k_select_top_k, dim3(1), dim3(256), smem, nullptr, dsel, dn, ds, n_blocks, k);
    hip_ok(hipGetLastError(), "select_top_k_blocks");
    int n = 0;
    hip_ok(hipMemcpy(&n, dn, 4, hipMemcpyDeviceToHost), "select_top_k_blocks");
    if (is_device(selected))
        hip_ok(hipMemcpy(selected, dsel, (size_t)n * 4, hipMemcpyDeviceToDevice), "select_top_k_blocks");
    else
        hip_ok(hipMemcpy(selected, dsel, (size_t)n * 4, hipMemcpyDeviceToHost), "select_top_k_blocks");
    return n;
}

// ---- LSH diagnostics (ops_lsh.c:447-668) ---------------------------------------------

extern "C" void lsh_stats_reset_atomic(t_lsh_stats_atomic *s)
{
    if (!s)
        return;
    uint64_t *f[] = {&s->total_queries, &s->validated_queries, &s->topk_hits, &s->topk_total,
                     &s->recall_scaled, &s->validation_count, &s->total_used_k, &s->k_samples};
    for (uint64_t *p : f)
        __atomic_store_n(p, 0, __ATOMIC_SEQ_CST);
}

extern "C" void lsh_stats_print_atomic(const t_lsh_stats_atomic *s, int sparse_k)
{
    if (!s)
        return;
    const uint64_t total_q = __atomic_load_n(&s->total_queries, __ATOMIC_SEQ_CST);
    const uint64_t validated = __atomic_load_n(&s->validated_queries, __ATOMIC_SEQ_CST);
    const uint64_t hits = __atomic_load_n(&s->topk_hits, __ATOMIC_SEQ_CST);
    const uint64_t total = __atomic_load_n(&s->topk_total, __ATOMIC_SEQ_CST);
    const uint64_t used_k = __atomic_load_n(&s->total_used_k, __ATOMIC_SEQ_CST);
    const uint64_t k_samples = __atomic_load_n(&s->k_samples, __ATOMIC_SEQ_CST);
    if (validated == 0 || total == 0) {
        printf("[LSH Stats] No validation data collected.\n");
        fflush(stdout);
        return;
    }
    const float recall = (float)hits / (float)total;
    const float avg_k = k_samples > 0 ? (float)used_k / (float)k_samples : 0.0f;
    const float savings = sparse_k > 0 ? (1.0f - avg_k / (float)sparse_k) * 100.0f : 0.0f;
    printf("[LSH Stats] Queries: %lu (validated: %lu)\n", (unsigned long)total_q, (unsigned long)validated);
    printf("[LSH Stats] Recall: %.1f%% (target: >80%%)\n", recall * 100.0f);
    printf("[LSH Stats] Avg Dynamic K: %.1f (savings: %.1f%%)\n", avg_k, savings);
    if (recall < 0.8f)
        printf("[LSH Stats] WARNING: Recall below 80%% - sparse attention degraded!\n");
    else
        printf("[LSH Stats] Recall acceptable\n");
    fflush(stdout);
}

extern "C" float lsh_validate_recall(const float *query, const uint16_t *keys, int n_keys, int dim,
                                     const int *lsh_indices, int lsh_k, int actual_k)
{
    if (actual_k > n_keys)
        actual_k = n_keys;
    if (lsh_k > actual_k)
        lsh_k = actual_k;
    if (actual_k > kValMaxTopK)
        actual_k = kValMaxTopK;
    if (actual_k <= 0)
        return NAN;   // the reference divides 0 hits by actual_k = 0
    const int stride = n_keys > kValMaxKeys ? n_keys / kValMaxKeys : 1;
    const int actual_n = n_keys > kValMaxKeys ? kValMaxKeys : n_keys;
    std::lock_guard<std::mutex> g(rt().mu);
    const float *dq = (const float *)in_dev(query, (size_t)dim * 4, kS0);
    const uint16_t *dk = (const uint16_t *)in_dev(keys, (size_t)n_keys * dim * 2, kS2);
    const int nl = lsh_k > 0 ? lsh_k : 0;
    const int *dl = (const int *)in_dev(lsh_indices, (size_t)nl * 4, kS3);
    int *dh = (int *)scratch(kS1, 4);
    hipLaunchKernelGGL(k_validate_recall, dim3(1), dim3(256), 0, nullptr, dh, dq, dk, actual_n, stride, dim,
                       nl ? dl : nullptr, nl, actual_k);
    hip_ok(hipGetLastError(), "lsh_validate_recall");
    int hits = 0;
    hip_ok(hipMemcpy(&hits, dh, 4, hipMemcpyDeviceToHost), "lsh_validate_recall");
    return (float)hits / (float)actual_k;
}

extern "C" int adaptive_k_cutoff(const float *scores, const int *indices, int n_cand, float threshold)
{
    (void)indices;
    if (n_cand <= 0)
        return 1;
    std::lock_guard<std::mutex> g(rt().mu);
    const float *ds = (const float *)in_dev(scores, (size_t)n_cand * 4, kS0);
    int *dk = (int *)scratch(kS1, 4);
    hipLaunchKernelGGL(k_adaptive_k, dim3(1), dim3(1), 0, nullptr, dk, ds, n_cand, threshold);
    hip_ok(hipGetLastError(), "adaptive_k_cutoff");
    int k = 1;
    hip_ok(hipMemcpy(&k, dk, 4, hipMemcpyDeviceToHost), "adaptive_k_cutoff");
    return k;
}

// ---- linear KV cache and its attention (kv_cache.c, ops_attention.c:41-245) -------------

// arena_alloc_or_die / arena_try_alloc (arena.c:80-115): 64-byte aligned bump
// allocation, zeroed; fatal when the arena is too small
static void *arena_take(t_arena *a, size_t size)
{
    const size_t padding = (64 - (a->offset % 64)) % 64;
    if (padding > a->size - a->offset || size > a->size - a->offset - padding) {
        fprintf(stderr, "Fatal: arena OOM (requested %zu bytes, %zu/%zu used)\n", size, a->offset, a->size);
        exit(1);
    }
    a->offset += padding;
    void *p = a->base + a->offset;
    a->offset += size;
    memset(p, 0, size);
    return p;
}

static t_tensor view3(void *data, int d0, int d1, int d2)
{
    t_tensor t{};
    t.data = data;
    t.ndim = 3;
    t.shape[0] = d0;
    t.shape[1] = d1;
    t.shape[2] = d2;
    t.shape[3] = 1;
    t.stride[0] = d1 * d2;
    t.stride[1] = d2;
    t.stride[2] = 1;
    t.size = (size_t)d0 * d1 * d2;
    t.dtype = DTYPE_BF16;
    return t;
}

static void linear_drop(Runtime &r, std::unordered_map<const t_kv_cache *, Runtime::Linear>::iterator it)
{
    hip_ok(hipDeviceSynchronize(), "kv cache release");
    hip_ok(hipFree(it->second.k), "kv cache release");
    hip_ok(hipFree(it->second.v), "kv cache release");
    r.linear.erase(it);
}

extern "C" void kv_cache_init(t_kv_cache *c, t_arena *a, t_kv_init_params *p)
{
    c->max_seq_len = p->max_seq;
    c->num_heads = p->num_heads;
    c->head_dim = p->head_dim;
    c->current_seq_len = 0;
    const size_t bytes = (size_t)p->max_seq * p->num_heads * p->head_dim * sizeof(t_bf16);
    c->k = view3(arena_take(a, bytes), p->max_seq, p->num_heads, p->head_dim);
    c->v = view3(arena_take(a, bytes), p->max_seq, p->num_heads, p->head_dim);
    std::lock_guard<std::mutex> g(rt().mu);
    Runtime &r = rt();
    auto it = r.linear.find(c);
    if (it != r.linear.end())
        linear_drop(r, it);
    Runtime::Linear &m = r.linear[c];
    m.rows = (size_t)p->max_seq;
    m.row = (size_t)p->num_heads * p->head_dim;
    m.hk = c->k.data;
    m.hv = c->v.data;
    m.max_seq = c->max_seq_len;
    m.heads = c->num_heads;
    m.dim = c->head_dim;
    hip_ok(hipMalloc((void **)&m.k, bytes ? bytes : 2), "kv_cache_init");
    hip_ok(hipMalloc((void **)&m.v, bytes ? bytes : 2), "kv_cache_init");
    // zero like the arena rows, so rows past the current length read the same
    hip_ok(hipMemset(m.k, 0, bytes ? bytes : 2), "kv_cache_init");
    hip_ok(hipMemset(m.v, 0, bytes ? bytes : 2), "kv_cache_init");
}

// The mirror kv_cache_init made for the struct at c, or null: an entry is
// used only while the struct still names the arena rows and the shape it was
// made for (a struct freed and its address reused by another cache, or a
// cache the caller re-pointed, does not), and a stale entry is released.
static Runtime::Linear *linear_entry(const t_kv_cache *c)
{
    Runtime &r = rt();
    auto it = r.linear.find(c);
    if (it == r.linear.end())
        return nullptr;
    const Runtime::Linear &m = it->second;
    if (m.hk == c->k.data && m.hv == c->v.data && m.max_seq == c->max_seq_len && m.heads == c->num_heads &&
        m.dim == c->head_dim)
        return &it->second;
    linear_drop(r, it);
    return nullptr;
}

// the device rows of a cache: its mirror, or a staged copy of the host rows
// [0, n) (a cache this library did not create)
static const Runtime::Linear &linear_dev(const t_kv_cache *c, int n, Runtime::Linear &tmp)
{
    if (const Runtime::Linear *m = linear_entry(c))
        return *m;
    tmp.row = (size_t)c->num_heads * c->head_dim;
    const size_t bytes = (size_t)n * tmp.row * 2;
    tmp.k = (uint16_t *)in_dev(c->k.data, bytes, kS6);
    tmp.v = (uint16_t *)in_dev(c->v.data, bytes, kS7);
    return tmp;
}

extern "C" void kv_cache_release(const t_kv_cache *c)
{
    std::lock_guard<std::mutex> g(rt().mu);
    Runtime &r = rt();
    auto it = r.linear.find(c);
    if (it != r.linear.end())
        linear_drop(r, it);
}

extern "C" void kv_cache_append(t_kv_cache *c, const t_tensor *k_in, const t_tensor *v_in)
{
    if (c->current_seq_len >= c->max_seq_len) {
        fprintf(stderr, "KV Cache Full!\n");
        return;
    }
    std::lock_guard<std::mutex> g(rt().mu);
    Runtime::Linear *m = linear_entry(c);
    const int idx = c->current_seq_len;
    const int row = c->num_heads * c->head_dim;
    uint16_t *hk = (uint16_t *)c->k.data + (size_t)idx * row, *hv = (uint16_t *)c->v.data + (size_t)idx * row;
    if (k_in->dtype == DTYPE_F32) {
        // rounded to bf16 on the device: into the mirror's row, or (a cache
        // without a mirror) into a staging row; then copied to the host row
        const float *fk = (const float *)in_dev(k_in->data, (size_t)row * 4, kS0);
        const float *fv = (const float *)in_dev(v_in->data, (size_t)row * 4, kS2);
        uint16_t *mk = m ? m->k : (uint16_t *)scratch(kS6, (size_t)row * 2);
        uint16_t *mv = m ? m->v : (uint16_t *)scratch(kS7, (size_t)row * 2);
        const int at = m ? idx : 0;
        ok(be42_kv_linear_append(mk, mv, at, fk, fv, row, nullptr), "kv_cache_append");
        hip_ok(hipMemcpy(hk, mk + (size_t)at * row, (size_t)row * 2, hipMemcpyDeviceToHost), "kv_cache_append");
        hip_ok(hipMemcpy(hv, mv + (size_t)at * row, (size_t)row * 2, hipMemcpyDeviceToHost), "kv_cache_append");
    } else {
        memcpy(hk, k_in->data, (size_t)row * 2);
        memcpy(hv, v_in->data, (size_t)row * 2);
        if (m) {
            hip_ok(hipMemcpy(m->k + (size_t)idx * row, hk, (size_t)row * 2, hipMemcpyHostToDevice), "kv_cache_append");
            hip_ok(hipMemcpy(m->v + (size_t)idx * row, hv, (size_t)row * 2, hipMemcpyHostToDevice), "kv_cache_append");
        }
    }
    c->current_seq_len++;
}

extern "C" void kv_cache_evict(t_kv_cache *c, t_evict_params *p)
{
    if (p->keep_k <= 0) {
        fprintf(stderr, "Warning: kv_cache_evict keep_k=%d invalid\n", p->keep_k);
        return;
    }
    int keep_k = p->keep_k;
    if (keep_k > c->current_seq_len)
        keep_k = c->current_seq_len;
    if (keep_k > c->max_seq_len)
        keep_k = c->max_seq_len;
    if (c->current_seq_len <= keep_k)
        return;
    const int n = c->current_seq_len, heads = c->num_heads, dim = c->head_dim;
    // the reference takes its sort buffer from the scratch arena (and gives
    // it back): the same arena must be large enough
    {
        const size_t padding = (64 - (p->scratch->offset % 64)) % 64;
        const size_t need = (size_t)n * 8;
        if (padding > p->scratch->size - p->scratch->offset || need > p->scratch->size - p->scratch->offset - padding) {
            fprintf(stderr, "Fatal: arena OOM (requested %zu bytes, %zu/%zu used)\n", need, p->scratch->offset,
                    p->scratch->size);
            exit(1);
        }
    }
    std::lock_guard<std::mutex> g(rt().mu);
    Runtime::Linear tmp;
    const Runtime::Linear &m = linear_dev(c, n, tmp);
    const uint16_t *dq = (const uint16_t *)in_dev(p->q->data, (size_t)heads * dim * 2, kS0);
    const uint16_t *dw = (const uint16_t *)in_dev(p->w->data, (size_t)heads * 2, kS2);
    int new_len = n;
    ok(be42_kv_linear_evict(m.k, m.v, n, heads, dim, dq, dw, keep_k, &new_len, nullptr), "kv_cache_evict");
    const size_t bytes = (size_t)new_len * heads * dim * 2;
    hip_ok(hipMemcpy(c->k.data, m.k, bytes, hipMemcpyDeviceToHost), "kv_cache_evict");
    hip_ok(hipMemcpy(c->v.data, m.v, bytes, hipMemcpyDeviceToHost), "kv_cache_evict");
    c->current_seq_len = new_len;
}

static void linear_attention(float *out, const float *q, const uint16_t *dk, const uint16_t *dv, const int *idx_host,
                             int n_tok, int n_heads, int n_kv, int hd, float scale, const char *what)
{
    const size_t qb = (size_t)n_heads * hd * 4;
    const float *dq = (const float *)in_dev(q, qb, kS0);
    const int *di = idx_host ? (const int *)in_dev(idx_host, (size_t)(n_tok > 0 ? n_tok : 0) * 4, kS3) : nullptr;
    bool st;
    float *o = (float *)out_dev(out, qb, kS1, &st);
    const size_t wsb = be42_linear_attention_workspace_bytes(n_tok, n_heads, n_kv, hd);
    void *ws = scratch(kS5, wsb ? wsb : 16);
    ok(be42_linear_attention(o, dq, dk, dv, di, n_tok, n_heads, n_kv, hd, scale, ws, wsb, nullptr), what);
    out_done(out, o, qb, st);
}

extern "C" void flash_attention_head(float *out, const float *q, const t_bf16 *k_cache, const t_bf16 *v_cache,
                                     int seq_len, int head_dim, float scale)
{
    std::lock_guard<std::mutex> g(rt().mu);
    const size_t bytes = (size_t)(seq_len > 0 ? seq_len : 0) * head_dim * 2;
    const uint16_t *dk = (const uint16_t *)in_dev(k_cache, bytes, kS6);
    const uint16_t *dv = (const uint16_t *)in_dev(v_cache, bytes, kS7);
    linear_attention(out, q, dk, dv, nullptr, seq_len, 1, 1, head_dim, scale, "flash_attention_head");
}

extern "C" void op_attention_dense(t_attention_params *p, int kv_len)
{
    std::lock_guard<std::mutex> g(rt().mu);
    Runtime::Linear tmp;
    const Runtime::Linear &m = linear_dev(p->kv_cache, kv_len, tmp);
    linear_attention(p->output, p->q, m.k, m.v, nullptr, kv_len, p->n_heads, p->n_kv_heads, p->head_dim, p->scale,
                     "op_attention_dense");
}

extern "C" void op_attention_sparse(t_attention_params *p)
{
    std::lock_guard<std::mutex> g(rt().mu);
    Runtime::Linear tmp;
    const t_kv_cache *c = p->kv_cache;
    const Runtime::Linear &m = linear_dev(c, c->current_seq_len, tmp);
    // positions must name rows the device holds: the whole cache for one that
    // kv_cache_init made, the first current_seq_len rows of a staged one
    const int rows = m.rows ? (int)m.rows : c->current_seq_len;
    for (int i = 0; i < p->attend_k; i++)
        if (p->topk_idx[i] < 0 || p->topk_idx[i] >= rows)
            die("op_attention_sparse", "position out of the cache");
    linear_attention(p->output, p->q, m.k, m.v, p->topk_idx, p->attend_k, p->n_heads, p->n_kv_heads, p->head_dim,
                     p->scale, "op_attention_sparse");
}

extern "C" void op_multihead_attention(t_attention_params *p)
{
    const int kv_len = p->kv_cache->current_seq_len;
    if (p->topk_idx != nullptr && p->attend_k > 0 && p->attend_k < kv_len)
        op_attention_sparse(p);
    else
        op_attention_dense(p, kv_len);
}

// ---- paged attention ------------------------------------------------------------------

extern "C" void op_paged_attention_sparse(float *output, const float *q, t_block_manager *bm,
                                          const int *selected_blocks, int n_selected, int n_heads, int n_kv_heads,
                                          int head_dim, float scale)
{
    std::lock_guard<std::mutex> g(rt().mu);
    paged_attention(output, q, pool_of(bm, "op_paged_attention_sparse"), selected_blocks, n_selected, n_heads,
                    n_kv_heads, head_dim, scale, "op_paged_attention_sparse");
}

extern "C" void op_paged_attention(float *output, const float *q, t_paged_kv_cache *pkv, int n_heads,
                                   int n_kv_heads, int head_dim, float scale)
{
    std::lock_guard<std::mutex> g(rt().mu);
    t_block_manager *bm = pkv->bm;
    const int n = pkv->n_blocks;
    std::vector<int> sel;
    sel.reserve(n > 0 ? n : 0);
    const int base = pkv->layer_idx * bm->max_logical;
    for (int i = 0; i < n; i++)
        if (bm->page_table[base + i] >= 0)
            sel.push_back(bm->page_table[base + i]);
    paged_attention(output, q, pool_of(bm, "op_paged_attention"), sel.data(), (int)sel.size(), n_heads,
                    n_kv_heads, head_dim, scale, "op_paged_attention");
}
