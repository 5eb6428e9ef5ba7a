// decode.hip -- the decode step of a Llama-style decoder on gfx950: the
// per-token operations around the quantized GEMVs and the paged attention,
// and the loop that chains them (transformer_forward,
// src/inference/inference.c:60-696, paged path).
//
// embedding (row-scaled codes)                  inference.c:88 (extension: quantized table)
// op_rmsnorm                                    src/compute/ops_norm.c:27-138
// rope_cache_init / rope_apply_multihead_cached src/compute/ops_rope.c:30-95, :192-228
// op_silu_mul -> op_silu_mul_fused_f32          src/compute/ops_silu.c:67, ops_activation.c:48-105
// residual add (simd_add_f32)                   src/compute/simd_kernels.h:359
// sample_argmax (argmax_simd_f32)               src/compute/sampler.c:42-148
//
// Every elementwise operation reproduces the reference's rounding: RMSNorm
// sums squares in the 8-lane FMA order of compute_rms_f32_avx2 and divides
// and square-roots in IEEE; RoPE evaluates x0*c - x1*s and x0*s + x1*c as the
// compiled loop does (one FMA each); SiLU uses the vector Schraudolph exp
// (clamp, fused multiply-add, round to nearest).  The GEMVs are the library's
// MFMA GEMVs (fp32-accurate), attention is the fused paged attention (dense
// while a layer has <= sparse_k pages, else the LSH route).
#include <algorithm>
#include <type_traits>
#include <cmath>
#include <cstring>
#include <initializer_list>
#include <vector>

#include "attn_dev.h"
#include "be42_common.h"
#include "paged_dev.h"
#include "paged_step.h"
#include "xdigits.h"

namespace be42 {

constexpr int kMaxBatch = 16;

// Parameters of one step, written by the host into pinned memory and copied
// to the device at the start of the step: with them in device memory the
// launch sequence of a step is the same for every position, so it is
// captured once as a HIP graph and replayed.
struct StepHead {
    int pos;
    int tokens[kMaxBatch];
};

// tokens from device memory: the step's parameters, or the previous step's
// argmax
template <bool FP8>
__global__ __launch_bounds__(256) void k_embed(float *__restrict__ x, const uint8_t *__restrict__ emb,
                                               const float *__restrict__ emb_s, const int *__restrict__ tok_p,
                                               int dim)
{
    const int b = blockIdx.y, i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= dim)
        return;
    const int tok = tok_p[b];
    const uint8_t c = emb[(size_t)tok * dim + i];
    const float v = FP8 ? fp8_to_f32(c) : (float)(int8_t)c;
    x[(size_t)b * dim + i] = v * emb_s[tok];
}

// Row kernels of the decode step (RMSNorm, SiLU*up), written straight as the
// next GEMV's digit planes.  The digit scale needs the row's max |h|, so a row
// is spread over workgroups this way: block (c, b) of a row of n elements
// evaluates the whole row in registers (thread t holds float4 number
// t + kRowT * j, j < NV) and reduces it itself, then writes only chunk c of the
// digit planes (elements [kChunk c, kChunk (c + 1)), zero past n; kChunk is
// the planes' burst, so the chunks tile the padded row).  Every block thus
// takes the row's few KiB from L2 and does a little redundant arithmetic,
// instead of one block doing the whole row's digit split.
constexpr int kRowT = 256;
constexpr int kChunk = 4 * kRowT;
constexpr int kRowNV = 16;                       // rows up to 16384 elements
constexpr int kRowMax = kChunk * kRowNV;

__device__ __forceinline__ float f4_absmax(float4 a)
{
    return fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w)));
}

__device__ __forceinline__ float4 f4_zero() { return make_float4(0.f, 0.f, 0.f, 0.f); }

// block (kRowT threads) reductions; every thread gets the result
__device__ __forceinline__ float block_sum4(float v, float *red)
{
    v = wave_sum_dpp(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

__device__ __forceinline__ float block_max4(float v, float *red)
{
    v = wave_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0)
        red[4 + (threadIdx.x >> 6)] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[4], red[5]), fmaxf(red[6], red[7]));
}

// chunk c of row b's digit planes (and fp32 out) from the row in registers;
// c < 0: every chunk (one block per row, for many rows)
template <bool FP8, int NV>
__device__ __forceinline__ void row_chunk_digits(const float4 (&h)[NV], int n, uint8_t *__restrict__ dig,
                                                 float *__restrict__ out, int B, int b, int c, float *red)
{
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; j++)
        m = fmaxf(m, f4_absmax(h[j]));
    const float amax = block_max4(m, red);
    const float sc = digit_scale<FP8>(amax);
    const int Kp = (int)xdig_kp(n, FP8);
    if (c <= 0 && threadIdx.x == 0)
        xdig_scales(dig, n, B, FP8)[b] = sc;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        if (j == c || c < 0) {
            const int i = (int)threadIdx.x + kRowT * j, k0 = 4 * i;
            if (k0 < Kp) {
                const float xe[4] = {h[j].x, h[j].y, h[j].z, h[j].w};
                store_digit_words<FP8>(xe, sc, dig, B, Kp, b, k0);
            }
            if (out && 4 * i < n)
                ((float4 *)(out + (size_t)b * n))[i] = h[j];
        }
    }
}

// xn = rmsnorm(x [+ delta]) of row b (op_rmsnorm, ops_norm.c:126-138):
// ss = sum x^2, inv = 1 / sqrtf(ss / dim + eps), h = (x * inv) * w.  With
// delta the residual add of inference.c:525/:577 comes first and the sum
// x + delta is written to x_out (chunk c by block c; x_out is not x, so no
// block reads a value another has already updated).  The sum of squares is
// a tree (per-thread fused multiply-adds, then DPP and LDS sums), not the
// reference's 8 sequential lanes: equal to fp32 rounding, far inside the
// decode tolerance.
template <bool FP8, int NV>
__global__ __launch_bounds__(kRowT) void k_rmsnorm(float *__restrict__ out, uint8_t *__restrict__ dig,
                                                  const float *__restrict__ x, float *__restrict__ x_out,
                                                  const float *__restrict__ delta, const uint16_t *__restrict__ w,
                                                  int dim, int B, float eps, bool all_chunks)
{
    __shared__ float red[8];
    const int b = blockIdx.y, c = all_chunks ? -1 : (int)blockIdx.x, n4 = dim >> 2;
    const float4 *x4 = (const float4 *)(x + (size_t)b * dim);
    const float4 *d4 = delta ? (const float4 *)(delta + (size_t)b * dim) : nullptr;
    const uint2 *w4 = (const uint2 *)w;
    float4 v[NV], dv[NV];
    uint2 wv[NV];
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int i = min((int)threadIdx.x + kRowT * j, n4 - 1);
        v[j] = x4[i];
        wv[j] = w4[i];
        if (d4)
            dv[j] = d4[i];
    }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int i = threadIdx.x + kRowT * j;
        if (d4) {
            v[j] = make_float4(v[j].x + dv[j].x, v[j].y + dv[j].y, v[j].z + dv[j].z, v[j].w + dv[j].w);
            if ((j == c || c < 0) && i < n4)
                ((float4 *)(x_out + (size_t)b * dim))[i] = v[j];
        }
        if (i >= n4)
            v[j] = f4_zero();
        ss = __fmaf_rn(v[j].x, v[j].x, ss);
        ss = __fmaf_rn(v[j].y, v[j].y, ss);
        ss = __fmaf_rn(v[j].z, v[j].z, ss);
        ss = __fmaf_rn(v[j].w, v[j].w, ss);
    }
    ss = block_sum4(ss, red);
    const float inv = __fdiv_rn(1.0f, sqrtf(__fdiv_rn(ss, (float)dim) + eps));
    float4 h[NV];
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const uint2 wj = wv[j];
        h[j] = make_float4((v[j].x * inv) * bf16_to_f32((uint16_t)(wj.x & 0xFFFF)),
                           (v[j].y * inv) * bf16_to_f32((uint16_t)(wj.x >> 16)),
                           (v[j].z * inv) * bf16_to_f32((uint16_t)(wj.y & 0xFFFF)),
                           (v[j].w * inv) * bf16_to_f32((uint16_t)(wj.y >> 16)));
        if ((int)threadIdx.x + kRowT * j >= n4)
            h[j] = f4_zero();
    }
    row_chunk_digits<FP8, NV>(h, dim, dig, out, B, b, c, red);
}

// h = (g * sigmoid(g)) * u for row b (op_silu_mul_fused_f32): blocks of 8 use
// the vector Schraudolph exp (clamp, fused multiply-add, round to nearest),
// the n % 8 remainder the scalar one; written as GEMV digit planes of the
// down projection (and to out if not NULL).  Element for element the
// reference's arithmetic.
__device__ __forceinline__ float silu_mul1(float gv, float uv, bool vec)
{
    float e;
    if (vec) {
        float xv = 0.0f - gv;
        xv = fmaxf(xv, -87.0f);
        xv = fminf(xv, 87.0f);
        e = __int_as_float(__float2int_rn(__fmaf_rn(xv, 12102203.0f, 1065353216.0f)));
    } else {
        e = fast_expf(-gv);
    }
    const float sig = __fdiv_rn(1.0f, 1.0f + e);
    return (gv * sig) * uv;
}

template <bool FP8, int NV>
__global__ __launch_bounds__(kRowT) void k_silu_mul(float *__restrict__ out, uint8_t *__restrict__ dig,
                                                   const float *__restrict__ g, const float *__restrict__ u, int n,
                                                   int B, bool all_chunks)
{
    __shared__ float red[8];
    const int b = blockIdx.y, c = all_chunks ? -1 : (int)blockIdx.x, n4 = n >> 2, nvec = n & ~7;
    const float4 *g4 = (const float4 *)(g + (size_t)b * n), *u4 = (const float4 *)(u + (size_t)b * n);
    float4 gv[NV], uv[NV];
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int i = min((int)threadIdx.x + kRowT * j, n4 - 1);
        gv[j] = g4[i];
        uv[j] = u4[i];
    }
    float4 h[NV];
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int i = threadIdx.x + kRowT * j, e0 = 4 * i;
        h[j] = make_float4(silu_mul1(gv[j].x, uv[j].x, e0 < nvec), silu_mul1(gv[j].y, uv[j].y, e0 + 1 < nvec),
                           silu_mul1(gv[j].z, uv[j].z, e0 + 2 < nvec), silu_mul1(gv[j].w, uv[j].w, e0 + 3 < nvec));
        if (i >= n4)
            h[j] = f4_zero();
    }
    row_chunk_digits<FP8, NV>(h, n, dig, out, B, b, c, red);
}

// k_silu_mul of a whole row by one 1024-thread block (the decoder's batched
// steps, without an fp32 copy): the same elements, maximum and digits as the
// 256-thread chunked kernel -- a maximum does not depend on its order -- in
// a quarter of the per-thread work.  NV * 4096 >= the digit planes' row.
constexpr int kWideT = 1024;
template <bool FP8, int NV>
__global__ __launch_bounds__(kWideT) void k_silu_mul_wide(uint8_t *__restrict__ dig, const float *__restrict__ g,
                                                         const float *__restrict__ u, int n, int B)
{
    __shared__ float red[kWideT / kWave];
    const int b = blockIdx.x, tid = threadIdx.x, n4 = n >> 2, nvec = n & ~7;
    const float4 *g4 = (const float4 *)(g + (size_t)b * n), *u4 = (const float4 *)(u + (size_t)b * n);
    float4 gv[NV], uv[NV];
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int i = min(tid + kWideT * j, n4 - 1);
        gv[j] = g4[i];
        uv[j] = u4[i];
    }
    float4 h[NV];
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int i = tid + kWideT * j, e0 = 4 * i;
        h[j] = make_float4(silu_mul1(gv[j].x, uv[j].x, e0 < nvec), silu_mul1(gv[j].y, uv[j].y, e0 + 1 < nvec),
                           silu_mul1(gv[j].z, uv[j].z, e0 + 2 < nvec), silu_mul1(gv[j].w, uv[j].w, e0 + 3 < nvec));
        if (i >= n4)
            h[j] = f4_zero();
        m = fmaxf(m, f4_absmax(h[j]));
    }
    m = wave_max(m);
    if ((tid & (kWave - 1)) == 0)
        red[tid / kWave] = m;
    __syncthreads();
    float amax = 0.0f;
#pragma unroll
    for (int w = 0; w < kWideT / kWave; w++)
        amax = fmaxf(amax, red[w]);
    const float sc = digit_scale<FP8>(amax);
    const int Kp = (int)xdig_kp(n, FP8);
    if (tid == 0)
        xdig_scales(dig, n, B, FP8)[b] = sc;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int k0 = 4 * (tid + kWideT * j);
        if (k0 < Kp) {
            const float xe[4] = {h[j].x, h[j].y, h[j].z, h[j].w};
            store_digit_words<FP8>(xe, sc, dig, B, Kp, b, k0);
        }
    }
}

// argmax_simd_f32: the maximum value wins; among equal maxima in the
// 8-lane part (indices below 8*floor(n/8), n >= 8) the lowest lane (i % 8),
// then the first index; tail entries win only with a strictly larger value.
// In one pass: (max, smallest key (i % 8, i) among the elements equal to
// it) is an associative pair, so kArgChunks blocks per row reduce their
// chunks of the 8-lane part, and the last block of the row to finish
// (counted with an atomic in cnt[row], which it resets for the next call)
// combines the chunks in order and applies the tail rule.
constexpr int kArgChunks = 64;
struct ArgPart {
    float vm;
    int pad;
    unsigned long long key;
};

__device__ __forceinline__ void arg_merge(float &vm, unsigned long long &key, float v2, unsigned long long k2)
{
    if (v2 > vm || (v2 == vm && k2 < key)) {
        vm = v2;
        key = k2;
    }
}

__global__ __launch_bounds__(256) void k_argmax(int *__restrict__ out, const float *__restrict__ logits, int n,
                                                ArgPart *__restrict__ parts, int *__restrict__ cnt)
{
    __shared__ float rv[4];
    __shared__ unsigned long long rk[4];
    __shared__ int last;
    const int row = blockIdx.y, c = blockIdx.x;
    const float *x = logits + (size_t)row * n;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int main = n < 8 ? 0 : (n & ~7);
    const int cs = ((main + kArgChunks - 1) / kArgChunks + 7) & ~7;
    const int lo = min(c * cs, main), hi = min(lo + cs, main);
    float vm = -INFINITY;
    unsigned long long key = ~0ull;
    for (int i0 = lo; i0 < hi; i0 += 8 * 256) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int i = i0 + j * 256 + threadIdx.x;
            v[j] = i < hi ? x[i] : -INFINITY;
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int i = i0 + j * 256 + threadIdx.x;
            if (i < hi)
                arg_merge(vm, key, v[j], ((unsigned long long)(i & 7) << 32) | (unsigned)i);
        }
    }
    for (int o = 32; o > 0; o >>= 1) {
        const float v2 = __shfl_xor(vm, o);
        const unsigned long long k2 = __shfl_xor(key, o);
        arg_merge(vm, key, v2, k2);
    }
    if (lane == 0) {
        rv[wave] = vm;
        rk[wave] = key;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++)
            arg_merge(vm, key, rv[w], rk[w]);
        parts[(size_t)row * kArgChunks + c] = ArgPart{vm, 0, key};
        __threadfence();
        last = atomicAdd(&cnt[row], 1) == kArgChunks - 1;
    }
    __syncthreads();
    if (!last)
        return;
    __threadfence();
    if (wave == 0) {
        float cv = -INFINITY;
        unsigned long long ck = ~0ull;
        if (lane < kArgChunks) {
            const ArgPart p = parts[(size_t)row * kArgChunks + lane];
            cv = p.vm;
            ck = p.key;
        }
        for (int o = 32; o > 0; o >>= 1) {
            const float v2 = __shfl_xor(cv, o);
            const unsigned long long k2 = __shfl_xor(ck, o);
            arg_merge(cv, ck, v2, k2);
        }
        if (lane == 0) {
            // tail: first index of the largest value; wins only if strictly larger
            float tm = -INFINITY;
            int ti = -1;
            for (int i = main; i < n; i++)
                if (ti < 0 || x[i] > tm) {
                    tm = x[i];
                    ti = i;
                }
            int res;
            if (main == 0 || (ti >= 0 && tm > cv))
                res = ti >= 0 ? ti : 0;
            else
                res = ck == ~0ull ? 0 : (int)(ck & 0xFFFFFFFFu);
            out[row] = res;
            cnt[row] = 0;
        }
    }
}

// RoPE of a prefill chunk in place: token t (position p0 + t), KV head h:
// q heads of h's group and k head h, with the arithmetic of the decode
// step's rotation (k_rope_append_dev): y0 = fma(x0, c, -(x1 s)),
// y1 = fma(x0, s, x1 c); positions at or past rope_len are not rotated.
__global__ __launch_bounds__(256) void k_rope_rows(float *__restrict__ q, float *__restrict__ k,
                                                   const float *__restrict__ cos_t, const float *__restrict__ sin_t,
                                                   int p0, int rope_len, int H, int KV, int hd)
{
    const int t = blockIdx.x, h = blockIdx.y, half = hd / 2, G = H / KV, pos = p0 + t;
    if (pos >= rope_len)
        return;
    for (int i = threadIdx.x; i < (G + 1) * half; i += blockDim.x) {
        const int j = i / half, pr = i % half;
        float *base = j < G ? q + ((size_t)t * H + h * G + j) * hd : k + ((size_t)t * KV + h) * hd;
        const float cs = cos_t[(size_t)pos * half + pr], sn = sin_t[(size_t)pos * half + pr];
        const float x0 = base[pr], x1 = base[pr + half];
        base[pr] = __fmaf_rn(x0, cs, -(x1 * sn));
        base[pr + half] = __fmaf_rn(x0, sn, x1 * cs);
    }
}

// ---- the fused layer of a one-sequence decode step ------------------------------
// At batch 1 every operation of a layer but the attention is a few
// microseconds of dependent memory round trips on a few CUs, and a launch of
// its own costs about as much again.  One launch per layer runs, after the
// layer's attention: the o projection, the residual add and RMSNorm, gate/up
// with SiLU*up, the down projection, then the next layer's residual add,
// RMSNorm, q/k/v and its RoPE + K/V append + seal -- with a grid barrier
// between dependent phases.  Every block is resident (one per CU), keeps its
// own copy of the phase's activation digit planes in LDS (it computes them
// from the fp32 vector itself), and streams its row tiles of the phase's
// weights straight from HBM into MFMA operand registers.  A phase's input
// vector is loaded first; half of the block's weight loads leave while the
// other half of its waves compute the digit planes; the phase's row scales
// and output addresses load with the vector, so that only the cross-wave sum
// and the stores follow the last matrix instruction.  (Weight loads issued
// before a barrier were measured to slow the barrier itself more than they
// gained, and so was a barrier in which every block reads a packed array of
// all the arrival flags.)
//
// Coherence: the activations one block writes and another reads go through
// device-scope (agent) atomic stores and loads, which act at the device's
// coherence point, so the barrier needs no L2 write-back or invalidate: a
// block waits for its own stores (vmcnt), publishes an arrival flag, block 0
// gathers every flag and publishes a release flag.  Flags hold increasing
// barrier numbers (a per-decoder launch counter times kFBars plus the
// barrier index), so graph replays need no reset.  Every wait is bounded: a
// barrier that does not complete within ~kFSpinMax polls sets an error flag
// the host reports, and the launch runs on (its results are then invalid).
//
// Arithmetic: the row kernels' (RMSNorm sums of squares in the same thread
// layout and tree, the same digit split and SiLU), and the GEMV's single
// rounding of exact INT8 digit sums -- so with INT8 weights a fused step
// equals the step of separate launches bit for bit; FP8 digit sums are fp32
// matrix-core accumulations in another order.
constexpr int kFT = 512;                  // threads per block
constexpr int kFW = kFT / kWave;          // waves per block
constexpr int kFMaxU = 12;                // MFMA steps (128 k-bytes) one wave holds in registers
constexpr int kFMaxTiles = 8;             // 16-row tiles of one block in one phase
constexpr int kFDigBytes = 84 * 1024;     // LDS digit planes; also keeps one block per CU
constexpr int kFBars = 8;                 // barrier numbers per launch
constexpr unsigned kFSpinMax = 1u << 16;  // polls (about 1 us each) before a wait gives up

__device__ __forceinline__ float ld_dev(const float *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(float *p, float v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(__attribute__((address_space(1))) float *p, float v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Device-scope (sc1) direct-to-LDS loads of a vector other blocks wrote:
// lane l of wave w moves floats 4 (64 w + l + 256 q) .. + 3 for q = 0, 1, ...
// (threads < kRowT, n floats, n a multiple of 4) into dst at the same float
// index.  The caller waits (vmcnt) before reading dst.
__device__ __forceinline__ void vec_to_lds(const float *src, float *dst, int n)
{
    const int tid = threadIdx.x, wave = tid >> 6;
    if (tid >= kRowT)
        return;
    for (int q = 0; (wave * 64 + q * kRowT) * 4 < n; q++) {
        const int i4 = tid + q * kRowT;
        if (4 * i4 < n)
            __builtin_amdgcn_global_load_lds((const void *)(src + 4 * i4),
                                             (lds_void *)(dst + 4 * (wave * 64 + q * kRowT)), 16, 0, 16);
    }
}

// One projection phase: up to three weight matrices over the same input
// (q/k/v), or gate/up pairs (silu: tile pair p = gate tile p, up tile p, and
// y[0] takes silu(gate) * up).  units: tiles, or pairs.
struct FPhase {
    const uint8_t *w[3];
    const float *sw[3];
    float *y[3];
    int n[3], tend[3];
    int nseg, K, steps, units, silu;
};

// The embedding row of a step's token: codes [vocab][dim] (INT8 or FP8) and
// one scale per row, as k_embed dequantizes them.
struct EmbRow {
    const uint8_t *emb;
    const float *scale;
    const int *tok;   // the token (device memory)
};

struct FusedArgs {
    FPhase o, gu, down, qkv;      // qkv.nseg == 0: the last layer
    const float *att;
    float *X, *Hb, *XB, *H2, *q, *k, *v;
    const uint16_t *ffn_norm, *attn_norm;   // this layer's FFN norm, the next layer's attention norm
    be42_kv_pool P;
    const AppendStepArgs *app;              // the next layer's append
    const float *cos_t, *sin_t;
    const int *pos_p;
    int rope_len, dim, hidden, qd, kd, H, KV;
    float eps;
    unsigned *flags, *gen;
    int *err;
    unsigned spin_max;   // polls before a grid-barrier wait gives up
    unsigned bias;       // added to the numbers waited for (0; a test sets it so no wait completes)
    float *att_out;      // the next layer's dense attention output (null: a launch of its own)
    float att_scale;
    EmbRow er;           // k_fused_layer<..., START>: the step's token, whose embedding is layer 0's input
    int pf_route;        // the next layer's attention routes: warm the L2 with its routing tables
};

struct GridBar {
    unsigned *flags;
    unsigned base;
    int nb;
    int *err;
    unsigned spin_max, bias;
};

__device__ __forceinline__ bool flag_before(unsigned v, unsigned target) { return (int)(v - target) < 0; }

// Arrive, run `during` (loads of the next phase's weights), then wait for
// every block.  After a timed-out wait (error flag set) later barriers do not
// wait again; whether to wait is decided once per block.
template <class F>
__device__ __forceinline__ void grid_barrier(const GridBar &gb, unsigned idx, F &&during)
{
    __shared__ int failed;
    const unsigned target = gb.base + idx, awaited = target + gb.bias;
    wait_vmcnt<0>();              // this thread's stores have completed
    __syncthreads();
    // arrive, then read the error word (its round trip overlaps the wait)
    if (threadIdx.x == 0) {
        __hip_atomic_store(gb.flags + blockIdx.x * 32, target, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        failed = __hip_atomic_load(gb.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
    }
    during();
    __syncthreads();
    const bool skip = failed;
    if (blockIdx.x == 0 && !skip) {
        for (int i = threadIdx.x; i < gb.nb; i += blockDim.x) {
            unsigned spins = 0;
            while (flag_before(__hip_atomic_load(gb.flags + i * 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                               awaited))
                if (++spins > gb.spin_max) {
                    atomicExch(gb.err, 1);
                    break;
                }
        }
        __syncthreads();
        if (threadIdx.x == 0)
            __hip_atomic_store(gb.flags + gb.nb * 32, target, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (threadIdx.x == 0 && !skip) {
        unsigned spins = 0;
        while (flag_before(__hip_atomic_load(gb.flags + gb.nb * 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                           awaited))
            if (++spins > gb.spin_max) {
                atomicExch(gb.err, 2);
                break;
            }
    }
    __syncthreads();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

__device__ __forceinline__ int ph_count(const FPhase &ph, int b, int nb)
{
    const int c = ph.units > b ? (ph.units - 1 - b) / nb + 1 : 0;
    return ph.silu ? 2 * c : c;
}

// tile slot j of block b -> (segment, tile within the segment)
__device__ __forceinline__ void ph_slot(const FPhase &ph, int b, int nb, int j, int &seg, int &lt)
{
    if (ph.silu) {
        seg = j & 1;
        lt = b + (j >> 1) * nb;
        return;
    }
    const int T = b + j * nb;
    seg = (int)(ph.nseg > 1 && T >= ph.tend[0]) + (int)(ph.nseg > 2 && T >= ph.tend[1]);
    lt = T - (seg == 0 ? 0 : (seg == 1 ? ph.tend[0] : ph.tend[1]));
}

template <class T>
__device__ __forceinline__ T seg_sel(const T (&a)[3], int seg)
{
    return seg == 0 ? a[0] : (seg == 1 ? a[1] : a[2]);
}

// seg_sel for a per-lane seg: the three entries are first made scalars, so
// that the choice is a per-lane select and not an indexed (vector) load
// from the kernel arguments, which the next dependent load would wait for.
// Pointers come back as global-memory pointers (a generic one would make
// its loads and stores flat accesses, which LDS waits also count).
template <class T>
using gptr = __attribute__((address_space(1))) T *;
__device__ __forceinline__ int sgpr(int v) { return __builtin_amdgcn_readfirstlane(v); }
template <class T>
__device__ __forceinline__ gptr<T> sgpr(T *p)
{
    const uint64_t u = (uint64_t)(uintptr_t)p;
    return (gptr<T>)(((uint64_t)(uint32_t)sgpr((int)(uint32_t)(u >> 32)) << 32) | (uint32_t)sgpr((int)(uint32_t)u));
}
__device__ __forceinline__ int seg_sel_lane(const int (&a)[3], int seg)
{
    const int a0 = sgpr(a[0]), a1 = sgpr(a[1]), a2 = sgpr(a[2]);
    return seg == 0 ? a0 : (seg == 1 ? a1 : a2);
}
template <class T>
__device__ __forceinline__ gptr<T> seg_sel_lane(T *const (&a)[3], int seg)
{
    const gptr<T> a0 = sgpr(a[0]), a1 = sgpr(a[1]), a2 = sgpr(a[2]);
    return seg == 0 ? a0 : (seg == 1 ? a1 : a2);
}

// wave -> (tile slot, step range): the tiles rounded up to a power of two
// share the 8 waves, each tile's waves splitting its K steps
struct FWave {
    int j, s0, s1, wpt;
    bool on;
};
__device__ __forceinline__ FWave ph_wave(int nt, int steps, int wave)
{
    const int np = nt <= 1 ? 1 : (nt <= 2 ? 2 : (nt <= 4 ? 4 : 8));
    FWave w;
    w.wpt = kFW / np;
    w.j = wave / w.wpt;
    const int gw = wave % w.wpt;
    w.on = w.j < nt;
    w.s0 = gw * steps / w.wpt;
    w.s1 = (gw + 1) * steps / w.wpt;
    return w;
}

// this wave's weight fragments of the phase (waves lo .. hi-1 only): lane
// (r, g) holds row r of its tile, k bytes 128 s + 16 g .. + 15 and
// 128 s + 64 + 16 g .. + 15 of each of its steps s (so each load instruction
// reads 64 contiguous bytes of each of 16 rows; the digit fragments use the
// same k positions)
__device__ __forceinline__ void ph_prefetch(const FPhase &ph, int b, int nb, v8i (&fr)[kFMaxU], int lo, int hi)
{
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    if (wave < lo || wave >= hi)
        return;
    const FWave fw = ph_wave(ph_count(ph, b, nb), ph.steps, wave);
    if (!fw.on)
        return;
    int seg, lt;
    ph_slot(ph, b, nb, fw.j, seg, lt);
    const int row = min(lt * 16 + r, seg_sel(ph.n, seg) - 1);
    const uint8_t *wr = seg_sel(ph.w, seg) + (size_t)row * ph.K + 16 * g;
#pragma unroll
    for (int u = 0; u < kFMaxU; u++) {
        const int s = fw.s0 + u;
        if (s < fw.s1) {
            const v4i lo = *(const v4i *)(wr + (size_t)s * 128), hi = *(const v4i *)(wr + (size_t)s * 128 + 64);
            fr[u] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
    }
}

// What thread i (< 16 x the block's tiles) of a phase needs after the
// matrix instructions: its row's weight scale and where its output goes
// (for gate/up: the scale of its gate or up row, and the output of pair
// i / 16).  Loaded when the phase starts, so that these dependent loads
// overlap the input vector's instead of following the last MFMA.
struct FOut {
    gptr<float> y;   // output element, nullptr if none
    float sw;     // row scale (0 past the rows)
    int ok;       // the row exists
    int tail;     // gate/up: the pair's row is past the last multiple of 8
};
__device__ __forceinline__ FOut ph_out(const FPhase &ph, int b, int nb)
{
    FOut o{nullptr, 0.0f, 0, 0};
    const int nt = ph_count(ph, b, nb), i = threadIdx.x;
    if (i < nt * 16) {
        const int j = i >> 4, r = i & 15;
        int seg, lt;
        ph_slot(ph, b, nb, j, seg, lt);
        const int row = lt * 16 + r;
        if (row < seg_sel_lane(ph.n, seg)) {
            o.ok = 1;
            o.sw = seg_sel_lane(ph.sw, seg)[row];
            if (!ph.silu)
                o.y = seg_sel_lane(ph.y, seg) + row;
        }
    }
    if (ph.silu && i < (nt / 2) * 16) {
        int seg, lt;
        ph_slot(ph, b, nb, 2 * (i >> 4), seg, lt);
        const int row = lt * 16 + (i & 15);
        const int n0 = sgpr(ph.n[0]);
        if (row < n0) {
            o.y = sgpr(ph.y[0]) + row;
            o.tail = row >= (n0 & ~7);
        }
    }
    return o;
}

// The phase's MFMAs against the digit planes in LDS (dig[d][Kp]), the
// cross-wave sum of each tile's partials, and the outputs (device-scope
// stores).  sx: the digit scale of the input; oo: ph_out of this thread.
template <bool FP8>
__device__ __forceinline__ void ph_compute(const FPhase &ph, int b, int nb, const v8i (&fr)[kFMaxU],
                                           const uint8_t *dig, int Kp, float sx, long long (*part)[16], float *ybuf,
                                           const FOut &oo)
{
    constexpr int ND = FP8 ? kF8Digits : kI8Digits;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, c = lane & 15, g = lane >> 4;
    const int nt = ph_count(ph, b, nb);
    const FWave fw = ph_wave(nt, ph.steps, wave);
    using Acc = typename std::conditional<FP8, v4f, v4i>::type;
    Acc acc = Acc{0, 0, 0, 0};
    if (fw.on) {
#pragma unroll
        for (int u = 0; u < kFMaxU; u++) {
            const int s = fw.s0 + u;
            if (s < fw.s1) {
                v8i bf = v8i{0, 0, 0, 0, 0, 0, 0, 0};
                if (c < ND) {
                    const uint8_t *dp = dig + (size_t)c * Kp + (size_t)s * 128 + 16 * g;
                    const v4i lo = *(const v4i *)dp, hi = *(const v4i *)(dp + 64);
                    bf = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                }
                if constexpr (FP8) {
                    acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(fr[u], bf, acc, 0, 0, 0, 127, 0, 127);
                } else {
                    const v4i alo = {fr[u][0], fr[u][1], fr[u][2], fr[u][3]}, ahi = {fr[u][4], fr[u][5], fr[u][6], fr[u][7]};
                    const v4i blo = {bf[0], bf[1], bf[2], bf[3]}, bhi = {bf[4], bf[5], bf[6], bf[7]};
                    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo, blo, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi, bhi, acc, 0, 0, 0);
                }
            }
        }
    }
    // lane l holds rows 4 (l / 16) + e of digit column l % 16: combine the
    // digit columns of each row (exact int64 / fp64) into part[wave][row]
#pragma unroll
    for (int e = 0; e < 4; e++) {
        if constexpr (FP8) {
            double t = 0.0;
#pragma unroll
            for (int d = 0; d < ND; d++)
                t += (double)__shfl(acc[e], (lane & 48) + d, kWave) * kF8DigitW[d];
            if (c == 0)
                part[wave][4 * g + e] = __double_as_longlong(t);
        } else {
            long long t = 0;
#pragma unroll
            for (int d = 0; d < ND; d++)
                t += (long long)__shfl(acc[e], (lane & 48) + d, kWave) *
                     (d == 0 ? (long long)kI8Base * kI8Base : (d == 1 ? (long long)kI8Base : 1ll));
            if (c == 0)
                part[wave][4 * g + e] = t;
        }
    }
    __syncthreads();
    const double sxw = FP8 ? 1.0 : 1.0 / (double)(kI8Base * kI8Base);
    const int i = threadIdx.x;
    if (i < nt * 16) {
        const int j = i >> 4, r = i & 15;
        const int w0 = j * fw.wpt;   // the tile's waves (wpt is the same for every wave)
        double tot;
        if constexpr (FP8) {
            tot = 0.0;
            for (int w = 0; w < fw.wpt; w++)
                tot += __longlong_as_double(part[w0 + w][r]);
        } else {
            long long it = 0;
            for (int w = 0; w < fw.wpt; w++)
                it += part[w0 + w][r];
            tot = (double)it;
        }
        const float y = oo.ok ? (float)(tot * ((double)sx * sxw * (double)oo.sw)) : 0.0f;
        if (ph.silu)
            ybuf[i] = y;
        else if (oo.y)
            st_dev(oo.y, y);
    }
    if (ph.silu) {
        __syncthreads();
        if (oo.y) {
            const int p = i >> 4, r = i & 15;
            st_dev(oo.y, silu_mul1(ybuf[2 * p * 16 + r], ybuf[(2 * p + 1) * 16 + r], !oo.tail));
        }
    }
}

// fp32 staging of a phase's input vector in LDS, after its digit planes
__device__ __forceinline__ float *dig_stage(uint8_t *dig, int nd, int K)
{
    return (float *)(dig + (((size_t)nd * K + 15) & ~(size_t)15));
}

// Waves 0-3 of a block wait for each other through an LDS counter (waves
// 4-7 take no part: they may be stalled issuing weight loads, and a block
// barrier would hold waves 0-3 behind them).  Every call adds 4 to the
// target; the wait is bounded like the grid barrier's.
struct QuadSync {
    int *cnt;     // LDS, 0 at kernel start
    int target;
    int *err;     // the launch's error flag
};
__device__ __forceinline__ void quad_sync(QuadSync &q)
{
    q.target += 4;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if ((threadIdx.x & 63) == 0)
        __hip_atomic_fetch_add(q.cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    unsigned spins = 0;
    while (__hip_atomic_load(q.cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < q.target) {
        __builtin_amdgcn_s_sleep(1);
        if (++spins > kFSpinMax * 16) {
            if ((threadIdx.x & 63) == 0)
                atomicExch(q.err, 3);
            break;
        }
    }
    asm volatile("" ::: "memory");
}

// max over waves 0-3 of a per-lane value (red: 4 floats of LDS)
__device__ __forceinline__ float quad_max(float v, float *red, QuadSync &q)
{
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = v;
    quad_sync(q);
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// Digit planes of a vector written by other blocks (K a multiple of 128,
// at most kRowT * 4 * kFVecG).  Waves 0-3 stage it in LDS with device-scope
// loads; once those have left, waves 4-7 issue their weight loads of the
// phase (`mid`) while waves 0-3 wait for the vector, compute the scale and
// the digit planes, and only then issue theirs.  Returns the scale (in every
// thread).
constexpr int kFVecG = 8;
template <bool FP8, class Mid>
__device__ __forceinline__ float vec_digits(const float *x, int K, uint8_t *dig, float *red, QuadSync &q, Mid &&mid)
{
    constexpr int ND = FP8 ? kF8Digits : kI8Digits;
    const int tid = threadIdx.x;
    float *stage = dig_stage(dig, ND, K);
    vec_to_lds(x, stage, K);
    asm volatile("" ::: "memory");
    __syncthreads();              // the vector's loads leave before any weight load of the block
    if (tid >= kRowT) {
        mid();
    } else {
        wait_vmcnt<0>();
        quad_sync(q);
        float m = 0.0f;
#pragma unroll
        for (int g = 0; g < kFVecG; g++) {
            const int i4 = tid + g * kRowT;
            if (4 * i4 < K)
                m = fmaxf(m, f4_absmax(*(const float4 *)(stage + 4 * i4)));
        }
        const float sc = digit_scale<FP8>(quad_max(m, red + 8, q));
#pragma unroll
        for (int g = 0; g < kFVecG; g++) {
            const int i4 = tid + g * kRowT;
            if (4 * i4 < K) {
                const float4 x4 = *(const float4 *)(stage + 4 * i4);
                const float xe[4] = {x4.x, x4.y, x4.z, x4.w};
                uint32_t word[ND];
                digit_words<FP8>(xe, sc, word);
#pragma unroll
                for (int d = 0; d < ND; d++)
                    *(uint32_t *)(dig + (size_t)d * K + 4 * i4) = word[d];
            }
        }
        if (tid == 0)
            red[12] = sc;
        asm volatile("" ::: "memory");
        mid();
    }
    __syncthreads();
    return red[12];
}

// x + delta (both written by other blocks), RMSNorm with w, into digit
// planes, with the work split as in vec_digits; block b writes its share of
// x + delta to x_out.  Threads < kRowT (waves 0-3) hold the row exactly as
// k_rmsnorm's threads do (same sum of squares, same reduction tree).  EMB:
// the row is instead the embedding of er's token, formed as k_embed forms it
// (x and delta unused).
template <bool FP8, int NV, bool EMB = false, class Mid>
__device__ __forceinline__ float norm_digits(const float *x, const float *delta, const uint16_t *w, float *x_out,
                                             int dim, float eps, uint8_t *dig, float *red, int b, int nb,
                                             QuadSync &q, Mid &&mid, const EmbRow &er = EmbRow{})
{
    constexpr int ND = FP8 ? kF8Digits : kI8Digits;
    const int tid = threadIdx.x, n4 = dim >> 2;
    float *sx_ = dig_stage(dig, ND, dim), *sd_ = sx_ + dim;
    if constexpr (!EMB) {
        vec_to_lds(x, sx_, dim);
        vec_to_lds(delta, sd_, dim);
    }
    asm volatile("" ::: "memory");
    __syncthreads();              // the vectors' loads leave before any weight load of the block
    if (tid >= kRowT) {
        mid();
    } else {
        float4 v[NV], h[NV];
        uint2 wv[NV];
        if constexpr (EMB) {
            const int tok = *er.tok;
            const float es = er.scale[tok];
            const uint8_t *row = er.emb + (size_t)tok * dim;
            auto dq = [](uint32_t c) { return FP8 ? fp8_to_f32((uint8_t)c) : (float)(int8_t)(uint8_t)c; };
#pragma unroll
            for (int j = 0; j < NV; j++) {
                const int i = min(tid + kRowT * j, n4 - 1);
                const uint32_t c4 = *(const uint32_t *)(row + 4 * i);
                v[j] = make_float4(dq(c4 & 0xFFu) * es, dq((c4 >> 8) & 0xFFu) * es, dq((c4 >> 16) & 0xFFu) * es,
                                   dq(c4 >> 24) * es);
                wv[j] = ((const uint2 *)w)[i];
            }
        } else {
            wait_vmcnt<0>();
            quad_sync(q);
#pragma unroll
            for (int j = 0; j < NV; j++) {
                const int i = min(tid + kRowT * j, n4 - 1);
                const float4 xv = *(const float4 *)(sx_ + 4 * i), dv = *(const float4 *)(sd_ + 4 * i);
                v[j] = make_float4(xv.x + dv.x, xv.y + dv.y, xv.z + dv.z, xv.w + dv.w);
                wv[j] = ((const uint2 *)w)[i];
            }
        }
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < NV; j++) {
            const int i = tid + kRowT * j;
            if (i < n4 && i % nb == b) {
                float *o = x_out + 4 * i;
                st_dev(o, v[j].x);
                st_dev(o + 1, v[j].y);
                st_dev(o + 2, v[j].z);
                st_dev(o + 3, v[j].w);
            }
            if (i >= n4)
                v[j] = f4_zero();
            ss = __fmaf_rn(v[j].x, v[j].x, ss);
            ss = __fmaf_rn(v[j].y, v[j].y, ss);
            ss = __fmaf_rn(v[j].z, v[j].z, ss);
            ss = __fmaf_rn(v[j].w, v[j].w, ss);
        }
        ss = wave_sum_dpp(ss);
        if ((tid & 63) == 0)
            red[tid >> 6] = ss;
        quad_sync(q);
        const float tot = (red[0] + red[1]) + (red[2] + red[3]);
        const float inv = __fdiv_rn(1.0f, sqrtf(__fdiv_rn(tot, (float)dim) + eps));
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < NV; j++) {
            const uint2 wj = wv[j];
            h[j] = make_float4((v[j].x * inv) * bf16_to_f32((uint16_t)(wj.x & 0xFFFF)),
                               (v[j].y * inv) * bf16_to_f32((uint16_t)(wj.x >> 16)),
                               (v[j].z * inv) * bf16_to_f32((uint16_t)(wj.y & 0xFFFF)),
                               (v[j].w * inv) * bf16_to_f32((uint16_t)(wj.y >> 16)));
            if (tid + kRowT * j >= n4)
                h[j] = f4_zero();
            m = fmaxf(m, f4_absmax(h[j]));
        }
        const float sc = digit_scale<FP8>(quad_max(m, red + 8, q));
#pragma unroll
        for (int j = 0; j < NV; j++) {
            const int i = tid + kRowT * j;
            if (i < n4) {
                const float xe[4] = {h[j].x, h[j].y, h[j].z, h[j].w};
                uint32_t word[ND];
                digit_words<FP8>(xe, sc, word);
#pragma unroll
                for (int d = 0; d < ND; d++)
                    *(uint32_t *)(dig + (size_t)d * dim + 4 * i) = word[d];
            }
        }
        if (tid == 0)
            red[12] = sc;
        asm volatile("" ::: "memory");
        mid();
    }
    __syncthreads();
    return red[12];
}

// The next layer's dense attention for KV head kvh, after this block's K/V
// append (blocks 0 .. KV-1 of the tail): what a one-query k_attn_fused launch
// at 16 waves computes over the sequence's pages, from this block's 8 waves
// (the scores and weights of every token as there, the values summed in the
// 16-wave layout: attn_values_layout), so the step's output is the same bit
// for bit.  The page list is the one the append leaves -- the slot's table
// before it, the appended token's page at its logical position, holding
// position + 1 tokens -- formed here from the append's arguments, since block
// 0 publishes the table and token count and other blocks do not wait for it.
// qs: the G rotated query rows of the group (LDS); lds: free LDS for the
// phases' shared state and the 16 partial outputs.
constexpr int kTailAttnOff = 4096;   // bytes of the tail's scratch before the attention state
template <bool BF16KV, int HD, int G>
__device__ __forceinline__ void tail_attention(const FusedArgs &A, int kvh, const float *qs, uint8_t *lds)
{
    using SH = AttnShared<HD, G, kFW>;
    constexpr size_t kRedOff = (sizeof(SH) + 15) & ~(size_t)15;
    static_assert(kTailAttnOff + kRedOff + 16 * G * HD * 4 <= kFDigBytes, "tail attention LDS");
    static_assert((G + 3) * HD * 4 <= kTailAttnOff, "tail scratch");
    SH &S = *reinterpret_cast<SH *>(lds);
    S.red = reinterpret_cast<float *>(lds + kRedOff);
    const be42_kv_pool &P = A.P;
    const AppendStepArgs &a = *A.app;
    const int off = a.pos[0] % kPg, blk = a.pos[0] / kPg, phys = a.phys[0], slot = a.slot[0];
    const int ns = min(blk + 1, kFusedMaxPages);
    for (int i = threadIdx.x; i < G * HD; i += blockDim.x)
        S.qs[i / HD][i % HD] = qs[i];
    for (int i = threadIdx.x; i < ns; i += blockDim.x) {
        const int ph = i == blk ? phys : P.page_table[(size_t)slot * a.max_logical + i];
        S.pphys[i] = ph;
        S.pnt[i] = ph == phys ? off + 1 : P.ntok[ph];
    }
    __syncthreads();
    attn_scores<BF16KV, HD, G, kFW, 8>(P, S, kvh, ns, A.att_scale, 0, kFW);
    __syncthreads();
    attn_weights(S, ns, nullptr);
    __syncthreads();
    attn_values_layout<BF16KV, HD, G, kFW, 16, 8>(P, S, 0, kvh, ns, A.H, A.att_out, nullptr);
}

template <bool FP8, bool BF16KV, int NV, bool START>
__global__ __launch_bounds__(kFT, 1) void k_fused_layer(const FusedArgs A)
{
    __shared__ __align__(16) uint8_t dig[kFDigBytes];
    __shared__ long long part[kFW][16];
    __shared__ float ybuf[kFMaxTiles * 16];
    __shared__ float red[16];
    __shared__ int qcnt;
    const int b = blockIdx.x, nb = gridDim.x;
    if (threadIdx.x == 0)
        qcnt = 0;
    __syncthreads();
    QuadSync quad{&qcnt, 0, A.err};
    GridBar gb{A.flags, __hip_atomic_load(A.gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) * kFBars, nb, A.err,
               A.spin_max, A.bias};
    v8i fr[kFMaxU];
#pragma unroll
    for (int u = 0; u < kFMaxU; u++)
        fr[u] = v8i{0, 0, 0, 0, 0, 0, 0, 0};
    // A phase's input vector is loaded first (waves 0-3); then waves 4-7
    // issue their weight loads of the phase while waves 0-3 compute the
    // digit planes, and waves 0-3 issue theirs after (a vector load queued
    // behind the phase's weight stream would hold up the digits).
    auto wload = [&](const FPhase &ph) {
        const FPhase *pp = &ph;
        return [pp, b, nb, &fr] { ph_prefetch(*pp, b, nb, fr, 0, kFW); };
    };
    FOut oo;
    float sx;
    if constexpr (!START) {
        // o projection of the attention output
        oo = ph_out(A.o, b, nb);
        sx = vec_digits<FP8>(A.att, A.qd, dig, red, quad, wload(A.o));
        ph_compute<FP8>(A.o, b, nb, fr, dig, A.qd, sx, part, ybuf, oo);
        grid_barrier(gb, 1, [] {});
        // h = x + o, RMSNorm, gate/up, SiLU * up
        oo = ph_out(A.gu, b, nb);
        sx = norm_digits<FP8, NV>(A.X, A.XB, A.ffn_norm, A.Hb, A.dim, A.eps, dig, red, b, nb, quad, wload(A.gu));
        ph_compute<FP8>(A.gu, b, nb, fr, dig, A.dim, sx, part, ybuf, oo);
        grid_barrier(gb, 2, [] {});
        // down projection
        oo = ph_out(A.down, b, nb);
        sx = vec_digits<FP8>(A.H2, A.hidden, dig, red, quad, wload(A.down));
        ph_compute<FP8>(A.down, b, nb, fr, dig, A.hidden, sx, part, ybuf, oo);
        if (A.qkv.nseg == 0) {
            // last layer: h and the down output stay for the final norm
            if (b == 0 && threadIdx.x == 0)
                __hip_atomic_store(A.gen, gb.base / kFBars + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
        grid_barrier(gb, 3, [] {});
    }
    // next layer: x = h + down (the step's first launch: x = the token's
    // embedding), RMSNorm, q/k/v
    oo = ph_out(A.qkv, b, nb);
    if constexpr (START)
        sx = norm_digits<FP8, NV, true>(nullptr, nullptr, A.attn_norm, A.X, A.dim, A.eps, dig, red, b, nb, quad,
                                        wload(A.qkv), A.er);
    else
        sx = norm_digits<FP8, NV>(A.Hb, A.XB, A.attn_norm, A.X, A.dim, A.eps, dig, red, b, nb, quad, wload(A.qkv));
    ph_compute<FP8>(A.qkv, b, nb, fr, dig, A.dim, sx, part, ybuf, oo);
    grid_barrier(gb, 4, [] {});
    if (b == 0 && threadIdx.x == 0)
        __hip_atomic_store(A.gen, gb.base / kFBars + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (b >= A.KV) {
        if (A.pf_route && b < A.KV + 8 && threadIdx.x < kWave) {
            // Blocks KV .. KV + 7 (one per XCD; they have no tail): the next
            // layer's routing tables (its page hashes and page-table row, the
            // projection) into their XCD's L2, one word per 128-byte line into
            // an LDS word nobody reads, so that the router's first loads hit L2.
            const AppendStepArgs &ap = *A.app;
            const size_t base = (size_t)ap.slot[0] * ap.max_logical;
            const int hd = A.P.head_dim, n = ap.pos[0] / kPg + 1;
            const int lh = (n + 63) / 64, lt = (n + 31) / 32, lp = (hd * 16 + 31) / 32;
            for (int li = threadIdx.x; li < lh + lt + lp; li += kWave) {
                const void *src = li < lh        ? (const void *)(A.P.page_hash + base + min(li * 64, n - 1))
                                  : li < lh + lt ? (const void *)(A.P.page_table + base + min((li - lh) * 32, n - 1))
                                                 : (const void *)(A.P.hpT + min((li - lh - lt) * 32, hd * 16 - 1));
                __builtin_amdgcn_global_load_lds(src, (lds_void *)(dig + kFDigBytes - 256), 4, 0, 0);
            }
            wait_vmcnt<0>();   // the LDS writes land before the workgroup ends
        }
        return;
    }
    // RoPE of the q heads of KV head b and of k head b, K/V append and seal
    const int hd = A.P.head_dim, half = hd / 2, G = A.H / A.KV, tid = threadIdx.x;
    float *qs = (float *)dig, *ks = qs + G * hd, *vs = ks + hd, *cs = vs + hd;
    float *qrow = A.q + (size_t)b * G * hd, *krow = A.k + (size_t)b * hd;
    for (int i = tid; i < G * hd; i += kFT)
        qs[i] = ld_dev(qrow + i);
    for (int i = tid; i < hd; i += kFT) {
        ks[i] = ld_dev(krow + i);
        vs[i] = ld_dev(A.v + (size_t)b * hd + i);
    }
    __syncthreads();
    const int pos = *A.pos_p;
    if (pos < A.rope_len) {
        for (int i = tid; i < (G + 1) * half; i += kFT) {
            const int j = i / half, pr = i % half;
            float *base = j < G ? qs + j * hd : ks;
            const float c = A.cos_t[(size_t)pos * half + pr], sn = A.sin_t[(size_t)pos * half + pr];
            const float x0 = base[pr], x1 = base[pr + half];
            base[pr] = __fmaf_rn(x0, c, -(x1 * sn));
            base[pr + half] = __fmaf_rn(x0, sn, x1 * c);
        }
    }
    __syncthreads();
    // the rotated rows for the attention launch that follows (and captures)
    for (int i = tid; i < G * hd; i += kFT)
        qrow[i] = qs[i];
    for (int i = tid; i < hd; i += kFT)
        krow[i] = ks[i];
    if (A.app->n > 0)
        append_seal_tail<BF16KV>(A.P, *A.app, 0, b, ks, vs, cs);
    if (A.att_out) {
        wait_vmcnt<0>();   // this block's K/V row is in memory
        __syncthreads();
        if (hd == 128 && G == 3)
            tail_attention<BF16KV, 128, 3>(A, b, qs, dig + kTailAttnOff);
        else
            tail_attention<BF16KV, 64, 1>(A, b, qs, dig + kTailAttnOff);
    }
}

// Tokens of one prefill pass (positions p0 .. p0 + T - 1 of one sequence).
constexpr int kPrefillChunk = 1024;

}  // namespace be42

using namespace be42;

struct be42_decoder {
    be42_decoder_config c;
    std::vector<be42_decoder_layer> layers;
    be42_decoder_weights w;
    be42_kv_pool *pool = nullptr;
    float *cos_t = nullptr, *sin_t = nullptr;
    // activations [max_batch][...]
    float *x = nullptr, *xb = nullptr, *xn = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *att = nullptr, *hb = nullptr,
          *hb2 = nullptr, *logits = nullptr;
    void *xdig = nullptr;
    size_t xdig_bytes = 0;
    int *sel = nullptr, *nsel = nullptr, *slots = nullptr, *next = nullptr;
    ArgPart *arg_parts = nullptr;   // [max_batch][kArgChunks] argmax partials
    int *arg_cnt = nullptr;         // [max_batch] chunk counters, zero between calls
    void *attn_ws = nullptr;
    size_t attn_ws_bytes = 0;
    int *cand = nullptr, *ncand = nullptr;
    float *capture_q = nullptr;   // optional [n_layers][max_batch][n_heads * head_dim]
    float *capture_k = nullptr, *capture_v = nullptr;   // optional [n_layers][max_batch][n_kv * head_dim]
    int *capture_sel = nullptr;   // optional [n_layers][max_batch][sel stride]: routed selections
    int *capture_nsel = nullptr;  // optional [n_layers][max_batch] pages attended
    // step parameters: StepHead then AppendStepArgs[n_layers], two pinned host
    // copies (steps alternate, so the host never rewrites a buffer a queued
    // step still has to read) and their device copies
    size_t params_bytes = 0;
    void *params_host[2] = {nullptr, nullptr}, *params_dev[2] = {nullptr, nullptr};
    hipEvent_t params_free[2] = {nullptr, nullptr};
    int parity = 0;
    int *next_host = nullptr;     // pinned copy of d->next: the argmax [kMaxBatch], then the error word
    hipStream_t gstream = nullptr;
    hipEvent_t ev_in = nullptr, ev_out = nullptr;
    struct Key {
        int batch = -1, sparse = -1, dev_tokens = -1;
        const float *logits = nullptr;
        const float *cq = nullptr, *ck = nullptr, *cv = nullptr;
        const int *cn = nullptr, *cs = nullptr;
        bool operator==(const Key &o) const
        {
            return batch == o.batch && sparse == o.sparse && dev_tokens == o.dev_tokens && logits == o.logits &&
                   cq == o.cq && ck == o.ck && cv == o.cv && cn == o.cn && cs == o.cs;
        }
    } key[2];
    hipGraphExec_t exec[2] = {nullptr, nullptr};
    bool use_graph = true;
    // the fused layer of one-sequence steps: grid = the CU count; barrier
    // flags [(nb + 1) * 32], launch counter, error flag (device, zeroed at create)
    bool fused = false;
    bool fail_barriers = false;   // test: every grid-barrier wait gives up
    int fnb = 0;
    unsigned *fflags = nullptr;
    // a fused launch's error flag seen set: the decoder's state is invalid and
    // every later step or prefill is refused (the device flag stays set)
    int fault = 0;
    // prefill activations [kPrefillChunk][...], digit planes, and the chunk's
    // metadata (tokens [T], visible lengths [T], slots [n_layers][T]) with
    // its pinned host copy; allocated by the first prefill
    float *px = nullptr, *pxn = nullptr, *pq = nullptr, *pk = nullptr, *pv = nullptr, *patt = nullptr,
          *pxb = nullptr, *phb = nullptr, *phb2 = nullptr;
    void *pdig = nullptr;
    int *pmeta = nullptr, *pmeta_host = nullptr;
    size_t pmeta_bytes = 0;
    // the chunk's page selections [kPrefillChunk][psel_stride] and counts
    int *psel = nullptr, *pnsel = nullptr;
    int psel_stride = 0;
};

// Whether the fused layer kernel serves this shape at batch 1 (sets d->fnb).
static bool fused_layer_fits(const be42_decoder_config &c, be42_decoder *d)
{
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        return false;
    const int qd = c.n_heads * c.head_dim, kd = c.n_kv_heads * c.head_dim, nd = c.wkind ? kF8Digits : kI8Digits;
    if (c.dim % 128 || c.hidden_dim % 128 || qd % 128 || kd % 16 || c.dim > 4096 ||
        c.hidden_dim > kRowT * 4 * kFVecG || qd > kRowT * 4 * kFVecG ||
        (size_t)(nd + 4) * std::max(c.hidden_dim, qd) + 16 > (size_t)kFDigBytes ||
        (size_t)(nd + 8) * c.dim + 16 > (size_t)kFDigBytes ||
        (size_t)(c.n_heads / c.n_kv_heads + 2) * c.head_dim * 4 + 1024 > (size_t)kFDigBytes || c.n_kv_heads > cus)
        return false;
    // one block per CU, but no more blocks than the largest phase has row
    // tiles (or gate/up tile pairs): a small model's barriers then gather
    // fewer blocks
    const int units_max = std::max(std::max((c.dim + 15) / 16, (c.hidden_dim + 15) / 16),
                                   (qd + 2 * kd + 15) / 16 + 2);
    const int nb = std::max(std::min(cus, units_max), c.n_kv_heads);
    // every block's tiles (rounded up to a power of two) share its 8 waves,
    // and a wave's K steps must fit its registers
    auto ok = [&](int units, bool pairs, int K) {
        const int cnt = (units + nb - 1) / nb * (pairs ? 2 : 1);
        if (cnt > kFMaxTiles)
            return false;
        const int np = cnt <= 1 ? 1 : (cnt <= 2 ? 2 : (cnt <= 4 ? 4 : 8));
        const int wpt = kFW / np, steps = K / 128;
        return (steps + wpt - 1) / wpt <= kFMaxU;
    };
    if (!ok((c.dim + 15) / 16, false, qd) || !ok((c.hidden_dim + 15) / 16, true, c.dim) ||
        !ok((c.dim + 15) / 16, false, c.hidden_dim) || !ok((qd + 2 * kd + 15) / 16 + 2, false, c.dim))
        return false;
    d->fnb = nb;
    return true;
}

static int dec_fail(be42_decoder *d, int rc)
{
    be42_decoder_destroy(d);
    return rc;
}

extern "C" int be42_decoder_create(be42_decoder **out, const be42_decoder_config *cfg,
                                   const be42_decoder_weights *w, const float *hpT_host)
{
    BE42_CHECK(out && cfg && w && w->layers, "be42_decoder_create: null pointer");
    *out = nullptr;
    const be42_decoder_config &c = *cfg;
    BE42_CHECK(c.n_layers > 0 && c.dim > 0 && c.n_heads > 0 && c.n_kv_heads > 0 && c.n_heads % c.n_kv_heads == 0 &&
                   c.head_dim > 0 && c.head_dim % 8 == 0 && c.hidden_dim > 0 && c.vocab > 0 && c.max_seq > 0 &&
                   c.max_batch > 0 && c.max_batch <= 16 && c.dim % 16 == 0 && c.hidden_dim % 16 == 0 && c.dim <= kRowMax && c.hidden_dim <= kRowMax &&
                   c.hidden_dim <= 40960 && c.dim <= 40960 &&
                   (c.n_heads * c.head_dim) % 16 == 0,
               "be42_decoder_create: unsupported shape");
    BE42_CHECK(c.wkind == 0 || c.wkind == 1, "be42_decoder_create: weight kind %d", c.wkind);
    be42_decoder *d = new be42_decoder();
    d->c = c;
    d->layers.assign(w->layers, w->layers + c.n_layers);
    d->w = *w;
    d->w.layers = d->layers.data();
    const int pages = (c.max_seq + 15) / 16;
    int rc = be42_kv_create(&d->pool, c.kv_kind, c.n_layers * c.max_batch, c.n_kv_heads, c.head_dim, pages,
                            hpT_host);
    if (rc)
        return dec_fail(d, rc);
    // RoPE tables from the host's libm, as rope_cache_init builds them
    const int half = c.head_dim / 2;
    const int rope_len = c.rope_len > 0 ? c.rope_len : c.max_seq;
    std::vector<float> ct((size_t)rope_len * half), st((size_t)rope_len * half), inv(half);
    for (int i = 0; i < half; i++)
        inv[i] = 1.0f / powf(c.rope_theta, (float)(i * 2) / (float)c.head_dim);
    for (int p = 0; p < rope_len; p++)
        for (int i = 0; i < half; i++) {
            const float a = (float)p * inv[i];
            ct[(size_t)p * half + i] = cosf(a);
            st[(size_t)p * half + i] = sinf(a);
        }
    const int B = c.max_batch, qd = c.n_heads * c.head_dim, kd = c.n_kv_heads * c.head_dim;
    const int wide = std::max(std::max(c.dim, qd), c.hidden_dim);
    hipError_t e = hipSuccess;
    auto alloc = [&](void **p, size_t bytes) {
        if (e == hipSuccess)
            e = hipMalloc(p, bytes ? bytes : 4);
    };
    alloc((void **)&d->cos_t, ct.size() * 4);
    alloc((void **)&d->sin_t, st.size() * 4);
    alloc((void **)&d->x, (size_t)B * c.dim * 4);
    alloc((void **)&d->xb, (size_t)B * wide * 4);
    alloc((void **)&d->xn, (size_t)B * c.dim * 4);
    alloc((void **)&d->q, (size_t)B * qd * 4);
    alloc((void **)&d->k, (size_t)B * kd * 4);
    alloc((void **)&d->v, (size_t)B * kd * 4);
    alloc((void **)&d->att, (size_t)B * qd * 4);
    alloc((void **)&d->hb, (size_t)B * c.hidden_dim * 4);
    alloc((void **)&d->hb2, (size_t)B * c.hidden_dim * 4);
    alloc((void **)&d->logits, (size_t)B * c.vocab * 4);
    alloc((void **)&d->sel, (size_t)B * std::max(c.sparse_k, 64) * 4);
    alloc((void **)&d->nsel, (size_t)B * 4);
    alloc((void **)&d->slots, (size_t)c.n_layers * B * 4);
    alloc((void **)&d->next, (size_t)(kMaxBatch + 1) * 4);   // tokens, then the step's error word
    alloc((void **)&d->arg_parts, (size_t)B * kArgChunks * sizeof(ArgPart));
    alloc((void **)&d->arg_cnt, (size_t)B * 4);
    alloc((void **)&d->cand, (size_t)B * std::max(c.cand_cap, 1) * 4);
    alloc((void **)&d->ncand, (size_t)B * 4);
    d->xdig_bytes = std::max(be42_gemv_xdig_bytes(wide, B, c.wkind), be42_gemv_xdig_bytes(c.dim, B, c.wkind));
    alloc(&d->xdig, d->xdig_bytes);
    d->attn_ws_bytes = be42_attn_workspace_bytes(B, c.n_heads, c.head_dim, std::max(c.sparse_k, 64), 4);
    alloc(&d->attn_ws, d->attn_ws_bytes);
    if (e == hipSuccess)
        e = hipMemcpy(d->cos_t, ct.data(), ct.size() * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = hipMemcpy(d->sin_t, st.data(), st.size() * 4, hipMemcpyHostToDevice);
    std::vector<int> slots((size_t)c.n_layers * B);
    for (size_t i = 0; i < slots.size(); i++)
        slots[i] = (int)i;
    if (e == hipSuccess)
        e = hipMemcpy(d->slots, slots.data(), slots.size() * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        be42_decoder_destroy(d);
        return hip_fail(e, "be42_decoder_create", __FILE__, __LINE__);
    }
    d->params_bytes = sizeof(StepHead) + (size_t)c.n_layers * sizeof(AppendStepArgs);
    for (int i = 0; i < 2; i++) {
        if (e == hipSuccess)
            e = hipHostMalloc(&d->params_host[i], d->params_bytes, hipHostMallocDefault);
        alloc(&d->params_dev[i], d->params_bytes);
        if (e == hipSuccess)
            e = hipEventCreateWithFlags(&d->params_free[i], hipEventDisableTiming);
    }
    if (e == hipSuccess)
        e = hipHostMalloc((void **)&d->next_host, (kMaxBatch + 1) * sizeof(int), hipHostMallocDefault);
    if (e == hipSuccess)
        e = hipStreamCreateWithFlags(&d->gstream, hipStreamNonBlocking);
    if (e == hipSuccess)
        e = hipEventCreateWithFlags(&d->ev_in, hipEventDisableTiming);
    if (e == hipSuccess)
        e = hipEventCreateWithFlags(&d->ev_out, hipEventDisableTiming);
    if (e == hipSuccess)
        e = hipMemset(d->next, 0, (size_t)(kMaxBatch + 1) * 4);
    if (e == hipSuccess)
        e = hipMemset(d->arg_cnt, 0, (size_t)B * 4);
    {
        const char *ng = getenv("BE42_DECODE_NO_GRAPH");
        d->use_graph = !(ng && ng[0] == '1');
    }
    if (e == hipSuccess && fused_layer_fits(c, d)) {
        const char *fz = getenv("BE42_DECODE_FUSED");
        if (!(fz && fz[0] == '0')) {
            const size_t fbytes = ((size_t)d->fnb + 1) * 128 + 256;
            e = hipMalloc((void **)&d->fflags, fbytes);
            if (e == hipSuccess)
                e = hipMemset(d->fflags, 0, fbytes);
            d->fused = e == hipSuccess;
            const char *fb = getenv("BE42_DECODE_FAIL_BARRIERS");
            d->fail_barriers = fb && fb[0] == '1';
        }
    }
    if (e == hipSuccess)
        d->next_host[kMaxBatch] = 0;
    if (e != hipSuccess) {
        be42_decoder_destroy(d);
        return hip_fail(e, "be42_decoder_create", __FILE__, __LINE__);
    }
    *out = d;
    return BE42_OK;
}

extern "C" void be42_decoder_destroy(be42_decoder *d)
{
    if (!d)
        return;
    if (d->gstream)
        (void)hipStreamSynchronize(d->gstream);
    for (int i = 0; i < 2; i++) {
        if (d->exec[i])
            (void)hipGraphExecDestroy(d->exec[i]);
        if (d->params_host[i])
            (void)hipHostFree(d->params_host[i]);
        if (d->params_dev[i])
            (void)hipFree(d->params_dev[i]);
        if (d->params_free[i])
            (void)hipEventDestroy(d->params_free[i]);
    }
    if (d->next_host)
        (void)hipHostFree(d->next_host);
    if (d->ev_in)
        (void)hipEventDestroy(d->ev_in);
    if (d->ev_out)
        (void)hipEventDestroy(d->ev_out);
    if (d->gstream)
        (void)hipStreamDestroy(d->gstream);
    if (d->pool)
        be42_kv_destroy(d->pool);
    if (d->pmeta_host)
        (void)hipHostFree(d->pmeta_host);
    void *ptrs[] = {d->cos_t, d->sin_t, d->x, d->xb, d->xn, d->q, d->k, d->v, d->att, d->hb, d->hb2, d->logits, d->sel,
                    d->nsel, d->slots, d->next, d->cand, d->ncand, d->xdig, d->attn_ws, d->arg_parts, d->arg_cnt, d->fflags,
                    d->px, d->pxn, d->pq, d->pk, d->pv, d->patt, d->pxb, d->phb, d->phb2, d->pdig, d->pmeta,
                    d->psel, d->pnsel};
    for (void *p : ptrs)
        if (p)
            (void)hipFree(p);
    delete d;
}

extern "C" be42_kv_pool *be42_decoder_pool(be42_decoder *d)
{
    return d ? d->pool : nullptr;
}

static int gemv(be42_decoder *d, float *y, const void *w, const float *s, int n, int k, int B, hipStream_t st)
{
    return d->c.wkind == 0 ? be42_gemv_q8_prepared(y, (const int8_t *)w, s, d->xdig, n, k, B, st)
                           : be42_gemv_fp8_prepared(y, (const uint8_t *)w, s, d->xdig, n, k, B, st);
}

// projections that share one input, in one launch
static int gemv_multi(be42_decoder *d, std::initializer_list<be42_gemv_seg> segs, int k, int B, hipStream_t st)
{
    return be42_gemv_prepared_multi(segs.begin(), (int)segs.size(), d->xdig, k, B, d->c.wkind, st);
}

#define DEC_TRY(x)                                                                                                 \
    do {                                                                                                           \
        const int rc_ = (x);                                                                                       \
        if (rc_)                                                                                                   \
            return rc_;                                                                                            \
    } while (0)

// Calls f(integral_constant FP8, integral_constant NV) for a row of n
// elements (n <= kRowMax), NV = ceil(n / kChunk).
template <class F>
static void launch_rows(bool fp8, int n, F &&f)
{
    using T = std::true_type;
    using Fa = std::false_type;
    const int nv = (n + kChunk - 1) / kChunk;
    auto pick = [&](auto f8) {
        if (nv <= 1) f(f8, std::integral_constant<int, 1>());
        else if (nv <= 2) f(f8, std::integral_constant<int, 2>());
        else if (nv <= 3) f(f8, std::integral_constant<int, 3>());
        else if (nv <= 4) f(f8, std::integral_constant<int, 4>());
        else if (nv <= 6) f(f8, std::integral_constant<int, 6>());
        else if (nv <= 8) f(f8, std::integral_constant<int, 8>());
        else if (nv <= 12) f(f8, std::integral_constant<int, 12>());
        else f(f8, std::integral_constant<int, 16>());
    };
    if (fp8)
        pick(T());
    else
        pick(Fa());
}

// The fused layer launch after layer l's attention (batch 1).
static FPhase one_phase(const void *w, const float *sw, float *y, int n, int K)
{
    FPhase p{};
    p.w[0] = (const uint8_t *)w;
    p.sw[0] = sw;
    p.y[0] = y;
    p.n[0] = n;
    p.nseg = 1;
    p.K = K;
    p.steps = K / 128;
    p.units = (n + 15) / 16;
    p.tend[0] = p.units;
    return p;
}

// att_out: the fused launch also computes the next layer's dense attention
// into it (enqueue_step's tail_att), else null.  start_tok: the step's first
// launch (l = -1): the embedding of that token, layer 0's RMSNorm, q/k/v,
// RoPE and append (and, with att_out, its attention).
static int launch_fused_layer(be42_decoder *d, int l, const AppendStepArgs *app, const int *pos_p, int rope_len,
                              hipStream_t st, float *att_out, float att_scale, const int *start_tok = nullptr,
                              bool pf_route = false)
{
    const be42_decoder_config &c = d->c;
    const bool start = start_tok != nullptr;
    const be42_decoder_layer &L = d->w.layers[start ? 0 : l];
    const int dim = c.dim, hidden = c.hidden_dim, qd = c.n_heads * c.head_dim, kd = c.n_kv_heads * c.head_dim;
    FusedArgs A{};
    A.o = one_phase(L.wo, L.so, d->xb, dim, qd);
    A.gu = one_phase(L.w1, L.s1, d->hb, hidden, dim);
    A.gu.w[1] = (const uint8_t *)L.w3;
    A.gu.sw[1] = L.s3;
    A.gu.n[1] = hidden;
    A.gu.nseg = 2;
    A.gu.silu = 1;
    A.down = one_phase(L.w2, L.s2, d->xb, dim, hidden);
    if (start || l + 1 < c.n_layers) {
        const be42_decoder_layer &N = d->w.layers[start ? 0 : l + 1];
        A.qkv = one_phase(N.wq, N.sq, d->q, qd, dim);
        A.qkv.w[1] = (const uint8_t *)N.wk;
        A.qkv.w[2] = (const uint8_t *)N.wv;
        A.qkv.sw[1] = N.sk;
        A.qkv.sw[2] = N.sv;
        A.qkv.y[1] = d->k;
        A.qkv.y[2] = d->v;
        A.qkv.n[1] = A.qkv.n[2] = kd;
        A.qkv.nseg = 3;
        A.qkv.tend[0] = qd / 16;
        A.qkv.tend[1] = qd / 16 + kd / 16;
        A.qkv.tend[2] = qd / 16 + 2 * (kd / 16);
        A.qkv.units = A.qkv.tend[2];
        A.attn_norm = N.attn_norm;
        A.app = app + (start ? 0 : l + 1);
    } else {
        A.qkv.nseg = 0;
        A.app = app + l;
    }
    A.att = d->att;
    A.X = d->x;
    A.Hb = d->xn;
    A.XB = d->xb;
    A.H2 = d->hb;
    A.q = d->q;
    A.k = d->k;
    A.v = d->v;
    A.ffn_norm = L.ffn_norm;
    A.P = *d->pool;
    A.cos_t = d->cos_t;
    A.sin_t = d->sin_t;
    A.pos_p = pos_p;
    A.rope_len = rope_len;
    A.dim = dim;
    A.hidden = hidden;
    A.qd = qd;
    A.kd = kd;
    A.H = c.n_heads;
    A.KV = c.n_kv_heads;
    A.eps = c.norm_eps;
    A.flags = d->fflags;
    A.gen = d->fflags + ((size_t)d->fnb + 1) * 32;
    A.err = d->next + kMaxBatch;
    A.spin_max = d->fail_barriers ? 64u : kFSpinMax;
    A.bias = d->fail_barriers ? 1u << 24 : 0u;
    A.att_out = start || l + 1 < c.n_layers ? att_out : nullptr;
    A.att_scale = att_scale;
    A.er = EmbRow{(const uint8_t *)d->w.emb, d->w.emb_s, start_tok};
    A.pf_route = pf_route && (start || l + 1 < c.n_layers);
    const int nv = (dim + kChunk - 1) / kChunk;
    const bool fp8 = c.wkind != 0, bf16 = c.kv_kind == BE42_KV_BF16;
    auto go = [&](auto f8, auto kb, auto nvc) {
        if (start)
            hipLaunchKernelGGL((k_fused_layer<decltype(f8)::value, decltype(kb)::value, decltype(nvc)::value, true>),
                               dim3(d->fnb), dim3(kFT), 0, st, A);
        else
            hipLaunchKernelGGL((k_fused_layer<decltype(f8)::value, decltype(kb)::value, decltype(nvc)::value, false>),
                               dim3(d->fnb), dim3(kFT), 0, st, A);
    };
    auto pick_nv = [&](auto f8, auto kb) {
        switch (nv) {
        case 1: go(f8, kb, std::integral_constant<int, 1>()); break;
        case 2: go(f8, kb, std::integral_constant<int, 2>()); break;
        case 3: go(f8, kb, std::integral_constant<int, 3>()); break;
        default: go(f8, kb, std::integral_constant<int, 4>()); break;
        }
    };
    if (fp8)
        bf16 ? pick_nv(std::true_type(), std::true_type()) : pick_nv(std::true_type(), std::false_type());
    else
        bf16 ? pick_nv(std::false_type(), std::true_type()) : pick_nv(std::false_type(), std::false_type());
    BE42_LAUNCH_CHECK();
    return BE42_OK;
}

// The launches of one step.  Everything that changes from step to step (the
// position, the tokens, the page bookkeeping of the appends) is read from
// device memory at params_dev, so this sequence depends only on the key
// (batch, dense or sparse attention, token source, output buffers).
static int enqueue_step(be42_decoder *d, int B, bool sparse, bool dev_tokens, float *logits_out, int parity,
                        hipStream_t st)
{
    const be42_decoder_config &c = d->c;
    const int dim = c.dim, hd = c.head_dim, H = c.n_heads, KV = c.n_kv_heads;
    const int qd = H * hd, kd = KV * hd, fp8 = c.wkind;
    uint8_t *params = (uint8_t *)d->params_dev[parity];
    const StepHead *head = (const StepHead *)params;
    const AppendStepArgs *app = (const AppendStepArgs *)(params + sizeof(StepHead));
    BE42_HIP(hipMemcpyAsync(params, d->params_host[parity], d->params_bytes, hipMemcpyHostToDevice, st));
    const int *tok = dev_tokens ? d->next : head->tokens;
    // one sequence: the embedding, layer 0's norm, q/k/v, RoPE and append in
    // one fused launch (below), and everything of a layer after its
    // attention (and the next layer's q/k/v and append) in one fused launch
    const bool fz = d->fused && B == 1;
    const dim3 eg((dim + 255) / 256, B);
    if (!fz) {
        if (fp8)
            hipLaunchKernelGGL(k_embed<true>, eg, dim3(256), 0, st, d->x, (const uint8_t *)d->w.emb, d->w.emb_s,
                               tok, dim);
        else
            hipLaunchKernelGGL(k_embed<false>, eg, dim3(256), 0, st, d->x, (const uint8_t *)d->w.emb, d->w.emb_s,
                               tok, dim);
        BE42_LAUNCH_CHECK();
    }
    uint8_t *dig = (uint8_t *)d->xdig;
    // the residual stream alternates between x and xn: a norm with a pending
    // delta writes x + delta to the other buffer
    float *xcur = d->x, *xalt = d->xn;
    // RMSNorm (+ residual) straight into the GEMV digit planes
    auto norm = [&](const uint16_t *wn, const float *delta) {
        float *xo = delta ? xalt : nullptr;
        launch_rows(fp8, dim, [&](auto f8, auto nv) {
            hipLaunchKernelGGL((k_rmsnorm<decltype(f8)::value, decltype(nv)::value>),
                               dim3((dim + kChunk - 1) / kChunk, B), dim3(kRowT), 0, st, nullptr, dig, xcur, xo,
                               delta, wn, dim, B, c.norm_eps, false);
        });
        if (delta)
            std::swap(xcur, xalt);
        return hipGetLastError();
    };
    const float scale = 1.0f / sqrtf((float)hd);
    const int rope_len = c.rope_len > 0 ? c.rope_len : c.max_seq;
    const be42_kv_pool &P = *d->pool;
    // dense: every page in logical order from the device page table; the
    // fused kernel reads each sequence's page count from the device
    const int dense_max = std::min(c.sparse_k, P.max_logical);
    const float *pending = nullptr;   // residual delta not yet added to x
    const bool fused_route = c.sparse_k <= 64 && c.cand_cap <= 256 && H / KV <= 4 && (hd == 64 || hd == 128);
    // dense steps of one sequence: each fused launch also runs the next
    // layer's attention (its tail has the rotated q and the appended K/V), for
    // the group shapes it is built for and selections of <= 64 pages
    const bool tail_att = fz && !sparse && dense_max <= kFusedMaxPages &&
                          ((hd == 128 && H / KV == 3) || (hd == 64 && H / KV == 1));
    if (fz)
        DEC_TRY(launch_fused_layer(d, -1, app, &head->pos, rope_len, st, tail_att ? d->att : nullptr, scale, tok,
                                   sparse && fused_route));
    for (int l = 0; l < c.n_layers; l++) {
        const be42_decoder_layer &L = d->w.layers[l];
        if (!fz) {
            BE42_HIP(norm(L.attn_norm, pending));
            DEC_TRY(gemv_multi(d, {{L.wq, L.sq, d->q, qd}, {L.wk, L.sk, d->k, kd}, {L.wv, L.sv, d->v, kd}}, dim, B,
                               st));
            // RoPE of q and k, the K/V append and the seal of filled pages: one launch
            DEC_TRY(launch_rope_append_step_dev(P, app + l, B, d->q, d->k, d->v, d->cos_t, d->sin_t, &head->pos,
                                                rope_len, H, st));
        }
        if (d->capture_q)
            BE42_HIP(hipMemcpyAsync(d->capture_q + (size_t)l * c.max_batch * qd, d->q, (size_t)B * qd * 4,
                                    hipMemcpyDeviceToDevice, st));
        if (d->capture_k)
            BE42_HIP(hipMemcpyAsync(d->capture_k + (size_t)l * c.max_batch * kd, d->k, (size_t)B * kd * 4,
                                    hipMemcpyDeviceToDevice, st));
        if (d->capture_v)
            BE42_HIP(hipMemcpyAsync(d->capture_v + (size_t)l * c.max_batch * kd, d->v, (size_t)B * kd * 4,
                                    hipMemcpyDeviceToDevice, st));
        const int *lslots = d->slots + (size_t)l * c.max_batch;
        bool att_digits = false;   // the attention wrote d->att's digit planes into d->xdig
        if (!sparse) {
            if (!tail_att)
                DEC_TRY(be42_paged_attention(d->pool, d->q, B, H,
                                             P.page_table + (size_t)l * c.max_batch * P.max_logical,
                                             P.n_logical + (size_t)l * c.max_batch, P.max_logical, dense_max, scale,
                                             d->att, dense_max <= 64 ? 1 : 4, d->attn_ws, d->attn_ws_bytes, st));
        } else if (fused_route) {
            // route + attention in one launch; without the fused layer a split
            // launch also writes the o projection's digit planes
            DEC_TRY(lsh_attention_digits(*d->pool, d->q, lslots, B, H, c.sparse_k, c.cand_cap, scale, d->att,
                                         d->sel, d->nsel, std::max(c.sparse_k, 64), fz ? nullptr : d->xdig,
                                         fp8 != 0, &att_digits, d->next + kMaxBatch, st));
        } else {
            const int stride = std::max(c.sparse_k, 64);
            DEC_TRY(be42_lsh_route(d->pool, d->q, lslots, B, H, c.sparse_k, c.cand_cap, d->sel, d->nsel, stride,
                                   d->cand, d->ncand, nullptr, st));
            DEC_TRY(be42_paged_attention(d->pool, d->q, B, H, d->sel, d->nsel, stride, c.sparse_k, scale, d->att,
                                         c.sparse_k <= 64 ? 1 : 4, d->attn_ws, d->attn_ws_bytes, st));
        }
        if (d->capture_sel && sparse) {
            const int stride = std::max(c.sparse_k, 64);
            BE42_HIP(hipMemcpyAsync(d->capture_sel + (size_t)l * c.max_batch * stride, d->sel,
                                    (size_t)B * stride * 4, hipMemcpyDeviceToDevice, st));
        }
        if (d->capture_nsel) {
            const int *src = !sparse ? P.n_logical + (size_t)l * c.max_batch : d->nsel;
            BE42_HIP(hipMemcpyAsync(d->capture_nsel + (size_t)l * c.max_batch, src, (size_t)B * 4,
                                    hipMemcpyDeviceToDevice, st));
        }
        if (fz) {
            DEC_TRY(launch_fused_layer(d, l, app, &head->pos, rope_len, st, tail_att ? d->att : nullptr, scale,
                                       nullptr, sparse && fused_route));
            continue;
        }
        if (!att_digits)
            DEC_TRY(be42_gemv_prepare(d->xdig, d->att, qd, B, fp8, st));
        DEC_TRY(gemv(d, d->xb, L.wo, L.so, dim, qd, B, st));
        BE42_HIP(norm(L.ffn_norm, d->xb));                 // x += attention output
        DEC_TRY(gemv_multi(d, {{L.w1, L.s1, d->hb, c.hidden_dim}, {L.w3, L.s3, d->hb2, c.hidden_dim}}, dim, B, st));
        const int nvw = (int)((xdig_kp(c.hidden_dim, fp8) + 4 * kWideT - 1) / (4 * kWideT));
        if (nvw <= 2) {
            auto wide = [&](auto f8, auto nv) {
                hipLaunchKernelGGL((k_silu_mul_wide<decltype(f8)::value, decltype(nv)::value>), dim3(B),
                                   dim3(kWideT), 0, st, dig, d->hb, d->hb2, c.hidden_dim, B);
            };
            if (fp8)
                nvw <= 1 ? wide(std::true_type(), std::integral_constant<int, 1>())
                         : wide(std::true_type(), std::integral_constant<int, 2>());
            else
                nvw <= 1 ? wide(std::false_type(), std::integral_constant<int, 1>())
                         : wide(std::false_type(), std::integral_constant<int, 2>());
        } else {
            launch_rows(fp8, c.hidden_dim, [&](auto f8, auto nv) {
                hipLaunchKernelGGL((k_silu_mul<decltype(f8)::value, decltype(nv)::value>),
                                   dim3((c.hidden_dim + kChunk - 1) / kChunk, B), dim3(kRowT), 0, st, nullptr, dig,
                                   d->hb, d->hb2, c.hidden_dim, B, false);
            });
        }
        BE42_LAUNCH_CHECK();
        DEC_TRY(gemv(d, d->xb, L.w2, L.s2, dim, c.hidden_dim, B, st));
        pending = d->xb;
    }
    // final residual + norm, lm_head, argmax
    if (fz) {
        // the fused launches leave h in xn and the last down output in xb
        xcur = d->xn;
        xalt = d->x;
        pending = d->xb;
    }
    BE42_HIP(norm(d->w.final_norm, pending));
    float *lg = logits_out ? logits_out : d->logits;
    DEC_TRY(gemv(d, lg, d->w.out, d->w.out_s, c.vocab, dim, B, st));
    hipLaunchKernelGGL(k_argmax, dim3(kArgChunks, B), dim3(256), 0, st, d->next, lg, c.vocab, d->arg_parts,
                       d->arg_cnt);
    BE42_LAUNCH_CHECK();
    BE42_HIP(hipMemcpyAsync(d->next_host, d->next, (size_t)(kMaxBatch + 1) * 4, hipMemcpyDeviceToHost, st));
    return BE42_OK;
}

static int launch_step(be42_decoder *d, int B, int pos, bool host_tokens, float *logits_out, hipStream_t caller,
                       bool *queued);

// The fused launches' error flag as the last finished step copied it to the
// host (wait: for the decoder's queued work first).  Once it is seen set the
// decoder's results and cache are invalid, and every later call is refused.
static int fault_check(be42_decoder *d, bool wait, const char *what)
{
    if (!d->fault) {
        if (wait) {
            BE42_HIP(hipEventSynchronize(d->ev_out));
            d->fault = d->next_host[kMaxBatch];
        } else {
            const hipError_t q = hipEventQuery(d->ev_out);
            if (q == hipSuccess)
                d->fault = d->next_host[kMaxBatch];
            else if (q == hipErrorNotReady)
                (void)hipGetLastError();
            else
                BE42_HIP(q);
        }
    }
    BE42_CHECK(d->fault == 0,
               "%s: a bounded wait gave up in an earlier step (code %d: 1-2 a grid barrier of the fused layer, 3 its "
               "wave sync, 4 the split attention's); the decoder's results and cache are invalid (destroy it)",
               what, d->fault);
    return BE42_OK;
}

extern "C" int be42_decoder_status(be42_decoder *d)
{
    BE42_CHECK(d, "be42_decoder_status: null decoder");
    return fault_check(d, true, "be42_decoder_status");
}

extern "C" int be42_decoder_step(be42_decoder *d, const int *tokens, int batch, int pos, int *next_tokens,
                                 float *logits_out, void *stream)
{
    BE42_CHECK(d, "be42_decoder_step: null decoder");
    const be42_decoder_config &c = d->c;
    BE42_CHECK(batch > 0 && batch <= c.max_batch, "be42_decoder_step: batch %d (max %d)", batch, c.max_batch);
    BE42_CHECK(pos >= 0 && pos < c.max_seq, "be42_decoder_step: position %d (max %d)", pos, c.max_seq);
    hipStream_t caller = as_stream(stream);
    const int B = batch;
    for (int b = 0; tokens && b < B; b++)
        BE42_CHECK(tokens[b] >= 0 && tokens[b] < c.vocab, "be42_decoder_step: token %d out of range", tokens[b]);
    DEC_TRY(fault_check(d, false, "be42_decoder_step"));
    // host parameters of this step into the pinned buffer of this parity,
    // once the step that used it last has copied it
    const int par = d->parity;
    BE42_HIP(hipEventSynchronize(d->params_free[par]));
    uint8_t *ph = (uint8_t *)d->params_host[par];
    StepHead *head = (StepHead *)ph;
    AppendStepArgs *app = (AppendStepArgs *)(ph + sizeof(StepHead));
    head->pos = pos;
    for (int b = 0; b < kMaxBatch; b++)
        head->tokens[b] = tokens && b < B ? tokens[b] : 0;
    int slot_ids[kMaxBatch], positions[kMaxBatch];
    for (int b = 0; b < B; b++)
        positions[b] = pos;
    // the appends are planned on the host before anything is queued; a step
    // that fails before its work is queued gives the pages back
    PlanUndo undo;
    int rc = BE42_OK;
    for (int l = 0; l < c.n_layers && rc == BE42_OK; l++) {
        for (int b = 0; b < B; b++)
            slot_ids[b] = l * c.max_batch + b;
        rc = plan_append_step(d->pool, slot_ids, positions, B, app + l, &undo);
    }
    bool queued = false;
    if (rc == BE42_OK)
        rc = launch_step(d, B, pos, tokens != nullptr, logits_out, caller, &queued);
    if (rc != BE42_OK) {
        if (!queued)
            undo_append_plans(d->pool, undo);
        return rc;
    }
    if (next_tokens) {
        DEC_TRY(fault_check(d, true, "be42_decoder_step"));
        memcpy(next_tokens, d->next_host, (size_t)B * sizeof(int));
    }
    return BE42_OK;
}

// Queue the planned step (parameters already in the pinned buffer of this
// parity) on the decoder's stream, as a graph replay or kernel by kernel;
// *queued tells whether any of its work reached the device.
static int launch_step(be42_decoder *d, int B, int pos, bool host_tokens, float *logits_out, hipStream_t caller,
                       bool *queued)
{
    const be42_decoder_config &c = d->c;
    const int par = d->parity;
    const int pages = pos / 16 + 1;
    be42_decoder::Key key;
    key.batch = B;
    key.sparse = pages > c.sparse_k ? 1 : 0;
    key.dev_tokens = host_tokens ? 0 : 1;
    key.logits = logits_out;
    key.cq = d->capture_q;
    key.ck = d->capture_k;
    key.cs = d->capture_sel;
    key.cv = d->capture_v;
    key.cn = d->capture_nsel;
    // the step runs on the decoder's own stream, ordered after the caller's work
    hipStream_t st = d->gstream;
    BE42_HIP(hipEventRecord(d->ev_in, caller));
    BE42_HIP(hipStreamWaitEvent(st, d->ev_in, 0));
    if (!d->use_graph) {
        *queued = true;   // launched one by one: a failure can come after some of them
        DEC_TRY(enqueue_step(d, B, key.sparse, key.dev_tokens, logits_out, par, st));
    } else {
        if (!d->exec[par] || !(d->key[par] == key)) {
            if (d->exec[par]) {
                BE42_HIP(hipStreamSynchronize(st));
                BE42_HIP(hipGraphExecDestroy(d->exec[par]));
                d->exec[par] = nullptr;
            }
            hipGraph_t graph = nullptr;
            BE42_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
            const int rc = enqueue_step(d, B, key.sparse, key.dev_tokens, logits_out, par, st);
            const hipError_t ce = hipStreamEndCapture(st, &graph);
            if (rc) {
                if (graph)
                    (void)hipGraphDestroy(graph);
                return rc;
            }
            BE42_HIP(ce);
            const hipError_t ie = hipGraphInstantiate(&d->exec[par], graph, nullptr, nullptr, 0);
            (void)hipGraphDestroy(graph);
            BE42_HIP(ie);
            d->key[par] = key;
        }
        *queued = true;
        BE42_HIP(hipGraphLaunch(d->exec[par], st));
    }
    BE42_HIP(hipEventRecord(d->params_free[par], st));
    d->parity ^= 1;
    BE42_HIP(hipEventRecord(d->ev_out, st));
    BE42_HIP(hipStreamWaitEvent(caller, d->ev_out, 0));
    return BE42_OK;
}

extern "C" int be42_decoder_next_tokens(be42_decoder *d, const int **dev_ptr)
{
    BE42_CHECK(d && dev_ptr, "be42_decoder_next_tokens: null pointer");
    *dev_ptr = d->next;
    return BE42_OK;
}

// Inspection: copy each layer's rotated queries ([n_layers][max_batch]
// [n_heads * head_dim]) and attended page counts ([n_layers][max_batch]) of
// every step into device buffers; NULL stops either.
extern "C" int be42_decoder_capture(be42_decoder *d, float *q_dst, int *nsel_dst)
{
    BE42_CHECK(d, "be42_decoder_capture: null decoder");
    d->capture_q = q_dst;
    d->capture_nsel = nsel_dst;
    return BE42_OK;
}

// Inspection: copy each layer's post-RoPE K and V rows of every step (the
// values the step appends to the page pool, [n_layers][max_batch]
// [n_kv * head_dim]) into device buffers; NULL stops either.
extern "C" int be42_decoder_capture_kv(be42_decoder *d, float *k_dst, float *v_dst)
{
    BE42_CHECK(d, "be42_decoder_capture_kv: null decoder");
    d->capture_k = k_dst;
    d->capture_v = v_dst;
    return BE42_OK;
}

// Inspection: on routed steps, copy each layer's selection (physical page
// ids in attention order, [n_layers][max_batch][max(sparse_k, 64)]; the
// counts are those of be42_decoder_capture) into a device buffer; NULL stops.
extern "C" int be42_decoder_capture_sel(be42_decoder *d, int *sel_dst)
{
    BE42_CHECK(d, "be42_decoder_capture_sel: null decoder");
    d->capture_sel = sel_dst;
    return BE42_OK;
}

// ---- prefill ------------------------------------------------------------------
// A prompt of n tokens of one sequence in passes of up to kPrefillChunk
// tokens, each pass layer by layer over all of its tokens: the projections
// are GEMMs over the activation digit planes (every weight tile read once
// per pass, and each output equal to the decode GEMV's), RMSNorm, RoPE and
// SiLU*up are the decode step's row kernels, the pass's K/V rows are
// appended (pages sealed as they fill), and each token's attention sees the
// cache as the decode step at its position saw it.  The argmax (and the
// logits) of the prompt's last token follow through the final norm, the
// lm_head GEMV and the argmax of the decode step.  For INT8 weights the
// result is bit-identical to n single-sequence decode steps (the KV pages,
// LSH index and logits); for FP8 it differs only by the order of the fp32
// accumulations inside the matrix cores.
// This is the fixed layout of forward_prefill_batch
// (src/inference/inference.c:718-1112), whose activations are token-major
// but described to op_matmul as [dim][batch] (:812-843).

static int prefill_alloc(be42_decoder *d)
{
    if (d->px)
        return BE42_OK;
    const be42_decoder_config &c = d->c;
    const size_t T = kPrefillChunk;
    const int qd = c.n_heads * c.head_dim, kd = c.n_kv_heads * c.head_dim;
    const int wide = std::max(std::max(c.dim, qd), c.hidden_dim);
    hipError_t e = hipSuccess;
    auto alloc = [&](void **p, size_t bytes) {
        if (e == hipSuccess)
            e = hipMalloc(p, bytes);
    };
    alloc((void **)&d->px, T * c.dim * 4);
    alloc((void **)&d->pxn, T * c.dim * 4);
    alloc((void **)&d->pq, T * qd * 4);
    alloc((void **)&d->pk, T * kd * 4);
    alloc((void **)&d->pv, T * kd * 4);
    alloc((void **)&d->patt, T * qd * 4);
    alloc((void **)&d->pxb, T * c.dim * 4);
    alloc((void **)&d->phb, T * c.hidden_dim * 4);
    alloc((void **)&d->phb2, T * c.hidden_dim * 4);
    alloc(&d->pdig, be42_gemm_xdig_bytes(wide, (int)T, c.wkind));
    d->pmeta_bytes = ((2 + (size_t)c.n_layers) * T + (size_t)c.n_layers * append_run_list_cap((int)T)) * sizeof(int);
    alloc((void **)&d->pmeta, d->pmeta_bytes);
    d->psel_stride = prefix_sel_stride(c.sparse_k);
    alloc((void **)&d->psel, T * d->psel_stride * sizeof(int));
    alloc((void **)&d->pnsel, T * sizeof(int));
    if (e == hipSuccess)
        e = hipHostMalloc((void **)&d->pmeta_host, d->pmeta_bytes, hipHostMallocDefault);
    if (e != hipSuccess) {
        void **ptrs[] = {(void **)&d->px, (void **)&d->pxn, (void **)&d->pq, (void **)&d->pk, (void **)&d->pv,
                         (void **)&d->patt, (void **)&d->pxb, (void **)&d->phb, (void **)&d->phb2, &d->pdig,
                         (void **)&d->pmeta, (void **)&d->psel, (void **)&d->pnsel};
        for (void **p : ptrs)
            if (*p) {
                (void)hipFree(*p);
                *p = nullptr;
            }
        if (d->pmeta_host) {
            (void)hipHostFree(d->pmeta_host);
            d->pmeta_host = nullptr;
        }
        return hip_fail(e, "be42_decoder_prefill", __FILE__, __LINE__);
    }
    return BE42_OK;
}

static int pgemm(be42_decoder *d, float *y, const void *w, const float *s, int n, int k, int T, hipStream_t st)
{
    return d->c.wkind == 0 ? be42_gemm_q8_prepared(y, (const int8_t *)w, s, d->pdig, n, k, T, st)
                           : be42_gemm_fp8_prepared(y, (const uint8_t *)w, s, d->pdig, n, k, T, st);
}

static int pgemm_multi(be42_decoder *d, std::initializer_list<be42_gemv_seg> segs, int k, int T, hipStream_t st)
{
    return be42_gemm_prepared_multi(segs.begin(), (int)segs.size(), d->pdig, k, T, d->c.wkind, st);
}

// One pass: tokens, visible lengths, slots and each layer's page lists
// (runs[l], lists at the metadata's offset list_off[l]) at d->pmeta (device),
// positions p0 .. p0 + T - 1 of sequence seq.  Leaves the residual stream's
// last row and its pending delta in *x_last / *delta_last.
static int prefill_pass(be42_decoder *d, int seq, int T, int p0, const AppendRun *runs, const size_t *list_off,
                        const float **x_last, const float **delta_last, float **x_alt_last, hipStream_t st)
{
    const be42_decoder_config &c = d->c;
    const int dim = c.dim, hd = c.head_dim, H = c.n_heads, KV = c.n_kv_heads;
    const int qd = H * hd, kd = KV * hd, fp8 = c.wkind;
    const int *tok = d->pmeta, *lim = d->pmeta + T;
    const dim3 eg((dim + 255) / 256, T);
    if (fp8)
        hipLaunchKernelGGL(k_embed<true>, eg, dim3(256), 0, st, d->px, (const uint8_t *)d->w.emb, d->w.emb_s, tok,
                           dim);
    else
        hipLaunchKernelGGL(k_embed<false>, eg, dim3(256), 0, st, d->px, (const uint8_t *)d->w.emb, d->w.emb_s, tok,
                           dim);
    BE42_LAUNCH_CHECK();
    uint8_t *dig = (uint8_t *)d->pdig;
    float *xcur = d->px, *xalt = d->pxn;
    auto norm = [&](const uint16_t *wn, const float *delta) {
        float *xo = delta ? xalt : nullptr;
        launch_rows(fp8, dim, [&](auto f8, auto nv) {
            hipLaunchKernelGGL((k_rmsnorm<decltype(f8)::value, decltype(nv)::value>),
                               dim3(1, T), dim3(kRowT), 0, st, nullptr, dig, xcur, xo, delta, wn, dim, T,
                               c.norm_eps, true);
        });
        if (delta)
            std::swap(xcur, xalt);
        return hipGetLastError();
    };
    const float scale = 1.0f / sqrtf((float)hd);
    const int rope_len = c.rope_len > 0 ? c.rope_len : c.max_seq;
    const float *pending = nullptr;
    for (int l = 0; l < c.n_layers; l++) {
        const be42_decoder_layer &L = d->w.layers[l];
        BE42_HIP(norm(L.attn_norm, pending));
        DEC_TRY(pgemm_multi(d, {{L.wq, L.sq, d->pq, qd}, {L.wk, L.sk, d->pk, kd}, {L.wv, L.sv, d->pv, kd}}, dim, T,
                            st));
        hipLaunchKernelGGL(k_rope_rows, dim3(T, KV), dim3(256), 0, st, d->pq, d->pk, d->cos_t, d->sin_t, p0,
                           rope_len, H, KV, hd);
        BE42_LAUNCH_CHECK();
        // the pass's K/V rows and the pages they fill: one launch each
        DEC_TRY(launch_append_run(*d->pool, runs[l], d->pmeta + list_off[l], d->pk, d->pv, st));
        DEC_TRY(lsh_attention_prefix(*d->pool, d->pq, d->pmeta + (size_t)(2 + l) * T, lim, T, H, c.sparse_k,
                                     c.cand_cap, scale, d->patt, d->psel, d->pnsel, d->psel_stride, st));
        DEC_TRY(xdig_prepare(d->pdig, d->patt, qd, T, fp8 != 0, st));
        DEC_TRY(pgemm(d, d->pxb, L.wo, L.so, dim, qd, T, st));
        BE42_HIP(norm(L.ffn_norm, d->pxb));                 // x += attention output
        DEC_TRY(pgemm_multi(d, {{L.w1, L.s1, d->phb, c.hidden_dim}, {L.w3, L.s3, d->phb2, c.hidden_dim}}, dim, T,
                            st));
        launch_rows(fp8, c.hidden_dim, [&](auto f8, auto nv) {
            hipLaunchKernelGGL((k_silu_mul<decltype(f8)::value, decltype(nv)::value>),
                               dim3(1, T), dim3(kRowT), 0, st, nullptr, dig, d->phb, d->phb2, c.hidden_dim, T,
                               true);
        });
        BE42_LAUNCH_CHECK();
        DEC_TRY(pgemm(d, d->pxb, L.w2, L.s2, dim, c.hidden_dim, T, st));
        pending = d->pxb;
    }
    *x_last = xcur + (size_t)(T - 1) * dim;
    *delta_last = pending + (size_t)(T - 1) * dim;
    *x_alt_last = xalt + (size_t)(T - 1) * dim;
    return BE42_OK;
}

extern "C" int be42_decoder_prefill(be42_decoder *d, int seq, const int *tokens, int n, int pos0, int *next_token,
                                    float *logits_out, void *stream)
{
    BE42_CHECK(d && tokens, "be42_decoder_prefill: null pointer");
    const be42_decoder_config &c = d->c;
    BE42_CHECK(seq >= 0 && seq < c.max_batch, "be42_decoder_prefill: sequence %d (max_batch %d)", seq, c.max_batch);
    BE42_CHECK(n > 0 && pos0 >= 0 && pos0 + n <= c.max_seq, "be42_decoder_prefill: positions %d .. %d (max_seq %d)",
               pos0, pos0 + n - 1, c.max_seq);
    BE42_CHECK(c.sparse_k <= 64 && c.cand_cap <= 256 && c.n_heads / c.n_kv_heads <= 4 &&
                   (c.head_dim == 64 || c.head_dim == 128),
               "be42_decoder_prefill: needs sparse_k <= 64, cand_cap <= 256, <= 4 heads per KV head and head_dim "
               "64 or 128 (the decode step serves the others token by token)");
    for (int i = 0; i < n; i++)
        BE42_CHECK(tokens[i] >= 0 && tokens[i] < c.vocab, "be42_decoder_prefill: token %d out of range", tokens[i]);
    DEC_TRY(fault_check(d, false, "be42_decoder_prefill"));
    DEC_TRY(prefill_alloc(d));
    hipStream_t caller = as_stream(stream), st = d->gstream;
    BE42_HIP(hipEventRecord(d->ev_in, caller));
    BE42_HIP(hipStreamWaitEvent(st, d->ev_in, 0));
    const float *x_last = nullptr, *delta_last = nullptr;
    float *xo_last = nullptr;
    for (int c0 = 0; c0 < n; c0 += kPrefillChunk) {
        const int T = std::min(kPrefillChunk, n - c0), p0 = pos0 + c0;
        // the previous pass has copied the metadata before it is rewritten
        BE42_HIP(hipStreamSynchronize(st));
        int *mh = d->pmeta_host;
        for (int t = 0; t < T; t++) {
            mh[t] = tokens[c0 + t];
            mh[T + t] = p0 + t + 1;
        }
        for (int l = 0; l < c.n_layers; l++)
            for (int t = 0; t < T; t++)
                mh[(size_t)(2 + l) * T + t] = l * c.max_batch + seq;
        // every layer's pages for the pass, allocated before anything is queued
        std::vector<AppendRun> runs(c.n_layers);
        std::vector<size_t> off(c.n_layers);
        size_t o = (2 + (size_t)c.n_layers) * T;
        for (int l = 0; l < c.n_layers; l++) {
            off[l] = o;
            DEC_TRY(plan_append_run(d->pool, l * c.max_batch + seq, p0, T, mh + o, &runs[l]));
            o += runs[l].list_len;
        }
        BE42_HIP(hipMemcpyAsync(d->pmeta, mh, o * sizeof(int), hipMemcpyHostToDevice, st));
        DEC_TRY(prefill_pass(d, seq, T, p0, runs.data(), off.data(), &x_last, &delta_last, &xo_last, st));
    }
    // the last token: final residual + norm (one row, into the decode GEMV's
    // digit planes), lm_head, argmax into the sequence's feedback slot
    const int dim = c.dim;
    launch_rows(c.wkind, dim, [&](auto f8, auto nv) {
        hipLaunchKernelGGL((k_rmsnorm<decltype(f8)::value, decltype(nv)::value>), dim3((dim + kChunk - 1) / kChunk, 1),
                           dim3(kRowT), 0, st, nullptr, (uint8_t *)d->xdig, x_last, xo_last, delta_last,
                           d->w.final_norm, dim, 1, c.norm_eps, false);
    });
    BE42_LAUNCH_CHECK();
    float *lg = logits_out ? logits_out : d->logits + (size_t)seq * c.vocab;
    DEC_TRY(gemv(d, lg, d->w.out, d->w.out_s, c.vocab, dim, 1, st));
    hipLaunchKernelGGL(k_argmax, dim3(kArgChunks, 1), dim3(256), 0, st, d->next + seq, lg, c.vocab,
                       d->arg_parts + (size_t)seq * kArgChunks, d->arg_cnt + seq);
    BE42_LAUNCH_CHECK();
    BE42_HIP(hipMemcpyAsync(d->next_host, d->next + seq, sizeof(int), hipMemcpyDeviceToHost, st));
    BE42_HIP(hipEventRecord(d->ev_out, st));
    BE42_HIP(hipStreamWaitEvent(caller, d->ev_out, 0));
    if (next_token) {
        BE42_HIP(hipEventSynchronize(d->ev_out));
        *next_token = d->next_host[0];
    }
    return BE42_OK;
}
