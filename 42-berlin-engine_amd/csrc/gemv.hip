// gemv.hip -- decode GEMV for per-row-scaled INT8 / FP8 E4M3 weights on gfx950.
//
// Replaces the n == 1 GEMV of op_matmul (src/compute/ops_matmul.c:366-417;
// structure of matvec_bf16_f32_blocked :57-153) for quantized weights:
//     y[b][i] = w_scale[i] * sum_j w[i][j] * x[b][j],   x fp32, batch <= 16.
//
// The weight stream goes straight from HBM into the matrix cores with no
// per-element dequantisation: the fp32 activations are split once per call
// into fixed-point digits of the MFMA input type, so that
//     x[b][j] = s_b * sum_d digit_d[b][j] * R^-d   (R = 254 for INT8, 30 for FP8)
// (INT8 to ~2^-24 relative to max|x[b]|, FP8 to ~1.2e-6), and each digit
// plane is one MFMA operand.
//   INT8: 3 int8 digits in [-127, 127], v_mfma_i32_16x16x64_i8, exact int32
//         accumulators, recombined in fp64 in the epilogue.
//   FP8:  4 integer digits in [-15, 15] stored as E4M3 codes (exact),
//         v_mfma_scale_f32_16x16x128_f8f6f4 with unit scales, fp32 accumulators.
// The per-row scale is applied once per output, in the epilogue.
//
// A lane (r = lane % 16, g = lane / 16) loads 16 (INT8) or 32 (FP8)
// contiguous bytes of weight row r per MFMA; the same k positions of digit
// column r form the B operand.  Tiling and K-split are described at k_gemv.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <type_traits>

#include "be42_common.h"
#include "xdigits.h"

namespace be42 {

// Digit planes of the activations.  Grid (chunks of kPrepChunk k, batch):
// every block recomputes the row absmax (x is small and L2-resident), then
// writes the digits of its chunk, 4 consecutive k per thread as one dword per
// plane.  Layout dig[d][b][0..Kp), zero beyond K.
constexpr int kPrepChunk = 1024;

// Per-thread partial absmax of x[0..K) (K % 4 == 0 on this path) with four
// independent 16-byte loads in flight per iteration.
__device__ __forceinline__ float absmax_vec(const float *x, int K)
{
    const float4 *x4 = (const float4 *)x;
    const int n4 = K >> 2;
    float m0 = 0.f, m1 = 0.f, m2 = 0.f, m3 = 0.f;
    int i = threadIdx.x;
    for (; i + 3 * (int)blockDim.x < n4; i += 4 * blockDim.x) {
        const float4 a = x4[i], b = x4[i + blockDim.x], c = x4[i + 2 * blockDim.x], d = x4[i + 3 * blockDim.x];
        m0 = fmaxf(m0, fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))));
        m1 = fmaxf(m1, fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
        m2 = fmaxf(m2, fmaxf(fmaxf(fabsf(c.x), fabsf(c.y)), fmaxf(fabsf(c.z), fabsf(c.w))));
        m3 = fmaxf(m3, fmaxf(fmaxf(fabsf(d.x), fabsf(d.y)), fmaxf(fabsf(d.z), fabsf(d.w))));
    }
    for (; i < n4; i += blockDim.x) {
        const float4 a = x4[i];
        m0 = fmaxf(m0, fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))));
    }
    return fmaxf(fmaxf(m0, m1), fmaxf(m2, m3));
}

template <bool FP8>
__global__ __launch_bounds__(256) void k_gemv_prep(const float *__restrict__ x, int K, int Kp, int B,
                                                   uint8_t *__restrict__ dig, float *__restrict__ sx)
{
    __shared__ float red[4];
    const int b = blockIdx.y;
    const float *xr = x + (size_t)b * K;
    const float m = wave_max(absmax_vec(xr, K));
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = m;
    __syncthreads();
    const float amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float s = digit_scale<FP8>(amax);
    if (blockIdx.x == 0 && threadIdx.x == 0)
        sx[b] = s;
    const int k0 = blockIdx.x * kPrepChunk + threadIdx.x * 4;
    if (k0 >= Kp)
        return;
    const float4 xv4 = k0 < K ? *(const float4 *)(xr + k0) : make_float4(0.f, 0.f, 0.f, 0.f);
    const float xe[4] = {xv4.x, xv4.y, xv4.z, xv4.w};
    store_digit_words<FP8>(xe, s, dig, B, Kp, b, k0);
}

// The same digit planes for rows of at most 1024 * NV elements in one round
// trip to memory: thread t loads float4 t of every 256-float4 chunk of the
// row at once (zero past K), so the absmax needs no second pass.  Register j
// holds chunk (blockIdx.x + j) mod chunks, so register 0 is already this
// block's element (a register picked by blockIdx.x would be an indexed access,
// which the compiler places in scratch memory).  Same grid and layout as
// k_gemv_prep; the maximum is order-free, so the digits are the same bytes.
template <bool FP8, int NV>
__global__ __launch_bounds__(256) void k_gemv_prep_row(const float *__restrict__ x, int K, int Kp, int B,
                                                       uint8_t *__restrict__ dig, float *__restrict__ sx)
{
    __shared__ float red[4];
    const int b = blockIdx.y, t = threadIdx.x, nch = gridDim.x;
    const float4 *x4 = (const float4 *)(x + (size_t)b * K);
    const int n4 = K >> 2;
    // unconditional loads at a clamped index, zeroed after: straight-line
    // code keeps every load in flight at once and the array in registers
    float4 v[NV];
    bool in[NV];
#pragma unroll
    for (int j = 0; j < NV; j++) {
        int c = (int)blockIdx.x + j;
        c = c >= nch ? c - nch : c;
        const int i = 256 * c + t;
        in[j] = j < nch && i < n4;
        v[j] = x4[min(i, n4 - 1)];
    }
#pragma unroll
    for (int j = 0; j < NV; j++)
        if (!in[j])
            v[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    float m = 0.f;
#pragma unroll
    for (int j = 0; j < NV; j++)
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
    m = wave_max(m);
    if ((t & 63) == 0)
        red[t >> 6] = m;
    __syncthreads();
    const float amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float s = digit_scale<FP8>(amax);
    if (blockIdx.x == 0 && t == 0)
        sx[b] = s;
    const float xe[4] = {v[0].x, v[0].y, v[0].z, v[0].w};
    store_digit_words<FP8>(xe, s, dig, B, Kp, b, blockIdx.x * kPrepChunk + t * 4);
}

__constant__ double kF8Weight[kF8Digits] = {1.0, 1.0 / 30, 1.0 / 900, 1.0 / 27000};

// Up to three weight matrices that share one input (the q/k/v or gate/up
// projections of a decode step) stream in one launch: their rows are
// numbered one after another, and a row tile may straddle two of them.
constexpr int kMaxSegs = 3;
struct GemvSegs {
    const uint8_t *w[kMaxSegs];
    const float *sw[kMaxSegs];
    float *y[kMaxSegs];
    int n[kMaxSegs];
    int nseg, total;
};

__device__ __forceinline__ int seg_of(const GemvSegs &S, int row, int *local)
{
    static_assert(kMaxSegs == 3, "segment lookup written for three segments");
    // branch-free: the segment ends are uniform, the row is per lane
    const int e1 = S.n[0], e2 = S.n[0] + S.n[1];
    const bool s1 = S.nseg > 1 && row >= e1;
    const bool s2 = S.nseg > 2 && row >= e2;
    *local = row - (s2 ? e2 : (s1 ? e1 : 0));
    return (int)s1 + (int)s2;
}

// a[sg] for a lane-varying segment number, by selects over the kernel
// argument's entries (uniform, so scalar loads): indexing the by-value
// argument with sg itself costs dependent vector loads from the argument
// buffer before the first weight load can be addressed.
// Accesses through global-address-space pointers.  A pointer that went
// through seg_pick is no longer known to be global, and a plain dereference
// becomes a flat access, which also counts against the LDS / scalar counter
// (stage barriers wait on that one to drain) and makes the compiler wait on
// it early.
__device__ __forceinline__ float ld_global(const float *p)
{
    return *(const __attribute__((address_space(1))) float *)p;
}
__device__ __forceinline__ v4i ld_global_v4(const uint8_t *p)
{
    return *(const __attribute__((address_space(1))) v4i *)p;
}
__device__ __forceinline__ void st_global(float *p, float v) { *(__attribute__((address_space(1))) float *)p = v; }

template <class T>
__device__ __forceinline__ T seg_pick(const T (&a)[kMaxSegs], int sg)
{
    T v = a[0];
    asm volatile("" : "+s"(v));   // each entry its own scalar value: not re-fused into a[sg]
#pragma unroll
    for (int i = 1; i < kMaxSegs; i++) {
        T ai = a[i];
        asm volatile("" : "+s"(ai));
        v = sg == i ? ai : v;
    }
    return v;
}

// Epilogue operands of a lane, loaded at kernel start so their latency hides
// under the weight stream.  In the epilogue loop over o = lane + 64 j the
// lane's output row within a tile is always r = lane % 16 and its batch rows
// are g + 4 j (g = lane / 16), j < 4.
template <int RT>
struct EpiOps {
    float sw[RT];
    float *y[RT];
    int n[RT];
    float sx[4];
};

template <int RT>
__device__ __forceinline__ void epi_load(EpiOps<RT> &E, const GemvSegs &S, const float *sx, int row0, int r, int g,
                                         int B)
{
#pragma unroll
    for (int t = 0; t < RT; t++) {
        const int row = row0 + t * 16 + r;
        if (row < S.total) {
            int local;
            const int sg = seg_of(S, row, &local);
            E.sw[t] = ld_global(seg_pick(S.sw, sg) + local);
            E.y[t] = seg_pick(S.y, sg) + local;
            E.n[t] = seg_pick(S.n, sg);
        } else {
            E.sw[t] = 0.0f;
            E.y[t] = nullptr;
            E.n[t] = 0;
        }
    }
#pragma unroll
    for (int j = 0; j < 4; j++)
        E.sx[j] = g + 4 * j < B ? sx[g + 4 * j] : 0.0f;
}

// y for row tile t from the digit sums of each (row, batch row): raw(d, bb)
// returns the sum of digit plane d of batch row bb for the lane's row.
template <bool FP8, int RT, class RawAt>
__device__ __forceinline__ void epi_store(const EpiOps<RT> &E, int t, int g, int B, RawAt raw)
{
    constexpr int ND = FP8 ? kF8Digits : kI8Digits;
    using Tot = typename std::conditional<FP8, double, long long>::type;
    const double sxw = FP8 ? 1.0 : 1.0 / (double)(kI8Base * kI8Base);
    if (!E.y[t])
        return;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int bb = g + 4 * j;
        if (bb >= B)
            break;
        Tot tot = 0;
#pragma unroll
        for (int d = 0; d < ND; d++) {
            const Tot dsum = raw(d, bb);
            // digit weights: INT8 254^(2-d) (exact in int64), FP8 30^-d
            if constexpr (FP8)
                tot = tot + dsum * kF8Weight[d];
            else
                tot = tot + dsum * (Tot)(d == 0 ? kI8Base * kI8Base : (d == 1 ? kI8Base : 1));
        }
        st_global(E.y[t] + (size_t)bb * E.n[t], (float)((double)tot * ((double)E.sx[j] * sxw * (double)E.sw[t])));
    }
}

// Main GEMV kernel.
// Operands of one MFMA: A = 16 weight rows x STEP k (row r = lane % 16, k
// slice lane / 16), B = STEP k x 16 columns, where column c of column group nc
// is digit plane d = (16*nc + c) % ND of batch row b = (16*nc + c) / ND.
// A batch of <= 5 (INT8) or <= 4 (FP8) rows therefore needs one MFMA per
// weight tile: NC = ceil(batch * ND / 16) MFMAs in general.
//   INT8: STEP 64, 16 bytes per lane, v_mfma_i32_16x16x64_i8, exact int32.
//   FP8:  STEP 128, 32 bytes per lane, unit-scale v_mfma_scale_f32_16x16x128_f8f6f4.
// A block holds WAVES waves in WAVES/KS groups; a group owns one tile of
// 16*RT rows and its KS waves split K into contiguous slices.  A wave loads a
// burst of U MFMA steps (RT*U KiB of INT8 weights) with unconditional 16-byte
// loads, then runs its MFMAs.  With PF the next burst is loaded into a
// second register set before the MFMAs of the current one, so a wave keeps
// one burst in flight while it computes; without PF the latency is hidden by
// the other resident waves alone.  Epilogue: raw accumulators go through LDS
// one row tile at a time and the group's first wave sums slices and digit
// columns per output, weighting digit d by 254^(2-d) in exact int64 (INT8) or
// 30^-d in fp64 (FP8).
template <bool FP8, int RT, int U, int KS, int NC, int WAVES, bool PF>
__global__ __launch_bounds__(WAVES * 64) void k_gemv(const GemvSegs S, const uint8_t *__restrict__ dig,
                                                     const float *__restrict__ sx, int K, int Kp, int B)
{
    constexpr int ND = FP8 ? kF8Digits : kI8Digits;
    constexpr int STEP = FP8 ? 128 : 64;
    constexpr int NV = FP8 ? 2 : 1;          // 16-byte loads per lane per operand
    constexpr int GROUPS = WAVES / KS;
    using Tot = typename std::conditional<FP8, double, long long>::type;
    using Acc = typename std::conditional<FP8, v4f, v4i>::type;
    using Raw = typename std::conditional<FP8, float, int>::type;
    __shared__ Raw part[WAVES][16][NC * 16];

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int group = wave / KS, slice = wave % KS;
    const int r = lane & 15, g = lane >> 4;
    const int row0 = (blockIdx.x * GROUPS + group) * 16 * RT;
    const int nburst = Kp / (STEP * U);
    const int b0 = (nburst * slice) / KS, b1 = (nburst * (slice + 1)) / KS;
    EpiOps<RT> E;
    if (slice == 0)
        epi_load<RT>(E, S, sx, row0, r, g, B);

    Acc acc[RT][NC];
#pragma unroll
    for (int t = 0; t < RT; t++)
#pragma unroll
        for (int c = 0; c < NC; c++)
            acc[t][c] = Acc{0, 0, 0, 0};

    // Every load is unconditional and in bounds, so the loop carries no
    // branches and the next burst stays in flight across the MFMAs: rows past
    // the last read the last row and columns past the batch read plane 0
    // (neither is ever written out); k past K reads the row's last 16 bytes
    // against digits that are zero there.
    const uint8_t *wrow[RT];
#pragma unroll
    for (int t = 0; t < RT; t++) {
        int local;
        const int sg = seg_of(S, min(row0 + t * 16 + r, S.total - 1), &local);
        wrow[t] = seg_pick(S.w, sg) + (size_t)local * K;
    }
    const uint8_t *xcolp[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const int col = 16 * c + r, bb = col / ND, d = col % ND;
        xcolp[c] = dig + ((size_t)d * B + (bb < B ? bb : 0)) * Kp;
    }
    const int klast = K - 16;

    auto load = [&](int bi, v4i (&wd)[RT][U][NV], v4i (&xd)[NC][U][NV]) {
        const int kb = bi * STEP * U + g * 16 * NV;
#pragma unroll
        for (int t = 0; t < RT; t++)
#pragma unroll
            for (int u = 0; u < U; u++)
#pragma unroll
                for (int v = 0; v < NV; v++)
                    wd[t][u][v] = ld_global_v4(wrow[t] + min(kb + u * STEP + 16 * v, klast));
#pragma unroll
        for (int c = 0; c < NC; c++)
#pragma unroll
            for (int u = 0; u < U; u++)
#pragma unroll
                for (int v = 0; v < NV; v++)
                    xd[c][u][v] = *(const v4i *)(xcolp[c] + kb + u * STEP + 16 * v);
    };
    auto compute = [&](const v4i (&wd)[RT][U][NV], const v4i (&xd)[NC][U][NV]) {
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int t = 0; t < RT; t++)
#pragma unroll
                for (int c = 0; c < NC; c++) {
                    if constexpr (FP8) {
                        const v8i a = {wd[t][u][0][0], wd[t][u][0][1], wd[t][u][0][2], wd[t][u][0][3],
                                       wd[t][u][1][0], wd[t][u][1][1], wd[t][u][1][2], wd[t][u][1][3]};
                        const v8i bb = {xd[c][u][0][0], xd[c][u][0][1], xd[c][u][0][2], xd[c][u][0][3],
                                        xd[c][u][1][0], xd[c][u][1][1], xd[c][u][1][2], xd[c][u][1][3]};
                        acc[t][c] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, bb, acc[t][c], 0, 0, 0,
                                                                                     127, 0, 127);
                    } else {
                        acc[t][c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wd[t][u][0], xd[c][u][0], acc[t][c],
                                                                          0, 0, 0);
                    }
                }
    };
    if constexpr (PF) {
        v4i wa[RT][U][NV], xa[NC][U][NV], wb[RT][U][NV], xb[NC][U][NV];
        if (b0 < b1)
            load(b0, wa, xa);
        for (int bi = b0; bi < b1; bi += 2) {
            if (bi + 1 < b1)
                load(bi + 1, wb, xb);
            compute(wa, xa);
            if (bi + 1 >= b1)
                break;
            if (bi + 2 < b1)
                load(bi + 2, wa, xa);
            compute(wb, xb);
        }
    } else {
        v4i wv[RT][U][NV], xv[NC][U][NV];
        for (int bi = b0; bi < b1; bi++) {
            load(bi, wv, xv);
            compute(wv, xv);
        }
    }

    // C layout of a 16x16 MFMA: lane holds rows 4*(lane/16)+j of column lane%16.
    // One row tile at a time through LDS: slices and digit columns are summed
    // per output by the group's first wave.
#pragma unroll
    for (int t = 0; t < RT; t++) {
        if (t > 0)
            __syncthreads();
#pragma unroll
        for (int c = 0; c < NC; c++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                part[wave][4 * g + j][16 * c + r] = acc[t][c][j];
        __syncthreads();
        if (slice == 0)
            epi_store<FP8, RT>(E, t, g, B, [&](int d, int bb) {
                Tot dsum = 0;
#pragma unroll
                for (int sl = 0; sl < KS; sl++)
                    dsum += (Tot)part[group * KS + sl][r][bb * ND + d];
                return dsum;
            });
    }
}

// Streaming GEMV with the weights and the digit planes moved HBM -> LDS by
// the direct-to-LDS loads of gfx950 (global_load_lds_dwordx4), P stages deep,
// so the bytes in flight sit in LDS instead of VGPRs.  A block is WAVES waves
// (one or two per SIMD); wave w owns RT row tiles of 16 rows over the whole of K.
// A stage is 128 k-bytes: per row tile 2 KB of weights (two wave-wide loads,
// lane l writing LDS bytes [16l, 16l+16) of each, and later reading exactly
// those back as its MFMA A operand) in a ring private to the wave, and
// NC*2 KB of digit planes in a ring shared by the block.  Digit load j covers
// column group j/2 and 16-byte pieces 4*(j%2)..+3 of the stage, lane l
// carrying column 16*(j/2) + l%16 and piece 4*(j%2) + l/16, so that each
// 16-lane group of a B-operand read touches 256 contiguous bytes.  The
// block's 2*NC digit loads are spread over its waves (DI per wave; a wave
// past the last one reloads piece 0 into a spare 1 KB, keeping the per-stage
// load count uniform for the wait counts).
// Iteration s: wait for this wave's loads of stage s, barrier (all waves'
// loads of stage s are in LDS and every wave is done with stage s-1), issue
// stage s+P-1 into the slot stage s-1 used, run stage s's MFMAs.
template <bool FP8, int RT, int NC, int P, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void k_gemv_dma(const GemvSegs S, const uint8_t *__restrict__ dig,
                                                         const float *__restrict__ sx, int K, int Kp, int B)
{
    constexpr int ND = FP8 ? kF8Digits : kI8Digits;
    constexpr int COLS = NC * 16;
    constexpr int WI = 2 * RT;                       // weight loads per wave per stage
    constexpr int NDL = 2 * NC;                      // digit loads per block per stage
    constexpr int DI = (NDL + WAVES - 1) / WAVES;    // digit loads per wave per stage
    constexpr int PER = WI + DI;
    constexpr int WRING = WAVES * P * WI * 1024;
    constexpr int DRING = P * NDL * 1024;
    constexpr int PART = WAVES * 16 * COLS * 4;
    constexpr int LDS_BYTES = (WRING + DRING + 1024) > PART ? (WRING + DRING + 1024) : PART;
    static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
    static_assert(P >= 2 && (P - 2) * PER < 64, "stages");
    using Tot = typename std::conditional<FP8, double, long long>::type;
    using Acc = typename std::conditional<FP8, v4f, v4i>::type;
    using Raw = typename std::conditional<FP8, float, int>::type;
    __shared__ __align__(1024) uint8_t lds[LDS_BYTES];
    uint8_t *wring = lds, *dring = lds + WRING, *spare = lds + WRING + DRING;

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = lane & 15, g = lane >> 4;
    const int row0 = (blockIdx.x * WAVES + wave) * 16 * RT;
    const int nst = Kp / 128;
    EpiOps<RT> E;
    epi_load<RT>(E, S, sx, row0, r, g, B);

    Acc acc[RT][NC];
#pragma unroll
    for (int t = 0; t < RT; t++)
#pragma unroll
        for (int c = 0; c < NC; c++)
            acc[t][c] = Acc{0, 0, 0, 0};

    // per-lane sources: weight rows (rows past the end read the last row)
    // and digit columns (columns past the batch read plane 0 of row 0)
    const uint8_t *wrow[RT];
#pragma unroll
    for (int t = 0; t < RT; t++) {
        int local;
        const int sg = seg_of(S, min(row0 + t * 16 + r, S.total - 1), &local);
        wrow[t] = seg_pick(S.w, sg) + (size_t)local * K;
    }
    const int klast = K - 16;
    // weight load v of a tile: FP8 bytes 32g + 16v (one MFMA step, two loads);
    // INT8 bytes 64v + 16g (MFMA step v)
    const int woff0 = FP8 ? 32 * g : 16 * g, woff1 = FP8 ? 32 * g + 16 : 64 + 16 * g;
    const uint8_t *dsrc[DI];
    uint8_t *ddst[DI];
#pragma unroll
    for (int i = 0; i < DI; i++) {
        const int j = wave * DI + i;
        const int jj = j < NDL ? j : 0;
        const int col = 16 * (jj / 2) + r, q = 4 * (jj % 2) + g;
        const int bb = col / ND, d = col % ND;
        dsrc[i] = dig + ((size_t)d * B + (bb < B ? bb : 0)) * Kp + 16 * q;
        ddst[i] = j < NDL ? dring + j * 1024 : spare;
    }

    auto issue = [&](int st) {
        const int slot = st % P;
        uint8_t *wbase = wring + ((wave * P + slot) * WI) * 1024;
#pragma unroll
        for (int t = 0; t < RT; t++) {
            __builtin_amdgcn_global_load_lds((const void *)(wrow[t] + min(st * 128 + woff0, klast)),
                                             (lds_void *)(wbase + (2 * t) * 1024), 16, 0, 0);
            __builtin_amdgcn_global_load_lds((const void *)(wrow[t] + min(st * 128 + woff1, klast)),
                                             (lds_void *)(wbase + (2 * t + 1) * 1024), 16, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < DI; i++)
            __builtin_amdgcn_global_load_lds((const void *)(dsrc[i] + (size_t)st * 128),
                                             (lds_void *)(ddst[i] == spare ? spare : ddst[i] + slot * NDL * 1024),
                                             16, 0, 0);
        // the wait counts assume every load of stage st is issued before any
        // load of a later stage: keep the compiler from interleaving stages
        asm volatile("" ::: "memory");
    };
    auto compute = [&](int st) {
        const int slot = st % P;
        const uint8_t *wbase = wring + ((wave * P + slot) * WI) * 1024 + lane * 16;
        const uint8_t *dbase = dring + slot * NDL * 1024;
        if constexpr (FP8) {
            v8i a[RT];
#pragma unroll
            for (int t = 0; t < RT; t++) {
                const v4i a0 = *(const v4i *)(wbase + (2 * t) * 1024), a1 = *(const v4i *)(wbase + (2 * t + 1) * 1024);
                a[t] = v8i{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
            }
#pragma unroll
            for (int c = 0; c < NC; c++) {
                // pieces 2g and 2g+1 of column 16c + r: load 2c + g/2, lanes r + 16*((2g) % 4) and +16
                const uint8_t *xp = dbase + (2 * c + (g >> 1)) * 1024 + (r + 16 * ((2 * g) & 3)) * 16;
                const v4i b0 = *(const v4i *)xp, b1 = *(const v4i *)(xp + 256);
                const v8i bb = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
#pragma unroll
                for (int t = 0; t < RT; t++)
                    acc[t][c] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[t], bb, acc[t][c], 0, 0, 0, 127,
                                                                                 0, 127);
            }
        } else {
#pragma unroll
            for (int u = 0; u < 2; u++) {
                v4i a[RT];
#pragma unroll
                for (int t = 0; t < RT; t++)
                    a[t] = *(const v4i *)(wbase + (2 * t + u) * 1024);
#pragma unroll
                for (int c = 0; c < NC; c++) {
                    const v4i bb = *(const v4i *)(dbase + (2 * c + u) * 1024 + lane * 16);
#pragma unroll
                    for (int t = 0; t < RT; t++)
                        acc[t][c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t], bb, acc[t][c], 0, 0, 0);
                }
            }
        }
    };

#pragma unroll
    for (int st = 0; st < P - 1; st++)
        if (st < nst)
            issue(st);
    for (int st = 0; st < nst; st++) {
        if (st + P - 2 < nst)
            stage_barrier<(P - 2) * PER>();
        else
            stage_barrier<0>();
        if (st + P - 1 < nst)
            issue(st + P - 1);
        compute(st);
    }
    wait_vmcnt<0>();
    __syncthreads();

    // epilogue: each wave combines the digit columns of its own rows
    Raw(*part)[16][COLS] = (Raw(*)[16][COLS])lds;
#pragma unroll
    for (int t = 0; t < RT; t++) {
        if (t > 0)
            __syncthreads();
#pragma unroll
        for (int c = 0; c < NC; c++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                part[wave][4 * g + j][16 * c + r] = acc[t][c][j];
        __syncthreads();
        epi_store<FP8, RT>(E, t, g, B, [&](int d, int bb) { return (Tot)part[wave][r][bb * ND + d]; });
    }
}

// Partial sums of split-K launches, [ks][b][row]: the digit-combined sum of
// each K range before any scale (exact integers for INT8), added up in K
// order and scaled by a second launch (k_gemv_part_sum), so that a split
// GEMV rounds once, like an unsplit one.  Shared by every launch on the
// device, so split-K GEMVs on one device must not run concurrently (one
// stream).
constexpr size_t kGemvPartFloats = (size_t)1 << 20;   // entries (8 MiB)
__device__ double g_gemv_part[kGemvPartFloats];

// Streaming GEMV for many rows (the lm_head) with the digit planes resident in
// LDS one K-slice at a time.
// Operand roles are the transpose of k_gemv's: A = one digit plane (16 batch
// rows x 128 k; lane (r, g) holds batch row r, k bytes 32g .. 32g+31 for FP8,
// 64v + 16g .. +15 for the two INT8 sub-steps v), B = 16 weight rows (lane
// (r, g) holds row r at the same k).  A lane's accumulator j is then the sum
// of batch row 4g + j for weight row r, so it holds every digit plane of its
// own outputs and recombines them in registers: no LDS epilogue.
// A block of WAVES waves owns 16*RT*WAVES rows over the whole of K.  K is cut
// into slices of KSL bytes; the digits of a slice (ND planes x 16 batch rows x
// KSL, 2 KB per plane and 128-byte step, laid out [piece p][batch row][16
// bytes] so that each 16-lane read is one 256-byte run) are moved HBM -> LDS
// once per block by direct-to-LDS loads, double buffered, so a block crosses
// one barrier per slice instead of one per stage.  A wave streams its weights
// into a register ring of D stages; a stage is one row tile over SB steps of
// 128 k, i.e. 16 rows x 128*SB contiguous bytes each.  Stage order: slice,
// then tile, then step; the ring runs across tile and slice boundaries.
template <bool FP8, int RT, int SB, int KSL, int D, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void k_gemv_slab(const GemvSegs S, const uint8_t *__restrict__ dig,
                                                          const float *__restrict__ sx, int K, int Kp, int B,
                                                          int nsl)
{
    constexpr int ND = FP8 ? kF8Digits : kI8Digits;
    constexpr int STEPS = KSL / 128;                 // 128-k steps per slice
    constexpr int SPT = STEPS / SB;                  // stages per tile per slice
    constexpr int NST = RT * SPT;                    // stages per slice per wave
    constexpr int WL = 2 * SB;                       // weight loads per stage
    constexpr int SLB = ND * STEPS * 2048;           // LDS bytes per slice
    constexpr int NDMA = ND * STEPS * 2;             // 1 KB loads per slice
    constexpr int DI = NDMA / WAVES;                 // of them per wave
    static_assert(STEPS % SB == 0 && NST % D == 0 && D >= 2 && D <= NST, "stage ring");
    static_assert(NDMA % WAVES == 0, "slice loads split evenly over the waves");
    static_assert(2 * SLB <= 160 * 1024, "LDS budget");
    static_assert((D - 1) * WL < 64, "vmcnt");
    using Acc = typename std::conditional<FP8, v4f, v4i>::type;
    __shared__ __align__(1024) uint8_t lds[2 * SLB];

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = lane & 15, g = lane >> 4;
    const int row0 = (blockIdx.x * WAVES + wave) * 16 * RT;
    // blockIdx.y = ks: this block covers slices ks*nsl .. ks*nsl + nsl-1 of K
    const int ks = blockIdx.y, ksplit = gridDim.y;

    Acc acc[RT][ND];
#pragma unroll
    for (int t = 0; t < RT; t++)
#pragma unroll
        for (int d = 0; d < ND; d++)
            acc[t][d] = Acc{0, 0, 0, 0};

    const uint8_t *wrow[RT];
#pragma unroll
    for (int t = 0; t < RT; t++) {
        int local;
        const int sg = seg_of(S, min(row0 + t * 16 + r, S.total - 1), &local);
        wrow[t] = seg_pick(S.w, sg) + (size_t)local * K;
    }
    const int klast = K - 16;
    const int woff0 = FP8 ? 32 * g : 16 * g, woff1 = FP8 ? 32 * g + 16 : 64 + 16 * g;

    // epilogue operands, loaded up front and without branches (rows and
    // batch rows past the end read the last one and are masked): fetched
    // after the last weight stage, their loads would add a few microseconds
    // to every block
    float e_sw[RT], e_sx[4];
    float *e_y[RT];
    int e_n[RT];
#pragma unroll
    for (int t = 0; t < RT; t++) {
        const int row = row0 + t * 16 + r;
        const bool in = row < S.total;
        int local;
        const int sg = seg_of(S, in ? row : S.total - 1, &local);
        e_sw[t] = ld_global(seg_pick(S.sw, sg) + local);
        e_y[t] = in ? seg_pick(S.y, sg) + local : nullptr;
        e_n[t] = seg_pick(S.n, sg);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float v = ld_global(sx + min(4 * g + j, B - 1));
        e_sx[j] = 4 * g + j < B ? v : 0.0f;
    }

    // slice loads: load j of a slice carries plane d, step st, half h; lane
    // l brings batch row l % 16 (clamped to the batch), piece l / 16 + 4h
    const uint8_t *dsrc[DI];
    int ddst[DI];
#pragma unroll
    for (int i = 0; i < DI; i++) {
        const int j = wave * DI + i;
        const int d = j / (STEPS * 2), st = (j / 2) % STEPS, h = j % 2;
        const int b = min(r, B - 1);
        dsrc[i] = dig + ((size_t)d * B + b) * Kp + st * 128 + 16 * (g + 4 * h);
        ddst[i] = (d * STEPS + st) * 2048 + h * 1024;
    }
    // Blocks start at different slices (slice s of block b covers k bytes
    // KSL * ((s + b) mod nsl) ..), so that at any moment the blocks read
    // spread-out k ranges of their rows rather than all the same one.
    const int sk0 = blockIdx.x % nsl;
    auto kslice = [&](int s) { return (ks * nsl + (s + sk0 < nsl ? s + sk0 : s + sk0 - nsl)) * KSL; };
    auto issue_slice = [&](int s) {
        uint8_t *buf = lds + (s & 1) * SLB;
        const int kb = kslice(s);
#pragma unroll
        for (int i = 0; i < DI; i++)
            __builtin_amdgcn_global_load_lds((const void *)(dsrc[i] + kb), (lds_void *)(buf + ddst[i]), 16, 0, 0);
        asm volatile("" ::: "memory");
    };

    // A stage's weights, one 32-byte MFMA operand per step: FP8 bytes 32g ..
    // 32g+31 of the step, INT8 bytes 16g .. +15 (low half) and 64+16g .. +15
    // (high half).  Held as 8-dword vectors so each operand sits in
    // consecutive registers from the load on.
    v8i wr[D][SB];
    // weights of stage i (tile i / SPT, step group i % SPT) of slice s
    auto issue = [&](int s, int i, v8i (&w)[SB]) {
        const int t = i / SPT, q = i % SPT;
        const int kb = kslice(s) + q * SB * 128;
#pragma unroll
        for (int u = 0; u < SB; u++) {
            const v4i lo = ld_global_v4(wrow[t] + min(kb + u * 128 + woff0, klast));
            const v4i hi = ld_global_v4(wrow[t] + min(kb + u * 128 + woff1, klast));
            w[u] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        }
        asm volatile("" ::: "memory");
    };
    // stage i of slice s, digits from LDS buffer s & 1
    auto compute = [&](const v8i (&w)[SB], int i, int s) {
        const int t = i / SPT, q = i % SPT;
        const uint8_t *buf = lds + (s & 1) * SLB;
#pragma unroll
        for (int u = 0; u < SB; u++) {
            const int st = q * SB + u;
#pragma unroll
            for (int d = 0; d < ND; d++) {
                const uint8_t *pl = buf + (d * STEPS + st) * 2048 + r * 16;
                if constexpr (FP8) {
                    const v4i a0 = *(const v4i *)(pl + (2 * g) * 256), a1 = *(const v4i *)(pl + (2 * g + 1) * 256);
                    const v8i a = __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7);
                    acc[t][d] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, w[u], acc[t][d], 0, 0, 0, 127, 0,
                                                                                 127);
                } else {
                    const v4i a0 = *(const v4i *)(pl + g * 256), a1 = *(const v4i *)(pl + (4 + g) * 256);
                    const v4i w0 = __builtin_shufflevector(w[u], w[u], 0, 1, 2, 3);
                    const v4i w1 = __builtin_shufflevector(w[u], w[u], 4, 5, 6, 7);
                    acc[t][d] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, w0, acc[t][d], 0, 0, 0);
                    acc[t][d] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, w1, acc[t][d], 0, 0, 0);
                }
            }
            // keep each step's LDS reads next to its matrix instructions:
            // merging the identical reads of different tiles, or gathering a
            // whole slice's reads ahead of its matrix instructions, would not
            // fit the registers (the empty asm ties the accumulators here)
#pragma unroll
            for (int d = 0; d < ND; d++)
                asm volatile("" : "+v"(acc[t][d]));
            asm volatile("" ::: "memory");
        }
    };
    // one slice: stage i computes while stage i + D - 1 (of this slice or
    // the next) is issued; the ring slot of a stage is its number mod D,
    // static because NST is a multiple of D.  The last slice issues its own
    // last stage again in place of the stages past the end (same addresses
    // as the load just before, served by the L2), so that every slice runs
    // the same code and keeps the same number of loads in flight.
    auto slice = [&](int s, int snext) {
#pragma unroll
        for (int i = 0; i < NST; i++) {
            const int ii = i + D - 1;
            if (ii < NST)
                issue(s, ii, wr[ii % D]);
            else if (snext > s)
                issue(snext, ii - NST, wr[ii % D]);
            else
                issue(s, NST - 1, wr[ii % D]);
            compute(wr[i % D], i, s);
        }
    };

    issue_slice(0);
    if (nsl > 1)
        issue_slice(1);
#pragma unroll
    for (int j = 0; j < D - 1; j++)
        issue(0, j, wr[j]);
    // Slice s is in LDS once this wave's loads older than the D-1 weight
    // stages in flight have landed: at s = 0 everything but slice 1's loads
    // and those stages; later, slice s's loads were issued a whole slice
    // (NST >= D stages) ago.  Every wave is then done with slice s-1, whose
    // buffer takes slice s+1.
    if (nsl > 1)
        stage_barrier<DI + (D - 1) * WL>();
    else
        stage_barrier<(D - 1) * WL>();
    for (int s = 0; s < nsl; s++) {
        if (s > 0) {
            stage_barrier<(D - 1) * WL>();
            if (s + 1 < nsl)
                issue_slice(s + 1);
        }
        slice(s, min(s + 1, nsl - 1));
    }
    wait_vmcnt<0>();

    constexpr double kI8W[3] = {(double)(kI8Base * kI8Base), (double)kI8Base, 1.0};
    const double sxw = FP8 ? 1.0 : 1.0 / (double)(kI8Base * kI8Base);
    // one K range's share of y[b][row]; with a K split it goes to the
    // partial buffer [ks][b][row] instead of y
#pragma unroll
    for (int t = 0; t < RT; t++) {
        if (!e_y[t])
            continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int b = 4 * g + j;
            if (b >= B)
                break;
            double tot = 0.0;
            if constexpr (FP8) {
#pragma unroll
                for (int d = 0; d < ND; d++)
                    tot += (double)acc[t][d][j] * kF8Weight[d];
            } else {
                long long it = 0;
#pragma unroll
                for (int d = 0; d < ND; d++)
                    it += (long long)acc[t][d][j] * (long long)kI8W[d];
                tot = (double)it;
            }
            if (ksplit == 1)
                st_global(e_y[t] + (size_t)b * e_n[t], (float)(tot * ((double)e_sx[j] * sxw * (double)e_sw[t])));
            else
                g_gemv_part[((size_t)ks * B + b) * S.total + row0 + t * 16 + r] = tot;
        }
    }
}

// y[b][row] = (sum over the K ranges of a split launch, in K order) times the
// scales, as the unsplit epilogue forms it (sxw: 254^-2 for INT8, 1 for FP8).
__global__ __launch_bounds__(256) void k_gemv_part_sum(const GemvSegs S, const float *__restrict__ sx, double sxw,
                                                       int B, int ksplit)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= B * S.total)
        return;
    const int b = i / S.total, row = i % S.total;
    double tot = 0.0;
    for (int q = 0; q < ksplit; q++)
        tot += g_gemv_part[((size_t)q * B + b) * S.total + row];
    int local;
    const int sg = seg_of(S, row, &local);
    const float sw = seg_pick(S.sw, sg)[local];
    st_global(seg_pick(S.y, sg) + (size_t)b * seg_pick(S.n, sg) + local,
              (float)(tot * ((double)sx[b] * sxw * (double)sw)));
}

// Block-cooperative streaming GEMV for many rows.
// The 8 waves of a block read the same 16-row tile at the same time, wave w
// taking its own SPW 128-byte steps of k, so that a block streams whole
// 16-row x K regions (16 KiB .. 64 KiB of consecutive rows) one after
// another: the DRAM pages of a region are read together, with every load
// instruction covering whole 128-byte lines of 8 rows and the non-temporal
// hint.  Loads go straight to LDS (global_load_lds), into a ring of D stages
// per wave (a stage is 16 rows x 128 bytes); the matrix operands are read
// back from LDS in the MFMA lane layout.  A wave's k range of the activation
// digits stays in registers for the whole launch (A operand: batch row r,
// k bytes 32g .. 32g+31 of the step for FP8; 16g .. and 64+16g .. for INT8),
// so the block never re-reads them.  At the end of a tile each wave combines
// its digit sums into one partial per (row, batch row) -- exact int64 for
// INT8, fp64 for FP8 -- and after a barrier every wave adds up 32 of the
// tile's 256 outputs over the 8 partials, in wave order, and writes y (or
// the split-K partial).  Partials are double buffered (tile parity), with a
// third buffer for tile 0, which is added up after tile 1's barrier.
// Blocks cover tpb consecutive tiles; blockIdx.y selects a k range of a
// split launch.
constexpr int kCoopWaves = 8;
constexpr int kCoopMaxTiles = 64;                // tiles per block (their weight scales sit in LDS)
constexpr int kCoopHalf = 1040;                  // 8 rows x 128 bytes, + 16-byte pad
constexpr int kCoopSlot = 2 * kCoopHalf;         // one stage: 16 rows x 128 bytes

// LDS position of 16-byte chunk c of row rr (0..7 within a half): rows two
// apart rotate their chunks by two, so that the 16 rows of an operand read
// land in 16 different 16-byte bank groups (the pad shifts the second half)
__device__ __forceinline__ int coop_pos(int c, int rr) { return (c + 2 * (rr >> 1)) & 7; }

// LDS reads of this wave have completed, and the barrier leaves loads in
// flight alone (a workgroup barrier from the language would drain them)
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((63 & 15) | ((63 >> 4) << 14) | (7 << 4) | (0 << 8));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <bool FP8, int SPW, int D>
__global__ __launch_bounds__(kCoopWaves * 64) void k_gemv_coop(const GemvSegs S, const uint8_t *__restrict__ dig,
                                                               const float *__restrict__ sx, int K, int Kp, int B,
                                                               int tpb)
{
    constexpr int ND = FP8 ? kF8Digits : kI8Digits;
    static_assert(D >= 2 && (D - 1) * 2 < 64, "ring");
    using Acc = typename std::conditional<FP8, v4f, v4i>::type;
    using Tot = typename std::conditional<FP8, double, long long>::type;
    __shared__ __align__(16) uint8_t ring[kCoopWaves * D * kCoopSlot];
    __shared__ __align__(16) Tot red[3][kCoopWaves][64][4];
    __shared__ float lsw[kCoopMaxTiles * 16];

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = lane & 15, g = lane >> 4;
    const int ks = blockIdx.y, ksplit = gridDim.y;
    const int ntile = (S.total + 15) >> 4;
    const int tile0 = blockIdx.x * tpb;
    const int nst = tpb * SPW;
    // first 128-byte step of k of this wave: the k ranges rotate with the
    // block, so that at the start the blocks' waves do not all read the same
    // digits at once
    const int step0 = (ks * kCoopWaves + ((wave + blockIdx.x) & (kCoopWaves - 1))) * SPW;
    const int klast = K - 16;
    uint8_t *myring = ring + wave * D * kCoopSlot;

    // stage i: tile i / SPW, step i % SPW, ring slot i % D; stages past the
    // end load the last one again (into a free slot) so that every
    // iteration keeps the same number of loads in flight
    const int drr = lane >> 3;
    const int dc = ((lane & 7) - 2 * (drr >> 1)) & 7;    // chunk this lane brings (inverse of coop_pos)
    auto issue = [&](int i) {
        const int ic = min(i, nst - 1);
        const int t = ic / SPW, q = ic - t * SPW;
        const int tile = min(tile0 + t, ntile - 1);
        const int kb = min((step0 + q) * 128 + 16 * dc, klast);
        uint8_t *dst = myring + (i % D) * kCoopSlot;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            int local;
            const int sg = seg_of(S, min(tile * 16 + 8 * h + drr, S.total - 1), &local);
            const uint8_t *src = seg_pick(S.w, sg) + (size_t)local * K + kb;
            __builtin_amdgcn_global_load_lds((const void *)src, (lds_void *)(dst + h * kCoopHalf), 16, 0, 2);
        }
        asm volatile("" ::: "memory");
    };
    // ring prologue first, so that weights stream while the digits load
#pragma unroll
    for (int j = 0; j < D - 1; j++)
        issue(j);

    // this wave's k range of the digits, kept for the whole launch
    v8i a[SPW][ND];
    {
        const int b = min(r, B - 1);
#pragma unroll
        for (int q = 0; q < SPW; q++)
#pragma unroll
            for (int d = 0; d < ND; d++) {
                const uint8_t *p = dig + ((size_t)d * B + b) * Kp + (size_t)(step0 + q) * 128;
                const v4i lo = ld_global_v4(p + (FP8 ? 32 * g : 16 * g));
                const v4i hi = ld_global_v4(p + (FP8 ? 32 * g + 16 : 64 + 16 * g));
                a[q][d] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
            }
    }
    // the output this lane adds up at the end of every tile (lanes < 32):
    // number o = 32 * wave + lane, held by lane o / 4 of each wave
    const int o_src = (32 * wave + lane) >> 2, o_j = lane & 3;
    const int o_r = o_src & 15, o_b = 4 * (o_src >> 4) + o_j;
    double o_sx = (double)ld_global(sx + min(o_b, B - 1)) * (FP8 ? 1.0 : 1.0 / (double)(kI8Base * kI8Base));
    // (every GEMV epilogue forms y = tot * ((sx * sxw) * sw) in fp64 and rounds once)
    // weight scales of the block's rows, staged in LDS before the loop: a
    // plain load inside it would make the compiler wait for every load in
    // flight (it cannot count plain loads apart from the ones into LDS);
    // the first tile's barrier publishes them
    for (int i = threadIdx.x; i < tpb * 16; i += kCoopWaves * 64) {
        int local;
        const int sg = seg_of(S, min(tile0 * 16 + i, S.total - 1), &local);
        lsw[i] = ld_global(seg_pick(S.sw, sg) + local);
    }
    // the batch scale converted here, not next to its first use in the loop
    // (where the compiler would wait for every load in flight first)
    asm volatile("" : "+v"(o_sx));

    Acc acc[ND];
#pragma unroll
    for (int d = 0; d < ND; d++)
        acc[d] = Acc{0, 0, 0, 0};
    const int rr = r & 7;
    const int roff = (r >> 3) * kCoopHalf + rr * 128;
    const int p0 = coop_pos(FP8 ? 2 * g : g, rr) * 16, p1 = coop_pos(FP8 ? 2 * g + 1 : 4 + g, rr) * 16;

    constexpr long long kI8W[3] = {(long long)kI8Base * kI8Base, (long long)kI8Base, 1};
    // the 256 outputs of tile t, 32 per wave: lane l < 32 of wave w adds up
    // output 32w + l (held by lane o / 4, batch row 4g + o % 4 of that lane)
    // over the 8 waves' partials in buffer buf, in wave order
    auto reduce_tile = [&](int t, int buf) {
        if (lane < 32) {
            Tot tot = 0;
#pragma unroll
            for (int w = 0; w < kCoopWaves; w++)
                tot += red[buf][w][o_src][o_j];
            const int row = (tile0 + t) * 16 + o_r;
            if (tile0 + t < ntile && row < S.total && o_b < B) {
                // y[b][local] of the row's segment, or the partial [ks][b][row]
                int local;
                const int sg = seg_of(S, row, &local);
                if (ksplit == 1)
                    st_global(seg_pick(S.y, sg) + (size_t)o_b * seg_pick(S.n, sg) + local,
                              (float)((double)tot * (o_sx * (double)lsw[t * 16 + o_r])));
                else
                    g_gemv_part[((size_t)ks * B + o_b) * S.total + row] = (double)tot;
            }
        }
    };
    for (int t = 0; t < tpb; t++) {
#pragma unroll
        for (int q = 0; q < SPW; q++) {
            const int i = t * SPW + q;
            // the slot refilled next was read by stage i - 1, whose reads
            // have returned (the matrix instructions used them)
            issue(i + D - 1);
            wait_vmcnt<(D - 1) * 2>();
            asm volatile("" ::: "memory");
            // operand reads as inline assembly: the compiler cannot tell the
            // slot apart from the ones still being filled, and would wait for
            // every load in flight before an LDS read it knows of
            const uint32_t base = (uint32_t)(uintptr_t)(myring + (i % D) * kCoopSlot + roff);
            v4i w0, w1;
            asm volatile("ds_read_b128 %0, %1" : "=v"(w0) : "v"(base + p0));
            asm volatile("ds_read_b128 %0, %1" : "=v"(w1) : "v"(base + p1));
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(w0), "+v"(w1));
#pragma unroll
            for (int d = 0; d < ND; d++) {
                if constexpr (FP8) {
                    const v8i w = __builtin_shufflevector(w0, w1, 0, 1, 2, 3, 4, 5, 6, 7);
                    acc[d] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[q][d], w, acc[d], 0, 0, 0, 127, 0,
                                                                              127);
                } else {
                    const v4i a0 = __builtin_shufflevector(a[q][d], a[q][d], 0, 1, 2, 3);
                    const v4i a1 = __builtin_shufflevector(a[q][d], a[q][d], 4, 5, 6, 7);
                    acc[d] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, w0, acc[d], 0, 0, 0);
                    acc[d] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, w1, acc[d], 0, 0, 0);
                }
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
        // this wave's share of the tile: digit sums combined per output.
        // Tile 0 goes to a third buffer and is added up together with tile
        // 1 after the second barrier: the waves start unevenly (each first
        // waits for its k range of the digits), and the first tile then
        // needs no barrier of its own.
        const int buf = t == 0 ? 2 : (t & 1);
        Tot *mine = &red[buf][wave][lane][0];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            Tot v = 0;
#pragma unroll
            for (int d = 0; d < ND; d++) {
                if constexpr (FP8)
                    v += (double)acc[d][j] * kF8Weight[d];
                else
                    v += (long long)acc[d][j] * kI8W[d];
            }
            mine[j] = v;
        }
#pragma unroll
        for (int d = 0; d < ND; d++)
            acc[d] = Acc{0, 0, 0, 0};
        if (t == 0 && tpb > 1)
            continue;
        lds_barrier();
        if (t == 1)
            reduce_tile(0, 2);
        reduce_tile(t, buf);
    }
    wait_vmcnt<0>();
}

template <bool FP8, int SPW, int D>
static void launch_coop(const GemvSegs &S, const uint8_t *dig, const float *sx, int k, int Kp, int batch, int ksplit,
                        int tpb, hipStream_t s)
{
    const int ntile = (S.total + 15) / 16;
    const int blocks = (ntile + tpb - 1) / tpb;
    hipLaunchKernelGGL((k_gemv_coop<FP8, SPW, D>), dim3(blocks, ksplit), dim3(kCoopWaves * 64), 0, s, S, dig, sx, k,
                       Kp, batch, tpb);
    if (ksplit > 1)
        hipLaunchKernelGGL(k_gemv_part_sum, dim3((batch * S.total + 255) / 256), dim3(256), 0, s, S, sx,
                           FP8 ? 1.0 : 1.0 / (double)(kI8Base * kI8Base), batch, ksplit);
}

template <bool FP8, int RT, int SB, int KSL, int D, int WAVES>
static void launch_slab(const GemvSegs &S, const uint8_t *dig, const float *sx, int k, int Kp, int batch, int ksplit,
                        hipStream_t s)
{
    const int blocks = (S.total + 16 * RT * WAVES - 1) / (16 * RT * WAVES);
    hipLaunchKernelGGL((k_gemv_slab<FP8, RT, SB, KSL, D, WAVES>), dim3(blocks, ksplit), dim3(WAVES * 64), 0, s, S,
                       dig, sx, k, Kp, batch, Kp / KSL / ksplit);
    if (ksplit > 1)
        hipLaunchKernelGGL(k_gemv_part_sum, dim3((batch * S.total + 255) / 256), dim3(256), 0, s, S, sx,
                           FP8 ? 1.0 : 1.0 / (double)(kI8Base * kI8Base), batch, ksplit);
}

template <bool FP8, int RT, int NC, int P, int WAVES>
static void launch_dma(const GemvSegs &S, const uint8_t *dig, const float *sx, int k, int Kp, int batch,
                       hipStream_t s)
{
    const int tiles = (S.total + 16 * RT - 1) / (16 * RT);
    const int blocks = (tiles + WAVES - 1) / WAVES;
    hipLaunchKernelGGL((k_gemv_dma<FP8, RT, NC, P, WAVES>), dim3(blocks), dim3(WAVES * 64), 0, s, S, dig, sx, k,
                       Kp, batch);
}

// Generic path for shapes the MFMA path does not take (k % 16 != 0, unaligned
// pointers, batch > 16): one block per output row, fp32 dot of the
// dequantized row, reduction through LDS.
template <bool FP8>
__global__ __launch_bounds__(256) void k_gemv_generic(float *y, const uint8_t *W, const float *sw,
                                                      const float *x, int N, int K, int B)
{
    __shared__ float red[4];
    const int row = blockIdx.x;
    const uint8_t *wr = W + (size_t)row * K;
    for (int b = 0; b < B; b++) {
        const float *xb = x + (size_t)b * K;
        float s = 0.0f;
        for (int k = threadIdx.x; k < K; k += blockDim.x) {
            float w;
            if (FP8) {
                const uint8_t c = wr[k];
                const int e = (c >> 3) & 0xF, m = c & 7;
                w = (e == 0) ? (float)m * (1.0f / 512.0f)
                             : __uint_as_float((uint32_t)(e + 120) << 23) * (1.0f + (float)m * 0.125f);
                w = (c & 0x80) ? -w : w;
            } else {
                w = (float)(int8_t)wr[k];
            }
            s = __fmaf_rn(w, xb[k], s);
        }
        s = wave_sum(s);
        if ((threadIdx.x & 63) == 0)
            red[threadIdx.x >> 6] = s;
        __syncthreads();
        if (threadIdx.x == 0)
            y[(size_t)b * N + row] = ((red[0] + red[1]) + (red[2] + red[3])) * sw[row];
        __syncthreads();
    }
}

int xdig_prepare(void *buf, const float *x, int k, int batch, bool fp8, hipStream_t s)
{
    const int Kp = (int)xdig_kp(k, fp8);
    uint8_t *dig = (uint8_t *)buf;
    const size_t dbytes = (size_t)xdig_layout(fp8).nd * batch * Kp;
    float *sx = (float *)(dig + ((dbytes + 255) & ~(size_t)255));
    const int chunks = (Kp + kPrepChunk - 1) / kPrepChunk;
    const dim3 grid(chunks, batch);
    // one load per thread and register slot: rows up to 16 chunks (16384 k)
    // in one round trip; longer rows by the two-pass kernel
    auto row = [&](auto f8) {
        constexpr bool F = decltype(f8)::value;
        if (chunks <= 1)
            hipLaunchKernelGGL((k_gemv_prep_row<F, 1>), grid, dim3(256), 0, s, x, k, Kp, batch, dig, sx);
        else if (chunks <= 2)
            hipLaunchKernelGGL((k_gemv_prep_row<F, 2>), grid, dim3(256), 0, s, x, k, Kp, batch, dig, sx);
        else if (chunks <= 4)
            hipLaunchKernelGGL((k_gemv_prep_row<F, 4>), grid, dim3(256), 0, s, x, k, Kp, batch, dig, sx);
        else if (chunks <= 8)
            hipLaunchKernelGGL((k_gemv_prep_row<F, 8>), grid, dim3(256), 0, s, x, k, Kp, batch, dig, sx);
        else if (chunks <= 16)
            hipLaunchKernelGGL((k_gemv_prep_row<F, 16>), grid, dim3(256), 0, s, x, k, Kp, batch, dig, sx);
        else
            hipLaunchKernelGGL(k_gemv_prep<F>, grid, dim3(256), 0, s, x, k, Kp, batch, dig, sx);
    };
    if (fp8)
        row(std::true_type{});
    else
        row(std::false_type{});
    BE42_LAUNCH_CHECK();
    return BE42_OK;
}

template <bool FP8, int RT, int U, int NC, int KS, int WAVES, bool PF>
static void launch_cfg(const GemvSegs &S, const uint8_t *dig, const float *sx, int k, int Kp, int batch,
                       hipStream_t s)
{
    static_assert(WAVES % KS == 0, "a row group is KS whole waves");
    constexpr int GROUPS = WAVES / KS;
    const int tiles = (S.total + 16 * RT - 1) / (16 * RT);
    const int blocks = (tiles + GROUPS - 1) / GROUPS;
    hipLaunchKernelGGL((k_gemv<FP8, RT, U, KS, NC, WAVES, PF>), dim3(blocks), dim3(WAVES * 64), 0, s, S, dig, sx, k,
                       Kp, batch);
}

// Launch shape per (dtype, column groups NC, rows n, k), measured on MI355X
// over the decode projections of configs[0] and configs[4] and the four
// configs[1] shapes at batch 1 / 4 / 8 / 16 (rows n count all segments of a
// launch).  RT row tiles of 16 per wave, U MFMA steps per burst, KS waves
// splitting K per row group, WAVES per block, PF register double buffering.
struct TileCfg {
    int rt, u, ks, waves, pf;
    int dma;        // 1: k_gemv_dma with u = pipeline stages (ks, pf unused); 3: k_gemv_slab
    int split = 1;  // k_gemv_slab: K ranges per row range
};
constexpr TileCfg dma_tile(int rt, int stages, int waves) { return TileCfg{rt, stages, 0, waves, 0, 1}; }
constexpr TileCfg slab_tile(int rt, int stages, int steps, int waves, int slice_steps, int split = 1)
{
    return TileCfg{rt, stages, steps, waves, slice_steps, 3, split};
}

// Split-K slab shape for n rows: 128 rows per range with 256-byte ring
// stages (or, past 8192 rows, 256 rows with 512-byte stages) and the largest
// split of the 512-byte slices that keeps the grid within 256 blocks and the
// partials within their buffer; split 0 if none.
static TileCfg split_slab_tile(int n, int k, int batch, bool fp8)
{
    const int rt = n > 8192 ? 2 : 1;
    const int ranges = (n + 128 * rt - 1) / (128 * rt);
    const int nsl = (int)(xdig_kp(k, fp8) / 512);
    for (int d = nsl; d >= 2; d--)
        if (nsl % d == 0 && ranges * d <= 256 && (size_t)d * batch * n <= kGemvPartFloats)
            return slab_tile(rt, 2, 2 * rt, 8, 4, d);
    return slab_tile(rt, 2, 2 * rt, 8, 4, 0);
}

static TileCfg pick_tile(bool fp8, int nc, int n, int k, int batch)
{
    // 3+ column groups (FP8 batch >= 9, INT8 batch >= 11) otherwise: the
    // LDS-resident digit slab kernel; many rows (k > 4096): one block of 8
    // waves x 4 row tiles per row range, each ring stage 16 rows x 512
    // contiguous bytes; long rows, or FP8 at 4096 .. 14336 rows: split K,
    // partials added by a second launch
    // the block-cooperative kernel when k splits into 8 wave ranges of at
    // most 4 steps (k <= 4096): many rows (the lm_head) at any batch,
    // 8193 .. 32768 rows at one column group (measured: 14336 x 4096 FP8
    // batch 1 -6%, INT8 batch 4 -16%), and past 4096 rows at 2-4 column
    // groups (measured against the other kernels at batch 4-16, with five
    // FP8 digit planes then: the 3B model's q/k/v (5120 x 3072) FP8 batch 4
    // 15.7 -> 9.4 us, INT8 batch 16 19.2 -> 10.6 us; gate/up (16384 x 3072)
    // FP8 batch 8 17.8 -> 15.7 us; 14336 x 4096 INT8 batch 16 19.6 ->
    // 17.5 us; with four planes FP8 batch 16 is 4 groups, and 14336 x 4096
    // runs 29.1 -> 26.7 us here instead of on the split slab kernel).
    if (n > 32768 || (n > 8192 && nc < 3) || (n > 4096 && nc >= 2 && nc <= 4)) {
        const int steps = (int)(xdig_kp(k, fp8) / 128);
        if (steps % kCoopWaves == 0 && steps / kCoopWaves <= 4)
            return TileCfg{0, 6, 0, kCoopWaves, 0, 4, 1};
    }
    if (nc >= 3) {
        if (n > 32768)
            return slab_tile(4, 2, 4, 8, 4);
        if (k >= 8192 || (fp8 && n >= 4096 && n <= 14336)) {
            const TileCfg c = split_slab_tile(n, k, batch, fp8);
            if (c.split > 1)
                return c;
        }
    }
    if (fp8) {
        if (nc == 1) {
            if (n <= 4096)
                return k <= 4096 ? TileCfg{1, 4, 4, 4, 1} : TileCfg{1, 2, 8, 8, 0};
            if (n <= 8192)
                return {2, 2, 8, 8, 1};
            return n <= 32768 ? TileCfg{2, 1, 4, 8, 1} : TileCfg{2, 1, 4, 4, 1};
        }
        if (nc == 2) {
            if (n <= 4096)
                return k <= 4096 ? TileCfg{1, 1, 8, 8, 1} : TileCfg{1, 1, 8, 8, 0};
            return n <= 8192 ? TileCfg{2, 4, 2, 4, 0} : dma_tile(1, 4, 4);
        }
        if (nc == 3) {
            if (n <= 4096)
                return {1, 1, 4, 4, 1};
            if (n <= 8192)
                return {2, 2, 4, 4, 0};
            return n <= 32768 ? dma_tile(1, 4, 4) : dma_tile(2, 3, 8);
        }
        if (n <= 4096)
            return k <= 4096 ? TileCfg{1, 1, 4, 4, 0} : TileCfg{1, 2, 4, 4, 1};
        if (n <= 8192)
            return {4, 2, 4, 4, 0};
        return n <= 32768 ? dma_tile(1, 4, 4) : dma_tile(2, 3, 4);
    }
    if (nc == 1) {
        if (n <= 2048)
            return k <= 1024 ? TileCfg{1, 8, 8, 8, 1} : TileCfg{1, 4, 8, 8, 1};
        if (n <= 4096)
            return k <= 4096 ? TileCfg{1, 8, 4, 4, 1} : TileCfg{1, 2, 8, 8, 1};
        return n <= 32768 ? TileCfg{2, 2, 4, 4, 0} : TileCfg{2, 2, 4, 4, 1};
    }
    if (n <= 4096)
        return k <= 4096 ? TileCfg{1, 2, 4, 4, 0} : TileCfg{1, 2, 8, 8, 1};
    if (n <= 8192)
        return {4, 2, 4, 4, 1};
    return n <= 32768 ? dma_tile(1, 5, 4) : dma_tile(1, 3, 8);
}

#define BE42_TILE(RT, U, KS, W, PF)                                                                                \
    if (!c.dma && c.rt == RT && c.u == U && c.ks == KS && c.waves == W && c.pf == PF)                            \
        return launch_cfg<FP8, RT, U, NC, KS, W, PF>(S, dig, sx, k, Kp, batch, s), true;
#define BE42_DMA(RT, P, W)                                                                                         \
    if (c.dma == 1 && c.rt == RT && c.u == P && c.waves == W)                                                     \
        return launch_dma<FP8, RT, NC, P, W>(S, dig, sx, k, Kp, batch, s), true;

// The shapes pick_tile returns for each (dtype, NC); false if c is not one.
template <bool FP8, int NC>
static bool launch_tile(const TileCfg &c, const GemvSegs &S, const uint8_t *dig, const float *sx, int k, int Kp,
                        int batch, hipStream_t s)
{
    if constexpr (FP8 && NC == 1) {
        BE42_TILE(1, 4, 4, 4, 1) BE42_TILE(1, 2, 8, 8, 0) BE42_TILE(2, 2, 8, 8, 1) BE42_TILE(2, 1, 4, 8, 1)
        BE42_TILE(2, 1, 4, 4, 1)
    } else if constexpr (FP8 && NC == 2) {
        BE42_TILE(1, 1, 8, 8, 1) BE42_TILE(1, 1, 8, 8, 0) BE42_TILE(2, 4, 2, 4, 0) BE42_DMA(1, 4, 4)
    } else if constexpr (FP8 && NC == 3) {
        BE42_TILE(1, 1, 4, 4, 1) BE42_TILE(2, 2, 4, 4, 0) BE42_DMA(1, 4, 4) BE42_DMA(2, 3, 8)
    } else if constexpr (FP8) {
        BE42_TILE(1, 1, 4, 4, 0) BE42_TILE(1, 2, 4, 4, 1) BE42_TILE(4, 2, 4, 4, 0) BE42_DMA(1, 4, 4)
        BE42_DMA(2, 3, 4)
    } else if constexpr (NC == 1) {
        BE42_TILE(1, 8, 8, 8, 1) BE42_TILE(1, 4, 8, 8, 1) BE42_TILE(1, 8, 4, 4, 1) BE42_TILE(1, 2, 8, 8, 1)
        BE42_TILE(2, 2, 4, 4, 0) BE42_TILE(2, 2, 4, 4, 1)
    } else {
        BE42_TILE(1, 2, 4, 4, 0) BE42_TILE(1, 2, 8, 8, 1) BE42_TILE(4, 2, 4, 4, 1) BE42_DMA(1, 5, 4)
        BE42_DMA(1, 3, 8)
    }
    return false;
}
#undef BE42_TILE
#undef BE42_DMA

// NC = ceil(batch * digits / 16) MFMA column groups.
template <bool FP8>
static int segs_launch(const GemvSegs &S, const void *buf, int k, int batch, hipStream_t s)
{
    const int Kp = (int)xdig_kp(k, FP8);
    const uint8_t *dig = (const uint8_t *)buf;
    const size_t dbytes = (size_t)xdig_layout(FP8).nd * batch * Kp;
    const float *sx = (const float *)(dig + ((dbytes + 255) & ~(size_t)255));
    const int nc = (batch * (FP8 ? kF8Digits : kI8Digits) + 15) / 16;
    TileCfg c = pick_tile(FP8, nc, S.total, k, batch);
    // BE42_GEMV_TILE = "kind,rt,u,ks,waves,pf[,split]" forces one launch
    // shape (kind 0 register path, 1 k_gemv_dma, 3 k_gemv_slab with u = ring
    // stages, ks = steps per stage, pf = steps per slice, split = K ranges;
    // 4 k_gemv_coop with pf = tiles per block, 0 for the default)
    if (const char *e = getenv("BE42_GEMV_TILE")) {
        TileCfg f{};
        const int got = sscanf(e, "%d,%d,%d,%d,%d,%d,%d", &f.dma, &f.rt, &f.u, &f.ks, &f.waves, &f.pf, &f.split);
        if (got == 6)
            f.split = 1;
        if (got >= 6)
            c = f;
    }
    bool ok = false;
    if (c.dma == 4) {
        const int steps = Kp / 128;
        BE42_CHECK(c.split >= 1 && steps % (kCoopWaves * c.split) == 0 && steps / (kCoopWaves * c.split) <= 4 &&
                       (c.split == 1 || (size_t)c.split * batch * S.total <= kGemvPartFloats),
                   "be42 gemv: cooperative split %d does not fit k=%d rows=%d batch=%d", c.split, k, S.total, batch);
        const int spw = steps / (kCoopWaves * c.split);
        const int ntile = (S.total + 15) / 16;
        // tiles per block: about 256 blocks in all, unless forced (pf)
        const int tpb = c.pf > 0 ? c.pf : std::max(1, (ntile * c.split + 255) / 256);
        BE42_CHECK(tpb <= kCoopMaxTiles, "be42 gemv: %d tiles per block exceed %d (rows=%d)", tpb, kCoopMaxTiles,
                   S.total);
        switch (spw) {
        case 1: launch_coop<FP8, 1, 6>(S, dig, sx, k, Kp, batch, c.split, tpb, s); break;
        case 2: launch_coop<FP8, 2, 6>(S, dig, sx, k, Kp, batch, c.split, tpb, s); break;
        case 3: launch_coop<FP8, 3, 6>(S, dig, sx, k, Kp, batch, c.split, tpb, s); break;
        default: launch_coop<FP8, 4, 6>(S, dig, sx, k, Kp, batch, c.split, tpb, s); break;
        }
        BE42_LAUNCH_CHECK();
        return BE42_OK;
    }
    if (c.dma == 3) {
        BE42_CHECK(c.split >= 1 && c.pf > 0 && Kp % (c.pf * 128 * c.split) == 0 &&
                       (c.split == 1 || (size_t)c.split * batch * S.total <= kGemvPartFloats),
                   "be42 gemv: slab split %d does not fit k=%d rows=%d batch=%d", c.split, k, S.total, batch);
#define BE42_SLAB(RT, SB, KSL, D, W)                                                                               \
    if (!ok && c.rt == RT && c.ks == SB && c.pf * 128 == KSL && c.u == D && c.waves == W) {                       \
        launch_slab<FP8, RT, SB, KSL, D, W>(S, dig, sx, k, Kp, batch, c.split, s);                                 \
        ok = true;                                                                                                 \
    }
        BE42_SLAB(4, 4, 512, 2, 8) BE42_SLAB(2, 4, 512, 2, 8) BE42_SLAB(1, 2, 512, 2, 8) BE42_SLAB(4, 1, 512, 4, 8)
        BE42_SLAB(2, 1, 512, 4, 8) BE42_SLAB(1, 1, 512, 4, 8)
#undef BE42_SLAB
        BE42_CHECK(ok, "be42 gemv: no slab kernel for (%d,%d,%d,%d,%d)", c.rt, c.u, c.ks, c.waves, c.pf);
        BE42_LAUNCH_CHECK();
        return BE42_OK;
    }
    if constexpr (FP8) {
        switch (nc) {
        case 1: ok = launch_tile<true, 1>(c, S, dig, sx, k, Kp, batch, s); break;
        case 2: ok = launch_tile<true, 2>(c, S, dig, sx, k, Kp, batch, s); break;
        case 3: ok = launch_tile<true, 3>(c, S, dig, sx, k, Kp, batch, s); break;
        case 4: ok = launch_tile<true, 4>(c, S, dig, sx, k, Kp, batch, s); break;
        default: ok = launch_tile<true, 5>(c, S, dig, sx, k, Kp, batch, s); break;
        }
    } else {
        switch (nc) {
        case 1: ok = launch_tile<false, 1>(c, S, dig, sx, k, Kp, batch, s); break;
        case 2: ok = launch_tile<false, 2>(c, S, dig, sx, k, Kp, batch, s); break;
        default: ok = launch_tile<false, 3>(c, S, dig, sx, k, Kp, batch, s); break;
        }
    }
    BE42_CHECK(ok, "be42 gemv: no kernel for tile (%d,%d,%d,%d,%d,%d) at nc %d", c.rt, c.u, c.ks, c.waves, c.pf,
               c.dma, nc);
    BE42_LAUNCH_CHECK();
    return BE42_OK;
}

static GemvSegs one_seg(float *y, const uint8_t *w, const float *sw, int n)
{
    GemvSegs S{};
    S.w[0] = w;
    S.sw[0] = sw;
    S.y[0] = y;
    S.n[0] = n;
    S.nseg = 1;
    S.total = n;
    return S;
}

template <bool FP8>
static int prepared_launch(float *y, const uint8_t *w, const float *sw, const void *buf, int n, int k,
                           int batch, hipStream_t s)
{
    return segs_launch<FP8>(one_seg(y, w, sw, n), buf, k, batch, s);
}

static bool fast_path(const void *w, int k, int batch)
{
    return batch <= 16 && (k % 16) == 0 && (((uintptr_t)w) & 15) == 0;
}

static bool x_aligned(const float *x) { return (((uintptr_t)x) & 15) == 0; }

template <bool FP8>
static int gemv_launch(float *y, const uint8_t *w, const float *sw, const float *x, int n, int k,
                       int batch, void *stream)
{
    const char *name = FP8 ? "be42_gemv_fp8" : "be42_gemv_q8";
    BE42_CHECK(y && w && sw && x, "%s: null pointer", name);
    BE42_CHECK(n >= 0 && k > 0 && batch >= 0, "%s: bad shape n=%d k=%d batch=%d", name, n, k, batch);
    if (n == 0 || batch == 0)
        return BE42_OK;
    hipStream_t s = as_stream(stream);
    if (!fast_path(w, k, batch) || !x_aligned(x)) {
        hipLaunchKernelGGL(k_gemv_generic<FP8>, dim3(n), dim3(256), 0, s, y, w, sw, x, n, k, batch);
        BE42_LAUNCH_CHECK();
        return BE42_OK;
    }
    void *buf = workspace(xdig_bytes(k, batch, FP8), s);
    if (!buf)
        return BE42_ENOMEM;
    int rc = xdig_prepare(buf, x, k, batch, FP8, s);
    if (rc)
        return rc;
    return prepared_launch<FP8>(y, w, sw, buf, n, k, batch, s);
}

// ---- GEMV without allocation ------------------------------------------------------
// be42_gemv_noalloc keeps its digit planes in a fixed device array instead of
// the grow-only workspace.  Each GPU holds its own copy for the life of the
// process; host code reaches it only through the address hipGetSymbolAddress
// returns for the current device (the array's name is a host-side stand-in).
constexpr size_t kNoAllocScratchBytes = (size_t)8 << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void *g_scratch_dev[kMaxDevices];

// Look up the scratch address of `device` (which must be current).
int gemv_scratch_init(int device)
{
    BE42_CHECK(device >= 0 && device < kMaxDevices, "gemv scratch: device %d out of range", device);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_dev[device])
        return BE42_OK;
    void *p = nullptr;
    BE42_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    BE42_CHECK(p != nullptr, "gemv scratch: no device address for device %d", device);
    g_scratch_dev[device] = p;
    return BE42_OK;
}

static int gemv_scratch(void **out)
{
    int dev = 0;
    BE42_HIP(hipGetDevice(&dev));
    const int rc = gemv_scratch_init(dev);
    if (rc)
        return rc;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    *out = g_scratch_dev[dev];
    return BE42_OK;
}

}  // namespace be42

using namespace be42;

extern "C" int be42_gemv_noalloc(float *y, const void *w, const float *w_scale, const float *x, int n, int k,
                                 int batch, int fp8, void *stream)
{
    BE42_CHECK(y && w && w_scale && x, "be42_gemv_noalloc: null pointer");
    BE42_CHECK(n >= 0 && k > 0 && batch >= 0, "be42_gemv_noalloc: bad shape n=%d k=%d batch=%d", n, k, batch);
    if (n == 0 || batch == 0)
        return BE42_OK;
    hipStream_t s = as_stream(stream);
    const uint8_t *wb = (const uint8_t *)w;
    if (!fast_path(w, k, batch) || !x_aligned(x)) {
        // the per-row kernel reads x directly and needs no scratch
        if (fp8)
            hipLaunchKernelGGL(k_gemv_generic<true>, dim3(n), dim3(256), 0, s, y, wb, w_scale, x, n, k, batch);
        else
            hipLaunchKernelGGL(k_gemv_generic<false>, dim3(n), dim3(256), 0, s, y, wb, w_scale, x, n, k, batch);
        BE42_LAUNCH_CHECK();
        return BE42_OK;
    }
    const size_t need = xdig_bytes(k, batch, fp8 != 0);
    BE42_CHECK(need <= kNoAllocScratchBytes,
               "be42_gemv_noalloc: k=%d at batch %d needs %zu bytes of digit planes, more than the %zu-byte scratch "
               "(use be42_gemv_%s)", k, batch, need, kNoAllocScratchBytes, fp8 ? "fp8" : "q8");
    void *buf = nullptr;
    int rc = gemv_scratch(&buf);
    if (rc)
        return rc;
    rc = xdig_prepare(buf, x, k, batch, fp8 != 0, s);
    if (rc)
        return rc;
    return fp8 ? prepared_launch<true>(y, wb, w_scale, buf, n, k, batch, s)
               : prepared_launch<false>(y, wb, w_scale, buf, n, k, batch, s);
}

extern "C" int be42_gemv_q8(float *y, const int8_t *w, const float *w_scale, const float *x, int n,
                            int k, int batch, void *stream)
{
    return gemv_launch<false>(y, (const uint8_t *)w, w_scale, x, n, k, batch, stream);
}

extern "C" int be42_gemv_fp8(float *y, const uint8_t *w, const float *w_scale, const float *x, int n,
                             int k, int batch, void *stream)
{
    return gemv_launch<true>(y, w, w_scale, x, n, k, batch, stream);
}

extern "C" size_t be42_gemv_xdig_bytes(int k, int batch, int fp8)
{
    if (k <= 0 || batch <= 0 || batch > 16)
        return 0;
    return xdig_bytes(k, batch, fp8 != 0);
}

extern "C" int be42_gemv_prepare(void *xdig, const float *x, int k, int batch, int fp8, void *stream)
{
    BE42_CHECK(xdig && x, "be42_gemv_prepare: null pointer");
    BE42_CHECK(k > 0 && k % 16 == 0 && batch > 0 && batch <= 16 && x_aligned(x),
               "be42_gemv_prepare: needs k %% 16 == 0, 1 <= batch <= 16 and 16-byte aligned x (k=%d batch=%d)",
               k, batch);
    return xdig_prepare(xdig, x, k, batch, fp8 != 0, as_stream(stream));
}

extern "C" int be42_gemv_q8_prepared(float *y, const int8_t *w, const float *w_scale, const void *xdig,
                                     int n, int k, int batch, void *stream)
{
    BE42_CHECK(y && w && w_scale && xdig, "be42_gemv_q8_prepared: null pointer");
    BE42_CHECK(n >= 0 && fast_path(w, k, batch) && batch > 0,
               "be42_gemv_q8_prepared: needs 16-byte aligned weights, k %% 16 == 0, 1 <= batch <= 16");
    if (n == 0)
        return BE42_OK;
    return prepared_launch<false>(y, (const uint8_t *)w, w_scale, xdig, n, k, batch, as_stream(stream));
}

extern "C" int be42_gemv_fp8_prepared(float *y, const uint8_t *w, const float *w_scale, const void *xdig,
                                      int n, int k, int batch, void *stream)
{
    BE42_CHECK(y && w && w_scale && xdig, "be42_gemv_fp8_prepared: null pointer");
    BE42_CHECK(n >= 0 && fast_path(w, k, batch) && batch > 0,
               "be42_gemv_fp8_prepared: needs 16-byte aligned weights, k %% 16 == 0, 1 <= batch <= 16");
    if (n == 0)
        return BE42_OK;
    return prepared_launch<true>(y, w, w_scale, xdig, n, k, batch, as_stream(stream));
}

extern "C" int be42_gemv_prepared_multi(const be42_gemv_seg *segs, int nseg, const void *xdig, int k, int batch,
                                        int fp8, void *stream)
{
    BE42_CHECK(segs && xdig && nseg >= 1 && nseg <= kMaxSegs, "be42_gemv_prepared_multi: bad arguments");
    BE42_CHECK(k > 0 && k % 16 == 0 && batch > 0 && batch <= 16,
               "be42_gemv_prepared_multi: needs k %% 16 == 0 and 1 <= batch <= 16 (k=%d batch=%d)", k, batch);
    GemvSegs S{};
    S.nseg = nseg;
    for (int i = 0; i < nseg; i++) {
        BE42_CHECK(segs[i].w && segs[i].w_scale && segs[i].y && segs[i].n > 0 &&
                       (((uintptr_t)segs[i].w) & 15) == 0,
                   "be42_gemv_prepared_multi: segment %d needs weights (16-byte aligned), scales, output, n > 0", i);
        BE42_CHECK(S.total <= INT32_MAX - segs[i].n, "be42_gemv_prepared_multi: too many rows");
        S.w[i] = (const uint8_t *)segs[i].w;
        S.sw[i] = segs[i].w_scale;
        S.y[i] = segs[i].y;
        S.n[i] = segs[i].n;
        S.total += segs[i].n;
    }
    hipStream_t s = as_stream(stream);
    return fp8 ? segs_launch<true>(S, xdig, k, batch, s) : segs_launch<false>(S, xdig, k, batch, s);
}
