// gemm.hip -- prefill GEMM for per-token-quantized activations against
// per-row-quantized weights on gfx950 matrix cores.
//
// Replaces the n > 1 (tiled GEMM) branch of op_matmul
// (src/compute/ops_matmul.c:366-477, tiling pattern of gemm_bf16_f32_tiled
// :231-330 and ops_gemm_bf16_tiled, src/compute/gemm.c:92) for quantized
// operands, both K-contiguous:
//     INT8: Y[m][n] = ((float)sum_k xq[m][k] * wq[n][k] * sx[m]) * sw[n]
//           int32 accumulation is exact (|acc| < 127^2 * K < 2^31 for
//           K < 133144), so Y is bit-identical to any exact evaluation.
//     FP8:  Y[m][n] = (sum_k e4m3(xq[m][k]) * e4m3(wq[n][k]) * sx[m]) * sw[n]
//           with fp32 accumulation in the matrix core (products are exact).
// xq / sx come from the per-token quantizers (quant_f32_to_int8,
// ops_quant.c:229, and the amax/224 E4M3 encoder, ops_quant.c:103).
//
// Tiling.  A workgroup computes a BM x BN tile of Y (tokens x features) with
// WGM x WGN waves, each owning (BM/WGM) x (BN/WGN) = TM x TN tiles of 16x16.
// K advances in stages of 128 bytes: the stage's X rows and W rows are
// copied global -> registers -> LDS (rows padded to 144 bytes so that the
// 16-byte fragment reads of 16 consecutive rows hit distinct banks), double
// buffered with one barrier per stage; the global loads of stage s+1 are in
// flight while the MFMAs of stage s run.
//   INT8: v_mfma_i32_16x16x64_i8, lane (r = lane%16, g = lane/16) supplies
//         the 16 bytes k = 16g..16g+15 of its row; 2 MFMA steps per stage.
//   FP8:  v_mfma_scale_f32_16x16x128_f8f6f4 with unit E8M0 scales (127), lane
//         supplies the 32 bytes k = 32g..32g+31; 1 step per stage.
// A and B fragments use the same k assignment, so every product pairs equal
// k.  The accumulator of a 16x16 tile holds, in lane l, rows 4*(l/16)+j
// (j = 0..3) of column l%16.
#include "be42_common.h"

namespace be42 {

constexpr int kGemmBK = 128;          // bytes of k per stage
constexpr int kGemmLd = kGemmBK + 16; // padded LDS row

template <bool FP8, int BM, int BN, int WGM, int WGN>
__global__ __launch_bounds__(WGM *WGN * 64) void k_gemm(float *__restrict__ Y, const uint8_t *__restrict__ X,
                                                        const float *__restrict__ sx,
                                                        const uint8_t *__restrict__ W,
                                                        const float *__restrict__ sw, int M, int N, int K,
                                                        int tiles_n)
{
    constexpr int NT = WGM * WGN * 64;
    constexpr int TM = BM / WGM / 16, TN = BN / WGN / 16;
    constexpr int CHUNKS = (BM + BN) * (kGemmBK / 16);   // 16-byte chunks per stage
    constexpr int CPT = CHUNKS / NT;
    static_assert(CHUNKS % NT == 0, "stage chunks must divide over the threads");
    constexpr int KI = FP8 ? 128 : 64;                   // k per MFMA
    constexpr int LB = KI / 4;                           // bytes per lane per MFMA
    __shared__ __align__(16) uint8_t lds[2][(BM + BN) * kGemmLd];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // tile order: consecutive workgroups walk down M within a column of N
    // tiles, so the W tile they share stays hot in L2
    const int tm_count = (M + BM - 1) / BM;
    const int bid = blockIdx.x;
    const int bn = bid / tm_count, bm = bid % tm_count;
    if (bn >= tiles_n)
        return;
    const int m0 = bm * BM, n0 = bn * BN;
    const int wm = wave / WGN, wn = wave % WGN;

    // global chunk c of a stage: row c / 8 of [X rows | W rows], 16-byte column c % 8
    const uint8_t *src[CPT];
    int dst[CPT];
#pragma unroll
    for (int i = 0; i < CPT; i++) {
        const int c = tid + i * NT;
        const int row = c >> 3, col = (c & 7) * 16;
        if (row < BM) {
            const int gm = min(m0 + row, M - 1);
            src[i] = X + (size_t)gm * K + col;
        } else {
            const int gn = min(n0 + row - BM, N - 1);
            src[i] = W + (size_t)gn * K + col;
        }
        dst[i] = row * kGemmLd + col;
    }
    const int nk = (K + kGemmBK - 1) / kGemmBK;
    v4i stage[CPT];
    auto gload = [&](int ks) {
        const int kb = ks * kGemmBK;
#pragma unroll
        for (int i = 0; i < CPT; i++) {
            const int col = ((tid + i * NT) & 7) * 16;
            stage[i] = kb + col < K ? *(const v4i *)(src[i] + kb) : v4i{0, 0, 0, 0};
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < CPT; i++)
            *(v4i *)(&lds[buf][dst[i]]) = stage[i];
    };

    using Acc = typename std::conditional<FP8, v4f, v4i>::type;
    Acc acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
            acc[i][j] = Acc{0, 0, 0, 0};

    const int r = lane & 15, g = lane >> 4;
    const int arow0 = wm * (TM * 16) + r;
    const int brow0 = BM + wn * (TN * 16) + r;

    gload(0);
    sstore(0);
    __syncthreads();
    for (int ks = 0; ks < nk; ks++) {
        const int cur = ks & 1;
        if (ks + 1 < nk)
            gload(ks + 1);
        const uint8_t *L = lds[cur];
#pragma unroll
        for (int kk = 0; kk < kGemmBK / KI; kk++) {
            const int kof = kk * KI + g * LB;
            if constexpr (FP8) {
                v8i a[TM], b[TN];
#pragma unroll
                for (int i = 0; i < TM; i++) {
                    const v4i lo = *(const v4i *)(L + (arow0 + i * 16) * kGemmLd + kof);
                    const v4i hi = *(const v4i *)(L + (arow0 + i * 16) * kGemmLd + kof + 16);
                    a[i] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                }
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const v4i lo = *(const v4i *)(L + (brow0 + j * 16) * kGemmLd + kof);
                    const v4i hi = *(const v4i *)(L + (brow0 + j * 16) * kGemmLd + kof + 16);
                    b[j] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                }
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[i], b[j], acc[i][j], 0, 0,
                                                                                     0, 127, 0, 127);
            } else {
                v4i a[TM], b[TN];
#pragma unroll
                for (int i = 0; i < TM; i++)
                    a[i] = *(const v4i *)(L + (arow0 + i * 16) * kGemmLd + kof);
#pragma unroll
                for (int j = 0; j < TN; j++)
                    b[j] = *(const v4i *)(L + (brow0 + j * 16) * kGemmLd + kof);
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], acc[i][j], 0, 0, 0);
            }
        }
        if (ks + 1 < nk)
            sstore(cur ^ 1);
        __syncthreads();
    }

    // epilogue: lane l holds rows 4*(l/16)+e of column l%16 of each tile
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int n = n0 + wn * (TN * 16) + j * 16 + r;
        if (n >= N)
            continue;
        const float swn = sw[n];
#pragma unroll
        for (int i = 0; i < TM; i++) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = m0 + wm * (TM * 16) + i * 16 + 4 * g + e;
                if (m < M) {
                    float v;
                    if constexpr (FP8)
                        v = acc[i][j][e];
                    else
                        v = (float)acc[i][j][e];
                    Y[(size_t)m * N + n] = (v * sx[m]) * swn;
                }
            }
        }
    }
}

template <bool FP8, int BM, int BN, int WGM, int WGN>
static void launch_gemm(float *Y, const uint8_t *X, const float *sx, const uint8_t *W, const float *sw, int M,
                        int N, int K, hipStream_t s)
{
    const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
    hipLaunchKernelGGL((k_gemm<FP8, BM, BN, WGM, WGN>), dim3(tm * tn), dim3(WGM * WGN * 64), 0, s, Y, X, sx, W, sw,
                       M, N, K, tn);
}

// Tile choice: 128 x 128 workgroups of 4 waves (2 x 2, 64 x 64 per wave)
// when the grid fills the chip, else 64 x 128.
template <bool FP8>
static void gemm_dispatch(float *Y, const uint8_t *X, const float *sx, const uint8_t *W, const float *sw, int M,
                          int N, int K, hipStream_t s)
{
    const long tiles128 = (long)((M + 127) / 128) * ((N + 127) / 128);
    if (tiles128 >= 512)
        launch_gemm<FP8, 128, 128, 2, 2>(Y, X, sx, W, sw, M, N, K, s);
    else
        launch_gemm<FP8, 64, 128, 2, 2>(Y, X, sx, W, sw, M, N, K, s);
}

}  // namespace be42

using namespace be42;

static int gemm_entry(bool fp8, float *y, const void *xq, const float *sx, const void *wq, const float *sw, int m,
                      int n, int k, void *stream)
{
    const char *name = fp8 ? "be42_gemm_fp8" : "be42_gemm_i8";
    BE42_CHECK(y && xq && sx && wq && sw, "%s: null pointer", name);
    BE42_CHECK(m >= 0 && n >= 0 && k > 0 && k % 16 == 0, "%s: bad shape m=%d n=%d k=%d (k must be a multiple of 16)",
               name, m, n, k);
    BE42_CHECK(((uintptr_t)xq & 15) == 0 && ((uintptr_t)wq & 15) == 0, "%s: operands must be 16-byte aligned", name);
    BE42_CHECK(fp8 || k < 133144, "%s: k=%d would overflow the int32 accumulator", name, k);
    if (m == 0 || n == 0)
        return BE42_OK;
    if (fp8)
        gemm_dispatch<true>(y, (const uint8_t *)xq, sx, (const uint8_t *)wq, sw, m, n, k, as_stream(stream));
    else
        gemm_dispatch<false>(y, (const uint8_t *)xq, sx, (const uint8_t *)wq, sw, m, n, k, as_stream(stream));
    BE42_LAUNCH_CHECK();
    return BE42_OK;
}

extern "C" int be42_gemm_i8(float *y, const int8_t *xq, const float *sx, const int8_t *wq, const float *sw, int m,
                            int n, int k, void *stream)
{
    return gemm_entry(false, y, xq, sx, wq, sw, m, n, k, stream);
}

extern "C" int be42_gemm_fp8(float *y, const uint8_t *xq, const float *sx, const uint8_t *wq, const float *sw,
                             int m, int n, int k, void *stream)
{
    return gemm_entry(true, y, xq, sx, wq, sw, m, n, k, stream);
}
