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
// Two kernels: k_gemm_dma (K a multiple of 128, the prefill shapes), whose
// stages go global -> LDS by the direct-to-LDS loads and whose tiles run on
// the 32x32 matrix-core steps (described at the kernel), and k_gemm for any
// K that is a multiple of 16:
// A workgroup computes a BM x BN tile of Y (tokens x features) with
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
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "be42_common.h"
#include "xdigits.h"

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

// Chunk slot of 16-byte chunk c in LDS row R of the DMA-staged GEMM: rows
// are 128 bytes, chunks XOR-permuted so that 16 consecutive rows read at the
// same chunk fall on 16 distinct (row parity, slot) pairs, i.e. on distinct
// banks whether the LDS serves 8 lanes x 16 bytes over 32 banks or 16 lanes
// over 64 banks per cycle.
__device__ __forceinline__ int dma_slot(int R, int c) { return c ^ ((R & 7) ^ ((R >> 3) & 1)); }

// Scheduling hint: NM matrix-core instructions, each followed by its share of
// ND LDS reads (the first ND % NM take one more).
template <int NM, int ND, int I = 0>
__device__ __forceinline__ void sched_interleave()
{
    if constexpr (I < NM) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        constexpr int d = ND / NM + (I < ND % NM ? 1 : 0);
        if constexpr (d > 0)
            __builtin_amdgcn_sched_group_barrier(0x100, d, 0);
        sched_interleave<NM, ND, I + 1>();
    }
}

// Large-tile GEMM whose stages move global -> LDS through the direct-to-LDS
// loads of gfx950 (global_load_lds_dwordx4), so no VGPRs or LDS-store
// instructions are spent on staging.  A workgroup of WGM x WGN waves owns a
// BM x BN tile of Y, each wave (BM/WGM) x (BN/WGN) = TM x TN tiles of 32x32
// on the 32x32 matrix-core instructions, which do twice the work of the
// 16x16 ones per operand byte read from LDS:
//   FP8:  v_mfma_scale_f32_32x32x64_f8f6f4 with unit scales, lane
//         (r = lane%32, h = lane/32) supplying 32 bytes of row r;
//   INT8: two v_mfma_i32_32x32x32_i8, 16 bytes each.
// The accumulator of a 32x32 tile holds, in lane l, rows
// 8*(i/4) + 4*(l/32) + i%4 (i = 0..15) of column l%32.
// A stage is 128 k-bytes of the BM + BN rows (X rows first, then W rows),
// laid out in LDS as 128-byte rows with chunks placed by dma_slot; one load
// instruction fills 1 KB = 8 rows, lane l writing LDS bytes [16l, 16l+16),
// i.e. row l/8, slot l%8, so each lane fetches global chunk
// dma_slot(row, l%8) and the 8 lanes of a row read one full 128-byte line.
// NS stages are resident in a ring (see the main loop).  Within a stage the
// LDS reads of step 1 are interleaved with the matrix-core instructions of
// step 0, and those of the next stage's step 0 with step 1.  Workgroup ids
// are spread over the 8 XCDs round-robin by the hardware; they are remapped
// so that each XCD walks a contiguous run of the grouped tile order.
// K must be a multiple of 128 and M*K, N*K below 2^32 (32-bit offsets);
// rows past M or N read the last row and are not stored.
template <bool FP8, int BM, int BN, int WGM, int WGN, int NS>
__global__ __launch_bounds__(WGM *WGN * 64) void k_gemm_dma(float *__restrict__ Y, const uint8_t *__restrict__ X,
                                                            const float *__restrict__ sx,
                                                            const uint8_t *__restrict__ W,
                                                            const float *__restrict__ sw, int M, int N, int K,
                                                            int tiles_m, int tiles_n, int tiles)
{
    constexpr int NW = WGM * WGN;
    constexpr int TM = BM / WGM / 32, TN = BN / WGN / 32;
    constexpr int SBYTES = (BM + BN) * 128;              // one stage
    constexpr int DPW = (BM + BN) / 8 / NW;              // 1 KB loads per wave per stage
    static_assert((BM + BN) % (8 * NW) == 0, "stage loads must divide over the waves");
    static_assert(BM % 32 == 0 && BN % 32 == 0, "32-row blocks");
    using AccT = typename std::conditional<FP8, v16f, v16i>::type;
    extern __shared__ __align__(1024) uint8_t lds_dyn[];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int b = blockIdx.x, nb = gridDim.x;
    const int per = nb / 8, rem = nb % 8, x = b % 8, i8 = b / 8;
    const int tile = (x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per) + i8;
    if (tile >= tiles)
        return;
    // grouped order: runs of 8 M-tiles, N-tiles within a run, so that the
    // 32 workgroups an XCD holds at once cover 8 x 4 tiles and share their X
    // and W slabs in its L2
    int bm, bn;
    {
        constexpr int GM = 8;
        const int span = GM * tiles_n;
        const int first = tile / span * GM, gsz = min(tiles_m - first, GM), t = tile % span;
        bm = first + t % gsz;
        bn = t / gsz;
    }

    const int m0 = bm * BM, n0 = bn * BN;
    const int wm = wave / WGN, wn = wave % WGN;

    // byte offsets of this lane's 16-byte chunk in X or W (which one is
    // uniform over each load: BM is a multiple of 8); the host keeps M*K
    // and N*K below 2^32
    uint32_t src[DPW];
#pragma unroll
    for (int j = 0; j < DPW; j++) {
        const int row = (wave * DPW + j) * 8 + (lane >> 3);
        const uint32_t off = dma_slot(row, lane & 7) * 16;
        if (row < BM)
            src[j] = (uint32_t)min(m0 + row, M - 1) * (uint32_t)K + off;
        else
            src[j] = (uint32_t)min(n0 + row - BM, N - 1) * (uint32_t)K + off;
    }
    auto issue = [&](int st) {
        uint8_t *base = lds_dyn + (st % NS) * SBYTES + wave * DPW * 1024;
#pragma unroll
        for (int j = 0; j < DPW; j++) {
            const uint8_t *g = (wave * DPW + j) * 8 < BM ? X : W;
            __builtin_amdgcn_global_load_lds((const void *)(g + src[j] + (size_t)st * 128),
                                             (lds_void *)(base + j * 1024), 16, 0, 0);
        }
        // the wait counts assume every load of stage st is issued before any
        // load of a later stage: keep the compiler from interleaving stages
        asm volatile("" ::: "memory");
    };

    AccT acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
            acc[i][j] = AccT{};

    const int r = lane & 31, h = lane >> 5;
    // row r of every 32-row block has the same slot permutation
    const int arow = (wm * TM * 32 + r) * 128, brow = (BM + wn * TN * 32 + r) * 128;
    // a stage is two steps of 64 k-bytes; a step's fragment is 32 bytes a
    // lane, chunks c0 and c1 of its row:
    //   FP8  one 32x32x64 instruction, k = 64u + 32h .. +31: c0 = 4u + 2h, c1 = c0 + 1
    //   INT8 two 32x32x32 instructions, k = 64u + 16h .. +15 (c0 = 4u + h) and
    //        k = 64u + 32 + 16h .. +15 (c1 = 4u + 2 + h)
    struct Frags {
        v8i a[TM], b[TN];
    };
    const int c0 = FP8 ? 2 * h : h, c1 = FP8 ? 2 * h + 1 : 2 + h;
    auto load = [&](int buf, int u, Frags &f) {
        const uint8_t *L = lds_dyn + buf * SBYTES;
        auto rd = [&](int rowoff, int c) -> v4i { return *(const v4i *)(L + rowoff + dma_slot(r, c) * 16); };
#pragma unroll
        for (int i = 0; i < TM + TN; i++) {
            const int ro = i < TM ? arow + i * 32 * 128 : brow + (i - TM) * 32 * 128;
            const v4i lo = rd(ro, 4 * u + c0), hi = rd(ro, 4 * u + c1);
            const v8i v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            if (i < TM)
                f.a[i] = v;
            else
                f.b[i - TM] = v;
        }
    };
    auto mfma = [&](const Frags &f) {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) {
                if constexpr (FP8) {
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.a[i], f.b[j], acc[i][j], 0, 0, 0,
                                                                                127, 0, 127);
                } else {
                    const v4i alo = {f.a[i][0], f.a[i][1], f.a[i][2], f.a[i][3]};
                    const v4i ahi = {f.a[i][4], f.a[i][5], f.a[i][6], f.a[i][7]};
                    const v4i blo = {f.b[j][0], f.b[j][1], f.b[j][2], f.b[j][3]};
                    const v4i bhi = {f.b[j][4], f.b[j][5], f.b[j][6], f.b[j][7]};
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(alo, blo, acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ahi, bhi, acc[i][j], 0, 0, 0);
                }
            }
    };
    // the LDS reads of the next step go between the matrix-core instructions
    // of this one
    auto interleave = [&]() {
        if constexpr (FP8)
            sched_interleave<TM * TN, (TM + TN) * 2>();
    };

    // Stages s .. s+NS-1 are resident (the first NS issued up front).  The
    // loads of stage s+NS are issued once every wave has read its last
    // fragments of stage s (the barrier before the last step of s), which is
    // also where stage s+1 is waited for (NS-2 later stages may still be in
    // flight).
    const int nk = K / 128;
#pragma unroll
    for (int st = 0; st < NS; st++)
        if (st < nk)
            issue(st);
    if (nk >= NS)
        wait_vmcnt<(NS - 1) * DPW>();
    else
        wait_vmcnt<0>();
    __syncthreads();
    Frags F[2];
    load(0, 0, F[0]);
    for (int st = 0; st < nk; st++) {
        const int buf = st % NS, nbuf = (st + 1) % NS;
        // step 0: read step 1's fragments while the matrix cores run step 0
        __builtin_amdgcn_sched_barrier(0);
        load(buf, 1, F[1]);
        mfma(F[0]);
        interleave();
        __builtin_amdgcn_sched_barrier(0);
        // step 1: stage st+1 must have landed and every wave be done with
        // stage st before its buffer takes stage st+NS; then read stage
        // st+1's first fragments (past the last stage the read is of stale
        // LDS and unused)
        if (st + 1 < nk) {
            if (st + NS - 1 < nk)
                wait_vmcnt<(NS - 2) * DPW>();
            else
                wait_vmcnt<0>();
            __syncthreads();
            if (st + NS < nk)
                issue(st + NS);
        }
        load(nbuf, 0, F[0]);
        mfma(F[1]);
        interleave();
    }

#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int n = n0 + wn * (TN * 32) + j * 32 + r;
        if (n >= N)
            continue;
        const float swn = sw[n];
#pragma unroll
        for (int i = 0; i < TM; i++) {
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int m = m0 + wm * (TM * 32) + i * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
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

template <bool FP8, int BM, int BN, int WGM, int WGN, int NS>
static void launch_gemm_dma(float *Y, const uint8_t *X, const float *sx, const uint8_t *W, const float *sw, int M,
                            int N, int K, hipStream_t s)
{
    const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
    const size_t lds = (size_t)NS * (BM + BN) * 128;
    static_assert(NS * (BM + BN) * 128 <= 160 * 1024, "LDS budget");
    static bool attr = false;
    if (!attr) {
        (void)hipFuncSetAttribute((const void *)k_gemm_dma<FP8, BM, BN, WGM, WGN, NS>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        attr = true;
    }
    hipLaunchKernelGGL((k_gemm_dma<FP8, BM, BN, WGM, WGN, NS>), dim3(tm * tn), dim3(WGM * WGN * 64), lds, s, Y, X, sx,
                       W, sw, M, N, K, tm, tn, tm * tn);
}

template <bool FP8, int BM, int BN, int WGM, int WGN>
static void launch_gemm(float *Y, const uint8_t *X, const float *sx, const uint8_t *W, const float *sw, int M,
                        int N, int K, hipStream_t s)
{
    const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
    hipLaunchKernelGGL((k_gemm<FP8, BM, BN, WGM, WGN>), dim3(tm * tn), dim3(WGM * WGN * 64), 0, s, Y, X, sx, W, sw,
                       M, N, K, tn);
}

// Kernel and tile choice.  K a multiple of 128 (and operands under 4 GiB):
// the direct-to-LDS kernel, at 256 x 256 when that grid alone fills the 256
// CUs, at 64 x 128 (4 waves of 32 x 64, a 4-stage ring) when 128 x 128 tiles
// would leave CUs idle (fewer than 256 tiles: M = 512 at N = 4096), else at
// 128 x 128.  Otherwise the register-staged 16x16 kernel at 128 x 128 when
// its grid holds two workgroups per CU, else 64 x 128.
// BE42_GEMM_TILE = 1..5 forces one of the five (1, 2 and 5 only where K
// allows; 5 is the 64 x 128 direct-to-LDS tile).
template <bool FP8>
static void gemm_dispatch(float *Y, const uint8_t *X, const float *sx, const uint8_t *W, const float *sw, int M,
                          int N, int K, hipStream_t s)
{
    const long tiles128 = (long)((M + 127) / 128) * ((N + 127) / 128);
    const long tiles256 = (long)((M + 255) / 256) * ((N + 255) / 256);
    const bool dma = K % 128 == 0 && (size_t)M * K < (1ull << 32) && (size_t)N * K < (1ull << 32);
    const char *e = getenv("BE42_GEMM_TILE");
    const int force = e ? atoi(e) : 0;
    if (dma && (force == 1 || (!force && tiles256 >= 256)))
        launch_gemm_dma<FP8, 256, 256, 2, 4, 2>(Y, X, sx, W, sw, M, N, K, s);
    else if (dma && (force == 5 || (!force && tiles128 < 256)))
        launch_gemm_dma<FP8, 64, 128, 2, 2, 4>(Y, X, sx, W, sw, M, N, K, s);
    else if (dma && (force == 2 || !force))
        launch_gemm_dma<FP8, 128, 128, 2, 2, 2>(Y, X, sx, W, sw, M, N, K, s);
    else if (force == 3 || (!force && tiles128 >= 512))
        launch_gemm<FP8, 128, 128, 2, 2>(Y, X, sx, W, sw, M, N, K, s);
    else
        launch_gemm<FP8, 64, 128, 2, 2>(Y, X, sx, W, sw, M, N, K, s);
}

// Prefill GEMM with fp32 activations: the decode GEMV's arithmetic for many
// tokens at once.  X arrives as the GEMV's digit planes (xdigits.h, one batch
// row per token, dig[d][m][Kp]), so each weight tile is read once for all
// the tokens of a workgroup instead of once per token, and every output is
// formed exactly as the GEMV forms it: INT8 digit sums are exact int32,
// combined in int64 and scaled once in fp64, y = tot * ((sx * 254^-2) * sw),
// so the result is bit-identical to the GEMV's for the same row; FP8 digit
// sums are fp32 matrix-core accumulations combined in fp64 (equal to the
// GEMV's to fp32 accumulation order).
// A workgroup of WGM x WGN waves owns BT = 16 WGM tokens x BN = 16 TN WGN
// features; wave (wm, wn) holds, for its 16 tokens, one 16x16 accumulator
// per digit plane and feature tile, so the epilogue combines a token's
// digits in registers.  LDS rows of a stage: digit d of token row t at
// d * BT + t, then the BN weight rows; stages of 128 k-bytes go global ->
// registers -> LDS (rows padded to 144 bytes), double buffered with one
// barrier per stage, as in k_gemm.  Chunks past K read as zero.
template <bool FP8, int WGM, int WGN, int TN>
__global__ __launch_bounds__(WGM *WGN * 64) void k_gemm_dig(float *__restrict__ Y, const uint8_t *__restrict__ dig,
                                                            const float *__restrict__ sx,
                                                            const uint8_t *__restrict__ W,
                                                            const float *__restrict__ sw, int M, int N, int K,
                                                            int Kp, int tiles_m)
{
    constexpr int ND = FP8 ? kF8Digits : kI8Digits;
    constexpr int NT = WGM * WGN * 64;
    constexpr int BT = 16 * WGM, BN = 16 * TN * WGN, XR = ND * BT;
    constexpr int CHUNKS = (XR + BN) * (kGemmBK / 16);
    constexpr int CPT = (CHUNKS + NT - 1) / NT;
    constexpr int KI = FP8 ? 128 : 64;
    constexpr int LB = KI / 4;
    __shared__ __align__(16) uint8_t lds[2][(XR + BN) * kGemmLd];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int bm = blockIdx.x % tiles_m, bn = blockIdx.x / tiles_m;
    const int m0 = bm * BT, n0 = bn * BN;
    const int wm = wave / WGN, wn = wave % WGN;

    const uint8_t *src[CPT];
    int dst[CPT];
    bool live[CPT];
#pragma unroll
    for (int i = 0; i < CPT; i++) {
        const int c = min(tid + i * NT, CHUNKS - 1);
        live[i] = tid + i * NT < CHUNKS;
        const int row = c >> 3, col = (c & 7) * 16;
        if (row < XR) {
            const int d = row / BT, t = min(m0 + row % BT, M - 1);
            src[i] = dig + ((size_t)d * M + t) * Kp + col;
        } else {
            src[i] = W + (size_t)min(n0 + row - XR, N - 1) * K + col;
        }
        dst[i] = row * kGemmLd + col;
    }
    const int nk = (K + kGemmBK - 1) / kGemmBK;
    v4i stage[CPT];
    auto gload = [&](int ks) {
        const int kb = ks * kGemmBK;
#pragma unroll
        for (int i = 0; i < CPT; i++) {
            const int col = (min(tid + i * NT, CHUNKS - 1) & 7) * 16;
            stage[i] = kb + col < K ? *(const v4i *)(src[i] + kb) : v4i{0, 0, 0, 0};
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < CPT; i++)
            if (live[i])
                *(v4i *)(&lds[buf][dst[i]]) = stage[i];
    };

    using Acc = typename std::conditional<FP8, v4f, v4i>::type;
    Acc acc[ND][TN];
#pragma unroll
    for (int i = 0; i < ND; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
            acc[i][j] = Acc{0, 0, 0, 0};

    const int r = lane & 15, g = lane >> 4;
    const int arow0 = wm * 16 + r;                   // + d * BT
    const int brow0 = XR + wn * (TN * 16) + r;       // + j * 16

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
                v8i a[ND], b[TN];
#pragma unroll
                for (int i = 0; i < ND; i++) {
                    const v4i lo = *(const v4i *)(L + (arow0 + i * BT) * kGemmLd + kof);
                    const v4i hi = *(const v4i *)(L + (arow0 + i * BT) * kGemmLd + kof + 16);
                    a[i] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                }
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const v4i lo = *(const v4i *)(L + (brow0 + j * 16) * kGemmLd + kof);
                    const v4i hi = *(const v4i *)(L + (brow0 + j * 16) * kGemmLd + kof + 16);
                    b[j] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                }
#pragma unroll
                for (int i = 0; i < ND; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[i], b[j], acc[i][j], 0, 0,
                                                                                     0, 127, 0, 127);
            } else {
                v4i a[ND], b[TN];
#pragma unroll
                for (int i = 0; i < ND; i++)
                    a[i] = *(const v4i *)(L + (arow0 + i * BT) * kGemmLd + kof);
#pragma unroll
                for (int j = 0; j < TN; j++)
                    b[j] = *(const v4i *)(L + (brow0 + j * 16) * kGemmLd + kof);
#pragma unroll
                for (int i = 0; i < ND; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], acc[i][j], 0, 0, 0);
            }
        }
        if (ks + 1 < nk)
            sstore(cur ^ 1);
        __syncthreads();
    }

    // lane l holds tokens 4*(l/16)+e of feature column l%16 of every tile
    const double sxw = FP8 ? 1.0 : 1.0 / (double)(kI8Base * kI8Base);
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int n = n0 + wn * (TN * 16) + j * 16 + r;
        if (n >= N)
            continue;
        const double swn = (double)sw[n];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int m = m0 + wm * 16 + 4 * g + e;
            if (m >= M)
                continue;
            double tot;
            if constexpr (FP8) {
                tot = 0.0;
#pragma unroll
                for (int d = 0; d < ND; d++)
                    tot += (double)acc[d][j][e] * kF8DigitW[d];
            } else {
                const long long it = (long long)acc[0][j][e] * ((long long)kI8Base * kI8Base) +
                                     (long long)acc[1][j][e] * kI8Base + (long long)acc[2][j][e];
                tot = (double)it;
            }
            Y[(size_t)m * N + n] = (float)(tot * ((double)sx[m] * sxw * swn));
        }
    }
}

template <bool FP8, int WGM, int WGN, int TN>
static void launch_gemm_dig(float *Y, const uint8_t *dig, const float *sx, const uint8_t *W, const float *sw, int M,
                            int N, int K, hipStream_t s)
{
    const int tm = (M + 16 * WGM - 1) / (16 * WGM), tn = (N + 16 * TN * WGN - 1) / (16 * TN * WGN);
    hipLaunchKernelGGL((k_gemm_dig<FP8, WGM, WGN, TN>), dim3(tm * tn), dim3(WGM * WGN * 64), 0, s, Y, dig, sx, W, sw,
                       M, N, K, (int)xdig_kp(K, FP8), tm);
}

// The digit-plane GEMM on the direct-to-LDS stages and 32x32 matrix-core
// steps of k_gemm_dma (K a multiple of 128).  A workgroup of WGM x WGN waves
// owns BT = 32 WGM tokens x BN = 32 TN WGN features; wave (wm, wn) holds,
// for its 32 tokens, one 32x32 accumulator per digit plane and feature tile.
// A stage's LDS rows: digit d of token row t at d * BT + t, then the BN
// weight rows, 128 bytes each with chunks placed by dma_slot.  The epilogue
// is k_gemm_dig's: digits combined in registers, one fp64 scaling.
// Up to three weight matrices that share the activations (q/k/v, gate/up):
// feature tiles are numbered through the segments one after another
// (segment s owns tiles [tn_end[s-1], tn_end[s])), so one launch covers them.
constexpr int kDigSegs = 3;
struct DigSegs {
    const uint8_t *w[kDigSegs];
    const float *sw[kDigSegs];
    float *y[kDigSegs];
    int n[kDigSegs], tn_end[kDigSegs];
    int nseg;
};

template <bool FP8, int WGM, int WGN, int TN, int NS>
__global__ __launch_bounds__(WGM *WGN * 64) void k_gemm_dig_dma(const DigSegs S, const uint8_t *__restrict__ dig,
                                                                const float *__restrict__ sx, int M, int K, int Kp,
                                                                int tiles_m, int tiles)
{
    constexpr int ND = FP8 ? kF8Digits : kI8Digits;
    constexpr int NW = WGM * WGN;
    constexpr int BT = 32 * WGM, BN = 32 * TN * WGN, XR = ND * BT, R = XR + BN;
    constexpr int SBYTES = R * 128;
    constexpr int DPW = R / 8 / NW;
    static_assert(R % (8 * NW) == 0, "stage loads must divide over the waves");
    static_assert(XR % 8 == 0, "a load instruction stays within the digit rows or the weight rows");
    using AccT = typename std::conditional<FP8, v16f, v16i>::type;
    extern __shared__ __align__(1024) uint8_t lds_dyn[];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int b = blockIdx.x, nb = gridDim.x;
    const int per = nb / 8, rem = nb % 8, x = b % 8, i8 = b / 8;
    const int tile = (x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per) + i8;
    if (tile >= tiles)
        return;
    // token tiles innermost: the workgroups of one XCD share a weight slab
    const int bm = tile % tiles_m, bng = tile / tiles_m;
    const int sg = (S.nseg > 1 && bng >= S.tn_end[0]) + (S.nseg > 2 && bng >= S.tn_end[1]);
    const int bn = bng - (sg == 0 ? 0 : S.tn_end[sg - 1]);
    const uint8_t *__restrict__ W = S.w[sg];
    const float *__restrict__ sw = S.sw[sg];
    float *__restrict__ Y = S.y[sg];
    const int N = S.n[sg];
    const int m0 = bm * BT, n0 = bn * BN;
    const int wm = wave / WGN, wn = wave % WGN;

    // byte offset of this lane's 16-byte chunk (digit planes or weights)
    uint32_t src[DPW];
#pragma unroll
    for (int j = 0; j < DPW; j++) {
        const int row = (wave * DPW + j) * 8 + (lane >> 3);
        const uint32_t off = dma_slot(row, lane & 7) * 16;
        if (row < XR) {
            const int d = row / BT, t = min(m0 + row % BT, M - 1);
            src[j] = ((uint32_t)d * (uint32_t)M + (uint32_t)t) * (uint32_t)Kp + off;
        } else {
            src[j] = (uint32_t)min(n0 + row - XR, N - 1) * (uint32_t)K + off;
        }
    }
    auto issue = [&](int st) {
        uint8_t *base = lds_dyn + (st % NS) * SBYTES + wave * DPW * 1024;
#pragma unroll
        for (int j = 0; j < DPW; j++) {
            const uint8_t *g = (wave * DPW + j) * 8 < XR ? dig : W;
            __builtin_amdgcn_global_load_lds((const void *)(g + src[j] + (size_t)st * 128),
                                             (lds_void *)(base + j * 1024), 16, 0, 0);
        }
        asm volatile("" ::: "memory");
    };

    AccT acc[ND][TN];
#pragma unroll
    for (int i = 0; i < ND; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
            acc[i][j] = AccT{};

    const int r = lane & 31, h = lane >> 5;
    const int arow = (wm * 32 + r) * 128, brow = (XR + wn * TN * 32 + r) * 128;
    struct Frags {
        v8i a[ND], b[TN];
    };
    const int c0 = FP8 ? 2 * h : h, c1 = FP8 ? 2 * h + 1 : 2 + h;
    auto load = [&](int buf, int u, Frags &f) {
        const uint8_t *L = lds_dyn + buf * SBYTES;
        auto rd = [&](int rowoff, int c) -> v4i { return *(const v4i *)(L + rowoff + dma_slot(r, c) * 16); };
#pragma unroll
        for (int i = 0; i < ND + TN; i++) {
            const int ro = i < ND ? arow + i * BT * 128 : brow + (i - ND) * 32 * 128;
            const v4i lo = rd(ro, 4 * u + c0), hi = rd(ro, 4 * u + c1);
            const v8i v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            if (i < ND)
                f.a[i] = v;
            else
                f.b[i - ND] = v;
        }
    };
    auto mfma = [&](const Frags &f) {
#pragma unroll
        for (int i = 0; i < ND; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) {
                if constexpr (FP8) {
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.a[i], f.b[j], acc[i][j], 0, 0, 0,
                                                                                127, 0, 127);
                } else {
                    const v4i alo = {f.a[i][0], f.a[i][1], f.a[i][2], f.a[i][3]};
                    const v4i ahi = {f.a[i][4], f.a[i][5], f.a[i][6], f.a[i][7]};
                    const v4i blo = {f.b[j][0], f.b[j][1], f.b[j][2], f.b[j][3]};
                    const v4i bhi = {f.b[j][4], f.b[j][5], f.b[j][6], f.b[j][7]};
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(alo, blo, acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ahi, bhi, acc[i][j], 0, 0, 0);
                }
            }
    };
    auto interleave = [&]() {
        if constexpr (FP8)
            sched_interleave<ND * TN, (ND + TN) * 2>();
    };

    const int nk = K / 128;
#pragma unroll
    for (int st = 0; st < NS; st++)
        if (st < nk)
            issue(st);
    if (nk >= NS)
        wait_vmcnt<(NS - 1) * DPW>();
    else
        wait_vmcnt<0>();
    __syncthreads();
    Frags F[2];
    load(0, 0, F[0]);
    for (int st = 0; st < nk; st++) {
        const int buf = st % NS, nbuf = (st + 1) % NS;
        __builtin_amdgcn_sched_barrier(0);
        load(buf, 1, F[1]);
        mfma(F[0]);
        interleave();
        __builtin_amdgcn_sched_barrier(0);
        if (st + 1 < nk) {
            if (st + NS - 1 < nk)
                wait_vmcnt<(NS - 2) * DPW>();
            else
                wait_vmcnt<0>();
            __syncthreads();
            if (st + NS < nk)
                issue(st + NS);
        }
        load(nbuf, 0, F[0]);
        mfma(F[1]);
        interleave();
    }

    // lane l holds tokens 8*(e/4) + 4*(l/32) + e%4 of feature column l%32
    const double sxw = FP8 ? 1.0 : 1.0 / (double)(kI8Base * kI8Base);
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int n = n0 + wn * (TN * 32) + j * 32 + r;
        if (n >= N)
            continue;
        const double swn = (double)sw[n];
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int m = m0 + wm * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
            if (m >= M)
                continue;
            double tot;
            if constexpr (FP8) {
                tot = 0.0;
#pragma unroll
                for (int d = 0; d < ND; d++)
                    tot += (double)acc[d][j][e] * kF8DigitW[d];
            } else {
                const long long it = (long long)acc[0][j][e] * ((long long)kI8Base * kI8Base) +
                                     (long long)acc[1][j][e] * kI8Base + (long long)acc[2][j][e];
                tot = (double)it;
            }
            Y[(size_t)m * N + n] = (float)(tot * ((double)sx[m] * sxw * swn));
        }
    }
}

template <bool FP8, int WGM, int WGN, int TN, int NS>
static void launch_gemm_dig_dma(DigSegs S, const uint8_t *dig, const float *sx, int M, int K, hipStream_t s)
{
    constexpr int ND = FP8 ? kF8Digits : kI8Digits;
    constexpr int BT = 32 * WGM, BN = 32 * TN * WGN;
    constexpr size_t lds = (size_t)NS * (ND * BT + BN) * 128;
    static_assert(lds <= 160 * 1024, "LDS budget");
    const int tm = (M + BT - 1) / BT;
    int tn = 0;
    for (int i = 0; i < S.nseg; i++) {
        tn += (S.n[i] + BN - 1) / BN;
        S.tn_end[i] = tn;
    }
    static bool attr = false;
    if (!attr) {
        (void)hipFuncSetAttribute((const void *)k_gemm_dig_dma<FP8, WGM, WGN, TN, NS>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        attr = true;
    }
    hipLaunchKernelGGL((k_gemm_dig_dma<FP8, WGM, WGN, TN, NS>), dim3(tm * tn), dim3(WGM * WGN * 64), lds, s, S, dig,
                       sx, M, K, (int)xdig_kp(K, FP8), tm, tm * tn);
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

// ---- prefill GEMM over activation digit planes ------------------------------

extern "C" size_t be42_gemm_xdig_bytes(int k, int m, int fp8)
{
    if (k <= 0 || m <= 0)
        return 0;
    return xdig_bytes(k, m, fp8 != 0);
}

extern "C" int be42_gemm_prepare(void *xdig, const float *x, int k, int m, int fp8, void *stream)
{
    BE42_CHECK(xdig && x, "be42_gemm_prepare: null pointer");
    BE42_CHECK(k > 0 && k % 16 == 0 && m > 0 && m <= 65535 && ((uintptr_t)x & 15) == 0,
               "be42_gemm_prepare: needs k %% 16 == 0, 1 <= m <= 65535 and 16-byte aligned x (k=%d m=%d)", k, m);
    return xdig_prepare(xdig, x, k, m, fp8 != 0, as_stream(stream));
}

static int gemm_dig_run(bool fp8, const be42_gemv_seg *segs, int nseg, const void *xdig, int k, int m,
                        void *stream, const char *name)
{
    BE42_CHECK(segs && xdig && nseg >= 1 && nseg <= kDigSegs, "%s: null pointer or %d segments (1..%d)", name, nseg,
               kDigSegs);
    BE42_CHECK(k > 0 && k % 16 == 0 && m > 0 && m <= 65535, "%s: bad shape k=%d m=%d (k %% 16 == 0, m <= 65535)",
               name, k, m);
    BE42_CHECK(fp8 || k < 133144, "%s: k=%d would overflow the int32 accumulator", name, k);
    DigSegs S{};
    S.nseg = nseg;
    size_t nmax = 0;
    for (int i = 0; i < nseg; i++) {
        BE42_CHECK(segs[i].w && segs[i].w_scale && segs[i].y && segs[i].n > 0, "%s: segment %d: null pointer or n %d",
                   name, i, segs[i].n);
        BE42_CHECK(((uintptr_t)segs[i].w & 15) == 0, "%s: weights must be 16-byte aligned", name);
        S.w[i] = (const uint8_t *)segs[i].w;
        S.sw[i] = segs[i].w_scale;
        S.y[i] = segs[i].y;
        S.n[i] = segs[i].n;
        nmax = std::max(nmax, (size_t)segs[i].n);
    }
    const uint8_t *dig = (const uint8_t *)xdig;
    const float *sx = xdig_scales((void *)xdig, k, m, fp8);
    hipStream_t s = as_stream(stream);
    // K a multiple of 128 and 32-bit offsets: the direct-to-LDS kernel, all
    // segments in one launch; else the register-staged one per segment
    const int nd = xdig_layout(fp8).nd;
    const bool dma = k % 128 == 0 && (size_t)nd * m * xdig_kp(k, fp8) < (1ull << 32) && nmax * k < (1ull << 32);
    const char *e = getenv("BE42_GEMM_DIG");
    const int force = e ? atoi(e) : 0;
    if (dma && force != 1) {
        if (fp8) {
            // 64 tokens x 256 features: each wave's 4 digit fragments and 2
            // weight fragments feed 8 matrix instructions (with 128 features,
            // 5 fragments fed 4, and the LDS reads bounded the loop: the 3B
            // shapes 15-20% slower)
            if (force == 3)
                launch_gemm_dig_dma<true, 2, 2, 2, 2>(S, dig, sx, m, k, s);
            else
                launch_gemm_dig_dma<true, 2, 4, 2, 2>(S, dig, sx, m, k, s);
        } else {
            if (force == 3)
                launch_gemm_dig_dma<false, 2, 2, 2, 3>(S, dig, sx, m, k, s);
            else
                launch_gemm_dig_dma<false, 2, 4, 2, 2>(S, dig, sx, m, k, s);
        }
    } else {
        for (int i = 0; i < nseg; i++) {
            if (fp8)
                launch_gemm_dig<true, 4, 2, 4>(S.y[i], dig, sx, S.w[i], S.sw[i], m, S.n[i], k, s);
            else
                launch_gemm_dig<false, 4, 2, 4>(S.y[i], dig, sx, S.w[i], S.sw[i], m, S.n[i], k, s);
        }
    }
    BE42_LAUNCH_CHECK();
    return BE42_OK;
}

static int gemm_dig_entry(bool fp8, float *y, const void *w, const float *sw, const void *xdig, int n, int k, int m,
                          void *stream)
{
    const char *name = fp8 ? "be42_gemm_fp8_prepared" : "be42_gemm_q8_prepared";
    BE42_CHECK(y && w && sw && xdig, "%s: null pointer", name);
    BE42_CHECK(n > 0, "%s: bad shape n=%d", name, n);
    const be42_gemv_seg seg = {w, sw, y, n};
    return gemm_dig_run(fp8, &seg, 1, xdig, k, m, stream, name);
}

extern "C" int be42_gemm_prepared_multi(const be42_gemv_seg *segs, int nseg, const void *xdig, int k, int m, int fp8,
                                        void *stream)
{
    return gemm_dig_run(fp8 != 0, segs, nseg, xdig, k, m, stream, "be42_gemm_prepared_multi");
}

extern "C" int be42_gemm_q8_prepared(float *y, const int8_t *w, const float *w_scale, const void *xdig, int n, int k,
                                     int m, void *stream)
{
    return gemm_dig_entry(false, y, w, w_scale, xdig, n, k, m, stream);
}

extern "C" int be42_gemm_fp8_prepared(float *y, const uint8_t *w, const float *w_scale, const void *xdig, int n,
                                      int k, int m, void *stream)
{
    return gemm_dig_entry(true, y, w, w_scale, xdig, n, k, m, stream);
}
