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
    std::unordered_map<const t_block_manager *, be42_kv_pool *> pools;
    std::unordered_map<const t_lsh_ctx *, float *> ctx_hpT;
    struct Index {
        uint16_t *hash = nullptr;   // [LSH_MAX_BLOCKS]
        float *sum = nullptr;       // [LSH_MAX_DIM]
        int uploaded = 0;           // block hashes already on the device
    };
    std::unordered_map<const t_lsh_index *, Index> indexes;
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

be42_kv_pool *pool_of(const t_block_manager *bm, const char *what)
{
    Runtime &r = rt();
    auto it = r.pools.find(bm);
    if (it == r.pools.end())
        die(what, "block manager was not created by block_manager_init of this library");
    return it->second;
}

// host mirror of the pool's allocator state
void sync_manager(t_block_manager *bm, be42_kv_pool *pool)
{
    ok(be42_kv_export(pool, bm->page_table, bm->free_stack, &bm->free_top, bm->logical_len), "be42_kv_export");
}

const float *ctx_hpT(const t_lsh_ctx *ctx)
{
    Runtime &r = rt();
    auto it = r.ctx_hpT.find(ctx);
    if (it != r.ctx_hpT.end())
        return it->second;
    float *d = nullptr;
    hip_ok(hipMalloc((void **)&d, sizeof(ctx->hp_transposed)), "lsh ctx");
    hip_ok(hipMemcpy(d, ctx->hp_transposed, sizeof(ctx->hp_transposed), hipMemcpyHostToDevice), "lsh ctx upload");
    r.ctx_hpT[ctx] = d;
    return d;
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
    }
    return x;
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
    // b [k][n] -> x [n][k]; y [n][m] in chunks of 16 tokens; out = y^T [m][n]
    const float *bd = (const float *)in_dev(b->data, (size_t)k * n * 4, kS0);
    float *x = (float *)scratch(kS2, (size_t)n * k * 4);
    float *y = (float *)scratch(kS3, (size_t)n * m * 4);
    hipLaunchKernelGGL(k_transpose, dim3((n + 31) / 32, (k + 31) / 32), dim3(256), 0, nullptr, x, bd, k, n);
    hip_ok(hipGetLastError(), "op_matmul transpose");
    for (int c0 = 0; c0 < n; c0 += kGemvBatch) {
        const int bc = n - c0 < kGemvBatch ? n - c0 : kGemvBatch;
        ok(fp8 ? be42_gemv_fp8(y + (size_t)c0 * m, (const uint8_t *)w, ws, x + (size_t)c0 * k, m, k, bc, nullptr)
               : be42_gemv_q8(y + (size_t)c0 * m, (const int8_t *)w, ws, x + (size_t)c0 * k, m, k, bc, nullptr),
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
    std::lock_guard<std::mutex> g(rt().mu);
    Runtime &r = rt();
    auto it = r.ctx_hpT.find(ctx);
    if (it != r.ctx_hpT.end())
        hip_ok(hipMemcpy(it->second, ctx->hp_transposed, sizeof(ctx->hp_transposed), hipMemcpyHostToDevice),
               "lsh_init");
}

extern "C" void lsh_ctx_release(const t_lsh_ctx *ctx)
{
    std::lock_guard<std::mutex> g(rt().mu);
    Runtime &r = rt();
    auto it = r.ctx_hpT.find(ctx);
    if (it != r.ctx_hpT.end()) {
        hip_ok(hipDeviceSynchronize(), "lsh_ctx_release");
        hip_ok(hipFree(it->second), "lsh_ctx_release");
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
    if (acc->count == 0)
        acc->start_pos = pos;
    const float *dk = (const float *)in_dev(key, (size_t)dim * 4, kS0);
    hipLaunchKernelGGL(k_lsh_accumulate, dim3((dim + 255) / 256), dim3(256), 0, nullptr, x.sum, dk, dim);
    hip_ok(hipGetLastError(), "lsh_update");
    acc->count++;
    if (acc->count >= LSH_BLOCK_SIZE) {
        uint16_t *dh = (uint16_t *)scratch(kS1, 2);
        hipLaunchKernelGGL(k_lsh_commit, dim3(1), dim3(256), 0, nullptr, dh, x.sum, ctx_hpT(ctx), dim, ctx->dim,
                           acc->count);
        hip_ok(hipGetLastError(), "lsh_update");
        uint16_t h = 0;
        hip_ok(hipMemcpy(&h, dh, 2, hipMemcpyDeviceToHost), "lsh_update");
        lsh_insert_block(idx, h, acc->start_pos, acc->count);
        acc->count = 0;
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
    if (x.uploaded > nb)
        x.uploaded = 0;
    if (x.uploaded < nb)
        hip_ok(hipMemcpy(x.hash + x.uploaded, idx->block_hashes + x.uploaded, (size_t)(nb - x.uploaded) * 2,
                         hipMemcpyHostToDevice),
               "lsh_find_candidates");
    x.uploaded = nb;
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
    rt().pools[bm] = pool;
    return 0;
}

extern "C" void block_manager_free(t_block_manager *bm)
{
    std::lock_guard<std::mutex> g(rt().mu);
    Runtime &r = rt();
    auto it = r.pools.find(bm);
    if (it != r.pools.end()) {
        hip_ok(hipDeviceSynchronize(), "block_manager_free");
        be42_kv_destroy(it->second);
        r.pools.erase(it);
    }
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
