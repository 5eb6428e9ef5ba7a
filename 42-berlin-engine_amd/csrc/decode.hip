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
#include <cmath>
#include <cstring>
#include <vector>

#include "be42_common.h"
#include "xdigits.h"

namespace be42 {

constexpr int kMaxBatch = 64;

struct TokArgs {
    int tok[kMaxBatch];
};

// tokens from the kernel argument, or (dev_tok != NULL) from the device
// argmax of the previous step
template <bool FP8>
__global__ __launch_bounds__(256) void k_embed(float *__restrict__ x, const uint8_t *__restrict__ emb,
                                               const float *__restrict__ emb_s, const TokArgs t,
                                               const int *__restrict__ dev_tok, int dim)
{
    const int b = blockIdx.y, i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= dim)
        return;
    const int tok = dev_tok ? dev_tok[b] : t.tok[b];
    const uint8_t c = emb[(size_t)tok * dim + i];
    const float v = FP8 ? fp8_to_f32(c) : (float)(int8_t)c;
    x[(size_t)b * dim + i] = v * emb_s[tok];
}

// block-wide max of non-negative values (blockDim.x a multiple of 64, <= 1024)
__device__ __forceinline__ float block_max(float v, float *red)
{
    v = wave_max(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0)
        red[wave] = v;
    __syncthreads();
    float r = 0.0f;
    for (int w = 0; w < nw; w++)
        r = fmaxf(r, red[w]);
    return r;
}

// Write row b of the GEMV digit planes from LDS values v[0..K) (zero past K).
template <bool FP8>
__device__ __forceinline__ void row_digits(const float *v, int K, uint8_t *dig, int B, int b, float *red)
{
    float m = 0.0f;
    for (int i = threadIdx.x; i < K; i += blockDim.x)
        m = fmaxf(m, fabsf(v[i]));
    const float amax = block_max(m, red);
    const float s = digit_scale<FP8>(amax);
    const int Kp = (int)xdig_kp(K, FP8);
    if (threadIdx.x == 0)
        xdig_scales(dig, K, B, FP8)[b] = s;
    for (int k0 = threadIdx.x * 4; k0 < Kp; k0 += blockDim.x * 4) {
        float xe[4];
#pragma unroll
        for (int e = 0; e < 4; e++)
            xe[e] = k0 + e < K ? v[k0 + e] : 0.0f;
        store_digit_words<FP8>(xe, s, dig, B, Kp, b, k0);
    }
}

// xn = rmsnorm(x [+ delta]) per row b, written as GEMV digit planes (and, if
// out != NULL, as fp32); with delta, x is updated in place first (the
// residual add of inference.c:525/:577 fused with the next norm).  The sum
// of squares follows compute_rms_f32_avx2: 8 FMA chains (chain l over
// i = l (mod 8), in order), ((s0+s4)+(s1+s5)) + ((s2+s6)+(s3+s7)), fused
// scalar remainder; ss / dim; inv = 1 / sqrtf(ss + eps); (x * inv) * w.
template <bool FP8>
__global__ __launch_bounds__(1024) void k_rmsnorm(float *__restrict__ out, uint8_t *__restrict__ dig,
                                                 float *__restrict__ x, const float *__restrict__ delta,
                                                 const uint16_t *__restrict__ w, int dim, int B, float eps)
{
    extern __shared__ float xs[];
    __shared__ float inv_s, red[16];
    const int b = blockIdx.x;
    float *xr = x + (size_t)b * dim;
    const float *dr = delta ? delta + (size_t)b * dim : nullptr;
    for (int i = threadIdx.x; i < dim; i += blockDim.x) {
        float v = xr[i];
        if (dr) {
            v = v + dr[i];
            xr[i] = v;
        }
        xs[i] = v;
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        const int main = dim & ~7;
        float s = 0.0f;
        if (lane < 8) {
            // 32 elements of the chain are loaded before their 32 dependent FMAs
            for (int c0 = 0; c0 < main; c0 += 8 * 32) {
                float v[32];
#pragma unroll
                for (int j = 0; j < 32; j++) {
                    const int i = c0 + lane + 8 * j;
                    v[j] = i < main ? xs[i] : 0.0f;
                }
#pragma unroll
                for (int j = 0; j < 32; j++)
                    s = __fmaf_rn(v[j], v[j], s);      // the zero padding adds exact zeros
            }
        }
        const float t = s + __shfl_down(s, 4, 8);
        const float u = t + __shfl_down(t, 1, 8);
        float ss = u + __shfl_down(u, 2, 8);
        if (lane == 0) {
            for (int i = main; i < dim; i++)
                ss = __fmaf_rn(xs[i], xs[i], ss);
            ss = __fdiv_rn(ss, (float)dim);
            inv_s = __fdiv_rn(1.0f, __fsqrt_rn(ss + eps));
        }
    }
    __syncthreads();
    const float inv = inv_s;
    for (int i = threadIdx.x; i < dim; i += blockDim.x) {
        const float v = (xs[i] * inv) * bf16_to_f32(w[i]);
        xs[i] = v;
        if (out)
            out[(size_t)b * dim + i] = v;
    }
    __syncthreads();
    row_digits<FP8>(xs, dim, dig, B, b, red);
}

// q [B][nq*hd], k [B][nk*hd] rotated at position pos (table rows [pos][hd/2])
__global__ __launch_bounds__(256) void k_rope(float *__restrict__ q, float *__restrict__ k,
                                              const float *__restrict__ cos_t, const float *__restrict__ sin_t,
                                              int pos, int nq, int nk, int hd)
{
    const int half = hd / 2, b = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (nq + nk) * half)
        return;
    const int h = i / half, j = i % half;
    float *base = h < nq ? q + ((size_t)b * nq + h) * hd : k + ((size_t)b * nk + (h - nq)) * hd;
    const float c = cos_t[(size_t)pos * half + j], s = sin_t[(size_t)pos * half + j];
    const float x0 = base[j], x1 = base[j + half];
    base[j] = __fmaf_rn(x0, c, -(x1 * s));
    base[j + half] = __fmaf_rn(x0, s, x1 * c);
}

// h = (g * sigmoid(g)) * u for row b (op_silu_mul_fused_f32): blocks of 8 use
// the vector Schraudolph exp (clamp, fused multiply-add, round to nearest),
// the n % 8 remainder the scalar one; written as GEMV digit planes of the
// down projection (and to out if not NULL).
template <bool FP8>
__global__ __launch_bounds__(1024) void k_silu_mul(float *__restrict__ out, uint8_t *__restrict__ dig,
                                                   const float *__restrict__ g, const float *__restrict__ u, int n,
                                                   int B)
{
    extern __shared__ float hs[];
    __shared__ float red[16];
    const int b = blockIdx.x;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float gv = g[(size_t)b * n + i], uv = u[(size_t)b * n + i];
        float e;
        if (i < (n & ~7)) {
            float xv = 0.0f - gv;
            xv = fmaxf(xv, -87.0f);
            xv = fminf(xv, 87.0f);
            e = __int_as_float(__float2int_rn(__fmaf_rn(xv, 12102203.0f, 1065353216.0f)));
        } else {
            e = fast_expf(-gv);
        }
        const float sig = __fdiv_rn(1.0f, 1.0f + e);
        const float h = (gv * sig) * uv;
        hs[i] = h;
        if (out)
            out[(size_t)b * n + i] = h;
    }
    __syncthreads();
    row_digits<FP8>(hs, n, dig, B, b, red);
}

// argmax_simd_f32: the maximum value wins; among equal maxima in the
// 8-lane part (indices below 8*floor(n/8), n >= 8) the lowest lane (i % 8),
// then the first index; tail entries win only with a strictly larger value.
__global__ __launch_bounds__(1024) void k_argmax(int *__restrict__ out, const float *__restrict__ logits, int n)
{
    __shared__ float redv[16], redt[16];
    __shared__ unsigned long long redk[16];
    __shared__ float vmax_s, tmax_s;
    const float *x = logits + (size_t)blockIdx.x * n;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int main = n < 8 ? 0 : (n & ~7);
    float vm = -INFINITY, tm = -INFINITY;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        if (i < main)
            vm = fmaxf(vm, x[i]);
        else
            tm = fmaxf(tm, x[i]);
    }
    vm = wave_max(vm);
    tm = wave_max(tm);
    if (lane == 0) {
        redv[wave] = vm;
        redt[wave] = tm;
    }
    __syncthreads();
    if (wave == 0) {
        float a = lane < nw ? redv[lane] : -INFINITY, t = lane < nw ? redt[lane] : -INFINITY;
        a = wave_max(a);
        t = wave_max(t);
        if (lane == 0) {
            vmax_s = a;
            tmax_s = t;
        }
    }
    __syncthreads();
    const float vmax = vmax_s, tmax = tmax_s;
    const bool tail_wins = main == 0 || tmax > vmax;
    const float target = tail_wins ? tmax : vmax;
    // smallest key among the winners: (lane, index) in the vector part, index in the tail
    unsigned long long key = ~0ull;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const bool in_vec = i < main;
        if (in_vec != tail_wins && x[i] == target) {
            const unsigned long long k =
                tail_wins ? (unsigned long long)i : ((unsigned long long)(i & 7) << 32) | (unsigned)i;
            key = k < key ? k : key;
        }
    }
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long other = __shfl_xor(key, o);
        key = other < key ? other : key;
    }
    if (lane == 0)
        redk[wave] = key;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long k = ~0ull;
        for (int w = 0; w < nw; w++)
            k = redk[w] < k ? redk[w] : k;
        out[blockIdx.x] = k == ~0ull ? 0 : (int)(k & 0xFFFFFFFFu);
    }
}

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
    void *attn_ws = nullptr;
    size_t attn_ws_bytes = 0;
    int *cand = nullptr, *ncand = nullptr;
    float *capture_q = nullptr;   // optional [n_layers][max_batch][n_heads * head_dim]
    int *capture_nsel = nullptr;  // optional [n_layers][max_batch] pages attended
};

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
                   c.max_batch > 0 && c.max_batch <= 16 && c.dim % 16 == 0 && c.hidden_dim % 16 == 0 &&
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
    alloc((void **)&d->next, (size_t)B * 4);
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
    if ((size_t)c.hidden_dim * 4 > 65536) {
        if (e == hipSuccess)
            e = hipFuncSetAttribute((const void *)k_silu_mul<true>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    c.hidden_dim * 4);
        if (e == hipSuccess)
            e = hipFuncSetAttribute((const void *)k_silu_mul<false>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    c.hidden_dim * 4);
    }
    if ((size_t)c.dim * 4 > 65536) {
        if (e == hipSuccess)
            e = hipFuncSetAttribute((const void *)k_rmsnorm<true>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    c.dim * 4);
        if (e == hipSuccess)
            e = hipFuncSetAttribute((const void *)k_rmsnorm<false>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    c.dim * 4);
    }
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
    if (d->pool)
        be42_kv_destroy(d->pool);
    void *ptrs[] = {d->cos_t, d->sin_t, d->x, d->xb, d->xn, d->q, d->k, d->v, d->att, d->hb, d->hb2, d->logits, d->sel,
                    d->nsel, d->slots, d->next, d->cand, d->ncand, d->xdig, d->attn_ws};
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

#define DEC_TRY(x)                                                                                                 \
    do {                                                                                                           \
        const int rc_ = (x);                                                                                       \
        if (rc_)                                                                                                   \
            return rc_;                                                                                            \
    } while (0)

extern "C" int be42_decoder_step(be42_decoder *d, const int *tokens, int batch, int pos, int *next_tokens,
                                 float *logits_out, void *stream)
{
    BE42_CHECK(d, "be42_decoder_step: null decoder");
    const be42_decoder_config &c = d->c;
    BE42_CHECK(batch > 0 && batch <= c.max_batch, "be42_decoder_step: batch %d (max %d)", batch, c.max_batch);
    BE42_CHECK(pos >= 0 && pos < c.max_seq, "be42_decoder_step: position %d (max %d)", pos, c.max_seq);
    hipStream_t st = as_stream(stream);
    const int B = batch, dim = c.dim, hd = c.head_dim, H = c.n_heads, KV = c.n_kv_heads;
    const int qd = H * hd, kd = KV * hd, fp8 = c.wkind;
    TokArgs ta;
    memset(&ta, 0, sizeof ta);
    for (int b = 0; tokens && b < B; b++) {
        BE42_CHECK(tokens[b] >= 0 && tokens[b] < c.vocab, "be42_decoder_step: token %d out of range", tokens[b]);
        ta.tok[b] = tokens[b];
    }
    // the device argmax of the previous step is always in [0, vocab)
    const int *dev_tok = tokens ? nullptr : d->next;
    const dim3 eg((dim + 255) / 256, B);
    if (fp8)
        hipLaunchKernelGGL(k_embed<true>, eg, dim3(256), 0, st, d->x, (const uint8_t *)d->w.emb, d->w.emb_s, ta,
                           dev_tok, dim);
    else
        hipLaunchKernelGGL(k_embed<false>, eg, dim3(256), 0, st, d->x, (const uint8_t *)d->w.emb, d->w.emb_s, ta,
                           dev_tok, dim);
    BE42_LAUNCH_CHECK();
    const size_t norm_lds = (size_t)dim * 4, silu_lds = (size_t)c.hidden_dim * 4;
    uint8_t *dig = (uint8_t *)d->xdig;
    // RMSNorm (+ residual) straight into the GEMV digit planes
    auto norm = [&](const uint16_t *wn, const float *delta) {
        if (fp8)
            hipLaunchKernelGGL(k_rmsnorm<true>, dim3(B), dim3(1024), norm_lds, st, nullptr, dig, d->x, delta, wn,
                               dim, B, c.norm_eps);
        else
            hipLaunchKernelGGL(k_rmsnorm<false>, dim3(B), dim3(1024), norm_lds, st, nullptr, dig, d->x, delta, wn,
                               dim, B, c.norm_eps);
        return hipGetLastError();
    };
    const float scale = 1.0f / sqrtf((float)hd);
    const float *pending = nullptr;   // residual delta not yet added to x
    int slot_ids[kMaxBatch], positions[kMaxBatch];
    for (int b = 0; b < B; b++)
        positions[b] = pos;
    const int pages = pos / 16 + 1;
    for (int l = 0; l < c.n_layers; l++) {
        const be42_decoder_layer &L = d->w.layers[l];
        BE42_HIP(norm(L.attn_norm, pending));
        DEC_TRY(gemv(d, d->q, L.wq, L.sq, qd, dim, B, st));
        DEC_TRY(gemv(d, d->k, L.wk, L.sk, kd, dim, B, st));
        DEC_TRY(gemv(d, d->v, L.wv, L.sv, kd, dim, B, st));
        if (pos < (c.rope_len > 0 ? c.rope_len : c.max_seq)) {   // no rotation past the table
            hipLaunchKernelGGL(k_rope, dim3(((H + KV) * (hd / 2) + 255) / 256, B), dim3(256), 0, st, d->q, d->k,
                               d->cos_t, d->sin_t, pos, H, KV, hd);
            BE42_LAUNCH_CHECK();
        }
        if (d->capture_q)
            BE42_HIP(hipMemcpyAsync(d->capture_q + (size_t)l * c.max_batch * qd, d->q, (size_t)B * qd * 4,
                                    hipMemcpyDeviceToDevice, st));
        for (int b = 0; b < B; b++)
            slot_ids[b] = l * c.max_batch + b;
        DEC_TRY(be42_kv_append_step(d->pool, slot_ids, positions, B, d->k, d->v, st));
        const int *lslots = d->slots + (size_t)l * c.max_batch;
        if (pages <= c.sparse_k) {
            // dense: every page in logical order, straight from the device page table
            const be42_kv_pool &P = *d->pool;
            DEC_TRY(be42_paged_attention(d->pool, d->q, B, H, P.page_table + (size_t)l * c.max_batch * P.max_logical,
                                         P.n_logical + (size_t)l * c.max_batch, P.max_logical, pages, scale,
                                         d->att, pages <= 64 ? 1 : 4, d->attn_ws, d->attn_ws_bytes, st));
        } else {
            const int stride = std::max(c.sparse_k, 64);
            DEC_TRY(be42_lsh_route(d->pool, d->q, lslots, B, H, c.sparse_k, c.cand_cap, d->sel, d->nsel, stride,
                                   d->cand, d->ncand, nullptr, st));
            DEC_TRY(be42_paged_attention(d->pool, d->q, B, H, d->sel, d->nsel, stride, c.sparse_k, scale, d->att,
                                         c.sparse_k <= 64 ? 1 : 4, d->attn_ws, d->attn_ws_bytes, st));
        }
        if (d->capture_nsel) {
            const int *src = pages <= c.sparse_k ? d->pool->n_logical + (size_t)l * c.max_batch : d->nsel;
            BE42_HIP(hipMemcpyAsync(d->capture_nsel + (size_t)l * c.max_batch, src, (size_t)B * 4,
                                    hipMemcpyDeviceToDevice, st));
        }
        DEC_TRY(be42_gemv_prepare(d->xdig, d->att, qd, B, fp8, st));
        DEC_TRY(gemv(d, d->xb, L.wo, L.so, dim, qd, B, st));
        BE42_HIP(norm(L.ffn_norm, d->xb));                 // x += attention output
        DEC_TRY(gemv(d, d->hb, L.w1, L.s1, c.hidden_dim, dim, B, st));
        DEC_TRY(gemv(d, d->hb2, L.w3, L.s3, c.hidden_dim, dim, B, st));
        if (fp8)
            hipLaunchKernelGGL(k_silu_mul<true>, dim3(B), dim3(1024), silu_lds, st, nullptr, dig, d->hb, d->hb2,
                               c.hidden_dim, B);
        else
            hipLaunchKernelGGL(k_silu_mul<false>, dim3(B), dim3(1024), silu_lds, st, nullptr, dig, d->hb, d->hb2,
                               c.hidden_dim, B);
        BE42_LAUNCH_CHECK();
        DEC_TRY(gemv(d, d->xb, L.w2, L.s2, dim, c.hidden_dim, B, st));
        pending = d->xb;
    }
    // final residual + norm, lm_head, argmax
    BE42_HIP(norm(d->w.final_norm, pending));
    float *lg = logits_out ? logits_out : d->logits;
    DEC_TRY(gemv(d, lg, d->w.out, d->w.out_s, c.vocab, dim, B, st));
    hipLaunchKernelGGL(k_argmax, dim3(B), dim3(1024), 0, st, d->next, lg, c.vocab);
    BE42_LAUNCH_CHECK();
    if (next_tokens)
        BE42_HIP(hipMemcpyAsync(next_tokens, d->next, (size_t)B * 4, hipMemcpyDeviceToHost, st));
    if (next_tokens)
        BE42_HIP(hipStreamSynchronize(st));
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
