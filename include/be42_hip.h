/*
 * be42_hip.h -- device-level C ABI of the gfx950 decode hot-path library
 * (lib42be_hip.so).
 *
 * Every pointer argument is device memory (HBM) unless stated otherwise and
 * every entry point enqueues its work on `stream` (a hipStream_t, NULL for
 * the default stream) and returns without synchronising.  Return value:
 * BE42_OK or a negative BE42_E* code; be42_last_error() then holds a message.
 *
 * The reference-signature entry points built on top of these (op_matmul,
 * paged_kv_append, lsh_hash, op_paged_attention_sparse, ...) are declared in
 * be42_ref_abi.h.
 */
#ifndef BE42_HIP_H
#define BE42_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BE42_OK        0
#define BE42_EINVAL   (-1)
#define BE42_EHIP     (-2)
#define BE42_ENOMEM   (-3)
#define BE42_ENODEV   (-4)

/* ---- runtime plumbing ----------------------------------------------------- */
/* Select `device` for the calling thread and upload the constant tables. */
int         be42_init(int device);
const char *be42_last_error(void);
int         be42_device_count(void);
int         be42_sync(void *stream);
void       *be42_malloc(size_t bytes);
int         be42_free(void *ptr);
int         be42_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream);
int         be42_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream);
int         be42_memset(void *dst, int value, size_t bytes, void *stream);

/* ---- quant codecs ------------------------------------------------------------
 * Row-wise versions of quant_f32_to_int8 (src/compute/ops_quant.c:229-270) and
 * quant_f32_to_fp8 (ops_quant.c:103-136): one scale per row of `cols` values.
 * Codes and scales are bit-identical to the reference. */
int be42_quant_rows_int8(int8_t *q, float *scales, const float *x, int rows, int cols, void *stream);
int be42_quant_rows_fp8(uint8_t *q, float *scales, const float *x, int rows, int cols, void *stream);
/* (float)q * scale[row], dequant_int8_to_f32_avx2 (ops_quant.c:275-305) row-wise */
int be42_dequant_rows_int8(float *out, const int8_t *q, const float *scales, int rows, int cols,
                           void *stream);
/* g_fp8_lut[q] (ops_quant.c:18-63): E4M3 with bias 7 and no NaN (0x7F -> 480) */
int be42_fp8_decode(float *out, const uint8_t *q, size_t n, void *stream);

/* ---- decode GEMV ---------------------------------------------------------------
 * y[b*n + i] = w_scale[i] * sum_j w[i*k + j] * x[b*k + j] for b < batch <= 16:
 * per-output-row scaled INT8 or FP8 E4M3 weights [n][k] against fp32
 * activations [batch][k], fp32 output [batch][n].  Replaces the n == 1 GEMV of
 * op_matmul (src/compute/ops_matmul.c:366-417, matvec_bf16_f32_blocked :57)
 * for the quantized weight dtypes. */
int be42_gemv_q8(float *y, const int8_t *w, const float *w_scale, const float *x,
                 int n, int k, int batch, void *stream);
int be42_gemv_fp8(float *y, const uint8_t *w, const float *w_scale, const float *x,
                  int n, int k, int batch, void *stream);

/* The same GEMV in two steps, for callers that reuse one activation for
 * several weight matrices (q/k/v, gate/up) or time the weight stream alone:
 * be42_gemv_prepare splits x [batch][k] (k % 16 == 0, batch <= 16) into the
 * MFMA digit planes held in `xdig` (be42_gemv_xdig_bytes(k, batch, fp8) bytes
 * of device memory); be42_gemv_{q8,fp8}_prepared then stream the weights. */
size_t be42_gemv_xdig_bytes(int k, int batch, int fp8);
int be42_gemv_prepare(void *xdig, const float *x, int k, int batch, int fp8, void *stream);
int be42_gemv_q8_prepared(float *y, const int8_t *w, const float *w_scale, const void *xdig,
                          int n, int k, int batch, void *stream);
int be42_gemv_fp8_prepared(float *y, const uint8_t *w, const float *w_scale, const void *xdig,
                           int n, int k, int batch, void *stream);

#ifdef __cplusplus
}
#endif
#endif
