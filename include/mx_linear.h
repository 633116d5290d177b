/*
 * mx_linear.h — C ABI of the projections on either side of the attention (MI355X, gfx950).
 *
 * Y = X W^T over f16 weights: the producer of the attention's inputs (the q|k|v projection, the Whisper decoder's
 * cross-attention key/value cache) and the consumer of its output (attn_output). Replaces, in dooms.cpp 0.6.1:
 *
 *   reference (file:line)                                                                  replaced by
 *   -------------------------------------------------------------------------------------  -------------------------
 *   matvec1  src/backend/metal/llama_kernels.h:96-126 (one token: "qkv" with the RMS norm,   mx_linear, M <= 8
 *       "attn_output" accumulating into the residual; metal_llama_decoder.mm:160-190,         (f32 input rows)
 *       318-325)
 *   matvecm  llama_kernels.h:809-842 (the Whisper decoder's prompt rows, M <= 8)              mx_linear, M <= 8
 *   matmul<TM,TN> / matmul_big + rms_scale  llama_kernels.h:164-300, 309-450 (prompt         mx_linear, M > 8
 *       chunks; metal_llama_decoder.mm:191-235, 346-352)                                      (half operands)
 *   encode_cross: matmul_big into scratch, then to_half into the cross cache                 mx_linear with
 *       (metal_whisper_decoder.mm:295-316, llama_kernels.h:772-775), per layer for K and V    MX_LINEAR_OUT_F16,
 *       (set_audio, metal_whisper_decoder.mm:505-513)                                         count = 2 n_layer
 *   MatvecParams / GemmParams (flags bits 0-2)  llama_kernels.h:28-34, 166-170                mx_linear_desc
 *
 * Arithmetic, as the reference's kernels: weights are f16, accumulation f32. With M <= 8 the input rows stay f32 (the
 * matvec kernels): y = (W . (x * gamma)) * rms_scale + bias. With M > 8 the input is rounded to half after the
 * normalization (the matmul kernels' staging, llama_kernels.h:186-199): y = W . half(x * gamma * rms_scale) + bias.
 * rms_scale = 1 / sqrt(mean(x^2) + eps) of the row (rms_scale, llama_kernels.h:312-328).
 *
 * Errors, streams and threading as mx_attn.h (the same codes and mx_attn_last_error()).
 */
#ifndef MX_LINEAR_H
#define MX_LINEAR_H

#include "mx_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Flags: bits 0-2 are the reference's GemmParams / MatvecParams flags (llama_kernels.h:31, 168). */
#define MX_LINEAR_RMS_NORM 1u    /* the input row is RMS-normalized and multiplied by gamma first */
#define MX_LINEAR_ACCUMULATE 2u  /* y += result (the residual stream) instead of y = result */
#define MX_LINEAR_BIAS 4u        /* + bias[n] */
#define MX_LINEAR_OUT_F16 8u     /* y is IEEE binary16 (a cache row), rounded once; otherwise f32 */

typedef struct mx_linear_desc {
    int32_t M;         /* input rows (tokens) */
    int32_t N;         /* output features = weight rows */
    int32_t K;         /* input features = weight columns; a multiple of 32 */
    uint32_t flags;    /* MX_LINEAR_* */
    int64_t x_stride;  /* floats between input rows (>= K, a multiple of 4) */
    int64_t y_stride;  /* elements between output rows (>= N; a multiple of 4 for f32, 8 for f16 output) */
    float eps;         /* RMS-norm epsilon (rms_eps) */
    int32_t reserved;  /* must be 0 */
} mx_linear_desc;

/*
 * Bytes of device workspace mx_linear needs for this descriptor: for M > 8, M * round_up(K, 64) halves (256-byte
 * rounded) for the input rows staged once as half(x * gamma * rms_scale) (the values the reference's matmul stages
 * per tile, with its rms_scale buffer folded in); 0 for M <= 8.
 */
MX_ATTN_API size_t mx_linear_workspace_bytes(const mx_linear_desc * desc);

/*
 * count products that share the input X and the shape: Y[i] = X W[i]^T (flags as desc). W, Y and bias are HOST arrays
 * of count device pointers (bias may be NULL without MX_LINEAR_BIAS; an entry may be NULL for no bias on that matrix).
 *
 *   W[i]     device, f16, [N][K] row-major (the reference's weight layout: row n is output feature n)
 *   X        device, f32, [M][x_stride]
 *   Y[i]     device, [M][y_stride], f32 or (MX_LINEAR_OUT_F16) f16
 *   gamma    device, f32 [K], with MX_LINEAR_RMS_NORM (else ignored)
 *   bias[i]  device, f32 [N], with MX_LINEAR_BIAS
 *
 * All device pointers 16-byte aligned. 1 <= count <= 64. Y[i] must not overlap X.
 */
MX_ATTN_API int32_t mx_linear(const mx_linear_desc * desc, int32_t count, const uint16_t * const * W, const float * X,
                              void * const * Y, const float * gamma, const float * const * bias, void * workspace,
                              size_t ws_bytes, mx_attn_stream stream);

#ifdef __cplusplus
}
#endif

#endif /* MX_LINEAR_H */
