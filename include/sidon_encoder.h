/*
 * sidon_encoder.h -- C ABI of the encoder pieces around the attention
 * (MI355X / gfx950), in the same library as sidon_flexrel.h and under the
 * same conventions (device pointers owned by the caller, work enqueued on
 * `stream` with no host synchronisation and no allocation, SIDON_OK or a
 * negative SIDON_E_* code, sidon_last_error()).
 */
#ifndef SIDON_ENCODER_H
#define SIDON_ENCODER_H

#include "sidon_flexrel.h"

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Residual add + LayerNorm over the rows of the fp32 stream x [R, C]
 * (row-major, contiguous), in place.  Replaces res_norm / _res_norm_kernel of
 * src/sidon_triton/triton_encoder.py:61-100 (the op the encoder runs before
 * and after every residual GEMM, e.g. :491-503):
 *
 *   x_r  = x_r + bias + y_r          bias [C] fp32 and y [R, C] fp32, each optional (NULL)
 *   x_r  = LN1(x_r)                  if n1_w != NULL
 *   x_r is stored back               if write_x != 0
 *   xn_r = LN2(x_r)                  if n2_w != NULL; xn [R, C] fp16 (xn_fp16 != 0) or fp32
 *
 * LN(v) = (v - mean) * rsqrt(var + eps) * w + b over the C columns (biased
 * variance), weights and biases fp32 [C].  C must be a multiple of 4 in
 * [4, 2048]; fp32 pointers 16-byte aligned, an fp16 xn 8-byte aligned.
 */
int sidon_res_norm(float* x, const float* y, const float* bias, const float* n1_w, const float* n1_b,
                   float eps1, int write_x, const float* n2_w, const float* n2_b, float eps2, void* xn,
                   int xn_fp16, int R, int C, sidon_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SIDON_ENCODER_H */
