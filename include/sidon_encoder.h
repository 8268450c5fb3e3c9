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

/*
 * GLU of the pointwise conv's output: g[r, c] = h[r, c] * sigmoid(h[r, C + c])
 * for h [R, 2C] and g [R, C] fp16 (row-major, contiguous), math in fp32.
 * Replaces glu / _glu_kernel of src/sidon_triton/triton_encoder.py:113-133.
 */
int sidon_glu(const void* h, void* g, int R, int C, sidon_stream_t stream);

/*
 * In-place SiLU of n fp16 values: h = h * sigmoid(h), math in fp32.  Replaces
 * the in-place F.silu of the feed-forward modules
 * (src/sidon_triton/triton_encoder.py:485-486, :505-506).
 */
int sidon_silu(void* h, int64_t n, sidon_stream_t stream);

/*
 * Causal depthwise conv + LayerNorm + SiLU over B items of T frames:
 *
 *   out[b, t, c] = silu(LN_c(sum_{k<K} dwt[k, c] * g[b, t + k - (K-1), c]))
 *
 * with g = 0 before frame 0 (left padding of K - 1 frames) and LN over the C
 * channels (fp32, biased variance, weights ln_w / ln_b fp32 [C]).  g is
 * src [B*T, C] fp16 when glu_input == 0; when glu_input != 0, src is the
 * pointwise conv's output h [B*T, 2C] fp16 and g = GLU(h) is formed on the fly,
 * rounded to fp16 as sidon_glu stores it.  dwt [K, C] fp32, out [B*T, C] fp16.
 * C even in [2, 2048]; K in {3, 7, 15, 31}; fp16 pointers 4-byte aligned, fp32
 * pointers 8-byte aligned.  Replaces causal_dw_norm / _causal_dw_norm_kernel of
 * src/sidon_triton/triton_encoder.py:136-181 (glu_input = 0 is that
 * signature; glu_input = 1 also absorbs :120-133).
 */
int sidon_causal_dw_norm(const void* src, int glu_input, const float* dwt, const float* ln_w,
                         const float* ln_b, float eps, void* out, int B, int T, int C, int K,
                         sidon_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SIDON_ENCODER_H */
