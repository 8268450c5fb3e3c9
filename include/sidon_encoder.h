/*
 * sidon_encoder.h -- C ABI of the encoder pieces around the attention
 * (MI355X / gfx950), in the same library as sidon_flexrel.h and under the
 * same conventions (device pointers owned by the caller, work enqueued on
 * `stream` with no host synchronisation and no allocation, SIDON_OK or a
 * negative SIDON_E_* code, sidon_last_error()).
 */
#ifndef SIDON_ENCODER_H
#define SIDON_ENCODER_H

#include <stddef.h>

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
 * (src/sidon_triton/triton_encoder.py:498-499, :507-508).
 */
int sidon_silu(void* h, int64_t n, sidon_stream_t stream);

/*
 * The feed-forward module's input projection with its bias and SiLU fused:
 *
 *   y[m, n] = act(fp16(x[m, :] . w[n, :] + bias[n]))     act: 1 = SiLU, 0 = none
 *
 * x [M, K] and w [N, K] fp16 (row strides ldx, ldw; both K-contiguous),
 * fp32 sums, y [M, N] fp16 (row stride ldy); bias fp16 [N] or NULL.  SiLU
 * is taken in fp32 on the fp16-rounded sum and rounded to fp16, as
 * sidon_silu does after a separate GEMM.  Replaces the torch.addmm(b1, xn,
 * W1^T) + in-place F.silu pair of src/sidon_triton/triton_encoder.py:498-499
 * and :507-508.  Shapes: M >= 1, N a multiple of 256, K a multiple of 64;
 * strides multiples of 8; x, w, y 16-byte aligned, bias 8-byte aligned.
 * sidon_gemm_bias_act_fits(M, N, K) says whether a shape is supported (pure
 * host function); sidon_gemm_bias_act_preferred(M, N, K) whether the kernel
 * is expected to beat a library GEMM followed by sidon_silu on the current
 * device (its 320 x 256 tiles keep >= 3/4 of the CUs busy in every round).
 * Neither has a counterpart in the reference.
 */
int sidon_gemm_bias_act_fits(int M, int N, int K);
int sidon_gemm_bias_act_preferred(int M, int N, int K);
int sidon_gemm_bias_act(const void* x, int ldx, const void* w, int ldw, const void* bias, void* y, int ldy,
                        int M, int N, int K, int act, sidon_stream_t stream);

/*
 * The same projection on hipBLASLt, for the shapes where the kernel above
 * leaves CUs idle:
 *
 *   y[m, n] = act(x[m, :] . w[n, :] + bias[n])     act: 1 = SiLU, 0 = none
 *
 * x [M, K], w [N, K] fp16 (row strides ldx, ldw; K-contiguous), fp32 sums,
 * bias fp16 [N] or NULL, y [M, N] fp16 (row stride ldy).  The bias and the
 * SiLU run in hipBLASLt's epilogue on the fp32 sum, with one rounding to
 * fp16 (the kernel above and the reference round the biased sum to fp16
 * before the SiLU: the two differ by at most about one fp16 ulp).  Replaces
 * the torch.addmm(b1, xn, W1^T) + in-place F.silu pair of
 * src/sidon_triton/triton_encoder.py:498-499 and :507-508.  Shapes: M, N,
 * K >= 1, strides >= the row lengths, every operand 2-byte aligned.  The
 * kernel is hipBLASLt's first heuristic choice that needs no workspace,
 * kept per problem; the first call on a device creates its hipBLASLt handle
 * and must not run during stream capture.
 */
int sidon_gemm_lt_act(const void* x, int ldx, const void* w, int ldw, const void* bias, void* y, int ldy, int M,
                      int N, int K, int act, sidon_stream_t stream);

/*
 * Residual projection, accumulated into the fp32 stream in place:
 *
 *   y[m, n] += x[m, :] . w[n, :]        m < M, n < N, fp32 sums
 *
 * x [M, K] and w [N, K] fp16 row-major (K contiguous: activations and a torch
 * Linear weight), y [M, N] fp32 row-major, updated in place.  Replaces the
 * torch.addmm(x, a, w.t(), out_dtype=torch.float32, out=x) of res(),
 * src/sidon_triton/triton_encoder.py:491-492.  64 x 64 output tiles, K split
 * over the workgroup's 4 wavefronts and summed in a fixed order: the result
 * does not depend on timing.  Shapes: M >= 1, N a multiple of 64, K a
 * multiple of 128; ldx, ldw multiples of 8 and >= K, ldy a multiple of 4 and
 * >= N; x, w, y 16-byte aligned; x and w must not overlap y (checked on the byte ranges
 * the call touches: SIDON_E_SHAPE).  sidon_gemm_res_fits(M, N, K) says whether
 * a shape is supported (pure host function); sidon_gemm_res_preferred(M, N,
 * K) whether the kernel is expected to beat a library GEMM on the current
 * device (its tiles fit one per compute unit).  Neither has a counterpart in
 * the reference.
 */
int sidon_gemm_res_fits(int M, int N, int K);
int sidon_gemm_res_preferred(int M, int N, int K);
int sidon_gemm_res(const void* x, int ldx, const void* w, int ldw, float* y, int ldy, int M, int N, int K,
                   sidon_stream_t stream);

/*
 * Plain GEMM on rocBLAS with the kernel chosen per problem by timing:
 *
 *   y[m, n] = x[m, :] . w[n, :] + beta * y[m, n]      m < M, n < N, fp32 sums
 *
 * x [M, K] and w [N, K] row-major with row strides ldx, ldw >= K (K
 * contiguous); y [M, N] row-major with row stride ldy >= N.  dtype 0: fp32
 * x, w, y; 1: fp16 x, w, y (beta must be 0); 2: fp16 x, w and fp32 y.
 * Used for the pointwise conv's first F.linear of the encoder
 * (src/sidon_triton/triton_encoder.py:504; dtype 1) and the framing matmul
 * of the front end (src/sidon_triton/frontend.py:222; dtype 0).  dtype 2
 * with beta 1 is the form of the residual projections of res() (:491-492),
 * which the encoder keeps on torch.addmm.
 *
 * sidon_gemm_nt runs the kernel recorded for the problem (shape, strides,
 * dtype, beta != 0) by sidon_gemm_nt_tune or sidon_gemm_nt_pin, else
 * rocBLAS's default.  The tuner times rocBLAS's default and every solution
 * it lists for the problem, on scratch: y and y_check are two distinct buffers of y's
 * shape and row stride (both overwritten; y's contents are the beta term
 * while timing).  It records for the current device the fastest kernel whose
 * product agrees with the default's -- at beta = 0 and, when beta != 0, with
 * the problem's beta from identical contents; fp32 output: every row and
 * column within 1e-5 relative; fp16 output: every element within one fp16
 * ulp and the whole within 1e-4 -- and writes its solution index to
 * *solution_out (INT_MIN: the default) when that is not NULL.  When rocBLAS
 * lists no kernel or none passes that gate, it records
 * rocBLAS's default and returns SIDON_OK (SIDON_GEMM_TUNE_FORCE_FALLBACK=1
 * takes that path for every problem, for tests).  Each candidate's timed
 * calls are queued behind a short hold kernel (one lane, 400 us) so that
 * they run back to back on the device and its own speed is measured, not
 * the host's launch rate.  The tuner
 * synchronises the stream and fails during stream capture; tune before
 * capturing.  Every candidate is deterministic (rocBLAS atomics disabled),
 * but the choice is by timing, so two processes may keep different kernels
 * (outputs differing in the last bits).  Each device's rocBLAS handle gets a
 * fixed 32 MiB workspace, allocated on the first call on that device and
 * never freed, so graphs never point at memory rocBLAS has freed; any kernel
 * may use it (rocBLAS answers no workspace-size query for these GEMMs), so
 * calls on two streams of one device must not overlap.  Neither function has a
 * counterpart in the reference.
 */
int sidon_gemm_nt(const void* x, int ldx, const void* w, int ldw, void* y, int ldy, int M, int N, int K, int dtype,
                  float beta, sidon_stream_t stream);
int sidon_gemm_nt_tune(const void* x, int ldx, const void* w, int ldw, void* y, void* y_check, int ldy, int M,
                       int N, int K, int dtype, float beta, sidon_stream_t stream, int* solution_out);
/*
 * Record rocBLAS solution `solution` (an index sidon_gemm_nt_tune returned
 * in an earlier run; INT_MIN = rocBLAS's default) for the problem
 * (M, N, K, ldx, ldw, ldy, dtype, beta != 0) on the current device, so runs
 * are reproducible.  The first sidon_gemm_nt call of the problem fails with
 * SIDON_E_SHAPE, before running anything, if rocBLAS does not list the kernel
 * for this exact problem (shape, strides, types).  No counterpart in the
 * reference.
 */
int sidon_gemm_nt_pin(int M, int N, int K, int ldx, int ldw, int ldy, int dtype, int beta_nonzero,
                      int solution);
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

/*
 * Fbank framing: frames[b, f, i] = chunk[b, 160 f + i - 160] (0 outside
 * [0, S)) for f < F = S / 160, i < 400 -- the (160, 160) edge padding and the
 * 400-sample frames with hop 160 of frontend.py:219-221, ready for the framing
 * GEMM with the [400, 514] transform.  chunk [B, S] fp32 (S a positive
 * multiple of 320), frames [B, F, 400] fp32, 16-byte aligned.
 */
int sidon_fbank_frames(const float* chunk, float* frames, int B, int S, sidon_stream_t stream);

/*
 * Fbank front end, after the framing GEMM.  Replaces the log-mel part of
 * SeamlessFbank._masked, src/sidon_triton/frontend.py:218-229:
 *
 *   logmel[r, m] = log(max(sum_k mel[k, m] * (spec[r, k]^2 + spec[r, 257 + k]^2), 1.192092955078125e-07))
 *
 * spec [R, 514] fp32 (real 257 | imaginary 257 of each frame's 512-point
 * rDFT, as the framing GEMM writes it), logmel [R, 80] fp32.  The mel bank
 * is passed sparse: triangle m covers bins [mel_lo[m], mel_lo[m] + mel_len[m])
 * with weights mel_w[m * max_len + i]; 1 <= max_len <= 257.
 */
int sidon_fbank_logmel(const float* spec, const float* mel_w, const int* mel_lo, const int* mel_len, int max_len,
                       float* logmel, int R, sidon_stream_t stream);

/* Bytes of the workspace sidon_fbank_normalize needs for B items of F frames. */
size_t sidon_fbank_workspace_bytes(int B, int F);

/*
 * Per-bin normalization of B items of F frames (F even: a bucket of 160 F
 * samples), replacing frontend.py:230-240.  valid [B] int32 on the device
 * holds each item's true sample count; its true frames are
 * tf = 1 + (valid + 320 - 400) / 160 (floor, clamped to [0, F]).  For every mel
 * bin, over the frames f < tf:
 *
 *   feats[b, f, m] = (logmel[b, f, m] - mean) / sqrt(var + 1e-7)      (var with ddof 1)
 *
 * feats[b, tf, m] = 1.0 when tf is odd (the extractor's pad frame), and 0 for
 * every later frame.  feats [B, F, 80] fp32 is also the stacked
 * [B, F / 2, 160] encoder input.  workspace: device memory of at least
 * sidon_fbank_workspace_bytes(B, F) bytes (overwritten); feats must not alias
 * logmel.  tf = 1 gives 0/0 like the reference.
 */
int sidon_fbank_normalize(const float* logmel, const int* valid, float* workspace, size_t workspace_bytes,
                          float* feats, int B, int F, sidon_stream_t stream);

/*
 * sidon_fbank_normalize without a workspace argument: the same kernels and
 * results (bit for bit), with the statistics held in a static device array
 * of the library (1.9 MiB per device, kept until the process ends) instead
 * of caller memory.  No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops).  It allocates nothing and calls no allocating routine.  B <= 32
 * items (any F); larger B returns SIDON_E_SHAPE.  Every call on one device
 * shares that device's array, so calls that overlap on one GPU (two streams,
 * two threads) race; every word a call reads is written earlier in the same
 * call, so consecutive calls need no clearing.  The first call on a device
 * looks up the array's device address (hipGetSymbolAddress, once per device)
 * and must run outside stream capture; later calls launch three kernels and
 * nothing else (no memset, no copy), so they may be captured into a graph.
 */
int sidon_fbank_normalize_noalloc(const float* logmel, const int* valid, float* feats, int B, int F,
                                  sidon_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SIDON_ENCODER_H */
