/*
 * sidon_flexrel.h -- C ABI of the MI355X (gfx950) relative_key flash attention.
 *
 * Math (per batch b, head h, query row i in [0, L), head_dim 64):
 *
 *   s_ij = ( q_i . k_j  +  q_i . rel[ clamp(j - i, -64, +8) + 64 ] ) / 8
 *   o_i  = sum_{j < LK_b} softmax_j(s_ij) v_j        (keys j >= LK_b weigh 0)
 *
 * LK_b = lens[b] (device int32), or L when lens is NULL.  Every query row
 * i < L is computed and stored, including rows i >= LK_b (bucket padding);
 * callers compare only rows i < LK_b.  Inside the kernel LK_b is clamped to
 * [0, L], so an out-of-range length never reads past the buffers; a row with
 * LK_b == 0 is written as zeros (the reference would produce 0/0 = NaN).
 *
 * Arithmetic: fp16 operands, fp32 MFMA accumulation, fp32 online softmax in
 * base-2 units, probabilities rounded to fp16 before the PV product, fp16
 * output.
 *
 * Conventions shared by every entry point:
 *   - all tensors are device pointers owned by the caller; the library keeps
 *     no per-call state and allocates nothing;
 *   - strides are in ELEMENTS, ordered (batch, head, row); the head-dim
 *     stride is 1 (64 contiguous fp16 per row);
 *   - base pointers must be 16-byte aligned and every stride a multiple of 8
 *     elements (each 64-wide row is read as 16-byte vectors);
 *   - work is enqueued on `stream` (a hipStream_t; NULL = the legacy default
 *     stream) with no host synchronisation and no host read of device data,
 *     so calls may be captured into a HIP graph;
 *   - return value: SIDON_OK (0) or a negative SIDON_E_* code; nothing is
 *     launched when an argument is rejected.  sidon_last_error() returns a
 *     thread-local description of the last failure.
 */
#ifndef SIDON_FLEXREL_H
#define SIDON_FLEXREL_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t without pulling in the HIP headers. */
typedef struct ihipStream_t* sidon_stream_t;

#define SIDON_FLEXREL_HEAD_DIM 64
#define SIDON_FLEXREL_LEFT 64
#define SIDON_FLEXREL_RIGHT 8
#define SIDON_FLEXREL_NUM_POS 73

#define SIDON_OK 0
#define SIDON_E_NULL (-1)      /* a required pointer is NULL */
#define SIDON_E_SHAPE (-2)     /* B, H, L or head_dim out of range */
#define SIDON_E_STRIDE (-3)    /* stride not a multiple of 8 or too large */
#define SIDON_E_ALIGN (-4)     /* base pointer not 16-byte aligned */
#define SIDON_E_LAUNCH (-5)    /* the HIP launch itself failed */
#define SIDON_E_DEVICE (-6)    /* no usable HIP device / wrong architecture */
#define SIDON_E_CONFIG (-7)    /* SIDON_FLEXREL_VARIANT names no kernel (split8, w64, w32, auto) */

/*
 * Strided [B, H, L, 64] attention.
 *
 * Replaces the Triton launcher behind
 *   flexrel_attention(q, k, v, r, out=None)   src/sidon_triton/flexrel_triton.py:249-278
 * (q/k/v/out [B,H,L,64] with arbitrary batch/head/row strides, r [73,64]
 * contiguous), extended with the key-length vector `lens` of
 *   _flexrel_body(..., LENS, ...)             src/sidon_triton/triton_encoder.py:210-226
 * (NULL = no padding, the flexrel_triton.py behaviour).
 *
 * q_strides/k_strides/v_strides/o_strides: int64[3] = (batch, head, row).
 * rel: [73, 64] fp16 contiguous.  head_dim must be 64.
 */
int sidon_flexrel_fwd(const void* q, const void* k, const void* v,
                      const void* rel, const int32_t* lens, void* out,
                      int B, int H, int L, int head_dim,
                      const int64_t* q_strides, const int64_t* k_strides,
                      const int64_t* v_strides, const int64_t* o_strides,
                      sidon_stream_t stream);

/*
 * Encoder layout: fused QKV GEMM output in, context rows out.
 *
 * Replaces
 *   flexrel_attention(qkv, batch, heads, rel, lens)   src/sidon_triton/triton_encoder.py:346-371
 * qkv: [B*L, 3*H*64] fp16 row-major (q | k | v column blocks, head h at
 * columns h*64 of each block), out: [B*L, H*64] fp16 row-major, rel [73,64]
 * fp16, lens int32 [B] on the device (NULL = every item has L valid keys).
 */
int sidon_flexrel_fwd_qkv(const void* qkv, const void* rel,
                          const int32_t* lens, void* out,
                          int B, int H, int L, sidon_stream_t stream);

/*
 * Launch shape chosen for a given (B, H, L): queries per workgroup and the
 * number of key splits merged inside a workgroup.  Host function: it
 * launches nothing and reads the current device's compute-unit count once
 * (hipGetDeviceProperties); exposed so tests and benchmarks can report it.
 * It reports the shape of calls whose K and V rows share one row stride
 * (the fused QKV layout of sidon_flexrel_fwd_qkv); sidon_flexrel_fwd with K
 * and V rows of different strides launches 64 rows x 8 key splits (512
 * threads) instead.  Returns SIDON_E_CONFIG when SIDON_FLEXREL_VARIANT holds
 * an unknown value.  Has no counterpart in the reference (Triton picks
 * BLOCK_M/BLOCK_N at src/sidon_triton/triton_encoder.py:340-343).
 */
int sidon_flexrel_launch_shape(int B, int H, int L, int* queries_per_block,
                               int* key_splits, int* workgroups,
                               int* threads_per_block);

/*
 * Test hook.  With `on` nonzero, every wavefront of the 64-row kernel
 * discards what its hand-scheduled key-step loop computed and runs its steps
 * again through the kernel's compiled general code -- the path a wavefront
 * takes when a probability leaves the fp16 range -- so that tests can require
 * the two to agree bit for bit on every row.  Process-wide; read by every
 * sidon_flexrel_fwd / sidon_flexrel_fwd_qkv call (a captured graph keeps the
 * value of its capture).  Slower; never needed in production.  Has no
 * counterpart in the reference.
 */
void sidon_flexrel_debug_rerun_all(int on);

/* Thread-local text of the last error ("" when none). */
const char* sidon_last_error(void);

/* Library version string, e.g. "sidon-flexrel 0.3.0 gfx950". */
const char* sidon_version(void);

#ifdef __cplusplus
}
#endif

#endif /* SIDON_FLEXREL_H */
