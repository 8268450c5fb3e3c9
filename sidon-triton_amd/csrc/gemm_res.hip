// gemm_res.hip -- the encoder's residual projections, accumulated into the
// fp32 residual stream in place (MI355X / gfx950).
//
//   Y[m, n] += X[m, :] . W[n, :]       X [M, K], W [N, K] fp16 (K contiguous), Y [M, N] fp32
//
// This is the torch.addmm(x, a, w.t(), out_dtype=torch.float32, out=x) of the
// res() helper of src/sidon_triton/triton_encoder.py:491-492, called four
// times per layer (feed-forward outputs with K = 4096, attention
// out-projection and pointwise conv 2 with K = 1024; N = 1024).  At the
// encoder's short chunks (M = 750-1500 rows) a library GEMM's large tiles
// leave most compute units idle (M = 750, N = 1024: 48 tiles of 128 x 128 for
// 256 CUs), so this kernel uses small output tiles and splits K inside the
// workgroup instead.
//
// Tiling.  A workgroup owns a 64 x 64 tile of Y and runs 8 wavefronts (two
// per SIMD, so one's LDS reads overlap the other's products).  The K loop
// walks 128-wide slices: the X and W slices are copied global -> LDS with
// global_load_lds_dwordx4 into a ring of kStages buffers (copies of the next
// kStages - 1 slices in flight), and wavefront w takes k16 step w of every
// slice for the whole 64 x 64 tile (2 x 2 blocks of v_mfma_f32_32x32x16_f16,
// Y^T = W . X^T, so a lane holds four consecutive columns of one row).  At
// the end wavefront w + 4 hands its partial tile to wavefront w through LDS,
// the four sums meet in LDS, and each wavefront adds 8 rows of them in
// wavefront order to Y and stores Y: the result does not depend on timing,
// and the only difference from a one-pass GEMM is the summation order.
// 16-byte chunk c of the 128-byte LDS row r sits at chunk c ^ ((r >> 1) & 7),
// so the operand reads (16 rows per 16 lanes) are bank-conflict free.
//
// Measured on MI355X (N = 1024, graph replays): M = 750: 8.1 us at K = 1024
// and 16.8 us at K = 4096, against 9.4 and 19.5 us for torch.addmm
// (hipBLASLt); from M = 1500 on (more tiles than compute units) the library's
// larger tiles win (13.6 against 10.7 us, 29.7 against 22.9 us), so the
// encoder calls this kernel only while its tiles fit one per compute unit.
// 4 wavefronts: 5-15% slower; tiles with the row tile fastest over the whole
// grid instead of in groups of 4: level at M = 750, 20-40% slower from 3000.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "sidon_encoder.h"
#include "sidon_host.h"

#define SIDON_API extern "C" __attribute__((visibility("default")))
#define SIDON_INLINE __attribute__((always_inline))

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kTile = 64;                          // rows of X and of W per workgroup
constexpr int kSliceK = 128;                       // K per ring buffer
constexpr int kStages = 3;
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kSteps = kSliceK / 16;               // k16 steps per slice
constexpr int kStepsPerWave = kSteps / kWaves;
constexpr int kRowBytes = 128;                     // one LDS row: 64 halves of K
constexpr int kHalves = kSliceK / 64;              // 128-byte row halves per slice row
constexpr int kOperand = kTile * kHalves * kRowBytes;   // bytes of the X (or W) part of a stage
constexpr int kStage = 2 * kOperand;
constexpr int kCopies = kStage / 1024;             // 1 KB copy instructions per slice
constexpr int kCopiesPerWave = kCopies / kWaves;
constexpr int kRedStride = 68;                     // fp32 per row of a partial tile in LDS
constexpr int kRedParts = 4;                       // partial tiles in LDS at once
constexpr int kRedBytes = kRedParts * kTile * kRedStride * 4;
constexpr int kRowsPerWave = kTile / kWaves;       // rows each wavefront finishes
constexpr int kLanesPerRow = 64 / kRowsPerWave;
constexpr int kColsPerLane = kTile / kLanesPerRow;
constexpr int kGroupM = 4;                         // tile order: groups of kGroupM row tiles, N next
constexpr int kLdsBytes = kStages * kStage > kRedBytes ? kStages * kStage : kRedBytes;
static_assert(kSteps % kWaves == 0 && kCopies % kWaves == 0, "even split over the wavefronts");
static_assert(kWaves == kRedParts || kWaves == 2 * kRedParts, "4 or 8 wavefronts");
static_assert(kLdsBytes <= 160 * 1024, "LDS budget of one CU");

#define LDS_PTR(T, p) ((__attribute__((address_space(3))) T*)(p))

struct ResParams {
  const _Float16* x;
  const _Float16* w;
  float* y;
  int ldx, ldw, ldy;  // row strides (elements)
  int M, N, K;
  int tiles_m;
};

__device__ __forceinline__ int row_swz(int r) { return (r >> 1) & 7; }

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// Copy of 1 KB (8 rows of 128 bytes) global -> LDS; lane l's 16 bytes land at
// lds_addr + 16 l.  Completion is awaited with wait_vmcnt.
__device__ __forceinline__ void dma_1k(uint32_t lds_addr, const char* gbase, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :: "s"(lds_addr), "v"(voff), "s"(gbase) : "memory", "m0");
}
#pragma clang diagnostic pop

template <int N>
__device__ __forceinline__ void wait_vmcnt() { asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory"); }

// Wait until the oldest slice in flight has landed while the `newer` slices
// issued after it (kPer copies each) stay in flight.
template <int kPer, int kMax>
__device__ __forceinline__ void wait_slice(int newer) {
  if constexpr (kMax > 0) {
    if (newer >= kMax) {
      wait_vmcnt<kPer * kMax>();
      return;
    }
    wait_slice<kPer, kMax - 1>(newer);
  } else {
    (void)newer;
    wait_vmcnt<0>();
  }
}

// Barrier after this wavefront's LDS reads have retired (no vmcnt wait: the
// copies of later slices stay in flight).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__global__ void __launch_bounds__(kThreads) gemm_res_kernel(const ResParams p) {
  __shared__ __attribute__((aligned(16))) char smem[kLdsBytes];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  // Each XCD (workgroups are dispatched round-robin over the 8) takes a
  // contiguous range of tile numbers, walked in groups of kGroupM row tiles
  // with the row tile fastest: the workgroups an XCD runs at once cover a
  // few row blocks of X and a few row blocks of W, whose K slices its L2
  // serves to all of them.
  const int nwg = gridDim.x;
  const int bid = blockIdx.x;
  const int xcd = bid & 7;
  const int per = nwg >> 3;
  const int rem = nwg & 7;
  const int lin = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + (bid >> 3);
  int tm, tn;
  if (kGroupM > 0) {
    const int tiles_n = p.N / kTile;
    const int gsize = kGroupM * tiles_n;
    const int first = (lin / gsize) * kGroupM;
    const int gm = min(p.tiles_m - first, kGroupM);
    const int r = lin - (lin / gsize) * gsize;
    tm = first + r % gm;
    tn = r / gm;
  } else {
    tn = lin / p.tiles_m;
    tm = lin - tn * p.tiles_m;
  }
  const int m0 = tm * kTile;
  const int n0 = tn * kTile;

  // Copy instruction i of a slice (wavefront w issues i = w + 4 j): 8 rows of
  // 128 bytes, row-half hf of rows 8 r8 .. 8 r8 + 7 of the X part (i <
  // kCopies / 2) or of the W part.  LDS: part, then half, then row.  X rows
  // >= M re-read row M - 1 (their results are never stored).
  const uint32_t lds0 = (uint32_t)(uintptr_t)LDS_PTR(char, smem);
  uint32_t voff[kCopiesPerWave];
  uint32_t lofs[kCopiesPerWave];
#pragma unroll
  for (int j = 0; j < kCopiesPerWave; ++j) {
    const int i = w + kWaves * j;
    const bool xi = i < kCopies / 2;
    const int ii = xi ? i : i - kCopies / 2;   // within the part
    const int hf = ii / (kTile / 8);           // row half
    const int r = 8 * (ii % (kTile / 8)) + (lane >> 3);
    const int c = (lane & 7) ^ row_swz(r);     // global chunk landing at chunk position lane % 8
    voff[j] = xi ? (uint32_t)min(m0 + r, p.M - 1) * (uint32_t)p.ldx * 2u + (uint32_t)(hf * 128 + c * 16)
                 : (uint32_t)(n0 + r) * (uint32_t)p.ldw * 2u + (uint32_t)(hf * 128 + c * 16);
    lofs[j] = (xi ? 0u : (uint32_t)kOperand) + (uint32_t)(hf * kTile * kRowBytes) + (uint32_t)(ii % (kTile / 8)) * 1024u;
  }
  const char* xg = reinterpret_cast<const char*>(p.x);
  const char* wg = reinterpret_cast<const char*>(p.w);
  auto issue = [&](int kt) SIDON_INLINE {
    const uint32_t base = lds0 + (uint32_t)((kt % kStages) * kStage);
#pragma unroll
    for (int j = 0; j < kCopiesPerWave; ++j) {
      const bool xi = w + kWaves * j < kCopies / 2;  // wave-uniform
      dma_1k(base + lofs[j], (xi ? xg : wg) + kt * (kSliceK * 2), voff[j]);
    }
  };

  // Operand reads: lane (n, g) reads LDS row 32 b + n of a part, chunk
  // 2 s' + g of the row half holding k16 step s (s' = s % 4).
  const int ln = lane & 31;
  const int lg = lane >> 5;
  const int swz = row_swz(ln);  // rows 32 b + ln share the swizzle of row ln

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  const int kslices = p.K / kSliceK;
#pragma unroll
  for (int kt = 0; kt < kStages - 1; ++kt)
    if (kt < kslices) issue(kt);
  for (int kt = 0; kt < kslices; ++kt) {
    // Slice kt has landed for every wavefront, and every wavefront is done
    // with slice kt - 1, whose buffer the copy of slice kt + kStages - 1
    // refills.
    wait_slice<kCopiesPerWave, kStages - 2>(min(kStages - 2, kslices - 1 - kt));
    lds_barrier();
    if (kt + kStages - 1 < kslices) issue(kt + kStages - 1);
    const char* st = smem + (kt % kStages) * kStage;
#pragma unroll
    for (int q = 0; q < kStepsPerWave; ++q) {
      const int s = w + kWaves * q;
      const int hf = s >> 2;
      const int chunk = ((2 * (s & 3) + lg) ^ swz) << 4;
      h8 xa[2], wb[2];
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        xa[b] = *reinterpret_cast<const h8*>(st + hf * kTile * kRowBytes + (32 * b + ln) * kRowBytes + chunk);
        wb[b] = *reinterpret_cast<const h8*>(st + kOperand + hf * kTile * kRowBytes + (32 * b + ln) * kRowBytes + chunk);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wb[j], xa[i], acc[i][j], 0, 0, 0);
    }
  }
  lds_barrier();  // every wavefront is done with the ring (the partial tiles reuse it)

  // acc[i][j]: rows 32 i + ln of the tile, columns 32 j + 8 (e / 4) + 4 lg +
  // (e % 4).  Partial tile `part` at part * 64 rows of kRedStride fp32; with 8
  // wavefronts, wavefront w + 4 first hands its partial to wavefront w, which
  // adds it to its own (the two hold the same elements in the same lanes).
  float* red = reinterpret_cast<float*>(smem);
  auto put = [&](int part) SIDON_INLINE {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f4 v = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
          *reinterpret_cast<f4*>(red + (part * kTile + 32 * i + ln) * kRedStride + 32 * j + 8 * q + 4 * lg) = v;
        }
  };
  if (kWaves > kRedParts) {
    if (w >= kRedParts) put(w - kRedParts);
    lds_barrier();
    if (w < kRedParts) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f4 v =
                *reinterpret_cast<const f4*>(red + (w * kTile + 32 * i + ln) * kRedStride + 32 * j + 8 * q + 4 * lg);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[i][j][4 * q + e] += v[e];
          }
    }
    lds_barrier();
  }
  if (w < kRedParts) put(w);
  lds_barrier();

  // Wavefront w finishes rows kRowsPerWave w + [0, kRowsPerWave): lane takes
  // row kRowsPerWave w + lane / kLanesPerRow, kColsPerLane columns from
  // kColsPerLane (lane % kLanesPerRow); partial tiles summed in order.
  const int row = kRowsPerWave * w + lane / kLanesPerRow;
  const int col = kColsPerLane * (lane % kLanesPerRow);
  f4 sum[kColsPerLane / 4];
#pragma unroll
  for (int t = 0; t < kColsPerLane / 4; ++t) sum[t] = *reinterpret_cast<const f4*>(red + row * kRedStride + col + 4 * t);
#pragma unroll
  for (int s = 1; s < kRedParts; ++s)
#pragma unroll
    for (int t = 0; t < kColsPerLane / 4; ++t)
      sum[t] += *reinterpret_cast<const f4*>(red + (s * kTile + row) * kRedStride + col + 4 * t);
  const int gm = m0 + row;
  if (gm < p.M) {
    float* yrow = p.y + (int64_t)gm * p.ldy + n0 + col;
#pragma unroll
    for (int t = 0; t < kColsPerLane / 4; ++t) {
      f4 v = *reinterpret_cast<const f4*>(yrow + 4 * t);
      v += sum[t];
      *reinterpret_cast<f4*>(yrow + 4 * t) = v;
    }
  }
}

}  // namespace

SIDON_API int sidon_gemm_res_fits(int M, int N, int K) {
  return M >= 1 && N >= kTile && N % kTile == 0 && K >= kSliceK && K % kSliceK == 0 ? 1 : 0;
}

SIDON_API int sidon_gemm_res_preferred(int M, int N, int K) {
  if (!sidon_gemm_res_fits(M, N, K)) return 0;
  if (sidon::check_device() != SIDON_OK) return 0;
  const int64_t tiles = (int64_t)((M + kTile - 1) / kTile) * (N / kTile);
  return tiles <= sidon::compute_units() ? 1 : 0;
}

SIDON_API int sidon_gemm_res(const void* x, int ldx, const void* w, int ldw, float* y, int ldy, int M, int N, int K,
                             sidon_stream_t stream) {
  using sidon::fail;
  sidon::clear_error();
  if (!x || !w || !y) return fail(SIDON_E_NULL, "x, w and y must be non-NULL");
  if (!sidon_gemm_res_fits(M, N, K))
    return fail(SIDON_E_SHAPE, "M=%d N=%d K=%d: need M >= 1, N a multiple of %d, K a multiple of %d", M, N, K, kTile,
                kSliceK);
  if (ldx < K || ldw < K || ldy < N || ldx % 8 != 0 || ldw % 8 != 0 || ldy % 4 != 0)
    return fail(SIDON_E_STRIDE, "row strides ldx=%d ldw=%d (multiples of 8, >= K) ldy=%d (multiple of 4, >= N)", ldx,
                ldw, ldy);
  if ((int64_t)M * ldx * 2 >= (int64_t(1) << 32) || (int64_t)N * ldw * 2 >= (int64_t(1) << 32))
    return fail(SIDON_E_SHAPE, "X and W must each span less than 4 GiB");
  if (!sidon::aligned16(x) || !sidon::aligned16(w) || !sidon::aligned16(y))
    return fail(SIDON_E_ALIGN, "x, w and y must be 16-byte aligned");
  // Workgroups read X and W while others already add into Y: the byte
  // ranges the call touches must be disjoint.
  {
    const uintptr_t xb = reinterpret_cast<uintptr_t>(x), wb = reinterpret_cast<uintptr_t>(w);
    const uintptr_t yb = reinterpret_cast<uintptr_t>(y);
    const uintptr_t xe = xb + (uintptr_t)(((int64_t)(M - 1) * ldx + K) * 2);
    const uintptr_t we = wb + (uintptr_t)(((int64_t)(N - 1) * ldw + K) * 2);
    const uintptr_t ye = yb + (uintptr_t)(((int64_t)(M - 1) * ldy + N) * 4);
    if ((xb < ye && yb < xe) || (wb < ye && yb < we))
      return fail(SIDON_E_SHAPE, "x and w must not overlap y (the kernel reads them while adding into y)");
  }
  int rc;
  if ((rc = sidon::check_device())) return rc;
  ResParams p;
  p.x = static_cast<const _Float16*>(x);
  p.w = static_cast<const _Float16*>(w);
  p.y = y;
  p.ldx = ldx;
  p.ldw = ldw;
  p.ldy = ldy;
  p.M = M;
  p.N = N;
  p.K = K;
  p.tiles_m = (M + kTile - 1) / kTile;
  const int64_t tiles = (int64_t)p.tiles_m * (N / kTile);
  if (tiles >= (int64_t(1) << 31)) return fail(SIDON_E_SHAPE, "too many tiles");
  hipLaunchKernelGGL(gemm_res_kernel, dim3((unsigned)tiles), dim3(kThreads), 0, reinterpret_cast<hipStream_t>(stream),
                     p);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(SIDON_E_LAUNCH, "gemm launch failed: %s", hipGetErrorString(err));
  return SIDON_OK;
}
