// gemm.hip -- the conformer FFN's input projection with its bias and SiLU
// fused, for MI355X (gfx950).
//
//   Y[m, n] = act(X[m, :] . W[n, :] + bias[n])        act = SiLU or identity
//
// X [M, K] and W [N, K] fp16 (both K-contiguous: activations and a torch
// Linear weight), fp32 accumulation, Y [M, N] fp16.  This is the
// torch.addmm(b1, xn, W1^T) + F.silu_ pair of the FFN modules of
// src/sidon_triton/triton_encoder.py:498-499 and :507-508, in one pass: the
// bias is added to the fp32 sum and rounded to fp16 (as the addmm stores it),
// then SiLU is taken in fp32 and rounded to fp16 (as the in-place SiLU does),
// so the only difference from the two-step form is the GEMM's summation order.
//
// Tiling.  A workgroup owns a 320 x 256 tile of Y and runs 8 wavefronts (two
// per SIMD), wavefront (wm, wn) owning rows 160 wm + [0, 160) and columns
// 64 wn + [0, 64) as 5 x 2 blocks of v_mfma_f32_32x32x16_f16 (Y^T = W . X^T,
// so a lane holds four consecutive columns of one row).  The K loop walks
// 64-wide slices: X and W slices (40 KB + 32 KB) are copied global -> LDS
// with global_load_lds_dwordx4 into one of two buffers while the other is
// consumed; one barrier per slice.  The operands of each k16 step are read
// from LDS while the previous step's 10 MFMAs run.  16-byte chunk c of the
// 128-byte LDS row r sits at chunk c ^ ((r >> 1) & 7), so the operand reads
// (16 rows per 16 lanes) are bank-conflict free.  The epilogue stages each
// wavefront's 160 x 64 fp16 result in LDS and writes whole 128-byte row
// segments.  At M = 4800, N = 4096 the 240 tiles fill 240 CUs in one round.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "sidon_encoder.h"
#include "sidon_host.h"

#define SIDON_API extern "C" __attribute__((visibility("default")))
#define SIDON_INLINE __attribute__((always_inline))

namespace {

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kTileM = 320;
constexpr int kTileN = 256;
// K slices of 64 in a ring of two (copy of slice k + 1 in flight while slice
// k is consumed).  Measured at M = 4800: slices of 32 in a ring of three or
// four (prefetch distance 2-3) are 5% slower -- the loop is bound by LDS
// traffic (copies plus operand reads, about 115 B/clock per CU), not by copy
// latency.
constexpr int kTileK = 64;
constexpr int kStages = 2;
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kWaveM = 160;                       // rows per wavefront
constexpr int kWaveN = 64;                        // columns per wavefront
constexpr int kBM = kWaveM / 32;                  // 5 row blocks
constexpr int kBN = kWaveN / 32;                  // 2 column blocks
constexpr int kRowBytes = kTileK * 2;             // bytes per LDS row
constexpr int kChunks = kRowBytes / 16;           // 16-byte chunks per row
constexpr int kRowsPerCopy = 1024 / kRowBytes;    // rows per 1 KB copy instruction
constexpr int kStageA = kTileM * kRowBytes;
constexpr int kStageB = kTileN * kRowBytes;
constexpr int kStage = kStageA + kStageB;
constexpr int kCopiesA = kStageA / 1024;
constexpr int kCopies = kStage / 1024;            // copy instructions per slice
constexpr int kCopySlots = (kCopies + kWaves - 1) / kWaves;
constexpr int kFullWaves = kCopies - kWaves * (kCopySlots - 1);  // wavefronts issuing kCopySlots copies
constexpr int kEpiWave = kWaveM * kWaveN * 2;     // 20 KB of fp16 per wavefront
constexpr int kLdsBytes = kStages * kStage > kWaves * kEpiWave ? kStages * kStage : kWaves * kEpiWave;
static_assert(kChunks == 4 || kChunks == 8, "32- or 64-wide K slices");

// Chunk position of 16-byte chunk c of LDS row r: c ^ swz(r).  A 16-lane
// group reads 16 consecutive rows at one logical chunk; the map spreads them
// over all 64 banks (rows of 64 bytes: 4 per 64 banks; of 128: 2).
__device__ __forceinline__ int row_swz(int r) { return kChunks == 8 ? (r >> 1) & 7 : (r >> 2) & 3; }
static_assert(kLdsBytes <= 160 * 1024, "LDS budget of one CU");

#define LDS_PTR(T, p) ((__attribute__((address_space(3))) T*)(p))

struct GemmParams {
  const _Float16* x;
  const _Float16* w;
  const _Float16* bias;
  _Float16* y;
  int ldx, ldw, ldy;  // row strides (elements)
  int M, N, K;
  int tiles_m;
  int act;  // 1: SiLU
};

// Copy of 1 KB (8 rows of 128 bytes) global -> LDS; lane l's 16 bytes land
// at lds_addr + 16 l.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma_1k(uint32_t lds_addr, const char* gbase, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :: "s"(lds_addr), "v"(voff), "s"(gbase) : "memory", "m0");
}
#pragma clang diagnostic pop

template <int N>
__device__ __forceinline__ void wait_vmcnt() { asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory"); }

// Wait until slice kt has landed while up to `newer` later slices (of kPer
// copies each, issued after it by this wavefront) stay in flight.
template <int kPer>
__device__ __forceinline__ void wait_slice(int newer) {
  if (newer >= 2) {
    wait_vmcnt<2 * kPer>();
  } else if (newer == 1) {
    wait_vmcnt<kPer>();
  } else {
    wait_vmcnt<0>();
  }
}

// SiLU as the encoder's in-place SiLU kernel computes it (fp32, hardware
// exponential and reciprocal, rounded to fp16); the empty asm keeps the
// product and the conversion from fusing into one mixed-precision rounding.
__device__ __forceinline__ _Float16 silu16(_Float16 h) {
  const float x = (float)h;
  float y = x * __builtin_amdgcn_rcpf(1.f + __expf(-x));
  asm volatile("" : "+v"(y));
  return (_Float16)y;
}

__global__ void __launch_bounds__(kThreads) gemm_bias_act_kernel(const GemmParams p) {
  __shared__ __attribute__((aligned(16))) char smem[kLdsBytes];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = w >> 2;  // 0..1
  const int wn = w & 3;   // 0..3

  // Tiles are numbered with M fastest; each XCD (workgroups are dispatched
  // round-robin over the 8) takes a contiguous range, so its tiles share a
  // few column blocks of W, which stay in its L2.
  const int nwg = gridDim.x;
  const int bid = blockIdx.x;
  const int xcd = bid & 7;
  const int per = nwg >> 3;
  const int rem = nwg & 7;
  const int lin = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + (bid >> 3);
  const int tn = lin / p.tiles_m;
  const int tm = lin - tn * p.tiles_m;
  const int m0 = tm * kTileM;
  const int n0 = tn * kTileN;

  // Copy instruction i (of kCopies per slice; wavefront w issues i = w + 8 j):
  // rows kRowsPerCopy i' + lane / kChunks of the X slice (i < kCopiesA) or of
  // the W slice; lane offsets fixed for the whole loop (X rows >= M re-read
  // row M - 1, whose results are never stored).
  const uint32_t lds0 = (uint32_t)(uintptr_t)LDS_PTR(char, smem);
  uint32_t voff[kCopySlots];
#pragma unroll
  for (int j = 0; j < kCopySlots; ++j) {
    const int i = min(w + kWaves * j, kCopies - 1);
    const bool xi = i < kCopiesA;
    const int r = (xi ? kRowsPerCopy * i : kRowsPerCopy * (i - kCopiesA)) + lane / kChunks;
    const int c = (lane % kChunks) ^ row_swz(r);  // global chunk that lands at chunk position lane % kChunks
    voff[j] = xi ? (uint32_t)min(m0 + r, p.M - 1) * (uint32_t)p.ldx * 2u + (uint32_t)c * 16u
                 : (uint32_t)(n0 + r) * (uint32_t)p.ldw * 2u + (uint32_t)c * 16u;
  }
  const char* xg = reinterpret_cast<const char*>(p.x);
  const char* wg = reinterpret_cast<const char*>(p.w);
  auto issue = [&](int kt) {
    const uint32_t base = lds0 + (kt % kStages) * kStage;
#pragma unroll
    for (int j = 0; j < kCopySlots; ++j) {
      const int i = w + kWaves * j;
      if (i < kCopies) {  // wave-uniform
        const bool xi = i < kCopiesA;
        dma_1k(base + i * 1024, (xi ? xg : wg) + kt * kRowBytes, voff[j]);
      }
    }
  };

  // Operand reads: lane (n, g) reads LDS row r = 32 blk + n, chunk 2 s + g
  // (k = 16 s + 8 g + [0, 8) of the slice) for k16 step s.
  const int ln = lane & 31;
  const int lg = lane >> 5;
  int aoff[kBM], boff[kBN];  // row byte offsets within a stage
#pragma unroll
  for (int b = 0; b < kBM; ++b) aoff[b] = (kWaveM * wm + 32 * b + ln) * kRowBytes;
#pragma unroll
  for (int b = 0; b < kBN; ++b) boff[b] = kStageA + (kWaveN * wn + 32 * b + ln) * kRowBytes;
  const int swz = row_swz(ln);  // rows 32 b + ln share the swizzle of row ln

  f32x16 acc[kBM][kBN];
#pragma unroll
  for (int i = 0; i < kBM; ++i)
#pragma unroll
    for (int j = 0; j < kBN; ++j) acc[i][j] = f32x16{};

  const int kslices = p.K / kTileK;
#pragma unroll
  for (int kt = 0; kt < kStages - 1; ++kt)
    if (kt < kslices) issue(kt);
  for (int kt = 0; kt < kslices; ++kt) {
    // Slice kt has landed for every wavefront, and nobody reads slice kt - 1
    // any more, whose buffer the copy of slice kt + kStages - 1 refills.
    const int newer = min(kStages - 2, kslices - 1 - kt);
    if (w < kFullWaves) {
      wait_slice<kCopySlots>(newer);
    } else {
      wait_slice<kCopySlots - 1>(newer);
    }
    __syncthreads();
    if (kt + kStages - 1 < kslices) issue(kt + kStages - 1);
    const char* st = smem + (kt % kStages) * kStage;
    // Operands of k16 step s + 1 are read while the 10 MFMAs of step s run
    // (two register sets; the scheduling barriers keep the compiler from
    // interleaving the reads into the MFMA group, where each would wait).
    h8 xa[2][kBM], wb[2][kBN];
    auto load = [&](int s, int set) SIDON_INLINE {
      const int chunk = ((2 * s + lg) ^ swz) << 4;
#pragma unroll
      for (int b = 0; b < kBM; ++b) xa[set][b] = *reinterpret_cast<const h8*>(st + aoff[b] + chunk);
#pragma unroll
      for (int b = 0; b < kBN; ++b) wb[set][b] = *reinterpret_cast<const h8*>(st + boff[b] + chunk);
    };
    load(0, 0);
#pragma unroll
    for (int s = 0; s < kTileK / 16; ++s) {
      const int cur = s & 1;
      if (s + 1 < kTileK / 16) load(s + 1, cur ^ 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < kBM; ++i)
#pragma unroll
        for (int j = 0; j < kBN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wb[cur][j], xa[cur][i], acc[i][j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  __syncthreads();  // every wavefront is done with the ring (the epilogue reuses it)

  // Epilogue.  acc[i][j] is Y^T for rows 32 i + n (lane column n) and
  // columns 32 j + 8 (e / 4) + 4 g + (e % 4): four consecutive columns per
  // group e / 4.  Bias add (rounded to fp16 as addmm stores it), SiLU, and
  // the fp16 tile of this wavefront into its own 20 KB of LDS (row stride
  // 128 bytes, 8-byte unit u at u ^ (row & 15)), then whole rows out.
  char* ep = smem + w * kEpiWave;
#pragma unroll
  for (int j = 0; j < kBN; ++j) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int col = kWaveN * wn + 32 * j + 8 * q + 4 * lg;  // within the tile
      h4 bv = {};
      if (p.bias != nullptr) bv = *reinterpret_cast<const h4*>(p.bias + n0 + col);
#pragma unroll
      for (int i = 0; i < kBM; ++i) {
        h4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          _Float16 hsum = (_Float16)(acc[i][j][4 * q + e] + (float)bv[e]);
          v[e] = p.act == 1 ? silu16(hsum) : hsum;
        }
        const int row = 32 * i + ln;                 // within the wavefront's 160
        const int unit = (col - kWaveN * wn) >> 2;   // 8-byte unit within the 128-byte row
        *reinterpret_cast<h4*>(ep + row * 128 + ((unit ^ (row & 15)) << 3)) = v;
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): own LDS writes done (wave-private region)
  // Rows 8 t + lane / 8, 16-byte chunk lane % 8 (units 2 c, 2 c + 1).
  const int c = lane & 7;
#pragma unroll 4
  for (int t = 0; t < kWaveM / 8; ++t) {
    const int row = 8 * t + (lane >> 3);
    const int gm = m0 + kWaveM * wm + row;
    const h4 lo = *reinterpret_cast<const h4*>(ep + row * 128 + (((2 * c) ^ (row & 15)) << 3));
    const h4 hi = *reinterpret_cast<const h4*>(ep + row * 128 + (((2 * c + 1) ^ (row & 15)) << 3));
    if (gm < p.M) {
      const h8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      *reinterpret_cast<h8*>(p.y + (int64_t)gm * p.ldy + n0 + kWaveN * wn + 8 * c) = v;
    }
  }
}

}  // namespace

SIDON_API int sidon_gemm_bias_act_fits(int M, int N, int K) {
  return M >= 1 && N >= kTileN && N % kTileN == 0 && K >= kTileK && K % kTileK == 0 ? 1 : 0;
}

// One workgroup per CU (its LDS fills one): the kernel pays off when its
// tiles keep at least three quarters of the CUs busy in every dispatch round
// (at N = 4096, K = 1024: M = 4800 gives 240 tiles on 256 CUs, 17% faster
// than hipBLASLt's GEMM followed by the SiLU pass; M = 1500 gives 80 and is
// slower).
SIDON_API int sidon_gemm_bias_act_preferred(int M, int N, int K) {
  if (!sidon_gemm_bias_act_fits(M, N, K)) return 0;
  if (sidon::check_device() != SIDON_OK) return 0;
  const int64_t tiles = (int64_t)((M + kTileM - 1) / kTileM) * (N / kTileN);
  const int64_t cus = sidon::compute_units();
  const int64_t rounds = (tiles + cus - 1) / cus;
  return 4 * tiles >= 3 * rounds * cus ? 1 : 0;
}

SIDON_API int sidon_gemm_bias_act(const void* x, int ldx, const void* w, int ldw, const void* bias, void* y, int ldy,
                                  int M, int N, int K, int act, sidon_stream_t stream) {
  using sidon::fail;
  sidon::clear_error();
  if (!x || !w || !y) return fail(SIDON_E_NULL, "x, w and y must be non-NULL");
  if (!sidon_gemm_bias_act_fits(M, N, K))
    return fail(SIDON_E_SHAPE, "M=%d N=%d K=%d: need M >= 1, N a multiple of %d, K a multiple of %d", M, N, K,
                kTileN, kTileK);
  if (ldx < K || ldw < K || ldy < N || (ldx | ldw | ldy) % 8 != 0)
    return fail(SIDON_E_STRIDE, "row strides ldx=%d ldw=%d ldy=%d must be multiples of 8 and >= K, K, N", ldx, ldw,
                ldy);
  if ((int64_t)M * ldx * 2 >= (int64_t(1) << 32) || (int64_t)N * ldw * 2 >= (int64_t(1) << 32))
    return fail(SIDON_E_SHAPE, "X and W must each span less than 4 GiB");
  if (act != 0 && act != 1) return fail(SIDON_E_SHAPE, "act=%d: 0 (none) or 1 (SiLU)", act);
  if (!sidon::aligned16(x) || !sidon::aligned16(w) || !sidon::aligned16(y) || (bias && ((uintptr_t)bias & 7) != 0))
    return fail(SIDON_E_ALIGN, "x, w, y must be 16-byte aligned and bias 8-byte aligned");
  int rc;
  if ((rc = sidon::check_device())) return rc;
  GemmParams p;
  p.x = static_cast<const _Float16*>(x);
  p.w = static_cast<const _Float16*>(w);
  p.bias = static_cast<const _Float16*>(bias);
  p.y = static_cast<_Float16*>(y);
  p.ldx = ldx;
  p.ldw = ldw;
  p.ldy = ldy;
  p.M = M;
  p.N = N;
  p.K = K;
  p.tiles_m = (M + kTileM - 1) / kTileM;
  p.act = act;
  const int64_t tiles = (int64_t)p.tiles_m * (N / kTileN);
  if (tiles >= (int64_t(1) << 31)) return fail(SIDON_E_SHAPE, "too many tiles");
  hipLaunchKernelGGL(gemm_bias_act_kernel, dim3((unsigned)tiles), dim3(kThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), p);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(SIDON_E_LAUNCH, "gemm launch failed: %s", hipGetErrorString(err));
  return SIDON_OK;
}
