// flexrel_fwd.hip -- relative_key flash attention for MI355X (gfx950 / CDNA4).
//
// Computes, for every (batch b, head h, query row i < L):
//
//   s_ij = (q_i . k_j + q_i . rel[clamp(j - i, -64, 8) + 64]) / sqrt(64)
//   o_i  = sum_{j < LK_b} softmax_j(s_ij) v_j
//
// the encoder self-attention of src/sidon_triton/triton_encoder.py:210-312
// (kernel body) behind the launcher of :346-371, and the strided [B,H,L,64]
// form of src/sidon_triton/flexrel_triton.py:249-278.
//
// Work decomposition.  One workgroup owns 64 query rows of one (b, h) and has
// 8 wavefronts (two per SIMD); wavefront w runs an independent online softmax
// over the key steps w, w + 8, w + 16, ... (32 keys each; round-robin, so the
// few steps that need the per-score bias gather or the key mask fall at the
// same time for all wavefronts) and the 8 partial results are merged through
// LDS at the end.  Each wavefront runs a software pipeline in which every
// dependency crosses a half-step boundary:
//
//   * K and V step tiles (32 keys x 64 dims, 4 KB each) are copied
//     global -> LDS with global_load_lds_dwordx4 (no register staging) into a
//     per-wavefront ring of two K and two V slots; step u issues the copies
//     of K(u+2) and V(u+1).  16-byte chunks are XOR swizzled by row so both
//     LDS read patterns below are bank-conflict free;
//   * scores are formed transposed, S^T = K . Q^T, with
//     v_mfma_f32_32x32x16_f16 on two 32-query column blocks (Q^T stays in
//     registers): every lane holds scores of one query only, so the softmax
//     row state is per lane.  K rows are fed to the MFMA A operand with bits
//     2 and 3 of the row index swapped, which makes the 8 probabilities a lane
//     owns per 16-key PV step contiguous keys: the score accumulator, rounded
//     to fp16, is the B operand of O^T += V^T . P^T without any shuffle;
//   * the V^T operand comes straight from the key-major V tile through
//     ds_read_b64_tr_b16 (LDS transpose read);
//   * step u is two half steps, one per column block: each issues 4 PV and
//     4 QK MFMAs (of steps u - 1 and u, or u - 1 and u + 1), one tile copy
//     and the LDS operand reads of a later step next to the exp2 work of
//     its column block;
//   * softmax with a lazily updated running max: probabilities are
//     exp2(s * log2(e)/8 + bias - m) with the max m of earlier steps.  While the
//     step's probabilities stay inside the fp16 range (a query's 32 values
//     sum below 2^15), m, the row sum and O need no rescaling; a step that
//     leaves it, and the first step, take the exact max-update path.  The
//     row sums are taken on the matrix core from the fp16-rounded
//     probabilities (the values the PV product uses) and checked one half
//     step later, before the scores they came from are overwritten;
//   * relative bias: q . rel^T for the 64 rows x 73 positions is computed once
//     per workgroup with MFMA into LDS (fp32).  Steps entirely left
//     (j - i <= -64) or right (j - i >= 8) of a 32-row column block see a
//     per-row constant bias, folded into the exp2 argument; only the ~4
//     "band" steps per column block gather the bias per score;
//   * keys >= LK: the one straddling step reads clamped (valid) rows and sets
//     their scores to -inf; steps starting at or past LK are never visited.
#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <type_traits>

#include "flexrel_device.h"
#include "sidon_flexrel.h"
#include "sidon_host.h"

#define SIDON_API extern "C" __attribute__((visibility("default")))
// Kernel-body lambdas index register arrays with their arguments; inlined,
// every index is a constant and the arrays stay in registers.
#define SIDON_INLINE __attribute__((always_inline))

namespace {

using namespace sidon_flexrel;
#define LDS_PTR SIDON_LDS_PTR

constexpr int kRows = 64;       // query rows per workgroup (two 32-column blocks)
// Key splits per workgroup: 8 wavefronts, two per SIMD (one per SIMD leaves
// the SIMD idle on every dependency stall of its wavefront).
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kStages = 2;                   // ring depth (K and V) per wavefront
constexpr int kWaveRing = 2 * kStages * kTile;  // K slots, then V slots
constexpr int kQrOff = kWaves * kWaveRing;
constexpr int kQStageOff = kQrOff + kRows * kQrStride * 4;  // Q block, 64 rows x 128 B
constexpr int kLdsBytes = kQStageOff + kRows * kD * 2;
// Split merge (reuses the ring and table area after the key loop).
constexpr int kMergeStride = 68;             // fp32 per partial-output row
constexpr int kMergeMlOff = kWaves * kRows * kMergeStride * 4;
static_assert(kMergeMlOff + kWaves * kRows * 2 * 4 <= kLdsBytes, "merge area too small");
static_assert(kLdsBytes <= 160 * 1024, "LDS budget of one CU");

// kSameStride: K and V rows have the same stride (always the case for the
// fused QKV layout), so one set of copy offsets serves both.
template <bool kSameStride>
__global__ void __launch_bounds__(kThreads)
flexrel_fwd_kernel(const Params p) {
  __shared__ __attribute__((aligned(16))) char smem[kLdsBytes];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 31;  // query column of this lane (within a 32-block)
  const int g = lane >> 5;  // lane half

  // Workgroups are dispatched round-robin over the 8 XCDs; give each XCD a
  // contiguous range of (b, h, query block) so one head's K/V stays in one
  // XCD's L2.
  const int lin = xcd_linear(blockIdx.x, gridDim.x);
  const int bh = lin / p.nqb;
  const int qblk = lin - bh * p.nqb;
  const int b = bh / p.H;
  const int h = bh - b * p.H;

  int LK = p.L;
  if (p.lens != nullptr) LK = min(max(p.lens[b], 0), p.L);
  LK = __builtin_amdgcn_readfirstlane(LK);
  const int q0 = p.row0 + qblk * kRows;
  const float scale = p.scale;

  const _Float16* qbase = p.q + b * p.qsb + h * p.qsh;
  const char* kbase = reinterpret_cast<const char*>(p.k + b * p.ksb + h * p.ksh);
  const char* vbase = reinterpret_cast<const char*>(p.v + b * p.vsb + h * p.vsh);
  const int64_t kstride = (int64_t)p.ksl * 2;  // bytes
  const int64_t vstride = (int64_t)p.vsl * 2;

  // Key steps: T steps of 32 keys cover [0, LK); this wavefront takes steps
  // w + 8 u, u = 0 .. nu - 1.
  const int T = (LK + kStep - 1) / kStep;
  const int nu = T > w ? (T - w + kWaves - 1) / kWaves : 0;
  const bool active = nu > 0;

  char* ring = smem + w * kWaveRing;
  const uint32_t ring_lds = (uint32_t)(uintptr_t)LDS_PTR(char, ring);

  // Copy of one step tile (K or V) into an LDS slot: LDS chunk position
  // 64 i + lane = (row 8 i + lane / 8, swizzled chunk lane % 8).  Lane
  // offsets are taken from base - 3072 (instruction i adds 1024 i), which
  // keeps them non-negative.
  uint32_t koff[4], voff_own[4];
  // Offsets for the last step T - 1 when it straddles LK: rows past LK re-read
  // row LK - 1 (in bounds); their scores are masked.
  uint32_t koff_last[4], voff_last_own[4];
  const int last_row = LK - 1 - (T - 1) * kStep;  // in [0, 31]
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 8 * i + (lane >> 3);
    const int rc = min(r, last_row);
    const uint32_t c16 = 16u * ((lane & 7) ^ tile_swz(r)) + 3072u - 1024u * i;
    koff[i] = (uint32_t)(r * kstride) + c16;
    koff_last[i] = (uint32_t)(rc * kstride) + c16;
    voff_own[i] = kSameStride ? 0u : (uint32_t)(r * vstride) + c16;
    voff_last_own[i] = kSameStride ? 0u : (uint32_t)(rc * vstride) + c16;
  }
  const uint32_t (&voff)[4] = kSameStride ? koff : voff_own;
  const uint32_t (&voff_last)[4] = kSameStride ? koff_last : voff_last_own;
  // Local step u -> global step; local steps past the wavefront's range
  // (prefetches whose data is never used) re-read step T - 1, so every copy
  // stays in bounds and every step issues the same number of copies.
  auto gstep = [&](int u) SIDON_INLINE { return min(w + kWaves * u, T - 1); };
  // may_straddle == false promises that step u is not T - 1 with LK % 32 != 0
  // (no select then).  Branch-free, so a copy can sit in a scheduled block.
  auto copy_tile = [&](const char* base, int64_t stride, const uint32_t (&off)[4],
                       const uint32_t (&off_last)[4], int u, uint32_t slot, bool may_straddle) {
    const int t = gstep(u);
    const char* gb = base + (int64_t)(t * kStep) * stride - 3072;
    const bool straddle = may_straddle && t == T - 1;
    dma_tile(slot, gb, straddle ? off_last[0] : off[0], straddle ? off_last[1] : off[1],
             straddle ? off_last[2] : off[2], straddle ? off_last[3] : off[3]);
  };
  // Ring slots: K(u) and V(u) live in slot u % 2 of their halves of the ring.
  constexpr uint32_t kVRing = kStages * kTile;

  // First copies, all in flight together: this wavefront's 8 rows of the Q
  // block into the Q staging area; the rel rows of its q.rel table block
  // (wavefronts 0-5) into its last V slot, unused until step 0 refills it;
  // and K(0), K(1), V(0).  Rows are clamped into range (Q rows >= L and rel
  // rows >= 73 are zeroed after reading).  16-byte chunks are swizzled like
  // the step tiles.
  const uint32_t q_lds = (uint32_t)(uintptr_t)LDS_PTR(char, smem + kQStageOff);
  {
    const int r = 8 * w + (lane >> 3);
    const int row0 = min(q0 + 8 * w, p.L - 1);
    const char* gq = reinterpret_cast<const char*>(qbase + (int64_t)row0 * p.qsl);
    const uint32_t off = (uint32_t)((min(q0 + r, p.L - 1) - row0) * p.qsl * 2) +
                         16u * ((lane & 7) ^ tile_swz(r));
    dma_1k(q_lds + 1024u * w, gq, off);
  }
  const int tab_j = w;  // q.rel block of this wavefront (if < 6): j = 3 qb + pb
  if (tab_j < 6) {
    const int pb = tab_j % 3;
    uint32_t roff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 8 * i + (lane >> 3);
      roff[i] = (uint32_t)(min(32 * pb + r, kNumPos - 1) * kD * 2) + 16u * ((lane & 7) ^ tile_swz(r)) +
                3072u - 1024u * i;
    }
    dma_tile(ring_lds + kVRing + (kStages - 1) * kTile, reinterpret_cast<const char*>(p.rel) - 3072,
             roff[0], roff[1], roff[2], roff[3]);
  }
  if (active) {
#pragma unroll
    for (int i = 0; i < kStages; ++i) copy_tile(kbase, kstride, koff, koff_last, i, ring_lds + i * kTile, true);
#pragma unroll
    for (int i = 0; i + 1 < kStages; ++i)
      copy_tile(vbase, vstride, voff, voff_last, i, ring_lds + kVRing + i * kTile, true);
    wait_vmcnt<4 * (2 * kStages - 1)>();  // the Q rows and rel rows have landed
  } else {
    wait_vmcnt<0>();
  }
  lds_barrier();  // the whole Q block is in LDS

  // Q^T as the MFMA B operand: lane (n, g) of block qb holds query
  // q0 + 32 qb + n, dims 16 s + 8 g + [0, 8) for k-step s.  Rows >= L are 0.
  h8 qop[2][4];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int r = 32 * qb + n;
    const char* qrow = smem + kQStageOff + r * 128;
#pragma unroll
    for (int s = 0; s < 4; ++s) qop[qb][s] = *reinterpret_cast<const h8*>(qrow + (((2 * s + g) ^ tile_swz(r)) << 4));
    if (q0 + r >= p.L) {
#pragma unroll
      for (int s = 0; s < 4; ++s) qop[qb][s] = h8{};
    }
  }

  // q.rel^T * scale for the 64 rows: 6 blocks of 32 positions x 32 queries,
  // block j = 3 qb + pb (positions 32 pb + [0, 32)) computed by wavefront j
  // as rel . Q^T; rows of rel >= 73 are 0.
  float* qr_tab = reinterpret_cast<float*>(smem + kQrOff);
  if (tab_j < 6) {
    const int pb = tab_j % 3;
    const int qsel = tab_j / 3;
    const int pos = 32 * pb + n;
    const char* rrow = ring + kVRing + (kStages - 1) * kTile + n * 128;
    f32x16 acc = {};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      h8 e = *reinterpret_cast<const h8*>(rrow + (((2 * s + g) ^ tile_swz(n)) << 4));
      if (pos >= kNumPos) e = h8{};
      const h8 qs = qsel ? qop[1][s] : qop[0][s];
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(e, qs, acc, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int pos0 = 32 * pb + 8 * i + 4 * g;
      if (pos0 < kQrStride) {
        const f4 val = {acc[4 * i] * scale, acc[4 * i + 1] * scale, acc[4 * i + 2] * scale,
                        acc[4 * i + 3] * scale};
        *reinterpret_cast<f4*>(qr_tab + (32 * qsel + n) * kQrStride + pos0) = val;
      }
    }
  }
  lds_barrier();  // the q.rel table is complete

  float qr_l[2], qr_r[2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    qr_l[qb] = qr_tab[(32 * qb + n) * kQrStride];                 // j - i <= -64
    qr_r[qb] = qr_tab[(32 * qb + n) * kQrStride + kNumPos - 1];   // j - i >= 8
  }

  f32x16 oacc[2][2] = {};   // O^T: dims 32 db + 8 (i/4) + 4 g + i%4, query n
  float m_run[2] = {-INFINITY, -INFINITY};
  f32x16 sacc[2];           // S^T per column block (step u, or u + 1 once consumed)
  h8 pk[2][2] = {};         // fp16 probabilities per column block and 16-key half
  h8 kop[4];                // K operands (16 dims per k-step) of one step
  h8 vop[2][2];             // V^T operands [hh][db] of one step

  // K operands: lane (m, g) holds key row perm(m) of the tile, dims
  // 16 s + 8 g + [0, 8).
  const int kperm = mfma_row_perm(n);
  const char* krow0 = ring + kperm * 128;
  const int kswz = tile_swz(kperm);
  // The swizzled chunk offsets differ per lane and per k-step, so the eight
  // addresses (two slots x four k-steps) are formed once, not per step.
  const char* kaddr[2][4];
#pragma unroll
  for (int sl = 0; sl < 2; ++sl)
#pragma unroll
    for (int s = 0; s < 4; ++s) kaddr[sl][s] = krow0 + sl * kTile + (((2 * s + g) ^ kswz) << 4);
  auto load_k = [&](uint32_t slot) SIDON_INLINE {
    const int sl = slot != 0;
#pragma unroll
    for (int s = 0; s < 4; ++s)
      kop[s] = *reinterpret_cast<const h8*>(sl ? kaddr[1][s] : kaddr[0][s]);
  };
  // V^T operands via transpose reads: group G of 16 lanes, source lane
  // (a, bq) reads V[key0 + a][d0 + 4 bq .. +4) with key0 = 16 hh + 8 (G / 2)
  // + 4 hf and d0 = 32 db + 16 (G % 2).  hh adds 2048 bytes (an immediate);
  // hf and db flip one chunk bit each through the swizzle, so four per-lane
  // bases cover all eight reads.
  const int tr_G = lane >> 4;
  const int tr_a = (lane >> 2) & 3;
  const int tr_b = lane & 3;
  int tr_off[2][2];  // [hf][db] byte offset for hh = 0
#pragma unroll
  for (int hf = 0; hf < 2; ++hf)
#pragma unroll
    for (int db = 0; db < 2; ++db) {
      const int row = 8 * (tr_G >> 1) + 4 * hf + tr_a;
      const int chunk = 4 * db + 2 * (tr_G & 1) + (tr_b >> 1);
      tr_off[hf][db] = row * 128 + ((chunk ^ tile_swz(row)) << 4) + 8 * (tr_b & 1);
    }
  auto load_v = [&](uint32_t slot) SIDON_INLINE {
    const char* vt = ring + kVRing + slot;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        const h4 lo = __builtin_bit_cast(
            h4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(s4, vt + tr_off[0][db] + 2048 * hh)));
        const h4 hi = __builtin_bit_cast(
            h4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(s4, vt + tr_off[1][db] + 2048 * hh)));
        vop[hh][db] = cat(lo, hi);
      }
    }
  };
  // S^T of column block qb = K . Q^T (4 MFMAs); O^T += V^T . P^T for column
  // block qb (4 MFMAs).
  auto qk = [&](int qb) SIDON_INLINE {
    sacc[qb] = f32x16{};
#pragma unroll
    for (int s = 0; s < 4; ++s)
      sacc[qb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kop[s], qop[qb][s], sacc[qb], 0, 0, 0);
  };
  auto pv = [&](int qb) SIDON_INLINE {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int db = 0; db < 2; ++db)
        oacc[qb][db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vop[hh][db], pk[qb][hh], oacc[qb][db], 0, 0, 0);
  };

  // Row sums on the matrix core: rs = ones . P^T with v_mfma_f32_32x32x16_f16
  // (the PV product's B operand layout), so every element of lane (n, g) is
  // the step's sum of query n's fp16 probabilities -- the values the PV
  // product uses.  Each output column reads its own query only, so a
  // non-finite probability of one query never reaches another's sum.  One
  // accumulator serves both column blocks: block 0's sums are read at the
  // start of the half step that issues block 1's.
  // Kept live in registers across the loop (otherwise it is rebuilt with two
  // 64-bit moves before every row-sum pair).
  h8 ones = {1, 1, 1, 1, 1, 1, 1, 1};
  asm volatile("" : "+v"(ones));
  f32x16 rs;
  float l_run[2] = {0.f, 0.f};
  auto rowsum = [&](int qb) SIDON_INLINE {
    asm volatile("" : "+v"(ones));
    rs = __builtin_amdgcn_mfma_f32_32x32x16_f16(ones, pk[qb][0], f32x16{}, 0, 0, 0);
    rs = __builtin_amdgcn_mfma_f32_32x32x16_f16(ones, pk[qb][1], rs, 0, 0, 0);
  };

  // p = exp2(s * scale + nb) for column block qb (nb = bias - m), rounded to
  // fp16: the B operand of the PV product.
  auto emit = [&](int qb, int i, const f2& e) SIDON_INLINE {
    const h2 ph = __builtin_convertvector(e, h2);
    pk[qb][i >> 3][i & 7] = ph[0];
    pk[qb][i >> 3][(i & 7) + 1] = ph[1];
  };
  // Keys [8 part, 8 part + 8) of the lane's 16 (part -1: all).
  auto probs_fast = [&](int qb, float nb, int part = -1) SIDON_INLINE {
#pragma unroll
    for (int i = 0; i < 16; i += 2)
      if (part < 0 || (i >> 3) == part)
        emit(qb, i, f2{fast_exp2(fmaf(sacc[qb][i], scale, nb)), fast_exp2(fmaf(sacc[qb][i + 1], scale, nb))});
  };
  // p = exp2(y - m) from explicit biased scores y.
  auto probs_y = [&](int qb, const float (&y)[16], float m) {
#pragma unroll
    for (int i = 0; i < 16; i += 2) emit(qb, i, f2{fast_exp2(y[i] - m), fast_exp2(y[i + 1] - m)});
  };

  // Probabilities of column block qb of step u for the general cases (band
  // gather, masked keys) and the exact max update, from the scores still in
  // sacc[qb].
  auto general = [&](int u, int qb, bool first, bool need_sum) SIDON_INLINE {
    const int k0 = (w + kWaves * u) * kStep;
    const int qlo = q0 + 32 * qb;
    const bool left = k0 + (kStep - 1) - qlo <= -kLeft;
    const bool right = k0 - (qlo + 31) >= kRight;
    const bool masked = k0 + kStep > LK;
    const bool band = !left && !right;
    const float off = left ? qr_l[qb] : (right ? qr_r[qb] : 0.f);
    // y = s * scale + bias (log2 units); masked keys -> -inf.
    auto biased = [&](float (&y)[16]) {
      if (band) {
        const float* qrow = qr_tab + (32 * qb + n) * kQrStride;
        const int d0 = k0 + 8 * g - (qlo + n) + kLeft;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int idx = min(max(d0 + 16 * (i >> 3) + (i & 7), 0), kLeft + kRight);
          y[i] = fmaf(sacc[qb][i], scale, qrow[idx]);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) y[i] = fmaf(sacc[qb][i], scale, off);
      }
      if (masked) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = k0 + 16 * (i >> 3) + 8 * g + (i & 7);
          if (key >= LK) y[i] = -INFINITY;
        }
      }
    };
    auto probs = [&](float m) SIDON_INLINE {
      if (band || masked) {
        float y[16];
        biased(y);
        probs_y(qb, y, m);
      } else {
        probs_fast(qb, off - m);
      }
    };
    // Recompute with the running max; then raise the max of the queries
    // that need it: all at the first step (the max is -inf), else those whose
    // step sum left the fp16-safe range (need_sum).  The decision is per
    // query, never per wavefront, so one row cannot change the rounding of
    // another; a row whose max does not change gets bit-identical values.
    {
      if (!first) probs(m_run[qb]);
      if (first || need_sum) {
        const bool need = first || !(rs[0] < kSumLimit);
        float y[16];
        biased(y);
        float mx = y[0];
#pragma unroll
        for (int i = 1; i < 16; ++i) mx = fmaxf(mx, y[i]);
        mx = pair_max(mx);
        const float m_new = need ? fmaxf(m_run[qb], mx) : m_run[qb];
        const float alpha = fast_exp2(m_run[qb] - m_new);  // 1 if unchanged, 0 from -inf
        oacc[qb][0] *= alpha;
        oacc[qb][1] *= alpha;
        l_run[qb] *= alpha;
        m_run[qb] = m_new;
        probs(m_new);
      }
      rowsum(qb);
    }
  };
  // Deferred check of block qb of step u (its row sums were issued a half
  // step ago; its probabilities are consumed by the next PV product): a step
  // sum outside the fp16-safe range sends the block through the max update.
  // Then the step sums join the running sums.
  auto settle = [&](int u, int qb) SIDON_INLINE {
    // All of rs stays live up to here, so no register of the in-flight row
    // sum is reused (and waited for) before it lands.
    asm volatile("" : "+v"(rs));
    if (__builtin_expect(__builtin_amdgcn_ballot_w64(!(rs[0] < kSumLimit)) != 0, 0)) general(u, qb, false, true);
    l_run[qb] += rs[0];
  };

  // Softmax of column block qb of step u in its half step, in two parts
  // around the settling of the other block's previous softmax:
  //   1. `pre` (the PV product, 4 MFMAs) and the exp2 work of keys 0-7;
  //   2. `post` (the QK product, 4 MFMAs, and the next operand reads), the
  //      tile copy `dma`, keys 8-15 and the row sums (2 MFMAs).
  // The settle sits between them: the row sums it reads have had the PV
  // product's time to land, and `post` overwrites the scores it may need.
  // The common case is a plain step (no band, no mask, not the first step)
  // with the constant bias off_plain; the other steps redo the
  // probabilities at the end.  The MFMAs never sit in a branch, so their
  // accumulators stay in place.  (Instruction order inside each part is left
  // to the compiler: with two wavefronts per SIMD it interleaves MFMA and
  // VALU work across them better than a fixed in-wave pattern.)
  auto half_step = [&](int u, int qb, auto&& dma, auto&& pre, auto&& post, bool plain,
                       float off_plain) SIDON_INLINE {
    // The LDS reads of the previous half step are done (so the slot refilled
    // below is free), and the copy this half step reads has landed.
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), seen by the compiler
    wait_vmcnt<4 * (2 * kStages - 3)>();
    const float nb = off_plain - m_run[qb];
    pre();
    probs_fast(qb, nb, 0);
    asm volatile("" : "+v"(pk[qb][0]));
    if (qb == 0) {
      if (u > 0) settle(u - 1, 1);
    } else {
      settle(u, 0);
    }
    post();
    dma();
    probs_fast(qb, nb, 1);
    rowsum(qb);
    // Pin the common-case results here, so the compiler does not sink their
    // computation into the branch below.
    asm volatile("" : "+v"(pk[qb][0]), "+v"(pk[qb][1]));
    if (__builtin_expect(!plain, 0)) general(u, qb, u == 0, false);
  };

  // Software pipeline over this wavefront's steps.  Step u is two half
  // steps; every dependency crosses a half-step boundary and every register
  // set is reused in place:
  //   A(u): O^T block 0 += V^T(u-1) P^T(u-1);  settle block 1 of step u-1;
  //         S^T(u) block 1 = K(u) . Q^T, read K(u+1) operands;
  //         softmax of step u, block 0
  //   B(u): O^T block 1 += V^T(u-1) P^T(u-1);  settle block 0 of step u;
  //         S^T(u+1) block 0 = K(u+1) . Q^T, read V(u) operands;
  //         softmax of step u, block 1
  // The ring has two K and two V slots: A(u) copies K(u+2) into the slot
  // K(u) was read from (during A(u-1)), B(u) copies V(u+1) into the slot V(u-1)
  // was read from; the vmcnt(4) before each half step leaves only the newest
  // copy in flight, so K(u+1) has landed for A(u) and V(u) for B(u).  c0 and
  // c1 are the byte offsets of slots u % 2 and (u+1) % 2.
  if (active) {
    wait_vmcnt<0>();  // K(0), K(1), V(0)
    load_k(0);
    load_v(0);        // finite operands for the zero probabilities of step -1
    qk(0);            // S^T(0) block 0
    const bool ragged = LK % kStep != 0;  // step T - 1 straddles LK
    // Plain steps (see half_step) are u in [1, uM) with u <= uL (both column
    // blocks entirely left of the window, j - i <= -64) or u >= uR (both
    // entirely right, j - i >= 8); uM is the first step that straddles LK.
    // (Arithmetic shifts: floor and ceiling divisions by 256 = 8 steps of 32.)
    const int uL = (q0 - 95 - kStep * w) >> 8;
    const int uR = -((-(q0 + 71 - kStep * w)) >> 8);
    const int uM = ((LK - kStep - kStep * w) >> 8) + 1;
    // Tile sources, advanced by 8 steps per step of this wavefront; copies
    // of step T - 1 (the last one, also for prefetches past the range) read
    // from klast / vlast.
    const int64_t kinc = (int64_t)kWaves * kStep * kstride;
    const int64_t vinc = (int64_t)kWaves * kStep * vstride;
    const char* gk = kbase + (int64_t)(w + 2 * kWaves) * kStep * kstride - 3072;  // K(2)
    const char* gv = vbase + (int64_t)(w + kWaves) * kStep * vstride - 3072;      // V(1)
    const char* klast = kbase + (int64_t)(T - 1) * kStep * kstride - 3072;
    const char* vlast = vbase + (int64_t)(T - 1) * kStep * vstride - 3072;
    uint32_t c0 = 0, c1 = kTile;
    // Lane offsets of the next copies: the plain ones, switched once (for K
    // and V separately) to the clamped ones when the copies reach step T - 1
    // of a ragged LK -- no per-copy select.
    uint32_t kcur[4], vcur[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kcur[i] = koff[i];
      vcur[i] = voff[i];
    }
    for (int u = 0; u < nu; ++u) {
      // Wavefronts w and w + 4 share a SIMD, and the issue arbiter favours
      // the older one; alternate the wave priority per step so both finish
      // together (a lone wavefront leaves its SIMD half idle).
      if (((u + (w >> 2)) & 1) != 0) {
        __builtin_amdgcn_s_setprio(1);
      } else {
        __builtin_amdgcn_s_setprio(0);
      }
      // Plain step: both column blocks entirely left (j - i <= -64) or both
      // entirely right (j - i >= 8) of the window, and not the first or the
      // masked step.
      const bool both_left = u <= uL;
      const bool plain = u > 0 && (both_left || u >= uR) && u < uM;
      const float off0 = both_left ? qr_l[0] : qr_r[0];
      const float off1 = both_left ? qr_l[1] : qr_r[1];
      const bool k_last = w + kWaves * (u + 2) >= T - 1;
      const bool v_last = w + kWaves * (u + 1) >= T - 1;
      if (ragged && k_last) {
#pragma unroll
        for (int i = 0; i < 4; ++i) kcur[i] = koff_last[i];
      }
      if (ragged && v_last) {
#pragma unroll
        for (int i = 0; i < 4; ++i) vcur[i] = voff_last[i];
      }
      half_step(
          u, 0,
          [&]() SIDON_INLINE {
            dma_tile(ring_lds + c0, k_last ? klast : gk, kcur[0], kcur[1], kcur[2], kcur[3]);
          },
          [&]() SIDON_INLINE { pv(0); },
          [&]() SIDON_INLINE {
            qk(1);
            load_k(c1);
          },
          plain, off0);
      half_step(
          u, 1,
          [&]() SIDON_INLINE {
            dma_tile(ring_lds + kVRing + c1, v_last ? vlast : gv, vcur[0], vcur[1], vcur[2], vcur[3]);
          },
          [&]() SIDON_INLINE { pv(1); },
          [&]() SIDON_INLINE {
            qk(0);
            load_v(c0);
          },
          plain, off1);
      const uint32_t c = c0;
      c0 = c1;
      c1 = c;
      gk += kinc;
      gv += vinc;
    }
    __builtin_amdgcn_s_setprio(0);
    settle(nu - 1, 1);
    wait_lgkm0();
    pv(0);            // PV of the last step
    pv(1);
  }
  wait_vmcnt<0>();  // the last (unused) prefetches have landed before LDS is reused

  // ---- merge the key splits ----
  float l_tot[2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) l_tot[qb] = l_run[qb];

  lds_barrier();  // every wavefront is done with its ring and the q.rel table
  float* mo = reinterpret_cast<float*>(smem);
  float* ml = reinterpret_cast<float*>(smem + kMergeMlOff);
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    float* dst = mo + (w * kRows + 32 * qb + n) * kMergeStride;
#pragma unroll
    for (int db = 0; db < 2; ++db) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f4 val = {oacc[qb][db][4 * j], oacc[qb][db][4 * j + 1], oacc[qb][db][4 * j + 2],
                        oacc[qb][db][4 * j + 3]};
        *reinterpret_cast<f4*>(dst + 32 * db + 8 * j + 4 * g) = val;
      }
    }
    if (g == 0) {
      ml[(w * kRows + 32 * qb + n) * 2] = m_run[qb];
      ml[(w * kRows + 32 * qb + n) * 2 + 1] = l_tot[qb];
    }
  }
  lds_barrier();

  // Wavefront w finalises kRows / kWaves rows, kCols dims per lane.
  constexpr int kLanesPerRow = 64 / (kRows / kWaves);
  constexpr int kCols = kD / kLanesPerRow;  // 16 (4 waves) or 8 (8 waves)
  const int r = (kRows / kWaves) * w + lane / kLanesPerRow;
  const int c = kCols * (lane % kLanesPerRow);
  float mmax = -INFINITY;
#pragma unroll
  for (int s = 0; s < kWaves; ++s) mmax = fmaxf(mmax, ml[(s * kRows + r) * 2]);
  float lsum = 0.f;
  f4 o[kCols / 4] = {};
#pragma unroll
  for (int s = 0; s < kWaves; ++s) {
    const float ms = ml[(s * kRows + r) * 2];
    const float f = ms == -INFINITY ? 0.f : fast_exp2(ms - mmax);
    lsum += ml[(s * kRows + r) * 2 + 1] * f;
    const float* src = mo + (s * kRows + r) * kMergeStride + c;
#pragma unroll
    for (int j = 0; j < kCols / 4; ++j) o[j] += *reinterpret_cast<const f4*>(src + 4 * j) * f;
  }
  const int row = q0 + r;
  if (row < p.L) {
    const float inv = lsum > 0.f ? __builtin_amdgcn_rcpf(lsum) : 0.f;
    _Float16* dst = p.out + b * p.osb + h * p.osh + (int64_t)row * p.osl + c;
#pragma unroll
    for (int j = 0; j < kCols / 8; ++j) {
      const h8 v = {(_Float16)(o[2 * j][0] * inv), (_Float16)(o[2 * j][1] * inv),
                    (_Float16)(o[2 * j][2] * inv), (_Float16)(o[2 * j][3] * inv),
                    (_Float16)(o[2 * j + 1][0] * inv), (_Float16)(o[2 * j + 1][1] * inv),
                    (_Float16)(o[2 * j + 1][2] * inv), (_Float16)(o[2 * j + 1][3] * inv)};
      *reinterpret_cast<h8*>(dst + 8 * j) = v;
    }
  }
}

// ---------------------------------------------------------------------------
// host side

using sidon::aligned16;
using sidon::check_device;
using sidon::fail;

int check_strides(const char* name, const int64_t* st) {
  if (st == nullptr) return fail(SIDON_E_NULL, "%s_strides is NULL", name);
  for (int i = 0; i < 3; ++i) {
    if (st[i] < 0 || (st[i] & 7) != 0)
      return fail(SIDON_E_STRIDE, "%s stride[%d] = %lld must be a non-negative multiple of 8",
                  name, i, (long long)st[i]);
  }
  if (st[2] >= (int64_t(1) << 25))
    return fail(SIDON_E_STRIDE, "%s row stride %lld too large (< 2^25 elements)", name,
                (long long)st[2]);
  return SIDON_OK;
}

}  // namespace

namespace sidon {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_err[0] = '\0'; }

// One architecture check per device (gfx950 only).
namespace {
constexpr int kMaxDevices = 64;
std::once_flag g_dev_flags[kMaxDevices];
int g_dev_status[kMaxDevices];
int g_dev_cus[kMaxDevices];
}  // namespace

// The one-time query of device dev: 1 (gfx950), -1 (query failed), -2 (other
// architecture).  g_dev_status / g_dev_cus are written only inside the
// call_once and read only after it returned, which orders every read after
// the write on any thread.
int device_status(int dev) {
  std::call_once(g_dev_flags[dev], [dev]() {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
      g_dev_status[dev] = -1;
      return;
    }
    g_dev_cus[dev] = prop.multiProcessorCount;
    g_dev_status[dev] = strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : -2;
  });
  return g_dev_status[dev];
}

int check_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(SIDON_E_DEVICE, "hipGetDevice failed");
  if (dev < 0 || dev >= kMaxDevices) return fail(SIDON_E_DEVICE, "device index %d out of range", dev);
  const int st = device_status(dev);
  if (st == -1) return fail(SIDON_E_DEVICE, "hipGetDeviceProperties failed on device %d", dev);
  if (st != 1) return fail(SIDON_E_DEVICE, "device %d is not gfx950", dev);
  return SIDON_OK;
}

// Compute units of the current device (MI355X: 256); 256 when no gfx950
// device can be queried (host-only shape queries).
int compute_units() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices || device_status(dev) != 1) return 256;
  return g_dev_cus[dev];
}

}  // namespace sidon

namespace {

// Kernel variants: the 64-row workgroup with 8 key splits and one workgroup
// per compute unit (flexrel_fwd_kernel, any K / V strides); the 64-row
// workgroup with 4 key splits and two workgroups per compute unit
// (flexrel_w64.hip); the 32-row workgroup with 4 key splits
// (flexrel_w32.hip) for short sequences.
enum Variant { kSplit8 = 0, kW64 = 3, kW32 = 4 };

std::atomic<int> g_rerun_all{0};  // sidon_flexrel_debug_rerun_all

// SIDON_FLEXREL_VARIANT=split8|w64|w32 forces one variant (A/B timing and
// tests); unset, empty or "auto" picks by shape; any other value is an error
// (SIDON_E_CONFIG), so a mistyped override never runs silently on the
// automatic choice.  Read at every call that plans a launch (tests switch it
// between calls); a graph captured under one setting keeps that launch.
constexpr int kAuto = -1, kBadVariant = -2;
int forced_variant() {
  const char* e = getenv("SIDON_FLEXREL_VARIANT");
  if (e == nullptr || e[0] == '\0' || strcmp(e, "auto") == 0) return kAuto;
  if (strcmp(e, "split8") == 0) return (int)kSplit8;
  if (strcmp(e, "w64") == 0) return (int)kW64;
  if (strcmp(e, "w32") == 0) return (int)kW32;
  return kBadVariant;
}

// Automatic choice, from launch timings on MI355X (B = 1; H = 16 at
// L = 150 .. 4800, H = 1, 4, 8 at L = 512 .. 8000): when the 32-row kernel's
// workgroups (B H ceil(L / 32)) fit one per compute unit and the keys are
// few (L <= 1024), it is the fastest (its fixed costs -- q.rel table, steps
// near the diagonal, merge -- are half the 64-row kernel's, and no
// workgroup shares a compute unit; its compiled one-block step costs more
// than the 64-row kernel's hand-scheduled two-block step, so long key
// ranges favour the 64-row kernel whatever the grid: H = 1, L = 8000: 48.9
// against 35.1 us; H = 4, L = 2048: 16.3 against 14.6 us; H = 8, L = 1024:
// 10.6 against 11.2 us; H = 8, L = 600: 8.2 against 10.4 us).
// Otherwise the two-workgroups-per-CU 64-row kernel is the fastest or level
// with the fastest at every length (its key-step loop keeps the matrix core
// busy with two wavefronts per SIMD; the 32-row kernel's pairs contend in
// their latency-bound phases, the 8-split kernel's steps cost more).  K and
// V rows of different strides take the 8-split kernel, whatever the override.
constexpr int kW32MaxKeys = 1024;
int choose_variant(int B, int H, int L, bool same_stride, Variant* out) {
  if (!same_stride) {  // the other kernels are built for K and V rows of one stride
    *out = kSplit8;
    return SIDON_OK;
  }
  const int f = forced_variant();
  if (f == kBadVariant)
    return fail(SIDON_E_CONFIG, "SIDON_FLEXREL_VARIANT=%s is not one of split8, w64, w32, auto",
                getenv("SIDON_FLEXREL_VARIANT"));
  if (f != kAuto) {
    *out = (Variant)f;
    return SIDON_OK;
  }
  const long long w32_blocks = (long long)B * H * ((L + w32_rows() - 1) / w32_rows());
  *out = L <= kW32MaxKeys && w32_blocks <= sidon::compute_units() ? kW32 : kW64;
  return SIDON_OK;
}

// One launch: `rows` query rows per workgroup, nqb blocks per (b, h) from
// query row row0.
struct Launch {
  Variant kernel;  // kSplit8, kW64 or kW32
  int rows, splits, threads, nqb, row0;
  long long nwg;
};
struct Plan {
  int n;
  Launch l[2];
};

Launch launch_of(Variant kernel, int B, int H, int nqb, int row0) {
  Launch x;
  x.kernel = kernel;
  x.rows = kernel == kW64 ? w64_rows() : kernel == kW32 ? w32_rows() : kRows;
  x.splits = kernel == kSplit8 ? kWaves : 4;
  x.threads = kernel == kW64 ? w64_threads() : kernel == kW32 ? w32_threads() : kThreads;
  x.nqb = nqb;
  x.row0 = row0;
  x.nwg = (long long)B * H * nqb;
  return x;
}

int plan_of(int B, int H, int L, bool same_stride, Plan* pl) {
  Variant v;
  const int rc = choose_variant(B, H, L, same_stride, &v);
  if (rc) return rc;
  const int rows = v == kW64 ? w64_rows() : v == kW32 ? w32_rows() : kRows;
  pl->n = 1;
  pl->l[0] = launch_of(v, B, H, (L + rows - 1) / rows, 0);
  return SIDON_OK;
}

}  // namespace

namespace {
// The plan of a call whose K and V rows have the same stride or not, with
// the grid-size check of every launch.
int checked_plan(int B, int H, int L, bool same_stride, Plan* pl) {
  if (B < 1 || H < 1 || L < 1) return fail(SIDON_E_SHAPE, "B=%d H=%d L=%d must be >= 1", B, H, L);
  const int rc = plan_of(B, H, L, same_stride, pl);
  if (rc) return rc;
  long long total = 0;
  for (int i = 0; i < pl->n; ++i) total += pl->l[i].nwg;
  if (total >= (1LL << 31)) return fail(SIDON_E_SHAPE, "grid of %lld workgroups too large", total);
  return SIDON_OK;
}
}  // namespace

SIDON_API int sidon_flexrel_launch_shape(int B, int H, int L, int* queries_per_block,
                                         int* key_splits, int* workgroups, int* threads_per_block) {
  sidon::clear_error();
  Plan pl;
  const int rc = checked_plan(B, H, L, true, &pl);
  if (rc) return rc;
  long long total = 0;
  for (int i = 0; i < pl.n; ++i) total += pl.l[i].nwg;
  // The first launch's shape; workgroups counts every launch of the call.
  if (queries_per_block) *queries_per_block = pl.l[0].rows;
  if (key_splits) *key_splits = pl.l[0].splits;
  if (workgroups) *workgroups = (int)total;
  if (threads_per_block) *threads_per_block = pl.l[0].threads;
  return SIDON_OK;
}

SIDON_API int sidon_flexrel_fwd(const void* q, const void* k, const void* v, const void* rel,
                                const int32_t* lens, void* out, int B, int H, int L, int head_dim,
                                const int64_t* q_strides, const int64_t* k_strides,
                                const int64_t* v_strides, const int64_t* o_strides,
                                sidon_stream_t stream) {
  sidon::clear_error();
  if (!q || !k || !v || !rel || !out) return fail(SIDON_E_NULL, "q, k, v, rel and out must be non-NULL");
  if (head_dim != kD) return fail(SIDON_E_SHAPE, "head_dim must be 64 (got %d)", head_dim);
  if (B < 1 || H < 1 || L < 1) return fail(SIDON_E_SHAPE, "B=%d H=%d L=%d must be >= 1", B, H, L);
  int rc;
  if ((rc = check_strides("q", q_strides)) || (rc = check_strides("k", k_strides)) ||
      (rc = check_strides("v", v_strides)) || (rc = check_strides("out", o_strides)))
    return rc;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(rel) || !aligned16(out))
    return fail(SIDON_E_ALIGN, "q, k, v, rel and out must be 16-byte aligned");
  // the device first: the plan reads its compute-unit count
  if ((rc = check_device())) return rc;
  Plan pl;
  if ((rc = checked_plan(B, H, L, k_strides[2] == v_strides[2], &pl))) return rc;

  Params p;
  p.q = static_cast<const _Float16*>(q);
  p.k = static_cast<const _Float16*>(k);
  p.v = static_cast<const _Float16*>(v);
  p.rel = static_cast<const _Float16*>(rel);
  p.lens = lens;
  p.out = static_cast<_Float16*>(out);
  p.qsb = q_strides[0];
  p.qsh = q_strides[1];
  p.qsl = (int)q_strides[2];
  p.ksb = k_strides[0];
  p.ksh = k_strides[1];
  p.ksl = (int)k_strides[2];
  p.vsb = v_strides[0];
  p.vsh = v_strides[1];
  p.vsl = (int)v_strides[2];
  p.osb = o_strides[0];
  p.osh = o_strides[1];
  p.osl = (int)o_strides[2];
  p.B = B;
  p.H = H;
  p.L = L;
  p.scale = 1.4426950408889634f / 8.0f;  // log2(e) / sqrt(64)
  p.rerun_all = g_rerun_all.load(std::memory_order_relaxed);

  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t err = hipSuccess;
  for (int i = 0; i < pl.n && err == hipSuccess; ++i) {
    const Launch& x = pl.l[i];
    p.nqb = x.nqb;
    p.row0 = x.row0;
    if (x.kernel == kW64) {
      err = launch_w64(p, (int)x.nwg, true, s);
    } else if (x.kernel == kW32) {
      err = launch_w32(p, (int)x.nwg, true, s);
    } else {
      if (p.ksl == p.vsl)
        hipLaunchKernelGGL(flexrel_fwd_kernel<true>, dim3((unsigned)x.nwg), dim3(kThreads), 0, s, p);
      else
        hipLaunchKernelGGL(flexrel_fwd_kernel<false>, dim3((unsigned)x.nwg), dim3(kThreads), 0, s, p);
      err = hipGetLastError();
    }
  }
  if (err != hipSuccess) return fail(SIDON_E_LAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
  return SIDON_OK;
}

SIDON_API int sidon_flexrel_fwd_qkv(const void* qkv, const void* rel, const int32_t* lens, void* out,
                                    int B, int H, int L, sidon_stream_t stream) {
  sidon::clear_error();
  if (!qkv || !out || !rel) return fail(SIDON_E_NULL, "qkv, rel and out must be non-NULL");
  if (B < 1 || H < 1 || L < 1) return fail(SIDON_E_SHAPE, "B=%d H=%d L=%d must be >= 1", B, H, L);
  const int64_t hid = (int64_t)H * kD;
  const int64_t in_st[3] = {(int64_t)L * 3 * hid, kD, 3 * hid};
  const int64_t out_st[3] = {(int64_t)L * hid, kD, hid};
  const _Float16* base = static_cast<const _Float16*>(qkv);
  return sidon_flexrel_fwd(base, base + hid, base + 2 * hid, rel, lens, out, B, H, L, kD, in_st,
                           in_st, in_st, out_st, stream);
}

// Test hook: with `on` nonzero, every wavefront of the 64-row kernel discards
// its hand-scheduled loop's results and runs its steps again through the
// compiled general code (the path a wavefront takes when a probability
// leaves the fp16 range), so that the two can be compared bit for bit on
// every row.  Read at each sidon_flexrel_fwd call (a captured graph keeps the
// value of its capture).
SIDON_API void sidon_flexrel_debug_rerun_all(int on) { g_rerun_all.store(on != 0, std::memory_order_relaxed); }

SIDON_API const char* sidon_last_error(void) { return sidon::g_err; }

SIDON_API const char* sidon_version(void) { return "sidon-flexrel 0.3.0 gfx950"; }
