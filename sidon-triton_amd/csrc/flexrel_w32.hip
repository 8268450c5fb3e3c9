// flexrel_w32.hip -- relative_key flash attention for short sequences, 32
// query rows per workgroup (MI355X / gfx950).  Same math and results
// contract as flexrel_fwd.hip (src/sidon_triton/triton_encoder.py:210-312):
//
//   s_ij = (q_i . k_j + q_i . rel[clamp(j - i, -64, 8) + 64]) / sqrt(64)
//   o_i  = sum_{j < LK_b} softmax_j(s_ij) v_j
//
// Why a second shape.  At a few hundred keys a launch of flexrel_w64.hip (64
// rows, two 32-row blocks per wavefront) has 16 ceil(L / 64) workgroups for
// 256 compute units, and a workgroup's time is latency-bound work whose length
// grows with the rows a wavefront owns: the q.rel table, the steps near the
// diagonal that gather the bias per score, the merge.  One 32-row block per
// workgroup gives twice the workgroups and halves that work on the critical
// path; the key-step loop runs through compiler-scheduled code (a wavefront
// has at most a few steps at these lengths).
//
// Work decomposition: 4 wavefronts; wavefront w takes the key steps w, w + 4,
// w + 8, ... (32 keys each) for all 32 rows, and the four partial results are
// merged through LDS.  Per step: S^T = K . Q^T (4 v_mfma_f32_32x32x16_f16, Q^T
// in registers), the softmax through the exact general form (per-score bias
// gather near the diagonal, constant bias left or right of the window, key
// mask at LK, running max raised per query when a step's probabilities would
// leave the fp16 range), row sums on the matrix core and O^T += V^T . P^T
// (4 MFMAs).  K operands are loaded from global memory into registers (two
// buffers); V tiles pass through a two-slot LDS ring per wavefront
// (global_load_lds_dwordx4, read transposed with ds_read_b64_tr_b16).  The
// loads of step u + 1 are issued before the arithmetic of step u.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "flexrel_device.h"

#define SIDON_INLINE __attribute__((always_inline))

namespace sidon_flexrel {
namespace {

constexpr int kRows = 32;    // query rows per workgroup = per wavefront
constexpr int kWaves = 4;    // key splits
constexpr int kThreads = 64 * kWaves;
// LDS: V slot 0 of wavefront w at 4 KB w, V slot 1 at 16 KB + 4 KB w, then the
// q.rel table (32 rows of kQrStride fp32).
constexpr int kVSlot1 = kWaves * kTile;
constexpr int kQrOff = 2 * kWaves * kTile;
constexpr int kPreBytes = kQrOff + kRows * kQrStride * 4;
// Prologue staging in the V slot 1 region, which the loop fills only after
// the q.rel table is built: the Q block (32 rows), rel rows 0-63, rel rows
// 64-79 (row 72 repeated past it).
constexpr int kQStageOff = kVSlot1;
constexpr int kRelOff = kQStageOff + kRows * kD * 2;
constexpr int kRel2Off = kRelOff + 2 * kTile;
static_assert(kRel2Off + 16 * kD * 2 <= kQrOff, "the staged rows fit the V slot 1 region");
constexpr int kMergeStride = 68;  // fp32 per partial-output row
constexpr int kMergeMlOff = kWaves * kRows * kMergeStride * 4;
constexpr int kMergeBytes = kMergeMlOff + kWaves * kRows * 2 * 4;
constexpr int kLdsBytes = kPreBytes > kMergeBytes ? kPreBytes : kMergeBytes;
static_assert(kLdsBytes <= 64 * 1024, "at least two workgroups per compute unit");

__global__ void __launch_bounds__(kThreads) flexrel_w32_kernel(const Params p) {
  __shared__ __attribute__((aligned(16))) char smem[kLdsBytes];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 31;  // query column of this lane
  const int g = lane >> 5;  // lane half

  const int lin = xcd_linear(blockIdx.x, gridDim.x);
  const int bh = lin / p.nqb;
  const int qblk = lin - bh * p.nqb;
  const int b = bh / p.H;
  const int h = bh - b * p.H;

  const int q0 = p.row0 + qblk * kRows;
  const float scale = p.scale;
  const _Float16* qbase = p.q + b * p.qsb + h * p.qsh;
  // The valid length: a scalar load, awaited at its first use below.
  int lk_raw = p.L;
  if (p.lens != nullptr) lk_raw = p.lens[__builtin_amdgcn_readfirstlane(b)];

  // ---- prologue: the Q rows and rel rows staged in LDS (wavefront 0: Q,
  // 1 and 2: rel rows 0-63, 3: rel rows 64-79) ----
  const uint32_t smem_lds = (uint32_t)(uintptr_t)SIDON_LDS_PTR(char, smem);
  auto stage_rows = [&](uint32_t lds, const char* src, int64_t stride, int row0, int rmax, int nk) SIDON_INLINE {
    // rows row0 + [0, 8 nk) of src (clamped to rmax) into LDS at lds, swizzled
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (i >= nk) break;
      const int r = 8 * i + (lane >> 3);
      const uint32_t off = (uint32_t)((min(row0 + r, rmax) - row0) * stride) + 16u * ((lane & 7) ^ tile_swz(r));
      dma_1k(lds + 1024u * i, src + row0 * stride, off);
    }
  };
  if (w == 0) {
    const int row0 = min(q0, p.L - 1);
    stage_rows(smem_lds + kQStageOff, reinterpret_cast<const char*>(qbase), (int64_t)p.qsl * 2, row0, p.L - 1, 4);
  } else if (w < 3) {
    stage_rows(smem_lds + kRelOff + 4096u * (w - 1), reinterpret_cast<const char*>(p.rel), kD * 2, 32 * (w - 1),
               kNumPos - 1, 4);
  } else {
    stage_rows(smem_lds + kRel2Off, reinterpret_cast<const char*>(p.rel), kD * 2, 64, kNumPos - 1, 2);
  }

  const int LK = __builtin_amdgcn_readfirstlane(min(max(lk_raw, 0), p.L));
  const char* kbase = reinterpret_cast<const char*>(p.k + b * p.ksb + h * p.ksh);
  const char* vbase = reinterpret_cast<const char*>(p.v + b * p.vsb + h * p.vsh);
  const int64_t kstride = (int64_t)p.ksl * 2;  // bytes (V rows have the same stride)

  // Key steps: T steps of 32 keys cover [0, LK); this wavefront takes steps
  // w + 4 u, u = 0 .. nu - 1.
  const int T = (LK + kStep - 1) / kStep;
  const int nu = T > w ? (T - w + kWaves - 1) / kWaves : 0;
  const bool active = nu > 0;
  const int last_row = LK - 1 - (T - 1) * kStep;  // in [0, 31] when T > 0
  const bool ragged = LK % kStep != 0;           // step T - 1 straddles LK
  const LaneTab lt = lane_tab(lane, kstride, last_row);

  const uint32_t ring_lds = smem_lds + w * kTile;  // V slot 0 of this wavefront
  auto copy_v = [&](int u, uint32_t slot) SIDON_INLINE {
    const int t = w + kWaves * u;
    const char* gb = vbase + (int64_t)(t * kStep) * kstride - 3072;
    const bool last = ragged && t == T - 1;
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = last ? lt.voff_last[i] : lt.voff[i];
    dma_tile(slot, gb, o[0], o[1], o[2], o[3]);
  };
  auto load_k = [&](int u, h8 (&dst)[4]) SIDON_INLINE {
    const int t = w + kWaves * u;
    const char* gb = kbase + (int64_t)(t * kStep) * kstride + ((ragged && t == T - 1) ? lt.kofs_last : lt.kofs);
#pragma unroll
    for (int s = 0; s < 4; ++s) dst[s] = *reinterpret_cast<const h8*>(gb + 32 * s);
  };

  // V(0) into slot 0 and K(0) into buffer 0, in flight with the staging.
  h8 kop[2][4];
  if (active) {
    copy_v(0, ring_lds);
    load_k(0, kop[0]);
    // the staged rows have landed: every memory operation but the 8 issued
    // last (the copy and the K loads)
    wait_vmcnt<8>();
  } else {
    wait_vmcnt<0>();
  }
  lds_barrier();  // the Q block and the rel rows are in LDS

  // Q^T as the MFMA B operand: lane (n, g) holds query q0 + n, dims 16 s +
  // 8 g + [0, 8) for k-step s.  Rows >= L are 0.
  h8 qop[4];
  {
    const char* qrow = smem + kQStageOff + n * 128;
#pragma unroll
    for (int s = 0; s < 4; ++s) qop[s] = *reinterpret_cast<const h8*>(qrow + (((2 * s + g) ^ tile_swz(n)) << 4));
    if (q0 + n >= p.L) {
#pragma unroll
      for (int s = 0; s < 4; ++s) qop[s] = h8{};
    }
  }

  // q.rel^T * scale for the 32 rows: three (32 positions x 32 rows) tiles
  // rel . Q^T, tile w on wavefront w < 3.  Rel rows >= 73 are 0.
  float* qr_tab = reinterpret_cast<float*>(smem + kQrOff);
  if (w < 3) {
    const int pb = w;
    const int pos = 32 * pb + n;
    const char* rrow = pb < 2 ? smem + kRelOff + pb * kTile + n * 128 : smem + kRel2Off + min(n, 15) * 128;
    f32x16 acc = {};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      h8 e = *reinterpret_cast<const h8*>(rrow + (((2 * s + g) ^ tile_swz(n)) << 4));
      if (pos >= kNumPos) e = h8{};
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(e, qop[s], acc, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int pos0 = 32 * pb + 8 * i + 4 * g;
      if (pos0 < kQrStride) {
        const f4 val = {acc[4 * i] * scale, acc[4 * i + 1] * scale, acc[4 * i + 2] * scale, acc[4 * i + 3] * scale};
        *reinterpret_cast<f4*>(qr_tab + n * kQrStride + pos0) = val;
      }
    }
  }

  f32x16 oacc[2] = {};  // O^T: dims 32 db + 8 (i/4) + 4 g + i%4, query n
  float m_run = -INFINITY;
  f4 lsum = {};         // running row sum (rowsum below): each value is the query's sum
  f32x16 sacc;          // S^T of the current step
  h8 pk[2];             // fp16 probabilities [16-key half]
  h8 vop[2][2];         // V^T operands [hh][db] of one step

  auto load_v = [&](int sl) SIDON_INLINE {
    const char* vt = smem + w * kTile + (sl ? kVSlot1 : 0);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        const h4 lo = __builtin_bit_cast(
            h4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(SIDON_LDS_PTR(s4, vt + lt.tr_off[0][db] + 2048 * hh)));
        const h4 hi = __builtin_bit_cast(
            h4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(SIDON_LDS_PTR(s4, vt + lt.tr_off[1][db] + 2048 * hh)));
        vop[hh][db] = cat(lo, hi);
      }
    }
  };

  // Row sums on the matrix core with v_mfma_f32_16x16x32_f16 (the selector
  // operand of flexrel_w64.hip): read as a 16x16x32 B operand, the
  // probability tile of lane l = c + 16 j holds query c + 16 (j % 2), keys
  // 8 (j / 2) + [0, 8) of the 16-key half; the A operand "sel" of lane l is 1
  // where bit 4 of l equals bit 2 of l, so the four rows lane l receives are
  // its own query's sum.
  const _Float16 sel_v = (((lane >> 4) ^ (lane >> 2)) & 1) == 0 ? (_Float16)1 : (_Float16)0;
  const h8 sel = {sel_v, sel_v, sel_v, sel_v, sel_v, sel_v, sel_v, sel_v};

  auto emit = [&](int i, const f2& e) SIDON_INLINE {
    const h2 ph = __builtin_convertvector(e, h2);
    pk[i >> 3][i & 7] = ph[0];
    pk[i >> 3][(i & 7) + 1] = ph[1];
  };

  const float* qrow_tab = qr_tab;  // row n of the table (set after the barrier below)
  float ql = 0.f, qrr = 0.f;       // the bias left / right of the window for query n

  // Step u of this wavefront, from K(u) in kop[bf] and V(u) in ring slot bf:
  // scores, probabilities with the running max, row sums, PV.  The max is
  // set exactly at the first step and raised for the queries whose fp16
  // probabilities would not be finite (a step sum >= 2^15 in fp32), decided
  // per query, never per wavefront.
  auto step = [&](int u, int bf) SIDON_INLINE {
    if (u + 1 < nu) {
      // the transpose reads of V(u - 1) (slot bf ^ 1) are done: prefetch
      // K(u + 1) into buffer bf ^ 1 and V(u + 1) into slot bf ^ 1
      wait_lgkm0();
      load_k(u + 1, kop[bf ^ 1]);
      copy_v(u + 1, ring_lds + (bf ^ 1) * kVSlot1);
    }
    load_v(bf);
    {
      f32x16 acc = {};
#pragma unroll
      for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kop[bf][s], qop[s], acc, 0, 0, 0);
      sacc = acc;
    }
    const int k0 = (w + kWaves * u) * kStep;
    const bool left = k0 + (kStep - 1) - q0 <= -kLeft;
    const bool right = k0 - (q0 + kRows - 1) >= kRight;
    const bool masked = k0 + kStep > LK;
    const float off = left ? ql : qrr;
    float y[16];
    if (!left && !right) {
      const int d0 = k0 + 8 * g - (q0 + n) + kLeft;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int idx = min(max(d0 + 16 * (i >> 3) + (i & 7), 0), kLeft + kRight);
        y[i] = fmaf(sacc[i], scale, qrow_tab[idx]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) y[i] = fmaf(sacc[i], scale, off);
    }
    if (masked) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = k0 + 16 * (i >> 3) + 8 * g + (i & 7);
        if (key >= LK) y[i] = -INFINITY;
      }
    }
    auto probs = [&](float m) SIDON_INLINE {
      float sum = 0.f;
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        const f2 e = {fast_exp2(y[i] - m), fast_exp2(y[i + 1] - m)};
        sum += e[0] + e[1];
        emit(i, e);
      }
      return sum;
    };
    bool need = u == 0;
    if (!need) {
      const float own = probs(m_run);
      const auto pr = __builtin_amdgcn_permlane32_swap(__float_as_uint(own), __float_as_uint(own), false, false);
      need = !(__uint_as_float(pr[0]) + __uint_as_float(pr[1]) < kSumLimit);
    }
    if (__builtin_amdgcn_ballot_w64(need) != 0) {
      float mx = y[0];
#pragma unroll
      for (int i = 1; i < 16; ++i) mx = fmaxf(mx, y[i]);
      mx = pair_max(mx);
      const float m_new = need ? fmaxf(m_run, mx) : m_run;
      const float alpha = fast_exp2(m_run - m_new);  // 1 if unchanged, 0 from -inf
      if (u != 0 && __builtin_amdgcn_ballot_w64(alpha != 1.f) != 0) {
        oacc[0] *= alpha;
        oacc[1] *= alpha;
      }
      lsum *= alpha;
      m_run = m_new;
      probs(m_new);
    }
    lsum = __builtin_amdgcn_mfma_f32_16x16x32_f16(sel, pk[0], lsum, 0, 0, 0);
    lsum = __builtin_amdgcn_mfma_f32_16x16x32_f16(sel, pk[1], lsum, 0, 0, 0);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int db = 0; db < 2; ++db)
        oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vop[hh][db], pk[hh], oacc[db], 0, 0, 0);
  };

  lds_barrier();  // the q.rel table is complete
  qrow_tab = qr_tab + n * kQrStride;
  ql = qrow_tab[0];
  qrr = qrow_tab[kNumPos - 1];

  for (int u = 0; u < nu; u += 2) {
    wait_vmcnt<0>();  // K(u) and V(u) have landed
    step(u, 0);
    if (u + 1 >= nu) break;
    wait_vmcnt<0>();
    step(u + 1, 1);
  }

  // ---- merge the key splits ----
  wait_vmcnt<0>();  // (no copy is in flight: the last step issues none)
  lds_barrier();    // every wavefront is done with its ring and the q.rel table
  float* mo = reinterpret_cast<float*>(smem);
  float* ml = reinterpret_cast<float*>(smem + kMergeMlOff);
  {
    float* dst = mo + (w * kRows + n) * kMergeStride;
#pragma unroll
    for (int db = 0; db < 2; ++db) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f4 val = {oacc[db][4 * j], oacc[db][4 * j + 1], oacc[db][4 * j + 2], oacc[db][4 * j + 3]};
        *reinterpret_cast<f4*>(dst + 32 * db + 8 * j + 4 * g) = val;
      }
    }
    if (g == 0) {
      ml[(w * kRows + n) * 2] = m_run;
      ml[(w * kRows + n) * 2 + 1] = lsum[0];
    }
  }
  lds_barrier();

  // Wavefront w finalises rows 8 w + [0, 8), eight lanes per row, 8 dims per
  // lane.
  const int r = 8 * w + (lane >> 3);
  const int c = 8 * (lane & 7);
  float mmax = -INFINITY;
#pragma unroll
  for (int s = 0; s < kWaves; ++s) mmax = fmaxf(mmax, ml[(s * kRows + r) * 2]);
  float total = 0.f;
  f4 o[2] = {};
#pragma unroll
  for (int s = 0; s < kWaves; ++s) {
    const float ms = ml[(s * kRows + r) * 2];
    const float f = ms == -INFINITY ? 0.f : fast_exp2(ms - mmax);
    total += ml[(s * kRows + r) * 2 + 1] * f;
    const float* src = mo + (s * kRows + r) * kMergeStride + c;
    o[0] += *reinterpret_cast<const f4*>(src) * f;
    o[1] += *reinterpret_cast<const f4*>(src + 4) * f;
  }
  const int row = q0 + r;
  if (row < p.L) {
    const float inv = total > 0.f ? __builtin_amdgcn_rcpf(total) : 0.f;
    _Float16* dst = p.out + b * p.osb + h * p.osh + (int64_t)row * p.osl + c;
    const h8 v = {(_Float16)(o[0][0] * inv), (_Float16)(o[0][1] * inv), (_Float16)(o[0][2] * inv),
                  (_Float16)(o[0][3] * inv), (_Float16)(o[1][0] * inv), (_Float16)(o[1][1] * inv),
                  (_Float16)(o[1][2] * inv), (_Float16)(o[1][3] * inv)};
    *reinterpret_cast<h8*>(dst) = v;
  }
}

}  // namespace

int w32_rows() { return kRows; }
int w32_threads() { return kThreads; }

// Only K and V rows of the same stride (one set of lane offsets serves both).
hipError_t launch_w32(const Params& p, int nwg, bool same_stride, hipStream_t stream) {
  if (!same_stride) return hipErrorInvalidValue;
  hipLaunchKernelGGL(flexrel_w32_kernel, dim3(nwg), dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace sidon_flexrel
