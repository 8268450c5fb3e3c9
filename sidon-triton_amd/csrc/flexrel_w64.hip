// flexrel_w64.hip -- relative_key flash attention, 64 query rows per
// workgroup and two workgroups per compute unit (MI355X / gfx950).  Same
// math and results contract as flexrel_fwd.hip
// (src/sidon_triton/triton_encoder.py:210-312):
//
//   s_ij = (q_i . k_j + q_i . rel[clamp(j - i, -64, 8) + 64]) / sqrt(64)
//   o_i  = sum_{j < LK_b} softmax_j(s_ij) v_j
//
// Work decomposition.  One workgroup owns 64 query rows of one (b, h) and has
// 4 wavefronts; wavefront w runs an online softmax for all 64 rows (two
// 32-query column blocks) over the key steps w, w + 4, w + 8, ... (32 keys
// each), and the four partial results are merged through LDS at the end.
// A workgroup needs at most 256 registers per lane and 73 KB of LDS, so two
// workgroups share a compute unit: every SIMD runs two wavefronts, and one
// issues its vector work while the other's products hold the matrix core
// (one wavefront alone issues a vector instruction only every ~5.4 cycles,
// which leaves the matrix core idle for part of each step), and one
// workgroup's prologue and merge overlap the other's key steps.
//
// Per wavefront and step (32 keys), for each block J: S^T = K . Q^T (4
// v_mfma_f32_32x32x16_f16, Q^T in registers), the exp2 softmax with the lazily
// updated running max of flexrel_fwd.hip, the row sums on the matrix core (2
// v_mfma_f32_16x16x32_f16) and O^T += V^T . P^T (4 MFMAs).  K and V tiles
// pass through LDS, copied with global_load_lds_dwordx4: K through one slot
// per wavefront (tile j + 3 copied once tile j + 2 is in registers; two
// register buffers), V through a two-slot ring read transposed with
// ds_read_b64_tr_b16.
// The key-step loop is hand-scheduled assembly (flexrel_w64_step.inc,
// written and checked by gen_w64_step.py); a wavefront whose probabilities
// leave the fp16 range reruns its steps through the C++ code below, which
// computes the same values for every query that stays in range.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "flexrel_device.h"
#include "flexrel_w64_step.inc"

#define SIDON_INLINE __attribute__((always_inline))

namespace sidon_flexrel {
namespace {

constexpr int kRows = 64;      // query rows per workgroup = per wavefront
constexpr int kBlocks = 2;     // 32-query column blocks per wavefront
constexpr int kWaves = 4;      // key splits
constexpr int kThreads = 64 * kWaves;
// LDS: three tiles per wavefront -- V slots 0 and 1 and one K slot -- each
// kind in its own 16 KB region (tile of wavefront w at 4 KB w), then the
// q.rel table.
constexpr int kSlotStride = kWaves * kTile;      // 16 KB: V slot 0, V slot 1, K
constexpr int kVSlot1 = kSlotStride;
constexpr int kKSlot = 2 * kSlotStride;
constexpr int kQrOff = 3 * kSlotStride;
// q.rel table rows: position p (0..72) at float kQrPad + p; floats
// [0, kQrPad) repeat position 0 and [kQrPad + 73, kQrPad + 81) position 72,
// so a run of 8 consecutive positions clamped to [0, 72] is 8 consecutive
// floats of the row from the clamped start -- the band steps read a lane's
// 16 biases as two such runs (ds_read2_b32).
constexpr int kQrPad = 8;
constexpr int kQrRow = 92;  // floats per row: kQrPad + 73 + 8, rounded up to 16 bytes
constexpr int kPreBytes = kQrOff + kRows * kQrRow * 4;
// Prologue staging, over regions the loop fills only after the q.rel table
// is built: the Q block (64 rows) and rel rows 0-63 in the V slot 1 region,
// rel rows 64-79 (row 72 repeated past it) after the table.
constexpr int kQStageOff = kVSlot1;
constexpr int kRelOff = kQStageOff + kRows * kD * 2;
static_assert(kRelOff + 2 * kTile == kKSlot, "Q block and rel rows 0-63 fill the V slot 1 region");
constexpr int kRel2Off = kPreBytes;
constexpr int kMergeStride = 68;                            // fp32 per partial-output row
constexpr int kMergeMlOff = kWaves * kRows * kMergeStride * 4;
constexpr int kMergeBytes = kMergeMlOff + kWaves * kRows * 2 * 4;
constexpr int kLdsBytes = kPreBytes + 2048 > kMergeBytes ? kPreBytes + 2048 : kMergeBytes;
static_assert(2 * kLdsBytes <= 160 * 1024, "two workgroups per CU");

typedef float f32x4 __attribute__((ext_vector_type(4)));

// The per-lane offsets (LaneTab, lane_tab) are formed twice: for the
// prologue and the key-step loop, and again from a fresh lane id after the
// loop (for the rerun and the merge), so that no lane-dependent value has to
// survive the loop, which holds all 256 registers.

__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
flexrel_w64_kernel(const Params p) {
  __shared__ __attribute__((aligned(16))) char smem[kLdsBytes];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 31;  // query column of this lane (within a 32-block)
  const int g = lane >> 5;  // lane half

  const int lin = xcd_linear(blockIdx.x, gridDim.x);
  const int bh = lin / p.nqb;
  const int qblk = lin - bh * p.nqb;
  const int b = bh / p.H;
  const int h = bh - b * p.H;

  const int q0 = p.row0 + qblk * kRows;
  const float scale = p.scale;
  const _Float16* qbase = p.q + b * p.qsb + h * p.qsh;
  // The valid length: a scalar load (uniform address), awaited at its first
  // use below -- a vector load would be awaited with every copy in flight.
  int lk_raw = p.L;
  if (p.lens != nullptr) lk_raw = p.lens[__builtin_amdgcn_readfirstlane(b)];

  // ---- prologue, part 1: the Q rows and rel rows, which do not depend on
  // the valid length, are staged in LDS before that length is read ----
  const uint32_t q_lds = (uint32_t)(uintptr_t)SIDON_LDS_PTR(char, smem + kQStageOff);
  const uint32_t rel_lds = (uint32_t)(uintptr_t)SIDON_LDS_PTR(char, smem + kRelOff);
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
  if (w < 2) {
    const int row0 = min(q0 + 32 * w, p.L - 1);
    stage_rows(q_lds + 4096u * w, reinterpret_cast<const char*>(qbase), (int64_t)p.qsl * 2, row0,
               p.L - 1, 4);
  } else {
    stage_rows(rel_lds + 4096u * (w - 2), reinterpret_cast<const char*>(p.rel), kD * 2, 32 * (w - 2),
               kNumPos - 1, 4);
  }
  if (w == 1)
    stage_rows((uint32_t)(uintptr_t)SIDON_LDS_PTR(char, smem + kRel2Off), reinterpret_cast<const char*>(p.rel),
               kD * 2, 64, kNumPos - 1, 2);

  const int LK = __builtin_amdgcn_readfirstlane(min(max(lk_raw, 0), p.L));

  const char* kbase = reinterpret_cast<const char*>(p.k + b * p.ksb + h * p.ksh);
  const char* vbase = reinterpret_cast<const char*>(p.v + b * p.vsb + h * p.vsh);
  const int64_t kstride = (int64_t)p.ksl * 2;  // bytes (V rows have the same stride)

  // Key steps: T steps of 32 keys cover [0, LK); this wavefront takes steps
  // w + 4 u, u = 0 .. nu - 1.
  const int T = (LK + kStep - 1) / kStep;
  const int nu = T > w ? (T - w + kWaves - 1) / kWaves : 0;
  const bool active = nu > 0;

  // Step classes per block J (32 rows at q0 + 32 J): steps u <= uL[J] lie
  // entirely left of the window (j - i <= -64), u >= uR[J] entirely right
  // (j - i >= 8); uM is the first step that straddles LK (at most one: the
  // wavefront's last).  (Arithmetic shifts: floor and ceiling divisions by
  // 128 = 4 steps of 32.)
  int uL[kBlocks], uR[kBlocks];
#pragma unroll
  for (int J = 0; J < kBlocks; ++J) {
    uL[J] = (q0 + 32 * J - 95 - kStep * w) >> 7;
    uR[J] = -((-(q0 + 32 * J + 39 - kStep * w)) >> 7);
  }
  const int uM = ((LK - kStep - kStep * w) >> 7) + 1;
  // Processing order: the special steps first -- the band steps [cL, cR)
  // where some block needs the per-score bias gather, then the straddling
  // step -- and then the plain steps [0, cL), [cR, uE).  The first processed
  // step sets the running max exactly; a wavefront with no special step runs
  // its first plain step through the special code for that.
  const int uE = min(uM, nu);
  const int cL = min(max(uL[0] + 1, 0), uE);
  const int cR = min(max(uR[kBlocks - 1], cL), uE);
  const int nS = (cR - cL) + (nu - uE);
  const int nSlow = nu > 0 ? max(nS, 1) : 0;
  auto u_of = [&](int j) SIDON_INLINE {
    if (j < cR - cL) return cL + j;
    if (j < nS) return uE;
    const int k = j - nS;
    return k + (k >= cL ? cR - cL : 0);
  };

  char* ring = smem + w * kTile;  // V slot 0 of this wavefront
  const uint32_t ring_lds = (uint32_t)(uintptr_t)SIDON_LDS_PTR(char, ring);

  const int last_row = LK - 1 - (T - 1) * kStep;  // in [0, 31]
  const LaneTab lt = lane_tab(lane, kstride, last_row);
  const bool ragged = LK % kStep != 0;  // step T - 1 straddles LK

  // Global step and tile base of processing index j (clamped to the last
  // index: prefetches past it re-read the last processed step).
  auto step_of = [&](int j) SIDON_INLINE { return w + kWaves * u_of(min(j, nu - 1)); };
  // Copy of the K or V tile of processing index j into an LDS slot (K and V
  // rows share the stride, so one set of lane offsets serves both).
  auto copy_v = [&](const LaneTab& t, int j, uint32_t slot, const char* base) SIDON_INLINE {
    const int step = step_of(j);
    const char* gb = base + (int64_t)(step * kStep) * kstride - 3072;
    const bool last = ragged && step == T - 1;
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t a = t.voff[i], c = t.voff_last[i];
      o[i] = last ? c : a;
    }
    dma_tile(slot, gb, o[0], o[1], o[2], o[3]);
  };
  auto load_k = [&](const LaneTab& lt_, int j, h8 (&dst)[4]) SIDON_INLINE {
    const int t = step_of(j);
    const char* gb = kbase + (int64_t)(t * kStep) * kstride + ((ragged && t == T - 1) ? lt_.kofs_last : lt_.kofs);
#pragma unroll
    for (int s = 0; s < 4; ++s) dst[s] = *reinterpret_cast<const h8*>(gb + 32 * s);
  };

  // ---- prologue, part 2: V(0) and K(2) copied into their slots, K(0) and
  // K(1) loaded into registers -- all in flight with the staging ----
  h8 kop[2][4];  // K operands, buffers 0 and 1
  if (active) {
    copy_v(lt, 0, ring_lds, vbase);           // V(0) into V slot 0
    copy_v(lt, 2, ring_lds + kKSlot, kbase);  // K(2) into the K slot
    load_k(lt, 0, kop[0]);
    load_k(lt, 1, kop[1]);
    // the staged rows have landed: every memory operation but the 16 issued
    // last (the two copies above, then the K loads: at least 8 instructions
    // of 16 bytes per lane)
    wait_vmcnt<16>();
  } else {
    wait_vmcnt<0>();
  }
  lds_barrier();  // the Q block and the rel rows are in LDS

  // Q^T as the MFMA B operand: lane (n, g) of block J holds query
  // q0 + 32 J + n, dims 16 s + 8 g + [0, 8) for k-step s.  Rows >= L are 0.
  h8 qop[kBlocks][4];
#pragma unroll
  for (int J = 0; J < kBlocks; ++J) {
    const int r = 32 * J + n;
    const char* qrow = smem + kQStageOff + r * 128;
#pragma unroll
    for (int s = 0; s < 4; ++s) qop[J][s] = *reinterpret_cast<const h8*>(qrow + (((2 * s + g) ^ tile_swz(r)) << 4));
    if (q0 + r >= p.L) {
#pragma unroll
      for (int s = 0; s < 4; ++s) qop[J][s] = h8{};
    }
  }

  // q.rel^T * scale for the 64 rows, as twenty (16 positions x 16 rows)
  // tiles rel . Q^T of v_mfma_f32_16x16x32_f16: wavefront w takes rows
  // 16 w + [0, 16) and all five position blocks (positions 0-79; rel rows
  // >= 73 are 0; positions 73-79 are not stored: the row's padding repeats
  // position 72 there, and position 0 before it) -- five independent
  // two-product chains per wavefront.  Lane l supplies position (A) and row
  // (B) l % 16, dims 32 t + 8 (l / 16) + [0, 8) of k-step t, and receives
  // positions 4 (l / 16) + [0, 4) of row l % 16.
  float* qr_tab = reinterpret_cast<float*>(smem + kQrOff);
  {
    const int c16 = lane & 15, kg = lane >> 4;
    const int qr = 16 * w + c16;
    h8 qb[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int c = 4 * t + kg;
      qb[t] = *reinterpret_cast<const h8*>(smem + kQStageOff + qr * 128 + ((c ^ tile_swz(qr)) << 4));
      if (q0 + qr >= p.L) qb[t] = h8{};
    }
    f32x4 acc[5];
#pragma unroll
    for (int pb = 0; pb < 5; ++pb) {
      const int pos = 16 * pb + c16;
      const int r2 = min(pos - 64, 15);
      acc[pb] = f32x4{};
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int c = 4 * t + kg;
        const char* src = pb < 4 ? smem + kRelOff + pos * 128 + ((c ^ tile_swz(pos)) << 4)
                                 : smem + kRel2Off + r2 * 128 + ((c ^ tile_swz(r2)) << 4);
        h8 e = *reinterpret_cast<const h8*>(src);
        if (pos >= kNumPos) e = h8{};
        acc[pb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(e, qb[t], acc[pb], 0, 0, 0);
      }
    }
    float* qrow = qr_tab + qr * kQrRow + kQrPad;  // position 0 of row qr
#pragma unroll
    for (int pb = 0; pb < 5; ++pb) {
      const int pos0 = 16 * pb + 4 * kg;
      if (pos0 + 3 < kNumPos - 1) {
        const f4 val = {acc[pb][0] * scale, acc[pb][1] * scale, acc[pb][2] * scale, acc[pb][3] * scale};
        *reinterpret_cast<f4*>(qrow + pos0) = val;
      } else if (pos0 == kNumPos - 1) {  // position 72 and the padding after it
        const float e = acc[pb][0] * scale;
        const f4 val = {e, e, e, e};
        *reinterpret_cast<f4*>(qrow + pos0) = val;
        *reinterpret_cast<f4*>(qrow + pos0 + 4) = val;
        qrow[pos0 + 8] = e;
      }
      if (pos0 == 0) {  // the padding before position 0
        const float e = acc[pb][0] * scale;
        const f4 val = {e, e, e, e};
        *reinterpret_cast<f4*>(qrow - 8) = val;
        *reinterpret_cast<f4*>(qrow - 4) = val;
      }
    }
  }

  f32x16 oacc[kBlocks][2];  // O^T: dims 32 db + 8 (i/4) + 4 g + i%4, query n
  float m_run[kBlocks];
  // Running row sums per block, accumulated on the matrix core (see rowsum
  // below): the four values of a lane are its query's sum.
  f32x4 lsum[kBlocks];
  // Every value bound to a register of the key-step loop is defined at its
  // entry, or the compiler may place other inputs in that register.
  f32x16 sacc[2] = {};   // S^T of the current and the next item
  h8 pk[2][2] = {};      // fp16 probabilities [buffer][16-key half]
  h8 vop[2][2];          // V^T operands [hh][db] of one step

  auto load_v = [&](const LaneTab& t, int sl) SIDON_INLINE {
    const char* vt = ring + (sl ? kVSlot1 : 0);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        const h4 lo = __builtin_bit_cast(
            h4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(SIDON_LDS_PTR(s4, vt + t.tr_off[0][db] + 2048 * hh)));
        const h4 hi = __builtin_bit_cast(
            h4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(SIDON_LDS_PTR(s4, vt + t.tr_off[1][db] + 2048 * hh)));
        vop[hh][db] = cat(lo, hi);
      }
    }
  };
  auto qk_with = [&](const h8 (&qo)[4], const h8 (&k)[4]) SIDON_INLINE {
    f32x16 acc = {};
#pragma unroll
    for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(k[s], qo[s], acc, 0, 0, 0);
    return acc;
  };
  auto qk = [&](int J, const h8 (&k)[4]) SIDON_INLINE { return qk_with(qop[J], k); };
  // Q^T operands of block J read again from global memory (the rerun: the
  // staged Q block in LDS is overwritten by then), with the same values as
  // qop: lane (n, g) holds query q0 + 32 J + n, dims 16 s + 8 g + [0, 8);
  // rows >= L are 0.
  auto load_q = [&](const LaneTab& t, int J, h8 (&dst)[4]) SIDON_INLINE {
    const int row = q0 + 32 * J + t.n;
    const _Float16* src = qbase + (int64_t)min(row, p.L - 1) * p.qsl + 8 * t.g;
#pragma unroll
    for (int s = 0; s < 4; ++s) dst[s] = row < p.L ? *reinterpret_cast<const h8*>(src + 16 * s) : h8{};
  };
  auto pv = [&](int J, int bf) SIDON_INLINE {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int db = 0; db < 2; ++db)
        oacc[J][db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vop[hh][db], pk[bf][hh], oacc[J][db], 0, 0, 0);
  };

  // Row sums on the matrix core with v_mfma_f32_16x16x32_f16: read as a
  // 16x16x32 B operand, the probability tile of lane l = c + 16 j (column
  // c = l % 16, k-group j = l / 16) holds query c + 16 (j % 2), keys 8 (j / 2)
  // + [0, 8) of the 16-key half.  The A operand "sel" of lane l (row l % 16,
  // k-group l / 16) is 1 where bit 4 of l equals bit 2 of l: output row i
  // then sums the k-groups of parity (i / 4) % 2, i.e. all 16 keys of query
  // c + 16 ((i / 4) % 2), and the four rows lane l receives (4 (l / 16) +
  // [0, 4)) are exactly its own query's sum.
  const _Float16 sel_v = (((lane >> 4) ^ (lane >> 2)) & 1) == 0 ? (_Float16)1 : (_Float16)0;
  h8 sel = {sel_v, sel_v, sel_v, sel_v, sel_v, sel_v, sel_v, sel_v};
  asm volatile("" : "+v"(sel));
  auto accumulate_with = [&](const h8& sl, int J, int bf) SIDON_INLINE {
    lsum[J] = __builtin_amdgcn_mfma_f32_16x16x32_f16(sl, pk[bf][0], lsum[J], 0, 0, 0);
    lsum[J] = __builtin_amdgcn_mfma_f32_16x16x32_f16(sl, pk[bf][1], lsum[J], 0, 0, 0);
  };
  auto accumulate = [&](int J, int bf) SIDON_INLINE {
    asm volatile("" : "+v"(sel));
    accumulate_with(sel, J, bf);
  };

  auto emit = [&](int bf, int i, const f2& e) SIDON_INLINE {
    const h2 ph = __builtin_convertvector(e, h2);
    pk[bf][i >> 3][i & 7] = ph[0];
    pk[bf][i >> 3][(i & 7) + 1] = ph[1];
  };
  // p = exp2(s * scale + nb), the lane's 16 keys.
  auto probs_fast = [&](int bf, float nb) SIDON_INLINE {
#pragma unroll
    for (int i = 0; i < 16; i += 2)
      emit(bf, i, f2{fast_exp2(fmaf(sacc[bf][i], scale, nb)), fast_exp2(fmaf(sacc[bf][i + 1], scale, nb))});
  };

  // Item (u, J) through the general code, from the scores in sacc[0]:
  // probabilities into pk[0] with the running max, then the exact max update
  // for the queries that need it (all at the first step, else those whose
  // step sum is not finite -- a probability past the fp16 range), decided
  // per query from its own sum, never per wavefront, so one row cannot
  // change the rounding of another.  A query that needs no update keeps its
  // max, and its probabilities are the ones the hand-scheduled loop forms.
  auto item = [&](const LaneTab& t, const float (&ql)[kBlocks], const float (&qrr)[kBlocks], int j, int u,
                  int J, int sb) SIDON_INLINE {
    const int n = t.n, g = t.g;
    int k0 = (w + kWaves * u) * kStep;
    asm volatile("" : "+s"(k0));
    const int qlo = q0 + 32 * J;
    const bool left = k0 + (kStep - 1) - qlo <= -kLeft;
    const bool right = k0 - (qlo + 31) >= kRight;
    const bool masked = k0 + kStep > LK;
    const bool band = !left && !right;
    const bool first = j == 0;
    const float off = left ? ql[J] : (right ? qrr[J] : 0.f);
    float y[16];
    if (band) {
      const float* qrow = qr_tab + (32 * J + n) * kQrRow + kQrPad;
      const int d0 = k0 + 8 * g - (qlo + n) + kLeft;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int idx = min(max(d0 + 16 * (i >> 3) + (i & 7), 0), kLeft + kRight);
        y[i] = fmaf(sacc[sb][i], scale, qrow[idx]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) y[i] = fmaf(sacc[sb][i], scale, off);
    }
    if (masked) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = k0 + 16 * (i >> 3) + 8 * g + (i & 7);
        if (key >= LK) y[i] = -INFINITY;
      }
    }
    auto probs = [&](float m) SIDON_INLINE {
      if (band || masked) {
#pragma unroll
        for (int i = 0; i < 16; i += 2) emit(sb, i, f2{fast_exp2(y[i] - m), fast_exp2(y[i + 1] - m)});
      } else {  // the plain form, bit for bit as the loop computes it
        probs_fast(sb, off - m);
      }
    };
    bool need = first;
    if (!first) {
      probs(m_run[J]);
      float own = 0.f;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int e = 0; e < 8; ++e) own += (float)pk[sb][hh][e];
      const auto pr = __builtin_amdgcn_permlane32_swap(__float_as_uint(own), __float_as_uint(own), false, false);
      need = !(__uint_as_float(pr[0]) + __uint_as_float(pr[1]) < INFINITY);
    }
    if (__builtin_amdgcn_ballot_w64(need) != 0) {
      float mx = y[0];
#pragma unroll
      for (int i = 1; i < 16; ++i) mx = fmaxf(mx, y[i]);
      mx = pair_max(mx);
      const float m_new = need ? fmaxf(m_run[J], mx) : m_run[J];
      const float alpha = fast_exp2(m_run[J] - m_new);  // 1 if unchanged, 0 from -inf
      if (!first && __builtin_amdgcn_ballot_w64(alpha != 1.f) != 0) {
        oacc[J][0] *= alpha;
        oacc[J][1] *= alpha;
      }
      lsum[J] *= alpha;
      m_run[J] = m_new;
      probs(m_new);
    }
  };

#pragma unroll
  for (int J = 0; J < kBlocks; ++J) {
    oacc[J][0] = f32x16{};
    oacc[J][1] = f32x16{};
    m_run[J] = -INFINITY;
    lsum[J] = f32x4{};
  }

  if (active) {
    // Entry state of the loop: S^T of item (0, 0) in sacc[0], K(0) and K(1)
    // in the two K buffers, K(2) in the K slot, V(0) in ring slot 0 and in
    // the V operands (finite operands for the zero probabilities of the
    // items before the first), probabilities and sums 0; no copy in flight.
    // (Formed before the barrier below, behind which the slowest
    // wavefront's part of the q.rel table lands.)
    wait_vmcnt<0>();
    load_v(lt, 0);
    sacc[0] = qk(0, kop[0]);
  }
  lds_barrier();  // the q.rel table is complete

  if (active) {
    // The first pass runs every step through the hand-scheduled loop of
    // flexrel_w64_step.inc; it checks no step sum: a probability past the
    // fp16 range becomes inf and makes its block's running sum non-finite
    // (inf, or NaN through the other query's zero weight in the row-sum
    // product).  Such a wavefront discards its partial results and runs all
    // its steps again through `item` above, one step at a time.
    for (bool safe = false;; safe = true) {
      if (safe) {
#pragma unroll
        for (int J = 0; J < kBlocks; ++J) {
          oacc[J][0] = f32x16{};
          oacc[J][1] = f32x16{};
          m_run[J] = -INFINITY;
          lsum[J] = f32x4{};
        }
        for (int j = 0; j < nu; ++j) {
          // every lane-dependent value formed again at every step (none
          // survives the hand-scheduled loop, and none is kept across the
          // steps here: with the accumulators, Q^T and the row state live,
          // keeping the lane offsets too spilled them to scratch, and a
          // scratch segment slows every launch, rerun or not)
          const LaneTab t1 = lane_tab(fresh_lane_id(), kstride, last_row);
          float ql[kBlocks], qrr[kBlocks];
#pragma unroll
          for (int J = 0; J < kBlocks; ++J) {
            ql[J] = qr_tab[(32 * J + t1.n) * kQrRow + kQrPad];
            qrr[J] = qr_tab[(32 * J + t1.n) * kQrRow + kQrPad + kNumPos - 1];
          }
          const int u = u_of(j);
          const int ln = t1.n + 32 * t1.g;
          const _Float16 sv = (((ln >> 4) ^ (ln >> 2)) & 1) == 0 ? (_Float16)1 : (_Float16)0;
          const h8 sel1 = {sv, sv, sv, sv, sv, sv, sv, sv};
          wait_lgkm0();  // the reads of the previous V tile are done
          copy_v(t1, j, ring_lds, vbase);
          wait_vmcnt<0>();
          load_v(t1, 0);
#pragma unroll
          for (int J = 0; J < kBlocks; ++J) {
            // the K and Q^T operands read for each block (only one block's
            // are live at a time)
            h8 ko[4], qo[4];
            load_k(t1, j, ko);
            load_q(t1, J, qo);
            sacc[0] = qk_with(qo, ko);
            // (every item, the plain ones too: their probabilities take the
            // loop's plain form, and a query past the fp16 range must not
            // reach the row-sum product, where its inf would turn the sum of
            // the other query of its lane group into NaN)
            item(t1, ql, qrr, j, u, J, 0);
            accumulate_with(sel1, J, 0);
            pv(J, 0);
          }
        }
        break;
      }
      // Loop state: j, the load bases (V of step j + 1, K of step j + 2) and
      // their advances for the plain steps (by 4 key steps, or across the
      // band at index jump), the scalars of the processing order, and the
      // per-lane LDS addresses of the V operand reads (slot 0) and of the
      // lane's q.rel row.
      int jreg = 0;
      const int jump = nS + cL;
      const int64_t dstep = (int64_t)(kWaves * kStep) * kstride;
      const int64_t djump = dstep * (1 + cR - cL);
      const char* gk = kbase;
      const char* gv = vbase;
      const uint64_t kb = (uint64_t)(uintptr_t)(kbase - 3072), vb = (uint64_t)(uintptr_t)(vbase - 3072);
      const uint32_t rowb = (uint32_t)(kStep * kstride);
      const int tlast = ragged ? T - 1 : -1;
      uint32_t ka[4], tv[2][2];
#pragma unroll
      for (int s = 0; s < 4; ++s)
        ka[s] = ring_lds + (uint32_t)(lt.kperm * 128 + (((2 * s + g) ^ tile_swz(lt.kperm)) << 4));
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int db = 0; db < 2; ++db) tv[hf][db] = ring_lds + (uint32_t)lt.tr_off[hf][db];
      const uint32_t qbase_lds = (uint32_t)(uintptr_t)SIDON_LDS_PTR(float, qr_tab + n * kQrRow + kQrPad);
      const int laned = 8 * g - n;
      const int g8 = 8 * g;
      // (The loop writes M0 for its LDS copies; the clobber says so.  The
      // compiler treats M0 as reserved and warns; no compiled code of these
      // kernels relies on M0 across the statement.)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
      asm volatile(SIDON_W64_LOOP
                   : "+{v[0:15]}"(oacc[0][0]), "+{v[16:31]}"(oacc[0][1]), "+{v[32:47]}"(oacc[1][0]),
                     "+{v[48:63]}"(oacc[1][1]), "+{v[64:79]}"(sacc[0]), "+{v[80:95]}"(sacc[1]),
                     "+{v[96:99]}"(pk[0][0]), "+{v[100:103]}"(pk[0][1]), "+{v[104:107]}"(pk[1][0]),
                     "+{v[108:111]}"(pk[1][1]), "+{v[112:115]}"(lsum[0]), "+{v[116:119]}"(lsum[1]),
                     "+{v[120:123]}"(sel), "+{v[152:155]}"(qop[0][0]), "+{v[156:159]}"(qop[0][1]),
                     "+{v[160:163]}"(qop[0][2]), "+{v[164:167]}"(qop[0][3]), "+{v[168:171]}"(qop[1][0]),
                     "+{v[172:175]}"(qop[1][1]), "+{v[176:179]}"(qop[1][2]), "+{v[180:183]}"(qop[1][3]),
                     "+{v[184:187]}"(kop[0][0]), "+{v[188:191]}"(kop[0][1]), "+{v[192:195]}"(kop[0][2]),
                     "+{v[196:199]}"(kop[0][3]), "+{v[200:203]}"(kop[1][0]), "+{v[204:207]}"(kop[1][1]),
                     "+{v[208:211]}"(kop[1][2]), "+{v[212:215]}"(kop[1][3]), "+{v[216:219]}"(vop[0][0]),
                     "+{v[220:223]}"(vop[0][1]), "+{v[224:227]}"(vop[1][0]), "+{v[228:231]}"(vop[1][1]),
                     "+{s64}"(jreg), "+{s[70:71]}"(gk),
                     "+{s[72:73]}"(gv), [m0] "+v"(m_run[0]), [m1] "+v"(m_run[1])
                   : "{s65}"(nu), "{s66}"(jump), "{s67}"(ring_lds), "{s68}"(scale), "{s[74:75]}"(dstep),
                     "{s[76:77]}"(djump), [nslow] "s"(nSlow), [w] "s"(w), [q0] "s"(q0), [lk] "s"(LK),
                     [tlast] "s"(tlast), [cl] "s"(cL), [nband] "s"(cR - cL), [ns] "s"(nS), [ue] "s"(uE),
                     [rowb] "s"(rowb), [kblo] "s"((uint32_t)kb), [kbhi] "s"((uint32_t)(kb >> 32)),
                     [vblo] "s"((uint32_t)vb), [vbhi] "s"((uint32_t)(vb >> 32)), [ko0] "v"(lt.voff[0]),
                     [ko1] "v"(lt.voff[1]), [ko2] "v"(lt.voff[2]), [ko3] "v"(lt.voff[3]), [kl0] "v"(lt.voff_last[0]),
                     [kl1] "v"(lt.voff_last[1]), [kl2] "v"(lt.voff_last[2]), [kl3] "v"(lt.voff_last[3]),
                     [ka0] "v"(ka[0]), [ka1] "v"(ka[1]), [ka2] "v"(ka[2]), [ka3] "v"(ka[3]), [tv00] "v"(tv[0][0]), [tv01] "v"(tv[0][1]),
                     [tv10] "v"(tv[1][0]), [tv11] "v"(tv[1][1]), [qbase] "v"(qbase_lds), [laned] "v"(laned),
                     [g8] "v"(g8)
                   : SIDON_W64_VGPR_CLOBBERS, SIDON_W64_SGPR_CLOBBERS, "vcc", "m0", "scc", "memory");
#pragma clang diagnostic pop
      uint64_t overflow = 0;
#pragma unroll
      for (int J = 0; J < kBlocks; ++J) overflow |= __builtin_amdgcn_ballot_w64(!(lsum[J][0] < INFINITY));
      // (The statement returns with every LDS read and copy retired, so its
      // register outputs -- the V^T operands read below among them -- are
      // final: a wait placed here in compiled code would not order the
      // register-only products after it.)
      if (__builtin_expect(overflow != 0 || p.rerun_all != 0, 0)) continue;
      pv(0, 0);  // PV of items (nu - 1, 0) and (nu - 1, 1)
      pv(1, 1);
      break;
    }
  }
  wait_vmcnt<0>();  // the last (unused) prefetches have landed before LDS is reused

  // ---- merge the key splits ----
  lds_barrier();  // every wavefront is done with its ring and the q.rel table
  const int lane1 = fresh_lane_id();
  const int n1 = lane1 & 31, g1 = lane1 >> 5;
  float* mo = reinterpret_cast<float*>(smem);
  float* ml = reinterpret_cast<float*>(smem + kMergeMlOff);
#pragma unroll
  for (int J = 0; J < kBlocks; ++J) {
    float* dst = mo + (w * kRows + 32 * J + n1) * kMergeStride;
#pragma unroll
    for (int db = 0; db < 2; ++db) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f4 val = {oacc[J][db][4 * j], oacc[J][db][4 * j + 1], oacc[J][db][4 * j + 2], oacc[J][db][4 * j + 3]};
        *reinterpret_cast<f4*>(dst + 32 * db + 8 * j + 4 * g1) = val;
      }
    }
    if (g1 == 0) {
      ml[(w * kRows + 32 * J + n1) * 2] = m_run[J];
      ml[(w * kRows + 32 * J + n1) * 2 + 1] = lsum[J][0];
    }
  }
  lds_barrier();

  // Wavefront w finalises rows 16 w + [0, 16), four lanes per row, 16 dims
  // per lane.
  const int r = 16 * w + (lane1 >> 2);
  const int c = 16 * (lane1 & 3);
  float mmax = -INFINITY;
#pragma unroll
  for (int s = 0; s < kWaves; ++s) mmax = fmaxf(mmax, ml[(s * kRows + r) * 2]);
  float total = 0.f;
  f4 o[4] = {};
#pragma unroll
  for (int s = 0; s < kWaves; ++s) {
    const float ms = ml[(s * kRows + r) * 2];
    const float f = ms == -INFINITY ? 0.f : fast_exp2(ms - mmax);
    total += ml[(s * kRows + r) * 2 + 1] * f;
    const float* src = mo + (s * kRows + r) * kMergeStride + c;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] += *reinterpret_cast<const f4*>(src + 4 * j) * f;
  }
  const int row = q0 + r;
  if (row < p.L) {
    const float inv = total > 0.f ? __builtin_amdgcn_rcpf(total) : 0.f;
    _Float16* dst = p.out + b * p.osb + h * p.osh + (int64_t)row * p.osl + c;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const h8 v = {(_Float16)(o[2 * j][0] * inv), (_Float16)(o[2 * j][1] * inv), (_Float16)(o[2 * j][2] * inv),
                    (_Float16)(o[2 * j][3] * inv), (_Float16)(o[2 * j + 1][0] * inv),
                    (_Float16)(o[2 * j + 1][1] * inv), (_Float16)(o[2 * j + 1][2] * inv),
                    (_Float16)(o[2 * j + 1][3] * inv)};
      *reinterpret_cast<h8*>(dst + 8 * j) = v;
    }
  }
}

}  // namespace

int w64_rows() { return kRows; }
int w64_threads() { return kThreads; }

// Only K and V rows of the same stride (the fused QKV layout, and any
// [B, H, L, 64] views that share a row stride).
hipError_t launch_w64(const Params& p, int nwg, bool same_stride, hipStream_t stream) {
  if (!same_stride) return hipErrorInvalidValue;
  hipLaunchKernelGGL(flexrel_w64_kernel, dim3(nwg), dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace sidon_flexrel
