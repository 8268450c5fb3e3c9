// flexrel_wide.hip -- relative_key flash attention, 128 query rows per
// wavefront (MI355X / gfx950).  Same math and results contract as
// flexrel_fwd.hip (src/sidon_triton/triton_encoder.py:210-312):
//
//   s_ij = (q_i . k_j + q_i . rel[clamp(j - i, -64, 8) + 64]) / sqrt(64)
//   o_i  = sum_{j < LK_b} softmax_j(s_ij) v_j
//
// Work decomposition.  One workgroup owns 128 query rows of one (b, h) and
// has 4 wavefronts, one per SIMD; wavefront w runs an online softmax for all
// 128 rows over the key steps w, w + 4, w + 8, ... (32 keys each) and the
// four partial results are merged through LDS at the end.  Against the
// 64-row kernel (two wavefronts per SIMD, 8 key splits) every K/V tile copy
// and every LDS operand read serves twice the query rows, the first-step
// exact max update and the merge are amortised over twice the keys, and
// the wavefront has four column blocks of independent work to interleave
// on its matrix core and vector ALU.
//
// Per wavefront and step (32 keys): for each 32-query column block J the
// score tile S^T = K . Q^T (4 v_mfma_f32_32x32x16_f16, Q^T in registers),
// the exp2 softmax with the lazily updated running max of flexrel_fwd.hip,
// the step's row sums on the matrix core (2 v_mfma_f32_16x16x32_f16, see
// rowsum below) and O^T += V^T . P^T (4 MFMAs, accumulators in AGPRs).
// The items (step u, block J) form one software pipeline: phase (u, J)
// issues the PV product of item i - 2, the softmax of item i, the deferred
// check of item i - 1 and the score product of item i + 1, so every
// dependency crosses a phase boundary and the matrix core always has
// independent products beside the softmax.
//
// Registers (one wavefront per SIMD: 512 per lane): O^T accumulators 128
// VGPRs, two score tiles 32, two probability tiles 16; the MFMA source
// operands that only the matrix core reads -- Q^T (64), the K and V
// operands of a step (32) -- are allocated to AGPRs, which the MFMAs read
// directly.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include <type_traits>

#include "flexrel_device.h"
#include "flexrel_wide_step.inc"

#define SIDON_INLINE __attribute__((always_inline))

namespace sidon_flexrel {
namespace {

constexpr int kRows = 128;     // query rows per workgroup = per wavefront
constexpr int kBlocks = 4;     // 32-query column blocks per wavefront
constexpr int kWaves = 4;      // key splits, one wavefront per SIMD
constexpr int kThreads = 64 * kWaves;
constexpr int kWaveRing = 4 * kTile;  // K slots 0, 1 then V slots 0, 1
constexpr int kQrOff = kWaves * kWaveRing;
constexpr int kQStageOff = kQrOff + kRows * kQrStride * 4;  // Q block, 128 rows x 128 B
constexpr int kRelOff = kQStageOff + kRows * kD * 2;        // rel rows, 3 tiles of 32
constexpr int kPreBytes = kRelOff + 3 * kTile;
constexpr int kMergeStride = 68;                            // fp32 per partial-output row
constexpr int kMergeMlOff = kWaves * kRows * kMergeStride * 4;
constexpr int kMergeBytes = kMergeMlOff + kWaves * kRows * 2 * 4;
constexpr int kLdsBytes = kPreBytes > kMergeBytes ? kPreBytes : kMergeBytes;
static_assert(kLdsBytes <= 160 * 1024, "LDS budget of one CU");

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <bool kSameStride>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
flexrel_wide_kernel(const Params p) {
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
  // w + 4 u, u = 0 .. nu - 1.
  const int T = (LK + kStep - 1) / kStep;
  const int nu = T > w ? (T - w + kWaves - 1) / kWaves : 0;
  const bool active = nu > 0;

  // Step classes per block J (32 rows at q0 + 32 J): steps u <= uL[J] are
  // entirely left of the window (j - i <= -64), u >= uR[J] entirely right
  // (j - i >= 8); uM is the first step that straddles LK (at most one: the
  // wavefront's last).  (Arithmetic shifts: floor and ceiling divisions by
  // 128 = 4 steps of 32.)  uL grows and uR grows with J.
  int uL[kBlocks], uR[kBlocks];
#pragma unroll
  for (int J = 0; J < kBlocks; ++J) {
    uL[J] = (q0 + 32 * J - 95 - kStep * w) >> 7;
    uR[J] = -((-(q0 + 32 * J + 39 - kStep * w)) >> 7);
  }
  const int uM = ((LK - kStep - kStep * w) >> 7) + 1;
  // Processing order.  The online softmax (lazy max, per-query exact
  // updates) does not depend on the order of the steps, so a wavefront runs
  // its special steps first -- the band steps [cL, cR) where some block
  // needs the per-score bias gather, then the straddling step -- through the
  // general code, and then its plain steps (every block entirely left,
  // u < cL, or entirely right, u in [cR, uE)) through a loop with no
  // rare-path branch beyond the overflow check.  The first processed step
  // sets the running max exactly; a wavefront with no special step runs its
  // first plain step through the general code for that.
  const int uE = min(uM, nu);            // steps [uE, nu) straddle LK
  const int cL = min(max(uL[0] + 1, 0), uE);
  const int cR = min(max(uR[kBlocks - 1], cL), uE);
  const int nS = (cR - cL) + (nu - uE);  // special steps
  const int nSlow = nu > 0 ? max(nS, 1) : 0;
  // Local step of processing index j (j < nu); plain_u for indices >= nS
  // (branch-free: the plain steps are [0, cL) then [cR, uE)).
  auto plain_u = [&](int j) SIDON_INLINE {
    const int k = j - nS;
    return k + (k >= cL ? cR - cL : 0);
  };
  auto u_of = [&](int j) SIDON_INLINE {
    if (j < cR - cL) return cL + j;
    if (j < nS) return uE;
    return plain_u(j);
  };

  char* ring = smem + w * kWaveRing;
  const uint32_t ring_lds = (uint32_t)(uintptr_t)SIDON_LDS_PTR(char, ring);
  constexpr uint32_t kVRing = 2 * kTile;

  // Tile copy lane offsets (LDS chunk position 64 i + lane = row 8 i +
  // lane / 8, swizzled chunk lane % 8), from base - 3072; the last step T - 1
  // re-reads row LK - 1 for its rows past LK (their scores are masked).
  uint32_t koff[4], voff_own[4], koff_last[4], voff_last_own[4];
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
  const bool ragged = LK % kStep != 0;  // step T - 1 straddles LK
  // Copy of the step at processing index j into an LDS slot; prefetches past
  // the last index re-read the last processed step, so every copy stays in
  // bounds.  kPlain: the step is known not to straddle LK (no select).
  auto copy_step = [&](const char* base, int64_t stride, const uint32_t (&off)[4], const uint32_t (&off_last)[4],
                       int j, uint32_t slot, auto plain_tag) SIDON_INLINE {
    constexpr bool kPlain = decltype(plain_tag)::value;
    const int jc = min(j, nu - 1);
    const int t = w + kWaves * (kPlain ? plain_u(jc) : u_of(jc));
    const char* gb = base + (int64_t)(t * kStep) * stride - 3072;
    if (kPlain) {
      dma_tile(slot, gb, off[0], off[1], off[2], off[3]);
    } else {
      // (selected by value: a select between the two arrays would become a
      // pointer select through scratch memory)
      const bool last = ragged && t == T - 1;
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t a = off[i], b = off_last[i];
        o[i] = last ? b : a;
      }
      dma_tile(slot, gb, o[0], o[1], o[2], o[3]);
    }
  };

  // ---- prologue: Q rows, rel rows and the first K/V tiles, all in flight ----
  const uint32_t q_lds = (uint32_t)(uintptr_t)SIDON_LDS_PTR(char, smem + kQStageOff);
  {
    // wavefront w: Q rows 32 w + [0, 32) (rows >= L clamped, zeroed below)
    uint32_t qoff[4];
    const int row0 = min(q0 + 32 * w, p.L - 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 32 * w + 8 * i + (lane >> 3);
      qoff[i] = (uint32_t)((min(q0 + r, p.L - 1) - row0) * p.qsl * 2) + 16u * ((lane & 7) ^ tile_swz(r)) + 3072u -
                1024u * i;
    }
    dma_tile(q_lds + 4096u * w, reinterpret_cast<const char*>(qbase + (int64_t)row0 * p.qsl) - 3072, qoff[0],
             qoff[1], qoff[2], qoff[3]);
  }
  if (w < 3) {
    // rel rows 32 w + [0, 32) (rows >= 73 clamped, zeroed below)
    uint32_t roff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 8 * i + (lane >> 3);
      roff[i] = (uint32_t)(min(32 * w + r, kNumPos - 1) * kD * 2) + 16u * ((lane & 7) ^ tile_swz(r)) + 3072u -
                1024u * i;
    }
    dma_tile((uint32_t)(uintptr_t)SIDON_LDS_PTR(char, smem + kRelOff) + kTile * w,
             reinterpret_cast<const char*>(p.rel) - 3072, roff[0], roff[1], roff[2], roff[3]);
  }
  if (active) {
    // K(0), V(0), K(1), V(1) (processing order): the order of the copies in the loop
    copy_step(kbase, kstride, koff, koff_last, 0, ring_lds, std::false_type{});
    copy_step(vbase, vstride, voff, voff_last, 0, ring_lds + kVRing, std::false_type{});
    copy_step(kbase, kstride, koff, koff_last, 1, ring_lds + kTile, std::false_type{});
    copy_step(vbase, vstride, voff, voff_last, 1, ring_lds + kVRing + kTile, std::false_type{});
    wait_vmcnt<16>();  // Q and rel rows landed (the four K/V tiles may still fly)
  } else {
    wait_vmcnt<0>();
  }
  lds_barrier();  // the whole Q block and the rel rows are in LDS

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

  // q.rel^T * scale for the 128 rows: wavefront w computes query block w for
  // the three 32-position blocks pb as rel . Q^T (Q^T of block w read from
  // the staging area); rel rows >= 73 are 0.
  float* qr_tab = reinterpret_cast<float*>(smem + kQrOff);
  {
    const int r = 32 * w + n;
    const char* qrow = smem + kQStageOff + r * 128;
    h8 qw[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) qw[s] = *reinterpret_cast<const h8*>(qrow + (((2 * s + g) ^ tile_swz(r)) << 4));
    if (q0 + r >= p.L) {
#pragma unroll
      for (int s = 0; s < 4; ++s) qw[s] = h8{};
    }
#pragma unroll
    for (int pb = 0; pb < 3; ++pb) {
      const int pos = 32 * pb + n;
      const char* rrow = smem + kRelOff + pb * kTile + n * 128;
      f32x16 acc = {};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        h8 e = *reinterpret_cast<const h8*>(rrow + (((2 * s + g) ^ tile_swz(n)) << 4));
        if (pos >= kNumPos) e = h8{};
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(e, qw[s], acc, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int pos0 = 32 * pb + 8 * i + 4 * g;
        if (pos0 < kQrStride) {
          const f4 val = {acc[4 * i] * scale, acc[4 * i + 1] * scale, acc[4 * i + 2] * scale,
                          acc[4 * i + 3] * scale};
          *reinterpret_cast<f4*>(qr_tab + r * kQrStride + pos0) = val;
        }
      }
    }
  }
  lds_barrier();  // the q.rel table is complete

  float qr_l[kBlocks], qr_r[kBlocks];
#pragma unroll
  for (int J = 0; J < kBlocks; ++J) {
    qr_l[J] = qr_tab[(32 * J + n) * kQrStride];                // j - i <= -64
    qr_r[J] = qr_tab[(32 * J + n) * kQrStride + kNumPos - 1];  // j - i >= 8
  }

  f32x16 oacc[kBlocks][2];  // O^T: dims 32 db + 8 (i/4) + 4 g + i%4, query n (AGPRs)
#pragma unroll
  for (int J = 0; J < kBlocks; ++J) {
    oacc[J][0] = f32x16{};
    oacc[J][1] = f32x16{};
  }
  float m_run[kBlocks];
  // Running row sums per block, accumulated on the matrix core (see rowsum
  // below): the four values of a lane are its query's sum.
  f32x4 lsum[kBlocks];
#pragma unroll
  for (int J = 0; J < kBlocks; ++J) {
    m_run[J] = -INFINITY;
    lsum[J] = f32x4{};
  }
  // S^T of items i (buffer i & 1) and i + 1.  Zeroed: every value bound to
  // a register of the key-step loop must be defined at its entry, or the
  // compiler may place other inputs in that register.
  f32x16 sacc[2] = {};
  h8 pk[2][2] = {};      // fp16 probabilities [buffer][16-key half]
  h8 kop[4];             // K operands (16 dims per k-step) of one step
  h8 vop[2][2];          // V^T operands [hh][db] of one step
  f32x4 rs = {};         // row sums of the latest item

  // K operands: lane (m, g) holds key row perm(m) of the tile, dims
  // 16 s + 8 g + [0, 8); the swizzled addresses of both slots, formed once.
  const int kperm = mfma_row_perm(n);
  const char* krow0 = ring + kperm * 128;
  const int kswz = tile_swz(kperm);
  const char* kaddr[2][4];
#pragma unroll
  for (int sl = 0; sl < 2; ++sl)
#pragma unroll
    for (int s = 0; s < 4; ++s) kaddr[sl][s] = krow0 + sl * kTile + (((2 * s + g) ^ kswz) << 4);
  auto load_k = [&](int sl) SIDON_INLINE {
#pragma unroll
    for (int s = 0; s < 4; ++s) kop[s] = *reinterpret_cast<const h8*>(sl ? kaddr[1][s] : kaddr[0][s]);
  };
  // V^T operands via transpose reads (ds_read_b64_tr_b16): group G of 16
  // lanes, source lane (a, bq) reads V[key0 + a][d0 + 4 bq .. +4) with key0 =
  // 16 hh + 8 (G / 2) + 4 hf and d0 = 32 db + 16 (G % 2).
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
  auto load_v = [&](int sl) SIDON_INLINE {
    const char* vt = ring + kVRing + (sl ? kTile : 0);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        const h4 lo = __builtin_bit_cast(
            h4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(SIDON_LDS_PTR(s4, vt + tr_off[0][db] + 2048 * hh)));
        const h4 hi = __builtin_bit_cast(
            h4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(SIDON_LDS_PTR(s4, vt + tr_off[1][db] + 2048 * hh)));
        vop[hh][db] = cat(lo, hi);
      }
    }
  };
  // S^T of block J into score buffer bf (4 MFMAs); O^T of block J += V^T . P^T
  // with the probabilities of buffer bf (4 MFMAs).
  auto qk = [&](int J, int bf) SIDON_INLINE {
    f32x16 acc = {};
#pragma unroll
    for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kop[s], qop[J][s], acc, 0, 0, 0);
    sacc[bf] = acc;
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
  // [0, 4)) are exactly its own query's sum.  Half the matrix-core time of a
  // 32x32x16 row sum, with the same fp32 sums of the fp16-rounded values the
  // PV product uses.
  const _Float16 sel_v = (((lane >> 4) ^ (lane >> 2)) & 1) == 0 ? (_Float16)1 : (_Float16)0;
  h8 sel = {sel_v, sel_v, sel_v, sel_v, sel_v, sel_v, sel_v, sel_v};
  asm volatile("" : "+v"(sel));
  auto rowsum = [&](int bf) SIDON_INLINE {
    asm volatile("" : "+v"(sel));
    rs = __builtin_amdgcn_mfma_f32_16x16x32_f16(sel, pk[bf][0], f32x4{}, 0, 0, 0);
    rs = __builtin_amdgcn_mfma_f32_16x16x32_f16(sel, pk[bf][1], rs, 0, 0, 0);
  };
  // The same row sums added to block J's running sums (the hand-scheduled
  // plain step issues exactly these two products per item).
  auto accumulate = [&](int J, int bf) SIDON_INLINE {
    asm volatile("" : "+v"(sel));
    lsum[J] = __builtin_amdgcn_mfma_f32_16x16x32_f16(sel, pk[bf][0], lsum[J], 0, 0, 0);
    lsum[J] = __builtin_amdgcn_mfma_f32_16x16x32_f16(sel, pk[bf][1], lsum[J], 0, 0, 0);
  };

  auto emit = [&](int bf, int i, const f2& e) SIDON_INLINE {
    const h2 ph = __builtin_convertvector(e, h2);
    pk[bf][i >> 3][i & 7] = ph[0];
    pk[bf][i >> 3][(i & 7) + 1] = ph[1];
  };
  // p = exp2(s * scale + nb), keys [8 part, 8 part + 8) of the lane's 16.
  auto probs_fast = [&](int bf, float nb, int part) SIDON_INLINE {
#pragma unroll
    for (int i = 8 * part; i < 8 * part + 8; i += 2)
      emit(bf, i, f2{fast_exp2(fmaf(sacc[bf][i], scale, nb)), fast_exp2(fmaf(sacc[bf][i + 1], scale, nb))});
  };
  auto probs_y = [&](int bf, const float (&y)[16], float m) {
#pragma unroll
    for (int i = 0; i < 16; i += 2) emit(bf, i, f2{fast_exp2(y[i] - m), fast_exp2(y[i + 1] - m)});
  };


  // Probabilities of item (u, J) in buffer bf for the general cases (band
  // gather, masked keys) and the exact max update, from the scores still in
  // sacc[bf].
  auto general = [&](int u, int J, int bf, bool first, bool need_sum) SIDON_INLINE {
    // Everything below depends on k0 through this fence, so none of it is
    // speculated into the common path (the masks and gathers cost more than
    // the plain step itself).
    int k0 = (w + kWaves * u) * kStep;
    asm volatile("" : "+s"(k0));
    const int qlo = q0 + 32 * J;
    const bool left = k0 + (kStep - 1) - qlo <= -kLeft;
    const bool right = k0 - (qlo + 31) >= kRight;
    const bool masked = k0 + kStep > LK;
    const bool band = !left && !right;
    const float off = left ? qr_l[J] : (right ? qr_r[J] : 0.f);
    auto biased = [&](float (&y)[16]) {
      if (band) {
        const float* qrow = qr_tab + (32 * J + n) * kQrStride;
        const int d0 = k0 + 8 * g - (qlo + n) + kLeft;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int idx = min(max(d0 + 16 * (i >> 3) + (i & 7), 0), kLeft + kRight);
          y[i] = fmaf(sacc[bf][i], scale, qrow[idx]);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) y[i] = fmaf(sacc[bf][i], scale, off);
      }
      if (masked) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = k0 + 16 * (i >> 3) + 8 * g + (i & 7);
          if (key >= LK) y[i] = -INFINITY;
        }
      }
    };
    // Every call needs the biased scores (the max, or the band / mask
    // probabilities), so they are formed once.
    float y[16];
    biased(y);
    auto probs = [&](float m) SIDON_INLINE {
      if (band || masked) {
        probs_y(bf, y, m);
      } else {  // the plain form, bit for bit as the common path computes it
        probs_fast(bf, off - m, 0);
        probs_fast(bf, off - m, 1);
      }
    };
    // Recompute with the running max; then raise the max of the queries that
    // need it: all at the first step (the max is -inf), else those with a
    // probability past the fp16 range (inf, so a non-finite step sum; every
    // finite fp16 probability is safe: the sums and products are fp32).  Per
    // query, never per wavefront, so one row cannot change the rounding of
    // another -- and the sum that decides is the query's own: the
    // matrix-core row sum also multiplies the other query of the lane group
    // by 0, and 0 * inf = NaN, so an overflowing neighbour (a garbage padded
    // row, say) would read as an overflow there.
    if (!first) probs(m_run[J]);
    if (first || need_sum) {
      bool need = first;
      if (!first) {
        float own = 0.f;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int e = 0; e < 8; ++e) own += (float)pk[bf][hh][e];
        const auto pr = __builtin_amdgcn_permlane32_swap(__float_as_uint(own), __float_as_uint(own), false, false);
        need = !(__uint_as_float(pr[0]) + __uint_as_float(pr[1]) < INFINITY);
      }
      float mx = y[0];
#pragma unroll
      for (int i = 1; i < 16; ++i) mx = fmaxf(mx, y[i]);
      mx = pair_max(mx);
      const float m_new = need ? fmaxf(m_run[J], mx) : m_run[J];
      const float alpha = fast_exp2(m_run[J] - m_new);  // 1 if unchanged, 0 from -inf
      // (At the first step nothing has been accumulated for the block yet.)
      if (!first && __builtin_amdgcn_ballot_w64(alpha != 1.f) != 0) {
        oacc[J][0] *= alpha;
        oacc[J][1] *= alpha;
      }
      lsum[J] *= alpha;
      m_run[J] = m_new;
      probs(m_new);
    }
    rowsum(bf);
  };
  // Deferred check of item (u, J) (buffer bf; its row sums were issued one
  // phase ago, its probabilities are consumed by the next PV product): a
  // non-finite step sum sends the block through the max update (which
  // decides per query from the query's own sum and leaves every probability
  // finite).  Then the item's row sums join the running sums.
  auto settle = [&](int u, int J, int bf) SIDON_INLINE {
    asm volatile("" : "+v"(rs));
    if (__builtin_expect(__builtin_amdgcn_ballot_w64(!(rs[0] < INFINITY)) != 0, 0)) general(u, J, bf, false, true);
    accumulate(J, bf);
  };

  if (active) {
    wait_vmcnt<8>();  // K(0), V(0)
    load_k(0);
    load_v(0);        // finite operands for the zero probabilities of items -2 and -1
    qk(0, 0);         // S^T of item (0, 0)
    // One step through the general code (index j, local step u = u_of(j),
    // 32 keys): every item whose block is not plain (band, straddling LK, or
    // the wavefront's first step) takes the general form.
    auto step = [&](int j) SIDON_INLINE {
      const int u = u_of(j);
      const int u_prev = u_of(max(j - 1, 0));  // (j = 0: item i - 1 does not exist and rs is 0)
      const int sl = j & 1;  // ring slot of this step's K and V
      // Phase J: item i = 4 j + J in buffer J & 1.
#pragma unroll
      for (int J = 0; J < kBlocks; ++J) {
        const int bf = J & 1;
        const int Jm2 = (J + 2) & 3, Jm1 = (J + 3) & 3, Jp1 = (J + 1) & 3;
        const bool is_left = u <= uL[J];
        const bool plain = j > 0 && (is_left || u >= uR[J]) && u < uM;
        const float nb = (is_left ? qr_l[J] : qr_r[J]) - m_run[J];
        if (J == 1) wait_vmcnt<12>();  // V(j) landed
        if (J == 2) wait_vmcnt<8>();   // K(j + 1) landed
        pv(Jm2, bf);  // item i - 2 (its buffer is this item's)
        probs_fast(bf, nb, 0);
        asm volatile("" : "+v"(pk[bf][0]));
        settle(J == 0 ? u_prev : u, Jm1, bf ^ 1);  // item i - 1 (J == 0: the previous step's block 3)
        qk(Jp1, bf ^ 1);      // item i + 1 (J == 3: the next step's block 0, K operands loaded in phase 2)
        if (J == 0) {
          wait_lgkm0();  // the K(j) operand reads are done: refill slot sl with K(j + 2)
          copy_step(kbase, kstride, koff, koff_last, j + 2, ring_lds + sl * kTile, std::false_type{});
        }
        if (J == 2) {
          wait_lgkm0();  // the V(j) operand reads are done: refill slot sl with V(j + 2)
          copy_step(vbase, vstride, voff, voff_last, j + 2, ring_lds + kVRing + sl * kTile, std::false_type{});
        }
        if (J == 1) load_v(sl);      // V operands of step j (after the PV of item (j - 1, 3))
        if (J == 2) load_k(sl ^ 1);  // K operands of step j + 1 (after the QK of item (j, 3))
        probs_fast(bf, nb, 1);
        rowsum(bf);
        asm volatile("" : "+v"(pk[bf][0]), "+v"(pk[bf][1]));
        if (__builtin_expect(!plain, 0)) general(u, J, bf, j == 0, false);
      }
    };

    // The first pass runs every step through the hand-scheduled loop of
    // flexrel_wide_step.inc: the special steps (band, straddling LK, the
    // first) with exactly the general code's arithmetic per item, then the
    // plain steps ordered for one wavefront per SIMD -- which issues a vector
    // instruction about every 5.4 cycles (v_exp_f32: 9.1) while a 32x32x16
    // product holds the matrix core for 32, so the two must run side by
    // side.  It checks no step sum: a probability past the fp16 range becomes
    // inf and makes its block's running sum non-finite (inf, or NaN through
    // the other query's zero weight).  Such a wavefront discards its partial
    // results and runs all its steps again through the C++ general code,
    // which raises the running max exactly where needed and computes the
    // same values as the first pass for every query whose probabilities stay
    // finite.
    for (bool safe = false;; safe = true) {
      if (safe) {
        wait_vmcnt<0>();  // the last prefetches have landed
        wait_lgkm0();
        copy_step(kbase, kstride, koff, koff_last, 0, ring_lds, std::false_type{});
        copy_step(vbase, vstride, voff, voff_last, 0, ring_lds + kVRing, std::false_type{});
        copy_step(kbase, kstride, koff, koff_last, 1, ring_lds + kTile, std::false_type{});
        copy_step(vbase, vstride, voff, voff_last, 1, ring_lds + kVRing + kTile, std::false_type{});
#pragma unroll
        for (int J = 0; J < kBlocks; ++J) {
          oacc[J][0] = f32x16{};
          oacc[J][1] = f32x16{};
          m_run[J] = -INFINITY;
          lsum[J] = f32x4{};
        }
        pk[0][0] = pk[0][1] = pk[1][0] = pk[1][1] = h8{};
        rs = f32x4{};
        wait_vmcnt<8>();  // K(0), V(0)
        load_k(0);
        load_v(0);
        qk(0, 0);
        for (int j = 0; j < nu; ++j) step(j);
        settle(u_of(nu - 1), 3, 1);
        break;
      }
      // Loop state: j, the copy bases and their advances for the plain
      // steps (by 4 key steps, or across the band at index jump), the
      // scalars of the processing order, and the per-lane LDS addresses of
      // the operand reads (slot 0) and of the lane's q.rel row.
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
      for (int s = 0; s < 4; ++s) ka[s] = (uint32_t)(uintptr_t)SIDON_LDS_PTR(char, kaddr[0][s]);
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int db = 0; db < 2; ++db) tv[hf][db] = ring_lds + (uint32_t)tr_off[hf][db];
      const uint32_t qbase = (uint32_t)(uintptr_t)SIDON_LDS_PTR(float, qr_tab + n * kQrStride);
      const int laned = 8 * g - n;
      const int g8 = 8 * g;
      // (The loop writes M0 for its LDS copies; the clobber says so.  The
      // compiler treats M0 as reserved and warns; no compiled code of these
      // kernels relies on M0 across the statement.)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
      asm volatile(SIDON_WIDE_LOOP
                   : "+{v[0:15]}"(oacc[0][0]), "+{v[16:31]}"(oacc[0][1]), "+{v[32:47]}"(oacc[1][0]),
                     "+{v[48:63]}"(oacc[1][1]), "+{v[64:79]}"(oacc[2][0]), "+{v[80:95]}"(oacc[2][1]),
                     "+{v[96:111]}"(oacc[3][0]), "+{v[112:127]}"(oacc[3][1]), "+{v[128:143]}"(sacc[0]),
                     "+{v[144:159]}"(sacc[1]), "+{v[160:163]}"(pk[0][0]), "+{v[164:167]}"(pk[0][1]),
                     "+{v[168:171]}"(pk[1][0]), "+{v[172:175]}"(pk[1][1]), "+{v[176:179]}"(lsum[0]),
                     "+{v[180:183]}"(lsum[1]), "+{v[184:187]}"(lsum[2]), "+{v[188:191]}"(lsum[3]),
                     "+{v[192:195]}"(sel), "+{a[0:3]}"(qop[0][0]), "+{a[4:7]}"(qop[0][1]), "+{a[8:11]}"(qop[0][2]),
                     "+{a[12:15]}"(qop[0][3]), "+{a[16:19]}"(qop[1][0]), "+{a[20:23]}"(qop[1][1]),
                     "+{a[24:27]}"(qop[1][2]), "+{a[28:31]}"(qop[1][3]), "+{a[32:35]}"(qop[2][0]),
                     "+{a[36:39]}"(qop[2][1]), "+{a[40:43]}"(qop[2][2]), "+{a[44:47]}"(qop[2][3]),
                     "+{a[48:51]}"(qop[3][0]), "+{a[52:55]}"(qop[3][1]), "+{a[56:59]}"(qop[3][2]),
                     "+{a[60:63]}"(qop[3][3]), "+{a[64:67]}"(kop[0]), "+{a[68:71]}"(kop[1]), "+{a[72:75]}"(kop[2]),
                     "+{a[76:79]}"(kop[3]), "+{a[80:83]}"(vop[0][0]), "+{a[84:87]}"(vop[0][1]),
                     "+{a[88:91]}"(vop[1][0]), "+{a[92:95]}"(vop[1][1]), "+{s64}"(jreg), "+{s[70:71]}"(gk),
                     "+{s[72:73]}"(gv), [m0] "+v"(m_run[0]), [m1] "+v"(m_run[1]), [m2] "+v"(m_run[2]),
                     [m3] "+v"(m_run[3])
                   : "{s65}"(nu), "{s66}"(jump), "{s67}"(ring_lds), "{s68}"(scale), "{s[74:75]}"(dstep),
                     "{s[76:77]}"(djump), [nslow] "s"(nSlow), [w] "s"(w), [q0] "s"(q0), [lk] "s"(LK),
                     [tlast] "s"(tlast), [cl] "s"(cL), [nband] "s"(cR - cL), [ns] "s"(nS), [ue] "s"(uE),
                     [rowb] "s"(rowb), [kblo] "s"((uint32_t)kb), [kbhi] "s"((uint32_t)(kb >> 32)),
                     [vblo] "s"((uint32_t)vb), [vbhi] "s"((uint32_t)(vb >> 32)), [ko0] "v"(koff[0]),
                     [ko1] "v"(koff[1]), [ko2] "v"(koff[2]), [ko3] "v"(koff[3]), [kl0] "v"(koff_last[0]),
                     [kl1] "v"(koff_last[1]), [kl2] "v"(koff_last[2]), [kl3] "v"(koff_last[3]), [ka0] "v"(ka[0]),
                     [ka1] "v"(ka[1]), [ka2] "v"(ka[2]), [ka3] "v"(ka[3]), [tv00] "v"(tv[0][0]),
                     [tv01] "v"(tv[0][1]), [tv10] "v"(tv[1][0]), [tv11] "v"(tv[1][1]), [qbase] "v"(qbase),
                     [laned] "v"(laned), [g8] "v"(g8)
                   : SIDON_WIDE_VGPR_CLOBBERS, SIDON_WIDE_SGPR_CLOBBERS, "vcc", "m0", "scc", "memory");
#pragma clang diagnostic pop
      uint64_t overflow = 0;
#pragma unroll
      for (int J = 0; J < kBlocks; ++J) overflow |= __builtin_amdgcn_ballot_w64(!(lsum[J][0] < INFINITY));
      if (__builtin_expect(overflow != 0, 0)) continue;
      break;
    }
    // (The statement returns with every LDS read retired, so its register
    // outputs -- the V^T operands read below among them -- are final: a wait
    // placed here in compiled code would not order the register-only
    // products after it.)
    pv(2, 0);  // PV of items (nu - 1, 2) and (nu - 1, 3)
    pv(3, 1);
  }
  wait_vmcnt<0>();  // the last (unused) prefetches have landed before LDS is reused

  // ---- merge the key splits ----
  lds_barrier();  // every wavefront is done with its ring and the q.rel table
  float* mo = reinterpret_cast<float*>(smem);
  float* ml = reinterpret_cast<float*>(smem + kMergeMlOff);
#pragma unroll
  for (int J = 0; J < kBlocks; ++J) {
    float* dst = mo + (w * kRows + 32 * J + n) * kMergeStride;
#pragma unroll
    for (int db = 0; db < 2; ++db) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f4 val = {oacc[J][db][4 * j], oacc[J][db][4 * j + 1], oacc[J][db][4 * j + 2], oacc[J][db][4 * j + 3]};
        *reinterpret_cast<f4*>(dst + 32 * db + 8 * j + 4 * g) = val;
      }
    }
    if (g == 0) {
      ml[(w * kRows + 32 * J + n) * 2] = m_run[J];
      ml[(w * kRows + 32 * J + n) * 2 + 1] = lsum[J][0];
    }
  }
  lds_barrier();

  // Wavefront w finalises rows 32 w + [0, 32), two lanes per row, 32 dims
  // per lane.
  const int r = 32 * w + (lane >> 1);
  const int c = 32 * (lane & 1);
  float mmax = -INFINITY;
#pragma unroll
  for (int s = 0; s < kWaves; ++s) mmax = fmaxf(mmax, ml[(s * kRows + r) * 2]);
  float total = 0.f;
  f4 o[8] = {};
#pragma unroll
  for (int s = 0; s < kWaves; ++s) {
    const float ms = ml[(s * kRows + r) * 2];
    const float f = ms == -INFINITY ? 0.f : fast_exp2(ms - mmax);
    total += ml[(s * kRows + r) * 2 + 1] * f;
    const float* src = mo + (s * kRows + r) * kMergeStride + c;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] += *reinterpret_cast<const f4*>(src + 4 * j) * f;
  }
  const int row = q0 + r;
  if (row < p.L) {
    const float inv = total > 0.f ? __builtin_amdgcn_rcpf(total) : 0.f;
    _Float16* dst = p.out + b * p.osb + h * p.osh + (int64_t)row * p.osl + c;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const h8 v = {(_Float16)(o[2 * j][0] * inv), (_Float16)(o[2 * j][1] * inv), (_Float16)(o[2 * j][2] * inv),
                    (_Float16)(o[2 * j][3] * inv), (_Float16)(o[2 * j + 1][0] * inv),
                    (_Float16)(o[2 * j + 1][1] * inv), (_Float16)(o[2 * j + 1][2] * inv),
                    (_Float16)(o[2 * j + 1][3] * inv)};
      *reinterpret_cast<h8*>(dst + 8 * j) = v;
    }
  }
}

}  // namespace

int wide_rows() { return kRows; }
int wide_threads() { return kThreads; }

// Only K and V rows of the same stride (the fused QKV layout, and any
// [B, H, L, 64] views that share a row stride): the host uses the 64-row
// kernel otherwise.
hipError_t launch_wide(const Params& p, int nwg, bool same_stride, hipStream_t stream) {
  if (!same_stride) return hipErrorInvalidValue;
  hipLaunchKernelGGL(flexrel_wide_kernel<true>, dim3(nwg), dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace sidon_flexrel
