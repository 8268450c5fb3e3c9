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
// 8 wavefronts; wavefront w runs an independent online softmax over the w-th
// eighth of the key range [0, LK) and the 8 partial results are merged
// through LDS at the end.  Inside a wavefront the keys advance in steps of 32:
//
//   * wavefront w takes steps w, w + 8, w + 16, ... (round-robin, so the few
//     steps that need the per-score bias gather or the key mask fall at the
//     same time for all wavefronts of a workgroup);
//   * K and V step tiles (32 keys x 64 dims, 4 KB each) are copied
//     global -> LDS with global_load_lds_dwordx4 (no register staging) into a
//     per-wavefront ring of two K and two V slots: the copy of K(u+2) and
//     V(u+1) is in flight while step u computes.  16-byte chunks are XOR
//     swizzled by row so both LDS read patterns below are bank-conflict free;
//   * per step a wavefront runs an MFMA phase (S^T of step u, O^T update of
//     step u - 1, then the copies and LDS operand reads for the next step)
//     and a VALU-only softmax phase;
//   * scores are formed transposed, S^T = K . Q^T, with
//     v_mfma_f32_32x32x16_f16 on two 32-query column blocks (Q^T stays in
//     registers): every lane holds scores of one query only, so the softmax
//     row state is per lane.  K rows are fed to the MFMA A operand with bits
//     2 and 3 of the row index swapped, which makes the 8 probabilities a lane
//     owns per 16-key PV step contiguous keys: the score accumulator, rounded
//     to fp16, is the B operand of O^T += V^T . P^T without any shuffle;
//   * the V^T operand comes straight from the key-major V tile through
//     ds_read_b64_tr_b16 (LDS transpose read);
//   * softmax with a lazily updated running max: probabilities are
//     exp2(s * log2(e)/8 + bias - m) with the max m of earlier steps.  While the
//     step's probabilities stay inside the fp16 range (a lane's 16 values
//     summing below 2^15), m, the row sum and O need no rescaling; a step
//     that leaves it, and the first step, take the exact max-update path.
//     The row sum is accumulated in fp32 with plain adds (v_dot2_f32_f16
//     shares the matrix pipe and would stall the other wavefront's MFMAs);
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
#include <string.h>

#include <mutex>

#include "sidon_flexrel.h"

#define SIDON_API extern "C" __attribute__((visibility("default")))

namespace {

constexpr int kD = 64;          // head dim
constexpr int kLeft = 64;       // clamp window: j - i in [-64, 8]
constexpr int kRight = 8;
constexpr int kNumPos = 73;     // rows of the relative table
constexpr int kStep = 32;       // keys per pipeline step
constexpr int kRows = 64;       // query rows per workgroup (two 32-column blocks)
constexpr int kWaves = 8;       // key splits per workgroup, one wavefront each
constexpr int kThreads = 64 * kWaves;
constexpr int kTile = kStep * kD * 2;      // bytes of one K or V step tile
constexpr int kWaveRing = 4 * kTile;       // K slot 0, K slot 1, V slot 0, V slot 1
constexpr int kQrStride = 76;              // fp32 per row of the q.rel table
// A lane's 16 probabilities of one step summing below 2^15 are each below the
// fp16 maximum, so their fp16 rounding is finite; a larger (or non-finite)
// sum sends the query through the exact max update.
constexpr float kSumLimit = 32768.f;
constexpr int kQrOff = kWaves * kWaveRing;
constexpr int kLdsBytes = kQrOff + kRows * kQrStride * 4;
// Split merge (reuses the ring and table area after the key loop).
constexpr int kMergeStride = 68;           // fp32 per partial-output row
constexpr int kMergeMlOff = kWaves * kRows * kMergeStride * 4;
static_assert(kMergeMlOff + kWaves * kRows * 2 * 4 <= kLdsBytes, "merge area too small");
static_assert(kLdsBytes <= 160 * 1024, "LDS budget of one CU");

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define LDS_PTR(T, p) ((__attribute__((address_space(3))) T*)(p))

struct Params {
  const _Float16* q;
  const _Float16* k;
  const _Float16* v;
  const _Float16* rel;
  const int32_t* lens;
  _Float16* out;
  int64_t qsb, qsh;  // batch / head strides (elements)
  int64_t ksb, ksh;
  int64_t vsb, vsh;
  int64_t osb, osh;
  int qsl, ksl, vsl, osl;  // row strides (elements, < 2^25)
  int B, H, L;
  int nqb;                 // query blocks per (b, h)
  float scale;             // log2(e) / sqrt(64)
};

// 16-byte chunk c of tile row r is stored at chunk position c ^ tile_swz(r).
// The map is a bijection of row bits 1..3, which keeps the 16 rows of every
// ds_read_b128 quarter-wave on distinct banks, and puts row bit 1 on chunk
// bit 1, which spreads the four rows of every ds_read_b64_tr_b16 group.
__device__ __forceinline__ int tile_swz(int row) {
  return ((row >> 2) & 1) | (row & 2) | ((row >> 1) & 4);
}

// Key row fed to A-operand lane m of S^T = K.Q^T: bits 2 and 3 of m swapped.
// With the 32x32 accumulator layout (lane half g holds rows 8*(i/4) + 4g +
// i%4) element i of lane half g is then key 16*(i >> 3) + 8g + (i & 7).
__device__ __forceinline__ int mfma_row_perm(int m) {
  return (m & 0x13) | ((m >> 1) & 4) | ((m << 1) & 8);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// x of lane l and of lane l ^ 32 (the other half of the wavefront) combined
// with max / sum.  v_permlane32_swap applied to (x, x) leaves one half's
// value in each result register, so any symmetric combination of the two is
// the combination over the lane pair.
__device__ __forceinline__ float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Asynchronous copy global -> LDS, 16 bytes per lane: lane l's bytes
// gbase[voff_l .. +16) land at LDS byte address lds_addr + 16 l.  Issued as
// inline assembly so that the compiler does not wait for the copy before
// unrelated LDS reads; completion is awaited with wait_vmcnt below.
// M0 is written here; nothing else in this translation unit uses M0 (the
// clobber documents it -- the compiler treats M0 as reserved).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma_x4(uint32_t lds_addr, const char* gbase, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :: "s"(lds_addr), "v"(voff), "s"(gbase) : "memory", "m0");
}
#pragma clang diagnostic pop

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}

__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ h8 cat(h4 a, h4 b) {
  return h8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

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
  const int nwg = gridDim.x;
  const int bid = blockIdx.x;
  const int xcd = bid & 7;
  const int per = nwg >> 3;
  const int rem = nwg & 7;
  const int lin = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + (bid >> 3);
  const int bh = lin / p.nqb;
  const int qblk = lin - bh * p.nqb;
  const int b = bh / p.H;
  const int h = bh - b * p.H;

  int LK = p.L;
  if (p.lens != nullptr) LK = min(max(p.lens[b], 0), p.L);
  LK = __builtin_amdgcn_readfirstlane(LK);
  const int q0 = qblk * kRows;
  const float scale = p.scale;

  const _Float16* qbase = p.q + b * p.qsb + h * p.qsh;
  const char* kbase = reinterpret_cast<const char*>(p.k + b * p.ksb + h * p.ksh);
  const char* vbase = reinterpret_cast<const char*>(p.v + b * p.vsb + h * p.vsh);
  const int64_t kstride = (int64_t)p.ksl * 2;  // bytes
  const int64_t vstride = (int64_t)p.vsl * 2;

  // Key steps: T steps of 32 keys cover [0, LK).  Wavefront w takes steps
  // t = w + 8 u, u = 0 .. nu - 1 (round-robin, so the few "band" and masked
  // steps of a workgroup fall into the same one or two phases).
  const int T = (LK + kStep - 1) / kStep;
  const int U = (T + kWaves - 1) / kWaves;          // phases of the slowest wavefront
  const int nu = T > w ? (T - w + kWaves - 1) / kWaves : 0;
  const bool active = nu > 0;

  char* ring = smem + w * kWaveRing;
  const uint32_t ring_lds = (uint32_t)(uintptr_t)LDS_PTR(char, ring);

  // Copy of one step tile (K or V) into an LDS slot: 4 instructions of 64
  // lanes x 16 bytes; LDS chunk position 64 i + lane = (row 8 i + lane / 8,
  // swizzled chunk lane % 8).
  uint32_t koff[4], voff_own[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 8 * i + (lane >> 3);
    const uint32_t c16 = 16u * ((lane & 7) ^ tile_swz(r));
    koff[i] = (uint32_t)(r * kstride) + c16;
    voff_own[i] = kSameStride ? 0u : (uint32_t)(r * vstride) + c16;
  }
  const uint32_t (&voff)[4] = kSameStride ? koff : voff_own;
  // Local step u of this wavefront -> global step; local steps past the
  // wavefront's range (prefetches whose data is never used) re-read step
  // T - 1, so every copy stays in bounds and every phase issues the same
  // number of copies.
  auto gstep = [&](int u) { return min(w + kWaves * u, T - 1); };
  auto copy_tile = [&](const char* base, int64_t stride, const uint32_t (&off)[4], int u,
                       uint32_t slot) {
    const int k0 = gstep(u) * kStep;
    const char* gb = base + (int64_t)k0 * stride;
    if (k0 + kStep <= LK) {
#pragma unroll
      for (int i = 0; i < 4; ++i) dma_x4(slot + 1024u * i, gb, off[i]);
    } else {
      // Rows past LK re-read row LK - 1 (in bounds); their scores are masked.
      const int last = LK - 1 - k0;  // >= 0: every step holds a valid key
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 8 * i + (lane >> 3);
        const uint32_t c16 = 16u * ((lane & 7) ^ tile_swz(r));
        dma_x4(slot + 1024u * i, gb, (uint32_t)(min(r, last) * stride) + c16);
      }
    }
  };
  auto k_slot = [&](int u) { return ring_lds + (uint32_t)((u & 1) * kTile); };
  auto v_slot = [&](int u) { return ring_lds + (uint32_t)(2 * kTile + (u & 1) * kTile); };

  // First copies K(0), K(1), V(0) -- the steady-state order (K of the next
  // step, then V of the current one) -- before the Q and table loads, so all
  // of them are in flight together.
  if (active) {
    copy_tile(kbase, kstride, koff, 0, k_slot(0));
    copy_tile(kbase, kstride, koff, 1, k_slot(1));
    copy_tile(vbase, vstride, voff, 0, v_slot(0));
  }

  // Q^T as the MFMA B operand: lane (n, g) of block qb holds query
  // q0 + 32 qb + n, dims 16 s + 8 g + [0, 8) for k-step s.  Rows >= L are 0.
  h8 qop[2][4];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int row = q0 + 32 * qb + n;
    const _Float16* src = qbase + (int64_t)min(row, p.L - 1) * p.qsl + 8 * g;
#pragma unroll
    for (int s = 0; s < 4; ++s) qop[qb][s] = *reinterpret_cast<const h8*>(src + 16 * s);
    if (row >= p.L) {
#pragma unroll
      for (int s = 0; s < 4; ++s) qop[qb][s] = h8{};
    }
  }
  // rel rows for the q.rel table (wavefronts 0..5, see below); rows >= 73 are 0.
  const int qr_pb = w % 3;
  const int qr_qb = w / 3;
  h8 eop[4];
  {
    const int pos = 32 * qr_pb + n;
    const _Float16* src = p.rel + min(pos, kNumPos - 1) * kD + 8 * g;
#pragma unroll
    for (int s = 0; s < 4; ++s) eop[s] = *reinterpret_cast<const h8*>(src + 16 * s);
    if (pos >= kNumPos) {
#pragma unroll
      for (int s = 0; s < 4; ++s) eop[s] = h8{};
    }
  }
  // Every load above, the first tile copies included, has landed.  (A wait
  // the compiler sees, so it does not re-wait for these loads in the loop.)
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)

  // q.rel^T * scale for the 64 rows: wavefront w < 6 computes positions
  // 32 (w % 3) + [0, 32) for column block w / 3 as rel . Q^T.
  float* qr_tab = reinterpret_cast<float*>(smem + kQrOff);
  if (w < 6) {
    f32x16 acc = {};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const h8 qsel = qr_qb ? qop[1][s] : qop[0][s];
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(eop[s], qsel, acc, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int pos0 = 32 * qr_pb + 8 * j + 4 * g;
      if (pos0 < kQrStride) {
        const f4 val = {acc[4 * j] * scale, acc[4 * j + 1] * scale, acc[4 * j + 2] * scale,
                        acc[4 * j + 3] * scale};
        *reinterpret_cast<f4*>(qr_tab + (32 * qr_qb + n) * kQrStride + pos0) = val;
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
  float l_run[2] = {0.f, 0.f};
  f32x16 sacc[2];           // S^T of the step in flight
  h8 pk[2][2];              // fp16 probabilities: [column block][16-key half]
  float lt[2];              // their sums
  h8 kop[4] = {};           // K operands of the next QK product (k-steps 0..3)
  h8 vop[2][2] = {};        // V^T operands of the next PV product [hh][db]
  pk[0][0] = pk[0][1] = pk[1][0] = pk[1][1] = h8{};

  // K operands: lane (m, g) holds key row perm(m) of the tile, dims
  // 16 s + 8 g + [0, 8).
  const int kperm = mfma_row_perm(n);
  const char* krow0 = ring + kperm * 128;
  const int kswz = tile_swz(kperm);
  auto load_k = [&](int u) {
    const char* krow = krow0 + (u & 1) * kTile;
#pragma unroll
    for (int s = 0; s < 4; ++s)
      kop[s] = *reinterpret_cast<const h8*>(krow + (((2 * s + g) ^ kswz) << 4));
  };
  // V^T operands via transpose reads: group G of 16 lanes, source lane
  // (a, bq) reads V[key0 + a][d0 + 4 bq .. +4) with key0 = 16 hh + 8 (G / 2)
  // + 4 hf and d0 = 32 db + 16 (G % 2).
  const int tr_G = lane >> 4;
  const int tr_a = (lane >> 2) & 3;
  const int tr_b = lane & 3;
  // Byte offset of the source of (hh, hf, db): row = 16 hh + 8 (G / 2) +
  // 4 hf + a, chunk = (4 db + 2 (G % 2) + bq / 2) ^ tile_swz(row).  hh adds
  // 2048 (an immediate); hf and db flip one chunk bit each through the
  // swizzle, so four per-lane bases cover all eight reads.
  int tr_off[2][2];  // [hf][db] byte offset for hh = 0
#pragma unroll
  for (int hf = 0; hf < 2; ++hf)
#pragma unroll
    for (int db = 0; db < 2; ++db) {
      const int row = 8 * (tr_G >> 1) + 4 * hf + tr_a;
      const int chunk = 4 * db + 2 * (tr_G & 1) + (tr_b >> 1);
      tr_off[hf][db] = row * 128 + ((chunk ^ tile_swz(row)) << 4) + 8 * (tr_b & 1);
    }
  auto load_v = [&](int u) {
    const char* vt = ring + 2 * kTile + (u & 1) * kTile;
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

  // MFMA phase u: O^T += V^T(u - 1) . P^T(u - 1), then S^T(u) = K(u) . Q^T.
  // Branch-free (one register assignment for O): where there is no step
  // u - 1 the probabilities are 0 and add exactly 0 (V is finite), and past
  // the wavefront's range S^T is computed on a valid dummy tile and unused.
  // The K operands are read here (their latency hides behind the PV MFMAs);
  // P is dead once PV is issued, so S^T can reuse its registers.
  auto mfma_phase = [&](int u) {
    load_k(u);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        oacc[0][db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vop[hh][db], pk[0][hh], oacc[0][db], 0, 0, 0);
        oacc[1][db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vop[hh][db], pk[1][hh], oacc[1][db], 0, 0, 0);
      }
    }
    sacc[0] = f32x16{};
    sacc[1] = f32x16{};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      sacc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kop[s], qop[0][s], sacc[0], 0, 0, 0);
      sacc[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kop[s], qop[1][s], sacc[1], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    // While the MFMAs run: copies of K(u + 2) and V(u + 1) into the slots
    // whose operands were read in phase u - 1; then K(u + 1) and V(u) (issued
    // one phase earlier) have landed for the next two LDS operand reads.
    if (u < nu) {
      copy_tile(kbase, kstride, koff, u + 2, k_slot(u + 2));
      copy_tile(vbase, vstride, voff, u + 1, v_slot(u + 1));
      wait_vmcnt<8>();
    }
  };

  // p = exp2(s * scale + nb) for a step without band or mask (nb = bias - m).
  auto probs_fast = [&](int qb, float nb) {
    float sum = 0.f;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f2 e = {fast_exp2(fmaf(sacc[qb][8 * hh + 2 * j], scale, nb)),
                      fast_exp2(fmaf(sacc[qb][8 * hh + 2 * j + 1], scale, nb))};
        const h2 ph = __builtin_convertvector(e, h2);
        pk[qb][hh][2 * j] = ph[0];
        pk[qb][hh][2 * j + 1] = ph[1];
        sum += e[0] + e[1];
      }
    }
    lt[qb] = sum;
  };
  // p = exp2(y - m) from explicit biased scores y.
  auto probs_y = [&](int qb, const float (&y)[16], float m) {
    float sum = 0.f;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f2 e = {fast_exp2(y[8 * hh + 2 * j] - m), fast_exp2(y[8 * hh + 2 * j + 1] - m)};
        const h2 ph = __builtin_convertvector(e, h2);
        pk[qb][hh][2 * j] = ph[0];
        pk[qb][hh][2 * j + 1] = ph[1];
        sum += e[0] + e[1];
      }
    }
    lt[qb] = sum;
  };

  // Softmax phase u: probabilities of step u (from sacc), plus the copies and
  // LDS operand reads that feed the next MFMA phase.
  auto softmax_phase = [&](int u) {
    if (u >= nu) {
      // No step u: the next MFMA phase's PV adds nothing.
      pk[0][0] = pk[0][1] = pk[1][0] = pk[1][1] = h8{};
      return;
    }

    const int k0 = (w + kWaves * u) * kStep;
    const bool masked = k0 + kStep > LK;
    bool band[2];
    float off[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const int qlo = q0 + 32 * qb;
      const bool left = k0 + (kStep - 1) - qlo <= -kLeft;
      const bool right = k0 - (qlo + 31) >= kRight;
      band[qb] = !left && !right;
      off[qb] = left ? qr_l[qb] : (right ? qr_r[qb] : 0.f);
    }
    const bool first = u == 0;  // the running max is still -inf

    if (!first && !masked && !band[0] && !band[1]) {
      probs_fast(0, off[0] - m_run[0]);
      probs_fast(1, off[1] - m_run[1]);
      if (__builtin_amdgcn_ballot_w64(!(fmaxf(lt[0], lt[1]) < kSumLimit)) != 0) {
        // A probability of some query left the fp16 range: exact max update
        // for those queries only (others keep bit-identical values).
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          const bool need = pair_max(lt[qb] < kSumLimit ? 0.f : 1.f) > 0.f;
          float mx = sacc[qb][0];
#pragma unroll
          for (int i = 1; i < 16; ++i) mx = fmaxf(mx, sacc[qb][i]);
          mx = pair_max(fmaf(mx, scale, off[qb]));
          const float m_new = need ? fmaxf(m_run[qb], mx) : m_run[qb];
          const float alpha = fast_exp2(m_run[qb] - m_new);
          l_run[qb] *= alpha;
          oacc[qb][0] *= alpha;
          oacc[qb][1] *= alpha;
          m_run[qb] = m_new;
          probs_fast(qb, off[qb] - m_new);
        }
      }
    } else {
      // y = s * scale + bias (log2 units); masked keys -> -inf.
      auto biased = [&](int qb, float (&y)[16]) {
        if (band[qb]) {
          const float* qrow = qr_tab + (32 * qb + n) * kQrStride;
          const int d0 = k0 + 8 * g - (q0 + 32 * qb + n) + kLeft;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int idx = min(max(d0 + 16 * (i >> 3) + (i & 7), 0), kLeft + kRight);
            y[i] = fmaf(sacc[qb][i], scale, qrow[idx]);
          }
        } else {
#pragma unroll
          for (int i = 0; i < 16; ++i) y[i] = fmaf(sacc[qb][i], scale, off[qb]);
        }
        if (masked) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = k0 + 16 * (i >> 3) + 8 * g + (i & 7);
            if (key >= LK) y[i] = -INFINITY;
          }
        }
      };
      // The same formula on the first call and after a max update, so rows
      // whose max did not change get bit-identical values.
      auto probs = [&](int qb, float m) {
        if (band[qb] || masked) {
          float y[16];
          biased(qb, y);
          probs_y(qb, y, m);
        } else {
          probs_fast(qb, off[qb] - m);
        }
      };
      if (!first) {
        probs(0, m_run[0]);
        probs(1, m_run[1]);
      }
      if (first || __builtin_amdgcn_ballot_w64(!(fmaxf(lt[0], lt[1]) < kSumLimit)) != 0) {
        // Exact max update for the queries that need it: the first step, or a
        // probability of this query left the fp16 range.  The decision is per
        // query (lane pair), never per wavefront, so one row cannot change
        // the rounding of another.
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          const bool need = first || pair_max(lt[qb] < kSumLimit ? 0.f : 1.f) > 0.f;
          float y[16];
          biased(qb, y);
          float mx = y[0];
#pragma unroll
          for (int i = 1; i < 16; ++i) mx = fmaxf(mx, y[i]);
          mx = pair_max(mx);
          const float m_new = need ? fmaxf(m_run[qb], mx) : m_run[qb];
          const float alpha = fast_exp2(m_run[qb] - m_new);  // 1 if unchanged, 0 from -inf
          l_run[qb] *= alpha;
          oacc[qb][0] *= alpha;
          oacc[qb][1] *= alpha;
          m_run[qb] = m_new;
          probs(qb, m_new);
        }
      }
    }
    l_run[0] += lt[0];
    l_run[1] += lt[1];
    load_v(u);  // V(u) operands for the next MFMA phase
  };

  // Each wavefront alternates an MFMA phase (PV of step u - 1, QK of step
  // u, then the copies for later steps) and a softmax phase (VALU only, then
  // the V operand reads of step u).  Wavefronts run free: the two sharing a SIMD drift
  // apart, so one's matrix work tends to overlap the other's exp2 work.
  for (int u = 0; u <= U; ++u) {
    mfma_phase(u);
    if (u < U) softmax_phase(u);
  }
  wait_vmcnt<0>();  // the last (unused) prefetches have landed before LDS is reused

  // ---- merge the 8 key splits ----
  float l_tot[2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) l_tot[qb] = pair_sum(l_run[qb]);

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

  // Wavefront w finalises rows 8 w + lane / 8, dims 8 (lane % 8) + [0, 8).
  const int r = 8 * w + (lane >> 3);
  const int c = 8 * (lane & 7);
  float mmax = -INFINITY;
#pragma unroll
  for (int s = 0; s < kWaves; ++s) mmax = fmaxf(mmax, ml[(s * kRows + r) * 2]);
  float lsum = 0.f;
  f4 o0 = {0.f, 0.f, 0.f, 0.f};
  f4 o1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < kWaves; ++s) {
    const float ms = ml[(s * kRows + r) * 2];
    const float f = ms == -INFINITY ? 0.f : fast_exp2(ms - mmax);
    lsum += ml[(s * kRows + r) * 2 + 1] * f;
    const float* src = mo + (s * kRows + r) * kMergeStride + c;
    o0 += *reinterpret_cast<const f4*>(src) * f;
    o1 += *reinterpret_cast<const f4*>(src + 4) * f;
  }
  const int row = q0 + r;
  if (row < p.L) {
    const float inv = lsum > 0.f ? __builtin_amdgcn_rcpf(lsum) : 0.f;
    const h8 o = {(_Float16)(o0[0] * inv), (_Float16)(o0[1] * inv), (_Float16)(o0[2] * inv),
                  (_Float16)(o0[3] * inv), (_Float16)(o1[0] * inv), (_Float16)(o1[1] * inv),
                  (_Float16)(o1[2] * inv), (_Float16)(o1[3] * inv)};
    *reinterpret_cast<h8*>(p.out + b * p.osb + h * p.osh + (int64_t)row * p.osl + c) = o;
  }
}

// ---------------------------------------------------------------------------
// host side

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

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

// One architecture check per device (gfx950 only).
int check_device() {
  static std::once_flag flags[64];
  static int status[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(SIDON_E_DEVICE, "hipGetDevice failed");
  if (dev < 0 || dev >= 64) return fail(SIDON_E_DEVICE, "device index %d out of range", dev);
  std::call_once(flags[dev], [dev]() {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
      status[dev] = -1;
      return;
    }
    status[dev] = strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : -2;
  });
  if (status[dev] == -1) return fail(SIDON_E_DEVICE, "hipGetDeviceProperties failed on device %d", dev);
  if (status[dev] != 1) return fail(SIDON_E_DEVICE, "device %d is not gfx950", dev);
  return SIDON_OK;
}

}  // namespace

SIDON_API int sidon_flexrel_launch_shape(int B, int H, int L, int* queries_per_block,
                                         int* key_splits, int* workgroups, int* threads_per_block) {
  if (B < 1 || H < 1 || L < 1) return fail(SIDON_E_SHAPE, "B=%d H=%d L=%d must be >= 1", B, H, L);
  const long long nqb = (L + kRows - 1) / kRows;
  const long long nwg = (long long)B * H * nqb;
  if (nwg >= (1LL << 31)) return fail(SIDON_E_SHAPE, "grid of %lld workgroups too large", nwg);
  if (queries_per_block) *queries_per_block = kRows;
  if (key_splits) *key_splits = kWaves;
  if (workgroups) *workgroups = (int)nwg;
  if (threads_per_block) *threads_per_block = kThreads;
  return SIDON_OK;
}

SIDON_API int sidon_flexrel_fwd(const void* q, const void* k, const void* v, const void* rel,
                                const int32_t* lens, void* out, int B, int H, int L, int head_dim,
                                const int64_t* q_strides, const int64_t* k_strides,
                                const int64_t* v_strides, const int64_t* o_strides,
                                sidon_stream_t stream) {
  g_err[0] = '\0';
  if (!q || !k || !v || !rel || !out) return fail(SIDON_E_NULL, "q, k, v, rel and out must be non-NULL");
  if (head_dim != kD) return fail(SIDON_E_SHAPE, "head_dim must be 64 (got %d)", head_dim);
  if (B < 1 || H < 1 || L < 1) return fail(SIDON_E_SHAPE, "B=%d H=%d L=%d must be >= 1", B, H, L);
  int rc;
  if ((rc = check_strides("q", q_strides)) || (rc = check_strides("k", k_strides)) ||
      (rc = check_strides("v", v_strides)) || (rc = check_strides("out", o_strides)))
    return rc;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(rel) || !aligned16(out))
    return fail(SIDON_E_ALIGN, "q, k, v, rel and out must be 16-byte aligned");
  int wg_threads = 0, nwg = 0, nq = 0, nk = 0;
  if ((rc = sidon_flexrel_launch_shape(B, H, L, &nq, &nk, &nwg, &wg_threads))) return rc;
  if ((rc = check_device())) return rc;

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
  p.nqb = (L + kRows - 1) / kRows;
  p.scale = 1.4426950408889634f / 8.0f;  // log2(e) / sqrt(64)

  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (p.ksl == p.vsl)
    hipLaunchKernelGGL(flexrel_fwd_kernel<true>, dim3(nwg), dim3(kThreads), 0, s, p);
  else
    hipLaunchKernelGGL(flexrel_fwd_kernel<false>, dim3(nwg), dim3(kThreads), 0, s, p);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(SIDON_E_LAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
  return SIDON_OK;
}

SIDON_API int sidon_flexrel_fwd_qkv(const void* qkv, const void* rel, const int32_t* lens, void* out,
                                    int B, int H, int L, sidon_stream_t stream) {
  g_err[0] = '\0';
  if (!qkv || !out || !rel) return fail(SIDON_E_NULL, "qkv, rel and out must be non-NULL");
  if (B < 1 || H < 1 || L < 1) return fail(SIDON_E_SHAPE, "B=%d H=%d L=%d must be >= 1", B, H, L);
  const int64_t hid = (int64_t)H * kD;
  const int64_t in_st[3] = {(int64_t)L * 3 * hid, kD, 3 * hid};
  const int64_t out_st[3] = {(int64_t)L * hid, kD, hid};
  const _Float16* base = static_cast<const _Float16*>(qkv);
  return sidon_flexrel_fwd(base, base + hid, base + 2 * hid, rel, lens, out, B, H, L, kD, in_st,
                           in_st, in_st, out_st, stream);
}

SIDON_API const char* sidon_last_error(void) { return g_err; }

SIDON_API const char* sidon_version(void) { return "sidon-flexrel 0.2.0 gfx950"; }
