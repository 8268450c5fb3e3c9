// flexrel_device.h -- device helpers and launch parameters shared by the
// relative_key attention kernels (flexrel_fwd.hip: 64 query rows per
// workgroup, 8 key splits; flexrel_w64.hip: 64 rows per wavefront, 4 key splits, two
// workgroups per compute unit; flexrel_w32.hip: 32 rows per wavefront, 4 key
// splits, for short sequences).  Internal to the library.
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

namespace sidon_flexrel {

constexpr int kD = 64;          // head dim
constexpr int kLeft = 64;       // clamp window: j - i in [-64, 8]
constexpr int kRight = 8;
constexpr int kNumPos = 73;     // rows of the relative table
constexpr int kStep = 32;       // keys per pipeline step
constexpr int kTile = kStep * kD * 2;  // bytes of one K or V step tile (4 KB)
constexpr int kQrStride = 76;   // fp32 per row of the q.rel table
// A query's 32 probabilities of one step summing below 2^15 are each below
// the fp16 maximum, so their fp16 rounding is finite; a larger (or
// non-finite) sum sends the query through the exact max update.
constexpr float kSumLimit = 32768.f;

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define SIDON_LDS_PTR(T, p) ((__attribute__((address_space(3))) T*)(p))

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
  int nqb;                 // query blocks per (b, h) in this launch
  int row0;                // first query row of block 0 (a launch may cover rows [row0, L))
  float scale;             // log2(e) / sqrt(64)
  int rerun_all;           // test hook (sidon_flexrel_debug_rerun_all): every 64-row wavefront reruns
};

// 16-byte chunk c of tile row r is stored at chunk position c ^ tile_swz(r)
// (LDS: 64 banks of 4 bytes).  The map is a bijection of row bits 1..3, which
// keeps the 16 rows of every 16-lane ds_read_b128 group on distinct banks.
// It puts row bit 1 on chunk bit 2: a 32-lane half of a ds_read_b64_tr_b16
// reads rows with bits 0-1 varying and chunk bits 0-1 varying (lane bits 1
// and 4), so row bit 1 must land on the one chunk bit that does not vary.
__device__ __forceinline__ int tile_swz(int row) {
  return ((row >> 2) & 1) | ((row >> 2) & 2) | ((row << 1) & 4);
}

// Key row fed to A-operand lane m of S^T = K.Q^T: bits 2 and 3 of m swapped.
// With the 32x32 accumulator layout (lane half g holds rows 8*(i/4) + 4g +
// i%4) element i of lane half g is then key 16*(i >> 3) + 8g + (i & 7).
__device__ __forceinline__ int mfma_row_perm(int m) {
  return (m & 0x13) | ((m >> 1) & 4) | ((m << 1) & 8);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// x of lane l and of lane l ^ 32 (the other half of the wavefront) combined
// with max.  v_permlane32_swap applied to (x, x) leaves one half's
// value in each result register, so any symmetric combination of the two is
// the combination over the lane pair.
__device__ __forceinline__ float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Asynchronous copy global -> LDS of one 4 KB tile: four instructions of
// 64 lanes x 16 bytes.  Instruction i adds 1024 i to both addresses: lane l's
// bytes gbase[voff_i,l + 1024 i .. +16) land at LDS byte address
// lds_addr + 1024 i + 16 l.  Issued as inline assembly so that the compiler
// does not wait for the copy before unrelated LDS reads; completion is
// awaited with wait_vmcnt below.  M0 is written here; nothing else in the
// library's kernels uses M0 (the clobber documents it -- the compiler treats
// M0 as reserved).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma_tile(uint32_t lds_addr, const char* gbase, uint32_t v0, uint32_t v1,
                                         uint32_t v2, uint32_t v3) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %5\n\t"
      "global_load_lds_dwordx4 %2, %5 offset:1024\n\t"
      "global_load_lds_dwordx4 %3, %5 offset:2048\n\t"
      "global_load_lds_dwordx4 %4, %5 offset:3072"
      :: "s"(lds_addr), "v"(v0), "v"(v1), "v"(v2), "v"(v3), "s"(gbase) : "memory", "m0");
}
__device__ __forceinline__ void dma_1k(uint32_t lds_addr, const char* gbase, uint32_t v0) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :: "s"(lds_addr), "v"(v0), "s"(gbase) : "memory", "m0");
}
#pragma clang diagnostic pop

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}

__device__ __forceinline__ void wait_lgkm0() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ h8 cat(h4 a, h4 b) {
  return h8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// Workgroups are dispatched round-robin over the 8 XCDs; linear work index
// of workgroup `bid` such that each XCD gets a contiguous range (one head's
// K/V then stays in one XCD's L2).
__device__ __forceinline__ int xcd_linear(int bid, int nwg) {
  const int xcd = bid & 7;
  const int per = nwg >> 3;
  const int rem = nwg & 7;
  return (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + (bid >> 3);
}

// Per-lane offsets of the 4-wavefront kernels (flexrel_w64.hip,
// flexrel_w32.hip), formed from the lane id.
struct LaneTab {
  int n, g;                        // query column in a 32-block, lane half
  uint32_t voff[4], voff_last[4];  // tile copy offsets from base - 3072: any step, the last step
  uint32_t kofs, kofs_last;        // K operand row offsets for global loads: any step, the last step
  int kperm;                       // key row held by the K operand lane
  int tr_off[2][2];                // V^T transpose-read offsets [hf][db] for hh = 0
};

// Tile copy lane offsets: LDS chunk position 64 i + lane = row 8 i + lane / 8,
// swizzled chunk lane % 8; the last step T - 1 re-reads row LK - 1 (last_row
// of the tile) for its rows past LK (their scores are masked).  K operands:
// lane (m, g) of the MFMA A operand holds key row perm(m), dims 16 s + 8 g +
// [0, 8) for k-step s (bytes 32 s + 16 g of the row).  V^T operands via
// transpose reads (ds_read_b64_tr_b16): group G of 16 lanes, source lane
// (a, bq) reads V[key0 + a][d0 + 4 bq .. +4) with key0 = 16 hh + 8 (G / 2) +
// 4 hf and d0 = 32 db + 16 (G % 2).
__device__ __forceinline__ LaneTab lane_tab(int lane, int64_t kstride, int last_row) {
  LaneTab t;
  t.n = lane & 31;
  t.g = lane >> 5;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 8 * i + (lane >> 3);
    const int rc = min(r, last_row);
    const uint32_t c16 = 16u * ((lane & 7) ^ tile_swz(r)) + 3072u - 1024u * i;
    t.voff[i] = (uint32_t)(r * kstride) + c16;
    t.voff_last[i] = (uint32_t)(rc * kstride) + c16;
  }
  t.kperm = mfma_row_perm(t.n);
  t.kofs = (uint32_t)(t.kperm * kstride) + 16u * t.g;
  t.kofs_last = (uint32_t)(min(t.kperm, last_row) * kstride) + 16u * t.g;
  const int tr_G = lane >> 4, tr_a = (lane >> 2) & 3, tr_b = lane & 3;
#pragma unroll
  for (int hf = 0; hf < 2; ++hf)
#pragma unroll
    for (int db = 0; db < 2; ++db) {
      const int row = 8 * (tr_G >> 1) + 4 * hf + tr_a;
      const int chunk = 4 * db + 2 * (tr_G & 1) + (tr_b >> 1);
      t.tr_off[hf][db] = row * 128 + ((chunk ^ tile_swz(row)) << 4) + 8 * (tr_b & 1);
    }
  return t;
}

// The lane id from an opaque instruction pair: never merged with an earlier
// computation of it, so it is formed again instead of kept live.
__device__ __forceinline__ int fresh_lane_id() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

}  // namespace sidon_flexrel

namespace sidon_flexrel {
// Launch of the 64-row, two-workgroups-per-CU kernel (flexrel_w64.hip), with
// p.nqb = query blocks of 64 rows per (b, h).
int w64_rows();
int w64_threads();
hipError_t launch_w64(const Params& p, int nwg, bool same_stride, hipStream_t stream);
// Launch of the 32-row kernel (flexrel_w32.hip), with p.nqb = query blocks
// of 32 rows per (b, h).
int w32_rows();
int w32_threads();
hipError_t launch_w32(const Params& p, int nwg, bool same_stride, hipStream_t stream);
}  // namespace sidon_flexrel
