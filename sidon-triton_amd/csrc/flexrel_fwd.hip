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
// Work decomposition (one workgroup = NQ x NK wavefronts of 64 lanes):
//   * a wavefront owns 32 query rows and one key split; the NQ wavefronts of
//     a split share its K / V^T tiles (64 keys each) staged in LDS, loaded
//     through registers one tile ahead of the MFMA work;
//   * the NK key splits of a workgroup cover [0, LK) in contiguous tile
//     ranges and are merged through LDS at the end (flash-decoding style
//     split, kept inside one workgroup so no workspace is needed);
//   * scores are formed transposed, S^T = K . Q^T, with
//     v_mfma_f32_32x32x16_f16: every lane then holds one query column, so
//     the softmax row state (max, sum, rescale factor) is per-lane and the
//     only cross-lane step is one swap between the two 32-lane halves;
//   * O^T += V^T . P^T reuses the S^T accumulator registers directly as the
//     B operand (after rounding P to fp16).  The K rows loaded into the A
//     operand are permuted (bits 2 and 3 of the row index swapped) so that
//     the 8 keys a lane contributes to each PV step are contiguous, which
//     makes every V^T operand one 16-byte LDS read;
//   * the relative bias: Q.rel^T for the 32 rows x 73 positions is one small
//     MFMA product per wavefront kept in LDS (fp32).  Key tiles entirely left
//     (j - i <= -64) or right (j - i >= 8) of every row of the wavefront see a
//     per-row constant bias, which is folded into the exp2 argument and the
//     running max; only the 2-3 "band" tiles per row block gather it per
//     score;
//   * keys >= LK are zero-filled on load and their scores set to -inf in the
//     one tile that straddles LK; tiles starting at or past LK are never
//     visited.
#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "sidon_flexrel.h"

#define SIDON_API extern "C" __attribute__((visibility("default")))

namespace {

constexpr int kD = 64;           // head dim
constexpr int kLeft = 64;        // clamp window: j - i in [-64, 8]
constexpr int kRight = 8;
constexpr int kNumPos = 73;      // rows of the relative table
constexpr int kBN = 64;          // keys per tile
constexpr int kWQ = 32;          // query rows per wavefront
constexpr int kQrStride = 76;    // fp32 per row of the LDS q.rel table
constexpr int kTileBytes = kBN * kD * 2;
constexpr int kMergeFloats = 34 * 64;  // m, l, 32 accumulators per lane

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

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

// LDS K tile: row = key (128 bytes = 8 chunks of 8 fp16).  Chunk c of key row
// r is stored at chunk position c ^ key_swz(r).  The 8 lanes that read one
// 128-byte wavefront slice hit keys {b..b+3, b+8..b+11}; key_swz is distinct
// over them, so the slice is bank-conflict free.
__device__ __forceinline__ int key_swz(int key) {
  return (key & 3) | ((key >> 1) & 4);
}

// Key row loaded into A-operand lane m of the S^T = K.Q^T MFMA: bits 2 and 3
// of m swapped.  With the 32x32 accumulator layout (lane group g holds rows
// 8*(i/4) + 4g + i%4) the 8 P^T values a lane feeds to PV step hh are then
// keys 16*hh + 8g + [0, 8) of the 32-key block.
__device__ __forceinline__ int mfma_row_perm(int m) {
  return (m & 0x13) | ((m >> 1) & 4) | ((m << 1) & 8);
}

__device__ __forceinline__ float fast_exp2(float x) {
  return __builtin_amdgcn_exp2f(x);
}

template <int NQ, int NK>
__global__ void __launch_bounds__(64 * NQ * NK)
flexrel_fwd_kernel(const Params p) {
  constexpr int GT = 64 * NQ;                      // threads per key split
  constexpr int KCH = (kBN * kD / 8) / GT;         // 16-B K chunks / thread
  constexpr int VBL = ((kBN / 4) * (kD / 8)) / GT; // 4x8 V blocks / thread
  constexpr int KV_BYTES = NK * 2 * kTileBytes;
  constexpr int QR_BYTES = NQ * kWQ * kQrStride * 4;
  static_assert(KCH * GT == 512 && VBL * GT == 128, "NQ must be 1 or 2");
  static_assert((NK - 1) * NQ * kMergeFloats * 4 <= KV_BYTES,
                "merge buffer must fit in the K/V tiles");
  __shared__ __attribute__((aligned(16))) char smem[KV_BYTES + QR_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int qi = w % NQ;    // query sub-block of this wavefront
  const int ki = w / NQ;    // key split of this wavefront
  const int n = lane & 31;  // query column of this lane
  const int g = lane >> 5;  // lane half
  const int tg = qi * 64 + lane;

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
  const int qb = lin - bh * p.nqb;
  const int b = bh / p.H;
  const int h = bh - b * p.H;

  int LK = p.L;
  if (p.lens != nullptr) LK = min(max(p.lens[b], 0), p.L);
  const int q0 = qb * (kWQ * NQ) + kWQ * qi;
  const float scale = p.scale;

  const _Float16* qbase = p.q + b * p.qsb + h * p.qsh;
  const _Float16* kbase = p.k + b * p.ksb + h * p.ksh;
  const _Float16* vbase = p.v + b * p.vsb + h * p.vsh;

  // Q^T as the MFMA B operand: lane (n, g) holds query q0 + n, dims
  // 16*s + 8*g + [0, 8) for k-step s.  Rows >= L are zero.
  h8 qop[4];
  {
    const int row = q0 + n;
    if (row < p.L) {
      const _Float16* src = qbase + (int64_t)row * p.qsl + 8 * g;
#pragma unroll
      for (int s = 0; s < 4; ++s) qop[s] = *reinterpret_cast<const h8*>(src + 16 * s);
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) qop[s] = h8{};
    }
  }

  // q.rel^T for this wavefront's 32 rows (raw dot products), computed by the
  // split-0 wavefronts as (rel . Q^T): 3 position blocks of 32 (73 used).
  float* qr_tab = reinterpret_cast<float*>(smem + KV_BYTES) + qi * (kWQ * kQrStride);
  if (ki == 0) {
#pragma unroll
    for (int pb = 0; pb < 3; ++pb) {
      f32x16 acc = {};
      const int pos = 32 * pb + n;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        h8 e = {};
        if (pos < kNumPos) e = *reinterpret_cast<const h8*>(p.rel + pos * kD + 16 * s + 8 * g);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(e, qop[s], acc, 0, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int pos0 = 32 * pb + 8 * j + 4 * g;
        if (pos0 < kQrStride) {
          const f4 val = {acc[4 * j], acc[4 * j + 1], acc[4 * j + 2], acc[4 * j + 3]};
          *reinterpret_cast<f4*>(qr_tab + n * kQrStride + pos0) = val;
        }
      }
    }
  }

  char* Ks = smem + ki * 2 * kTileBytes;
  char* Vt = Ks + kTileBytes;
  const int T = (LK + kBN - 1) / kBN;  // key tiles that hold a valid key
  const int tb = (ki * T) / NK;
  const int te = ((ki + 1) * T) / NK;
  const int niter = (T + NK - 1) / NK;

  u4 kreg[KCH];
  u4 vreg[4 * VBL];

  auto load_tile = [&](int t) {
    const int n0 = t * kBN;
    const _Float16* kt = kbase + (int64_t)n0 * p.ksl;
    const _Float16* vt = vbase + (int64_t)n0 * p.vsl;
#pragma unroll
    for (int j = 0; j < KCH; ++j) {
      const int c = tg + GT * j;
      const int key = c >> 3;
      u4 val = {0u, 0u, 0u, 0u};
      if (n0 + key < LK) val = *reinterpret_cast<const u4*>(kt + key * p.ksl + 8 * (c & 7));
      kreg[j] = val;
    }
#pragma unroll
    for (int j = 0; j < VBL; ++j) {
      const int bb = tg + GT * j;
      const int dc = bb & 7;
      const int k4 = bb >> 3;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = 4 * k4 + r;
        u4 val = {0u, 0u, 0u, 0u};
        if (n0 + key < LK) val = *reinterpret_cast<const u4*>(vt + key * p.vsl + 8 * dc);
        vreg[4 * j + r] = val;
      }
    }
  };

  // K rows go to LDS as loaded (swizzled chunks).  V is transposed on the
  // way in: a thread holds 4 keys x 8 dims and writes, per dim, the 4 keys
  // as one 8-byte piece of the V^T row (V^T row d = 64 keys = 8 chunks,
  // chunk c stored at c ^ (d & 7)).
  auto store_tile = [&]() {
#pragma unroll
    for (int j = 0; j < KCH; ++j) {
      const int c = tg + GT * j;
      const int key = c >> 3;
      *reinterpret_cast<u4*>(Ks + key * 128 + (((c & 7) ^ key_swz(key)) << 4)) = kreg[j];
    }
#pragma unroll
    for (int j = 0; j < VBL; ++j) {
      const int bb = tg + GT * j;
      const int dc = bb & 7;
      const int k4 = bb >> 3;
      const int c8 = k4 >> 1;
      const int half = (k4 & 1) * 8;
#pragma unroll
      for (int wi = 0; wi < 4; ++wi) {
        const uint32_t a0 = vreg[4 * j + 0][wi];
        const uint32_t a1 = vreg[4 * j + 1][wi];
        const uint32_t a2 = vreg[4 * j + 2][wi];
        const uint32_t a3 = vreg[4 * j + 3][wi];
        const u2 lo = {(a0 & 0xFFFFu) | (a1 << 16), (a2 & 0xFFFFu) | (a3 << 16)};
        const u2 hi = {(a0 >> 16) | (a1 & 0xFFFF0000u), (a2 >> 16) | (a3 & 0xFFFF0000u)};
        const int d0 = 8 * dc + 2 * wi;
        const int d1 = d0 + 1;
        *reinterpret_cast<u2*>(Vt + d0 * 128 + ((c8 ^ (d0 & 7)) << 4) + half) = lo;
        *reinterpret_cast<u2*>(Vt + d1 * 128 + ((c8 ^ (d1 & 7)) << 4) + half) = hi;
      }
    }
  };

  if (tb < te) {
    load_tile(tb);
  } else {
#pragma unroll
    for (int j = 0; j < KCH; ++j) kreg[j] = u4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < 4 * VBL; ++j) vreg[j] = u4{0u, 0u, 0u, 0u};
  }
  store_tile();
  __syncthreads();  // K/V tile 0 and the q.rel table are in LDS

  const float* qr_row = qr_tab + n * kQrStride;
  const float qr_left = qr_row[0] * scale;             // bias of j - i <= -64
  const float qr_right = qr_row[kNumPos - 1] * scale;  // bias of j - i >= 8
  const int iq = q0 + n;

  float m_run = -INFINITY;  // running max (log2 units, true scores)
  float l_run = 0.f;        // running sum of this lane's keys
  f32x16 oacc[2] = {};      // O^T: dims 32*db + 8*(i/4) + 4g + i%4, query n

  for (int it = 0; it < niter; ++it) {
    const int t = tb + it;
    const bool have = t < te;
    const bool have_next = t + 1 < te;
    if (have_next) load_tile(t + 1);
    if (have) {
      const int n0 = t * kBN;
      f32x16 sacc[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        sacc[kb] = f32x16{};
        const int key = 32 * kb + mfma_row_perm(n);
        const char* krow = Ks + key * 128;
        const int sw = key_swz(key);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const h8 kop = *reinterpret_cast<const h8*>(krow + (((2 * s + g) ^ sw) << 4));
          sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kop, qop[s], sacc[kb], 0, 0, 0);
        }
      }
      // Lane (n, g), element i of block kb holds key
      // n0 + 32*kb + 16*(i >> 3) + 8*g + (i & 7).
      const bool left = n0 + (kBN - 1) + kLeft <= q0;
      const bool right = n0 >= q0 + (kWQ - 1) + kRight;
      const bool masked = n0 + kBN > LK;
      float off = 0.f;
      if (left) off = qr_left;
      if (right) off = qr_right;
      if (!left && !right) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = n0 + 32 * kb + 16 * (i >> 3) + 8 * g + (i & 7);
            const int rel = min(max(key - iq, -kLeft), kRight) + kLeft;
            sacc[kb][i] += qr_row[rel];
          }
        }
      }
      if (masked) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = n0 + 32 * kb + 16 * (i >> 3) + 8 * g + (i & 7);
            if (key >= LK) sacc[kb][i] = -INFINITY;
          }
        }
      }
      float mx = sacc[0][0];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sacc[kb][i]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run, fmaf(mx, scale, off));
      const float alpha = fast_exp2(m_run - m_new);
      const float nb = off - m_new;
      float ls = 0.f;
      h8 pop[2][2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float pv = fast_exp2(fmaf(sacc[kb][i], scale, nb));
          ls += pv;
          pop[kb][i >> 3][i & 7] = (_Float16)pv;
        }
      }
      l_run = l_run * alpha + ls;
      m_run = m_new;
      oacc[0] *= alpha;
      oacc[1] *= alpha;
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        const int d = 32 * db + n;
        const char* vrow = Vt + d * 128;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const h8 vop = *reinterpret_cast<const h8*>(vrow + (((4 * kb + 2 * hh + g) ^ (d & 7)) << 4));
            oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vop, pop[kb][hh], oacc[db], 0, 0, 0);
          }
        }
      }
    }
    __syncthreads();  // every wavefront is done reading tile t
    if (have_next) store_tile();
    __syncthreads();  // tile t + 1 is in LDS
  }

  float l_tot = l_run + __shfl_xor(l_run, 32);

  if constexpr (NK > 1) {
    // Merge the key splits: splits 1.. park (m, l, O^T) in the K/V area,
    // split 0 rescales everything to the common max and sums.
    float* mb = reinterpret_cast<float*>(smem);
    if (ki > 0) {
      float* dst = mb + ((ki - 1) * NQ + qi) * kMergeFloats;
      dst[lane] = m_run;
      dst[64 + lane] = l_tot;
#pragma unroll
      for (int r = 0; r < 32; ++r) dst[(2 + r) * 64 + lane] = oacc[r >> 4][r & 15];
    }
    __syncthreads();
    if (ki != 0) return;
    float mmax = m_run;
#pragma unroll
    for (int kk = 1; kk < NK; ++kk) mmax = fmaxf(mmax, mb[((kk - 1) * NQ + qi) * kMergeFloats + lane]);
    const float f0 = (m_run == -INFINITY) ? 0.f : fast_exp2(m_run - mmax);
    l_tot *= f0;
    oacc[0] *= f0;
    oacc[1] *= f0;
#pragma unroll
    for (int kk = 1; kk < NK; ++kk) {
      const float* src = mb + ((kk - 1) * NQ + qi) * kMergeFloats;
      const float mk = src[lane];
      const float fk = (mk == -INFINITY) ? 0.f : fast_exp2(mk - mmax);
      l_tot += src[64 + lane] * fk;
#pragma unroll
      for (int r = 0; r < 32; ++r) oacc[r >> 4][r & 15] += src[(2 + r) * 64 + lane] * fk;
    }
  }

  if (iq < p.L) {
    const float inv = l_tot > 0.f ? __builtin_amdgcn_rcpf(l_tot) : 0.f;
    _Float16* dst = p.out + b * p.osb + h * p.osh + (int64_t)iq * p.osl;
#pragma unroll
    for (int db = 0; db < 2; ++db) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d0 = 32 * db + 8 * j + 4 * g;
        const h4 o = {(_Float16)(oacc[db][4 * j] * inv), (_Float16)(oacc[db][4 * j + 1] * inv),
                      (_Float16)(oacc[db][4 * j + 2] * inv), (_Float16)(oacc[db][4 * j + 3] * inv)};
        *reinterpret_cast<h4*>(dst + d0) = o;
      }
    }
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

struct Shape {
  int nq;   // query sub-blocks (wavefronts) per key split
  int nk;   // key splits per workgroup
};

// Enough workgroups to cover the 256 CUs several times over: key splits
// shrink each workgroup's serial work when (b, h, query block) count is low.
Shape pick_shape(int B, int H, int L) {
  const long long rows = (long long)B * H * ((L + 63) / 64);
  if (rows >= 512) return {2, 2};
  return {2, 4};
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

template <int NQ, int NK>
hipError_t launch(const Params& p, int nwg, hipStream_t stream) {
  hipLaunchKernelGGL((flexrel_fwd_kernel<NQ, NK>), dim3(nwg), dim3(64 * NQ * NK), 0, stream, p);
  return hipGetLastError();
}

}  // namespace

SIDON_API int sidon_flexrel_launch_shape(int B, int H, int L, int* queries_per_block,
                                         int* key_splits, int* workgroups, int* threads_per_block) {
  if (B < 1 || H < 1 || L < 1) return fail(SIDON_E_SHAPE, "B=%d H=%d L=%d must be >= 1", B, H, L);
  const Shape s = pick_shape(B, H, L);
  const long long nqb = (L + kWQ * s.nq - 1) / (kWQ * s.nq);
  const long long nwg = (long long)B * H * nqb;
  if (nwg >= (1LL << 31)) return fail(SIDON_E_SHAPE, "grid of %lld workgroups too large", nwg);
  if (queries_per_block) *queries_per_block = kWQ * s.nq;
  if (key_splits) *key_splits = s.nk;
  if (workgroups) *workgroups = (int)nwg;
  if (threads_per_block) *threads_per_block = 64 * s.nq * s.nk;
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
  p.nqb = (L + nq - 1) / nq;
  p.scale = 1.4426950408889634f / 8.0f;  // log2(e) / sqrt(64)

  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t err;
  if (nq == 64 && nk == 2) err = launch<2, 2>(p, nwg, s);
  else if (nq == 64 && nk == 4) err = launch<2, 4>(p, nwg, s);
  else return fail(SIDON_E_LAUNCH, "no kernel instance for %d queries x %d splits", nq, nk);
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

SIDON_API const char* sidon_version(void) { return "sidon-flexrel 0.1.0 gfx950"; }
