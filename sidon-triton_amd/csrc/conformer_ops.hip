// conformer_ops.hip -- the conformer layer's elementwise and convolution
// kernels around its GEMMs (MI355X / gfx950):
//
//   glu              g = h[:, :C] * sigmoid(h[:, C:])                  fp16 -> fp16
//   silu (in place)  h = h * sigmoid(h)                                 fp16
//   causal_dw_norm   out[t] = silu(LN(sum_k w[k] * g[t + k - (K-1)]))   fp16 -> fp16
//
// They replace _glu_kernel / glu and _causal_dw_norm_kernel / causal_dw_norm
// of src/sidon_triton/triton_encoder.py:113-181, and the in-place F.silu of
// the feed-forward modules (:498-499, :507-508).  causal_dw_norm can also read
// the pointwise conv's output h [R, 2C] and form g = GLU(h) on the fly (g is
// rounded to fp16 exactly as glu stores it), which saves the g round trip
// through HBM.
//
// causal_dw_norm maps one thread to a channel pair and one block to BT
// consecutive frames of one batch item over all C channels.  The thread
// keeps its 2 K taps and BT accumulator pairs in registers and walks the
// BT + K - 1 source frames once, adding each frame's g into every output
// frame it reaches: each g element is read once per block (plus the K - 1
// frames of left context the block shares with its neighbour), and every
// output frame sums its taps in order k = 0 .. K-1.  LayerNorm reduces the
// block's BT rows at once (wavefront butterflies, then one LDS exchange).
#include <hip/hip_runtime.h>

#include <stdint.h>

#include <algorithm>

#include "sidon_encoder.h"
#include "sidon_host.h"
#include "sidon_wave.h"

#define SIDON_API extern "C" __attribute__((visibility("default")))

namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef float f8 __attribute__((ext_vector_type(8)));

constexpr int kMaxC = 2048;      // channels: one thread per pair, <= 1024 threads
constexpr int kEwThreads = 256;  // glu / silu block size
constexpr int kXcds = 8;         // accelerator complex dies of an MI355X
constexpr int kStageRows = 4;    // causal_dw_norm: source rows each thread loads per pass

// sigmoid(x) = 1 / (1 + e^-x) with the hardware exponential and reciprocal
// (each within about 1 ulp in fp32; the results are rounded to fp16).
__device__ __forceinline__ float sigmoid(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }

// GLU of one element as glu stores it: the fp32 product rounded to fp32,
// then to fp16.  The empty asm keeps the compiler from fusing the product and
// the conversion into one mixed-precision instruction, whose single rounding
// can differ from the two.
__device__ __forceinline__ _Float16 glu1(float a, float b) {
  float prod = a * sigmoid(b);
  asm volatile("" : "+v"(prod));
  return (_Float16)prod;
}

// SiLU of one element, rounded the same way (fp32, then fp16).
__device__ __forceinline__ _Float16 silu1(float x) {
  float y = x * sigmoid(x);
  asm volatile("" : "+v"(y));
  return (_Float16)y;
}

// ---- glu / silu -------------------------------------------------------------

// kVec chunks of 8 columns per thread (loads first, then math); requires
// C % 8 == 0 and 16-byte aligned rows.
constexpr int kVec = 4;
__global__ void __launch_bounds__(kEwThreads) glu_vec_kernel(const _Float16* __restrict__ h, _Float16* __restrict__ g,
                                                             int64_t n8, int c8) {
  const int64_t i0 = ((int64_t)blockIdx.x * kEwThreads * kVec) + threadIdx.x;
  h8 a[kVec], b[kVec];
#pragma unroll
  for (int v = 0; v < kVec; ++v) {
    const int64_t i = i0 + (int64_t)v * kEwThreads;
    if (i < n8) {
      const int64_t row = i / c8;
      const int64_t col = i - row * c8;
      a[v] = reinterpret_cast<const h8*>(h)[row * 2 * c8 + col];
      b[v] = reinterpret_cast<const h8*>(h)[row * 2 * c8 + c8 + col];
    }
  }
#pragma unroll
  for (int v = 0; v < kVec; ++v) {
    const int64_t i = i0 + (int64_t)v * kEwThreads;
    if (i < n8) {
      h8 o;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = glu1((float)a[v][j], (float)b[v][j]);
      reinterpret_cast<h8*>(g)[i] = o;
    }
  }
}

__global__ void __launch_bounds__(kEwThreads) glu_scalar_kernel(const _Float16* __restrict__ h,
                                                                _Float16* __restrict__ g, int64_t n, int C) {
  const int64_t i = (int64_t)blockIdx.x * kEwThreads + threadIdx.x;
  if (i >= n) return;
  const int64_t row = i / C;
  const int64_t col = i - row * C;
  const float a = (float)h[row * 2 * C + col];
  const float b = (float)h[row * 2 * C + C + col];
  g[i] = glu1(a, b);
}

__global__ void __launch_bounds__(kEwThreads) silu_vec_kernel(_Float16* __restrict__ h, int64_t n8) {
  const int64_t i0 = ((int64_t)blockIdx.x * kEwThreads * kVec) + threadIdx.x;
  h8 x[kVec];
#pragma unroll
  for (int v = 0; v < kVec; ++v) {
    const int64_t i = i0 + (int64_t)v * kEwThreads;
    if (i < n8) x[v] = reinterpret_cast<const h8*>(h)[i];
  }
#pragma unroll
  for (int v = 0; v < kVec; ++v) {
    const int64_t i = i0 + (int64_t)v * kEwThreads;
    if (i < n8) {
#pragma unroll
      for (int j = 0; j < 8; ++j) x[v][j] = silu1((float)x[v][j]);
      reinterpret_cast<h8*>(h)[i] = x[v];
    }
  }
}

__global__ void __launch_bounds__(kEwThreads) silu_scalar_kernel(_Float16* __restrict__ h, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kEwThreads + threadIdx.x;
  if (i >= n) return;
  h[i] = silu1((float)h[i]);
}

// ---- causal depthwise conv + LayerNorm + SiLU --------------------------------

struct DwParams {
  const _Float16* src;  // g [B*T, C] or h [B*T, 2C] (kGlu)
  const float* dwt;     // [K, C] taps
  const float* ln_w;
  const float* ln_b;
  _Float16* out;        // [B*T, C]
  float eps;
  int T, C;
  int vec8;             // C % 8 == 0 and src 16-byte aligned: 8-channel tile loads
};

using sidon::wave_sum;

// Sums v[t] over the block's threads for every t < BT (result in every
// thread).  red holds BT floats per wavefront.
template <int BT>
__device__ __forceinline__ void block_sums(float (&v)[BT], float* red, int nwaves) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int t = 0; t < BT; ++t) v[t] = wave_sum(v[t]);
  if (lane == 0) {
#pragma unroll
    for (int t = 0; t < BT; ++t) red[wave * BT + t] = v[t];
  }
  __syncthreads();
#pragma unroll
  for (int t = 0; t < BT; ++t) v[t] = 0.f;
  for (int w = 0; w < nwaves; ++w) {
#pragma unroll
    for (int t = 0; t < BT; ++t) v[t] += red[w * BT + t];
  }
  __syncthreads();  // red is reused by the next reduction
}

// One block: output frames [t0, t0 + BT) of one item, all C channels (tiles
// numbered item-major over a 1-D grid).
//   1. The block stages g of source frames t0 - (K - 1) .. t0 + BT - 1 in LDS
//      (fp16, zeros outside [0, T)), every thread loading whole 16-byte
//      chunks of four rows at a time from clamped (always valid) rows, so
//      the four rows' loads are in flight together.
//   2. Thread i owns channels 2i, 2i + 1: its 2 K taps and BT accumulator
//      pairs sit in registers; it walks the BT + K - 1 staged frames once,
//      adding frame j into output i through tap k = j - i, so every output
//      sums its taps in order k = 0 .. K-1.
//   3. LayerNorm over the C channels of the BT rows (two passes, block
//      reductions), SiLU, fp16 store.
template <int K, int BT, bool kGlu>
__global__ void __launch_bounds__(1024) causal_dw_norm_kernel(const DwParams p) {
  extern __shared__ __attribute__((aligned(16))) char dw_smem[];
  __shared__ float red[16 * BT];
  constexpr int kRows = BT + K - 1;
  _Float16* tile = reinterpret_cast<_Float16*>(dw_smem);  // [kRows][C]
  const int C = p.C;
  const int nthreads = blockDim.x;
  const int nwaves = nthreads >> 6;
  // Workgroups go to the 8 XCDs round-robin; give each XCD a contiguous run
  // of tiles, so the K - 1 frames a tile shares with its left neighbour are
  // usually in the same L2.
  const int ntiles = (p.T + BT - 1) / BT;
  const int nblk = gridDim.x;
  const int xcd = blockIdx.x % kXcds;
  const int tile_id = xcd * (nblk / kXcds) + min(xcd, nblk % kXcds) + blockIdx.x / kXcds;
  const int b = tile_id / ntiles;
  const int t0 = (tile_id - b * ntiles) * BT;
  const int s0 = t0 - (K - 1);
  const int64_t row0 = (int64_t)b * p.T;
  const int64_t src_stride = kGlu ? 2 * (int64_t)C : (int64_t)C;

  // 1. stage g
  {
    const int width = p.vec8 ? 8 : 2;          // channels per chunk
    const int cpr = C / width;                 // chunks per row
    const int rpp = nthreads / cpr;            // rows per pass (>= 1: C / 2 <= nthreads)
    const int r_first = threadIdx.x / cpr;
    const int cc = (threadIdx.x - r_first * cpr) * width;
    if (r_first < rpp) {
      // kStageRows rows per pass: the loads of all of them are issued before
      // any is used (rows past the tile repeat the last one and are not stored).
      for (int r = r_first; r < kRows; r += kStageRows * rpp) {
        if (p.vec8) {
          h8 a[kStageRows], gate[kStageRows];
#pragma unroll
          for (int u = 0; u < kStageRows; ++u) {
            const int sc = min(max(s0 + min(r + u * rpp, kRows - 1), 0), p.T - 1);
            const _Float16* src = p.src + (row0 + sc) * src_stride + cc;
            a[u] = *reinterpret_cast<const h8*>(src);
            if (kGlu) gate[u] = *reinterpret_cast<const h8*>(src + C);
          }
#pragma unroll
          for (int u = 0; u < kStageRows; ++u) {
            const int rr = r + u * rpp;
            if (rr < kRows) {
              const int s = s0 + rr;
              h8 g = a[u];
              if (kGlu) {
#pragma unroll
                for (int e = 0; e < 8; ++e) g[e] = glu1((float)a[u][e], (float)gate[u][e]);
              }
              if (s < 0 || s >= p.T) g = h8{};
              *reinterpret_cast<h8*>(tile + rr * C + cc) = g;
            }
          }
        } else {
          h2 a[kStageRows], gate[kStageRows];
#pragma unroll
          for (int u = 0; u < kStageRows; ++u) {
            const int sc = min(max(s0 + min(r + u * rpp, kRows - 1), 0), p.T - 1);
            const _Float16* src = p.src + (row0 + sc) * src_stride + cc;
            a[u] = *reinterpret_cast<const h2*>(src);
            if (kGlu) gate[u] = *reinterpret_cast<const h2*>(src + C);
          }
#pragma unroll
          for (int u = 0; u < kStageRows; ++u) {
            const int rr = r + u * rpp;
            if (rr < kRows) {
              const int s = s0 + rr;
              h2 g = a[u];
              if (kGlu) g = h2{glu1((float)a[u][0], (float)gate[u][0]), glu1((float)a[u][1], (float)gate[u][1])};
              if (s < 0 || s >= p.T) g = h2{};
              *reinterpret_cast<h2*>(tile + rr * C + cc) = g;
            }
          }
        }
      }
    }
  }
  __syncthreads();

  // 2. conv
  const int c = 2 * threadIdx.x;
  const bool on = c < C;  // threads past C hold zeros
  f2 w[K];
#pragma unroll
  for (int k = 0; k < K; ++k) w[k] = on ? *reinterpret_cast<const f2*>(p.dwt + (int64_t)k * C + c) : f2{0.f, 0.f};
  f2 acc[BT];
#pragma unroll
  for (int t = 0; t < BT; ++t) acc[t] = f2{0.f, 0.f};
  if (on) {
#pragma unroll
    for (int j = 0; j < kRows; ++j) {
      const h2 gh = *reinterpret_cast<const h2*>(tile + j * C + c);
      const f2 gv = {(float)gh[0], (float)gh[1]};
#pragma unroll
      for (int i = 0; i < BT; ++i) {
        const int k = j - i;
        if (k >= 0 && k < K) {
          acc[i][0] = fmaf(gv[0], w[k][0], acc[i][0]);
          acc[i][1] = fmaf(gv[1], w[k][1], acc[i][1]);
        }
      }
    }
  }

  // 3. LayerNorm over the C channels of every row (two passes), then SiLU.
  float v[BT];
#pragma unroll
  for (int t = 0; t < BT; ++t) v[t] = acc[t][0] + acc[t][1];
  block_sums<BT>(v, red, nwaves);
  const float inv_c = 1.f / (float)C;
#pragma unroll
  for (int t = 0; t < BT; ++t) {
    const float mean = v[t] * inv_c;
    acc[t][0] = on ? acc[t][0] - mean : 0.f;
    acc[t][1] = on ? acc[t][1] - mean : 0.f;
    v[t] = acc[t][0] * acc[t][0] + acc[t][1] * acc[t][1];
  }
  block_sums<BT>(v, red, nwaves);
  if (!on) return;
  const f2 lw = *reinterpret_cast<const f2*>(p.ln_w + c);
  const f2 lb = *reinterpret_cast<const f2*>(p.ln_b + c);
#pragma unroll
  for (int t = 0; t < BT; ++t) {
    if (t0 + t >= p.T) continue;
    const float rstd = rsqrtf(v[t] * inv_c + p.eps);
    const float y0 = acc[t][0] * rstd * lw[0] + lb[0];
    const float y1 = acc[t][1] * rstd * lw[1] + lb[1];
    *reinterpret_cast<h2*>(p.out + (row0 + t0 + t) * C + c) = h2{silu1(y0), silu1(y1)};
  }
}

constexpr int kLdsBudget = 160 * 1024;  // LDS of one CU

int dw_lds_bytes(int bt, int K, int C) { return (bt + K - 1) * C * 2; }

// Frames per block: the candidate that minimises (blocks per compute unit,
// rounded up) x (staged frames per block), within the LDS of one CU.  Blocks
// are counted per CU, not per resident slot: two blocks sharing a CU run no
// faster than one after the other (T = 1500, C = 1024: 376 blocks of 4
// frames, two per CU, take 15.9 us against 13.0 us for 188 blocks of 8).
int pick_bt(int K, int B, int T, int C) {
  static const int kCands[] = {20, 16, 8, 4};
  int best = 0;
  long best_cost = 0;
  const int cus = sidon::compute_units();
  for (int bt : kCands) {
    const int lds = dw_lds_bytes(bt, K, C) + 16 * bt * 4;
    if (lds > kLdsBudget) continue;
    const long blocks = (long)((T + bt - 1) / bt) * B;
    const long cost = ((blocks + cus - 1) / cus) * (bt + K - 1);
    if (best == 0 || cost < best_cost) {
      best = bt;
      best_cost = cost;
    }
  }
  return best;
}

template <int K, int BT>
hipError_t launch_dw_bt(const DwParams& p, int B, bool glu_input, int threads, hipStream_t stream) {
  const dim3 grid((unsigned)(((p.T + BT - 1) / BT) * B));
  const size_t lds = (size_t)dw_lds_bytes(BT, K, p.C);
  if (glu_input) {
    auto fn = causal_dw_norm_kernel<K, BT, true>;
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    hipLaunchKernelGGL(fn, grid, dim3(threads), lds, stream, p);
  } else {
    auto fn = causal_dw_norm_kernel<K, BT, false>;
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    hipLaunchKernelGGL(fn, grid, dim3(threads), lds, stream, p);
  }
  return hipGetLastError();
}

template <int K>
hipError_t launch_dw(const DwParams& p, int B, bool glu_input, hipStream_t stream) {
  const int threads = 64 * ((p.C / 2 + 63) / 64);
  switch (pick_bt(K, B, p.T, p.C)) {
    case 20: return launch_dw_bt<K, 20>(p, B, glu_input, threads, stream);
    case 16: return launch_dw_bt<K, 16>(p, B, glu_input, threads, stream);
    case 8: return launch_dw_bt<K, 8>(p, B, glu_input, threads, stream);
    case 4: return launch_dw_bt<K, 4>(p, B, glu_input, threads, stream);
    default: return hipErrorInvalidConfiguration;
  }
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace

SIDON_API int sidon_glu(const void* h, void* g, int R, int C, sidon_stream_t stream) {
  using sidon::fail;
  sidon::clear_error();
  if (!h || !g) return fail(SIDON_E_NULL, "h and g must be non-NULL");
  if (R < 1 || C < 1) return fail(SIDON_E_SHAPE, "R=%d and C=%d must be >= 1", R, C);
  if (!aligned(h, 2) || !aligned(g, 2)) return fail(SIDON_E_ALIGN, "fp16 tensors must be 2-byte aligned");
  int rc;
  if ((rc = sidon::check_device())) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const auto* hp = static_cast<const _Float16*>(h);
  auto* gp = static_cast<_Float16*>(g);
  if (C % 8 == 0 && aligned(h, 16) && aligned(g, 16)) {
    const int64_t n8 = (int64_t)R * (C / 8);
    const int64_t per_block = (int64_t)kEwThreads * kVec;
    hipLaunchKernelGGL(glu_vec_kernel, dim3((unsigned)((n8 + per_block - 1) / per_block)), dim3(kEwThreads), 0, s, hp,
                       gp, n8, C / 8);
  } else {
    const int64_t n = (int64_t)R * C;
    hipLaunchKernelGGL(glu_scalar_kernel, dim3((unsigned)((n + kEwThreads - 1) / kEwThreads)), dim3(kEwThreads), 0, s,
                       hp, gp, n, C);
  }
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(SIDON_E_LAUNCH, "glu launch failed: %s", hipGetErrorString(err));
  return SIDON_OK;
}

SIDON_API int sidon_silu(void* h, int64_t n, sidon_stream_t stream) {
  using sidon::fail;
  sidon::clear_error();
  if (!h) return fail(SIDON_E_NULL, "h must be non-NULL");
  if (n < 1) return fail(SIDON_E_SHAPE, "n=%lld must be >= 1", (long long)n);
  if (!aligned(h, 2)) return fail(SIDON_E_ALIGN, "fp16 tensors must be 2-byte aligned");
  int rc;
  if ((rc = sidon::check_device())) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  auto* hp = static_cast<_Float16*>(h);
  if (n % 8 == 0 && aligned(h, 16)) {
    const int64_t n8 = n / 8;
    const int64_t per_block = (int64_t)kEwThreads * kVec;
    hipLaunchKernelGGL(silu_vec_kernel, dim3((unsigned)((n8 + per_block - 1) / per_block)), dim3(kEwThreads), 0, s, hp,
                       n8);
  } else {
    hipLaunchKernelGGL(silu_scalar_kernel, dim3((unsigned)((n + kEwThreads - 1) / kEwThreads)), dim3(kEwThreads), 0, s,
                       hp, n);
  }
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(SIDON_E_LAUNCH, "silu launch failed: %s", hipGetErrorString(err));
  return SIDON_OK;
}

SIDON_API int sidon_causal_dw_norm(const void* src, int glu_input, const float* dwt, const float* ln_w,
                                   const float* ln_b, float eps, void* out, int B, int T, int C, int K,
                                   sidon_stream_t stream) {
  using sidon::fail;
  sidon::clear_error();
  if (!src || !dwt || !ln_w || !ln_b || !out) return fail(SIDON_E_NULL, "every pointer must be non-NULL");
  if (B < 1 || T < 1 || C < 2 || C > kMaxC || (C & 1) != 0)
    return fail(SIDON_E_SHAPE, "B=%d and T=%d must be >= 1 and C=%d even in [2, %d]", B, T, C, kMaxC);
  if (K != 3 && K != 7 && K != 15 && K != 31)
    return fail(SIDON_E_SHAPE, "K=%d: supported kernel sizes are 3, 7, 15 and 31", K);
  if ((int64_t)B * T > INT32_MAX / 2) return fail(SIDON_E_SHAPE, "B*T=%lld rows is too large", (long long)B * T);
  if (!aligned(src, 4) || !aligned(out, 4)) return fail(SIDON_E_ALIGN, "fp16 tensors must be 4-byte aligned");
  if (!aligned(dwt, 8) || !aligned(ln_w, 8) || !aligned(ln_b, 8))
    return fail(SIDON_E_ALIGN, "fp32 tensors must be 8-byte aligned");
  int rc;
  if ((rc = sidon::check_device())) return rc;
  const int vec8 = C % 8 == 0 && aligned(src, 16);
  const DwParams p{static_cast<const _Float16*>(src), dwt, ln_w, ln_b, static_cast<_Float16*>(out), eps, T, C, vec8};
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool g = glu_input != 0;
  hipError_t err;
  switch (K) {
    case 3: err = launch_dw<3>(p, B, g, s); break;
    case 7: err = launch_dw<7>(p, B, g, s); break;
    case 15: err = launch_dw<15>(p, B, g, s); break;
    default: err = launch_dw<31>(p, B, g, s); break;
  }
  if (err != hipSuccess) return fail(SIDON_E_LAUNCH, "causal_dw_norm launch failed: %s", hipGetErrorString(err));
  return SIDON_OK;
}
