// conformer_ops.hip -- the conformer layer's elementwise and convolution
// kernels around its GEMMs (MI355X / gfx950):
//
//   glu              g = h[:, :C] * sigmoid(h[:, C:])                  fp16 -> fp16
//   silu (in place)  h = h * sigmoid(h)                                 fp16
//   causal_dw_norm   out[t] = silu(LN(sum_k w[k] * g[t + k - (K-1)]))   fp16 -> fp16
//
// They replace _glu_kernel / glu and _causal_dw_norm_kernel / causal_dw_norm
// of src/sidon_triton/triton_encoder.py:113-181, and the in-place F.silu of
// the feed-forward modules (:485-486, :505-506).  causal_dw_norm can also read
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

#include "sidon_encoder.h"
#include "sidon_host.h"

#define SIDON_API extern "C" __attribute__((visibility("default")))

namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef float f8 __attribute__((ext_vector_type(8)));

constexpr int kBT = 16;          // output frames per causal_dw_norm block
constexpr int kMaxC = 2048;      // channels: one thread per pair, <= 1024 threads
constexpr int kEwThreads = 256;  // glu / silu block size

__device__ __forceinline__ float sigmoid(float x) { return 1.f / (1.f + __expf(-x)); }

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

// 8 columns per thread; requires C % 8 == 0 and 16-byte aligned rows.
__global__ void __launch_bounds__(kEwThreads) glu_vec_kernel(const _Float16* __restrict__ h, _Float16* __restrict__ g,
                                                             int64_t n8, int c8) {
  const int64_t i = (int64_t)blockIdx.x * kEwThreads + threadIdx.x;
  if (i >= n8) return;
  const int64_t row = i / c8;
  const int64_t col = i - row * c8;
  const h8 a = reinterpret_cast<const h8*>(h)[row * 2 * c8 + col];
  const h8 b = reinterpret_cast<const h8*>(h)[row * 2 * c8 + c8 + col];
  h8 o;
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = glu1((float)a[j], (float)b[j]);
  reinterpret_cast<h8*>(g)[i] = o;
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
  const int64_t i = (int64_t)blockIdx.x * kEwThreads + threadIdx.x;
  if (i >= n8) return;
  h8 v = reinterpret_cast<h8*>(h)[i];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    v[j] = silu1((float)v[j]);
  }
  reinterpret_cast<h8*>(h)[i] = v;
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
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Sums v[t] over the block's threads for every t < kBT (result in every
// thread).  red holds kBT floats per wavefront.
__device__ __forceinline__ void block_sums(float (&v)[kBT], float* red, int nwaves) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int t = 0; t < kBT; ++t) v[t] = wave_sum(v[t]);
  if (lane == 0) {
#pragma unroll
    for (int t = 0; t < kBT; ++t) red[wave * kBT + t] = v[t];
  }
  __syncthreads();
#pragma unroll
  for (int t = 0; t < kBT; ++t) v[t] = 0.f;
  for (int w = 0; w < nwaves; ++w) {
#pragma unroll
    for (int t = 0; t < kBT; ++t) v[t] += red[w * kBT + t];
  }
  __syncthreads();  // red is reused by the next reduction
}

template <int K, bool kGlu>
__global__ void __launch_bounds__(1024) causal_dw_norm_kernel(const DwParams p) {
  __shared__ float red[16 * kBT];
  const int nwaves = blockDim.x >> 6;
  const int b = blockIdx.y;
  const int t0 = blockIdx.x * kBT;
  const int c = 2 * threadIdx.x;
  const bool on = c < p.C;  // threads past C hold zeros
  const int64_t row0 = (int64_t)b * p.T;
  const int64_t src_stride = kGlu ? 2 * (int64_t)p.C : (int64_t)p.C;

  f2 w[K];
#pragma unroll
  for (int k = 0; k < K; ++k) w[k] = on ? *reinterpret_cast<const f2*>(p.dwt + (int64_t)k * p.C + c) : f2{0.f, 0.f};

  f2 acc[kBT];
#pragma unroll
  for (int t = 0; t < kBT; ++t) acc[t] = f2{0.f, 0.f};

  // Source frame s = t0 + j - (K - 1) = (t0 + i) + k - (K - 1) feeds output
  // frame t0 + i through tap k = j - i, for i in [j - (K - 1), j].
#pragma unroll
  for (int j = 0; j < kBT + K - 1; ++j) {
    const int s = t0 + j - (K - 1);
    f2 gv = {0.f, 0.f};
    if (on && s >= 0 && s < p.T) {
      const _Float16* srow = p.src + (row0 + s) * src_stride + c;
      const h2 a = *reinterpret_cast<const h2*>(srow);
      if (kGlu) {
        const h2 gate = *reinterpret_cast<const h2*>(srow + p.C);
        gv = f2{(float)glu1((float)a[0], (float)gate[0]), (float)glu1((float)a[1], (float)gate[1])};
      } else {
        gv = f2{(float)a[0], (float)a[1]};
      }
    }
#pragma unroll
    for (int i = 0; i < kBT; ++i) {
      const int k = j - i;
      if (k >= 0 && k < K) {
        acc[i][0] = fmaf(gv[0], w[k][0], acc[i][0]);
        acc[i][1] = fmaf(gv[1], w[k][1], acc[i][1]);
      }
    }
  }

  // LayerNorm over the C channels of every row (two passes), then SiLU.
  float v[kBT];
#pragma unroll
  for (int t = 0; t < kBT; ++t) v[t] = acc[t][0] + acc[t][1];
  block_sums(v, red, nwaves);
  const float inv_c = 1.f / (float)p.C;
#pragma unroll
  for (int t = 0; t < kBT; ++t) {
    const float mean = v[t] * inv_c;
    acc[t][0] = on ? acc[t][0] - mean : 0.f;
    acc[t][1] = on ? acc[t][1] - mean : 0.f;
    v[t] = acc[t][0] * acc[t][0] + acc[t][1] * acc[t][1];
  }
  block_sums(v, red, nwaves);
  if (!on) return;
  const f2 lw = *reinterpret_cast<const f2*>(p.ln_w + c);
  const f2 lb = *reinterpret_cast<const f2*>(p.ln_b + c);
#pragma unroll
  for (int t = 0; t < kBT; ++t) {
    if (t0 + t >= p.T) continue;
    const float rstd = rsqrtf(v[t] * inv_c + p.eps);
    float y0 = acc[t][0] * rstd * lw[0] + lb[0];
    float y1 = acc[t][1] * rstd * lw[1] + lb[1];
    y0 = y0 * sigmoid(y0);
    y1 = y1 * sigmoid(y1);
    *reinterpret_cast<h2*>(p.out + (row0 + t0 + t) * p.C + c) = h2{(_Float16)y0, (_Float16)y1};
  }
}

template <int K>
hipError_t launch_dw(const DwParams& p, int B, bool glu_input, hipStream_t stream) {
  const int threads = 64 * ((p.C / 2 + 63) / 64);
  const dim3 grid((p.T + kBT - 1) / kBT, B);
  if (glu_input) {
    hipLaunchKernelGGL((causal_dw_norm_kernel<K, true>), grid, dim3(threads), 0, stream, p);
  } else {
    hipLaunchKernelGGL((causal_dw_norm_kernel<K, false>), grid, dim3(threads), 0, stream, p);
  }
  return hipGetLastError();
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
    hipLaunchKernelGGL(glu_vec_kernel, dim3((unsigned)((n8 + kEwThreads - 1) / kEwThreads)), dim3(kEwThreads), 0, s, hp,
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
    hipLaunchKernelGGL(silu_vec_kernel, dim3((unsigned)((n8 + kEwThreads - 1) / kEwThreads)), dim3(kEwThreads), 0, s, hp,
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
  const DwParams p{static_cast<const _Float16*>(src), dwt, ln_w, ln_b, static_cast<_Float16*>(out), eps, T, C};
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
