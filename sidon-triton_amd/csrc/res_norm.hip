// res_norm.hip -- residual add + LayerNorm rows of the encoder's fp32 stream
// (MI355X / gfx950).
//
// For every row r of x [R, C] fp32 (in place):
//
//   x_r  = x_r + bias + y_r            (each term optional)
//   x_r  = LN1(x_r)                    (optional)
//   store x_r                          (optional)
//   xn_r = LN2(x_r) -> fp16 or fp32    (optional)
//
// with LN(v) = (v - mean(v)) / sqrt(var(v) + eps) * w + b over the C columns
// (two-pass mean and variance in fp32).  This is _res_norm_kernel /
// res_norm of src/sidon_triton/triton_encoder.py:61-100, the op that feeds
// the fused QKV GEMM of the attention sub-block and takes the running bias of
// the accumulating residual GEMMs (:438-443, :491-503).
//
// One wavefront per row: lane l holds columns 4 (l + 64 j), j < NC, as
// 16-byte vectors, so every load and store instruction of a wavefront covers
// 1 KB of contiguous row.  The op streams HBM: 4 C bytes read (plus 4 C if
// y) and 2 C or 4 C bytes written per row.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "sidon_encoder.h"
#include "sidon_host.h"
#include "sidon_wave.h"

#define SIDON_API extern "C" __attribute__((visibility("default")))

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));

constexpr int kRowsPerBlock = 4;  // one wavefront per row
constexpr int kMaxChunks = 8;     // C <= 64 * 4 * 8 = 2048

struct RNParams {
  float* x;
  const float* y;
  const float* bias;
  const float* n1_w;
  const float* n1_b;
  const float* n2_w;
  const float* n2_b;
  void* xn;
  float eps1, eps2;
  int R, C;
  int write_x, xn_fp16;
};

using sidon::wave_sum;

// v <- LN(v) over the row (chunks past C hold 0 and stay 0; full: C == 256 NC).
template <int NC>
__device__ __forceinline__ void layer_norm(f4 (&v)[NC], int lane, int C, const float* w, const float* b,
                                           float eps, bool full) {
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NC; ++j) s += (v[j][0] + v[j][1]) + (v[j][2] + v[j][3]);
  const float mean = wave_sum(s) / (float)C;
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = 4 * (lane + 64 * j);
    if (full || c < C) {
      v[j] -= mean;
      q += (v[j][0] * v[j][0] + v[j][1] * v[j][1]) + (v[j][2] * v[j][2] + v[j][3] * v[j][3]);
    }
  }
  const float rstd = rsqrtf(wave_sum(q) / (float)C + eps);
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = 4 * (lane + 64 * j);
    if (full || c < C) {
      const f4 wv = *reinterpret_cast<const f4*>(w + c);
      const f4 bv = *reinterpret_cast<const f4*>(b + c);
      v[j] = v[j] * rstd * wv + bv;
    }
  }
}

// Mode bits: a kernel instantiated with kMode >= 0 has its options fixed at
// compile time (no per-element branches, loads hoisted freely); kMode = -1
// reads them from the parameters.
constexpr int kY = 1, kBias = 2, kNorm1 = 4, kWriteX = 8, kNorm2 = 16, kFp16 = 32, kFull = 64;
constexpr int kModeBiasNorm = kBias | kNorm2 | kFp16 | kFull;                     // x + b -> LN2 (fp16)
constexpr int kModeFinal = kBias | kNorm1 | kWriteX | kNorm2 | kFp16 | kFull;     // x = LN1(x + b) -> LN2

template <int NC, int kMode>
__global__ void __launch_bounds__(64 * kRowsPerBlock) res_norm_kernel(const RNParams p) {
  constexpr bool kFixed = kMode >= 0;
  const bool has_y = kFixed ? (kMode & kY) != 0 : p.y != nullptr;
  const bool has_bias = kFixed ? (kMode & kBias) != 0 : p.bias != nullptr;
  const bool norm1 = kFixed ? (kMode & kNorm1) != 0 : p.n1_w != nullptr;
  const bool write_x = kFixed ? (kMode & kWriteX) != 0 : p.write_x != 0;
  const bool norm2 = kFixed ? (kMode & kNorm2) != 0 : p.n2_w != nullptr;
  const bool fp16 = kFixed ? (kMode & kFp16) != 0 : p.xn_fp16 != 0;
  const bool full = kFixed && (kMode & kFull) != 0;  // C == 256 NC: every chunk in range
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= p.R) return;
  const size_t base = (size_t)row * p.C;
  f4 v[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = 4 * (lane + 64 * j);
    v[j] = f4{0.f, 0.f, 0.f, 0.f};
    if (full || c < p.C) {
      v[j] = *reinterpret_cast<const f4*>(p.x + base + c);
      if (has_bias) v[j] += *reinterpret_cast<const f4*>(p.bias + c);
      if (has_y) v[j] += *reinterpret_cast<const f4*>(p.y + base + c);
    }
  }
  if (norm1) layer_norm<NC>(v, lane, p.C, p.n1_w, p.n1_b, p.eps1, full);
  if (write_x) {
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int c = 4 * (lane + 64 * j);
      if (full || c < p.C) *reinterpret_cast<f4*>(p.x + base + c) = v[j];
    }
  }
  if (norm2) {
    layer_norm<NC>(v, lane, p.C, p.n2_w, p.n2_b, p.eps2, full);
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int c = 4 * (lane + 64 * j);
      if (full || c < p.C) {
        if (fp16) {
          *reinterpret_cast<h4*>(static_cast<_Float16*>(p.xn) + base + c) = __builtin_convertvector(v[j], h4);
        } else {
          *reinterpret_cast<f4*>(static_cast<float*>(p.xn) + base + c) = v[j];
        }
      }
    }
  }
}

template <int NC>
hipError_t launch(const RNParams& p, hipStream_t stream) {
  const int blocks = (p.R + kRowsPerBlock - 1) / kRowsPerBlock;
  const int mode = (p.y ? kY : 0) | (p.bias ? kBias : 0) | (p.n1_w ? kNorm1 : 0) | (p.write_x ? kWriteX : 0) |
                   (p.n2_w ? kNorm2 : 0) | (p.xn_fp16 ? kFp16 : 0) | (p.C == 256 * NC ? kFull : 0);
  if (mode == kModeBiasNorm) {
    hipLaunchKernelGGL((res_norm_kernel<NC, kModeBiasNorm>), dim3(blocks), dim3(64 * kRowsPerBlock), 0, stream, p);
  } else if (mode == kModeFinal) {
    hipLaunchKernelGGL((res_norm_kernel<NC, kModeFinal>), dim3(blocks), dim3(64 * kRowsPerBlock), 0, stream, p);
  } else {
    hipLaunchKernelGGL((res_norm_kernel<NC, -1>), dim3(blocks), dim3(64 * kRowsPerBlock), 0, stream, p);
  }
  return hipGetLastError();
}

}  // namespace

SIDON_API int sidon_res_norm(float* x, const float* y, const float* bias, const float* n1_w,
                             const float* n1_b, float eps1, int write_x, const float* n2_w,
                             const float* n2_b, float eps2, void* xn, int xn_fp16, int R, int C,
                             sidon_stream_t stream) {
  using sidon::aligned16;
  using sidon::fail;
  sidon::clear_error();
  if (!x) return fail(SIDON_E_NULL, "x must be non-NULL");
  if ((n1_w == nullptr) != (n1_b == nullptr)) return fail(SIDON_E_NULL, "norm1 needs both weight and bias");
  if ((n2_w == nullptr) != (n2_b == nullptr)) return fail(SIDON_E_NULL, "norm2 needs both weight and bias");
  if (n2_w && !xn) return fail(SIDON_E_NULL, "norm2 needs an xn output");
  if (R < 1 || C < 4 || C > 64 * 4 * kMaxChunks || (C & 3) != 0)
    return fail(SIDON_E_SHAPE, "R=%d must be >= 1 and C=%d a multiple of 4 in [4, %d]", R, C,
                64 * 4 * kMaxChunks);
  const void* ptrs[] = {x, y, bias, n1_w, n1_b, n2_w, n2_b};
  for (const void* ptr : ptrs)
    if (ptr && !aligned16(ptr)) return fail(SIDON_E_ALIGN, "fp32 tensors must be 16-byte aligned");
  if (xn && (reinterpret_cast<uintptr_t>(xn) & (xn_fp16 ? 7u : 15u)) != 0)
    return fail(SIDON_E_ALIGN, "xn must be %d-byte aligned", xn_fp16 ? 8 : 16);
  int rc;
  if ((rc = sidon::check_device())) return rc;
  RNParams p{x, y, bias, n1_w, n1_b, n2_w, n2_b, xn, eps1, eps2, R, C, write_x != 0, xn_fp16 != 0};
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int nc = (C + 255) / 256;
  hipError_t err;
  switch (nc) {
    case 1: err = launch<1>(p, s); break;
    case 2: err = launch<2>(p, s); break;
    case 3: err = launch<3>(p, s); break;
    case 4: err = launch<4>(p, s); break;
    case 5: err = launch<5>(p, s); break;
    case 6: err = launch<6>(p, s); break;
    case 7: err = launch<7>(p, s); break;
    default: err = launch<8>(p, s); break;
  }
  if (err != hipSuccess) return fail(SIDON_E_LAUNCH, "res_norm launch failed: %s", hipGetErrorString(err));
  return SIDON_OK;
}
