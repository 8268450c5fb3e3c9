// fbank.hip -- the encoder's fbank front end around its framing GEMM
// (MI355X / gfx950).  The framing GEMM (frames [R, 400] x the [400, 514]
// DC-removal / pre-emphasis / window / rDFT matrix, fp32) runs on rocBLAS
// (sidon_gemm_nt, the kernel chosen by timing);
// these kernels do the rest of src/sidon_triton/frontend.py:218-240:
//
//   logmel     spec [R, 514] (re 257 | im 257) -> log(max(power . mel, 1.19e-7)) [R, 80]
//   normalize  per (item, mel bin) over the item's true frames:
//              (x - mean) / sqrt(var_ddof1 + 1e-7); the frame after an odd
//              count of true frames is 1.0; later frames 0.  [B, F, 80] is
//              also the stride-2 stacked [B, F / 2, 160] layout.
//
// logmel: 12 frames per block; their 257 powers go to LDS, then thread
// (m, lane) sums the nonzero span of mel triangle m (sparse: start bin,
// length, weights) for 4 of the frames, loading each weight once.
// normalize: statistics are per-tile two-pass sums (fixed tiles of frames,
// one block per (tile, item)), merged by a fixed pairwise tree, one block per (bin group, item) --
// deterministic, no atomics -- through a caller-provided workspace; a third
// kernel applies them to every frame.  frames: the edge padding and framing
// that feed the framing GEMM.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include <mutex>

#include "sidon_encoder.h"
#include "sidon_host.h"

#define SIDON_API extern "C" __attribute__((visibility("default")))

namespace {

constexpr int kBins = 257;
constexpr int kSpecWidth = 2 * kBins;
constexpr int kMel = 80;
constexpr int kFrameShift = 160;
constexpr int kFrameSize = 400;
constexpr int kEdgePad = 160;
constexpr float kMelFloor = 1.192092955078125e-07f;
constexpr float kVarEps = 1e-7f;
constexpr float kPadValue = 1.0f;
constexpr int kLmFrames = 12;        // logmel: frames per block
constexpr int kLmLanes = 3;          // logmel: threads per mel bin (each kLmFrames / kLmLanes frames)
constexpr int kLmThreads = 256;      // logmel: threads per block (kMel * kLmLanes = 240 sum)
constexpr int kLanes = 4;            // normalize: frame lanes x 80 bins per block
constexpr int kApplyFrames = 64;     // normalize: frames per apply block
constexpr int kMaxTiles = 64;
constexpr int kStatsCache = 40;      // statistics: frames per lane held in registers
constexpr int kMergeBins = 10;       // merge: mel bins per block (8 blocks per item)
constexpr int kMergeThreads = 320;   // merge: threads per block (32 tile pairs x 10 bins)

// frames[b, f, i] = chunk[b, 160 f + i - 160] (zero outside [0, S)): the
// (160, 160) edge padding and the 400 / 160 framing in one pass, 4 samples
// per thread.
// Block (x, item b): 256 of the item's F * 100 16-byte frame chunks; 32-bit
// index math within the item (F * 100 < 2^32; the division by 100 is a
// multiply).
__global__ void __launch_bounds__(256) frames_kernel(const float* __restrict__ chunk, float* __restrict__ frames,
                                                    int S, int F, bool vec4) {
  constexpr uint32_t kPerRow = kFrameSize / 4;  // 100 chunks of 4 samples
  const uint32_t q = blockIdx.x * 256u + threadIdx.x;
  if (q >= (uint32_t)F * kPerRow) return;
  const uint32_t f = q / kPerRow;
  const int i = (int)(q - f * kPerRow) * 4;     // 0, 4, ..., 396
  const int t0 = (int)f * kFrameShift + i - kEdgePad;
  const float* src = chunk + (int64_t)blockIdx.y * S;
  float4 v;
  if (t0 >= 0 && t0 + 3 < S && vec4) {
    v = *reinterpret_cast<const float4*>(src + t0);  // t0 % 4 == 0; rows 16-byte aligned
  } else {
    v.x = (t0 >= 0 && t0 < S) ? src[t0] : 0.f;
    v.y = (t0 + 1 >= 0 && t0 + 1 < S) ? src[t0 + 1] : 0.f;
    v.z = (t0 + 2 >= 0 && t0 + 2 < S) ? src[t0 + 2] : 0.f;
    v.w = (t0 + 3 >= 0 && t0 + 3 < S) ? src[t0 + 3] : 0.f;
  }
  *reinterpret_cast<float4*>(frames + ((int64_t)blockIdx.y * F + f) * kFrameSize + i) = v;
}

__global__ void __launch_bounds__(kLmThreads) logmel_kernel(const float* __restrict__ spec,
                                                          const float* __restrict__ mel_w,
                                                          const int* __restrict__ mel_lo,
                                                          const int* __restrict__ mel_len, int max_len,
                                                          float* __restrict__ out, int R) {
  __shared__ float power[kLmFrames][kBins + 3];
  const int f0 = blockIdx.x * kLmFrames;
  // Power spectra of the block's frames, every load of a thread in flight
  // together (consecutive threads read consecutive bins of a frame).
  {
    constexpr int kPer = (kLmFrames * kBins + kLmThreads - 1) / kLmThreads;
    float re[kPer], im[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int idx = threadIdx.x + kLmThreads * j;
      const int f = idx / kBins;
      const int k = idx - f * kBins;
      const bool ok = idx < kLmFrames * kBins && f0 + f < R;
      const float* row = spec + (int64_t)(f0 + f) * kSpecWidth;
      re[j] = ok ? row[k] : 0.f;
      im[j] = ok ? row[kBins + k] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int idx = threadIdx.x + kLmThreads * j;
      const int f = idx / kBins;
      if (idx < kLmFrames * kBins) power[f][idx - f * kBins] = re[j] * re[j] + im[j] * im[j];
    }
  }
  __syncthreads();
  // Thread (mel m, lane fl) sums frames fl, fl + kLmLanes, ...: each weight
  // is loaded once for kLmFrames / kLmLanes frames.  Every sum keeps the
  // order i = 0 .. n - 1.
  const int t = threadIdx.x;
  if (t >= kMel * kLmLanes) return;
  const int m = t % kMel;
  const int fl = t / kMel;
  const int lo = mel_lo[m];
  const int n = mel_len[m];
  const float* wm = mel_w + m * max_len;
  constexpr int kPerLane = kLmFrames / kLmLanes;
  float acc[kPerLane] = {};
#pragma unroll 4
  for (int i = 0; i < n; ++i) {
    const float wv = wm[i];
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) acc[j] = fmaf(wv, power[fl + kLmLanes * j][lo + i], acc[j]);
  }
#pragma unroll
  for (int j = 0; j < kPerLane; ++j) {
    const int r = f0 + fl + kLmLanes * j;
    if (r < R) out[(int64_t)r * kMel + m] = logf(fmaxf(acc[j], kMelFloor));
  }
}

// True frames of the exact-length extractor for `samples` valid samples:
// 1 + (samples + 2 * 160 - 400) / 160 (floor), clamped to [0, F].
__device__ __forceinline__ int true_frames(int samples, int F) {
  const int t = samples + 2 * kEdgePad - kFrameSize;
  const int n = t < 0 ? 0 : t / kFrameShift + 1;
  return min(n, F);
}

// Block (tile g, item b): two-pass sums over the true frames of tile g.
__global__ void __launch_bounds__(kLanes * kMel) stats_kernel(const float* __restrict__ x,
                                                             const int* __restrict__ valid,
                                                             float* __restrict__ part, int F, int G) {
  __shared__ float red[kLanes][kMel];
  const int b = blockIdx.y;
  const int g = blockIdx.x;
  const int m = threadIdx.x % kMel;
  const int fl = threadIdx.x / kMel;
  const int tf = true_frames(valid[b], F);
  const int per = (F + G - 1) / G;
  const int f0 = g * per;
  const int f1 = min(f0 + per, tf);
  const int n = max(f1 - f0, 0);
  const float* xb = x + (int64_t)b * F * kMel;
  // Tiles of up to kLanes * kStatsCache frames are held in registers, loaded
  // in one round (one memory latency for both passes); longer tiles stream.
  // Either way the sums run over f = f0 + fl, f0 + fl + kLanes, ... in order.
  const int nl = f1 > f0 + fl ? (f1 - f0 - fl + kLanes - 1) / kLanes : 0;
  float xv[kStatsCache];
  const bool cached = nl <= kStatsCache;
  if (cached) {
#pragma unroll
    for (int j = 0; j < kStatsCache; ++j) xv[j] = j < nl ? xb[(int64_t)(f0 + fl + kLanes * j) * kMel + m] : 0.f;
  }
  float s = 0.f;
  if (cached) {
#pragma unroll
    for (int j = 0; j < kStatsCache; ++j)
      if (j < nl) s += xv[j];
  } else {
#pragma unroll 8
    for (int f = f0 + fl; f < f1; f += kLanes) s += xb[(int64_t)f * kMel + m];
  }
  red[fl][m] = s;
  __syncthreads();
  const float mean = n > 0 ? ((red[0][m] + red[1][m]) + (red[2][m] + red[3][m])) / (float)n : 0.f;
  __syncthreads();
  float q = 0.f;
  if (cached) {
#pragma unroll
    for (int j = 0; j < kStatsCache; ++j) {
      if (j < nl) {
        const float d = xv[j] - mean;
        q = fmaf(d, d, q);
      }
    }
  } else {
#pragma unroll 8
    for (int f = f0 + fl; f < f1; f += kLanes) {
      const float d = xb[(int64_t)f * kMel + m] - mean;
      q = fmaf(d, d, q);
    }
  }
  red[fl][m] = q;
  __syncthreads();
  if (fl == 0) {
    float* dst = part + (((int64_t)b * G + g) * kMel + m) * 3;
    dst[0] = (float)n;
    dst[1] = mean;
    dst[2] = (red[0][m] + red[1][m]) + (red[2][m] + red[3][m]);
  }
}

// Block (bin group, item b): merge item b's tile sums of kMergeBins bins by
// a fixed pairwise tree (Chan et al.'s update of count, mean and sum of
// squared deviations) in LDS; writes (mean, sqrt(var + eps)) per bin after
// the partials.
__global__ void __launch_bounds__(kMergeThreads) merge_kernel(const int* __restrict__ valid, float* __restrict__ part,
                                                             int F, int G, int B) {
  constexpr int kVals = kMergeBins * 3;  // floats per tile of this group
  __shared__ float sp[kMaxTiles * kVals];
  const int b = blockIdx.y;
  const int m0 = blockIdx.x * kMergeBins;
  const float* src = part + (int64_t)b * G * kMel * 3 + m0 * 3;
  // The group's partials into LDS, every load in flight at once (one memory
  // latency): tile g's kVals floats sit at src + g * kMel * 3.
  {
    constexpr int kPer = (kMaxTiles * kVals + kMergeThreads - 1) / kMergeThreads;
    float v[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = threadIdx.x + kMergeThreads * j;
      const int g = i / kVals;
      v[j] = g < G ? src[(int64_t)g * kMel * 3 + (i - g * kVals)] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = threadIdx.x + kMergeThreads * j;
      if (i / kVals < G) sp[i] = v[j];
    }
  }
  __syncthreads();
  // Pairwise tree over the tiles, the same for every call (deterministic):
  // level l merges tile g + 2^l into tile g for g a multiple of 2^(l+1).
  for (int stride = 1; stride < G; stride *= 2) {
    const int pairs = (G + 2 * stride - 1) / (2 * stride);
    for (int t = threadIdx.x; t < pairs * kMergeBins; t += kMergeThreads) {
      const int mm = t % kMergeBins;
      const int g = (t / kMergeBins) * 2 * stride;
      if (g + stride < G) {
        float* a = sp + g * kVals + mm * 3;
        const float* c = sp + (g + stride) * kVals + mm * 3;
        const float na = a[0], nb = c[0];
        if (nb > 0.f) {
          if (na <= 0.f) {
            a[0] = nb;
            a[1] = c[1];
            a[2] = c[2];
          } else {
            const float nt = na + nb;
            const float d = c[1] - a[1];
            a[1] += d * (nb / nt);
            a[2] += c[2] + d * d * (na * nb / nt);
            a[0] = nt;
          }
        }
      }
    }
    __syncthreads();
  }
  const int mm = threadIdx.x;
  if (mm >= kMergeBins) return;
  const int tf = true_frames(valid[b], F);
  const float mean = sp[mm * 3 + 1];
  const float m2 = sp[mm * 3 + 2];
  float* stats = part + (int64_t)B * G * kMel * 3 + ((int64_t)b * kMel + m0 + mm) * 2;
  stats[0] = mean;
  stats[1] = sqrtf(m2 / (float)(tf - 1) + kVarEps);
}

// Block (frame range, item b): normalize the range's frames.
__global__ void __launch_bounds__(kLanes * kMel) apply_kernel(const float* __restrict__ x,
                                                             const int* __restrict__ valid,
                                                             const float* __restrict__ part,
                                                             float* __restrict__ out, int F, int G, int B) {
  const int b = blockIdx.y;
  const int m = threadIdx.x % kMel;
  const int fl = threadIdx.x / kMel;
  const int tf = true_frames(valid[b], F);
  const float* stats = part + (int64_t)B * G * kMel * 3 + ((int64_t)b * kMel + m) * 2;
  const float mean = stats[0];
  const float denom = stats[1];
  const float* xb = x + (int64_t)b * F * kMel;
  float* ob = out + (int64_t)b * F * kMel;
  const int fbase = blockIdx.x * kApplyFrames;
  // All of the thread's loads first (one memory latency), then the stores.
  constexpr int kPer = kApplyFrames / kLanes;
  float x_in[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int f = fbase + fl + kLanes * j;
    x_in[j] = f < tf ? xb[(int64_t)f * kMel + m] : 0.f;  // tf <= F
  }
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int f = fbase + fl + kLanes * j;
    if (f < F) {
      const float v = f < tf ? (x_in[j] - mean) / denom : ((f == tf && (tf & 1)) ? kPadValue : 0.f);
      ob[(int64_t)f * kMel + m] = v;
    }
  }
}

int tiles_for(int F) { return F / 128 < 1 ? 1 : (F / 128 > kMaxTiles ? kMaxTiles : F / 128); }

// Scratch of sidon_fbank_normalize_noalloc: the normalize workspace of up
// to kScratchItems items of any length (tiles_for() caps the tiles at
// kMaxTiles), 1.9 MiB in all, one copy per device for the life of the
// process.  Every word a call reads was written earlier in the same call, so
// nothing needs clearing between calls.
constexpr int kScratchItems = 32;
constexpr size_t kScratchFloats = (size_t)kScratchItems * (kMaxTiles * kMel * 3 + kMel * 2);
static __device__ __align__(256) float scratch[kScratchFloats];

// Device address of `scratch` per device, taken once per device with that
// device current (host code must never pass the symbol itself to a kernel).
constexpr int kMaxDevices = 64;
std::once_flag g_scratch_once[kMaxDevices];
float* g_scratch[kMaxDevices] = {};
hipError_t g_scratch_err[kMaxDevices] = {};

int normalize_launch(const float* logmel, const int* valid, float* workspace, float* feats, int B, int F,
                     hipStream_t s) {
  using sidon::fail;
  const int G = tiles_for(F);
  hipLaunchKernelGGL(stats_kernel, dim3(G, B), dim3(kLanes * kMel), 0, s, logmel, valid, workspace, F, G);
  hipError_t err = hipGetLastError();
  if (err == hipSuccess) {
    hipLaunchKernelGGL(merge_kernel, dim3(kMel / kMergeBins, B), dim3(kMergeThreads), 0, s, valid, workspace, F, G, B);
    err = hipGetLastError();
  }
  if (err == hipSuccess) {
    hipLaunchKernelGGL(apply_kernel, dim3((F + kApplyFrames - 1) / kApplyFrames, B), dim3(kLanes * kMel), 0, s,
                       logmel, valid, workspace, feats, F, G, B);
    err = hipGetLastError();
  }
  if (err != hipSuccess) return fail(SIDON_E_LAUNCH, "fbank normalize launch failed: %s", hipGetErrorString(err));
  return SIDON_OK;
}

}  // namespace

SIDON_API int sidon_fbank_logmel(const float* spec, const float* mel_w, const int* mel_lo, const int* mel_len,
                                 int max_len, float* logmel, int R, sidon_stream_t stream) {
  using sidon::fail;
  sidon::clear_error();
  if (!spec || !mel_w || !mel_lo || !mel_len || !logmel) return fail(SIDON_E_NULL, "every pointer must be non-NULL");
  if (R < 1 || max_len < 1 || max_len > kBins) return fail(SIDON_E_SHAPE, "R=%d must be >= 1 and max_len=%d in [1, %d]", R, max_len, kBins);
  int rc;
  if ((rc = sidon::check_device())) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(logmel_kernel, dim3((unsigned)((R + kLmFrames - 1) / kLmFrames)), dim3(kLmThreads), 0, s, spec,
                     mel_w, mel_lo, mel_len, max_len, logmel, R);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(SIDON_E_LAUNCH, "fbank logmel launch failed: %s", hipGetErrorString(err));
  return SIDON_OK;
}

SIDON_API int sidon_fbank_frames(const float* chunk, float* frames, int B, int S, sidon_stream_t stream) {
  using sidon::fail;
  sidon::clear_error();
  if (!chunk || !frames) return fail(SIDON_E_NULL, "chunk and frames must be non-NULL");
  if (B < 1 || S < 2 * kFrameShift || S % (2 * kFrameShift) != 0)
    return fail(SIDON_E_SHAPE, "B=%d must be >= 1 and S=%d a positive multiple of %d", B, S, 2 * kFrameShift);
  if (!sidon::aligned16(frames)) return fail(SIDON_E_ALIGN, "frames must be 16-byte aligned");
  int rc;
  if ((rc = sidon::check_device())) return rc;
  const int F = S / kFrameShift;
  // 16-byte source loads when every item's row starts 16-byte aligned (S is a
  // multiple of 320, so that holds when the chunk pointer is aligned).
  const bool vec4 = sidon::aligned16(chunk);
  const unsigned blocks = (unsigned)(((int64_t)F * (kFrameSize / 4) + 255) / 256);
  for (int b0 = 0; b0 < B; b0 += 65535) {  // items on grid y, at most 65535 per launch
    const int nb = B - b0 < 65535 ? B - b0 : 65535;
    hipLaunchKernelGGL(frames_kernel, dim3(blocks, (unsigned)nb), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       chunk + (int64_t)b0 * S, frames + (int64_t)b0 * F * kFrameSize, S, F, vec4);
  }
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(SIDON_E_LAUNCH, "fbank frames launch failed: %s", hipGetErrorString(err));
  return SIDON_OK;
}

SIDON_API size_t sidon_fbank_workspace_bytes(int B, int F) {
  if (B < 1 || F < 1) return 0;
  return (size_t)B * (tiles_for(F) * kMel * 3 + kMel * 2) * sizeof(float);
}

SIDON_API int sidon_fbank_normalize(const float* logmel, const int* valid, float* workspace, size_t workspace_bytes,
                                    float* feats, int B, int F, sidon_stream_t stream) {
  using sidon::fail;
  sidon::clear_error();
  if (!logmel || !valid || !workspace || !feats) return fail(SIDON_E_NULL, "every pointer must be non-NULL");
  if (B < 1 || F < 2 || (F & 1) != 0) return fail(SIDON_E_SHAPE, "B=%d must be >= 1 and F=%d even and >= 2", B, F);
  if (workspace_bytes < sidon_fbank_workspace_bytes(B, F))
    return fail(SIDON_E_SHAPE, "workspace of %zu bytes is smaller than the %zu needed", workspace_bytes,
                sidon_fbank_workspace_bytes(B, F));
  if (logmel == feats) return fail(SIDON_E_SHAPE, "feats must not alias logmel");
  int rc;
  if ((rc = sidon::check_device())) return rc;
  return normalize_launch(logmel, valid, workspace, feats, B, F, reinterpret_cast<hipStream_t>(stream));
}

SIDON_API int sidon_fbank_normalize_noalloc(const float* logmel, const int* valid, float* feats, int B, int F,
                                            sidon_stream_t stream) {
  using sidon::fail;
  sidon::clear_error();
  if (!logmel || !valid || !feats) return fail(SIDON_E_NULL, "every pointer must be non-NULL");
  if (B < 1 || F < 2 || (F & 1) != 0) return fail(SIDON_E_SHAPE, "B=%d must be >= 1 and F=%d even and >= 2", B, F);
  if (B > kScratchItems || sidon_fbank_workspace_bytes(B, F) > sizeof(scratch))
    return fail(SIDON_E_SHAPE, "B=%d items exceed the %d the static scratch holds (use sidon_fbank_normalize)", B,
                kScratchItems);
  if (logmel == feats) return fail(SIDON_E_SHAPE, "feats must not alias logmel");
  int rc;
  if ((rc = sidon::check_device())) return rc;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(SIDON_E_DEVICE, "no usable HIP device");
  std::call_once(g_scratch_once[dev], [dev]() {
    void* ptr = nullptr;
    g_scratch_err[dev] = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    g_scratch[dev] = g_scratch_err[dev] == hipSuccess ? static_cast<float*>(ptr) : nullptr;
  });
  if (g_scratch[dev] == nullptr)
    return fail(SIDON_E_DEVICE, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                hipGetErrorString(g_scratch_err[dev]));
  return normalize_launch(logmel, valid, g_scratch[dev], feats, B, F, reinterpret_cast<hipStream_t>(stream));
}
