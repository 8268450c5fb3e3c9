// blaslt.hip -- library GEMMs with a fused activation on hipBLASLt:
//
//   y[m, n] = act(x[m, :] . w[n, :] + bias[n])     act: 1 = SiLU, 0 = none
//
// x [M, K] and w [N, K] fp16, row-major and K-contiguous; fp32 sums; y [M, N]
// fp16.  The bias and the SiLU run in hipBLASLt's epilogue
// (HIPBLASLT_EPILOGUE_SWISH_BIAS_EXT: bias added to the fp32 sum, x *
// sigmoid(x) in fp32, one rounding to fp16), so the SiLU of the feed-forward
// input projection costs no pass of its own.  In hipBLASLt's column-major
// terms this is y^T = op(w) . x^T with op = transpose, the bias one value per
// row of y^T.
//
// The kernel is hipBLASLt's first heuristic choice for the problem with no
// workspace (no split-K partials: a call shares no memory with other calls
// and its sums are always taken in the same order), looked up once per
// problem and kept.  The first call of a device creates its handle, so it
// must not run during stream capture.

#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <climits>
#include <map>
#include <mutex>
#include <tuple>

#include "sidon_encoder.h"
#include "sidon_host.h"

#define SIDON_API extern "C" __attribute__((visibility("default")))

namespace {

using sidon::fail;

constexpr int kMaxDevices = 64;

// One problem: the descriptor (epilogue, transposes), the layouts and the
// chosen algorithm.  The bias pointer is set on the descriptor per call.
struct Plan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
  hipblasLtMatmulAlgo_t algo{};
};

using Key = std::tuple<int, int, int, int, int, int, int, int, bool>;

std::mutex g_mu;  // guards the handles, the plans and the descriptors' bias pointers
hipblasLtHandle_t g_handle[kMaxDevices] = {};
std::map<Key, Plan> g_plans;

void destroy(Plan& p) {
  if (p.a) hipblasLtMatrixLayoutDestroy(p.a);
  if (p.b) hipblasLtMatrixLayoutDestroy(p.b);
  if (p.c) hipblasLtMatrixLayoutDestroy(p.c);
  if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
  p = Plan{};
}

// Called with g_mu held.
int plan_for(int dev, const Key& key, int M, int N, int K, int ldx, int ldw, int ldy, int act, bool has_bias,
             Plan** out) {
  if (g_handle[dev] == nullptr) {
    hipblasLtHandle_t h = nullptr;
    if (hipblasLtCreate(&h) != HIPBLAS_STATUS_SUCCESS)
      return fail(SIDON_E_LAUNCH, "hipblasLtCreate failed on device %d", dev);
    g_handle[dev] = h;
  }
  auto it = g_plans.find(key);
  if (it != g_plans.end()) {
    *out = &it->second;
    return SIDON_OK;
  }
  Plan p;
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  const hipblasLtEpilogue_t epi = act ? (has_bias ? HIPBLASLT_EPILOGUE_SWISH_BIAS_EXT : HIPBLASLT_EPILOGUE_SWISH_EXT)
                                      : (has_bias ? HIPBLASLT_EPILOGUE_BIAS : HIPBLASLT_EPILOGUE_DEFAULT);
  const hipDataType bias_type = HIP_R_16F;
  bool ok = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) ==
                 HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) ==
                 HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi)) ==
                 HIPBLAS_STATUS_SUCCESS;
  if (has_bias)
    ok = ok && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bias_type,
                                               sizeof(bias_type)) == HIPBLAS_STATUS_SUCCESS;
  // column-major: A = w as K x N (ld ldw), B = x as K x M (ld ldx), C = D = y^T as N x M (ld ldy)
  ok = ok && hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16F, K, N, ldw) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16F, K, M, ldx) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&p.c, HIP_R_16F, N, M, ldy) == HIPBLAS_STATUS_SUCCESS;
  if (!ok) {
    destroy(p);
    return fail(SIDON_E_LAUNCH, "hipBLASLt descriptor set-up failed");
  }
  hipblasLtMatmulPreference_t pref = nullptr;
  const uint64_t no_workspace = 0;
  hipblasLtMatmulHeuristicResult_t res[1];
  int found = 0;
  ok = hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &no_workspace,
                                                   sizeof(no_workspace)) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatmulAlgoGetHeuristic(g_handle[dev], p.desc, p.a, p.b, p.c, p.c, pref, 1, res, &found) ==
                 HIPBLAS_STATUS_SUCCESS;
  if (pref) hipblasLtMatmulPreferenceDestroy(pref);
  if (!ok || found < 1 || res[0].state != HIPBLAS_STATUS_SUCCESS || res[0].workspaceSize != 0) {
    destroy(p);
    return fail(SIDON_E_SHAPE, "hipBLASLt has no kernel without workspace for M=%d N=%d K=%d", M, N, K);
  }
  p.algo = res[0].algo;
  *out = &g_plans.emplace(key, p).first->second;
  return SIDON_OK;
}

}  // namespace

SIDON_API int sidon_gemm_lt_act(const void* x, int ldx, const void* w, int ldw, const void* bias, void* y, int ldy,
                                int M, int N, int K, int act, sidon_stream_t stream) {
  sidon::clear_error();
  if (!x || !w || !y) return fail(SIDON_E_NULL, "x, w and y must be non-NULL");
  if (M < 1 || N < 1 || K < 1 || (act != 0 && act != 1))
    return fail(SIDON_E_SHAPE, "M=%d, N=%d and K=%d must be >= 1 and act=%d in {0, 1}", M, N, K, act);
  if (ldx < K || ldw < K || ldy < N)
    return fail(SIDON_E_STRIDE, "row strides ldx=%d, ldw=%d (>= K=%d) and ldy=%d (>= N=%d)", ldx, ldw, K, ldy, N);
  if ((int64_t)M * ldx > INT32_MAX || (int64_t)N * ldw > INT32_MAX || (int64_t)M * ldy > INT32_MAX)
    return fail(SIDON_E_SHAPE, "operands of more than 2^31 - 1 elements");
  if (((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(y) |
        reinterpret_cast<uintptr_t>(bias)) & 1u) != 0)
    return fail(SIDON_E_ALIGN, "x, w, bias and y must be 2-byte aligned");
  int rc, dev = 0;
  if ((rc = sidon::check_device())) return rc;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(SIDON_E_DEVICE, "no usable HIP device");
  const bool has_bias = bias != nullptr;
  const Key key{dev, M, N, K, ldx, ldw, ldy, act, has_bias};
  std::lock_guard<std::mutex> lock(g_mu);
  Plan* p = nullptr;
  if ((rc = plan_for(dev, key, M, N, K, ldx, ldw, ldy, act, has_bias, &p))) return rc;
  if (has_bias && hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias,
                                                  sizeof(bias)) != HIPBLAS_STATUS_SUCCESS)
    return fail(SIDON_E_LAUNCH, "hipBLASLt bias pointer not accepted");
  const float one = 1.f, zero = 0.f;
  const hipblasStatus_t st = hipblasLtMatmul(g_handle[dev], p->desc, &one, w, p->a, x, p->b, &zero, y, p->c, y,
                                             p->c, &p->algo, nullptr, 0, reinterpret_cast<hipStream_t>(stream));
  if (st != HIPBLAS_STATUS_SUCCESS) return fail(SIDON_E_LAUNCH, "hipblasLtMatmul failed (status %d)", (int)st);
  return SIDON_OK;
}
