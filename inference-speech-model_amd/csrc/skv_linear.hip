// Decode-batch projections, y = x W^T (+ b), through hipBLASLt with one cached plan
// per (device, dtype, shape, strides, bias or not).
//
// torch's linear builds the matmul descriptor and matrix layouts and asks hipBLASLt's
// heuristic for an algorithm on every call (~19 us of host time at the decode
// shapes); a decode step of a 32-layer model makes ~190 such calls. Here the
// descriptor, the layouts and the heuristic's first algorithm are kept per shape, so a
// call is a map lookup, the bias pointer and one hipblasLtMatmul. Plans take no
// workspace (the heuristic is asked for algorithms that need none), so a call
// allocates nothing, and the algorithm is the one torch's linear runs at these shapes
// (the same descriptor settings: fp32 compute and scale, A = W transposed, bias epilogue).
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "skv_common.h"

using namespace skv;

namespace {

constexpr int kMaxDevices = 64;

struct LinearPlan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
  hipblasLtMatmulAlgo_t algo{};
};

// (device, dtype, m, n, k, ldx, ldw, ldy, bias)
using PlanKey = std::tuple<int, int32_t, int32_t, int32_t, int32_t, int64_t, int64_t, int64_t, bool>;

std::mutex g_linear_mu;
hipblasLtHandle_t g_lt[kMaxDevices] = {};
std::map<PlanKey, LinearPlan> g_linear_plans;

hipDataType lt_type(int32_t dtype) {
  return dtype == SKV_BF16 ? HIP_R_16BF : dtype == SKV_F16 ? HIP_R_16F : HIP_R_32F;
}

// Builds the plan of `key` (caller holds g_linear_mu); SKV_OK, or an error code with the message recorded.
int make_plan(hipblasLtHandle_t lt, const PlanKey& key, LinearPlan& p) {
  const int32_t dtype = std::get<1>(key), m = std::get<2>(key), n = std::get<3>(key), k = std::get<4>(key);
  const int64_t ldx = std::get<5>(key), ldw = std::get<6>(key), ldy = std::get<7>(key);
  const bool has_bias = std::get<8>(key);
  const hipDataType t = lt_type(dtype);
  // Column-major view of the row-major product: D (n x m, ld ldy) = op(A) B with A = W
  // stored as k x n (ld ldw) and transposed, B = x stored as k x m (ld ldx).
  hipblasStatus_t st = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F);
  if (st != HIPBLAS_STATUS_SUCCESS) return fail(SKV_EINVAL, "skv_linear: hipblasLtMatmulDescCreate returned %d", (int)st);
  const int32_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  st = hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta));
  if (st == HIPBLAS_STATUS_SUCCESS) st = hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb));
  if (st == HIPBLAS_STATUS_SUCCESS && has_bias) {
    const uint32_t epi = HIPBLASLT_EPILOGUE_BIAS;
    const int32_t bt = (int32_t)t;
    st = hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi));
    if (st == HIPBLAS_STATUS_SUCCESS)
      st = hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof(bt));
  }
  if (st == HIPBLAS_STATUS_SUCCESS) st = hipblasLtMatrixLayoutCreate(&p.a, t, (uint64_t)k, (uint64_t)n, ldw);
  if (st == HIPBLAS_STATUS_SUCCESS) st = hipblasLtMatrixLayoutCreate(&p.b, t, (uint64_t)k, (uint64_t)m, ldx);
  if (st == HIPBLAS_STATUS_SUCCESS) st = hipblasLtMatrixLayoutCreate(&p.d, t, (uint64_t)n, (uint64_t)m, ldy);
  if (st != HIPBLAS_STATUS_SUCCESS) return fail(SKV_EINVAL, "skv_linear: descriptor set-up returned %d", (int)st);
  hipblasLtMatmulPreference_t pref = nullptr;
  st = hipblasLtMatmulPreferenceCreate(&pref);
  if (st != HIPBLAS_STATUS_SUCCESS) return fail(SKV_EINVAL, "skv_linear: preference set-up returned %d", (int)st);
  const uint64_t no_workspace = 0;
  st = hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &no_workspace,
                                             sizeof(no_workspace));
  hipblasLtMatmulHeuristicResult_t res{};
  int found = 0;
  if (st == HIPBLAS_STATUS_SUCCESS)
    st = hipblasLtMatmulAlgoGetHeuristic(lt, p.desc, p.a, p.b, p.d, p.d, pref, 1, &res, &found);
  hipblasLtMatmulPreferenceDestroy(pref);
  if (st != HIPBLAS_STATUS_SUCCESS || found < 1 || res.workspaceSize != 0)
    return fail(SKV_EUNSUPPORTED, "skv_linear: no workspace-free hipBLASLt algorithm for m=%d n=%d k=%d dtype=%d", m,
                n, k, dtype);
  p.algo = res.algo;
  return SKV_OK;
}

void destroy_plan(LinearPlan& p) {
  if (p.a) hipblasLtMatrixLayoutDestroy(p.a);
  if (p.b) hipblasLtMatrixLayoutDestroy(p.b);
  if (p.d) hipblasLtMatrixLayoutDestroy(p.d);
  if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
  p = LinearPlan{};
}

}  // namespace

int skv_linear(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* bias, void* y, int64_t ldy,
               int32_t m, int32_t n, int32_t k, int32_t dtype, void* stream) {
  if (elt_bytes(dtype) == 0) return fail(SKV_EDTYPE, "skv_linear: unknown dtype %d", dtype);
  if (m < 0 || n <= 0 || k <= 0 || ldx < k || ldw < k || ldy < n)
    return fail(SKV_EINVAL, "skv_linear: bad sizes m=%d n=%d k=%d ldx=%lld ldw=%lld ldy=%lld", m, n, k,
                (long long)ldx, (long long)ldw, (long long)ldy);
  if (m == 0) return SKV_OK;
  if (!x || !w || !y) return fail(SKV_EINVAL, "skv_linear: null pointer argument");
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(SKV_EINVAL, "skv_linear: no current device");
  std::lock_guard<std::mutex> lock(g_linear_mu);
  if (!g_lt[dev]) {
    const hipblasStatus_t st = hipblasLtCreate(&g_lt[dev]);
    if (st != HIPBLAS_STATUS_SUCCESS) {
      g_lt[dev] = nullptr;
      return fail(SKV_EINVAL, "skv_linear: hipblasLtCreate returned %d", (int)st);
    }
  }
  const PlanKey key{dev, dtype, m, n, k, ldx, ldw, ldy, bias != nullptr};
  auto it = g_linear_plans.find(key);
  if (it == g_linear_plans.end()) {
    LinearPlan p;
    const int rc = make_plan(g_lt[dev], key, p);
    if (rc != SKV_OK) {
      destroy_plan(p);
      return rc;
    }
    it = g_linear_plans.emplace(key, p).first;
  }
  LinearPlan& p = it->second;
  if (bias) {
    const hipblasStatus_t st =
        hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias));
    if (st != HIPBLAS_STATUS_SUCCESS) return fail(SKV_EINVAL, "skv_linear: bias pointer returned %d", (int)st);
  }
  const float alpha = 1.f, beta = 0.f;
  const hipblasStatus_t st = hipblasLtMatmul(g_lt[dev], p.desc, &alpha, w, p.a, x, p.b, &beta, y, p.d, y, p.d,
                                             &p.algo, nullptr, 0, (hipStream_t)stream);
  if (st != HIPBLAS_STATUS_SUCCESS) return fail(SKV_EINVAL, "skv_linear: hipblasLtMatmul returned %d", (int)st);
  return SKV_OK;
}
