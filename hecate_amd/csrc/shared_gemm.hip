// shared_gemm.hip - the prefill shared expert's two projections as plain library GEMMs (hipBLASLt: f16 operands,
// fp32 accumulation and output). The shared expert is a dense bf16 MLP (its weights are exact in f16), so it needs no
// dequantisation and a library GEMM runs it near the MFMA peak. The reference keeps the shared expert outside its
// routed op as well (runtime/tier/tier_split.py:548-560: at decode into the accumulator, at prefill through the model's
// own shared-expert forward). The routed int4 experts stay on the hand-written grouped GEMM.
//
// lt_gemm: D[n][m] (row-major, leading dimension ldd) = X[n][k] . W[m][k]^T. In hipBLASLt's column-major terms that is
// D^T (m x n, ld ldd) = op(A) B with A = W seen as k x m (ld k, op = transpose) and B = X seen as k x n (ld k).
// One library handle per device and one plan (descriptors + the heuristic's algorithm) per shape, made on first use
// under a mutex and kept for the process; after that a call only queues the GEMM on the stream.
#include "hmoe_dev.h"

#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

namespace hmoe {

namespace {

struct LtPlan
{
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo{};
};

std::mutex g_lt_mu;
hipblasLtHandle_t g_lt[64] = {};
std::map<std::tuple<int, int, int, int, int, size_t>, LtPlan> g_plans;   // (device, m, n, k, ldd, workspace)

int lt_fail(const char* what, hipblasStatus_t s)
{
    return set_error(HMOE_ERR_HIP, "shared expert GEMM: %s failed (hipBLASLt status %d)", what, (int) s);
}

#define LT_TRY(call)                                             \
    do {                                                         \
        const hipblasStatus_t s_ = (call);                       \
        if (s_ != HIPBLAS_STATUS_SUCCESS) return lt_fail(#call, s_); \
    } while (0)

int make_plan(hipblasLtHandle_t h, int m, int n, int k, int ldd, size_t ws_bytes, LtPlan& p)
{
    LT_TRY(hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F));
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    LT_TRY(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)));
    LT_TRY(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)));
    LT_TRY(hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16F, k, m, k));
    LT_TRY(hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16F, k, n, k));
    LT_TRY(hipblasLtMatrixLayoutCreate(&p.c, HIP_R_32F, m, n, ldd));
    hipblasLtMatmulPreference_t pref = nullptr;
    LT_TRY(hipblasLtMatmulPreferenceCreate(&pref));
    const uint64_t wsb = ws_bytes;
    hipblasStatus_t s = hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb,
                                                              sizeof(wsb));
    hipblasLtMatmulHeuristicResult_t res{};
    int found = 0;
    if (s == HIPBLAS_STATUS_SUCCESS)
        s = hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.a, p.b, p.c, p.c, pref, 1, &res, &found);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (s != HIPBLAS_STATUS_SUCCESS) return lt_fail("hipblasLtMatmulAlgoGetHeuristic", s);
    if (found < 1 || res.workspaceSize > ws_bytes)
        return set_error(HMOE_ERR_HIP, "shared expert GEMM: no algorithm for m %d n %d k %d within %zu workspace bytes",
                         m, n, k, ws_bytes);
    p.algo = res.algo;
    return HMOE_OK;
}

}  // namespace

int lt_gemm(const _Float16* W, const _Float16* X, float* D, int m, int n, int k, int ldd, void* ws, size_t ws_bytes,
            hipStream_t st)
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return set_error(HMOE_ERR_HIP, "shared expert GEMM: current device");
    const LtPlan* plan = nullptr;
    hipblasLtHandle_t h = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_lt_mu);
        if (!g_lt[dev]) LT_TRY(hipblasLtCreate(&g_lt[dev]));
        h = g_lt[dev];
        const auto key = std::make_tuple(dev, m, n, k, ldd, ws_bytes);
        auto it = g_plans.find(key);
        if (it == g_plans.end())
        {
            LtPlan p;
            if (int rc = make_plan(h, m, n, k, ldd, ws_bytes, p)) return rc;
            it = g_plans.emplace(key, p).first;
        }
        plan = &it->second;                                      // (map nodes do not move)
    }
    const float alpha = 1.0f, beta = 0.0f;
    LT_TRY(hipblasLtMatmul(h, plan->desc, &alpha, W, plan->a, X, plan->b, &beta, D, plan->c, D, plan->c, &plan->algo,
                           ws, ws_bytes, st));
    return HMOE_OK;
}

}  // namespace hmoe
