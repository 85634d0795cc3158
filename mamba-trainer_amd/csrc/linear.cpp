// Linear::apply for bf16 activations (nn/linear.rs:155-185) through hipBLASLt:
//   y[M,N] = (x[M,K] @ w[K,N]) * col_scale[N] + residual[M,N]
// with f32 accumulation.  For the int8 fake-quantized projections w holds the
// integer codes (exact in bf16) and col_scale the per-output-channel scales,
// so the dequantisation is the GEMM's alpha vector; the residual add of the
// stack (models/hybrid.rs:446-456) is its beta * C.
//
// Row-major y = x w is column-major D = W X with D (N x M), W (N x K) and
// X (K x M), so the output channels are D's rows and the scale vector is
// hipBLASLt's per-row alpha vector.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "m3_internal.hpp"

namespace m3 {

namespace {

struct Plan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    bool ok = false;
};

struct DeviceState {
    hipblasLtHandle_t handle = nullptr;
    std::map<std::tuple<size_t, size_t, size_t, bool, size_t>, Plan> plans;
};

std::mutex g_mu;
std::map<int, DeviceState> g_dev;

bool build_plan(hipblasLtHandle_t h, size_t m, size_t k, size_t n, bool scaled, size_t ws,
                Plan &p) {
    if (hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS)
        return false;
    hipblasOperation_t op = HIPBLAS_OP_N;
    hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &op, sizeof(op));
    hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &op, sizeof(op));
    if (scaled) {
        int32_t mode = HIPBLASLT_POINTER_MODE_ALPHA_DEVICE_VECTOR_BETA_HOST;
        hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_POINTER_MODE, &mode, sizeof(mode));
    }
    if (hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16BF, n, k, static_cast<int64_t>(n)) !=
            HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16BF, k, m, static_cast<int64_t>(k)) !=
            HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&p.c, HIP_R_16BF, n, m, static_cast<int64_t>(n)) !=
            HIPBLAS_STATUS_SUCCESS)
        return false;
    hipblasLtMatmulPreference_t pref = nullptr;
    if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return false;
    uint64_t wsb = ws;
    hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb,
                                          sizeof(wsb));
    hipblasLtMatmulHeuristicResult_t res[4];
    int count = 0;
    const hipblasStatus_t st =
        hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.a, p.b, p.c, p.c, pref, 4, res, &count);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (st != HIPBLAS_STATUS_SUCCESS || count == 0) return false;
    for (int i = 0; i < count; ++i) {
        if (res[i].state == HIPBLAS_STATUS_SUCCESS && res[i].workspaceSize <= ws) {
            p.algo = res[i].algo;
            p.ok = true;
            return true;
        }
    }
    return false;
}

}  // namespace

hipError_t launch_linear(size_t m, size_t k, size_t n, const void *x, const void *w,
                         const float *col_scale, const void *residual, void *y, void *workspace,
                         size_t workspace_bytes, hipStream_t s) {
    if (m == 0 || n == 0) return hipSuccess;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const bool scaled = col_scale != nullptr;
    const size_t ws = workspace ? workspace_bytes : 0;
    Plan *plan = nullptr;
    hipblasLtHandle_t handle = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        DeviceState &d = g_dev[dev];
        if (d.handle == nullptr && hipblasLtCreate(&d.handle) != HIPBLAS_STATUS_SUCCESS) {
            d.handle = nullptr;
            return hipErrorInitializationError;
        }
        handle = d.handle;
        auto key = std::make_tuple(m, k, n, scaled, ws);
        auto it = d.plans.find(key);
        if (it == d.plans.end()) {
            Plan p;
            if (!build_plan(handle, m, k, n, scaled, ws, p)) return hipErrorNotSupported;
            it = d.plans.emplace(key, p).first;
        }
        plan = &it->second;
    }
    const float one = 1.0f;
    const float beta = residual ? 1.0f : 0.0f;
    const void *alpha = scaled ? static_cast<const void *>(col_scale) : static_cast<const void *>(&one);
    const hipblasStatus_t st =
        hipblasLtMatmul(handle, plan->desc, alpha, w, plan->a, x, plan->b, &beta,
                        residual ? residual : y, plan->c, y, plan->c, &plan->algo, workspace, ws, s);
    return st == HIPBLAS_STATUS_SUCCESS ? hipSuccess : hipErrorLaunchFailure;
}

}  // namespace m3
