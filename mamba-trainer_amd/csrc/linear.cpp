// Linear::apply for bf16 activations (nn/linear.rs:155-185) through hipBLASLt:
//   y[M,N] = (x[M,K] @ w[K,N]) * col_scale[N] + residual[M,N]
// with f32 accumulation.  For the int8 fake-quantized projections w holds the
// integer codes (exact in bf16) and col_scale the per-output-channel scales,
// so the dequantisation is the GEMM's alpha vector; the residual add of the
// stack (models/hybrid.rs:446-456) is its beta * C.
//
// Row-major y = x w is column-major D = W X with D (N x M), W (N x K) and
// X (K x M), so the output channels are D's rows and the scale vector is
// hipBLASLt's per-row alpha vector.  A weight given transposed, w^T [N, K]
// row-major, is W^T column-major (K x N) with transpose A: hipBLASLt's
// kernels for that layout measured ~15 % faster at the prefill's shapes
// (torch.mm at 32768 x 768 by 768 x {5400, 768, 32000}: 323 / 48 / 1386 us
// against 365 / 57 / 1602 us).
//
// Up to 512 rows and 4096 columns (K a multiple of 128, N of 8, 16-byte
// aligned buffers) the product runs on the weight-streaming kernel of
// skinny_gemm.hip instead, with the same epilogue.
//
// Plan choice follows the reference's tuned plans (tensor/matmul.rs:1636-1943:
// timing probes once per shape): the first call for a shape asks hipBLASLt's
// heuristic for up to kCandidates algorithms, times each on the caller's data
// into a scratch output (the caller's buffers, including an in-place
// residual, are left untouched), keeps the fastest and blocks on the stream
// to read the timings.  Each timed run follows a write of kFlushBytes, more
// than the L2 and Infinity Cache hold, so a plan is judged on weights read
// from HBM, as a model's layers meet them, and each candidate keeps its best
// of kProbeRounds interleaved rounds.  Later calls with the shape launch the kept
// plan asynchronously.  M3_LINEAR_TUNE=0 keeps the heuristic's first choice
// (no probe, no blocking), for runs that must pick the same algorithm in
// every process.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

#include "m3_internal.hpp"

namespace m3 {

namespace {

constexpr int kCandidates = 8;
constexpr int kProbeRounds = 3;
constexpr size_t kFlushBytes = size_t(512) << 20;

struct Plan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    std::vector<hipblasLtMatmulAlgo_t> candidates;
    bool ok = false;
};

struct DeviceState {
    hipblasLtHandle_t handle = nullptr;
    std::map<std::tuple<size_t, size_t, size_t, bool, bool, size_t>, Plan> plans;
};

std::mutex g_mu;
std::map<int, DeviceState> g_dev;

bool build_plan(hipblasLtHandle_t h, size_t m, size_t k, size_t n, bool scaled, bool wt, size_t ws,
                Plan &p) {
    if (hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS)
        return false;
    hipblasOperation_t op = HIPBLAS_OP_N, opa = wt ? HIPBLAS_OP_T : HIPBLAS_OP_N;
    hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opa, sizeof(opa));
    hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &op, sizeof(op));
    if (scaled) {
        int32_t mode = HIPBLASLT_POINTER_MODE_ALPHA_DEVICE_VECTOR_BETA_HOST;
        hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_POINTER_MODE, &mode, sizeof(mode));
    }
    if ((wt ? hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16BF, k, n, static_cast<int64_t>(k))
            : hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16BF, n, k, static_cast<int64_t>(n))) !=
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
    hipblasLtMatmulHeuristicResult_t res[kCandidates];
    int count = 0;
    const hipblasStatus_t st =
        hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.a, p.b, p.c, p.c, pref, kCandidates, res, &count);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (st != HIPBLAS_STATUS_SUCCESS || count == 0) return false;
    for (int i = 0; i < count; ++i)
        if (res[i].state == HIPBLAS_STATUS_SUCCESS && res[i].workspaceSize <= ws)
            p.candidates.push_back(res[i].algo);
    if (p.candidates.empty()) return false;
    p.algo = p.candidates.front();
    p.ok = true;
    return true;
}

bool tuning_enabled() {
    const char *v = std::getenv("M3_LINEAR_TUNE");
    return v == nullptr || std::strcmp(v, "0") != 0;
}

// Times every candidate of `p` (one warm-up each, then kProbeRounds rounds of
// one run per candidate, each after the cache flush) with beta = 0 into a
// scratch [m, n] output and keeps the one with the lowest best time.  Any
// failure leaves the heuristic's first choice in place; without the flush
// buffer the runs are timed warm.
void tune_plan(hipblasLtHandle_t h, size_t m, size_t n, Plan &p, const void *alpha, const void *w,
               const void *x, void *workspace, size_t ws, hipStream_t s) {
    const size_t nc = p.candidates.size();
    if (nc < 2) return;
    void *scratch = nullptr, *flush = nullptr;
    if (hipMalloc(&scratch, m * n * 2) != hipSuccess) {
        (void)hipGetLastError();
        return;
    }
    if (hipMalloc(&flush, kFlushBytes) != hipSuccess) {
        (void)hipGetLastError();
        flush = nullptr;
    }
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess) {
        const float zero = 0.0f;
        auto run = [&](size_t i) {
            return hipblasLtMatmul(h, p.desc, alpha, w, p.a, x, p.b, &zero, scratch, p.c, scratch, p.c,
                                   &p.candidates[i], workspace, ws, s) == HIPBLAS_STATUS_SUCCESS;
        };
        std::vector<float> best(nc, -1.0f);   // -1: failed or not timed
        std::vector<char> usable(nc, 0);
        for (size_t i = 0; i < nc; ++i) usable[i] = run(i) ? 1 : 0;
        for (int round = 0; round < kProbeRounds; ++round) {
            for (size_t i = 0; i < nc; ++i) {
                if (!usable[i]) continue;
                if (flush) (void)hipMemsetAsync(flush, round * 16 + static_cast<int>(i), kFlushBytes, s);
                bool ok = hipEventRecord(e0, s) == hipSuccess && run(i);
                ok = ok && hipEventRecord(e1, s) == hipSuccess && hipEventSynchronize(e1) == hipSuccess;
                float ms = 0.0f;
                if (!ok || hipEventElapsedTime(&ms, e0, e1) != hipSuccess) {
                    usable[i] = 0;
                    continue;
                }
                if (best[i] < 0.0f || ms < best[i]) best[i] = ms;
            }
        }
        size_t pick = nc;
        for (size_t i = 0; i < nc; ++i)
            if (usable[i] && best[i] >= 0.0f && (pick == nc || best[i] < best[pick])) pick = i;
        if (pick < nc) p.algo = p.candidates[pick];
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipStreamSynchronize(s);
    (void)hipFree(scratch);
    if (flush) (void)hipFree(flush);
    (void)hipGetLastError();
}

}  // namespace

hipError_t launch_linear(size_t m, size_t k, size_t n, const void *x, const void *w,
                         bool w_transposed, const float *col_scale, const void *residual, void *y,
                         void *workspace, size_t workspace_bytes, hipStream_t s) {
    if (m == 0 || n == 0) return hipSuccess;
    // few rows (a decode step's tokens): the weight-streaming kernel
    if (skinny_gemm_supported(m, k, n, x, w, col_scale, residual, y))
        return launch_skinny_gemm(m, k, n, x, w, w_transposed, col_scale, residual, y, s);
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
        auto key = std::make_tuple(m, k, n, scaled, w_transposed, ws);
        auto it = d.plans.find(key);
        const float one = 1.0f;
        const void *alpha = scaled ? static_cast<const void *>(col_scale) : static_cast<const void *>(&one);
        if (it == d.plans.end()) {
            Plan p;
            if (!build_plan(handle, m, k, n, scaled, w_transposed, ws, p)) return hipErrorNotSupported;
            // no probe while the stream is being captured into a graph: its
            // allocations, fills and waits cannot be captured, so a shape
            // first met under capture keeps hipBLASLt's first choice
            hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
            if (hipStreamIsCapturing(s, &cap) != hipSuccess) {
                (void)hipGetLastError();
                cap = hipStreamCaptureStatusActive;
            }
            if (tuning_enabled() && cap == hipStreamCaptureStatusNone)
                tune_plan(handle, m, n, p, alpha, w, x, workspace, ws, s);
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
