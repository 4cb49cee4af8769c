// gemm.cpp -- the prefill GEMMs: y[m][n] (+)= x[m][k] . W[n][k]^T with bf16
// operands and fp32 accumulation, on hipBLASLt (plain library GEMMs; the
// fused work around them lives in rows.hip and the attention kernels).
//
// hipBLASLt is column-major.  The row-major buffers map onto it without
// copies: W [n][k] is a k x n column-major matrix (ld k) used transposed,
// x [m][k] is k x m (ld k), and y [m][n] is the n x m result (ld n).  An
// accumulating call passes y as C with beta = 1 (the residual add of the
// reference's Gemm(..., accumulate) calls, VulkanBackend.cs:782-856).
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "weights.hpp"

namespace hymt {
namespace {

constexpr size_t kWorkspace = 64u << 20;

struct Plan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    size_t ws = 0;
};

struct DeviceState {
    hipblasLtHandle_t handle = nullptr;
    void *workspace = nullptr;
    std::map<std::tuple<int, int, int, bool, bool>, Plan> plans;
};

std::mutex g_mu;
std::map<int, DeviceState> g_dev;

void destroy_plan(Plan &p) {
    if (p.a) hipblasLtMatrixLayoutDestroy(p.a);
    if (p.b) hipblasLtMatrixLayoutDestroy(p.b);
    if (p.c) hipblasLtMatrixLayoutDestroy(p.c);
    if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
    p = Plan{};
}

// hipBLASLt status -> a HIP error code the C ABI maps (no device, bad shape,
// or an internal failure)
hipError_t as_hip(hipblasStatus_t st) {
    switch (st) {
    case HIPBLAS_STATUS_SUCCESS: return hipSuccess;
    case HIPBLAS_STATUS_ALLOC_FAILED: return hipErrorOutOfMemory;
    case HIPBLAS_STATUS_INVALID_VALUE:
    case HIPBLAS_STATUS_NOT_SUPPORTED: return hipErrorInvalidValue;
    default: return hipErrorUnknown;
    }
}

constexpr int kCandidates = 8;

hipError_t time_candidates(DeviceState &d, const Plan &p, const hipblasLtMatmulHeuristicResult_t *res, int found,
                           const uint16_t *W, const uint16_t *x, int n, int m, bool y_bf16, bool acc,
                           hipStream_t s, int &best) {
    void *scratch = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t e = hipMalloc(&scratch, (size_t)n * m * (y_bf16 ? 2 : 4));
    if (e == hipSuccess) e = hipMemsetAsync(scratch, 0, (size_t)n * m * (y_bf16 ? 2 : 4), s);
    if (e == hipSuccess) e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    const float alpha = 1.0f, beta = acc ? 1.0f : 0.0f;
    float best_ms = 0.f;
    bool have = false;
    best = 0;
    for (int i = 0; i < found && e == hipSuccess; i++) {
        if (res[i].state != HIPBLAS_STATUS_SUCCESS || res[i].workspaceSize > kWorkspace) continue;
        auto run = [&]() {
            return hipblasLtMatmul(d.handle, p.desc, &alpha, W, p.a, x, p.b, &beta, scratch, p.c, scratch, p.c,
                                   &res[i].algo, d.workspace, res[i].workspaceSize, s);
        };
        if (run() != HIPBLAS_STATUS_SUCCESS) continue;  // warm-up; a candidate that fails is skipped
        e = hipEventRecord(e0, s);
        for (int r = 0; r < 3 && e == hipSuccess; r++)
            if (run() != HIPBLAS_STATUS_SUCCESS) e = hipErrorUnknown;
        if (e == hipSuccess) e = hipEventRecord(e1, s);
        if (e == hipSuccess) e = hipEventSynchronize(e1);
        float ms = 0.f;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
        if (e == hipSuccess && (!have || ms < best_ms)) {
            have = true;
            best_ms = ms;
            best = i;
        }
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (scratch) {
        (void)hipStreamSynchronize(s);
        (void)hipFree(scratch);
    }
    return e;
}

hipError_t make_plan(DeviceState &d, int n, int k, int m, bool y_bf16, bool acc, const uint16_t *W,
                     const uint16_t *x, hipStream_t s, Plan &p) {
    const hipDataType yt = y_bf16 ? HIP_R_16BF : HIP_R_32F;
    hipblasStatus_t st = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F);
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    if (st == HIPBLAS_STATUS_SUCCESS)
        st = hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta));
    if (st == HIPBLAS_STATUS_SUCCESS)
        st = hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb));
    if (st == HIPBLAS_STATUS_SUCCESS) st = hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16BF, k, n, k);
    if (st == HIPBLAS_STATUS_SUCCESS) st = hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16BF, k, m, k);
    if (st == HIPBLAS_STATUS_SUCCESS) st = hipblasLtMatrixLayoutCreate(&p.c, yt, n, m, n);
    hipblasLtMatmulPreference_t pref = nullptr;
    if (st == HIPBLAS_STATUS_SUCCESS) st = hipblasLtMatmulPreferenceCreate(&pref);
    const uint64_t wsmax = kWorkspace;
    if (st == HIPBLAS_STATUS_SUCCESS)
        st = hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsmax,
                                                   sizeof(wsmax));
    hipblasLtMatmulHeuristicResult_t res[kCandidates];
    int found = 0;
    if (st == HIPBLAS_STATUS_SUCCESS)
        st = hipblasLtMatmulAlgoGetHeuristic(d.handle, p.desc, p.a, p.b, p.c, p.c, pref, kCandidates, res, &found);
    if (pref) hipblasLtMatmulPreferenceDestroy(pref);
    if (st == HIPBLAS_STATUS_SUCCESS && found < 1) st = HIPBLAS_STATUS_NOT_SUPPORTED;
    if (st != HIPBLAS_STATUS_SUCCESS) {
        destroy_plan(p);
        return as_hip(st);
    }
    int best = 0;
    if (found > 1) {
        // The heuristic's first choice is not always the fastest at these
        // shapes: time each candidate once on the call's operands, writing a
        // scratch output (beta = 0 or 1 alike), and keep the fastest.
        hipError_t e = time_candidates(d, p, res, found, W, x, n, m, y_bf16, acc, s, best);
        if (e != hipSuccess) {
            destroy_plan(p);
            return e;
        }
    }
    p.algo = res[best].algo;
    p.ws = res[best].workspaceSize;
    return hipSuccess;
}

}  // namespace

hipError_t gemm_bf16(hipStream_t s, const uint16_t *W, int n, int k, const uint16_t *x, int m, void *y,
                     bool y_bf16, bool accumulate) {
    if (n < 1 || k < 1 || m < 0 || (accumulate && y_bf16)) return hipErrorInvalidValue;
    if (m == 0) return hipSuccess;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lk(g_mu);
    DeviceState &d = g_dev[dev];
    if (!d.handle) {
        hipblasStatus_t st = hipblasLtCreate(&d.handle);
        if (st != HIPBLAS_STATUS_SUCCESS) {
            d.handle = nullptr;
            return as_hip(st);
        }
        e = hipMalloc(&d.workspace, kWorkspace);
        if (e != hipSuccess) {
            d.workspace = nullptr;
            return e;
        }
    }
    const auto key = std::make_tuple(n, k, m, y_bf16, accumulate);
    auto it = d.plans.find(key);
    if (it == d.plans.end()) {
        Plan p;
        e = make_plan(d, n, k, m, y_bf16, accumulate, W, x, s, p);
        if (e != hipSuccess) return e;
        it = d.plans.emplace(key, p).first;
    }
    const Plan &p = it->second;
    const float alpha = 1.0f, beta = accumulate ? 1.0f : 0.0f;
    hipblasStatus_t st = hipblasLtMatmul(d.handle, p.desc, &alpha, W, p.a, x, p.b, &beta, y, p.c, y, p.c, &p.algo,
                                         d.workspace, p.ws, s);
    return as_hip(st);
}

}  // namespace hymt
