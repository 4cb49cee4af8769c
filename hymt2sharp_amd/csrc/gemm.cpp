// gemm.cpp -- the prefill GEMMs: y[m][n] (+)= x[m][k] . W[n][k]^T with bf16
// operands and fp32 accumulation, on hipBLASLt or on this library's MFMA
// kernel (gemm_mfma.hip) (the fused work around them lives in rows.hip and
// the attention kernels).
//
// hipBLASLt is column-major.  The row-major buffers map onto it without
// copies: W [n][k] is a k x n column-major matrix (ld k) used transposed,
// x [m][k] is k x m (ld k), and y [m][n] is the n x m result (ld ldy >= n).
// An accumulating call passes y as C with beta = 1 (the residual add of the
// reference's Gemm(..., accumulate) calls, VulkanBackend.cs:782-856).
//
// All state -- the hipBLASLt handle, the split-K workspace, the chosen
// algorithms -- belongs to one GemmState, which a context owns: two contexts
// on one device never share a workspace, and no lock is needed (calls on one
// context come from one thread, in stream order).
//
// Algorithm choice, by HYMT_HIP_GEMM (read when the state is created):
//  unset   the MFMA kernel wherever its shape rules allow (gemm_mfma_fits),
//  (=mfma) hipBLASLt's first heuristic choice for the call's exact shape
//          otherwise: no timing, so identical inputs give identical bits in
//          every context and process.  Measured per shape (us, MFMA plan /
//          hipBLASLt's first choice): the MFMA kernel is faster for q/k/v, o
//          and down at every m from 512 to 2048 and for gate/up at 512;
//          hipBLASLt by 1-5 % for the gate/up GEMM alone from 1024 rows on,
//          which the model's prefill runs fused with its SwiGLU on the MFMA
//          kernel instead (gemm_swiglu: one launch, half the output bytes,
//          no row kernel);
//  library hipBLASLt's first heuristic choice for every shape;
//  auto    the first call of a shape in an m bucket (m rounded up to a power
//          of two, at least 256) times up to kCandidates of hipBLASLt's
//          candidates and the MFMA kernel on the call's operands and keeps
//          the fastest; a later m in the same bucket reuses that choice (for
//          hipBLASLt, when the heuristic offers the algorithm for the new m,
//          else its first choice).  The pick can differ between processes
//          with timing noise, and with it the summation order and the bits;
//  hipblaslt  as auto over hipBLASLt's candidates only.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <map>
#include <tuple>

#include "ktimer.hpp"
#include "weights.hpp"

namespace hymt {

namespace {

constexpr size_t kWorkspace = 64u << 20;
constexpr int kCandidates = 16;

struct Layouts {
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    size_t ws = 0;
    bool mfma = false;  // the MFMA kernel, when the call's operands fit it
};

struct Choice {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatmulAlgo_t algo{};  // the timed algorithm of the bucket
    bool mfma = false;             // the MFMA kernel timed fastest
};

enum GemmMode { kHeuristic = 0, kAuto = 1, kLibTimed = 3, kPlanned = 4 };

void destroy_layouts(Layouts &l) {
    if (l.a) hipblasLtMatrixLayoutDestroy(l.a);
    if (l.b) hipblasLtMatrixLayoutDestroy(l.b);
    if (l.c) hipblasLtMatrixLayoutDestroy(l.c);
    l = Layouts{};
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

int bucket_of(int m) {
    int b = 256;
    while (b < m) b *= 2;
    return b;
}

bool same_algo(const hipblasLtMatmulAlgo_t &x, const hipblasLtMatmulAlgo_t &y) {
    return std::memcmp(&x, &y, sizeof(x)) == 0;
}

}  // namespace

struct GemmState {
    int mode = kHeuristic;
    hipblasLtHandle_t handle = nullptr;
    void *workspace = nullptr;
    void *scratch = nullptr;  // timing output of the candidate runs
    size_t scratch_bytes = 0;
    GemmSplitWs split{};      // the MFMA kernel's split-k partials and tickets
    // (n, k, m bucket, y_bf16, accumulate) -> descriptor and timed algorithm
    std::map<std::tuple<int, int, int, bool, bool>, Choice> choices;
    // (n, k, m, ldy, y_bf16, accumulate) -> layouts and the algorithm used
    std::map<std::tuple<int, int, int, int, bool, bool>, Layouts> layouts;
};

GemmState *gemm_state_create() {
    GemmState *g = new (std::nothrow) GemmState();
    if (g) {
        const char *e = std::getenv("HYMT_HIP_GEMM");
        g->mode = kPlanned;
        if (e && !std::strcmp(e, "library")) g->mode = kHeuristic;
        if (e && !std::strcmp(e, "auto")) g->mode = kAuto;
        if (e && !std::strcmp(e, "hipblaslt")) g->mode = kLibTimed;
    }
    return g;
}

void gemm_state_destroy(GemmState *g) {
    if (!g) return;
    for (auto &kv : g->layouts) destroy_layouts(kv.second);
    for (auto &kv : g->choices)
        if (kv.second.desc) hipblasLtMatmulDescDestroy(kv.second.desc);
    if (g->workspace) (void)hipFree(g->workspace);
    if (g->scratch) (void)hipFree(g->scratch);
    if (g->split.part) (void)hipFree(g->split.part);
    if (g->split.ticket) (void)hipFree(g->split.ticket);
    if (g->handle) hipblasLtDestroy(g->handle);
    delete g;
}

namespace {

// The MFMA kernel with its plan for the shape; a split plan first makes sure
// the state holds room for its partials and tickets (allocated on the stream's
// first such call, zeroed once; every call leaves the tickets zero).
hipError_t run_mfma(GemmState &g, const uint16_t *W, int n, int k, const uint16_t *x, int m, void *y, int ldy,
                    bool y_bf16, bool acc, hipStream_t s) {
    const GemmPlan p = gemm_mfma_plan(n, k, m);
    if (p.split == 2) {
        const size_t need = gemm_split_bytes(n, m, p);
        const int tickets = gemm_split_tiles(n, m, p);  // one per tile
        hipError_t e = hipSuccess;
        if (need > g.split.part_bytes) {
            e = hipStreamSynchronize(s);
            if (e == hipSuccess && g.split.part) e = hipFree(g.split.part);
            g.split.part = nullptr;
            g.split.part_bytes = 0;
            if (e == hipSuccess) e = hipMalloc(&g.split.part, need);
            if (e != hipSuccess) return e;
            g.split.part_bytes = need;
        }
        if (tickets > g.split.tickets) {
            e = hipStreamSynchronize(s);
            if (e == hipSuccess && g.split.ticket) e = hipFree(g.split.ticket);
            g.split.ticket = nullptr;
            g.split.tickets = 0;
            if (e == hipSuccess) e = hipMalloc(&g.split.ticket, (size_t)tickets * 32 * sizeof(unsigned));
            if (e == hipSuccess) e = hipMemsetAsync(g.split.ticket, 0, (size_t)tickets * 32 * sizeof(unsigned), s);
            if (e != hipSuccess) return e;
            g.split.tickets = tickets;
        }
    }
    return gemm_bf16_mfma(W, n, k, x, m, y, ldy, y_bf16, acc, s, p, &g.split);
}

hipblasStatus_t make_desc(hipblasLtMatmulDesc_t &desc) {
    hipblasStatus_t st = hipblasLtMatmulDescCreate(&desc, HIPBLAS_COMPUTE_32F, HIP_R_32F);
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    if (st == HIPBLAS_STATUS_SUCCESS)
        st = hipblasLtMatmulDescSetAttribute(desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta));
    if (st == HIPBLAS_STATUS_SUCCESS)
        st = hipblasLtMatmulDescSetAttribute(desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb));
    return st;
}

hipblasStatus_t make_layouts(int n, int k, int m, int ldy, bool y_bf16, Layouts &l) {
    hipblasStatus_t st = hipblasLtMatrixLayoutCreate(&l.a, HIP_R_16BF, k, n, k);
    if (st == HIPBLAS_STATUS_SUCCESS) st = hipblasLtMatrixLayoutCreate(&l.b, HIP_R_16BF, k, m, k);
    if (st == HIPBLAS_STATUS_SUCCESS)
        st = hipblasLtMatrixLayoutCreate(&l.c, y_bf16 ? HIP_R_16BF : HIP_R_32F, n, m, ldy);
    return st;
}

hipblasStatus_t heuristic(GemmState &g, hipblasLtMatmulDesc_t desc, const Layouts &l,
                          hipblasLtMatmulHeuristicResult_t *res, int &found) {
    hipblasLtMatmulPreference_t pref = nullptr;
    hipblasStatus_t st = hipblasLtMatmulPreferenceCreate(&pref);
    const uint64_t wsmax = kWorkspace;
    if (st == HIPBLAS_STATUS_SUCCESS)
        st = hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsmax,
                                                   sizeof(wsmax));
    found = 0;
    if (st == HIPBLAS_STATUS_SUCCESS)
        st = hipblasLtMatmulAlgoGetHeuristic(g.handle, desc, l.a, l.b, l.c, l.c, pref, kCandidates, res, &found);
    if (pref) hipblasLtMatmulPreferenceDestroy(pref);
    if (st == HIPBLAS_STATUS_SUCCESS && found < 1) st = HIPBLAS_STATUS_NOT_SUPPORTED;
    return st;
}

// Time the usable candidates -- hipBLASLt's and, with_mfma, the MFMA kernel
// (best = -1) -- on the call's operands, writing the state's scratch output
// (beta = 0 or 1 alike): each runs once to warm up, then kRounds rounds time
// every candidate once in turn, so that a drift of the clock over the tuning
// weighs on all candidates alike; the fastest median wins.  (Three
// back-to-back runs per candidate let such drift pick a candidate 25 % slower
// than the best on the 12288 x 2048 gate/up GEMM.)
hipError_t time_candidates(GemmState &g, hipblasLtMatmulDesc_t desc, const Layouts &l,
                           const hipblasLtMatmulHeuristicResult_t *res, int found, const uint16_t *W,
                           const uint16_t *x, int n, int k, int m, int ldy, bool y_bf16, bool acc, bool with_mfma,
                           hipStream_t s, int &best) {
    constexpr int kRounds = 5;
    best = 0;
    const size_t ybytes = ((size_t)(m - 1) * ldy + n) * (y_bf16 ? 2 : 4);
    hipError_t e = hipSuccess;
    if (ybytes > g.scratch_bytes) {
        e = hipStreamSynchronize(s);
        if (e == hipSuccess && g.scratch) e = hipFree(g.scratch);
        g.scratch = nullptr;
        g.scratch_bytes = 0;
        if (e == hipSuccess) e = hipMalloc(&g.scratch, ybytes);
        if (e != hipSuccess) return e;
        g.scratch_bytes = ybytes;
    }
    e = hipMemsetAsync(g.scratch, 0, ybytes, s);
    const float alpha = 1.0f, beta = acc ? 1.0f : 0.0f;
    // candidate i >= 0: hipBLASLt's res[i]; -1: the MFMA kernel
    auto run = [&](int i) -> bool {
        if (i < 0) return run_mfma(g, W, n, k, x, m, g.scratch, ldy, y_bf16, acc, s) == hipSuccess;
        return hipblasLtMatmul(g.handle, desc, &alpha, W, l.a, x, l.b, &beta, g.scratch, l.c, g.scratch, l.c,
                               &res[i].algo, g.workspace, res[i].workspaceSize, s) == HIPBLAS_STATUS_SUCCESS;
    };
    int usable[kCandidates + 1], nu = 0;
    if (with_mfma && e == hipSuccess && run(-1)) usable[nu++] = -1;
    for (int i = 0; i < found && e == hipSuccess; i++) {
        if (res[i].state != HIPBLAS_STATUS_SUCCESS || res[i].workspaceSize > kWorkspace) continue;
        if (run(i)) usable[nu++] = i;  // warm-up; a candidate that fails is skipped
    }
    if (nu < 2) {
        if (nu == 1) best = usable[0];
        return e;
    }
    hipEvent_t ev[2 * (kCandidates + 1)] = {};
    for (int j = 0; j < 2 * nu && e == hipSuccess; j++) e = hipEventCreate(&ev[j]);
    float ms[kCandidates + 1][kRounds] = {};
    for (int r = 0; r < kRounds && e == hipSuccess; r++) {
        for (int j = 0; j < nu && e == hipSuccess; j++) {
            e = hipEventRecord(ev[2 * j], s);
            if (e == hipSuccess && !run(usable[j])) e = hipErrorUnknown;
            if (e == hipSuccess) e = hipEventRecord(ev[2 * j + 1], s);
        }
        if (e == hipSuccess) e = hipEventSynchronize(ev[2 * nu - 1]);
        for (int j = 0; j < nu && e == hipSuccess; j++) e = hipEventElapsedTime(&ms[j][r], ev[2 * j], ev[2 * j + 1]);
    }
    float best_ms = 0.f;
    for (int j = 0; j < nu && e == hipSuccess; j++) {
        float v[kRounds];
        std::memcpy(v, ms[j], sizeof(v));
        std::sort(v, v + kRounds);
        if (j == 0 || v[kRounds / 2] < best_ms) {
            best_ms = v[kRounds / 2];
            best = usable[j];
        }
    }
    for (int j = 0; j < 2 * nu; j++)
        if (ev[j]) (void)hipEventDestroy(ev[j]);
    return e;
}

}  // namespace

bool gemm_swiglu(GemmState *g, hipStream_t s, const uint16_t *Wg, const uint16_t *Wu, bool separate, int f, int k,
                 const uint16_t *x, int m, const uint16_t *gu, uint16_t *act, hipError_t &err) {
    err = hipSuccess;
    if (!g || m < 1 || f < 1) return false;
    // gu (null: any 16-byte aligned buffer) and its up half gu + f: their
    // alignment is all that enters (f % 8 == 0 below)
    const bool gu_al = ((uintptr_t)gu & 15u) == 0;
    auto mfma_unsplit = [&](const uint16_t *W, int n) {
        return gemm_mfma_fits(W, n, k, x, m, act, 2 * f) && g->mode == kPlanned && gemm_mfma_plan(n, k, m).split == 1;
    };
    const bool unfused_mfma = separate ? mfma_unsplit(Wg, f) && mfma_unsplit(Wu, f)
                                       : Wu == Wg + (size_t)f * k && mfma_unsplit(Wg, 2 * f);
    // launch_rows_swiglu_bf16's 16-byte kernel
    const bool rows_x8 = f % 8 == 0 && gu_al && ((uintptr_t)act & 15u) == 0 && (size_t)m * (f / 8) <= (1u << 30);
    if (!unfused_mfma || !rows_x8 || !gemm_swiglu_fits(Wg, Wu, f, k, x, m, act, f)) return false;
    err = gemm_swiglu_mfma(Wg, Wu, f, k, x, m, act, f, s, gemm_mfma_plan(2 * f, k, m));
    return true;
}

hipError_t gemm_bf16(GemmState *g, hipStream_t s, const uint16_t *W, int n, int k, const uint16_t *x, int m,
                     void *y, int ldy, bool y_bf16, bool accumulate) {
    if (!g || n < 1 || k < 1 || m < 0 || ldy < n || (accumulate && y_bf16)) return hipErrorInvalidValue;
    if (m == 0) return hipSuccess;
    const bool fits = gemm_mfma_fits(W, n, k, x, m, y, ldy);
    if (fits && g->mode == kPlanned)
        return run_mfma(*g, W, n, k, x, m, y, ldy, y_bf16, accumulate, s);
    hipError_t e = hipSuccess;
    if (!g->handle) {
        hipblasStatus_t st = hipblasLtCreate(&g->handle);
        if (st != HIPBLAS_STATUS_SUCCESS) {
            g->handle = nullptr;
            return as_hip(st);
        }
    }
    if (!g->workspace) {
        e = hipMalloc(&g->workspace, kWorkspace);
        if (e != hipSuccess) {
            g->workspace = nullptr;
            return e;
        }
    }
    const auto ckey = std::make_tuple(n, k, bucket_of(m), y_bf16, accumulate);
    auto cit = g->choices.find(ckey);
    const bool first_in_bucket = cit == g->choices.end();
    if (first_in_bucket) {
        Choice ch;
        hipblasStatus_t st = make_desc(ch.desc);
        if (st != HIPBLAS_STATUS_SUCCESS) {
            if (ch.desc) hipblasLtMatmulDescDestroy(ch.desc);
            return as_hip(st);
        }
        cit = g->choices.emplace(ckey, ch).first;
    }
    Choice &ch = cit->second;
    const auto lkey = std::make_tuple(n, k, m, ldy, y_bf16, accumulate);
    auto lit = g->layouts.find(lkey);
    if (lit == g->layouts.end()) {
        Layouts l;
        hipblasLtMatmulHeuristicResult_t res[kCandidates];
        int found = 0;
        hipblasStatus_t st = make_layouts(n, k, m, ldy, y_bf16, l);
        if (st == HIPBLAS_STATUS_SUCCESS) st = heuristic(*g, ch.desc, l, res, found);
        if (st != HIPBLAS_STATUS_SUCCESS) {
            destroy_layouts(l);
            if (first_in_bucket) {
                hipblasLtMatmulDescDestroy(ch.desc);
                g->choices.erase(cit);
            }
            return as_hip(st);
        }
        int pick = 0;
        const bool timed = g->mode == kAuto || g->mode == kLibTimed;
        if (!timed) {
            // the heuristic's first choice for this exact shape
            ch.mfma = false;
            ch.algo = res[0].algo;
        } else if (first_in_bucket) {
            const bool with_mfma = fits && g->mode == kAuto;
            if (found > 1 || with_mfma) {
                e = time_candidates(*g, ch.desc, l, res, found, W, x, n, k, m, ldy, y_bf16, accumulate, with_mfma, s,
                                    pick);
                if (e != hipSuccess) {
                    destroy_layouts(l);
                    hipblasLtMatmulDescDestroy(ch.desc);
                    g->choices.erase(cit);
                    return e;
                }
            }
            ch.mfma = pick < 0;
            if (pick < 0) pick = 0;  // hipBLASLt's first choice stays the fallback
            ch.algo = res[pick].algo;
        } else {
            for (int i = 0; i < found; i++)
                if (res[i].state == HIPBLAS_STATUS_SUCCESS && same_algo(res[i].algo, ch.algo)) {
                    pick = i;
                    break;
                }
        }
        l.algo = res[pick].algo;
        l.ws = res[pick].workspaceSize;
        l.mfma = ch.mfma;
        lit = g->layouts.emplace(lkey, l).first;
    }
    const Layouts &l = lit->second;
    if (l.mfma && fits) return run_mfma(*g, W, n, k, x, m, y, ldy, y_bf16, accumulate, s);
    const float alpha = 1.0f, beta = accumulate ? 1.0f : 0.0f;
    KernelSpan span(y_bf16 ? "gemm_bf16_out_bf16" : "gemm_bf16_out_f32", s);
    hipblasStatus_t st = hipblasLtMatmul(g->handle, ch.desc, &alpha, W, l.a, x, l.b, &beta, y, l.c, y, l.c, &l.algo,
                                         g->workspace, l.ws, s);
    return as_hip(st);
}

}  // namespace hymt
