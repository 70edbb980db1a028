// blaslt.cpp -- the vendor comparator: hipBLASLt FP16 GEMM, FP32 compute.
//
// Counterpart of the reference's cublasReference / cublasGemm
// (bench/check-gemm.cu:147-154, bench/measure.cu:104-109). Row-major C = A B is
// computed as the column-major C^T = B^T A^T by passing B as the first operand,
// so no transpose is materialised. Fairness rules from the build plan (D10/H10):
// a 64 MiB workspace, and the fastest of the heuristic's top candidates measured
// on the caller's own buffers (best of three interleaved passes), cached per
// (M, N, K, C type).

#include "ridge_gemm.h"

#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <tuple>
#include <vector>

namespace {

constexpr size_t kWorkspaceBytes = 64ull << 20;

struct Plan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    size_t workspace = 0;
};

struct Handle {
    hipblasLtHandle_t lt = nullptr;
    void* workspace = nullptr;
    std::map<std::tuple<int, int, int, int>, Plan> plans;
};

void destroyPlan(Plan& p) {
    if (p.la) hipblasLtMatrixLayoutDestroy(p.la);
    if (p.lb) hipblasLtMatrixLayoutDestroy(p.lb);
    if (p.lc) hipblasLtMatrixLayoutDestroy(p.lc);
    if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
    p = Plan{};
}

int makeLayouts(Plan& p, int M, int N, int K, int cF32) {
    hipblasStatus_t st = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F);
    if (st != HIPBLAS_STATUS_SUCCESS) return (int)st;
    const int32_t opN = HIPBLAS_OP_N;
    if ((st = hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opN, sizeof(opN))) !=
        HIPBLAS_STATUS_SUCCESS)
        return (int)st;
    if ((st = hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opN, sizeof(opN))) !=
        HIPBLAS_STATUS_SUCCESS)
        return (int)st;
    // Column-major view: first operand B^T is N x K (ld N), second A^T is K x M
    // (ld K), result C^T is N x M (ld N).
    if ((st = hipblasLtMatrixLayoutCreate(&p.la, HIP_R_16F, N, K, N)) != HIPBLAS_STATUS_SUCCESS) return (int)st;
    if ((st = hipblasLtMatrixLayoutCreate(&p.lb, HIP_R_16F, K, M, K)) != HIPBLAS_STATUS_SUCCESS) return (int)st;
    if ((st = hipblasLtMatrixLayoutCreate(&p.lc, cF32 ? HIP_R_32F : HIP_R_16F, N, M, N)) != HIPBLAS_STATUS_SUCCESS)
        return (int)st;
    return 0;
}

int run(Handle* h, const Plan& p, const void* A, const void* B, void* C, hipStream_t stream) {
    const float alpha = 1.0f, beta = 0.0f;
    return (int)hipblasLtMatmul(h->lt, p.desc, &alpha, B, p.la, A, p.lb, &beta, C, p.lc, C, p.lc, &p.algo,
                                h->workspace, p.workspace, stream);
}

}  // namespace

extern "C" {

int ridge_blaslt_create(void** handle) {
    if (handle == nullptr) return (int)hipErrorInvalidValue;
    Handle* h = new Handle();
    hipblasStatus_t st = hipblasLtCreate(&h->lt);
    if (st != HIPBLAS_STATUS_SUCCESS) {
        delete h;
        return (int)st;
    }
    hipError_t e = hipMalloc(&h->workspace, kWorkspaceBytes);
    if (e != hipSuccess) {
        hipblasLtDestroy(h->lt);
        delete h;
        return (int)e;
    }
    *handle = h;
    return 0;
}

int ridge_blaslt_destroy(void* handle) {
    Handle* h = static_cast<Handle*>(handle);
    if (h == nullptr) return 0;
    for (auto& kv : h->plans) destroyPlan(kv.second);
    hipError_t err = hipSuccess;
    if (h->workspace) err = hipFree(h->workspace);
    if (h->lt) hipblasLtDestroy(h->lt);
    delete h;
    return (int)err;
}

int ridge_blaslt_prepare(void* handle, const void* A, const void* B, void* C, int M, int N, int K, int c_is_f32,
                         int candidates, int iters, void* stream) {
    Handle* h = static_cast<Handle*>(handle);
    if (h == nullptr || M <= 0 || N <= 0 || K <= 0) return (int)hipErrorInvalidValue;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const auto key = std::make_tuple(M, N, K, c_is_f32 ? 1 : 0);
    auto it = h->plans.find(key);
    if (it != h->plans.end()) {
        destroyPlan(it->second);
        h->plans.erase(it);
    }
    Plan p;
    int rc = makeLayouts(p, M, N, K, c_is_f32);
    if (rc != 0) {
        destroyPlan(p);
        return rc;
    }
    hipblasLtMatmulPreference_t pref = nullptr;
    hipblasStatus_t pst = hipblasLtMatmulPreferenceCreate(&pref);
    const uint64_t ws = kWorkspaceBytes;
    if (pst == HIPBLAS_STATUS_SUCCESS)
        pst = hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws));
    if (pst != HIPBLAS_STATUS_SUCCESS) {
        if (pref) hipblasLtMatmulPreferenceDestroy(pref);
        destroyPlan(p);
        return (int)pst;
    }
    if (candidates < 1) candidates = 1;
    std::vector<hipblasLtMatmulHeuristicResult_t> res(candidates);
    int returned = 0;
    hipblasStatus_t st = hipblasLtMatmulAlgoGetHeuristic(h->lt, p.desc, p.la, p.lb, p.lc, p.lc, pref, candidates,
                                                         res.data(), &returned);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (st != HIPBLAS_STATUS_SUCCESS || returned == 0) {
        destroyPlan(p);
        return st != HIPBLAS_STATUS_SUCCESS ? (int)st : (int)HIPBLAS_STATUS_NOT_SUPPORTED;
    }
    // Each usable candidate is timed over `iters` launches in kPasses
    // interleaved passes and keeps its fastest pass: one pass per candidate let
    // the clock's state at that moment pick between kernels a few percent apart
    // (the same box chose a 110 us kernel in one call and a 120 us one in another).
    constexpr int kPasses = 3;
    std::vector<float> fastest(returned, 1e30f);
    std::vector<char> usable(returned, 0);
    int best = -1;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t err = hipEventCreate(&e0);
    if (err == hipSuccess) err = hipEventCreate(&e1);
    for (int c = 0; c < returned && err == hipSuccess; ++c) {
        if (res[c].state != HIPBLAS_STATUS_SUCCESS || res[c].workspaceSize > kWorkspaceBytes) continue;
        p.algo = res[c].algo;
        p.workspace = res[c].workspaceSize;
        if (run(h, p, A, B, C, s) != 0) continue;  // warm-up and validity probe
        usable[c] = 1;
        if (iters < 1) {
            best = c;
            break;
        }
    }
    for (int pass = 0; pass < kPasses && iters >= 1 && err == hipSuccess; ++pass) {
        for (int c = 0; c < returned && err == hipSuccess; ++c) {
            if (!usable[c]) continue;
            p.algo = res[c].algo;
            p.workspace = res[c].workspaceSize;
            err = hipEventRecord(e0, s);
            for (int i = 0; i < iters && err == hipSuccess; ++i)
                if (run(h, p, A, B, C, s) != 0) err = hipErrorLaunchFailure;
            if (err == hipSuccess) err = hipEventRecord(e1, s);
            if (err == hipSuccess) err = hipEventSynchronize(e1);
            float ms = 0.0f;
            if (err == hipSuccess) err = hipEventElapsedTime(&ms, e0, e1);
            if (err == hipSuccess && ms < fastest[c]) fastest[c] = ms;
        }
    }
    if (iters >= 1) {
        for (int c = 0; c < returned; ++c)
            if (usable[c] && (best < 0 || fastest[c] < fastest[best])) best = c;
    }
    if (e0) (void)hipEventDestroy(e0);  // teardown: nothing to recover from
    if (e1) (void)hipEventDestroy(e1);
    if (err != hipSuccess) {
        destroyPlan(p);
        return (int)err;
    }
    if (best < 0) {
        destroyPlan(p);
        return (int)HIPBLAS_STATUS_NOT_SUPPORTED;
    }
    p.algo = res[best].algo;
    p.workspace = res[best].workspaceSize;
    h->plans[key] = p;
    return 0;
}

int ridge_blaslt_gemm(void* handle, const void* A, const void* B, void* C, int M, int N, int K, int c_is_f32,
                      void* stream) {
    Handle* h = static_cast<Handle*>(handle);
    if (h == nullptr) return (int)hipErrorInvalidValue;
    const auto key = std::make_tuple(M, N, K, c_is_f32 ? 1 : 0);
    auto it = h->plans.find(key);
    if (it == h->plans.end()) {
        const int rc = ridge_blaslt_prepare(handle, A, B, C, M, N, K, c_is_f32, 1, 0, stream);
        if (rc != 0) return rc;
        it = h->plans.find(key);
    }
    return run(h, it->second, A, B, C, static_cast<hipStream_t>(stream));
}

}  // extern "C"
