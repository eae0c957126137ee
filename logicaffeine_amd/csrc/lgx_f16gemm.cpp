// lgx_f16gemm.cpp -- the plain binary16 GEMM of the opt-in fast prefill,
// through hipBLASLt: y[m][n] (binary32, or binary16 rounded from the
// binary32 accumulation) = x[m][k] (binary16) . w[n][k]^T (binary16).  In
// hipBLASLt's column-major terms this is D (n x m, ld n) = op(A) . B with
// A = w stored k x n (ld k, op = T) and B = x stored k x m (ld k): the "TN"
// form, both operands k-contiguous.  One plan (descriptors + algorithm) per
// (m, n, k, output type), kept for the object's lifetime; the workspace is
// allocated once.  The algorithm is hipBLASLt's first heuristic pick, or
// with LGX_F16GEMM_TUNE=N the fastest of its first N picks, each timed
// twice on the first call's own operands (a synchronising step on that
// call's stream; the outputs it writes are the call's own).
#include <hipblaslt/hipblaslt.h>

#include <cstdlib>
#include <map>
#include <tuple>
#include <vector>

#include "lgx_internal.h"

namespace lgxi {

namespace {
constexpr size_t kWorkspace = 64ull << 20;

const char* blas_name(hipblasStatus_t s) {
    switch (s) {
        case HIPBLAS_STATUS_SUCCESS: return "success";
        case HIPBLAS_STATUS_NOT_INITIALIZED: return "not initialized";
        case HIPBLAS_STATUS_ALLOC_FAILED: return "allocation failed";
        case HIPBLAS_STATUS_INVALID_VALUE: return "invalid value";
        case HIPBLAS_STATUS_ARCH_MISMATCH: return "architecture mismatch";
        case HIPBLAS_STATUS_EXECUTION_FAILED: return "execution failed";
        case HIPBLAS_STATUS_NOT_SUPPORTED: return "not supported";
        default: return "error";
    }
}
}  // namespace

struct F16Gemm {
    struct Plan {
        hipblasLtMatmulDesc_t desc = nullptr;
        hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
        hipblasLtMatmulAlgo_t algo{};
    };
    hipblasLtHandle_t h = nullptr;
    void* ws = nullptr;
    std::map<std::tuple<int, int, int, bool>, Plan> plans;

    ~F16Gemm() {
        for (auto& kv : plans) {
            Plan& p = kv.second;
            if (p.a) (void)hipblasLtMatrixLayoutDestroy(p.a);
            if (p.b) (void)hipblasLtMatrixLayoutDestroy(p.b);
            if (p.c) (void)hipblasLtMatrixLayoutDestroy(p.c);
            if (p.desc) (void)hipblasLtMatmulDescDestroy(p.desc);
        }
        if (ws) (void)hipFree(ws);
        if (h) (void)hipblasLtDestroy(h);
    }
};

#define LGX_BLAS(call)                                                                           \
    do {                                                                                         \
        hipblasStatus_t s_ = (call);                                                             \
        if (s_ != HIPBLAS_STATUS_SUCCESS)                                                        \
            return fail(LGX_HIP_ERROR, "%s: %s", #call, blas_name(s_));                          \
    } while (0)

lgx_status f16gemm_create(F16Gemm** out) {
    F16Gemm* g = new F16Gemm();
    hipblasStatus_t s = hipblasLtCreate(&g->h);
    if (s != HIPBLAS_STATUS_SUCCESS) {
        delete g;
        return fail(LGX_HIP_ERROR, "hipblasLtCreate: %s", blas_name(s));
    }
    if (hipMalloc(&g->ws, kWorkspace) != hipSuccess) {
        g->ws = nullptr;
        delete g;
        return fail(LGX_OUT_OF_MEMORY, "binary16 GEMM workspace of %zu bytes", kWorkspace);
    }
    *out = g;
    return LGX_OK;
}

void f16gemm_destroy(F16Gemm* g) { delete g; }

static lgx_status make_plan(F16Gemm* g, const uint16_t* w, const uint16_t* x, void* y, int m, int n,
                            int k, bool y16, hipStream_t stream, F16Gemm::Plan& p) {
    LGX_BLAS(hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F));
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    LGX_BLAS(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)));
    LGX_BLAS(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)));
    LGX_BLAS(hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16F, (uint64_t)k, (uint64_t)n, (int64_t)k));
    LGX_BLAS(hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16F, (uint64_t)k, (uint64_t)m, (int64_t)k));
    LGX_BLAS(hipblasLtMatrixLayoutCreate(&p.c, y16 ? HIP_R_16F : HIP_R_32F, (uint64_t)n, (uint64_t)m,
                                         (int64_t)n));
    hipblasLtMatmulPreference_t pref = nullptr;
    LGX_BLAS(hipblasLtMatmulPreferenceCreate(&pref));
    const uint64_t wsb = kWorkspace;
    hipblasStatus_t s = hipblasLtMatmulPreferenceSetAttribute(
        pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb, sizeof(wsb));
    const char* tv = std::getenv("LGX_F16GEMM_TUNE");
    const int want = std::min(std::max(tv ? std::atoi(tv) : 1, 1), 16);
    std::vector<hipblasLtMatmulHeuristicResult_t> res(want);
    int nres = 0;
    if (s == HIPBLAS_STATUS_SUCCESS)
        s = hipblasLtMatmulAlgoGetHeuristic(g->h, p.desc, p.a, p.b, p.c, p.c, pref, want, res.data(), &nres);
    (void)hipblasLtMatmulPreferenceDestroy(pref);
    if (s != HIPBLAS_STATUS_SUCCESS || nres < 1)
        return fail(LGX_UNSUPPORTED, "no hipBLASLt algorithm for the binary16 GEMM m=%d n=%d k=%d (%s)",
                    m, n, k, blas_name(s));
    p.algo = res[0].algo;
    if (nres == 1) return LGX_OK;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
        if (e0) (void)hipEventDestroy(e0);
        return fail(LGX_HIP_ERROR, "GEMM tuning events");
    }
    const float alpha = 1.0f, beta = 0.0f;
    float best = 0.0f;
    for (int i = 0; i < nres; ++i) {
        if (res[i].workspaceSize > kWorkspace) continue;
        float tmin = 0.0f;
        for (int rep = 0; rep < 2; ++rep) {
            (void)hipEventRecord(e0, stream);
            const hipblasStatus_t r = hipblasLtMatmul(g->h, p.desc, &alpha, w, p.a, x, p.b, &beta, y, p.c, y,
                                                      p.c, &res[i].algo, g->ws, kWorkspace, stream);
            (void)hipEventRecord(e1, stream);
            float ms = 0.0f;
            if (r != HIPBLAS_STATUS_SUCCESS || hipEventSynchronize(e1) != hipSuccess ||
                hipEventElapsedTime(&ms, e0, e1) != hipSuccess) {
                tmin = -1.0f;
                break;
            }
            tmin = rep == 0 ? ms : std::min(tmin, ms);
        }
        if (tmin > 0.0f && (best == 0.0f || tmin < best)) {
            best = tmin;
            p.algo = res[i].algo;
        }
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return LGX_OK;
}

static lgx_status get_plan(F16Gemm* g, const uint16_t* w, const uint16_t* x, void* y, bool y16, int m,
                           int n, int k, void* stream, const F16Gemm::Plan** out) {
    if (m <= 0 || n <= 0 || k <= 0) return fail(LGX_INVALID_ARGUMENT, "GEMM m=%d n=%d k=%d", m, n, k);
    auto key = std::make_tuple(m, n, k, y16);
    auto it = g->plans.find(key);
    if (it == g->plans.end()) {
        F16Gemm::Plan p;
        const lgx_status st = make_plan(g, w, x, y, m, n, k, y16, (hipStream_t)stream, p);
        if (st != LGX_OK) {
            if (p.a) (void)hipblasLtMatrixLayoutDestroy(p.a);
            if (p.b) (void)hipblasLtMatrixLayoutDestroy(p.b);
            if (p.c) (void)hipblasLtMatrixLayoutDestroy(p.c);
            if (p.desc) (void)hipblasLtMatmulDescDestroy(p.desc);
            return st;
        }
        it = g->plans.emplace(key, p).first;
    }
    *out = &it->second;
    return LGX_OK;
}

lgx_status f16gemm_prepare(F16Gemm* g, const uint16_t* w, const uint16_t* x, void* y, bool y16, int m,
                           int n, int k, void* stream) {
    const F16Gemm::Plan* p = nullptr;
    return get_plan(g, w, x, y, y16, m, n, k, stream, &p);
}

lgx_status f16gemm_run(F16Gemm* g, const uint16_t* w, const uint16_t* x, void* y, bool y16, int m,
                       int n, int k, void* stream) {
    const F16Gemm::Plan* pp = nullptr;
    const lgx_status st = get_plan(g, w, x, y, y16, m, n, k, stream, &pp);
    if (st != LGX_OK) return st;
    const F16Gemm::Plan& p = *pp;
    const float alpha = 1.0f, beta = 0.0f;
    LGX_BLAS(hipblasLtMatmul(g->h, p.desc, &alpha, w, p.a, x, p.b, &beta, y, p.c, y, p.c, &p.algo, g->ws,
                             kWorkspace, (hipStream_t)stream));
    if (trace_on()) {
        int dev = -1;
        (void)hipGetDevice(&dev);
        trace_line("gemm dev=%d hipblaslt m=%d n=%d k=%d out=%s stream=%p", dev, m, n, k, y16 ? "f16" : "f32",
                   stream);
    }
    return LGX_OK;
}

}  // namespace lgxi
