// linear_lt.hip - the linear and linear_silu slots through the platform GEMM
// library (hipBLASLt) for wide 16-bit shapes.
//
// The slots are plain GEMMs y[n][co] = x[n][ci] W^T + b (then SiLU):
// src/ops/sparse/trellis_sparse_cpu.c:122-171 (linear, silu at :165-169).
// For Ci, Co >= 256 the library's tuned GEMMs (both operands staged through
// LDS in large output tiles) beat this library's MFMA linear kernel, whose
// weights reach each wavefront through the vector-memory path: on 316k rows
// 512 -> 2048 (SiLU) 844 against 525 TFLOP/s, 2048 -> 512 1241 against 670.
// Bias and SiLU (hipBLASLt's Swish with beta 1, x * sigmoid(x)) run in the
// library's epilogue on the fp32 sums; the result is rounded to the storage
// type to nearest even.  (This library's own kernels keep a positive value
// that would round to +0 as the smallest positive subnormal; below the
// smallest subnormal that is the only difference, and the subdivide logits,
// where it matters, are an 8-wide linear that never comes here.)
//
// Column-major view of the row-major buffers: W [co][ci] is a ci x co matrix
// (ld ci) used transposed, x [n][ci] a ci x n matrix (ld ci), y [n][co] a
// co x n matrix (ld co): y^T = W x^T, m = co, n = n, k = ci; the bias runs
// along m.  With a residual r [n][co] (same layout as y) the call computes
// y = r + x W^T + b with beta = 1: the residual is added to the fp32 sums
// before the one rounding.  Plans (descriptor, layouts, the heuristic's
// algorithm) are kept per shape.
#include "tsh_internal.h"

#include <hipblaslt/hipblaslt.h>

#include <map>
#include <tuple>

namespace tsh {

struct LinearLt {
    hipblasLtHandle_t handle = nullptr;
    struct Plan {
        hipblasLtMatmulDesc_t desc = nullptr;
        hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, ld = nullptr;
        hipblasLtMatmulAlgo_t algo{};
        size_t workspace = 0;
        bool ok = false;
    };
    std::map<std::tuple<int, int64_t, int, int, int, int>, Plan> plans;
    ~LinearLt() {
        for (auto & kv : plans) {
            Plan & p = kv.second;
            if (p.la != nullptr) hipblasLtMatrixLayoutDestroy(p.la);
            if (p.lb != nullptr) hipblasLtMatrixLayoutDestroy(p.lb);
            if (p.ld != nullptr) hipblasLtMatrixLayoutDestroy(p.ld);
            if (p.desc != nullptr) hipblasLtMatmulDescDestroy(p.desc);
        }
        if (handle != nullptr) hipblasLtDestroy(handle);
    }
};

bool linear_lt_wanted(int dtype, int64_t n, int ci, int co) {
    return (dtype == kF16 || dtype == kBF16) && ci >= 256 && co >= 256 && n >= 2048 && n <= INT32_MAX;
}

LinearLt * linear_lt_create() {
    LinearLt * lt = new LinearLt();
    if (hipblasLtCreate(&lt->handle) != HIPBLAS_STATUS_SUCCESS) {
        lt->handle = nullptr;
    }
    return lt;
}

void linear_lt_destroy(LinearLt * lt) { delete lt; }

// Plan for one shape, or nullptr when the library has none (the caller then
// runs its own kernel).  workspace_bytes: what the caller can lend.
static LinearLt::Plan * plan_for(LinearLt * lt, int dtype, int64_t n, int ci, int co, int silu, bool bias,
                                 size_t workspace_bytes) {
    if (lt == nullptr || lt->handle == nullptr) return nullptr;
    const auto key = std::make_tuple(dtype, n, ci, co, silu, bias ? 1 : 0);
    auto it = lt->plans.find(key);
    if (it != lt->plans.end()) return it->second.ok ? &it->second : nullptr;
    LinearLt::Plan & p = lt->plans[key];
    const hipDataType t = dtype == kBF16 ? HIP_R_16BF : HIP_R_16F;
    bool good = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS;
    const int32_t op_t = HIPBLAS_OP_T, op_n = HIPBLAS_OP_N;
    good = good && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &op_t, sizeof(op_t)) ==
                       HIPBLAS_STATUS_SUCCESS;
    good = good && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &op_n, sizeof(op_n)) ==
                       HIPBLAS_STATUS_SUCCESS;
    const uint32_t epi = silu ? (bias ? HIPBLASLT_EPILOGUE_SWISH_BIAS_EXT : HIPBLASLT_EPILOGUE_SWISH_EXT)
                              : (bias ? HIPBLASLT_EPILOGUE_BIAS : HIPBLASLT_EPILOGUE_DEFAULT);
    good = good && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi)) ==
                       HIPBLAS_STATUS_SUCCESS;
    if (bias) {
        const int32_t bt = HIP_R_32F;
        good = good && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt,
                                                       sizeof(bt)) == HIPBLAS_STATUS_SUCCESS;
    }
    if (silu) {
        const float beta1 = 1.0f;  // Swish(x, 1) = x * sigmoid(x)
        good = good && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE_ACT_ARG0_EXT, &beta1,
                                                       sizeof(beta1)) == HIPBLAS_STATUS_SUCCESS;
    }
    good = good && hipblasLtMatrixLayoutCreate(&p.la, t, (uint64_t) ci, (uint64_t) co, ci) == HIPBLAS_STATUS_SUCCESS;
    good = good && hipblasLtMatrixLayoutCreate(&p.lb, t, (uint64_t) ci, (uint64_t) n, ci) == HIPBLAS_STATUS_SUCCESS;
    good = good && hipblasLtMatrixLayoutCreate(&p.ld, t, (uint64_t) co, (uint64_t) n, co) == HIPBLAS_STATUS_SUCCESS;
    if (good) {
        hipblasLtMatmulPreference_t pref = nullptr;
        good = hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS;
        const uint64_t ws = workspace_bytes;
        good = good && hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws,
                                                             sizeof(ws)) == HIPBLAS_STATUS_SUCCESS;
        hipblasLtMatmulHeuristicResult_t res[1];
        int found = 0;
        good = good && hipblasLtMatmulAlgoGetHeuristic(lt->handle, p.desc, p.la, p.lb, p.ld, p.ld, pref, 1, res,
                                                       &found) == HIPBLAS_STATUS_SUCCESS &&
               found > 0 && res[0].state == HIPBLAS_STATUS_SUCCESS && res[0].workspaceSize <= workspace_bytes;
        if (good) {
            p.algo = res[0].algo;
            p.workspace = res[0].workspaceSize;
        }
        if (pref != nullptr) hipblasLtMatmulPreferenceDestroy(pref);
    }
    p.ok = good;
    return good ? &p : nullptr;
}

// Enqueues the GEMM on stream s (residual: nullptr, or r of y = r + x W^T + b;
// it may be y itself).  Returns false (nothing enqueued) when the library has
// no plan for the shape or refuses the call; the caller then runs its own
// kernel.
bool linear_lt_run(LinearLt * lt, int dtype, const void * x, const void * w16, const float * bias,
                   const void * residual, void * y, int64_t n, int ci, int co, int silu, void * workspace,
                   size_t workspace_bytes, hipStream_t s) {
    LinearLt::Plan * p = plan_for(lt, dtype, n, ci, co, silu, bias != nullptr, workspace_bytes);
    if (p == nullptr) return false;
    if (bias != nullptr &&
        hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias)) !=
            HIPBLAS_STATUS_SUCCESS) {
        return false;
    }
    const float alpha = 1.0f, beta = residual != nullptr ? 1.0f : 0.0f;
    const void * c = residual != nullptr ? residual : y;
    return hipblasLtMatmul(lt->handle, p->desc, &alpha, w16, p->la, x, p->lb, &beta, c, p->ld, y, p->ld, &p->algo,
                           workspace, p->workspace, s) == HIPBLAS_STATUS_SUCCESS;
}

}  // namespace tsh
