// gemm.hip -- the plain fp32 matrix products around the attention core (the
// QKV and output projections of the attention layers, and the per-head
// products of the attention backward), through hipBLASLt on the context's
// stream, with rocBLAS for any product hipBLASLt offers no algorithm for (or
// every product under MIMIR_TUNE blas=0).  These are library GEMMs: the
// path's own kernels are the fused core between them (attention.hip) and the
// backward's row passes (attention_bwd.hip).
//
// The reference computes them with LayerOps::matmul (LayerOps.hpp:977-1001):
// row-major C[M x N] = A[M x K] * B[K x N] in float32.  Both libraries are
// column-major, so the row-major product is taken as C^T = B^T A^T, which is
// the same memory.  Both compute in fp32 (HIPBLAS_COMPUTE_32F; rocBLAS's
// default math mode): no reduced-precision inner products.
//
// Measured on MI355X for the attention backward's per-head products (32
// heads of 1024 x 1024 x 128): hipBLASLt takes the transposed-operand score
// product S = Q K^T in 92 us where rocBLAS takes 168 (88 for the plain form
// on a transposed copy of K), and the key- and query-side products in 75-76
// us against 85-101; on half-size causal blocks it keeps its rate (77, 62
// and 64 us for 3/4 of the work) where rocBLAS drops to smaller tiles.
#include "internal.hpp"

#include <hipblaslt/hipblaslt.h>
#include <rocblas/rocblas.h>

#include <cstring>
#include <map>
#include <tuple>

namespace {

// The library workspace is this library's own allocation, so neither library
// reallocates it by itself: a captured graph (store.hip) holds its address.
// It starts at kWsBytes and grows when a product reports that it needs more
// (the old one is retired while graphs are alive).
constexpr size_t kWsBytes = size_t(32) << 20;
constexpr size_t kWsMax = size_t(4) << 30;

int ensure_workspace(mimir_ctx* ctx, size_t bytes) {
    if (ctx->blas_ws && ctx->blas_ws_bytes >= bytes) return MIMIR_OK;
    if (bytes < kWsBytes) bytes = kWsBytes;
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return mimir::fail(ctx, MIMIR_ENOMEM, "library workspace of %zu bytes: %s", bytes, hipGetErrorString(e));
    }
    if (ctx->blas && rocblas_set_workspace(static_cast<rocblas_handle>(ctx->blas), p, bytes) != rocblas_status_success) {
        (void)hipFree(p);
        return mimir::fail(ctx, MIMIR_EDEVICE, "rocblas_set_workspace failed");
    }
    if (int st = mimir::retire_or_free(ctx, ctx->blas_ws)) return st;
    ctx->blas_ws = p;
    ctx->blas_ws_bytes = bytes;
    return MIMIR_OK;
}

rocblas_handle rocblas_of(mimir_ctx* ctx, int* st) {
    if (!ctx->blas) {
        rocblas_handle h = nullptr;
        if (rocblas_create_handle(&h) != rocblas_status_success) {
            *st = mimir::fail(ctx, MIMIR_EDEVICE, "rocblas_create_handle failed");
            return nullptr;
        }
        if ((*st = ensure_workspace(ctx, kWsBytes)) != MIMIR_OK ||
            rocblas_set_workspace(h, ctx->blas_ws, ctx->blas_ws_bytes) != rocblas_status_success) {
            if (*st == MIMIR_OK) *st = mimir::fail(ctx, MIMIR_EDEVICE, "rocblas_set_workspace failed");
            (void)rocblas_destroy_handle(h);
            return nullptr;
        }
        ctx->blas = h;
    }
    rocblas_handle h = static_cast<rocblas_handle>(ctx->blas);
    if (rocblas_set_stream(h, ctx->stream) != rocblas_status_success) {
        *st = mimir::fail(ctx, MIMIR_EDEVICE, "rocblas_set_stream failed");
        return nullptr;
    }
    *st = MIMIR_OK;
    return h;
}

// One product shape's hipBLASLt descriptors and the algorithm its heuristic
// chose, kept for the context's life (`ok` false: no algorithm, rocBLAS).
struct LtPlan {
    bool ok = false;
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    size_t ws = 0;
};
// (trans_a, trans_b, m, n, k, lda, ldb, ldc, stride_a, stride_b, stride_c, batch) of the column-major call
using LtKey = std::tuple<int, int, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t,
                         int64_t>;
constexpr size_t kMaxPlans = 1024;
struct LtState {
    hipblasLtHandle_t handle = nullptr;
    bool failed = false;  // the handle could not be created: rocBLAS only
    std::map<LtKey, LtPlan> plans;
};

void destroy_plan(LtPlan& p) {
    if (p.a) (void)hipblasLtMatrixLayoutDestroy(p.a);
    if (p.b) (void)hipblasLtMatrixLayoutDestroy(p.b);
    if (p.c) (void)hipblasLtMatrixLayoutDestroy(p.c);
    if (p.desc) (void)hipblasLtMatmulDescDestroy(p.desc);
    p = LtPlan{};
}

LtState* lt_of(mimir_ctx* ctx) {
    if (ctx->tune.blas_lt == 0) return nullptr;
    if (!ctx->blaslt) {
        auto* s = new LtState;
        if (hipblasLtCreate(&s->handle) != HIPBLAS_STATUS_SUCCESS) {
            s->handle = nullptr;
            s->failed = true;
        }
        ctx->blaslt = s;
    }
    auto* s = static_cast<LtState*>(ctx->blaslt);
    return s->failed ? nullptr : s;
}

bool layout(hipblasLtMatrixLayout_t* l, int64_t rows, int64_t cols, int64_t ld, int64_t stride, int64_t batch) {
    if (hipblasLtMatrixLayoutCreate(l, HIP_R_32F, static_cast<uint64_t>(rows), static_cast<uint64_t>(cols), ld) !=
        HIPBLAS_STATUS_SUCCESS)
        return false;
    if (batch == 1) return true;
    const int32_t b32 = static_cast<int32_t>(batch);
    return hipblasLtMatrixLayoutSetAttribute(*l, HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT, &b32, sizeof b32) ==
               HIPBLAS_STATUS_SUCCESS &&
           hipblasLtMatrixLayoutSetAttribute(*l, HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET, &stride,
                                             sizeof stride) == HIPBLAS_STATUS_SUCCESS;
}

// The plan for column-major C[m x n] = op(A)[m x k] op(B)[k x n], made on
// first use (a host-side heuristic query, no device work).
LtPlan* plan_of(mimir_ctx* ctx, LtState* s, bool ta, bool tb, int64_t m, int64_t n, int64_t k, int64_t lda,
                int64_t ldb, int64_t ldc, int64_t sa, int64_t sb, int64_t sc, int64_t batch) {
    const LtKey key{ta, tb, m, n, k, lda, ldb, ldc, sa, sb, sc, batch};
    auto it = s->plans.find(key);
    if (it != s->plans.end()) return &it->second;
    // Shapes vary with sequence lengths: past kMaxPlans the cache starts over
    // rather than growing without bound (a plan is a host-side heuristic
    // query away).  Plans are only used within the call that looks them up.
    if (s->plans.size() >= kMaxPlans) {
        for (auto& kv : s->plans) destroy_plan(kv.second);
        s->plans.clear();
    }
    LtPlan p;
    const int32_t opa = ta ? HIPBLAS_OP_T : HIPBLAS_OP_N, opb = tb ? HIPBLAS_OP_T : HIPBLAS_OP_N;
    bool good = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS &&
                hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opa, sizeof opa) ==
                    HIPBLAS_STATUS_SUCCESS &&
                hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opb, sizeof opb) ==
                    HIPBLAS_STATUS_SUCCESS &&
                layout(&p.a, ta ? k : m, ta ? m : k, lda, sa, batch) &&
                layout(&p.b, tb ? n : k, tb ? k : n, ldb, sb, batch) && layout(&p.c, m, n, ldc, sc, batch);
    if (good) {
        hipblasLtMatmulPreference_t pref = nullptr;
        const uint64_t max_ws = ctx->blas_ws_bytes;
        hipblasLtMatmulHeuristicResult_t res[1];
        int found = 0;
        good = hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS &&
               hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &max_ws,
                                                     sizeof max_ws) == HIPBLAS_STATUS_SUCCESS &&
               hipblasLtMatmulAlgoGetHeuristic(s->handle, p.desc, p.a, p.b, p.c, p.c, pref, 1, res, &found) ==
                   HIPBLAS_STATUS_SUCCESS &&
               found > 0 && res[0].state == HIPBLAS_STATUS_SUCCESS && res[0].workspaceSize <= max_ws;
        if (pref) (void)hipblasLtMatmulPreferenceDestroy(pref);
        if (good) {
            p.algo = res[0].algo;
            p.ws = res[0].workspaceSize;
        }
    }
    if (!good) destroy_plan(p);  // keeps ok = false: this shape goes to rocBLAS
    p.ok = good;
    return &s->plans.emplace(key, p).first->second;
}

}  // namespace

namespace mimir {

int gemm_f32(mimir_ctx* ctx, int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, const float* B,
             int64_t ldb, float* C, int64_t ldc) {
    return gemm_f32_ex(ctx, false, false, M, N, K, 1.0f, A, lda, 0, B, ldb, 0, 0.0f, C, ldc, 0, 1);
}

bool gemm_lt(mimir_ctx* ctx) { return lt_of(ctx) != nullptr; }

int gemm_f32_ex(mimir_ctx* ctx, bool trans_a, bool trans_b, int64_t M, int64_t N, int64_t K, float alpha,
                const float* A, int64_t lda, int64_t stride_a, const float* B, int64_t ldb, int64_t stride_b,
                float beta, float* C, int64_t ldc, int64_t stride_c, int64_t batch) {
    if (M == 0 || N == 0 || batch == 0) return MIMIR_OK;
    const int64_t lim = INT32_MAX;
    if (M > lim || N > lim || K > lim || lda > lim || ldb > lim || ldc > lim || batch > lim)
        return fail(ctx, MIMIR_EINVAL, "matrix product: dimensions exceed the 32-bit library limit");
    // Row-major C = op(A) op(B) is column-major C^T = op(B)^T op(A)^T: the
    // operands swap and each keeps its own transpose flag.  K == 0 with
    // beta == 0 gives C = 0 (an empty sum), which rocBLAS takes.
    // hipBLASLt only where the output's batch matrices do not overlap: some
    // of its algorithms (split reductions) treat the output's batches as
    // disjoint ranges, which the attention layers' interleaved heads (row
    // stride the whole width, batch stride one head) are not.  Those products
    // take rocBLAS, which honours any stride.
    const bool disjoint = batch == 1 || stride_c >= ldc * M;
    if (K > 0 && disjoint) {
        if (LtState* s = lt_of(ctx)) {
            if (int st = ensure_workspace(ctx, kWsBytes)) return st;
            LtPlan* p = plan_of(ctx, s, trans_b, trans_a, N, M, K, ldb, lda, ldc, stride_b, stride_a, stride_c, batch);
            if (p->ok) {
                const hipblasStatus_t r = hipblasLtMatmul(s->handle, p->desc, &alpha, B, p->a, A, p->b, &beta, C, p->c,
                                                          C, p->c, &p->algo, ctx->blas_ws, ctx->blas_ws_bytes,
                                                          ctx->stream);
                if (r == HIPBLAS_STATUS_SUCCESS) return MIMIR_OK;
                return fail(ctx, MIMIR_EDEVICE, "hipBLASLt matmul failed (status %d)", (int)r);
            }
        }
    }
    int st = MIMIR_OK;
    rocblas_handle h = rocblas_of(ctx, &st);
    if (!h) return st;
    const rocblas_operation ob = trans_b ? rocblas_operation_transpose : rocblas_operation_none;
    const rocblas_operation oa = trans_a ? rocblas_operation_transpose : rocblas_operation_none;
    const auto n32 = static_cast<rocblas_int>(N), m32 = static_cast<rocblas_int>(M), k32 = static_cast<rocblas_int>(K);
    for (;;) {
        rocblas_status s;
        if (batch == 1)
            s = rocblas_sgemm(h, ob, oa, n32, m32, k32, &alpha, B, static_cast<rocblas_int>(ldb), A,
                              static_cast<rocblas_int>(lda), &beta, C, static_cast<rocblas_int>(ldc));
        else
            s = rocblas_sgemm_strided_batched(h, ob, oa, n32, m32, k32, &alpha, B, static_cast<rocblas_int>(ldb),
                                              stride_b, A, static_cast<rocblas_int>(lda), stride_a, &beta, C,
                                              static_cast<rocblas_int>(ldc), stride_c,
                                              static_cast<rocblas_int>(batch));
        if (s == rocblas_status_success) return MIMIR_OK;
        if (s != rocblas_status_memory_error || ctx->blas_ws_bytes >= kWsMax)
            return fail(ctx, MIMIR_EDEVICE, "rocBLAS sgemm failed (status %d)", (int)s);
        if (int st2 = ensure_workspace(ctx, ctx->blas_ws_bytes * 4)) return st2;  // grow and try again
    }
}

void gemm_release(mimir_ctx* ctx) {
    if (ctx->blaslt) {
        auto* s = static_cast<LtState*>(ctx->blaslt);
        for (auto& kv : s->plans) destroy_plan(kv.second);
        if (s->handle) (void)hipblasLtDestroy(s->handle);
        delete s;
        ctx->blaslt = nullptr;
    }
    if (ctx->blas) (void)rocblas_destroy_handle(static_cast<rocblas_handle>(ctx->blas));
    ctx->blas = nullptr;
    if (ctx->blas_ws) (void)hipFree(ctx->blas_ws);
    ctx->blas_ws = nullptr;
    ctx->blas_ws_bytes = 0;
}

}  // namespace mimir
