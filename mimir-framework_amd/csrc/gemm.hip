// gemm.hip -- the plain fp32 matrix products around the attention core (the
// QKV and output projections of the attention layers, and the per-head
// products of the attention backward), through rocBLAS on the context's
// stream.  These are library GEMMs: the path's own kernels are the fused core
// between them (attention.hip) and the backward's row passes
// (attention_bwd.hip).
//
// The reference computes them with LayerOps::matmul (LayerOps.hpp:977-1001):
// row-major C[M x N] = A[M x K] * B[K x N] in float32.  rocBLAS is
// column-major, so the row-major product is taken as C^T = B^T A^T, which is
// the same memory.  rocBLAS's default math mode keeps fp32 arithmetic (no
// reduced-precision inner products).
#include "internal.hpp"

#include <rocblas/rocblas.h>

namespace {

// The handle's workspace is this library's own allocation, so the library
// never reallocates it by itself: a captured graph (store.hip) holds its
// address.  It starts at kWsBytes and grows when a product reports that it
// needs more (the old one is retired while graphs are alive).
constexpr size_t kWsBytes = size_t(32) << 20;
constexpr size_t kWsMax = size_t(4) << 30;

int set_workspace(mimir_ctx* ctx, rocblas_handle h, size_t bytes) {
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return mimir::fail(ctx, MIMIR_ENOMEM, "library workspace of %zu bytes: %s", bytes, hipGetErrorString(e));
    }
    if (rocblas_set_workspace(h, p, bytes) != rocblas_status_success) {
        (void)hipFree(p);
        return mimir::fail(ctx, MIMIR_EDEVICE, "rocblas_set_workspace failed");
    }
    if (int st = mimir::retire_or_free(ctx, ctx->blas_ws)) return st;
    ctx->blas_ws = p;
    ctx->blas_ws_bytes = bytes;
    return MIMIR_OK;
}

rocblas_handle handle_of(mimir_ctx* ctx, int* st) {
    if (!ctx->blas) {
        rocblas_handle h = nullptr;
        if (rocblas_create_handle(&h) != rocblas_status_success) {
            *st = mimir::fail(ctx, MIMIR_EDEVICE, "rocblas_create_handle failed");
            return nullptr;
        }
        if ((*st = set_workspace(ctx, h, kWsBytes)) != MIMIR_OK) {
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

}  // namespace

namespace mimir {

int gemm_f32(mimir_ctx* ctx, int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, const float* B,
             int64_t ldb, float* C, int64_t ldc) {
    return gemm_f32_ex(ctx, false, false, M, N, K, 1.0f, A, lda, 0, B, ldb, 0, 0.0f, C, ldc, 0, 1);
}

int gemm_f32_ex(mimir_ctx* ctx, bool trans_a, bool trans_b, int64_t M, int64_t N, int64_t K, float alpha,
                const float* A, int64_t lda, int64_t stride_a, const float* B, int64_t ldb, int64_t stride_b,
                float beta, float* C, int64_t ldc, int64_t stride_c, int64_t batch) {
    if (M == 0 || N == 0 || batch == 0) return MIMIR_OK;
    const int64_t lim = INT32_MAX;
    if (M > lim || N > lim || K > lim || lda > lim || ldb > lim || ldc > lim || batch > lim)
        return fail(ctx, MIMIR_EINVAL, "matrix product: dimensions exceed the 32-bit library limit");
    int st = MIMIR_OK;
    rocblas_handle h = handle_of(ctx, &st);
    if (!h) return st;
    // Row-major C = op(A) op(B) is column-major C^T = op(B)^T op(A)^T: the
    // operands swap and each keeps its own transpose flag.  K == 0 with
    // beta == 0 gives C = 0 (an empty sum).
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
        if (int st2 = set_workspace(ctx, h, ctx->blas_ws_bytes * 4)) return st2;  // grow and try again
    }
}

void gemm_release(mimir_ctx* ctx) {
    if (ctx->blas) (void)rocblas_destroy_handle(static_cast<rocblas_handle>(ctx->blas));
    ctx->blas = nullptr;
    if (ctx->blas_ws) (void)hipFree(ctx->blas_ws);
    ctx->blas_ws = nullptr;
    ctx->blas_ws_bytes = 0;
}

}  // namespace mimir
