// softmax.hip -- max-subtracted row softmax / log-softmax for gfx950.
//
// Same row layout as norm.hip (rows.hpp): TPR threads hold the row in VGPRs
// as 16-byte vectors;
// the row max and the sum of exponentials are wave-uniform DPP reductions, so
// each element is read from HBM once and written once.  Rows too wide for
// the register budget are split over many workgroups (longrow.hip); rows of
// a width that is not a multiple of 4, or unaligned, are held in registers
// with 4-byte columns up to 4096 floats (softmax_rows_scalar); wider
// unaligned rows take one workgroup per row with three strided passes.
//
// Arithmetic (per row): m = max_j x[j]; e[j] = expf(x[j] - m); s = sum e[j];
//   MIMIR_SOFTMAX_DIV_EPS  y = e / (s + 1e-9f)    LayerOps::softmax_inplace,
//                                                  LayerOps.hpp:952-974
//   MIMIR_SOFTMAX_MUL_INV  y = e * (1.0f / s)     LayerOps::softmax_forward,
//                                                  LayerOps.hpp:325-361
//   MIMIR_SOFTMAX_LOG      y = (x - m) - logf(s)  LogSoftmax, LayerOps.hpp:345-353
#include "common.hpp"
#include "internal.hpp"

#include <math.h>

using namespace mimir;

namespace {

struct SoftmaxArgs {
    const float* x;
    float* y;
    int64_t rows;
    int64_t cols;
};

template <int MODE>
__device__ __forceinline__ float finish(float xv, float e, float m, float s, float inv_or_log) {
    if constexpr (MODE == MIMIR_SOFTMAX_DIV_EPS) return e / s;  // s already holds sum + 1e-9f
    else if constexpr (MODE == MIMIR_SOFTMAX_MUL_INV) return e * inv_or_log;
    else return (xv - m) - inv_or_log;
}

template <int MODE>
__device__ __forceinline__ void row_constants(float sum, float* s, float* aux) {
    if constexpr (MODE == MIMIR_SOFTMAX_DIV_EPS) {
        *s = sum + 1e-9f;
        *aux = 0.0f;
    } else if constexpr (MODE == MIMIR_SOFTMAX_MUL_INV) {
        *s = sum;
        *aux = 1.0f / sum;
    } else {
        *s = sum;
        *aux = logf(sum);
    }
}

// KEEP: y through the caches (mimir_ctx_set_output_caching).
template <int MODE, int TPR, int VPT, int BS, bool KEEP>
__global__ __launch_bounds__(BS) void softmax_rows_vec(SoftmaxArgs a) {
    constexpr int RPB = BS / TPR;
    constexpr int NW = TPR / kWave;
    __shared__ float lds[2][BS / kWave];
    const int t = threadIdx.x % TPR;
    const int sub = threadIdx.x / TPR;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + sub;
    if constexpr (NW == 1) {
        if (row >= a.rows) return;
    }
    const int64_t c4n = row < a.rows ? (a.cols >> 2) : 0;  // rows past the end touch no memory
    const int64_t base = row * a.cols;

    f4 v[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t c4 = static_cast<int64_t>(j) * TPR + t;
        v[j] = (c4 < c4n) ? ld4<true>(a.x + base + 4 * c4) : f4(-INFINITY);
    }
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < VPT; ++j) m = fmaxf(m, fmaxf(fmaxf(v[j].x, v[j].y), fmaxf(v[j].z, v[j].w)));
    m = row_max<NW>(m, lds[0], sub);

    f4 e[VPT];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t c4 = static_cast<int64_t>(j) * TPR + t;
        if (c4 < c4n) {
#pragma unroll
            for (int k = 0; k < 4; ++k) e[j][k] = expf(v[j][k] - m);
            s += (e[j].x + e[j].y) + (e[j].z + e[j].w);
        } else {
            e[j] = f4(0.0f);
        }
    }
    float sum, aux;
    row_constants<MODE>(row_sum<NW>(s, lds[1], sub), &sum, &aux);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t c4 = static_cast<int64_t>(j) * TPR + t;
        if (c4 < c4n) {
            f4 o;
#pragma unroll
            for (int k = 0; k < 4; ++k) o[k] = finish<MODE>(v[j][k], e[j][k], m, sum, aux);
            st_out<KEEP>(a.y + base + 4 * c4, o);
        }
    }
}

template <int MODE>
__global__ __launch_bounds__(kBlock) void softmax_rows_generic(SoftmaxArgs a) {
    constexpr int NW = kBlock / kWave;
    __shared__ float lds[2][NW];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * a.cols;
    const float* x = a.x + base;
    float* y = a.y + base;
    float m = -INFINITY;
    for (int64_t c = threadIdx.x; c < a.cols; c += kBlock) m = fmaxf(m, x[c]);
    m = block_max<NW>(m, lds[0]);
    float s = 0.0f;
    for (int64_t c = threadIdx.x; c < a.cols; c += kBlock) s += expf(x[c] - m);
    float sum, aux;
    row_constants<MODE>(block_sum<NW>(s, lds[1]), &sum, &aux);
    for (int64_t c = threadIdx.x; c < a.cols; c += kBlock) {
        const float xv = x[c];
        y[c] = finish<MODE>(xv, expf(xv - m), m, sum, aux);
    }
}

// Rows the vector kernel cannot take (a width that is not a multiple of 4,
// or unaligned pointers), up to kBlock*VPT floats: the row held in registers
// with 4-byte columns, one kBlock-thread workgroup per row -- one read of
// the row, and the same max / sum / finish as softmax_rows_generic.
template <int MODE, int VPT, bool KEEP>
__global__ __launch_bounds__(kBlock) void softmax_rows_scalar(SoftmaxArgs a) {
    constexpr int NW = kBlock / kWave;
    __shared__ float lds[2][NW];
    const int t = threadIdx.x;
    const int64_t base = static_cast<int64_t>(blockIdx.x) * a.cols;
    float v[VPT], e[VPT];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t c = static_cast<int64_t>(j) * kBlock + t;
        v[j] = c < a.cols ? __builtin_nontemporal_load(a.x + base + c) : 0.0f;
        if (c < a.cols) m = fmaxf(m, v[j]);
    }
    m = block_max<NW>(m, lds[0]);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        e[j] = 0.0f;
        if (static_cast<int64_t>(j) * kBlock + t < a.cols) {
            e[j] = expf(v[j] - m);
            s += e[j];
        }
    }
    float sum, aux;
    row_constants<MODE>(block_sum<NW>(s, lds[1]), &sum, &aux);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t c = static_cast<int64_t>(j) * kBlock + t;
        if (c < a.cols) {
            const float o = finish<MODE>(v[j], e[j], m, sum, aux);
            if constexpr (KEEP) a.y[base + c] = o;
            else st_stream(a.y + base + c, o);
        }
    }
}

template <int MODE, int VPT>
int launch_scalar(mimir_ctx* ctx, const SoftmaxArgs& a) {
    const unsigned grid = static_cast<unsigned>(a.rows);
    if (ctx->keep_outputs) softmax_rows_scalar<MODE, VPT, true><<<grid, kBlock, 0, ctx->stream>>>(a);
    else softmax_rows_scalar<MODE, VPT, false><<<grid, kBlock, 0, ctx->stream>>>(a);
    return launched(ctx, "softmax_rows_scalar");
}

template <int MODE, int TPR, int VPT, int BS>
int launch_vec(mimir_ctx* ctx, const SoftmaxArgs& a) {
    unsigned blocks;
    if (!grid_for(a.rows, BS / TPR, BS, &blocks))
        return fail(ctx, MIMIR_EINVAL, "softmax: %lld rows exceed the grid limit", (long long)a.rows);
    if (ctx->keep_outputs) softmax_rows_vec<MODE, TPR, VPT, BS, true><<<blocks, BS, 0, ctx->stream>>>(a);
    else softmax_rows_vec<MODE, TPR, VPT, BS, false><<<blocks, BS, 0, ctx->stream>>>(a);
    return launched(ctx, "softmax_rows_vec");
}

template <int MODE>
int dispatch(mimir_ctx* ctx, const SoftmaxArgs& a) {
    const int64_t c4 = a.cols / 4;
    const bool vec = (a.cols % 4) == 0 && aligned16(a.x) && aligned16(a.y);
    if (vec) {
        const RowShape s = shape_fits(ctx->tune.softmax, c4) ? ctx->tune.softmax : default_softmax_shape(c4);
#define MIMIR_SOFTMAX_CASE(T, V, B) \
        if (s.tpr == T && s.vpt == V && s.bs == B) return launch_vec<MODE, T, V, B>(ctx, a);
        MIMIR_ROW_SHAPES(MIMIR_SOFTMAX_CASE)
#undef MIMIR_SOFTMAX_CASE
        if (longrow_applies(a.rows, a.cols)) return longrow_softmax(ctx, MODE, a.x, a.y, a.rows, a.cols);
    }
    if (!dispatch_fits(a.rows, kBlock))
        return fail(ctx, MIMIR_EINVAL, "softmax: %lld rows exceed the grid limit", (long long)a.rows);
    if (!vec && a.cols <= 4 * kBlock) return launch_scalar<MODE, 4>(ctx, a);
    if (!vec && a.cols <= 8 * kBlock) return launch_scalar<MODE, 8>(ctx, a);
    if (!vec && a.cols <= 16 * kBlock) return launch_scalar<MODE, 16>(ctx, a);
    softmax_rows_generic<MODE><<<static_cast<unsigned>(a.rows), kBlock, 0, ctx->stream>>>(a);
    return launched(ctx, "softmax_rows_generic");
}

}  // namespace

extern "C" int mimir_softmax_fwd(mimir_ctx* ctx, const float* x, float* y, int64_t rows,
                                 int64_t cols, int mode) {
    if (!ctx) return MIMIR_EINVAL;
    MIMIR_REQUIRE(ctx, rows >= 0 && cols > 0, "Softmax: invalid shape (rows=%lld, cols=%lld)",
                  (long long)rows, (long long)cols);
    MIMIR_REQUIRE(ctx, mode == MIMIR_SOFTMAX_DIV_EPS || mode == MIMIR_SOFTMAX_MUL_INV ||
                           mode == MIMIR_SOFTMAX_LOG,
                  "Softmax: unknown mode %d", mode);
    if (rows == 0) return MIMIR_OK;
    MIMIR_REQUIRE(ctx, x && y, "Softmax: null tensor");
    MIMIR_ENTER(ctx);
    const SoftmaxArgs a{x, y, rows, cols};
    switch (mode) {
        case MIMIR_SOFTMAX_DIV_EPS: return dispatch<MIMIR_SOFTMAX_DIV_EPS>(ctx, a);
        case MIMIR_SOFTMAX_MUL_INV: return dispatch<MIMIR_SOFTMAX_MUL_INV>(ctx, a);
        default: return dispatch<MIMIR_SOFTMAX_LOG>(ctx, a);
    }
}
