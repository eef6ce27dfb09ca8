// longrow.hip -- row reductions split over many workgroups, for rows too
// long for one workgroup's registers (more than 16384 floats).
//
// The reference's RMSNorm and Softmax layers normalise the whole input as one
// row (LayerOpsExt.hpp:345-378, LayerOps.hpp:325-361), and so does LayerNorm
// when in_features is unset (LayerOps.hpp:276); a transformer's activations
// make that row millions of elements long.  One workgroup per row would leave
// all but one CU idle, so such rows are cut into chunks of 4096 floats (one
// workgroup per chunk, or two for LayerNorm, for the statistics):
//   1. partial : per chunk, the partial statistic (sum, sum of squares,
//                sum of squared deviations, or softmax's (max, sum of exp));
//   2. combine : one 1024-thread workgroup per row folds the chunk partials
//                in a fixed order (per-thread strided sums with eight loads in
//                flight, then the DPP/LDS tree), so the result does not
//                depend on scheduling;
//   3. apply   : per quarter chunk (128 threads x 2 float4), the elementwise
//                normalisation with the row stats.
// LayerNorm's variance is two-pass within each chunk: the chunk is held in
// registers, so its sum and its squared deviations about its own mean come
// from one read.  The combine merges the chunks in float64 by the pairwise
// formula of Chan, Golub and LeVeque (1979):
//   M2 = sum_c M2_c + sum_c n_c (mean_c - mean)^2,
// which equals the reference's sum((x - mean)^2) (LayerOps.hpp:296-303) up
// to float rounding inside a chunk, without a second read of the row.  The
// sums are taken of x - x0, x0 the row's first element (shifted data), and
// the row mean reaches the apply pass as a float pair hi + lo, so a row whose
// mean is large against its spread keeps its precision.  Every
// op reads x twice (statistics, then apply) and writes y once; the second
// read walks the row backwards, so that its first part can come from the MALL
// (measured on one 2^25-float row, 128 MiB: the apply pass moves its 256 MiB
// of read and write at 7.3 TB/s, above the HBM stream rate).
// Partials live in the context's scratch buffer, reused in stream order.
#include "common.hpp"
#include "internal.hpp"

#include <math.h>

using namespace mimir;

namespace {

constexpr int kChunkVec = 4;                          // float4 per thread per chunk
constexpr int64_t kChunk4 = kChunkVec * kBlock;       // float4 per chunk (1024)
constexpr int64_t kChunkFloats = 4 * kChunk4;         // 4096 floats

enum Stat { kChan = 0, kSumSq = 1, kSumSqAdd = 3, kSoftmax = 4 };

struct LongArgs {
    const float* x;
    const float* r;
    float* r_out;
    const float* g;
    const float* b;
    int64_t w_len;
    float* y;
    int64_t rows;
    int64_t cols;
    int64_t nchunks;
    float eps;
    float* partial;  // [rows][nchunks][2]
    float* stats;    // [rows][4]
    int reverse;     // this pass walks the chunks last to first
};

// Passes alternate direction: a pass starts where the previous one ended, so
// the start of its walk is still in the 256 MiB Infinity Cache (MALL) and
// only the part of the row beyond the cache comes again from HBM.
__device__ __forceinline__ int64_t chunk_of(const LongArgs& a) {
    return a.reverse ? a.nchunks - 1 - static_cast<int64_t>(blockIdx.x) : static_cast<int64_t>(blockIdx.x);
}

// Number of floats in a chunk (the last one may be short).
__device__ __forceinline__ float chunk_len(const LongArgs& a, int64_t chunk) {
    const int64_t left = a.cols - chunk * kChunkFloats;
    return static_cast<float>(left < kChunkFloats ? left : kChunkFloats);
}

// Sum of one double per thread over a workgroup of BS threads, in a fixed
// tree order; every thread gets the total.
template <int BS>
__device__ __forceinline__ double block_sum_f64(double v, double* lds) {
    lds[threadIdx.x] = v;
    __syncthreads();
#pragma unroll
    for (int h = BS / 2; h > 0; h >>= 1) {
        if (static_cast<int>(threadIdx.x) < h) lds[threadIdx.x] += lds[threadIdx.x + h];
        __syncthreads();
    }
    const double t = lds[0];
    __syncthreads();  // lds is reused by the caller's next reduction
    return t;
}

// Pass 1: one chunk's partial statistic.
// CPW chunks per workgroup (chunks CPW*b .. CPW*b + CPW - 1 of the row, in
// the forward order): every chunk's loads are issued before the first
// chunk's reductions, so a workgroup keeps CPW chunks in flight; each
// chunk's partial is the one-chunk computation, bit for bit.
// BS threads hold a chunk, VPT = kChunk4 / BS float4 each (the chunk, its
// partial's definition and the combine are the same for every BS; only the
// order of the sums inside a chunk differs).
template <int S, int CPW = 1, int BS = kBlock>
__global__ __launch_bounds__(BS) void lr_partial(LongArgs a) {
    constexpr int VPT = static_cast<int>(kChunk4) / BS;
    static_assert(VPT * BS == kChunk4, "a chunk fills the workgroup's slots");
    __shared__ float lds[2][BS / kWave];
    const int64_t row = blockIdx.y;
    const int64_t c4n = a.cols >> 2;
    const int64_t base = row * a.cols;
    f4 vv[CPW][VPT];
    bool okk[CPW][VPT];
#pragma unroll
    for (int i = 0; i < CPW; ++i) {
        const int64_t chunk = CPW == 1 ? chunk_of(a) : static_cast<int64_t>(blockIdx.x) * CPW + i;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int64_t c4 = chunk * kChunk4 + static_cast<int64_t>(j) * BS + threadIdx.x;
            okk[i][j] = chunk < a.nchunks && c4 < c4n;
            if constexpr (S == kSumSqAdd) {
                if (okk[i][j]) {
                    vv[i][j] = ld4<false>(a.x + base + 4 * c4) + ld4<false>(a.r + base + 4 * c4);
                    st4<false>(a.r_out + base + 4 * c4, vv[i][j]);  // the updated residual, re-read by the last pass
                }
            } else {
                if (okk[i][j]) vv[i][j] = ld4<false>(a.x + base + 4 * c4);  // kept in the caches for the next pass
            }
        }
    }
#pragma unroll
    for (int i = 0; i < CPW; ++i) {
        const int64_t chunk = CPW == 1 ? chunk_of(a) : static_cast<int64_t>(blockIdx.x) * CPW + i;
        f4* v = vv[i];
        const bool* ok = okk[i];
        float p0 = 0.0f, p1 = 0.0f;
        if constexpr (S == kSoftmax) {
            float m = -INFINITY;
#pragma unroll
            for (int j = 0; j < VPT; ++j)
                if (ok[j]) m = fmaxf(m, fmaxf(fmaxf(v[j].x, v[j].y), fmaxf(v[j].z, v[j].w)));
            m = block_max<BS / kWave>(m, lds[0]);
            float s = 0.0f;
            if (m != -INFINITY) {  // an all -inf chunk contributes nothing
#pragma unroll
                for (int j = 0; j < VPT; ++j)
                    if (ok[j])
                        s += (expf(v[j].x - m) + expf(v[j].y - m)) + (expf(v[j].z - m) + expf(v[j].w - m));
            }
            p0 = m;
            p1 = block_sum<BS / kWave>(s, lds[1]);
        } else if constexpr (S == kChan) {
            const float x0 = a.x[base];  // the shift
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < VPT; ++j) {
                if (!ok[j]) continue;
                v[j] -= x0;
                s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
            }
            p0 = block_sum<BS / kWave>(s, lds[0]);
            const float mc = chunk < a.nchunks ? p0 / chunk_len(a, chunk) : 0.0f;  // recomputed bit for bit by the combine
            float q = 0.0f;
#pragma unroll
            for (int j = 0; j < VPT; ++j) {
                if (!ok[j]) continue;
                const f4 d = v[j] - mc;
                q += (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
            }
            p1 = block_sum<BS / kWave>(q, lds[1]);
        } else {
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < VPT; ++j)
                if (ok[j]) s += (v[j].x * v[j].x + v[j].y * v[j].y) + (v[j].z * v[j].z + v[j].w * v[j].w);
            p0 = block_sum<BS / kWave>(s, lds[0]);
        }
        if (threadIdx.x == 0 && chunk < a.nchunks) {
            float* p = a.partial + 2 * (row * a.nchunks + chunk);
            p[0] = p0;
            p[1] = p1;
        }
    }
}
// Pass 2: fold one row's chunk partials (fixed order) into its statistics.
//   kChan  -> stats = (mean hi, mean lo, 1/sqrt(var+eps))
//   kSumSq / kSumSqAdd -> stats = (rms, -) kSoftmax -> stats = (max, sum)
// Thread t folds chunks t, t + kCombine, t + 2*kCombine, ... in that order,
// then the workgroup tree adds the threads; kCombineU partials per thread are
// loaded before the first is folded, so a row of up to kCombine*kCombineU
// chunks (32M floats) costs one memory round trip per pass instead of one
// per chunk.
constexpr int kCombine = 1024;
constexpr int kCombineU = 8;

// The first pass over `rows` rows: CPW chunks per workgroup (MIMIR_TUNE
// lrcpw=1/2/4 overrides).  Measured on MI355X on one 2^25-float row: the
// LayerNorm statistic (two block reductions per chunk) gains from two chunks
// per workgroup, 75.2 -> 69.8 us for the whole op, while the one-reduction
// passes lose 1-2% (softmax 67.2 -> 68.7 us, RMSNorm 65.0 -> 65.9 us) and
// all lose at four.
template <int S, int BS>
void launch_partial_bs(mimir_ctx* ctx, const LongArgs& a, int64_t rows, int cpw) {
    const dim3 grid(static_cast<unsigned>((a.nchunks + cpw - 1) / cpw), static_cast<unsigned>(rows));
    if (cpw == 4) lr_partial<S, 4, BS><<<grid, BS, 0, ctx->stream>>>(a);
    else if (cpw == 2) lr_partial<S, 2, BS><<<grid, BS, 0, ctx->stream>>>(a);
    else lr_partial<S, 1, BS><<<grid, BS, 0, ctx->stream>>>(a);
}

// Threads per chunk (MIMIR_TUNE lrpart=256 / 512 overrides): 512 (2 float4
// each) for the LayerNorm statistic, 256 (4 each) for the others.  Measured
// on MI355X on one 2^25-float row, whole op, 256 / 512 threads: LayerNorm
// 67.3-67.5 / 66.7 us, softmax 65.3-65.7 / 65.6-66.1, RMSNorm 62.6 / 62.4-62.5
// (128 threads, 8 float4 each: 1.3-2 us slower for LayerNorm and softmax).
template <int S>
void launch_partial(mimir_ctx* ctx, const LongArgs& a, int64_t rows) {
    const int over = ctx->tune.lr_cpw;
    const int cpw = over == 1 || over == 2 || over == 4 ? over : (S == kChan ? 2 : 1);
    const int bs = ctx->tune.lr_part_bs == 256 || ctx->tune.lr_part_bs == 512 ? ctx->tune.lr_part_bs
                                                                             : (S == kChan ? 512 : kBlock);
    if (bs == 512) launch_partial_bs<S, 512>(ctx, a, rows, cpw);
    else launch_partial_bs<S, kBlock>(ctx, a, rows, cpw);
}

template <int S>
__global__ __launch_bounds__(kCombine) void lr_combine(LongArgs a) {
    constexpr int NW = kCombine / kWave;
    __shared__ float lds[2][NW];
    const int64_t row = blockIdx.x;
    const float2* p = reinterpret_cast<const float2*>(a.partial) + row * a.nchunks;
    const int64_t nc = a.nchunks;
    // f(chunk, partial) for this thread's chunks, in chunk order.
    auto each = [&](auto&& f) {
        for (int64_t c0 = threadIdx.x; c0 < nc; c0 += static_cast<int64_t>(kCombine) * kCombineU) {
            float2 v[kCombineU];
#pragma unroll
            for (int u = 0; u < kCombineU; ++u) {
                const int64_t c = c0 + static_cast<int64_t>(u) * kCombine;
                if (c < nc) v[u] = p[c];
            }
#pragma unroll
            for (int u = 0; u < kCombineU; ++u) {
                const int64_t c = c0 + static_cast<int64_t>(u) * kCombine;
                if (c < nc) f(c, v[u]);
            }
        }
    };
    const float n = static_cast<float>(a.cols);
    if constexpr (S == kSoftmax) {
        float m = -INFINITY;
        each([&](int64_t, float2 q) { m = fmaxf(m, q.x); });
        m = block_max<NW>(m, lds[0]);
        float s = 0.0f;
        each([&](int64_t, float2 q) {
            if (q.x != -INFINITY) s += q.y * expf(q.x - m);
        });
        s = block_sum<NW>(s, lds[1]);
        if (threadIdx.x == 0) {
            a.stats[4 * row] = m;
            a.stats[4 * row + 1] = s;
        }
    } else if constexpr (S == kChan) {
        __shared__ double lds64[kCombine];
        double s = 0.0;
        each([&](int64_t, float2 q) { s += static_cast<double>(q.x); });
        const double mean = block_sum_f64<kCombine>(s, lds64) / static_cast<double>(a.cols);
        double m2 = 0.0;
        each([&](int64_t c, float2 q) {
            const float ncl = chunk_len(a, c);
            const double d = static_cast<double>(q.x / ncl) - mean;  // the chunk mean the partial used
            m2 += static_cast<double>(q.y) + static_cast<double>(ncl) * d * d;
        });
        m2 = block_sum_f64<kCombine>(m2, lds64);
        if (threadIdx.x == 0) {
            const double mu = static_cast<double>(a.x[row * a.cols]) + mean;  // undo the shift
            const float hi = static_cast<float>(mu);
            a.stats[4 * row] = hi;
            a.stats[4 * row + 1] = static_cast<float>(mu - static_cast<double>(hi));
            a.stats[4 * row + 2] = 1.0f / sqrtf(static_cast<float>(m2 / static_cast<double>(a.cols)) + a.eps);
        }
    } else {
        float s = 0.0f;
        each([&](int64_t, float2 q) { s += q.x; });
        s = block_sum<NW>(s, lds[0]);
        if (threadIdx.x == 0) a.stats[4 * row] = sqrtf(s / n + a.eps);
    }
}

template <int MODE>
__device__ __forceinline__ float softmax_out(float xv, float m, float s) {
    if constexpr (MODE == MIMIR_SOFTMAX_DIV_EPS) return expf(xv - m) / (s + 1e-9f);
    else if constexpr (MODE == MIMIR_SOFTMAX_MUL_INV) return expf(xv - m) * (1.0f / s);
    else return (xv - m) - logf(s);
}

// Pass 3: normalise one chunk.  K: 0 LayerNorm, 1 RMSNorm, 2 add+RMSNorm, 3 softmax.
// KEEP: y through the caches (mimir_ctx_set_output_caching).
// Each workgroup of BS threads takes a piece of BS*VPT float4 of the row,
// VPT per thread a workgroup-width apart (256 x 4: one chunk).  Pieces are
// walked as chunks are (chunk_of).
template <int K, int MODE, bool KEEP, int BS = kBlock, int VPT = kChunkVec>
__global__ __launch_bounds__(BS) void lr_apply(LongArgs a) {
    const int64_t row = blockIdx.y;
    const int64_t c4n = a.cols >> 2;
    const int64_t npieces = (c4n + BS * VPT - 1) / (BS * VPT);
    const int64_t piece = a.reverse ? npieces - 1 - static_cast<int64_t>(blockIdx.x) : static_cast<int64_t>(blockIdx.x);
    const int64_t base = row * a.cols;
    const float s0 = a.stats[4 * row];
    const float s1 = a.stats[4 * row + 1];
    const float s2 = a.stats[4 * row + 2];
    const float* src = (K == 2) ? a.r_out : a.x;  // add+RMSNorm re-reads the residual it wrote
    f4 v[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t c4 = piece * (BS * VPT) + static_cast<int64_t>(j) * BS + threadIdx.x;
        if (c4 < c4n) v[j] = ld4<true>(src + base + 4 * c4);
    }
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t c4 = piece * (BS * VPT) + static_cast<int64_t>(j) * BS + threadIdx.x;
        if (c4 >= c4n) continue;
        const int64_t c = 4 * c4;
        f4 o;
        if constexpr (K == 0) {
            o = ((v[j] - s0) - s1) * s2;
            if (a.g) {
                o *= *reinterpret_cast<const f4*>(a.g + c);
                if (a.b) o += *reinterpret_cast<const f4*>(a.b + c);
            }
        } else if constexpr (K == 1 || K == 2) {
            o = v[j] / s0;
            if (a.g) {
                if (c + 3 < a.w_len) {  // weights cover the whole vector: one 16-byte load
                    o *= *reinterpret_cast<const f4*>(a.g + c);
                } else {
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        if (c + k < a.w_len) o[k] *= a.g[c + k];
                }
            }
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) o[k] = softmax_out<MODE>(v[j][k], s0, s1);
        }
        st_out<KEEP>(a.y + base + c, o);
    }
}

int setup(mimir_ctx* ctx, LongArgs& a, int64_t rows, int64_t cols) {
    a.rows = rows;
    a.cols = cols;
    a.nchunks = (cols + kChunkFloats - 1) / kChunkFloats;
    const size_t bytes = sizeof(float) * (2 * static_cast<size_t>(rows) * a.nchunks + 4 * rows);
    void* s = nullptr;
    if (int st = ensure_scratch(ctx, bytes, &s)) return st;
    a.partial = static_cast<float*>(s);
    a.stats = a.partial + 2 * rows * a.nchunks;
    return MIMIR_OK;
}

}  // namespace

// Rows wider than a register-resident workgroup takes, however many: the
// grid is chunks x rows (rows up to 65535, the grid's y limit used here).
bool mimir::longrow_applies(int64_t rows, int64_t cols) {
    return cols > 16384 && rows <= 65535 && dispatch_fits((cols + kChunkFloats - 1) / kChunkFloats, kBlock);
}

namespace {

template <int K, int MODE, int BS, int VPT>
void launch_apply_shape(mimir_ctx* ctx, const LongArgs& a) {
    const int64_t npieces = ((a.cols >> 2) + BS * VPT - 1) / (BS * VPT);
    const dim3 grid(static_cast<unsigned>(npieces), static_cast<unsigned>(a.rows));
    if (ctx->keep_outputs) lr_apply<K, MODE, true, BS, VPT><<<grid, BS, 0, ctx->stream>>>(a);
    else lr_apply<K, MODE, false, BS, VPT><<<grid, BS, 0, ctx->stream>>>(a);
}

// The apply pass's workgroup shape: 128 threads x 2 float4 (a quarter of a
// chunk) by default, measured on MI355X on one 2^25-float row against one
// chunk per 256 x 4: softmax 66.7 -> 64.6-64.9 us, RMSNorm 64.4-65.0 ->
// 62.0-62.2, LayerNorm 69.4-69.6 -> 66.9-67.0 for the whole op (256 x 1,
// 128 x 1, 512 x 1 and 1024 x 1 in between).  MIMIR_TUNE lrapply=256x4
// selects the chunk shape, which is also the fallback when a row has more
// quarter chunks than one launch dimension holds.
template <int K, int MODE>
void launch_apply(mimir_ctx* ctx, dim3, const LongArgs& a) {
    constexpr int BS = 128, VPT = 2;
    const bool chunk = ctx->tune.lr_apply_bs == kBlock && ctx->tune.lr_apply_vpt == kChunkVec;
    if (!chunk && dispatch_fits(((a.cols >> 2) + BS * VPT - 1) / (BS * VPT), BS))
        launch_apply_shape<K, MODE, BS, VPT>(ctx, a);
    else
        launch_apply_shape<K, MODE, kBlock, kChunkVec>(ctx, a);  // longrow_applies checked this one
}

}  // namespace

int mimir::longrow_norm(mimir_ctx* ctx, int kind, const float* x, const float* r, float* r_out,
                        const float* g, const float* b, int64_t w_len, float* y, int64_t rows, int64_t cols,
                        float eps) {
    LongArgs a{x, r, r_out, g, b, w_len, y, 0, 0, 0, eps, nullptr, nullptr, 0};
    if (int st = setup(ctx, a, rows, cols)) return st;
    const dim3 grid(static_cast<unsigned>(a.nchunks), static_cast<unsigned>(rows));
    const unsigned nrows = static_cast<unsigned>(rows);
    LongArgs fwd = a, rev = a;
    rev.reverse = 1;
    if (kind == 0) {
        launch_partial<kChan>(ctx, fwd, rows);
        lr_combine<kChan><<<nrows, kCombine, 0, ctx->stream>>>(fwd);
        launch_apply<0, 0>(ctx, grid, rev);
    } else if (kind == 1) {
        launch_partial<kSumSq>(ctx, fwd, rows);
        lr_combine<kSumSq><<<nrows, kCombine, 0, ctx->stream>>>(fwd);
        launch_apply<1, 0>(ctx, grid, rev);
    } else {
        launch_partial<kSumSqAdd>(ctx, fwd, rows);
        lr_combine<kSumSqAdd><<<nrows, kCombine, 0, ctx->stream>>>(fwd);
        launch_apply<2, 0>(ctx, grid, rev);
    }
    return launched(ctx, "longrow_norm");
}

int mimir::longrow_softmax(mimir_ctx* ctx, int mode, const float* x, float* y, int64_t rows, int64_t cols) {
    LongArgs a{x, nullptr, nullptr, nullptr, nullptr, 0, y, 0, 0, 0, 0.0f, nullptr, nullptr, 0};
    if (int st = setup(ctx, a, rows, cols)) return st;
    const dim3 grid(static_cast<unsigned>(a.nchunks), static_cast<unsigned>(rows));
    LongArgs rev = a;
    rev.reverse = 1;
    launch_partial<kSoftmax>(ctx, a, rows);
    lr_combine<kSoftmax><<<static_cast<unsigned>(rows), kCombine, 0, ctx->stream>>>(a);
    switch (mode) {
        case MIMIR_SOFTMAX_DIV_EPS: launch_apply<3, MIMIR_SOFTMAX_DIV_EPS>(ctx, grid, rev); break;
        case MIMIR_SOFTMAX_MUL_INV: launch_apply<3, MIMIR_SOFTMAX_MUL_INV>(ctx, grid, rev); break;
        default: launch_apply<3, MIMIR_SOFTMAX_LOG>(ctx, grid, rev); break;
    }
    return launched(ctx, "longrow_softmax");
}

// ---------------------------------------------------------------------------
// LayerNorm backward over long rows (Model.cpp:7719-7821 with a group of the
// whole input, or of more than 16384 floats): the row statistics come from
// the forward's passes (lr_partial / lr_combine<kChan>), then
//   lr_bwd_partial : per chunk, sum(dxh) and sum(dxh * xh), dxh = dy * gamma;
//   lr_bwd_combine : per row, their totals, added in float64 in chunk order;
//   lr_bwd_apply   : per (chunk, group of kLongBwdRows rows), dx =
//                    inv_std/n * ((n*dxh - S1) - xh*S2) for its rows in
//                    order, and the chunk's column sums of dy*xh and dy over
//                    those rows, each column owned by one thread: added into
//                    dgamma / dbeta when there is one group, else written to
//                    the group's slot for the caller's slot sums.
// ---------------------------------------------------------------------------
namespace {

struct LongBwdArgs {
    const float* x;
    const float* dy;
    const float* g;  // gamma, or null (no affine transform)
    float* dx;
    float* dgamma;   // += ; null: not wanted
    float* dbeta;    // += ; null: not wanted
    int64_t rows;
    int64_t cols;
    int64_t nchunks;
    const float* stats;  // [rows][4]: mean hi, mean lo, inv_std
    float* partial;      // [rows][nchunks][2]
    float* sums;         // [rows][2]: S1, S2
    int acc;             // dx += instead of dx =
    int params16;        // dgamma / dbeta 16-byte aligned: vector read-modify-writes
    float* slots;        // [groups][2*cols] column sums per row group, or null (add into dgamma / dbeta)
};

__device__ __forceinline__ float sum4(f4 v) { return (v.x + v.y) + (v.z + v.w); }

__global__ __launch_bounds__(kBlock) void lr_bwd_partial(LongBwdArgs a) {
    __shared__ float lds[2][kBlock / kWave];
    const int64_t row = blockIdx.y;
    const int64_t chunk = blockIdx.x;
    const int64_t c4n = a.cols >> 2;
    const int64_t base = row * a.cols;
    const float m0 = a.stats[4 * row], m1 = a.stats[4 * row + 1], inv = a.stats[4 * row + 2];
    float p = 0.0f, q = 0.0f;
#pragma unroll
    for (int j = 0; j < kChunkVec; ++j) {
        const int64_t c4 = chunk * kChunk4 + static_cast<int64_t>(j) * kBlock + threadIdx.x;
        if (c4 < c4n) {
            const f4 xv = ld4<false>(a.x + base + 4 * c4);  // kept in the caches for the apply pass
            const f4 gv = ld4<false>(a.dy + base + 4 * c4);
            const f4 dxh = a.g ? gv * *reinterpret_cast<const f4*>(a.g + 4 * c4) : gv;
            const f4 xh = ((xv - m0) - m1) * inv;
            p += sum4(dxh);
            q += sum4(dxh * xh);
        }
    }
    p = block_sum<kBlock / kWave>(p, lds[0]);
    q = block_sum<kBlock / kWave>(q, lds[1]);
    if (threadIdx.x == 0) {
        a.partial[2 * (row * a.nchunks + chunk)] = p;
        a.partial[2 * (row * a.nchunks + chunk) + 1] = q;
    }
}

__global__ __launch_bounds__(kCombine) void lr_bwd_combine(LongBwdArgs a) {
    __shared__ double lds64[kCombine];
    const int64_t row = blockIdx.x;
    const float2* p = reinterpret_cast<const float2*>(a.partial) + row * a.nchunks;
    double s = 0.0, t = 0.0;
    for (int64_t c0 = threadIdx.x; c0 < a.nchunks; c0 += static_cast<int64_t>(kCombine) * kCombineU) {
        float2 v[kCombineU];
#pragma unroll
        for (int u = 0; u < kCombineU; ++u) {
            const int64_t c = c0 + static_cast<int64_t>(u) * kCombine;
            if (c < a.nchunks) v[u] = p[c];
        }
#pragma unroll
        for (int u = 0; u < kCombineU; ++u) {
            if (c0 + static_cast<int64_t>(u) * kCombine < a.nchunks) {
                s += static_cast<double>(v[u].x);
                t += static_cast<double>(v[u].y);
            }
        }
    }
    s = block_sum_f64<kCombine>(s, lds64);
    t = block_sum_f64<kCombine>(t, lds64);
    if (threadIdx.x == 0) {
        a.sums[2 * row] = static_cast<float>(s);
        a.sums[2 * row + 1] = static_cast<float>(t);
    }
}

template <bool KEEP>
__global__ __launch_bounds__(kBlock) void lr_bwd_apply(LongBwdArgs a) {
    const int64_t chunk = blockIdx.x;
    const int64_t c4n = a.cols >> 2;
    const float n = static_cast<float>(a.cols);
    const float invF = 1.0f / n;
    f4 gm[kChunkVec], dg[kChunkVec], db[kChunkVec];
#pragma unroll
    for (int j = 0; j < kChunkVec; ++j) {
        const int64_t c4 = chunk * kChunk4 + static_cast<int64_t>(j) * kBlock + threadIdx.x;
        gm[j] = (a.g && c4 < c4n) ? *reinterpret_cast<const f4*>(a.g + 4 * c4) : f4(1.0f);
        dg[j] = f4(0.0f);
        db[j] = f4(0.0f);
    }
    const int64_t r0 = static_cast<int64_t>(blockIdx.y) * kLongBwdRows;
    const int64_t r1 = r0 + kLongBwdRows < a.rows ? r0 + kLongBwdRows : a.rows;
    for (int64_t row = r0; row < r1; ++row) {
        const int64_t base = row * a.cols;
        const float m0 = a.stats[4 * row], m1 = a.stats[4 * row + 1], inv = a.stats[4 * row + 2];
        const float S1 = a.sums[2 * row], S2 = a.sums[2 * row + 1];
        const float k = inv * invF;
#pragma unroll
        for (int j = 0; j < kChunkVec; ++j) {
            const int64_t c4 = chunk * kChunk4 + static_cast<int64_t>(j) * kBlock + threadIdx.x;
            if (c4 >= c4n) continue;
            const f4 xv = ld4<true>(a.x + base + 4 * c4);
            const f4 gv = ld4<true>(a.dy + base + 4 * c4);
            const f4 xh = ((xv - m0) - m1) * inv;
            const f4 dxh = gv * gm[j];
            dg[j] += gv * xh;
            db[j] += gv;
            f4 o = k * ((n * dxh - S1) - xh * S2);
            if (a.acc) o = ld4<true>(a.dx + base + 4 * c4) + o;
            st_out<KEEP>(a.dx + base + 4 * c4, o);
        }
    }
    if (a.slots) {  // this row group's slot: dgamma sums, then dbeta sums (16-byte aligned)
        f4* sg = reinterpret_cast<f4*>(a.slots + static_cast<int64_t>(blockIdx.y) * 2 * a.cols);
#pragma unroll
        for (int j = 0; j < kChunkVec; ++j) {
            const int64_t c4 = chunk * kChunk4 + static_cast<int64_t>(j) * kBlock + threadIdx.x;
            if (c4 >= c4n) continue;
            sg[c4] = dg[j];
            sg[c4n + c4] = db[j];
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < kChunkVec; ++j) {
        const int64_t c4 = chunk * kChunk4 + static_cast<int64_t>(j) * kBlock + threadIdx.x;
        if (c4 >= c4n) continue;
        if (a.params16) {
            if (a.dgamma) *reinterpret_cast<f4*>(a.dgamma + 4 * c4) += dg[j];
            if (a.dbeta) *reinterpret_cast<f4*>(a.dbeta + 4 * c4) += db[j];
            continue;
        }
        for (int e = 0; e < 4; ++e) {
            if (a.dgamma) a.dgamma[4 * c4 + e] += dg[j][e];
            if (a.dbeta) a.dbeta[4 * c4 + e] += db[j][e];
        }
    }
}

}  // namespace

int mimir::longrow_ln_bwd(mimir_ctx* ctx, const float* x, const float* dy, const float* gamma, float* dx,
                          float* dgamma, float* dbeta, int64_t rows, int64_t cols, float eps, int accumulate,
                          float** slots, int64_t* nslots, float** tmp, const ScratchSpan* fixed) {
    const int64_t groups = (rows + kLongBwdRows - 1) / kLongBwdRows;
    const bool use_slots = groups > 1 && dgamma;
    *slots = nullptr;
    *nslots = 0;
    *tmp = nullptr;
    LongArgs a{x, nullptr, nullptr, nullptr, nullptr, 0, nullptr, 0, 0, 0, eps, nullptr, nullptr, 0};
    a.rows = rows;
    a.cols = cols;
    a.nchunks = (cols + kChunkFloats - 1) / kChunkFloats;
    // partials [rows][nchunks][2] (the statistics pass's, then this pass's),
    // stats [rows][4], sums [rows][2]; then, with slots, [groups][2*cols] and
    // the slot sums' [kSlotGroups][2*cols], each 256-byte aligned.
    const size_t head = (sizeof(float) * (2 * static_cast<size_t>(rows) * a.nchunks + 6 * rows) + 255) & ~size_t(255);
    const size_t slot_bytes = use_slots ? sizeof(float) * static_cast<size_t>(groups) * 2 * cols : 0;
    const size_t tmp_bytes = use_slots ? sizeof(float) * static_cast<size_t>(kSlotGroups) * 2 * cols : 0;
    void* s = nullptr;
    if (int st = get_scratch(ctx, fixed, head + slot_bytes + tmp_bytes, &s)) return st;
    a.partial = static_cast<float*>(s);
    a.stats = a.partial + 2 * rows * a.nchunks;
    float* slot_base = use_slots ? reinterpret_cast<float*>(static_cast<char*>(s) + head) : nullptr;
    const dim3 grid(static_cast<unsigned>(a.nchunks), static_cast<unsigned>(rows));
    launch_partial<kChan>(ctx, a, rows);
    lr_combine<kChan><<<static_cast<unsigned>(rows), kCombine, 0, ctx->stream>>>(a);
    LongBwdArgs b{x, dy, gamma, dx, dgamma, dbeta, rows, cols, a.nchunks, a.stats, a.partial,
                  a.stats + 4 * rows, accumulate ? 1 : 0, aligned16(dgamma) && aligned16(dbeta) ? 1 : 0, slot_base};
    lr_bwd_partial<<<grid, kBlock, 0, ctx->stream>>>(b);
    lr_bwd_combine<<<static_cast<unsigned>(rows), kCombine, 0, ctx->stream>>>(b);
    const dim3 agrid(static_cast<unsigned>(a.nchunks), static_cast<unsigned>(groups));
    if (ctx->keep_outputs) lr_bwd_apply<true><<<agrid, kBlock, 0, ctx->stream>>>(b);
    else lr_bwd_apply<false><<<agrid, kBlock, 0, ctx->stream>>>(b);
    if (int st = launched(ctx, "longrow_ln_bwd")) return st;
    if (use_slots) {
        *slots = slot_base;
        *nslots = groups;
        *tmp = reinterpret_cast<float*>(reinterpret_cast<char*>(slot_base) + slot_bytes);
    }
    return MIMIR_OK;
}
