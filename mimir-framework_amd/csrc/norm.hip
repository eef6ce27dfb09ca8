// norm.hip -- LayerNorm, RMSNorm and residual-add + RMSNorm for gfx950.
//
// Row layout (rows.hpp): a row of `cols` fp32 is held in VGPRs by TPR
// threads, each owning VPT 16-byte vectors at float4 columns t, t+TPR, ...,
// so every load instruction of a wave covers 1 KiB of contiguous row.  Each
// input byte crosses HBM once: the row is loaded, reduced (DPP wave
// reductions, LDS only to combine the waves of one row) and written from
// registers.  Rows too wide for that register budget are split over many
// workgroups (longrow.hip).  Rows whose width is not a multiple of 4 or whose
// buffers are not 16-byte aligned are held in registers with 4-byte columns
// up to 4096 floats (norm_rows_scalar); wider unaligned rows take the generic
// kernel: one workgroup per row, scalar strided passes.
//
// Arithmetic follows the reference step by step:
//   LayerNorm  LayerOps::layernorm_forward, LayerOps.hpp:264-319
//              mean = sum/n; var = sum((x-mean)^2)/n (two-pass);
//              inv_std = 1/sqrt(var+eps); y = (x-mean)*inv_std [*g [+b]]
//   RMSNorm    LayerOpsExt::rms_norm_forward, LayerOpsExt.hpp:345-378 and
//              Normalization::rms_norm, Layers.hpp:1003-1021
//              rms = sqrt(sum(x^2)/n + eps); y = x/rms [*w]
//   add+RMS    h = x + r (LayerOps::add_forward, LayerOps.hpp:154-169), then
//              RMSNorm of h; h is also written out (the updated residual).
#include "common.hpp"
#include "internal.hpp"
#include "pointwise.hpp"

using namespace mimir;


namespace {

// AddLayer: the runtime's fused Add -> LayerNorm (h = x + r, written when
// r_out is set, then LayerNorm of h).
enum class Norm { Layer, Rms, AddRms, AddLayer };

struct NormArgs {
    const float* x;
    const float* r;   // AddRms: residual in
    float* r_out;     // AddRms: residual out (x + r)
    const float* g;   // gamma / weight (may be null)
    const float* b;   // beta (LayerNorm, may be null)
    float* y;
    int64_t rows;
    int64_t cols;
    int64_t w_len;    // RMSNorm: weight applies to columns < w_len
    float eps;
    float inv_n;      // 1 / cols (set at launch)
    const float* wp;  // RMSNorm weight shorter than the row (set at launch; g is then 1.0)
    // LayerNorm epilogue (the runtime's fusion): a chain of elementwise
    // steps on the normalised value before it is stored (y, when set, gets
    // the LayerNorm output itself); operands index epi.ins.
    FuseProgram epi;
};

// Scale by the RMSNorm weight where the column is below w_len.
__device__ __forceinline__ f4 rms_scale(f4 o, const float* w, int64_t w_len, int64_t c) {
    if (c + 3 < w_len) {
        const f4 g = *reinterpret_cast<const f4*>(w + c);
        o *= g;
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (c + k < w_len) o[k] *= w[c + k];
    }
    return o;
}

// 1.0f and -0.0f for every column a vector row kernel holds, on each GPU,
// standing in for an absent scale and bias (filled at context creation).
__device__ __align__(16) float unit_weights[2][kUnitCols];

__global__ __launch_bounds__(kBlock) void fill_unit_weights(float* p) {
    const int i = blockIdx.x * kBlock + threadIdx.x;
    if (i < kUnitCols) {
        p[i] = 1.0f;
        p[kUnitCols + i] = -0.0f;
    }
}

// The instruction budget of these kernels is tight: at 8 TB/s one SIMD's
// share of HBM moves a wave's 4 KiB (1 KiB loaded and stored per row slice
// and tensor) in about 1300 cycles, ~320 wave64 VALU instructions, so every
// per-element divide and bounds mask shows in the rate.  FULL: the row fills
// every thread slot (cols == 4*TPR*VPT and no row past the end), so no
// column is masked.  Per element the divisions of the reference become
// multiplications by per-row reciprocals (1/n from the host, v_rsq for
// 1/sqrt): within 2 ulp of the divided form.
//
// KEEP: y through the caches (mimir_ctx_set_output_caching); r_out is always
// streamed (it is read by a later block, not the next op).  EPI: the
// LayerNorm output goes through a.epi before it is stored.
template <Norm K, int TPR, int VPT, int BS, bool KEEP, bool EPI, bool FULL>
__global__ __launch_bounds__(BS) void norm_rows_vec(NormArgs a) {
    constexpr int RPB = BS / TPR;  // rows per workgroup
    constexpr int NW = TPR / kWave;  // waves per row
    __shared__ __attribute__((aligned(16))) float lds[2][BS / kWave];
    const int t = threadIdx.x % TPR;
    const int sub = threadIdx.x / TPR;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + sub;
    if constexpr (NW == 1 && !FULL) {
        if (row >= a.rows) return;  // whole wavefront leaves together
    }
    // Rows past the end (only in the last workgroup) keep taking part in the
    // workgroup barriers but touch no memory.
    const int c4n = FULL ? TPR * VPT : (row < a.rows ? static_cast<int>(a.cols >> 2) : 0);
    auto live = [&](int j) { return FULL || j * TPR + t < c4n; };
    const float* x = a.x + row * a.cols + 4 * t;
    float* y = a.y + row * a.cols + 4 * t;

    // LayerNorm: issue the row's loads at raised wave priority, so the loads
    // of resident rows are not held up behind other waves' reduction math.
    constexpr bool kLayer = K == Norm::Layer || K == Norm::AddLayer;
    if constexpr (kLayer) __builtin_amdgcn_s_setprio(3);
    // The per-column weights (L2-resident) are loaded right behind the row,
    // with no condition: an absent scale or bias arrives as the context's
    // 1.0 / -0.0 columns (x * 1 and x + (-0) are x exactly).  A conditional
    // or later load would put its latency after the reduction, or make the
    // reduction wait for it.
    f4 v[VPT], gv[VPT], bv[VPT];
    auto load_weights = [&]() {
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int c4 = j * TPR + t;
            gv[j] = live(j) ? *reinterpret_cast<const f4*>(a.g + 4 * c4) : f4(0.0f);
            if constexpr (kLayer) bv[j] = live(j) ? *reinterpret_cast<const f4*>(a.b + 4 * c4) : f4(0.0f);
        }
    };
    if constexpr (K == Norm::AddRms || K == Norm::AddLayer) {
        const float* r = a.r + row * a.cols + 4 * t;
        f4 rr[VPT];
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            v[j] = live(j) ? ld4<true>(x + 4 * j * TPR) : f4(0.0f);
            rr[j] = live(j) ? ld4<true>(r + 4 * j * TPR) : f4(0.0f);
        }
        if constexpr (kLayer) __builtin_amdgcn_s_setprio(0);
        load_weights();
        float* ro = a.r_out + row * a.cols + 4 * t;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            v[j] = v[j] + rr[j];  // one IEEE add per element, as add_forward
            // add + RMSNorm's updated residual: a plain store, measured
            // faster than a streamed one beside the streamed y (4 points of
            // 8 TB/s at configs[1]).  The runtime's fused Add ->
            // LayerNorm streams its sum (a later block reads it).
            if (live(j) && (K == Norm::AddRms || a.r_out)) st4<K == Norm::AddLayer>(ro + 4 * j * TPR, v[j]);
        }
    } else {
#pragma unroll
        for (int j = 0; j < VPT; ++j) v[j] = live(j) ? ld4<true>(x + 4 * j * TPR) : f4(0.0f);
        if constexpr (kLayer) __builtin_amdgcn_s_setprio(0);
        load_weights();
    }

    if constexpr (kLayer) {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < VPT; ++j) s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
        const float sw = wave_sum(s);
        float mean, var;
        if constexpr (NW == 1) {
            mean = sw * a.inv_n;
            float q = 0.0f;
#pragma unroll
            for (int j = 0; j < VPT; ++j) {
                if (live(j)) {
                    const f4 d = v[j] - mean;
                    q += (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
                }
            }
            var = wave_sum(q) * a.inv_n;
        } else if constexpr (FULL) {
            // Mean and variance with one exchange between the row's waves.
            // Each wave holds kPer = 256*VPT values (a power of two, so its
            // mean S_w * (1/kPer) is exact) and reduces them to (S_w, M2_w
            // about its own mean); one LDS round combines the parts by the
            // pairwise update of Chan, Golub and LeVeque (1979):
            //   mean = sum_w S_w / n,  M2 = sum_w M2_w + kPer * sum_w (S_w/kPer - mean)^2,
            // the reference's two-pass mean and variance, regrouped.
            constexpr float kPer = 256.0f * VPT;
            constexpr float kInvPer = 1.0f / kPer;
            const float mw = sw * kInvPer;
            float q = 0.0f;
#pragma unroll
            for (int j = 0; j < VPT; ++j) {
                const f4 d = v[j] - mw;
                q += (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
            }
            const float m2w = wave_sum(q);
            float2* part = reinterpret_cast<float2*>(&lds[0][0]);
            if ((threadIdx.x & (kWave - 1)) == 0) part[threadIdx.x / kWave] = make_float2(sw, m2w);
            __syncthreads();
            float2 p[NW];
#pragma unroll
            for (int i = 0; i < NW; ++i) p[i] = part[sub * NW + i];
            float S = 0.0f;
#pragma unroll
            for (int i = 0; i < NW; ++i) S += p[i].x;
            mean = S * a.inv_n;
            float M2 = 0.0f, D = 0.0f;
#pragma unroll
            for (int i = 0; i < NW; ++i) {
                const float d = p[i].x * kInvPer - mean;
                M2 += p[i].y;
                D += d * d;
            }
            var = (M2 + kPer * D) * a.inv_n;
        } else {
            // Partial rows: waves hold different counts; two exchanges, the
            // plain two-pass order.
            mean = row_sum<NW, false>(s, lds[0], sub) * a.inv_n;
            float q = 0.0f;
#pragma unroll
            for (int j = 0; j < VPT; ++j) {
                if (live(j)) {
                    const f4 d = v[j] - mean;
                    q += (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
                }
            }
            var = row_sum<NW, false>(q, lds[1], sub) * a.inv_n;
        }
        const float inv_std = __builtin_amdgcn_rsqf(var + a.eps);
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            if (live(j)) {
                const int c4 = j * TPR + t;
                f4 o = (v[j] - mean) * inv_std;
                o = o * gv[j] + bv[j];
                if constexpr (EPI) {
                    const int64_t off = row * a.cols + 4 * c4;
                    const int ns = a.epi.n_steps;
                    if (a.y) {
                        if (ns == 0) st_out<KEEP>(a.y + off, o);
                        else st4<true>(a.y + off, o);
                    }
                    for (int k = 0; k < ns; ++k) {
                        const FuseStep st = a.epi.steps[k];
                        const bool bin = st.kind == kFuseAdd || st.kind == kFuseMul;
                        const f4 w = bin && st.operand >= 0 ? ld4<true>(a.epi.ins[st.operand] + off) : o;
                        o = fuse_step4(st.kind, o, w);
                        if (st.store >= 0) {
                            if (k + 1 == ns) st_out<KEEP>(a.epi.outs[st.store] + off, o);
                            else st4<true>(a.epi.outs[st.store] + off, o);
                        }
                    }
                } else {
                    st_out<KEEP>(y + 4 * j * TPR, o);
                }
            }
        }
    } else {
        float q = 0.0f;
#pragma unroll
        for (int j = 0; j < VPT; ++j)
            q += (v[j].x * v[j].x + v[j].y * v[j].y) + (v[j].z * v[j].z + v[j].w * v[j].w);
        const float inv_rms = __builtin_amdgcn_rsqf(row_sum<NW, false>(q, lds[0], sub) * a.inv_n + a.eps);
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            if (live(j)) {
                const int c4 = j * TPR + t;
                f4 o = v[j] * inv_rms * gv[j];
                // A weight shorter than the row scales its prefix only.
                if (a.wp) o = rms_scale(o, a.wp, a.w_len, 4 * c4);
                st_out<KEEP>(y + 4 * j * TPR, o);
            }
        }
    }
}

// Generic rows: one workgroup per row, scalar strided passes over global
// memory (the re-reads of a row hit L2).  Any width, any alignment.
template <Norm K>
__global__ __launch_bounds__(kBlock) void norm_rows_generic(NormArgs a) {
    constexpr int NW = kBlock / kWave;
    __shared__ float lds[2][NW];
    const int64_t row = blockIdx.x;
    const int64_t base = row * a.cols;
    const float n = static_cast<float>(a.cols);
    const float* x = a.x + base;
    float* y = a.y + base;

    if constexpr (K == Norm::Layer) {
        float s = 0.0f;
        for (int64_t c = threadIdx.x; c < a.cols; c += kBlock) s += x[c];
        const float mean = block_sum<NW>(s, lds[0]) / n;
        float q = 0.0f;
        for (int64_t c = threadIdx.x; c < a.cols; c += kBlock) {
            const float d = x[c] - mean;
            q += d * d;
        }
        const float var = block_sum<NW>(q, lds[1]) / n;
        const float inv_std = 1.0f / sqrtf(var + a.eps);
        for (int64_t c = threadIdx.x; c < a.cols; c += kBlock) {
            float o = (x[c] - mean) * inv_std;
            if (a.g) {
                o *= a.g[c];
                if (a.b) o += a.b[c];
            }
            y[c] = o;
        }
    } else {
        const float* h = x;
        float q = 0.0f;
        if constexpr (K == Norm::AddRms) {
            const float* r = a.r + base;
            float* ro = a.r_out + base;
            for (int64_t c = threadIdx.x; c < a.cols; c += kBlock) {
                const float v = x[c] + r[c];
                ro[c] = v;
                q += v * v;
            }
            h = ro;  // the second pass reads back this thread's own writes
        } else {
            for (int64_t c = threadIdx.x; c < a.cols; c += kBlock) q += x[c] * x[c];
        }
        const float rms = sqrtf(block_sum<NW>(q, lds[0]) / n + a.eps);
        for (int64_t c = threadIdx.x; c < a.cols; c += kBlock) {
            float o = h[c] / rms;
            if (a.g && c < a.w_len) o *= a.g[c];
            y[c] = o;
        }
    }
}

template <Norm K, int TPR, int VPT, int BS, bool EPI = false>
int launch_vec(mimir_ctx* ctx, const NormArgs& args) {
    unsigned blocks;
    if (!grid_for(args.rows, BS / TPR, BS, &blocks))
        return fail(ctx, MIMIR_EINVAL, "norm: %lld rows exceed the grid limit", (long long)args.rows);
    NormArgs a = args;
    a.inv_n = 1.0f / static_cast<float>(a.cols);
    const float* one = ctx->unit_weights;
    const float* negzero = one + kUnitCols;
    if constexpr (K == Norm::Layer || K == Norm::AddLayer) {
        if (!a.g) a.g = one;
        if (!a.b) a.b = negzero;
    } else if (!a.g) {
        a.g = one;
    } else if (a.w_len < a.cols) {
        a.wp = a.g;
        a.g = one;
    }
    const bool full = a.cols == 4LL * TPR * VPT && a.rows % (BS / TPR) == 0;
    if (ctx->keep_outputs) {
        if (full) norm_rows_vec<K, TPR, VPT, BS, true, EPI, true><<<blocks, BS, 0, ctx->stream>>>(a);
        else norm_rows_vec<K, TPR, VPT, BS, true, EPI, false><<<blocks, BS, 0, ctx->stream>>>(a);
    } else {
        if (full) norm_rows_vec<K, TPR, VPT, BS, false, EPI, true><<<blocks, BS, 0, ctx->stream>>>(a);
        else norm_rows_vec<K, TPR, VPT, BS, false, EPI, false><<<blocks, BS, 0, ctx->stream>>>(a);
    }
    return launched(ctx, "norm_rows_vec");
}

// The default LayerNorm shapes (rows.hpp default_norm_shape), the ones the
// runtime's fused LayerNorm is compiled for.
#define MIMIR_LN_FUSED_SHAPES(X) \
    X(64, 1, 256)                \
    X(128, 1, 256)               \
    X(64, 4, 64)                 \
    X(512, 1, 512)               \
    X(256, 4, 256)               \
    X(512, 4, 512)               \
    X(1024, 4, 1024)

// Rows the vector kernels cannot take (a width that is not a multiple of 4,
// so rows start off 16-byte alignment, or unaligned pointers), up to
// kBlock*VPT floats: the same register-resident scheme with 4-byte columns.
// One kBlock-thread workgroup per row; thread t holds columns t, t+kBlock,
// ...; one read of the row (and of the residual for add + RMSNorm, whose
// sum is written once), two reductions (LayerNorm) or one (RMSNorm).
template <Norm K, int VPT, bool KEEP>
__global__ __launch_bounds__(kBlock) void norm_rows_scalar(NormArgs a) {
    constexpr int NW = kBlock / kWave;
    __shared__ float lds[2][NW];
    const int t = threadIdx.x;
    const int64_t base = static_cast<int64_t>(blockIdx.x) * a.cols;
    float v[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t c = static_cast<int64_t>(j) * kBlock + t;
        v[j] = c < a.cols ? __builtin_nontemporal_load(a.x + base + c) : 0.0f;
    }
    if constexpr (K == Norm::AddRms) {  // h = x + residual (one IEEE add, as add_forward), streamed out
        float rr[VPT];
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int64_t c = static_cast<int64_t>(j) * kBlock + t;
            rr[j] = c < a.cols ? __builtin_nontemporal_load(a.r + base + c) : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int64_t c = static_cast<int64_t>(j) * kBlock + t;
            v[j] = v[j] + rr[j];
            if (c < a.cols) st_stream(a.r_out + base + c, v[j]);
        }
    }
    const float n = static_cast<float>(a.cols);
    auto put = [&](int64_t c, float o) {
        if constexpr (KEEP) a.y[base + c] = o;
        else st_stream(a.y + base + c, o);
    };
    if constexpr (K == Norm::Layer) {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < VPT; ++j) s += v[j];
        const float mean = row_sum<NW, false>(s, lds[0], 0) / n;
        float q = 0.0f;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            if (static_cast<int64_t>(j) * kBlock + t < a.cols) {
                const float d = v[j] - mean;
                q += d * d;
            }
        }
        const float var = row_sum<NW, false>(q, lds[1], 0) / n;
        const float inv_std = 1.0f / sqrtf(var + a.eps);
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int64_t c = static_cast<int64_t>(j) * kBlock + t;
            if (c < a.cols) {
                float o = (v[j] - mean) * inv_std;
                if (a.g) {
                    o *= a.g[c];
                    if (a.b) o += a.b[c];
                }
                put(c, o);
            }
        }
    } else {
        float q = 0.0f;
#pragma unroll
        for (int j = 0; j < VPT; ++j) q += v[j] * v[j];
        const float rms = sqrtf(row_sum<NW, false>(q, lds[0], 0) / n + a.eps);
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int64_t c = static_cast<int64_t>(j) * kBlock + t;
            if (c < a.cols) {
                float o = v[j] / rms;
                if (a.g && c < a.w_len) o *= a.g[c];
                put(c, o);
            }
        }
    }
}

template <Norm K, int VPT>
int launch_scalar(mimir_ctx* ctx, const NormArgs& a) {
    const unsigned grid = static_cast<unsigned>(a.rows);
    if (ctx->keep_outputs) norm_rows_scalar<K, VPT, true><<<grid, kBlock, 0, ctx->stream>>>(a);
    else norm_rows_scalar<K, VPT, false><<<grid, kBlock, 0, ctx->stream>>>(a);
    return launched(ctx, "norm_rows_scalar");
}

template <Norm K>
int dispatch(mimir_ctx* ctx, const NormArgs& a) {
    bool vec = (a.cols % 4) == 0 && aligned16(a.x) && aligned16(a.y) &&
               (!a.g || aligned16(a.g)) && (!a.b || aligned16(a.b));
    if constexpr (K == Norm::AddRms) vec = vec && aligned16(a.r) && aligned16(a.r_out);
    const int64_t c4 = a.cols / 4;
    if (vec) {
        const RowShape over = K == Norm::Layer ? ctx->tune.layernorm : ctx->tune.rmsnorm;
        const RowShape s = shape_fits(over, c4) ? over
                           : (K == Norm::Layer ? default_layernorm_shape(c4) : default_norm_shape(c4));
#define MIMIR_NORM_CASE(T, V, B) \
        if (s.tpr == T && s.vpt == V && s.bs == B) return launch_vec<K, T, V, B>(ctx, a);
        MIMIR_ROW_SHAPES(MIMIR_NORM_CASE)
#undef MIMIR_NORM_CASE
        // Rows too wide for one workgroup's registers: split each row.
        if (longrow_applies(a.rows, a.cols))
            return longrow_norm(ctx, K == Norm::Layer ? 0 : (K == Norm::Rms ? 1 : 2), a.x, a.r, a.r_out, a.g, a.b,
                                a.w_len, a.y, a.rows, a.cols, a.eps);
    }
    if (!dispatch_fits(a.rows, kBlock))
        return fail(ctx, MIMIR_EINVAL, "norm: %lld rows exceed the grid limit", (long long)a.rows);
    if (!vec && a.cols <= 4 * kBlock) return launch_scalar<K, 4>(ctx, a);
    if (!vec && a.cols <= 8 * kBlock) return launch_scalar<K, 8>(ctx, a);
    if (!vec && a.cols <= 16 * kBlock) return launch_scalar<K, 16>(ctx, a);
    norm_rows_generic<K><<<static_cast<unsigned>(a.rows), kBlock, 0, ctx->stream>>>(a);
    return launched(ctx, "norm_rows_generic");
}

}  // namespace

int mimir::norm_init(mimir_ctx* ctx) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(unit_weights));
    if (e != hipSuccess) return hip_fail(ctx, e, "hipGetSymbolAddress(unit_weights)");
    fill_unit_weights<<<(kUnitCols + kBlock - 1) / kBlock, kBlock, 0, ctx->stream>>>(static_cast<float*>(p));
    if (int st = launched(ctx, "fill_unit_weights")) return st;
    e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamSynchronize");
    ctx->unit_weights = static_cast<const float*>(p);
    return MIMIR_OK;
}

bool mimir::layernorm_fusable(const mimir_ctx* ctx, int64_t cols, const float* g, const float* b) {
    if (cols <= 0 || cols % 4 != 0 || (g && !aligned16(g)) || (b && !aligned16(b))) return false;
    // With a LayerNorm shape override the unfused kernel would reduce in
    // another order: keep the unfused path then, so both agree bit for bit.
    if (shape_fits(ctx->tune.layernorm, cols / 4)) return false;
    return default_layernorm_shape(cols / 4).tpr != 0;
}

int mimir::layernorm_fused(mimir_ctx* ctx, const LnFused& f) {
    NormArgs a{f.x, f.r, f.h, f.g, f.b, f.y, f.rows, f.cols, f.cols, f.eps};
    a.epi = f.epi;
    if (f.rows == 0) return MIMIR_OK;
    MIMIR_ENTER(ctx);
    const RowShape s = default_layernorm_shape(f.cols / 4);
#define MIMIR_LN_FUSED_CASE(T, V, B)                                                                  \
    if (s.tpr == T && s.vpt == V && s.bs == B)                                                       \
        return f.r ? launch_vec<Norm::AddLayer, T, V, B, true>(ctx, a) : launch_vec<Norm::Layer, T, V, B, true>(ctx, a);
    MIMIR_LN_FUSED_SHAPES(MIMIR_LN_FUSED_CASE)
#undef MIMIR_LN_FUSED_CASE
    return fail(ctx, MIMIR_EINVAL, "fused LayerNorm: no row shape for %lld columns", (long long)f.cols);
}

extern "C" {

int mimir_layernorm_fwd(mimir_ctx* ctx, const float* x, const float* gamma, const float* beta,
                        float* y, int64_t groups, int64_t n, float eps) {
    if (!ctx) return MIMIR_EINVAL;
    MIMIR_REQUIRE(ctx, n > 0 && groups >= 0, "LayerNorm: invalid normalized_size (groups=%lld, n=%lld)",
                  (long long)groups, (long long)n);
    MIMIR_REQUIRE(ctx, !(beta && !gamma), "LayerNorm: bias without scale (use_bias needs affine)");
    if (groups == 0) return MIMIR_OK;
    MIMIR_REQUIRE(ctx, x && y, "LayerNorm: null tensor");
    MIMIR_ENTER(ctx);
    NormArgs a{x, nullptr, nullptr, gamma, beta, y, groups, n, n, eps};
    return dispatch<Norm::Layer>(ctx, a);
}

int mimir_rmsnorm_fwd(mimir_ctx* ctx, const float* x, const float* w, int64_t w_len, float* y,
                      int64_t rows, int64_t cols, float eps) {
    if (!ctx) return MIMIR_EINVAL;
    MIMIR_REQUIRE(ctx, rows >= 0 && cols > 0 && w_len >= 0, "RMSNorm: invalid shape (rows=%lld, cols=%lld)",
                  (long long)rows, (long long)cols);
    if (rows == 0) return MIMIR_OK;
    MIMIR_REQUIRE(ctx, x && y, "RMSNorm: null tensor");
    MIMIR_ENTER(ctx);
    NormArgs a{x, nullptr, nullptr, (w && w_len > 0) ? w : nullptr, nullptr, y, rows, cols, w ? w_len : 0, eps};
    return dispatch<Norm::Rms>(ctx, a);
}

int mimir_add_rmsnorm_fwd(mimir_ctx* ctx, const float* x, const float* residual,
                          float* residual_out, const float* w, float* y, int64_t rows,
                          int64_t cols, float eps) {
    if (!ctx) return MIMIR_EINVAL;
    MIMIR_REQUIRE(ctx, rows >= 0 && cols > 0, "add+RMSNorm: invalid shape (rows=%lld, cols=%lld)",
                  (long long)rows, (long long)cols);
    if (rows == 0) return MIMIR_OK;
    MIMIR_REQUIRE(ctx, x && residual && residual_out && y, "add+RMSNorm: null tensor");
    MIMIR_REQUIRE(ctx, static_cast<const void*>(y) != static_cast<const void*>(residual_out),
                  "add+RMSNorm: y must not alias residual_out");
    MIMIR_ENTER(ctx);
    NormArgs a{x, residual, residual_out, w, nullptr, y, rows, cols, w ? cols : 0, eps};
    return dispatch<Norm::AddRms>(ctx, a);
}

}  // extern "C"
