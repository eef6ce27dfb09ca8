// elementwise.hip -- GELU, SiLU, gated products, add (with the reference's
// broadcast rules) and multiply for gfx950.
//
// Streaming layout: each thread owns VPT 16-byte vectors spaced one
// workgroup-width apart (so each wave instruction moves 1 KiB of contiguous
// data), issues all its loads before any arithmetic, and writes with
// non-temporal stores: every input byte is read once and every output byte
// written once.  VPT = 1 (one vector per thread, many waves in flight) in
// 128-thread workgroups streams fastest on MI355X (kEwBlock); 2 and 4 vectors
// per thread and 64-1024-thread workgroups stay available for sweeps
// (MIMIR_TUNE ew=, ewbs=).  Buffers that are not 16-byte aligned, and the
// n % 4 tail, run through a scalar grid-stride kernel with the same
// per-element functor.
#include "common.hpp"
#include "internal.hpp"
#include "pointwise.hpp"

#include <math.h>

using namespace mimir;

namespace {

struct Gelu {
    __device__ float operator()(float x) const { return gelu1(x); }
};
struct Silu {
    __device__ float operator()(float x) const { return silu1(x); }
};
// multiply_forward(silu_forward(gate), up): LayerOps.hpp:570-581 then :205-230.
struct SiluMul {
    __device__ float operator()(float g, float u) const { return silu1(g) * u; }
};
// multiply_forward(gelu_forward(gate), up).
struct GeluMul {
    __device__ float operator()(float g, float u) const { return gelu1(g) * u; }
};
struct Add {
    __device__ float operator()(float a, float b) const { return a + b; }
};
struct Mul {
    __device__ float operator()(float a, float b) const { return a * b; }
};
// computeBranchMerge AVERAGE, Model.cpp:4434-4460: (a + b) * 0.5f, two roundings.
struct Average {
    __device__ float operator()(float a, float b) const { return (a + b) * 0.5f; }
};
// computeBranchMerge MAX, Model.cpp:4408-4432.  The AVX2 body's vmaxps
// returns its second operand unless the first is greater (so b for a NaN on
// either side and for equal zeros); the scalar tail's std::max(a, b) returns
// a unless a < b.
struct MaxBody {
    __device__ float operator()(float a, float b) const { return a > b ? a : b; }
};
struct MaxTail {
    __device__ float operator()(float a, float b) const { return a < b ? b : a; }
};

template <class F>
__device__ __forceinline__ f4 map4(F f, f4 a) {
    return f4{f(a.x), f(a.y), f(a.z), f(a.w)};
}
template <class F>
__device__ __forceinline__ f4 map4(F f, f4 a, f4 b) {
    return f4{f(a.x, b.x), f(a.y, b.y), f(a.z, b.z), f(a.w, b.w)};
}

// BS: the workgroup size (rows.hpp ew_block); VPT float4 per thread, a
// workgroup-width apart.
template <class F, int VPT, bool KEEP, int BS = kBlock>
__global__ __launch_bounds__(BS) void unary_vec(const float* x, float* y, int64_t n4, F f) {
    const int64_t first = static_cast<int64_t>(blockIdx.x) * VPT * BS + threadIdx.x;
    f4 v[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t i = first + static_cast<int64_t>(j) * BS;
        if (i < n4) v[j] = ld4<true>(x + 4 * i);
    }
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t i = first + static_cast<int64_t>(j) * BS;
        if (i < n4) st_out<KEEP, kStoreThrough>(y + 4 * i, map4(f, v[j]));  // one read, one write: written through
    }
}

template <class F, int VPT, bool KEEP, int BS = kBlock>
__global__ __launch_bounds__(BS) void binary_vec(const float* a, const float* b, float* y,
                                                 int64_t n4, F f) {
    const int64_t first = static_cast<int64_t>(blockIdx.x) * VPT * BS + threadIdx.x;
    f4 va[VPT], vb[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t i = first + static_cast<int64_t>(j) * BS;
        if (i < n4) {
            va[j] = ld4<true>(a + 4 * i);
            vb[j] = ld4<true>(b + 4 * i);
        }
    }
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t i = first + static_cast<int64_t>(j) * BS;
        if (i < n4) st_out<KEEP>(y + 4 * i, map4(f, va[j], vb[j]));
    }
}

template <class F>
__global__ __launch_bounds__(kBlock) void unary_scalar(const float* x, float* y, int64_t n, F f) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
        y[i] = f(x[i]);
}

template <class F>
__global__ __launch_bounds__(kBlock) void binary_scalar(const float* a, const float* b, float* y,
                                                        int64_t n, F f) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
        y[i] = f(a[i], b[i]);
}

// add_forward scalar broadcast, LayerOps.hpp:181-188: y[i] = big[i] + small[0].
__global__ __launch_bounds__(kBlock) void add_scalar_kernel(const float* big, const float* small,
                                                            float* y, int64_t n) {
    const float s = small[0];
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
        y[i] = big[i] + s;
}

// add_forward repeat broadcast, LayerOps.hpp:194-197: y[i] = big[i] + small[i % small_n],
// as `rows` rows of small_n.  Each thread keeps its 16 bytes of `small` in
// registers and walks the rows (blockIdx.y strided).
template <bool KEEP>
__global__ __launch_bounds__(kBlock) void add_repeat_vec(const float* big, const float* small,
                                                         float* y, int64_t rows, int64_t small_n4) {
    const int64_t c4 = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (c4 >= small_n4) return;
    const f4 s = *reinterpret_cast<const f4*>(small + 4 * c4);
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
        const int64_t i = r * small_n4 + c4;
        st_out<KEEP>(y + 4 * i, ld4<true>(big + 4 * i) + s);
    }
}

__global__ __launch_bounds__(kBlock) void add_repeat_scalar(const float* big, const float* small,
                                                            float* y, int64_t n, int64_t small_n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
        y[i] = big[i] + small[i % small_n];
}

unsigned stride_grid(int64_t n) {
    const int64_t b = (n + kBlock - 1) / kBlock;
    return static_cast<unsigned>(b < 1 ? 1 : (b > 65536 ? 65536 : b));
}

template <class F, int VPT, int BS = kBlock>
int launch_unary(mimir_ctx* ctx, const float* x, float* y, int64_t n4, F f, const char* name) {
    unsigned blocks;
    if (!grid_for(n4, static_cast<int64_t>(VPT) * BS, BS, &blocks))
        return fail(ctx, MIMIR_EINVAL, "%s: n=%lld exceeds the grid limit", name, (long long)(4 * n4));
    if (ctx->keep_outputs) unary_vec<F, VPT, true, BS><<<blocks, BS, 0, ctx->stream>>>(x, y, n4, f);
    else unary_vec<F, VPT, false, BS><<<blocks, BS, 0, ctx->stream>>>(x, y, n4, f);
    return launched(ctx, name);
}

template <class F, int VPT, int BS = kBlock>
int launch_binary(mimir_ctx* ctx, const float* a, const float* b, float* y, int64_t n4, F f,
                  const char* name) {
    unsigned blocks;
    if (!grid_for(n4, static_cast<int64_t>(VPT) * BS, BS, &blocks))
        return fail(ctx, MIMIR_EINVAL, "%s: n=%lld exceeds the grid limit", name, (long long)(4 * n4));
    if (ctx->keep_outputs) binary_vec<F, VPT, true, BS><<<blocks, BS, 0, ctx->stream>>>(a, b, y, n4, f);
    else binary_vec<F, VPT, false, BS><<<blocks, BS, 0, ctx->stream>>>(a, b, y, n4, f);
    return launched(ctx, name);
}

template <class F>
int run_unary(mimir_ctx* ctx, const float* x, float* y, int64_t n, F f, const char* name) {
    int64_t done = 0;
    if (aligned16(x) && aligned16(y)) {
        const int64_t n4 = n / 4;
        if (n4 > 0) {
            int st;
            switch (ctx->tune.ew_vpt) {
                case 2: st = launch_unary<F, 2>(ctx, x, y, n4, f, name); break;
                case 4: st = launch_unary<F, 4>(ctx, x, y, n4, f, name); break;
                default:
                    st = with_block(ew_block(ctx->tune), [&](auto bs) {
                        return launch_unary<F, 1, decltype(bs)::value>(ctx, x, y, n4, f, name);
                    });
                    break;
            }
            if (st) return st;
        }
        done = n4 * 4;
    }
    if (n > done) {
        unary_scalar<F><<<stride_grid(n - done), kBlock, 0, ctx->stream>>>(x + done, y + done, n - done, f);
        return launched(ctx, name);
    }
    return MIMIR_OK;
}

template <class F>
int run_binary(mimir_ctx* ctx, const float* a, const float* b, float* y, int64_t n, F f,
               const char* name) {
    int64_t done = 0;
    if (aligned16(a) && aligned16(b) && aligned16(y)) {
        const int64_t n4 = n / 4;
        if (n4 > 0) {
            int st;
            switch (ctx->tune.ew_vpt) {
                case 2: st = launch_binary<F, 2>(ctx, a, b, y, n4, f, name); break;
                case 4: st = launch_binary<F, 4>(ctx, a, b, y, n4, f, name); break;
                default:
                    st = with_block(ew_block(ctx->tune), [&](auto bs) {
                        return launch_binary<F, 1, decltype(bs)::value>(ctx, a, b, y, n4, f, name);
                    });
                    break;
            }
            if (st) return st;
        }
        done = n4 * 4;
    }
    if (n > done) {
        binary_scalar<F><<<stride_grid(n - done), kBlock, 0, ctx->stream>>>(a + done, b + done, y + done,
                                                                          n - done, f);
        return launched(ctx, name);
    }
    return MIMIR_OK;
}

// One 16-byte vector per thread; the steps run in registers, each binary
// step loading its operand where it is used (many waves in flight hide the
// latency: the kernel stays small).  The program is uniform across the grid,
// so its branches never diverge.
template <bool KEEP, int BS = kBlock>
__global__ __launch_bounds__(BS) void fused_chain_vec(const FuseProgram p, int64_t n4) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * BS + threadIdx.x;
    if (i >= n4) return;
    f4 v = ld4<true>(p.ins[0] + 4 * i);
    for (int k = 0; k < p.n_steps; ++k) {
        const FuseStep st = p.steps[k];
        const bool bin = st.kind == kFuseAdd || st.kind == kFuseMul;
        const f4 o = bin && st.operand >= 0 ? ld4<true>(p.ins[st.operand] + 4 * i) : v;
        v = fuse_step4(st.kind, v, o);
        // The chain's last value is what the next layer reads; the
        // intermediates a later layer needs are streamed out.
        if (st.store >= 0) {
            if (k + 1 == p.n_steps) st_out<KEEP>(p.outs[st.store] + 4 * i, v);
            else st4<true>(p.outs[st.store] + 4 * i, v);
        }
    }
}

__global__ __launch_bounds__(kBlock) void fused_chain_scalar(const FuseProgram p, int64_t first, int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = first + static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
        float v = p.ins[0][i];
        for (int k = 0; k < p.n_steps; ++k) {
            const FuseStep st = p.steps[k];
            v = fuse_step1(st.kind, v, st.operand >= 0 ? p.ins[st.operand][i] : v);
            if (st.store >= 0) p.outs[st.store][i] = v;
        }
    }
}

}  // namespace

int mimir::fused_chain(mimir_ctx* ctx, const FuseProgram& p, int64_t n) {
    if (n == 0) return MIMIR_OK;
    bool aligned = true;
    for (int k = 0; k < p.n_ins; ++k) aligned = aligned && aligned16(p.ins[k]);
    for (int k = 0; k < p.n_outs; ++k) aligned = aligned && aligned16(p.outs[k]);
    MIMIR_ENTER(ctx);
    int64_t done = 0;
    if (aligned && n / 4 > 0) {
        const int64_t n4 = n / 4;
        const int st = with_block(ew_block(ctx->tune), [&](auto bsc) {
            constexpr int BS = decltype(bsc)::value;
            unsigned blocks;
            if (!grid_for(n4, BS, BS, &blocks)) return fail(ctx, MIMIR_EINVAL, "fused chain: grid too large");
            if (ctx->keep_outputs) fused_chain_vec<true, BS><<<blocks, BS, 0, ctx->stream>>>(p, n4);
            else fused_chain_vec<false, BS><<<blocks, BS, 0, ctx->stream>>>(p, n4);
            return launched(ctx, "fused_chain_vec");
        });
        if (st) return st;
        done = n4 * 4;
    }
    if (n > done) {
        fused_chain_scalar<<<stride_grid(n - done), kBlock, 0, ctx->stream>>>(p, done, n);
        return launched(ctx, "fused_chain_scalar");
    }
    return MIMIR_OK;
}

extern "C" {

int mimir_gelu_fwd(mimir_ctx* ctx, const float* x, float* y, int64_t n) {
    if (!ctx) return MIMIR_EINVAL;
    MIMIR_REQUIRE(ctx, n >= 0, "GELU: n < 0");
    if (n == 0) return MIMIR_OK;
    MIMIR_REQUIRE(ctx, x && y, "GELU: null tensor");
    MIMIR_ENTER(ctx);
    return run_unary(ctx, x, y, n, Gelu{}, "gelu");
}

int mimir_silu_fwd(mimir_ctx* ctx, const float* x, float* y, int64_t n) {
    if (!ctx) return MIMIR_EINVAL;
    MIMIR_REQUIRE(ctx, n >= 0, "SiLU: n < 0");
    if (n == 0) return MIMIR_OK;
    MIMIR_REQUIRE(ctx, x && y, "SiLU: null tensor");
    MIMIR_ENTER(ctx);
    return run_unary(ctx, x, y, n, Silu{}, "silu");
}

int mimir_silu_mul_fwd(mimir_ctx* ctx, const float* gate, const float* up, float* y, int64_t n) {
    if (!ctx) return MIMIR_EINVAL;
    MIMIR_REQUIRE(ctx, n >= 0, "SiLU*up: n < 0");
    if (n == 0) return MIMIR_OK;
    MIMIR_REQUIRE(ctx, gate && up && y, "SiLU*up: null tensor");
    MIMIR_ENTER(ctx);
    return run_binary(ctx, gate, up, y, n, SiluMul{}, "silu_mul");
}

int mimir_gelu_mul_fwd(mimir_ctx* ctx, const float* gate, const float* up, float* y, int64_t n) {
    if (!ctx) return MIMIR_EINVAL;
    MIMIR_REQUIRE(ctx, n >= 0, "GELU*up: n < 0");
    if (n == 0) return MIMIR_OK;
    MIMIR_REQUIRE(ctx, gate && up && y, "GELU*up: null tensor");
    MIMIR_ENTER(ctx);
    return run_binary(ctx, gate, up, y, n, GeluMul{}, "gelu_mul");
}

int mimir_add_fwd(mimir_ctx* ctx, const float* a, int64_t na, const float* b, int64_t nb,
                  float* y) {
    if (!ctx) return MIMIR_EINVAL;
    // LayerOps.hpp:150-152: both inputs must be non-empty.
    MIMIR_REQUIRE(ctx, na > 0 && nb > 0, "Add: inputs must be non-empty");
    MIMIR_REQUIRE(ctx, a && b && y, "Add: null tensor");
    if (na == nb) {  // LayerOps.hpp:154-169
        MIMIR_ENTER(ctx);
        return run_binary(ctx, a, b, y, na, Add{}, "add");
    }
    const float* big = a;
    const float* small = b;
    int64_t big_n = na, small_n = nb;
    if (nb > na) {  // LayerOps.hpp:172-177
        big = b;
        small = a;
        big_n = nb;
        small_n = na;
    }
    MIMIR_REQUIRE(ctx, small_n == 1 || big_n % small_n == 0,
                  "Add: input sizes must match or be broadcastable (%lld vs %lld)", (long long)na,
                  (long long)nb);
    MIMIR_ENTER(ctx);
    if (small_n == 1) {
        add_scalar_kernel<<<stride_grid(big_n), kBlock, 0, ctx->stream>>>(big, small, y, big_n);
        return launched(ctx, "add_scalar_kernel");
    }
    const int64_t rows = big_n / small_n;
    if (small_n % 4 == 0 && aligned16(big) && aligned16(small) && aligned16(y)) {
        const int64_t small_n4 = small_n / 4;
        unsigned bx;
        if (!grid_for(small_n4, kBlock, kBlock, &bx))
            return fail(ctx, MIMIR_EINVAL, "Add: operand of %lld exceeds the grid limit", (long long)small_n);
        // Enough rows per launch to give every CU work; each thread then strides rows.
        const int64_t want_y = (static_cast<int64_t>(2048) + bx - 1) / bx;
        const unsigned by = static_cast<unsigned>(rows < want_y ? rows : (want_y > 65535 ? 65535 : want_y));
        if (ctx->keep_outputs)
            add_repeat_vec<true><<<dim3(bx, by), kBlock, 0, ctx->stream>>>(big, small, y, rows, small_n4);
        else
            add_repeat_vec<false><<<dim3(bx, by), kBlock, 0, ctx->stream>>>(big, small, y, rows, small_n4);
        return launched(ctx, "add_repeat_vec");
    }
    add_repeat_scalar<<<stride_grid(big_n), kBlock, 0, ctx->stream>>>(big, small, y, big_n, small_n);
    return launched(ctx, "add_repeat_scalar");
}

int mimir_branch_merge_fwd(mimir_ctx* ctx, const float* a, int64_t na, const float* b, int64_t nb,
                           float* y, int merge_op) {
    if (!ctx) return MIMIR_EINVAL;
    MIMIR_REQUIRE(ctx, na >= 0 && nb >= 0, "branch merge: negative size");
    MIMIR_REQUIRE(ctx, merge_op >= MIMIR_MERGE_ADD && merge_op <= MIMIR_MERGE_ATTENTION_WEIGHTED,
                  "branch merge: unknown merge operation %d", merge_op);
    if (merge_op == MIMIR_MERGE_CONCATENATE) {  // Model.cpp:4462-4468: a then b
        MIMIR_REQUIRE(ctx, (na == 0 || (a && y)) && (nb == 0 || (b && y)), "branch merge: null tensor");
        if (na > 0)
            if (int st = mimir_copy(ctx, y, a, static_cast<size_t>(na) * 4)) return st;
        return nb > 0 ? mimir_copy(ctx, y + na, b, static_cast<size_t>(nb) * 4) : MIMIR_OK;
    }
    // Every other operation reads branch2[i] for i < branch1.size().
    MIMIR_REQUIRE(ctx, nb >= na,
                  "branch merge: the source branch has %lld floats, fewer than the %lld it is merged with",
                  (long long)nb, (long long)na);
    if (na == 0) return MIMIR_OK;
    MIMIR_REQUIRE(ctx, a && b && y, "branch merge: null tensor");
    MIMIR_ENTER(ctx);
    switch (merge_op) {
        case MIMIR_MERGE_MULTIPLY:
            return run_binary(ctx, a, b, y, na, Mul{}, "merge_mul");
        case MIMIR_MERGE_AVERAGE:
            return run_binary(ctx, a, b, y, na, Average{}, "merge_average");
        case MIMIR_MERGE_MAX: {
            const int64_t body = na / 8 * 8;  // the 8-wide AVX2 loop, then the tail
            if (body > 0)
                if (int st = run_binary(ctx, a, b, y, body, MaxBody{}, "merge_max")) return st;
            return na > body ? run_binary(ctx, a + body, b + body, y + body, na - body, MaxTail{}, "merge_max")
                             : MIMIR_OK;
        }
        default:  // ADD (:4355-4380); GATED, ATTENTION_WEIGHTED: copy then += (:4470-4477)
            return run_binary(ctx, a, b, y, na, Add{}, "merge_add");
    }
}

int mimir_mul_fwd(mimir_ctx* ctx, const float* a, int64_t na, const float* b, int64_t nb,
                  float* y) {
    if (!ctx) return MIMIR_EINVAL;
    // LayerOps.hpp:209-211
    MIMIR_REQUIRE(ctx, na == nb && na >= 0, "Multiply: input sizes must match (%lld vs %lld)",
                  (long long)na, (long long)nb);
    if (na == 0) return MIMIR_OK;
    MIMIR_REQUIRE(ctx, a && b && y, "Multiply: null tensor");
    MIMIR_ENTER(ctx);
    return run_binary(ctx, a, b, y, na, Mul{}, "mul");
}

}  // extern "C"
