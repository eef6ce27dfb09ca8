// backward.hip -- backward of the path's ops for gfx950: the branches of
// Model::backwardPass (Model.cpp:7305-9153) for LayerNorm, GELU, SiLU,
// Multiply, Add and Embedding.
//
// The reference builds with -std=c++17 (CMakeLists.txt:8-10, no GNU
// extensions), so GCC does not contract a*b+c into FMAs there; this file
// turns contraction off as well, so every product and sum is rounded where
// the reference rounds it.  That keeps Multiply's and Add's gradients, and
// accumulate_grad's `dst += src` (Model.cpp:7329-7341), bit-identical.
//
// Kernels:
//   dact_vec / dact_scalar   GELU and SiLU input gradients (3 streams)
//   mul_bwd_*                Multiply: da = dy*b, db = dy*a (5 streams)
//   add_bwd_*                Add: the big operand's gradient is dy itself;
//                            the broadcast operand's is a column (or total)
//                            sum of dy, reduced in two deterministic passes
//   ln_bwd_vec               LayerNorm, rows held in VGPRs as in the forward
//                            (rows.hpp shapes), a persistent grid: each
//                            workgroup slot keeps its dgamma/dbeta column
//                            sums in registers over the rows it visits and
//                            writes them once; sum_slots adds the slots in a
//                            fixed order into grad_weights
//   ln_bwd_scalar            the same with 4-byte columns: rows up to 4096
//                            floats that are not 16-byte aligned or whose
//                            width is not a multiple of 4
//   ln_stats_generic, ln_bwd_params_part, ln_bwd_generic  any other width /
//                            alignment
//   embed_sort_*, embed_bwd_* scatter-add of dy rows into the gradient table:
//                            (id, token) pairs are sorted by id, stably (a
//                            counting sort up to 64K tokens, rocPRIM's radix
//                            sort above); an id with fewer than 32 tokens has its
//                            rows added in token order by one workgroup --
//                            the reference's sequence of float adds, bit for
//                            bit -- and a more frequent id's rows are summed
//                            in 32-token segments in parallel, then the
//                            segment sums in a fixed grouping (deterministic,
//                            the reference's sum to float32 rounding).
#include "common.hpp"
#include "internal.hpp"
#include "ids.hpp"

#include <math.h>
#include <mutex>

#include <rocprim/block/block_radix_sort.hpp>
#include <rocprim/block/block_scan.hpp>
#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/iterator/counting_iterator.hpp>
#include <rocprim/iterator/transform_iterator.hpp>

#pragma clang fp contract(off)

using namespace mimir;

namespace {

// ---------------------------------------------------------------------------
// Elementwise input gradients
// ---------------------------------------------------------------------------

// GELU branch, Model.cpp:9026-9051:
//   u = s*(x + c*x^3), t = tanh(u),
//   dgelu = 0.5*(1+t) + 0.5*x*(1-t*t)*du_dx,   du_dx = s*(1 + 3c*x^2)
// evaluated with e = exp(-2|u|) and r = 1/(1+e), for which
//   0.5*(1+t) = sigmoid(2u) = (u >= 0 ? r : e*r)   and   1 - t*t = 4*e*r^2
// exactly: the same function without the cancellation of 1+t and 1-t*t
// (the reference's float result carries a few ulp of 1 there, times
// 0.5*|x|*du_dx).  inf / NaN inputs give NaN, as in the reference.
__device__ __forceinline__ float dgelu1(float x) {
    const float s = __builtin_sqrtf(2.0f / 3.14159265359f);
    const float c = 0.044715f;
    const float u = s * (x + c * x * x * x);
    const float e = expf(-2.0f * fabsf(u));
    const float r = __builtin_amdgcn_rcpf(1.0f + e);
    const float half_1pt = u >= 0.0f ? r : e * r;
    const float sech2 = 4.0f * e * r * r;
    const float du_dx = s * (1.0f + 3.0f * c * x * x);
    return half_1pt + 0.5f * x * sech2 * du_dx;
}

// SiLU branch, Model.cpp:8021-8027: s = 1/(1+exp(-x)); dy_dx = s + x*s*(1-s).
__device__ __forceinline__ float dsilu1(float x) {
    const float s = 1.0f / (1.0f + expf(-x));
    const float ds = s * (1.0f - s);
    return s + x * ds;
}

struct DGelu {
    __device__ float operator()(float x) const { return dgelu1(x); }
};
struct DSilu {
    __device__ float operator()(float x) const { return dsilu1(x); }
};

// dx = dy * f'(x), or dx += that (accumulate_grad into a present gradient).
// KEEP: dx through the caches (mimir_ctx_set_output_caching), as for every
// *_vec kernel below with a KEEP parameter.
template <class F, bool ACC, bool KEEP, int BS = kBlock>
__global__ __launch_bounds__(BS) void dact_vec(const float* x, const float* dy, float* dx, int64_t n4, F f) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * BS + threadIdx.x;
    if (i >= n4) return;
    const f4 xv = ld4<true>(x + 4 * i);
    const f4 g = ld4<true>(dy + 4 * i);
    f4 o{g.x * f(xv.x), g.y * f(xv.y), g.z * f(xv.z), g.w * f(xv.w)};
    if constexpr (ACC) o = ld4<true>(dx + 4 * i) + o;
    st_out<KEEP>(dx + 4 * i, o);
}

template <class F, bool ACC>
__global__ __launch_bounds__(kBlock) void dact_scalar(const float* x, const float* dy, float* dx, int64_t n, F f) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
        float o = dy[i] * f(x[i]);
        if constexpr (ACC) o = dx[i] + o;
        dx[i] = o;
    }
}

unsigned stride_grid(int64_t n) {
    const int64_t b = (n + kBlock - 1) / kBlock;
    return static_cast<unsigned>(b < 1 ? 1 : (b > 65536 ? 65536 : b));
}

template <class F, bool ACC>
int run_dact(mimir_ctx* ctx, const float* x, const float* dy, float* dx, int64_t n, F f, const char* name) {
    int64_t done = 0;
    if (aligned16(x) && aligned16(dy) && aligned16(dx)) {
        const int64_t n4 = n / 4;
        if (n4 > 0) {
            const int st = with_block(ew_block(ctx->tune), [&](auto bsc) {
                constexpr int BS = decltype(bsc)::value;
                unsigned blocks;
                if (!grid_for(n4, BS, BS, &blocks))
                    return fail(ctx, MIMIR_EINVAL, "%s: n=%lld exceeds the grid limit", name, (long long)n);
                if (ctx->keep_outputs) dact_vec<F, ACC, true, BS><<<blocks, BS, 0, ctx->stream>>>(x, dy, dx, n4, f);
                else dact_vec<F, ACC, false, BS><<<blocks, BS, 0, ctx->stream>>>(x, dy, dx, n4, f);
                return launched(ctx, name);
            });
            if (st) return st;
        }
        done = n4 * 4;
    }
    if (n > done) {
        dact_scalar<F, ACC><<<stride_grid(n - done), kBlock, 0, ctx->stream>>>(x + done, dy + done, dx + done,
                                                                             n - done, f);
        return launched(ctx, name);
    }
    return MIMIR_OK;
}

// ---------------------------------------------------------------------------
// Multiply (Model.cpp:7647-7665) and Add (7541-7601)
// ---------------------------------------------------------------------------

// g0 = dy*b and g1 = dy*a are formed before either is accumulated, as in
// the reference, so da / db may alias dy (element for element).
template <bool ACC_A, bool ACC_B, bool KEEP, int BS = kBlock>
__global__ __launch_bounds__(BS) void mul_bwd_vec(const float* a, const float* b, const float* dy, float* da,
                                                  float* db, int64_t n4) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * BS + threadIdx.x;
    if (i >= n4) return;
    const f4 g = ld4<true>(dy + 4 * i);
    f4 g0 = g * ld4<true>(b + 4 * i);
    f4 g1 = g * ld4<true>(a + 4 * i);
    if (da) {
        if constexpr (ACC_A) g0 = ld4<true>(da + 4 * i) + g0;
    }
    if (db) {
        if constexpr (ACC_B) g1 = ld4<true>(db + 4 * i) + g1;
    }
    if (da) st_out<KEEP>(da + 4 * i, g0);
    if (db) st_out<KEEP>(db + 4 * i, g1);
}

// da == db (Multiply of a tensor with itself): the second accumulation adds
// onto the first, ((da) + g0) + g1, as two accumulate_grad calls on one name.
template <bool ACC_A>
__global__ __launch_bounds__(kBlock) void mul_bwd_same(const float* a, const float* b, const float* dy, float* d,
                                                       int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
        const float g = dy[i];
        const float g0 = g * b[i];
        const float g1 = g * a[i];
        float o = ACC_A ? d[i] + g0 : g0;
        d[i] = o + g1;
    }
}

template <bool ACC_A, bool ACC_B>
__global__ __launch_bounds__(kBlock) void mul_bwd_scalar(const float* a, const float* b, const float* dy, float* da,
                                                         float* db, int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
        const float g = dy[i];
        float g0 = g * b[i];
        float g1 = g * a[i];
        if (da && ACC_A) g0 = da[i] + g0;
        if (db && ACC_B) g1 = db[i] + g1;
        if (da) da[i] = g0;
        if (db) db[i] = g1;
    }
}

// dst = src or dst += src over n floats (accumulate_grad, Model.cpp:7329-7341).
template <bool ACC, bool KEEP>
__global__ __launch_bounds__(kBlock) void acc_vec(const float* src, float* dst, int64_t n4) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= n4) return;
    f4 o = ld4<true>(src + 4 * i);
    if constexpr (ACC) o = ld4<true>(dst + 4 * i) + o;
    st_out<KEEP>(dst + 4 * i, o);
}

template <bool ACC>
__global__ __launch_bounds__(kBlock) void acc_scalar(const float* src, float* dst, int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
        float o = src[i];
        if constexpr (ACC) o = dst[i] + o;
        dst[i] = o;
    }
}

// Equal sizes and no aliasing: da (+)= dy and db (+)= dy in one pass.
template <bool ACC_A, bool ACC_B, bool KEEP, int BS = kBlock>
__global__ __launch_bounds__(BS) void add_bwd_vec(const float* dy, float* da, float* db, int64_t n4) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * BS + threadIdx.x;
    if (i >= n4) return;
    const f4 g = ld4<true>(dy + 4 * i);
    // Every load before the stores, which are written through (two output
    // streams per input stream).
    const f4 oa = ACC_A && da ? ld4<true>(da + 4 * i) + g : g;
    const f4 ob = ACC_B && db ? ld4<true>(db + 4 * i) + g : g;
    if (da) st_out<KEEP, kStoreThrough>(da + 4 * i, oa);
    if (db) st_out<KEEP, kStoreThrough>(db + 4 * i, ob);
}

template <bool KEEP, int BS>
void launch_mul_bwd(mimir_ctx* ctx, unsigned blocks, bool A, bool B, const float* a, const float* b, const float* dy,
                    float* da, float* db, int64_t n4) {
    if (A && B) mul_bwd_vec<true, true, KEEP, BS><<<blocks, BS, 0, ctx->stream>>>(a, b, dy, da, db, n4);
    else if (A) mul_bwd_vec<true, false, KEEP, BS><<<blocks, BS, 0, ctx->stream>>>(a, b, dy, da, db, n4);
    else if (B) mul_bwd_vec<false, true, KEEP, BS><<<blocks, BS, 0, ctx->stream>>>(a, b, dy, da, db, n4);
    else mul_bwd_vec<false, false, KEEP, BS><<<blocks, BS, 0, ctx->stream>>>(a, b, dy, da, db, n4);
}

template <bool KEEP, int BS>
void launch_add_bwd(mimir_ctx* ctx, unsigned blocks, bool A, bool B, const float* dy, float* da, float* db,
                    int64_t n4) {
    if (A && B) add_bwd_vec<true, true, KEEP, BS><<<blocks, BS, 0, ctx->stream>>>(dy, da, db, n4);
    else if (A) add_bwd_vec<true, false, KEEP, BS><<<blocks, BS, 0, ctx->stream>>>(dy, da, db, n4);
    else if (B) add_bwd_vec<false, true, KEEP, BS><<<blocks, BS, 0, ctx->stream>>>(dy, da, db, n4);
    else add_bwd_vec<false, false, KEEP, BS><<<blocks, BS, 0, ctx->stream>>>(dy, da, db, n4);
}

int accumulate(mimir_ctx* ctx, const float* src, float* dst, int64_t n, bool acc, const char* name) {
    int64_t done = 0;
    if (aligned16(src) && aligned16(dst)) {
        const int64_t n4 = n / 4;
        if (n4 > 0) {
            unsigned blocks;
            if (!grid_for(n4, kBlock, kBlock, &blocks))
                return fail(ctx, MIMIR_EINVAL, "%s: n=%lld exceeds the grid limit", name, (long long)n);
            const bool k = ctx->keep_outputs != 0;
            if (acc && k) acc_vec<true, true><<<blocks, kBlock, 0, ctx->stream>>>(src, dst, n4);
            else if (acc) acc_vec<true, false><<<blocks, kBlock, 0, ctx->stream>>>(src, dst, n4);
            else if (k) acc_vec<false, true><<<blocks, kBlock, 0, ctx->stream>>>(src, dst, n4);
            else acc_vec<false, false><<<blocks, kBlock, 0, ctx->stream>>>(src, dst, n4);
            if (int st = launched(ctx, name)) return st;
        }
        done = n4 * 4;
    }
    if (n > done) {
        if (acc) acc_scalar<true><<<stride_grid(n - done), kBlock, 0, ctx->stream>>>(src + done, dst + done, n - done);
        else acc_scalar<false><<<stride_grid(n - done), kBlock, 0, ctx->stream>>>(src + done, dst + done, n - done);
        return launched(ctx, name);
    }
    return MIMIR_OK;
}

// ---------------------------------------------------------------------------
// Deterministic column sums: partial sums per slot, then slots in order
// ---------------------------------------------------------------------------

constexpr int kSumLanes = 16;  // waves per sum_slots workgroup, one slot lane each

// out[c] (+)= sum over slots k of part[k*stride + c], c < width: wave l of
// the workgroup adds slots l, l+16, ... for 64 consecutive columns; the 16
// lane sums are then added in lane order.  Columns below `split` go to out0,
// the rest to out1 (dgamma | dbeta).
__global__ __launch_bounds__(kSumLanes * kWave) void sum_slots(const float* part, int64_t nslots, int64_t stride,
                                                               int64_t width, float* out0, float* out1, int64_t split,
                                                               int acc) {
    __shared__ float lds[kSumLanes][kWave];
    const int lane = threadIdx.x / kWave;
    const int col = threadIdx.x % kWave;
    const int64_t c = static_cast<int64_t>(blockIdx.x) * kWave + col;
    float s = 0.0f;
    if (c < width)
        for (int64_t k = lane; k < nslots; k += kSumLanes) s += part[k * stride + c];
    lds[lane][col] = s;
    __syncthreads();
    if (lane == 0 && c < width) {
        float t = lds[0][col];
#pragma unroll
        for (int l = 1; l < kSumLanes; ++l) t += lds[l][col];
        float* o = c < split ? out0 + c : out1 + (c - split);
        *o = acc ? *o + t : t;
    }
}

// The same with 16-byte columns (width, stride and split multiples of 4):
// each slot lane issues U loads before adding them in slot order, so the sum
// order (hence every bit of the result) is that of sum_slots.
template <int U>
__global__ __launch_bounds__(kSumLanes * kWave) void sum_slots4(const float* part, int64_t nslots, int64_t stride,
                                                                int64_t width, float* out0, float* out1,
                                                                int64_t split, int acc) {
    __shared__ f4 lds[kSumLanes][kWave];
    const int lane = threadIdx.x / kWave;
    const int col = threadIdx.x % kWave;
    const int64_t c4 = static_cast<int64_t>(blockIdx.x) * kWave + col;
    // The values accumulated onto are loaded first, off the critical path.
    float prev[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (acc && lane == 0 && 4 * c4 < width) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t c = 4 * c4 + i;
            prev[i] = c < split ? out0[c] : out1[c - split];
        }
    }
    f4 s = f4(0.0f);
    if (4 * c4 < width) {
        const f4* p = reinterpret_cast<const f4*>(part) + c4;
        const int64_t st4 = stride / 4;
        int64_t k = lane;
        for (; k + (U - 1) * kSumLanes < nslots; k += U * kSumLanes) {
            f4 v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) v[u] = p[(k + u * kSumLanes) * st4];
#pragma unroll
            for (int u = 0; u < U; ++u) s += v[u];
        }
        for (; k < nslots; k += kSumLanes) s += p[k * st4];
    }
    lds[lane][col] = s;
    __syncthreads();
    if (lane == 0 && 4 * c4 < width) {
        f4 t = lds[0][col];
#pragma unroll
        for (int l = 1; l < kSumLanes; ++l) t += lds[l][col];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t c = 4 * c4 + i;
            float* o = c < split ? out0 + c : out1 + (c - split);
            *o = acc ? prev[i] + t[i] : t[i];
        }
    }
}

// First level of a two-level slot sum for many slots: group g (blockIdx.y)
// of kGroups sums its contiguous range of slots for 64 float4 columns
// (blockIdx.x); its 4 waves take interleaved slots, each adding U loads at
// a time in slot order, and the 4 wave sums are added in wave order:
// lvl2[g*width + c] = the group's sum.  sum_slots4 then adds the kGroups
// rows in order.  (Folding that second level into this kernel with an
// arrival counter needs a device-scope release per block, which on this
// GPU writes back the XCD's L2 each time and costs far more than a launch.)
constexpr int kGroups = kSlotGroups;

template <int U>
__global__ __launch_bounds__(kBlock) void slot_groups4(const float* part, int64_t nslots, int64_t stride,
                                                       int64_t width, float* lvl2) {
    constexpr int W = kBlock / kWave;
    __shared__ f4 lds[W][kWave];
    const int w = threadIdx.x / kWave;
    const int col = threadIdx.x % kWave;
    const int64_t c4 = static_cast<int64_t>(blockIdx.x) * kWave + col;
    const int64_t per = (nslots + kGroups - 1) / kGroups;
    const int64_t k0 = static_cast<int64_t>(blockIdx.y) * per;
    const int64_t k1 = k0 + per < nslots ? k0 + per : nslots;
    f4 s = f4(0.0f);
    if (4 * c4 < width) {
        const f4* p = reinterpret_cast<const f4*>(part) + c4;
        const int64_t st4 = stride / 4;
        int64_t k = k0 + w;
        for (; k + (U - 1) * W < k1; k += U * W) {
            f4 v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) v[u] = p[(k + u * W) * st4];
#pragma unroll
            for (int u = 0; u < U; ++u) s += v[u];
        }
        for (; k < k1; k += W) s += p[k * st4];
    }
    lds[w][col] = s;
    __syncthreads();
    if (w == 0 && 4 * c4 < width) {
        f4 t = lds[0][col];
#pragma unroll
        for (int l = 1; l < W; ++l) t += lds[l][col];
        reinterpret_cast<f4*>(lvl2 + static_cast<int64_t>(blockIdx.y) * width)[c4] = t;
    }
}

// The slot sum in one launch, for up to kTileMaxSlots slots: workgroup b
// sums every slot for float4 columns kTileCols*b .. kTileCols*b + 7 of the
// summed width (one workgroup per CU at the LayerNorm backward's 2048
// columns).  Lane l of wave w holds column kTileCols*b + (l & 7) and slot
// lane q = 8w + (l >> 3) of kTileLanes, and adds slots q, q + 128, ... in
// order with U loads in flight (one round trip for 512 slots); each load
// instruction reads eight slots' 128 contiguous bytes.  The 128 slot lanes
// of a column are then added in a fixed order: the eight of a wave by three
// lane swaps (((q0 + q1) + (q2 + q3)) + ((q4 + q5) + (q6 + q7)), the same
// bits in every lane), the 16 waves through LDS in wave order.  The
// two-level form (slot_groups4, then sum_slots4) costs two launches of
// ~4.5 us each on MI355X.
constexpr int kTileCols = 8;
constexpr int kTileLanes = 1024 / kTileCols;
constexpr int64_t kTileMaxSlots = 2048;  // at most four rounds of U loads per slot lane

__device__ __forceinline__ f4 shfl_xor4(f4 v, int m) {
    f4 r;
    r.x = __shfl_xor(v.x, m);
    r.y = __shfl_xor(v.y, m);
    r.z = __shfl_xor(v.z, m);
    r.w = __shfl_xor(v.w, m);
    return r;
}

template <int U>
__global__ __launch_bounds__(1024) void sum_slots_tile(const float* part, int64_t nslots, int64_t stride,
                                                       int64_t width, float* out0, float* out1, int64_t split,
                                                       int acc) {
    constexpr int NW = 1024 / kWave;
    __shared__ f4 lds[NW][kTileCols];
    const int w = threadIdx.x / kWave;
    const int l = threadIdx.x % kWave;
    const int col = l & (kTileCols - 1);
    const int64_t q = (kWave / kTileCols) * w + (l / kTileCols);
    const int64_t c4 = static_cast<int64_t>(blockIdx.x) * kTileCols + col;
    f4 s = f4(0.0f);
    if (4 * c4 < width) {
        const f4* p = reinterpret_cast<const f4*>(part) + c4;
        const int64_t st4 = stride / 4;
        int64_t k = q;
        for (; k + (U - 1) * kTileLanes < nslots; k += U * kTileLanes) {
            f4 v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) v[u] = p[(k + u * kTileLanes) * st4];
#pragma unroll
            for (int u = 0; u < U; ++u) s += v[u];
        }
        for (; k < nslots; k += kTileLanes) s += p[k * st4];
    }
#pragma unroll
    for (int m = kTileCols; m < kWave; m <<= 1) s += shfl_xor4(s, m);  // the wave's slot lanes, pairwise
    if (l < kTileCols) lds[w][col] = s;
    __syncthreads();
    if (threadIdx.x < kTileCols && 4 * c4 < width) {
        f4 t = lds[0][col];
#pragma unroll
        for (int i = 1; i < NW; ++i) t += lds[i][col];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t c = 4 * c4 + i;
            float* o = c < split ? out0 + c : out1 + (c - split);
            *o = acc ? *o + t[i] : t[i];
        }
    }
}

// out[0] (+)= the sum of the first float of nslots slots (row stride
// `stride`): 1024 threads add slots t, t+1024, ... in order, then the block
// tree adds the threads in order.
__global__ __launch_bounds__(1024) void sum_total(const float* part, int64_t nslots, int64_t stride, float* out,
                                                  int acc) {
    __shared__ float lds[1024 / kWave];
    float s = 0.0f;
    for (int64_t k = threadIdx.x; k < nslots; k += 1024) s += part[k * stride];
    s = block_sum<1024 / kWave>(s, lds);
    if (threadIdx.x == 0) *out = acc ? *out + s : s;
}

// out (+)= the sum of nslots slot rows of `part` (row stride `stride`, first
// `width` columns; columns below `split` to out0, the rest to out1).  With
// `tmp` (kGroups*width floats) and many slots, two levels; else one.
int launch_sum_slots(mimir_ctx* ctx, const float* part, int64_t nslots, int64_t stride, int64_t width, float* out0,
                     float* out1, int64_t split, bool acc, float* tmp = nullptr) {
    unsigned blocks;
    if (width % 4 == 0 && stride % 4 == 0 && split % 4 == 0 && aligned16(part)) {
        if (nslots >= 4 * kGroups && nslots <= kTileMaxSlots) {
            if (!grid_for(width / 4, kTileCols, 1024, &blocks))
                return fail(ctx, MIMIR_EINVAL, "sum_slots: width %lld exceeds the grid limit", (long long)width);
            sum_slots_tile<4><<<blocks, 1024, 0, ctx->stream>>>(part, nslots, stride, width, out0, out1, split,
                                                               acc ? 1 : 0);
            return launched(ctx, "sum_slots_tile");
        }
        if (!grid_for(width / 4, kWave, kBlock, &blocks))
            return fail(ctx, MIMIR_EINVAL, "sum_slots: width %lld exceeds the grid limit", (long long)width);
        if (tmp && aligned16(tmp) && nslots >= 4 * kGroups) {
            slot_groups4<8><<<dim3(blocks, kGroups), kBlock, 0, ctx->stream>>>(part, nslots, stride, width, tmp);
            if (int st = launched(ctx, "slot_groups4")) return st;
            part = tmp;
            nslots = kGroups;
            stride = width;
        }
        sum_slots4<8><<<blocks, kSumLanes * kWave, 0, ctx->stream>>>(part, nslots, stride, width, out0, out1, split,
                                                                     acc ? 1 : 0);
        return launched(ctx, "sum_slots4");
    }
    if (width == 1) {
        sum_total<<<1, 1024, 0, ctx->stream>>>(part, nslots, stride, out0, acc ? 1 : 0);
        return launched(ctx, "sum_total");
    }
    if (!grid_for(width, kWave, kSumLanes * kWave, &blocks))
        return fail(ctx, MIMIR_EINVAL, "sum_slots: width %lld exceeds the grid limit", (long long)width);
    sum_slots<<<blocks, kSumLanes * kWave, 0, ctx->stream>>>(part, nslots, stride, width, out0, out1, split,
                                                             acc ? 1 : 0);
    return launched(ctx, "sum_slots");
}

// 16-byte columns per block of add_bcast_part: all kBlock threads for wide
// rows, else the next power of two above the row's float4 count.
__host__ __device__ inline int bcast_cols_per_block(int64_t w4) {
    int cw = 1;
    while (cw < kBlock && cw < w4) cw *= 2;
    return cw;
}

// Broadcast Add backward in one pass over dy, viewed as [rows x cols]
// (cols = the small operand's size): the big operand's gradient d_big (+)= dy
// (:7577), and per chunk of `chunk` rows the column sums of what the
// reference then reduces (:7586-7594) -- dy, or the updated d_big when it is
// the same buffer as dy (the reference's grad_out is that map entry).
// part[k*cols + c], rows in order.  VEC: 16-byte columns, four rows' loads in
// flight per thread (each element is read before it is written, so d_big may
// alias dy).
template <bool VEC>
__global__ __launch_bounds__(kBlock) void add_bcast_part(const float* dy, float* d_big, int acc_big, int64_t rows,
                                                         int64_t cols, int64_t chunk, float* part) {
    const int64_t r0 = static_cast<int64_t>(blockIdx.y) * chunk;
    const int64_t r1 = r0 + chunk < rows ? r0 + chunk : rows;
    const bool same = d_big == dy;
    if constexpr (VEC) {
        // cw = 16-byte columns per block (a power of two up to kBlock); narrow
        // rows pack L = kBlock / cw row lanes per block, lane l taking rows
        // l, l+L, ... of the chunk; the lanes are added in lane order.
        __shared__ f4 lds[kBlock];
        const int64_t w4 = cols / 4;
        const int cw = bcast_cols_per_block(w4);
        const int L = kBlock / cw;
        const int col = threadIdx.x % cw;
        const int lane = threadIdx.x / cw;
        const int64_t c4 = static_cast<int64_t>(blockIdx.x) * cw + col;
        const bool live = c4 < w4;
        const f4* src = reinterpret_cast<const f4*>(dy) + c4;
        f4* dst = d_big ? reinterpret_cast<f4*>(d_big) + c4 : nullptr;
        f4 s = f4(0.0f);
        if (live) {
            int64_t r = r0 + lane;
            for (; r + 3 * L < r1; r += 4 * L) {
                f4 v[4], o[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) v[u] = __builtin_nontemporal_load(src + (r + u * L) * w4);
                if (dst) {
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        o[u] = acc_big ? __builtin_nontemporal_load(dst + (r + u * L) * w4) + v[u] : v[u];
#pragma unroll
                    for (int u = 0; u < 4; ++u) st_stream(dst + (r + u * L) * w4, o[u]);
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) s += (same ? o[u] : v[u]);
            }
            for (; r < r1; r += L) {
                const f4 v = __builtin_nontemporal_load(src + r * w4);
                f4 o = v;
                if (dst) {
                    o = acc_big ? __builtin_nontemporal_load(dst + r * w4) + v : v;
                    st_stream(dst + r * w4, o);
                }
                s += (same ? o : v);
            }
        }
        if (L > 1) {
            lds[threadIdx.x] = s;
            __syncthreads();
            if (lane != 0) return;
            for (int l = 1; l < L; ++l) s += lds[l * cw + col];
        }
        if (live) reinterpret_cast<f4*>(part + static_cast<int64_t>(blockIdx.y) * cols)[c4] = s;
    } else {
        const int64_t c = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
        if (c >= cols) return;
        float s = 0.0f;
        for (int64_t r = r0; r < r1; ++r) {
            const float v = dy[r * cols + c];
            float o = v;
            if (d_big) {
                o = acc_big ? d_big[r * cols + c] + v : v;
                d_big[r * cols + c] = o;
            }
            s += (same ? o : v);
        }
        part[static_cast<int64_t>(blockIdx.y) * cols + c] = s;
    }
}

// The scalar broadcast (small_n == 1): the same over contiguous chunks of
// `chunk` floats (a multiple of 4 * kBlock when VEC), one block each;
// part[k] = the chunk's sum.
template <bool VEC>
__global__ __launch_bounds__(kBlock) void add_total_part(const float* dy, float* d_big, int acc_big, int64_t n,
                                                         int64_t chunk, float* part) {
    __shared__ float lds[kBlock / kWave];
    const int64_t i0 = static_cast<int64_t>(blockIdx.x) * chunk;
    const int64_t i1 = i0 + chunk < n ? i0 + chunk : n;
    const bool same = d_big == dy;
    float s = 0.0f;
    if constexpr (VEC) {
        const f4* src = reinterpret_cast<const f4*>(dy);
        f4* dst = reinterpret_cast<f4*>(d_big);
        const int64_t e4 = i1 / 4;
        f4 acc = f4(0.0f);
        int64_t i = i0 / 4 + threadIdx.x;
        for (; i + 3 * kBlock < e4; i += 4 * kBlock) {
            f4 v[4], o[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = __builtin_nontemporal_load(src + i + u * kBlock);
            if (dst) {
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    o[u] = acc_big ? __builtin_nontemporal_load(dst + i + u * kBlock) + v[u] : v[u];
#pragma unroll
                for (int u = 0; u < 4; ++u) st_stream(dst + i + u * kBlock, o[u]);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) acc += (same ? o[u] : v[u]);
        }
        for (; i < e4; i += kBlock) {
            const f4 v = __builtin_nontemporal_load(src + i);
            f4 o = v;
            if (dst) {
                o = acc_big ? __builtin_nontemporal_load(dst + i) + v : v;
                st_stream(dst + i, o);
            }
            acc += (same ? o : v);
        }
        s = (acc.x + acc.y) + (acc.z + acc.w);
        // The tail of n beyond the last multiple of 4 (last chunk only).
        for (int64_t k = 4 * e4 + threadIdx.x; k < i1; k += kBlock) {
            const float v = dy[k];
            float o = v;
            if (d_big) {
                o = acc_big ? d_big[k] + v : v;
                d_big[k] = o;
            }
            s += (same ? o : v);
        }
    } else {
        for (int64_t i = i0 + threadIdx.x; i < i1; i += kBlock) {
            const float v = dy[i];
            float o = v;
            if (d_big) {
                o = acc_big ? d_big[i] + v : v;
                d_big[i] = o;
            }
            s += (same ? o : v);
        }
    }
    s = block_sum<kBlock / kWave>(s, lds);
    if (threadIdx.x == 0) part[blockIdx.x] = s;
}

// Add backward with a broadcast operand (Model.cpp:7561-7594): d_big (+)= dy,
// then d_small (+)= the sum of dy over the big operand's tiles (small_n > 1)
// or over all of it (small_n == 1), in one pass over dy and a deterministic
// sum of the per-chunk partial sums.
int add_bcast_bwd(mimir_ctx* ctx, const float* dy, int64_t n_big, int64_t n_small, float* d_big, bool acc_big,
                  float* d_small, bool acc_small) {
    if (n_small == 1) {
        const bool vec = aligned16(dy) && (!d_big || aligned16(d_big));
        const int64_t chunk = 16 * 4 * kBlock;  // 16 KiB floats per block
        const int64_t nchunks = (n_big + chunk - 1) / chunk;
        void* s = nullptr;
        if (int st = ensure_scratch(ctx, sizeof(float) * static_cast<size_t>(nchunks), &s)) return st;
        unsigned blocks;
        if (!grid_for(nchunks, 1, kBlock, &blocks)) return fail(ctx, MIMIR_EINVAL, "Add backward: operand too large");
        if (vec) add_total_part<true><<<blocks, kBlock, 0, ctx->stream>>>(dy, d_big, acc_big, n_big, chunk,
                                                                         static_cast<float*>(s));
        else add_total_part<false><<<blocks, kBlock, 0, ctx->stream>>>(dy, d_big, acc_big, n_big, chunk,
                                                                      static_cast<float*>(s));
        if (int st = launched(ctx, "add_total_part")) return st;
        return launch_sum_slots(ctx, static_cast<float*>(s), nchunks, 1, 1, d_small, d_small, 1, acc_small);
    }
    const int64_t rows = n_big / n_small;
    const bool vec = n_small % 4 == 0 && aligned16(dy) && (!d_big || aligned16(d_big));
    // About 1024 workgroups over (column blocks x row chunks), chunks of at
    // least 8 rows: partial sums stay a few percent of dy.
    const int64_t cw = vec ? bcast_cols_per_block(n_small / 4) : kBlock;
    const int64_t lanes = vec ? kBlock / cw : 1;
    const int64_t cblocks = ((vec ? n_small / 4 : n_small) + cw - 1) / cw;
    int64_t nchunks = (1024 + cblocks - 1) / cblocks;
    if (nchunks > rows / (8 * lanes)) nchunks = rows / (8 * lanes);
    if (nchunks < 1) nchunks = 1;
    if (nchunks > 65535) nchunks = 65535;
    const int64_t chunk = (rows + nchunks - 1) / nchunks;
    nchunks = (rows + chunk - 1) / chunk;
    if (!dispatch_fits(cblocks, kBlock)) return fail(ctx, MIMIR_EINVAL, "Add backward: operand too large");
    void* s = nullptr;
    const size_t part_floats = static_cast<size_t>((nchunks + kGroups) * n_small);
    if (int st = ensure_scratch(ctx, sizeof(float) * part_floats, &s)) return st;
    float* part = static_cast<float*>(s);
    const dim3 grid(static_cast<unsigned>(cblocks), static_cast<unsigned>(nchunks));
    if (vec) add_bcast_part<true><<<grid, kBlock, 0, ctx->stream>>>(dy, d_big, acc_big, rows, n_small, chunk, part);
    else add_bcast_part<false><<<grid, kBlock, 0, ctx->stream>>>(dy, d_big, acc_big, rows, n_small, chunk, part);
    if (int st = launched(ctx, "add_bcast_part")) return st;
    return launch_sum_slots(ctx, part, nchunks, n_small, n_small, d_small, d_small, n_small, acc_small,
                            part + nchunks * n_small);
}

// ---------------------------------------------------------------------------
// LayerNorm backward (Model.cpp:7719-7821)
// ---------------------------------------------------------------------------

struct LnBwdArgs {
    const float* x;
    const float* dy;
    const float* g;  // gamma (null: not affine, gamma = 1)
    float* dx;
    float* part;     // [slots][2*cols] dgamma | dbeta partial sums (null: not wanted)
    float* stats;    // generic path: [rows][2] mean, inv_std
    int64_t rows;
    int64_t cols;
    float eps;
    int acc;         // dx += value instead of dx = value
};

// Two sums over one row at once (one LDS round).
template <int NW>
__device__ __forceinline__ void row_sum2(float& a, float& b, float* la, float* lb, int sub) {
    a = wave_sum(a);
    b = wave_sum(b);
    if constexpr (NW > 1) {
        if ((threadIdx.x & (kWave - 1)) == 0) {
            la[threadIdx.x / kWave] = a;
            lb[threadIdx.x / kWave] = b;
        }
        __syncthreads();
        float sa = la[sub * NW], sb = lb[sub * NW];
#pragma unroll
        for (int i = 1; i < NW; ++i) {
            sa += la[sub * NW + i];
            sb += lb[sub * NW + i];
        }
        a = sa;
        b = sb;
    }
}

__device__ __forceinline__ float hsum(f4 v) { return (v.x + v.y) + (v.z + v.w); }

// A persistent grid (fewer blocks than row groups): sub-row `sub` of block b
// visits rows sub + RPB*(b + k*grid) and keeps dgamma / dbeta for its
// TPR*VPT*4 columns in registers; the block writes one slot of partial sums.
// The two reduction rounds of a row use separate LDS arrays, so each
// array's reuse (next row) is separated from its reads by the other round's
// barrier: no leading barriers are needed.
template <int TPR, int VPT, int BS, bool KEEP>
__global__ __launch_bounds__(BS) void ln_bwd_vec(LnBwdArgs a) {
    constexpr int RPB = BS / TPR;
    constexpr int NW = TPR / kWave;
    __shared__ float lds[4][BS / kWave];
    const int t = threadIdx.x % TPR;
    const int sub = threadIdx.x / TPR;
    const int64_t c4n = a.cols >> 2;
    const float n = static_cast<float>(a.cols);
    const float invF = 1.0f / n;  // Model.cpp:7799
    f4 gm[VPT], dg[VPT], db[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t c4 = static_cast<int64_t>(j) * TPR + t;
        gm[j] = (a.g && c4 < c4n) ? *reinterpret_cast<const f4*>(a.g + 4 * c4) : f4(1.0f);
        dg[j] = f4(0.0f);
        db[j] = f4(0.0f);
    }
    const int64_t step = static_cast<int64_t>(gridDim.x) * RPB;
    // Row group `b`'s x and dy for this thread (zeros past the end).
    auto load_rows = [&](int64_t b, f4* xo, f4* go) {
        const int64_t r = b + sub;
        const int64_t l = r < a.rows ? c4n : 0;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int64_t c4 = static_cast<int64_t>(j) * TPR + t;
            const bool ok = c4 < l;
            xo[j] = ok ? ld4<true>(a.x + r * a.cols + 4 * c4) : f4(0.0f);
            go[j] = ok ? ld4<true>(a.dy + r * a.cols + 4 * c4) : f4(0.0f);
        }
    };
    f4 xv[VPT], gv[VPT];
    load_rows(static_cast<int64_t>(blockIdx.x) * RPB, xv, gv);
    for (int64_t base = static_cast<int64_t>(blockIdx.x) * RPB; base < a.rows; base += step) {
        const int64_t row = base + sub;
        const int64_t lim = row < a.rows ? c4n : 0;  // past-end rows join the barriers only
        const int64_t off = row * a.cols;
        // The next row group's loads go out before this one's reductions, so
        // each wave keeps memory busy while it waits at the barriers.
        f4 xn[VPT], gn[VPT];
        load_rows(base + step, xn, gn);
        // Two reduction rounds per row.  Round 1: sum(x) and sum(dxhat)
        // (dxhat = dy*gamma needs no statistics).  Round 2, with the mean:
        // sum((x-mean)^2) for the reference's two-pass variance and
        // sum(dxhat*(x-mean)), which times inv_std is the reference's
        // sum(dxhat*xhat) (:7783-7797) up to rounding.
        float s = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            s += hsum(xv[j]);
            s1 += hsum(gv[j] * gm[j]);
        }
        row_sum2<NW>(s, s1, lds[0], lds[1], sub);
        const float mean = s / n;  // :7765-7768
        float q = 0.0f, p2 = 0.0f;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int64_t c4 = static_cast<int64_t>(j) * TPR + t;
            if (c4 < lim) {
                const f4 d = xv[j] - mean;
                q += (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
                p2 += hsum(gv[j] * gm[j] * d);
            }
        }
        row_sum2<NW>(q, p2, lds[2], lds[3], sub);
        const float var = q / n;                          // :7770-7776
        const float inv_std = 1.0f / sqrtf(var + a.eps);  // :7777
        const float s2 = p2 * inv_std;
        const float k = inv_std * invF;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {  // :7783-7805
            const int64_t c4 = static_cast<int64_t>(j) * TPR + t;
            if (c4 < lim) {
                const f4 xh = (xv[j] - mean) * inv_std;
                const f4 dxh = gv[j] * gm[j];
                dg[j] += gv[j] * xh;
                db[j] += gv[j];
                f4 o = k * ((n * dxh - s1) - xh * s2);
                if (a.acc) o = ld4<true>(a.dx + off + 4 * c4) + o;
                st_out<KEEP>(a.dx + off + 4 * c4, o);
            }
        }
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            xv[j] = xn[j];
            gv[j] = gn[j];
        }
    }
    if (!a.part) return;
    // One slot per workgroup: the sub-rows' sums are added in sub-row order
    // through LDS, then written once.
    float* p = a.part + static_cast<int64_t>(blockIdx.x) * 2 * a.cols;
    if constexpr (RPB > 1) {
        __shared__ f4 comb[2 * TPR * VPT];
        for (int r = 0; r < RPB; ++r) {
            if (sub == r) {
#pragma unroll
                for (int j = 0; j < VPT; ++j) {
                    const int i = j * TPR + t;
                    comb[i] = r == 0 ? dg[j] : comb[i] + dg[j];
                    comb[TPR * VPT + i] = r == 0 ? db[j] : comb[TPR * VPT + i] + db[j];
                }
            }
            __syncthreads();
        }
        if (sub != 0) return;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            dg[j] = comb[j * TPR + t];
            db[j] = comb[TPR * VPT + j * TPR + t];
        }
    }
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t c4 = static_cast<int64_t>(j) * TPR + t;
        if (c4 < c4n) {
            *reinterpret_cast<f4*>(p + 4 * c4) = dg[j];
            *reinterpret_cast<f4*>(p + a.cols + 4 * c4) = db[j];
        }
    }
}

// Rows of up to 4096 floats whose 16-byte vectors do not line up (a width
// that is not a multiple of 4, or an unaligned pointer), and rows of at most
// 64 floats: ln_bwd_vec's scheme with 4-byte columns c = j*TPR + t, TPR
// threads per row and kBlock/TPR rows per workgroup (one wave per row up to
// 1024 floats: no barrier in the row sums, and four rows' loads in flight
// per workgroup; 16 or 32 lanes per row up to 64 floats, so a wave holds two
// or four rows and sums them with lane-group reductions).  Each row is read
// once; a thread reads dy[c] before it writes dx[c], so dx may alias dy.
template <int TPR, int VPT, bool KEEP>
__global__ __launch_bounds__(kBlock) void ln_bwd_scalar(LnBwdArgs a) {
    constexpr int RPB = kBlock / TPR;
    constexpr int NW = TPR / kWave;
    __shared__ float lds[4][kBlock / kWave];
    const int t = threadIdx.x % TPR;
    const int sub = threadIdx.x / TPR;
    const float n = static_cast<float>(a.cols);
    const float invF = 1.0f / n;  // Model.cpp:7799
    float gm[VPT], dg[VPT], db[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t c = static_cast<int64_t>(j) * TPR + t;
        gm[j] = (a.g && c < a.cols) ? a.g[c] : 1.0f;
        dg[j] = 0.0f;
        db[j] = 0.0f;
    }
    const int64_t step = static_cast<int64_t>(gridDim.x) * RPB;
    // Row group `b`'s x and dy for this thread (zeros past the end).
    auto load_rows = [&](int64_t b, float* xo, float* go) {
        const int64_t r = b + sub;
        const int64_t l = r < a.rows ? a.cols : 0;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int64_t c = static_cast<int64_t>(j) * TPR + t;
            const bool ok = c < l;
            xo[j] = ok ? __builtin_nontemporal_load(a.x + r * a.cols + c) : 0.0f;
            go[j] = ok ? __builtin_nontemporal_load(a.dy + r * a.cols + c) : 0.0f;
        }
    };
    float xv[VPT], gv[VPT];
    load_rows(static_cast<int64_t>(blockIdx.x) * RPB, xv, gv);
    for (int64_t base = static_cast<int64_t>(blockIdx.x) * RPB; base < a.rows; base += step) {
        const int64_t row = base + sub;
        const int64_t lim = row < a.rows ? a.cols : 0;  // past-end rows join the barriers only
        const int64_t off = row * a.cols;
        float xn[VPT], gn[VPT];
        load_rows(base + step, xn, gn);  // the next group's loads in flight during the reductions
        float s = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            s += xv[j];
            s1 += gv[j] * gm[j];
        }
        if constexpr (TPR < kWave) {
            s = group_sum<TPR>(s);
            s1 = group_sum<TPR>(s1);
        } else {
            row_sum2<NW>(s, s1, lds[0], lds[1], sub);
        }
        const float mean = s / n;  // :7765-7768
        float q = 0.0f, p2 = 0.0f;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            if (static_cast<int64_t>(j) * TPR + t < lim) {
                const float d = xv[j] - mean;
                q += d * d;
                p2 += gv[j] * gm[j] * d;
            }
        }
        if constexpr (TPR < kWave) {
            q = group_sum<TPR>(q);
            p2 = group_sum<TPR>(p2);
        } else {
            row_sum2<NW>(q, p2, lds[2], lds[3], sub);
        }
        const float var = q / n;                          // :7770-7776
        const float inv_std = 1.0f / sqrtf(var + a.eps);  // :7777
        const float s2 = p2 * inv_std;
        const float k = inv_std * invF;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {  // :7783-7805
            const int64_t c = static_cast<int64_t>(j) * TPR + t;
            if (c < lim) {
                const float xh = (xv[j] - mean) * inv_std;
                const float dxh = gv[j] * gm[j];
                dg[j] += gv[j] * xh;
                db[j] += gv[j];
                float o = k * ((n * dxh - s1) - xh * s2);
                if (a.acc) o = a.dx[off + c] + o;
                if constexpr (KEEP) a.dx[off + c] = o;
                else st_stream(a.dx + off + c, o);
            }
        }
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            xv[j] = xn[j];
            gv[j] = gn[j];
        }
    }
    if (!a.part) return;
    // One slot per workgroup: the sub-rows' sums are added in sub-row order
    // through LDS, then written once.
    float* p = a.part + static_cast<int64_t>(blockIdx.x) * 2 * a.cols;
    if constexpr (RPB > 1) {
        __shared__ float comb[2 * TPR * VPT];
        for (int r = 0; r < RPB; ++r) {
            if (sub == r) {
#pragma unroll
                for (int j = 0; j < VPT; ++j) {
                    const int i = j * TPR + t;
                    comb[i] = r == 0 ? dg[j] : comb[i] + dg[j];
                    comb[TPR * VPT + i] = r == 0 ? db[j] : comb[TPR * VPT + i] + db[j];
                }
            }
            __syncthreads();
        }
        if (sub != 0) return;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            dg[j] = comb[j * TPR + t];
            db[j] = comb[TPR * VPT + j * TPR + t];
        }
    }
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t c = static_cast<int64_t>(j) * TPR + t;
        if (c < a.cols) {
            p[c] = dg[j];
            p[a.cols + c] = db[j];
        }
    }
}

// Any width / alignment: one workgroup per row, strided passes (the re-reads
// of a row hit L2).  Three kernels, so that dx may overwrite dy: the row
// statistics (mean, inv_std) first, then the parameter gradients (which read
// dy), then dx.
__global__ __launch_bounds__(kBlock) void ln_stats_generic(LnBwdArgs a) {
    constexpr int NW = kBlock / kWave;
    __shared__ float lds[2][NW];
    const int64_t row = blockIdx.x;
    const float* x = a.x + row * a.cols;
    const float n = static_cast<float>(a.cols);
    float s = 0.0f;
    for (int64_t c = threadIdx.x; c < a.cols; c += kBlock) s += x[c];
    const float mean = block_sum<NW>(s, lds[0]) / n;
    float q = 0.0f;
    for (int64_t c = threadIdx.x; c < a.cols; c += kBlock) {
        const float d = x[c] - mean;
        q += d * d;
    }
    const float var = block_sum<NW>(q, lds[1]) / n;
    if (threadIdx.x == 0) {
        a.stats[2 * row] = mean;
        a.stats[2 * row + 1] = 1.0f / sqrtf(var + a.eps);
    }
}

__global__ __launch_bounds__(kBlock) void ln_bwd_generic(LnBwdArgs a) {
    constexpr int NW = kBlock / kWave;
    __shared__ float lds[2][NW];
    const int64_t row = blockIdx.x;
    const float* x = a.x + row * a.cols;
    const float* dy = a.dy + row * a.cols;
    float* dx = a.dx + row * a.cols;
    const float n = static_cast<float>(a.cols);
    const float mean = a.stats[2 * row];
    const float inv_std = a.stats[2 * row + 1];
    float s1 = 0.0f, s2 = 0.0f;
    for (int64_t c = threadIdx.x; c < a.cols; c += kBlock) {
        const float xh = (x[c] - mean) * inv_std;
        const float dxh = dy[c] * (a.g ? a.g[c] : 1.0f);
        s1 += dxh;
        s2 += dxh * xh;
    }
    row_sum2<NW>(s1, s2, lds[0], lds[1], 0);
    const float k = inv_std * (1.0f / n);
    // Each thread reads dy[c] before writing dx[c], so dx may alias dy.
    for (int64_t c = threadIdx.x; c < a.cols; c += kBlock) {
        const float xh = (x[c] - mean) * inv_std;
        const float dxh = dy[c] * (a.g ? a.g[c] : 1.0f);
        float o = k * ((n * dxh - s1) - xh * s2);
        if (a.acc) o = dx[c] + o;
        dx[c] = o;
    }
}

// Parameter gradients for the generic path: part[k][c] = sum over the rows r
// of chunk k of dy*xhat, part[k][cols + c] = sum of dy.
__global__ __launch_bounds__(kBlock) void ln_bwd_params_part(LnBwdArgs a, int64_t chunk) {
    const int64_t c = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (c >= a.cols) return;
    const int64_t r0 = static_cast<int64_t>(blockIdx.y) * chunk;
    const int64_t r1 = r0 + chunk < a.rows ? r0 + chunk : a.rows;
    float sg = 0.0f, sb = 0.0f;
    for (int64_t r = r0; r < r1; ++r) {
        const float g = a.dy[r * a.cols + c];
        const float xh = (a.x[r * a.cols + c] - a.stats[2 * r]) * a.stats[2 * r + 1];
        sg += g * xh;
        sb += g;
    }
    float* p = a.part + static_cast<int64_t>(blockIdx.y) * 2 * a.cols;
    p[c] = sg;
    p[a.cols + c] = sb;
}

// The persistent grid of the register-resident kernels: `groups` row groups
// on at most 512 workgroups (or the tuned count), one dgamma | dbeta slot per
// workgroup, then the slots' deterministic sum.  `run(grid, a)` launches the
// kernel with a.part set.
template <class Run>
int ln_bwd_persistent(mimir_ctx* ctx, LnBwdArgs a, int64_t groups, float* dgamma, float* dbeta, const char* name,
                      const ScratchSpan* fixed, Run run) {
    int64_t grid = ctx->tune.lnbwd_grid > 0 ? ctx->tune.lnbwd_grid : 512;
    if (grid > groups) grid = groups;
    const int64_t nslots = grid;
    float* tmp = nullptr;
    if (dgamma) {  // partial slots, then room for the second level of their sum
        void* s = nullptr;
        const size_t bytes = sizeof(float) * static_cast<size_t>((nslots + kGroups) * 2 * a.cols);
        if (int st = get_scratch(ctx, fixed, bytes, &s)) return st;
        a.part = static_cast<float*>(s);
        tmp = a.part + nslots * 2 * a.cols;
    }
    run(static_cast<unsigned>(grid), a);
    if (int st = launched(ctx, name)) return st;
    if (!dgamma) return MIMIR_OK;
    // dbeta null: sum only the dgamma half.
    return launch_sum_slots(ctx, a.part, nslots, 2 * a.cols, dbeta ? 2 * a.cols : a.cols, dgamma, dbeta, a.cols,
                            true, tmp);
}

template <int TPR, int VPT, int BS>
int launch_ln_bwd_vec(mimir_ctx* ctx, LnBwdArgs a, float* dgamma, float* dbeta, const ScratchSpan* fixed) {
    constexpr int RPB = BS / TPR;
    return ln_bwd_persistent(ctx, a, (a.rows + RPB - 1) / RPB, dgamma, dbeta, "ln_bwd_vec", fixed,
                             [ctx](unsigned grid, const LnBwdArgs& la) {
                                 if (ctx->keep_outputs) ln_bwd_vec<TPR, VPT, BS, true><<<grid, BS, 0, ctx->stream>>>(la);
                                 else ln_bwd_vec<TPR, VPT, BS, false><<<grid, BS, 0, ctx->stream>>>(la);
                             });
}

template <int TPR, int VPT>
int launch_ln_bwd_scalar(mimir_ctx* ctx, LnBwdArgs a, float* dgamma, float* dbeta, const ScratchSpan* fixed) {
    constexpr int RPB = kBlock / TPR;
    return ln_bwd_persistent(ctx, a, (a.rows + RPB - 1) / RPB, dgamma, dbeta, "ln_bwd_scalar", fixed,
                             [ctx](unsigned grid, const LnBwdArgs& la) {
                                 if (ctx->keep_outputs)
                                     ln_bwd_scalar<TPR, VPT, true><<<grid, kBlock, 0, ctx->stream>>>(la);
                                 else ln_bwd_scalar<TPR, VPT, false><<<grid, kBlock, 0, ctx->stream>>>(la);
                             });
}

int ln_bwd_generic_run(mimir_ctx* ctx, LnBwdArgs a, float* dgamma, float* dbeta, const ScratchSpan* fixed) {
    if (!dispatch_fits(a.rows, kBlock))
        return fail(ctx, MIMIR_EINVAL, "LayerNorm backward: %lld rows exceed the grid limit", (long long)a.rows);
    const int64_t cblocks = (a.cols + kBlock - 1) / kBlock;
    if (!dispatch_fits(cblocks, kBlock)) return fail(ctx, MIMIR_EINVAL, "LayerNorm backward: row too wide");
    int64_t nchunks = 0, chunk = a.rows;
    if (dgamma) {
        nchunks = (1024 + cblocks - 1) / cblocks;
        if (nchunks > a.rows) nchunks = a.rows;
        if (nchunks > 65535) nchunks = 65535;
        chunk = (a.rows + nchunks - 1) / nchunks;
        nchunks = (a.rows + chunk - 1) / chunk;
    }
    void* s = nullptr;
    const size_t bytes = sizeof(float) * static_cast<size_t>(2 * a.rows + nchunks * 2 * a.cols);
    if (int st = get_scratch(ctx, fixed, bytes, &s)) return st;
    a.stats = static_cast<float*>(s);
    a.part = a.stats + 2 * a.rows;
    const unsigned rows = static_cast<unsigned>(a.rows);
    ln_stats_generic<<<rows, kBlock, 0, ctx->stream>>>(a);
    if (int st = launched(ctx, "ln_stats_generic")) return st;
    if (dgamma) {
        ln_bwd_params_part<<<dim3(static_cast<unsigned>(cblocks), static_cast<unsigned>(nchunks)), kBlock, 0,
                             ctx->stream>>>(a, chunk);
        if (int st = launched(ctx, "ln_bwd_params_part")) return st;
    }
    ln_bwd_generic<<<rows, kBlock, 0, ctx->stream>>>(a);
    if (int st = launched(ctx, "ln_bwd_generic")) return st;
    if (!dgamma) return MIMIR_OK;
    return launch_sum_slots(ctx, a.part, nchunks, 2 * a.cols, dbeta ? 2 * a.cols : a.cols, dgamma, dbeta, a.cols,
                            true);
}

// ---------------------------------------------------------------------------
// Embedding backward (Model.cpp:7429-7461)
// ---------------------------------------------------------------------------

// Sort key of token t: its id, or `vocab` (sorted last, skipped) for the
// padding id and ids outside [0, vocab) (Model.cpp:7454-7455).  The counting
// sort's kernels call it per token; rocPRIM's radix sort reads the keys
// through it (a transform iterator over the token index) and the token
// indices from a counting iterator.  Either way nothing is staged.
template <int MODE>
struct EmbedKey {
    const void* ids;
    int32_t vocab;
    int32_t pad;
    __device__ uint32_t of_id(int32_t id) const {
        const bool use = !(pad >= 0 && id == pad) && id >= 0 && id < vocab;
        return use ? static_cast<uint32_t>(id) : static_cast<uint32_t>(vocab);
    }
    __device__ uint32_t operator()(int64_t t) const { return of_id(load_id<MODE>(ids, t)); }
};

// The end of the run of `id` that starts at sorted position i: each wave
// checks 64 keys per step and takes the first mismatch from a ballot (the
// result is wave-uniform).  Must be reached by all 64 lanes of the wave.
__device__ __forceinline__ int64_t run_end(const uint32_t* keys, int64_t i, int64_t n, uint32_t id) {
    const int lane = threadIdx.x & (kWave - 1);
    int64_t end = i + 1;
    for (;;) {
        const int64_t j = end + lane;
        const bool stop = j >= n || keys[j] != id;
        const unsigned long long m = __ballot(stop);
        if (m) return end + __builtin_ctzll(m);
        end += kWave;
    }
}

// Runs of at least kLongRun tokens (a frequent id) are summed in two levels
// instead of one token after another: the run's positions are cut at the
// multiples of kLongRun, embed_bwd_seg_partial sums each segment's dy rows
// (token order) into a slot of partial rows, all segments at once, and
// embed_bwd_seg_combine adds the run's slots onto the gradient row.  The
// workgroup at a run's first segment also lists the run (id, head, end) for
// the combine, whose grid then covers only the long runs.  The result is
// deterministic; it is the reference's sequential sum regrouped, so it
// agrees with it to the rounding of a float32 sum (the path's tolerance for
// sums), not bit for bit.  Shorter runs stay with embed_bwd_rows_vec, which
// adds in token order (bit-exact).
constexpr int kLongRun = 32;
constexpr int kLongBatch = 16;

// The long runs, appended in no fixed order (each entry's sum is fixed);
// `count` is zeroed before the segment kernels run.
struct LongRunEntry {
    uint32_t id, head, end, pad;
};
struct LongRunList {
    uint32_t* count;
    LongRunEntry* runs;
    uint32_t cap;  // entries: one per kLongRun positions, at least one per long run
};
__device__ __forceinline__ void list_long_run(const LongRunList& list, uint32_t id, int64_t head, int64_t end) {
    const uint32_t j = atomicAdd(list.count, 1u);
    if (j < list.cap) list.runs[j] = LongRunEntry{id, static_cast<uint32_t>(head), static_cast<uint32_t>(end), 0u};
}

__global__ void zero_count_kernel(uint32_t* count) {
    if (threadIdx.x == 0) *count = 0;
}

// The end of the run of `id` in the sorted keys, given a position j inside
// it: the first position after j whose key differs, or n.  Each step the 64
// lanes probe 64 evenly spaced positions of the range still open; since the
// keys are sorted the probes that still hold `id` form a prefix, and the end
// lies after the last of them and no later than the next probe -- log64 of
// the span steps (3 for 32768 keys).  Must be reached by all 64 lanes.
__device__ __forceinline__ int64_t run_end_search(const uint32_t* keys, int64_t j, int64_t n, uint32_t id) {
    const int lane = threadIdx.x & (kWave - 1);
    int64_t lo = j + 1, hi = n;  // keys[lo - 1] == id; the end is in [lo, hi]
    while (lo < hi) {
        const int64_t span = hi - lo;
        const int64_t step = (span + kWave - 1) / kWave;
        const int64_t q = lo + lane * step;
        const unsigned long long m = __ballot(q < hi && keys[q] == id);
        const int64_t cnt = __popcll(m);
        if (cnt == 0) return lo;
        const int64_t next = lo + cnt * step;  // the first probe past the run, or past hi
        lo = lo + (cnt - 1) * step + 1;
        if (next < hi) hi = next;
    }
    return lo;
}

// The long run through sorted position p = m * kLongRun, seen from p: its
// key, whether p is the run's first multiple of kLongRun (`first`), its head
// (valid when `first`) and end.  `is_long` when it has kLongRun tokens or
// more.  One ballot over positions p - kLongRun + 1 .. p finds the head of a
// run that starts there; a run through p - kLongRun as well is long.  A
// run of kLongRun tokens or more through p reaches p - kLongRun / 2 or
// p + kLongRun / 2 (its extents on the two sides of p add up to at least
// kLongRun - 1), so a run that reaches neither is short, known after the
// first round trip.  Must be reached by all 64 lanes of the wave.
struct LongRun {
    uint32_t id;
    bool first;
    bool is_long;
    int64_t head;
    int64_t end;
};
__device__ __forceinline__ LongRun long_run_at(const uint32_t* keys, int64_t p, int64_t n, uint32_t vocab) {
    LongRun r{keys[p], false, false, p, p + 1};
    // Loaded with the key: one round trip.
    const uint32_t before = p >= kLongRun ? keys[p - kLongRun] : ~0u;
    const uint32_t left = p >= kLongRun / 2 ? keys[p - kLongRun / 2] : ~0u;
    const uint32_t right = p + kLongRun / 2 < n ? keys[p + kLongRun / 2] : ~0u;
    if (r.id >= vocab || (left != r.id && right != r.id)) return r;
    r.first = before != r.id;
    const int lane = threadIdx.x & (kWave - 1);
    if (r.first) {
        const int64_t q = p - (kLongRun - 1) + lane;
        const unsigned long long m = __ballot(lane < kLongRun && q >= 0 && keys[q] == r.id);
        r.head = p - (kLongRun - 1) + __builtin_ctzll(m);  // lane kLongRun - 1 (position p) always matches
    }
    r.end = run_end_search(keys, p, n, r.id);
    r.is_long = !r.first || r.end - r.head >= kLongRun;
    return r;
}

// First level: workgroup (m, o) of position p = m * kLongRun in a long run
// sums the dy rows of its segment, positions p .. min(p + kLongRun, end) - 1
// (and head .. p - 1 before them when p is the run's first multiple), in
// token order, into partial slot m, for its o-th block of kSegCols 16-byte
// columns (one per thread).  Each thread requests kSegRows tokens' rows
// before adding the first.
constexpr int kSegCols = 256;
constexpr int kSegRows = 16;
__global__ __launch_bounds__(kSegCols) void embed_bwd_seg_partial(const uint32_t* keys, const uint32_t* toks,
                                                                  int64_t n, uint32_t vocab, const float* dy,
                                                                  float* part, int64_t dim4, LongRunList list) {
    const int64_t m = blockIdx.x;
    const int64_t p = m * kLongRun;
    if (p >= n) return;
    const LongRun r = long_run_at(keys, p, n, vocab);
    if (!r.is_long) return;
    if (r.first && blockIdx.y == 0 && threadIdx.x == 0) list_long_run(list, r.id, r.head, r.end);
    const int64_t c = static_cast<int64_t>(blockIdx.y) * kSegCols + threadIdx.x;
    if (c >= dim4) return;  // after the ballots of long_run_at
    const int64_t s0 = r.first ? r.head : p;
    const int64_t s1 = p + kLongRun < r.end ? p + kLongRun : r.end;
    const f4* src = reinterpret_cast<const f4*>(dy);
    f4 acc;
    bool started = false;
    for (int64_t j = s0; j < s1; j += kSegRows) {
        f4 v[kSegRows];
#pragma unroll
        for (int u = 0; u < kSegRows; ++u)
            if (j + u < s1) v[u] = __builtin_nontemporal_load(src + static_cast<int64_t>(toks[j + u]) * dim4 + c);
        __builtin_amdgcn_sched_barrier(0);  // the batch's loads are all issued before the first add
#pragma unroll
        for (int u = 0; u < kSegRows; ++u) {
            if (j + u < s1) {
                acc = started ? acc + v[u] : v[u];
                started = true;
            }
        }
    }
    reinterpret_cast<f4*>(part)[m * dim4 + c] = acc;
}

// Second level: work item (run, column block) adds the run's partial slots
// onto kCombineCols 16-byte columns of the id's gradient row.  Each of the
// workgroup's kCombineGroups waves sums every kCombineGroups-th slot
// (kLongBatch loads in flight per lane); the first wave adds the groups'
// sums, in group order, onto the gradient.  The grid strides over the
// listed runs' items, so with no long run every workgroup leaves after one
// load.
constexpr int kCombineCols = kWave;
constexpr int kCombineGroups = 4;
constexpr int64_t kCombineGrid = 1024;
__global__ __launch_bounds__(kWave * kCombineGroups) void embed_bwd_seg_combine(const uint32_t* count,
                                                                                 const LongRunEntry* runs,
                                                                                 uint32_t cap, const float* part,
                                                                                 float* grad, int64_t dim4) {
    __shared__ f4 sums[kCombineGroups - 1][kWave];
    const int64_t blocks = (dim4 + kCombineCols - 1) / kCombineCols;
    const int64_t listed = *count < cap ? *count : cap;
    const int64_t items = listed * blocks;
    const int grp = threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    const f4* src = reinterpret_cast<const f4*>(part);
    for (int64_t it = blockIdx.x; it < items; it += gridDim.x) {
        const LongRunEntry e = runs[it / blocks];
        const int64_t c = (it % blocks) * kCombineCols + lane;
        const int64_t m0 = (static_cast<int64_t>(e.head) + kLongRun - 1) / kLongRun;  // the run's first slot
        const int64_t m1 = (static_cast<int64_t>(e.end) - 1) / kLongRun + 1;
        f4* g = reinterpret_cast<f4*>(grad) + static_cast<int64_t>(e.id) * dim4;
        f4 acc = {0.f, 0.f, 0.f, 0.f};
        f4 gv = acc;
        if (c < dim4) {
            if (grp == 0) gv = __builtin_nontemporal_load(g + c);
            bool started = false;
            int64_t j = m0 + grp;
            for (; j + (kLongBatch - 1) * kCombineGroups < m1; j += kLongBatch * kCombineGroups) {
                f4 v[kLongBatch];
#pragma unroll
                for (int u = 0; u < kLongBatch; ++u) v[u] = src[(j + u * kCombineGroups) * dim4 + c];
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int u = 0; u < kLongBatch; ++u) {
                    acc = started ? acc + v[u] : v[u];
                    started = true;
                }
            }
            for (; j < m1; j += kCombineGroups) {
                const f4 v = src[j * dim4 + c];
                acc = started ? acc + v : v;
                started = true;
            }
        }
        if (grp > 0) sums[grp - 1][lane] = acc;
        __syncthreads();
        if (grp == 0 && c < dim4) {
            gv += acc;  // group 0 always holds slot m0
            for (int q = 1; q < kCombineGroups; ++q)
                if (m0 + q < m1) gv += sums[q - 1][lane];
            st_stream(g + c, gv);
        }
        __syncthreads();  // sums is reused by the next item
    }
}

// One workgroup per sorted position.  The first position of each id's run
// of fewer than kLongRun tokens (every run without `long_runs`) adds the
// run's dy rows (token order, the sort is stable) onto the id's gradient row;
// every other position leaves at once.  Each thread owns CPT 16-byte columns
// TPT apart.  The first token's row and the gradient row are requested
// before the run's end is known, so a run of one (the common case) waits for
// two memory round trips; the rest of a run is loaded kRunBatch tokens at a
// time, then added in token order.  Most workgroups leave at once, so the
// kernel is kept small in registers: two 1024-thread workgroups fit a CU.
constexpr int kRunBatch = 4;

// The first token's row and the gradient row, for the CPT columns of this
// thread that start at c0.
template <int TPT, int CPT>
__device__ __forceinline__ void embed_rows_load(const f4* g, const f4* src, uint32_t t0, int64_t c0, int64_t dim4,
                                                f4 (&acc)[CPT], f4 (&v)[CPT]) {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
        const int64_t c = c0 + static_cast<int64_t>(k) * TPT;
        if (c < dim4) {
            acc[k] = __builtin_nontemporal_load(g + c);
            v[k] = __builtin_nontemporal_load(src + static_cast<int64_t>(t0) * dim4 + c);
        }
    }
}

// The run at sorted positions i .. end - 1 (first token t0, its row and the
// gradient row already loaded for columns from threadIdx.x): adds the rows
// in token order onto the gradient row, column group by column group.
template <int TPT, int CPT>
__device__ __forceinline__ void embed_rows_sum(int64_t i, int64_t end, uint32_t t0, const uint32_t* toks,
                                               const f4* src, f4* g, int64_t dim4, f4 (&acc)[CPT], f4 (&v)[CPT]) {
    int64_t c0 = threadIdx.x;
    while (c0 < dim4) {
#pragma unroll
        for (int k = 0; k < CPT; ++k) acc[k] += v[k];
        for (int64_t j = i + 1; j < end; j += kRunBatch) {
            f4 w[kRunBatch][CPT];
#pragma unroll
            for (int u = 0; u < kRunBatch; ++u) {
                if (j + u < end) {
                    const int64_t row = static_cast<int64_t>(toks[j + u]) * dim4;
#pragma unroll
                    for (int k = 0; k < CPT; ++k) {
                        const int64_t c = c0 + static_cast<int64_t>(k) * TPT;
                        if (c < dim4) w[u][k] = __builtin_nontemporal_load(src + row + c);
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);  // the batch's loads are all issued before the first add
#pragma unroll
            for (int u = 0; u < kRunBatch; ++u) {
                if (j + u < end) {
#pragma unroll
                    for (int k = 0; k < CPT; ++k) acc[k] += w[u][k];
                }
            }
        }
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            const int64_t c = c0 + static_cast<int64_t>(k) * TPT;
            if (c < dim4) st_stream(g + c, acc[k]);
        }
        c0 += static_cast<int64_t>(TPT) * CPT;
        if (c0 < dim4) embed_rows_load<TPT, CPT>(g, src, t0, c0, dim4, acc, v);
    }
}

template <int TPT, int CPT>
__device__ __forceinline__ void embed_rows_position(int64_t i, const uint32_t* keys, const uint32_t* toks, int64_t n,
                                                    uint32_t vocab, const float* dy, float* grad, int64_t dim4,
                                                    int long_runs) {
    const uint32_t id = keys[i];
    const uint32_t t0 = toks[i];
    if (id >= vocab || (i > 0 && keys[i - 1] == id)) return;  // not a run's head
    const f4* src = reinterpret_cast<const f4*>(dy);
    f4* g = reinterpret_cast<f4*>(grad) + static_cast<int64_t>(id) * dim4;
    f4 acc[CPT], v[CPT];
    embed_rows_load<TPT, CPT>(g, src, t0, threadIdx.x, dim4, acc, v);
    if (long_runs && i + kLongRun <= n && keys[i + kLongRun - 1] == id) return;  // a long run: segments
    // Every lane of the wave takes part in the ballots of run_end.
    const int64_t end = run_end(keys, i, n, id);
    embed_rows_sum<TPT, CPT>(i, end, t0, toks, src, g, dim4, acc, v);
}

// The runs of the counting sort, in ascending id order: (id, first sorted
// position, token count, first token), and how many there are.
struct RunEntry {
    uint32_t id, start, count, tok;
};
struct RunList {
    const uint32_t* count;
    const RunEntry* runs;
};

// Run j of the list (no workgroup when j is past the list's end), the same
// sums as embed_rows_position at the run's head.
template <int TPT, int CPT>
__device__ __forceinline__ void embed_rows_run(int64_t j, const RunList& list, const uint32_t* toks,
                                               const float* dy, float* grad, int64_t dim4, int long_runs) {
    if (j >= *list.count) return;
    const RunEntry e = list.runs[j];
    if (long_runs && e.count >= static_cast<uint32_t>(kLongRun)) return;  // a long run: segments
    const f4* src = reinterpret_cast<const f4*>(dy);
    f4* g = reinterpret_cast<f4*>(grad) + static_cast<int64_t>(e.id) * dim4;
    f4 acc[CPT], v[CPT];
    embed_rows_load<TPT, CPT>(g, src, e.tok, threadIdx.x, dim4, acc, v);
    embed_rows_sum<TPT, CPT>(e.start, static_cast<int64_t>(e.start) + e.count, e.tok, toks, src, g, dim4, acc, v);
}

// RUNS: workgroup j takes run j of the counting sort's list; otherwise
// workgroup i takes sorted position i.  Separate instantiations, so each
// form is compiled on its own.
template <int TPT, int CPT, bool RUNS>
__global__ __launch_bounds__(TPT) void embed_bwd_rows_vec(const uint32_t* keys, const uint32_t* toks, int64_t n,
                                                          uint32_t vocab, const float* dy, float* grad, int64_t dim4,
                                                          int long_runs, RunList runs) {
    if constexpr (RUNS)
        embed_rows_run<TPT, CPT>(blockIdx.x, runs, toks, dy, grad, dim4, long_runs);
    else
        embed_rows_position<TPT, CPT>(blockIdx.x, keys, toks, n, vocab, dy, grad, dim4, long_runs);
}

// The rows kernel and the long runs' first level in one launch, so the two
// independent streams overlap: blocks [0, nslots) are the segments of
// embed_bwd_seg_partial (dispatched first, so the long segments start before
// the short rows), the blocks after them embed_bwd_rows_vec's (one per
// listed run with RUNS, else one per sorted position), the segment blocks
// each 1024 threads summing their segment's rows over whole 16-byte
// columns with kMergedSegRows tokens' loads in flight.  The segment path is
// kept small enough that the kernel stays at 64 registers, so two
// 1024-thread workgroups still fit a CU (the rows path's turnover needs
// them); its sums are embed_bwd_seg_partial's, in the same token order, bit
// for bit.
constexpr int kMergedSegRows = 8;
template <bool RUNS>
__global__ __launch_bounds__(1024, 8) void embed_bwd_rows_seg(const uint32_t* keys, const uint32_t* toks, int64_t n,
                                                               uint32_t vocab, const float* dy, float* grad,
                                                               float* part, int64_t dim4, LongRunList list,
                                                               RunList runs) {
    const int64_t nslots = (n + kLongRun - 1) / kLongRun;
    if (blockIdx.x >= nslots) {
        if constexpr (RUNS)
            embed_rows_run<1024, 1>(blockIdx.x - nslots, runs, toks, dy, grad, dim4, 1);
        else
            embed_rows_position<1024, 1>(blockIdx.x - nslots, keys, toks, n, vocab, dy, grad, dim4, 1);
        return;
    }
    const int64_t m = blockIdx.x;
    const int64_t p = m * kLongRun;
    if (p >= n) return;
    const LongRun r = long_run_at(keys, p, n, vocab);
    if (!r.is_long) return;
    if (r.first && threadIdx.x == 0) list_long_run(list, r.id, r.head, r.end);
    const int64_t s0 = r.first ? r.head : p;
    const int64_t s1 = p + kLongRun < r.end ? p + kLongRun : r.end;
    const f4* src = reinterpret_cast<const f4*>(dy);
    for (int64_t c = threadIdx.x; c < dim4; c += 1024) {
        f4 acc;
        bool started = false;
        for (int64_t j = s0; j < s1; j += kMergedSegRows) {
            f4 v[kMergedSegRows];
#pragma unroll
            for (int u = 0; u < kMergedSegRows; ++u)
                if (j + u < s1) v[u] = __builtin_nontemporal_load(src + static_cast<int64_t>(toks[j + u]) * dim4 + c);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < kMergedSegRows; ++u) {
                if (j + u < s1) {
                    acc = started ? acc + v[u] : v[u];
                    started = true;
                }
            }
        }
        reinterpret_cast<f4*>(part)[m * dim4 + c] = acc;
    }
}

__global__ __launch_bounds__(kBlock) void embed_bwd_rows_scalar(const uint32_t* keys, const uint32_t* toks,
                                                                int64_t n, uint32_t vocab, const float* dy,
                                                                float* grad, int64_t dim) {
    const int64_t i = blockIdx.x;
    const uint32_t id = keys[i];
    if (id >= vocab || (i > 0 && keys[i - 1] == id)) return;
    const int64_t end = run_end(keys, i, n, id);
    float* g = grad + static_cast<int64_t>(id) * dim;
    for (int64_t c = threadIdx.x; c < dim; c += kBlock) {
        float acc = g[c];
        for (int64_t j = i; j < end; ++j) acc += dy[static_cast<int64_t>(toks[j]) * dim + c];
        g[c] = acc;
    }
}

size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

// ---- The (id, token) sort as a counting sort ------------------------------
// Tokens are cut into blocks of kSortBlock.  A token's sorted position is
//   (tokens with a smaller key) + (tokens of earlier blocks with its key)
//   + (tokens earlier in its own block with its key),
// which is exactly the stable sort's order, so the result equals the radix
// sort's bit for bit.  Three launches:
//   embed_sort_count    per block: a stable sort of its keys in LDS gives
//                       each token's rank among its block's tokens of the
//                       same key, and the block's row of per-key counts
//                       (16-bit, every row zeroed by its block first)
//   embed_sort_offsets  per key: the counts over the blocks turned into each
//                       block's start (the key's offset within its chunk of
//                       kSortChunk keys plus the earlier blocks' counts),
//                       and each chunk's total
//   embed_sort_scatter  per token: the chunk prefix (scanned in LDS) + its
//                       block's start for its key + its rank
// Used up to kSortMaxBlocks blocks and kSortMaxTable count entries; above
// that the rocPRIM radix sort below.
constexpr int kSortBlock = 1024;
constexpr int64_t kSortMaxBlocks = 64;
constexpr int64_t kSortMaxTable = int64_t(1) << 24;
constexpr int kSortChunk = 256;  // keys per workgroup of embed_sort_offsets
constexpr int64_t kSortMaxKeys = int64_t(kSortBlock) * kSortChunk;  // chunk totals scanned by one workgroup

// The run list's per-key arrays (null `idx`: no list): each key's index among
// the keys with tokens within its chunk, its token count, and each chunk's
// number of such keys.
struct RunScan {
    uint32_t* idx;
    uint32_t* tot;
    uint32_t* chunk;
};

template <int MODE>
__global__ __launch_bounds__(kSortBlock) void embed_sort_count(const void* ids, int64_t n, int32_t vocab, int32_t pad,
                                                               uint32_t end_bit, uint16_t* cnt, int64_t pitch,
                                                               uint16_t* rank, uint32_t* zero) {
    using Sort = rocprim::block_radix_sort<uint32_t, kSortBlock, 1, uint32_t>;
    using Scan = rocprim::block_scan<uint32_t, kSortBlock>;
    __shared__ union {
        typename Sort::storage_type sort;
        typename Scan::storage_type scan;
    } st;
    __shared__ uint32_t sk[kSortBlock];
    const int64_t b = blockIdx.x;
    const int i = threadIdx.x;
    // This block's row of counts: zeroed here, the runs' counts stored after
    // the barriers below.
    uint4* row = reinterpret_cast<uint4*>(cnt + b * pitch);
    for (int64_t c = i; c < pitch / 8; c += kSortBlock) row[c] = uint4{0, 0, 0, 0};
    if (zero && b == 0 && i == 0) *zero = 0;  // a counter of the kernels after the sort
    const uint32_t v1 = static_cast<uint32_t>(vocab) + 1;  // keys 0 .. vocab; v1 pads the last block
    const int64_t t = b * kSortBlock + i;
    uint32_t key[1] = {v1};
    uint32_t idx[1] = {static_cast<uint32_t>(i)};
    if (t < n) key[0] = EmbedKey<MODE>{ids, vocab, pad}(t);
    Sort().sort(key, idx, st.sort, 0u, end_bit);  // LSD radix sort: stable, equal keys keep token order
    const uint32_t k = key[0];
    sk[i] = k;
    __syncthreads();  // sk complete; the sort's storage free for the scan
    const bool head = i == 0 || sk[i - 1] != k;
    const bool tail = i == kSortBlock - 1 || sk[i + 1] != k;
    uint32_t start = 0;
    Scan().inclusive_scan(head ? static_cast<uint32_t>(i) : 0u, start, st.scan, rocprim::maximum<uint32_t>());
    if (k >= v1) return;
    rank[b * kSortBlock + idx[0]] = static_cast<uint16_t>(i - start);
    if (tail) cnt[b * pitch + k] = static_cast<uint16_t>(i - start + 1);
}

__global__ __launch_bounds__(kSortChunk) void embed_sort_offsets(const uint16_t* cnt, int64_t nb, int64_t v1,
                                                                 int64_t pitch, uint32_t* start, uint32_t* chunk,
                                                                 RunScan rs) {
    using Scan = rocprim::block_scan<uint32_t, kSortChunk>;
    __shared__ typename Scan::storage_type st;
    const int64_t k = static_cast<int64_t>(blockIdx.x) * kSortChunk + threadIdx.x;
    uint32_t tot = 0;
    if (k < v1) {
        int64_t b = 0;
        for (; b + 8 <= nb; b += 8) {
            uint32_t v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = cnt[(b + u) * pitch + k];
#pragma unroll
            for (int u = 0; u < 8; ++u) tot += v[u];
        }
        for (; b < nb; ++b) tot += cnt[b * pitch + k];
    }
    uint32_t run = 0, total = 0;
    Scan().exclusive_scan(tot, run, 0u, total, st, rocprim::plus<uint32_t>());
    if (threadIdx.x == 0) chunk[blockIdx.x] = total;
    if (rs.idx) {  // the run list: keys below v1 - 1 (the skipped key) with tokens, numbered in key order
        __syncthreads();  // the scan's storage is reused
        uint32_t idx = 0, runs = 0;
        Scan().exclusive_scan(k < v1 - 1 && tot > 0 ? 1u : 0u, idx, 0u, runs, st, rocprim::plus<uint32_t>());
        if (threadIdx.x == 0) rs.chunk[blockIdx.x] = runs;
        if (k < v1) {
            rs.idx[k] = idx;
            rs.tot[k] = tot;
        }
    }
    if (k >= v1) return;
    int64_t b = 0;  // the counts again, from L2
    for (; b + 8 <= nb; b += 8) {
        uint32_t v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = cnt[(b + u) * pitch + k];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            start[(b + u) * pitch + k] = run;
            run += v[u];
        }
    }
    for (; b < nb; ++b) {
        start[b * pitch + k] = run;
        run += cnt[b * pitch + k];
    }
}

template <int MODE>
__global__ __launch_bounds__(kSortBlock) void embed_sort_scatter(const void* ids, int64_t n, int32_t vocab,
                                                                 int32_t pad, const uint32_t* start, int64_t pitch,
                                                                 const uint16_t* rank, const uint32_t* chunk,
                                                                 int64_t nchunks, uint32_t* skeys, uint32_t* stoks,
                                                                 RunScan rs, uint32_t* nruns, RunEntry* runs) {
    using Scan = rocprim::block_scan<uint32_t, kSortBlock>;
    __shared__ typename Scan::storage_type st;
    __shared__ uint32_t cpre[kSortBlock];
    __shared__ uint32_t rpre[kSortBlock];
    const int64_t b = blockIdx.x;
    const int64_t t = b * kSortBlock + threadIdx.x;
    const uint32_t c = threadIdx.x < nchunks ? chunk[threadIdx.x] : 0u;
    const uint32_t rc = rs.idx && threadIdx.x < nchunks ? rs.chunk[threadIdx.x] : 0u;
    const uint32_t k = t < n ? EmbedKey<MODE>{ids, vocab, pad}(t) : 0u;  // loaded beside the chunk totals
    uint32_t cp = 0;
    Scan().exclusive_scan(c, cp, 0u, st, rocprim::plus<uint32_t>());
    cpre[threadIdx.x] = cp;
    if (rs.idx) {
        __syncthreads();  // the scan's storage is reused
        uint32_t rp = 0, total = 0;
        Scan().exclusive_scan(rc, rp, 0u, total, st, rocprim::plus<uint32_t>());
        rpre[threadIdx.x] = rp;
        if (b == 0 && threadIdx.x == 0) *nruns = total;
    }
    __syncthreads();
    if (t >= n) return;
    const uint32_t s = start[b * pitch + k];
    const uint32_t r = rank[t];
    // The run list's fields for the key, loaded with the rest (one round trip).
    const uint32_t s0 = rs.idx ? start[k] : 0u;
    const uint32_t idx = rs.idx ? rs.idx[k] : 0u;
    const uint32_t tot = rs.idx ? rs.tot[k] : 0u;
    const uint32_t pos = cpre[k / kSortChunk] + s + r;
    if (pos >= n) return;  // cannot happen when the counts are consistent; keeps a fault out regardless
    skeys[pos] = k;
    stoks[pos] = static_cast<uint32_t>(t);
    // The run's first token (no earlier block holds its key, rank 0) lists it.
    if (rs.idx && k < static_cast<uint32_t>(vocab) && r == 0 && s == s0) {
        const uint32_t j = rpre[k / kSortChunk] + idx;
        if (j < n) runs[j] = RunEntry{k, pos, tot, static_cast<uint32_t>(t)};
    }
}

// ---- The same sort in one launch, for tables of at most kOnePassKeys keys --
// Workgroup b (kSortBlock tokens, as above) needs, for each of its tokens,
// the number of tokens with a smaller key and the number of earlier blocks'
// tokens with its key.  Instead of a counts table in HBM and two more
// launches, every workgroup counts all n keys into a histogram in LDS
// itself: the tokens before its block first (the histogram then holds the
// earlier blocks' counts, read off for its own keys), then the rest.  One
// exclusive scan of the histogram, with each key's count packed beside a
// flag for the keys below `vocab` that have tokens, gives both each key's
// first sorted position and its run's number in key order (both below
// 2^16: at most kOnePassBlocks blocks, kOnePassKeys keys).  Positions and
// run list are the three-launch sort's, bit for bit.  The histogram costs
// each workgroup n LDS atomics and a read of the ids (L2 after the first
// touch), issued before the block sort so its latency hides under it; the
// scan takes kOnePassPer keys per thread (odd, so the threads' strided LDS
// reads fall in distinct banks).
constexpr int kOnePassPer = 33;
constexpr int64_t kOnePassKeys = int64_t(kSortBlock) * kOnePassPer;  // 33792 keys: a 132 KiB histogram
constexpr int kOnePassBlocks = 32;  // more tokens per thread spill registers; larger launches take three
constexpr int kOnePassVec = kOnePassBlocks / 4;  // 16-byte vectors of ids per thread
static_assert(kOnePassKeys < 65536 && kOnePassBlocks * kSortBlock < 65536, "keys, counts and positions are held as 16 bits");

// Adds the keys of tokens in [from, to) to the histogram.  kp holds thread
// i's keys of tokens 4 (i + kSortBlock j) + e (e < 4, j < kOnePassVec), two
// 16-bit keys per word; slots past n hold v1 (no token).
__device__ __forceinline__ void count_keys(uint32_t* hist, const uint32_t (&kp)[2 * kOnePassVec], uint32_t v1,
                                           uint32_t from, uint32_t to) {
#pragma unroll
    for (int j = 0; j < kOnePassVec; ++j) {
        const uint32_t u = 4u * (threadIdx.x + static_cast<uint32_t>(kSortBlock) * j);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t k = (kp[2 * j + (e >> 1)] >> (16 * (e & 1))) & 0xffffu;
            if (k < v1 && u + e >= from && u + e < to) atomicAdd(hist + k, 1u);
        }
    }
}

template <int MODE>
__global__ __launch_bounds__(kSortBlock) void embed_sort_onepass(const void* ids, int64_t n64, int32_t vocab,
                                                                 int32_t pad, uint32_t end_bit, uint32_t* skeys,
                                                                 uint32_t* stoks, uint32_t* zero, uint32_t* nruns,
                                                                 RunEntry* runs) {
    using Sort = rocprim::block_radix_sort<uint32_t, kSortBlock, 1, uint32_t>;
    using Scan = rocprim::block_scan<uint32_t, kSortBlock>;
    __shared__ uint32_t hist[kOnePassKeys];
    __shared__ union {
        typename Sort::storage_type sort;
        uint32_t sk[kSortBlock];  // the block's keys in sorted order, after the sort
    } ss;
    __shared__ typename Scan::storage_type scan;
    const uint32_t b = blockIdx.x;
    const uint32_t i = threadIdx.x;
    const uint32_t n = static_cast<uint32_t>(n64);  // at most kOnePassBlocks * kSortBlock
    const uint32_t v1 = static_cast<uint32_t>(vocab) + 1;  // keys 0 .. vocab; v1 marks no token
    const uint32_t b0 = b * kSortBlock;
    const EmbedKey<MODE> kf{ids, vocab, pad};
    const uint32_t* w32 = static_cast<const uint32_t*>(ids);
    if (zero && b == 0 && i == 0) *zero = 0;  // a counter of the kernels after the sort
    // This thread's token first (the sort waits for it alone), then every
    // token's id word, as 16-byte vectors where the ids are aligned.
    const uint32_t own = b0 + i < n ? w32[b0 + i] : 0u;
    const bool vec = (reinterpret_cast<uintptr_t>(ids) & 15u) == 0;
    uint32_t w[kOnePassVec][4];
#pragma unroll
    for (int j = 0; j < kOnePassVec; ++j) {
        const uint32_t u = 4u * (i + static_cast<uint32_t>(kSortBlock) * j);
        if (vec && u + 3 < n) {
            const uint4 q = *reinterpret_cast<const uint4*>(w32 + u);
            w[j][0] = q.x, w[j][1] = q.y, w[j][2] = q.z, w[j][3] = q.w;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) w[j][e] = u + e < n ? w32[u + e] : 0u;
        }
    }
    for (uint32_t j = i; j < v1; j += kSortBlock) hist[j] = 0;  // under the loads
    uint32_t key[1] = {b0 + i < n ? kf.of_id(id_from_word<MODE>(own)) : v1};
    uint32_t idx[1] = {i};
    Sort().sort(key, idx, ss.sort, 0u, end_bit);  // stable: equal keys keep token order
    // Thread i now holds the block's i-th token in key order: its key k, its
    // token b0 + idx, and (below) its rank among the block's tokens of key k.
    const uint32_t k = key[0];
    __syncthreads();  // the sort's storage becomes sk
    ss.sk[i] = k;
    __syncthreads();
    const bool head = i == 0 || ss.sk[i - 1] != k;
    uint32_t first = 0;
    Scan().inclusive_scan(head ? i : 0u, first, scan, rocprim::maximum<uint32_t>());
    const uint32_t rank = i - first;
    uint32_t kp[2 * kOnePassVec];
#pragma unroll
    for (int j = 0; j < kOnePassVec; ++j) {
        const uint32_t u = 4u * (i + static_cast<uint32_t>(kSortBlock) * j);
        uint32_t kk[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) kk[e] = u + e < n ? kf.of_id(id_from_word<MODE>(w[j][e])) : v1;
        kp[2 * j] = kk[0] | kk[1] << 16;
        kp[2 * j + 1] = kk[2] | kk[3] << 16;
    }
    __syncthreads();  // the histogram is zeroed
    count_keys(hist, kp, v1, 0, b0);
    __syncthreads();
    const uint32_t earlier = k < v1 ? hist[k] : 0u;  // tokens of earlier blocks with key k
    __syncthreads();
    count_keys(hist, kp, v1, b0, n);
    __syncthreads();
    // Keys i * kOnePassPer .. + kOnePassPer - 1: (run flag << 16 | count),
    // then, in place, the exclusive prefix of those over the keys.
    uint32_t c[kOnePassPer];
    uint32_t sum = 0;
#pragma unroll
    for (int j = 0; j < kOnePassPer; ++j) {
        const uint32_t kk = i * kOnePassPer + j;
        const uint32_t cnt = kk < v1 ? hist[kk] : 0u;
        c[j] = cnt | (kk < static_cast<uint32_t>(vocab) && cnt > 0 ? 1u << 16 : 0u);
        sum += c[j];
    }
    uint32_t pre = 0, all = 0;
    Scan().exclusive_scan(sum, pre, 0u, all, scan, rocprim::plus<uint32_t>());
#pragma unroll
    for (int j = 0; j < kOnePassPer; ++j) {
        const uint32_t kk = i * kOnePassPer + j;
        if (kk < v1) hist[kk] = pre;
        pre += c[j];
    }
    if (nruns && b == 0 && i == 0) *nruns = all >> 16;
    __syncthreads();
    if (k >= v1) return;  // a padding slot of the last block
    const uint32_t h = hist[k];
    const uint32_t s0 = h & 0xffffu;
    const uint32_t pos = s0 + earlier + rank;
    const uint32_t t = b0 + idx[0];
    if (pos < n) {  // always, when the counts are consistent; kept as a bound regardless
        skeys[pos] = k;
        stoks[pos] = t;
    }
    // The run's first token (no earlier block holds its key, rank 0) lists it.
    if (runs && k < static_cast<uint32_t>(vocab) && earlier == 0 && rank == 0) {
        const uint32_t j = h >> 16;
        if (j < n) runs[j] = RunEntry{k, pos, (hist[k + 1] & 0xffffu) - s0, t};
    }
}

struct CountSortPlan {
    bool ok = false;
    bool runs = false;     // also the run list
    bool onepass = false;  // embed_sort_onepass (no counts table; only the run list in scratch)
    int64_t nb = 0, v1 = 0, pitch = 0, nchunks = 0;
    uint32_t end_bit = 0;
    size_t cnt_bytes = 0, start_bytes = 0, rank_bytes = 0, chunk_bytes = 0;
    size_t key_bytes = 0, list_bytes = 0;  // the run list's per-key arrays (x2), its count and entries
    size_t bytes() const {
        if (onepass) return runs ? list_bytes : 0;
        return cnt_bytes + start_bytes + rank_bytes + chunk_bytes + (runs ? 2 * key_bytes + chunk_bytes + list_bytes : 0);
    }
};

CountSortPlan count_sort_plan(int64_t n, int32_t vocab, bool runs, bool onepass) {
    CountSortPlan p;
    p.nb = (n + kSortBlock - 1) / kSortBlock;
    p.v1 = static_cast<int64_t>(vocab) + 1;
    p.pitch = (p.v1 + 7) / 8 * 8;  // 16-byte rows of counts, zeroed with 16-byte stores
    p.nchunks = (p.v1 + kSortChunk - 1) / kSortChunk;
    uint32_t bits = 1;
    while (bits < 32 && (static_cast<uint64_t>(p.v1) >> bits) != 0) ++bits;  // the padding key v1 included
    p.end_bit = bits;
    p.ok = p.nb <= kSortMaxBlocks && p.nb * p.pitch <= kSortMaxTable && p.v1 <= kSortMaxKeys;
    p.cnt_bytes = align256(sizeof(uint16_t) * static_cast<size_t>(p.nb * p.pitch));
    p.start_bytes = align256(sizeof(uint32_t) * static_cast<size_t>(p.nb * p.pitch));
    p.rank_bytes = align256(sizeof(uint16_t) * static_cast<size_t>(p.nb * kSortBlock));
    p.chunk_bytes = align256(sizeof(uint32_t) * static_cast<size_t>(p.nchunks));
    p.runs = runs;
    p.key_bytes = align256(sizeof(uint32_t) * static_cast<size_t>(p.v1));
    p.list_bytes = 256 + align256(sizeof(RunEntry) * static_cast<size_t>(n));
    p.onepass = onepass && p.ok && p.v1 <= kOnePassKeys && p.nb <= kOnePassBlocks;
    return p;
}

template <int MODE>
int count_sort(mimir_ctx* ctx, const CountSortPlan& p, const void* ids, int64_t n, int32_t vocab, int32_t pad,
               char* temp, uint32_t* skeys, uint32_t* stoks, uint32_t* zero, RunList* list) {
    const unsigned nb = static_cast<unsigned>(p.nb);
    if (p.onepass) {
        uint32_t* nruns = p.runs ? reinterpret_cast<uint32_t*>(temp) : nullptr;
        RunEntry* runs = p.runs ? reinterpret_cast<RunEntry*>(temp + 256) : nullptr;
        if (p.runs) *list = RunList{nruns, runs};
        embed_sort_onepass<MODE><<<nb, kSortBlock, 0, ctx->stream>>>(ids, n, vocab, pad, p.end_bit, skeys, stoks,
                                                                     zero, nruns, runs);
        return launched(ctx, "embed_sort_onepass");
    }
    uint16_t* cnt = reinterpret_cast<uint16_t*>(temp);
    uint32_t* start = reinterpret_cast<uint32_t*>(temp + p.cnt_bytes);
    uint16_t* rank = reinterpret_cast<uint16_t*>(temp + p.cnt_bytes + p.start_bytes);
    uint32_t* chunk = reinterpret_cast<uint32_t*>(temp + p.cnt_bytes + p.start_bytes + p.rank_bytes);
    RunScan rs{nullptr, nullptr, nullptr};
    uint32_t* nruns = nullptr;
    RunEntry* runs = nullptr;
    if (p.runs) {
        char* r = temp + p.cnt_bytes + p.start_bytes + p.rank_bytes + p.chunk_bytes;
        rs.idx = reinterpret_cast<uint32_t*>(r);
        rs.tot = reinterpret_cast<uint32_t*>(r + p.key_bytes);
        rs.chunk = reinterpret_cast<uint32_t*>(r + 2 * p.key_bytes);
        nruns = reinterpret_cast<uint32_t*>(r + 2 * p.key_bytes + p.chunk_bytes);
        runs = reinterpret_cast<RunEntry*>(r + 2 * p.key_bytes + p.chunk_bytes + 256);
        *list = RunList{nruns, runs};
    }
    embed_sort_count<MODE><<<nb, kSortBlock, 0, ctx->stream>>>(ids, n, vocab, pad, p.end_bit, cnt, p.pitch, rank,
                                                               zero);
    if (int st = launched(ctx, "embed_sort_count")) return st;
    embed_sort_offsets<<<static_cast<unsigned>(p.nchunks), kSortChunk, 0, ctx->stream>>>(cnt, p.nb, p.v1, p.pitch,
                                                                                       start, chunk, rs);
    if (int st = launched(ctx, "embed_sort_offsets")) return st;
    embed_sort_scatter<MODE><<<nb, kSortBlock, 0, ctx->stream>>>(ids, n, vocab, pad, start, p.pitch, rank, chunk,
                                                                 p.nchunks, skeys, stoks, rs, nruns, runs);
    return launched(ctx, "embed_sort_scatter");
}

// The (id, token) sort past the counting sort's limits (more than 64 blocks
// of tokens or too large a count table): rocPRIM's.  Below its merge-sort
// limit (2^20 pairs) its device radix sort is a block sort followed by merge
// passes; 8192-pair blocks (512 threads x 16) need two passes at 32768
// tokens.  Measured on
// MI355X at configs[3] (32768 pairs, 15-bit keys): 28.4 us, against 33.2 us
// for the default 1024-pair blocks (five passes), 40 us for 16384-pair
// blocks and 60 us for onesweep.
using EmbedSortConfig = rocprim::radix_sort_config<rocprim::default_config, rocprim::merge_sort_config<512, 512, 16>>;

template <int MODE>
int embed_bwd(mimir_ctx* ctx, const void* ids, int64_t n_ids, const float* dy, float* grad, int64_t table_len,
              int32_t vocab, int32_t dim, int32_t pad) {
    MIMIR_REQUIRE(ctx, n_ids >= 0, "Embedding backward: n_ids < 0");
    vocab = vocab < 1 ? 1 : vocab;  // Model.cpp:7434-7435
    dim = dim < 1 ? 1 : dim;
    MIMIR_REQUIRE(ctx, table_len >= static_cast<int64_t>(vocab) * dim,  // :7443-7447
                  "Embedding backward: invalid weight size (%lld < %d x %d)", (long long)table_len, vocab, dim);
    MIMIR_REQUIRE(ctx, vocab < 0x7fffffff, "Embedding backward: vocab too large");
    if (n_ids == 0) return MIMIR_OK;
    MIMIR_REQUIRE(ctx, ids && dy && grad, "Embedding backward: null tensor");
    MIMIR_REQUIRE(ctx, n_ids <= 0x7fffffffLL, "Embedding backward: %lld ids exceed the grid limit",
                  (long long)n_ids);
    MIMIR_ENTER(ctx);
    const unsigned n = static_cast<unsigned>(n_ids);
    unsigned end_bit = 1;
    while (end_bit < 32 && (static_cast<uint32_t>(vocab) >> end_bit) != 0) ++end_bit;
    const auto keys = rocprim::make_transform_iterator(rocprim::counting_iterator<int64_t>(0),
                                                       EmbedKey<MODE>{ids, vocab, pad});
    const rocprim::counting_iterator<uint32_t> toks(0);
    const CountSortPlan plan =
        count_sort_plan(n_ids, vocab, ctx->tune.embed_bwd_runs != 0, ctx->tune.embed_bwd_onepass != 0);
    const bool counting = plan.ok && ctx->tune.embed_bwd_sort != 0;
    size_t sort_bytes = 0;
    hipError_t e = hipSuccess;
    if (counting) {
        sort_bytes = plan.bytes();
    } else {
        e = rocprim::radix_sort_pairs<EmbedSortConfig>(nullptr, sort_bytes, keys, static_cast<uint32_t*>(nullptr),
                                                       toks, static_cast<uint32_t*>(nullptr), n, 0u, end_bit,
                                                       ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "radix_sort_pairs (size)");
    }
    const size_t vbytes = align256(sizeof(uint32_t) * n);
    const bool vec = (dim % 4) == 0 && aligned16(dy) && aligned16(grad);
    if (!vec && !dispatch_fits(n_ids, kBlock))  // the scalar rows kernel: a workgroup per sorted position
        return fail(ctx, MIMIR_EINVAL, "Embedding backward: %lld ids of %d-float rows exceed the grid limit",
                    (long long)n_ids, dim);
    const bool long_runs = vec && n_ids >= kLongRun;
    // Partial rows of the long runs' segments: one slot per kLongRun positions.
    const int64_t nslots = (n_ids + kLongRun - 1) / kLongRun;
    const size_t part_bytes = long_runs ? align256(sizeof(float) * static_cast<size_t>(nslots) * dim) : 0;
    // The long-run list: its count, then at most one entry per slot.
    const size_t list_bytes = long_runs ? 256 + align256(sizeof(LongRunEntry) * static_cast<size_t>(nslots)) : 0;
    void* s = nullptr;
    if (int st = ensure_scratch(ctx, 2 * vbytes + part_bytes + list_bytes + align256(sort_bytes), &s)) return st;
    char* base = static_cast<char*>(s);
    uint32_t* skeys = reinterpret_cast<uint32_t*>(base);
    uint32_t* stoks = reinterpret_cast<uint32_t*>(base + vbytes);
    float* part = reinterpret_cast<float*>(base + 2 * vbytes);
    LongRunList list{nullptr, nullptr, 0u};
    if (long_runs) {
        list.count = reinterpret_cast<uint32_t*>(base + 2 * vbytes + part_bytes);
        list.runs = reinterpret_cast<LongRunEntry*>(base + 2 * vbytes + part_bytes + 256);
        list.cap = static_cast<uint32_t>(nslots);
    }
    char* temp = base + 2 * vbytes + part_bytes + list_bytes;
    RunList runs{nullptr, nullptr};  // with the counting sort, its runs in id order (unless MIMIR_TUNE embruns=0)
    if (counting) {  // embed_sort_count zeroes the list's count
        if (int st = count_sort<MODE>(ctx, plan, ids, n_ids, vocab, pad, temp, skeys, stoks, list.count, &runs))
            return st;
    } else {
        e = rocprim::radix_sort_pairs<EmbedSortConfig>(temp, sort_bytes, keys, skeys, toks, stoks, n, 0u, end_bit,
                                                       ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "radix_sort_pairs");
        if (long_runs) {
            zero_count_kernel<<<1, kWave, 0, ctx->stream>>>(list.count);
            if (int st = launched(ctx, "zero_count_kernel")) return st;
        }
    }
    if (vec) {
        const uint32_t v = static_cast<uint32_t>(vocab);
        const int64_t dim4 = dim / 4;
        const int lr = long_runs ? 1 : 0;
        // Measured on MI355X at dim 4096 (MIMIR_TUNE gather=256/512/1024 picks a
        // variant): one 16-byte column per thread in 1024-thread workgroups
        // is fastest, 2-4 columns per thread in smaller ones ~2-4% slower.
        const int tpt = ctx->tune.gather_tpt ? ctx->tune.gather_tpt : (dim4 >= 1024 ? 1024 : dim4 >= 512 ? 512 : 256);
        // With the run list, a workgroup per run: at most min(n, vocab) of them.
        const int64_t rows_grid = runs.count && vocab < n_ids ? vocab : n_ids;
        const bool merged = long_runs && tpt == 1024 && dispatch_fits(rows_grid + nslots, 1024) &&
                            ctx->tune.embed_bwd_merged != 0;
        if (!dispatch_fits(rows_grid, tpt))
            return fail(ctx, MIMIR_EINVAL, "Embedding backward: %lld rows of %d threads exceed the grid limit",
                        (long long)rows_grid, tpt);
        const unsigned rg = static_cast<unsigned>(rows_grid);
        const bool by_run = runs.count != nullptr;
        if (merged) {
            const unsigned grid = static_cast<unsigned>(rows_grid + nslots);
            if (by_run)
                embed_bwd_rows_seg<true><<<grid, 1024, 0, ctx->stream>>>(skeys, stoks, n_ids, v, dy, grad, part, dim4,
                                                                        list, runs);
            else
                embed_bwd_rows_seg<false><<<grid, 1024, 0, ctx->stream>>>(skeys, stoks, n_ids, v, dy, grad, part,
                                                                         dim4, list, runs);
            if (int st = launched(ctx, "embed_bwd_rows_seg")) return st;
        } else {
            if (long_runs) {
                const dim3 pgrid(static_cast<unsigned>(nslots),
                                 static_cast<unsigned>((dim4 + kSegCols - 1) / kSegCols));
                embed_bwd_seg_partial<<<pgrid, kSegCols, 0, ctx->stream>>>(skeys, stoks, n_ids, v, dy, part, dim4,
                                                                           list);
                if (int st = launched(ctx, "embed_bwd_seg_partial")) return st;
            }
#define MIMIR_EMB_ROWS(T, C)                                                                                  \
    do {                                                                                                      \
        if (by_run)                                                                                           \
            embed_bwd_rows_vec<T, C, true><<<rg, T, 0, ctx->stream>>>(skeys, stoks, n_ids, v, dy, grad, dim4, lr, \
                                                                      runs);                                  \
        else                                                                                                  \
            embed_bwd_rows_vec<T, C, false><<<rg, T, 0, ctx->stream>>>(skeys, stoks, n_ids, v, dy, grad, dim4,  \
                                                                       lr, runs);                             \
    } while (0)
            if (tpt == 256)
                MIMIR_EMB_ROWS(256, 4);
            else if (tpt == 512)
                MIMIR_EMB_ROWS(512, 2);
            else
                MIMIR_EMB_ROWS(1024, 1);
#undef MIMIR_EMB_ROWS
            if (int st = launched(ctx, "embed_bwd_rows_vec")) return st;
        }
        if (!long_runs) return MIMIR_OK;
        // The long runs' segment partials are complete and listed (stream
        // order): add them.  At most nslots runs of `blocks` items each.
        const int64_t blocks = (dim4 + kCombineCols - 1) / kCombineCols;
        const int64_t items = nslots * blocks;
        const unsigned cgrid = static_cast<unsigned>(items < kCombineGrid ? items : kCombineGrid);
        embed_bwd_seg_combine<<<cgrid, kWave * kCombineGroups, 0, ctx->stream>>>(list.count, list.runs, list.cap,
                                                                                 part, grad, dim4);
        return launched(ctx, "embed_bwd_seg_combine");
    }
    embed_bwd_rows_scalar<<<n, kBlock, 0, ctx->stream>>>(skeys, stoks, n_ids, static_cast<uint32_t>(vocab), dy,
                                                         grad, dim);
    return launched(ctx, "embed_bwd_rows_scalar");
}

// Model.cpp:7719-7821 (the LayerNorm branch of backwardPass): dispatch over
// the kernels by row width and alignment.  Scratch comes from `fixed` when
// given (the no-allocation entry point), else from the context.
int layernorm_bwd(mimir_ctx* ctx, const float* x, const float* dy, const float* gamma, float* dx, float* dgamma,
                  float* dbeta, int64_t groups, int64_t n, float eps, int accumulate, const ScratchSpan* fixed) {
    if (!ctx) return MIMIR_EINVAL;
    MIMIR_REQUIRE(ctx, n > 0 && groups >= 0, "LayerNorm backward: invalid shape (groups=%lld, n=%lld)",
                  (long long)groups, (long long)n);
    MIMIR_REQUIRE(ctx, !(dgamma && !gamma) && !(dbeta && !dgamma),
                  "LayerNorm backward: dgamma needs gamma (affine), dbeta needs dgamma");
    if (groups == 0) return MIMIR_OK;
    MIMIR_REQUIRE(ctx, x && dy && dx, "LayerNorm backward: null tensor");
    MIMIR_ENTER(ctx);
    LnBwdArgs a{x, dy, gamma, dx, nullptr, nullptr, groups, n, eps, accumulate ? 1 : 0};
    const int64_t c4 = n / 4;
    const bool vec = (n % 4) == 0 && aligned16(x) && aligned16(dy) && aligned16(dx) && (!gamma || aligned16(gamma));
    // Rows too wide for one workgroup: chunked over the whole GPU; with more
    // than one group of rows, dgamma / dbeta come from per-group slots.
    if (vec && longrow_applies(groups, n)) {
        float* slots = nullptr;
        float* tmp = nullptr;
        int64_t nslots = 0;
        if (int st = longrow_ln_bwd(ctx, x, dy, gamma, dx, dgamma, dbeta, groups, n, eps, accumulate, &slots,
                                    &nslots, &tmp, fixed))
            return st;
        if (!slots) return MIMIR_OK;
        return launch_sum_slots(ctx, slots, nslots, 2 * n, dbeta ? 2 * n : n, dgamma, dbeta, n, true, tmp);
    }
    // Rows of at most 64 floats: two or four rows per wave (MIMIR_TUNE
    // lnbwd_narrow=0 keeps one row per wave, or per vector row of ln_bwd_vec).
    if (n <= 64 && ctx->tune.lnbwd_narrow != 0 && !(vec && shape_fits(ctx->tune.lnbwd, c4))) {
        if (n <= 16) return launch_ln_bwd_scalar<16, 1>(ctx, a, dgamma, dbeta, fixed);
        if (n <= 32) return launch_ln_bwd_scalar<16, 2>(ctx, a, dgamma, dbeta, fixed);
        return launch_ln_bwd_scalar<32, 2>(ctx, a, dgamma, dbeta, fixed);
    }
    if (vec) {
        const RowShape over = ctx->tune.lnbwd;
        const RowShape s = shape_fits(over, c4) ? over : default_norm_shape(c4);
#define MIMIR_LNBWD_CASE(T, V, B) \
        if (s.tpr == T && s.vpt == V && s.bs == B) return launch_ln_bwd_vec<T, V, B>(ctx, a, dgamma, dbeta, fixed);
        MIMIR_ROW_SHAPES(MIMIR_LNBWD_CASE)
#undef MIMIR_LNBWD_CASE
    }
    if (!vec && n <= 256) return launch_ln_bwd_scalar<64, 4>(ctx, a, dgamma, dbeta, fixed);
    if (!vec && n <= 1024) return launch_ln_bwd_scalar<64, 16>(ctx, a, dgamma, dbeta, fixed);
    if (!vec && n <= 2048) return launch_ln_bwd_scalar<128, 16>(ctx, a, dgamma, dbeta, fixed);
    if (!vec && n <= 4096) return launch_ln_bwd_scalar<256, 16>(ctx, a, dgamma, dbeta, fixed);
    return ln_bwd_generic_run(ctx, a, dgamma, dbeta, fixed);
}

// The no-allocation entry point's scratch: one array per GPU, reserved when
// the code object loads and held until the process ends.  Its name is a
// host-side stand-in in host code; the device address comes from
// hipGetSymbolAddress, once per device (noalloc_scratch_init).  The LayerNorm
// backward writes every slot it later reads, so nothing in it has to start
// at zero.  One context per GPU holds it at a time (g_noalloc_owner): its
// calls are ordered on its stream, and another context's call is refused,
// so no two calls can overlap on it.
constexpr size_t kNoAllocScratchBytes = size_t(32) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mutex;
void* g_noalloc_ptr[kMaxDevices] = {};
const mimir_ctx* g_noalloc_owner[kMaxDevices] = {};

}  // namespace

// The device address of this GPU's scratch array (ctx->device current).
int mimir::noalloc_scratch_init(mimir_ctx* ctx) {
    if (ctx->device < 0 || ctx->device >= kMaxDevices)
        return fail(ctx, MIMIR_EDEVICE, "device %d: no scratch slot for it", ctx->device);
    std::lock_guard<std::mutex> lock(g_noalloc_mutex);
    if (!g_noalloc_ptr[ctx->device]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) return hip_fail(ctx, e, "hipGetSymbolAddress(scratch)");
        g_noalloc_ptr[ctx->device] = ptr;
    }
    ctx->noalloc_scratch = g_noalloc_ptr[ctx->device];
    return MIMIR_OK;
}

// A context being destroyed (its stream drained) gives the array up.
void mimir::noalloc_scratch_release(mimir_ctx* ctx) {
    if (ctx->device < 0 || ctx->device >= kMaxDevices) return;
    std::lock_guard<std::mutex> lock(g_noalloc_mutex);
    if (g_noalloc_owner[ctx->device] == ctx) g_noalloc_owner[ctx->device] = nullptr;
}

extern "C" {

int mimir_layernorm_bwd(mimir_ctx* ctx, const float* x, const float* dy, const float* gamma, float* dx,
                        float* dgamma, float* dbeta, int64_t groups, int64_t n, float eps, int accumulate) {
    return layernorm_bwd(ctx, x, dy, gamma, dx, dgamma, dbeta, groups, n, eps, accumulate, nullptr);
}

int mimir_layernorm_bwd_noalloc(mimir_ctx* ctx, const float* x, const float* dy, const float* gamma, float* dx,
                                float* dgamma, float* dbeta, int64_t groups, int64_t n, float eps, int accumulate) {
    if (!ctx) return MIMIR_EINVAL;
    if (!ctx->noalloc_scratch)
        return fail(ctx, MIMIR_EDEVICE, "LayerNorm backward (no allocation): the device scratch is not set up");
    {
        std::lock_guard<std::mutex> lock(g_noalloc_mutex);
        const mimir_ctx*& owner = g_noalloc_owner[ctx->device];  // device checked by noalloc_scratch_init
        if (owner && owner != ctx)
            return fail(ctx, MIMIR_EBUSY,
                        "LayerNorm backward (no allocation): GPU %d's scratch array is held by another context "
                        "until it is destroyed",
                        ctx->device);
        owner = ctx;
    }
    const ScratchSpan fixed{ctx->noalloc_scratch, kNoAllocScratchBytes};
    return layernorm_bwd(ctx, x, dy, gamma, dx, dgamma, dbeta, groups, n, eps, accumulate, &fixed);
}

int mimir_gelu_bwd(mimir_ctx* ctx, const float* x, const float* dy, float* dx, int64_t n, int accumulate) {
    if (!ctx) return MIMIR_EINVAL;
    MIMIR_REQUIRE(ctx, n >= 0, "GELU backward: n < 0");
    if (n == 0) return MIMIR_OK;
    MIMIR_REQUIRE(ctx, x && dy && dx, "GELU backward: null tensor");
    MIMIR_ENTER(ctx);
    return accumulate ? run_dact<DGelu, true>(ctx, x, dy, dx, n, DGelu{}, "gelu_bwd")
                      : run_dact<DGelu, false>(ctx, x, dy, dx, n, DGelu{}, "gelu_bwd");
}

int mimir_silu_bwd(mimir_ctx* ctx, const float* x, const float* dy, float* dx, int64_t n, int accumulate) {
    if (!ctx) return MIMIR_EINVAL;
    MIMIR_REQUIRE(ctx, n >= 0, "SiLU backward: n < 0");
    if (n == 0) return MIMIR_OK;
    MIMIR_REQUIRE(ctx, x && dy && dx, "SiLU backward: null tensor");
    MIMIR_ENTER(ctx);
    return accumulate ? run_dact<DSilu, true>(ctx, x, dy, dx, n, DSilu{}, "silu_bwd")
                      : run_dact<DSilu, false>(ctx, x, dy, dx, n, DSilu{}, "silu_bwd");
}

int mimir_mul_bwd(mimir_ctx* ctx, const float* a, const float* b, const float* dy, float* da, float* db, int64_t n,
                  int acc_a, int acc_b) {
    if (!ctx) return MIMIR_EINVAL;
    MIMIR_REQUIRE(ctx, n >= 0, "Multiply backward: n < 0");
    if (n == 0 || (!da && !db)) return MIMIR_OK;
    MIMIR_REQUIRE(ctx, a && b && dy, "Multiply backward: null tensor");
    MIMIR_ENTER(ctx);
    const bool A = acc_a != 0, B = acc_b != 0;
    if (da && da == db) {
        if (A) mul_bwd_same<true><<<stride_grid(n), kBlock, 0, ctx->stream>>>(a, b, dy, da, n);
        else mul_bwd_same<false><<<stride_grid(n), kBlock, 0, ctx->stream>>>(a, b, dy, da, n);
        return launched(ctx, "mul_bwd_same");
    }
    int64_t done = 0;
    if (aligned16(a) && aligned16(b) && aligned16(dy) && (!da || aligned16(da)) && (!db || aligned16(db))) {
        const int64_t n4 = n / 4;
        if (n4 > 0) {
            const int st = with_block(ew_block(ctx->tune), [&](auto bsc) {
                constexpr int BS = decltype(bsc)::value;
                unsigned blocks;
                if (!grid_for(n4, BS, BS, &blocks))
                    return fail(ctx, MIMIR_EINVAL, "Multiply backward: n=%lld exceeds the grid limit", (long long)n);
                if (ctx->keep_outputs) launch_mul_bwd<true, BS>(ctx, blocks, A, B, a, b, dy, da, db, n4);
                else launch_mul_bwd<false, BS>(ctx, blocks, A, B, a, b, dy, da, db, n4);
                return launched(ctx, "mul_bwd_vec");
            });
            if (st) return st;
        }
        done = n4 * 4;
    }
    if (n > done) {
        const unsigned g = stride_grid(n - done);
        float* da2 = da ? da + done : nullptr;
        float* db2 = db ? db + done : nullptr;
        if (A && B) mul_bwd_scalar<true, true><<<g, kBlock, 0, ctx->stream>>>(a + done, b + done, dy + done, da2, db2, n - done);
        else if (A) mul_bwd_scalar<true, false><<<g, kBlock, 0, ctx->stream>>>(a + done, b + done, dy + done, da2, db2, n - done);
        else if (B) mul_bwd_scalar<false, true><<<g, kBlock, 0, ctx->stream>>>(a + done, b + done, dy + done, da2, db2, n - done);
        else mul_bwd_scalar<false, false><<<g, kBlock, 0, ctx->stream>>>(a + done, b + done, dy + done, da2, db2, n - done);
        return launched(ctx, "mul_bwd_scalar");
    }
    return MIMIR_OK;
}

int mimir_add_bwd(mimir_ctx* ctx, const float* dy, int64_t na, int64_t nb, float* da, float* db, int acc_a,
                  int acc_b) {
    if (!ctx) return MIMIR_EINVAL;
    MIMIR_REQUIRE(ctx, na > 0 && nb > 0, "Add backward: inputs must be non-empty");
    MIMIR_REQUIRE(ctx, dy, "Add backward: null tensor");
    const bool A = acc_a != 0, B = acc_b != 0;
    if (na == nb) {  // Model.cpp:7552-7555: both inputs receive dy, in that order
        if (!da && !db) return MIMIR_OK;
        MIMIR_ENTER(ctx);
        const bool alias = da == dy || db == dy || (da && da == db);
        if (!alias && aligned16(dy) && (!da || aligned16(da)) && (!db || aligned16(db)) && (na % 4) == 0) {
            return with_block(ew_block(ctx->tune), [&](auto bsc) {
                constexpr int BS = decltype(bsc)::value;
                unsigned blocks;
                if (!grid_for(na / 4, BS, BS, &blocks))
                    return fail(ctx, MIMIR_EINVAL, "Add backward: n=%lld exceeds the grid limit", (long long)na);
                if (ctx->keep_outputs) launch_add_bwd<true, BS>(ctx, blocks, A, B, dy, da, db, na / 4);
                else launch_add_bwd<false, BS>(ctx, blocks, A, B, dy, da, db, na / 4);
                return launched(ctx, "add_bwd_vec");
            });
        }
        // Aliased gradients: the second accumulation sees the first, as the
        // reference's in-place adds into its gradient map do.
        if (da)
            if (int st = accumulate(ctx, dy, da, na, A, "add_bwd")) return st;
        if (db)
            if (int st = accumulate(ctx, dy, db, nb, B || db == da, "add_bwd")) return st;
        return MIMIR_OK;
    }
    const bool a_big = na > nb;  // dy has the big operand's size
    const int64_t big_n = a_big ? na : nb, small_n = a_big ? nb : na;
    MIMIR_REQUIRE(ctx, small_n == 1 || big_n % small_n == 0,  // Model.cpp:7595-7599
                  "Add backward: broadcast unsupported (big=%lld, small=%lld)", (long long)big_n, (long long)small_n);
    float* d_big = a_big ? da : db;
    float* d_small = a_big ? db : da;
    MIMIR_ENTER(ctx);
    if (d_small)  // :7577 then :7580-7594, in one pass over dy
        return add_bcast_bwd(ctx, dy, big_n, small_n, d_big, a_big ? A : B, d_small, a_big ? B : A);
    if (d_big) return accumulate(ctx, dy, d_big, big_n, a_big ? A : B, "add_bwd");
    return MIMIR_OK;
}

int mimir_embedding_bwd(mimir_ctx* ctx, const int32_t* ids, int64_t n_ids, const float* dy, float* grad_table,
                        int64_t table_len, int32_t vocab, int32_t dim, int32_t padding_idx) {
    if (!ctx) return MIMIR_EINVAL;
    return embed_bwd<kIdsI32>(ctx, ids, n_ids, dy, grad_table, table_len, vocab, dim, padding_idx);
}

int mimir_embedding_f32ids_bwd(mimir_ctx* ctx, const float* ids, int64_t n_ids, const float* dy, float* grad_table,
                               int64_t table_len, int32_t vocab, int32_t dim, int32_t padding_idx) {
    if (!ctx) return MIMIR_EINVAL;
    return embed_bwd<kIdsF32>(ctx, ids, n_ids, dy, grad_table, table_len, vocab, dim, padding_idx);
}

}  // extern "C"

namespace mimir {

int embedding_bwd_launch(mimir_ctx* ctx, const void* ids, int mode, int64_t n_ids, const float* dy, float* grad,
                         int64_t table_len, int32_t vocab, int32_t dim, int32_t pad) {
    if (mode == kIdsF32) return embed_bwd<kIdsF32>(ctx, ids, n_ids, dy, grad, table_len, vocab, dim, pad);
    if (mode == kIdsI32AsF32) return embed_bwd<kIdsI32AsF32>(ctx, ids, n_ids, dy, grad, table_len, vocab, dim, pad);
    return embed_bwd<kIdsI32>(ctx, ids, n_ids, dy, grad, table_len, vocab, dim, pad);
}

}  // namespace mimir
