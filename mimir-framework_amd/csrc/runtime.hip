// runtime.hip -- context, device memory, copies and timing events of
// libmimir_hip.  Replaces the host storage the reference ops use
// (Model::tensor_store, Model.hpp:608-610; RuntimeAllocator::allocate_tensor,
// RuntimeAllocator.hpp:191-226; MemoryGuard accounting, MemoryGuard.hpp:75-130)
// with device-resident buffers and one HIP stream per context.
#include "common.hpp"
#include "internal.hpp"

#include <new>

using namespace mimir;

namespace {

// Streaming copy: one 16-byte vector per thread for the aligned body (the
// grid covers it in one pass up to 2^30 workgroups), bytes for the rest.
// KEEP: the copy stays in the caches (mimir_ctx_set_output_caching).
template <bool KEEP, int BS = kBlock>
__global__ __launch_bounds__(BS) void copy16_kernel(const u4* __restrict__ src,
                                                     u4* __restrict__ dst, int64_t n16) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * BS;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * BS + threadIdx.x; i < n16; i += stride) {
        const u4 v = __builtin_nontemporal_load(src + i);
        if constexpr (KEEP) dst[i] = v;
        else st_stream(dst + i, v);
    }
}

unsigned full_grid(int64_t n, int bs = kBlock) {
    const int64_t b = (n + bs - 1) / bs;
    return static_cast<unsigned>(b < 1 ? 1 : (b > (int64_t(1) << 30) ? (int64_t(1) << 30) : b));
}

__global__ __launch_bounds__(kBlock) void copy1_kernel(const uint8_t* __restrict__ src,
                                                        uint8_t* __restrict__ dst, int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
        dst[i] = src[i];
}

__global__ __launch_bounds__(kBlock) void fill_kernel(float* __restrict__ dst, int64_t n, float v) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
        dst[i] = v;
}

// Grid for a grid-stride loop over n items: enough blocks to cover every CU
// many times over, capped so the launch stays cheap.
unsigned stride_grid(int64_t n) {
    const int64_t b = (n + kBlock - 1) / kBlock;
    return static_cast<unsigned>(b < 1 ? 1 : (b > 65536 ? 65536 : b));
}

}  // namespace

int mimir::retire_or_free(mimir_ctx* ctx, void* p) {
    if (!p) return MIMIR_OK;
    if (ctx->graph_pins > 0) {
        ctx->retired.push_back(p);
        return MIMIR_OK;
    }
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamSynchronize");
    (void)hipFree(p);
    return MIMIR_OK;
}

void mimir::graph_pin(mimir_ctx* ctx) { ++ctx->graph_pins; }

int mimir::graph_unpin(mimir_ctx* ctx) {
    if (--ctx->graph_pins > 0 || ctx->retired.empty()) return MIMIR_OK;
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamSynchronize");
    for (void* p : ctx->retired) (void)hipFree(p);
    ctx->retired.clear();
    return MIMIR_OK;
}

int mimir::ensure_scratch(mimir_ctx* ctx, size_t bytes, void** out) {
    if (bytes > ctx->scratch_bytes) {
        if (ctx->scratch) {
            if (int st = retire_or_free(ctx, ctx->scratch)) return st;
            ctx->scratch = nullptr;
            ctx->scratch_bytes = 0;
        }
        const size_t want = bytes < (size_t(1) << 20) ? (size_t(1) << 20) : bytes;
        hipError_t e = hipMalloc(&ctx->scratch, want);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            ctx->scratch = nullptr;
            return fail(ctx, MIMIR_ENOMEM, "scratch of %zu bytes: %s", want, hipGetErrorString(e));
        }
        ctx->scratch_bytes = want;
    }
    *out = ctx->scratch;
    return MIMIR_OK;
}

extern "C" {

int mimir_ctx_create(int device, mimir_ctx** out) {
    if (!out) return MIMIR_EINVAL;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) return MIMIR_EDEVICE;
    if (device < 0 || device >= count) return MIMIR_EINVAL;
    if (hipSetDevice(device) != hipSuccess) return MIMIR_EDEVICE;
    mimir_ctx* ctx = new (std::nothrow) mimir_ctx();
    if (!ctx) return MIMIR_ENOMEM;
    ctx->device = device;
    ctx->tune = read_tuning();
    if (hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking) != hipSuccess) {
        delete ctx;
        return MIMIR_EDEVICE;
    }
    ctx->stream = ctx->own_stream;
    int init_st = noalloc_scratch_init(ctx);
    if (init_st == MIMIR_OK) init_st = norm_init(ctx);
    if (int st = init_st) {
        (void)hipStreamDestroy(ctx->own_stream);
        delete ctx;
        return st;
    }
    *out = ctx;
    return MIMIR_OK;
}

int mimir_ctx_destroy(mimir_ctx* ctx) {
    if (!ctx) return MIMIR_EINVAL;
    int st = enter(ctx);
    if (st == MIMIR_OK) {
        (void)hipStreamSynchronize(ctx->stream);
        gemm_release(ctx);
        for (auto& kv : ctx->allocs) (void)hipFree(kv.first);
        if (ctx->scratch) (void)hipFree(ctx->scratch);
        for (void* p : ctx->retired) (void)hipFree(p);
        (void)hipStreamDestroy(ctx->own_stream);
    }
    noalloc_scratch_release(ctx);  // after the stream drained (or could not be entered)
    delete ctx;
    return st;
}

int mimir_ctx_set_stream(mimir_ctx* ctx, void* hip_stream) {
    MIMIR_ENTER(ctx);
    // The context's scratch is reused in the order of its current stream:
    // finish what the old stream may still do with it before switching.
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamSynchronize");
    ctx->stream = hip_stream ? static_cast<hipStream_t>(hip_stream) : ctx->own_stream;
    return MIMIR_OK;
}

void* mimir_ctx_stream(mimir_ctx* ctx) { return ctx ? static_cast<void*>(ctx->stream) : nullptr; }

int mimir_ctx_set_output_caching(mimir_ctx* ctx, int keep) {
    if (!ctx) return MIMIR_EINVAL;
    ctx->keep_outputs = keep ? 1 : 0;
    return MIMIR_OK;
}

int mimir_ctx_set_alloc_limit(mimir_ctx* ctx, size_t bytes) {
    if (!ctx) return MIMIR_EINVAL;
    ctx->alloc_limit = bytes;
    return MIMIR_OK;
}

const char* mimir_last_error(const mimir_ctx* ctx) {
    return ctx ? ctx->last_error.c_str() : "null context";
}

int mimir_malloc(mimir_ctx* ctx, size_t bytes, void** dptr) {
    if (!ctx || !dptr) return MIMIR_EINVAL;
    *dptr = nullptr;
    MIMIR_REQUIRE(ctx, bytes > 0, "mimir_malloc: zero-byte allocation");
    if (ctx->alloc_limit && (bytes > ctx->alloc_limit || ctx->alloc_used > ctx->alloc_limit - bytes))
        return fail(ctx, MIMIR_ENOMEM, "mimir_malloc: %zu bytes over the context cap (%zu of %zu used)",
                    bytes, ctx->alloc_used, ctx->alloc_limit);
    MIMIR_ENTER(ctx);
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();  // clear the sticky-free error state of the runtime
        return fail(ctx, MIMIR_ENOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    }
    ctx->allocs[p] = bytes;
    ctx->alloc_used += bytes;
    *dptr = p;
    return MIMIR_OK;
}

int mimir_free(mimir_ctx* ctx, void* dptr) {
    if (!ctx) return MIMIR_EINVAL;
    if (!dptr) return MIMIR_OK;
    auto it = ctx->allocs.find(dptr);
    MIMIR_REQUIRE(ctx, it != ctx->allocs.end(), "mimir_free: %p was not allocated by this context",
                  dptr);
    MIMIR_ENTER(ctx);
    // Work already enqueued may still read the buffer.
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamSynchronize");
    e = hipFree(dptr);
    ctx->alloc_used -= it->second;
    ctx->allocs.erase(it);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipFree");
    return MIMIR_OK;
}

int mimir_upload(mimir_ctx* ctx, void* dst_dev, const void* src_host, size_t bytes) {
    if (!ctx) return MIMIR_EINVAL;
    if (bytes == 0) return MIMIR_OK;
    MIMIR_REQUIRE(ctx, dst_dev && src_host, "mimir_upload: null pointer");
    MIMIR_ENTER(ctx);
    hipError_t e = hipMemcpyAsync(dst_dev, src_host, bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "mimir_upload");
    return MIMIR_OK;
}

int mimir_download(mimir_ctx* ctx, void* dst_host, const void* src_dev, size_t bytes) {
    if (!ctx) return MIMIR_EINVAL;
    if (bytes == 0) return MIMIR_OK;
    MIMIR_REQUIRE(ctx, dst_host && src_dev, "mimir_download: null pointer");
    MIMIR_ENTER(ctx);
    hipError_t e = hipMemcpyAsync(dst_host, src_dev, bytes, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "mimir_download");
    return MIMIR_OK;
}

int mimir_copy(mimir_ctx* ctx, void* dst_dev, const void* src_dev, size_t bytes) {
    if (!ctx) return MIMIR_EINVAL;
    if (bytes == 0) return MIMIR_OK;
    MIMIR_REQUIRE(ctx, dst_dev && src_dev, "mimir_copy: null pointer");
    MIMIR_ENTER(ctx);
    const uint8_t* s = static_cast<const uint8_t*>(src_dev);
    uint8_t* d = static_cast<uint8_t*>(dst_dev);
    int64_t n16 = 0;
    if (aligned16(s) && aligned16(d)) {
        n16 = static_cast<int64_t>(bytes / 16);
        if (n16 > 0) {
            const int st = with_block(ew_block(ctx->tune), [&](auto bsc) {
                constexpr int BS = decltype(bsc)::value;
                if (ctx->keep_outputs)
                    copy16_kernel<true, BS><<<full_grid(n16, BS), BS, 0, ctx->stream>>>(
                        reinterpret_cast<const u4*>(s), reinterpret_cast<u4*>(d), n16);
                else
                    copy16_kernel<false, BS><<<full_grid(n16, BS), BS, 0, ctx->stream>>>(
                        reinterpret_cast<const u4*>(s), reinterpret_cast<u4*>(d), n16);
                return launched(ctx, "copy16_kernel");
            });
            if (st) return st;
        }
    }
    const int64_t rest = static_cast<int64_t>(bytes) - n16 * 16;
    if (rest > 0) {
        copy1_kernel<<<stride_grid(rest), kBlock, 0, ctx->stream>>>(s + n16 * 16, d + n16 * 16, rest);
        if (int st = launched(ctx, "copy1_kernel")) return st;
    }
    return MIMIR_OK;
}

int mimir_fill_f32(mimir_ctx* ctx, float* dst_dev, int64_t n, float value) {
    if (!ctx) return MIMIR_EINVAL;
    MIMIR_REQUIRE(ctx, n >= 0, "mimir_fill_f32: n < 0");
    if (n == 0) return MIMIR_OK;
    MIMIR_REQUIRE(ctx, dst_dev, "mimir_fill_f32: null pointer");
    MIMIR_ENTER(ctx);
    fill_kernel<<<stride_grid(n), kBlock, 0, ctx->stream>>>(dst_dev, n, value);
    return launched(ctx, "fill_kernel");
}

int mimir_sync(mimir_ctx* ctx) {
    MIMIR_ENTER(ctx);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamSynchronize");
    return MIMIR_OK;
}

int mimir_event_create(mimir_ctx* ctx, mimir_event** out) {
    if (!ctx || !out) return MIMIR_EINVAL;
    MIMIR_ENTER(ctx);
    mimir_event* ev = new (std::nothrow) mimir_event();
    if (!ev) return MIMIR_ENOMEM;
    ev->device = ctx->device;
    hipError_t e = hipEventCreate(&ev->ev);
    if (e != hipSuccess) {
        delete ev;
        return hip_fail(ctx, e, "hipEventCreate");
    }
    *out = ev;
    return MIMIR_OK;
}

int mimir_event_destroy(mimir_event* ev) {
    if (!ev) return MIMIR_EINVAL;
    (void)hipSetDevice(ev->device);
    (void)hipEventDestroy(ev->ev);
    delete ev;
    return MIMIR_OK;
}

int mimir_event_record(mimir_ctx* ctx, mimir_event* ev) {
    if (!ctx || !ev) return MIMIR_EINVAL;
    MIMIR_ENTER(ctx);
    hipError_t e = hipEventRecord(ev->ev, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipEventRecord");
    return MIMIR_OK;
}

int mimir_event_elapsed_ms(mimir_event* start, mimir_event* stop, float* ms) {
    if (!start || !stop || !ms) return MIMIR_EINVAL;
    if (hipEventSynchronize(stop->ev) != hipSuccess) return MIMIR_EDEVICE;
    if (hipEventElapsedTime(ms, start->ev, stop->ev) != hipSuccess) return MIMIR_EDEVICE;
    return MIMIR_OK;
}

}  // extern "C"
