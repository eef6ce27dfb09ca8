// internal.hpp -- host-side context and status plumbing shared by the
// translation units of libmimir_hip (not part of the public ABI).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/mimir_hip.h"
#include "rows.hpp"

struct mimir_ctx {
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;  // where ops are enqueued
    size_t alloc_limit = 0;        // 0 = unlimited
    size_t alloc_used = 0;
    std::unordered_map<void*, size_t> allocs;
    std::string last_error;
    mimir::Tuning tune;  // launch-shape override (MIMIR_TUNE), read at creation
    int keep_outputs = 0;  // 1: ops store outputs through the caches (mimir_ctx_set_output_caching)
    // Scratch for the partial results of multi-workgroup row reductions
    // (longrow.hip); grows on demand, reused in stream order.
    void* scratch = nullptr;
    size_t scratch_bytes = 0;
    // Device address of this GPU's fixed scratch array (backward.hip), for
    // the entry point that allocates nothing; set at context creation.
    void* noalloc_scratch = nullptr;
    // This GPU's columns of 1.0f then -0.0f (mimir::kUnitCols each), the
    // weights of a row kernel's absent scale / bias (norm.hip).
    const float* unit_weights = nullptr;
    // hipBLASLt state (handle and per-shape plans) and rocBLAS handle for the
    // attention layers' products (gemm.hip), created on first use, sharing a
    // workspace of this library's (grown on demand).
    void* blaslt = nullptr;
    void* blas = nullptr;
    void* blas_ws = nullptr;
    size_t blas_ws_bytes = 0;
    // Captured store graphs alive on this context (store.hip).  Their kernels
    // hold the addresses of the scratch and the library workspace as they
    // were at capture, so while any exists a buffer that must grow is retired
    // (kept allocated) rather than freed; the retired buffers are freed when
    // the last graph goes.
    int graph_pins = 0;
    std::vector<void*> retired;
};

struct mimir_event {
    hipEvent_t ev = nullptr;
    int device = 0;
};

namespace mimir {

// Record a message on the context and return `code`.
inline int fail(mimir_ctx* ctx, int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (ctx) ctx->last_error = buf;
    return code;
}

inline int hip_fail(mimir_ctx* ctx, hipError_t e, const char* what) {
    return fail(ctx, MIMIR_EDEVICE, "%s: %s", what, hipGetErrorString(e));
}

// Make the context's device current for this host thread.
inline int enter(mimir_ctx* ctx) {
    if (!ctx) return MIMIR_EINVAL;
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipGetDevice");
    if (cur != ctx->device) {
        e = hipSetDevice(ctx->device);
        if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
    }
    return MIMIR_OK;
}

// Status of the launch just enqueued.
inline int launched(mimir_ctx* ctx, const char* kernel) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(ctx, e, kernel);
    return MIMIR_OK;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// dispatch_fits / grid_for: launch-size checks (rows.hpp).

// Context scratch of at least `bytes` (runtime.hip).  Growing it waits for
// the work already enqueued, which may still read the old buffer (or, while
// captured graphs hold its address, retires the old buffer instead).
int ensure_scratch(mimir_ctx* ctx, size_t bytes, void** out);

// Free a device buffer that enqueued work or captured graphs may still use:
// retired while graphs are alive, else freed after the stream drains.
int retire_or_free(mimir_ctx* ctx, void* p);
// A captured graph starts / stops holding the context's buffers.
void graph_pin(mimir_ctx* ctx);
int graph_unpin(mimir_ctx* ctx);

// Row-major fp32 C[M x N] = A[M x K] * B[K x N] on the context's stream
// (rocBLAS; gemm.hip), and the release of its handle at context teardown.
int gemm_f32(mimir_ctx* ctx, int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, const float* B,
             int64_t ldb, float* C, int64_t ldc);
// The general form: row-major C = alpha op(A) op(B) + beta C over `batch`
// products whose operands sit `stride_*` floats apart; op(A) is M x K (A
// stored K x M when trans_a), op(B) is K x N (B stored N x K when trans_b).
int gemm_f32_ex(mimir_ctx* ctx, bool trans_a, bool trans_b, int64_t M, int64_t N, int64_t K, float alpha,
                const float* A, int64_t lda, int64_t stride_a, const float* B, int64_t ldb, int64_t stride_b,
                float beta, float* C, int64_t ldc, int64_t stride_c, int64_t batch);
void gemm_release(mimir_ctx* ctx);
// Whether products go to hipBLASLt (unless MIMIR_TUNE blas=0), where the
// transposed-operand forms run as fast as the plain ones.
bool gemm_lt(mimir_ctx* ctx);

// A chain of elementwise layers run as one kernel (store.hip's fusion):
// v = ins[0]; then each step k sets v = op_k(v, operand) -- GELU, SiLU, or
// an add / multiply with ins[operand] (operand -1: v itself) -- and, when
// store_k >= 0, writes v to outs[store_k].  Every tensor has n floats.  The
// per-element functions are the standalone kernels', so each stored value
// has the bits the unfused layers would give it.
constexpr int kFuseMax = 8;
enum FuseKind : int32_t { kFuseGelu = 1, kFuseSilu = 2, kFuseAdd = 3, kFuseMul = 4 };
struct FuseStep {
    int32_t kind;
    int32_t operand;
    int32_t store;
};
struct FuseProgram {
    const float* ins[kFuseMax];
    float* outs[kFuseMax];
    FuseStep steps[kFuseMax];
    int32_t n_ins, n_outs, n_steps;
};
int fused_chain(mimir_ctx* ctx, const FuseProgram& p, int64_t n);

// The runtime's fused LayerNorm (norm.hip): optionally an Add before it
// (h = x + r, written to h when set) and a chain of elementwise steps after
// it (epi, operands in epi.ins; y, when set, gets the LayerNorm output
// itself).  rows x cols, gamma / beta as mimir_layernorm_fwd.
struct LnFused {
    const float* x;
    const float* r;
    float* h;
    const float* g;
    const float* b;
    float* y;
    int64_t rows, cols;
    float eps;
    FuseProgram epi;
};
// Whether the fused LayerNorm takes rows of `cols` floats with these
// parameter pointers (the register-resident vector kernel).
bool layernorm_fusable(const mimir_ctx* ctx, int64_t cols, const float* g, const float* b);
int layernorm_fused(mimir_ctx* ctx, const LnFused& f);

// Look up this context's device address of the no-allocation scratch array
// (backward.hip); called once per context, with its device current.
int noalloc_scratch_init(mimir_ctx* ctx);
// Gives up the array if `ctx` holds it (context teardown, stream drained).
void noalloc_scratch_release(mimir_ctx* ctx);
// Widest row (floats) the register-resident row kernels hold, and the
// per-GPU set-up of their unit weights (norm.hip), run at context creation.
constexpr int kUnitCols = 4 * 4096;
int norm_init(mimir_ctx* ctx);

// Scratch for one call: a fixed span (the no-allocation entry point's device
// array) or, when `fixed` is null, the context's growable scratch.  A fixed
// span never grows: a call needing more is refused before any launch.
struct ScratchSpan {
    void* ptr;
    size_t bytes;
};
inline int get_scratch(mimir_ctx* ctx, const ScratchSpan* fixed, size_t bytes, void** out) {
    if (!fixed) return ensure_scratch(ctx, bytes, out);
    if (bytes > fixed->bytes)
        return fail(ctx, MIMIR_EINVAL, "this call needs %zu bytes of scratch; the no-allocation entry point has %zu",
                    bytes, fixed->bytes);
    *out = fixed->ptr;
    return MIMIR_OK;
}

// Rows too long for one workgroup's registers: split each row over many
// workgroups (longrow.hip).  `kind`: 0 LayerNorm, 1 RMSNorm,
// 2 add + RMSNorm; softmax `mode` as in mimir_softmax_fwd.
bool longrow_applies(int64_t rows, int64_t cols);
int longrow_norm(mimir_ctx* ctx, int kind, const float* x, const float* r, float* r_out, const float* g,
                 const float* b, int64_t w_len, float* y, int64_t rows, int64_t cols, float eps);
int longrow_softmax(mimir_ctx* ctx, int mode, const float* x, float* y, int64_t rows, int64_t cols);
// Second-level groups of the slot sums (backward.hip launch_sum_slots): its
// `tmp` holds kSlotGroups rows of the summed width.
constexpr int kSlotGroups = 16;
// LayerNorm backward of such rows (the forward's statistics, then two more
// passes); dgamma / dbeta are added onto, as the reference's grad_weights.
// The apply pass takes kLongBwdRows rows per workgroup: with more rows than
// that and dgamma wanted, it leaves one slot of column sums per row group,
// [*nslots][2*cols] at *slots with room for the slot sums at *tmp, for the
// caller to add into dgamma / dbeta; else *slots is null.
constexpr int64_t kLongBwdRows = 16;
int longrow_ln_bwd(mimir_ctx* ctx, const float* x, const float* dy, const float* gamma, float* dx, float* dgamma,
                   float* dbeta, int64_t rows, int64_t cols, float eps, int accumulate, float** slots,
                   int64_t* nslots, float** tmp, const ScratchSpan* fixed = nullptr);

// Embedding gather with an id mode (gather.hip); used by the C ABI and the
// device-resident runtime (store.hip).
enum : int { kIdsI32 = 0, kIdsF32 = 1, kIdsI32AsF32 = 2 };
int embedding_launch(mimir_ctx* ctx, const void* ids, int mode, int64_t n_ids, const float* table,
                     int64_t table_len, int32_t vocab, int32_t dim, int32_t pad, float* y);
// Its backward, the scatter-add into the gradient table (backward.hip).
int embedding_bwd_launch(mimir_ctx* ctx, const void* ids, int mode, int64_t n_ids, const float* dy, float* grad,
                         int64_t table_len, int32_t vocab, int32_t dim, int32_t pad);

}  // namespace mimir

#define MIMIR_ENTER(ctx)                         \
    do {                                         \
        if (!(ctx)) return MIMIR_EINVAL;         \
        const int _st = ::mimir::enter(ctx);     \
        if (_st != MIMIR_OK) return _st;         \
    } while (0)

#define MIMIR_REQUIRE(ctx, cond, ...)                                   \
    do {                                                                \
        if (!(cond)) return ::mimir::fail((ctx), MIMIR_EINVAL, __VA_ARGS__); \
    } while (0)
