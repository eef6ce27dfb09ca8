// gather.hip -- token-embedding gather for gfx950 (bit-exact).
//
// One workgroup (or a slice of one, for narrow rows) per token row: the id
// is read once per wave (wave-uniform), then the threads move the row as
// 16-byte vectors, one per thread per pass -- for the 4096-wide rows of the
// benchmark, 1024 threads each moving one vector.  Rows of padding / out-of-range ids are written as
// zeros without touching the table.  Payload moves as raw 32-bit words, so
// every bit pattern (NaN payloads, -0, denormals) is copied unchanged.
//
// Semantics: Model::forwardPassView inline gather, Model.cpp:1152-1205 (int
// ids) and Model.cpp:5301-5334 (float ids rounded with llround).
#include "common.hpp"
#include "internal.hpp"
#include "ids.hpp"

#include <math.h>

using namespace mimir;

namespace {

struct GatherArgs {
    const void* ids;
    int64_t n_ids;
    const float* table;
    int32_t vocab;
    int32_t dim;
    int32_t pad;
    float* y;
};

constexpr int kWavesPerBlock = kBlock / kWave;

// TPT threads per token row (BS / TPT token rows per workgroup), one 16-byte
// vector per thread per pass; rows wider than TPT vectors take several passes.
// Table rows are loaded through the caches, output rows stored non-temporal
// (unless KEEP: the context keeps outputs cached for a consumer launched next):
// a token that repeats an id already gathered in the same launch finds the
// row in L2 or the Infinity Cache.  At configs[3] 37% of the tokens repeat an
// id; measured on MI355X, 157 us against 172 us with non-temporal loads.
template <int MODE, int TPT, int BS, bool KEEP>
__global__ __launch_bounds__(BS) void embed_vec(GatherArgs a) {
    const int t = threadIdx.x % TPT;
    const int64_t token = static_cast<int64_t>(blockIdx.x) * (BS / TPT) + threadIdx.x / TPT;
    if (token >= a.n_ids) return;  // no barriers in this kernel
    const int32_t id = load_id<MODE>(a.ids, token);
    const bool copy = !(a.pad >= 0 && id == a.pad) && id >= 0 && id < a.vocab;
    const int64_t dim4 = a.dim >> 2;
    const u4* src = reinterpret_cast<const u4*>(a.table) + (copy ? static_cast<int64_t>(id) * dim4 : 0);
    u4* dst = reinterpret_cast<u4*>(a.y) + token * dim4;
    for (int64_t c = t; c < dim4; c += TPT) {
        const u4 v = copy ? src[c] : u4(0u);
        if constexpr (KEEP) dst[c] = v;
        else st_stream(dst + c, v);
    }
}

// Any dim / alignment: one wavefront per token, 32-bit words.
template <int MODE>
__global__ __launch_bounds__(kBlock) void embed_scalar(GatherArgs a) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t token = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
    if (token >= a.n_ids) return;
    const int32_t id = load_id<MODE>(a.ids, token);
    const bool copy = !(a.pad >= 0 && id == a.pad) && id >= 0 && id < a.vocab;
    const uint32_t* src = reinterpret_cast<const uint32_t*>(a.table) +
                          (copy ? static_cast<int64_t>(id) * a.dim : 0);
    uint32_t* dst = reinterpret_cast<uint32_t*>(a.y) + token * a.dim;
    for (int64_t c = lane; c < a.dim; c += kWave) dst[c] = copy ? src[c] : 0u;
}

template <int MODE, bool KEEP>
void launch_vec(int tpt, unsigned vb, hipStream_t stream, const GatherArgs& a) {
    switch (tpt) {
        case 64: embed_vec<MODE, 64, 256, KEEP><<<vb, 256, 0, stream>>>(a); break;
        case 128: embed_vec<MODE, 128, 256, KEEP><<<vb, 256, 0, stream>>>(a); break;
        case 256: embed_vec<MODE, 256, 256, KEEP><<<vb, 256, 0, stream>>>(a); break;
        case 512: embed_vec<MODE, 512, 512, KEEP><<<vb, 512, 0, stream>>>(a); break;
        default: embed_vec<MODE, 1024, 1024, KEEP><<<vb, 1024, 0, stream>>>(a); break;
    }
}

template <int MODE>
int run(mimir_ctx* ctx, const void* ids, int64_t n_ids, const float* table, int64_t table_len,
        int32_t vocab, int32_t dim, int32_t pad, float* y) {
    MIMIR_REQUIRE(ctx, n_ids >= 0, "Embedding: n_ids < 0");
    // Model.cpp:1176-1177: vocab and dim are clamped to at least 1.
    vocab = vocab < 1 ? 1 : vocab;
    dim = dim < 1 ? 1 : dim;
    // Model.cpp:1181-1182: the table must hold vocab*dim floats.
    MIMIR_REQUIRE(ctx, table_len >= static_cast<int64_t>(vocab) * dim,
                  "Embedding: invalid weight size (%lld < %d x %d)", (long long)table_len, vocab, dim);
    if (n_ids == 0) return MIMIR_OK;
    MIMIR_REQUIRE(ctx, ids && table && y, "Embedding: null tensor");
    MIMIR_ENTER(ctx);
    const GatherArgs a{ids, n_ids, table, vocab, dim, pad, y};
    unsigned blocks;
    if (!grid_for(n_ids, kWavesPerBlock, kBlock, &blocks))
        return fail(ctx, MIMIR_EINVAL, "Embedding: %lld ids exceed the grid limit", (long long)n_ids);
    if (dim % 4 == 0 && aligned16(table) && aligned16(y)) {
        const int64_t dim4 = dim / 4;
        int tpt = ctx->tune.gather_tpt;
        if (tpt != 64 && tpt != 128 && tpt != 256 && tpt != 512 && tpt != 1024)
            tpt = dim4 <= 64 ? 64 : dim4 <= 128 ? 128 : dim4 <= 256 ? 256 : dim4 <= 512 ? 512 : 1024;
        const int bs = tpt < kBlock ? kBlock : tpt;
        unsigned vb;
        if (!grid_for(n_ids, bs / tpt, bs, &vb))
            return fail(ctx, MIMIR_EINVAL, "Embedding: %lld ids exceed the grid limit", (long long)n_ids);
        if (ctx->keep_outputs) launch_vec<MODE, true>(tpt, vb, ctx->stream, a);
        else launch_vec<MODE, false>(tpt, vb, ctx->stream, a);
        return launched(ctx, "embed_vec");
    }
    embed_scalar<MODE><<<blocks, kBlock, 0, ctx->stream>>>(a);
    return launched(ctx, "embed_scalar");
}

}  // namespace

int mimir::embedding_launch(mimir_ctx* ctx, const void* ids, int mode, int64_t n_ids, const float* table,
                            int64_t table_len, int32_t vocab, int32_t dim, int32_t pad, float* y) {
    switch (mode) {
        case kIdsF32: return run<kIdsF32>(ctx, ids, n_ids, table, table_len, vocab, dim, pad, y);
        case kIdsI32AsF32: return run<kIdsI32AsF32>(ctx, ids, n_ids, table, table_len, vocab, dim, pad, y);
        default: return run<kIdsI32>(ctx, ids, n_ids, table, table_len, vocab, dim, pad, y);
    }
}

extern "C" {

int mimir_embedding_fwd(mimir_ctx* ctx, const int32_t* ids, int64_t n_ids, const float* table,
                        int64_t table_len, int32_t vocab, int32_t dim, int32_t padding_idx,
                        float* y) {
    if (!ctx) return MIMIR_EINVAL;
    return run<kIdsI32>(ctx, ids, n_ids, table, table_len, vocab, dim, padding_idx, y);
}

int mimir_embedding_f32ids_fwd(mimir_ctx* ctx, const float* ids, int64_t n_ids,
                               const float* table, int64_t table_len, int32_t vocab, int32_t dim,
                               int32_t padding_idx, float* y) {
    if (!ctx) return MIMIR_EINVAL;
    return run<kIdsF32>(ctx, ids, n_ids, table, table_len, vocab, dim, padding_idx, y);
}

}  // extern "C"
