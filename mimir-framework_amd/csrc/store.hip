// store.hip -- device-resident named tensor store and layer runner.
//
// The reference keeps every activation in Model::tensor_store /
// tensor_store_int (Model.hpp:608-610): host std::vectors looked up by name,
// each layer's output a fresh vector (Model.cpp:6674).  Here the names map to
// device buffers of a per-store pool:
//   * a layer's output always goes to a buffer that none of its inputs uses,
//     then the name is rebound and the old buffer returns to the pool, so an
//     output may take the name of an input ("x" -> "x") without aliasing;
//   * buffers are reference-counted by the names bound to them: Identity and
//     inference-time Dropout bind their output name to the input's buffer;
//   * every op runs on the context's stream, so a buffer released by one
//     layer can be reused by a later layer in stream order with no sync.
// The routing follows Model::forwardPassView (Model.cpp:4621-6824): see
// mimir_store_set_inputs / mimir_store_run in include/mimir_hip.h.
#include "common.hpp"
#include "internal.hpp"

#include <map>
#include <new>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

using namespace mimir;

namespace {

struct Buf {
    void* p = nullptr;
    size_t cap = 0;
    int refs = 0;
};

struct Slot {
    Buf* buf = nullptr;
    int64_t n = 0;
};

__global__ __launch_bounds__(kBlock) void fill_i32_kernel(int32_t* dst, int64_t n, int32_t v) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) dst[i] = v;
}

}  // namespace

struct mimir_store {
    mimir_ctx* ctx = nullptr;
    std::unordered_map<std::string, Slot> f32;
    std::unordered_map<std::string, Slot> i32;
    std::vector<std::unique_ptr<Buf>> bufs;
    std::multimap<size_t, Buf*> free_bufs;  // capacity -> idle buffer

    std::unordered_map<std::string, Slot>& map(int dtype) { return dtype == MIMIR_DTYPE_I32 ? i32 : f32; }

    // An idle buffer of at least `bytes` (best fit), or a new one.
    int acquire(size_t bytes, Buf** out) {
        bytes = (bytes + 255) & ~size_t(255);
        if (bytes == 0) bytes = 256;
        auto it = free_bufs.lower_bound(bytes);
        if (it != free_bufs.end() && it->first <= 2 * bytes) {
            *out = it->second;
            free_bufs.erase(it);
            return MIMIR_OK;
        }
        void* p = nullptr;
        const int st = mimir_malloc(ctx, bytes, &p);
        if (st != MIMIR_OK) return st;
        bufs.push_back(std::make_unique<Buf>());
        Buf* b = bufs.back().get();
        b->p = p;
        b->cap = bytes;
        *out = b;
        return MIMIR_OK;
    }

    void release(Buf* b) {
        if (b && --b->refs == 0) free_bufs.emplace(b->cap, b);
    }

    void bind(int dtype, const std::string& name, Buf* b, int64_t n) {
        ++b->refs;  // before releasing the old binding, which may be the same buffer
        auto& m = map(dtype);
        auto it = m.find(name);
        if (it != m.end()) {
            release(it->second.buf);
            it->second = Slot{b, n};
        } else {
            m.emplace(name, Slot{b, n});
        }
    }

    // A buffer holding nothing yet goes straight back to the pool on error.
    void discard(Buf* b) {
        if (b && b->refs == 0) free_bufs.emplace(b->cap, b);
    }

    void clear() {
        for (auto& kv : f32) release(kv.second.buf);
        for (auto& kv : i32) release(kv.second.buf);
        f32.clear();
        i32.clear();
    }
};

namespace {

int put_host(mimir_store* s, int dtype, const std::string& name, const void* host, int64_t n) {
    Buf* b = nullptr;
    int st = s->acquire(static_cast<size_t>(n) * 4, &b);
    if (st) return st;
    if (n > 0) {
        st = mimir_upload(s->ctx, b->p, host, static_cast<size_t>(n) * 4);
        if (st) {
            s->discard(b);
            return st;
        }
    }
    s->bind(dtype, name, b, n);
    return MIMIR_OK;
}

const char* layer_name(const mimir_layer& L) { return L.name ? L.name : "?"; }

// One layer of Model::forwardPassView's loop (Model.cpp:4795-6680), inference.
int run_layer(mimir_store* s, const mimir_layer& L) {
    mimir_ctx* ctx = s->ctx;
    static const char* const kDefaultInput[] = {"x"};
    const char* const* names = L.n_inputs > 0 ? L.inputs : kDefaultInput;
    const int n_in = L.n_inputs > 0 ? L.n_inputs : 1;
    const std::string out_name = (L.output && *L.output) ? L.output : "x";

    // RETRIEVE INPUTS (Model.cpp:4813-4856): float store first; Embedding
    // input 0 may come from the int store (ids read as floats), and when it
    // is missing there too, seq_len padding ids are stored under its name.
    struct In {
        const void* p;
        int64_t n;
        bool ids_i32;
    };
    std::vector<In> in;
    in.reserve(n_in);
    for (int k = 0; k < n_in; ++k) {
        const std::string name = names[k] ? names[k] : "";
        auto itf = s->f32.find(name);
        if (itf != s->f32.end()) {
            in.push_back(In{itf->second.buf->p, itf->second.n, false});
            continue;
        }
        if (L.type == MIMIR_LAYER_EMBEDDING && k == 0) {
            auto iti = s->i32.find(name);
            if (iti == s->i32.end()) {
                const int64_t len = L.seq_len > 0 ? L.seq_len : 1;
                const int32_t pad = L.padding_idx >= 0 ? L.padding_idx : 0;
                Buf* b = nullptr;
                if (int st = s->acquire(static_cast<size_t>(len) * 4, &b)) return st;
                MIMIR_ENTER(ctx);
                fill_i32_kernel<<<1, kBlock, 0, ctx->stream>>>(static_cast<int32_t*>(b->p), len, pad);
                if (int st = launched(ctx, "fill_i32_kernel")) {
                    s->discard(b);
                    return st;
                }
                s->bind(MIMIR_DTYPE_I32, name, b, len);
                iti = s->i32.find(name);
            }
            in.push_back(In{iti->second.buf->p, iti->second.n, true});
            continue;
        }
        return fail(ctx, MIMIR_EINVAL, "Missing input tensor: %s (layer %s)", name.c_str(), layer_name(L));
    }
    const int64_t N = in[0].n;
    const float* x = static_cast<const float*>(in[0].p);

    // Identity / inference Dropout: the output name shares the input buffer.
    if (L.type == MIMIR_LAYER_IDENTITY || L.type == MIMIR_LAYER_DROPOUT) {
        const std::string in0 = names[0] ? names[0] : "";
        Slot src = s->f32.at(in0);
        s->bind(MIMIR_DTYPE_F32, out_name, src.buf, src.n);
        return MIMIR_OK;
    }

    // Output size, checks where the reference throws.
    int64_t out_n = N;
    switch (L.type) {
        case MIMIR_LAYER_LAYERNORM:
        case MIMIR_LAYER_RMSNORM:
        case MIMIR_LAYER_GELU:
        case MIMIR_LAYER_SILU:
            break;
        case MIMIR_LAYER_SOFTMAX:
        case MIMIR_LAYER_LOGSOFTMAX:
            if (N == 0) return fail(ctx, MIMIR_EINVAL, "Softmax: empty input (layer %s)", layer_name(L));
            break;
        case MIMIR_LAYER_ADD:
        case MIMIR_LAYER_MULTIPLY:
            if (n_in < 2)
                return fail(ctx, MIMIR_EINVAL, "%s layer requires 2 inputs, got %d",
                            L.type == MIMIR_LAYER_ADD ? "Add" : "Multiply", n_in);
            out_n = L.type == MIMIR_LAYER_ADD ? (in[0].n > in[1].n ? in[0].n : in[1].n) : in[0].n;
            break;
        case MIMIR_LAYER_EMBEDDING: {
            const int64_t dim = L.embed_dim > 1 ? L.embed_dim : 1;
            out_n = N * dim;
            break;
        }
        default:
            return fail(ctx, MIMIR_EINVAL, "layer %s: type %d is not on this path", layer_name(L), L.type);
    }

    Buf* ob = nullptr;
    if (int st = s->acquire(static_cast<size_t>(out_n) * 4, &ob)) return st;
    float* y = static_cast<float*>(ob->p);
    int st = MIMIR_OK;
    switch (L.type) {
        case MIMIR_LAYER_LAYERNORM: {
            // LayerOps.hpp:276-285: group = in_features or N; gamma | beta block
            // only when affine; a null block means no affine transform.
            const int64_t n = L.in_features > 0 ? L.in_features : N;
            if (n <= 0 || N % n != 0) {
                st = fail(ctx, MIMIR_EINVAL, "LayerNorm: invalid normalized_size (layer %s)", layer_name(L));
                break;
            }
            const float* gamma = (L.affine && L.weights && L.weights_len > 0) ? L.weights : nullptr;
            const float* beta = (gamma && L.use_bias) ? L.weights + n : nullptr;
            if (gamma && L.weights_len < (beta ? 2 * n : n)) {
                st = fail(ctx, MIMIR_EINVAL, "LayerNorm: weight block of %lld < %lld (layer %s)",
                          (long long)L.weights_len, (long long)(beta ? 2 * n : n), layer_name(L));
                break;
            }
            st = mimir_layernorm_fwd(ctx, x, gamma, beta, y, N / n, n, L.eps);
            break;
        }
        case MIMIR_LAYER_RMSNORM: {
            // LayerOpsExt.hpp:364-375: weight i applies while i < getWeightsSize().
            const bool use_w = L.affine && L.weights && L.weights_len > 0;
            if (N > 0) st = mimir_rmsnorm_fwd(ctx, x, use_w ? L.weights : nullptr, use_w ? L.weights_len : 0, y, 1, N, L.eps);
            break;
        }
        case MIMIR_LAYER_SOFTMAX:
            st = mimir_softmax_fwd(ctx, x, y, 1, N, MIMIR_SOFTMAX_MUL_INV);
            break;
        case MIMIR_LAYER_LOGSOFTMAX:
            st = mimir_softmax_fwd(ctx, x, y, 1, N, MIMIR_SOFTMAX_LOG);
            break;
        case MIMIR_LAYER_GELU:
            st = mimir_gelu_fwd(ctx, x, y, N);
            break;
        case MIMIR_LAYER_SILU:
            st = mimir_silu_fwd(ctx, x, y, N);
            break;
        case MIMIR_LAYER_ADD:
            st = mimir_add_fwd(ctx, x, in[0].n, static_cast<const float*>(in[1].p), in[1].n, y);
            break;
        case MIMIR_LAYER_MULTIPLY:
            st = mimir_mul_fwd(ctx, x, in[0].n, static_cast<const float*>(in[1].p), in[1].n, y);
            break;
        case MIMIR_LAYER_EMBEDDING:
            // Model.cpp:5307-5312: the weight block must exist and hold vocab*dim.
            if (!L.weights || L.weights_len <= 0) {
                st = fail(ctx, MIMIR_EINVAL, "Embedding: weights not initialized (layer %s)", layer_name(L));
                break;
            }
            st = embedding_launch(ctx, in[0].p, in[0].ids_i32 ? kIdsI32AsF32 : kIdsF32, N, L.weights,
                                  L.weights_len, L.vocab_size, L.embed_dim, L.padding_idx, y);
            break;
    }
    if (st != MIMIR_OK) {
        s->discard(ob);
        return st;
    }
    s->bind(MIMIR_DTYPE_F32, out_name, ob, out_n);  // STORE OUTPUT, Model.cpp:6655,6674
    return MIMIR_OK;
}

}  // namespace

extern "C" {

int mimir_store_create(mimir_ctx* ctx, mimir_store** out) {
    if (!ctx || !out) return MIMIR_EINVAL;
    mimir_store* s = new (std::nothrow) mimir_store();
    if (!s) return MIMIR_ENOMEM;
    s->ctx = ctx;
    *out = s;
    return MIMIR_OK;
}

int mimir_store_destroy(mimir_store* s) {
    if (!s) return MIMIR_EINVAL;
    int st = MIMIR_OK;
    for (auto& b : s->bufs) {
        const int r = mimir_free(s->ctx, b->p);
        if (r != MIMIR_OK && st == MIMIR_OK) st = r;
    }
    delete s;
    return st;
}

int mimir_store_clear(mimir_store* s) {
    if (!s) return MIMIR_EINVAL;
    s->clear();
    return MIMIR_OK;
}

int mimir_store_put(mimir_store* s, const char* name, int dtype, const void* host, int64_t n) {
    if (!s) return MIMIR_EINVAL;
    MIMIR_REQUIRE(s->ctx, name && (dtype == MIMIR_DTYPE_F32 || dtype == MIMIR_DTYPE_I32) && n >= 0 &&
                              (n == 0 || host),
                  "mimir_store_put: invalid argument");
    return put_host(s, dtype, name, host, n);
}

int mimir_store_info(mimir_store* s, const char* name, int dtype, void** dptr, int64_t* n) {
    if (!s) return MIMIR_EINVAL;
    MIMIR_REQUIRE(s->ctx, name && dptr && n, "mimir_store_info: invalid argument");
    auto& m = s->map(dtype);
    auto it = m.find(name);
    MIMIR_REQUIRE(s->ctx, it != m.end(), "mimir_store_info: no tensor named %s", name);
    *dptr = it->second.buf->p;
    *n = it->second.n;
    return MIMIR_OK;
}

int mimir_store_get(mimir_store* s, const char* name, int dtype, void* host, int64_t cap, int64_t* n) {
    if (!s) return MIMIR_EINVAL;
    MIMIR_REQUIRE(s->ctx, name && n && cap >= 0, "mimir_store_get: invalid argument");
    auto& m = s->map(dtype);
    auto it = m.find(name);
    MIMIR_REQUIRE(s->ctx, it != m.end(), "mimir_store_get: no tensor named %s", name);
    *n = it->second.n;
    const int64_t k = cap < it->second.n ? cap : it->second.n;
    if (k > 0) {
        MIMIR_REQUIRE(s->ctx, host, "mimir_store_get: null host buffer");
        return mimir_download(s->ctx, host, it->second.buf->p, static_cast<size_t>(k) * 4);
    }
    return MIMIR_OK;
}

int mimir_store_set_inputs(mimir_store* s, const char* const* fnames, const float* const* fdata,
                           const int64_t* fsizes, int32_t nf, const char* const* inames,
                           const int32_t* const* idata, const int64_t* isizes, int32_t ni) {
    if (!s) return MIMIR_EINVAL;
    MIMIR_REQUIRE(s->ctx, nf >= 0 && ni >= 0 && (nf == 0 || (fnames && fdata && fsizes)) &&
                              (ni == 0 || (inames && idata && isizes)),
                  "mimir_store_set_inputs: invalid argument");
    s->clear();
    // Model.cpp:1396-1407: "x" = float_inputs["x"], else ["__input__"], else empty.
    int xi = -1;
    for (int32_t i = 0; i < nf && xi < 0; ++i)
        if (fnames[i] && std::string(fnames[i]) == "x") xi = i;
    for (int32_t i = 0; i < nf && xi < 0; ++i)
        if (fnames[i] && std::string(fnames[i]) == "__input__") xi = i;
    const float* x0 = xi >= 0 ? fdata[xi] : nullptr;
    const int64_t n0 = xi >= 0 ? fsizes[xi] : 0;
    // Model.cpp:4639-4642
    if (int st = put_host(s, MIMIR_DTYPE_F32, "x", x0, n0)) return st;
    Slot xs = s->f32.at("x");
    s->bind(MIMIR_DTYPE_F32, "__input__", xs.buf, xs.n);
    // Model.cpp:4645-4664: int inputs; "seq" also as text_ids / __input__ / x.
    for (int32_t i = 0; i < ni; ++i) {
        MIMIR_REQUIRE(s->ctx, inames[i] && isizes[i] >= 0, "mimir_store_set_inputs: bad int input %d", i);
        if (int st = put_host(s, MIMIR_DTYPE_I32, inames[i], idata[i], isizes[i])) return st;
    }
    auto seq = s->i32.find("seq");
    if (seq != s->i32.end()) {
        const Slot q = seq->second;
        for (const char* alias : {"text_ids", "__input__", "x"}) s->bind(MIMIR_DTYPE_I32, alias, q.buf, q.n);
    }
    // Model.cpp:4665-4668: every float input (overwrites "x" with itself).
    for (int32_t i = 0; i < nf; ++i) {
        MIMIR_REQUIRE(s->ctx, fnames[i] && fsizes[i] >= 0, "mimir_store_set_inputs: bad float input %d", i);
        if (i == xi) {
            if (std::string(fnames[i]) != "x") s->bind(MIMIR_DTYPE_F32, fnames[i], xs.buf, xs.n);
            continue;
        }
        if (int st = put_host(s, MIMIR_DTYPE_F32, fnames[i], fdata[i], fsizes[i])) return st;
    }
    return MIMIR_OK;
}

int mimir_store_run(mimir_store* s, const mimir_layer* layers, int32_t n_layers) {
    if (!s) return MIMIR_EINVAL;
    MIMIR_REQUIRE(s->ctx, n_layers >= 0 && (n_layers == 0 || layers), "mimir_store_run: invalid argument");
    for (int32_t i = 0; i < n_layers; ++i)
        if (int st = run_layer(s, layers[i])) return st;
    return MIMIR_OK;
}

}  // extern "C"
