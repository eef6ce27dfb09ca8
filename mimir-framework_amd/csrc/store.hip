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
//
// Training (mimir_store_run_training + mimir_store_backward) mirrors
// forwardPassView(training=true) and Model::backwardPass (Model.cpp:
// 7307-9153): the forward keeps each layer's input buffers by reference
// (nothing is copied: no buffer is ever written in place), and the backward
// routes gradients through a name -> buffer map with accumulate_grad's
// copy-or-add, calling the backward kernels (backward.hip) for each branch.
#include "common.hpp"
#include "internal.hpp"

#include <algorithm>
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

// A layer's inputs as a training forward saw them (forwardPassView's
// layer_inputs_multi / layer_input_sizes_multi, Model.cpp:4858-4878): the
// buffers are held by reference (the store never writes one in place).
struct Snap {
    std::vector<Slot> vals;    // empty for Add / Identity (sizes only, :4757-4766)
    std::vector<bool> ids_i32;  // Embedding ids read from the int store
    std::vector<int64_t> sizes;
};

struct mimir_store {
    mimir_ctx* ctx = nullptr;
    std::unordered_map<std::string, Slot> f32;
    std::unordered_map<std::string, Slot> i32;
    std::vector<Snap> snaps;                      // last mimir_store_run_training
    // The outputs of that run's layers that a residual merge reads
    // (forwardPassView's all_layer_outputs, Model.cpp:4734-4737, 6676-6678):
    // held by reference, as the snapshots are; empty slots elsewhere.
    std::vector<Slot> outs;
    std::unordered_map<std::string, Slot> grads;  // last mimir_store_backward
    std::vector<std::unique_ptr<Buf>> bufs;
    std::multimap<size_t, Buf*> free_bufs;  // capacity -> idle buffer
    // While a run is captured (mimir_store_capture): every buffer it acquires.
    std::vector<Buf*>* capture_log = nullptr;
    int fuse = 0;  // mimir_store_set_fusion
    std::vector<mimir_store_graph*> graphs;  // alive captured graphs

    std::unordered_map<std::string, Slot>& map(int dtype) { return dtype == MIMIR_DTYPE_I32 ? i32 : f32; }

    // An idle buffer of at least `bytes` (best fit), or a new one.
    int acquire(size_t bytes, Buf** out) {
        bytes = (bytes + 255) & ~size_t(255);
        if (bytes == 0) bytes = 256;
        auto it = free_bufs.lower_bound(bytes);
        if (it != free_bufs.end() && it->first <= 2 * bytes) {
            *out = it->second;
            free_bufs.erase(it);
            if (capture_log) capture_log->push_back(*out);
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
        if (capture_log) capture_log->push_back(b);
        return MIMIR_OK;
    }

    // Take an idle buffer out of the pool (it is about to be held).
    void unpool(Buf* b) {
        auto r = free_bufs.equal_range(b->cap);
        for (auto it = r.first; it != r.second; ++it)
            if (it->second == b) {
                free_bufs.erase(it);
                return;
            }
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

    void release_snaps() {
        for (auto& sn : snaps)
            for (auto& v : sn.vals) release(v.buf);
        snaps.clear();
        for (auto& o : outs) release(o.buf);
        outs.clear();
    }

    void release_grads() {
        for (auto& kv : grads) release(kv.second.buf);
        grads.clear();
    }

    void clear() {
        for (auto& kv : f32) release(kv.second.buf);
        for (auto& kv : i32) release(kv.second.buf);
        f32.clear();
        i32.clear();
        release_snaps();
        release_grads();
    }
};

// A captured mimir_store_run (mimir_store_capture).  Its kernels hold the
// device addresses of the buffers the run used, so the graph holds a
// reference on each of them (the pool never hands them out while it lives),
// and it keeps its own name -> buffer maps: `in`, the tensors bound when it
// was captured (what set_input writes), and `out`, the bindings after the
// run (what get reads).  Index 0: float tensors, 1: int tensors.
struct mimir_store_graph {
    mimir_store* store = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    std::vector<Buf*> held;
    std::unordered_map<std::string, Slot> in[2], out[2];
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

const char* type_name(int32_t t) {
    switch (t) {
        case MIMIR_LAYER_LAYERNORM: return "LayerNorm";
        case MIMIR_LAYER_RMSNORM: return "RMSNorm";
        case MIMIR_LAYER_SOFTMAX: return "Softmax";
        case MIMIR_LAYER_LOGSOFTMAX: return "LogSoftmax";
        case MIMIR_LAYER_GELU: return "GELU";
        case MIMIR_LAYER_SILU: return "SiLU";
        case MIMIR_LAYER_ADD: return "Add";
        case MIMIR_LAYER_MULTIPLY: return "Multiply";
        case MIMIR_LAYER_EMBEDDING: return "Embedding";
        case MIMIR_LAYER_IDENTITY: return "Identity";
        case MIMIR_LAYER_DROPOUT: return "Dropout";
        case MIMIR_LAYER_SELF_ATTENTION: return "SelfAttention";
        case MIMIR_LAYER_MULTIHEAD_ATTENTION: return "MultiHeadAttention";
        case MIMIR_LAYER_CROSS_ATTENTION: return "CrossAttention";
        default: return "?";
    }
}

// One layer of Model::forwardPassView's loop (Model.cpp:4795-6680); with
// `snap`, the training form that keeps the layer's inputs.  `ids_path`: the
// loop of the int-ids forward instead (Model.cpp:1143-1346), whose routing
// and layer switch are narrower (see mimir_store_run_ids).
int run_layer(mimir_store* s, const mimir_layer& L, Snap* snap, bool ids_path = false) {
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
        Buf* buf;
    };
    std::vector<In> in;
    in.reserve(n_in);
    // The int path's Embedding reads only its first input, from the int store
    // ("Int tensor not found", Model.cpp:1148 -> :936-948); every other layer
    // reads float inputs ("Tensor not found", :1214-1215 -> :918-930), with no
    // int fallback.
    const int n_read = (ids_path && L.type == MIMIR_LAYER_EMBEDDING) ? 1 : n_in;
    for (int k = 0; k < n_read; ++k) {
        const std::string name = names[k] ? names[k] : "";
        if (ids_path) {
            if (L.type == MIMIR_LAYER_EMBEDDING) {
                auto iti = s->i32.find(name);
                if (iti == s->i32.end())
                    return fail(ctx, MIMIR_EINVAL, "Int tensor not found: %s (layer %s)", name.c_str(), layer_name(L));
                in.push_back(In{iti->second.buf->p, iti->second.n, true, iti->second.buf});
            } else {
                auto itf = s->f32.find(name);
                if (itf == s->f32.end())
                    return fail(ctx, MIMIR_EINVAL, "Tensor not found: %s (layer %s)", name.c_str(), layer_name(L));
                in.push_back(In{itf->second.buf->p, itf->second.n, false, itf->second.buf});
            }
            continue;
        }
        auto itf = s->f32.find(name);
        if (itf != s->f32.end()) {
            in.push_back(In{itf->second.buf->p, itf->second.n, false, itf->second.buf});
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
            in.push_back(In{iti->second.buf->p, iti->second.n, true, iti->second.buf});
            continue;
        }
        return fail(ctx, MIMIR_EINVAL, "Missing input tensor: %s (layer %s)", name.c_str(), layer_name(L));
    }
    const int64_t N = in[0].n;
    const float* x = static_cast<const float*>(in[0].p);

    if (snap) {  // Model.cpp:4858-4878
        if (L.type == MIMIR_LAYER_DROPOUT)
            return fail(ctx, MIMIR_EINVAL, "Dropout (layer %s): its training form draws a random mask, which is "
                        "not on this path", layer_name(L));
        for (const In& v : in) snap->sizes.push_back(v.n);
        if (L.type != MIMIR_LAYER_ADD && L.type != MIMIR_LAYER_IDENTITY) {
            for (const In& v : in) {
                ++v.buf->refs;
                snap->vals.push_back(Slot{v.buf, v.n});
                snap->ids_i32.push_back(v.ids_i32);
            }
        }
    }

    if (ids_path) {  // the int path's reduced switch, Model.cpp:1242-1321 (strict mode)
        switch (L.type) {
            case MIMIR_LAYER_RMSNORM:
            case MIMIR_LAYER_SILU:
            case MIMIR_LAYER_MULTIPLY:
            case MIMIR_LAYER_IDENTITY:
            case MIMIR_LAYER_CROSS_ATTENTION:
                return fail(ctx, MIMIR_EINVAL, "forwardPass(int): layer type not supported in int path: %s (layer %s)",
                            type_name(L.type), layer_name(L));
            case MIMIR_LAYER_ADD:  // :1285
                if (n_in < 2) return fail(ctx, MIMIR_EINVAL, "Add requires 2 inputs (layer %s)", layer_name(L));
                break;
            default:
                break;
        }
    }

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
        case MIMIR_LAYER_SELF_ATTENTION:
        case MIMIR_LAYER_MULTIHEAD_ATTENTION: {  // Model.cpp:5904-5934 (int path :1291-1310)
            if (!L.weights || L.weights_len <= 0)
                return fail(ctx, MIMIR_EINVAL, "Attention: weights not initialized. Call allocateParams() first. "
                            "(layer %s)", layer_name(L));
            const int64_t seq = L.seq_len > 0 ? L.seq_len : 1;
            const int64_t e = L.embed_dim > 0 ? L.embed_dim : N;
            const int64_t heads = L.num_heads > 0 ? L.num_heads : 1;
            if (e <= 0 || e % heads != 0)  // LayerOps.hpp:1013-1015
                return fail(ctx, MIMIR_EINVAL, "SelfAttention: embed_dim must be divisible by num_heads (layer %s)",
                            layer_name(L));
            if (N != seq * e)  // :1021-1023
                return fail(ctx, MIMIR_EINVAL, "SelfAttention: input size mismatch (layer %s)", layer_name(L));
            out_n = seq * e;
            break;
        }
        case MIMIR_LAYER_CROSS_ATTENTION: {  // Model.cpp:5936-5990
            if (n_in < 2)
                return fail(ctx, MIMIR_EINVAL, "CrossAttention requires 2 inputs (query, key_value), got %d", n_in);
            if (!L.weights || L.weights_len <= 0)
                return fail(ctx, MIMIR_EINVAL, "CrossAttention: weights not initialized. Call allocateParams() "
                            "first. (layer %s)", layer_name(L));
            const int64_t heads = L.num_heads > 0 ? L.num_heads : 1;
            int64_t e = L.embed_dim;
            if (e <= 0 && L.head_dim > 0) e = static_cast<int64_t>(L.head_dim) * heads;
            if (e <= 0)
                return fail(ctx, MIMIR_EINVAL, "CrossAttention: embed_dim must be configured (set layer.embed_dim "
                            "or head_dim*num_heads) (layer %s)", layer_name(L));
            if (in[0].n % e != 0)
                return fail(ctx, MIMIR_EINVAL, "CrossAttention: query input size must be divisible by embed_dim "
                            "(layer %s)", layer_name(L));
            if (in[1].n % e != 0)
                return fail(ctx, MIMIR_EINVAL, "CrossAttention: key/value input size must be divisible by "
                            "embed_dim (layer %s)", layer_name(L));
            if (in[0].n == 0 || in[1].n == 0)
                return fail(ctx, MIMIR_EINVAL, "CrossAttention: invalid sequence lengths (layer %s)", layer_name(L));
            out_n = in[0].n;
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
            // The int path gathers the ids as ints (Model.cpp:1194-1203); the
            // float path reads int-store ids through a float cast.
            st = embedding_launch(ctx, in[0].p, ids_path ? kIdsI32 : in[0].ids_i32 ? kIdsI32AsF32 : kIdsF32, N,
                                  L.weights, L.weights_len, L.vocab_size, L.embed_dim, L.padding_idx, y);
            break;
        case MIMIR_LAYER_SELF_ATTENTION:
        case MIMIR_LAYER_MULTIHEAD_ATTENTION: {
            const int64_t seq = L.seq_len > 0 ? L.seq_len : 1;
            const int64_t e = L.embed_dim > 0 ? L.embed_dim : N;
            st = mimir_self_attention_fwd(ctx, x, seq, e, L.num_heads > 0 ? L.num_heads : 1, L.causal, L.weights,
                                          L.weights_len, y);
            break;
        }
        case MIMIR_LAYER_CROSS_ATTENTION: {
            const int64_t heads = L.num_heads > 0 ? L.num_heads : 1;
            const int64_t e = L.embed_dim > 0 ? L.embed_dim : static_cast<int64_t>(L.head_dim) * heads;
            st = mimir_cross_attention_fwd(ctx, x, in[0].n / e, static_cast<const float*>(in[1].p), in[1].n / e, e,
                                           heads, L.causal, L.weights, L.weights_len, y);
            break;
        }
    }
    if (st != MIMIR_OK) {
        s->discard(ob);
        return st;
    }
    s->bind(MIMIR_DTYPE_F32, out_name, ob, out_n);  // STORE OUTPUT, Model.cpp:6655,6674
    return MIMIR_OK;
}

// Every layer but the last stores its output through the caches, where the
// layer after it (the usual reader) finds much of it in L2 / the Infinity
// Cache; the last layer's output is streamed, and the context's own setting
// (mimir_ctx_set_output_caching) is restored on the way out.
struct ChainOutputs {
    mimir_ctx* ctx;
    int saved;
    explicit ChainOutputs(mimir_ctx* c) : ctx(c), saved(c->keep_outputs) {}
    void layer(int32_t i, int32_t n) { ctx->keep_outputs = i + 1 < n && !ctx->tune.chain_streamed ? 1 : saved; }
    ~ChainOutputs() { ctx->keep_outputs = saved; }
};

// Inference fusion (mimir_store_set_fusion): a run of consecutive
// elementwise layers -- GELU, SiLU, and Add / Multiply of equal sizes --
// each reading the previous one's output, runs as one kernel (fused_chain).
// The second operand of an Add / Multiply must be a tensor bound when the
// chain starts (not written inside it).  An intermediate output is written
// only when a layer after the chain reads its name, or it is "x"; the others
// are never materialised and their names are left unbound.  Values are the
// unfused layers' bits (the same per-element functions, a + b = b + a).
bool chain_type(int32_t t) {
    return t == MIMIR_LAYER_GELU || t == MIMIR_LAYER_SILU || t == MIMIR_LAYER_ADD || t == MIMIR_LAYER_MULTIPLY;
}

std::string input_name(const mimir_layer& L, int k) {
    if (L.n_inputs <= 0) return k == 0 ? "x" : "";
    return k < L.n_inputs && L.inputs[k] ? L.inputs[k] : "";
}

std::string output_name(const mimir_layer& L) { return (L.output && *L.output) ? L.output : "x"; }

// Extend a chain from layer j: consecutive elementwise layers each reading
// the previous output (written.back()), the second operand of an Add /
// Multiply bound in the store and not written by the group, all of n
// floats.  Appends their steps to p (operands into p.ins) and their output
// names to `written`; returns the first layer not taken.
int32_t extend_chain(mimir_store* s, const mimir_layer* layers, int32_t j, int32_t n_layers, int64_t n,
                     FuseProgram& p, std::vector<std::string>& written) {
    auto kind_of = [](int32_t t) {
        return t == MIMIR_LAYER_GELU ? kFuseGelu : t == MIMIR_LAYER_SILU ? kFuseSilu
               : t == MIMIR_LAYER_ADD ? kFuseAdd : kFuseMul;
    };
    for (; j < n_layers && p.n_steps < kFuseMax; ++j) {
        const mimir_layer& M = layers[j];
        if (!chain_type(M.type)) break;
        const std::string& cur = written.back();
        FuseStep st{kind_of(M.type), -1, -1};
        if (M.type == MIMIR_LAYER_GELU || M.type == MIMIR_LAYER_SILU) {
            if (input_name(M, 0) != cur) break;
        } else {
            if (M.n_inputs < 2) break;
            const std::string n0 = input_name(M, 0), n1 = input_name(M, 1);
            if (!(n0 == cur && n1 == cur)) {
                const std::string other = n0 == cur ? n1 : n1 == cur ? n0 : std::string();
                if (other.empty() || p.n_ins >= kFuseMax) break;
                if (std::find(written.begin(), written.end(), other) != written.end()) break;
                auto it = s->f32.find(other);
                if (it == s->f32.end() || it->second.n != n) break;
                st.operand = p.n_ins;
                p.ins[p.n_ins++] = static_cast<const float*>(it->second.buf->p);
            }
        }
        p.steps[p.n_steps++] = st;
        written.push_back(output_name(M));
    }
    return j;
}

// Whether output k of a fused group is written: the group's last; one a
// layer after the group reads; "x" when the group does not write "x" again.
bool materialise(const mimir_layer* layers, int32_t after, int32_t n_layers, const std::vector<std::string>& written,
                 size_t k) {
    const std::string& nm = written[k];
    if (k + 1 == written.size()) return true;
    for (int32_t q = after; q < n_layers; ++q) {
        const mimir_layer& L = layers[q];
        const int ni = L.n_inputs > 0 ? L.n_inputs : 1;
        for (int t = 0; t < ni; ++t)
            if (input_name(L, t) == nm) return true;
    }
    return nm == "x" && std::find(written.begin() + static_cast<long>(k) + 1, written.end(), nm) == written.end();
}

// Bind a fused group's outputs in layer order (a name written twice ends on
// its last value); an output not materialised is unbound.
void bind_group(mimir_store* s, const std::vector<std::string>& written, const std::vector<Buf*>& bufs, int64_t n) {
    for (size_t k = 0; k < written.size(); ++k) {
        if (Buf* b = bufs[k]) {
            s->bind(MIMIR_DTYPE_F32, written[k], b, n);
        } else {
            auto it = s->f32.find(written[k]);
            if (it != s->f32.end()) {
                s->release(it->second.buf);
                s->f32.erase(it);
            }
        }
    }
}

int run_fused_chain(mimir_store* s, const mimir_layer* layers, int32_t i, int32_t n_layers, int32_t* end,
                    ChainOutputs& chain) {
    *end = i;
    const mimir_layer& H = layers[i];
    if (!chain_type(H.type)) return MIMIR_OK;
    const bool bin = H.type == MIMIR_LAYER_ADD || H.type == MIMIR_LAYER_MULTIPLY;
    if (bin && H.n_inputs < 2) return MIMIR_OK;
    auto a = s->f32.find(input_name(H, 0));
    if (a == s->f32.end() || a->second.n == 0) return MIMIR_OK;
    const int64_t n = a->second.n;
    FuseProgram p{};
    p.ins[p.n_ins++] = static_cast<const float*>(a->second.buf->p);
    FuseStep head{H.type == MIMIR_LAYER_GELU ? kFuseGelu : H.type == MIMIR_LAYER_SILU ? kFuseSilu
                  : H.type == MIMIR_LAYER_ADD ? kFuseAdd : kFuseMul, -1, -1};
    if (bin) {  // v = in0, then v op in1
        auto b = s->f32.find(input_name(H, 1));
        if (b == s->f32.end() || b->second.n != n) return MIMIR_OK;
        head.operand = p.n_ins;
        p.ins[p.n_ins++] = static_cast<const float*>(b->second.buf->p);
    }
    p.steps[p.n_steps++] = head;
    std::vector<std::string> written{output_name(H)};
    const int32_t j = extend_chain(s, layers, i + 1, n_layers, n, p, written);
    if (written.size() < 2) return MIMIR_OK;
    std::vector<Buf*> bufs(written.size(), nullptr);
    for (size_t k = 0; k < written.size(); ++k) {
        if (!materialise(layers, j, n_layers, written, k)) continue;
        if (int st = s->acquire(static_cast<size_t>(n) * 4, &bufs[k])) {
            for (Buf* b : bufs) s->discard(b);
            return st;
        }
        p.steps[k].store = p.n_outs;
        p.outs[p.n_outs++] = static_cast<float*>(bufs[k]->p);
    }
    chain.layer(j - 1, n_layers);  // a layer after the chain reads its output
    if (int st = fused_chain(s->ctx, p, n)) {
        for (Buf* b : bufs) s->discard(b);
        return st;
    }
    bind_group(s, written, bufs, n);
    *end = j;
    return MIMIR_OK;
}

// The fused LayerNorm group: [Add ->] LayerNorm [-> elementwise chain], one
// kernel (norm.hip layernorm_fused).  The Add (equal sizes) must feed the
// LayerNorm; a LayerNorm with neither an Add before nor a chain after runs
// unfused.  Checks the LayerNorm layer as run_layer does and leaves any
// group it would refuse to the unfused path (which reports the error).
int run_fused_norm(mimir_store* s, const mimir_layer* layers, int32_t i, int32_t n_layers, int32_t* end,
                   ChainOutputs& chain) {
    *end = i;
    auto find = [&](const std::string& nm) -> const Slot* {
        auto it = s->f32.find(nm);
        return it == s->f32.end() ? nullptr : &it->second;
    };
    const mimir_layer& A = layers[i];
    const Slot* xin = nullptr;
    const Slot* rin = nullptr;
    int32_t ln = i;
    std::vector<std::string> written;
    if (A.type == MIMIR_LAYER_ADD) {
        if (i + 1 >= n_layers || A.n_inputs < 2) return MIMIR_OK;
        const mimir_layer& L = layers[i + 1];
        if (L.type != MIMIR_LAYER_LAYERNORM || input_name(L, 0) != output_name(A)) return MIMIR_OK;
        xin = find(input_name(A, 0));
        rin = find(input_name(A, 1));
        if (!xin || !rin || xin->n != rin->n) return MIMIR_OK;
        ln = i + 1;
        written.push_back(output_name(A));
    } else if (A.type == MIMIR_LAYER_LAYERNORM) {
        xin = find(input_name(A, 0));
        if (!xin) return MIMIR_OK;
    } else {
        return MIMIR_OK;
    }
    const mimir_layer& L = layers[ln];
    const int64_t N = xin->n;
    if (N == 0) return MIMIR_OK;
    const int64_t nrm = L.in_features > 0 ? L.in_features : N;  // LayerOps.hpp:276-285
    if (nrm <= 0 || N % nrm != 0) return MIMIR_OK;
    const float* gamma = (L.affine && L.weights && L.weights_len > 0) ? L.weights : nullptr;
    const float* beta = (gamma && L.use_bias) ? L.weights + nrm : nullptr;
    if (gamma && L.weights_len < (beta ? 2 * nrm : nrm)) return MIMIR_OK;
    if (!layernorm_fusable(s->ctx, nrm, gamma, beta)) return MIMIR_OK;
    written.push_back(output_name(L));
    const size_t first_epi = written.size();
    LnFused f{};
    const int32_t j = extend_chain(s, layers, ln + 1, n_layers, N, f.epi, written);
    if (!rin && f.epi.n_steps == 0) return MIMIR_OK;  // a LayerNorm alone: the unfused kernel
    std::vector<Buf*> bufs(written.size(), nullptr);
    for (size_t k = 0; k < written.size(); ++k) {
        if (!materialise(layers, j, n_layers, written, k)) continue;
        if (int st = s->acquire(static_cast<size_t>(N) * 4, &bufs[k])) {
            for (Buf* b : bufs) s->discard(b);
            return st;
        }
        float* out = static_cast<float*>(bufs[k]->p);
        if (rin && k == 0) f.h = out;
        else if (k + 1 == first_epi) f.y = out;
        else {
            f.epi.steps[k - first_epi].store = f.epi.n_outs;
            f.epi.outs[f.epi.n_outs++] = out;
        }
    }
    f.x = static_cast<const float*>(xin->buf->p);
    f.r = rin ? static_cast<const float*>(rin->buf->p) : nullptr;
    f.g = gamma;
    f.b = beta;
    f.rows = N / nrm;
    f.cols = nrm;
    f.eps = L.eps;
    chain.layer(j - 1, n_layers);
    if (int st = layernorm_fused(s->ctx, f)) {
        for (Buf* b : bufs) s->discard(b);
        return st;
    }
    bind_group(s, written, bufs, N);
    *end = j;
    return MIMIR_OK;
}

// accumulate_grad's destination (Model.cpp:7329-7341): the gradient of
// `name`, present (acc: add onto it) or new (written by the first
// contribution).  A present gradient of another size is the reference's
// "Gradient accumulate: size mismatch".
int grad_dst(mimir_store* s, const std::string& name, int64_t n, float** out, int* acc) {
    auto it = s->grads.find(name);
    if (it != s->grads.end() && it->second.n > 0) {
        if (it->second.n != n)
            return fail(s->ctx, MIMIR_EINVAL, "Gradient accumulate: size mismatch (%s: %lld vs %lld)", name.c_str(),
                        (long long)it->second.n, (long long)n);
        *out = static_cast<float*>(it->second.buf->p);
        *acc = 1;
        return MIMIR_OK;
    }
    Buf* b = nullptr;
    if (int st = s->acquire(static_cast<size_t>(n) * 4, &b)) return st;
    ++b->refs;
    if (it != s->grads.end()) {
        s->release(it->second.buf);
        it->second = Slot{b, n};
    } else {
        s->grads.emplace(name, Slot{b, n});
    }
    *out = static_cast<float*>(b->p);
    *acc = 0;
    return MIMIR_OK;
}

// accumulate_grad(grad_store[name], g) for a whole gradient g (Identity, the
// pass-through fallback); when name's gradient is g itself it doubles, as the
// reference's in-place add of a vector onto itself does.
int grad_pass(mimir_store* s, const std::string& name, const float* g, int64_t n) {
    float* d = nullptr;
    int acc = 0;
    if (int st = grad_dst(s, name, n, &d, &acc)) return st;
    return mimir_add_bwd(s->ctx, g, n, n, d, nullptr, acc, 0);
}

// One layer of Model::backwardPass (Model.cpp:7349-9141).
int backward_layer(mimir_store* s, const mimir_layer& L, const Snap& sn) {
    mimir_ctx* ctx = s->ctx;
    const std::string out_name = (L.output && *L.output) ? L.output : "x";
    auto it = s->grads.find(out_name);
    if (it == s->grads.end()) return MIMIR_OK;  // :7352-7356
    const Slot go = it->second;
    const float* g = static_cast<const float*>(go.buf->p);
    const int64_t gn = go.n;
    if (gn == 0) return MIMIR_OK;
    static const char* const kDefaultInput[] = {"x"};
    const char* const* names = L.n_inputs > 0 ? L.inputs : kDefaultInput;
    auto nm = [&](int k) { return std::string(names[k] ? names[k] : ""); };
    const int64_t n0 = sn.sizes.empty() ? 0 : sn.sizes[0];
    float* d0 = nullptr;
    float* d1 = nullptr;
    int a0 = 0, a1 = 0;
    switch (L.type) {
        case MIMIR_LAYER_EMBEDDING: {  // :7429-7461
            if (sn.vals.empty()) return MIMIR_OK;
            const int64_t vocab = L.vocab_size > 1 ? L.vocab_size : 1;
            const int64_t dim = L.embed_dim > 1 ? L.embed_dim : 1;
            const Slot& ids = sn.vals[0];
            if (gn != ids.n * dim) return MIMIR_OK;                               // shape mismatch: skipped
            if (!L.weights || L.weights_len < vocab * dim) return MIMIR_OK;       // weights invalid: skipped
            if (!L.grad_weights) return MIMIR_OK;
            return embedding_bwd_launch(ctx, ids.buf->p, sn.ids_i32[0] ? kIdsI32AsF32 : kIdsF32, ids.n, g,
                                        L.grad_weights, L.weights_len, L.vocab_size, L.embed_dim, L.padding_idx);
        }
        case MIMIR_LAYER_IDENTITY:  // :7463-7468
            if (gn != n0) return MIMIR_OK;
            return grad_pass(s, nm(0), g, gn);
        case MIMIR_LAYER_ADD: {  // :7541-7601
            if (sn.sizes.size() < 2 || L.n_inputs < 2) return MIMIR_OK;
            const int64_t n1 = sn.sizes[1];
            if (gn == n0 && gn == n1) {
                if (int st = grad_dst(s, nm(0), gn, &d0, &a0)) return st;
                if (int st = grad_dst(s, nm(1), gn, &d1, &a1)) return st;
                return mimir_add_bwd(ctx, g, gn, gn, d0, d1, a0, a1);
            }
            if (gn != n0 && gn != n1) return MIMIR_OK;
            const int big = gn == n0 ? 0 : 1;
            const int64_t small_n = big == 0 ? n1 : n0;
            if (int st = grad_dst(s, nm(big), gn, &d0, &a0)) return st;
            if (!(small_n == 1 || (small_n > 1 && gn % small_n == 0)))  // :7595-7599, after the big one's gradient
                return mimir_add_bwd(ctx, g, gn, gn, d0, nullptr, a0, 0);
            if (int st = grad_dst(s, nm(1 - big), small_n, &d1, &a1)) return st;
            return big == 0 ? mimir_add_bwd(ctx, g, gn, small_n, d0, d1, a0, a1)
                            : mimir_add_bwd(ctx, g, small_n, gn, d1, d0, a1, a0);
        }
        case MIMIR_LAYER_MULTIPLY: {  // :7647-7665
            if (sn.vals.size() < 2) return MIMIR_OK;
            if (gn != sn.vals[0].n || gn != sn.vals[1].n) return MIMIR_OK;
            if (int st = grad_dst(s, nm(0), gn, &d0, &a0)) return st;
            if (int st = grad_dst(s, nm(1), gn, &d1, &a1)) return st;
            return mimir_mul_bwd(ctx, static_cast<const float*>(sn.vals[0].buf->p),
                                 static_cast<const float*>(sn.vals[1].buf->p), g, d0, d1, gn, a0, a1);
        }
        case MIMIR_LAYER_LAYERNORM: {  // :7719-7821
            if (sn.vals.empty()) return MIMIR_OK;
            const Slot& x = sn.vals[0];
            if (gn != x.n) return MIMIR_OK;
            const int64_t N = x.n;
            const int64_t feat = L.in_features > 0 ? L.in_features : N;
            if (feat <= 0 || N % feat != 0) return MIMIR_OK;
            const bool affine = L.affine != 0;
            const bool has_bias = affine && L.use_bias;
            if (affine && (!L.weights || L.weights_len < feat * (has_bias ? 2 : 1))) return MIMIR_OK;
            if (int st = grad_dst(s, nm(0), N, &d0, &a0)) return st;
            float* dg = (affine && L.grad_weights) ? L.grad_weights : nullptr;
            float* db = (has_bias && dg) ? L.grad_weights + feat : nullptr;
            return mimir_layernorm_bwd(ctx, static_cast<const float*>(x.buf->p), g, affine ? L.weights : nullptr, d0,
                                       dg, db, N / feat, feat, L.eps, a0);
        }
        case MIMIR_LAYER_GELU:  // :9026-9051
        case MIMIR_LAYER_SILU: {  // :7993-8032
            if (sn.vals.empty() || gn != sn.vals[0].n) return MIMIR_OK;
            if (int st = grad_dst(s, nm(0), gn, &d0, &a0)) return st;
            const float* x = static_cast<const float*>(sn.vals[0].buf->p);
            return L.type == MIMIR_LAYER_GELU ? mimir_gelu_bwd(ctx, x, g, d0, gn, a0)
                                              : mimir_silu_bwd(ctx, x, g, d0, gn, a0);
        }
        case MIMIR_LAYER_SELF_ATTENTION:
        case MIMIR_LAYER_MULTIHEAD_ATTENTION: {  // :8034-8072 -> backward_self_attention (:6847-7062)
            if (sn.vals.empty()) return MIMIR_OK;
            const Slot& x = sn.vals[0];
            const int64_t seq = L.seq_len > 0 ? L.seq_len : 1;
            const int64_t e = L.embed_dim > 0 ? L.embed_dim : (x.n % seq == 0 ? x.n / seq : x.n);
            const int64_t heads = L.num_heads > 1 ? L.num_heads : 1;
            if (!L.weights || L.weights_len < 4 * e * e) return MIMIR_OK;  // "weights invalid": skipped
            // backward_self_attention's own refusals (:6860-6863): "failed", skipped
            if (e <= 0 || e % heads != 0 || x.n != seq * e || gn != seq * e) return MIMIR_OK;
            if (int st = grad_dst(s, nm(0), x.n, &d0, &a0)) return st;
            return mimir_self_attention_bwd(ctx, static_cast<const float*>(x.buf->p), g, seq, e, heads, L.causal,
                                            L.weights, L.weights_len, L.grad_weights, d0, a0);
        }
        case MIMIR_LAYER_CROSS_ATTENTION: {  // :8074-8130 -> backward_cross_attention (:7068-7300)
            if (sn.vals.size() < 2) return MIMIR_OK;  // "need 2 inputs": skipped
            const Slot& xq = sn.vals[0];
            const Slot& xkv = sn.vals[1];
            const int64_t heads = L.num_heads > 1 ? L.num_heads : 1;
            int64_t e = L.embed_dim;
            if (e <= 0 && L.head_dim > 0) e = static_cast<int64_t>(L.head_dim) * heads;
            if (e <= 0 || e % heads != 0) return MIMIR_OK;          // "invalid embed_dim": skipped
            if (xq.n % e != 0 || xkv.n % e != 0) return MIMIR_OK;   // "input size mismatch": skipped
            const int64_t lq = xq.n / e, lk = xkv.n / e;
            if (gn != lq * e) return MIMIR_OK;                      // "grad size mismatch": skipped
            if (!L.weights || L.weights_len < 4 * e * e) return MIMIR_OK;
            if (lq <= 0 || lk <= 0) return MIMIR_OK;                // backward_cross_attention's refusal
            if (int st = grad_dst(s, nm(0), xq.n, &d0, &a0)) return st;
            if (int st = grad_dst(s, nm(1), xkv.n, &d1, &a1)) return st;
            return mimir_cross_attention_bwd(ctx, static_cast<const float*>(xq.buf->p), lq,
                                             static_cast<const float*>(xkv.buf->p), lk, g, e, heads, L.causal,
                                             L.weights, L.weights_len, L.grad_weights, d0, a0, d1, a1);
        }
        default:  // RMSNorm, Softmax, LogSoftmax: the fallback at :9133-9140
            if (gn != n0) return MIMIR_OK;
            return grad_pass(s, nm(0), g, gn);
    }
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
    while (!s->graphs.empty()) {
        const int r = mimir_store_graph_destroy(s->graphs.back());
        if (r != MIMIR_OK && st == MIMIR_OK) st = r;
    }
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
    s->release_snaps();
    ChainOutputs chain(s->ctx);
    for (int32_t i = 0; i < n_layers;) {
        if (s->fuse) {
            int32_t end = i;
            if (int st = run_fused_norm(s, layers, i, n_layers, &end, chain)) return st;
            if (end == i)
                if (int st = run_fused_chain(s, layers, i, n_layers, &end, chain)) return st;
            if (end > i) {
                i = end;
                continue;
            }
        }
        chain.layer(i, n_layers);
        if (int st = run_layer(s, layers[i], nullptr)) return st;
        ++i;
    }
    return MIMIR_OK;
}

int mimir_store_set_fusion(mimir_store* s, int enable) {
    if (!s) return MIMIR_EINVAL;
    s->fuse = enable ? 1 : 0;
    return MIMIR_OK;
}

int mimir_store_set_input_ids(mimir_store* s, const int32_t* ids, int64_t n) {
    if (!s) return MIMIR_EINVAL;
    MIMIR_REQUIRE(s->ctx, n >= 0 && (n == 0 || ids), "mimir_store_set_input_ids: invalid argument");
    s->clear();  // Model.cpp:1046-1049
    if (int st = put_host(s, MIMIR_DTYPE_I32, "x", ids, n)) return st;
    const Slot xs = s->i32.at("x");
    s->bind(MIMIR_DTYPE_I32, "__input__", xs.buf, xs.n);
    return MIMIR_OK;
}

int mimir_store_run_ids(mimir_store* s, const mimir_layer* layers, int32_t n_layers, int training) {
    if (!s) return MIMIR_EINVAL;
    MIMIR_REQUIRE(s->ctx, n_layers >= 0 && (n_layers == 0 || layers), "mimir_store_run_ids: invalid argument");
    s->release_snaps();
    if (training) s->snaps.resize(static_cast<size_t>(n_layers));
    ChainOutputs chain(s->ctx);
    for (int32_t i = 0; i < n_layers; ++i) {
        chain.layer(i, n_layers);
        if (int st = run_layer(s, layers[i], training ? &s->snaps[i] : nullptr, true)) {
            s->release_snaps();
            return st;
        }
    }
    // Model.cpp:1348: the result is the float tensor "x" (no layers: an empty
    // result, :1033-1037).
    if (n_layers > 0 && s->f32.find("x") == s->f32.end()) {
        s->release_snaps();
        return fail(s->ctx, MIMIR_EINVAL, "Tensor not found: x");
    }
    return MIMIR_OK;
}

namespace {

// The source layer of layer i's residual merge, or -1 when the layer merges
// nothing: executeBranchComputation (Model.cpp:4550-4582) merges only for
// BranchType::RESIDUAL with a first branch source inside all_layer_outputs,
// which at layer i holds the outputs of layers 0..i.
int merge_source(const mimir_layer& L, int32_t i) {
    if (L.branch_type != MIMIR_BRANCH_RESIDUAL || L.n_branch_sources <= 0 || !L.branch_sources) return -1;
    const int32_t src = L.branch_sources[0];
    return src >= 0 && src <= i ? src : -1;
}

// After layer i of a training run: keep its output when a merge reads it,
// and merge it with its source's output when it is a residual layer
// (Model.cpp:6676-6685).  The merged tensor replaces the output under the
// same name, and is what a later merge reads as layer i's output.
int after_training_layer(mimir_store* s, const mimir_layer* layers, int32_t i, const std::vector<bool>& kept) {
    const mimir_layer& L = layers[i];
    const std::string out_name = (L.output && *L.output) ? L.output : "x";
    const Slot o = s->f32.at(out_name);
    const int src = merge_source(L, i);
    if (src >= 0) {
        const Slot b = src == i ? o : s->outs[src];
        const int64_t n = L.merge_op == MIMIR_MERGE_CONCATENATE ? o.n + b.n : o.n;
        Buf* mb = nullptr;
        if (int st = s->acquire(static_cast<size_t>(n) * 4, &mb)) return st;
        const int st = mimir_branch_merge_fwd(s->ctx, static_cast<const float*>(o.buf->p), o.n,
                                              static_cast<const float*>(b.buf->p), b.n,
                                              static_cast<float*>(mb->p), L.merge_op);
        if (st != MIMIR_OK) {
            s->discard(mb);
            return fail(s->ctx, st, "%s (layer %s, merged with layer %d)", mimir_last_error(s->ctx), layer_name(L),
                        src);
        }
        s->bind(MIMIR_DTYPE_F32, out_name, mb, n);
    }
    if (kept[i]) {
        const Slot m = s->f32.at(out_name);
        ++m.buf->refs;
        s->outs[i] = m;
    }
    return MIMIR_OK;
}

}  // namespace

int mimir_store_run_training(mimir_store* s, const mimir_layer* layers, int32_t n_layers) {
    if (!s) return MIMIR_EINVAL;
    MIMIR_REQUIRE(s->ctx, n_layers >= 0 && (n_layers == 0 || layers), "mimir_store_run_training: invalid argument");
    s->release_snaps();
    s->snaps.resize(static_cast<size_t>(n_layers));
    // Layers whose outputs a later (or their own) residual merge reads.
    std::vector<bool> kept(static_cast<size_t>(n_layers), false);
    bool merges = false;
    for (int32_t i = 0; i < n_layers; ++i) {
        const int src = merge_source(layers[i], i);
        if (src >= 0 && src < i) kept[src] = true;
        merges = merges || src >= 0;
    }
    if (merges) s->outs.resize(static_cast<size_t>(n_layers));
    ChainOutputs chain(s->ctx);
    for (int32_t i = 0; i < n_layers; ++i) {
        chain.layer(i, n_layers);
        int st = run_layer(s, layers[i], &s->snaps[i]);
        if (st == MIMIR_OK && merges) st = after_training_layer(s, layers, i, kept);
        if (st != MIMIR_OK) {
            s->release_snaps();
            return st;
        }
    }
    return MIMIR_OK;
}

namespace {

// Model::backwardPass with the loss gradient on the host (the reference's
// form) or already in device memory.
int store_backward(mimir_store* s, const mimir_layer* layers, int32_t n_layers, const float* loss_grad,
                   int64_t n_grad, bool device) {
    if (!s) return MIMIR_EINVAL;
    MIMIR_REQUIRE(s->ctx, n_layers >= 0 && (n_layers == 0 || layers) && n_grad >= 0 && (n_grad == 0 || loss_grad),
                  "mimir_store_backward: invalid argument");
    // Model.cpp:7313-7317: a backward needs the training forward's state.
    MIMIR_REQUIRE(s->ctx, static_cast<size_t>(n_layers) == s->snaps.size(),
                  "mimir_store_backward: no training forward of these %d layers (run_training first)", n_layers);
    s->release_grads();
    // Every layer's gradients but the first layer's (the model's input
    // gradients, read back by the caller) feed the backward of the layer
    // before it: they stay in the caches, as the forward's outputs do.
    ChainOutputs chain(s->ctx);
    chain.layer(0, n_layers + 1);
    Buf* b = nullptr;  // grad_store["x"] = loss_gradient (:7346)
    if (int st = s->acquire(static_cast<size_t>(n_grad) * 4, &b)) return st;
    if (n_grad > 0) {
        const size_t bytes = static_cast<size_t>(n_grad) * 4;
        const int st = device ? mimir_copy(s->ctx, b->p, loss_grad, bytes) : mimir_upload(s->ctx, b->p, loss_grad, bytes);
        if (st) {
            s->discard(b);
            return st;
        }
    }
    ++b->refs;
    s->grads.emplace("x", Slot{b, n_grad});
    for (int32_t i = n_layers - 1; i >= 0; --i) {
        chain.layer(n_layers - 1 - i, n_layers);
        if (int st = backward_layer(s, layers[i], s->snaps[i])) return st;
    }
    return MIMIR_OK;
}

}  // namespace

int mimir_store_backward(mimir_store* s, const mimir_layer* layers, int32_t n_layers, const float* loss_grad,
                         int64_t n_grad) {
    return store_backward(s, layers, n_layers, loss_grad, n_grad, false);
}

int mimir_store_backward_dev(mimir_store* s, const mimir_layer* layers, int32_t n_layers, const float* loss_grad,
                             int64_t n_grad) {
    return store_backward(s, layers, n_layers, loss_grad, n_grad, true);
}

int mimir_store_grad_info(mimir_store* s, const char* name, void** dptr, int64_t* n) {
    if (!s) return MIMIR_EINVAL;
    MIMIR_REQUIRE(s->ctx, name && dptr && n, "mimir_store_grad_info: invalid argument");
    auto it = s->grads.find(name);
    MIMIR_REQUIRE(s->ctx, it != s->grads.end(), "mimir_store_grad_info: no gradient reached %s", name);
    *dptr = it->second.buf->p;
    *n = it->second.n;
    return MIMIR_OK;
}

int mimir_store_grad_get(mimir_store* s, const char* name, float* host, int64_t cap, int64_t* n) {
    if (!s) return MIMIR_EINVAL;
    MIMIR_REQUIRE(s->ctx, name && n && cap >= 0, "mimir_store_grad_get: invalid argument");
    auto it = s->grads.find(name);
    MIMIR_REQUIRE(s->ctx, it != s->grads.end(), "mimir_store_grad_get: no gradient reached %s", name);
    *n = it->second.n;
    const int64_t k = cap < it->second.n ? cap : it->second.n;
    if (k > 0) {
        MIMIR_REQUIRE(s->ctx, host, "mimir_store_grad_get: null host buffer");
        return mimir_download(s->ctx, host, it->second.buf->p, static_cast<size_t>(k) * 4);
    }
    return MIMIR_OK;
}

int mimir_store_capture(mimir_store* s, const mimir_layer* layers, int32_t n_layers, mimir_store_graph** out) {
    if (!s || !out) return MIMIR_EINVAL;
    *out = nullptr;
    mimir_ctx* ctx = s->ctx;
    MIMIR_REQUIRE(ctx, n_layers >= 0 && (n_layers == 0 || layers), "mimir_store_capture: invalid argument");
    MIMIR_REQUIRE(ctx, ctx->stream != nullptr,
                  "mimir_store_capture: the context's stream is the null stream, which cannot be captured");
    MIMIR_ENTER(ctx);
    std::unique_ptr<mimir_store_graph> g(new (std::nothrow) mimir_store_graph());
    if (!g) return MIMIR_ENOMEM;
    g->store = s;
    // The inputs: the bindings now, each held by the graph from here on.
    g->in[0] = s->f32;
    g->in[1] = s->i32;
    for (auto& m : g->in)
        for (auto& kv : m) {
            Buf* b = kv.second.buf;
            if (b->refs++ == 0) s->unpool(b);  // (bound buffers are never pooled; for symmetry)
            if (std::find(g->held.begin(), g->held.end(), b) == g->held.end()) g->held.push_back(b);
            else --b->refs;
        }
    auto drop = [&]() {
        for (Buf* b : g->held) s->release(b);
        g->held.clear();
    };
    auto rebind_inputs = [&]() {
        for (int d = 0; d < 2; ++d) {
            auto& m = s->map(d == 0 ? MIMIR_DTYPE_F32 : MIMIR_DTYPE_I32);
            for (auto& kv : m) s->release(kv.second.buf);
            m.clear();
            for (auto& kv : g->in[d]) s->bind(d == 0 ? MIMIR_DTYPE_F32 : MIMIR_DTYPE_I32, kv.first, kv.second.buf,
                                              kv.second.n);
        }
    };
    // A first, eager run: every pool buffer, the scratch and the library
    // workspace the run needs then exist, so the captured run allocates
    // nothing.  The store never writes a buffer in place, so the inputs are
    // intact afterwards and are bound again.
    if (int st = mimir_store_run(s, layers, n_layers)) {
        drop();
        return st;
    }
    rebind_inputs();
    hipError_t e = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeRelaxed);
    if (e != hipSuccess) {
        drop();
        return hip_fail(ctx, e, "hipStreamBeginCapture");
    }
    std::vector<Buf*> log;
    s->capture_log = &log;
    const int st = mimir_store_run(s, layers, n_layers);
    s->capture_log = nullptr;
    hipGraph_t graph = nullptr;
    e = hipStreamEndCapture(ctx->stream, &graph);
    if (st != MIMIR_OK || e != hipSuccess) {
        if (graph) (void)hipGraphDestroy(graph);
        (void)hipGetLastError();
        drop();
        return st != MIMIR_OK ? st : hip_fail(ctx, e, "hipStreamEndCapture");
    }
    g->graph = graph;
    e = hipGraphInstantiate(&g->exec, graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(graph);
        drop();
        return hip_fail(ctx, e, "hipGraphInstantiate");
    }
    // Every buffer the captured run acquired, including intermediates it
    // released back to the pool (the graph writes them on each launch).
    for (Buf* b : log) {
        if (std::find(g->held.begin(), g->held.end(), b) != g->held.end()) continue;
        if (b->refs++ == 0) s->unpool(b);
        g->held.push_back(b);
    }
    g->out[0] = s->f32;
    g->out[1] = s->i32;
    graph_pin(ctx);
    s->graphs.push_back(g.get());
    mimir_store_graph* gp = g.release();
    // Compute what the outputs name now (the capture only recorded the run).
    if (int st2 = mimir_store_graph_launch(gp)) {
        (void)mimir_store_graph_destroy(gp);
        return st2;
    }
    *out = gp;
    return MIMIR_OK;
}

int mimir_store_graph_launch(mimir_store_graph* g) {
    if (!g) return MIMIR_EINVAL;
    mimir_ctx* ctx = g->store->ctx;
    MIMIR_ENTER(ctx);
    hipError_t e = hipGraphLaunch(g->exec, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipGraphLaunch");
    return MIMIR_OK;
}

int mimir_store_graph_set_input(mimir_store_graph* g, const char* name, int dtype, const void* host, int64_t n) {
    if (!g) return MIMIR_EINVAL;
    mimir_ctx* ctx = g->store->ctx;
    MIMIR_REQUIRE(ctx, name && n >= 0 && (n == 0 || host), "mimir_store_graph_set_input: invalid argument");
    auto& m = g->in[dtype == MIMIR_DTYPE_I32 ? 1 : 0];
    auto it = m.find(name);
    MIMIR_REQUIRE(ctx, it != m.end(), "mimir_store_graph_set_input: %s is not an input of the graph", name);
    MIMIR_REQUIRE(ctx, it->second.n == n, "mimir_store_graph_set_input: %s holds %lld elements, not %lld", name,
                  (long long)it->second.n, (long long)n);
    if (n == 0) return MIMIR_OK;
    return mimir_upload(ctx, it->second.buf->p, host, static_cast<size_t>(n) * 4);
}

int mimir_store_graph_get(mimir_store_graph* g, const char* name, int dtype, void* host, int64_t cap, int64_t* n) {
    if (!g) return MIMIR_EINVAL;
    mimir_ctx* ctx = g->store->ctx;
    MIMIR_REQUIRE(ctx, name && n && cap >= 0, "mimir_store_graph_get: invalid argument");
    auto& m = g->out[dtype == MIMIR_DTYPE_I32 ? 1 : 0];
    auto it = m.find(name);
    MIMIR_REQUIRE(ctx, it != m.end(), "mimir_store_graph_get: the graph binds no tensor named %s", name);
    *n = it->second.n;
    const int64_t k = cap < it->second.n ? cap : it->second.n;
    if (k > 0) {
        MIMIR_REQUIRE(ctx, host, "mimir_store_graph_get: null host buffer");
        return mimir_download(ctx, host, it->second.buf->p, static_cast<size_t>(k) * 4);
    }
    return MIMIR_OK;
}

int mimir_store_graph_destroy(mimir_store_graph* g) {
    if (!g) return MIMIR_EINVAL;
    mimir_store* s = g->store;
    mimir_ctx* ctx = s->ctx;
    int st = enter(ctx);
    // Launches still in flight read and write the held buffers.
    if (st == MIMIR_OK) {
        hipError_t e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) st = hip_fail(ctx, e, "hipStreamSynchronize");
    }
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    for (Buf* b : g->held) s->release(b);
    s->graphs.erase(std::remove(s->graphs.begin(), s->graphs.end(), g), s->graphs.end());
    const int st2 = graph_unpin(ctx);
    delete g;
    return st != MIMIR_OK ? st : st2;
}

}  // extern "C"
