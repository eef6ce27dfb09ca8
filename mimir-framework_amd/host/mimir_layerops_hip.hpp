// mimir_layerops_hip.hpp -- header-only C++ adapter that puts libmimir_hip
// (include/mimir_hip.h) behind the reference's own forward-op signatures, so
// Mimir's runtime can switch these ops to the MI355X without touching its
// callers.  Same names, argument meaning and exceptions as the reference
// (brit45/mimir-framework):
//
//   mimir_hip::LayerOps::layernorm_forward   LayerOps.hpp:264-319
//   mimir_hip::LayerOps::softmax_forward     LayerOps.hpp:325-361
//   mimir_hip::LayerOps::softmax_inplace     LayerOps.hpp:952-974
//   mimir_hip::LayerOps::gelu_forward        LayerOps.hpp:556-568
//   mimir_hip::LayerOps::silu_forward        LayerOps.hpp:570-581
//   mimir_hip::LayerOps::add_forward         LayerOps.hpp:142-199
//   mimir_hip::LayerOps::multiply_forward    LayerOps.hpp:205-230
//   mimir_hip::LayerOpsExt::rms_norm_forward LayerOpsExt.hpp:345-378
//   mimir_hip::Normalization::rms_norm       Layers.hpp:1003-1021
//   mimir_hip::embedding_forward(_float_ids) Model.cpp:1152-1205 / 5301-5334 (inline there)
//   mimir_hip::DeviceModel::forwardPassNamed Model.cpp:1352-1408, 4621-6824
//                                            (device-resident TensorStore)
//   mimir_hip::DeviceModel::backwardPass     Model.cpp:7307-9153
//
// The op templates take the reference's `Layer` (or anything with the same
// fields: eps, affine, use_bias, in_features, vocab_size, embed_dim,
// padding_idx, type_enum, getWeights(), getWeightsSize()).  The host-vector
// overloads upload, run and download; the `device::` functions take device
// pointers and only enqueue, for a device-resident TensorStore.
//
// Errors: invalid shapes throw std::runtime_error, as the reference does;
// device failures throw mimir_hip::Error (also a std::runtime_error).
#pragma once

#include <mimir_hip.h>

#include <cmath>
#include <cstddef>
#include <cstdint>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace mimir_hip {

class Error : public std::runtime_error {
public:
    Error(int status, const std::string& msg) : std::runtime_error(msg), status_(status) {}
    int status() const { return status_; }

private:
    int status_;
};

// One device + stream.  Context::instance() is the process-wide default,
// created on first use (as the reference's static compute engines are).
// The host-vector mirrors below all use it, each holding lock() for its
// whole call (uploads, launch, download), so host threads may call them at
// the same time; a caller that wants its threads to overlap on the GPU gives
// each thread a Context of its own and uses the device:: functions.
class Context {
public:
    explicit Context(int device = 0) {
        const int st = mimir_ctx_create(device, &ctx_);
        if (st != MIMIR_OK)
            throw Error(st, "mimir_ctx_create(device " + std::to_string(device) + ") failed");
    }
    ~Context() {
        if (ctx_) mimir_ctx_destroy(ctx_);
    }
    Context(const Context&) = delete;
    Context& operator=(const Context&) = delete;

    static Context& instance() {
        static Context ctx(0);
        return ctx;
    }

    mimir_ctx* get() const { return ctx_; }
    std::unique_lock<std::mutex> lock() { return std::unique_lock<std::mutex>(m_); }

    // MIMIR_EINVAL -> std::runtime_error (the reference's convention); others -> Error.
    void check(int st, const char* what) const {
        if (st == MIMIR_OK) return;
        std::string msg = std::string(what) + ": " + mimir_last_error(ctx_);
        if (st == MIMIR_EINVAL) throw std::runtime_error(msg);
        throw Error(st, msg);
    }
    void sync() const { check(mimir_sync(ctx_), "mimir_sync"); }

private:
    mimir_ctx* ctx_ = nullptr;
    std::mutex m_;
};

// Owning device buffer of T.
template <class T>
class DeviceBuffer {
public:
    DeviceBuffer(Context& ctx, size_t n) : ctx_(&ctx), n_(n) {
        if (n_) ctx_->check(mimir_malloc(ctx_->get(), n_ * sizeof(T), reinterpret_cast<void**>(&p_)),
                            "mimir_malloc");
    }
    DeviceBuffer(Context& ctx, const std::vector<T>& host) : DeviceBuffer(ctx, host.size()) {
        upload(host.data(), host.size());
    }
    DeviceBuffer(Context& ctx, const T* host, size_t n) : DeviceBuffer(ctx, n) { upload(host, n); }
    ~DeviceBuffer() {
        if (p_) mimir_free(ctx_->get(), p_);
    }
    DeviceBuffer(DeviceBuffer&& o) noexcept : ctx_(o.ctx_), p_(o.p_), n_(o.n_) { o.p_ = nullptr; }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;

    T* data() const { return p_; }
    size_t size() const { return n_; }
    void upload(const T* host, size_t n) {
        if (n) ctx_->check(mimir_upload(ctx_->get(), p_, host, n * sizeof(T)), "mimir_upload");
    }
    std::vector<T> download() const {
        std::vector<T> out(n_);
        if (n_) ctx_->check(mimir_download(ctx_->get(), out.data(), p_, n_ * sizeof(T)), "mimir_download");
        return out;
    }

private:
    Context* ctx_;
    T* p_ = nullptr;
    size_t n_ = 0;
};

// ---------------------------------------------------------------------------
// Device-resident entry points (enqueue only).
// ---------------------------------------------------------------------------
namespace device {

inline void layernorm(Context& c, const float* x, const float* gamma, const float* beta, float* y,
                      int64_t groups, int64_t n, float eps) {
    c.check(mimir_layernorm_fwd(c.get(), x, gamma, beta, y, groups, n, eps), "LayerNorm");
}
inline void rmsnorm(Context& c, const float* x, const float* w, int64_t w_len, float* y, int64_t rows,
                    int64_t cols, float eps) {
    c.check(mimir_rmsnorm_fwd(c.get(), x, w, w_len, y, rows, cols, eps), "RMSNorm");
}
inline void add_rmsnorm(Context& c, const float* x, const float* residual, float* residual_out,
                        const float* w, float* y, int64_t rows, int64_t cols, float eps) {
    c.check(mimir_add_rmsnorm_fwd(c.get(), x, residual, residual_out, w, y, rows, cols, eps),
            "add+RMSNorm");
}
inline void softmax(Context& c, const float* x, float* y, int64_t rows, int64_t cols, int mode) {
    c.check(mimir_softmax_fwd(c.get(), x, y, rows, cols, mode), "Softmax");
}
inline void gelu(Context& c, const float* x, float* y, int64_t n) {
    c.check(mimir_gelu_fwd(c.get(), x, y, n), "GELU");
}
inline void silu(Context& c, const float* x, float* y, int64_t n) {
    c.check(mimir_silu_fwd(c.get(), x, y, n), "SiLU");
}
inline void silu_mul(Context& c, const float* gate, const float* up, float* y, int64_t n) {
    c.check(mimir_silu_mul_fwd(c.get(), gate, up, y, n), "SiLU*up");
}
inline void gelu_mul(Context& c, const float* gate, const float* up, float* y, int64_t n) {
    c.check(mimir_gelu_mul_fwd(c.get(), gate, up, y, n), "GELU*up");
}
inline void add(Context& c, const float* a, int64_t na, const float* b, int64_t nb, float* y) {
    c.check(mimir_add_fwd(c.get(), a, na, b, nb, y), "Add");
}
inline void mul(Context& c, const float* a, int64_t na, const float* b, int64_t nb, float* y) {
    c.check(mimir_mul_fwd(c.get(), a, na, b, nb, y), "Multiply");
}
inline void embedding(Context& c, const int32_t* ids, int64_t n_ids, const float* table,
                      int64_t table_len, int32_t vocab, int32_t dim, int32_t pad, float* y) {
    c.check(mimir_embedding_fwd(c.get(), ids, n_ids, table, table_len, vocab, dim, pad, y), "Embedding");
}
inline void rope(Context& c, const float* q, float* q_out, int64_t q_heads, const float* k, float* k_out,
                 int64_t k_heads, int64_t batch, int64_t seq, int64_t head_dim, int64_t pos_offset,
                 const float* cos_tab, const float* sin_tab, int64_t table_rows) {
    c.check(mimir_rope_fwd(c.get(), q, q_out, q_heads, k, k_out, k_heads, batch, seq, head_dim,
                           pos_offset, cos_tab, sin_tab, table_rows),
            "RoPE");
}

inline void attention(Context& c, const float* q, int64_t ld_q, const float* k, const float* v, int64_t ld_kv,
                      float* out, int64_t ld_out, int64_t batch, int64_t q_len, int64_t kv_len, int64_t heads,
                      int64_t head_dim, float scale, bool causal) {
    c.check(mimir_attention_fwd(c.get(), q, ld_q, k, v, ld_kv, out, ld_out, batch, q_len, kv_len, heads,
                                head_dim, scale, causal ? 1 : 0),
            "Attention");
}

}  // namespace device

namespace detail {

// Run `op(device ptrs..., y)` on host vectors: upload inputs, allocate the
// output, download it (the PCIe-inclusive path of a host-vector caller).
template <class Op>
std::vector<float> run1(Context& c, const std::vector<float>& x, size_t out_n, Op op) {
    DeviceBuffer<float> dx(c, x);
    DeviceBuffer<float> dy(c, out_n);
    op(dx.data(), dy.data());
    return dy.download();
}

template <class Op>
std::vector<float> run2(Context& c, const std::vector<float>& a, const std::vector<float>& b,
                        size_t out_n, Op op) {
    DeviceBuffer<float> da(c, a);
    DeviceBuffer<float> db(c, b);
    DeviceBuffer<float> dy(c, out_n);
    op(da.data(), db.data(), dy.data());
    return dy.download();
}

}  // namespace detail

// ---------------------------------------------------------------------------
// Host-vector mirrors of the reference entry points.
// ---------------------------------------------------------------------------
namespace LayerOps {

template <class LayerT>
std::vector<float> layernorm_forward(const std::vector<float>& input, const LayerT& layer,
                                     bool training = true) {
    (void)training;
    Context& c = Context::instance();
    const auto held = c.lock();  // buffers below are freed before it is released
    const int64_t N = static_cast<int64_t>(input.size());
    const int64_t n = layer.in_features > 0 ? layer.in_features : N;
    if (n <= 0 || (N % n) != 0) throw std::runtime_error("LayerNorm: invalid normalized_size");
    const float* w = layer.affine ? layer.getWeights() : nullptr;
    const bool bias = layer.affine && layer.use_bias;
    std::vector<float> gamma, beta;
    if (w) {
        const size_t need = static_cast<size_t>(n) * (bias ? 2 : 1);
        if (layer.getWeightsSize() < need) throw std::runtime_error("LayerNorm: weight block too small");
        gamma.assign(w, w + n);
        if (bias) beta.assign(w + n, w + 2 * n);
    }
    DeviceBuffer<float> dg(c, gamma), db(c, beta);
    return detail::run1(c, input, input.size(), [&](const float* x, float* y) {
        device::layernorm(c, x, w ? dg.data() : nullptr, bias && w ? db.data() : nullptr, y, N / n, n,
                          layer.eps);
    });
}

template <class LayerT>
std::vector<float> softmax_forward(const std::vector<float>& input, const LayerT& layer) {
    Context& c = Context::instance();
    const auto held = c.lock();  // buffers below are freed before it is released
    const bool log = layer.type_enum == decltype(layer.type_enum)::LogSoftmax;
    return detail::run1(c, input, input.size(), [&](const float* x, float* y) {
        device::softmax(c, x, y, 1, static_cast<int64_t>(input.size()),
                        log ? MIMIR_SOFTMAX_LOG : MIMIR_SOFTMAX_MUL_INV);
    });
}

inline void softmax_inplace(std::vector<float>& x, int seq_len, int dim) {
    Context& c = Context::instance();
    const auto held = c.lock();  // buffers below are freed before it is released
    x = detail::run1(c, x, x.size(), [&](const float* in, float* y) {
        device::softmax(c, in, y, seq_len, dim, MIMIR_SOFTMAX_DIV_EPS);
    });
}

inline std::vector<float> gelu_forward(const std::vector<float>& input) {
    Context& c = Context::instance();
    const auto held = c.lock();  // buffers below are freed before it is released
    return detail::run1(c, input, input.size(), [&](const float* x, float* y) {
        device::gelu(c, x, y, static_cast<int64_t>(input.size()));
    });
}

inline std::vector<float> silu_forward(const std::vector<float>& input) {
    Context& c = Context::instance();
    const auto held = c.lock();  // buffers below are freed before it is released
    return detail::run1(c, input, input.size(), [&](const float* x, float* y) {
        device::silu(c, x, y, static_cast<int64_t>(input.size()));
    });
}

inline std::vector<float> add_forward(const std::vector<float>& input1, const std::vector<float>& input2) {
    if (input1.empty() || input2.empty()) throw std::runtime_error("Add: inputs must be non-empty");
    Context& c = Context::instance();
    const auto held = c.lock();  // buffers below are freed before it is released
    const size_t out_n = input1.size() > input2.size() ? input1.size() : input2.size();
    return detail::run2(c, input1, input2, out_n, [&](const float* a, const float* b, float* y) {
        device::add(c, a, static_cast<int64_t>(input1.size()), b, static_cast<int64_t>(input2.size()), y);
    });
}

inline std::vector<float> multiply_forward(const std::vector<float>& input1,
                                           const std::vector<float>& input2) {
    if (input1.size() != input2.size()) throw std::runtime_error("Multiply: input sizes must match");
    Context& c = Context::instance();
    const auto held = c.lock();  // buffers below are freed before it is released
    return detail::run2(c, input1, input2, input1.size(), [&](const float* a, const float* b, float* y) {
        device::mul(c, a, static_cast<int64_t>(input1.size()), b, static_cast<int64_t>(input2.size()), y);
    });
}

// Fused form of multiply_forward(silu_forward(gate), up): one pass, no intermediate vector.
inline std::vector<float> silu_mul_forward(const std::vector<float>& gate, const std::vector<float>& up) {
    if (gate.size() != up.size()) throw std::runtime_error("Multiply: input sizes must match");
    Context& c = Context::instance();
    const auto held = c.lock();  // buffers below are freed before it is released
    return detail::run2(c, gate, up, gate.size(), [&](const float* g, const float* u, float* y) {
        device::silu_mul(c, g, u, y, static_cast<int64_t>(gate.size()));
    });
}

// Steps 2-5 of self_attention_forward (LayerOps.hpp:1028-1089) on the QKV
// projection's output qkv [seq_len x 3*embed_dim] (Q | K | V column blocks):
// returns the attended heads [seq_len x embed_dim] that the reference then
// multiplies by out_weight (:1094).  The split copies are not made: Q, K and
// V are read in place through the row stride.  Same checks and messages.
inline std::vector<float> attention_core(const std::vector<float>& qkv, int seq_len, int embed_dim,
                                         int num_heads = 1, bool causal = false) {
    if (num_heads <= 0 || embed_dim % num_heads != 0)
        throw std::runtime_error("SelfAttention: embed_dim must be divisible by num_heads");
    if (seq_len < 0 || qkv.size() != static_cast<size_t>(seq_len) * 3 * static_cast<size_t>(embed_dim))
        throw std::runtime_error("SelfAttention: input size mismatch");
    const int head_dim = embed_dim / num_heads;
    Context& c = Context::instance();
    const auto held = c.lock();  // buffers below are freed before it is released
    return detail::run1(c, qkv, static_cast<size_t>(seq_len) * embed_dim, [&](const float* d, float* y) {
        device::attention(c, d, 3 * embed_dim, d + embed_dim, d + 2 * embed_dim, 3 * embed_dim, y, embed_dim, 1,
                          seq_len, seq_len, num_heads, head_dim, 1.0f / std::sqrt(static_cast<float>(head_dim)),
                          causal);
    });
}

// The core of cross_attention_forward (LayerOps.hpp:1163-1209) on its
// projections: Q [query_len x embed_dim] and KV [kv_len x 2*embed_dim]
// (K | V column blocks).  Returns [query_len x embed_dim].
inline std::vector<float> cross_attention_core(const std::vector<float>& Q, const std::vector<float>& KV,
                                               int query_len, int kv_len, int embed_dim, int num_heads = 1,
                                               bool causal = false) {
    if (num_heads <= 0 || embed_dim % num_heads != 0)
        throw std::runtime_error("CrossAttention: embed_dim must be divisible by num_heads");
    if (query_len <= 0 || kv_len <= 0 || embed_dim <= 0)
        throw std::runtime_error("CrossAttention: invalid dimensions");
    if (Q.size() != static_cast<size_t>(query_len) * embed_dim ||
        KV.size() != static_cast<size_t>(kv_len) * 2 * embed_dim)
        throw std::runtime_error("CrossAttention: input size mismatch");
    const int head_dim = embed_dim / num_heads;
    Context& c = Context::instance();
    const auto held = c.lock();  // buffers below are freed before it is released
    return detail::run2(c, Q, KV, Q.size(), [&](const float* q, const float* kv, float* y) {
        device::attention(c, q, embed_dim, kv, kv + embed_dim, 2 * embed_dim, y, embed_dim, 1, query_len, kv_len,
                          num_heads, head_dim, 1.0f / std::sqrt(static_cast<float>(head_dim)), causal);
    });
}

}  // namespace LayerOps

namespace LayerOpsExt {

template <class LayerT>
std::vector<float> rms_norm_forward(const std::vector<float>& input, const LayerT& layer) {
    Context& c = Context::instance();
    const auto held = c.lock();  // buffers below are freed before it is released
    if (input.empty()) return {};
    const float* w = layer.getWeights();
    const size_t wn = (layer.affine && w) ? layer.getWeightsSize() : 0;
    DeviceBuffer<float> dw(c, w, wn);
    return detail::run1(c, input, input.size(), [&](const float* x, float* y) {
        device::rmsnorm(c, x, wn ? dw.data() : nullptr, static_cast<int64_t>(wn), y, 1,
                        static_cast<int64_t>(input.size()), layer.eps);
    });
}

}  // namespace LayerOpsExt

namespace Normalization {

inline void rms_norm(std::vector<float>& data, const std::vector<float>& gamma, int normalized_size,
                     float eps = 1e-6f) {
    Context& c = Context::instance();
    const auto held = c.lock();  // buffers below are freed before it is released
    if (normalized_size <= 0 || gamma.size() < static_cast<size_t>(normalized_size))
        throw std::runtime_error("rms_norm: invalid normalized_size");
    const int64_t rows = static_cast<int64_t>(data.size()) / normalized_size;
    DeviceBuffer<float> dg(c, gamma);
    data = detail::run1(c, data, data.size(), [&](const float* x, float* y) {
        device::rmsnorm(c, x, dg.data(), normalized_size, y, rows, normalized_size, eps);
    });
}

}  // namespace Normalization

// The embedding gather of Model::forwardPassView (int ids), Model.cpp:1152-1205.
template <class LayerT>
std::vector<float> embedding_forward(const std::vector<int>& ids, const LayerT& layer) {
    Context& c = Context::instance();
    const auto held = c.lock();  // buffers below are freed before it is released
    const int32_t vocab = layer.vocab_size > 1 ? layer.vocab_size : 1;
    const int32_t dim = layer.embed_dim > 1 ? layer.embed_dim : 1;
    const float* w = layer.getWeights();
    if (!w) throw std::runtime_error("Embedding: weights not initialized");
    const size_t wn = layer.getWeightsSize();
    if (wn < static_cast<size_t>(vocab) * static_cast<size_t>(dim))
        throw std::runtime_error("Embedding: invalid weight size");
    if (ids.empty()) return {};
    static_assert(sizeof(int) == sizeof(int32_t), "int ids are 32-bit");
    DeviceBuffer<int32_t> di(c, reinterpret_cast<const int32_t*>(ids.data()), ids.size());
    DeviceBuffer<float> dt(c, w, wn);
    DeviceBuffer<float> dy(c, ids.size() * static_cast<size_t>(dim));
    device::embedding(c, di.data(), static_cast<int64_t>(ids.size()), dt.data(), static_cast<int64_t>(wn),
                      vocab, dim, layer.padding_idx, dy.data());
    return dy.download();
}

// Float-id form, Model.cpp:5301-5334 (ids rounded with llround).
template <class LayerT>
std::vector<float> embedding_forward_float_ids(const std::vector<float>& x, const LayerT& layer) {
    Context& c = Context::instance();
    const auto held = c.lock();  // buffers below are freed before it is released
    const int32_t vocab = layer.vocab_size > 1 ? layer.vocab_size : 1;
    const int32_t dim = layer.embed_dim > 1 ? layer.embed_dim : 1;
    const float* w = layer.getWeights();
    if (!w) throw std::runtime_error("Embedding: weights not initialized");
    const size_t wn = layer.getWeightsSize();
    if (wn < static_cast<size_t>(vocab) * static_cast<size_t>(dim))
        throw std::runtime_error("Embedding: invalid weight size");
    if (x.empty()) return {};
    DeviceBuffer<float> di(c, x);
    DeviceBuffer<float> dt(c, w, wn);
    DeviceBuffer<float> dy(c, x.size() * static_cast<size_t>(dim));
    c.check(mimir_embedding_f32ids_fwd(c.get(), di.data(), static_cast<int64_t>(x.size()), dt.data(),
                                       static_cast<int64_t>(wn), vocab, dim, layer.padding_idx, dy.data()),
            "Embedding");
    return dy.download();
}

// ---------------------------------------------------------------------------
// Device-resident runtime: Model::forwardPassNamed (Model.cpp:1352-1408,
// forwardPassView Model.cpp:4621-6824) over a reference layer list, with every
// activation held in HBM by a mimir_store and only "x" downloaded, and the
// training step's Model::backwardPass over the same store.  A training
// forward applies the layers' residual merges (Layer::branch_type RESIDUAL
// with branch_sources, Model.cpp:6676-6685) as the reference does.  Layer
// types: LayerNorm, RMSNorm, Softmax, LogSoftmax, GELU, SiLU, Add, Multiply,
// Embedding, Identity, Dropout, SelfAttention, MultiHeadAttention,
// CrossAttention (others throw at construction).
// ---------------------------------------------------------------------------
template <class LayerT>
class DeviceModel {
public:
    DeviceModel(Context& c, const std::vector<LayerT>& layers) : ctx_(&c), layers_(&layers) {
        ctx_->check(mimir_store_create(ctx_->get(), &store_), "mimir_store_create");
        for (const LayerT& L : layers) {
            const int t = type_of(L.type);
            if (t == 0) {
                mimir_store_destroy(store_);
                throw std::runtime_error("DeviceModel: layer type " + L.type + " (" + L.name +
                                         ") is not on the HIP path");
            }
            types_.push_back(t);
        }
        syncWeights();
    }
    ~DeviceModel() {
        if (store_) mimir_store_destroy(store_);
    }
    DeviceModel(const DeviceModel&) = delete;
    DeviceModel& operator=(const DeviceModel&) = delete;

    // Inference fusion (mimir_store_set_fusion): groups of layers that feed
    // each other run as one kernel; forwardPassNamed's "x" is unchanged bit
    // for bit, intermediate tensors nothing reads are not kept.
    void setFusion(bool enable) { ctx_->check(mimir_store_set_fusion(store_, enable ? 1 : 0), "DeviceModel fusion"); }

    // Upload every layer's weight block (Layer::getWeights / getWeightsSize);
    // call again after the host weights change.
    void syncWeights() {
        weights_.clear();
        for (const LayerT& L : *layers_) {
            const float* w = L.getWeights();
            const size_t n = w ? L.getWeightsSize() : 0;
            weights_.emplace_back(*ctx_, w, n);
        }
    }

    // Model::forwardPassNamed (Model.cpp:1352-1408).  training=true keeps each
    // layer's inputs on the device for backwardPass, as the reference's
    // forward_state does (Dropout is then refused: its mask is random).
    std::vector<float> forwardPassNamed(const std::unordered_map<std::string, std::vector<float>>& fin,
                                        const std::unordered_map<std::string, std::vector<int>>& iin,
                                        bool training = false) {
        std::vector<const char*> fn, in;
        std::vector<const float*> fd;
        std::vector<const int32_t*> id;
        std::vector<int64_t> fs, is;
        for (const auto& kv : fin) {
            fn.push_back(kv.first.c_str());
            fd.push_back(kv.second.data());
            fs.push_back(static_cast<int64_t>(kv.second.size()));
        }
        for (const auto& kv : iin) {
            in.push_back(kv.first.c_str());
            id.push_back(reinterpret_cast<const int32_t*>(kv.second.data()));
            is.push_back(static_cast<int64_t>(kv.second.size()));
        }
        ctx_->check(mimir_store_set_inputs(store_, fn.data(), fd.data(), fs.data(), static_cast<int32_t>(fn.size()),
                                           in.data(), id.data(), is.data(), static_cast<int32_t>(in.size())),
                    "DeviceModel inputs");
        build_layers();
        if (training)
            ctx_->check(mimir_store_run_training(store_, ls_.data(), static_cast<int32_t>(ls_.size())),
                        "DeviceModel forward (training)");
        else
            ctx_->check(mimir_store_run(store_, ls_.data(), static_cast<int32_t>(ls_.size())), "DeviceModel forward");
        int64_t n = 0;
        void* p = nullptr;
        ctx_->check(mimir_store_info(store_, "x", MIMIR_DTYPE_F32, &p, &n), "DeviceModel output");
        std::vector<float> out(static_cast<size_t>(n));
        ctx_->check(mimir_store_get(store_, "x", MIMIR_DTYPE_F32, out.data(), n, &n), "DeviceModel output");
        return out;
    }

    // Model::forwardPass(const std::vector<int>& input_ids, training)
    // (Model.cpp:1026-1349), the int-ids forward: the ids are the int
    // tensors "x" and "__input__"; Embedding layers gather them as ints and
    // the reduced layer switch of that path applies (RMSNorm, SiLU, Multiply
    // and Identity throw).  The reference's default is training=true.
    std::vector<float> forwardPass(const std::vector<int>& input_ids, bool training = true) {
        ctx_->check(mimir_store_set_input_ids(store_, reinterpret_cast<const int32_t*>(input_ids.data()),
                                              static_cast<int64_t>(input_ids.size())),
                    "DeviceModel ids");
        build_layers();
        ctx_->check(mimir_store_run_ids(store_, ls_.data(), static_cast<int32_t>(ls_.size()), training ? 1 : 0),
                    "DeviceModel forward (int ids)");
        if (ls_.empty()) return {};
        int64_t n = 0;
        void* p = nullptr;
        ctx_->check(mimir_store_info(store_, "x", MIMIR_DTYPE_F32, &p, &n), "DeviceModel output");
        std::vector<float> out(static_cast<size_t>(n));
        ctx_->check(mimir_store_get(store_, "x", MIMIR_DTYPE_F32, out.data(), n, &n), "DeviceModel output");
        return out;
    }

    // Model::backwardPass(loss_gradient) (Model.cpp:7307-9153) after a
    // training forward.  Parameter gradients are added into the layers'
    // grad_weights as the reference does (a vector of the wrong size is first
    // reset to zeros, :7448-7450, :7751-7753, :8057-8059, :8110-8112), for the
    // LayerNorm, Embedding and attention layers whose branches produce them;
    // the gradient that reached "__input__" is kept for getLastInputGradient().
    void backwardPass(const std::vector<float>& loss_gradient, std::vector<LayerT>& layers) {
        if (&layers != layers_ && layers.size() != layers_->size())
            throw std::runtime_error("DeviceModel::backwardPass: not the model's layer list");
        grads_.clear();
        for (size_t i = 0; i < layers.size(); ++i) {
            LayerT& L = layers[i];
            const size_t wn = weights_[i].size();
            if (wn && has_param_grads(types_[i])) {
                if (L.grad_weights.size() != wn) L.grad_weights.assign(wn, 0.0f);
                grads_.emplace_back(*ctx_, L.grad_weights);
            } else {
                grads_.emplace_back(*ctx_, size_t(0));
            }
            ls_[i].grad_weights = grads_[i].size() ? grads_[i].data() : nullptr;
        }
        ctx_->check(mimir_store_backward(store_, ls_.data(), static_cast<int32_t>(ls_.size()), loss_gradient.data(),
                                         static_cast<int64_t>(loss_gradient.size())),
                    "DeviceModel backward");
        for (size_t i = 0; i < layers.size(); ++i)
            if (grads_[i].size()) layers[i].grad_weights = grads_[i].download();
        has_input_grad_ = false;
        input_grad_.clear();
        void* p = nullptr;
        int64_t n = 0;
        if (mimir_store_grad_info(store_, "__input__", &p, &n) == MIMIR_OK) {
            input_grad_.resize(static_cast<size_t>(n));
            ctx_->check(mimir_store_grad_get(store_, "__input__", input_grad_.data(), n, &n), "DeviceModel input grad");
            has_input_grad_ = true;
        }
    }

    bool hasLastInputGradient() const { return has_input_grad_; }
    const std::vector<float>& getLastInputGradient() const { return input_grad_; }

    mimir_store* store() const { return store_; }

private:
    static bool has_param_grads(int t) {
        return t == MIMIR_LAYER_LAYERNORM || t == MIMIR_LAYER_EMBEDDING || t == MIMIR_LAYER_SELF_ATTENTION ||
               t == MIMIR_LAYER_MULTIHEAD_ATTENTION || t == MIMIR_LAYER_CROSS_ATTENTION;
    }

    static int type_of(const std::string& t) {
        static const std::unordered_map<std::string, int> m = {
            {"LayerNorm", MIMIR_LAYER_LAYERNORM}, {"RMSNorm", MIMIR_LAYER_RMSNORM},
            {"Softmax", MIMIR_LAYER_SOFTMAX},     {"LogSoftmax", MIMIR_LAYER_LOGSOFTMAX},
            {"GELU", MIMIR_LAYER_GELU},           {"SiLU", MIMIR_LAYER_SILU},
            {"Add", MIMIR_LAYER_ADD},             {"Multiply", MIMIR_LAYER_MULTIPLY},
            {"Embedding", MIMIR_LAYER_EMBEDDING}, {"Identity", MIMIR_LAYER_IDENTITY},
            {"Dropout", MIMIR_LAYER_DROPOUT},
            {"SelfAttention", MIMIR_LAYER_SELF_ATTENTION},
            {"MultiHeadAttention", MIMIR_LAYER_MULTIHEAD_ATTENTION},
            {"CrossAttention", MIMIR_LAYER_CROSS_ATTENTION}};
        auto it = m.find(t);
        return it == m.end() ? 0 : it->second;
    }

    // The C descriptors of the layer list (names point into *layers_).
    void build_layers() {
        ls_.assign(layers_->size(), mimir_layer{});
        names_.assign(layers_->size(), {});
        for (size_t i = 0; i < layers_->size(); ++i) {
            const LayerT& L = (*layers_)[i];
            for (const auto& nm : L.inputs) names_[i].push_back(nm.c_str());
            mimir_layer& c = ls_[i];
            c.type = types_[i];
            c.name = L.name.c_str();
            c.inputs = names_[i].data();
            c.n_inputs = static_cast<int32_t>(names_[i].size());
            c.output = L.output.c_str();
            c.weights = weights_[i].data();
            c.weights_len = static_cast<int64_t>(weights_[i].size());
            c.eps = L.eps;
            c.affine = L.affine;
            c.use_bias = L.use_bias;
            c.in_features = L.in_features;
            c.vocab_size = L.vocab_size;
            c.embed_dim = L.embed_dim;
            c.padding_idx = L.padding_idx;
            c.seq_len = L.seq_len;
            c.grad_weights = nullptr;
            // Branch fields, read by training forwards (Layers.hpp:214-219).
            c.branch_type = static_cast<int32_t>(L.branch_type);
            c.merge_op = static_cast<int32_t>(L.merge_op);
            static_assert(sizeof(L.branch_sources[0]) == sizeof(int32_t), "Layer::branch_sources is int");
            c.branch_sources = reinterpret_cast<const int32_t*>(L.branch_sources.data());
            c.n_branch_sources = static_cast<int32_t>(L.branch_sources.size());
            // Attention fields (Layers.hpp:174-178).
            c.num_heads = L.num_heads;
            c.head_dim = L.head_dim;
            c.causal = L.causal ? 1 : 0;
        }
    }

    Context* ctx_;
    const std::vector<LayerT>* layers_;
    mimir_store* store_ = nullptr;
    std::vector<int> types_;
    std::vector<DeviceBuffer<float>> weights_;
    std::vector<DeviceBuffer<float>> grads_;
    std::vector<mimir_layer> ls_;
    std::vector<std::vector<const char*>> names_;
    bool has_input_grad_ = false;
    std::vector<float> input_grad_;
};

}  // namespace mimir_hip
