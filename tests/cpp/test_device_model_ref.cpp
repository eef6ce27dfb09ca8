// test_device_model_ref.cpp -- the C++ adapter's DeviceModel instantiated on
// the reference's own `struct Layer` (Layers.hpp:86-309), whose weights live
// in the blocks Model::allocateParams hands out (Layer::getWeights through
// the weight_block), run on the GPU beside the reference's own
// Model::forwardPassNamed / Model::backwardPass on the same layers.
//
// Built by oracle/Makefile (target `adapter_ref`, only where the reference
// tree is present) against the reference headers and the reference runtime
// compiled in place (oracle/_ref/libmimir_ref_model.so); run by
// tests/test_gpu_cpp_adapter.py.  Standalone main() returning 0 / 1, like
// the reference's CTest programs.  Also the attention core's binding inside
// the reference's own self_attention_forward / cross_attention_forward.
#include "LayerOps.hpp"
#include "Model.hpp"
#include "mimir_layerops_hip.hpp"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

namespace {

int failures = 0;

#define CHECK(cond)                                                                   \
    do {                                                                              \
        if (!(cond)) {                                                                \
            std::fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond);      \
            ++failures;                                                               \
        }                                                                             \
    } while (0)

using FMap = std::unordered_map<std::string, std::vector<float>>;
using IMap = std::unordered_map<std::string, std::vector<int>>;

bool same_bits(const std::vector<float>& a, const std::vector<float>& b) {
    return a.size() == b.size() && (a.empty() || std::memcmp(a.data(), b.data(), a.size() * 4) == 0);
}

// |a - b| <= max(1e-6, 1e-5 |b|) elementwise.
bool close(const std::vector<float>& a, const std::vector<float>& b) {
    if (a.size() != b.size()) return false;
    for (size_t i = 0; i < a.size(); ++i)
        if (!(std::fabs(a[i] - b[i]) <= std::fmax(1e-6f, 1e-5f * std::fabs(b[i])))) return false;
    return true;
}

// Tests/test_runtime_residual_merge.cpp:9-47: layer 1 (named "my_residual",
// so Model::push's detectBranchType makes it RESIDUAL) merges its output with
// layer 0's by ADD, in training forwards only.
void residual_merge_kat(mimir_hip::Context& c) {
    Model m;
    m.push("skip", "Identity", 0);
    m.push("my_residual", "Multiply", 0);
    auto& layers = m.getMutableLayers();
    layers[0].inputs = {"x"};
    layers[0].output = "skip";
    layers[1].inputs = {"x", "scale"};
    layers[1].output = "x";
    CHECK(layers[1].branch_type == BranchType::RESIDUAL);
    layers[1].branch_sources = {0};
    layers[1].merge_op = MergeOperation::ADD;
    m.allocateParams();
    const FMap fin{{"x", {1.0f, 2.0f}}, {"scale", {2.0f, 3.0f}}};

    const std::vector<float> ref_train = m.forwardPassNamed(fin, IMap{}, true);
    const std::vector<float> ref_inf = m.forwardPassNamed(fin, IMap{}, false);
    CHECK(same_bits(ref_train, {3.0f, 8.0f}));
    CHECK(same_bits(ref_inf, {2.0f, 6.0f}));

    mimir_hip::DeviceModel<Layer> dm(c, m.getLayers());
    CHECK(same_bits(dm.forwardPassNamed(fin, IMap{}, true), ref_train));
    CHECK(same_bits(dm.forwardPassNamed(fin, IMap{}, false), ref_inf));

    // Every merge operation through the Layer field, against the reference.
    const MergeOperation ops[] = {MergeOperation::ADD, MergeOperation::MULTIPLY, MergeOperation::CONCATENATE,
                                  MergeOperation::MAX, MergeOperation::AVERAGE, MergeOperation::GATED,
                                  MergeOperation::ATTENTION_WEIGHTED};
    const FMap fin9{{"x", {1, -2, 3, -4, 5, -6, 7, -8, 0.5f}}, {"scale", {2, 3, -1, 0, 1, 1, -2, 2, 3}}};
    for (MergeOperation op : ops) {
        layers[1].merge_op = op;
        const std::vector<float> want = m.forwardPassNamed(fin9, IMap{}, true);
        CHECK(same_bits(dm.forwardPassNamed(fin9, IMap{}, true), want));
    }
}

// A LayerNorm whose gamma | beta come from the reference's weight block, then
// a residual GELU ("block_residual", source: the LayerNorm), then an Add:
// forward in both modes, and a training step whose gradients (grad_weights,
// the "__input__" gradient) must equal the reference's.  The reference's
// backward ignores the merge (backpropThroughBranch is never called), and so
// must the device's.
void weight_block_and_backward(mimir_hip::Context& c) {
    const int rows = 3, feat = 8;
    Model m;
    m.push("ln", "LayerNorm", 2 * feat);
    m.push("block_residual", "GELU", 0);
    m.push("out", "Add", 0);
    auto& layers = m.getMutableLayers();
    layers[0].inputs = {"__input__"};
    layers[0].output = "h";
    layers[0].in_features = feat;
    layers[1].inputs = {"h"};
    layers[1].output = "g";
    layers[1].branch_sources = {0};
    layers[2].inputs = {"g", "bias"};
    layers[2].output = "x";
    m.allocateParams();
    float* w = layers[0].getWeights();
    CHECK(w != nullptr && layers[0].getWeightsSize() == 2 * feat);
    for (int i = 0; i < feat; ++i) {
        w[i] = 1.0f + 0.05f * static_cast<float>(i);
        w[feat + i] = 0.01f * static_cast<float>(i) - 0.03f;
    }
    std::vector<float> x(rows * feat), bias(feat), loss(rows * feat);
    for (size_t i = 0; i < x.size(); ++i) {
        x[i] = std::sin(0.7f * static_cast<float>(i)) * 2.0f + 0.25f;
        loss[i] = std::cos(0.3f * static_cast<float>(i));
    }
    for (int i = 0; i < feat; ++i) bias[i] = 0.1f * static_cast<float>(i);
    const FMap fin{{"__input__", x}, {"bias", bias}};

    mimir_hip::DeviceModel<Layer> dm(c, m.getLayers());
    const std::vector<float> ref_inf = m.forwardPassNamed(fin, IMap{}, false);
    CHECK(close(dm.forwardPassNamed(fin, IMap{}, false), ref_inf));

    const std::vector<float> ref_train = m.forwardPassNamed(fin, IMap{}, true);
    m.backwardPass(loss);
    const std::vector<float> ref_gw = m.getLayers()[0].grad_weights;
    CHECK(m.hasLastInputGradient());
    const std::vector<float> ref_gin = m.getLastInputGradient();
    CHECK(!close(ref_train, ref_inf));  // the merge changed the training output

    std::vector<Layer> dev_layers = m.getLayers();  // grad_weights start from the reference's zeros
    for (auto& L : dev_layers) std::fill(L.grad_weights.begin(), L.grad_weights.end(), 0.0f);
    mimir_hip::DeviceModel<Layer> dt(c, dev_layers);
    CHECK(close(dt.forwardPassNamed(fin, IMap{}, true), ref_train));
    dt.backwardPass(loss, dev_layers);
    CHECK(dt.hasLastInputGradient());
    // Float32 sums over rows: held at 1e-5 of the summed magnitudes' scale.
    auto close_sum = [](const std::vector<float>& a, const std::vector<float>& b, float scale) {
        if (a.size() != b.size()) return false;
        for (size_t i = 0; i < a.size(); ++i)
            if (!(std::fabs(a[i] - b[i]) <= std::fmax(1e-6f, 1e-5f * scale))) return false;
        return true;
    };
    CHECK(close_sum(dev_layers[0].grad_weights, ref_gw, 8.0f));
    CHECK(close_sum(dt.getLastInputGradient(), ref_gin, 8.0f));
}

// Model::forwardPass(const std::vector<int>&, training) through the
// reference Layer list: a gather, LayerNorm and Add graph in both modes, and
// the int path's refusal of a Multiply (Model.cpp:1311-1319).
void int_ids_forward(mimir_hip::Context& c) {
    const int vocab = 10, dim = 8;
    Model m;
    m.push("tok", "Embedding", vocab * dim);
    m.push("ln", "LayerNorm", 2 * dim);
    m.push("res", "Add", 0);
    auto& layers = m.getMutableLayers();
    layers[0].inputs = {"x"};
    layers[0].output = "h";
    layers[0].vocab_size = vocab;
    layers[0].embed_dim = dim;
    layers[0].padding_idx = 2;
    layers[1].inputs = {"h"};
    layers[1].output = "n";
    layers[1].in_features = dim;
    layers[2].inputs = {"n", "h"};
    layers[2].output = "x";
    m.allocateParams();
    float* w = layers[0].getWeights();
    for (int i = 0; i < vocab * dim; ++i) w[i] = std::sin(0.1f * static_cast<float>(i));
    float* g = layers[1].getWeights();
    for (int i = 0; i < dim; ++i) {
        g[i] = 1.0f + 0.1f * static_cast<float>(i);
        g[dim + i] = 0.05f * static_cast<float>(i);
    }
    const std::vector<int> ids = {3, 2, 9, -1, 10, 3, 0};
    mimir_hip::DeviceModel<Layer> dm(c, m.getLayers());
    for (bool training : {false, true}) {
        const std::vector<float> want = m.forwardPass(ids, training);
        CHECK(close(dm.forwardPass(ids, training), want));
    }
    m.push("bad", "Multiply", 0);
    auto& l2 = m.getMutableLayers();
    l2[3].inputs = {"x", "x"};
    mimir_hip::DeviceModel<Layer> dbad(c, m.getLayers());
    bool ref_threw = false, dev_threw = false;
    try { m.forwardPass(ids, false); } catch (const std::exception&) { ref_threw = true; }
    try { dbad.forwardPass(ids, false); } catch (const std::exception&) { dev_threw = true; }
    CHECK(ref_threw && dev_threw);
}

// LayerOps::self_attention_forward / cross_attention_forward (LayerOps.hpp:
// 1004-1097, 1116-1216) at their own call shape: the reference computes the
// projections, the adapter's attention_core / cross_attention_core replaces
// steps 2-5 (the softmax fused into QK^T and PV on the device), and the
// reference's output projection follows.  Held normwise at 1e-4 of the
// largest output: the core's element-wise parity is tests/test_gpu_attention.py;
// this checks the binding (layouts, strides, scale, mask) at the call site.
void attention_at_call_site() {
    const int seq = 100, e = 64, heads = 4;
    std::vector<float> x(seq * e), wqkv(3 * e * e), wout(e * e);
    for (size_t i = 0; i < x.size(); ++i) x[i] = std::sin(0.37f * static_cast<float>(i)) * 1.3f;
    for (size_t i = 0; i < wqkv.size(); ++i) wqkv[i] = std::cos(0.11f * static_cast<float>(i) + 0.5f) * 0.2f;
    for (size_t i = 0; i < wout.size(); ++i) wout[i] = std::sin(0.23f * static_cast<float>(i) + 1.0f) * 0.15f;
    auto normwise = [](const std::vector<float>& a, const std::vector<float>& b) {
        if (a.size() != b.size() || b.empty()) return false;
        float m = 0.f;
        for (float v : b) m = std::fmax(m, std::fabs(v));
        for (size_t i = 0; i < a.size(); ++i)
            if (!(std::fabs(a[i] - b[i]) <= 1e-6f + 1e-4f * m)) return false;
        return true;
    };
    for (bool causal : {false, true}) {
        const std::vector<float> ref = LayerOps::self_attention_forward(x, wqkv, wout, seq, e, heads, causal);
        std::vector<float> qkv, out;
        LayerOps::matmul(x, wqkv, qkv, seq, e, 3 * e);
        const std::vector<float> att = mimir_hip::LayerOps::attention_core(qkv, seq, e, heads, causal);
        LayerOps::matmul(att, wout, out, seq, e, e);
        CHECK(normwise(out, ref));
    }
    // Cross attention: 37 queries over 90 keys.
    const int lq = 37, lk = 90;
    std::vector<float> xq(lq * e), xkv(lk * e), wq(e * e), wkv(2 * e * e);
    for (size_t i = 0; i < xq.size(); ++i) xq[i] = std::cos(0.29f * static_cast<float>(i));
    for (size_t i = 0; i < xkv.size(); ++i) xkv[i] = std::sin(0.17f * static_cast<float>(i) + 0.3f);
    for (size_t i = 0; i < wq.size(); ++i) wq[i] = std::sin(0.07f * static_cast<float>(i)) * 0.25f;
    for (size_t i = 0; i < wkv.size(); ++i) wkv[i] = std::cos(0.05f * static_cast<float>(i) + 0.2f) * 0.2f;
    for (bool causal : {false, true}) {
        const std::vector<float> ref =
            LayerOps::cross_attention_forward(xq, xkv, wq, wkv, wout, lq, lk, e, heads, causal);
        std::vector<float> q, kv, out;
        LayerOps::matmul(xq, wq, q, lq, e, e);
        LayerOps::matmul(xkv, wkv, kv, lk, e, 2 * e);
        const std::vector<float> att = mimir_hip::LayerOps::cross_attention_core(q, kv, lq, lk, e, heads, causal);
        LayerOps::matmul(att, wout, out, lq, e, e);
        CHECK(normwise(out, ref));
    }
    // The reference's refusal, with its message.
    std::string ref_msg, dev_msg;
    try { LayerOps::self_attention_forward(x, wqkv, wout, seq, e, 5, false); } catch (const std::exception& ex) { ref_msg = ex.what(); }
    std::vector<float> qkv;
    LayerOps::matmul(x, wqkv, qkv, seq, e, 3 * e);
    try { mimir_hip::LayerOps::attention_core(qkv, seq, e, 5, false); } catch (const std::exception& ex) { dev_msg = ex.what(); }
    CHECK(!ref_msg.empty() && ref_msg == dev_msg);
}

// DeviceModel<Layer> on a pre-norm attention block of reference Layers
// (LayerNorm -> SelfAttention -> Add), beside Model::forwardPassNamed, then a
// training step beside Model::backwardPass (the input gradient gathers the
// LayerNorm's and the Add's contributions).  Normwise at 1e-4: each layer's
// element-wise parity is tested on its own.
void attention_block_model(mimir_hip::Context& c) {
    const int seq = 24, e = 32, heads = 4;
    Model m;
    m.push("ln", "LayerNorm", 2 * e);
    m.push("attn", "SelfAttention", 4 * e * e);
    m.push("res", "Add", 0);
    auto& layers = m.getMutableLayers();
    layers[0].inputs = {"__input__"};
    layers[0].output = "h";
    layers[0].in_features = e;
    layers[1].inputs = {"h"};
    layers[1].output = "a";
    layers[1].seq_len = seq;
    layers[1].embed_dim = e;
    layers[1].num_heads = heads;
    layers[1].causal = true;
    layers[2].inputs = {"a", "__input__"};
    layers[2].output = "x";
    m.allocateParams();
    float* g = layers[0].getWeights();
    for (int i = 0; i < e; ++i) {
        g[i] = 1.0f + 0.03f * static_cast<float>(i % 7);
        g[e + i] = 0.01f * static_cast<float>(i % 5);
    }
    float* w = layers[1].getWeights();
    CHECK(w != nullptr && layers[1].getWeightsSize() >= static_cast<size_t>(4 * e * e));
    for (int i = 0; i < 4 * e * e; ++i) w[i] = std::sin(0.013f * static_cast<float>(i) + 0.4f) * 0.18f;
    std::vector<float> x(seq * e);
    for (size_t i = 0; i < x.size(); ++i) x[i] = std::cos(0.21f * static_cast<float>(i)) * 1.1f;
    const FMap fin{{"__input__", x}};
    auto normwise = [](const std::vector<float>& got, const std::vector<float>& ref) {
        float mx = 0.f;
        for (float v : ref) mx = std::fmax(mx, std::fabs(v));
        bool ok = got.size() == ref.size() && !ref.empty();
        for (size_t i = 0; ok && i < ref.size(); ++i) ok = std::fabs(got[i] - ref[i]) <= 1e-6f + 1e-4f * mx;
        return ok;
    };
    const std::vector<float> ref = m.forwardPassNamed(fin, IMap{}, false);
    mimir_hip::DeviceModel<Layer> dm(c, m.getLayers());
    CHECK(normwise(dm.forwardPassNamed(fin, IMap{}, false), ref));

    std::vector<float> loss(seq * e);
    for (size_t i = 0; i < loss.size(); ++i) loss[i] = std::sin(0.37f * static_cast<float>(i)) + 0.2f;
    m.forwardPassNamed(fin, IMap{}, true);
    m.backwardPass(loss);
    CHECK(m.hasLastInputGradient());
    std::vector<Layer> dev_layers = m.getLayers();  // grad_weights start from zeros, as the reference's did
    for (auto& L : dev_layers) std::fill(L.grad_weights.begin(), L.grad_weights.end(), 0.0f);
    mimir_hip::DeviceModel<Layer> dt(c, dev_layers);
    dt.forwardPassNamed(fin, IMap{}, true);
    dt.backwardPass(loss, dev_layers);
    CHECK(dt.hasLastInputGradient());
    CHECK(normwise(dt.getLastInputGradient(), m.getLastInputGradient()));
    CHECK(normwise(dev_layers[0].grad_weights, m.getLayers()[0].grad_weights));  // LayerNorm dgamma | dbeta
    CHECK(normwise(dev_layers[1].grad_weights, m.getLayers()[1].grad_weights));  // dWqkv | dWout
}

// DeviceModel<Layer> with the runtime's fusion on: Add -> LayerNorm -> GELU
// -> Multiply -> SiLU runs as one kernel.  Its "x" equals the unfused
// device run bit for bit, and the reference Model to the LayerNorm's
// tolerance (normwise 1e-5 of the largest output).
void fused_block_model(mimir_hip::Context& c) {
    const int rows = 16, feat = 256;
    Model m;
    m.push("res_add", "Add", 0);
    m.push("ln", "LayerNorm", 2 * feat);
    m.push("act", "GELU", 0);
    m.push("gate", "Multiply", 0);
    m.push("silu", "SiLU", 0);
    auto& layers = m.getMutableLayers();
    layers[0].inputs = {"inp", "res"};
    layers[0].output = "h";
    layers[1].inputs = {"h"};
    layers[1].output = "n";
    layers[1].in_features = feat;
    layers[2].inputs = {"n"};
    layers[2].output = "g";
    layers[3].inputs = {"g", "gate"};
    layers[3].output = "m";
    layers[4].inputs = {"m"};
    layers[4].output = "x";
    m.allocateParams();
    float* w = layers[1].getWeights();
    for (int i = 0; i < feat; ++i) {
        w[i] = 1.0f + 0.01f * static_cast<float>(i % 13);
        w[feat + i] = 0.02f * static_cast<float>(i % 7) - 0.05f;
    }
    std::vector<float> inp(rows * feat), res(rows * feat), gate(rows * feat);
    for (size_t i = 0; i < inp.size(); ++i) {
        inp[i] = std::sin(0.37f * static_cast<float>(i));
        res[i] = std::cos(0.11f * static_cast<float>(i)) * 0.5f;
        gate[i] = std::sin(0.05f * static_cast<float>(i) + 1.0f);
    }
    const FMap fin{{"inp", inp}, {"res", res}, {"gate", gate}};
    const std::vector<float> ref = m.forwardPassNamed(fin, IMap{}, false);
    mimir_hip::DeviceModel<Layer> plain(c, m.getLayers());
    mimir_hip::DeviceModel<Layer> fused(c, m.getLayers());
    fused.setFusion(true);
    const std::vector<float> a = plain.forwardPassNamed(fin, IMap{}, false);
    const std::vector<float> b = fused.forwardPassNamed(fin, IMap{}, false);
    CHECK(a.size() == ref.size() && b.size() == ref.size() &&
          std::memcmp(a.data(), b.data(), a.size() * sizeof(float)) == 0);
    float mx = 0.f;
    for (float v : ref) mx = std::fmax(mx, std::fabs(v));
    bool ok = !ref.empty();
    for (size_t i = 0; ok && i < ref.size(); ++i) ok = std::fabs(b[i] - ref[i]) <= 1e-6f + 1e-5f * mx;
    CHECK(ok);
}

}  // namespace

int main() {
    try {
        auto& c = mimir_hip::Context::instance();
        residual_merge_kat(c);
        weight_block_and_backward(c);
        int_ids_forward(c);
        attention_at_call_site();
        attention_block_model(c);
        fused_block_model(c);
    } catch (const std::exception& e) {
        std::fprintf(stderr, "FAIL: exception %s\n", e.what());
        return 1;
    }
    if (failures) {
        std::fprintf(stderr, "%d check(s) failed\n", failures);
        return 1;
    }
    std::printf("DeviceModel<Layer> matches the reference Model: all checks passed\n");
    return 0;
}
