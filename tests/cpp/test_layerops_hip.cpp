// test_layerops_hip.cpp -- the reference's known-answer tests for this path,
// run through the C++ adapter (mimir_layerops_hip.hpp) on the GPU.  Same
// inputs, expected values and absolute tolerances as brit45/mimir-framework
// Tests/ (file:line per block); standalone main() returning 0 / 1 like the
// reference's CTest programs.  Run by tests/test_gpu_cpp_adapter.py.
#include "mimir_layerops_hip.hpp"

#include <atomic>
#include <cmath>
#include <cstdio>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

namespace {

// The fields of the reference's `struct Layer` (Layers.hpp:86-309) the
// adapter reads; weights live in a plain vector as with weight_block == nullptr.
enum class LayerType { Softmax, LogSoftmax, Other };
enum class BranchType { NONE, RESIDUAL };
enum class MergeOperation { ADD, MULTIPLY, CONCATENATE, MAX, AVERAGE };

struct TestLayer {
    std::string name;
    std::string type;
    std::vector<std::string> inputs;
    std::string output;
    int seq_len = 0;
    LayerType type_enum = LayerType::Other;
    float eps = 1e-5f;
    bool affine = true;
    bool use_bias = true;
    int in_features = 0;
    int vocab_size = 0;
    int embed_dim = 0;
    int padding_idx = -1;
    std::vector<float> weights;
    std::vector<float> grad_weights;
    BranchType branch_type = BranchType::NONE;
    MergeOperation merge_op = MergeOperation::ADD;
    std::vector<int> branch_sources;
    int num_heads = 8;  // Layers.hpp:175
    int head_dim = 0;
    bool causal = false;
    const float* getWeights() const { return weights.data(); }
    size_t getWeightsSize() const { return weights.size(); }
};

bool nearf(float a, float b, float eps) { return std::fabs(a - b) <= eps; }

int failures = 0;

#define CHECK(cond)                                                   \
    do {                                                              \
        if (!(cond)) {                                                \
            std::fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond); \
            ++failures;                                               \
        }                                                             \
    } while (0)
#define CHECK_NEAR(a, b, e) CHECK(nearf((a), (b), (e)))

float sigmoid(float x) { return 1.0f / (1.0f + std::exp(-x)); }

template <class F>
bool throws(F f) {
    try {
        f();
    } catch (const std::runtime_error&) {
        return true;
    }
    return false;
}

}  // namespace

int main() {
    namespace LO = mimir_hip::LayerOps;
    try {
        // Tests/test_layers_all_types.cpp:203-239 -- activations
        {
            const std::vector<float> x = {-1.0f, 0.0f, 1.0f};
            const auto silu = LO::silu_forward(x);
            CHECK(silu.size() == 3);
            CHECK_NEAR(silu[1], 0.0f, 1e-6f);
            CHECK_NEAR(silu[2], 1.0f * sigmoid(1.0f), 1e-6f);
            const auto gelu = LO::gelu_forward({0.0f, 1.0f});
            CHECK(gelu.size() == 2);
            CHECK_NEAR(gelu[0], 0.0f, 1e-6f);
            CHECK_NEAR(gelu[1], 0.8413f, 2e-3f);
        }
        // :242-262 -- Softmax / LogSoftmax layers
        {
            TestLayer L;
            L.type_enum = LayerType::Softmax;
            const auto sm = LO::softmax_forward({0.0f, 0.0f}, L);
            CHECK(sm.size() == 2);
            CHECK_NEAR(sm[0], 0.5f, 1e-6f);
            CHECK_NEAR(sm[1], 0.5f, 1e-6f);
            L.type_enum = LayerType::LogSoftmax;
            const auto lsm = LO::softmax_forward({0.0f, 0.0f}, L);
            const float ln2 = std::log(2.0f);
            CHECK_NEAR(lsm[0], -ln2, 1e-5f);
            CHECK_NEAR(lsm[1], -ln2, 1e-5f);
        }
        // :265-301 -- LayerNorm, in_features = 4, gamma = 1, beta = 0, eps = 1e-6
        {
            TestLayer L;
            L.in_features = 4;
            L.eps = 1e-6f;
            L.weights = {1, 1, 1, 1, 0, 0, 0, 0};
            const auto out = LO::layernorm_forward({1, 2, 3, 4}, L, false);
            CHECK(out.size() == 4);
            float mean = 0.0f;
            for (float v : out) mean += v;
            mean /= 4.0f;
            float var = 0.0f;
            for (float v : out) var += (v - mean) * (v - mean);
            var /= 4.0f;
            CHECK_NEAR(mean, 0.0f, 1e-5f);
            CHECK_NEAR(var, 1.0f, 1e-4f);
            L.in_features = 3;  // :276-279, 4 % 3 != 0
            CHECK(throws([&] { LO::layernorm_forward({1, 2, 3, 4}, L); }));
        }
        // :304-323 -- RMSNorm layer (whole vector), w = 1, eps = 1e-6
        {
            TestLayer L;
            L.eps = 1e-6f;
            L.weights = {1.0f, 1.0f};
            const auto out = mimir_hip::LayerOpsExt::rms_norm_forward({3.0f, 4.0f}, L);
            const float rms = std::sqrt((9.0f + 16.0f) / 2.0f + 1e-6f);
            CHECK(out.size() == 2);
            CHECK_NEAR(out[0], 3.0f / rms, 1e-5f);
            CHECK_NEAR(out[1], 4.0f / rms, 1e-5f);
        }
        // :392-422 -- Add / Multiply
        {
            const std::vector<float> x = {1, 2, 3}, y = {4, 5, 6};
            const auto add = LO::add_forward(x, y);
            CHECK(add.size() == 3);
            CHECK_NEAR(add[0], 5.0f, 1e-6f);
            CHECK_NEAR(add[1], 7.0f, 1e-6f);
            CHECK_NEAR(add[2], 9.0f, 1e-6f);
            const auto mul = LO::multiply_forward(x, y);
            CHECK_NEAR(mul[0], 4.0f, 1e-6f);
            CHECK_NEAR(mul[1], 10.0f, 1e-6f);
            CHECK_NEAR(mul[2], 18.0f, 1e-6f);
            // LayerOps.hpp:150-152, :191, :209-211
            CHECK(throws([&] { LO::add_forward(x, {}); }));
            CHECK(throws([&] { LO::add_forward({1, 2, 3, 4, 5}, {1, 2}); }));
            CHECK(throws([&] { LO::multiply_forward(x, {1, 2}); }));
            // broadcast: (d_model) + (seq_len * d_model)
            const auto rep = LO::add_forward({1, 2, 3, 4, 5, 6, 7, 8}, {10, 20, 30, 40});
            CHECK(rep.size() == 8 && rep[0] == 11.0f && rep[4] == 15.0f && rep[7] == 48.0f);
            const auto sc = LO::add_forward({0.5f}, {1, 2, 3});
            CHECK(sc.size() == 3 && sc[0] == 1.5f && sc[2] == 3.5f);
        }
        // Tests/test_layers_named_routing.cpp:14-15,39-51 -- sum = a + b; x = sum * c
        {
            const auto s = LO::add_forward({1.0f, 2.0f}, {3.0f, 4.0f});
            const auto x = LO::multiply_forward(s, {2.0f, 2.0f});
            CHECK_NEAR(x[0], 8.0f, 1e-6f);
            CHECK_NEAR(x[1], 12.0f, 1e-6f);
        }
        // Tests/test_runtime_residual_merge.cpp:26-29,46-47 -- x*scale + skip
        {
            const std::vector<float> x = {1.0f, 2.0f};
            const auto out = LO::add_forward(LO::multiply_forward(x, {2.0f, 3.0f}), x);
            CHECK_NEAR(out[0], 3.0f, 1e-6f);
            CHECK_NEAR(out[1], 8.0f, 1e-6f);
        }
        // Tests/test_layers_all_types.cpp:509-533 -- Embedding, float ids
        {
            TestLayer L;
            L.vocab_size = 3;
            L.embed_dim = 2;
            L.weights = {0, 0, 1, 10, 2, 20};
            const auto out = mimir_hip::embedding_forward_float_ids({1.0f, 2.0f}, L);
            CHECK(out.size() == 4);
            CHECK_NEAR(out[0], 1.0f, 1e-6f);
            CHECK_NEAR(out[1], 10.0f, 1e-6f);
            CHECK_NEAR(out[2], 2.0f, 1e-6f);
            CHECK_NEAR(out[3], 20.0f, 1e-6f);
        }
        // Tests/test_runtime_embedding_int_inputs.cpp:8-18,45-74 -- int ids, padding_idx = 0
        {
            TestLayer L;
            L.vocab_size = 4;
            L.embed_dim = 4;
            L.padding_idx = 0;
            for (int id = 0; id < 4; ++id)
                for (int d = 0; d < 4; ++d) L.weights.push_back(static_cast<float>(id * 10 + d));
            auto out = mimir_hip::embedding_forward({1, 0, 2}, L);
            CHECK(out.size() == 12);
            CHECK_NEAR(out[0], 10.0f, 1e-6f);
            CHECK_NEAR(out[3], 13.0f, 1e-6f);
            for (int i = 4; i < 8; ++i) CHECK_NEAR(out[i], 0.0f, 1e-6f);
            CHECK_NEAR(out[8], 20.0f, 1e-6f);
            CHECK_NEAR(out[11], 23.0f, 1e-6f);
            out = mimir_hip::embedding_forward(std::vector<int>(5, 0), L);  // seq_len pad ids
            CHECK(out.size() == 20);
            for (float v : out) CHECK_NEAR(v, 0.0f, 1e-6f);
            L.weights.resize(15);  // Model.cpp:1181-1182
            CHECK(throws([&] { mimir_hip::embedding_forward({1}, L); }));
        }
        // LayerOps::softmax_inplace rows (LayerOps.hpp:952-974): causal 2x2
        {
            std::vector<float> s = {0.0f, -INFINITY, 0.0f, 0.0f};
            LO::softmax_inplace(s, 2, 2);
            CHECK_NEAR(s[0], 1.0f, 1e-6f);
            CHECK(s[1] == 0.0f);
            CHECK_NEAR(s[2], 0.5f, 1e-6f);
            CHECK_NEAR(s[3], 0.5f, 1e-6f);
        }
        // Device-resident chain: h = x + r (in place), y = RMSNorm(h) -- matches the
        // host composition add_forward then Normalization::rms_norm.
        {
            auto& c = mimir_hip::Context::instance();
            const int rows = 3, cols = 4096;
            std::vector<float> x(rows * cols), r(rows * cols), w(cols, 1.0f);
            for (int i = 0; i < rows * cols; ++i) {
                x[i] = std::sin(0.37f * i);
                r[i] = std::cos(0.11f * i);
            }
            mimir_hip::DeviceBuffer<float> dx(c, x), dr(c, r), dw(c, w), dy(c, x.size());
            mimir_hip::device::add_rmsnorm(c, dx.data(), dr.data(), dr.data(), dw.data(), dy.data(), rows,
                                           cols, 1e-6f);
            const auto h = dr.download();
            const auto y = dy.download();
            auto h_ref = LO::add_forward(x, r);
            CHECK(h == h_ref);  // bit-exact residual
            mimir_hip::Normalization::rms_norm(h_ref, w, cols, 1e-6f);
            for (size_t i = 0; i < y.size(); ++i)
                CHECK(std::fabs(y[i] - h_ref[i]) <= std::fmax(1e-6f, 1e-5f * std::fabs(h_ref[i])));
        }
        // Device-resident runtime: the reference runtime KATs through
        // DeviceModel::forwardPassNamed (Tests/test_layers_named_routing.cpp:14-51,
        // Tests/test_runtime_embedding_int_inputs.cpp:8-74).
        {
            auto& c = mimir_hip::Context::instance();
            std::vector<TestLayer> layers(2);
            layers[0].name = "sum";
            layers[0].type = "Add";
            layers[0].inputs = {"a", "b"};
            layers[0].output = "sum";
            layers[1].name = "x";
            layers[1].type = "Multiply";
            layers[1].inputs = {"sum", "c"};
            layers[1].output = "x";
            mimir_hip::DeviceModel<TestLayer> m(c, layers);
            std::unordered_map<std::string, std::vector<float>> fin{
                {"x", {0, 0}}, {"a", {1, 2}}, {"b", {3, 4}}, {"c", {2, 2}}};
            const auto out = m.forwardPassNamed(fin, {});
            CHECK(out.size() == 2);
            CHECK_NEAR(out[0], 8.0f, 1e-6f);
            CHECK_NEAR(out[1], 12.0f, 1e-6f);
            fin.erase("c");  // a missing named input throws
            CHECK(throws([&] { m.forwardPassNamed(fin, {}); }));

            std::vector<TestLayer> emb(1);
            emb[0].name = "emb";
            emb[0].type = "Embedding";
            emb[0].inputs = {"ids"};
            emb[0].output = "x";
            emb[0].vocab_size = 4;
            emb[0].embed_dim = 4;
            emb[0].padding_idx = 0;
            emb[0].seq_len = 5;
            for (int id = 0; id < 4; ++id)
                for (int d = 0; d < 4; ++d) emb[0].weights.push_back(static_cast<float>(id * 10 + d));
            mimir_hip::DeviceModel<TestLayer> me(c, emb);
            auto e = me.forwardPassNamed({}, {{"ids", {1, 0, 2}}});
            CHECK(e.size() == 12);
            CHECK_NEAR(e[0], 10.0f, 1e-6f);
            CHECK_NEAR(e[5], 0.0f, 1e-6f);
            CHECK_NEAR(e[11], 23.0f, 1e-6f);
            e = me.forwardPassNamed({}, {});  // missing ids -> seq_len padding ids -> zeros
            CHECK(e.size() == 20);
            for (float v : e) CHECK_NEAR(v, 0.0f, 1e-6f);
        }
        // Training step: DeviceModel::forwardPassNamed(training=true) then
        // backwardPass (Model.cpp:7307-9153), closed-form answers.
        {
            auto& c = mimir_hip::Context::instance();
            // d(__input__) of x = __input__ * c is loss * c (Multiply branch, :7647-7665).
            std::vector<TestLayer> mul(1);
            mul[0].name = "m";
            mul[0].type = "Multiply";
            mul[0].inputs = {"__input__", "c"};
            mul[0].output = "x";
            mimir_hip::DeviceModel<TestLayer> mm(c, mul);
            mm.forwardPassNamed({{"__input__", {1, 2}}, {"c", {3, 4}}}, {}, true);
            mm.backwardPass({1, 1}, mul);
            CHECK(mm.hasLastInputGradient());
            CHECK(mm.getLastInputGradient() == std::vector<float>({3, 4}));
            // LayerNorm over [1, 3]: xhat = [-1, 1] (up to eps), loss [1, 2]:
            // dgamma = loss * xhat, dbeta = loss, dx = 0 (:7719-7821).
            std::vector<TestLayer> ln(1);
            ln[0].name = "ln";
            ln[0].type = "LayerNorm";
            ln[0].inputs = {"__input__"};
            ln[0].output = "x";
            ln[0].in_features = 2;
            ln[0].weights = {1, 1, 0, 0};
            mimir_hip::DeviceModel<TestLayer> ml(c, ln);
            ml.forwardPassNamed({{"__input__", {1, 3}}}, {}, true);
            ml.backwardPass({1, 2}, ln);
            CHECK(ln[0].grad_weights.size() == 4);
            CHECK_NEAR(ln[0].grad_weights[0], -1.0f, 1e-4f);
            CHECK_NEAR(ln[0].grad_weights[1], 2.0f, 1e-4f);
            CHECK_NEAR(ln[0].grad_weights[2], 1.0f, 1e-6f);
            CHECK_NEAR(ln[0].grad_weights[3], 2.0f, 1e-6f);
            CHECK_NEAR(ml.getLastInputGradient()[0], 0.0f, 1e-5f);
            CHECK_NEAR(ml.getLastInputGradient()[1], 0.0f, 1e-5f);
            ml.forwardPassNamed({{"__input__", {1, 3}}}, {}, true);  // grad_weights accumulate across steps
            ml.backwardPass({1, 2}, ln);
            CHECK_NEAR(ln[0].grad_weights[3], 4.0f, 1e-6f);
            // Embedding scatter-add (:7429-7461): ids [1, 0, 2, 1], padding 0, dim 2.
            std::vector<TestLayer> emb(1);
            emb[0].name = "emb";
            emb[0].type = "Embedding";
            emb[0].inputs = {"ids"};
            emb[0].output = "x";
            emb[0].vocab_size = 3;
            emb[0].embed_dim = 2;
            emb[0].padding_idx = 0;
            emb[0].weights.assign(6, 0.5f);
            mimir_hip::DeviceModel<TestLayer> me(c, emb);
            me.forwardPassNamed({}, {{"ids", {1, 0, 2, 1}}}, true);
            me.backwardPass({1, 2, 3, 4, 5, 6, 7, 8}, emb);
            CHECK(emb[0].grad_weights == std::vector<float>({0, 0, 8, 10, 5, 6}));
        }
        {
            // The host-vector mirrors share Context::instance() and hold its
            // lock per call: four host threads calling them at once must get
            // what one thread gets.
            TestLayer ln;
            ln.in_features = 256;
            ln.weights.resize(512);
            for (int i = 0; i < 512; ++i) ln.weights[i] = i < 256 ? 1.0f + 0.001f * i : 0.01f * (i - 256);
            std::vector<float> xs(64 * 256);
            for (size_t i = 0; i < xs.size(); ++i) xs[i] = std::sin(0.37f * static_cast<float>(i)) * 3.0f;
            const std::vector<float> want_ln = mimir_hip::LayerOps::layernorm_forward(xs, ln);
            std::vector<float> want_sm = xs;
            mimir_hip::LayerOps::softmax_inplace(want_sm, 64, 256);
            const std::vector<float> want_add = mimir_hip::LayerOps::add_forward(xs, want_ln);
            std::atomic<int> bad{0};
            std::vector<std::thread> pool;
            for (int t = 0; t < 4; ++t)
                pool.emplace_back([&] {
                    try {
                        for (int k = 0; k < 25; ++k) {
                            if (mimir_hip::LayerOps::layernorm_forward(xs, ln) != want_ln) ++bad;
                            std::vector<float> sm = xs;
                            mimir_hip::LayerOps::softmax_inplace(sm, 64, 256);
                            if (sm != want_sm) ++bad;
                            if (mimir_hip::LayerOps::add_forward(xs, want_ln) != want_add) ++bad;
                        }
                    } catch (const std::exception& e) {
                        std::fprintf(stderr, "FAIL: thread exception: %s\n", e.what());
                        ++bad;
                    }
                });
            for (auto& th : pool) th.join();
            CHECK(bad.load() == 0);
        }
    } catch (const std::exception& e) {
        std::fprintf(stderr, "FAIL: unexpected exception: %s\n", e.what());
        return 1;
    }
    if (failures) {
        std::fprintf(stderr, "%d check(s) failed\n", failures);
        return 1;
    }
    std::printf("test_layerops_hip: all checks passed\n");
    return 0;
}
