// ref_harness.cpp -- TEST INFRASTRUCTURE ONLY.
//
// A thin C-ABI around the reference's own op functions, compiled from the
// reference headers where they lie (-I $(REF)/src, see oracle/Makefile) into
// oracle/_ref/libmimir_ref.so.  Used only to pin the C restatement in
// mimir_oracle.c (tests/) and to write golden fixtures (tests/golden/); it is
// never linked into the product library.
//
// Each entry point copies the plain buffers into std::vector<float>, fills a
// reference `Layer` (Layers.hpp:86-309) with weight_block == nullptr so that
// Layer::getWeights() returns Layer::weights (Layers.hpp:232-240), calls the
// reference function and copies the result out.  Exceptions -> status 1.
#include "LayerOps.hpp"
#include "LayerOpsExt.hpp"

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <vector>

namespace {

std::vector<float> vec(const float* p, int64_t n) {
    return n > 0 ? std::vector<float>(p, p + n) : std::vector<float>();
}

int put(const std::vector<float>& v, float* out) {
    if (!v.empty()) std::memcpy(out, v.data(), v.size() * sizeof(float));
    return 0;
}

}  // namespace

extern "C" {

// LayerOps::layernorm_forward, LayerOps.hpp:264-319.  params = [gamma(n) | beta(n)].
int ref_layernorm(const float* x, int64_t N, int32_t in_features, const float* params,
                  int64_t params_len, int32_t affine, int32_t use_bias, float eps, float* y) {
    try {
        Layer L;
        L.in_features = in_features;
        L.affine = affine != 0;
        L.use_bias = use_bias != 0;
        L.eps = eps;
        L.weights = vec(params, params_len);
        return put(LayerOps::layernorm_forward(vec(x, N), L, false), y);
    } catch (...) {
        return 1;
    }
}

// LayerOpsExt::rms_norm_forward, LayerOpsExt.hpp:345-378 (whole vector).
int ref_rms_norm_forward(const float* x, int64_t N, const float* w, int64_t w_len,
                         int32_t affine, float eps, float* y) {
    try {
        Layer L;
        L.affine = affine != 0;
        L.eps = eps;
        L.weights = vec(w, w_len);
        return put(LayerOpsExt::rms_norm_forward(vec(x, N), L), y);
    } catch (...) {
        return 1;
    }
}

// Normalization::rms_norm, Layers.hpp:1003-1021 (per row, in place).
int ref_rms_norm_rows(const float* x, int64_t rows, int64_t cols, const float* gamma,
                      float eps, float* y) {
    try {
        std::vector<float> d = vec(x, rows * cols);
        std::vector<float> g = vec(gamma, cols);
        Normalization::rms_norm(d, g, static_cast<int>(cols), eps);
        return put(d, y);
    } catch (...) {
        return 1;
    }
}

// LayerOps::add_forward, LayerOps.hpp:142-199.
int ref_add(const float* a, int64_t na, const float* b, int64_t nb, float* y) {
    try {
        return put(LayerOps::add_forward(vec(a, na), vec(b, nb)), y);
    } catch (...) {
        return 1;
    }
}

// LayerOps::multiply_forward, LayerOps.hpp:205-230.
int ref_mul(const float* a, int64_t na, const float* b, int64_t nb, float* y) {
    try {
        return put(LayerOps::multiply_forward(vec(a, na), vec(b, nb)), y);
    } catch (...) {
        return 1;
    }
}

// LayerOps::softmax_inplace, LayerOps.hpp:952-974.
int ref_softmax_inplace(const float* x, int64_t rows, int64_t dim, float* y) {
    try {
        std::vector<float> d = vec(x, rows * dim);
        LayerOps::softmax_inplace(d, static_cast<int>(rows), static_cast<int>(dim));
        return put(d, y);
    } catch (...) {
        return 1;
    }
}

// LayerOps::softmax_forward, LayerOps.hpp:325-361 (Softmax or LogSoftmax layer).
int ref_softmax_forward(const float* x, int64_t n, int32_t log_softmax, float* y) {
    try {
        Layer L;
        L.type_enum = log_softmax ? LayerType::LogSoftmax : LayerType::Softmax;
        return put(LayerOps::softmax_forward(vec(x, n), L), y);
    } catch (...) {
        return 1;
    }
}

// LayerOps::gelu_forward, LayerOps.hpp:556-568.
int ref_gelu(const float* x, int64_t n, float* y) {
    try {
        return put(LayerOps::gelu_forward(vec(x, n)), y);
    } catch (...) {
        return 1;
    }
}

// LayerOps::silu_forward, LayerOps.hpp:570-581.
int ref_silu(const float* x, int64_t n, float* y) {
    try {
        return put(LayerOps::silu_forward(vec(x, n)), y);
    } catch (...) {
        return 1;
    }
}

// LayerOps::self_attention_forward, LayerOps.hpp:1004-1097: input [seq, embed],
// qkv_weight [embed, 3 embed], out_weight [embed, embed].  `multihead` calls
// LayerOps::multihead_attention_forward (:1100-1113) instead.
int ref_self_attention(const float* input, const float* qkv_weight, const float* out_weight,
                       int32_t seq_len, int32_t embed_dim, int32_t num_heads, int32_t causal,
                       int32_t multihead, float* y) {
    try {
        const int64_t e = embed_dim;
        const std::vector<float> x = vec(input, static_cast<int64_t>(seq_len) * e);
        const std::vector<float> wq = vec(qkv_weight, 3 * e * e), wo = vec(out_weight, e * e);
        return put(multihead ? LayerOps::multihead_attention_forward(x, wq, wo, seq_len, embed_dim,
                                                                     num_heads, causal != 0)
                             : LayerOps::self_attention_forward(x, wq, wo, seq_len, embed_dim,
                                                                num_heads, causal != 0),
                   y);
    } catch (...) {
        return 1;
    }
}

// LayerOps::cross_attention_forward, LayerOps.hpp:1116-1216: query_input
// [query_len, embed], kv_input [kv_len, embed], q_weight [embed, embed],
// kv_weight [embed, 2 embed], out_weight [embed, embed].
int ref_cross_attention(const float* query_input, const float* kv_input, const float* q_weight,
                        const float* kv_weight, const float* out_weight, int32_t query_len,
                        int32_t kv_len, int32_t embed_dim, int32_t num_heads, int32_t causal,
                        float* y) {
    try {
        const int64_t e = embed_dim;
        return put(LayerOps::cross_attention_forward(
                       vec(query_input, static_cast<int64_t>(query_len) * e),
                       vec(kv_input, static_cast<int64_t>(kv_len) * e), vec(q_weight, e * e),
                       vec(kv_weight, 2 * e * e), vec(out_weight, e * e), query_len, kv_len,
                       embed_dim, num_heads, causal != 0),
                   y);
    } catch (...) {
        return 1;
    }
}

// ---------------------------------------------------------------------------
// CPU baseline timing: the inputs are turned into std::vector once, then only
// the reference call(s) of the path are timed (including the output vector
// each reference op allocates and value-initialises).  Returns the median
// wall time in seconds over `reps` calls after one warm-up call, or -1.
// ---------------------------------------------------------------------------
enum RefTimedOp {
    REF_T_ADD_RMSNORM = 0,  // add_forward(x, r) then Normalization::rms_norm (per row)
    REF_T_LAYERNORM = 1,    // layernorm_forward, in_features = cols, gamma|beta in b
    REF_T_SOFTMAX = 2,      // softmax_inplace(x, rows, cols)
    REF_T_GELU = 3,         // gelu_forward
    REF_T_SILU_MUL = 4,     // multiply_forward(silu_forward(gate), up)
    REF_T_ADD = 5,          // add_forward(a, b)
};

double ref_time_op(int op, const float* a, int64_t na, const float* b, int64_t nb,
                   const float* w, int64_t nw, int64_t rows, int64_t cols, float eps, int reps) {
    try {
        const std::vector<float> va = vec(a, na), vb = vec(b, nb), vw = vec(w, nw);
        std::vector<float> work = va;
        Layer L;
        L.in_features = static_cast<int>(cols);
        L.eps = eps;
        L.weights = vw;
        volatile float sink = 0.0f;
        auto once = [&]() {
            switch (op) {
                case REF_T_ADD_RMSNORM: {
                    std::vector<float> h = LayerOps::add_forward(va, vb);
                    Normalization::rms_norm(h, vw, static_cast<int>(cols), eps);
                    sink = sink + h[0];
                    break;
                }
                case REF_T_LAYERNORM: sink = sink + LayerOps::layernorm_forward(va, L, false)[0]; break;
                case REF_T_SOFTMAX:
                    LayerOps::softmax_inplace(work, static_cast<int>(rows), static_cast<int>(cols));
                    sink = sink + work[0];
                    break;
                case REF_T_GELU: sink = sink + LayerOps::gelu_forward(va)[0]; break;
                case REF_T_SILU_MUL:
                    sink = sink + LayerOps::multiply_forward(LayerOps::silu_forward(va), vb)[0];
                    break;
                case REF_T_ADD: sink = sink + LayerOps::add_forward(va, vb)[0]; break;
                default: throw std::runtime_error("unknown op");
            }
        };
        once();
        std::vector<double> t;
        for (int i = 0; i < reps; ++i) {
            if (op == REF_T_SOFTMAX) work = va;  // fresh logits, copy not timed
            const auto t0 = std::chrono::steady_clock::now();
            once();
            const auto t1 = std::chrono::steady_clock::now();
            t.push_back(std::chrono::duration<double>(t1 - t0).count());
        }
        std::sort(t.begin(), t.end());
        return t.empty() ? -1.0 : t[t.size() / 2];
    } catch (...) {
        return -1.0;
    }
}

}  // extern "C"
