// ref_model_harness.cpp -- TEST INFRASTRUCTURE ONLY.
//
// Drives the reference's own runtime, Model::forwardPassNamed
// (Model.cpp:1352-1408 -> forwardPassView, Model.cpp:4621-6824),
// Model::backwardPass (Model.cpp:7307-9153) and the SafeTensors
// save_checkpoint / load_checkpoint (Serialization.cpp), on a layer
// list described by plain C structs.  Compiled with the reference's sources
// in place (oracle/Makefile, target `ref_model`) into
// oracle/_ref/libmimir_ref_model.so; used only to pin the routing
// restatement in oracle/model_oracle.py and to write golden fixtures.
//
// Layers are created with Model::push (Model.cpp:3096-3148), parameterised
// through Model::getMutableLayers(), given weight blocks by
// Model::allocateParams (Model.cpp:3156-3184) and filled from the spec.
#include "Model.hpp"
#include "Serialization/Serialization.hpp"

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstring>
#include <sstream>
#include <string>
#include <unordered_map>
#include <vector>

extern "C" {

struct ref_layer_spec {
    const char* name;
    const char* type;     // reference type string, e.g. "LayerNorm", "Add"
    const char* inputs;   // comma-separated names ("" -> default {"x"})
    const char* output;   // "" -> "x"
    int64_t params_count;
    const float* weights; // params_count floats (may be null)
    float eps;
    int32_t affine;
    int32_t use_bias;
    int32_t in_features;
    int32_t vocab_size;
    int32_t embed_dim;
    int32_t padding_idx;
    int32_t seq_len;
    // Branch fields (Layers.hpp:214-219), set after Model::push's
    // detectBranchType: -1 keeps what it derived from the name.
    int32_t branch_type;
    int32_t merge_op;
    const int32_t* branch_sources;
    int32_t n_branch_sources;
    // Attention fields (Layers.hpp:174-178).
    int32_t num_heads;
    int32_t head_dim;
    int32_t causal;
};

// Layers from the specs, weights copied into the blocks allocateParams made.
static void build_model(Model& m, const ref_layer_spec* specs, int32_t n_layers) {
    for (int32_t i = 0; i < n_layers; ++i)
        m.push(specs[i].name, specs[i].type, static_cast<size_t>(specs[i].params_count));
    auto& layers = m.getMutableLayers();
    for (int32_t i = 0; i < n_layers; ++i) {
        Layer& L = layers[i];
        const ref_layer_spec& s = specs[i];
        L.inputs.clear();
        if (s.inputs && *s.inputs) {
            std::stringstream ss(s.inputs);
            std::string tok;
            while (std::getline(ss, tok, ',')) L.inputs.push_back(tok);
        }
        L.output = s.output ? s.output : "";
        L.eps = s.eps;
        L.affine = s.affine != 0;
        L.use_bias = s.use_bias != 0;
        L.in_features = s.in_features;
        L.vocab_size = s.vocab_size;
        L.embed_dim = s.embed_dim;
        L.padding_idx = s.padding_idx;
        L.seq_len = s.seq_len;
        if (s.branch_type >= 0) L.branch_type = static_cast<BranchType>(s.branch_type);
        if (s.merge_op >= 0) L.merge_op = static_cast<MergeOperation>(s.merge_op);
        L.branch_sources.assign(s.branch_sources, s.branch_sources + (s.branch_sources ? s.n_branch_sources : 0));
        L.num_heads = s.num_heads;
        L.head_dim = s.head_dim;
        L.causal = s.causal != 0;
    }
    m.allocateParams();
    for (int32_t i = 0; i < n_layers; ++i) {
        const ref_layer_spec& s = specs[i];
        if (s.params_count > 0 && s.weights) {
            float* w = layers[i].getWeights();
            std::memcpy(w, s.weights, static_cast<size_t>(s.params_count) * sizeof(float));
        }
    }
}

static void copy_error(const std::exception& e, char* err, int32_t err_cap) {
    if (err && err_cap > 0) {
        std::strncpy(err, e.what(), static_cast<size_t>(err_cap) - 1);
        err[err_cap - 1] = 0;
    }
}

static std::vector<float> run_forward(Model& m, const char* const* fnames, const float* const* fdata,
                                      const int64_t* fsizes, int32_t nf, const char* const* inames,
                                      const int32_t* const* idata, const int64_t* isizes, int32_t ni,
                                      bool training) {
    std::unordered_map<std::string, std::vector<float>> fin;
    std::unordered_map<std::string, std::vector<int>> iin;
    for (int32_t i = 0; i < nf; ++i) fin[fnames[i]] = std::vector<float>(fdata[i], fdata[i] + fsizes[i]);
    for (int32_t i = 0; i < ni; ++i) iin[inames[i]] = std::vector<int>(idata[i], idata[i] + isizes[i]);
    return m.forwardPassNamed(fin, iin, training);
}

// Named inputs: nf float tensors and ni int tensors.  Writes at most out_cap
// floats of the returned "x" to out and its size to *out_n.  Returns 0, or 1
// when the reference throws (message copied to err).  `training` is
// forwardPassNamed's flag (the training form applies residual merges).
int ref_model_forward(const ref_layer_spec* specs, int32_t n_layers, const char* const* fnames,
                      const float* const* fdata, const int64_t* fsizes, int32_t nf,
                      const char* const* inames, const int32_t* const* idata, const int64_t* isizes,
                      int32_t ni, float* out, int64_t out_cap, int64_t* out_n, char* err,
                      int32_t err_cap, int32_t training) {
    try {
        Model m;
        build_model(m, specs, n_layers);
        const std::vector<float> y =
            run_forward(m, fnames, fdata, fsizes, nf, inames, idata, isizes, ni, training != 0);
        *out_n = static_cast<int64_t>(y.size());
        const size_t n = std::min(static_cast<size_t>(out_cap), y.size());
        if (n) std::memcpy(out, y.data(), n * sizeof(float));
        return 0;
    } catch (const std::exception& e) {
        copy_error(e, err, err_cap);
        return 1;
    }
}

// Training step without the optimizer: forwardPassNamed(training=true), then
// Model::backwardPass(loss_grad) (Model.cpp:7307-9153).  Per layer i with
// grads_out[i] non-null, writes params_count floats of Layer::grad_weights
// (zeros where the reference left it empty).  The gradient that reached the
// tensor "__input__" (Model::getLastInputGradient) goes to in_grad (at most
// in_cap floats; *in_n = its size, or -1 when none reached it).
int ref_model_backward(const ref_layer_spec* specs, int32_t n_layers, const char* const* fnames,
                       const float* const* fdata, const int64_t* fsizes, int32_t nf,
                       const char* const* inames, const int32_t* const* idata, const int64_t* isizes,
                       int32_t ni, const float* loss_grad, int64_t n_grad, float* const* grads_out,
                       float* in_grad, int64_t in_cap, int64_t* in_n, char* err, int32_t err_cap) {
    try {
        Model m;
        build_model(m, specs, n_layers);
        run_forward(m, fnames, fdata, fsizes, nf, inames, idata, isizes, ni, true);
        m.backwardPass(std::vector<float>(loss_grad, loss_grad + n_grad));
        const auto& layers = m.getLayers();
        for (int32_t i = 0; i < n_layers; ++i) {
            if (!grads_out || !grads_out[i]) continue;
            const size_t pc = static_cast<size_t>(specs[i].params_count);
            const std::vector<float>& g = layers[i].grad_weights;
            for (size_t k = 0; k < pc; ++k) grads_out[i][k] = k < g.size() ? g[k] : 0.0f;
        }
        *in_n = -1;
        if (m.hasLastInputGradient()) {
            const std::vector<float>& g = m.getLastInputGradient();
            *in_n = static_cast<int64_t>(g.size());
            const size_t n = std::min(static_cast<size_t>(in_cap), g.size());
            if (n) std::memcpy(in_grad, g.data(), n * sizeof(float));
        }
        return 0;
    } catch (const std::exception& e) {
        copy_error(e, err, err_cap);
        return 1;
    }
}

// The int-ids forward, Model::forwardPass(const std::vector<int>&, training)
// (Model.cpp:1026-1349).  Writes at most out_cap floats of the result to out
// and its size to *out_n.  With loss_grad non-null, a training forward is
// followed by Model::backwardPass(loss_grad): grad_weights to grads_out[i],
// the "__input__" gradient to in_grad (*in_n = -1 when none reached it), as
// ref_model_backward.  Returns 0, or 1 when the reference throws.
int ref_model_forward_ids(const ref_layer_spec* specs, int32_t n_layers, const int32_t* ids, int64_t n_ids,
                          int32_t training, float* out, int64_t out_cap, int64_t* out_n, const float* loss_grad,
                          int64_t n_grad, float* const* grads_out, float* in_grad, int64_t in_cap, int64_t* in_n,
                          char* err, int32_t err_cap) {
    try {
        Model m;
        build_model(m, specs, n_layers);
        const std::vector<int> v(ids, ids + n_ids);
        const std::vector<float> y = m.forwardPass(v, training != 0);
        *out_n = static_cast<int64_t>(y.size());
        const size_t n = std::min(static_cast<size_t>(out_cap), y.size());
        if (n) std::memcpy(out, y.data(), n * sizeof(float));
        if (loss_grad) {
            m.backwardPass(std::vector<float>(loss_grad, loss_grad + n_grad));
            const auto& layers = m.getLayers();
            for (int32_t i = 0; i < n_layers; ++i) {
                if (!grads_out || !grads_out[i]) continue;
                const size_t pc = static_cast<size_t>(specs[i].params_count);
                const std::vector<float>& g = layers[i].grad_weights;
                for (size_t k = 0; k < pc; ++k) grads_out[i][k] = k < g.size() ? g[k] : 0.0f;
            }
            *in_n = -1;
            if (m.hasLastInputGradient()) {
                const std::vector<float>& g = m.getLastInputGradient();
                *in_n = static_cast<int64_t>(g.size());
                const size_t k = std::min(static_cast<size_t>(in_cap), g.size());
                if (k) std::memcpy(in_grad, g.data(), k * sizeof(float));
            }
        }
        return 0;
    } catch (const std::exception& e) {
        copy_error(e, err, err_cap);
        return 1;
    }
}

// Mimir::Serialization::save_checkpoint (Serialization.cpp) of a model built
// from the specs, SafeTensors format, the reference's default SaveOptions.
int ref_model_save_safetensors(const ref_layer_spec* specs, int32_t n_layers, const char* path, char* err,
                               int32_t err_cap) {
    try {
        Model m;
        build_model(m, specs, n_layers);
        Mimir::Serialization::SaveOptions o;
        o.format = Mimir::Serialization::CheckpointFormat::SafeTensors;
        o.include_git_info = false;
        std::string e;
        if (!Mimir::Serialization::save_checkpoint(m, path, o, &e)) {
            if (err && err_cap > 0) {
                std::strncpy(err, e.c_str(), static_cast<size_t>(err_cap) - 1);
                err[err_cap - 1] = 0;
            }
            return 1;
        }
        return 0;
    } catch (const std::exception& e) {
        copy_error(e, err, err_cap);
        return 1;
    }
}

// Mimir::Serialization::load_checkpoint (SafeTensors, weights only: no
// tokenizer / encoder / optimizer) into a model built from the specs; each
// layer's weight block afterwards goes to weights_out[i] (params_count
// floats, when non-null).  Returns 0, or 1 with the reference's message.
int ref_model_load_safetensors(const ref_layer_spec* specs, int32_t n_layers, const char* path, int32_t strict,
                               float* const* weights_out, char* err, int32_t err_cap) {
    try {
        Model m;
        build_model(m, specs, n_layers);
        Mimir::Serialization::LoadOptions o;
        o.format = Mimir::Serialization::CheckpointFormat::SafeTensors;
        o.strict_mode = strict != 0;
        o.load_tokenizer = false;
        o.load_encoder = false;
        o.load_optimizer = false;
        std::string e;
        if (!Mimir::Serialization::load_checkpoint(m, path, o, &e)) {
            if (err && err_cap > 0) {
                std::strncpy(err, e.c_str(), static_cast<size_t>(err_cap) - 1);
                err[err_cap - 1] = 0;
            }
            return 1;
        }
        auto& layers = m.getMutableLayers();
        for (int32_t i = 0; i < n_layers; ++i) {
            if (!weights_out || !weights_out[i] || specs[i].params_count <= 0) continue;
            std::memcpy(weights_out[i], layers[i].getWeights(), static_cast<size_t>(specs[i].params_count) * 4);
        }
        return 0;
    } catch (const std::exception& e) {
        copy_error(e, err, err_cap);
        return 1;
    }
}

// Seconds per Model::forwardPassNamed(training=false) of a model built once
// from the specs: the median of `reps` timed calls after one untimed call.
// -1 when the reference throws.
double ref_time_forward_named(const ref_layer_spec* specs, int32_t n_layers, const char* const* fnames,
                              const float* const* fdata, const int64_t* fsizes, int32_t nf,
                              const char* const* inames, const int32_t* const* idata, const int64_t* isizes,
                              int32_t ni, int32_t reps) {
    try {
        Model m;
        build_model(m, specs, n_layers);
        std::unordered_map<std::string, std::vector<float>> fin;
        std::unordered_map<std::string, std::vector<int>> iin;
        for (int32_t i = 0; i < nf; ++i) fin[fnames[i]] = std::vector<float>(fdata[i], fdata[i] + fsizes[i]);
        for (int32_t i = 0; i < ni; ++i) iin[inames[i]] = std::vector<int>(idata[i], idata[i] + isizes[i]);
        std::vector<double> t;
        for (int32_t r = 0; r <= reps; ++r) {
            const auto t0 = std::chrono::steady_clock::now();
            const std::vector<float> y = m.forwardPassNamed(fin, iin, false);
            const auto t1 = std::chrono::steady_clock::now();
            if (y.empty()) return -1.0;
            if (r > 0) t.push_back(std::chrono::duration<double>(t1 - t0).count());
        }
        std::sort(t.begin(), t.end());
        return t.empty() ? -1.0 : t[t.size() / 2];
    } catch (...) {
        return -1.0;
    }
}

// Seconds per training step -- Model::forwardPassNamed(training=true) then
// Model::backwardPass(loss_grad) -- of a model built once from the specs:
// the median of `reps` timed steps after one untimed step.  -1 when the
// reference throws.
double ref_time_train_step(const ref_layer_spec* specs, int32_t n_layers, const char* const* fnames,
                           const float* const* fdata, const int64_t* fsizes, int32_t nf,
                           const char* const* inames, const int32_t* const* idata, const int64_t* isizes,
                           int32_t ni, const float* loss_grad, int64_t n_grad, int32_t reps) {
    try {
        Model m;
        build_model(m, specs, n_layers);
        std::unordered_map<std::string, std::vector<float>> fin;
        std::unordered_map<std::string, std::vector<int>> iin;
        for (int32_t i = 0; i < nf; ++i) fin[fnames[i]] = std::vector<float>(fdata[i], fdata[i] + fsizes[i]);
        for (int32_t i = 0; i < ni; ++i) iin[inames[i]] = std::vector<int>(idata[i], idata[i] + isizes[i]);
        const std::vector<float> lg(loss_grad, loss_grad + n_grad);
        std::vector<double> t;
        for (int32_t r = 0; r <= reps; ++r) {
            const auto t0 = std::chrono::steady_clock::now();
            m.forwardPassNamed(fin, iin, true);
            m.backwardPass(lg);
            const auto t1 = std::chrono::steady_clock::now();
            if (r > 0) t.push_back(std::chrono::duration<double>(t1 - t0).count());
        }
        std::sort(t.begin(), t.end());
        return t.empty() ? -1.0 : t[t.size() / 2];
    } catch (...) {
        return -1.0;
    }
}

// Seconds per Mimir::Serialization::load_checkpoint (SafeTensors, weights
// only) into a model built once from the specs: the median of `reps` timed
// calls after one untimed call (page cache warm).  -1 on failure.
double ref_time_safetensors_load(const ref_layer_spec* specs, int32_t n_layers, const char* path, int32_t reps) {
    try {
        Model m;
        build_model(m, specs, n_layers);
        Mimir::Serialization::LoadOptions o;
        o.format = Mimir::Serialization::CheckpointFormat::SafeTensors;
        o.load_tokenizer = false;
        o.load_encoder = false;
        o.load_optimizer = false;
        std::vector<double> t;
        for (int32_t r = 0; r <= reps; ++r) {
            const auto t0 = std::chrono::steady_clock::now();
            if (!Mimir::Serialization::load_checkpoint(m, path, o, nullptr)) return -1.0;
            const auto t1 = std::chrono::steady_clock::now();
            if (r > 0) t.push_back(std::chrono::duration<double>(t1 - t0).count());
        }
        std::sort(t.begin(), t.end());
        return t.empty() ? -1.0 : t[t.size() / 2];
    } catch (...) {
        return -1.0;
    }
}

}  // extern "C"
