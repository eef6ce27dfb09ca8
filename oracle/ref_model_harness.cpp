// ref_model_harness.cpp -- TEST INFRASTRUCTURE ONLY.
//
// Drives the reference's own runtime, Model::forwardPassNamed
// (Model.cpp:1352-1408 -> forwardPassView, Model.cpp:4621-6824), on a layer
// list described by plain C structs.  Compiled with the reference's sources
// in place (oracle/Makefile, target `ref_model`) into
// oracle/_ref/libmimir_ref_model.so; used only to pin the routing
// restatement in oracle/model_oracle.py and to write golden fixtures.
//
// Layers are created with Model::push (Model.cpp:3096-3148), parameterised
// through Model::getMutableLayers(), given weight blocks by
// Model::allocateParams (Model.cpp:3156-3184) and filled from the spec.
#include "Model.hpp"

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
};

// Named inputs: nf float tensors and ni int tensors.  Writes at most out_cap
// floats of the returned "x" to out and its size to *out_n.  Returns 0, or 1
// when the reference throws (message copied to err).
int ref_model_forward(const ref_layer_spec* specs, int32_t n_layers, const char* const* fnames,
                      const float* const* fdata, const int64_t* fsizes, int32_t nf,
                      const char* const* inames, const int32_t* const* idata, const int64_t* isizes,
                      int32_t ni, float* out, int64_t out_cap, int64_t* out_n, char* err,
                      int32_t err_cap) {
    try {
        Model m;
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
        }
        m.allocateParams();
        for (int32_t i = 0; i < n_layers; ++i) {
            const ref_layer_spec& s = specs[i];
            if (s.params_count > 0 && s.weights) {
                float* w = layers[i].getWeights();
                std::memcpy(w, s.weights, static_cast<size_t>(s.params_count) * sizeof(float));
            }
        }
        std::unordered_map<std::string, std::vector<float>> fin;
        std::unordered_map<std::string, std::vector<int>> iin;
        for (int32_t i = 0; i < nf; ++i) fin[fnames[i]] = std::vector<float>(fdata[i], fdata[i] + fsizes[i]);
        for (int32_t i = 0; i < ni; ++i) iin[inames[i]] = std::vector<int>(idata[i], idata[i] + isizes[i]);
        const std::vector<float> y = m.forwardPassNamed(fin, iin, /*training=*/false);
        *out_n = static_cast<int64_t>(y.size());
        const size_t n = std::min(static_cast<size_t>(out_cap), y.size());
        if (n) std::memcpy(out, y.data(), n * sizeof(float));
        return 0;
    } catch (const std::exception& e) {
        if (err && err_cap > 0) {
            std::strncpy(err, e.what(), static_cast<size_t>(err_cap) - 1);
            err[err_cap - 1] = 0;
        }
        return 1;
    }
}

}  // extern "C"
