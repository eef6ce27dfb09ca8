"""The C++ adapter (mimir-framework_amd/host/mimir_layerops_hip.hpp) compiled
against the reference's own `struct Layer` (Layers.hpp:86-309, with
LayerTypes.hpp) instead of a stand-in: every function template the adapter
offers and the whole DeviceModel<Layer> class are instantiated explicitly,
so each field the adapter reads must exist with a usable type.  Syntax only
(no GPU, no link).  Skipped where the reference tree is absent."""
import os
import subprocess
import tempfile

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_SRC = "/root/reference/src"

pytestmark = pytest.mark.skipif(not os.path.exists(os.path.join(REF_SRC, "Layers.hpp")),
                                reason="reference tree absent")

TU = r'''
#include "Layers.hpp"
#include "mimir_layerops_hip.hpp"

template class mimir_hip::DeviceModel<Layer>;
template std::vector<float> mimir_hip::LayerOps::layernorm_forward<Layer>(const std::vector<float>&, const Layer&, bool);
template std::vector<float> mimir_hip::LayerOps::softmax_forward<Layer>(const std::vector<float>&, const Layer&);
template std::vector<float> mimir_hip::LayerOpsExt::rms_norm_forward<Layer>(const std::vector<float>&, const Layer&);
template std::vector<float> mimir_hip::embedding_forward<Layer>(const std::vector<int>&, const Layer&);
template std::vector<float> mimir_hip::embedding_forward_float_ids<Layer>(const std::vector<float>&, const Layer&);
'''


def _compile(src):
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "tu.cpp")
        with open(path, "w") as f:
            f.write(src)
        return subprocess.run(
            ["g++", "-std=c++17", "-fsyntax-only", "-mavx2", "-mfma", "-fopenmp", "-w",
             f"-I{REF_SRC}", f"-I{REF_SRC}/Models", f"-I{REPO}/include",
             f"-I{REPO}/mimir-framework_amd/host", path],
            capture_output=True, text=True, timeout=300)


def test_adapter_instantiates_on_the_reference_layer():
    p = _compile(TU)
    assert p.returncode == 0, p.stderr[-4000:]


def test_the_check_would_catch_a_missing_field():
    """The same instantiation against a Layer-like type without the branch
    fields must fail to compile: the check above is not vacuous."""
    p = _compile(TU.replace('#include "Layers.hpp"', '''#include "Layers.hpp"
struct NoBranch { std::string name, type, output; std::vector<std::string> inputs; int seq_len = 0;
  float eps = 1e-5f; bool affine = true, use_bias = true; int in_features = 0, vocab_size = 0, embed_dim = 0,
  padding_idx = -1; std::vector<float> grad_weights; const float* getWeights() const { return nullptr; }
  size_t getWeightsSize() const { return 0; } };''') + "template class mimir_hip::DeviceModel<NoBranch>;\n")
    assert p.returncode != 0 and "branch" in p.stderr
