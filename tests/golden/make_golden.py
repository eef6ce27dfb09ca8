"""Write the golden fixtures in this directory from the reference's own op
functions.

The reference (brit45/mimir-framework) is C++; oracle/Makefile compiles its
LayerOps.hpp / LayerOpsExt.hpp / Layers.hpp functions in place into
oracle/_ref/libmimir_ref.so (through oracle/ref_harness.cpp).  This script
runs those functions on seeded inputs and stores inputs and outputs as .npz
data, so parity stays pinned to the reference where the reference tree is
absent (the GPU box, a fresh clone).  Inputs drawn from mimir_hip.datagen are
not stored; their SHA-256 is, and the tests regenerate and check them.

Run from the repository root:  python tests/golden/make_golden.py [fixture ...]
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "oracle"))
sys.path.insert(0, os.path.join(REPO, "mimir-framework_amd"))

import oracle as O  # noqa: E402
from mimir_hip import datagen as G  # noqa: E402

SPECIALS = np.array([0.0, -0.0, 1e-30, -1e-30, 1e-40, 3.0, -3.0, 5.0, -5.0, 9.0, -9.0, 20.0,
                     -20.0, 88.0, -88.0, 100.0, -100.0, np.inf, -np.inf, np.nan], np.float32)


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main():
    if not O.ref_available():
        sys.exit("oracle/_ref/libmimir_ref.so is not built (needs the reference tree): make -C oracle")
    rng = np.random.default_rng(0x60D)
    manifest = {}

    def save(name, note, regenerated=None, **arrays):
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrays)
        manifest[name] = {
            "note": note,
            "arrays": {k: {"shape": list(v.shape), "dtype": str(v.dtype), "sha256": sha(v)}
                       for k, v in arrays.items()},
            "regenerated_inputs": regenerated or {},
        }

    # LayerOps::layernorm_forward, in_features = 512, affine, bias, eps 1e-5
    x, g, b, eps = G.cfg0_layernorm()
    y = O.ref_layernorm(x, 512, np.concatenate([g, b]), True, True, eps).reshape(x.shape)
    save("layernorm_cfg0", "LayerOps::layernorm_forward (LayerOps.hpp:264-319) on configs[0]",
         {"datagen.cfg0_layernorm": {"x": sha(x), "gamma": sha(g), "beta": sha(b)}}, y=y)

    # LayerNorm variants: odd group sizes, no bias, non-affine, one whole-vector group
    xs = (rng.standard_normal(4 * 33) * 2 + 0.5).astype(np.float32)
    gb = (1 + 0.02 * rng.standard_normal(66)).astype(np.float32)
    xw = rng.standard_normal(300).astype(np.float32)
    pw = np.concatenate([np.full(300, 1.5, np.float32), np.full(300, -0.25, np.float32)])
    save("layernorm_variants", "LayerOps::layernorm_forward variants",
         x33=xs, params33=gb,
         y33_gb=O.ref_layernorm(xs, 33, gb, True, True, 1e-5),
         y33_g=O.ref_layernorm(xs, 33, gb, True, False, 1e-5),
         y33_none=O.ref_layernorm(xs, 33, None, False, False, 1e-5),
         xw=xw, pw=pw, yw=O.ref_layernorm(xw, 0, pw, True, True, 1e-5))

    # configs[1] rows 0..7: add_forward then Normalization::rms_norm (per row)
    x, r, w, eps = G.cfg1_add_rmsnorm(rows=8)
    h = O.ref_add(x, r).reshape(x.shape)
    y = O.ref_rms_norm_rows(h, w, eps)
    save("add_rmsnorm_cfg1_rows8", "LayerOps::add_forward + Normalization::rms_norm (Layers.hpp:1003-1021) "
         "on the first 8 rows of configs[1]",
         {"datagen.cfg1_add_rmsnorm(rows=8)": {"x": sha(x), "residual": sha(r), "w": sha(w)}}, h=h, y=y)

    # RMSNorm layer, whole vector, weights shorter than the input
    xv = rng.standard_normal(1000).astype(np.float32)
    wv = (1 + 0.02 * rng.standard_normal(17)).astype(np.float32)
    save("rmsnorm_layer", "LayerOpsExt::rms_norm_forward (LayerOpsExt.hpp:345-378), whole vector",
         x=xv, w=wv, y=O.ref_rms_norm_forward(xv, wv, True, 1e-5), y_noaffine=O.ref_rms_norm_forward(xv, None, False, 1e-5))

    # configs[2] head 0, query rows 992..1023: LayerOps::softmax_inplace
    s = G.cfg2_softmax(batch=1, heads=1).reshape(1024, 1024)
    rows = s[992:]
    save("softmax_cfg2_rows", "LayerOps::softmax_inplace (LayerOps.hpp:952-974) on configs[2] head 0, "
         "query rows 992..1023", {"datagen.cfg2_softmax(batch=1, heads=1)": {"scores": sha(s)}},
         y=O.ref_softmax_inplace(rows))

    # Softmax / LogSoftmax layers (whole vector) and special rows
    v = (3 * rng.standard_normal(1000)).astype(np.float32)
    special_rows = np.stack([np.array([np.nan, 1, 2, 3, 4, 5, 6, 7], np.float32),
                             np.array([1, np.nan, 2, 3, 4, 5, 6, 7], np.float32),
                             np.array([np.inf, 1, 2, 3, 4, 5, 6, 7], np.float32),
                             np.array([1e30, -1e30, 0, 0, 0, 0, 0, 0], np.float32),
                             np.full(8, -np.inf, np.float32)])
    save("softmax_layer", "LayerOps::softmax_forward (LayerOps.hpp:325-361), Softmax and LogSoftmax",
         x=v, y=O.ref_softmax_forward(v, False), y_log=O.ref_softmax_forward(v, True),
         special=special_rows, special_y=O.ref_softmax_inplace(special_rows))

    # GELU / SiLU on a dense grid, specials and normals
    xa = np.concatenate([np.linspace(-12, 12, 8001, dtype=np.float32), SPECIALS,
                         rng.standard_normal(4096).astype(np.float32)])
    save("activations", "LayerOps::gelu_forward / silu_forward (LayerOps.hpp:556-581)",
         x=xa, gelu=O.ref_gelu(xa), silu=O.ref_silu(xa))

    # add_forward broadcast forms and multiply_forward, with IEEE specials
    a = np.tile(SPECIALS, SPECIALS.size)
    bb = np.repeat(SPECIALS, SPECIALS.size)
    big = rng.standard_normal(4096 * 3).astype(np.float32)
    small = rng.standard_normal(4096).astype(np.float32)
    save("add_mul", "LayerOps::add_forward / multiply_forward (LayerOps.hpp:142-230)",
         a=a, b=bb, add=O.ref_add(a, bb), mul=O.ref_mul(a, bb),
         big=big, small=small, add_repeat=O.ref_add(small, big),
         add_scalar=O.ref_add(big, small[:1]))

    with open(os.path.join(HERE, "MANIFEST.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
    print("wrote", sorted(manifest))




def write_model_graphs():
    """Outputs of the reference's Model::forwardPassNamed on tests/_graphs.py."""
    sys.path.insert(0, os.path.join(REPO, "tests"))
    import model_ref as MR
    from _graphs import graphs
    if not MR.available():
        sys.exit("oracle/_ref/libmimir_ref_model.so is not built: make -C oracle ref_model")
    outs = {name: MR.forward_named(layers, fin, iin) for name, layers, fin, iin in graphs()}
    np.savez_compressed(os.path.join(HERE, "model_graphs.npz"), **outs)
    path = os.path.join(HERE, "MANIFEST.json")
    manifest = json.load(open(path))
    manifest["model_graphs"] = {
        "note": "Model::forwardPassNamed (Model.cpp:1352-1408, 4621-6824) on the graphs of tests/_graphs.py",
        "arrays": {k: {"shape": list(v.shape), "dtype": str(v.dtype), "sha256": sha(v)} for k, v in outs.items()},
        "regenerated_inputs": {"tests/_graphs.py": "graphs()"},
    }
    with open(path, "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
    print("wrote model_graphs", sorted(outs))


def write_model_backward():
    """Gradients of the reference's Model::backwardPass on tests/_graphs.py
    train_graphs(): per graph, each layer's grad_weights and the gradient
    that reached "__input__"."""
    sys.path.insert(0, os.path.join(REPO, "tests"))
    import model_ref as MR
    from _graphs import train_graphs
    if not MR.available():
        sys.exit("oracle/_ref/libmimir_ref_model.so is not built: make -C oracle ref_model")
    outs = {}
    for name, layers, fin, iin, lg in train_graphs():
        grads, gin = MR.backward(layers, fin, iin, lg)
        if gin is not None:
            outs[f"{name}/__input__"] = gin
        for L, g in zip(layers, grads):
            if g is not None:
                outs[f"{name}/{L['name']}"] = g
    np.savez_compressed(os.path.join(HERE, "model_backward.npz"), **outs)
    path = os.path.join(HERE, "MANIFEST.json")
    manifest = json.load(open(path))
    manifest["model_backward"] = {
        "note": "Model::forwardPassNamed(training=true) then Model::backwardPass (Model.cpp:7307-9153) on "
                "tests/_graphs.py train_graphs(): grad_weights per layer and the __input__ gradient",
        "arrays": {k: {"shape": list(v.shape), "dtype": str(v.dtype), "sha256": sha(v)} for k, v in outs.items()},
        "regenerated_inputs": {"tests/_graphs.py": "train_graphs()"},
    }
    with open(path, "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
    print("wrote model_backward", len(outs), "arrays")


def write_safetensors_fixture():
    """tests/golden/ref_checkpoint.safetensors: Mimir::Serialization::
    save_checkpoint (SafeTensors, default options) of checkpoint_layers()."""
    sys.path.insert(0, os.path.join(REPO, "tests"))
    import model_ref as MR
    from _graphs import checkpoint_layers
    if not MR.available():
        sys.exit("oracle/_ref/libmimir_ref_model.so is not built: make -C oracle ref_model")
    path = os.path.join(HERE, "ref_checkpoint.safetensors")
    layers = checkpoint_layers()
    MR.save_safetensors(layers, path)
    data = open(path, "rb").read()
    path_manifest = os.path.join(HERE, "MANIFEST.json")
    manifest = json.load(open(path_manifest))
    manifest["ref_checkpoint"] = {
        "note": "Mimir::Serialization::save_checkpoint (SafeTensors, default SaveOptions, no git info) of "
                "tests/_graphs.py checkpoint_layers(); weights: the layers' blocks as drawn there",
        "file": {"bytes": len(data), "sha256": hashlib.sha256(data).hexdigest()},
        "regenerated_inputs": {"tests/_graphs.py": "checkpoint_layers()"},
    }
    with open(path_manifest, "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
    print("wrote ref_checkpoint.safetensors", len(data), "bytes")


def write_attention():
    """attention.npz: LayerOps::self_attention_forward (LayerOps.hpp:1004-1097)
    and cross_attention_forward (:1116-1216) on the one-hot cases of
    tests/_attention.py, in both mask modes.  The Q / K / V those cases select
    are regenerated by the tests; the outputs are stored."""
    sys.path.insert(0, os.path.join(REPO, "tests"))
    from _attention import CROSS_CASES, SELF_CASES, cross_case, self_case
    if not O.ref_available():
        sys.exit("oracle/_ref/libmimir_ref.so is not built: make -C oracle ref")
    outs = {}
    for seq, e, heads in SELF_CASES:
        x, w, q, k, v = self_case(seq, e, 1.5, seq * 1000 + e)
        for causal in (0, 1):
            outs[f"self_{seq}_{e}_{heads}_{causal}"] = O.ref_self_attention(
                x, w, np.eye(e, dtype=np.float32), seq, e, heads, bool(causal))
    for lq, lk, e, heads in CROSS_CASES:
        xq, xkv, wq, wkv, q, k, v = cross_case(lq, lk, e, 1.2, lq * 7 + lk)
        for causal in (0, 1):
            outs[f"cross_{lq}_{lk}_{e}_{heads}_{causal}"] = O.ref_cross_attention(
                xq, xkv, wq, wkv, np.eye(e, dtype=np.float32), lq, lk, e, heads, bool(causal))
    np.savez_compressed(os.path.join(HERE, "attention.npz"), **outs)
    path = os.path.join(HERE, "MANIFEST.json")
    manifest = json.load(open(path))
    manifest["attention"] = {
        "note": "LayerOps::self_attention_forward / cross_attention_forward (LayerOps.hpp:1004-1216) with "
                "one-hot inputs and an identity output projection: the attention core on the selected rows",
        "arrays": {k: {"shape": list(v.shape), "dtype": str(v.dtype), "sha256": sha(v)} for k, v in outs.items()},
        "regenerated_inputs": {"tests/_attention.py": "self_case / cross_case"},
    }
    with open(path, "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
    print("wrote attention", len(outs), "arrays")


WRITERS = {"ops": lambda: main(), "model_graphs": write_model_graphs, "model_backward": write_model_backward,
           "safetensors": write_safetensors_fixture, "attention": write_attention}

if __name__ == "__main__":
    # No argument: every fixture; else only the named ones (e.g. `attention`).
    for name in (sys.argv[1:] or list(WRITERS)):
        WRITERS[name]()
