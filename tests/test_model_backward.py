"""Pin the training-step restatement (oracle/model_oracle.py backward_named:
forwardPassNamed(training=true) then Model::backwardPass, Model.cpp:7307-9153)
against the reference's own Model compiled in place
(oracle/_ref/libmimir_ref_model.so) and against golden outputs of it."""
import os

import numpy as np
import pytest

import model_oracle as MO
import model_ref as MR
from _graphs import train_graphs
from _parity import assert_close, assert_close_sum

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "model_backward.npz")

needs_ref = pytest.mark.skipif(not MR.available(), reason="oracle/_ref/libmimir_ref_model.so not built")


def _compare(name, layers, got, ref):
    """Input gradients at the path's tolerance; grad_weights (float32 sums over
    tokens) at that tolerance relative to the magnitudes summed."""
    grads, gin, mags = got
    rgrads, rgin = ref
    assert (gin is None) == (rgin is None), f"{name}: input gradient presence"
    if gin is not None:
        assert_close(gin, rgin, f"{name} input gradient")
    for L, a, b, m in zip(layers, grads, rgrads, mags):
        assert (a is None) == (b is None)
        if a is not None:
            assert_close_sum(a, b, m, f"{name} {L['name']} grad_weights")


@needs_ref
@pytest.mark.parametrize("case", train_graphs(), ids=lambda c: c[0])
def test_backward_restatement_matches_reference_model(case):
    name, layers, fin, iin, lg = case
    _compare(name, layers, MO.backward_named(layers, fin, iin, lg, scales=True), MR.backward(layers, fin, iin, lg))


def gold_of(name, layers, z):
    gin = z[f"{name}/__input__"] if f"{name}/__input__" in z.files else None
    grads = [z[f"{name}/{L['name']}"] if f"{name}/{L['name']}" in z.files else None for L in layers]
    return grads, gin


def test_backward_matches_golden_reference_outputs():
    with np.load(GOLD) as z:
        for name, layers, fin, iin, lg in train_graphs():
            _compare(name, layers, MO.backward_named(layers, fin, iin, lg, scales=True), gold_of(name, layers, z))


def test_same_name_aliasing_is_the_references():
    # The reference's gradient map adds a layer's input gradient onto its own
    # output gradient when both are named "x"; a restatement that replaced it
    # instead would give different LayerNorm grad_weights.
    g = {c[0]: c for c in train_graphs()}
    name, layers, fin, iin, lg = g["same_name_aliasing"]
    with np.load(GOLD) as z:
        ref = gold_of(name, layers, z)[0][0]
    renamed = [dict(L) for L in layers]
    for i, L in enumerate(renamed):
        L["inputs"] = [f"t{i}"] * (2 if L["type"] == "Add" else 1)
        L["output"] = f"t{i + 1}" if i + 1 < len(renamed) else "x"
    fin2 = {"t0": fin["x"]}
    plain = MO.backward_named(renamed, fin2, iin, lg)[0][0]
    assert not np.allclose(plain, ref, rtol=1e-3)
