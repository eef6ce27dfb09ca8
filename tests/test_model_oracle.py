"""Pin the runtime-routing restatement (oracle/model_oracle.py) against the
reference's own Model::forwardPassNamed, compiled in place into
oracle/_ref/libmimir_ref_model.so, and against golden outputs of it."""
import json
import os

import numpy as np
import pytest

import model_oracle as MO
import model_ref as MR
from _graphs import error_graphs, graphs
from _parity import assert_close

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "model_graphs.npz")

needs_ref = pytest.mark.skipif(not MR.available(), reason="oracle/_ref/libmimir_ref_model.so not built")


@needs_ref
@pytest.mark.parametrize("case", graphs(), ids=lambda c: c[0])
def test_routing_matches_reference_model(case):
    name, layers, fin, iin = case
    ref = MR.forward_named(layers, fin, iin)
    got = MO.forward_named(layers, fin, iin)
    assert_close(got, ref, name)


@needs_ref
@pytest.mark.parametrize("case", error_graphs(), ids=lambda c: c[0])
def test_errors_match_reference_model(case):
    name, layers, fin, iin = case
    with pytest.raises(MR.RefModelError):
        MR.forward_named(layers, fin, iin)
    with pytest.raises(MO.ModelError):
        MO.forward_named(layers, fin, iin)


def test_routing_matches_golden_reference_outputs():
    with np.load(GOLD) as z:
        gold = {k: z[k] for k in z.files}
    for name, layers, fin, iin in graphs():
        assert_close(MO.forward_named(layers, fin, iin), gold[name], name)


def test_reference_kats_through_routing():
    # Tests/test_layers_named_routing.cpp:43-51 and test_runtime_embedding_int_inputs.cpp:45-74
    g = {c[0]: c for c in graphs()}
    _, layers, fin, iin = g["named_routing"]
    np.testing.assert_allclose(MO.forward_named(layers, fin, iin), [8, 12], atol=1e-6)
    _, layers, fin, iin = g["embedding_int_ids"]
    np.testing.assert_allclose(MO.forward_named(layers, fin, iin),
                               [10, 11, 12, 13, 0, 0, 0, 0, 20, 21, 22, 23], atol=1e-6)
    _, layers, fin, iin = g["embedding_missing_ids"]
    out = MO.forward_named(layers, fin, iin)
    assert out.shape == (20,) and not out.any()
