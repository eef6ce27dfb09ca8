"""The int-ids forward, Model::forwardPass(const std::vector<int>& ids,
training) (Model.cpp:1026-1349): the routing restatement
(oracle/model_oracle.py forward_ids / backward_ids) against the reference's
own Model compiled in place (oracle/_ref), in inference and training form,
with the backwardPass that follows a training forward; and the cases the
reference throws on (its narrower layer switch, int / float store lookups)."""
import zlib

import numpy as np
import pytest

import model_oracle as MO
import model_ref as MR
from _graphs import ids_error_graphs, ids_graphs
from _parity import assert_bitexact, assert_close, assert_close_sum

pytestmark = pytest.mark.skipif(not MR.available(), reason="oracle/_ref/libmimir_ref_model.so not built")


def _loss(name, n):
    return np.random.default_rng(zlib.crc32(name.encode())).standard_normal(n).astype(np.float32)


@pytest.mark.parametrize("training", [False, True])
@pytest.mark.parametrize("graph", ids_graphs(), ids=lambda g: g[0])
def test_ids_forward_matches_reference(graph, training):
    name, layers, ids = graph
    if training and any(L["type"] == "Dropout" for L in layers):
        pytest.skip("a training Dropout draws a random mask")
    ref = MR.forward_ids(layers, ids, training)
    got = MO.forward_ids(layers, ids, training)
    if name.startswith("ids_extreme") or name in ("ids_empty", "no_layers"):
        assert_bitexact(got, ref, name, allow_empty=True)  # a gather: bit for bit
    else:
        assert_close(got, ref, name)


@pytest.mark.parametrize("graph", [g for g in ids_graphs() if g[0] != "ids_default_names"], ids=lambda g: g[0])
def test_ids_backward_matches_reference(graph):
    name, layers, ids = graph
    out = MR.forward_ids(layers, ids, True)
    lg = _loss(name, out.size)
    _, (rg, rin) = MR.forward_ids(layers, ids, True, loss_grad=lg)
    gg, gin, mags = MO.backward_ids(layers, ids, lg, scales=True)
    assert (rin is None) == (gin is None)
    for i, (a, b) in enumerate(zip(gg, rg)):
        if b is not None:
            assert_close_sum(a, b, mags[i] if mags[i] is not None else np.abs(b), f"{name} grad_weights[{i}]",
                             allow_empty=True)


@pytest.mark.parametrize("graph", ids_error_graphs(), ids=lambda g: g[0])
def test_ids_errors_match_reference(graph):
    name, layers, ids = graph
    with pytest.raises(MR.RefModelError) as r:
        MR.forward_ids(layers, ids, False)
    with pytest.raises(MO.ModelError) as o:
        MO.forward_ids(layers, ids, False)
    # The reference's own message (less the layer context the device adds).
    assert str(o.value) == str(r.value), name


def test_ids_path_differs_from_the_float_path():
    """The same RMSNorm graph runs through forwardPassNamed (float ids) but
    not through the int path: the two switches are not the same."""
    name, layers, ids = ids_error_graphs()[0]
    assert name == "ids_refuses_rmsnorm"
    MR.forward_named(layers, {}, {"x": ids})
    MO.forward_named(layers, {}, {"x": ids})
