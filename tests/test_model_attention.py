"""The reference Model's attention layers through the compiled runtime
(oracle/_ref, Model::forwardPassNamed, Model.cpp:5904-5990): the harness
passes num_heads / head_dim / causal / seq_len / embed_dim to the reference's
Layer, so the layer computes the reference's own LayerOps function on them
(the runtime library and the op library compile those inline functions
separately, -O2 and -O3, so the two agree to the layer's float32 tolerance,
not bit for bit), and the refusals carry the messages the device runtime
reproduces."""
import numpy as np
import pytest

import model_ref as MR
import oracle as O
from _attention import assert_within, attention_layer64, cross_attention_layer64
from _attention_graphs import error_graphs, single_graphs

pytestmark = pytest.mark.skipif(not (MR.available() and O.ref_available()), reason="oracle/_ref not built")


@pytest.mark.parametrize("graph", single_graphs(), ids=lambda g: g[0])
def test_model_layer_is_the_layer_function(graph):
    name, layers, fin, iin = graph
    L = layers[0]
    w = L["weights"]
    got = MR.forward_named(layers, fin, iin)
    if L["type"] == "CrossAttention":
        e = L.get("embed_dim") or L["head_dim"] * L["num_heads"]
        lq, lk = fin["q"].size // e, fin["kv"].size // e
        parts = (w[:e * e].reshape(e, e), w[e * e:3 * e * e].reshape(e, 2 * e), w[3 * e * e:4 * e * e].reshape(e, e))
        ref = O.ref_cross_attention(fin["q"], fin["kv"], *parts, lq, lk, e, L["num_heads"], L.get("causal", False))
        _, tol = cross_attention_layer64(fin["q"].reshape(lq, e), fin["kv"].reshape(lk, e), *parts, L["num_heads"],
                                         L.get("causal", False))
    else:
        e, seq = L["embed_dim"], L["seq_len"]
        wqkv, wout = w[:3 * e * e].reshape(e, 3 * e), w[3 * e * e:].reshape(e, e)
        ref = O.ref_self_attention(fin["x"], wqkv, wout, seq, e, L["num_heads"], L["causal"],
                                   multihead=L["type"] == "MultiHeadAttention")
        _, tol = attention_layer64(fin["x"].reshape(seq, e), wqkv, wout, L["num_heads"], L["causal"])
    assert_within(got, ref.ravel(), 2 * tol.ravel(), name)


@pytest.mark.parametrize("graph", error_graphs(), ids=lambda g: g[0])
def test_model_refusals(graph):
    name, layers, fin, iin, msg = graph
    with pytest.raises(MR.RefModelError, match=msg.replace("(", r"\(").replace(")", r"\)")):
        MR.forward_named(layers, fin, iin)
