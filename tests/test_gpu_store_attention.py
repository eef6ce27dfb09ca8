"""The device runtime's attention layers (mimir_store_run with
SelfAttention / MultiHeadAttention / CrossAttention layers) against the
reference's own compiled Model::forwardPassNamed (oracle/_ref):
- each layer alone, held element-wise to the whole-layer tolerance
  (tests/_attention.py: projection rounding carried through the core and the
  output projection), against float64 and the reference;
- a pre-norm residual block (LayerNorm -> SelfAttention -> Add -> LayerNorm
  -> GELU), held normwise to 1e-4 of its largest output (each layer's
  element-wise parity is tested on its own);
- the reference's refusals, with its messages; and the int-ids forward,
  which runs SelfAttention and refuses CrossAttention as the reference does.
The training step through these layers is tested in
tests/test_gpu_attention_bwd.py."""
import numpy as np
import pytest

import mimir_hip as M
import model_ref as MR
from _attention import assert_within, attention_layer64, cross_attention_layer64
from _attention_graphs import block_graph, error_graphs, single_graphs
from _parity import assert_bitexact, assert_close_normwise

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not MR.available(), reason="oracle/_ref not built")]


@pytest.fixture(scope="module")
def store(ctx):
    s = M.Store(ctx)
    yield s
    s.close()


def _tol(layers, fin):
    L = layers[0]
    w = L["weights"]
    if L["type"] == "CrossAttention":
        e = L.get("embed_dim") or L["head_dim"] * L["num_heads"]
        parts = (w[:e * e].reshape(e, e), w[e * e:3 * e * e].reshape(e, 2 * e), w[3 * e * e:4 * e * e].reshape(e, e))
        return cross_attention_layer64(fin["q"].reshape(-1, e), fin["kv"].reshape(-1, e), *parts, L["num_heads"],
                                       L.get("causal", False))
    e, seq = L["embed_dim"], L["seq_len"]
    return attention_layer64(fin["x"].reshape(seq, e), w[:3 * e * e].reshape(e, 3 * e), w[3 * e * e:].reshape(e, e),
                             L["num_heads"], L["causal"])


@pytest.mark.parametrize("graph", single_graphs(), ids=lambda g: g[0])
def test_attention_layer_in_store(ctx, store, graph):
    name, layers, fin, iin = graph
    print(f"store attention {name}", flush=True)
    g = M.DeviceGraph(ctx, layers)
    try:
        got = store.forward_named(g, fin, iin)
        want, tol = _tol(layers, fin)
        assert_within(got, want.ravel(), tol.ravel(), name + " vs float64")
        assert_within(got, MR.forward_named(layers, fin, iin), 2 * tol.ravel(), name + " vs reference Model")
        assert_bitexact(store.forward_named(g, fin, iin), got, name + " (second run)")
    finally:
        g.close()


@pytest.mark.parametrize("causal", [False, True])
def test_attention_block_in_store(ctx, store, causal):
    name, layers, fin, iin = block_graph(causal=causal)
    g = M.DeviceGraph(ctx, layers)
    try:
        got = store.forward_named(g, fin, iin)
        assert_close_normwise(got, MR.forward_named(layers, fin, iin), name, rel=1e-4)
    finally:
        g.close()


@pytest.mark.parametrize("graph", error_graphs(), ids=lambda g: g[0])
def test_attention_refusals(ctx, store, graph):
    name, layers, fin, iin, msg = graph
    with pytest.raises(MR.RefModelError, match=msg.replace("(", r"\(").replace(")", r"\)")):
        MR.forward_named(layers, fin, iin)
    g = M.DeviceGraph(ctx, layers)
    try:
        with pytest.raises(M.MimirError) as e:
            store.forward_named(g, fin, iin)
        assert e.value.status == M.EINVAL and msg in str(e.value), str(e.value)
    finally:
        g.close()


def test_attention_in_int_ids_path(ctx, store):
    """Model::forwardPass(ids): Embedding -> SelfAttention runs (Model.cpp:
    1291-1310); CrossAttention is not in the int path's switch."""
    r = np.random.default_rng(3)
    vocab, e, seq = 20, 32, 6
    emb = dict(name="tok", type="Embedding", inputs=["x"], output="h", vocab_size=vocab, embed_dim=e,
               weights=(0.5 * r.standard_normal(vocab * e)).astype(np.float32))
    att = dict(name="attn", type="SelfAttention", inputs=["h"], output="x", seq_len=seq, embed_dim=e, num_heads=4,
               causal=True, weights=(r.standard_normal(4 * e * e) / np.sqrt(e)).astype(np.float32))
    ids = r.integers(0, vocab, seq).astype(np.int32)
    g = M.DeviceGraph(ctx, [emb, att])
    try:
        got = store.forward_ids(g, ids, training=False)
        assert_close_normwise(got, MR.forward_ids([emb, att], ids, training=False), "int path attention", rel=1e-4)
    finally:
        g.close()
    cross = dict(att, type="CrossAttention", inputs=["h", "h"])
    with pytest.raises(MR.RefModelError, match="not supported in int path: CrossAttention"):
        MR.forward_ids([emb, cross], ids, training=False)
    g = M.DeviceGraph(ctx, [emb, cross])
    try:
        with pytest.raises(M.MimirError, match="not supported in int path: CrossAttention"):
            store.forward_ids(g, ids, training=False)
    finally:
        g.close()
