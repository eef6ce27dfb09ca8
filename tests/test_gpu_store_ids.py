"""The int-ids forward on the device (mimir_store_set_input_ids /
mimir_store_run_ids, the twin of Model::forwardPass(const std::vector<int>&,
training), Model.cpp:1026-1349) against the reference's own Model compiled in
place: outputs in inference and training form, the backwardPass after a
training forward, and EINVAL with the reference's message wherever it
throws."""
import zlib

import numpy as np
import pytest

import mimir_hip as M
import model_oracle as MO
import model_ref as MR
from _graphs import ids_error_graphs, ids_graphs
from _parity import assert_bitexact, assert_close_normwise, assert_close_sum

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not MR.available(), reason="oracle/_ref/libmimir_ref_model.so not built")]


def _loss(name, n):
    return np.random.default_rng(zlib.crc32(name.encode())).standard_normal(n).astype(np.float32)


def _dev(ctx, layers):
    return M.DeviceGraph(ctx, layers), M.Store(ctx)


@pytest.mark.parametrize("training", [False, True])
@pytest.mark.parametrize("graph", ids_graphs(), ids=lambda g: g[0])
def test_ids_forward_on_device(ctx, graph, training):
    name, layers, ids = graph
    if training and any(L["type"] == "Dropout" for L in layers):
        pytest.skip("a training Dropout draws a random mask")
    print("ids graph", name, "training", training, flush=True)
    ref = MR.forward_ids(layers, ids, training)
    g, st = _dev(ctx, layers)
    try:
        got = st.forward_ids(g, ids, training)
    finally:
        st.close()
        g.close()
    if name.startswith("ids_extreme") or name in ("ids_empty", "no_layers"):
        assert_bitexact(got, ref, name, allow_empty=True)
    else:
        assert_close_normwise(got, ref, name)


@pytest.mark.parametrize("graph", [g for g in ids_graphs() if g[0] != "ids_default_names"], ids=lambda g: g[0])
def test_ids_training_step_on_device(ctx, graph):
    name, layers, ids = graph
    print("ids graph backward", name, flush=True)
    out = MR.forward_ids(layers, ids, True)
    lg = _loss(name, out.size)
    _, (r_grads, r_in) = MR.forward_ids(layers, ids, True, loss_grad=lg)
    _, _, mags = MO.backward_ids(layers, ids, lg, scales=True)
    g, st = _dev(ctx, layers)
    try:
        grads, gin = st.train_step_ids(g, ids, lg)
    finally:
        st.close()
        g.close()
    assert (gin is None) == (r_in is None), name
    for L, a, b, m in zip(layers, grads, r_grads, mags):
        if b is not None:
            assert a is not None, f"{name} {L['name']}: no device gradient block"
            assert_close_sum(a, b, m, f"{name} {L['name']} grad_weights", allow_empty=True)


@pytest.mark.parametrize("graph", ids_error_graphs(), ids=lambda g: g[0])
def test_ids_errors_on_device(ctx, graph):
    name, layers, ids = graph
    with pytest.raises(MR.RefModelError) as r:
        MR.forward_ids(layers, ids, False)
    g, st = _dev(ctx, layers)
    try:
        with pytest.raises(M.MimirError) as e:
            st.forward_ids(g, ids, False)
    finally:
        st.close()
        g.close()
    assert e.value.status == M.EINVAL, name
    # The reference's message, followed by the device's layer context.
    assert str(r.value) in str(e.value), (name, str(r.value), str(e.value))
