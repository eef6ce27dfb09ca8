"""Training step on the device-resident store (mimir_store_run_training +
mimir_store_backward) against the reference's own Model::backwardPass
(golden outputs of the compiled reference, tests/golden/model_backward.npz)
and the routing restatement (oracle/model_oracle.py backward_named).

Input gradients: |gpu - ref| <= max(1e-6, 1e-5*|ref|); grad_weights (float32
sums over tokens) the same relative to the magnitudes summed."""
import os

import numpy as np
import pytest

import mimir_hip as M
import model_oracle as MO
from _graphs import train_graphs
from _parity import assert_bitexact, assert_close, assert_close_sum

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "model_backward.npz")


def _gold(name, layers, z):
    gin = z[f"{name}/__input__"] if f"{name}/__input__" in z.files else None
    grads = [z[f"{name}/{L['name']}"] if f"{name}/{L['name']}" in z.files else None for L in layers]
    return grads, gin


def _check(name, layers, got_grads, got_in, ref_grads, ref_in, mags, what):
    assert (got_in is None) == (ref_in is None), f"{name} {what}: __input__ gradient presence"
    if ref_in is not None:
        assert_close(got_in, ref_in, f"{name} {what} __input__ gradient")
    for L, a, b, m in zip(layers, got_grads, ref_grads, mags):
        if b is None:
            continue
        assert a is not None, f"{name} {L['name']}: no device gradient block"
        assert_close_sum(a, b, m, f"{name} {what} {L['name']} grad_weights")


@pytest.mark.parametrize("case", train_graphs(), ids=lambda c: c[0])
def test_train_step_matches_reference(ctx, case):
    name, layers, fin, iin, lg = case
    graph = M.DeviceGraph(ctx, layers)
    store = M.Store(ctx)
    try:
        grads, gin = store.train_step(graph, fin, iin, lg)
        o_grads, o_in, mags = MO.backward_named(layers, fin, iin, lg, scales=True)
        with np.load(GOLD) as z:
            r_grads, r_in = _gold(name, layers, z)
        _check(name, layers, grads, gin, r_grads, r_in, mags, "vs reference")
        _check(name, layers, grads, gin, o_grads, o_in, mags, "vs restatement")
        # grad_weights accumulate across steps (the reference never clears
        # Layer::grad_weights in backwardPass): a second identical step doubles them.
        grads2, _ = store.train_step(graph, fin, iin, lg)
        for L, a, b, m in zip(layers, grads, grads2, mags):
            if a is not None and m is not None:
                assert_close_sum(b, 2 * a.astype(np.float64), 2 * m, f"{name} {L['name']} second step")
    finally:
        store.close()
        graph.close()


def test_train_errors(ctx):
    store = M.Store(ctx)
    drop = M.DeviceGraph(ctx, [dict(name="d", type="Dropout")])
    ln = M.DeviceGraph(ctx, [dict(name="ln", type="LayerNorm", in_features=4)])
    try:
        store.set_inputs({"x": np.ones(8, np.float32)})
        with pytest.raises(M.MimirError, match="Dropout"):
            store.run_training(drop)
        store.run(ln)  # an inference run keeps no training state
        with pytest.raises(M.MimirError, match="training"):
            store.backward(ln, np.ones(8, np.float32))
        store.run_training(ln)
        store.backward(ln, np.ones(8, np.float32))
        assert store.grad("__input__") is None  # nothing routed to __input__
        g = store.grad("x")
        assert g is not None and g.shape == (8,)
    finally:
        store.close()
        drop.close()
        ln.close()


def test_train_step_allocates_nothing_on_repeat():
    """After one training step the store's pool holds every activation,
    snapshot and gradient buffer: a cap at the bytes already allocated does
    not stop a second step."""
    c = M.Context(0)
    name, layers, fin, iin, lg = [c_ for c_ in train_graphs() if c_[0] == "block_train"][0]
    graph = M.DeviceGraph(c, layers)
    store = M.Store(c)
    try:
        store.train_step(graph, fin, iin, lg)
        c.set_alloc_limit(1)  # any new device allocation would now fail with ENOMEM
        store.train_step(graph, fin, iin, lg)
    finally:
        c.set_alloc_limit(0)
        store.close()
        graph.close()
        c.close()


@pytest.mark.parametrize("case", train_graphs(), ids=lambda c: c[0])
def test_device_loss_gradient_matches_host(ctx, case):
    """mimir_store_backward_dev (loss gradient already on the GPU) gives the
    same bits as the host form, for the input gradient and grad_weights."""
    name, layers, fin, iin, lg = case
    graph = M.DeviceGraph(ctx, layers)
    store = M.Store(ctx)
    dlg = ctx.to_device(np.ascontiguousarray(lg, np.float32).ravel())
    try:
        store.set_inputs(fin, iin)
        store.run_training(graph)
        store.backward(graph, lg)
        host_grads, host_in = graph.grads(), store.grad("__input__")
        graph.zero_grads()
        store.set_inputs(fin, iin)  # the first step rebound names its layers write (e.g. "x")
        store.run_training(graph)
        store.backward(graph, dlg)
        dev_grads, dev_in = graph.grads(), store.grad("__input__")
        assert (host_in is None) == (dev_in is None)
        if host_in is not None:
            assert_bitexact(dev_in, host_in, f"{name} __input__ gradient")
        for L, a, b in zip(layers, host_grads, dev_grads):
            if a is not None:
                assert_bitexact(b, a, f"{name} {L['name']} grad_weights")
    finally:
        dlg.free()
        store.close()
        graph.close()
