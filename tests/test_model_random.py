"""The routing restatement (oracle/model_oracle.py) against the reference's
own Model, compiled in place (oracle/_ref), on 300 seeded random graphs
(tests/_random_graphs.py): forwardPassNamed, and forwardPassNamed(training)
+ backwardPass on 200 more.  Both must throw on the same graphs (the
backward throws on some graphs whose forward runs: a gradient accumulated
onto a name rebound to another size, Model.cpp:7335); otherwise
outputs within |d| <= max(1e-6, 1e-5*|ref|), gradients the same relative to
the magnitudes summed."""
import numpy as np
import pytest

import model_oracle as MO
import model_ref as MR
from _parity import assert_close, assert_close_sum
from _random_graphs import random_graph

pytestmark = pytest.mark.skipif(not MR.available(), reason="oracle/_ref/libmimir_ref_model.so not built")

FORWARD_SEEDS = range(300)
TRAIN_SEEDS = range(1000, 1200)


def _run(fn, err, *args):
    try:
        return fn(*args), None
    except err as e:
        return None, str(e)


def _loss_grad(seed, layers, fin, iin):
    out, e = _run(MR.forward_named, MR.RefModelError, layers, fin, iin)
    if e is not None:
        return None
    return np.random.default_rng(seed + 7).standard_normal(out.size).astype(np.float32)


@pytest.mark.parametrize("seed", FORWARD_SEEDS)
def test_random_forward_matches_reference(seed):
    name, layers, fin, iin = random_graph(seed)
    ref, rerr = _run(MR.forward_named, MR.RefModelError, layers, fin, iin)
    got, gerr = _run(MO.forward_named, MO.ModelError, layers, fin, iin)
    assert (rerr is None) == (gerr is None), f"{name}: reference error {rerr!r}, restatement error {gerr!r}"
    if ref is not None:
        assert_close(got, ref, name, allow_empty=True)


@pytest.mark.parametrize("seed", TRAIN_SEEDS)
def test_random_backward_matches_reference(seed):
    name, layers, fin, iin = random_graph(seed, training=True)
    lg = _loss_grad(seed, layers, fin, iin)
    if lg is None:
        with pytest.raises(MO.ModelError):
            MO.backward_named(layers, fin, iin, np.zeros(0, np.float32))
        return
    ref, rerr = _run(MR.backward, MR.RefModelError, layers, fin, iin, lg)
    got, gerr = _run(lambda *a: MO.backward_named(*a, scales=True), MO.ModelError, layers, fin, iin, lg)
    assert (rerr is None) == (gerr is None), f"{name}: reference error {rerr!r}, restatement error {gerr!r}"
    if rerr is not None:
        return
    (r_grads, r_in), (o_grads, o_in, mags) = ref, got
    assert (o_in is None) == (r_in is None), f"{name}: __input__ gradient presence"
    if r_in is not None:
        assert_close(o_in, r_in, f"{name} __input__ gradient", allow_empty=True)
    for L, a, b, m in zip(layers, o_grads, r_grads, mags):
        if b is None:
            assert a is None or not np.any(a), f"{name} {L['name']}: gradient where the reference has none"
            continue
        assert_close_sum(a, b, m, f"{name} {L['name']} grad_weights", allow_empty=True)


def test_random_graphs_mostly_run():
    """The generator is not vacuous: most graphs run, some throw, and the
    graphs cover every layer type."""
    ran = 0
    seen = set()
    for seed in FORWARD_SEEDS:
        name, layers, fin, iin = random_graph(seed)
        seen.update(L["type"] for L in layers)
        ran += _run(MR.forward_named, MR.RefModelError, layers, fin, iin)[1] is None
    assert 0.75 * len(FORWARD_SEEDS) <= ran < len(FORWARD_SEEDS), ran
    assert seen == set(MO.SUPPORTED), seen


def test_normwise_tolerance_catches_rewiring():
    """A planted routing mistake -- one layer input rebound to another tensor
    of the same size -- moves the reference's own result by far more than the
    normwise tolerance the device tests use (1e-5 of max|ref|): of the graphs
    where the rewired result differs at all, at least 95% move by more than
    1e-3 of it.  A rewiring can be neutral up to rounding: seed 66's LayerNorm
    reading g instead of LogSoftmax(g), whose constant offset it removes."""
    from _parity import assert_close_normwise

    rewired = caught = 0
    for seed in FORWARD_SEEDS:
        name, layers, fin, iin = random_graph(seed)
        ref, err = _run(MR.forward_named, MR.RefModelError, layers, fin, iin)
        if err is not None or ref.size == 0:
            continue
        rng = np.random.default_rng(seed)
        for i, L in enumerate(layers):
            cur = (L.get("inputs") or ["x"])[0]
            if L["type"] == "Embedding":
                continue
            # the size of `cur` where layer i reads it: the prefix graph, then an Identity onto "x"
            probe = layers[:i] + [dict(name="probe", type="Identity", inputs=[cur], output="x")]
            val, err = _run(MR.forward_named, MR.RefModelError, probe, fin, iin)
            cands = [k for k in fin if k != cur and err is None and np.asarray(fin[k]).size == val.size]
            if not cands:
                continue
            W = dict(L, inputs=[str(rng.choice(cands))] + list(L.get("inputs") or ["x"])[1:])
            bad, err = _run(MR.forward_named, MR.RefModelError, layers[:i] + [W] + layers[i + 1:], fin, iin)
            if err is not None or bad.shape != ref.shape or np.array_equal(bad, ref):
                continue
            rewired += 1
            big = float(np.abs(bad - ref).max()) > 1e-3 * float(np.abs(ref).max())
            if big:
                with pytest.raises(AssertionError):
                    assert_close_normwise(bad, ref, name)
            caught += big
    assert rewired >= 50, rewired
    assert caught >= 0.95 * rewired, (caught, rewired)
