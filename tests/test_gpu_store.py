"""The device-resident runtime (mimir_store_* in include/mimir_hip.h) against
the routing oracle on the graphs of tests/_graphs.py, which the CPU tests pin
to the reference's own Model::forwardPassNamed."""
import numpy as np
import pytest

import mimir_hip as M
import model_oracle as MO
from _graphs import error_graphs, graphs
from _parity import assert_bitexact, assert_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def store(ctx):
    s = M.Store(ctx)
    yield s
    s.close()


@pytest.mark.parametrize("case", graphs(), ids=lambda c: c[0])
def test_store_matches_routing_oracle(ctx, store, case):
    name, layers, fin, iin = case
    g = M.DeviceGraph(ctx, layers)
    try:
        got = store.forward_named(g, fin, iin)
        assert_close(got, MO.forward_named(layers, fin, iin), name)
        # A second run reuses the pooled buffers and gives the same bits.
        again = store.forward_named(g, fin, iin)
        assert_bitexact(again, got, name + " (second run)")
    finally:
        g.close()


@pytest.mark.parametrize("case", error_graphs(), ids=lambda c: c[0])
def test_store_errors_where_reference_throws(ctx, store, case):
    name, layers, fin, iin = case
    g = M.DeviceGraph(ctx, layers)
    try:
        with pytest.raises(M.MimirError) as e:
            store.forward_named(g, fin, iin)
        assert e.value.status == M.EINVAL
    finally:
        g.close()


def test_store_intermediates_stay_named(ctx, store):
    """Every layer output stays addressable by name on the device, with the
    value the oracle computes for that tensor."""
    name, layers, fin, iin = [c for c in graphs() if c[0] == "block_chain"][0]
    g = M.DeviceGraph(ctx, layers)
    try:
        store.forward_named(g, fin, iin)
        for upto in range(1, len(layers)):
            out_name = layers[upto - 1]["output"]
            sub = [dict(L) for L in layers[:upto]]
            sub[-1]["output"] = "x"
            ref = MO.forward_named(sub, fin, iin)
            assert_close(store.get(out_name), ref, out_name)
        ids = store.get("text_ids", M._lib.DTYPE_I32)
        assert_bitexact(ids, np.asarray(iin["seq"], np.int32), "seq alias")
    finally:
        g.close()


def test_store_allocates_nothing_on_a_repeat_run(ctx):
    """After one forward, the pool holds every buffer the graph needs: a cap at
    the bytes already allocated does not stop a second forward."""
    c = M.Context(0)
    s = M.Store(c)
    name, layers, fin, iin = [c_ for c_ in graphs() if c_[0] == "wide_ln_residual"][0]
    g = M.DeviceGraph(c, layers)
    try:
        first = s.forward_named(g, fin, iin)
        # Any new device allocation would now fail with ENOMEM.
        c.set_alloc_limit(1)
        second = s.forward_named(g, fin, iin)
        assert_bitexact(second, first, "repeat run")
    finally:
        c.set_alloc_limit(0)
        g.close()
        s.close()
        c.close()
