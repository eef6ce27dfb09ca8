"""Captured forwards (mimir_store_capture / _graph_launch / _graph_set_input /
_graph_get): a mimir_store_run recorded as a HIP graph and replayed.

Every replay is checked against an eager run of the same layers on the same
inputs in a second store, bit for bit (the same kernels on the same data),
with eager work and synchronisations on the capturing store between the
replays: the named-routing and runtime graphs of tests/_graphs.py, seeded
random layer graphs, the attention layers (library GEMMs inside the graph),
a scratch that grows while a graph is alive, and the refusals."""
import numpy as np
import pytest

import mimir_hip as M
from _attention_graphs import block_graph
from _graphs import graphs
from _parity import assert_bitexact
from _random_graphs import random_graph

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def stores(ctx):
    a, b = M.Store(ctx), M.Store(ctx)
    yield a, b
    a.close()
    b.close()


def _fresh_inputs(fin, iin, rng, layers):
    """New values of the same sizes for every input (int ids within the
    vocabularies of the graph's Embedding layers)."""
    vocab = max([L.get("vocab_size", 1) for L in layers if L["type"] == "Embedding"] or [1])
    f2 = {k: rng.standard_normal(np.asarray(v).size).astype(np.float32) for k, v in fin.items()}
    i2 = {k: rng.integers(-2, vocab + 2, np.asarray(v).size).astype(np.int32) for k, v in iin.items()}
    return f2, i2


def _check_replays(ctx, stores, name, layers, fin, iin, replays=3, seed=0):
    cap, eager = stores
    rng = np.random.default_rng(seed)
    g = M.DeviceGraph(ctx, layers)
    try:
        want = eager.forward_named(g, fin, iin)
        with cap.capture(g, fin, iin) as sg:
            assert_bitexact(sg.get("x"), want, f"{name}: the capture's own launch")
            for k in range(replays):
                f2, i2 = _fresh_inputs(fin, iin, rng, layers)
                for nm, v in f2.items():
                    sg.set_input(nm, v)
                for nm, v in i2.items():
                    sg.set_input(nm, v)
                sg.launch()
                # eager work on the capturing store between launch and read
                cap.forward_named(g, f2, i2)
                assert_bitexact(sg.get("x"), eager.forward_named(g, f2, i2), f"{name}: replay {k}")
                ctx.sync()
    finally:
        g.close()


@pytest.mark.parametrize("graph", [g for g in graphs() if g[0] != "embedding_missing_ids"], ids=lambda g: g[0])
def test_graph_replays_match_eager(ctx, stores, graph):
    name, layers, fin, iin = graph
    print(f"store graph {name}", flush=True)
    _check_replays(ctx, stores, name, layers, fin, iin)


def test_graph_with_padding_ids_made_in_the_run(ctx, stores):
    """An Embedding whose ids are missing stores seq_len padding ids during
    the run (a buffer the captured run itself fills)."""
    name, layers, fin, iin = next(g for g in graphs() if g[0] == "embedding_missing_ids")
    _check_replays(ctx, stores, name, layers, fin, iin, replays=2)


@pytest.mark.parametrize("seed", range(12))
def test_random_graph_replays(ctx, stores, seed):
    name, layers, fin, iin = random_graph(1000 + seed)
    print(f"store graph {name}", flush=True)
    _check_replays(ctx, stores, name, layers, fin, iin, seed=seed)


@pytest.mark.parametrize("causal", [False, True])
def test_attention_block_graph(ctx, stores, causal):
    """LayerNorm -> SelfAttention -> Add -> LayerNorm -> GELU: the attention
    layer's projections are library GEMMs, recorded into the graph."""
    name, layers, fin, iin = block_graph(seq=96, e=128, heads=4, causal=causal)
    _check_replays(ctx, stores, name, layers, fin, iin, replays=4)


def test_graph_survives_scratch_growth(ctx, stores):
    """The context's scratch grows (a larger attention layer runs eagerly)
    while a captured graph that uses the old one is alive: the old buffer is
    kept for the graph, and both keep giving the eager results."""
    cap, eager = stores
    _, small, fin, iin = block_graph(seq=32, e=64, heads=2, causal=True, seed=7)
    _, big, bfin, biin = block_graph(seq=512, e=256, heads=4, causal=False, seed=8)
    gs, gb = M.DeviceGraph(ctx, small), M.DeviceGraph(ctx, big)
    try:
        with cap.capture(gs, fin, iin) as sg:
            got_big = cap.forward_named(gb, bfin, biin)  # grows the scratch past the graph's
            sg.launch()
            assert_bitexact(sg.get("x"), eager.forward_named(gs, fin, iin), "graph after the scratch grew")
            assert_bitexact(got_big, eager.forward_named(gb, bfin, biin), "the larger layer")
    finally:
        gs.close()
        gb.close()


def test_graph_refusals(ctx, stores):
    cap, _ = stores
    name, layers, fin, iin = graphs()[0]
    g = M.DeviceGraph(ctx, layers)
    try:
        with cap.capture(g, fin, iin) as sg:
            with pytest.raises(M.MimirError, match="not an input of the graph"):
                sg.set_input("nope", np.zeros(2, np.float32))
            with pytest.raises(M.MimirError, match="holds 2 elements, not 3"):
                sg.set_input("a", np.zeros(3, np.float32))
            with pytest.raises(M.MimirError, match="binds no tensor named"):
                sg.get("nope")
        # A capture whose run fails (here in its first, eager pass) leaves the
        # store usable.
        bad = [dict(name="m", type="Add", inputs=["missing", "a"], output="x")]
        gbad = M.DeviceGraph(ctx, bad)
        try:
            with pytest.raises(M.MimirError, match="Missing input tensor: missing"):
                cap.capture(gbad, fin, iin)
        finally:
            gbad.close()
        assert_bitexact(cap.forward_named(g, fin, iin), np.array([8, 12], np.float32), "eager after a failed capture")
    finally:
        g.close()


def test_store_close_destroys_its_graphs(ctx):
    """Closing the store destroys its captured graphs; their StoreGraph
    objects then refuse to launch, and closing them again is a no-op."""
    name, layers, fin, iin = graphs()[0]
    s = M.Store(ctx)
    g = M.DeviceGraph(ctx, layers)
    try:
        sg = s.capture(g, fin, iin)
        sg.launch()
        assert_bitexact(sg.get("x"), np.array([8, 12], np.float32), "named routing")
        s.close()  # destroys sg's graph too
        assert not sg.handle
        with pytest.raises(M.MimirError, match="closed"):
            sg.launch()
        sg.close()  # safe: nothing left to destroy
        sg.close()
    finally:
        g.close()


def test_device_graph_close_waits_for_its_store_graphs(ctx):
    """A DeviceGraph refuses to free its weights while a captured graph that
    replays them is open, and frees them once that graph is closed."""
    name, layers, fin, iin = graphs()[0]
    s = M.Store(ctx)
    g = M.DeviceGraph(ctx, layers)
    try:
        sg = s.capture(g, fin, iin)
        with pytest.raises(M.MimirError, match="still replay"):
            g.close()
        sg.launch()  # the weights are still there
        assert_bitexact(sg.get("x"), np.array([8, 12], np.float32), "replay after a refused close")
        sg.close()
        g.close()
    finally:
        s.close()
        g.close()
