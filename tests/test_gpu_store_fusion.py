"""Inference fusion in the device runtime (mimir_store_set_fusion): chains of
GELU / SiLU / equal-size Add and Multiply layers run as one kernel.

A fused run is held to the unfused run of the same layers bit for bit: its
"x", and every name it leaves bound (the intermediates a later layer reads
are materialised), on the runtime graphs of tests/_graphs.py, seeded random
layer graphs and attention blocks; the names of intermediates nothing reads
are left unbound (the proof that the chain fused); and a captured forward
records the fused kernels."""
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
    fused, plain = M.Store(ctx), M.Store(ctx)
    fused.set_fusion(True)
    yield fused, plain
    fused.close()
    plain.close()


def _bound(store, names):
    out = {}
    for nm in names:
        try:
            out[nm] = store.get(nm)
        except M.MimirError:
            pass
    return out


def _names(layers, fin):
    return sorted({L.get("output") or "x" for L in layers} | set(fin) | {"x"})


def _compare(ctx, stores, name, layers, fin, iin):
    fused, plain = stores
    g = M.DeviceGraph(ctx, layers)
    try:
        try:
            want = plain.forward_named(g, fin, iin)
        except M.MimirError as e:  # a graph the reference refuses: the fused run refuses it the same way
            with pytest.raises(M.MimirError) as f:
                fused.forward_named(g, fin, iin)
            assert f.value.status == e.status and str(f.value) == str(e), f"{name}: {f.value} vs {e}"
            return
        ref = _bound(plain, _names(layers, fin))
        got = fused.forward_named(g, fin, iin)
        assert_bitexact(got, want, f"{name}: x")
        for nm, v in _bound(fused, _names(layers, fin)).items():
            assert nm in ref, f"{name}: {nm} bound only in the fused run"
            assert_bitexact(v, ref[nm], f"{name}: {nm}")
    finally:
        g.close()


@pytest.mark.parametrize("graph", graphs(), ids=lambda g: g[0])
def test_fused_graphs_match_unfused(ctx, stores, graph):
    name, layers, fin, iin = graph
    _compare(ctx, stores, name, layers, fin, iin)


@pytest.mark.parametrize("seed", range(40))
def test_fused_random_graphs_match_unfused(ctx, stores, seed):
    name, layers, fin, iin = random_graph(2000 + seed)
    _compare(ctx, stores, name, layers, fin, iin)


@pytest.mark.parametrize("causal", [False, True])
def test_fused_attention_block(ctx, stores, causal):
    name, layers, fin, iin = block_graph(seq=64, e=128, heads=4, causal=causal)
    _compare(ctx, stores, name, layers, fin, iin)


def _chain_graph(n=4096 * 3 + 2):
    """inp -> GELU -> a; a * gate -> b; SiLU(b) -> c; c + res -> x, with b
    read again by a final Add (so it is materialised) and a, c not."""
    r = np.random.default_rng(3)
    fin = {k: (2 * r.standard_normal(n)).astype(np.float32) for k in ("inp", "gate", "res")}
    layers = [dict(name="g", type="GELU", inputs=["inp"], output="a"),
              dict(name="m", type="Multiply", inputs=["a", "gate"], output="b"),
              dict(name="s", type="SiLU", inputs=["b"], output="c"),
              dict(name="r", type="Add", inputs=["res", "c"], output="x"),
              dict(name="late", type="Add", inputs=["x", "b"], output="y")]
    return layers, fin


def test_chain_fuses_and_keeps_what_is_read_later(ctx, stores):
    fused, plain = stores
    layers, fin = _chain_graph()
    g = M.DeviceGraph(ctx, layers)
    try:
        for s in (fused, plain):
            s.set_inputs(fin, {})
            s.run(g)
        for nm in ("x", "b", "y"):
            assert_bitexact(fused.get(nm), plain.get(nm), nm)
        for nm in ("a", "c"):  # fused away: nothing after the chain reads them
            with pytest.raises(M.MimirError, match="no tensor named"):
                fused.get(nm)
            plain.get(nm)
        # reference values by the unfused per-layer ops
        x, a = ctx.to_device(fin["inp"]), ctx.empty(fin["inp"].size)
        try:
            ctx.gelu(x, a, fin["inp"].size)
            want_b = a.numpy() * fin["gate"]
        finally:
            x.free()
            a.free()
        assert_bitexact(fused.get("b"), want_b.astype(np.float32), "b = gelu(inp) * gate")
    finally:
        g.close()


def test_chain_with_the_value_on_both_sides(ctx, stores):
    """Add(v, v) and Multiply(v, v) inside a chain, and "x" written twice."""
    r = np.random.default_rng(4)
    fin = {"x": r.standard_normal(1000).astype(np.float32)}
    layers = [dict(name="a", type="SiLU", inputs=["x"], output="x"),
              dict(name="b", type="Add", inputs=["x", "x"], output="x"),
              dict(name="c", type="Multiply", inputs=["x", "x"], output="t"),
              dict(name="d", type="GELU", inputs=["t"], output="x")]
    _compare(ctx, stores, "both_sides", layers, fin, {})


def test_captured_fused_forward(ctx, stores):
    fused, plain = stores
    layers, fin = _chain_graph(2048)
    g = M.DeviceGraph(ctx, layers)
    try:
        with fused.capture(g, fin, {}) as sg:
            r = np.random.default_rng(5)
            for k in range(3):
                f2 = {nm: r.standard_normal(v.size).astype(np.float32) for nm, v in fin.items()}
                for nm, v in f2.items():
                    sg.set_input(nm, v)
                sg.launch()
                plain.set_inputs(f2, {})
                plain.run(g)
                assert_bitexact(sg.get("y"), plain.get("y"), f"replay {k}")
    finally:
        g.close()


# ---- LayerNorm groups: [Add ->] LayerNorm [-> elementwise chain] -----------

def _ln_block(rows=64, cols=512, seed=6, bias=True, affine=True, h_read_later=False):
    """Add(inp, res) -> h; LayerNorm(h) -> n; GELU -> g; g * gate -> m;
    SiLU -> x (the bench's runtime block), optionally with h read again."""
    r = np.random.default_rng(seed)
    n = rows * cols
    fin = {"inp": r.standard_normal(n).astype(np.float32), "res": r.standard_normal(n).astype(np.float32),
           "gate": r.standard_normal(n).astype(np.float32)}
    w = np.concatenate([1 + 0.1 * r.standard_normal(cols), 0.1 * r.standard_normal(cols)]).astype(np.float32)
    layers = [dict(name="add", type="Add", inputs=["inp", "res"], output="h"),
              dict(name="ln", type="LayerNorm", inputs=["h"], output="n", in_features=cols, eps=1e-5,
                   affine=affine, use_bias=bias, weights=w if affine else None),
              dict(name="act", type="GELU", inputs=["n"], output="g"),
              dict(name="gate", type="Multiply", inputs=["g", "gate"], output="m"),
              dict(name="silu", type="SiLU", inputs=["m"], output="x")]
    if h_read_later:
        layers.append(dict(name="res2", type="Add", inputs=["x", "h"], output="y"))
    return layers, fin


@pytest.mark.parametrize("cols", [4, 256, 512, 4096, 16384])
@pytest.mark.parametrize("h_read_later", [False, True])
def test_add_layernorm_chain_fuses(ctx, stores, cols, h_read_later):
    fused, plain = stores
    layers, fin = _ln_block(rows=max(1, 65536 // cols), cols=cols, h_read_later=h_read_later)
    _compare(ctx, stores, f"ln_block_{cols}", layers, fin, {})
    names = set(_bound(fused, ["h", "n", "g", "m"]))
    assert names == ({"h"} if h_read_later else set()), f"left bound after the fused block: {names}"


@pytest.mark.parametrize("affine,bias", [(True, False), (False, False)])
def test_layernorm_epilogue_variants(ctx, stores, affine, bias):
    layers, fin = _ln_block(rows=32, cols=1024, affine=affine, bias=bias)
    _compare(ctx, stores, f"ln_affine{affine}_bias{bias}", layers[1:], {"h": fin["inp"], "gate": fin["gate"]}, {})


def test_layernorm_output_read_later_is_kept(ctx, stores):
    fused, _ = stores
    layers, fin = _ln_block(rows=16, cols=2048)
    layers = layers + [dict(name="late", type="Add", inputs=["x", "n"], output="y")]
    _compare(ctx, stores, "ln_out_read_later", layers, fin, {})
    fused.get("n")


def test_layernorm_groups_that_stay_unfused(ctx, stores):
    """A broadcast Add before the LayerNorm, rows too wide for one workgroup
    (the long-row kernels), a width that is not a multiple of 4 (the scalar
    kernel), and a LayerNorm the reference refuses: all give the unfused
    results or errors."""
    r = np.random.default_rng(9)
    g = np.concatenate([np.ones(6), np.zeros(6)]).astype(np.float32)
    cases = [
        ("broadcast_add", [dict(name="a", type="Add", inputs=["x", "bias"], output="h"),
                           dict(name="ln", type="LayerNorm", inputs=["h"], output="n", in_features=64),
                           dict(name="s", type="SiLU", inputs=["n"], output="x")],
         {"x": r.standard_normal(64 * 8).astype(np.float32), "bias": r.standard_normal(64).astype(np.float32)}),
        ("long_rows", [dict(name="ln", type="LayerNorm", inputs=["x"], output="n", in_features=65536),
                       dict(name="s", type="GELU", inputs=["n"], output="x")],
         {"x": r.standard_normal(65536 * 2).astype(np.float32)}),
        ("odd_width", [dict(name="ln", type="LayerNorm", inputs=["x"], output="n", in_features=6, weights=g),
                       dict(name="s", type="GELU", inputs=["n"], output="x")],
         {"x": r.standard_normal(6 * 5).astype(np.float32)}),
        ("refused", [dict(name="ln", type="LayerNorm", inputs=["x"], output="n", in_features=7),
                     dict(name="s", type="GELU", inputs=["n"], output="x")],
         {"x": r.standard_normal(20).astype(np.float32)}),
    ]
    for name, layers, fin in cases:
        _compare(ctx, stores, name, layers, fin, {})


def test_layernorm_shape_override_keeps_it_unfused(ctx):
    """With a LayerNorm launch-shape override the unfused kernel reduces in
    another order, so fusion leaves the LayerNorm alone: still bit-exact."""
    import os
    old = os.environ.get("MIMIR_TUNE")
    os.environ["MIMIR_TUNE"] = "layernorm=256x4x256"
    try:
        c = M.Context(0)
    finally:
        if old is None:
            del os.environ["MIMIR_TUNE"]
        else:
            os.environ["MIMIR_TUNE"] = old
    try:
        f, p = M.Store(c), M.Store(c)
        f.set_fusion(True)
        layers, fin = _ln_block(rows=64, cols=4096)
        _compare(c, (f, p), "override", layers, fin, {})
        f.close()
        p.close()
    finally:
        c.close()
