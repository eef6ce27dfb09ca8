"""Residual merges on the device: mimir_branch_merge_fwd against the
restatement of Model::computeBranchMerge (oracle.branch_merge, pinned to the
compiled reference by tests/test_model_merge.py), bit for bit; and the
device store's training forward and backward (mimir_store_run_training /
mimir_store_backward) against the reference's own Model on the merge graphs
of tests/_graphs.py and on 120 random training graphs with merges."""
import zlib

import numpy as np
import pytest

import mimir_hip as M
import model_oracle as MO
import model_ref as MR
import oracle as O
from _graphs import MERGE_OPS, merge_error_graphs, merge_graphs
from _parity import assert_bitexact, assert_close_normwise, assert_close_sum
from _random_graphs import random_graph
from test_model_merge import MERGE_SEEDS, _BITEXACT

pytestmark = pytest.mark.gpu
needs_ref = pytest.mark.skipif(not MR.available(), reason="oracle/_ref/libmimir_ref_model.so not built")


def _loss(name, n):
    return np.random.default_rng(zlib.crc32(name.encode())).standard_normal(n).astype(np.float32)


SPECIALS = np.array([np.nan, 1, -0.0, 0.0, np.inf, -np.inf, 2, np.nan, -3, 0.0, -0.0, np.nan, 5, 1e-40,
                     -1e-40, 3.4e38], np.float32)


@pytest.mark.parametrize("op", MERGE_OPS)
@pytest.mark.parametrize("n,off", [(1, 0), (7, 0), (8, 0), (9, 0), (13, 1), (1000, 3), (1 << 20, 0),
                                   ((1 << 20) + 5, 2)])
def test_branch_merge_kernel_bitexact(ctx, op, n, off):
    print(f"branch_merge {op} n={n} off={off}", flush=True)
    rng = np.random.default_rng(n + off)
    a = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n + 5).astype(np.float32)
    k = min(n, SPECIALS.size)
    a[:k] = SPECIALS[:k]
    b[:k] = SPECIALS[::-1][:k]
    a[n - k:n] = SPECIALS[:k]                   # specials in the MAX tail too
    b[n - k:n] = np.roll(SPECIALS, 3)[:k]
    want = O.branch_merge(a, b, op)
    # Offsets of a few floats leave the buffers off 16-byte alignment.
    da = ctx.to_device(np.concatenate([np.zeros(off, np.float32), a]))
    db = ctx.to_device(np.concatenate([np.zeros(off, np.float32), b]))
    dy = ctx.empty(want.size + off)
    ctx.branch_merge(da.offset(off), n, db.offset(off), b.size, dy.offset(off), op)
    assert_bitexact(dy.numpy()[off:], want, f"{op} n={n}")
    for d in (da, db, dy):
        d.free()


def test_branch_merge_refuses_a_short_source(ctx):
    a, b, y = ctx.empty(8), ctx.empty(5), ctx.empty(8)
    with pytest.raises(M.MimirError) as e:
        ctx.branch_merge(a, 8, b, 5, y, "ADD")
    assert e.value.status == M.EINVAL
    ctx.branch_merge(a, 8, b, 5, ctx.empty(13), "CONCATENATE")  # any sizes concatenate
    with pytest.raises(M.MimirError):
        ctx.branch_merge(a, 8, b, 8, y, 7)  # not a MergeOperation


def _train_forward(ctx, layers, fin, iin):
    graph = M.DeviceGraph(ctx, layers)
    store = M.Store(ctx)
    try:
        return store.forward_named(graph, fin, iin, training=True), store.forward_named(graph, fin, iin)
    finally:
        store.close()
        graph.close()


@needs_ref
@pytest.mark.parametrize("graph", merge_graphs(), ids=lambda g: g[0])
def test_store_merge_forward_matches_reference(ctx, graph):
    name, layers, fin, iin = graph
    print("merge graph", name, flush=True)
    ref = MR.forward_named(layers, fin, iin, training=True)
    got, inf = _train_forward(ctx, layers, fin, iin)
    if name in _BITEXACT:
        assert_bitexact(got, ref, name)
    else:
        assert_close_normwise(got, ref, name)
    assert_close_normwise(inf, MR.forward_named(layers, fin, iin), name + " inference (no merge)")


def test_store_merge_kat(ctx):
    """Tests/test_runtime_residual_merge.cpp:40-47 on the device."""
    name, layers, fin, iin = merge_graphs()[0]
    got, inf = _train_forward(ctx, layers, fin, iin)
    assert got.tolist() == [3.0, 8.0] and inf.tolist() == [2.0, 6.0]


@needs_ref
@pytest.mark.parametrize("graph", merge_graphs(), ids=lambda g: g[0])
def test_store_merge_backward_matches_reference(ctx, graph):
    name, layers, fin, iin = graph
    print("merge graph backward", name, flush=True)
    out = MR.forward_named(layers, fin, iin, training=True)
    lg = _loss(name, out.size)
    r_grads, r_in = MR.backward(layers, fin, iin, lg)
    _, _, mags = MO.backward_named(layers, fin, iin, lg, scales=True)
    graph = M.DeviceGraph(ctx, layers)
    store = M.Store(ctx)
    try:
        _, gin = store.train_step(graph, fin, iin, lg)
        # A repeated step reuses every buffer, gives the same input gradient
        # and adds the same parameter gradients again.
        grads, gin2 = store.train_step(graph, fin, iin, lg)
    finally:
        store.close()
        graph.close()
    assert (gin is None) == (r_in is None), name
    if r_in is not None:
        assert_close_normwise(gin, r_in, name + " __input__ gradient")
        assert_bitexact(gin2, gin, name + " repeated step")
    for L, a, b, m in zip(layers, grads, r_grads, mags):
        if b is not None:
            assert_close_sum(a / 2, b, m, f"{name} {L['name']} grad_weights (two steps)", allow_empty=True)


@pytest.mark.parametrize("graph", merge_error_graphs(), ids=lambda g: g[0])
def test_store_merge_short_source_is_refused(ctx, graph):
    name, layers, fin, iin = graph
    g = M.DeviceGraph(ctx, layers)
    store = M.Store(ctx)
    try:
        with pytest.raises(M.MimirError) as e:
            store.forward_named(g, fin, iin, training=True)
        assert e.value.status == M.EINVAL
        store.forward_named(g, fin, iin)  # inference does not merge
    finally:
        store.close()
        g.close()


@needs_ref
@pytest.mark.parametrize("seed", MERGE_SEEDS)
def test_random_merge_graphs_on_device(ctx, seed):
    name, layers, fin, iin = random_graph(seed, training=True, merges=True)
    try:
        out = MR.forward_named(layers, fin, iin, training=True)
        ferr = None
    except MR.RefModelError as e:
        out, ferr = None, str(e)
    graph = M.DeviceGraph(ctx, layers)
    store = M.Store(ctx)
    try:
        if ferr is not None:
            with pytest.raises(M.MimirError) as e:
                store.forward_named(graph, fin, iin, training=True)
            assert e.value.status == M.EINVAL, f"{name}: reference threw {ferr!r}"
            return
        got = store.forward_named(graph, fin, iin, training=True)
        assert_close_normwise(got, out, name, allow_empty=True)
        lg = _loss(name, out.size)
        try:
            r_grads, r_in = MR.backward(layers, fin, iin, lg)
        except MR.RefModelError as e:
            with pytest.raises(M.MimirError):
                store.train_step(graph, fin, iin, lg)
            return
        graph.zero_grads()
        grads, gin = store.train_step(graph, fin, iin, lg)
        _, _, mags = MO.backward_named(layers, fin, iin, lg, scales=True)
        assert (gin is None) == (r_in is None), name
        if r_in is not None:
            assert_close_normwise(gin, r_in, f"{name} __input__ gradient", allow_empty=True)
        for L, a, b, m in zip(layers, grads, r_grads, mags):
            if b is not None:
                assert_close_sum(a, b, m, f"{name} {L['name']} grad_weights", allow_empty=True)
    finally:
        store.close()
        graph.close()
