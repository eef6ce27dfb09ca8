"""Residual merges of the training forward: the routing restatement
(oracle/model_oracle.py, oracle.branch_merge) against the reference's own
Model compiled in place (oracle/_ref), forwardPassNamed(training=true) and
backwardPass, on tests/_graphs.py's merge graphs and on seeded random
training graphs with merges (tests/_random_graphs.py, merges=True).

The merge is one or two IEEE float32 operations per element (or a copy), so
the training outputs of the merge-only graphs must be bit-identical; graphs
that also run LayerNorm / GELU / SiLU are held to the path's tolerance.  The
reference's backward ignores merges (backpropThroughBranch is never called),
and so does the restatement: their gradients must agree."""
import zlib

import numpy as np
import pytest

import model_oracle as MO
import model_ref as MR
import oracle as O
from _graphs import MERGE_OPS, merge_error_graphs, merge_graphs
from _parity import assert_bitexact, assert_close, assert_close_sum
from _random_graphs import random_graph

pytestmark = pytest.mark.skipif(not MR.available(), reason="oracle/_ref/libmimir_ref_model.so not built")

MERGE_SEEDS = range(2000, 2120)
_BITEXACT = ("residual_merge_kat",) + tuple(f"merge_{op.lower()}_specials" for op in MERGE_OPS)


def _loss(name, n):
    return np.random.default_rng(zlib.crc32(name.encode())).standard_normal(n).astype(np.float32)


@pytest.mark.parametrize("graph", merge_graphs(), ids=lambda g: g[0])
def test_merge_training_forward_matches_reference(graph):
    name, layers, fin, iin = graph
    ref = MR.forward_named(layers, fin, iin, training=True)
    got = MO.forward_named(layers, fin, iin, training=True)
    if name in _BITEXACT:
        assert_bitexact(got, ref, name)
    else:
        assert_close(got, ref, name)
    # Inference never merges (Model.cpp:4729-4732: has_branches needs training).
    assert_close(MO.forward_named(layers, fin, iin), MR.forward_named(layers, fin, iin), name + " inference")


def test_merge_kat_values():
    """Tests/test_runtime_residual_merge.cpp:40-47: main [2, 6] + skip [1, 2]."""
    name, layers, fin, iin = merge_graphs()[0]
    assert name == "residual_merge_kat"
    assert MO.forward_named(layers, fin, iin, training=True).tolist() == [3.0, 8.0]
    assert MO.forward_named(layers, fin, iin).tolist() == [2.0, 6.0]


@pytest.mark.parametrize("graph", merge_graphs(), ids=lambda g: g[0])
def test_merge_backward_matches_reference(graph):
    name, layers, fin, iin = graph
    out = MR.forward_named(layers, fin, iin, training=True)
    lg = _loss(name, out.size)
    rg, rin = MR.backward(layers, fin, iin, lg)
    gg, gin, mags = MO.backward_named(layers, fin, iin, lg, scales=True)
    assert (rin is None) == (gin is None), name
    if rin is not None:
        assert_close(gin, rin, name + " input grad")
    for i, (a, b) in enumerate(zip(gg, rg)):
        if b is not None:
            assert_close_sum(a, b, mags[i] if mags[i] is not None else np.abs(b), f"{name} grad_weights[{i}]")


def test_merge_is_absent_from_the_reference_backward():
    """A LayerNorm whose output only a merge reads: if the backward routed the
    merged output's gradient into the merge's source, the LayerNorm would get
    parameter gradients.  The reference gives it none (backpropThroughBranch,
    Model.cpp:4584-4613, is never called), and neither does the restatement."""
    r = np.random.default_rng(5)
    d = 16
    layers = [dict(name="ln", type="LayerNorm", inputs=["v"], output="h", in_features=d,
                   weights=np.concatenate([np.ones(d), np.zeros(d)]).astype(np.float32)),
              dict(name="act_residual", type="GELU", inputs=["v"], output="x", branch_sources=[0])]
    fin = {"v": r.standard_normal(4 * d).astype(np.float32)}
    lg = r.standard_normal(4 * d).astype(np.float32)
    out = MR.forward_named(layers, fin, {}, training=True)
    assert not np.array_equal(out, MR.forward_named(layers, fin, {}))  # the merge happened
    rg, _ = MR.backward(layers, fin, {}, lg)
    gg, _ = MO.backward_named(layers, fin, {}, lg)
    assert not rg[0].any() and not gg[0].any()


@pytest.mark.parametrize("op", MERGE_OPS)
@pytest.mark.parametrize("n", [0, 1, 7, 8, 9, 16, 23])
def test_branch_merge_closed_forms(op, n):
    """oracle.branch_merge against the definition of each operation, with the
    MAX body/tail split at the largest multiple of 8."""
    rng = np.random.default_rng(n)
    a = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n + 3).astype(np.float32)
    got = O.branch_merge(a, b, op)
    b0 = b[:n]
    want = {"ADD": a + b0, "GATED": a + b0, "ATTENTION_WEIGHTED": a + b0, "MULTIPLY": a * b0,
            "AVERAGE": (a + b0) * np.float32(0.5), "MAX": np.maximum(a, b0),
            "CONCATENATE": np.concatenate([a, b])}[op]
    assert_bitexact(got, want, op, allow_empty=n == 0)
    # Planted mistakes the checks reject: swapped branches for CONCATENATE,
    # a missing halving for AVERAGE.
    if op == "CONCATENATE" and n:
        assert not np.array_equal(got, np.concatenate([b, a]))
    if op == "AVERAGE" and n:
        assert not np.array_equal(got, a + b0)


def test_branch_merge_max_nan_and_zero_rules():
    """vmaxps (a > b ? a : b) over the 8-aligned body, std::max (a < b ? b : a)
    over the tail: NaN and signed-zero ties pick the second operand in the
    body, the first in the tail."""
    a = np.array([np.nan, 1, 0.0, -0.0, 2, 2, 2, 2, np.nan, 1, 0.0, -0.0], np.float32)
    b = np.array([1, np.nan, -0.0, 0.0, 2, 2, 2, 2, 1, np.nan, -0.0, 0.0], np.float32)
    y = O.branch_merge(a, b, "MAX")
    assert y[0] == 1 and np.isnan(y[1])                      # body: second operand
    assert np.signbit(y[2]) and not np.signbit(y[3])
    assert np.isnan(y[8]) and y[9] == 1                      # tail: first operand
    assert not np.signbit(y[10]) and np.signbit(y[11])


@pytest.mark.parametrize("graph", merge_error_graphs(), ids=lambda g: g[0])
def test_short_source_is_refused(graph):
    name, layers, fin, iin = graph
    with pytest.raises(MO.ModelError):
        MO.forward_named(layers, fin, iin, training=True)
    # Inference does not merge, so the same graph runs.
    MO.forward_named(layers, fin, iin)


@pytest.mark.parametrize("seed", MERGE_SEEDS)
def test_random_merge_training_matches_reference(seed):
    name, layers, fin, iin = random_graph(seed, training=True, merges=True)
    try:
        ref = MR.forward_named(layers, fin, iin, training=True)
        rerr = None
    except MR.RefModelError as e:
        ref, rerr = None, str(e)
    try:
        got = MO.forward_named(layers, fin, iin, training=True)
        gerr = None
    except MO.ModelError as e:
        got, gerr = None, str(e)
    assert (rerr is None) == (gerr is None), f"{name}: reference error {rerr!r}, restatement error {gerr!r}"
    if ref is None:
        return
    assert_close(got, ref, name, allow_empty=True)
    lg = _loss(name, ref.size)
    try:
        rg, rin = MR.backward(layers, fin, iin, lg)
    except MR.RefModelError:
        with pytest.raises(MO.ModelError):
            MO.backward_named(layers, fin, iin, lg)
        return
    gg, gin, mags = MO.backward_named(layers, fin, iin, lg, scales=True)
    assert (rin is None) == (gin is None), name
    if rin is not None:
        assert_close(gin, rin, name + " input grad", allow_empty=True)
    for i, (a, b) in enumerate(zip(gg, rg)):
        if b is not None:
            assert_close_sum(a, b, mags[i] if mags[i] is not None else np.abs(b), f"{name} grad_weights[{i}]")
