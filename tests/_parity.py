"""Parity predicates shared by the tests.

Tolerance: an element passes when
|got - ref| <= max(1e-6, 1e-5 * |ref|); NaN must meet NaN and +-inf the same
infinity.  Integer / byte / copy results are compared bit for bit.
"""
import numpy as np

REL = 1e-5
ABS = 1e-6


def err_stats(got, ref):
    g = np.asarray(got, np.float64).ravel()
    r = np.asarray(ref, np.float64).ravel()
    fin = np.isfinite(r)
    d = np.abs(g[fin] - r[fin])
    tol = np.maximum(ABS, REL * np.abs(r[fin]))
    if d.size == 0:
        return 0.0, 0.0, 0.0
    rel = d / np.maximum(np.abs(r[fin]), 1e-30)
    return float(d.max()), float(rel.max()), float((d / tol).max())


def _nonempty(a, what, allow_empty):
    # A comparison of nothing proves nothing: an empty result fails unless the
    # test says an empty result is what it expects.
    assert allow_empty or np.asarray(a).size > 0, f"{what}: nothing to compare (empty result)"


def assert_close(got, ref, what="", rel=REL, abs_=ABS, allow_empty=False):
    got = np.asarray(got)
    ref = np.asarray(ref)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} != {ref.shape}"
    _nonempty(ref, what, allow_empty)
    g = got.astype(np.float64).ravel()
    r = ref.astype(np.float64).ravel()
    nan_r = np.isnan(r)
    assert np.array_equal(np.isnan(g), nan_r), f"{what}: NaN pattern differs"
    inf_r = np.isinf(r)
    assert np.array_equal(g[inf_r], r[inf_r]) and not np.isinf(g[~inf_r]).any(), \
        f"{what}: infinities differ"
    fin = np.isfinite(r)
    d = np.abs(g[fin] - r[fin])
    tol = np.maximum(abs_, rel * np.abs(r[fin]))
    bad = d > tol
    if bad.any():
        idx = np.flatnonzero(fin)[np.argmax(d / tol)]
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {fin.sum()} elements out of tolerance; worst at flat "
            f"index {idx}: got {g[idx]!r} ref {r[idx]!r} (|d|={abs(g[idx]-r[idx]):.3g})")


def assert_bitexact(got, ref, what="", allow_empty=False):
    got = np.ascontiguousarray(got)
    ref = np.ascontiguousarray(ref)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} != {ref.shape}"
    _nonempty(ref, what, allow_empty)
    gv = got.view(np.uint32) if got.dtype.itemsize == 4 else got.view(np.uint8)
    rv = ref.view(np.uint32) if ref.dtype.itemsize == 4 else ref.view(np.uint8)
    diff = np.flatnonzero(gv.ravel() != rv.ravel())
    assert diff.size == 0, (f"{what}: {diff.size} elements differ bitwise; first at {diff[0]}: "
                            f"got {got.ravel()[diff[0]]!r} ref {ref.ravel()[diff[0]]!r}")


def assert_close_or_nearer_exact(got, ref, exact, what="", allow_empty=False):
    """For reductions over long rows.  The reference sums in float32 one
    element at a time (LayerOps.hpp:291-303, 963-967; LayerOpsExt.hpp:357-361),
    whose rounding error grows like u*sqrt(n) and passes 1e-5 relative beyond
    about 10^4 elements; the HIP kernels reduce in a tree.  An element passes
    when it is within tolerance of the reference, or -- where it is not --
    when it is within tolerance of the float64 exact value AND nearer to that
    value than the reference is (the deviation is the reference's own error)."""
    got = np.asarray(got, np.float64).ravel()
    r = np.asarray(ref, np.float64).ravel()
    e = np.asarray(exact, np.float64).ravel()
    assert got.shape == r.shape == e.shape, what
    _nonempty(r, what, allow_empty)
    assert np.array_equal(np.isnan(got), np.isnan(r)), f"{what}: NaN pattern differs"
    inf_r = np.isinf(r)
    assert np.array_equal(got[inf_r], r[inf_r]), f"{what}: infinities differ"
    fin = np.isfinite(r)
    g, r, e = got[fin], r[fin], e[fin]
    near_ref = np.abs(g - r) <= np.maximum(ABS, REL * np.abs(r))
    near_exact = np.abs(g - e) <= np.maximum(ABS, REL * np.abs(e))
    nearer = np.abs(g - e) < np.abs(r - e)
    bad = ~(near_ref | (near_exact & nearer))
    if bad.any():
        i = np.flatnonzero(bad)[0]
        raise AssertionError(f"{what}: {int(bad.sum())} elements fail; first: got {g[i]!r} "
                             f"ref {r[i]!r} exact {e[i]!r}")


def assert_close_sum(got, ref, scale, what="", allow_empty=False):
    """For results that are float32 sums (gradient accumulations over tokens):
    |got - ref| <= max(1e-6, 1e-5 * max(|ref|, scale)), scale = the sum of the
    magnitudes added into the element.  Two float32 summation orders differ
    by up to ~u * scale, so a tolerance relative to the (possibly cancelled)
    result alone would reject correct sums."""
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    sc = np.zeros_like(ref) if scale is None else np.asarray(scale, np.float64).ravel()
    assert got.shape == ref.shape, f"{what}: shape {got.shape} != {ref.shape}"
    _nonempty(ref, what, allow_empty)
    assert np.array_equal(np.isnan(got), np.isnan(ref)), f"{what}: NaN pattern differs"
    fin = np.isfinite(ref)
    d = np.abs(got[fin] - ref[fin])
    tol = np.maximum(ABS, REL * np.maximum(np.abs(ref[fin]), sc[fin]))
    bad = d > tol
    if bad.any():
        idx = np.flatnonzero(fin)[np.argmax(d / tol)]
        raise AssertionError(f"{what}: {int(bad.sum())} of {fin.sum()} elements out of tolerance; worst at "
                             f"{idx}: got {got[idx]!r} ref {ref[idx]!r} scale {sc[idx]:.3g}")


def assert_close_normwise(got, ref, what="", rel=REL, abs_=ABS, allow_empty=False):
    """|got - ref| <= max(abs_, rel * max|ref|) for every element: the error
    measured against the size of the whole result rather than of each element.
    For composed layer graphs, where an element near zero can come out of a
    cancellation (LayerNorm's x - mean on offset data, an Add of opposite
    signs) and carry the rounding error of the larger values it came from;
    the routing mistakes such a test is for (a wrong input, broadcast or
    in-place binding) move the result by a large fraction of its size."""
    got = np.asarray(got)
    ref = np.asarray(ref)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} != {ref.shape}"
    _nonempty(ref, what, allow_empty)
    g = got.astype(np.float64).ravel()
    r = ref.astype(np.float64).ravel()
    assert np.array_equal(np.isnan(g), np.isnan(r)), f"{what}: NaN pattern differs"
    inf_r = np.isinf(r)
    assert np.array_equal(g[inf_r], r[inf_r]) and not np.isinf(g[~inf_r]).any(), f"{what}: infinities differ"
    fin = np.isfinite(r)
    if not fin.any():
        return
    tol = max(abs_, rel * float(np.abs(r[fin]).max()))
    d = np.abs(g[fin] - r[fin])
    if (d > tol).any():
        idx = np.flatnonzero(fin)[np.argmax(d)]
        raise AssertionError(f"{what}: {int((d > tol).sum())} of {fin.sum()} elements beyond {tol:.3g}; worst at "
                             f"flat index {idx}: got {g[idx]!r} ref {r[idx]!r} (|d|={abs(g[idx] - r[idx]):.3g})")


# The device sums the dy rows of an id with at least this many tokens in
# 32-token segments, then the segments in order: deterministic, and the
# reference's token-order sum to float32 rounding.  Rarer ids keep the
# reference's sequence of adds.
EMBED_LONG_RUN = 32


def assert_embedding_scatter(got, ref, counts, scale, what=""):
    """Embedding backward (a scatter-add into the gradient table, [vocab, dim]):
    rows of ids with fewer than EMBED_LONG_RUN tokens must equal ref bit for
    bit; rows of more frequent ids are float32 sums held to assert_close_sum
    with `scale` (|gradient row| + the sum of the |dy| rows added)."""
    got = np.asarray(got, np.float32).reshape(counts.size, -1)
    ref = np.asarray(ref, np.float32).reshape(counts.size, -1)
    short = counts < EMBED_LONG_RUN
    assert_bitexact(got[short], ref[short], what + " (ids with fewer than 32 tokens)", allow_empty=True)
    if (~short).any():
        sc = np.asarray(scale, np.float64).reshape(counts.size, -1)
        assert_close_sum(got[~short], ref[~short], sc[~short], what + " (frequent ids, segment sums)")
