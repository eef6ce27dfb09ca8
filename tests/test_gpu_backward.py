"""Backward ops (libmimir_hip, backward.hip) against the CPU oracle's
restatement of Model::backwardPass (Model.cpp:7305-9153) on the same seeded
inputs.

Tolerances: input gradients |gpu - ref| <= max(1e-6, 1e-5*|ref|) (widths
beyond 4096 may instead be nearer the float64 value than the reference);
gradient sums over tokens (dgamma, dbeta, a broadcast operand's gradient)
the same bound relative to the magnitudes summed (float32 sums in another
order differ by ~u * that); Multiply / Add gradients and accumulate_grad bit
for bit; the Embedding scatter-add bit for bit for ids with fewer than 32
tokens, and for more frequent ids (summed in segments) as a gradient sum."""
import os

import numpy as np
import pytest

import mimir_hip as M
import oracle as O
import _exact as X
from _parity import (assert_bitexact, assert_close, assert_close_or_nearer_exact, assert_close_sum,
                     assert_embedding_scatter)

pytestmark = pytest.mark.gpu

rng = np.random.default_rng(0xBAC)


def dev(ctx, a, offset=0):
    a = np.ascontiguousarray(a)
    buf = ctx.empty(a.size + offset, a.dtype)
    view = buf.offset(offset, a.shape) if offset else buf
    ctx.upload(view, a)
    return buf, view


# ---------------------------------------------------------------------------
# LayerNorm
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("cols", [1, 3, 4, 64, 100, 256, 512, 1000, 1023, 1024, 2047, 2048, 4095, 4096, 4099, 4100,
                                  8192, 20000])
@pytest.mark.parametrize("affine", ["gb", "g", "none"])
def test_layernorm_bwd(ctx, cols, affine):
    rows = 37 if cols <= 4096 else 5
    x = (1.5 * rng.standard_normal((rows, cols)) + 0.25).astype(np.float32)
    dy = rng.standard_normal((rows, cols)).astype(np.float32)
    g = (1 + 0.2 * rng.standard_normal(cols)).astype(np.float32) if affine != "none" else None
    has_b = affine == "gb"
    prev = rng.standard_normal(2 * cols).astype(np.float32)
    dx_ref, gp_ref = O.layernorm_bwd(x, dy, cols, g, has_b, 1e-5, prev[:cols * (2 if has_b else 1)] if g is not None
                                     else None)
    ex_dx, _, _, (sg, sb), dxs = X.layernorm_bwd(x, dy, cols, g, 1e-5)
    bufs = [dev(ctx, a) for a in (x, dy)]
    gb = dev(ctx, g) if g is not None else (None, None)
    dxb = ctx.empty(x.shape)
    dgb = dev(ctx, prev[:cols]) if g is not None else (None, None)
    dbb = dev(ctx, prev[cols:]) if has_b else (None, None)
    try:
        ctx.layernorm_bwd(bufs[0][1], bufs[1][1], gb[1], dxb, dgb[1], dbb[1], rows, cols, 1e-5)
        dx = dxb.numpy()
        # dx = inv/n * (n*dxh - sum - xhat*sum2) cancels: held to the tolerance
        # relative to the terms' magnitude (dxs); beyond 4096 it may instead be
        # nearer the float64 value than the reference.
        assert_close_or_nearer_exact(dx.ravel(), dx_ref, ex_dx, f"dx cols={cols}")
        if cols <= 4096:
            assert_close_sum(dx.ravel(), dx_ref, dxs, f"dx cols={cols}")
        if g is not None:
            assert_close_sum(dgb[1].numpy(), gp_ref[:cols], np.abs(prev[:cols]) + sg, "dgamma")
        if has_b:
            assert_close_sum(dbb[1].numpy(), gp_ref[cols:], np.abs(prev[cols:]) + sb, "dbeta")
        # accumulate_grad into a present gradient: dx += value
        base = rng.standard_normal(x.shape).astype(np.float32)
        ctx.upload(dxb, base)
        ctx.layernorm_bwd(bufs[0][1], bufs[1][1], gb[1], dxb, None, None, rows, cols, 1e-5, accumulate=True)
        assert_bitexact(dxb.numpy().ravel(), O.accumulate(base, dx.ravel()), f"dx accumulate cols={cols}")
    finally:
        for b in (bufs[0][0], bufs[1][0], gb[0], dgb[0], dbb[0], dxb):
            if b is not None:
                b.free()


@pytest.mark.parametrize("rows,cols", [(8192, 4096), (3000, 512), (1025, 64), (70000, 16), (8192, 4095), (3000, 1023),
                                       (70000, 17), (100, 4096), (300, 64), (2000, 20)])
def test_layernorm_bwd_many_rows(ctx, rows, cols):
    # Many rows per persistent-grid slot: dgamma / dbeta sums over thousands of
    # tokens (odd widths: the 4-byte-column kernel).  100 and 300 rows: slot
    # counts that are not a multiple of the one-launch slot sum's 128 slot
    # lanes; 20 columns: its last tile of 8 float4 columns half empty.
    x = rng.standard_normal((rows, cols), dtype=np.float32)
    dy = rng.standard_normal((rows, cols), dtype=np.float32)
    g = (1 + 0.02 * rng.standard_normal(cols)).astype(np.float32)
    dx_ref, gp_ref = O.layernorm_bwd(x, dy, cols, g, True, 1e-5)
    _, _, _, (sg, sb), dxs = X.layernorm_bwd(x, dy, cols, g, 1e-5)
    (bx, vx), (bd, vd), (bg, vg) = dev(ctx, x), dev(ctx, dy), dev(ctx, g)
    dxb = ctx.empty(x.shape)
    dgb, dbb = ctx.to_device(np.zeros(cols, np.float32)), ctx.to_device(np.zeros(cols, np.float32))
    try:
        ctx.layernorm_bwd(vx, vd, vg, dxb, dgb, dbb, rows, cols, 1e-5)
        assert_close_sum(dxb.numpy().ravel(), dx_ref, dxs, "dx")
        assert_close_sum(dgb.numpy(), gp_ref[:cols], sg, "dgamma")
        assert_close_sum(dbb.numpy(), gp_ref[cols:], sb, "dbeta")
        # Deterministic: a second run gives the same bits.
        d1 = dgb.numpy().copy()
        ctx.upload(dgb, np.zeros(cols, np.float32))
        ctx.layernorm_bwd(vx, vd, vg, dxb, dgb, None, rows, cols, 1e-5)
        assert_bitexact(dgb.numpy(), d1, "dgamma rerun")
    finally:
        for b in (bx, bd, bg, dxb, dgb, dbb):
            b.free()


def test_layernorm_bwd_unaligned_and_inplace(ctx):
    rows, cols = 9, 256
    x = rng.standard_normal((rows, cols), dtype=np.float32)
    dy = rng.standard_normal((rows, cols), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    dx_ref, gp_ref = O.layernorm_bwd(x, dy, cols, g, True, 1e-5)
    (bx, vx), (bd, vd), (bg, vg) = dev(ctx, x, 1), dev(ctx, dy, 1), dev(ctx, g, 1)
    dgb, dbb = ctx.to_device(np.zeros(cols, np.float32)), ctx.to_device(np.zeros(cols, np.float32))
    try:
        ctx.layernorm_bwd(vx, vd, vg, vd, dgb, dbb, rows, cols, 1e-5)  # unaligned (4-byte columns), dx over dy
        _, _, _, (sg, sb), dxs = X.layernorm_bwd(x, dy, cols, g, 1e-5)
        assert_close_sum(vd.numpy().ravel(), dx_ref, dxs, "dx unaligned in place")
        assert_close_sum(dgb.numpy(), gp_ref[:cols], sg, "dgamma unaligned")
        assert_close_sum(dbb.numpy(), gp_ref[cols:], sb, "dbeta unaligned")
        # Aligned (register-resident rows), dx over dy as well.
        (ax, avx), (ad, avd), (ag, avg) = dev(ctx, x), dev(ctx, dy), dev(ctx, g)
        ctx.upload(dgb, np.zeros(cols, np.float32))
        ctx.layernorm_bwd(avx, avd, avg, avd, dgb, None, rows, cols, 1e-5)
        assert_close_sum(avd.numpy().ravel(), dx_ref, dxs, "dx aligned in place")
        assert_close_sum(dgb.numpy(), gp_ref[:cols], sg, "dgamma aligned, dx over dy")
        for b in (ax, ad, ag):
            b.free()
    finally:
        for b in (bx, bd, bg, dgb, dbb):
            b.free()


def test_layernorm_bwd_errors(ctx):
    d = ctx.to_device(np.ones(8, np.float32))
    try:
        with pytest.raises(M.MimirError):
            ctx.layernorm_bwd(d, d, None, d, d, None, 2, 4, 1e-5)  # dgamma without gamma
        with pytest.raises(M.MimirError):
            ctx.layernorm_bwd(d, d, d, d, None, d, 2, 4, 1e-5)  # dbeta without dgamma
        with pytest.raises(M.MimirError):
            ctx.layernorm_bwd(d, d, None, d, None, None, 2, 0, 1e-5)
    finally:
        d.free()


# ---------------------------------------------------------------------------
# GELU / SiLU
# ---------------------------------------------------------------------------

SPECIALS = np.array([0.0, -0.0, 1e-30, -1e-40, 3.0, -3.0, 5.0, -5.0, 9.0, -9.0, 20.0, -20.0, 88.0, -88.0,
                     100.0, -100.0, 1e20, -1e20, np.inf, -np.inf, np.nan], np.float32)


@pytest.mark.parametrize("offset", [0, 1])
@pytest.mark.parametrize("acc", [False, True])
def test_gelu_silu_bwd(ctx, offset, acc):
    x = np.concatenate([np.linspace(-10, 10, 40001, dtype=np.float32), SPECIALS,
                        rng.standard_normal(50001).astype(np.float32) * 3])
    dy = rng.standard_normal(x.size).astype(np.float32)
    base = rng.standard_normal(x.size).astype(np.float32)
    (bx, vx), (bd, vd), (bo, vo) = dev(ctx, x, offset), dev(ctx, dy, offset), dev(ctx, base, offset)
    try:
        for name, fn, ref_fn, ex in (("gelu", ctx.gelu_bwd, O.gelu_bwd, X.dgelu), ("silu", ctx.silu_bwd,
                                                                                   O.silu_bwd, X.dsilu)):
            ctx.upload(vo, base)
            fn(vx, vd, vo, x.size, accumulate=acc)
            got = vo.numpy()
            ref = ref_fn(x, dy)
            exact = dy.astype(np.float64) * ex(x)
            if acc:
                ref = O.accumulate(base, ref)
                exact = base.astype(np.float64) + exact
            # GELU: the reference's 1+tanh and 1-tanh^2 cancel for |x| > 3; the
            # kernel's logistic form does not, and must then be nearer the
            # float64 value than the reference when it leaves the tolerance.
            assert_close_or_nearer_exact(got, ref, exact, f"{name}_bwd acc={acc}")
            if name == "silu":
                assert_close(got, ref, f"{name}_bwd acc={acc}")
            else:
                ok = np.abs(x) <= 3
                assert_close(got[ok], ref[ok], "gelu_bwd |x|<=3")
    finally:
        for b in (bx, bd, bo):
            b.free()


# ---------------------------------------------------------------------------
# Multiply / Add (bit-exact)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n", [1, 7, 4096, 100003])
def test_mul_bwd_bitexact(ctx, n):
    a, b, dy, pa, pb = (rng.standard_normal(n).astype(np.float32) for _ in range(5))
    ra, rb = O.mul_bwd(a, b, dy)
    ba, bb, bdy = ctx.to_device(a), ctx.to_device(b), ctx.to_device(dy)
    da, db = ctx.to_device(pa), ctx.to_device(pb)
    try:
        ctx.mul_bwd(ba, bb, bdy, da, db, n)
        assert_bitexact(da.numpy(), ra, "da")
        assert_bitexact(db.numpy(), rb, "db")
        ctx.upload(da, pa)
        ctx.upload(db, pb)
        ctx.mul_bwd(ba, bb, bdy, da, db, n, acc_a=True, acc_b=True)
        assert_bitexact(da.numpy(), O.accumulate(pa, ra), "da accumulate")
        assert_bitexact(db.numpy(), O.accumulate(pb, rb), "db accumulate")
        # da aliases dy (output and first input share a name): products first.
        ctx.mul_bwd(ba, bb, bdy, bdy, db, n, acc_a=True)
        assert_bitexact(bdy.numpy(), O.accumulate(dy, ra), "da aliasing dy")
        # Multiply(x, x): both accumulations land on one buffer, in order.
        ctx.upload(bdy, dy)
        ctx.upload(da, pa)
        ctx.mul_bwd(ba, ba, bdy, da, da, n, acc_a=True, acc_b=True)
        r0, r1 = O.mul_bwd(a, a, dy)
        assert_bitexact(da.numpy(), O.accumulate(O.accumulate(pa, r0), r1), "da == db")
    finally:
        for d in (ba, bb, bdy, da, db):
            d.free()


@pytest.mark.parametrize("na,nb", [(4096, 4096), (4097, 4097), (64 * 4096, 4096), (4096, 64 * 4096),
                                   (3 * 48, 48), (8192 * 4096, 1), (1, 1000), (999, 999)])
def test_add_bwd(ctx, na, nb):
    n = max(na, nb)
    dy = rng.standard_normal(n).astype(np.float32)
    pa = rng.standard_normal(na).astype(np.float32)
    pb = rng.standard_normal(nb).astype(np.float32)
    bdy, da, db = ctx.to_device(dy), ctx.to_device(pa), ctx.to_device(pb)
    try:
        for acc in (False, True):
            ctx.upload(da, pa)
            ctx.upload(db, pb)
            ctx.add_bwd(bdy, na, nb, da, db, acc_a=acc, acc_b=acc)
            for got, mine, prev in ((da.numpy(), na, pa), (db.numpy(), nb, pb)):
                if mine == n:
                    assert_bitexact(got, O.accumulate(prev, dy) if acc else dy, f"big operand acc={acc}")
                else:
                    s = O.add_bwd_small(dy, mine)
                    ref = O.accumulate(prev, s) if acc else s
                    scale = np.abs(dy.astype(np.float64)).reshape(-1, mine).sum(axis=0) + (np.abs(prev) if acc else 0)
                    assert_close_sum(got, ref, scale, f"small operand acc={acc}")
    finally:
        for d in (bdy, da, db):
            d.free()


def test_add_bwd_aliasing_is_the_references(ctx):
    # Add(x, x) -> x: the reference adds dy onto itself twice (4*dy).
    dy = rng.standard_normal(1000).astype(np.float32)
    d = ctx.to_device(dy)
    try:
        ctx.add_bwd(d, 1000, 1000, d, d, acc_a=True, acc_b=True)
        assert_bitexact(d.numpy(), (dy + dy) + (dy + dy), "x + x")
        # Broadcast with the big operand's gradient aliasing dy: the small
        # operand's sum reads the doubled dy.
        dy2 = rng.standard_normal(64 * 32).astype(np.float32)
        big = ctx.to_device(dy2)
        small = ctx.to_device(np.zeros(32, np.float32))
        ctx.add_bwd(big, 64 * 32, 32, big, small, acc_a=True, acc_b=False)
        assert_bitexact(big.numpy(), dy2 + dy2, "big aliasing dy")
        assert_close_sum(small.numpy(), O.add_bwd_small(dy2 + dy2, 32),
                         2 * np.abs(dy2.astype(np.float64)).reshape(-1, 32).sum(axis=0), "small after doubling")
        big.free()
        small.free()
    finally:
        d.free()


def test_add_bwd_errors(ctx):
    d = ctx.to_device(np.ones(10, np.float32))
    try:
        with pytest.raises(M.MimirError):
            ctx.add_bwd(d, 10, 3, d, d)  # not broadcastable
        with pytest.raises(M.MimirError):
            ctx.add_bwd(d, 0, 3, d, d)
    finally:
        d.free()


# ---------------------------------------------------------------------------
# Embedding scatter-add: ids with fewer than 32 tokens bit-exact (token order),
# more frequent ids summed in segments (sum tolerance), always deterministic
# ---------------------------------------------------------------------------

def _scatter_counts_scale(ids, dy, gt, vocab, dim, pad):
    """Per row of the gradient table: how many tokens add into it, and
    |row| + the sum of their |dy| rows -- both through the oracle's own id
    mapping (padding, out-of-range ids, float-id rounding)."""
    n = np.asarray(ids).size
    counts = O.embedding_bwd(ids, np.ones((n, 1), np.float32), np.zeros(vocab, np.float32), vocab, 1, pad)
    scale = O.embedding_bwd(ids, np.abs(dy), np.abs(gt), vocab, dim, pad)
    return counts.astype(np.int64), scale


def _check_scatter(got, ref, ids, dy, gt, vocab, dim, pad, what):
    counts, scale = _scatter_counts_scale(ids, dy, gt, vocab, dim, pad)
    assert_embedding_scatter(got, ref, counts, scale, what)


@pytest.mark.parametrize("vocab,dim,n,pad", [(32000, 4096, 2048, -1), (50, 64, 5000, 3), (7, 6, 100, 0),
                                             (1000, 128, 32768, -1), (1, 4, 10, -1)])
@pytest.mark.parametrize("float_ids", [False, True])
def test_embedding_bwd(ctx, vocab, dim, n, pad, float_ids):
    ids = rng.integers(-2, vocab + 2, n).astype(np.int32)
    ids[: n // 4] = min(5, vocab - 1)  # one row hit many times
    arg = ids.astype(np.float32) + np.float32(0.25) if float_ids else ids
    dy = rng.standard_normal((n, dim)).astype(np.float32)
    gt = rng.standard_normal(vocab * dim).astype(np.float32)
    ref = O.embedding_bwd(arg, dy, gt, vocab, dim, pad)
    bi, bdy, bg = ctx.to_device(arg), ctx.to_device(dy), ctx.to_device(gt)
    try:
        ctx.embedding_bwd(bi, n, bdy, bg, gt.size, vocab, dim, pad, float_ids=float_ids)
        got = bg.numpy()
        _check_scatter(got, ref, arg, dy, gt, vocab, dim, pad, "grad table")
        ctx.upload(bg, gt)  # the same call again: the same bits
        ctx.embedding_bwd(bi, n, bdy, bg, gt.size, vocab, dim, pad, float_ids=float_ids)
        assert_bitexact(bg.numpy(), got, "repeated call")
    finally:
        for d in (bi, bdy, bg):
            d.free()


def _embedding_bwd_gpu(c, ids, dy, gt, vocab, dim, pad):
    bi, bdy, bg = c.to_device(ids), c.to_device(dy), c.to_device(gt)
    try:
        c.embedding_bwd(bi, ids.size, bdy, bg, gt.size, vocab, dim, pad)
        return bg.numpy()
    finally:
        for d in (bi, bdy, bg):
            d.free()


@pytest.mark.parametrize("case", ["262144 tokens", "long runs", "padding block"])
def test_embedding_bwd_repeats(ctx, case):
    """Many tokens per id: a 64-id table hit by 2^18 tokens (runs of ~4000,
    padding and out-of-range ids mixed in), blocks of 4096 tokens of a single
    id, and a block of padding only."""
    vocab, dim, pad = 64, 8, -1
    if case == "262144 tokens":
        n = 64 * 4096
        ids = rng.integers(-1, vocab + 1, n).astype(np.int32)
    elif case == "long runs":
        n = 3 * 4096 + 7
        ids = np.full(n, 5, np.int32)
        ids[4096:8192] = 7
    else:
        pad = 2
        n = 2 * 4096 + 100
        ids = rng.integers(0, vocab, n).astype(np.int32)
        ids[4096:8192] = pad
    dy = rng.standard_normal((n, dim)).astype(np.float32)
    gt = rng.standard_normal(vocab * dim).astype(np.float32)
    ref = O.embedding_bwd(ids, dy, gt, vocab, dim, pad)
    _check_scatter(_embedding_bwd_gpu(ctx, ids, dy, gt, vocab, dim, pad), ref, ids, dy, gt, vocab, dim, pad, case)


@pytest.mark.parametrize("case", ["zipf ids, dim 4096", "runs around the long-run threshold, dim 132"])
def test_embedding_bwd_long_runs(ctx, case):
    """Ids with 32 tokens or more: their rows are summed in 32-token segments
    (segments cut at multiples of 32 in sorted order), then the segment sums
    onto the gradient row in four slot groups per 64-column block.  Zipf(1.0)
    ids are what a text batch looks like (the top id is ~9% of the tokens);
    the second case puts runs of 1, 31, 32, 33, 63, 64, 65 and 200 tokens next
    to each other, with 33 16-byte columns per row (a partial column block,
    runs of 1 to 7 slots).  Rarer ids stay bit-exact; two calls give the same
    bits."""
    if case.startswith("zipf"):
        vocab, dim, n = 2000, 4096, 8192
        r = np.arange(1, vocab + 1, dtype=np.float64) ** -1.0
        ids = rng.choice(vocab, n, p=r / r.sum()).astype(np.int32)
    else:
        vocab, dim = 40, 132
        ids = np.concatenate([np.full(k, i, np.int32) for i, k in enumerate([1, 31, 32, 33, 63, 64, 65, 200, 3])])
        ids = rng.permutation(ids)
        n = ids.size
    dy = rng.standard_normal((n, dim)).astype(np.float32)
    gt = rng.standard_normal(vocab * dim).astype(np.float32)
    ref = O.embedding_bwd(ids, dy, gt, vocab, dim, -1)
    got = _embedding_bwd_gpu(ctx, ids, dy, gt, vocab, dim, -1)
    _check_scatter(got, ref, ids, dy, gt, vocab, dim, -1, case)
    assert_bitexact(_embedding_bwd_gpu(ctx, ids, dy, gt, vocab, dim, -1), got, case + ", second call")
    counts, _ = _scatter_counts_scale(ids, dy, gt, vocab, dim, -1)
    assert (counts >= 32).any() and (counts < 32).any()  # both paths ran


def _tuned(tune):
    old = os.environ.get("MIMIR_TUNE")
    os.environ["MIMIR_TUNE"] = tune
    try:
        return M.Context(0)
    finally:
        if old is None:
            del os.environ["MIMIR_TUNE"]
        else:
            os.environ["MIMIR_TUNE"] = old


@pytest.fixture(scope="module")
def sort_ctxs():
    """Contexts whose Embedding backward sorts with rocPRIM's radix sort and
    takes a workgroup per sorted position (MIMIR_TUNE embsort=0), sorts by
    counting but keeps the per-position rows kernel (embruns=0), or counts in
    three launches instead of one (emb1pass=0), beside the default (the
    counting sort in one launch up to 32 blocks and 33792 keys, a workgroup per listed
    run)."""
    cs = {"radix": _tuned("embsort=0"), "positions": _tuned("embruns=0"), "three": _tuned("emb1pass=0")}
    yield cs
    for c in cs.values():
        c.close()


@pytest.mark.parametrize("vocab,n,dist,float_ids", [
    (32000, 32768, "uniform", False), (32000, 32768, "zipf", False), (32000, 32768, "uniform", True),
    (1023, 65536, "uniform", False), (1024, 65535, "zipf", False), (1025, 1025, "uniform", True),
    (1, 3000, "uniform", False), (70000, 4097, "uniform", False), (32000, 65537, "uniform", False),
    (5, 1024, "one id", False), (33791, 20000, "uniform", False), (33792, 9000, "zipf", True),
    (5, 65536, "one id", False), (100, 32769, "uniform", False), (40, 32768, "zipf", True)])
def test_embedding_bwd_counting_sort_matches_radix_sort(ctx, sort_ctxs, vocab, n, dist, float_ids):
    """The counting sort (up to 64 blocks of 1024 tokens; in one launch up to
    32 blocks and 33792 keys, else three) puts every (id, token) pair where the stable radix
    sort does, and its run list names every run the per-position kernel
    finds, so the gradients are the same bits: chunk edges of the key scan
    (vocab + 1 around 1024), padding and out-of-range ids (the skipped key), a
    last partial block, the 64-block limit and just past it (the radix sort
    on both sides), a table or a launch past the one-launch limits (70000
    ids, 33793 keys, 33 blocks)."""
    dim = 64
    if dist == "zipf":
        r = np.arange(1, vocab + 1, dtype=np.float64) ** -1.0
        ids = rng.choice(vocab, n, p=r / r.sum()).astype(np.int32)
    elif dist == "one id":
        ids = np.full(n, 3, np.int32)
    else:
        ids = rng.integers(-2, vocab + 2, n).astype(np.int32)
    pad = 1 if vocab > 1 else -1
    arg = ids.astype(np.float32) + np.float32(0.25) if float_ids else ids
    dy = rng.standard_normal((n, dim)).astype(np.float32)
    gt = rng.standard_normal(vocab * dim).astype(np.float32)
    got = {}
    for name, c in (("counting", ctx), ("radix", sort_ctxs["radix"]), ("positions", sort_ctxs["positions"]),
                    ("three", sort_ctxs["three"])):
        bi, bdy, bg = c.to_device(arg), c.to_device(dy), c.to_device(gt)
        try:
            c.embedding_bwd(bi, n, bdy, bg, gt.size, vocab, dim, pad, float_ids=float_ids)
            got[name] = bg.numpy()
        finally:
            for d in (bi, bdy, bg):
                d.free()
    assert_bitexact(got["counting"], got["radix"], f"{dist} ids, vocab {vocab}, {n} tokens")
    assert_bitexact(got["positions"], got["radix"], f"{dist} ids, vocab {vocab}, {n} tokens, per position")
    assert_bitexact(got["three"], got["radix"], f"{dist} ids, vocab {vocab}, {n} tokens, three-launch count")
    ref = O.embedding_bwd(arg, dy, gt, vocab, dim, pad)
    _check_scatter(got["counting"], ref, arg, dy, gt, vocab, dim, pad, "grad table")


@pytest.mark.parametrize("n", [4099, 32768])
def test_embedding_bwd_ids_off_alignment(ctx, sort_ctxs, n):
    """Ids starting 4 bytes past a 16-byte boundary: the one-launch sort reads
    them word by word instead of as 16-byte vectors, and places the pairs
    where the radix sort does."""
    vocab, dim = 3000, 64
    ids = rng.integers(-1, vocab + 1, n).astype(np.int32)
    dy = rng.standard_normal((n, dim)).astype(np.float32)
    gt = rng.standard_normal(vocab * dim).astype(np.float32)
    got = {}
    for name, c in (("counting", ctx), ("radix", sort_ctxs["radix"])):
        buf = c.empty(n + 1, np.int32)
        bi = buf.offset(1, (n,))
        c.upload(bi, ids)
        bdy, bg = c.to_device(dy), c.to_device(gt)
        try:
            c.embedding_bwd(bi, n, bdy, bg, gt.size, vocab, dim, 2)
            got[name] = bg.numpy()
        finally:
            for d in (buf, bdy, bg):
                d.free()
    assert_bitexact(got["counting"], got["radix"], f"{n} ids off alignment")
    ref = O.embedding_bwd(ids, dy, gt, vocab, dim, 2)
    _check_scatter(got["counting"], ref, ids, dy, gt, vocab, dim, 2, "ids off alignment")


def test_embedding_bwd_unaligned_rows_and_errors(ctx):
    vocab, dim, n = 9, 5, 300
    ids = rng.integers(0, vocab, n).astype(np.int32)
    dy = rng.standard_normal((n, dim)).astype(np.float32)
    gt = np.zeros(vocab * dim, np.float32)
    ref = O.embedding_bwd(ids, dy, gt, vocab, dim, -1)
    bi, bdy, bg = ctx.to_device(ids), ctx.to_device(dy), ctx.to_device(gt)
    try:
        ctx.embedding_bwd(bi, n, bdy, bg, gt.size, vocab, dim, -1)
        assert_bitexact(bg.numpy(), ref, "dim 5 (scalar rows)")
        with pytest.raises(M.MimirError):
            ctx.embedding_bwd(bi, n, bdy, bg, gt.size - 1, vocab, dim, -1)  # table too small
        # The scalar rows kernel (dim 5) takes a 256-thread workgroup per id:
        # 2^24 + 1 ids exceed the dispatch's 2^32 work-items, refused before
        # any launch (the buffers are far shorter than such a call would read).
        with pytest.raises(M.MimirError) as e:
            ctx.embedding_bwd(bi, (1 << 24) + 1, bdy, bg, gt.size, vocab, dim, -1)
        assert e.value.status == M.EINVAL and "grid limit" in str(e.value)
        assert_bitexact(bg.numpy(), ref, "untouched by the refused call")
    finally:
        for d in (bi, bdy, bg):
            d.free()


def _ln_bwd_exact(x, dy, g, eps):
    """float64 LayerNorm backward of rows of x: (dx, sum over rows of dy*xh, sum of dy)."""
    x64, dy64 = x.astype(np.float64), dy.astype(np.float64)
    mu = x64.mean(1, keepdims=True)
    sig = np.sqrt(((x64 - mu) ** 2).mean(1, keepdims=True) + eps)
    xh = (x64 - mu) / sig
    dxh = dy64 * (1.0 if g is None else g.astype(np.float64))
    dx = (dxh - dxh.mean(1, keepdims=True) - xh * (dxh * xh).mean(1, keepdims=True)) / sig
    return dx, (dy64 * xh).sum(0), dy64.sum(0)


@pytest.mark.parametrize("rows,cols,affine,acc,shift", [(1, 1 << 20, True, False, 0), (3, 20004, False, True, 0),
                                                        (2, 65536, True, True, 0), (2, 20000, True, False, 1),
                                                        (40, 20004, True, False, 0), (1040, 16388, True, True, 0)])
def test_layernorm_bwd_long_rows(ctx, rows, cols, affine, acc, shift):
    """Rows wider than one workgroup takes (a LayerNorm with in_features unset
    normalises the whole input): the chunked path.  Offset rows (mean 3), the
    reference's sequential sums against the float64 value: dx within tolerance
    of the oracle or nearer the float64 value than it; dgamma / dbeta (added
    onto random values) and the accumulated dx within tolerance.  shift=1
    puts dgamma / dbeta one float off 16-byte alignment (scalar updates).
    Past 16 rows the apply pass works in groups of 16 rows whose column sums
    go to slots (40 rows: 3 slots; 1040 rows: 65, the two-level slot sum);
    dgamma / dbeta are then sums over many rows and are held to the
    sum-aware rule (1e-5 of the magnitudes summed)."""
    r = np.random.default_rng(cols + rows)
    x = (3 + r.standard_normal((rows, cols))).astype(np.float32)
    dy = r.standard_normal((rows, cols)).astype(np.float32)
    g = (1 + 0.1 * r.standard_normal(cols)).astype(np.float32) if affine else None
    dx0 = r.standard_normal((rows, cols)).astype(np.float32) if acc else np.zeros((rows, cols), np.float32)
    gp0 = r.standard_normal(2 * cols).astype(np.float32)
    bx, bdy, bdx = ctx.to_device(x), ctx.to_device(dy), ctx.to_device(dx0)
    bg = ctx.to_device(g) if affine else None
    keep = []

    def params(v):
        full = ctx.to_device(np.concatenate([np.zeros(shift, np.float32), v]))
        keep.append(full)
        return full.offset(shift, (cols,)) if shift else full
    bdg = params(gp0[:cols].copy()) if affine else None
    bdb = params(gp0[cols:].copy()) if affine else None
    try:
        ctx.layernorm_bwd(bx, bdy, bg, bdx, bdg, bdb, rows, cols, 1e-5, accumulate=acc)
        got = bdx.numpy()
        ref, gp = O.layernorm_bwd(x, dy, cols, g, has_bias=affine, eps=1e-5,
                                  grad_params=gp0 if affine else None)
        ex_dx, ex_dg, ex_db = _ln_bwd_exact(x, dy, g, 1e-5)
        assert_close_or_nearer_exact(got, dx0 + ref.reshape(rows, cols), dx0.astype(np.float64) + ex_dx,
                                     "dx accumulated" if acc else "dx")
        if affine:
            x64 = x.astype(np.float64)
            xh = (x64 - x64.mean(1, keepdims=True)) / np.sqrt(x64.var(1, keepdims=True) + 1e-5)
            mg = np.abs(gp0[:cols]) + np.abs(dy * xh).sum(0)
            mb = np.abs(gp0[cols:]) + np.abs(dy).sum(0)
            assert_close_sum(bdg.numpy(), gp0[:cols] + ex_dg, mg, "dgamma")
            assert_close_sum(bdb.numpy(), gp0[cols:] + ex_db, mb, "dbeta")
    finally:
        for d in [bx, bdy, bdx, bg] + keep:
            if d is not None:
                d.free()
