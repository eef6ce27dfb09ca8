"""HIP path (libmimir_hip via its C ABI) against the CPU oracle on the same
seeded inputs, plus the edge cases the reference's semantics define.

Tolerance: |gpu - ref| <= max(1e-6, 1e-5*|ref|) for the floating-point ops;
gather, residual add and multiply must be bit-identical."""
import numpy as np
import pytest

import mimir_hip as M
import oracle as O
import _exact as X
from _parity import assert_bitexact, assert_close, assert_close_or_nearer_exact
from mimir_hip import datagen as G

pytestmark = pytest.mark.gpu

rng = np.random.default_rng(7)

SPECIALS = np.array([0.0, -0.0, 1e-30, -1e-30, 1e-40, -1e-40, 3.0, -3.0, 5.0, -5.0, 9.0, -9.0,
                     20.0, -20.0, 88.0, -88.0, 100.0, -100.0, 3e38, -3e38, np.inf, -np.inf,
                     np.nan], np.float32)


def run(ctx, fn, *arrays, out_shape, offset=0):
    """Upload inputs (optionally `offset` floats into their buffers, to take
    the unaligned paths), run fn(dev_inputs..., dev_out), download."""
    dev = []
    for a in arrays:
        if a is None:
            dev.append(None)
            continue
        a = np.ascontiguousarray(a)
        buf = ctx.empty(a.size + offset, a.dtype)
        view = buf.offset(offset, a.shape) if offset else buf
        ctx.upload(view, a)
        dev.append((buf, view))
    n_out = int(np.prod(out_shape))
    ybuf = ctx.empty(max(n_out + offset, 1))
    y = ybuf.offset(offset, out_shape) if offset else ybuf
    try:
        fn(*[None if d is None else d[1] for d in dev], y)
        out = np.empty(out_shape, np.float32)
        if n_out:
            ctx.download(out, y)
        return out
    finally:
        for d in dev:
            if d is not None:
                d[0].free()
        ybuf.free()


# ---------------------------------------------------------------------------
# LayerNorm
# ---------------------------------------------------------------------------

def test_layernorm_cfg0(ctx):
    x, g, b, eps = G.cfg0_layernorm()
    got = run(ctx, lambda dx, dg, db, y: ctx.layernorm(dx, dg, db, y, 256, 512, eps), x, g, b,
              out_shape=x.shape)
    assert_close(got, O.layernorm(x, 512, g, b, eps).reshape(x.shape), "cfg0 layernorm")


@pytest.mark.parametrize("cols", [1, 3, 4, 64, 100, 256, 512, 1000, 1024, 2048, 4096, 4100, 8192,
                                  16384, 20000])
@pytest.mark.parametrize("affine", ["gb", "g", "none"])
def test_layernorm_shapes(ctx, cols, affine):
    rows = 9
    x = (rng.standard_normal((rows, cols), dtype=np.float32) * 1.5 + 0.25)
    g = (1 + 0.02 * rng.standard_normal(cols)).astype(np.float32) if affine != "none" else None
    b = (0.02 * rng.standard_normal(cols)).astype(np.float32) if affine == "gb" else None
    got = run(ctx, lambda dx, dg, db, y: ctx.layernorm(dx, dg, db, y, rows, cols, 1e-5), x, g, b,
              out_shape=x.shape)
    ref = O.layernorm(x, cols, g, b, 1e-5).reshape(x.shape)
    assert_close_or_nearer_exact(got, ref, X.layernorm(x, cols, g, b, 1e-5), f"LN cols={cols}")
    if cols <= 4096:  # the BASELINE widths: strict tolerance against the reference
        assert_close(got, ref, f"LN cols={cols}")


@pytest.mark.parametrize("cols", [512, 4096])
def test_layernorm_unaligned_and_inplace(ctx, cols):
    x, g, b, eps = G.cfg4_layernorm(rows=5, cols=cols)
    ref = O.layernorm(x, cols, g, b, eps).reshape(x.shape)
    got = run(ctx, lambda dx, dg, db, y: ctx.layernorm(dx, dg, db, y, 5, cols, eps), x, g, b,
              out_shape=x.shape, offset=1)
    assert_close(got, ref, "LN unaligned")
    dx = ctx.to_device(x)
    dg, db = ctx.to_device(g), ctx.to_device(b)
    ctx.layernorm(dx, dg, db, dx, 5, cols, eps)  # y aliases x
    assert_close(dx.numpy(), ref, "LN in place")
    for d in (dx, dg, db):
        d.free()


def test_layernorm_errors(ctx):
    d = ctx.to_device(np.ones(8, np.float32))
    with pytest.raises(M.MimirError) as e:
        ctx.layernorm(d, None, None, d, 2, 0, 1e-5)
    assert e.value.status == M.EINVAL
    with pytest.raises(M.MimirError) as e:
        ctx.layernorm(d, None, d, d, 2, 4, 1e-5)  # bias without scale
    assert e.value.status == M.EINVAL
    ctx.layernorm(d, None, None, d, 0, 4, 1e-5)  # zero groups: nothing to do
    d.free()


# ---------------------------------------------------------------------------
# RMSNorm and residual add + RMSNorm
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("cols", [1, 7, 64, 512, 4096, 6000, 16384])
def test_rmsnorm_rows(ctx, cols):
    rows = 11
    x = rng.standard_normal((rows, cols), dtype=np.float32)
    w = (1 + 0.02 * rng.standard_normal(cols)).astype(np.float32)
    got = run(ctx, lambda dx, dw, y: ctx.rmsnorm(dx, dw, cols, y, rows, cols, 1e-6), x, w,
              out_shape=x.shape)
    ref = O.rmsnorm_rows(x, w, 1e-6)
    assert_close_or_nearer_exact(got, ref, X.rmsnorm(x, cols, w, cols, 1e-6), f"RMS cols={cols}")
    if cols <= 4096:
        assert_close(got, ref, f"RMS cols={cols}")


@pytest.mark.parametrize("n,wn", [(2, 2), (4096, 4096), (100000, 17), (1000, 0), (262144, 262144)])
def test_rmsnorm_whole_vector_layer(ctx, n, wn):
    x = rng.standard_normal(n, dtype=np.float32)
    w = (1 + 0.02 * rng.standard_normal(wn)).astype(np.float32) if wn else None
    got = run(ctx, lambda dx, dw, y: ctx.rmsnorm(dx, dw, wn, y, 1, n, 1e-5), x, w, out_shape=(n,))
    assert_close_or_nearer_exact(got, O.rmsnorm_whole(x, w, 1e-5), X.rmsnorm(x, n, w, wn, 1e-5),
                                 f"RMS whole n={n}")


@pytest.mark.parametrize("cols", [4096, 1000, 3])
def test_add_rmsnorm(ctx, cols):
    x, r, w, eps = G.cfg1_add_rmsnorm(rows=64, cols=4096)
    x, r, w = x[:, :cols].copy(), r[:, :cols].copy(), w[:cols].copy()
    y_ref, h_ref = O.add_rmsnorm(x, r, w, eps)
    dx, dr, dw = ctx.to_device(x), ctx.to_device(r), ctx.to_device(w)
    dh, dy = ctx.empty(x.shape), ctx.empty(x.shape)
    ctx.add_rmsnorm(dx, dr, dh, dw, dy, 64, cols, eps)
    assert_bitexact(dh.numpy(), h_ref, "residual out")
    assert_close(dy.numpy(), y_ref, "y")
    ctx.add_rmsnorm(dx, dr, dr, dw, dy, 64, cols, eps)  # in-place residual
    assert_bitexact(dr.numpy(), h_ref, "residual in place")
    assert_close(dy.numpy(), y_ref, "y (in place residual)")
    with pytest.raises(M.MimirError):
        ctx.add_rmsnorm(dx, dr, dh, dw, dh, 64, cols, eps)  # y aliasing residual_out
    for d in (dx, dr, dw, dh, dy):
        d.free()


# ---------------------------------------------------------------------------
# Softmax
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("mode", [M.SOFTMAX_DIV_EPS, M.SOFTMAX_MUL_INV, M.SOFTMAX_LOG])
def test_softmax_cfg2_head(ctx, mode):
    s = G.cfg2_softmax(batch=1, heads=1).reshape(1024, 1024)
    got = run(ctx, lambda dx, y: ctx.softmax(dx, y, 1024, 1024, mode), s, out_shape=s.shape)
    ref = O.softmax_rows(s, mode)
    if mode == M.SOFTMAX_LOG:  # (x - m) - log(sum) cancels: the reference's sum error shows
        assert_close_or_nearer_exact(got, ref, X.softmax(s, mode), f"softmax mode {mode}")
    else:
        assert_close(got, ref, f"softmax mode {mode}")


@pytest.mark.parametrize("cols", [1, 2, 5, 64, 256, 1000, 1024, 2048, 4096, 8192, 16384, 16385,
                                  70000])
@pytest.mark.parametrize("mode", [M.SOFTMAX_DIV_EPS, M.SOFTMAX_LOG])
def test_softmax_shapes(ctx, cols, mode):
    rows = 6
    s = (3 * rng.standard_normal((rows, cols))).astype(np.float32)
    s[0, cols // 2:] = -np.inf
    got = run(ctx, lambda dx, y: ctx.softmax(dx, y, rows, cols, mode), s, out_shape=s.shape)
    ref = O.softmax_rows(s, mode)
    assert_close_or_nearer_exact(got, ref, X.softmax(s, mode), f"softmax cols={cols}")
    if cols <= 4096 and mode != M.SOFTMAX_LOG:
        assert_close(got, ref, f"softmax cols={cols}")


def test_softmax_special_rows(ctx):
    s = np.stack([np.full(8, -np.inf, np.float32),
                  np.array([np.nan, 1, 2, 3, 4, 5, 6, 7], np.float32),
                  np.array([1, np.nan, 2, 3, 4, 5, 6, 7], np.float32),
                  np.array([np.inf, 1, 2, 3, 4, 5, 6, 7], np.float32),
                  np.array([1e30, -1e30, 0, 0, 0, 0, 0, 0], np.float32),
                  np.zeros(8, np.float32)])
    for mode in (M.SOFTMAX_DIV_EPS, M.SOFTMAX_MUL_INV, M.SOFTMAX_LOG):
        got = run(ctx, lambda dx, y: ctx.softmax(dx, y, 6, 8, mode), s, out_shape=s.shape)
        assert_close(got, O.softmax_rows(s, mode), f"special rows mode {mode}")


def test_softmax_inplace_and_unaligned(ctx):
    s = (3 * rng.standard_normal((33, 1024))).astype(np.float32)
    ref = O.softmax_rows(s)
    got = run(ctx, lambda dx, y: ctx.softmax(dx, y, 33, 1024), s, out_shape=s.shape, offset=3)
    assert_close(got, ref, "unaligned")
    d = ctx.to_device(s)
    ctx.softmax(d, d, 33, 1024)
    assert_close(d.numpy(), ref, "in place")
    with pytest.raises(M.MimirError):
        ctx.softmax(d, d, 33, 0)
    with pytest.raises(M.MimirError):
        ctx.softmax(d, d, 33, 1024, 7)
    d.free()


# ---------------------------------------------------------------------------
# Elementwise
# ---------------------------------------------------------------------------

def _grid():
    return np.concatenate([np.linspace(-12, 12, 100003, dtype=np.float32), SPECIALS,
                           rng.standard_normal(65536 * 3 + 5, dtype=np.float32)])


@pytest.mark.parametrize("offset", [0, 1])
def test_gelu_silu(ctx, offset):
    x = _grid()
    for name, fn, ref in (("gelu", ctx.gelu, O.gelu), ("silu", ctx.silu, O.silu)):
        got = run(ctx, lambda dx, y: fn(dx, y, x.size), x, out_shape=x.shape, offset=offset)
        assert_close(got, ref(x), name)


@pytest.mark.parametrize("offset", [0, 2])
def test_gated_products(ctx, offset):
    g = _grid()
    u = rng.standard_normal(g.size, dtype=np.float32) * 2
    u[:SPECIALS.size] = SPECIALS
    for name, fn, ref in (("silu_mul", ctx.silu_mul, O.silu_mul), ("gelu_mul", ctx.gelu_mul, O.gelu_mul)):
        got = run(ctx, lambda dg, du, y: fn(dg, du, y, g.size), g, u, out_shape=g.shape, offset=offset)
        assert_close(got, ref(g, u), name)


@pytest.mark.parametrize("na,nb", [(1, 1), (1000, 1000), (1001, 1001), (4096 * 8, 4096),
                                   (4096, 4096 * 8), (12, 1), (1, 12), (30, 10), (10, 30),
                                   (4096 * 3 + 0, 3)])
def test_add_broadcast_bitexact(ctx, na, nb):
    a = rng.standard_normal(na, dtype=np.float32)
    b = rng.standard_normal(nb, dtype=np.float32)
    got = run(ctx, lambda da, db, y: ctx.add(da, na, db, nb, y), a, b, out_shape=(max(na, nb),))
    assert_bitexact(got, O.add(a, b), f"add {na}+{nb}")


def test_add_mul_specials_bitexact(ctx):
    a = np.tile(SPECIALS, SPECIALS.size)
    b = np.repeat(SPECIALS, SPECIALS.size)
    n = a.size
    for offset in (0, 1):
        got = run(ctx, lambda da, db, y: ctx.add(da, n, db, n, y), a, b, out_shape=(n,), offset=offset)
        assert_bitexact(got, O.add(a, b), "add specials")
        got = run(ctx, lambda da, db, y: ctx.mul(da, n, db, n, y), a, b, out_shape=(n,), offset=offset)
        assert_bitexact(got, O.mul(a, b), "mul specials")


def test_elementwise_errors(ctx):
    d = ctx.to_device(np.ones(12, np.float32))
    for na, nb in ((0, 4), (4, 0), (5, 3)):
        with pytest.raises(M.MimirError) as e:
            ctx.add(d, na, d, nb, d)
        assert e.value.status == M.EINVAL
    with pytest.raises(M.MimirError):
        ctx.mul(d, 4, d, 3, d)
    d.free()


# ---------------------------------------------------------------------------
# Embedding gather (bit-exact)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dim", [4096, 1, 3, 64, 100, 256, 1024, 2052, 8192])
@pytest.mark.parametrize("pad", [-1, 0, 5])
def test_embedding_int_ids(ctx, dim, pad):
    vocab = 300
    table = G.normal(3, 0, (vocab, dim), 0.02)
    ids = rng.integers(-20, vocab + 20, size=1000, dtype=np.int32)
    ids[:8] = [0, 5, -1, vocab, vocab - 1, 2**31 - 1, -2**31, 5]
    got = run(ctx, lambda di, dt, y: ctx.embedding(di, ids.size, dt, table.size, vocab, dim, pad, y),
              ids, table, out_shape=(ids.size, dim))
    assert_bitexact(got, O.embedding(ids, table, vocab, dim, pad), f"gather dim={dim} pad={pad}")


def test_embedding_float_ids(ctx):
    vocab, dim = 1000, 128
    table = G.normal(3, 0, (vocab, dim), 0.02)
    special = np.array([1.0, 1.5, 2.5, -0.5, -1.5, 0.49999997, 999.5, 998.5, np.nan, np.inf,
                        -np.inf, 4294967808.0, -4294966784.0, 1e20, -1e20, 9.3e18, 2**31, -2**31,
                        3.0e9, 7.0], np.float32)
    ids = np.concatenate([special, rng.uniform(-10, vocab + 10, 5000).astype(np.float32)])
    for pad in (-1, 7):
        got = run(ctx, lambda di, dt, y: ctx.embedding(di, ids.size, dt, table.size, vocab, dim, pad, y,
                                                       float_ids=True),
                  ids, table, out_shape=(ids.size, dim))
        assert_bitexact(got, O.embedding(ids, table, vocab, dim, pad), f"float ids pad={pad}")


def test_embedding_payload_bits_unchanged(ctx):
    # NaN payloads, -0 and denormals must be copied as raw words.
    words = np.array([0x7fc00001, 0xffc12345, 0x80000000, 0x00000001, 0x807fffff, 0x7f800000,
                      0x3f800000, 0x7fa00000], np.uint32)
    table = np.tile(words, 64).view(np.float32).reshape(16, 32)
    ids = np.arange(16, dtype=np.int32)[::-1].copy()
    got = run(ctx, lambda di, dt, y: ctx.embedding(di, 16, dt, table.size, 16, 32, -1, y), ids, table,
              out_shape=(16, 32))
    assert_bitexact(got, table[ids], "payload bits")


def test_embedding_errors_and_clamps(ctx):
    t = ctx.to_device(np.ones(6, np.float32))
    i = ctx.to_device(np.zeros(2, np.int32))
    y = ctx.empty(16)
    with pytest.raises(M.MimirError) as e:
        ctx.embedding(i, 2, t, 6, 4, 2, -1, y)  # 6 < 4*2
    assert e.value.status == M.EINVAL
    ctx.embedding(i, 2, t, 6, 0, 0, -1, y)  # vocab, dim clamp to 1: rows of table[0]
    np.testing.assert_array_equal(y.numpy()[:2], [1.0, 1.0])
    for d in (t, i, y):
        d.free()


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("B,S,H,Hk,D", [(2, 64, 4, 4, 128), (1, 33, 3, 1, 64), (2, 17, 2, 5, 8),
                                        (1, 9, 2, 2, 96), (1, 5, 3, 2, 6), (1, 40, 2, 2, 512)])
def test_rope_qk(ctx, B, S, H, Hk, D):
    pos_offset = 3
    rows = S + pos_offset + 2
    cos_t, sin_t = M.rope_table(rows, D)
    q = rng.standard_normal((B, S, H, D), dtype=np.float32)
    k = rng.standard_normal((B, S, Hk, D), dtype=np.float32)
    dq, dk = ctx.to_device(q), ctx.to_device(k)
    dqo, dko = ctx.empty(q.shape), ctx.empty(k.shape)
    dc, ds = ctx.to_device(cos_t), ctx.to_device(sin_t)
    ctx.rope(dq, dqo, H, dk, dko, Hk, B, S, D, pos_offset, dc, ds, rows)
    assert_close(dqo.numpy(), O.rope(q, cos_t, sin_t, pos_offset), "q")
    assert_close(dko.numpy(), O.rope(k, cos_t, sin_t, pos_offset), "k")
    ctx.rope(dq, dq, H, dk, dk, Hk, B, S, D, pos_offset, dc, ds, rows)  # in place
    assert_close(dq.numpy(), O.rope(q, cos_t, sin_t, pos_offset), "q in place")
    assert_close(dk.numpy(), O.rope(k, cos_t, sin_t, pos_offset), "k in place")
    ctx.rope(dq, dqo, H, None, None, 0, B, S, D, 0, dc, ds, rows)  # q only
    with pytest.raises(M.MimirError):
        ctx.rope(dq, dqo, H, dk, dko, Hk, B, S, D, rows - S + 1, dc, ds, rows)  # past the table
    with pytest.raises(M.MimirError):
        ctx.rope(dq, dqo, H, dk, dko, Hk, B, S, D + 1, 0, dc, ds, rows)  # odd head_dim
    for d in (dq, dk, dqo, dko, dc, ds):
        d.free()


@pytest.mark.parametrize("ppt", [1, 2, 4])
def test_rope_slots_per_thread(ppt):
    """Each slots-per-thread form of the vector kernel (MIMIR_TUNE rope=n; 4
    is the default), on a tail that leaves part of the last workgroup's
    slots empty: q and k match the oracle, the same bits in every form."""
    import os
    old = os.environ.get("MIMIR_TUNE")
    os.environ["MIMIR_TUNE"] = f"rope={ppt}"
    try:
        c = M.Context(0)
    finally:
        if old is None:
            del os.environ["MIMIR_TUNE"]
        else:
            os.environ["MIMIR_TUNE"] = old
    B, S, H, Hk, D = 3, 37, 5, 3, 64
    r = np.random.default_rng(40 + ppt)
    cos_t, sin_t = M.rope_table(S + 1, D)
    q = r.standard_normal((B, S, H, D), dtype=np.float32)
    k = r.standard_normal((B, S, Hk, D), dtype=np.float32)
    try:
        dq, dk, dc, ds = c.to_device(q), c.to_device(k), c.to_device(cos_t), c.to_device(sin_t)
        c.rope(dq, dq, H, dk, dk, Hk, B, S, D, 1, dc, ds, S + 1)
        assert_close(dq.numpy(), O.rope(q, cos_t, sin_t, 1), f"q rope={ppt}")
        assert_close(dk.numpy(), O.rope(k, cos_t, sin_t, 1), f"k rope={ppt}")
        for d in (dq, dk, dc, ds):
            d.free()
    finally:
        c.close()


# ---------------------------------------------------------------------------
# Long rows split over many workgroups (longrow.hip)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("cpw", [1, 2, 4])
def test_longrow_chunks_per_workgroup(ctx, cpw):
    """The long rows' first pass with 1, 2 or 4 chunks per workgroup
    (MIMIR_TUNE lrcpw; two for LayerNorm and one for the others by default)
    computes each chunk's partial the same way: LayerNorm and softmax over
    rows with a partial last chunk and a chunk count that is not a multiple
    of the chunks per workgroup give the default's bits."""
    import os
    old = os.environ.get("MIMIR_TUNE")
    os.environ["MIMIR_TUNE"] = f"lrcpw={cpw}"
    try:
        c = M.Context(0)
    finally:
        if old is None:
            del os.environ["MIMIR_TUNE"]
        else:
            os.environ["MIMIR_TUNE"] = old
    try:
        rows, cols = 3, 4096 * 7 + 20  # 8 chunks, the last partial
        x = (rng.standard_normal((rows, cols), dtype=np.float32) * 1.3 + 0.2)
        g = (1 + 0.05 * rng.standard_normal(cols)).astype(np.float32)
        b = (0.05 * rng.standard_normal(cols)).astype(np.float32)
        for name, f in (("layernorm", lambda cc: (lambda dx, dg, db, y: cc.layernorm(dx, dg, db, y, rows, cols, 1e-5))),
                        ("softmax", lambda cc: (lambda dx, dg, db, y: cc.softmax(dx, y, rows, cols)))):
            got = run(c, f(c), x, g, b, out_shape=x.shape)
            want = run(ctx, f(ctx), x, g, b, out_shape=x.shape)
            assert_bitexact(got, want, f"{name} lrcpw={cpw}")
    finally:
        c.close()


@pytest.mark.parametrize("bs", [256, 512])
def test_longrow_first_pass_threads_per_chunk(ctx, bs):
    """The long rows' first pass with 256 or 512 threads per 4096-float chunk
    (MIMIR_TUNE lrpart; 512 for the LayerNorm statistic by default, 256 for
    the others) sums each chunk in a different order: LayerNorm, RMSNorm and
    softmax over rows with a partial last chunk stay within the oracle's
    tolerance (or nearer the exact value) either way."""
    import os
    old = os.environ.get("MIMIR_TUNE")
    os.environ["MIMIR_TUNE"] = f"lrpart={bs}"
    try:
        c = M.Context(0)
    finally:
        if old is None:
            del os.environ["MIMIR_TUNE"]
        else:
            os.environ["MIMIR_TUNE"] = old
    try:
        rows, cols = 3, 4096 * 7 + 20
        x = (rng.standard_normal((rows, cols), dtype=np.float32) * 1.3 + 0.2)
        g = (1 + 0.05 * rng.standard_normal(cols)).astype(np.float32)
        b = (0.05 * rng.standard_normal(cols)).astype(np.float32)
        got = run(c, lambda dx, dg, db, y: c.layernorm(dx, dg, db, y, rows, cols, 1e-5), x, g, b, out_shape=x.shape)
        assert_close_or_nearer_exact(got, O.layernorm(x, cols, g, b, 1e-5).reshape(x.shape),
                                     X.layernorm(x, cols, g, b, 1e-5), f"long LN lrpart={bs}")
        got = run(c, lambda dx, dw, y: c.rmsnorm(dx, dw, cols, y, rows, cols, 1e-6), x, g, out_shape=x.shape)
        assert_close_or_nearer_exact(got, O.rmsnorm_rows(x, g, 1e-6), X.rmsnorm(x, cols, g, cols, 1e-6),
                                     f"long RMSNorm lrpart={bs}")
        got = run(c, lambda dx, y: c.softmax(dx, y, rows, cols), x, out_shape=x.shape)
        assert_close_or_nearer_exact(got, O.softmax_rows(x, M.SOFTMAX_DIV_EPS), X.softmax(x, M.SOFTMAX_DIV_EPS),
                                     f"long softmax lrpart={bs}")
    finally:
        c.close()


@pytest.mark.parametrize("rows,cols", [(3, 4096 * 7 + 20), (1, 4096 * 64 * 3 + 4), (2, 70000)])
def test_longrow_apply_shapes_agree(ctx, rows, cols):
    """The apply pass in its default shape (128 threads x 2 float4) and in the
    chunk shape (MIMIR_TUNE lrapply=256x4) reads the same row statistics and
    applies the same per-element formula: LayerNorm, RMSNorm, add+RMSNorm
    and softmax, over rows whose last chunk is partial, give the same bits."""
    import os
    old = os.environ.get("MIMIR_TUNE")
    os.environ["MIMIR_TUNE"] = "lrapply=256x4"
    try:
        c = M.Context(0)
    finally:
        if old is None:
            del os.environ["MIMIR_TUNE"]
        else:
            os.environ["MIMIR_TUNE"] = old
    try:
        x = (rng.standard_normal((rows, cols), dtype=np.float32) * 1.3 + 0.2)
        r = rng.standard_normal((rows, cols), dtype=np.float32)
        g = (1 + 0.05 * rng.standard_normal(cols)).astype(np.float32)
        b = (0.05 * rng.standard_normal(cols)).astype(np.float32)
        ops = (("layernorm", lambda cc: (lambda dx, dr, dg, db, y: cc.layernorm(dx, dg, db, y, rows, cols, 1e-5))),
               ("rmsnorm", lambda cc: (lambda dx, dr, dg, db, y: cc.rmsnorm(dx, dg, cols, y, rows, cols, 1e-6))),
               ("softmax", lambda cc: (lambda dx, dr, dg, db, y: cc.softmax(dx, y, rows, cols))))
        for name, f in ops:
            got = run(c, f(c), x, r, g, b, out_shape=x.shape)
            want = run(ctx, f(ctx), x, r, g, b, out_shape=x.shape)
            assert_bitexact(got, want, f"{name} lrapply=256x4")
        outs = []
        for cc in (c, ctx):
            dx, dr, dg = cc.to_device(x), cc.to_device(r), cc.to_device(g)
            dy, dro = cc.empty(x.shape), cc.empty(x.shape)
            cc.add_rmsnorm(dx, dr, dro, dg, dy, rows, cols, 1e-6)
            outs.append((dy.numpy(), dro.numpy()))
            for d in (dx, dr, dg, dy, dro):
                d.free()
        assert_bitexact(outs[0][0], outs[1][0], "add+RMSNorm y lrapply=256x4")
        assert_bitexact(outs[0][1], outs[1][1], "add+RMSNorm residual lrapply=256x4")
    finally:
        c.close()


@pytest.mark.parametrize("rows,cols", [(1, 1 << 20), (3, 65536), (2, 20004), (1, 4097 * 4), (2, 20001),
                                       (300, 20004)])
def test_longrow_layernorm_rmsnorm(ctx, rows, cols):
    x = (rng.standard_normal((rows, cols), dtype=np.float32) * 1.3 + 0.2)
    g = (1 + 0.05 * rng.standard_normal(cols)).astype(np.float32)
    b = (0.05 * rng.standard_normal(cols)).astype(np.float32)
    got = run(ctx, lambda dx, dg, db, y: ctx.layernorm(dx, dg, db, y, rows, cols, 1e-5), x, g, b,
              out_shape=x.shape)
    assert_close_or_nearer_exact(got, O.layernorm(x, cols, g, b, 1e-5).reshape(x.shape),
                                 X.layernorm(x, cols, g, b, 1e-5), "long LN")
    wl = cols // 3  # the whole-vector layer: weights shorter than the row
    got = run(ctx, lambda dx, dw, y: ctx.rmsnorm(dx, dw, wl, y, rows, cols, 1e-6), x, g, out_shape=x.shape)
    ref = np.concatenate([O.rmsnorm_whole(x[i], g[:wl], 1e-6) for i in range(rows)]).reshape(x.shape)
    assert_close_or_nearer_exact(got, ref, X.rmsnorm(x, cols, g, wl, 1e-6), "long RMSNorm")


def test_longrow_layernorm_offset_rows(ctx):
    """Rows whose mean dwarfs their spread, and chunks of different means:
    the per-chunk deviations and their float64 merge must still give the
    two-pass variance."""
    rows, cols = 3, 5 * 4096 * 4 + 4096
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    x[0] = 1000.0 + 0.5 * x[0]
    x[1, : cols // 2] += 40.0  # two halves with different means
    x[2] = np.float32(3.25)  # constant row: variance 0, y = beta
    g = (1 + 0.05 * rng.standard_normal(cols)).astype(np.float32)
    b = (0.05 * rng.standard_normal(cols)).astype(np.float32)
    got = run(ctx, lambda dx, dg, db, y: ctx.layernorm(dx, dg, db, y, rows, cols, 1e-5), x, g, b,
              out_shape=x.shape)
    assert_close_or_nearer_exact(got, O.layernorm(x, cols, g, b, 1e-5).reshape(x.shape),
                                 X.layernorm(x, cols, g, b, 1e-5), "long LN, offset rows")
    assert_bitexact(got[2], b, "constant row")


def test_longrow_add_rmsnorm_inplace(ctx):
    rows, cols = 2, 3 * 4096 * 4 + 8
    x = rng.standard_normal((rows, cols), dtype=np.float32)
    r = rng.standard_normal((rows, cols), dtype=np.float32)
    w = (1 + 0.02 * rng.standard_normal(cols)).astype(np.float32)
    y_ref, h_ref = O.add_rmsnorm(x, r, w, 1e-6)
    dx, dr, dw, dy = ctx.to_device(x), ctx.to_device(r), ctx.to_device(w), ctx.empty(x.shape)
    ctx.add_rmsnorm(dx, dr, dr, dw, dy, rows, cols, 1e-6)
    assert_bitexact(dr.numpy(), h_ref, "residual")
    assert_close_or_nearer_exact(dy.numpy(), y_ref, X.rmsnorm(h_ref, cols, w, cols, 1e-6), "y")
    for d in (dx, dr, dw, dy):
        d.free()


@pytest.mark.parametrize("mode", [M.SOFTMAX_DIV_EPS, M.SOFTMAX_MUL_INV, M.SOFTMAX_LOG])
def test_longrow_softmax_with_masked_chunks(ctx, mode):
    rows, cols = 4, 9 * 4096
    s = (3 * rng.standard_normal((rows, cols))).astype(np.float32)
    s[0, 4096:3 * 4096] = -np.inf          # whole chunks masked
    s[1, :] = -np.inf                        # an all -inf row -> NaN, as the reference
    s[1, 5] = -np.inf
    s[2, 12345] = np.nan                     # NaN -> the row is NaN
    got = run(ctx, lambda dx, y: ctx.softmax(dx, y, rows, cols, mode), s, out_shape=s.shape)
    assert_close_or_nearer_exact(got, O.softmax_rows(s, mode), X.softmax(s, mode), f"long softmax {mode}")
    assert np.isnan(got[1]).all() and np.isnan(got[2]).all()


@pytest.mark.parametrize("mode", [M.SOFTMAX_DIV_EPS, M.SOFTMAX_LOG])
def test_longrow_softmax_many_rows(ctx, mode):
    """Many wide rows (a vocabulary-sized log-softmax): chunks x rows."""
    rows, cols = 300, 20004
    s = (3 * rng.standard_normal((rows, cols))).astype(np.float32)
    got = run(ctx, lambda dx, y: ctx.softmax(dx, y, rows, cols, mode), s, out_shape=s.shape)
    assert_close_or_nearer_exact(got, O.softmax_rows(s, mode), X.softmax(s, mode), f"wide softmax {mode}")


def test_longrow_softmax_layer_whole_vector(ctx):
    x = (3 * rng.standard_normal(1 << 21)).astype(np.float32)
    got = run(ctx, lambda dx, y: ctx.softmax(dx, y, 1, x.size, M.SOFTMAX_MUL_INV), x, out_shape=x.shape)
    ref = O.softmax_rows(x, M.SOFTMAX_MUL_INV)[0]
    assert_close_or_nearer_exact(got, ref, X.softmax(x, 1)[0], "whole-vector softmax")
    assert abs(got.sum(dtype=np.float64) - 1.0) < 1e-5


def _long_ops(c, rows, cols, wl):
    """The long-row forward ops as (name, launch closure, oracle, float64 value)."""
    return (
        ("layernorm", lambda dx, dg, db, y: c.layernorm(dx, dg, db, y, rows, cols, 1e-5),
         lambda x, g, b: O.layernorm(x, cols, g, b, 1e-5).reshape(x.shape),
         lambda x, g, b: X.layernorm(x, cols, g, b, 1e-5)),
        ("rmsnorm", lambda dx, dg, db, y: c.rmsnorm(dx, dg, wl, y, rows, cols, 1e-6),
         lambda x, g, b: np.stack([O.rmsnorm_whole(x[i], g[:wl], 1e-6) for i in range(rows)]).reshape(x.shape),
         lambda x, g, b: X.rmsnorm(x, cols, g, wl, 1e-6)),
        ("softmax", lambda dx, dg, db, y: c.softmax(dx, y, rows, cols, M.SOFTMAX_MUL_INV),
         lambda x, g, b: O.softmax_rows(x, M.SOFTMAX_MUL_INV),
         lambda x, g, b: X.softmax(x, M.SOFTMAX_MUL_INV)),
    )


def test_longrow_repeat_launches_give_the_same_bits(ctx):
    """The combine folds the chunk partials in a fixed order, whatever order
    the first pass's workgroups ran in: repeated launches give the same
    bits, with calls of other shapes in between (1025 chunks with a short
    last one, 18 chunks over 5 rows, 65 and 193 chunks), each within the
    path's tolerance of the oracle."""
    shapes = [(1, 4096 * 1024 + 12),
              (5, 70000),
              (2, 4096 * 65),
              (1, 4096 * 64 * 3 + 4)]
    first = {}
    for rep in range(3):
        for rows, cols in shapes:
            x = (np.random.default_rng(rows * 7 + cols).standard_normal((rows, cols), dtype=np.float32) * 1.7
                 + 0.3)
            g = (1 + 0.05 * np.random.default_rng(cols).standard_normal(cols)).astype(np.float32)
            b = (0.05 * np.random.default_rng(cols + 1).standard_normal(cols)).astype(np.float32)
            for name, f, ref, exact in _long_ops(ctx, rows, cols, cols // 2):
                got = run(ctx, f, x, g, b, out_shape=x.shape)
                key = (rows, cols, name)
                if rep == 0:
                    first[key] = got
                    assert_close_or_nearer_exact(got, ref(x, g, b), exact(x, g, b), f"{name} {rows}x{cols}")
                else:
                    assert_bitexact(got, first[key], f"{name} {rows}x{cols} launch {rep}")


# ---------------------------------------------------------------------------
# Output store policy (mimir_ctx_set_output_caching): same bits either way
# ---------------------------------------------------------------------------

def test_output_caching_gives_the_same_bits(ctx):
    """Every op's output with outputs kept in the caches equals the streamed
    result bit for bit (only the store instruction differs)."""
    rows, cols = 64, 4096
    x = rng.standard_normal((rows, cols), dtype=np.float32)
    r = rng.standard_normal((rows, cols), dtype=np.float32)
    g = (1 + 0.05 * rng.standard_normal(cols)).astype(np.float32)
    b = (0.05 * rng.standard_normal(cols)).astype(np.float32)
    long_x = rng.standard_normal(1 << 17, dtype=np.float32)
    table = rng.standard_normal((100, 256), dtype=np.float32)
    ids = rng.integers(-2, 102, 300).astype(np.int32)
    q = rng.standard_normal((2, 16, 4, 64), dtype=np.float32)
    cos_t, sin_t = M.rope_table(16, 64)
    dev = {k: ctx.to_device(v) for k, v in dict(x=x, r=r, g=g, b=b, long_x=long_x, table=table, ids=ids, q=q,
                                                 c=cos_t, s=sin_t).items()}
    outs = {}

    def run_all(tag):
        res = {}
        y = ctx.empty(x.shape)
        h = ctx.empty(x.shape)
        yl = ctx.empty(long_x.shape)
        ye = ctx.empty((ids.size, 256))
        qo = ctx.empty(q.shape)
        try:
            ctx.layernorm(dev["x"], dev["g"], dev["b"], y, rows, cols, 1e-5); res["ln"] = y.numpy()
            ctx.rmsnorm(dev["x"], dev["g"], cols, y, rows, cols, 1e-6); res["rms"] = y.numpy()
            ctx.add_rmsnorm(dev["x"], dev["r"], h, dev["g"], y, rows, cols, 1e-6)
            res["addrms_y"], res["addrms_h"] = y.numpy(), h.numpy()
            ctx.softmax(dev["x"], y, rows, cols); res["softmax"] = y.numpy()
            ctx.gelu(dev["x"], y, x.size); res["gelu"] = y.numpy()
            ctx.silu_mul(dev["x"], dev["r"], y, x.size); res["silu_mul"] = y.numpy()
            ctx.add(dev["x"], x.size, dev["r"], r.size, y); res["add"] = y.numpy()
            ctx.add(dev["x"], x.size, dev["g"], cols, y); res["add_repeat"] = y.numpy()
            ctx.layernorm(dev["long_x"], None, None, yl, 1, long_x.size, 1e-5); res["ln_long"] = yl.numpy()
            ctx.softmax(dev["long_x"], yl, 1, long_x.size); res["softmax_long"] = yl.numpy()
            ctx.embedding(dev["ids"], ids.size, dev["table"], table.size, 100, 256, -1, ye); res["gather"] = ye.numpy()
            ctx.rope(dev["q"], qo, 4, None, None, 0, 2, 16, 64, 0, dev["c"], dev["s"], 16); res["rope"] = qo.numpy()
        finally:
            for a in (y, h, yl, ye, qo):
                a.free()
        outs[tag] = res

    try:
        run_all("streamed")
        ctx.set_output_caching(True)
        run_all("kept")
    finally:
        ctx.set_output_caching(False)
        for a in dev.values():
            a.free()
    for k, v in outs["streamed"].items():
        assert_bitexact(outs["kept"][k], v, f"{k}: kept vs streamed")


@pytest.mark.parametrize("cols", [1023, 2047, 4095])
def test_odd_widths_register_resident(ctx, cols):
    """Widths that are not a multiple of 4 (rows start off 16-byte alignment)
    take the 4-byte-column kernels (norm_rows_scalar, softmax_rows_scalar):
    LayerNorm, RMSNorm with a weight block shorter than the row, add + RMSNorm
    with the residual updated in place (bit-exact), and softmax
    with a masked column, an all -inf row (NaN, as the reference) and a NaN
    row: within tolerance of the oracle or nearer the float64 value, since
    the reference's sequential float sums over ~4000 terms carry ~1e-6 of
    error into outputs near zero (LayerNorm's mean, LogSoftmax's log(sum))."""
    rows = 9
    x = (0.7 + 1.3 * rng.standard_normal((rows, cols))).astype(np.float32)
    g = (1 + 0.05 * rng.standard_normal(cols)).astype(np.float32)
    b = (0.05 * rng.standard_normal(cols)).astype(np.float32)
    got = run(ctx, lambda dx, dg, db, y: ctx.layernorm(dx, dg, db, y, rows, cols, 1e-5), x, g, b, out_shape=x.shape)
    assert_close_or_nearer_exact(got, O.layernorm(x, cols, g, b, 1e-5).reshape(x.shape),
                                 X.layernorm(x, cols, g, b, 1e-5), f"LN cols={cols}")
    wl = cols // 2
    got = run(ctx, lambda dx, dw, y: ctx.rmsnorm(dx, dw, wl, y, rows, cols, 1e-6), x, g, out_shape=x.shape)
    ref = np.stack([O.rmsnorm_whole(x[i], g[:wl], 1e-6) for i in range(rows)])
    assert_close_or_nearer_exact(got, ref, X.rmsnorm(x, cols, g, wl, 1e-6), f"RMSNorm cols={cols}")
    r = rng.standard_normal((rows, cols)).astype(np.float32)
    y_ref, h_ref = O.add_rmsnorm(x, r, g, 1e-6)
    dx, dr, dw, dy = ctx.to_device(x), ctx.to_device(r), ctx.to_device(g), ctx.empty((rows, cols))
    try:
        ctx.add_rmsnorm(dx, dr, dr, dw, dy, rows, cols, 1e-6)  # residual updated in place
        assert_bitexact(dr.numpy(), h_ref.reshape(rows, cols), f"add+RMSNorm residual cols={cols}")
        assert_close_or_nearer_exact(dy.numpy(), y_ref.reshape(rows, cols),
                                     X.rmsnorm(h_ref.reshape(rows, cols), cols, g, cols, 1e-6),
                                     f"add+RMSNorm cols={cols}")
    finally:
        for d in (dx, dr, dw, dy):
            d.free()
    s = (3 * x).astype(np.float32)
    s[1, 5] = -np.inf
    s[2, :] = -np.inf
    s[3, cols // 2] = np.nan
    for mode in (M.SOFTMAX_DIV_EPS, M.SOFTMAX_MUL_INV, M.SOFTMAX_LOG):
        got = run(ctx, lambda dx, y: ctx.softmax(dx, y, rows, cols, mode), s, out_shape=s.shape)
        assert_close_or_nearer_exact(got, O.softmax_rows(s, mode), X.softmax(s, mode), f"softmax cols={cols} mode {mode}")
