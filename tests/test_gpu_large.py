"""Tensors of more than 2^31 elements (8 GiB of fp32 each), forward and
backward: every index on the path is 64-bit.  The inputs are filled on the device (constants, with a
few rows uploaded where values must differ), and the results are checked at
the head, around element 2^31 and at the tail, against the oracle where a
row is not constant.  Peak device memory: 24 GiB of the MI355X's 288."""
import numpy as np
import pytest

import oracle as O
from _parity import assert_bitexact, assert_close

pytestmark = pytest.mark.gpu

BIG = (1 << 31) + 4096  # elements: past the int32 range by one 4096-wide row


def _slice(ctx, buf, start, n):
    out = np.empty(n, np.float32)
    ctx.download(out, buf.offset(start, (n,)))
    return out


def test_add_past_2_31(ctx):
    a, b, y = ctx.empty(BIG), ctx.empty(BIG), ctx.empty(BIG)
    try:
        ctx.fill(a, 1.5)
        ctx.fill(b, 2.25)
        ctx.add(a, BIG, b, BIG, y)
        for start in (0, (1 << 31) - 2048, BIG - 4096):
            assert_bitexact(_slice(ctx, y, start, 4096), np.full(4096, 3.75, np.float32), f"add at {start}")
    finally:
        for d in (a, b, y):
            d.free()


def test_layernorm_rows_past_2_31(ctx):
    cols = 4096
    rows = BIG // cols  # 2^19 + 1 rows
    x, y = ctx.empty((rows, cols)), ctx.empty((rows, cols))
    rng = np.random.default_rng(31)
    g = (1 + 0.05 * rng.standard_normal(cols)).astype(np.float32)
    b = (0.05 * rng.standard_normal(cols)).astype(np.float32)
    tail = rng.standard_normal((2, cols)).astype(np.float32)  # the last two rows differ
    dg, db = ctx.to_device(g), ctx.to_device(b)
    try:
        ctx.fill(x, 0.75)
        ctx.upload(x.offset((rows - 2) * cols, (2, cols)), tail)
        ctx.layernorm(x, dg, db, y, rows, cols, 1e-5)
        assert_bitexact(_slice(ctx, y, 0, cols), b, "constant row 0 -> beta")
        assert_bitexact(_slice(ctx, y, (rows - 3) * cols, cols), b, "constant row before the tail -> beta")
        got = _slice(ctx, y, (rows - 2) * cols, 2 * cols).reshape(2, cols)
        assert_close(got, O.layernorm(tail, cols, g, b, 1e-5).reshape(2, cols), "last rows (past 2^31)")
    finally:
        for d in (x, y, dg, db):
            d.free()


def test_gather_output_past_2_31(ctx):
    vocab, dim = 1000, 4096
    n = BIG // dim  # output [n x 4096] past 2^31 elements
    rng = np.random.default_rng(32)
    table = rng.standard_normal((vocab, dim)).astype(np.float32)
    ids = rng.integers(-1, vocab + 1, n).astype(np.int32)
    dt, di, y = ctx.to_device(table), ctx.to_device(ids), ctx.empty((n, dim))
    try:
        ctx.embedding(di, n, dt, table.size, vocab, dim, -1, y)
        for t in (0, n // 2, n - 2, n - 1):
            want = table[ids[t]] if 0 <= ids[t] < vocab else np.zeros(dim, np.float32)
            assert_bitexact(_slice(ctx, y, t * dim, dim), want, f"token {t}")
    finally:
        for d in (dt, di, y):
            d.free()


def test_softmax_rows_past_2_31(ctx):
    cols = 1024
    rows = BIG // cols
    x, y = ctx.empty((rows, cols)), ctx.empty((rows, cols))
    tail = (3 * np.random.default_rng(33).standard_normal((1, cols))).astype(np.float32)
    try:
        ctx.fill(x, -2.0)
        ctx.upload(x.offset((rows - 1) * cols, (1, cols)), tail)
        ctx.softmax(x, y, rows, cols)
        flat = O.softmax_rows(np.full((1, cols), -2.0, np.float32))[0]
        assert_close(_slice(ctx, y, 0, cols), flat, "constant row 0")
        assert_close(_slice(ctx, y, (rows - 1) * cols, cols), O.softmax_rows(tail)[0], "last row (past 2^31)")
    finally:
        for d in (x, y):
            d.free()


def test_gelu_bwd_past_2_31(ctx):
    x, dy, dx = ctx.empty(BIG), ctx.empty(BIG), ctx.empty(BIG)
    try:
        ctx.fill(x, 0.75)
        ctx.fill(dy, 2.0)
        tail = np.random.default_rng(34).standard_normal(4096).astype(np.float32)
        ctx.upload(x.offset(BIG - 4096, (4096,)), tail)
        ctx.gelu_bwd(x, dy, dx, BIG)
        one = O.gelu_bwd(np.full(4096, 0.75, np.float32), np.full(4096, 2.0, np.float32))
        for start in (0, (1 << 31) - 4096):  # the random tail starts at element 2^31
            assert_close(_slice(ctx, dx, start, 4096), one, f"gelu_bwd at {start}")
        assert_close(_slice(ctx, dx, BIG - 4096, 4096), O.gelu_bwd(tail, np.full(4096, 2.0, np.float32)),
                     "gelu_bwd tail (past 2^31)")
    finally:
        for d in (x, dy, dx):
            d.free()


def test_add_bwd_past_2_31(ctx):
    dy, da, db = ctx.empty(BIG), ctx.empty(BIG), ctx.empty(BIG)
    try:
        ctx.fill(dy, 1.25)
        ctx.add_bwd(dy, BIG, BIG, da, db)
        want = np.full(4096, 1.25, np.float32)
        for start in (0, (1 << 31) - 2048, BIG - 4096):
            assert_bitexact(_slice(ctx, da, start, 4096), want, f"da at {start}")
            assert_bitexact(_slice(ctx, db, start, 4096), want, f"db at {start}")
    finally:
        for d in (dy, da, db):
            d.free()


def test_layernorm_bwd_rows_past_2_31(ctx):
    """Constant rows of x with a constant dy (x - mean = 0: those rows add
    nothing to dgamma, and 0.5 each to dbeta), then two random rows at the
    end, past element 2^31.  dx of a constant row and of the last rows, and
    dgamma / dbeta, are held to the oracle.  eps = 1 keeps 1/sqrt(var + eps)
    of the constant rows at 1, so their dx is not an amplified rounding
    difference."""
    cols = 4096
    rows = BIG // cols  # 2^19 + 1 rows
    x, dy, dx = ctx.empty((rows, cols)), ctx.empty((rows, cols)), ctx.empty((rows, cols))
    rng = np.random.default_rng(35)
    g = (1 + 0.05 * rng.standard_normal(cols)).astype(np.float32)
    xt = rng.standard_normal((2, cols)).astype(np.float32)
    dyt = rng.standard_normal((2, cols)).astype(np.float32)
    dg_, dgam, dbet = ctx.to_device(g), ctx.to_device(np.zeros(cols, np.float32)), ctx.to_device(
        np.zeros(cols, np.float32))
    try:
        ctx.fill(x, 0.75)
        ctx.fill(dy, 0.5)
        ctx.upload(x.offset((rows - 2) * cols, (2, cols)), xt)
        ctx.upload(dy.offset((rows - 2) * cols, (2, cols)), dyt)
        ctx.layernorm_bwd(x, dy, dg_, dx, dgam, dbet, rows, cols, 1.0)
        const_dx, _ = O.layernorm_bwd(np.full(cols, 0.75, np.float32), np.full(cols, 0.5, np.float32), cols, g,
                                      has_bias=True, eps=1.0)
        assert_close(_slice(ctx, dx, 0, cols), const_dx, "dx of constant row 0")
        assert_close(_slice(ctx, dx, (rows - 3) * cols, cols), const_dx, "dx of the constant row before the tail")
        want_dx, gp = O.layernorm_bwd(xt, dyt, cols, g, has_bias=True, eps=1.0)
        got = _slice(ctx, dx, (rows - 2) * cols, 2 * cols)
        assert_close(got, want_dx.ravel(), "dx of the last rows (past 2^31)")
        # dgamma: only the tail rows contribute; dbeta: (rows - 2) * 0.5 + the tail's dy
        assert_close(dgam.numpy(), gp[:cols], "dgamma")
        want_db = np.float64(rows - 2) * 0.5 + dyt.astype(np.float64).sum(0)
        assert_close(dbet.numpy(), want_db.astype(np.float32), "dbeta")
    finally:
        for d in (x, dy, dx, dg_, dgam, dbet):
            d.free()


def test_attention_past_2_31(ctx):
    """The attention core, forward and backward, on a fused QKV buffer of
    more than 2^31 floats (172 sequences x 1024 tokens x 32 heads of 128,
    causal): the last sequence lies wholly past element 2^31 of the QKV and
    dQKV buffers and is held to float64 (two heads forward, one backward);
    the first, constant sequence to its closed form (every probability
    row averages one value of V)."""
    from _attention import assert_attention_close, assert_bwd_close, attention64, attention_bwd64
    b, seq, heads, hd = 172, 1024, 32, 128
    w = heads * hd
    rows = b * seq
    assert (rows - seq) * 3 * w > 1 << 31
    r = np.random.default_rng(41)
    last = (0.5 * r.standard_normal((seq, 3 * w))).astype(np.float32)
    last_dout = r.standard_normal((seq, w)).astype(np.float32)
    qkv, out = ctx.empty((rows, 3 * w)), ctx.empty((rows, w))
    dout, g = ctx.empty((rows, w)), ctx.empty((rows, 3 * w))
    try:
        ctx.fill(qkv, 0.25)
        ctx.upload(qkv.offset((rows - seq) * 3 * w, (seq, 3 * w)), last)
        print("attention forward past 2^31", flush=True)
        ctx.attention(qkv, qkv.offset(w), qkv.offset(2 * w), out, b, seq, seq, heads, hd, True, ld_q=3 * w,
                      ld_kv=3 * w)
        assert_close(_slice(ctx, out, 0, seq * w), np.full(seq * w, 0.25, np.float32), "constant first sequence")
        got = _slice(ctx, out, (rows - seq) * w, seq * w).reshape(seq, w)
        parts = [np.ascontiguousarray(last[:, i * w:(i + 1) * w]) for i in range(3)]
        for h in (0, heads - 1):
            sl = slice(h * hd, (h + 1) * hd)
            q, k, v = (np.ascontiguousarray(p[:, sl]) for p in parts)
            want, mag, cond = attention64(q, k, v, 1, True, O.attention_scale(hd))
            assert_attention_close(got[:, sl], want, mag, cond, f"last sequence head {h}")
        ctx.fill(dout, 0.5)
        ctx.upload(dout.offset((rows - seq) * w, (seq, w)), last_dout)
        print("attention backward past 2^31", flush=True)
        ctx.attention_bwd(qkv, qkv.offset(w), qkv.offset(2 * w), dout, g, g.offset(w), g.offset(2 * w), b, seq, seq,
                          heads, hd, True, ld_q=3 * w, ld_kv=3 * w, ld_dout=w, ld_dq=3 * w, ld_dkv=3 * w)
        tail = _slice(ctx, g, (rows - seq) * 3 * w, seq * 3 * w).reshape(seq, 3 * w)
        q, k, v = (np.ascontiguousarray(p[:, :hd]) for p in parts)
        want, tol = attention_bwd64(q, k, v, last_dout[:, :hd], 1, True, O.attention_scale(hd))
        for j, name in enumerate(("dq", "dk", "dv")):
            assert_bwd_close(tail[:, j * w:j * w + hd], want[j], tol[j], f"last sequence head 0 {name}")
        # The constant first sequence: dv_j = 0.5 * sum_{i >= j} 1 / (i + 1)
        # (P is 1/(i+1) on the visible keys), dq and dk vanish up to rounding.
        head = _slice(ctx, g, 0, seq * 3 * w).reshape(seq, 3 * w)
        dv_want = 0.5 * np.cumsum((1.0 / np.arange(1, seq + 1))[::-1])[::-1]
        assert_close(head[:, 2 * w], dv_want.astype(np.float32), "constant first sequence dv", rel=1e-4)
        assert np.abs(head[:, :2 * w]).max() < 1e-5, "constant first sequence dq / dk"
    finally:
        for d in (qkv, out, dout, g):
            d.free()
