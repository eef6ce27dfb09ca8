"""The BASELINE configurations at full size on the GPU.

The CPU oracle is too slow to restate every element at these sizes, so each
test combines (a) exact whole-tensor checks where numpy computes the same
IEEE result (gather = fancy indexing, residual add = float32 add), (b) the
oracle on a seeded sample of rows, and (c) size-independent invariants
(softmax rows sum to 1 with masked entries exactly 0, RoPE preserves every
pair's norm, RMSNorm rows have unit mean square)."""
import numpy as np
import pytest

import mimir_hip as M
import oracle as O
from _parity import assert_bitexact, assert_close
from mimir_hip import datagen as G

pytestmark = pytest.mark.gpu

sample_rng = np.random.default_rng(11)


def _sample(n, k):
    return np.sort(sample_rng.choice(n, size=min(k, n), replace=False))


def test_cfg1_add_rmsnorm_full(ctx):
    x, r, w, eps = G.cfg1_add_rmsnorm()
    rows, cols = x.shape
    dx, dr, dw = ctx.to_device(x), ctx.to_device(r), ctx.to_device(w)
    dy = ctx.empty(x.shape)
    ctx.add_rmsnorm(dx, dr, dr, dw, dy, rows, cols, eps)
    h = dr.numpy()
    y = dy.numpy()
    for d in (dx, dr, dw, dy):
        d.free()
    assert_bitexact(h, x + r, "residual'")
    idx = _sample(rows, 256)
    y_ref, _ = O.add_rmsnorm(x[idx], r[idx], w, eps)
    assert_close(y[idx], y_ref, "sampled rows")
    ms = np.mean((y.astype(np.float64) / w) ** 2, axis=1)
    assert np.all(np.abs(ms - 1.0) < 1e-4)


def test_cfg2_causal_softmax_full(ctx):
    s = G.cfg2_softmax()
    B, H, Q, K = s.shape
    d = ctx.to_device(s)
    dy = ctx.empty(s.shape)
    ctx.softmax(d, dy, B * H * Q, K, M.SOFTMAX_DIV_EPS)
    y = dy.numpy()
    d.free()
    dy.free()
    y2 = y.reshape(-1, K)
    s2 = s.reshape(-1, K)
    assert np.all(np.abs(y2.sum(axis=1, dtype=np.float64) - 1.0) < 1e-5)
    mask = np.triu(np.ones((Q, K), bool), 1)
    assert not y[:, :, mask].any(), "masked entries must be exactly 0"
    assert np.all(y[:, :, 0, 0] == 1.0)
    idx = _sample(B * H * Q, 2048)
    assert_close(y2[idx], O.softmax_rows(s2[idx]), "sampled rows")


def test_cfg3_gather_full_bitexact(ctx):
    table, ids = G.cfg3_gather()
    vocab, dim = table.shape
    dt, di = ctx.to_device(table), ctx.to_device(ids)
    dy = ctx.empty((ids.size, dim))
    ctx.embedding(di, ids.size, dt, table.size, vocab, dim, -1, dy)
    y = dy.numpy()
    for d in (dt, di, dy):
        d.free()
    assert_bitexact(y, table[ids.ravel()], "cfg3 gather")


def test_cfg3_rope_full(ctx):
    q, k, theta = G.cfg3_rope()
    B, S, H, D = q.shape
    cos_t, sin_t = M.rope_table(S, D, theta)
    dq, dk = ctx.to_device(q), ctx.to_device(k)
    dc, ds = ctx.to_device(cos_t), ctx.to_device(sin_t)
    ctx.rope(dq, dq, H, dk, dk, H, B, S, D, 0, dc, ds, S)
    qo, ko = dq.numpy(), dk.numpy()
    for d in (dq, dk, dc, ds):
        d.free()
    half = D // 2
    for name, x, y in (("q", q, qo), ("k", k, ko)):
        n_in = x[..., :half].astype(np.float64) ** 2 + x[..., half:].astype(np.float64) ** 2
        n_out = y[..., :half].astype(np.float64) ** 2 + y[..., half:].astype(np.float64) ** 2
        assert np.allclose(n_out, n_in, rtol=2e-6, atol=1e-6), f"{name}: pair norms not preserved"
        assert_bitexact(y[:, 0], x[:, 0], f"{name}: position 0 is the identity")
        for b in (0, B - 1):
            sidx = _sample(S, 64)
            assert_close(y[b, sidx], O.rope(x[b:b + 1, sidx], cos_t[sidx], sin_t[sidx])[0],
                         f"{name}: sampled positions")


def test_cfg4_layernorm_full(ctx):
    x, g, b, eps = G.cfg4_layernorm()
    rows, cols = x.shape
    dx, dg, db = ctx.to_device(x), ctx.to_device(g), ctx.to_device(b)
    dy = ctx.empty(x.shape)
    ctx.layernorm(dx, dg, db, dy, rows, cols, eps)
    y = dy.numpy()
    for d in (dx, dg, db, dy):
        d.free()
    idx = _sample(rows, 256)
    assert_close(y[idx], O.layernorm(x[idx], cols, g, b, eps).reshape(len(idx), cols), "sampled rows")
    z = (y.astype(np.float64) - b) / g
    assert np.all(np.abs(z.mean(axis=1)) < 1e-5)
    assert np.all(np.abs(z.var(axis=1) - 1.0) < 1e-4)


def test_cfg4_gelu_swiglu_add_full(ctx):
    a = G.cfg4_gelu()
    n = a.size
    da = ctx.to_device(a)
    dy = ctx.empty(a.shape)
    ctx.gelu(da, dy, n)
    y = dy.numpy().ravel()
    idx = _sample(n, 1 << 20)
    assert_close(y[idx], O.gelu(a.ravel()[idx]), "gelu sample")
    gate, up = G.cfg4_swiglu()
    ctx.upload(da, gate)
    du = ctx.to_device(up)
    ctx.silu_mul(da, du, dy, n)
    y = dy.numpy().ravel()
    assert_close(y[idx], O.silu_mul(gate.ravel()[idx], up.ravel()[idx]), "silu*up sample")
    for d in (da, du, dy):
        d.free()
    a, b = G.cfg4_add()
    da, db = ctx.to_device(a), ctx.to_device(b)
    dy = ctx.empty(a.shape)
    ctx.add(da, a.size, db, b.size, dy)
    assert_bitexact(dy.numpy(), a + b, "residual add")
    for d in (da, db, dy):
        d.free()
