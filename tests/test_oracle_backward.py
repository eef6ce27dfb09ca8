"""Pin the backward restatements of oracle/mimir_oracle.c (the branches of
Model::backwardPass, Model.cpp:7305-9153) by mathematics: float64 closed
forms of each derivative, themselves checked against central finite
differences of the float64 forward, and brute force for the scatter-add and
the products.  (The compiled reference pins the same functions through whole
graphs in test_model_backward.py.)"""
import numpy as np
import pytest

import oracle as O
from _parity import assert_bitexact, assert_close

rng = np.random.default_rng(0xB0B)
K = np.sqrt(np.float64(np.float32(2.0) / np.float32(3.14159265359)))  # sqrt(2/pi) as the reference rounds it


def assert_scaled(got, exact, scale, what):
    """|got - exact| <= 1e-6 + 1e-5 * scale, scale = the sum of the magnitudes
    that were added (the condition of a float32 sum)."""
    d = np.abs(np.asarray(got, np.float64) - exact)
    bad = d > 1e-6 + 1e-5 * scale
    assert not bad.any(), f"{what}: {int(bad.sum())} elements out of the scaled bound, worst |d|={d.max():.3g}"


def ln_fwd64(x, g, b, eps):
    m = x.mean(axis=1, keepdims=True)
    v = ((x - m) ** 2).mean(axis=1, keepdims=True)
    y = (x - m) / np.sqrt(v + eps)
    return y * g + b


def ln_bwd64(x, dy, g, eps):
    """dL/dx, dL/dgamma, dL/dbeta of y = xhat*g + b, per row."""
    m = x.mean(axis=1, keepdims=True)
    v = ((x - m) ** 2).mean(axis=1, keepdims=True)
    inv = 1.0 / np.sqrt(v + eps)
    xh = (x - m) * inv
    dxh = dy * g
    dx = inv * (dxh - dxh.mean(axis=1, keepdims=True) - xh * (dxh * xh).mean(axis=1, keepdims=True))
    return dx, (dy * xh).sum(axis=0), dy.sum(axis=0)


def gelu64(x):
    return 0.5 * x * (1 + np.tanh(K * (x + 0.044715 * x ** 3)))


def dgelu64(x):
    u = K * (x + 0.044715 * x ** 3)
    t = np.tanh(u)
    return 0.5 * (1 + t) + 0.5 * x * (1 - t * t) * K * (1 + 3 * 0.044715 * x * x)


def silu64(x):
    return x / (1 + np.exp(-x))


def dsilu64(x):
    s = 1 / (1 + np.exp(-x))
    return s + x * s * (1 - s)


def test_closed_forms_match_finite_differences():
    # The float64 derivatives used below against central differences of the
    # float64 forward (h = 1e-6): pins the closed forms themselves.
    x = rng.standard_normal((3, 7))
    dy = rng.standard_normal((3, 7))
    g = 1 + 0.3 * rng.standard_normal(7)
    b = 0.3 * rng.standard_normal(7)
    eps, h = 1e-5, 1e-6
    dx, dg, db = ln_bwd64(x, dy, g, eps)
    num = np.zeros_like(x)
    for i in np.ndindex(x.shape):
        e = np.zeros_like(x)
        e[i] = h
        num[i] = ((ln_fwd64(x + e, g, b, eps) - ln_fwd64(x - e, g, b, eps)) * dy).sum() / (2 * h)
    np.testing.assert_allclose(dx, num, rtol=1e-6, atol=1e-8)
    num_g = np.array([((ln_fwd64(x, g + h * np.eye(7)[j], b, eps) - ln_fwd64(x, g - h * np.eye(7)[j], b, eps))
                       * dy).sum() / (2 * h) for j in range(7)])
    np.testing.assert_allclose(dg, num_g, rtol=1e-6, atol=1e-8)
    np.testing.assert_allclose(db, dy.sum(axis=0), rtol=1e-12)
    xs = np.linspace(-6, 6, 241)
    np.testing.assert_allclose(dgelu64(xs), (gelu64(xs + h) - gelu64(xs - h)) / (2 * h), rtol=1e-6, atol=1e-8)
    np.testing.assert_allclose(dsilu64(xs), (silu64(xs + h) - silu64(xs - h)) / (2 * h), rtol=1e-6, atol=1e-8)


@pytest.mark.parametrize("feat,affine,bias", [(64, True, True), (64, True, False), (64, False, False),
                                              (4096, True, True), (5, True, True)])
def test_layernorm_bwd_closed_form(feat, affine, bias):
    rows = 12
    x = (1.5 * rng.standard_normal((rows, feat)) + 0.3).astype(np.float32)
    dy = rng.standard_normal((rows, feat)).astype(np.float32)
    g = (1 + 0.2 * rng.standard_normal(feat)).astype(np.float32) if affine else None
    prev = rng.standard_normal(feat * (2 if bias else 1)).astype(np.float32) if affine else None
    dx, gp = O.layernorm_bwd(x, dy, feat, g, bias, 1e-5, prev)
    edx, edg, edb = ln_bwd64(x.astype(np.float64), dy.astype(np.float64),
                             1.0 if g is None else g.astype(np.float64), 1e-5)
    assert_close(dx, edx.ravel().astype(np.float32), "dx")
    if affine:
        # Sums over tokens added onto the previous block: the error bound scales
        # with the magnitudes summed (|prev| + sum |dy*xhat|), not with the
        # possibly cancelled result.
        xh = ln_fwd64(x.astype(np.float64), 1.0, 0.0, 1e-5)
        sg = np.abs(prev[:feat]) + np.abs(dy * xh).sum(axis=0)
        assert_scaled(gp[:feat], prev[:feat] + edg, sg, "dgamma (added onto the block)")
        if bias:
            assert_scaled(gp[feat:], prev[feat:] + edb, np.abs(prev[feat:]) + np.abs(dy).sum(axis=0), "dbeta")
    else:
        assert gp is None
    # A plausible mistake (dropping the xhat * mean(dxhat*xhat) term) fails the same check.
    m = x.mean(axis=1, keepdims=True, dtype=np.float64)
    inv = 1 / np.sqrt(((x - m) ** 2).mean(axis=1, keepdims=True) + 1e-5)
    dxh = dy * (1.0 if g is None else g)
    wrong = inv * (dxh - dxh.mean(axis=1, keepdims=True))
    with pytest.raises(AssertionError):
        assert_close(wrong.ravel().astype(np.float32), edx.ravel().astype(np.float32), "planted")


def test_layernorm_bwd_whole_vector_and_errors():
    x = rng.standard_normal(300).astype(np.float32)
    dy = rng.standard_normal(300).astype(np.float32)
    dx, _ = O.layernorm_bwd(x, dy, 0, None)  # in_features 0: one group of N
    edx = ln_bwd64(x[None].astype(np.float64), dy[None].astype(np.float64), 1.0, 1e-5)[0]
    assert_close(dx, edx.ravel().astype(np.float32), "whole vector")
    with pytest.raises(O.OracleError):
        O.layernorm_bwd(x, dy, 7, None)  # 300 % 7 != 0: the reference skips the layer


def test_gelu_silu_bwd_closed_form():
    x = np.concatenate([np.linspace(-8, 8, 20001), rng.standard_normal(5000) * 3]).astype(np.float32)
    dy = rng.standard_normal(x.size).astype(np.float32)
    x64, dy64 = x.astype(np.float64), dy.astype(np.float64)
    g = O.gelu_bwd(x, dy)
    # The reference's 0.5*(1+t) and 1-t*t both cancel once |x| > 3 (t -> +-1):
    # there its float32 result carries an absolute error of a few ulp of 1
    # times 0.5*|x|*du/dx, so the strict tolerance applies where |x| <= 3 and
    # a bound of that size beyond.
    ok = np.abs(x) <= 3
    assert_close(g[ok], (dy64 * dgelu64(x64))[ok].astype(np.float32), "gelu_bwd |x|<=3")
    du = K * (1 + 3 * 0.044715 * x64 * x64)
    assert_scaled(g[~ok], (dy64 * dgelu64(x64))[~ok], (np.abs(dy64) * (1 + np.abs(x64) * du) * 0.1)[~ok],
                  "gelu_bwd |x|>3")
    # A plausible mistake (du/dx without the 3*c*x^2 term) fails the strict region.
    wrong = dy64 * (0.5 * (1 + np.tanh(K * (x64 + 0.044715 * x64 ** 3)))
                    + 0.5 * x64 * (1 - np.tanh(K * (x64 + 0.044715 * x64 ** 3)) ** 2) * K)
    with pytest.raises(AssertionError):
        assert_close(wrong[ok].astype(np.float32), (dy64 * dgelu64(x64))[ok].astype(np.float32), "planted")
    assert_close(O.silu_bwd(x, dy), (dy64 * dsilu64(x64)).astype(np.float32), "silu_bwd")
    # Specials follow the reference's float expressions: inf/NaN inputs give NaN.
    sp = np.array([np.inf, -np.inf, np.nan, 0.0, -0.0], np.float32)
    one = np.ones(5, np.float32)
    g = O.gelu_bwd(sp, one)
    assert np.isnan(g[:3]).all() and g[3] == 0.5 and g[4] == 0.5
    s = O.silu_bwd(sp, one)
    assert np.isnan(s[:3]).all() and s[3] == 0.5  # x*ds = inf*0 at +-inf, as in the reference


def test_mul_bwd_and_accumulate_bitexact():
    a, b, dy = (rng.standard_normal(1000).astype(np.float32) for _ in range(3))
    da, db = O.mul_bwd(a, b, dy)
    assert_bitexact(da, dy * b, "da")
    assert_bitexact(db, dy * a, "db")
    assert_bitexact(O.accumulate(a, b), a + b, "accumulate")


@pytest.mark.parametrize("n_big,n_small", [(4096, 1), (64 * 48, 48), (10, 10), (7 * 5, 5)])
def test_add_bwd_small_sums(n_big, n_small):
    dy = rng.standard_normal(n_big).astype(np.float32)
    got = O.add_bwd_small(dy, n_small)
    exact = dy.astype(np.float64).reshape(-1, n_small).sum(axis=0)
    np.testing.assert_allclose(got, exact, rtol=1e-5, atol=2e-5 * np.sqrt(n_big / n_small))
    # Sequential float32 order, as the reference (Model.cpp:7582-7593).
    seq = np.zeros(n_small, np.float32)
    for t in range(n_big // n_small):
        seq += dy[t * n_small:(t + 1) * n_small]
    assert_bitexact(got, seq, "sequential order")
    with pytest.raises(O.OracleError):
        O.add_bwd_small(dy[:10], 3)


@pytest.mark.parametrize("float_ids", [False, True])
def test_embedding_bwd_brute_force(float_ids):
    vocab, dim, pad = 11, 24, 3
    ids = rng.integers(-2, vocab + 2, 200).astype(np.int32)
    ids[:20] = 4  # a row hit many times
    dy = rng.standard_normal((ids.size, dim)).astype(np.float32)
    gt0 = rng.standard_normal(vocab * dim).astype(np.float32)
    ref = gt0.reshape(vocab, dim).copy()
    keep = (ids != pad) & (ids >= 0) & (ids < vocab)
    np.add.at(ref, ids[keep], dy[keep])  # unbuffered, in token order: the reference's sequence of adds
    arg = ids.astype(np.float32) + (0.3 if float_ids else 0.0) if float_ids else ids
    got = O.embedding_bwd(arg, dy, gt0, vocab, dim, pad)
    assert_bitexact(got, ref.ravel(), "scatter-add")
    with pytest.raises(O.OracleError):
        O.embedding_bwd(ids, dy, gt0[:-1], vocab, dim, pad)  # table smaller than vocab*dim
