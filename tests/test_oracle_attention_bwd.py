"""Pins of the attention backward's oracle (oracle_attention_bwd, the float64
model tests/_attention.attention_bwd64 and its layer forms) on the CPU:

- the C restatement against the reference's own Model::backwardPass
  (oracle/_ref), bit for bit: with one-hot input rows and an identity output
  projection the reference's dWqkv rows are its core's dq | dk | dv exactly
  (tests/_attention.ref_core_bwd_case);
- the float64 gradients against central finite differences of the float64
  forward (the mathematics, independent of the reference);
- the float32 restatement within the float64 model's bound, element-wise
  (first-order propagation, 1e-5 of each product's summed magnitudes) and
  normwise (relative error <= 1e-5, the path's relative tolerance; the
  reference itself is ~1e-6);
- plausible mistakes planted in a float64 restatement (no row-dot term, a
  transposed operand, a missing scale, the diagonal masked, softmax of
  unscaled scores) each fail those checks;
- the reference's whole-layer backward (SelfAttention, MultiHeadAttention,
  CrossAttention through Model::backwardPass) within the layer models."""
import numpy as np
import pytest

import model_ref as MR
import oracle as O
from _attention import (assert_bwd_close, attention_bwd64, cross_attention_bwd64, layer_case, ref_core_bwd_case,
                        self_attention_bwd64)

def _bwd_fails(got, ref, tol):
    try:
        assert_bwd_close(got, ref, tol, "planted")
    except AssertionError:
        return True
    return False


ref_only = pytest.mark.skipif(not MR.available(), reason="oracle/_ref not built")

# (seq, E, heads, causal, seed, amplitude of the Q/K/V weights: scores ~ amp^2)
CORE_CASES = [(8, 16, 2, True, 1, 1.0), (24, 32, 4, False, 2, 1.0), (33, 48, 3, True, 3, 1.0),
              (40, 64, 1, False, 4, 1.0), (64, 128, 2, True, 5, 1.0), (64, 64, 1, True, 6, 3.0),
              (100, 128, 1, False, 7, 2.0), (1, 8, 1, True, 8, 1.0), (130, 160, 5, True, 9, 1.5)]


@ref_only
@pytest.mark.parametrize("case", CORE_CASES, ids=lambda c: "x".join(map(str, c[:4])))
def test_oracle_is_the_reference_backward(case):
    seq, e, heads, causal, seed, amp = case
    q, k, v, dy, dq, dk, dv = ref_core_bwd_case(seq, e, heads, causal, seed, amp)
    gq, gk, gv = O.attention_bwd(q, k, v, dy, heads, causal)
    for name, got, want in (("dq", gq, dq), ("dk", gk, dk), ("dv", gv, dv)):
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"{name} differs from the reference"


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("lq,lk", [(4, 4), (3, 5), (5, 2)])
def test_float64_gradient_is_the_derivative(causal, lq, lk):
    """d/dX sum(dout * attention(q, k, v)) by central differences."""
    r = np.random.default_rng(lq * 10 + lk + causal)
    heads, hd = 2, 3
    w = heads * hd
    q, k, v, dout = r.standard_normal((lq, w)), r.standard_normal((lk, w)), r.standard_normal((lk, w)), \
        r.standard_normal((lq, w))
    scale = 0.7
    (dq, dk, dv), _ = attention_bwd64(q, k, v, dout, heads, causal, scale)

    def f(q_, k_, v_):
        return float((dout * O.attention_float64(q_, k_, v_, heads, causal, scale)[0]).sum())

    h = 1e-6
    for name, arr, grad in (("q", q, dq), ("k", k, dk), ("v", v, dv)):
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            a1, a2 = arr.copy(), arr.copy()
            a1[idx] += h
            a2[idx] -= h
            args1 = {"q": (a1, k, v), "k": (q, a1, v), "v": (q, k, a1)}[name]
            args2 = {"q": (a2, k, v), "k": (q, a2, v), "v": (q, k, a2)}[name]
            num[idx] = (f(*args1) - f(*args2)) / (2 * h)
        np.testing.assert_allclose(grad, num, rtol=1e-6, atol=1e-8, err_msg=f"d{name}")


def _core_inputs(lq, lk, w, seed, amp=1.0):
    r = np.random.default_rng(seed)
    return tuple((amp * r.standard_normal(s)).astype(np.float32) for s in ((lq, w), (lk, w), (lk, w))) + \
        (r.standard_normal((lq, w)).astype(np.float32),)


# (q_len, kv_len, heads, head_dim, causal, amp)
BOUND_CASES = [(64, 64, 2, 32, True, 1.0), (37, 90, 4, 16, False, 1.0), (90, 37, 1, 64, True, 2.0),
               (128, 128, 1, 128, True, 3.0), (17, 300, 2, 48, False, 1.0)]


@pytest.mark.parametrize("case", BOUND_CASES, ids=lambda c: "x".join(map(str, c)))
def test_oracle_within_float64_bound(case):
    lq, lk, heads, hd, causal, amp = case
    q, k, v, dout = _core_inputs(lq, lk, heads * hd, lq + lk + hd, amp)
    got = O.attention_bwd(q, k, v, dout, heads, causal)
    want, tol = attention_bwd64(q, k, v, dout, heads, causal, O.attention_scale(hd))
    for name, g, w_, t in zip(("dq", "dk", "dv"), got, want, tol):
        assert_bwd_close(g, w_, t, name)
        # the bound is met with room: the restatement's (= the reference's) error stays under 5% of it
        assert np.max(np.abs(g - w_) / t) < 0.05, name


def _variant64(q, k, v, dout, heads, causal, scale, mistake):
    """The float64 core backward with one planted mistake."""
    q, k, v, dout = (np.asarray(a, np.float64) for a in (q, k, v, dout))
    lq, w = q.shape
    lk = k.shape[0]
    hd = w // heads
    diag = 0 if mistake == "mask_diagonal" else 1
    mask = (np.arange(lk)[None, :] >= np.arange(lq)[:, None] + diag) if causal else np.zeros((lq, lk), bool)
    dq, dk, dv = np.zeros((lq, w)), np.zeros((lk, w)), np.zeros((lk, w))
    for h in range(heads):
        sl = slice(h * hd, (h + 1) * hd)
        Q, K, V, D = q[:, sl], k[:, sl], v[:, sl], dout[:, sl]
        s = (Q @ K.T) * (1.0 if mistake == "unscaled_scores" else scale)
        s = np.where(mask, -np.inf, s)
        with np.errstate(invalid="ignore"):  # "mask_diagonal" masks row 0 whole: NaN there
            P = np.exp(s - s.max(1, keepdims=True))
            P /= P.sum(1, keepdims=True)
        G = D @ V.T
        r = 0.0 if mistake == "no_row_dot" else (P * G).sum(1, keepdims=True)
        dS = P * (G - r)
        dv[:, sl] = (P if mistake == "dv_not_transposed" else P.T) @ D
        dq[:, sl] = (1.0 if mistake == "dq_unscaled" else scale) * (dS @ K)
        dk[:, sl] = scale * ((dS if mistake == "dk_not_transposed" else dS.T) @ Q)
    return dq, dk, dv


@pytest.mark.parametrize("mistake", ["no_row_dot", "dv_not_transposed", "dq_unscaled", "dk_not_transposed",
                                     "mask_diagonal", "unscaled_scores"])
def test_planted_mistakes_fail(mistake):
    lq = lk = 48
    heads, hd = 2, 32
    q, k, v, dout = _core_inputs(lq, lk, heads * hd, 5)
    scale = O.attention_scale(hd)
    got = O.attention_bwd(q, k, v, dout, heads, True)
    _, tol = attention_bwd64(q, k, v, dout, heads, True, scale)
    wrong = _variant64(q, k, v, dout, heads, True, scale, mistake)
    right = _variant64(q, k, v, dout, heads, True, scale, "none")
    assert not any(_bwd_fails(g, w_, t) for g, w_, t in zip(got, right, tol)), "the unplanted variant must pass"
    assert any(_bwd_fails(g, w_, t) for g, w_, t in zip(got, wrong, tol)), f"{mistake} was not caught"


def test_oracle_edges():
    # no keys: dq = 0, dk / dv empty; no queries: nothing written
    q, k, v, dout = _core_inputs(5, 0, 8, 1)
    dq, dk, dv = O.attention_bwd(q, k, v, dout, 2, False)
    assert np.array_equal(dq, np.zeros_like(dq)) and dk.size == 0 and dv.size == 0
    q, k, v, dout = _core_inputs(0, 4, 8, 1)
    dq, dk, dv = O.attention_bwd(q, k, v, dout, 2, True)
    assert dq.size == 0
    # one key: P = 1, so dS = 0, dq = dk = 0 and dv = dout
    q, k, v, dout = _core_inputs(1, 1, 8, 2)
    dq, dk, dv = O.attention_bwd(q, k, v, dout, 2, True)
    assert not dq.any() and not dk.any()
    assert np.array_equal(dv, dout)
    with pytest.raises(O.OracleError):
        O.attention_bwd(q, k, v, dout, 3, False)


# ---- whole layers through the reference's Model::backwardPass ---------------

SELF_LAYERS = [(40, 64, 4, True, "SelfAttention"), (33, 96, 3, False, "MultiHeadAttention"),
               (64, 128, 2, True, "SelfAttention"), (1, 32, 8, False, "SelfAttention"),
               (100, 64, 1, True, "MultiHeadAttention")]


def self_layer_case(seq, e, heads, causal, kind, seed, amp=1.0):
    x, w = layer_case(seq, e, seed, amp)
    dy = np.random.default_rng(seed + 100).standard_normal((seq, e)).astype(np.float32)
    L = dict(name="attn", type=kind, inputs=["__input__"], output="x", seq_len=seq, embed_dim=e, num_heads=heads,
             causal=causal, weights=w)
    return L, x, dy


@ref_only
@pytest.mark.parametrize("case", SELF_LAYERS, ids=lambda c: f"{c[4]}_{c[0]}x{c[1]}h{c[2]}{'c' if c[3] else ''}")
def test_reference_self_attention_backward_within_model(case):
    seq, e, heads, causal, kind = case
    L, x, dy = self_layer_case(seq, e, heads, causal, kind, seq + e, amp=1.5)
    grads, ig = MR.backward([L], {"x": x.ravel()}, {}, dy.ravel())
    w = L["weights"]
    (dx, dwqkv, dwout), (tx, twqkv, twout) = self_attention_bwd64(
        x, w[:3 * e * e].reshape(e, 3 * e), w[3 * e * e:].reshape(e, e), dy, heads, causal)
    assert_bwd_close(ig, dx, tx, "dx")
    assert_bwd_close(grads[0][:3 * e * e], dwqkv, twqkv, "dWqkv")
    assert_bwd_close(grads[0][3 * e * e:], dwout, twout, "dWout")


def cross_layer_case(lq, lk, e, heads, causal, seed, grad_of="query"):
    """A CrossAttention layer whose query (grad_of="query") or key/value
    input is "__input__", the name whose gradient the reference reports."""
    r = np.random.default_rng(seed)
    w = (r.standard_normal(4 * e * e) / np.sqrt(e)).astype(np.float32)
    xq = r.standard_normal((lq, e)).astype(np.float32)
    xkv = r.standard_normal((lk, e)).astype(np.float32)
    dy = r.standard_normal((lq, e)).astype(np.float32)
    inputs = ["__input__", "kv"] if grad_of == "query" else ["q", "__input__"]
    fin = {"x": xq.ravel(), "kv": xkv.ravel()} if grad_of == "query" else {"x": xkv.ravel(), "q": xq.ravel()}
    L = dict(name="cross", type="CrossAttention", inputs=inputs, output="x", embed_dim=e, num_heads=heads,
             causal=causal, weights=w)
    return L, fin, xq, xkv, dy


def cross_model(L, xq, xkv, dy):
    e = L["embed_dim"]
    w = L["weights"]
    return cross_attention_bwd64(xq, xkv, w[:e * e].reshape(e, e), w[e * e:3 * e * e].reshape(e, 2 * e),
                                 w[3 * e * e:].reshape(e, e), dy, L["num_heads"], L["causal"])


@ref_only
@pytest.mark.parametrize("grad_of", ["query", "kv"])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("lq,lk,e,heads", [(37, 90, 64, 4), (50, 20, 32, 2)])
def test_reference_cross_attention_backward_within_model(lq, lk, e, heads, causal, grad_of):
    L, fin, xq, xkv, dy = cross_layer_case(lq, lk, e, heads, causal, lq + lk, grad_of)
    grads, ig = MR.backward([L], fin, {}, dy.ravel())
    (dxq, dxkv, dwq, dwkv, dwout), (txq, txkv, twq, twkv, twout) = cross_model(L, xq, xkv, dy)
    if grad_of == "query":
        assert_bwd_close(ig, dxq, txq, "dxq")
    else:
        assert_bwd_close(ig, dxkv, txkv, "dxkv")
    assert_bwd_close(grads[0][:e * e], dwq, twq, "dWq")
    assert_bwd_close(grads[0][e * e:3 * e * e], dwkv, twkv, "dWkv")
    assert_bwd_close(grads[0][3 * e * e:], dwout, twout, "dWout")
