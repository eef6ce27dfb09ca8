"""Attention cases shared by the CPU pin tests (tests/test_oracle_attention.py),
the golden writer (tests/golden/make_golden.py) and the GPU parity tests.

The reference's attention functions (LayerOps::self_attention_forward,
LayerOps.hpp:1004-1097; cross_attention_forward, :1116-1216) wrap the core in
two projections.  With one-hot input rows (row m = e_(m mod E)) and an
identity output projection both projections are exact in float32 (each output
is one product 1*w plus products 0*w), so the reference's output IS its
attention core on Q / K / V = the selected rows of the projection weights."""
import numpy as np

import oracle as O

# (seq_len, embed_dim, num_heads): head_dim = embed_dim / num_heads.
SELF_CASES = [(1, 8, 1), (8, 8, 1), (5, 16, 2), (24, 32, 4), (33, 32, 1), (64, 64, 2), (100, 128, 1),
              (130, 96, 3), (40, 48, 3), (70, 80, 1)]
# (query_len, kv_len, embed_dim, num_heads)
CROSS_CASES = [(1, 7, 8, 1), (9, 4, 16, 2), (40, 65, 64, 2), (33, 100, 128, 1)]


def one_hot_rows(n, e):
    x = np.zeros((n, e), np.float32)
    x[np.arange(n), np.arange(n) % e] = 1.0
    return x


def self_case(seq, e, amp, seed):
    """(input, qkv_weight, q, k, v): q/k/v are the rows the one-hot input selects."""
    rng = np.random.default_rng(seed)
    w = (amp * rng.standard_normal((e, 3 * e))).astype(np.float32)
    x = one_hot_rows(seq, e)
    rows = w[np.arange(seq) % e]
    return x, w, rows[:, :e].copy(), rows[:, e:2 * e].copy(), rows[:, 2 * e:].copy()


def cross_case(q_len, kv_len, e, amp, seed):
    """(xq, xkv, q_weight, kv_weight, q, k, v)."""
    rng = np.random.default_rng(seed)
    wq = (amp * rng.standard_normal((e, e))).astype(np.float32)
    wkv = (amp * rng.standard_normal((e, 2 * e))).astype(np.float32)
    xq, xkv = one_hot_rows(q_len, e), one_hot_rows(kv_len, e)
    q = wq[np.arange(q_len) % e].copy()
    kv = wkv[np.arange(kv_len) % e]
    return xq, xkv, wq, wkv, q, kv[:, :e].copy(), kv[:, e:].copy()


def attention64(q, k, v, heads, causal, scale):
    """float64 softmax attention: (out, mag, cond) -- oracle.attention_float64,
    whose cond term (the propagated rounding of the float32 scores) the
    restatement pinned to the reference stays within a quarter of even where
    the scores reach +-50 (tests/test_oracle_attention.py)."""
    return O.attention_float64(q, k, v, heads, causal, scale)


def assert_attention_close(got, ref, mag, cond, what=""):
    """|got - ref| <= max(1e-6, 1e-5 * max(|ref|, mag)) + cond (attention64)."""
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    mag = np.asarray(mag, np.float64).ravel()
    cond = np.asarray(cond, np.float64).ravel()
    assert got.shape == ref.shape, f"{what}: shape {got.shape} != {ref.shape}"
    assert ref.size, f"{what}: empty"
    assert np.array_equal(np.isnan(got), np.isnan(ref)), f"{what}: NaN pattern differs"
    fin = np.isfinite(ref)
    d = np.abs(got[fin] - ref[fin])
    tol = np.maximum(1e-6, 1e-5 * np.maximum(np.abs(ref[fin]), mag[fin])) + cond[fin]
    bad = d > tol
    if bad.any():
        idx = np.flatnonzero(fin)[np.argmax(d / tol)]
        raise AssertionError(f"{what}: {int(bad.sum())} of {fin.sum()} elements out of tolerance; worst at {idx}: "
                             f"got {got[idx]!r} ref {ref[idx]!r} mag {mag[idx]:.3g} cond {cond[idx]:.3g}")


def _core_layer_tol(q, k, v, qa, ka, va, heads, causal, scale):
    """float64 core output with its tolerance given projection-error scales
    qa / ka / va (1e-5 * sum of |terms| of each projected element)."""
    out, mag, cond = attention64(q, k, v, heads, causal, scale)
    q, k, v, qa, ka, va = (np.asarray(a, np.float64) for a in (q, k, v, qa, ka, va))
    lq, w = q.shape
    lk = k.shape[0]
    hd = w // heads
    sc = abs(float(np.float32(scale)))
    extra = np.zeros((lq, w))
    mask = np.arange(lk)[None, :] > np.arange(lq)[:, None]
    for h in range(heads):
        sl = slice(h * hd, (h + 1) * hd)
        s = (q[:, sl] @ k[:, sl].T) * float(np.float32(scale))
        if causal:
            s = np.where(mask, -np.inf, s)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        ds = sc * (qa[:, sl] @ np.abs(k[:, sl]).T + np.abs(q[:, sl]) @ ka[:, sl].T)  # score error bound
        extra[:, sl] = p @ va[:, sl] + (p * ds) @ np.abs(v[:, sl]) + (p * ds).sum(1, keepdims=True) * np.abs(out[:, sl])
    tol = np.maximum(1e-6, 1e-5 * np.maximum(np.abs(out), mag)) + cond + extra
    return out, tol


def attention_layer64(x, wqkv, wout, heads, causal):
    """float64 LayerOps::self_attention_forward with a first-order tolerance:
    each projection's float32 rounding (1e-5 of its summed magnitudes), carried
    through the core (values directly, scores through both operands), the
    core's own bound (attention64), and the output projection (|W| times the
    core's bound, plus its own rounding).  Returns (out, tol)."""
    x, wqkv, wout = (np.asarray(a, np.float64) for a in (x, wqkv, wout))
    e = x.shape[1]
    qkv, qkv_a = x @ wqkv, 1e-5 * (np.abs(x) @ np.abs(wqkv))
    att, att_tol = _core_layer_tol(qkv[:, :e], qkv[:, e:2 * e], qkv[:, 2 * e:], qkv_a[:, :e], qkv_a[:, e:2 * e],
                                   qkv_a[:, 2 * e:], heads, causal, 1.0 / np.sqrt(np.float32(e // heads)))
    out = att @ wout
    return out, att_tol @ np.abs(wout) + 1e-5 * (np.abs(att) @ np.abs(wout)) + 1e-6


def cross_attention_layer64(xq, xkv, wq, wkv, wout, heads, causal):
    """float64 LayerOps::cross_attention_forward with the same tolerance."""
    xq, xkv, wq, wkv, wout = (np.asarray(a, np.float64) for a in (xq, xkv, wq, wkv, wout))
    e = xq.shape[1]
    q, qa = xq @ wq, 1e-5 * (np.abs(xq) @ np.abs(wq))
    kv, kva = xkv @ wkv, 1e-5 * (np.abs(xkv) @ np.abs(wkv))
    att, att_tol = _core_layer_tol(q, kv[:, :e], kv[:, e:], qa, kva[:, :e], kva[:, e:], heads, causal,
                                   1.0 / np.sqrt(np.float32(e // heads)))
    out = att @ wout
    return out, att_tol @ np.abs(wout) + 1e-5 * (np.abs(att) @ np.abs(wout)) + 1e-6


def assert_within(got, ref, tol, what=""):
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    tol = np.asarray(tol, np.float64).ravel()
    assert got.shape == ref.shape and ref.size, f"{what}: shape"
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    d = np.abs(got - ref)
    bad = d > tol
    if bad.any():
        i = int(np.argmax(d / tol))
        raise AssertionError(f"{what}: {int(bad.sum())} of {d.size} out of tolerance; worst at {i}: got {got[i]!r} "
                             f"ref {ref[i]!r} tol {tol[i]:.3g}")


def layer_case(seq, e, seed, amp=1.0):
    """Random SelfAttention inputs: x, the [Wqkv | Wout] block, with weights
    scaled 1/sqrt(E) so the projections keep unit scale (scores ~ amp^2)."""
    r = np.random.default_rng(seed)
    x = (amp * r.standard_normal((seq, e))).astype(np.float32)
    w = (r.standard_normal(4 * e * e) / np.sqrt(e)).astype(np.float32)
    return x, w


# ---------------------------------------------------------------------------
# Backward (backward_self_attention / backward_cross_attention, Model.cpp:
# 6847-7300): float64 gradients with a first-order bound on their float32
# rounding.  Every product is charged GAMMA of its summed magnitudes (|A||B|,
# the classical bound gamma_n |A||B| with gamma_n ~ n u, which 1e-5 covers for
# the head dimensions here and, with the sqrt(n) growth of real rounding, for
# the sequence lengths), elementwise steps a few u, and each input's own
# error bound (eq, ek, ev, eo: the projections' rounding) is carried through
# by the derivative's absolute value.
# ---------------------------------------------------------------------------
GAMMA = 1e-5
EW = 4 * O.U32  # an elementwise subtract / multiply / exp step


def _softmax_rows64(s, mask):
    if mask is not None:
        s = np.where(mask, -np.inf, s)
    p = np.exp(s - s.max(axis=1, keepdims=True))
    return p / p.sum(axis=1, keepdims=True)


def attention_bwd64(q, k, v, dout, heads, causal, scale, eq=None, ek=None, ev=None, eo=None):
    """float64 (dq, dk, dv) of the core for one sequence (q [lq, W], k / v
    [lk, W], dout [lq, W]) and their bounds (tq, tk, tv); eq..eo: error bounds
    of the inputs (None = exact).  A floor of 1e-6 of each gradient's largest
    magnitude covers elements whose terms all vanish."""
    q, k, v, dout = (np.asarray(a, np.float64) for a in (q, k, v, dout))
    z = lambda a, e: np.zeros_like(a) if e is None else np.asarray(e, np.float64)
    eq, ek, ev, eo = z(q, eq), z(k, ek), z(v, ev), z(dout, eo)
    lq, w = q.shape
    lk = k.shape[0]
    hd = w // heads
    sc = float(np.float32(scale))
    asc = abs(sc)
    mask = (np.arange(lk)[None, :] > np.arange(lq)[:, None]) if causal else None
    dq, dk, dv = np.zeros((lq, w)), np.zeros((lk, w)), np.zeros((lk, w))
    tq, tk, tv = np.zeros((lq, w)), np.zeros((lk, w)), np.zeros((lk, w))
    for h in range(heads):
        sl = slice(h * hd, (h + 1) * hd)
        Q, K, V, D = q[:, sl], k[:, sl], v[:, sl], dout[:, sl]
        aQ, aK, aV, aD = np.abs(Q), np.abs(K), np.abs(V), np.abs(D)
        P = _softmax_rows64(sc * (Q @ K.T), mask)
        eS = asc * (eq[:, sl] @ aK.T + aQ @ ek[:, sl].T) + GAMMA * asc * (aQ @ aK.T)
        eP = P * (eS + (P * eS).sum(1, keepdims=True)) + GAMMA * P
        G = D @ V.T
        eG = eo[:, sl] @ aV.T + aD @ ev[:, sl].T + GAMMA * (aD @ aV.T)
        r = (P * G).sum(1, keepdims=True)
        er = (eP * np.abs(G) + P * eG).sum(1, keepdims=True) + GAMMA * (P * np.abs(G)).sum(1, keepdims=True)
        dS = P * (G - r)
        eDS = eP * np.abs(G - r) + P * (eG + er) + EW * P * (np.abs(G) + np.abs(r))
        if mask is not None:
            dS = np.where(mask, 0.0, dS)
            eDS = np.where(mask, 0.0, eDS)
        aDS = np.abs(dS)
        dv[:, sl] = P.T @ D
        tv[:, sl] = eP.T @ aD + P.T @ eo[:, sl] + GAMMA * (P.T @ aD)
        dq[:, sl] = sc * (dS @ K)
        tq[:, sl] = asc * (eDS @ aK + aDS @ ek[:, sl] + GAMMA * (aDS @ aK))
        dk[:, sl] = sc * (dS.T @ Q)
        tk[:, sl] = asc * (eDS.T @ aQ + aDS.T @ eq[:, sl] + GAMMA * (aDS.T @ aQ))
    out = []
    for g, t in ((dq, tq), (dk, tk), (dv, tv)):
        out.append(t + 1e-6 * (np.abs(g).max() if g.size else 0.0))
    return (dq, dk, dv), tuple(out)


def _proj64(x, w):
    """x @ w in float64 and the bound of its float32 rounding."""
    return x @ w, GAMMA * (np.abs(x) @ np.abs(w))


def self_attention_bwd64(x, wqkv, wout, dy, heads, causal):
    """float64 backward_self_attention with bounds: ((dx, dWqkv, dWout),
    (tx, tWqkv, tWout))."""
    x, wqkv, wout, dy = (np.asarray(a, np.float64) for a in (x, wqkv, wout, dy))
    e = x.shape[1]
    scale = 1.0 / np.sqrt(np.float32(e // heads))
    qkv, eqkv = _proj64(x, wqkv)
    datt, edatt = _proj64(dy, wout.T)
    q, k, v = qkv[:, :e], qkv[:, e:2 * e], qkv[:, 2 * e:]
    (dq, dk, dv), (tq, tk, tv) = attention_bwd64(q, k, v, datt, heads, causal, scale, eqkv[:, :e],
                                                 eqkv[:, e:2 * e], eqkv[:, 2 * e:], edatt)
    att, tatt = _core_layer_tol(q, k, v, eqkv[:, :e], eqkv[:, e:2 * e], eqkv[:, 2 * e:], heads, causal, scale)
    dqkv, tqkv = np.concatenate([dq, dk, dv], 1), np.concatenate([tq, tk, tv], 1)
    dwout = att.T @ dy
    twout = tatt.T @ np.abs(dy) + GAMMA * (np.abs(att).T @ np.abs(dy))
    dwqkv = x.T @ dqkv
    twqkv = np.abs(x).T @ tqkv + GAMMA * (np.abs(x).T @ np.abs(dqkv))
    dx = dqkv @ wqkv.T
    tx = tqkv @ np.abs(wqkv).T + GAMMA * (np.abs(dqkv) @ np.abs(wqkv).T)
    return (dx, dwqkv, dwout), (tx, twqkv, twout)


def cross_attention_bwd64(xq, xkv, wq, wkv, wout, dy, heads, causal):
    """float64 backward_cross_attention with bounds: ((dxq, dxkv, dWq, dWkv,
    dWout), (their bounds))."""
    xq, xkv, wq, wkv, wout, dy = (np.asarray(a, np.float64) for a in (xq, xkv, wq, wkv, wout, dy))
    e = xq.shape[1]
    scale = 1.0 / np.sqrt(np.float32(e // heads))
    q, eq = _proj64(xq, wq)
    kv, ekv = _proj64(xkv, wkv)
    datt, edatt = _proj64(dy, wout.T)
    k, v = kv[:, :e], kv[:, e:]
    (dq, dk, dv), (tq, tk, tv) = attention_bwd64(q, k, v, datt, heads, causal, scale, eq, ekv[:, :e], ekv[:, e:],
                                                 edatt)
    att, tatt = _core_layer_tol(q, k, v, eq, ekv[:, :e], ekv[:, e:], heads, causal, scale)
    dkv, tkv = np.concatenate([dk, dv], 1), np.concatenate([tk, tv], 1)
    dwout = att.T @ dy
    twout = tatt.T @ np.abs(dy) + GAMMA * (np.abs(att).T @ np.abs(dy))
    dwq, twq = xq.T @ dq, np.abs(xq).T @ tq + GAMMA * (np.abs(xq).T @ np.abs(dq))
    dwkv, twkv = xkv.T @ dkv, np.abs(xkv).T @ tkv + GAMMA * (np.abs(xkv).T @ np.abs(dkv))
    dxq, txq = dq @ wq.T, tq @ np.abs(wq).T + GAMMA * (np.abs(dq) @ np.abs(wq).T)
    dxkv, txkv = dkv @ wkv.T, tkv @ np.abs(wkv).T + GAMMA * (np.abs(dkv) @ np.abs(wkv).T)
    return (dxq, dxkv, dwq, dwkv, dwout), (txq, txkv, twq, twkv, twout)


# The path's relative tolerance applied normwise: ||got - ref|| <= 1e-5 ||ref||
# (the reference's own backward is ~1e-6 from float64 on the tests' shapes).
NORM_REL = 1e-5


def assert_bwd_close(got, ref, tol, what, norm_rel=NORM_REL):
    """Element-wise |got - ref| <= tol and ||got - ref|| <= norm_rel ||ref||."""
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    tol = np.asarray(tol, np.float64).ravel()
    assert got.shape == ref.shape, f"{what}: shape {got.shape} != {ref.shape}"
    assert np.isfinite(got).all(), f"{what}: non-finite values"
    d = np.abs(got - ref)
    if (d > tol).any():
        i = int(np.argmax(d / tol))
        raise AssertionError(f"{what}: {int((d > tol).sum())} of {d.size} beyond the bound; worst at {i}: got "
                             f"{got[i]!r} ref {ref[i]!r} bound {tol[i]:.3g}")
    nref = np.linalg.norm(ref)
    if nref > 0:
        rel = np.linalg.norm(got - ref) / nref
        assert rel <= norm_rel, f"{what}: normwise relative error {rel:.3g} > {norm_rel}"


def ref_core_bwd_case(seq, e, heads, causal, seed, amp=1.0):
    """The reference's own backward core, observed through Model::backwardPass
    (oracle/_ref): a SelfAttention layer with one-hot input rows (seq <= E)
    and an identity output projection makes qkv the selected rows of Wqkv and
    dAtt = dY exactly, and dWqkv's first seq rows are then dq | dk | dv
    exactly (each is one product 1 * dqkv plus products with 0).  Returns
    (q, k, v, dy, dq, dk, dv)."""
    import model_ref as MR
    assert seq <= e
    r = np.random.default_rng(seed)
    wqkv = (amp * r.standard_normal((e, 3 * e))).astype(np.float32)
    w = np.concatenate([wqkv.ravel(), np.eye(e, dtype=np.float32).ravel()])
    x = one_hot_rows(seq, e)
    dy = r.standard_normal((seq, e)).astype(np.float32)
    L = dict(name="attn", type="SelfAttention", inputs=["x"], output="x", seq_len=seq, embed_dim=e, num_heads=heads,
             causal=causal, weights=w)
    grads, _ = MR.backward([L], {"x": x.ravel()}, {}, dy.ravel())
    dw = grads[0][:3 * e * e].reshape(e, 3 * e)[:seq]
    rows = wqkv[np.arange(seq)]
    return (rows[:, :e].copy(), rows[:, e:2 * e].copy(), rows[:, 2 * e:].copy(), dy, dw[:, :e].copy(),
            dw[:, e:2 * e].copy(), dw[:, 2 * e:].copy())
