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
