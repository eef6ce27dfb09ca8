"""Pin the attention restatement (oracle_attention in oracle/mimir_oracle.c):
- against the reference's own self_attention_forward / multihead_attention_
  forward / cross_attention_forward, compiled in place (oracle/_ref), through
  one-hot inputs and an identity output projection: bit-exact;
- against float64 softmax attention at the path's tolerance: the sum-aware
  bound 1e-5 * sum_j p_j |v_j| plus the propagated rounding of the float32
  scores (tests/_attention.py attention64), which the restatement must keep
  within a quarter of even for score ranges of +-50;
- on closed-form special cases (a causal first row returns V's first row;
  zero keys give the plain mean of the visible values);
- with planted mistakes (no 1/sqrt(d) scale, the mask reversed, K and V
  swapped, a head's columns shifted), each of which one of these checks
  rejects."""
import numpy as np
import pytest

import oracle as O
from _attention import CROSS_CASES, SELF_CASES, assert_attention_close, attention64, cross_case, self_case
from _parity import assert_bitexact, assert_close_sum

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")


@needs_ref
@pytest.mark.parametrize("seq,e,heads", SELF_CASES)
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("multihead", [False, True])
def test_self_attention_matches_reference(seq, e, heads, causal, multihead):
    x, w, q, k, v = self_case(seq, e, 1.5, seq * 1000 + e)
    ref = O.ref_self_attention(x, w, np.eye(e, dtype=np.float32), seq, e, heads, causal, multihead)
    assert_bitexact(O.attention(q, k, v, heads, causal), ref, f"self {seq}x{e} h{heads} causal={causal}")


@needs_ref
@pytest.mark.parametrize("lq,lk,e,heads", CROSS_CASES)
@pytest.mark.parametrize("causal", [False, True])
def test_cross_attention_matches_reference(lq, lk, e, heads, causal):
    xq, xkv, wq, wkv, q, k, v = cross_case(lq, lk, e, 1.2, lq * 7 + lk)
    ref = O.ref_cross_attention(xq, xkv, wq, wkv, np.eye(e, dtype=np.float32), lq, lk, e, heads, causal)
    assert_bitexact(O.attention(q[None], k[None], v[None], heads, causal)[0], ref,
                    f"cross {lq}x{lk} e{e} causal={causal}")


@needs_ref
def test_reference_refuses_heads_that_do_not_divide():
    x, w, q, k, v = self_case(4, 12, 1.0, 3)
    with pytest.raises(O.OracleError):
        O.ref_self_attention(x, w, np.eye(12, dtype=np.float32), 4, 12, 5)
    with pytest.raises(O.OracleError):
        O.attention(q, k, v, 5)


@pytest.mark.parametrize("batch,lq,lk,heads,hd", [(1, 1, 1, 1, 4), (2, 17, 17, 2, 16), (3, 64, 64, 4, 32),
                                                   (1, 50, 120, 1, 128), (2, 96, 40, 2, 64)])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("amp", [0.5, 2.0])
def test_against_float64(batch, lq, lk, heads, hd, causal, amp):
    rng = np.random.default_rng(batch * 131 + lq + lk + hd)
    w = heads * hd
    q = (amp * rng.standard_normal((batch, lq, w))).astype(np.float32)
    k = (amp * rng.standard_normal((batch, lk, w))).astype(np.float32)
    v = rng.standard_normal((batch, lk, w)).astype(np.float32)
    got = O.attention(q, k, v, heads, causal)
    want, mag, cond = attention64(q, k, v, heads, causal, O.attention_scale(hd))
    assert_attention_close(got, want, mag, cond, "oracle vs float64")


@pytest.mark.parametrize("hd", [32, 128])
@pytest.mark.parametrize("amp", [1.0, 4.0, 6.0])
def test_score_rounding_model(hd, amp):
    """The score-rounding term of the tolerance: the restatement's own error
    against float64 stays below a quarter of it and of the sum-aware bound
    together, from well-conditioned (amp 1) to score ranges of +-50 (amp 6),
    where the sum-aware bound alone is exceeded."""
    r = np.random.default_rng(99)
    q, k = ((amp * r.standard_normal((2, 150, hd))).astype(np.float32) for _ in range(2))
    v = r.standard_normal((2, 150, hd)).astype(np.float32)
    want, mag, cond = attention64(q, k, v, 1, True, O.attention_scale(hd))
    got = O.attention(q, k, v, 1, True)
    assert_attention_close(got, want, mag / 4, cond / 4, "within a quarter of the bound")


def test_closed_forms():
    rng = np.random.default_rng(7)
    lq, w, heads = 20, 32, 2
    q = rng.standard_normal((lq, w)).astype(np.float32)
    k = rng.standard_normal((lq, w)).astype(np.float32)
    v = rng.standard_normal((lq, w)).astype(np.float32)
    # Causal query 0 sees key 0 alone: p = 1 * (1 / (1 + 1e-9f)) = 1 exactly.
    assert_bitexact(O.attention(q, k, v, heads, True)[0], v[0], "causal row 0")
    # Zero keys: every visible score is 0, the weights are uniform.
    z = np.zeros_like(k)
    got = O.attention(q, z, v, heads, True)
    want = np.cumsum(v.astype(np.float64), axis=0) / np.arange(1, lq + 1)[:, None]
    assert_close_sum(got, want, np.cumsum(np.abs(v), axis=0) / np.arange(1, lq + 1)[:, None], "prefix mean")
    # Empty shapes.
    assert O.attention(np.zeros((2, 0, w), np.float32), np.zeros((2, 3, w), np.float32),
                       np.zeros((2, 3, w), np.float32), heads).shape == (2, 0, w)
    # No keys: every sum is empty, the outputs are zero.
    assert not O.attention(q[None], np.zeros((1, 0, w), np.float32), np.zeros((1, 0, w), np.float32),
                           heads).any()


def _fails(fn):
    try:
        fn()
    except AssertionError:
        return True
    return False


def test_planted_mistakes_are_caught():
    """Mistakes planted in the restatement's inputs or arguments (on the CPU)
    fail the float64 check: the check is strong enough to see each one."""
    rng = np.random.default_rng(11)
    b, l, heads, hd = 2, 40, 2, 16
    w = heads * hd
    q, k, v = (rng.standard_normal((b, l, w)).astype(np.float32) for _ in range(3))
    want, mag, cond = attention64(q, k, v, heads, True, O.attention_scale(hd))
    check = lambda got: assert_attention_close(got, want, mag, cond, "planted")  # noqa: E731
    check(O.attention(q, k, v, heads, True))  # the unplanted restatement passes
    assert _fails(lambda: check(O.attention(q, k, v, heads, True, scale=1.0)))          # scale dropped
    assert _fails(lambda: check(O.attention(q, k, v, heads, False)))                    # mask dropped
    rev = O.attention(q[:, ::-1], k[:, ::-1], v[:, ::-1], heads, True)[:, ::-1]         # mask reversed
    assert _fails(lambda: check(rev))
    assert _fails(lambda: check(O.attention(q, v, k, heads, True)))                     # K and V swapped
    assert _fails(lambda: check(O.attention(q, np.roll(k, 1, axis=2), v, heads, True)))  # head columns shifted


def test_oracle_reproduces_golden_fixture():
    """tests/golden/attention.npz (the reference's outputs, written by
    tests/golden/make_golden.py): the restatement reproduces them bit for bit
    where the reference tree is absent."""
    import os
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "attention.npz")
    with np.load(path) as z:
        gold = {k: z[k] for k in z.files}
    n = 0
    for seq, e, heads in SELF_CASES:
        _, _, q, k, v = self_case(seq, e, 1.5, seq * 1000 + e)
        for causal in (0, 1):
            assert_bitexact(O.attention(q, k, v, heads, bool(causal)), gold[f"self_{seq}_{e}_{heads}_{causal}"])
            n += 1
    for lq, lk, e, heads in CROSS_CASES:
        _, _, _, _, q, k, v = cross_case(lq, lk, e, 1.2, lq * 7 + lk)
        for causal in (0, 1):
            got = O.attention(q[None], k[None], v[None], heads, bool(causal))[0]
            assert_bitexact(got, gold[f"cross_{lq}_{lk}_{e}_{heads}_{causal}"])
            n += 1
    assert n == len(gold)


@needs_ref
@pytest.mark.parametrize("seq,e,heads", [(50, 64, 4), (130, 96, 3), (64, 128, 1)])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("amp", [1.0, 2.5])
def test_layer_tolerance_model(seq, e, heads, causal, amp):
    """The whole-layer tolerance (projections, core, output projection; see
    tests/_attention.py attention_layer64): the compiled reference's own
    self_attention_forward with random weights stays within a quarter of it
    against float64, and a planted mistake (no 1/sqrt(d) scale) does not."""
    from _attention import assert_within, attention_layer64, layer_case
    x, w = layer_case(seq, e, seq * 3 + e, amp)
    wqkv, wout = w[:3 * e * e].reshape(e, 3 * e), w[3 * e * e:].reshape(e, e)
    want, tol = attention_layer64(x, wqkv, wout, heads, causal)
    ref = O.ref_self_attention(x, wqkv, wout, seq, e, heads, causal)
    assert_within(ref, want, tol / 4, "reference vs float64")
    qkv = x.astype(np.float64) @ wqkv
    att = O.attention(qkv[:, :e], qkv[:, e:2 * e], qkv[:, 2 * e:], heads, causal, scale=1.0)
    with pytest.raises(AssertionError):
        assert_within(att.astype(np.float64) @ wout, want, tol, "no scale")


@needs_ref
@pytest.mark.parametrize("causal", [False, True])
def test_cross_layer_tolerance_model(causal):
    from _attention import assert_within, cross_attention_layer64
    r = np.random.default_rng(4)
    lq, lk, e, heads = 37, 90, 64, 4
    xq = r.standard_normal((lq, e)).astype(np.float32)
    xkv = r.standard_normal((lk, e)).astype(np.float32)
    wq, wkv, wout = ((r.standard_normal(s) / np.sqrt(e)).astype(np.float32) for s in ((e, e), (e, 2 * e), (e, e)))
    want, tol = cross_attention_layer64(xq, xkv, wq, wkv, wout, heads, causal)
    ref = O.ref_cross_attention(xq, xkv, wq, wkv, wout, lq, lk, e, heads, causal)
    assert_within(ref, want, tol / 4, "reference vs float64")
