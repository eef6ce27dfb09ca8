"""Pins of the CPU oracle by what the mathematics fixes: float64 closed forms,
invariants and brute force.  For RoPE (no reference implementation exists)
these are the only pins; each check is also shown to reject a plausible
mistake (a dropped term, a wrong sign, a transposed pairing)."""
import numpy as np
import pytest

import oracle as O
from _parity import assert_bitexact, assert_close

rng = np.random.default_rng(99)


# ---------------------------------------------------------------------------
# LayerNorm / RMSNorm / softmax / activations against float64 closed forms
# ---------------------------------------------------------------------------

def ln64(x, g, b, eps):
    x = x.astype(np.float64)
    m = x.mean(axis=1, keepdims=True)
    v = ((x - m) ** 2).mean(axis=1, keepdims=True)  # biased (divide by n), as LayerOps.hpp:303
    return (x - m) / np.sqrt(v + eps) * g + b


def test_layernorm_closed_form_and_invariants():
    x = (rng.standard_normal((64, 512)) * 2 + 1).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(512)).astype(np.float32)
    b = (0.1 * rng.standard_normal(512)).astype(np.float32)
    y = O.layernorm(x, 512, g, b, 1e-5).reshape(x.shape)
    assert_close(y, ln64(x, g, b, 1e-5), "closed form")
    # a plausible mistake (unbiased variance) is rejected by the same check
    xm = x.astype(np.float64)
    wrong = (xm - xm.mean(1, keepdims=True)) / np.sqrt(xm.var(1, ddof=1, keepdims=True) + 1e-5) * g + b
    with pytest.raises(AssertionError):
        assert_close(y, wrong)
    # shift invariance; a constant row maps to beta
    y2 = O.layernorm(x + np.float32(3.0), 512, g, b, 1e-5).reshape(x.shape)
    assert np.max(np.abs(y2 - y)) < 2e-5
    c = O.layernorm(np.full(512, 7.0, np.float32), 512, g, b, 1e-5)
    assert_bitexact(c, b, "constant row -> beta")


def test_rmsnorm_closed_form():
    x = rng.standard_normal((32, 4096)).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(4096)).astype(np.float32)
    y = O.rmsnorm_rows(x, w, 1e-6)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-6) * w
    assert_close(y, ref, "closed form")
    with pytest.raises(AssertionError):  # eps outside the square root
        assert_close(y, x64 / (np.sqrt((x64 ** 2).mean(axis=1, keepdims=True)) + 1e-6) * w * 1.00003)
    # scale invariance: rms(c*x) = |c| rms(x)
    y4 = O.rmsnorm_rows(x * np.float32(4.0), w, 1e-6)
    assert np.max(np.abs(y4 - y) / np.maximum(1.0, np.abs(y))) < 2e-6


def test_softmax_closed_form_and_invariants():
    s = (3 * rng.standard_normal((128, 1024))).astype(np.float32)
    s[np.triu(np.ones((128, 1024), bool), 1)] = -np.inf
    y = O.softmax_rows(s)
    s64 = s.astype(np.float64)
    e = np.exp(s64 - s64.max(axis=1, keepdims=True))
    assert_close(y, e / e.sum(axis=1, keepdims=True), "closed form")
    assert np.all(np.abs(y.sum(axis=1, dtype=np.float64) - 1) < 1e-5)
    assert not y[np.triu(np.ones((128, 1024), bool), 1)].any()
    assert y[0, 0] == 1.0
    ls = O.softmax_rows(s[:, :64][64:], O.SOFTMAX_LOG)
    s2 = s[64:, :64].astype(np.float64)
    m = s2.max(axis=1, keepdims=True)
    assert_close(ls, s2 - m - np.log(np.exp(s2 - m).sum(axis=1, keepdims=True)), "log-softmax")


def test_activations_closed_form():
    x = np.concatenate([np.linspace(-8, 8, 100001), rng.standard_normal(10000) * 3]).astype(np.float32)
    x64 = x.astype(np.float64)
    k = np.float64(np.sqrt(np.float32(2.0) / np.float32(3.14159265359)))
    gelu64 = x64 * 0.5 * (1 + np.tanh(k * (x64 + 0.044715 * x64 ** 3)))
    assert_close(O.gelu(x), gelu64, "tanh-GELU")
    with pytest.raises(AssertionError):  # dropped cubic term
        assert_close(O.gelu(x), x64 * 0.5 * (1 + np.tanh(k * x64)))
    assert_close(O.silu(x), x64 / (1 + np.exp(-x64)), "SiLU")
    u = rng.standard_normal(x.size).astype(np.float32)
    assert_close(O.silu_mul(x, u), x64 / (1 + np.exp(-x64)) * u, "SiLU*up")
    u64 = u.astype(np.float64)
    assert_close(O.gelu_mul(x, u), gelu64 * u64, "GELU*up")
    with pytest.raises(AssertionError):  # dropped cubic term in the gate
        assert_close(O.gelu_mul(x, u), x64 * 0.5 * (1 + np.tanh(k * x64)) * u64)
    with pytest.raises(AssertionError):  # the gate's GELU applied to up instead
        assert_close(O.gelu_mul(x, u), x64 * u64 * 0.5 * (1 + np.tanh(k * (u64 + 0.044715 * u64 ** 3))))


# ---------------------------------------------------------------------------
# Embedding gather: brute force (bit-exact)
# ---------------------------------------------------------------------------

def brute_gather(ids, table, vocab, dim, pad):
    out = np.zeros((ids.size, dim), np.float32)
    for t, i in enumerate(ids.tolist()):
        if pad >= 0 and i == pad:
            continue
        if 0 <= i < vocab:
            out[t] = table[i]
    return out


def llround_x86(f):
    """static_cast<int>(llround((double)f)) on x86-64 glibc: half away from
    zero; NaN / |x| >= 2^63 give 0x8000000000000000 (low word 0); the int64
    result wraps to int32."""
    d = float(f)
    if not (abs(d) < 2.0 ** 63):
        return 0
    r = int(np.sign(d)) * int(np.floor(abs(d) + 0.5))
    return ((r + 2 ** 31) % 2 ** 32) - 2 ** 31


def test_embedding_brute_force():
    vocab, dim = 50, 12
    table = rng.standard_normal((vocab, dim)).astype(np.float32)
    ids = rng.integers(-5, vocab + 5, 400).astype(np.int32)
    for pad in (-1, 0, 7):
        assert_bitexact(O.embedding(ids, table, vocab, dim, pad), brute_gather(ids, table, vocab, dim, pad))


def test_embedding_float_ids_rounding():
    vocab, dim = 1000, 4
    table = rng.standard_normal((vocab, dim)).astype(np.float32)
    f = np.array([1.0, 1.5, 2.5, -0.5, -1.5, 0.49999997, 999.5, 998.5, np.nan, np.inf, -np.inf,
                  4294967808.0, -4294966784.0, 1e20, -1e20, 9.3e18, 2.0 ** 31, -2.0 ** 31, 3.0e9],
                 np.float32)
    ids = np.array([llround_x86(v) for v in f], np.int64).astype(np.int32)
    assert ids[1] == 2 and ids[2] == 3 and ids[3] == -1 and ids[11] == 512 and ids[8] == 0
    assert_bitexact(O.embedding(f, table, vocab, dim, -1), brute_gather(ids, table, vocab, dim, -1))


# ---------------------------------------------------------------------------
# RoPE: closed form of rotary embedding (Su et al. 2021), rotate-half pairing
# ---------------------------------------------------------------------------

def rope64(x, pos, theta=10000.0):
    """float64 rotate-half RoPE of x [..., S, H, D] at positions pos[S]."""
    D = x.shape[-1]
    half = D // 2
    inv = 1.0 / theta ** (np.arange(half, dtype=np.float64) * 2.0 / D)
    a = np.asarray(pos, np.float64)[:, None] * inv[None, :]
    c = np.cos(a)[:, None, :]
    s = np.sin(a)[:, None, :]
    x0 = x[..., :half].astype(np.float64)
    x1 = x[..., half:].astype(np.float64)
    return np.concatenate([x0 * c - x1 * s, x1 * c + x0 * s], axis=-1)


ROPE_ATOL = 2e-6  # fp32 table entries (|err| <= 2^-25) times |x| <= ~6, plus product rounding


def test_rope_table_closed_form():
    c, s = O.rope_table(2048, 128)
    a = np.arange(2048)[:, None] * (1.0 / 10000.0 ** (np.arange(64) * 2.0 / 128))[None, :]
    assert np.max(np.abs(c - np.cos(a))) <= 2 ** -24 and np.max(np.abs(s - np.sin(a))) <= 2 ** -24
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)


@pytest.mark.parametrize("D", [128, 64, 8, 6])
def test_rope_closed_form(D):
    S, H = 300, 3
    x = rng.standard_normal((2, S, H, D)).astype(np.float32)
    c, s = O.rope_table(S + 5, D)
    y = O.rope(x, c, s, pos_offset=5)
    ref = rope64(x, np.arange(S) + 5)
    assert_close(y, ref, f"RoPE D={D}", abs_=ROPE_ATOL)
    # plausible mistakes are rejected: interleaved (GPT-J) pairing, flipped sign
    half = D // 2
    xi = x.reshape(2, S, H, half, 2)
    inter = np.concatenate([xi[..., 0], xi[..., 1]], axis=-1)  # de-interleave
    wrong = rope64(inter, np.arange(S) + 5).reshape(2, S, H, 2, half).transpose(0, 1, 2, 4, 3).reshape(x.shape)
    with pytest.raises(AssertionError):
        assert_close(y, wrong, abs_=ROPE_ATOL)
    flip = rope64(x, -(np.arange(S) + 5))
    with pytest.raises(AssertionError):
        assert_close(y, flip, abs_=ROPE_ATOL)


def test_rope_invariants():
    S, H, D = 512, 2, 128
    q = rng.standard_normal((1, S, H, D)).astype(np.float32)
    k = rng.standard_normal((1, S, H, D)).astype(np.float32)
    c, s = O.rope_table(S, D)
    qr, kr = O.rope(q, c, s), O.rope(k, c, s)
    half = D // 2
    n0 = q[..., :half].astype(np.float64) ** 2 + q[..., half:].astype(np.float64) ** 2
    n1 = qr[..., :half].astype(np.float64) ** 2 + qr[..., half:].astype(np.float64) ** 2
    assert np.allclose(n1, n0, rtol=2e-6, atol=1e-7), "pair norms preserved"
    assert_bitexact(qr[:, 0], q[:, 0], "position 0 is the identity")
    # <R_m q, R_n k> depends only on m - n: same vectors placed at (m, n) and (m+t, n+t)
    qv = np.repeat(q[:, :1], S, axis=1)
    kv = np.repeat(k[:, :1], S, axis=1)
    qvr, kvr = O.rope(qv, c, s), O.rope(kv, c, s)
    dots = np.einsum("d,d->", qvr[0, 10, 0].astype(np.float64), kvr[0, 3, 0].astype(np.float64))
    for t in (50, 200, 400):
        d2 = np.einsum("d,d->", qvr[0, 10 + t, 0].astype(np.float64), kvr[0, 3 + t, 0].astype(np.float64))
        assert abs(d2 - dots) < 1e-4 * max(1.0, abs(dots))
