"""The fused attention core (mimir_attention_fwd, csrc/attention.hip) against
the CPU restatement (oracle_attention, pinned bit-exact to the reference's
compiled self_attention_forward / cross_attention_forward) and float64
softmax attention, on the same seeded inputs; against the reference's own
outputs stored in tests/golden/attention.npz; and, at the benchmark's full
size, through properties that do not need the oracle's O(L^2) loops on every
head.

Tolerance (floating point): the output is a float32 weighted sum over
float32 scores, so each element is held to
  |gpu - ref| <= max(1e-6, 1e-5 * max(|ref|, sum_j p_j |v_j|)) + cond,
cond = the propagated rounding of the float32 scores (tests/_attention.py
attention64), against float64 and against the oracle.
"""
import os

import numpy as np
import pytest

import mimir_hip as M
import oracle as O
from _attention import CROSS_CASES, SELF_CASES, assert_attention_close, attention64, cross_case, self_case
from _parity import assert_bitexact, assert_close_sum

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def gpu_attention(ctx, q, k, v, heads, causal, scale=None, offset=0, fused=False):
    """Run mimir_attention_fwd on [batch, len, width] arrays.  offset: the
    buffers start `offset` floats in (the unaligned path); fused: q / k / v
    are the column blocks of one [batch*len, 3*width] buffer (needs
    q_len == kv_len)."""
    b, lq, w = q.shape
    lk = k.shape[1]
    hd = w // heads
    out = np.empty((b, lq, w), np.float32)
    bufs = []
    try:
        if fused:
            assert lq == lk
            qkv = np.concatenate([q, k, v], axis=2).reshape(b * lq, 3 * w)
            buf = ctx.empty(qkv.size + offset)
            bufs.append(buf)
            ctx.upload(buf.offset(offset, qkv.shape), qkv)
            dq, dk, dv = (buf.offset(offset + i * w) for i in range(3))
            ld_in = (3 * w, 3 * w)
        else:
            views = []
            for a in (q, k, v):
                buf = ctx.empty(a.size + offset)
                bufs.append(buf)
                view = buf.offset(offset, a.shape)
                ctx.upload(view, np.ascontiguousarray(a))
                views.append(view)
            dq, dk, dv = views
            ld_in = (w, w)
        ybuf = ctx.empty(max(out.size + offset, 1))
        bufs.append(ybuf)
        y = ybuf.offset(offset, out.shape)
        ctx.attention(dq, dk, dv, y, b, lq, lk, heads, hd, causal, scale, ld_q=ld_in[0], ld_kv=ld_in[1])
        if out.size:
            ctx.download(out, y)
        return out
    finally:
        for buf in bufs:
            buf.free()


def check(got, q, k, v, heads, causal, what, oracle=True):
    hd = q.shape[2] // heads
    want, mag, cond = attention64(q, k, v, heads, causal, O.attention_scale(hd))
    assert_attention_close(got, want, mag, cond, what + " vs float64")
    if oracle:
        # Both sides carry their own score rounding: twice the term.
        assert_attention_close(got, O.attention(q, k, v, heads, causal), mag, 2 * cond, what + " vs oracle")


def rand_qkv(seed, b, lq, lk, w, amp=1.0):
    r = np.random.default_rng(seed)
    q = (amp * r.standard_normal((b, lq, w))).astype(np.float32)
    k = (amp * r.standard_normal((b, lk, w))).astype(np.float32)
    v = r.standard_normal((b, lk, w)).astype(np.float32)
    return q, k, v


SHAPES = [  # (batch, q_len, kv_len, heads, head_dim)
    (1, 1, 1, 1, 4), (1, 5, 5, 1, 8), (2, 31, 31, 2, 16), (1, 32, 32, 1, 32), (2, 33, 33, 3, 32),
    (1, 127, 127, 2, 64), (1, 128, 128, 1, 128), (2, 129, 129, 2, 128), (1, 200, 200, 4, 48),
    (3, 70, 70, 2, 96), (1, 300, 300, 1, 80), (2, 257, 257, 2, 24),
    # cross attention: q_len != kv_len, both orders
    (2, 40, 100, 2, 64), (1, 150, 33, 1, 128), (1, 1, 300, 2, 32), (2, 200, 1, 1, 16),
]


@pytest.mark.parametrize("b,lq,lk,heads,hd", SHAPES)
@pytest.mark.parametrize("causal", [False, True])
def test_attention_matches_oracle(ctx, b, lq, lk, heads, hd, causal):
    q, k, v = rand_qkv(b * 1009 + lq * 31 + lk + hd, b, lq, lk, heads * hd, amp=1.5)
    print(f"attention b={b} lq={lq} lk={lk} h={heads} d={hd} causal={causal}", flush=True)
    check(gpu_attention(ctx, q, k, v, heads, causal), q, k, v, heads, causal, f"{b}x{lq}x{lk} h{heads} d{hd}")


@pytest.mark.parametrize("b,l,heads,hd", [(1, 64, 2, 32), (2, 130, 4, 128), (1, 100, 3, 64)])
@pytest.mark.parametrize("causal", [False, True])
def test_fused_qkv_buffer(ctx, b, l, heads, hd, causal):
    """q / k / v as the column blocks of one [T, 3E] QKV buffer (the layout of
    the reference's qkv projection output, LayerOps.hpp:1031-1043)."""
    q, k, v = rand_qkv(l + hd, b, l, l, heads * hd)
    print(f"attention fused b={b} l={l} h={heads} d={hd} causal={causal}", flush=True)
    check(gpu_attention(ctx, q, k, v, heads, causal, fused=True), q, k, v, heads, causal, "fused")


@pytest.mark.parametrize("b,lq,lk,heads,hd,offset", [(1, 40, 40, 2, 5, 0), (2, 33, 70, 1, 7, 0),
                                                      (1, 64, 64, 2, 30, 0), (1, 50, 50, 2, 32, 1),
                                                      (2, 129, 129, 1, 128, 3), (1, 20, 20, 3, 1, 0)])
@pytest.mark.parametrize("causal", [False, True])
def test_scalar_path(ctx, b, lq, lk, heads, hd, offset, causal):
    """Head sizes that are not multiples of 4, or buffers not 16-byte aligned:
    the kernel's scalar-load path."""
    q, k, v = rand_qkv(hd * 7 + offset, b, lq, lk, heads * hd)
    print(f"attention scalar b={b} lq={lq} lk={lk} h={heads} d={hd} off={offset} causal={causal}", flush=True)
    check(gpu_attention(ctx, q, k, v, heads, causal, offset=offset), q, k, v, heads, causal, "scalar path")


def test_golden_reference_outputs(ctx):
    """The reference's own outputs (one-hot inputs, identity output projection)."""
    with np.load(os.path.join(GOLD, "attention.npz")) as z:
        gold = {k: z[k] for k in z.files}
    for seq, e, heads in SELF_CASES:
        _, _, q, k, v = self_case(seq, e, 1.5, seq * 1000 + e)
        for causal in (0, 1):
            ref = gold[f"self_{seq}_{e}_{heads}_{causal}"]
            got = gpu_attention(ctx, q[None], k[None], v[None], heads, bool(causal))[0]
            _, mag, cond = attention64(q, k, v, heads, bool(causal), O.attention_scale(e // heads))
            assert_attention_close(got, ref, mag, 2 * cond, f"golden self {seq}x{e} h{heads} causal={causal}")
    for lq, lk, e, heads in CROSS_CASES:
        _, _, _, _, q, k, v = cross_case(lq, lk, e, 1.2, lq * 7 + lk)
        for causal in (0, 1):
            ref = gold[f"cross_{lq}_{lk}_{e}_{heads}_{causal}"]
            got = gpu_attention(ctx, q[None], k[None], v[None], heads, bool(causal))[0]
            _, mag, cond = attention64(q, k, v, heads, bool(causal), O.attention_scale(e // heads))
            assert_attention_close(got, ref, mag, 2 * cond, f"golden cross {lq}x{lk} causal={causal}")


def test_sharp_and_flat_softmax(ctx):
    """Large score ranges (one key dominates) and equal scores (uniform weights)."""
    q, k, v = rand_qkv(99, 2, 150, 150, 128, amp=6.0)  # scores up to about +-50
    check(gpu_attention(ctx, q, k, v, 1, True), q, k, v, 1, True, "sharp")
    z = np.zeros_like(k)
    got = gpu_attention(ctx, q, z, v, 2, True)
    check(got, q, z, v, 2, True, "zero keys")
    prefix = np.cumsum(v.astype(np.float64), axis=1) / np.arange(1, 151)[None, :, None]
    assert_close_sum(got, prefix, np.cumsum(np.abs(v), axis=1) / np.arange(1, 151)[None, :, None], "prefix mean")


def test_explicit_scale(ctx):
    """A caller-chosen scale (Model::computeAttention's AVX path applies none,
    Model.cpp:4236-4239)."""
    q, k, v = rand_qkv(5, 1, 96, 96, 64, amp=0.3)
    got = gpu_attention(ctx, q, k, v, 1, False, scale=1.0)
    want, mag, cond = attention64(q, k, v, 1, False, 1.0)
    assert_attention_close(got, want, mag, cond, "scale 1")
    assert_attention_close(got, O.attention(q, k, v, 1, False, scale=1.0), mag, 2 * cond, "scale 1 vs oracle")


def test_empty_shapes_and_no_keys(ctx):
    w = 64
    assert gpu_attention(ctx, *rand_qkv(1, 2, 0, 5, w), heads=2, causal=False).shape == (2, 0, w)
    q = np.random.default_rng(2).standard_normal((2, 17, w)).astype(np.float32)
    e = np.zeros((2, 0, w), np.float32)
    got = gpu_attention(ctx, q, e, e, 2, False)
    assert_bitexact(got, np.zeros_like(q), "no keys")  # sum = 0: 0 * (1 / 1e-9)


def test_invalid_arguments(ctx):
    q = ctx.empty(1024)
    try:
        with pytest.raises(M.MimirError, match="head_dim"):
            ctx.attention(q, q, q, q, 1, 2, 2, 1, 4096)
        with pytest.raises(M.MimirError, match="row strides"):
            ctx.attention(q, q, q, q, 1, 2, 2, 2, 16, ld_q=16)
        with pytest.raises(M.MimirError, match="invalid shape"):
            ctx.attention(q, q, q, q, 1, 2, 2, 0, 16)
    finally:
        q.free()


def test_full_size_properties(ctx):
    """The benchmark workload (8 sequences x 32 heads x 1024 tokens, head_dim
    128, causal) as one launch: the oracle on a sample of (sequence, head)
    pairs, and for every pair the first query's output, which is V's first
    row exactly (one visible key: p = 1 * (1 / (1 + 1e-9f)) = 1)."""
    b, l, heads, hd = 8, 1024, 32, 128
    w = heads * hd
    r = np.random.default_rng(2024)
    q, k, v = (r.standard_normal((b, l, w), dtype=np.float32) for _ in range(3))
    print("attention full size", flush=True)
    got = gpu_attention(ctx, q, k, v, heads, True, fused=True)
    assert_bitexact(got[:, 0], v[:, 0], "first query of every head")
    for bi, h in [(0, 0), (3, 17), (7, 31)]:
        sl = slice(h * hd, (h + 1) * hd)
        qs, ks, vs = (np.ascontiguousarray(a[bi:bi + 1, :, sl]) for a in (q, k, v))
        want, mag, cond = attention64(qs, ks, vs, 1, True, O.attention_scale(hd))
        assert_attention_close(got[bi:bi + 1, :, sl], want, mag, cond, f"full size b{bi} h{h} vs float64")
        assert_attention_close(got[bi:bi + 1, :, sl], O.attention(qs, ks, vs, 1, True), mag, 2 * cond,
                               f"b{bi} h{h} vs oracle")


@pytest.mark.parametrize("seq,e,heads", [(1, 16, 2), (50, 64, 4), (130, 96, 3), (64, 128, 1), (300, 256, 2)])
@pytest.mark.parametrize("causal", [False, True])
def test_self_attention_layer(ctx, seq, e, heads, causal):
    """mimir_self_attention_fwd (projections + fused core) against the
    compiled reference's self_attention_forward with random weights and
    float64, under the whole-layer tolerance (tests/_attention.py)."""
    from _attention import assert_within, attention_layer64, layer_case
    x, w = layer_case(seq, e, seq * 7 + e, 1.5)
    wqkv, wout = w[:3 * e * e].reshape(e, 3 * e), w[3 * e * e:].reshape(e, e)
    print(f"self attention layer seq={seq} e={e} h={heads} causal={causal}", flush=True)
    dx, dw, dy = ctx.to_device(x), ctx.to_device(w), ctx.empty((seq, e))
    try:
        ctx.self_attention(dx, seq, e, heads, causal, dw, w.size, dy)
        got = dy.numpy()
    finally:
        for d in (dx, dw, dy):
            d.free()
    want, tol = attention_layer64(x, wqkv, wout, heads, causal)
    assert_within(got, want, tol, "layer vs float64")
    assert_within(got, O.ref_self_attention(x, wqkv, wout, seq, e, heads, causal), 2 * tol, "layer vs reference")


@pytest.mark.parametrize("lq,lk,e,heads", [(37, 90, 64, 4), (200, 33, 128, 2), (1, 1, 32, 1)])
@pytest.mark.parametrize("causal", [False, True])
def test_cross_attention_layer(ctx, lq, lk, e, heads, causal):
    from _attention import assert_within, cross_attention_layer64
    r = np.random.default_rng(lq + lk + e)
    xq = r.standard_normal((lq, e)).astype(np.float32)
    xkv = r.standard_normal((lk, e)).astype(np.float32)
    wq, wkv, wout = ((r.standard_normal(s) / np.sqrt(e)).astype(np.float32) for s in ((e, e), (e, 2 * e), (e, e)))
    w = np.concatenate([wq.ravel(), wkv.ravel(), wout.ravel()])
    print(f"cross attention layer lq={lq} lk={lk} e={e} h={heads} causal={causal}", flush=True)
    dq, dkv, dw, dy = ctx.to_device(xq), ctx.to_device(xkv), ctx.to_device(w), ctx.empty((lq, e))
    try:
        ctx.cross_attention(dq, lq, dkv, lk, e, heads, causal, dw, w.size, dy)
        got = dy.numpy()
    finally:
        for d in (dq, dkv, dw, dy):
            d.free()
    want, tol = cross_attention_layer64(xq, xkv, wq, wkv, wout, heads, causal)
    assert_within(got, want, tol, "cross layer vs float64")
    assert_within(got, O.ref_cross_attention(xq, xkv, wq, wkv, wout, lq, lk, e, heads, causal), 2 * tol,
                  "cross layer vs reference")


def test_attention_layer_refusals(ctx):
    b = ctx.empty(4096)
    try:
        with pytest.raises(M.MimirError, match="divisible by num_heads"):
            ctx.self_attention(b, 4, 12, 5, False, b, 4096, b)
        with pytest.raises(M.MimirError, match="weight block"):
            ctx.self_attention(b, 4, 16, 2, False, b, 4 * 16 * 16 - 1, b)
        with pytest.raises(M.MimirError, match="invalid dimensions"):
            ctx.cross_attention(b, 0, b, 3, 16, 2, False, b, 4096, b)
    finally:
        b.free()


@pytest.mark.parametrize("b,lq,lk,heads,hd", [(1, 40, 40, 2, 160), (2, 33, 70, 1, 256), (1, 20, 20, 1, 200),
                                               (1, 9, 9, 2, 512), (1, 5, 7, 1, 1000)])
@pytest.mark.parametrize("causal", [False, True])
def test_wide_heads(ctx, b, lq, lk, heads, hd, causal):
    """Heads wider than 128 (the plain fp32 vector kernel): the reference
    accepts any head size."""
    q, k, v = rand_qkv(hd + lq, b, lq, lk, heads * hd)
    print(f"attention wide b={b} lq={lq} lk={lk} h={heads} d={hd} causal={causal}", flush=True)
    check(gpu_attention(ctx, q, k, v, heads, causal), q, k, v, heads, causal, f"wide d{hd}")
