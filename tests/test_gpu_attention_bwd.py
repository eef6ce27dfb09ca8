"""The attention backward on the GPU (csrc/attention_bwd.hip):
mimir_attention_bwd (the per-head core of backward_self_attention /
backward_cross_attention, Model.cpp:6892-7028, 7122-7246), the layer forms
mimir_self_attention_bwd / mimir_cross_attention_bwd, and the device
runtime's SelfAttention / MultiHeadAttention / CrossAttention branches of
mimir_store_backward (Model.cpp:8034-8130), against the float64 model
(tests/_attention.attention_bwd64 and its layer forms), the CPU restatement
oracle_attention_bwd (bit-exact to the reference's Model::backwardPass,
tests/test_oracle_attention_bwd.py) and the reference's own compiled
Model::backwardPass, on the same seeded inputs.

Tolerance (floating point; assert_bwd_close): element-wise, the float64
model's first-order bound -- 1e-5 of each product's summed magnitudes,
carried through the softmax, its backward and the projections -- and
normwise, relative error <= 1e-5.  Against the oracle or the reference
(each with its own rounding) both are doubled.  At the benchmark's size the
oracle's O(L^2) loops run on two heads; every head is held to two exact
consequences of softmax: the key-sum of dK is 0 (the rows of dS sum to 0)
and the key-sum of dV is the query-sum of dout (the rows of P sum to 1)."""
import os

import numpy as np
import pytest

import mimir_hip as M
import model_ref as MR
import oracle as O
from _attention import (NORM_REL, assert_bwd_close, attention_bwd64, cross_attention_bwd64, layer_case,
                        self_attention_bwd64)
from _attention_graphs import block_graph
from _parity import assert_close_normwise

pytestmark = pytest.mark.gpu


def _dev(ctx, a):
    a = np.ascontiguousarray(a, np.float32)
    d = ctx.empty(max(a.size, 1))
    if a.size:
        ctx.upload(d, a)
    return d


def gpu_core_bwd(ctx, q, k, v, dout, heads, causal, fused=False, scale=None):
    """mimir_attention_bwd on [batch, len, width] arrays; fused: q / k / v and
    dq / dk / dv are the column blocks of [batch*len, 3*width] buffers."""
    b, lq, w = q.shape
    lk = k.shape[1]
    hd = w // heads
    bufs = []
    try:
        if fused:
            assert lq == lk
            qkv = _dev(ctx, np.concatenate([q, k, v], axis=2))
            g = _dev(ctx, np.full((b, lq, 3 * w), np.nan, np.float32))
            bufs += [qkv, g]
            ins = (qkv, qkv.offset(w), qkv.offset(2 * w))
            outs = (g, g.offset(w), g.offset(2 * w))
            ld_in = ld_out = 3 * w
        else:
            ins = tuple(_dev(ctx, a) for a in (q, k, v))
            outs = tuple(_dev(ctx, np.full(a.shape, np.nan, np.float32)) for a in (q, k, v))
            bufs += list(ins) + list(outs)
            ld_in = ld_out = w
        do = _dev(ctx, dout)
        bufs.append(do)
        ctx.attention_bwd(ins[0], ins[1], ins[2], do, outs[0], outs[1], outs[2], b, lq, lk, heads, hd, causal,
                          scale, ld_q=ld_in, ld_kv=ld_in, ld_dout=w, ld_dq=ld_out, ld_dkv=ld_out)
        if fused:
            full = np.empty((b, lq, 3 * w), np.float32)
            ctx.download(full, g)
            return full[..., :w].copy(), full[..., w:2 * w].copy(), full[..., 2 * w:].copy()
        res = []
        for o, a in zip(outs, (q, k, v)):
            r = np.empty(a.shape, np.float32)
            if r.size:
                ctx.download(r, o)
            res.append(r)
        return tuple(res)
    finally:
        for d in bufs:
            d.free()


def rand_core(seed, b, lq, lk, w, amp=1.0):
    r = np.random.default_rng(seed)
    q, k, v = ((amp * r.standard_normal(s)).astype(np.float32) for s in ((b, lq, w), (b, lk, w), (b, lk, w)))
    return q, k, v, r.standard_normal((b, lq, w)).astype(np.float32)


def check_core(got, q, k, v, dout, heads, causal, what, oracle=True):
    hd = q.shape[2] // heads
    ref = O.attention_bwd(q, k, v, dout, heads, causal) if oracle else None
    for bi in range(q.shape[0]):
        want, tol = attention_bwd64(q[bi], k[bi], v[bi], dout[bi], heads, causal, O.attention_scale(hd))
        for j, name in enumerate(("dq", "dk", "dv")):
            assert_bwd_close(got[j][bi], want[j], tol[j], f"{what} {name}[{bi}] vs float64")
            if oracle:
                assert_bwd_close(got[j][bi], ref[j][bi], 2 * tol[j], f"{what} {name}[{bi}] vs oracle",
                                 2 * NORM_REL)


# (batch, q_len, kv_len, heads, head_dim, causal, amp): the softmax kernels'
# register forms (kv_len <= 256, <= 1024, <= 4096) and the streamed form
# (> 4096), self and cross shapes, causal rows past the last key, head_dim
# above 128.
CORE = [(1, 64, 64, 2, 32, True, 1.0), (1, 64, 64, 2, 32, False, 1.0), (3, 33, 33, 3, 20, True, 1.0),
        (1, 37, 90, 4, 16, False, 1.0), (1, 90, 37, 1, 64, True, 2.0), (1, 128, 128, 1, 128, True, 3.0),
        (1, 300, 300, 2, 48, True, 1.0), (1, 17, 1500, 2, 40, False, 1.0), (1, 5, 5000, 1, 32, True, 1.0),
        (1, 5, 5000, 1, 32, False, 1.0), (1, 1, 1, 1, 8, True, 1.0), (1, 1, 7, 3, 8, False, 1.0),
        (2, 257, 257, 1, 200, True, 1.0),
        # longer causal rows and cross shapes with keys past every query
        (1, 600, 600, 2, 32, True, 1.0), (1, 1000, 1000, 1, 64, True, 1.0), (1, 700, 300, 1, 32, True, 1.0),
        (1, 300, 700, 1, 32, True, 1.0), (2, 520, 520, 2, 16, True, 2.0),
        # odd head sizes: row strides and head offsets that are not 16-byte multiples
        (1, 45, 45, 3, 5, True, 1.0), (2, 33, 50, 2, 7, False, 1.0), (1, 260, 260, 2, 13, True, 1.0)]


@pytest.mark.parametrize("case", CORE, ids=lambda c: "x".join(map(str, c[:6])))
def test_core_backward(ctx, case):
    b, lq, lk, heads, hd, causal, amp = case
    print(f"attention_bwd core {case}", flush=True)
    q, k, v, dout = rand_core(lq * 7 + lk + hd, b, lq, lk, heads * hd, amp)
    check_core(gpu_core_bwd(ctx, q, k, v, dout, heads, causal), q, k, v, dout, heads, causal, str(case))


@pytest.mark.parametrize("causal", [False, True])
def test_core_backward_fused_layout(ctx, causal):
    """Q / K / V and dQ / dK / dV as the column blocks of one [rows, 3E]
    buffer each, the layout of the layers' qkv and dqkv."""
    q, k, v, dout = rand_core(11, 2, 70, 70, 4 * 32, 1.0)
    check_core(gpu_core_bwd(ctx, q, k, v, dout, 4, causal, fused=True), q, k, v, dout, 4, causal, "fused")


def _tuned_context(tune):
    old = os.environ.get("MIMIR_TUNE")
    os.environ["MIMIR_TUNE"] = tune
    try:
        return M.Context(0)
    finally:
        if old is None:
            del os.environ["MIMIR_TUNE"]
        else:
            os.environ["MIMIR_TUNE"] = old


@pytest.mark.parametrize("group", [1, 2])
def test_core_backward_head_groups(group):
    """Heads processed in groups (the scratch cap; forced small here through
    the tuning override) give the same gradients as one group."""
    c = _tuned_context(f"attnbwd_heads={group}")
    try:
        q, k, v, dout = rand_core(12, 2, 50, 60, 5 * 16, 1.0)
        check_core(gpu_core_bwd(c, q, k, v, dout, 5, True), q, k, v, dout, 5, True, f"groups of {group}")
    finally:
        c.close()


@pytest.mark.parametrize("blocks", [2, 3, 4])
@pytest.mark.parametrize("lq,lk", [(1000, 1000), (700, 300), (520, 900)])
def test_core_backward_causal_blocks(blocks, lq, lk):
    """The causal products over query / key blocks in other counts than the
    default two (a tuning override): ragged last blocks, cross shapes, and
    key blocks that no query sees (zeroed)."""
    c = _tuned_context(f"attnbwd_blocks={blocks}")
    try:
        q, k, v, dout = rand_core(lq + lk + blocks, 1, lq, lk, 2 * 32, 1.0)
        check_core(gpu_core_bwd(c, q, k, v, dout, 2, True), q, k, v, dout, 2, True, f"{blocks} blocks")
    finally:
        c.close()


@pytest.mark.parametrize("tune", ["blas=0", "blas=0,attnbwd_blocks=2"])
@pytest.mark.parametrize("causal", [False, True])
def test_core_backward_rocblas(tune, causal):
    """The rocBLAS-only path (MIMIR_TUNE blas=0): K and V transposed for the
    plain-form score products, dQ / dK / dV written in place, with and
    without causal blocks, and an odd head size."""
    c = _tuned_context(tune)
    try:
        q, k, v, dout = rand_core(15, 1, 520, 520, 3 * 20, 1.0)
        check_core(gpu_core_bwd(c, q, k, v, dout, 3, causal), q, k, v, dout, 3, causal, tune)
        q, k, v, dout = rand_core(16, 1, 260, 260, 2 * 13, 1.0)
        check_core(gpu_core_bwd(c, q, k, v, dout, 2, causal), q, k, v, dout, 2, causal, tune + ", head size 13")
    finally:
        c.close()


def test_core_backward_scale(ctx):
    q, k, v, dout = rand_core(13, 1, 40, 40, 64, 1.0)
    got = gpu_core_bwd(ctx, q, k, v, dout, 2, True, scale=0.37)
    ref = O.attention_bwd(q, k, v, dout, 2, True, scale=0.37)
    want, tol = attention_bwd64(q[0], k[0], v[0], dout[0], 2, True, 0.37)
    for j in range(3):
        assert_bwd_close(got[j][0], want[j], tol[j], "scale vs float64")
        assert_bwd_close(got[j][0], ref[j][0], 2 * tol[j], "scale vs oracle", 2 * NORM_REL)


def test_core_backward_empty(ctx):
    # no keys: dq = 0 (written), dk / dv empty
    q, k, v, dout = rand_core(14, 2, 6, 0, 16, 1.0)
    dq, dk, dv = gpu_core_bwd(ctx, q, k, v, dout, 2, True)
    assert np.array_equal(dq, np.zeros_like(dq)) and dk.size == 0 and dv.size == 0
    # no queries / no sequences: nothing written, no error
    q, k, v, dout = rand_core(14, 1, 0, 5, 16, 1.0)
    dq, dk, dv = gpu_core_bwd(ctx, q, k, v, dout, 2, False)
    assert np.isnan(dk).all() and np.isnan(dv).all()
    ctx.attention_bwd(None, None, None, None, None, None, None, 0, 4, 4, 2, 8)


def test_core_backward_refusals(ctx):
    q = _dev(ctx, np.zeros(64, np.float32))
    try:
        for kw, msg in ((dict(heads=0), "invalid shape"), (dict(ld_q=8), "row strides"),
                        (dict(scale=float("inf")), "scale must be finite")):
            args = dict(batch=1, q_len=2, kv_len=2, heads=2, head_dim=8, causal=False, scale=None, ld_q=None)
            args.update(kw)
            with pytest.raises(M.MimirError) as e:
                ctx.attention_bwd(q, q, q, q, q, q, q, args["batch"], args["q_len"], args["kv_len"], args["heads"],
                                  args["head_dim"], args["causal"], args["scale"], ld_q=args["ld_q"])
            assert e.value.status == M.EINVAL and msg in str(e.value), str(e.value)
    finally:
        q.free()


def test_core_backward_full_size(ctx):
    """The benchmark's shape (one sequence of 1024 tokens, 32 heads of 128,
    causal): heads 0 and 31 against the oracle and float64; every head
    against the two softmax identities; the first query's dq is exactly 0
    (its only probability is 1, so its dS row is 0)."""
    from mimir_hip import datagen as G
    seq, heads, hd = 1024, 32, 128
    w = heads * hd
    qkv = G.attention_qkv(batch=1, seq=seq, heads=heads, head_dim=hd).reshape(1, seq, 3 * w)
    q, k, v = qkv[..., :w], qkv[..., w:2 * w], qkv[..., 2 * w:]
    dout = np.random.default_rng(21).standard_normal((1, seq, w)).astype(np.float32)
    print("attention_bwd full size", flush=True)
    dq, dk, dv = gpu_core_bwd(ctx, q, k, v, dout, heads, True, fused=True)
    for h in (0, heads - 1):
        sl = slice(h * hd, (h + 1) * hd)
        qs, ks, vs, ds = (np.ascontiguousarray(a[..., sl]) for a in (q, k, v, dout))
        check_core((dq[..., sl], dk[..., sl], dv[..., sl]), qs, ks, vs, ds, 1, True, f"full size head {h}")
    assert not dq[0, 0].any(), "first query's dq"
    dk64, dv64 = dk[0].astype(np.float64), dv[0].astype(np.float64)
    # sum_j dk_j = scale sum_i (sum_j dS_ij) q_i = 0: bounded by the rounding of the terms
    bound = 1e-5 * np.abs(dk64).sum(0) + 1e-6
    assert (np.abs(dk64.sum(0)) <= bound).all(), "key-sum of dK"
    want = dout[0].astype(np.float64).sum(0)
    assert (np.abs(dv64.sum(0) - want) <= 1e-5 * np.abs(dout[0]).astype(np.float64).sum(0) + 1e-6).all(), \
        "key-sum of dV"


# ---- the layer forms --------------------------------------------------------

@pytest.mark.parametrize("seq,e,heads,causal", [(40, 64, 4, True), (33, 96, 3, False), (64, 128, 2, True),
                                                (1, 32, 8, False), (200, 256, 2, True)])
def test_self_attention_layer_backward(ctx, seq, e, heads, causal):
    x, w = layer_case(seq, e, seq + e, amp=1.5)
    dy = np.random.default_rng(seq).standard_normal((seq, e)).astype(np.float32)
    (dx, dwqkv, dwout), (tx, twqkv, twout) = self_attention_bwd64(
        x, w[:3 * e * e].reshape(e, 3 * e), w[3 * e * e:].reshape(e, e), dy, heads, causal)
    bufs = [_dev(ctx, a) for a in (x, dy, w, np.zeros(w.size, np.float32), np.full(x.shape, np.nan, np.float32))]
    try:
        dxb, dyb, wb, gwb, gxb = bufs
        ctx.self_attention_bwd(dxb, dyb, seq, e, heads, causal, wb, w.size, gwb, gxb)
        gw, gx = gwb.numpy(), gxb.numpy().reshape(seq, e)
        assert_bwd_close(gx, dx, tx, "dx")
        assert_bwd_close(gw[:3 * e * e], dwqkv, twqkv, "dWqkv")
        assert_bwd_close(gw[3 * e * e:], dwout, twout, "dWout")
        # accumulate: the weight gradients add onto what is there, dx adds
        # onto the buffer when asked; without a grad_weights block only dx.
        ctx.self_attention_bwd(dxb, dyb, seq, e, heads, causal, wb, w.size, gwb, gxb, accumulate=True)
        assert_bwd_close(gwb.numpy(), 2 * np.concatenate([dwqkv.ravel(), dwout.ravel()]),
                         2 * np.concatenate([twqkv.ravel(), twout.ravel()]), "accumulated dW")
        assert_bwd_close(gxb.numpy(), 2 * dx, 2 * tx, "accumulated dx")
        ctx.self_attention_bwd(dxb, dyb, seq, e, heads, causal, wb, w.size, None, gxb)
        assert_bwd_close(gxb.numpy(), dx, tx, "dx without weight gradients")
    finally:
        for b in bufs:
            b.free()


def test_self_attention_layer_backward_in_place(ctx):
    """grad_input may be grad_out itself (an input and output of one name:
    the reference adds dx into the gradient it read)."""
    seq, e, heads = 48, 64, 4
    x, w = layer_case(seq, e, 5)
    dy = np.random.default_rng(6).standard_normal((seq, e)).astype(np.float32)
    (dx, _, _), (tx, _, _) = self_attention_bwd64(x, w[:3 * e * e].reshape(e, 3 * e), w[3 * e * e:].reshape(e, e), dy,
                                                  heads, True)
    bufs = [_dev(ctx, a) for a in (x, dy, w)]
    try:
        xb, gb, wb = bufs
        ctx.self_attention_bwd(xb, gb, seq, e, heads, True, wb, w.size, None, gb, accumulate=True)
        assert_bwd_close(gb.numpy().reshape(seq, e), dy + dx, tx + 1e-7 * np.abs(dy), "dy + dx in place")
    finally:
        for b in bufs:
            b.free()


def _cross_parts(w, e):
    return w[:e * e].reshape(e, e), w[e * e:3 * e * e].reshape(e, 2 * e), w[3 * e * e:].reshape(e, e)


@pytest.mark.parametrize("lq,lk,e,heads,causal", [(37, 90, 64, 4, False), (37, 90, 64, 4, True),
                                                  (50, 20, 32, 2, True), (1, 7, 16, 1, False)])
def test_cross_attention_layer_backward(ctx, lq, lk, e, heads, causal):
    r = np.random.default_rng(lq + lk)
    w = (r.standard_normal(4 * e * e) / np.sqrt(e)).astype(np.float32)
    xq, xkv = r.standard_normal((lq, e)).astype(np.float32), r.standard_normal((lk, e)).astype(np.float32)
    dy = r.standard_normal((lq, e)).astype(np.float32)
    (dxq, dxkv, dwq, dwkv, dwout), (txq, txkv, twq, twkv, twout) = cross_attention_bwd64(
        xq, xkv, *_cross_parts(w, e), dy, heads, causal)
    bufs = [_dev(ctx, a) for a in (xq, xkv, dy, w, np.zeros(w.size, np.float32), np.zeros((lq, e), np.float32),
                                   np.zeros((lk, e), np.float32))]
    try:
        qb, kvb, dyb, wb, gwb, gqb, gkvb = bufs
        ctx.cross_attention_bwd(qb, lq, kvb, lk, dyb, e, heads, causal, wb, w.size, gwb, gqb, gkvb)
        gw = gwb.numpy()
        assert_bwd_close(gqb.numpy(), dxq, txq, "dxq")
        assert_bwd_close(gkvb.numpy(), dxkv, txkv, "dxkv")
        assert_bwd_close(gw[:e * e], dwq, twq, "dWq")
        assert_bwd_close(gw[e * e:3 * e * e], dwkv, twkv, "dWkv")
        assert_bwd_close(gw[3 * e * e:], dwout, twout, "dWout")
    finally:
        for b in bufs:
            b.free()


def test_cross_attention_layer_backward_shared_input(ctx):
    """Query and key/value from one tensor (inputs of one name): both
    gradients land in one buffer, dxq written then dxkv added."""
    n, e, heads = 40, 64, 4
    r = np.random.default_rng(17)
    w = (r.standard_normal(4 * e * e) / np.sqrt(e)).astype(np.float32)
    x = r.standard_normal((n, e)).astype(np.float32)
    dy = r.standard_normal((n, e)).astype(np.float32)
    (dxq, dxkv, *_), (txq, txkv, *_) = cross_attention_bwd64(x, x, *_cross_parts(w, e), dy, heads, True)
    bufs = [_dev(ctx, a) for a in (x, dy, w, np.full((n, e), np.nan, np.float32))]
    try:
        xb, dyb, wb, gb = bufs
        ctx.cross_attention_bwd(xb, n, xb, n, dyb, e, heads, True, wb, w.size, None, gb, gb, acc_kv=True)
        assert_bwd_close(gb.numpy(), dxq + dxkv, txq + txkv, "dxq + dxkv")
    finally:
        for b in bufs:
            b.free()


def test_layer_backward_refusals(ctx):
    b = _dev(ctx, np.zeros(4096, np.float32))
    try:
        for call, msg in ((lambda: ctx.self_attention_bwd(b, b, 4, 16, 5, False, b, 4096, None, b),
                           "embed_dim must be divisible by num_heads"),
                          (lambda: ctx.self_attention_bwd(b, b, 4, 16, 2, False, b, 100, None, b), "weight block"),
                          (lambda: ctx.cross_attention_bwd(b, 0, b, 3, b, 16, 2, False, b, 4096, None, b, b),
                           "invalid dimensions")):
            with pytest.raises(M.MimirError) as e:
                call()
            assert e.value.status == M.EINVAL and msg in str(e.value), str(e.value)
    finally:
        b.free()


# ---- the device runtime's training step -------------------------------------

ref_only = pytest.mark.skipif(not MR.available(), reason="oracle/_ref not built")


@pytest.fixture(scope="module")
def store(ctx):
    s = M.Store(ctx)
    yield s
    s.close()


def _train(ctx, store, layers, fin, loss):
    g = M.DeviceGraph(ctx, layers)
    try:
        return store.train_step(g, fin, {}, loss)
    finally:
        g.close()


@ref_only
@pytest.mark.parametrize("seq,e,heads,causal,kind", [(40, 64, 4, True, "SelfAttention"),
                                                     (33, 96, 3, False, "MultiHeadAttention"),
                                                     (64, 128, 2, True, "SelfAttention")])
def test_store_self_attention_training(ctx, store, seq, e, heads, causal, kind):
    x, w = layer_case(seq, e, seq + e, amp=1.5)
    dy = np.random.default_rng(seq + 100).standard_normal((seq, e)).astype(np.float32)
    L = dict(name="attn", type=kind, inputs=["__input__"], output="x", seq_len=seq, embed_dim=e, num_heads=heads,
             causal=causal, weights=w)
    grads, ig = _train(ctx, store, [L], {"x": x.ravel()}, dy.ravel())
    rgrads, rig = MR.backward([L], {"x": x.ravel()}, {}, dy.ravel())
    (dx, dwqkv, dwout), (tx, twqkv, twout) = self_attention_bwd64(
        x, w[:3 * e * e].reshape(e, 3 * e), w[3 * e * e:].reshape(e, e), dy, heads, causal)
    tw = np.concatenate([twqkv.ravel(), twout.ravel()])
    assert_bwd_close(ig, dx, tx, "input gradient vs float64")
    assert_bwd_close(grads[0], np.concatenate([dwqkv.ravel(), dwout.ravel()]), tw, "grad_weights vs float64")
    assert_bwd_close(ig, rig, 2 * tx, "input gradient vs reference", 2 * NORM_REL)
    assert_bwd_close(grads[0], rgrads[0], 2 * tw, "grad_weights vs reference", 2 * NORM_REL)


@ref_only
@pytest.mark.parametrize("grad_of", ["query", "kv"])
@pytest.mark.parametrize("causal", [False, True])
def test_store_cross_attention_training(ctx, store, causal, grad_of):
    lq, lk, e, heads = 37, 90, 64, 4
    r = np.random.default_rng(23)
    w = (r.standard_normal(4 * e * e) / np.sqrt(e)).astype(np.float32)
    xq, xkv = r.standard_normal((lq, e)).astype(np.float32), r.standard_normal((lk, e)).astype(np.float32)
    dy = r.standard_normal((lq, e)).astype(np.float32)
    inputs = ["__input__", "kv"] if grad_of == "query" else ["q", "__input__"]
    fin = {"x": xq.ravel(), "kv": xkv.ravel()} if grad_of == "query" else {"x": xkv.ravel(), "q": xq.ravel()}
    L = dict(name="cross", type="CrossAttention", inputs=inputs, output="x", embed_dim=e, num_heads=heads,
             causal=causal, weights=w)
    grads, ig = _train(ctx, store, [L], fin, dy.ravel())
    rgrads, rig = MR.backward([L], fin, {}, dy.ravel())
    (dxq, dxkv, dwq, dwkv, dwout), (txq, txkv, twq, twkv, twout) = cross_attention_bwd64(
        xq, xkv, *_cross_parts(w, e), dy, heads, causal)
    want_ig, tol_ig = (dxq, txq) if grad_of == "query" else (dxkv, txkv)
    tw = np.concatenate([twq.ravel(), twkv.ravel(), twout.ravel()])
    assert_bwd_close(ig, want_ig, tol_ig, "input gradient vs float64")
    assert_bwd_close(grads[0], np.concatenate([dwq.ravel(), dwkv.ravel(), dwout.ravel()]), tw,
                     "grad_weights vs float64")
    assert_bwd_close(ig, rig, 2 * tol_ig, "input gradient vs reference", 2 * NORM_REL)
    assert_bwd_close(grads[0], rgrads[0], 2 * tw, "grad_weights vs reference", 2 * NORM_REL)


def _block_on_input(causal):
    """block_graph (LayerNorm -> SelfAttention -> Add -> LayerNorm -> GELU)
    reading "__input__", the name whose gradient the reference reports."""
    name, layers, fin, _ = block_graph(causal=causal)
    layers = [dict(L, inputs=["__input__" if n == "inp" else n for n in L["inputs"]]) for L in layers]
    return layers, {"x": fin["inp"]}


@ref_only
@pytest.mark.parametrize("causal", [False, True])
def test_store_attention_block_training(ctx, store, causal):
    """A training step through a pre-norm residual block: every layer's
    weight gradient and the input gradient against the reference's
    Model::backwardPass, normwise (each op's element-wise parity is tested
    on its own)."""
    layers, fin = _block_on_input(causal)
    loss = np.random.default_rng(29).standard_normal(fin["x"].size).astype(np.float32)
    grads, ig = _train(ctx, store, layers, fin, loss)
    rgrads, rig = MR.backward(layers, fin, {}, loss)
    assert_close_normwise(ig, rig, "input gradient", rel=1e-4)
    for L, g, rg in zip(layers, grads, rgrads):
        if rg is not None:
            assert_close_normwise(g, rg, f"{L['name']} grad_weights", rel=1e-4)


@ref_only
def test_store_cross_attention_shared_name_training(ctx, store):
    """CrossAttention with query and key/value of one name ("h", a LayerNorm
    output): both gradients accumulate into "h" and flow on to the input."""
    e, n, heads = 64, 30, 4
    r = np.random.default_rng(31)
    g = np.concatenate([1 + 0.05 * r.standard_normal(e), 0.05 * r.standard_normal(e)]).astype(np.float32)
    layers = [dict(name="ln", type="LayerNorm", inputs=["__input__"], output="h", in_features=e, weights=g),
              dict(name="cross", type="CrossAttention", inputs=["h", "h"], output="x", embed_dim=e, num_heads=heads,
                   causal=True, weights=(r.standard_normal(4 * e * e) / np.sqrt(e)).astype(np.float32))]
    fin = {"x": r.standard_normal(n * e).astype(np.float32)}
    loss = r.standard_normal(n * e).astype(np.float32)
    grads, ig = _train(ctx, store, layers, fin, loss)
    rgrads, rig = MR.backward(layers, fin, {}, loss)
    assert_close_normwise(ig, rig, "input gradient", rel=1e-4)
    for L, gr, rg in zip(layers, grads, rgrads):
        assert_close_normwise(gr, rg, f"{L['name']} grad_weights", rel=1e-4)
