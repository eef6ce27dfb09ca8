"""mimir_hip.LayerOps -- the host-vector mirror of the reference's op API
(LayerOps.hpp / LayerOpsExt.hpp / Layers.hpp names and arguments) over the
HIP kernels -- called exactly as the reference's own functions are called,
against those functions compiled in place (oracle/_ref): the same inputs and
Layer fields, results within the path's tolerance (bit for bit for add,
multiply and the gather), and RuntimeError wherever the reference throws."""
import numpy as np
import pytest

import mimir_hip as M
import oracle as O
from _parity import assert_bitexact, assert_close

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")]

rng = np.random.default_rng(77)


@pytest.fixture(scope="module")
def ops(ctx):
    return M.LayerOps(ctx)


@pytest.mark.parametrize("groups,n", [(8, 512), (3, 4096), (1, 1000), (5, 33)])
@pytest.mark.parametrize("affine,use_bias,with_block", [(True, True, True), (True, False, True), (False, True, True),
                                                        (True, True, False)])
def test_layernorm_forward(ops, groups, n, affine, use_bias, with_block):
    x = (rng.standard_normal(groups * n) * 2 + 0.3).astype(np.float32)
    w = np.concatenate([1 + 0.1 * rng.standard_normal(n), 0.1 * rng.standard_normal(n)]).astype(np.float32)
    L = M.Layer(type="LayerNorm", in_features=n, affine=affine, use_bias=use_bias,
                weights=w if with_block else np.zeros(0, np.float32))
    ref = O.ref_layernorm(x, n, w if with_block else None, affine, use_bias, 1e-5)
    assert_close(ops.layernorm_forward(x, L), ref, "layernorm_forward")


def test_layernorm_forward_errors(ops):
    with pytest.raises(RuntimeError):  # LayerOps.hpp:276-279
        ops.layernorm_forward(np.ones(10, np.float32), M.Layer(type="LayerNorm", in_features=4))
    with pytest.raises(RuntimeError):
        O.ref_layernorm(np.ones(10, np.float32), 4)


@pytest.mark.parametrize("n,wn", [(4096, 4096), (1000, 17), (513, 0), (16384, 4096)])
def test_rms_norm_forward(ops, n, wn):
    x = rng.standard_normal(n).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(wn)).astype(np.float32)
    L = M.Layer(type="RMSNorm", eps=1e-5, weights=w)
    assert_close(ops.rms_norm_forward(x, L), O.ref_rms_norm_forward(x, w if wn else None, True, 1e-5),
                 "rms_norm_forward")


def test_rms_norm_rows_in_place(ops):
    x = rng.standard_normal((16, 4096)).astype(np.float32)
    g = (1 + 0.02 * rng.standard_normal(4096)).astype(np.float32)
    want = O.ref_rms_norm_rows(x, g, 1e-6)
    data = x.copy()
    ops.rms_norm(data, g, 4096, 1e-6)
    assert_close(data, want, "Normalization::rms_norm")


@pytest.mark.parametrize("log", [False, True])
def test_softmax_forward(ops, log):
    x = (3 * rng.standard_normal(5000)).astype(np.float32)
    L = M.Layer(type="LogSoftmax" if log else "Softmax")
    assert_close(ops.softmax_forward(x, L), O.ref_softmax_forward(x, log), "softmax_forward")


def test_softmax_inplace(ops):
    s = (3 * rng.standard_normal((64, 1024))).astype(np.float32)
    s[np.triu(np.ones((64, 1024), bool), 1)] = -np.inf
    want = O.ref_softmax_inplace(s)
    got = s.copy()
    ops.softmax_inplace(got, 64, 1024)
    assert_close(got, want, "softmax_inplace")


def test_activations(ops):
    x = np.concatenate([np.linspace(-8, 8, 20001, dtype=np.float32), rng.standard_normal(1000, dtype=np.float32)])
    assert_close(ops.gelu_forward(x), O.ref_gelu(x), "gelu_forward")
    assert_close(ops.silu_forward(x), O.ref_silu(x), "silu_forward")


@pytest.mark.parametrize("na,nb", [(1000, 1000), (1000, 1), (1, 1000), (4096, 256), (256, 4096)])
def test_add_forward_bitexact(ops, na, nb):
    a, b = rng.standard_normal(na).astype(np.float32), rng.standard_normal(nb).astype(np.float32)
    assert_bitexact(ops.add_forward(a, b), O.ref_add(a, b), "add_forward")


def test_add_multiply_errors(ops):
    for a, b in ((np.ones(5, np.float32), np.ones(2, np.float32)), (np.ones(0, np.float32), np.ones(2, np.float32))):
        with pytest.raises(RuntimeError):
            ops.add_forward(a, b)
        with pytest.raises(RuntimeError):
            O.ref_add(a, b)
    with pytest.raises(RuntimeError):
        ops.multiply_forward(np.ones(3, np.float32), np.ones(2, np.float32))
    with pytest.raises(RuntimeError):
        O.ref_mul(np.ones(3, np.float32), np.ones(2, np.float32))


def test_multiply_forward_bitexact(ops):
    a, b = rng.standard_normal(3001).astype(np.float32), rng.standard_normal(3001).astype(np.float32)
    assert_bitexact(ops.multiply_forward(a, b), O.ref_mul(a, b), "multiply_forward")


@pytest.mark.parametrize("float_ids", [False, True])
def test_embedding_forward_bitexact(ops, float_ids):
    vocab, dim = 50, 64
    table = rng.standard_normal(vocab * dim).astype(np.float32)
    ids = rng.integers(-3, vocab + 3, 300).astype(np.int32)
    arg = ids.astype(np.float32) + np.float32(0.3) if float_ids else ids
    L = M.Layer(type="Embedding", vocab_size=vocab, embed_dim=dim, padding_idx=4, weights=table)
    assert_bitexact(ops.embedding_forward(arg, L), O.embedding(arg, table, vocab, dim, 4).ravel(), "gather")
    with pytest.raises(RuntimeError):  # Model.cpp:1181-1182
        ops.embedding_forward(ids, M.Layer(type="Embedding", vocab_size=vocab, embed_dim=dim, weights=table[:-1]))


@pytest.mark.parametrize("seq,e,heads", [(40, 64, 2), (130, 96, 3), (1, 16, 1)])
@pytest.mark.parametrize("causal", [False, True])
def test_attention_core(ops, seq, e, heads, causal):
    """attention_core on the QKV projection, against the reference's own
    self_attention_forward fed one-hot inputs and an identity output
    projection (both projections exact: its output is the core itself)."""
    from _attention import assert_attention_close, attention64, self_case
    x, w, q, k, v = self_case(seq, e, 1.5, seq + e)
    ref = O.ref_self_attention(x, w, np.eye(e, dtype=np.float32), seq, e, heads, causal)
    qkv = np.concatenate([q, k, v], axis=1)
    got = ops.attention_core(qkv, seq, e, heads, causal).reshape(seq, e)
    _, mag, cond = attention64(q, k, v, heads, causal, O.attention_scale(e // heads))
    assert_attention_close(got, ref, mag, 2 * cond, "attention_core")


@pytest.mark.parametrize("causal", [False, True])
def test_cross_attention_core(ops, causal):
    from _attention import assert_attention_close, attention64, cross_case
    lq, lk, e, heads = 40, 65, 64, 2
    xq, xkv, wq, wkv, q, k, v = cross_case(lq, lk, e, 1.2, 9)
    ref = O.ref_cross_attention(xq, xkv, wq, wkv, np.eye(e, dtype=np.float32), lq, lk, e, heads, causal)
    got = ops.cross_attention_core(q, np.concatenate([k, v], axis=1), lq, lk, e, heads, causal).reshape(lq, e)
    _, mag, cond = attention64(q, k, v, heads, causal, O.attention_scale(e // heads))
    assert_attention_close(got, ref, mag, 2 * cond, "cross_attention_core")


def test_attention_core_errors(ops):
    with pytest.raises(RuntimeError, match="embed_dim must be divisible by num_heads"):
        ops.attention_core(np.zeros(4 * 36, np.float32), 4, 12, 5)
    with pytest.raises(RuntimeError, match="input size mismatch"):
        ops.attention_core(np.zeros(10, np.float32), 4, 12, 2)
    with pytest.raises(RuntimeError, match="invalid dimensions"):
        ops.cross_attention_core(np.zeros(0, np.float32), np.zeros(24, np.float32), 0, 1, 12, 2)
