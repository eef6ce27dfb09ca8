"""numpy front end for the CPU checkers.  TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
bench.py may import this module; the product (``mimir_hip``) never does.

Two libraries are wrapped:

* ``lib/libmimir_oracle.so`` -- the C restatement (``mimir_oracle.c``) of the
  reference algorithms, the parity checker for every HIP kernel;
* ``_ref/libmimir_ref.so`` -- the reference's own op functions compiled in
  place (``ref_harness.cpp``), used to pin the restatement.  It exists only
  where it was built from a reference tree; :func:`ref_available` says so.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_double, c_float, c_int32, c_int64, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "lib", "libmimir_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libmimir_ref.so")

SOFTMAX_DIV_EPS = 0  # LayerOps::softmax_inplace, LayerOps.hpp:952-974
SOFTMAX_MUL_INV = 1  # LayerOps::softmax_forward, LayerOps.hpp:325-361
SOFTMAX_LOG = 2      # LogSoftmax branch, LayerOps.hpp:345-353


class OracleError(RuntimeError):
    """Raised where the reference throws std::runtime_error (status 1)."""


def _load(path):
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built (run `make -C oracle`)")
    return ctypes.CDLL(path)


_o = None
_r = None


def _oracle():
    global _o
    if _o is None:
        lib = _load(ORACLE_SO)
        P = c_void_p
        sig = {
            "oracle_layernorm": [P, c_int64, c_int64, P, P, c_float, P],
            "oracle_rmsnorm_whole": [P, c_int64, P, c_int64, c_float, P],
            "oracle_rmsnorm_rows": [P, c_int64, c_int64, P, c_float, P],
            "oracle_add_rmsnorm": [P, P, c_int64, c_int64, P, c_float, P, P],
            "oracle_add": [P, c_int64, P, c_int64, P],
            "oracle_mul": [P, c_int64, P, c_int64, P],
            "oracle_softmax_rows": [P, c_int64, c_int64, c_int32, P],
            "oracle_gelu": [P, c_int64, P],
            "oracle_silu": [P, c_int64, P],
            "oracle_silu_mul": [P, P, c_int64, P],
            "oracle_gelu_mul": [P, P, c_int64, P],
            "oracle_embedding_i32": [P, c_int64, P, c_int64, c_int32, c_int32, c_int32, P],
            "oracle_embedding_f32": [P, c_int64, P, c_int64, c_int32, c_int32, c_int32, P],
            "oracle_rope_table": [c_int64, c_int64, c_double, P, P],
            "oracle_rope": [P, P, c_int64, c_int64, c_int64, c_int64, c_int64, P, P, c_int64],
            "oracle_accumulate": [P, P, c_int64],
            "oracle_layernorm_bwd": [P, P, c_int64, c_int64, P, c_int32, c_float, P, P],
            "oracle_gelu_bwd": [P, P, c_int64, P],
            "oracle_silu_bwd": [P, P, c_int64, P],
            "oracle_mul_bwd": [P, P, P, c_int64, P, P],
            "oracle_add_bwd_small": [P, c_int64, c_int64, P],
            "oracle_embedding_bwd_i32": [P, c_int64, P, P, c_int64, c_int32, c_int32, c_int32],
            "oracle_embedding_bwd_f32": [P, c_int64, P, P, c_int64, c_int32, c_int32, c_int32],
            "oracle_attention": [P, c_int64, P, P, c_int64, P, c_int64, c_int64, c_int64, c_int64,
                                 c_int64, c_int64, c_float, c_int32],
            "oracle_attention_bwd": [P, c_int64, P, P, c_int64, P, c_int64, P, c_int64, P, P, c_int64,
                                     c_int64, c_int64, c_int64, c_int64, c_int64, c_float, c_int32],
        }
        for name, args in sig.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = None if name in ("oracle_gelu", "oracle_silu", "oracle_silu_mul",
                                          "oracle_gelu_mul", "oracle_accumulate", "oracle_gelu_bwd",
                                          "oracle_silu_bwd", "oracle_mul_bwd") else c_int32
        _o = lib
    return _o


def ref_available() -> bool:
    return os.path.exists(REF_SO)


def _ref():
    global _r
    if _r is None:
        lib = _load(REF_SO)
        P = c_void_p
        sig = {
            "ref_layernorm": [P, c_int64, c_int32, P, c_int64, c_int32, c_int32, c_float, P],
            "ref_rms_norm_forward": [P, c_int64, P, c_int64, c_int32, c_float, P],
            "ref_rms_norm_rows": [P, c_int64, c_int64, P, c_float, P],
            "ref_add": [P, c_int64, P, c_int64, P],
            "ref_mul": [P, c_int64, P, c_int64, P],
            "ref_softmax_inplace": [P, c_int64, c_int64, P],
            "ref_softmax_forward": [P, c_int64, c_int32, P],
            "ref_gelu": [P, c_int64, P],
            "ref_silu": [P, c_int64, P],
            "ref_self_attention": [P, P, P, c_int32, c_int32, c_int32, c_int32, c_int32, P],
            "ref_cross_attention": [P, P, P, P, P, c_int32, c_int32, c_int32, c_int32, c_int32, P],
        }
        for name, args in sig.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = c_int32
        _r = lib
    return _r


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a):
    return None if a is None else a.ctypes.data_as(c_void_p)


def _check(status, what):
    if status:
        raise OracleError(f"{what}: invalid argument")


# --------------------------------------------------------------------------
# C restatement
# --------------------------------------------------------------------------

def layernorm(x, in_features, gamma=None, beta=None, eps=1e-5):
    x = _f32(x).ravel()
    g = None if gamma is None else _f32(gamma)
    b = None if beta is None else _f32(beta)
    y = np.empty_like(x)
    _check(_oracle().oracle_layernorm(_p(x), x.size, int(in_features), _p(g), _p(b),
                                      eps, _p(y)), "layernorm")
    return y


def rmsnorm_whole(x, w=None, eps=1e-5):
    x = _f32(x).ravel()
    w = None if w is None else _f32(w)
    y = np.empty_like(x)
    _check(_oracle().oracle_rmsnorm_whole(_p(x), x.size, _p(w), 0 if w is None else w.size,
                                          eps, _p(y)), "rmsnorm_whole")
    return y


def rmsnorm_rows(x, gamma=None, eps=1e-6):
    x = _f32(x)
    rows, cols = x.shape
    g = None if gamma is None else _f32(gamma)
    y = np.empty_like(x)
    _check(_oracle().oracle_rmsnorm_rows(_p(x), rows, cols, _p(g), eps, _p(y)), "rmsnorm_rows")
    return y


def add_rmsnorm(x, residual, gamma=None, eps=1e-6):
    x = _f32(x)
    r = _f32(residual)
    rows, cols = x.shape
    g = None if gamma is None else _f32(gamma)
    h = np.empty_like(x)
    y = np.empty_like(x)
    _check(_oracle().oracle_add_rmsnorm(_p(x), _p(r), rows, cols, _p(g), eps, _p(h), _p(y)),
           "add_rmsnorm")
    return y, h


def add(a, b):
    a = _f32(a).ravel()
    b = _f32(b).ravel()
    y = np.empty(max(a.size, b.size), np.float32)
    _check(_oracle().oracle_add(_p(a), a.size, _p(b), b.size, _p(y)), "add")
    return y


def mul(a, b):
    a = _f32(a).ravel()
    b = _f32(b).ravel()
    y = np.empty(a.size, np.float32)
    _check(_oracle().oracle_mul(_p(a), a.size, _p(b), b.size, _p(y)), "mul")
    return y


MERGE_OPS = ("ADD", "MULTIPLY", "CONCATENATE", "MAX", "AVERAGE", "GATED", "ATTENTION_WEIGHTED")


def branch_merge(b1, b2, op):
    """Model::computeBranchMerge(branch1, branch2, output, merge_op) with the
    hardware path the reference takes on an AVX2 host (Model.cpp:4344-4479):
    output has branch1's size (both, for CONCATENATE) and reads branch2[i]
    for i < branch1.size().  ADD (:4355-4380), and the default branch that
    GATED / ATTENTION_WEIGHTED take (copy, then +=, :4470-4477): b1 + b2.
    MULTIPLY (:4382-4406): b1 * b2.  AVERAGE (:4434-4460): (b1 + b2) * 0.5f.
    MAX (:4408-4432): the 8-wide _mm256_max_ps loop over the largest multiple
    of 8 (b1 > b2 ? b1 : b2), then the std::max tail (b1 < b2 ? b2 : b1).
    CONCATENATE (:4462-4468): b1 then b2.  Each element is one or two IEEE
    float32 operations, which numpy float32 arithmetic performs exactly so.
    Raises OracleError where the reference would read past branch2's end."""
    a = _f32(b1).ravel()
    b = _f32(b2).ravel()
    op = MERGE_OPS[op] if not isinstance(op, str) else op
    if op == "CONCATENATE":
        return np.concatenate([a, b])
    if b.size < a.size:
        raise OracleError("branch merge: branch2 shorter than branch1 (read out of bounds in the reference)")
    b = b[:a.size]
    with np.errstate(all="ignore"):
        if op == "MULTIPLY":
            return a * b
        if op == "AVERAGE":
            return (a + b) * np.float32(0.5)
        if op == "MAX":
            body = a.size // 8 * 8
            return np.concatenate([np.where(a[:body] > b[:body], a[:body], b[:body]),
                                   np.where(a[body:] < b[body:], b[body:], a[body:])])
        return a + b


def softmax_rows(x, mode=SOFTMAX_DIV_EPS):
    x = _f32(x)
    if x.ndim == 1:
        x = x.reshape(1, -1)
    rows, cols = x.shape
    y = np.empty_like(x)
    _check(_oracle().oracle_softmax_rows(_p(x), rows, cols, mode, _p(y)), "softmax_rows")
    return y


def _unary(name, x):
    x = _f32(x)
    y = np.empty_like(x)
    getattr(_oracle(), name)(_p(x), x.size, _p(y))
    return y


def gelu(x):
    return _unary("oracle_gelu", x)


def silu(x):
    return _unary("oracle_silu", x)


def silu_mul(gate, up):
    g, u = _f32(gate), _f32(up)
    y = np.empty_like(g)
    _oracle().oracle_silu_mul(_p(g), _p(u), g.size, _p(y))
    return y


def gelu_mul(gate, up):
    g, u = _f32(gate), _f32(up)
    y = np.empty_like(g)
    _oracle().oracle_gelu_mul(_p(g), _p(u), g.size, _p(y))
    return y


def embedding(ids, table, vocab, dim, padding_idx=-1):
    table = _f32(table).ravel()
    ids = np.asarray(ids)
    n = ids.size
    d = max(1, int(dim))
    y = np.empty(n * d, np.float32)
    if ids.dtype == np.float32:
        ids = np.ascontiguousarray(ids).ravel()
        st = _oracle().oracle_embedding_f32(_p(ids), n, _p(table), table.size, int(vocab),
                                            int(dim), int(padding_idx), _p(y))
    else:
        ids = np.ascontiguousarray(ids, dtype=np.int32).ravel()
        st = _oracle().oracle_embedding_i32(_p(ids), n, _p(table), table.size, int(vocab),
                                            int(dim), int(padding_idx), _p(y))
    _check(st, "embedding")
    return y.reshape(n, d)


def rope_table(rows, head_dim, theta=10000.0):
    half = head_dim // 2
    c = np.empty((rows, half), np.float32)
    s = np.empty((rows, half), np.float32)
    _check(_oracle().oracle_rope_table(rows, head_dim, theta, _p(c), _p(s)), "rope_table")
    return c, s


def rope(x, cos_tab, sin_tab, pos_offset=0):
    x = _f32(x)
    B, S, H, D = x.shape
    c, s = _f32(cos_tab), _f32(sin_tab)
    y = np.empty_like(x)
    _check(_oracle().oracle_rope(_p(x), _p(y), B, S, H, D, pos_offset, _p(c), _p(s),
                                 c.shape[0]), "rope")
    return y


# --------------------------------------------------------------------------
# C restatement: backward (Model::backwardPass branches)
# --------------------------------------------------------------------------

def accumulate(dst, src):
    """accumulate_grad's add (Model.cpp:7329-7341): returns dst + src."""
    d = _f32(dst).ravel().copy()
    s = _f32(src).ravel()
    assert d.size == s.size
    _oracle().oracle_accumulate(_p(d), _p(s), d.size)
    return d


def oracle_accumulate_inplace(dst, src):
    """accumulate_grad's add in place on dst (a float32 C-contiguous array;
    src may be dst itself, as in the reference's aliasing case)."""
    assert dst.dtype == np.float32 and dst.flags.c_contiguous and dst.size == src.size
    s = src if src is dst else _f32(src)
    _oracle().oracle_accumulate(_p(dst), _p(s), dst.size)


def layernorm_bwd(x, dy, in_features, gamma=None, has_bias=False, eps=1e-5, grad_params=None):
    """Returns (dx, grad_params): dx of x's shape; grad_params = the
    [dgamma | dbeta] block added onto the given one (zeros when None)."""
    x = _f32(x).ravel()
    dy = _f32(dy).ravel()
    assert x.size == dy.size
    feat = in_features if in_features > 0 else x.size
    g = None if gamma is None else _f32(gamma)
    gp = None
    if g is not None:
        gp = (np.zeros(feat * (2 if has_bias else 1), np.float32) if grad_params is None
              else _f32(grad_params).copy())
    dx = np.empty_like(x)
    _check(_oracle().oracle_layernorm_bwd(_p(x), _p(dy), x.size, int(in_features), _p(g), int(bool(has_bias)),
                                          eps, _p(dx), _p(gp)), "layernorm_bwd")
    return dx, gp


def gelu_bwd(x, dy):
    x, dy = _f32(x), _f32(dy)
    dx = np.empty_like(x)
    _oracle().oracle_gelu_bwd(_p(x), _p(dy), x.size, _p(dx))
    return dx


def silu_bwd(x, dy):
    x, dy = _f32(x), _f32(dy)
    dx = np.empty_like(x)
    _oracle().oracle_silu_bwd(_p(x), _p(dy), x.size, _p(dx))
    return dx


def mul_bwd(a, b, dy):
    a, b, dy = _f32(a), _f32(b), _f32(dy)
    da, db = np.empty_like(a), np.empty_like(a)
    _oracle().oracle_mul_bwd(_p(a), _p(b), _p(dy), a.size, _p(da), _p(db))
    return da, db


def add_bwd_small(dy, n_small):
    dy = _f32(dy).ravel()
    out = np.empty(n_small, np.float32)
    _check(_oracle().oracle_add_bwd_small(_p(dy), dy.size, int(n_small), _p(out)), "add_bwd_small")
    return out


def embedding_bwd(ids, dy, grad_table, vocab, dim, padding_idx=-1):
    """Returns grad_table + the scatter-added rows (ids int32, or float ids)."""
    dy = _f32(dy).ravel()
    gt = _f32(grad_table).ravel().copy()
    if np.asarray(ids).dtype == np.float32:
        ids = _f32(ids).ravel()
        fn = _oracle().oracle_embedding_bwd_f32
    else:
        ids = np.ascontiguousarray(ids, np.int32).ravel()
        fn = _oracle().oracle_embedding_bwd_i32
    _check(fn(_p(ids), ids.size, _p(dy), _p(gt), gt.size, int(vocab), int(dim), int(padding_idx)),
           "embedding_bwd")
    return gt


def attention_scale(head_dim):
    """1.0f / std::sqrt((float) head_dim), LayerOps.hpp:1047 (both IEEE, correctly rounded)."""
    return float(np.float32(1.0) / np.sqrt(np.float32(head_dim)))


def attention(q, k, v, heads, causal=False, scale=None):
    """The attention core of self_attention_forward / cross_attention_forward
    (oracle_attention).  q: [batch, q_len, width] (or [q_len, width]); k, v:
    [batch, kv_len, width]; width = heads * head_dim.  Returns [batch, q_len,
    width] (or [q_len, width])."""
    squeeze = np.ndim(q) == 2
    q, k, v = (np.asarray(a, np.float32) for a in (q, k, v))
    if squeeze:
        q, k, v = q[None], k[None], v[None]
    batch, q_len, width = q.shape
    kv_len = k.shape[1]
    if k.shape != (batch, kv_len, width) or v.shape != k.shape or width % heads:
        raise OracleError("attention: shape mismatch")
    head_dim = width // heads
    if scale is None:
        scale = attention_scale(head_dim)
    q, k, v = _f32(q), _f32(k), _f32(v)
    y = np.empty((batch, q_len, width), np.float32)
    _check(_oracle().oracle_attention(_p(q), width, _p(k), _p(v), width, _p(y), width, batch, q_len,
                                      kv_len, heads, head_dim, scale, int(causal)), "attention")
    return y[0] if squeeze else y


def attention_bwd(q, k, v, dout, heads, causal=False, scale=None):
    """The per-head core of backward_self_attention / backward_cross_attention
    (oracle_attention_bwd): (dq, dk, dv) from q [.., q_len, width], k / v
    [.., kv_len, width] and dout (the gradient of the attended heads, shaped
    like q)."""
    squeeze = np.ndim(q) == 2
    q, k, v, dout = (np.asarray(a, np.float32) for a in (q, k, v, dout))
    if squeeze:
        q, k, v, dout = q[None], k[None], v[None], dout[None]
    batch, q_len, width = q.shape
    kv_len = k.shape[1]
    if k.shape != (batch, kv_len, width) or v.shape != k.shape or dout.shape != q.shape or width % heads:
        raise OracleError("attention_bwd: shape mismatch")
    head_dim = width // heads
    if scale is None:
        scale = attention_scale(head_dim)
    q, k, v, dout = _f32(q), _f32(k), _f32(v), _f32(dout)
    dq = np.empty_like(q)
    dk = np.empty_like(k)
    dv = np.empty_like(v)
    _check(_oracle().oracle_attention_bwd(_p(q), width, _p(k), _p(v), width, _p(dout), width, _p(dq), width,
                                          _p(dk), _p(dv), width, batch, q_len, kv_len, heads, head_dim, scale,
                                          int(causal)), "attention_bwd")
    if squeeze:
        return dq[0], dk[0], dv[0]
    return dq, dk, dv


U32 = 2.0 ** -24  # float32 unit roundoff


def attention_float64(q, k, v, heads, causal, scale):
    """float64 softmax attention and the scales of its float32 rounding:
    (out, mag, cond), all shaped like q ([.., q_len, width]).
    mag  = sum_j p_j |v_j|: the scale of the float32 rounding of the weighted
           sum (two summation orders differ by ~u * mag);
    cond = u * sqrt(head_dim) * sum_j p_j A_j (|v_j| + |out|), A_j = scale *
           sum_k |q_k k_k|: the first-order effect on the output of rounding
           the float32 scores (d out / d s_j = p_j (v_j - out); a D-term
           float32 dot product is off by ~u sqrt(D) A_j).
    The path's tolerance for attention is max(1e-6, 1e-5 * max(|ref|, mag))
    + cond."""
    q, k, v = (np.asarray(a, np.float64) for a in (q, k, v))
    squeeze = q.ndim == 2
    if squeeze:
        q, k, v = q[None], k[None], v[None]
    b, lq, width = q.shape
    lk = k.shape[1]
    hd = width // heads
    sc = float(np.float32(scale))
    out = np.zeros((b, lq, width))
    mag = np.zeros((b, lq, width))
    cond = np.zeros((b, lq, width))
    mask = np.arange(lk)[None, :] > np.arange(lq)[:, None]
    for h in range(heads):
        sl = slice(h * hd, (h + 1) * hd)
        s = np.einsum("bid,bjd->bij", q[..., sl], k[..., sl]) * sc
        a = np.einsum("bid,bjd->bij", np.abs(q[..., sl]), np.abs(k[..., sl])) * abs(sc)
        if causal:
            s = np.where(mask[None], -np.inf, s)
        s = s - s.max(axis=2, keepdims=True) if lk else s
        p = np.exp(s)
        p /= np.maximum(p.sum(axis=2, keepdims=True), 1e-300)
        out[..., sl] = np.einsum("bij,bjd->bid", p, v[..., sl])
        mag[..., sl] = np.einsum("bij,bjd->bid", p, np.abs(v[..., sl]))
        pa = p * a
        cond[..., sl] = (np.einsum("bij,bjd->bid", pa, np.abs(v[..., sl])) +
                         pa.sum(axis=2)[..., None] * np.abs(out[..., sl])) * (U32 * np.sqrt(hd))
    if squeeze:
        return out[0], mag[0], cond[0]
    return out, mag, cond


# --------------------------------------------------------------------------
# The reference's own functions (compiled in place)
# --------------------------------------------------------------------------

def ref_layernorm(x, in_features, params=None, affine=True, use_bias=True, eps=1e-5):
    x = _f32(x).ravel()
    p = np.zeros(0, np.float32) if params is None else _f32(params)
    y = np.empty_like(x)
    _check(_ref().ref_layernorm(_p(x), x.size, int(in_features), _p(p), p.size, int(affine),
                                int(use_bias), eps, _p(y)), "ref_layernorm")
    return y


def ref_rms_norm_forward(x, w=None, affine=True, eps=1e-5):
    x = _f32(x).ravel()
    w = np.zeros(0, np.float32) if w is None else _f32(w)
    y = np.empty_like(x)
    _check(_ref().ref_rms_norm_forward(_p(x), x.size, _p(w), w.size, int(affine), eps, _p(y)),
           "ref_rms_norm_forward")
    return y


def ref_rms_norm_rows(x, gamma, eps=1e-6):
    x = _f32(x)
    rows, cols = x.shape
    g = _f32(gamma)
    y = np.empty_like(x)
    _check(_ref().ref_rms_norm_rows(_p(x), rows, cols, _p(g), eps, _p(y)), "ref_rms_norm_rows")
    return y


def ref_add(a, b):
    a = _f32(a).ravel()
    b = _f32(b).ravel()
    y = np.empty(max(a.size, b.size), np.float32)
    _check(_ref().ref_add(_p(a), a.size, _p(b), b.size, _p(y)), "ref_add")
    return y


def ref_mul(a, b):
    a = _f32(a).ravel()
    b = _f32(b).ravel()
    y = np.empty(a.size, np.float32)
    _check(_ref().ref_mul(_p(a), a.size, _p(b), b.size, _p(y)), "ref_mul")
    return y


def ref_softmax_inplace(x):
    x = _f32(x)
    rows, cols = x.shape
    y = np.empty_like(x)
    _check(_ref().ref_softmax_inplace(_p(x), rows, cols, _p(y)), "ref_softmax_inplace")
    return y


def ref_softmax_forward(x, log_softmax=False):
    x = _f32(x).ravel()
    y = np.empty_like(x)
    _check(_ref().ref_softmax_forward(_p(x), x.size, int(log_softmax), _p(y)),
           "ref_softmax_forward")
    return y


def ref_gelu(x):
    x = _f32(x).ravel()
    y = np.empty_like(x)
    _check(_ref().ref_gelu(_p(x), x.size, _p(y)), "ref_gelu")
    return y


def ref_silu(x):
    x = _f32(x).ravel()
    y = np.empty_like(x)
    _check(_ref().ref_silu(_p(x), x.size, _p(y)), "ref_silu")
    return y


def ref_self_attention(x, qkv_weight, out_weight, seq_len, embed_dim, num_heads, causal=False,
                       multihead=False):
    """LayerOps::self_attention_forward (or multihead_attention_forward)."""
    x, wq, wo = _f32(x).ravel(), _f32(qkv_weight).ravel(), _f32(out_weight).ravel()
    if x.size != seq_len * embed_dim or wq.size != 3 * embed_dim * embed_dim or wo.size != embed_dim ** 2:
        raise OracleError("ref_self_attention: size mismatch")
    y = np.empty(seq_len * embed_dim, np.float32)
    _check(_ref().ref_self_attention(_p(x), _p(wq), _p(wo), seq_len, embed_dim, num_heads, int(causal),
                                     int(multihead), _p(y)), "ref_self_attention")
    return y.reshape(seq_len, embed_dim)


def ref_cross_attention(xq, xkv, q_weight, kv_weight, out_weight, query_len, kv_len, embed_dim, num_heads,
                        causal=False):
    """LayerOps::cross_attention_forward."""
    a = [_f32(t).ravel() for t in (xq, xkv, q_weight, kv_weight, out_weight)]
    e = embed_dim
    if [t.size for t in a] != [query_len * e, kv_len * e, e * e, 2 * e * e, e * e]:
        raise OracleError("ref_cross_attention: size mismatch")
    y = np.empty(query_len * e, np.float32)
    _check(_ref().ref_cross_attention(*[_p(t) for t in a], query_len, kv_len, e, num_heads, int(causal),
                                      _p(y)), "ref_cross_attention")
    return y.reshape(query_len, e)


# --------------------------------------------------------------------------
# CPU baseline timing (bench.py's cpu_baseline leg)
# --------------------------------------------------------------------------

REF_T_ADD_RMSNORM, REF_T_LAYERNORM, REF_T_SOFTMAX, REF_T_GELU, REF_T_SILU_MUL, REF_T_ADD = range(6)


def ref_time_op(op, a, b=None, w=None, rows=0, cols=0, eps=1e-5, reps=3):
    """Median seconds of one call of the reference path `op` (ref_harness.cpp)."""
    lib = _ref()
    fn = lib.ref_time_op
    fn.argtypes = [c_int32, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_int64,
                   c_int64, c_float, c_int32]
    fn.restype = c_double
    a = _f32(a).ravel()
    b = np.zeros(0, np.float32) if b is None else _f32(b).ravel()
    w = np.zeros(0, np.float32) if w is None else _f32(w).ravel()
    t = fn(op, _p(a), a.size, _p(b), b.size, _p(w), w.size, rows, cols, eps, reps)
    if t < 0:
        raise OracleError(f"ref_time_op({op}) failed")
    return t


def time_port(fn, reps=3):
    """Median seconds of fn() (a call into the C restatement) after one warm-up."""
    import time
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]
