"""Host-vector mirror of the reference's op API over libmimir_hip.

Same names, argument meaning and error behaviour as the reference's forward
entry points (brit45/mimir-framework):

* ``layernorm_forward``   LayerOps.hpp:264-319
* ``rms_norm_forward``    LayerOpsExt.hpp:345-378 (whole vector)
* ``rms_norm``            Normalization::rms_norm, Layers.hpp:1003-1021 (per row, in place)
* ``softmax_forward``     LayerOps.hpp:325-361 (Softmax / LogSoftmax layer, whole vector)
* ``softmax_inplace``     LayerOps.hpp:952-974 (row softmax, in place)
* ``gelu_forward`` / ``silu_forward``  LayerOps.hpp:556-581
* ``add_forward`` / ``multiply_forward``  LayerOps.hpp:142-230
* ``embedding_forward``   the inline gather of Model.cpp:1152-1205 / 5301-5334
* ``attention_core``      steps 2-5 of self_attention_forward, LayerOps.hpp:1028-1089,
                          on the QKV projection's output (the softmax fused into QK^T / PV)
* ``cross_attention_core`` the same core of cross_attention_forward, :1163-1209

Inputs and outputs are host numpy vectors, so every call uploads, runs the
HIP kernel and downloads (the PCIe-inclusive path the reference's callers
would see).  Where the reference throws std::runtime_error these raise
RuntimeError.  Device-resident callers use :class:`mimir_hip.Context`'s op
methods directly.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import _lib
from .device import Context, MimirError


@dataclass
class Layer:
    """The op-parameter fields of the reference's ``struct Layer``
    (Layers.hpp:86-309) that this path reads."""
    type: str = ""
    eps: float = 1e-5           # Layers.hpp:139
    affine: bool = True         # :142
    use_bias: bool = True       # :197
    in_features: int = 0        # :112
    vocab_size: int = 0         # :149
    embed_dim: int = 0          # :150
    padding_idx: int = -1       # :151
    weights: np.ndarray = field(default_factory=lambda: np.zeros(0, np.float32))

    def getWeights(self):
        return self.weights

    def getWeightsSize(self):
        return int(np.asarray(self.weights).size)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32).ravel()


class LayerOps:
    """The reference op API bound to one device context."""

    def __init__(self, ctx: Context | None = None):
        self.ctx = ctx or Context(0)

    # -- helpers ----------------------------------------------------------
    def _run(self, fn, *arrays_in, out_size):
        ctx = self.ctx
        dev_in = [None if a is None else ctx.to_device(a) for a in arrays_in]
        y = ctx.empty(max(out_size, 1))
        try:
            try:
                fn(*dev_in, y)
            except MimirError as e:
                if e.status == _lib.EINVAL:
                    raise RuntimeError(str(e)) from e
                raise
            out = np.empty(out_size, np.float32)
            if out_size:
                ctx.download(out, y)
            return out
        finally:
            for d in dev_in:
                if d is not None:
                    d.free()
            y.free()

    # -- ops ----------------------------------------------------------------
    def layernorm_forward(self, input, layer: Layer, training=True):
        x = _f32(input)
        N = x.size
        n = layer.in_features if layer.in_features > 0 else N
        if n <= 0 or N % n:
            raise RuntimeError("LayerNorm: invalid normalized_size")
        # LayerOps.hpp:284-285: affine reads getWeights(), which is null for a
        # layer without a weight block -- then there is no affine transform.
        # A block shorter than gamma | beta is read out of bounds by the
        # reference; it is refused here.
        w = _f32(layer.getWeights()) if layer.affine and layer.getWeightsSize() > 0 else None
        gamma = beta = None
        if w is not None:
            need = 2 * n if layer.use_bias else n
            if w.size < need:
                raise RuntimeError(f"LayerNorm: {w.size} params for {need} needed")
            gamma = w[:n]
            beta = w[n:2 * n] if layer.use_bias else None
        return self._run(lambda dx, dg, db, y: self.ctx.layernorm(dx, dg, db, y, N // n, n, layer.eps),
                         x, gamma, beta, out_size=N)

    def rms_norm_forward(self, input, layer: Layer):
        x = _f32(input)
        w = _f32(layer.getWeights()) if layer.affine and layer.getWeightsSize() else None
        if x.size == 0:
            return x.copy()
        return self._run(lambda dx, dw, y: self.ctx.rmsnorm(dx, dw, 0 if w is None else w.size, y, 1,
                                                            x.size, layer.eps),
                         x, w, out_size=x.size)

    def rms_norm(self, data: np.ndarray, gamma, normalized_size, eps=1e-6):
        """In place on `data` (a float32 numpy array), like Normalization::rms_norm."""
        x = _f32(data)
        g = _f32(gamma)
        rows = x.size // normalized_size
        y = self._run(lambda dx, dg, dy: self.ctx.rmsnorm(dx, dg, normalized_size, dy, rows,
                                                          normalized_size, eps),
                      x, g, out_size=x.size)
        data.reshape(-1)[:] = y

    def softmax_forward(self, input, layer: Layer):
        x = _f32(input)
        mode = _lib.SOFTMAX_LOG if layer.type == "LogSoftmax" else _lib.SOFTMAX_MUL_INV
        return self._run(lambda dx, y: self.ctx.softmax(dx, y, 1, x.size, mode), x, out_size=x.size)

    def softmax_inplace(self, x: np.ndarray, seq_len, dim):
        v = _f32(x)
        y = self._run(lambda dx, dy: self.ctx.softmax(dx, dy, seq_len, dim, _lib.SOFTMAX_DIV_EPS), v,
                      out_size=v.size)
        x.reshape(-1)[:] = y

    def gelu_forward(self, input):
        x = _f32(input)
        if x.size == 0:
            return x.copy()
        return self._run(lambda dx, y: self.ctx.gelu(dx, y, x.size), x, out_size=x.size)

    def silu_forward(self, input):
        x = _f32(input)
        if x.size == 0:
            return x.copy()
        return self._run(lambda dx, y: self.ctx.silu(dx, y, x.size), x, out_size=x.size)

    def add_forward(self, input1, input2):
        a, b = _f32(input1), _f32(input2)
        if a.size == 0 or b.size == 0:
            raise RuntimeError("Add: inputs must be non-empty")
        return self._run(lambda da, db, y: self.ctx.add(da, a.size, db, b.size, y), a, b,
                         out_size=max(a.size, b.size))

    def multiply_forward(self, input1, input2):
        a, b = _f32(input1), _f32(input2)
        if a.size != b.size:
            raise RuntimeError("Multiply: input sizes must match")
        if a.size == 0:
            return a.copy()
        return self._run(lambda da, db, y: self.ctx.mul(da, a.size, db, b.size, y), a, b,
                         out_size=a.size)

    def embedding_forward(self, ids, layer: Layer):
        """The Model.cpp inline gather: int32 ids, or float ids rounded with llround."""
        ids = np.asarray(ids)
        float_ids = ids.dtype.kind == "f"
        ids = np.ascontiguousarray(ids, dtype=np.float32 if float_ids else np.int32).ravel()
        table = _f32(layer.getWeights())
        vocab = max(1, layer.vocab_size)
        dim = max(1, layer.embed_dim)
        if table.size < vocab * dim:
            raise RuntimeError("Embedding: invalid weight size")
        if ids.size == 0:
            return np.zeros(0, np.float32)
        ctx = self.ctx
        d_ids = ctx.to_device(ids)
        d_tab = ctx.to_device(table)
        y = ctx.empty(ids.size * dim)
        try:
            ctx.embedding(d_ids, ids.size, d_tab, table.size, layer.vocab_size, layer.embed_dim,
                          layer.padding_idx, y, float_ids=float_ids)
            return y.numpy()
        finally:
            d_ids.free()
            d_tab.free()
            y.free()

    def attention_core(self, qkv, seq_len, embed_dim, num_heads=1, causal=False):
        """Steps 2-5 of self_attention_forward on qkv [seq_len x 3*embed_dim]
        (Q | K | V column blocks): the attended heads [seq_len x embed_dim],
        flat, that the reference multiplies by out_weight."""
        x = _f32(qkv)
        if num_heads <= 0 or embed_dim % num_heads:
            raise RuntimeError("SelfAttention: embed_dim must be divisible by num_heads")
        if seq_len < 0 or x.size != seq_len * 3 * embed_dim:
            raise RuntimeError("SelfAttention: input size mismatch")
        hd = embed_dim // num_heads
        e = embed_dim
        return self._run(lambda d, y: self.ctx.attention(d, d.offset(e), d.offset(2 * e), y, 1, seq_len, seq_len,
                                                         num_heads, hd, causal, ld_q=3 * e, ld_kv=3 * e),
                         x, out_size=seq_len * e)

    def cross_attention_core(self, Q, KV, query_len, kv_len, embed_dim, num_heads=1, causal=False):
        """The core of cross_attention_forward on Q [query_len x E] and
        KV [kv_len x 2E] (K | V column blocks)."""
        q, kv = _f32(Q), _f32(KV)
        if num_heads <= 0 or embed_dim % num_heads:
            raise RuntimeError("CrossAttention: embed_dim must be divisible by num_heads")
        if query_len <= 0 or kv_len <= 0 or embed_dim <= 0:
            raise RuntimeError("CrossAttention: invalid dimensions")
        if q.size != query_len * embed_dim or kv.size != kv_len * 2 * embed_dim:
            raise RuntimeError("CrossAttention: input size mismatch")
        e = embed_dim
        return self._run(lambda dq, dkv, y: self.ctx.attention(dq, dkv, dkv.offset(e), y, 1, query_len, kv_len,
                                                               num_heads, e // num_heads, causal, ld_q=e,
                                                               ld_kv=2 * e),
                         q, kv, out_size=query_len * e)
