"""Seeded synthetic inputs for the benchmark configurations.

The reference ships no data generator for these shapes, so this one is the
build's own: numpy's PCG64 generator seeded with ``0x4D494D52 ("MIMR") +
16*config + tensor_index``, float32 standard normals (``standard_normal(...,
dtype=float32)``) scaled as each configuration states, int32 ids from
``integers``.  Inputs are made once on the host, so the HIP path and the CPU
checker see the same bytes.
"""
from __future__ import annotations

import numpy as np

SEED_BASE = 0x4D494D52


def rng(config: int, tensor: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(SEED_BASE + 16 * config + tensor))


def normal(config: int, tensor: int, shape, scale=1.0, shift=0.0) -> np.ndarray:
    x = rng(config, tensor).standard_normal(int(np.prod(shape)), dtype=np.float32).reshape(shape)
    if scale != 1.0:
        x *= np.float32(scale)
    if shift != 0.0:
        x += np.float32(shift)
    return x


def ids(config: int, tensor: int, shape, vocab: int) -> np.ndarray:
    return rng(config, tensor).integers(0, vocab, size=shape, dtype=np.int32)


def causal_scores(config: int, tensor: int, batch, heads, q, k, scale=3.0) -> np.ndarray:
    """Logits scale*N(0,1) of shape [batch, heads, q, k] with j > i set to -inf."""
    s = normal(config, tensor, (batch, heads, q, k), scale)
    mask = np.triu(np.ones((q, k), dtype=bool), 1)
    s[:, :, mask] = -np.inf
    return s


# --------------------------------------------------------------------------
# BASELINE configurations (shapes at full size; `rows` lets tests take a prefix)
# --------------------------------------------------------------------------

def cfg0_layernorm(rows=256, cols=512):
    x = normal(0, 0, (rows, cols))
    gamma = normal(0, 1, (cols,), 0.02, 1.0)
    beta = normal(0, 2, (cols,), 0.02)
    return x, gamma, beta, 1e-5


def cfg1_add_rmsnorm(rows=4096, cols=4096):
    x = normal(1, 0, (rows, cols))
    r = normal(1, 1, (rows, cols))
    w = normal(1, 2, (cols,), 0.02, 1.0)
    return x, r, w, 1e-6


def cfg2_softmax(batch=8, heads=32, q=1024, k=1024):
    return causal_scores(2, 0, batch, heads, q, k)


def cfg3_gather(batch=16, seq=2048, vocab=32000, dim=4096):
    table = normal(3, 0, (vocab, dim), 0.02)
    tok = ids(3, 1, (batch, seq), vocab)
    return table, tok


def cfg3_rope(batch=16, seq=2048, heads=32, head_dim=128):
    q = normal(3, 2, (batch, seq, heads, head_dim))
    k = normal(3, 3, (batch, seq, heads, head_dim))
    return q, k, 10000.0


def cfg4_layernorm(rows=8192, cols=4096):
    x = normal(4, 0, (rows, cols))
    gamma = normal(4, 1, (cols,), 0.02, 1.0)
    beta = normal(4, 2, (cols,), 0.02)
    return x, gamma, beta, 1e-5


def cfg4_gelu(rows=8192, cols=11008):
    return normal(4, 3, (rows, cols))


def cfg4_swiglu(rows=8192, cols=11008):
    return normal(4, 4, (rows, cols)), normal(4, 5, (rows, cols))


def cfg4_add(rows=8192, cols=4096):
    return normal(4, 6, (rows, cols)), normal(4, 7, (rows, cols))


# --------------------------------------------------------------------------
# Output gradients for the backward ops at the same shapes (N(0,1); the
# embedding's scaled by 0.01 like a small loss gradient)
# --------------------------------------------------------------------------

def attention_qkv(batch=8, seq=1024, heads=32, head_dim=128):
    """The fused QKV buffer of the attention benchmark: [batch*seq, 3*E]
    (E = heads*head_dim) N(0,1), Q | K | V column blocks -- the layout of
    self_attention_forward's projection output (LayerOps.hpp:1031-1043) --
    at configs[2]'s attention shape (8 sequences x 32 heads x 1024 tokens)."""
    return normal(2, 6, (batch * seq, 3 * heads * head_dim))


def attention_dout(batch=8, seq=1024, heads=32, head_dim=128):
    """The gradient of the attended heads for the attention backward
    benchmark: [batch*seq, E] N(0,1)."""
    return normal(2, 7, (batch * seq, heads * head_dim))


def cfg4_grad(shape, tensor=8):
    return normal(4, tensor, shape)


def cfg3_embedding_grad(batch=16, seq=2048, dim=4096):
    return normal(3, 4, (batch * seq, dim), 0.01)


def cfg3_ids(batch=16, seq=2048, vocab=32000):
    return ids(3, 1, (batch, seq), vocab)


def cfg3_ids_zipf(batch=16, seq=2048, vocab=32000, s=1.0):
    """Token ids as text has them: the id of frequency rank r drawn with
    probability proportional to r^-s (Zipf), ranks mapped to ids by a fixed
    permutation.  At s = 1 the most frequent id is ~9% of the tokens."""
    g = rng(3, 5)
    p = np.arange(1, vocab + 1, dtype=np.float64) ** -s
    ranks = g.choice(vocab, size=(batch, seq), p=p / p.sum())
    return g.permutation(vocab).astype(np.int32)[ranks]
