"""Layer graphs with the reference's attention layers (SelfAttention,
MultiHeadAttention, CrossAttention; Model.cpp:5904-5990) for the runtime
tests: the layer alone, and inside a pre-norm residual block of the path's
layers.  A graph is (name, layers, float_inputs, int_inputs) as in
tests/_graphs.py; weights are drawn scaled 1/sqrt(E) (unit-scale projections)."""
import numpy as np


def _w(r, e):
    return (r.standard_normal(4 * e * e) / np.sqrt(e)).astype(np.float32)


def single_graphs():
    r = np.random.default_rng(31)
    out = []
    for seq, e, heads, causal, kind in [(40, 64, 4, True, "SelfAttention"), (33, 96, 3, False, "SelfAttention"),
                                        (64, 128, 2, True, "MultiHeadAttention"), (1, 32, 8, False, "SelfAttention"),
                                        (100, 64, 1, False, "MultiHeadAttention")]:
        x = r.standard_normal(seq * e).astype(np.float32)
        L = dict(name=f"attn_{kind}_{seq}_{e}", type=kind, inputs=["x"], output="x", seq_len=seq, embed_dim=e,
                 num_heads=heads, causal=causal, weights=_w(r, e))
        out.append((L["name"], [L], {"x": x}, {}))
    lq, lk, e = 37, 90, 64
    for causal in (False, True):
        L = dict(name=f"cross_{int(causal)}", type="CrossAttention", inputs=["q", "kv"], output="x", embed_dim=e,
                 num_heads=4, causal=causal, weights=_w(r, e))
        out.append((L["name"], [L], {"q": r.standard_normal(lq * e).astype(np.float32),
                                     "kv": r.standard_normal(lk * e).astype(np.float32)}, {}))
    # CrossAttention sized by head_dim * num_heads (embed_dim unset).
    L = dict(name="cross_head_dim", type="CrossAttention", inputs=["q", "kv"], output="x", head_dim=16, num_heads=2,
             weights=_w(r, 32))
    out.append((L["name"], [L], {"q": r.standard_normal(5 * 32).astype(np.float32),
                                 "kv": r.standard_normal(7 * 32).astype(np.float32)}, {}))
    return out


def block_graph(seq=64, e=128, heads=4, causal=True, seed=5):
    """x -> LayerNorm -> SelfAttention -> + x -> LayerNorm -> GELU (a
    pre-norm transformer half-block built from the path's layers)."""
    r = np.random.default_rng(seed)
    g = np.concatenate([1 + 0.05 * r.standard_normal(e), 0.05 * r.standard_normal(e)]).astype(np.float32)
    layers = [dict(name="ln1", type="LayerNorm", inputs=["inp"], output="h", in_features=e, weights=g),
              dict(name="attn", type="SelfAttention", inputs=["h"], output="a", seq_len=seq, embed_dim=e,
                   num_heads=heads, causal=causal, weights=_w(r, e)),
              dict(name="res", type="Add", inputs=["a", "inp"], output="r"),
              dict(name="ln2", type="LayerNorm", inputs=["r"], output="n", in_features=e, weights=g),
              dict(name="act", type="GELU", inputs=["n"], output="x")]
    return "attention_block", layers, {"inp": r.standard_normal(seq * e).astype(np.float32)}, {}


def error_graphs():
    """Graphs the reference refuses, with the start of its message."""
    r = np.random.default_rng(8)
    e = 16
    x = r.standard_normal(4 * e).astype(np.float32)
    base = dict(type="SelfAttention", inputs=["x"], output="x", seq_len=4, embed_dim=e, num_heads=2, weights=_w(r, e))
    return [
        ("no_weights", [dict(base, name="a0", weights=None)], {"x": x}, {}, "Attention: weights not initialized"),
        ("heads_do_not_divide", [dict(base, name="a1", num_heads=5)], {"x": x}, {},
         "SelfAttention: embed_dim must be divisible by num_heads"),
        ("input_size_mismatch", [dict(base, name="a2", seq_len=5)], {"x": x}, {}, "SelfAttention: input size mismatch"),
        ("cross_one_input", [dict(base, name="c0", type="CrossAttention", inputs=["x"])], {"x": x}, {},
         "CrossAttention requires 2 inputs"),
        ("cross_not_divisible", [dict(base, name="c1", type="CrossAttention", inputs=["x", "kv"])],
         {"x": x, "kv": r.standard_normal(3 * e + 1).astype(np.float32)}, {},
         "CrossAttention: key/value input size must be divisible by embed_dim"),
        ("cross_no_embed_dim", [dict(base, name="c2", type="CrossAttention", inputs=["x", "x"], embed_dim=0)],
         {"x": x}, {}, "CrossAttention: embed_dim must be configured"),
    ]
