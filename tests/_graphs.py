"""Layer graphs for the runtime tests: each is (name, layers, float_inputs,
int_inputs).  Layers are dicts with the reference Layer fields
(Layers.hpp:86-309) and a host `weights` block; the same graph is run by the
reference's Model::forwardPassNamed (oracle/model_ref.py), by the routing
restatement (oracle/model_oracle.py) and by the device store (mimir_store)."""
import numpy as np


def _rng(seed):
    return np.random.default_rng(seed)


def graphs():
    out = []

    # Tests/test_layers_named_routing.cpp:14-51: sum = a + b; x = sum * c
    out.append(("named_routing",
                [dict(name="sum", type="Add", inputs=["a", "b"], output="sum"),
                 dict(name="x", type="Multiply", inputs=["sum", "c"], output="x")],
                {"x": [0, 0], "a": [1, 2], "b": [3, 4], "c": [2, 2]}, {}))

    # Tests/test_runtime_embedding_int_inputs.cpp: int ids, padding_idx 0
    tab = np.array([[i * 10 + d for d in range(4)] for i in range(4)], np.float32).ravel()
    emb = dict(name="emb", type="Embedding", inputs=["ids"], output="x", vocab_size=4, embed_dim=4,
               padding_idx=0, seq_len=5, weights=tab)
    out.append(("embedding_int_ids", [emb], {}, {"ids": [1, 0, 2]}))
    out.append(("embedding_missing_ids", [emb], {}, {}))

    # A pre-norm transformer block's elementwise / row-reduction chain on
    # [seq x d]: embedding -> LN (per token) -> GELU -> residual add -> RMSNorm
    # layer (whole vector) -> SiLU -> Multiply gate -> Softmax, with a "seq"
    # input (aliased to text_ids / __input__ / x in the int store).
    r = _rng(1)
    vocab, d, seq = 50, 64, 12
    table = (0.5 * r.standard_normal(vocab * d)).astype(np.float32)
    ln_w = np.concatenate([1 + 0.1 * r.standard_normal(d), 0.1 * r.standard_normal(d)]).astype(np.float32)
    rms_w = (1 + 0.1 * r.standard_normal(seq * d)).astype(np.float32)
    gate = r.standard_normal(seq * d).astype(np.float32)
    ids = r.integers(-3, vocab + 3, seq).astype(np.int32)
    out.append(("block_chain",
                [dict(name="tok", type="Embedding", inputs=["text_ids"], output="h", vocab_size=vocab,
                      embed_dim=d, padding_idx=1, weights=table),
                 dict(name="ln", type="LayerNorm", inputs=["h"], output="n", in_features=d, eps=1e-5,
                      weights=ln_w),
                 dict(name="act", type="GELU", inputs=["n"], output="g"),
                 dict(name="residual", type="Add", inputs=["g", "h"], output="h2"),
                 dict(name="rms", type="RMSNorm", inputs=["h2"], output="r", eps=1e-6, weights=rms_w),
                 dict(name="silu", type="SiLU", inputs=["r"], output="s"),
                 dict(name="gate", type="Multiply", inputs=["s", "gate"], output="m"),
                 dict(name="drop", type="Dropout", inputs=["m"], output="m2"),
                 dict(name="sm", type="Softmax", inputs=["m2"], output="x")],
                {"gate": gate}, {"seq": ids}))

    # Default names: every layer reads and writes "x"; broadcast adds (bias
    # vector over rows, then a scalar), LayerNorm over the whole vector
    # (in_features 0), a non-affine RMSNorm, LogSoftmax, Identity.
    r = _rng(2)
    x = (2 * r.standard_normal(6 * 32) + 0.3).astype(np.float32)
    bias = r.standard_normal(32).astype(np.float32)
    out.append(("default_names_broadcast",
                [dict(name="bias", type="Add", inputs=["x", "bias"]),
                 dict(name="scalar", type="Add", inputs=["one", "x"]),
                 dict(name="ln_all", type="LayerNorm", weights=np.ones(2 * 192, np.float32)),
                 dict(name="id", type="Identity"),
                 dict(name="rms", type="RMSNorm", affine=False, eps=1e-5),
                 dict(name="lsm", type="LogSoftmax")],
                {"x": x, "bias": bias, "one": [0.5]}, {}))

    # Float ids from the float store (llround), ids outside the vocab, an
    # out-of-range padding id, LN without bias, LN without a weight block.
    r = _rng(3)
    fids = np.array([0.0, 1.4, 1.5, 2.5, -0.5, 7.49, 7.5, 9.0, 100.0, -3.0], np.float32)
    table2 = r.standard_normal(8 * 16).astype(np.float32)
    out.append(("float_ids_ln_variants",
                [dict(name="e", type="Embedding", inputs=["ids_f"], output="e", vocab_size=8, embed_dim=16,
                      padding_idx=7, weights=table2),
                 dict(name="ln1", type="LayerNorm", inputs=["e"], output="a", in_features=16, use_bias=False,
                      weights=(1 + 0.2 * r.standard_normal(16)).astype(np.float32)),
                 dict(name="ln2", type="LayerNorm", inputs=["a"], output="x", in_features=4)],
                {"ids_f": fids}, {}))

    # A LayerNorm block at the BASELINE width: [32 tokens x 4096]
    r = _rng(4)
    xs = r.standard_normal(32 * 4096).astype(np.float32)
    res = r.standard_normal(32 * 4096).astype(np.float32)
    w2 = np.concatenate([1 + 0.02 * r.standard_normal(4096), 0.02 * r.standard_normal(4096)]).astype(np.float32)
    out.append(("wide_ln_residual",
                [dict(name="res_add", type="Add", inputs=["x", "res"], output="h"),
                 dict(name="ln", type="LayerNorm", inputs=["h"], output="x", in_features=4096, weights=w2),
                 dict(name="gelu", type="GELU")],
                {"x": xs, "res": res}, {}))
    return out


# Graphs on which the reference throws std::runtime_error.
def error_graphs():
    return [
        ("missing_input", [dict(name="x", type="Multiply", inputs=["sum", "c"])], {"x": [0, 0]}, {}),
        ("add_one_input", [dict(name="a", type="Add", inputs=["x"])], {"x": [1, 2]}, {}),
        ("ln_bad_group", [dict(name="ln", type="LayerNorm", in_features=4)], {"x": [1, 2, 3, 4, 5, 6]}, {}),
        ("add_not_broadcastable", [dict(name="a", type="Add", inputs=["x", "y"])],
         {"x": [1, 2, 3, 4, 5], "y": [1, 2]}, {}),
        ("mul_size_mismatch", [dict(name="m", type="Multiply", inputs=["x", "y"])],
         {"x": [1, 2, 3], "y": [1, 2]}, {}),
        ("embedding_table_too_small",
         [dict(name="e", type="Embedding", inputs=["ids"], vocab_size=4, embed_dim=4,
               weights=np.ones(15, np.float32))], {}, {"ids": [1]}),
    ]
