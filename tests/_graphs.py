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


# Graphs for a training step (forwardPassNamed(training=true) then
# Model::backwardPass): (name, layers, float_inputs, int_inputs, loss_grad).
# What the reference exposes after backwardPass is each layer's grad_weights
# and the gradient that reached "__input__", so every graph routes its
# gradient into parameters and/or "__input__".
def train_graphs():
    out = []

    # Embedding (repeated, padding and out-of-range ids) -> per-token LN ->
    # GELU -> residual Add -> RMSNorm layer -> SiLU -> gate Multiply -> Softmax.
    r = _rng(11)
    vocab, d, seq = 20, 64, 24
    table = (0.5 * r.standard_normal(vocab * d)).astype(np.float32)
    ln_w = np.concatenate([1 + 0.1 * r.standard_normal(d), 0.1 * r.standard_normal(d)]).astype(np.float32)
    rms_w = (1 + 0.1 * r.standard_normal(seq * d)).astype(np.float32)
    gate = r.standard_normal(seq * d).astype(np.float32)
    ids = r.integers(-2, vocab + 2, seq).astype(np.int32)
    ids[:4] = 5  # one row hit several times: its gradient is a sum in token order
    out.append(("block_train",
                [dict(name="tok", type="Embedding", inputs=["text_ids"], output="h", vocab_size=vocab,
                      embed_dim=d, padding_idx=1, weights=table),
                 dict(name="ln", type="LayerNorm", inputs=["h"], output="n", in_features=d, eps=1e-5,
                      weights=ln_w),
                 dict(name="act", type="GELU", inputs=["n"], output="g"),
                 dict(name="residual", type="Add", inputs=["g", "h"], output="h2"),
                 dict(name="rms", type="RMSNorm", inputs=["h2"], output="r", eps=1e-6, weights=rms_w),
                 dict(name="silu", type="SiLU", inputs=["r"], output="s"),
                 dict(name="gate", type="Multiply", inputs=["s", "gate"], output="m"),
                 dict(name="sm", type="Softmax", inputs=["m"], output="x")],
                {"gate": gate}, {"seq": ids}, r.standard_normal(seq * d).astype(np.float32)))

    # The gradient reaches "__input__" through LN (no bias), SiLU, a bias
    # broadcast Add, GELU, Multiply and Identity.
    r = _rng(12)
    rows, d = 10, 48
    xin = (1.5 * r.standard_normal(rows * d) + 0.2).astype(np.float32)
    out.append(("input_chain",
                [dict(name="ln", type="LayerNorm", inputs=["__input__"], output="a", in_features=d,
                      use_bias=False, weights=(1 + 0.2 * r.standard_normal(d)).astype(np.float32)),
                 dict(name="silu", type="SiLU", inputs=["a"], output="b"),
                 dict(name="bias", type="Add", inputs=["bvec", "b"], output="c"),
                 dict(name="gelu", type="GELU", inputs=["c"], output="e"),
                 dict(name="mul", type="Multiply", inputs=["e", "scale"], output="f"),
                 dict(name="id", type="Identity", inputs=["f"], output="x")],
                {"__input__": xin, "bvec": r.standard_normal(d).astype(np.float32),
                 "scale": r.standard_normal(rows * d).astype(np.float32)}, {},
                r.standard_normal(rows * d).astype(np.float32)))

    # "__input__" as the broadcast operand: its gradient is the per-position
    # sum over the tiles (repeat) and, through a scalar Add, the total sum.
    r = _rng(13)
    big = r.standard_normal(16 * 32).astype(np.float32)
    out.append(("broadcast_reduce",
                [dict(name="rep", type="Add", inputs=["big", "__input__"], output="h"),
                 dict(name="ln", type="LayerNorm", inputs=["h"], output="x", in_features=32,
                      weights=np.concatenate([np.ones(32), np.zeros(32)]).astype(np.float32))],
                {"big": big, "__input__": r.standard_normal(32).astype(np.float32)}, {},
                r.standard_normal(16 * 32).astype(np.float32)))
    out.append(("scalar_reduce",
                [dict(name="sc", type="Add", inputs=["__input__", "big"], output="h"),
                 dict(name="gelu", type="GELU", inputs=["h"], output="x")],
                {"big": big, "__input__": np.array([0.25], np.float32)}, {},
                r.standard_normal(16 * 32).astype(np.float32)))

    # Every layer reads and writes "x": the reference's gradient map then
    # adds a layer's input gradient onto its own output gradient (the same
    # vector), and Add(x, x) doubles it twice.  LN's grad_weights observe it.
    r = _rng(14)
    x = (r.standard_normal(8 * 16) + 0.5).astype(np.float32)
    out.append(("same_name_aliasing",
                [dict(name="ln", type="LayerNorm", in_features=16,
                      weights=np.concatenate([1 + 0.1 * r.standard_normal(16),
                                              0.1 * r.standard_normal(16)]).astype(np.float32)),
                 dict(name="gelu", type="GELU"),
                 dict(name="twice", type="Add", inputs=["x", "x"]),
                 dict(name="id", type="Identity"),
                 dict(name="rms", type="RMSNorm", affine=False, eps=1e-5),
                 dict(name="lsm", type="LogSoftmax")],
                {"x": x}, {}, r.standard_normal(8 * 16).astype(np.float32)))

    # Float ids (llround) with a padding id and ids outside the vocab; a
    # non-affine LN and a whole-vector LN (in_features 0).
    r = _rng(15)
    fids = np.array([0.0, 1.4, 1.5, 2.5, -0.5, 7.49, 7.5, 9.0, 100.0, -3.0, 2.0, 2.2], np.float32)
    out.append(("float_ids_train",
                [dict(name="e", type="Embedding", inputs=["ids_f"], output="e", vocab_size=8, embed_dim=16,
                      padding_idx=7, weights=r.standard_normal(8 * 16).astype(np.float32)),
                 dict(name="ln1", type="LayerNorm", inputs=["e"], output="a", in_features=16, affine=False),
                 dict(name="ln2", type="LayerNorm", inputs=["a"], output="x",
                      weights=np.concatenate([1 + 0.1 * r.standard_normal(12 * 16),
                                              0.1 * r.standard_normal(12 * 16)]).astype(np.float32))],
                {"ids_f": fids}, {}, r.standard_normal(12 * 16).astype(np.float32)))

    # A residual block at the BASELINE width, [32 tokens x 4096].
    r = _rng(16)
    xs = r.standard_normal(32 * 4096).astype(np.float32)
    w2 = np.concatenate([1 + 0.02 * r.standard_normal(4096), 0.02 * r.standard_normal(4096)]).astype(np.float32)
    out.append(("wide_block_train",
                [dict(name="ln", type="LayerNorm", inputs=["__input__"], output="n", in_features=4096,
                      weights=w2),
                 dict(name="gelu", type="GELU", inputs=["n"], output="g"),
                 dict(name="res", type="Add", inputs=["g", "__input__"], output="x")],
                {"__input__": xs}, {}, r.standard_normal(32 * 4096).astype(np.float32)))
    return out


# Training graphs with residual merges (forwardPassView with training=true,
# Model.cpp:6676-6685 -> executeBranchComputation :4550-4582 ->
# computeBranchMerge :4344-4479): (name, layers, float_inputs, int_inputs).
# A layer merges when its branch type is RESIDUAL (from its name, as
# Model::push's detectBranchType sets it, or set explicitly) and its first
# branch source is a layer at or before it.  The loss gradient is drawn by
# the caller at the training output's size.
MERGE_OPS = ("ADD", "MULTIPLY", "CONCATENATE", "MAX", "AVERAGE", "GATED", "ATTENTION_WEIGHTED")


def merge_graphs():
    out = []
    # Tests/test_runtime_residual_merge.cpp:9-47 exactly.
    out.append(("residual_merge_kat",
                [dict(name="skip", type="Identity", inputs=["x"], output="skip"),
                 dict(name="my_residual", type="Multiply", inputs=["x", "scale"], output="x",
                      branch_sources=[0], merge_op="ADD")],
                {"x": [1.0, 2.0], "scale": [2.0, 3.0]}, {}))

    # Every merge operation on a ragged length (the MAX body and its tail),
    # with NaN, infinities and signed zeros on both sides of the merge, so
    # MAX's two forms (vmaxps, std::max) are told apart.
    specials = np.array([np.nan, 1.0, -0.0, 0.0, np.inf, -np.inf, 2.0, np.nan, -3.0, 0.0, -0.0, np.nan, 5.0],
                        np.float32)
    other = np.array([1.0, np.nan, 0.0, -0.0, -np.inf, 7.0, np.nan, np.nan, -3.0, -0.0, 0.0, 4.0, np.nan],
                     np.float32)
    for op in MERGE_OPS:
        out.append((f"merge_{op.lower()}_specials",
                    [dict(name="src", type="Identity", inputs=["b"], output="skipped"),
                     dict(name="block_residual", type="Identity", inputs=["a"], output="x",
                          branch_sources=[0], merge_op=op)],
                    {"a": specials, "b": other}, {}))

    r = _rng(21)
    rows, d = 6, 40
    x = (1.3 * r.standard_normal(rows * d) + 0.3).astype(np.float32)
    ln_w = np.concatenate([1 + 0.1 * r.standard_normal(d), 0.1 * r.standard_normal(d)]).astype(np.float32)
    for op in MERGE_OPS:
        # A pre-norm block whose GELU output is merged with the LayerNorm
        # input's producer, then used downstream (so the merge changes the
        # gradient's inputs, not its routing).
        out.append((f"block_{op.lower()}",
                    [dict(name="inp", type="SiLU", inputs=["__input__"], output="h"),
                     dict(name="ln", type="LayerNorm", inputs=["h"], output="n", in_features=d, weights=ln_w),
                     dict(name="ffn_residual", type="GELU", inputs=["n"], output="g",
                          branch_sources=[0], merge_op=op),
                     dict(name="head", type="LayerNorm", inputs=["g"], output="x", in_features=d if op !=
                          "CONCATENATE" else 0, affine=False)],
                    {"__input__": x}, {}))

    # Sources: the layer itself (merged with its own output), a later layer
    # and a negative index (no merge), a longer source (its head is read), a
    # RESIDUAL type set on a neutral name, a GATE-typed layer with a source
    # (no merge: only RESIDUAL merges), and a chain where a merged output is
    # itself a later merge's source.
    r = _rng(22)
    v = r.standard_normal(24).astype(np.float32)
    long_src = r.standard_normal(48).astype(np.float32)
    out.append(("self_later_negative",
                [dict(name="a_shortcut", type="GELU", inputs=["v"], output="a", branch_sources=[0]),
                 dict(name="b_skip", type="SiLU", inputs=["a"], output="b", branch_sources=[2]),
                 dict(name="c_residual", type="GELU", inputs=["b"], output="c", branch_sources=[-1]),
                 dict(name="d", type="Add", inputs=["c", "a"], output="x")],
                {"v": v}, {}))
    out.append(("longer_source_and_chain",
                [dict(name="wide", type="GELU", inputs=["w"], output="w2"),
                 dict(name="plain", type="SiLU", inputs=["v"], output="p", branch_type="RESIDUAL",
                      branch_sources=[0], merge_op="AVERAGE"),
                 dict(name="gate", type="GELU", inputs=["p"], output="q", branch_sources=[1]),
                 dict(name="chain_residual", type="Multiply", inputs=["q", "v"], output="x",
                      branch_sources=[1], merge_op="MAX")],
                {"v": v, "w": long_src}, {}))
    # A merge into a name read later by its old value's consumers: the
    # merged tensor replaces the name, the source is the value layer s made.
    out.append(("rebound_source",
                [dict(name="s", type="GELU", inputs=["x"], output="h"),
                 dict(name="rebind", type="SiLU", inputs=["x"], output="h"),
                 dict(name="h_residual", type="Identity", inputs=["x"], output="x",
                      branch_sources=[0], merge_op="MULTIPLY"),
                 dict(name="sum", type="Add", inputs=["x", "h"], output="x")],
                {"x": v}, {}))
    return out


def merge_error_graphs():
    """A merge whose source is shorter than the layer's output: the
    reference reads past the source's end (undefined behaviour), the device
    and the restatement refuse it."""
    return [("short_source",
             [dict(name="s", type="Identity", inputs=["short"], output="s"),
              dict(name="r_residual", type="GELU", inputs=["x"], output="x", branch_sources=[0])],
             {"x": np.ones(8, np.float32), "short": np.ones(5, np.float32)}, {})]


# Graphs for the int-ids forward, Model::forwardPass(const std::vector<int>&
# ids, training) (Model.cpp:1026-1349): (name, layers, ids).  The first ones
# run; ids_error_graphs() hold the cases the reference throws on.
def ids_graphs():
    out = []
    r = _rng(31)
    vocab, d, seq = 20, 16, 12
    table = (0.5 * r.standard_normal(vocab * d)).astype(np.float32)
    ln_w = np.concatenate([1 + 0.1 * r.standard_normal(d), 0.1 * r.standard_normal(d)]).astype(np.float32)
    ids = r.integers(-2, vocab + 3, seq).astype(np.int32)
    ids[:3] = 4  # a repeated row: its gradient sums in token order
    ids[5] = 1   # the padding id
    emb = dict(name="tok", type="Embedding", inputs=["x"], output="h", vocab_size=vocab, embed_dim=d,
               padding_idx=1, weights=table)
    out.append(("ids_block",
                [emb,
                 dict(name="ln", type="LayerNorm", inputs=["h"], output="n", in_features=d, weights=ln_w),
                 dict(name="act", type="GELU", inputs=["n"], output="g"),
                 dict(name="res", type="Add", inputs=["g", "h"], output="a"),
                 dict(name="head", type="LogSoftmax", inputs=["a"], output="x")], ids))
    out.append(("ids_default_names",
                [dict(emb, inputs=[], output="x"),
                 dict(name="act", type="GELU"),
                 dict(name="drop", type="Dropout"),
                 dict(name="sm", type="Softmax")], ids))
    out.append(("ids_input_alias_and_broadcast",
                [dict(emb, inputs=["__input__"], output="e"),
                 dict(name="ln", type="LayerNorm", inputs=["e"], output="n", in_features=0, affine=False),
                 dict(name="bias", type="Add", inputs=["n", "n"], output="x")], ids))
    big = np.array([0, 3, (1 << 24) + 1, -(1 << 24) - 3, 2**31 - 1, -2**31, 7], np.int32)
    out.append(("ids_extreme_values", [dict(emb, output="x")], big))
    out.append(("ids_empty", [dict(emb, output="x")], np.zeros(0, np.int32)))
    out.append(("no_layers", [], ids))
    return out


def ids_error_graphs():
    r = _rng(32)
    table = r.standard_normal(5 * 4).astype(np.float32)
    emb = dict(name="tok", type="Embedding", inputs=["x"], output="h", vocab_size=5, embed_dim=4, weights=table)
    ids = np.array([1, 2, 3], np.int32)
    out = []
    for t in ("RMSNorm", "SiLU", "Multiply", "Identity"):  # the int path's strict default (:1311-1319)
        L = dict(name="op", type=t, inputs=["h"] + (["h"] if t == "Multiply" else []), output="x")
        out.append((f"ids_refuses_{t.lower()}", [emb, L], ids))
    out.append(("ids_missing_int_tensor", [dict(emb, inputs=["ids"])], ids))
    out.append(("ids_float_input_not_in_float_store", [emb, dict(name="g", type="GELU", inputs=["x"])], ids))
    out.append(("ids_no_x_result", [emb], ids))
    out.append(("ids_add_one_input", [emb, dict(name="a", type="Add", inputs=["h"], output="x")], ids))
    out.append(("ids_table_too_small", [dict(emb, weights=table[:19], output="x")], ids))
    return out


def checkpoint_layers():
    """The layers of the SafeTensors fixture tests/golden/ref_checkpoint.safetensors
    (written by the reference's save_checkpoint from these weights)."""
    r = _rng(0x5AFE)
    return [
        dict(name="tok", type="Embedding", inputs=["ids"], output="h", vocab_size=10, embed_dim=8,
             weights=r.standard_normal(80).astype(np.float32)),
        dict(name="ln", type="LayerNorm", inputs=["h"], output="n", in_features=8,
             weights=np.concatenate([1 + 0.1 * r.standard_normal(8), 0.1 * r.standard_normal(8)]).astype(np.float32)),
        dict(name="act", type="GELU", inputs=["n"], output="g"),
        dict(name="rms", type="RMSNorm", inputs=["g"], output="x",
             weights=(1 + 0.1 * r.standard_normal(24)).astype(np.float32)),
    ]
