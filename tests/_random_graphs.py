"""Seeded random layer graphs over the layer types of the path, for
differential tests against the reference's own Model (forwardPassNamed and
backwardPass, compiled in place: oracle/model_ref.py).

A graph is (name, layers, float_inputs, int_inputs), as in tests/_graphs.py.
The generator tracks the size of every named float tensor, so most graphs
run; about one in ten carries one deliberate error of a kind the reference
throws on (a missing input, an Add whose sizes do not broadcast
(LayerOps.hpp:190-192), a Multiply size mismatch (:209-211), a LayerNorm
group that does not divide its input).  What is varied:
- wiring: default names ("x" in and out), in-place outputs (a layer writing
  the name it reads), rebinding "x", "__input__" instead of "x", the int
  store's "seq" aliases (text_ids / __input__ / x);
- Add: equal sizes, a scalar, a repeated vector, either operand the small one;
- LayerNorm: per-row groups, the whole vector (in_features 0), affine with and
  without bias, no weight block;
- RMSNorm: affine or not; Softmax / LogSoftmax over the whole vector;
- Embedding: int ids (in range, out of range, padding), float ids rounded
  from the float store, a missing int input filled with seq_len padding ids.
"""
import numpy as np

FORWARD_TYPES = ("LayerNorm", "RMSNorm", "Softmax", "LogSoftmax", "GELU", "SiLU", "Add", "Multiply",
                 "Embedding", "Identity", "Dropout")
BACKWARD_TYPES = tuple(t for t in FORWARD_TYPES if t != "Dropout")
# Draw weights: the element-wise and row ops more often than the rest.
_WEIGHTS = {"LayerNorm": 3, "RMSNorm": 2, "Softmax": 1, "LogSoftmax": 1, "GELU": 2, "SiLU": 2, "Add": 3,
            "Multiply": 2, "Embedding": 1, "Identity": 1, "Dropout": 1}


MERGE_OPS = ("ADD", "MULTIPLY", "CONCATENATE", "MAX", "AVERAGE", "GATED", "ATTENTION_WEIGHTED")


def random_graph(seed, training=False, merges=False):
    """merges=True (training graphs): about a third of the layers also carry a
    residual merge (Model.cpp:6676-6685) -- RESIDUAL from a "_residual" /
    "_skip" / "_shortcut" name or set explicitly, a source drawn among the
    layers so far (or an index that merges nothing), any merge operation.
    A source must hold at least as many floats as the layer's output, or the
    reference reads past its end; CONCATENATE accepts any source."""
    rng = np.random.default_rng(seed)
    types = BACKWARD_TYPES if training else FORWARD_TYPES
    p = np.array([_WEIGHTS[t] for t in types], float)
    p /= p.sum()

    def vec(k, scale=1.0, off=0.0):
        return (off + scale * rng.standard_normal(k)).astype(np.float32)

    d = int(rng.choice([4, 8, 12, 16, 32, 64]))
    rows = int(rng.integers(1, 6))
    n = rows * d
    fin, iin, sizes = {}, {}, {}
    x = vec(n, float(rng.choice([0.5, 1.0, 3.0])), float(rng.choice([0.0, 0.5, -2.0])))
    fin["__input__" if rng.random() < 0.2 else "x"] = x
    sizes["x"] = sizes["__input__"] = n
    if rng.random() < 0.6:
        fin["g"], sizes["g"] = vec(n), n
    if rng.random() < 0.5:
        fin["bias"], sizes["bias"] = vec(d), d
    if rng.random() < 0.3:
        fin["one"], sizes["one"] = vec(1), 1
    int_sizes = {}  # int-store names (read only by an Embedding not finding them as floats)
    if rng.random() < 0.4:
        key = "seq" if rng.random() < 0.5 else "ids"
        iin[key] = rng.integers(-2, 60, int(rng.integers(1, 9))).astype(np.int32)
        for k in (["text_ids", "seq"] if key == "seq" else ["ids"]):
            int_sizes[k] = int(iin[key].size)
    broken = rng.random() < 0.1
    n_layers = int(rng.integers(1, 7))
    bad_at = int(rng.integers(0, n_layers)) if broken else -1
    layers = []
    out_sizes = []  # each layer's output size after its merge

    def pick(exclude=()):
        names = [k for k in sizes if k not in exclude]
        return str(rng.choice(names))

    for i in range(n_layers):
        t = str(rng.choice(types, p=p))
        L = dict(name=f"l{i}_{t.lower()}", type=t)
        bad = i == bad_at
        if t in ("Add", "Multiply"):
            a = pick()
            sa = sizes[a]
            if t == "Multiply":
                same = [k for k in sizes if sizes[k] == sa]
                b = str(rng.choice(same))
                if bad:
                    others = [k for k in sizes if sizes[k] != sa]
                    b = str(rng.choice(others)) if others else "nope"
                out_size = sa
            else:
                ok = [k for k in sizes if sizes[k] == sa or sizes[k] == 1 or sa == 1
                      or max(sizes[k], sa) % min(sizes[k], sa) == 0]
                b = str(rng.choice(ok))
                if bad:
                    nope = [k for k in sizes if k not in ok]
                    b = str(rng.choice(nope)) if nope else "nope"
                out_size = max(sa, sizes.get(b, 0))
            ins = [a, b] if rng.random() < 0.5 else [b, a]
            L["inputs"] = ins
        elif t == "Embedding":
            vocab = int(rng.choice([5, 10, 50]))
            dim = int(rng.choice([4, 8, 16]))
            pad = int(rng.choice([-1, 0, 1, vocab + 1]))
            L.update(vocab_size=vocab, embed_dim=dim, padding_idx=pad,
                     weights=(0.5 * rng.standard_normal(vocab * dim)).astype(np.float32))
            r = rng.random()
            small = [k for k in sizes if sizes[k] <= 64]
            if int_sizes and r < 0.5:
                src = str(rng.choice(sorted(int_sizes)))
            elif r < 0.7 or not small:
                src = "ids_missing"
                seq = int(rng.choice([0, 3, 5]))
                L["seq_len"] = seq
                # filled with padding ids on first use, then kept under that name
                int_sizes.setdefault(src, seq if seq > 0 else 1)
            else:
                src = str(rng.choice(small))
            count = sizes[src] if src in sizes else int_sizes[src]  # the float store is searched first
            L["inputs"] = [src]
            out_size = count * dim
        else:
            src = pick() if rng.random() < 0.75 else "x"
            if src != "x" or rng.random() < 0.5:
                L["inputs"] = [src]
            s = sizes[src]
            out_size = s
            if t == "LayerNorm":
                divs = [k for k in (d, s, s // 2 if s % 2 == 0 else 0, 0) if k == 0 or s % k == 0]
                nn = int(rng.choice(divs))
                if bad:
                    nn = s + 1
                L["in_features"] = nn
                L["eps"] = float(rng.choice([1e-5, 1e-6, 1e-3]))
                g = nn if nn > 0 else s
                r = rng.random()
                if r < 0.15:
                    L["affine"] = False
                elif r < 0.25:
                    pass  # no weight block: no affine transform
                else:
                    use_bias = rng.random() < 0.7
                    L["use_bias"] = use_bias
                    w = [1 + 0.2 * rng.standard_normal(g)] + ([0.2 * rng.standard_normal(g)] if use_bias else [])
                    L["weights"] = np.concatenate(w).astype(np.float32)
            elif t == "RMSNorm":
                L["eps"] = float(rng.choice([1e-5, 1e-6]))
                if rng.random() < 0.7:
                    L["weights"] = (1 + 0.2 * rng.standard_normal(s)).astype(np.float32)
                else:
                    L["affine"] = False
            if bad and t != "LayerNorm":
                L["inputs"] = ["nope"]
        r = rng.random()
        if r < 0.3:
            out = "x"
        elif r < 0.45 and L.get("inputs"):
            out = L["inputs"][0]  # in place
        else:
            out = f"h{int(rng.integers(0, 3))}"
        if out != "x" or rng.random() < 0.5:
            L["output"] = out
        if out in int_sizes:  # keep int-store names out of the float store
            out = "x"
            L["output"] = "x"
        if merges and rng.random() < 0.35:
            i_l = len(layers)
            op = str(rng.choice(MERGE_OPS))
            # Earlier layers with room enough, and the layer itself (always valid).
            ok = [j for j in range(i_l) if op == "CONCATENATE" or out_sizes[j] >= out_size] + [i_l]
            r = rng.random()
            src = int(rng.choice(ok)) if r < 0.85 else int(rng.choice([i_l + 1, -1, i_l + 5]))
            kind = rng.random()
            if kind < 0.5:
                L["name"] += str(rng.choice(["_residual", "_skip", "_shortcut"]))
            elif kind < 0.8:
                L["branch_type"] = "RESIDUAL"
            else:  # a source on a layer whose type does not merge
                L["branch_type"] = str(rng.choice(["GATE", "NONE", "SPLIT"]))
            L["branch_sources"] = [src]
            L["merge_op"] = op
            merging = L.get("branch_type", "RESIDUAL") == "RESIDUAL" and 0 <= src <= i_l
            if merging and op == "CONCATENATE":
                out_size += out_size if src == i_l else out_sizes[src]
        sizes[out] = out_size
        out_sizes.append(out_size)
        layers.append(L)
    return (f"seed{seed}", layers, fin, iin)
