"""Restatement of the reference runtime's forward routing for the layer types
of this path.  TEST INFRASTRUCTURE ONLY: the checker for the device-resident
runtime (mimir_store_run), pinned against the reference's own
Model::forwardPassNamed compiled in place (oracle/model_ref.py).

Follows brit45/mimir-framework Model.cpp:
  forwardPassNamedView   :1385-1408  "x" input = fin["x"] or fin["__input__"] or empty
  forwardPassView        :4638-4680  store "x" and "__input__"; replace the int store
                                      with the named ints ("seq" also under
                                      "text_ids", "__input__", "x"); then the
                                      named floats
  input lookup           :4795-4856  float store first; for Embedding input 0
                                      the int store (ids cast to float), else
                                      seq_len padding ids (stored under that
                                      name); else "Missing input tensor"
  dispatch               :4891-...   per layer type (the op functions of oracle.py)
  output                 :6655,6674  stored under layer.output or "x"
  residual merge         :6676-6685  training only: each layer's output is
                                      kept (all_layer_outputs); a RESIDUAL
                                      layer with a branch source merges its
                                      output with that layer's
                                      (executeBranchComputation :4550-4582,
                                      computeBranchMerge :4344-4479)
  result                 :6823       the float tensor "x"
The encoder's "mag"/"mod" injection (:4670-4700) belongs to the tokenizer /
encoder subsystem and is not restated: graphs here pass such tensors by name.
"""
from __future__ import annotations

import numpy as np

import oracle as O

SUPPORTED = ("LayerNorm", "RMSNorm", "Softmax", "LogSoftmax", "GELU", "SiLU", "Add", "Multiply",
             "Embedding", "Identity", "Dropout")


class ModelError(RuntimeError):
    """Where the reference throws std::runtime_error."""


def _layernorm(x, L):
    w = L.get("weights")
    n = L.get("in_features", 0)
    nn = n if n > 0 else x.size
    if nn <= 0 or x.size % nn:
        raise ModelError("LayerNorm: invalid normalized_size")
    gamma = beta = None
    # LayerOps.hpp:284-285: no weight block (params_count 0) -> no affine
    # transform; a block shorter than gamma|beta is read out of bounds by the
    # reference, and rejected here.
    if L.get("affine", True) and w is not None and np.asarray(w).size > 0:
        w = np.asarray(w, np.float32)
        need = 2 * nn if L.get("use_bias", True) else nn
        if w.size < need:
            raise ModelError("LayerNorm: weight block too small")
        gamma = w[:nn]
        if L.get("use_bias", True):
            beta = w[nn:2 * nn]
    return O.layernorm(x, nn, gamma, beta, L.get("eps", 1e-5))


def _rmsnorm(x, L):
    if x.size == 0:
        return x.copy()
    w = L.get("weights")
    use = L.get("affine", True) and w is not None and np.asarray(w).size > 0
    return O.rmsnorm_whole(x, np.asarray(w, np.float32) if use else None, L.get("eps", 1e-5))


def _embedding(x, L):
    w = L.get("weights")
    vocab = max(1, L.get("vocab_size", 0))
    dim = max(1, L.get("embed_dim", 0))
    if w is None or np.asarray(w).size == 0:
        raise ModelError("Embedding: weights not initialized")
    if np.asarray(w).size < vocab * dim:
        raise ModelError("Embedding: invalid weight size")
    return O.embedding(np.asarray(x, np.float32), np.asarray(w, np.float32), vocab, dim,
                       L.get("padding_idx", -1)).ravel()


def _apply(L, ins):
    t = L["type"]
    x = ins[0]
    if t == "LayerNorm":
        return _layernorm(x, L)
    if t == "RMSNorm":
        return _rmsnorm(x, L)
    if t in ("Softmax", "LogSoftmax"):
        if x.size == 0:
            raise ModelError("Softmax: empty input")
        mode = O.SOFTMAX_LOG if t == "LogSoftmax" else O.SOFTMAX_MUL_INV
        return O.softmax_rows(x, mode).ravel()
    if t == "GELU":
        return O.gelu(x)
    if t == "SiLU":
        return O.silu(x)
    if t in ("Add", "Multiply"):
        if len(ins) < 2:
            raise ModelError(f"{t} layer requires 2 inputs, got {len(ins)}")
        try:
            return O.add(ins[0], ins[1]) if t == "Add" else O.mul(ins[0], ins[1])
        except O.OracleError as e:
            raise ModelError(str(e)) from e
    if t == "Embedding":
        return _embedding(x, L)
    if t in ("Identity", "Dropout"):  # Dropout is the identity at inference (LayerOps.hpp:634-636)
        return x.copy()
    raise ModelError(f"unsupported layer type {t}")


def detect_branch_type(name):
    """Layer::detectBranchType (Layers.hpp:260-304), which Model::push runs on
    every layer's name (Model.cpp:3145): (branch_type, merge_op); merge_op
    keeps its default ADD where the reference leaves it."""
    def has(*w):
        return all(x in name for x in w)
    if has("residual") or has("shortcut") or has("skip"):
        return "RESIDUAL", "ADD"
    if has("concat"):
        return "SKIP_CONNECTION", "CONCATENATE"
    if has("dense", "connect"):
        return "DENSE_CONNECTION", "CONCATENATE"
    if has("attention", "branch"):
        return "ATTENTION_BRANCH", "ATTENTION_WEIGHTED"
    if has("inception") or has("multiscale"):
        return "MULTI_SCALE", "CONCATENATE"
    if has("gate"):
        return "GATE", "GATED"
    if has("split"):
        return "SPLIT", "ADD"
    if has("merge") or has("fusion"):
        return "MERGE", ("ADD" if has("add") else "MULTIPLY" if has("mul") else
                         "CONCATENATE" if has("concat") else "ADD")
    return "NONE", "ADD"


def merge_of(L, i):
    """(source layer, merge_op) of layer i's residual merge, or None:
    executeBranchComputation (Model.cpp:4550-4582) merges only a RESIDUAL
    layer whose first branch source indexes all_layer_outputs, which holds
    layers 0..i at that point."""
    bt, mop = detect_branch_type(L.get("name", ""))
    bt, mop = L.get("branch_type", bt), L.get("merge_op", mop)
    srcs = L.get("branch_sources", [])
    if bt != "RESIDUAL" or not srcs or not 0 <= srcs[0] <= i:
        return None
    return srcs[0], mop


def forward_named(layers, fin=None, iin=None, training=False):
    """Model::forwardPassNamed(fin, iin, training) for the layer types in
    SUPPORTED.  Returns the float32 "x" output.  The training form applies
    the residual merges (and refuses Dropout, whose training form draws a
    random mask)."""
    if training:
        return _forward_snap(layers, fin, iin)[0]
    fin = {k: np.ascontiguousarray(v, np.float32).ravel() for k, v in (fin or {}).items()}
    iin = {k: np.ascontiguousarray(v, np.int32).ravel() for k, v in (iin or {}).items()}
    x0 = fin.get("x", fin.get("__input__", np.zeros(0, np.float32)))
    fstore = {"x": x0, "__input__": x0}
    istore = dict(iin)
    if "seq" in iin:
        for alias in ("text_ids", "__input__", "x"):
            istore[alias] = iin["seq"]
    fstore.update(fin)
    for L in layers:
        names = L.get("inputs") or ["x"]
        ins = []
        for k, name in enumerate(names):
            if name in fstore:
                ins.append(fstore[name])
                continue
            if L["type"] == "Embedding" and k == 0:
                if name not in istore:
                    seq = L.get("seq_len", 0)
                    pad = L.get("padding_idx", -1)
                    istore[name] = np.full(seq if seq > 0 else 1, pad if pad >= 0 else 0, np.int32)
                ins.append(istore[name].astype(np.float32))
                continue
            raise ModelError(f"Missing input tensor: {name}")
        fstore[L.get("output") or "x"] = np.asarray(_apply(L, ins), np.float32).ravel()
    return fstore["x"].copy()


# ---------------------------------------------------------------------------
# Training step without the optimizer: forwardPassNamed(training=true) with
# the input snapshots, then Model::backwardPass (Model.cpp:7307-9153).
# ---------------------------------------------------------------------------

BACKWARD_SUPPORTED = ("LayerNorm", "RMSNorm", "Softmax", "LogSoftmax", "GELU", "SiLU", "Add", "Multiply",
                      "Embedding", "Identity")
# Model.cpp:7390-7402 (needs_input_values_for_backward): Add and Identity
# keep only the input sizes.
_SIZES_ONLY = ("Add", "Identity")


def _forward_snap(layers, fin, iin):
    """forward_named with the per-layer input snapshots the reference keeps in
    training mode (Model.cpp:4858-4878): (values or None, sizes), and the
    residual merges of the training form.  The backward then ignores the
    merges, as Model::backwardPass does: backpropThroughBranch
    (Model.cpp:4584-4613) is never called."""
    fin = {k: np.ascontiguousarray(v, np.float32).ravel() for k, v in (fin or {}).items()}
    iin = {k: np.ascontiguousarray(v, np.int32).ravel() for k, v in (iin or {}).items()}
    x0 = fin.get("x", fin.get("__input__", np.zeros(0, np.float32)))
    fstore = {"x": x0, "__input__": x0}
    istore = dict(iin)
    if "seq" in iin:
        for alias in ("text_ids", "__input__", "x"):
            istore[alias] = iin["seq"]
    fstore.update(fin)
    snaps = []
    outs = []
    for L in layers:
        if L["type"] not in BACKWARD_SUPPORTED:
            raise ModelError(f"unsupported layer type {L['type']} for backward")
        names = L.get("inputs") or ["x"]
        ins = []
        for k, name in enumerate(names):
            if name in fstore:
                ins.append(fstore[name])
                continue
            if L["type"] == "Embedding" and k == 0:
                if name not in istore:
                    seq = L.get("seq_len", 0)
                    pad = L.get("padding_idx", -1)
                    istore[name] = np.full(seq if seq > 0 else 1, pad if pad >= 0 else 0, np.int32)
                ins.append(istore[name].astype(np.float32))
                continue
            raise ModelError(f"Missing input tensor: {name}")
        vals = None if L["type"] in _SIZES_ONLY else [a.copy() for a in ins]
        snaps.append((vals, [a.size for a in ins]))
        out = L.get("output") or "x"
        fstore[out] = np.asarray(_apply(L, ins), np.float32).ravel()
        outs.append(fstore[out])  # all_layer_outputs (Model.cpp:6676-6678)
        m = merge_of(L, len(outs) - 1)
        if m is not None:  # Model.cpp:6681-6685
            try:
                outs[-1] = O.branch_merge(outs[-1], outs[m[0]], m[1])
            except O.OracleError as e:
                raise ModelError(str(e)) from e
            fstore[out] = outs[-1]
    return fstore["x"].copy(), snaps


def backward_named(layers, fin, iin, loss_grad, scales=False):
    """Returns (grads, input_grad) as oracle/model_ref.py's backward: the
    per-layer grad_weights (None for layers without parameters) and the
    gradient that reached "__input__" (None if none did).  With scales=True
    also returns, per layer, the float64 sum of the magnitudes added into each
    grad_weights element (the condition of those float32 sums; None where
    nothing was added), for tolerances that must not depend on cancellation.

    The gradient store mirrors the reference's std::unordered_map of vectors:
    accumulate_grad (Model.cpp:7329-7341) copies into an absent name and adds
    in place into a present one, and a branch's grad_out is a reference into
    that map, so a layer whose input and output share a name adds its input
    gradient onto its own output gradient (numpy in-place ops on the same
    array reproduce this)."""
    _, snaps = _forward_snap(layers, fin, iin)
    return _backward(layers, snaps, loss_grad, scales)


def _backward(layers, snaps, loss_grad, scales):
    """Model::backwardPass over the snapshots of a training forward."""
    grads = []
    for L in layers:
        w = L.get("weights")
        pc = int(L.get("params_count", 0 if w is None else np.asarray(w).size))
        grads.append(np.zeros(pc, np.float32) if pc > 0 else None)
    store = {"x": np.ascontiguousarray(loss_grad, np.float32).ravel().copy()}
    mags = [None] * len(layers)

    def acc(name, src):
        if name not in store:
            store[name] = np.array(src, np.float32, copy=True)
        else:
            dst = store[name]
            if dst.size != src.size:
                raise ModelError("Gradient accumulate: size mismatch")
            O.oracle_accumulate_inplace(dst, src)

    for i in range(len(layers) - 1, -1, -1):
        L = layers[i]
        out = L.get("output") or "x"
        if out not in store:
            continue
        g = store[out]
        names = L.get("inputs") or ["x"]
        vals, sizes = snaps[i]
        n0 = sizes[0] if sizes else 0
        t = L["type"]
        if t == "Embedding":  # :7429-7461
            ids = vals[0]
            vocab = max(1, L.get("vocab_size", 0))
            dim = max(1, L.get("embed_dim", 0))
            if g.size != ids.size * dim:
                continue
            wv = L.get("weights")
            if wv is None or np.asarray(wv).size < vocab * dim or grads[i] is None:
                continue
            grads[i] = O.embedding_bwd(ids, g, grads[i], vocab, dim, L.get("padding_idx", -1))
            m = np.zeros((vocab, dim))
            iid = np.array([int(np.round(v)) if abs(v - np.trunc(v)) != 0.5 else int(np.trunc(v) + np.sign(v))
                            for v in ids.astype(np.float64)], np.int64)
            keep = (iid >= 0) & (iid < vocab) & ~((L.get("padding_idx", -1) >= 0) & (iid == L.get("padding_idx", -1)))
            np.add.at(m, iid[keep], np.abs(g.reshape(-1, dim)[keep].astype(np.float64)))
            mags[i] = np.concatenate([m.ravel(), np.zeros(grads[i].size - m.size)])
        elif t == "Identity":  # :7463-7468
            if g.size != n0:
                continue
            acc(names[0], g)
        elif t == "Add":  # :7541-7601
            if len(sizes) < 2:
                continue
            n1 = sizes[1]
            if g.size == n0 and g.size == n1:
                acc(names[0], g)
                acc(names[1], g)
                continue
            if g.size != n0 and g.size != n1:
                continue
            big0 = g.size == n0
            big_name, small_name = (names[0], names[1]) if big0 else (names[1], names[0])
            small_n = n1 if big0 else n0
            acc(big_name, g)
            if small_n == 1 or (small_n > 1 and g.size % small_n == 0):
                acc(small_name, O.add_bwd_small(g, small_n))
        elif t == "Multiply":  # :7647-7665
            if len(vals) < 2 or g.size != vals[0].size or g.size != vals[1].size:
                continue
            g0, g1 = O.mul_bwd(vals[0], vals[1], g)
            acc(names[0], g0)
            acc(names[1], g1)
        elif t == "LayerNorm":  # :7719-7821
            x = vals[0]
            if g.size != x.size:
                continue
            N = x.size
            feat = L.get("in_features", 0) if L.get("in_features", 0) > 0 else N
            if feat <= 0 or N % feat:
                continue
            affine = bool(L.get("affine", True))
            has_bias = affine and bool(L.get("use_bias", True))
            gamma = None
            if affine:
                wv = L.get("weights")
                need = feat * (2 if has_bias else 1)
                if wv is None or np.asarray(wv).size < need:
                    continue
                gamma = np.asarray(wv, np.float32)[:feat]
            dx, gp = O.layernorm_bwd(x, g, feat, gamma, has_bias, L.get("eps", 1e-5),
                                     None if gamma is None else grads[i][:feat * (2 if has_bias else 1)])
            if gamma is not None:
                grads[i][:gp.size] = gp
                x64 = x.astype(np.float64).reshape(-1, feat)
                xh = (x64 - x64.mean(axis=1, keepdims=True)) / np.sqrt(x64.var(axis=1, keepdims=True) + 1e-5)
                g64 = np.abs(g.astype(np.float64).reshape(-1, feat))
                m = [(g64 * np.abs(xh)).sum(axis=0)] + ([g64.sum(axis=0)] if has_bias else [])
                mags[i] = np.concatenate(m + [np.zeros(grads[i].size - feat * len(m))])
            acc(names[0], dx)
        elif t == "GELU":  # :9026-9051
            if g.size != vals[0].size:
                continue
            acc(names[0], O.gelu_bwd(vals[0], g))
        elif t == "SiLU":  # :7993-8032
            if g.size != vals[0].size:
                continue
            acc(names[0], O.silu_bwd(vals[0], g))
        else:  # RMSNorm, Softmax, LogSoftmax: the fallback at :9133-9140
            if g.size == n0:
                acc(names[0], g)
    gin = store.get("__input__")
    if scales:
        return grads, (None if gin is None else gin.copy()), mags
    return grads, (None if gin is None else gin.copy())


# ---------------------------------------------------------------------------
# The int-ids forward, Model::forwardPassView(const std::vector<int>&,
# training) (Model.cpp:1030-1349), reached by Model::forwardPass(ids)
# (:1026-1028) and the Lua Mimir.Model.forward.
# ---------------------------------------------------------------------------

# The int path's switch (Model.cpp:1242-1321) for the types of this path; the
# others (RMSNorm, SiLU, Multiply, Identity) hit its strict-mode default.
INT_PATH_TYPES = ("LayerNorm", "GELU", "Softmax", "LogSoftmax", "Dropout", "Add", "Embedding")


def _forward_ids_snap(layers, ids, training):
    ids = np.ascontiguousarray(ids, np.int32).ravel()
    if not layers:  # :1033-1037: no layers -> an empty result
        return np.zeros(0, np.float32), []
    istore = {"x": ids, "__input__": ids}  # :1046-1049
    fstore = {}
    snaps = []
    for L in layers:
        names = L.get("inputs") or ["x"]
        t = L["type"]
        if t == "Embedding":  # :1145-1205
            if names[0] not in istore:
                raise ModelError(f"Int tensor not found: {names[0]}")
            v = istore[names[0]]
            snaps.append(([v.astype(np.float32)], [v.size]))  # ids snapshotted as floats (:1160-1165)
            w = L.get("weights")
            vocab = max(1, L.get("vocab_size", 0))
            dim = max(1, L.get("embed_dim", 0))
            if w is None or np.asarray(w).size == 0:
                raise ModelError("Embedding: weights not initialized")
            if np.asarray(w).size < vocab * dim:
                raise ModelError("Embedding: invalid weight size")
            out = O.embedding(v, np.asarray(w, np.float32), vocab, dim, L.get("padding_idx", -1)).ravel()
        else:
            ins = []
            for name in names:
                if name not in fstore:
                    raise ModelError(f"Tensor not found: {name}")
                ins.append(fstore[name])
            snaps.append((None if t in _SIZES_ONLY else [a.copy() for a in ins], [a.size for a in ins]))
            if t not in INT_PATH_TYPES:
                raise ModelError(f"forwardPass(int): layer type not supported in int path: {t}")
            if t == "Add" and len(ins) < 2:
                raise ModelError("Add requires 2 inputs")
            if t == "Dropout" and training:
                raise ModelError("Dropout: its training form draws a random mask")
            out = np.asarray(_apply(L, ins), np.float32).ravel()
        fstore[L.get("output") or "x"] = out
    if "x" not in fstore:  # :1348 getTensor("x")
        raise ModelError("Tensor not found: x")
    return fstore["x"].copy(), snaps


def forward_ids(layers, ids, training=True):
    """Model::forwardPass(const std::vector<int>& ids, training): the float
    "x" result (the reference's default is training=true; the int path has
    no residual merges)."""
    return _forward_ids_snap(layers, ids, training)[0]


def backward_ids(layers, ids, loss_grad, scales=False):
    """forwardPass(ids, training=true) then Model::backwardPass(loss_grad), as
    backward_named returns it."""
    _, snaps = _forward_ids_snap(layers, ids, True)
    return _backward(layers, snaps, loss_grad, scales)
