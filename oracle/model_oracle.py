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


def forward_named(layers, fin=None, iin=None):
    """Model::forwardPassNamed(fin, iin, training=false) for the layer types
    in SUPPORTED.  Returns the float32 "x" output."""
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
