"""ctypes front end for oracle/_ref/libmimir_ref_model.so: the reference's own
Model::forwardPassNamed (Model.cpp:1352-1408, 4621-6824) and
Model::backwardPass (Model.cpp:7307-9153) on a layer list.
TEST INFRASTRUCTURE ONLY (pins oracle/model_oracle.py; writes golden fixtures)."""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, Structure, c_char, c_char_p, c_float, c_int32, c_int64, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF_MODEL_SO = os.path.join(HERE, "_ref", "libmimir_ref_model.so")


class _Spec(Structure):
    _fields_ = [("name", c_char_p), ("type", c_char_p), ("inputs", c_char_p), ("output", c_char_p),
                ("params_count", c_int64), ("weights", c_void_p), ("eps", c_float),
                ("affine", c_int32), ("use_bias", c_int32), ("in_features", c_int32),
                ("vocab_size", c_int32), ("embed_dim", c_int32), ("padding_idx", c_int32),
                ("seq_len", c_int32), ("branch_type", c_int32), ("merge_op", c_int32),
                ("branch_sources", POINTER(c_int32)), ("n_branch_sources", c_int32),
                ("num_heads", c_int32), ("head_dim", c_int32), ("causal", c_int32)]

# The reference's BranchType and MergeOperation (Layers.hpp:59-80), in order.
BRANCH_TYPES = ("NONE", "RESIDUAL", "SKIP_CONNECTION", "DENSE_CONNECTION", "ATTENTION_BRANCH", "MULTI_SCALE",
                "GATE", "SPLIT", "MERGE")
MERGE_OPS = ("ADD", "MULTIPLY", "CONCATENATE", "MAX", "AVERAGE", "GATED", "ATTENTION_WEIGHTED")


class RefModelError(RuntimeError):
    pass


class _StdoutToStderr:
    """The reference's Model logs to stdout (std::cout); while it runs, file
    descriptor 1 points at stderr so a caller's stdout stays its own."""

    def __enter__(self):
        import sys
        sys.stdout.flush()
        self.saved = os.dup(1)
        os.dup2(2, 1)
        return self

    def __exit__(self, *exc):
        ctypes.CDLL(None).fflush(None)  # C stdio (and std::cout with it) before fd 1 returns
        os.dup2(self.saved, 1)
        os.close(self.saved)


_lib = None


def available() -> bool:
    return os.path.exists(REF_MODEL_SO)


def _load():
    global _lib
    if _lib is None:
        lib = ctypes.CDLL(REF_MODEL_SO)
        f = lib.ref_model_forward
        f.argtypes = [POINTER(_Spec), c_int32, POINTER(c_char_p), POINTER(c_void_p), POINTER(c_int64),
                      c_int32, POINTER(c_char_p), POINTER(c_void_p), POINTER(c_int64), c_int32,
                      c_void_p, c_int64, POINTER(c_int64), c_char_p, c_int32, c_int32]
        f.restype = c_int32
        b = lib.ref_model_backward
        b.argtypes = [POINTER(_Spec), c_int32, POINTER(c_char_p), POINTER(c_void_p), POINTER(c_int64),
                      c_int32, POINTER(c_char_p), POINTER(c_void_p), POINTER(c_int64), c_int32,
                      c_void_p, c_int64, POINTER(c_void_p), c_void_p, c_int64, POINTER(c_int64),
                      c_char_p, c_int32]
        b.restype = c_int32
        fi = lib.ref_model_forward_ids
        fi.argtypes = [POINTER(_Spec), c_int32, c_void_p, c_int64, c_int32, c_void_p, c_int64, POINTER(c_int64),
                       c_void_p, c_int64, POINTER(c_void_p), c_void_p, c_int64, POINTER(c_int64), c_char_p, c_int32]
        fi.restype = c_int32
        sv = lib.ref_model_save_safetensors
        sv.argtypes = [POINTER(_Spec), c_int32, c_char_p, c_char_p, c_int32]
        sv.restype = c_int32
        ld = lib.ref_model_load_safetensors
        ld.argtypes = [POINTER(_Spec), c_int32, c_char_p, c_int32, POINTER(c_void_p), c_char_p, c_int32]
        ld.restype = c_int32
        tl = lib.ref_time_safetensors_load
        tl.argtypes = [POINTER(_Spec), c_int32, c_char_p, c_int32]
        tl.restype = ctypes.c_double
        tf = lib.ref_time_forward_named
        tf.argtypes = [POINTER(_Spec), c_int32, POINTER(c_char_p), POINTER(c_void_p), POINTER(c_int64), c_int32,
                       POINTER(c_char_p), POINTER(c_void_p), POINTER(c_int64), c_int32, c_int32]
        tf.restype = ctypes.c_double
        ts = lib.ref_time_train_step
        ts.argtypes = [POINTER(_Spec), c_int32, POINTER(c_char_p), POINTER(c_void_p), POINTER(c_int64), c_int32,
                       POINTER(c_char_p), POINTER(c_void_p), POINTER(c_int64), c_int32, c_void_p, c_int64,
                       c_int32]
        ts.restype = ctypes.c_double
        _lib = lib
    return _lib


def _marshal(layers, fin, iin):
    fin = fin or {}
    iin = iin or {}
    keep = []
    specs = (_Spec * max(1, len(layers)))()
    for i, L in enumerate(layers):
        w = L.get("weights")
        w = None if w is None else np.ascontiguousarray(w, np.float32)
        srcs = (c_int32 * max(1, len(L.get("branch_sources", []))))(*L.get("branch_sources", []))
        keep += [w, srcs]
        specs[i] = _Spec(L["name"].encode(), L["type"].encode(), ",".join(L.get("inputs", [])).encode(),
                         L.get("output", "").encode(), int(L.get("params_count", 0 if w is None else w.size)),
                         None if w is None else w.ctypes.data, float(L.get("eps", 1e-5)),
                         int(L.get("affine", True)), int(L.get("use_bias", True)),
                         int(L.get("in_features", 0)), int(L.get("vocab_size", 0)),
                         int(L.get("embed_dim", 0)), int(L.get("padding_idx", -1)),
                         int(L.get("seq_len", 0)),
                         BRANCH_TYPES.index(L["branch_type"]) if "branch_type" in L else -1,
                         MERGE_OPS.index(L["merge_op"]) if "merge_op" in L else -1,
                         srcs, len(L.get("branch_sources", [])),
                         int(L.get("num_heads", 8)), int(L.get("head_dim", 0)), int(bool(L.get("causal", False))))
    fa = {k: np.ascontiguousarray(v, np.float32).ravel() for k, v in fin.items()}
    ia = {k: np.ascontiguousarray(v, np.int32).ravel() for k, v in iin.items()}
    keep += list(fa.values()) + list(ia.values())
    fn = (c_char_p * max(1, len(fa)))(*[k.encode() for k in fa])
    fd = (c_void_p * max(1, len(fa)))(*[v.ctypes.data for v in fa.values()])
    fs = (c_int64 * max(1, len(fa)))(*[v.size for v in fa.values()])
    inn = (c_char_p * max(1, len(ia)))(*[k.encode() for k in ia])
    idd = (c_void_p * max(1, len(ia)))(*[v.ctypes.data for v in ia.values()])
    isz = (c_int64 * max(1, len(ia)))(*[v.size for v in ia.values()])
    return keep, (specs, len(layers), fn, fd, fs, len(fa), inn, idd, isz, len(ia))


def forward_named(layers, fin=None, iin=None, out_cap=1 << 24, training=False):
    """layers: list of dicts (see oracle.model_oracle.Layer fields); fin/iin:
    {name: float32 / int32 array}.  Returns the float32 "x" output of
    forwardPassNamed(fin, iin, training)."""
    keep, args = _marshal(layers, fin, iin)
    out = np.empty(out_cap, np.float32)
    n = c_int64(0)
    err = ctypes.create_string_buffer(512)
    with _StdoutToStderr():
        st = _load().ref_model_forward(*args, out.ctypes.data, out_cap, ctypes.byref(n), err, 512,
                                       int(bool(training)))
    del keep
    if st:
        raise RefModelError(err.value.decode(errors="replace"))
    assert n.value <= out_cap, "output larger than out_cap"
    return out[:n.value].copy()


def backward(layers, fin, iin, loss_grad, in_cap=1 << 24):
    """forwardPassNamed(training=true) then backwardPass(loss_grad).  Returns
    (grads, input_grad): grads[i] = the layer's grad_weights (params_count
    floats, or None for a layer without parameters); input_grad = the gradient
    that reached "__input__" (None if none did)."""
    keep, args = _marshal(layers, fin, iin)
    g = np.ascontiguousarray(loss_grad, np.float32).ravel()
    grads = []
    for L in layers:
        w = L.get("weights")
        pc = int(L.get("params_count", 0 if w is None else np.asarray(w).size))
        grads.append(np.zeros(pc, np.float32) if pc > 0 else None)
    gp = (c_void_p * max(1, len(layers)))(*[0 if a is None else a.ctypes.data for a in grads])
    ig = np.empty(in_cap, np.float32)
    n = c_int64(0)
    err = ctypes.create_string_buffer(512)
    with _StdoutToStderr():
        st = _load().ref_model_backward(*args, g.ctypes.data, g.size, gp, ig.ctypes.data, in_cap,
                                        ctypes.byref(n), err, 512)
    del keep
    if st:
        raise RefModelError(err.value.decode(errors="replace"))
    assert n.value <= in_cap, "input gradient larger than in_cap"
    return grads, (None if n.value < 0 else ig[:n.value].copy())


def forward_ids(layers, ids, training=True, loss_grad=None, out_cap=1 << 24, in_cap=1 << 24):
    """Model::forwardPass(const std::vector<int>& ids, training) (the
    reference's default is training=true).  Returns the float32 output; with
    loss_grad (a training forward), also (grads, input_grad) of the
    backwardPass that follows, as backward() returns them."""
    keep, args = _marshal(layers, {}, {})
    ids = np.ascontiguousarray(ids, np.int32).ravel()
    out = np.empty(out_cap, np.float32)
    n = c_int64(0)
    grads, gp, ig, lg = [], None, None, None
    if loss_grad is not None:
        lg = np.ascontiguousarray(loss_grad, np.float32).ravel()
        for L in layers:
            w = L.get("weights")
            pc = int(L.get("params_count", 0 if w is None else np.asarray(w).size))
            grads.append(np.zeros(pc, np.float32) if pc > 0 else None)
        gp = (c_void_p * max(1, len(layers)))(*[0 if a is None else a.ctypes.data for a in grads])
        ig = np.empty(in_cap, np.float32)
    n_in = c_int64(0)
    err = ctypes.create_string_buffer(512)
    with _StdoutToStderr():
        st = _load().ref_model_forward_ids(args[0], args[1], ids.ctypes.data, ids.size, int(bool(training)),
                                           out.ctypes.data, out_cap, ctypes.byref(n),
                                           None if lg is None else lg.ctypes.data, 0 if lg is None else lg.size,
                                           gp, None if ig is None else ig.ctypes.data, in_cap, ctypes.byref(n_in),
                                           err, 512)
    del keep
    if st:
        raise RefModelError(err.value.decode(errors="replace"))
    y = out[:n.value].copy()
    if loss_grad is None:
        return y
    return y, (grads, None if n_in.value < 0 else ig[:n_in.value].copy())


def save_safetensors(layers, path):
    """The reference's save_checkpoint (SafeTensors) of a model with these layers."""
    keep, args = _marshal(layers, {}, {})
    err = ctypes.create_string_buffer(512)
    with _StdoutToStderr():
        st = _load().ref_model_save_safetensors(args[0], args[1], str(path).encode(), err, 512)
    del keep
    if st:
        raise RefModelError(err.value.decode(errors="replace"))


def load_safetensors(layers, path, strict=True):
    """The reference's load_checkpoint (SafeTensors, weights only) into a model
    with these layers; returns each layer's weight block afterwards (None for
    layers without one).  Raises RefModelError with the reference's message."""
    keep, args = _marshal(layers, {}, {})
    outs = []
    for L in layers:
        w = L.get("weights")
        pc = int(L.get("params_count", 0 if w is None else np.asarray(w).size))
        outs.append(np.zeros(pc, np.float32) if pc > 0 else None)
    ptrs = (c_void_p * max(1, len(layers)))(*[0 if a is None else a.ctypes.data for a in outs])
    err = ctypes.create_string_buffer(512)
    with _StdoutToStderr():
        st = _load().ref_model_load_safetensors(args[0], args[1], str(path).encode(), int(bool(strict)), ptrs, err,
                                                512)
    del keep
    if st:
        raise RefModelError(err.value.decode(errors="replace"))
    return outs


def time_safetensors_load(layers, path, reps=3):
    """Median seconds of the reference's load_checkpoint (SafeTensors, weights
    only) into a model built once with these layers (warm page cache)."""
    keep, args = _marshal(layers, {}, {})
    with _StdoutToStderr():
        t = _load().ref_time_safetensors_load(args[0], args[1], str(path).encode(), int(reps))
    del keep
    if t < 0:
        raise RefModelError("load_checkpoint failed")
    return t


def time_train_step(layers, fin, iin, loss_grad, reps=3):
    """Median seconds of one reference training step (forwardPassNamed with
    training=true, then backwardPass(loss_grad)) on a model built once."""
    keep, args = _marshal(layers, fin, iin)
    g = np.ascontiguousarray(loss_grad, np.float32).ravel()
    with _StdoutToStderr():
        t = _load().ref_time_train_step(*args, g.ctypes.data, g.size, int(reps))
    del keep
    if t < 0:
        raise RefModelError("training step failed")
    return t


def time_forward_named(layers, fin=None, iin=None, reps=3):
    """Median seconds of the reference's Model::forwardPassNamed (inference)
    on a model built once with these layers."""
    keep, args = _marshal(layers, fin, iin)
    with _StdoutToStderr():
        t = _load().ref_time_forward_named(*args, int(reps))
    del keep
    if t < 0:
        raise RefModelError("forwardPassNamed failed")
    return t
