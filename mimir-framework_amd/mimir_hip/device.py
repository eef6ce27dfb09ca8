"""Device context, buffers and the per-op calls of libmimir_hip.

Everything here is a thin layer over the C ABI: buffers are device memory
owned by a :class:`Context`, ops enqueue on the context's stream and return,
and a non-OK status raises :class:`MimirError` carrying the library's message.
"""
from __future__ import annotations

import ctypes
import weakref
from ctypes import byref, c_float, c_void_p

import numpy as np

from . import _lib
from ._lib import EDEVICE, EINVAL, ENOMEM, OK


class MimirError(RuntimeError):
    """A non-OK status from libmimir_hip (status code in ``.status``)."""

    def __init__(self, status, message):
        super().__init__(f"[status {status}] {message}")
        self.status = status


class DeviceArray:
    """A device buffer with a numpy-style shape and dtype."""

    def __init__(self, ctx, ptr, shape, dtype, owned=True):
        self.ctx = ctx
        self.ptr = ptr
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.owned = owned

    @property
    def size(self):
        n = 1
        for s in self.shape:
            n *= s
        return n

    @property
    def nbytes(self):
        return self.size * self.dtype.itemsize

    def offset(self, elements, shape=None):
        """A non-owning view starting `elements` items in."""
        return DeviceArray(self.ctx, self.ptr + elements * self.dtype.itemsize,
                           shape if shape is not None else (self.size - elements,),
                           self.dtype, owned=False)

    def numpy(self):
        out = np.empty(self.shape, self.dtype)
        self.ctx.download(out, self)
        return out

    def upload(self, arr):
        self.ctx.upload(self, arr)

    def free(self):
        if self.owned and self.ptr:
            self.ctx.free(self)
        self.ptr = 0

    def __int__(self):
        return self.ptr


def _ptr(x):
    if x is None:
        return None
    if isinstance(x, DeviceArray):
        return c_void_p(x.ptr) if x.ptr else None
    if isinstance(x, int):
        return c_void_p(x) if x else None
    raise TypeError(f"expected a DeviceArray or a device address, got {type(x)}")


class Context:
    """One HIP device + stream (``mimir_ctx``)."""

    def __init__(self, device=0):
        self.lib = _lib.load()
        h = c_void_p()
        st = self.lib.mimir_ctx_create(int(device), byref(h))
        if st != OK:
            raise MimirError(st, f"mimir_ctx_create(device={device}) failed")
        self.handle = h
        self.device = device

    # -- status ---------------------------------------------------------
    def check(self, st, what=""):
        if st != OK:
            msg = self.lib.mimir_last_error(self.handle)
            raise MimirError(st, (msg.decode() if msg else "") or what)

    def close(self):
        if getattr(self, "handle", None):
            self.lib.mimir_ctx_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- memory ---------------------------------------------------------
    def empty(self, shape, dtype=np.float32):
        shape = (shape,) if isinstance(shape, int) else tuple(shape)
        n = int(np.prod(shape)) * np.dtype(dtype).itemsize
        p = c_void_p()
        self.check(self.lib.mimir_malloc(self.handle, max(n, 1), byref(p)), "mimir_malloc")
        return DeviceArray(self, p.value, shape, dtype)

    def free(self, arr):
        self.check(self.lib.mimir_free(self.handle, _ptr(arr)), "mimir_free")

    def to_device(self, arr, dtype=None):
        a = np.ascontiguousarray(arr, dtype=dtype)
        d = self.empty(a.shape, a.dtype)
        self.upload(d, a)
        return d

    def upload(self, dst, arr):
        a = np.ascontiguousarray(arr)
        assert a.nbytes <= dst.nbytes, "upload larger than the buffer"
        self.check(self.lib.mimir_upload(self.handle, _ptr(dst), a.ctypes.data_as(c_void_p), a.nbytes),
                   "mimir_upload")

    def download(self, out, src):
        assert out.flags["C_CONTIGUOUS"] and out.nbytes <= src.nbytes
        self.check(self.lib.mimir_download(self.handle, out.ctypes.data_as(c_void_p), _ptr(src),
                                           out.nbytes), "mimir_download")

    def copy(self, dst, src, nbytes):
        self.check(self.lib.mimir_copy(self.handle, _ptr(dst), _ptr(src), nbytes), "mimir_copy")

    def fill(self, dst, value, n=None):
        n = dst.size if n is None else n
        self.check(self.lib.mimir_fill_f32(self.handle, _ptr(dst), n, value), "mimir_fill_f32")

    def sync(self):
        self.check(self.lib.mimir_sync(self.handle), "mimir_sync")

    def set_alloc_limit(self, nbytes):
        self.check(self.lib.mimir_ctx_set_alloc_limit(self.handle, nbytes))

    def set_output_caching(self, keep):
        """Ops enqueued next store their outputs through the caches (keep=True),
        for a consumer launched right after, or stream them (False, default)."""
        self.check(self.lib.mimir_ctx_set_output_caching(self.handle, 1 if keep else 0))

    # -- timing ---------------------------------------------------------
    def event(self):
        return Event(self)

    # -- ops (device pointers; enqueue only) -----------------------------
    def layernorm(self, x, gamma, beta, y, groups, n, eps):
        self.check(self.lib.mimir_layernorm_fwd(self.handle, _ptr(x), _ptr(gamma), _ptr(beta),
                                                _ptr(y), groups, n, eps))

    def rmsnorm(self, x, w, w_len, y, rows, cols, eps):
        self.check(self.lib.mimir_rmsnorm_fwd(self.handle, _ptr(x), _ptr(w), w_len, _ptr(y), rows,
                                              cols, eps))

    def add_rmsnorm(self, x, residual, residual_out, w, y, rows, cols, eps):
        self.check(self.lib.mimir_add_rmsnorm_fwd(self.handle, _ptr(x), _ptr(residual),
                                                  _ptr(residual_out), _ptr(w), _ptr(y), rows, cols,
                                                  eps))

    def softmax(self, x, y, rows, cols, mode=_lib.SOFTMAX_DIV_EPS):
        self.check(self.lib.mimir_softmax_fwd(self.handle, _ptr(x), _ptr(y), rows, cols, mode))

    def gelu(self, x, y, n):
        self.check(self.lib.mimir_gelu_fwd(self.handle, _ptr(x), _ptr(y), n))

    def silu(self, x, y, n):
        self.check(self.lib.mimir_silu_fwd(self.handle, _ptr(x), _ptr(y), n))

    def silu_mul(self, gate, up, y, n):
        self.check(self.lib.mimir_silu_mul_fwd(self.handle, _ptr(gate), _ptr(up), _ptr(y), n))

    def gelu_mul(self, gate, up, y, n):
        self.check(self.lib.mimir_gelu_mul_fwd(self.handle, _ptr(gate), _ptr(up), _ptr(y), n))

    def add(self, a, na, b, nb, y):
        self.check(self.lib.mimir_add_fwd(self.handle, _ptr(a), na, _ptr(b), nb, _ptr(y)))

    def mul(self, a, na, b, nb, y):
        self.check(self.lib.mimir_mul_fwd(self.handle, _ptr(a), na, _ptr(b), nb, _ptr(y)))

    def branch_merge(self, a, na, b, nb, y, merge_op):
        """merge_op: a MergeOperation name ("ADD", "MAX", ...) or its code."""
        op = _lib.MERGE_OPS.index(merge_op) if isinstance(merge_op, str) else int(merge_op)
        self.check(self.lib.mimir_branch_merge_fwd(self.handle, _ptr(a), na, _ptr(b), nb, _ptr(y), op))

    def embedding(self, ids, n_ids, table, table_len, vocab, dim, padding_idx, y, float_ids=False):
        fn = self.lib.mimir_embedding_f32ids_fwd if float_ids else self.lib.mimir_embedding_fwd
        self.check(fn(self.handle, _ptr(ids), n_ids, _ptr(table), table_len, vocab, dim,
                      padding_idx, _ptr(y)))

    def rope(self, q, q_out, q_heads, k, k_out, k_heads, batch, seq, head_dim, pos_offset,
             cos_tab, sin_tab, table_rows):
        self.check(self.lib.mimir_rope_fwd(self.handle, _ptr(q), _ptr(q_out), q_heads, _ptr(k),
                                           _ptr(k_out), k_heads, batch, seq, head_dim, pos_offset,
                                           _ptr(cos_tab), _ptr(sin_tab), table_rows))

    def attention(self, q, k, v, out, batch, q_len, kv_len, heads, head_dim, causal=False, scale=None,
                  ld_q=None, ld_kv=None, ld_out=None):
        """mimir_attention_fwd: softmax(Q K^T * scale, causal) V per head; the
        row strides default to heads * head_dim (separate Q / K / V / out)."""
        width = heads * head_dim
        if scale is None:
            scale = float(np.float32(1.0) / np.sqrt(np.float32(head_dim)))  # LayerOps.hpp:1047
        self.check(self.lib.mimir_attention_fwd(self.handle, _ptr(q), ld_q or width, _ptr(k), _ptr(v),
                                                ld_kv or width, _ptr(out), ld_out or width, batch, q_len,
                                                kv_len, heads, head_dim, float(scale), int(bool(causal))))

    def self_attention(self, x, seq_len, embed_dim, num_heads, causal, weights, weights_len, out):
        """mimir_self_attention_fwd: the SelfAttention layer on device buffers."""
        self.check(self.lib.mimir_self_attention_fwd(self.handle, _ptr(x), seq_len, embed_dim, num_heads,
                                                     int(bool(causal)), _ptr(weights), weights_len, _ptr(out)))

    def cross_attention(self, xq, query_len, xkv, kv_len, embed_dim, num_heads, causal, weights, weights_len, out):
        """mimir_cross_attention_fwd: the CrossAttention layer on device buffers."""
        self.check(self.lib.mimir_cross_attention_fwd(self.handle, _ptr(xq), query_len, _ptr(xkv), kv_len, embed_dim,
                                                      num_heads, int(bool(causal)), _ptr(weights), weights_len,
                                                      _ptr(out)))

    # -- backward (Model::backwardPass branches) -------------------------------

    def attention_bwd(self, q, k, v, dout, dq, dk, dv, batch, q_len, kv_len, heads, head_dim, causal=False,
                      scale=None, ld_q=None, ld_kv=None, ld_dout=None, ld_dq=None, ld_dkv=None):
        """mimir_attention_bwd: dq / dk / dv of the attention core from dout,
        strides as for attention() (default heads * head_dim)."""
        width = heads * head_dim
        if scale is None:
            scale = float(np.float32(1.0) / np.sqrt(np.float32(head_dim)))
        self.check(self.lib.mimir_attention_bwd(self.handle, _ptr(q), ld_q or width, _ptr(k), _ptr(v), ld_kv or width,
                                                _ptr(dout), ld_dout or width, _ptr(dq), ld_dq or width, _ptr(dk),
                                                _ptr(dv), ld_dkv or width, batch, q_len, kv_len, heads, head_dim,
                                                float(scale), int(bool(causal))))

    def self_attention_bwd(self, x, dy, seq_len, embed_dim, num_heads, causal, weights, weights_len, grad_weights,
                           dx, accumulate=False):
        """mimir_self_attention_bwd: backward_self_attention on device buffers
        (grad_weights may be None)."""
        self.check(self.lib.mimir_self_attention_bwd(self.handle, _ptr(x), _ptr(dy), seq_len, embed_dim, num_heads,
                                                     int(bool(causal)), _ptr(weights), weights_len,
                                                     _ptr(grad_weights), _ptr(dx), int(bool(accumulate))))

    def cross_attention_bwd(self, xq, query_len, xkv, kv_len, dy, embed_dim, num_heads, causal, weights, weights_len,
                            grad_weights, dxq, dxkv, acc_q=False, acc_kv=False):
        """mimir_cross_attention_bwd: backward_cross_attention on device buffers."""
        self.check(self.lib.mimir_cross_attention_bwd(self.handle, _ptr(xq), query_len, _ptr(xkv), kv_len, _ptr(dy),
                                                      embed_dim, num_heads, int(bool(causal)), _ptr(weights),
                                                      weights_len, _ptr(grad_weights), _ptr(dxq), int(bool(acc_q)),
                                                      _ptr(dxkv), int(bool(acc_kv))))

    def layernorm_bwd(self, x, dy, gamma, dx, dgamma, dbeta, groups, n, eps, accumulate=False):
        self.check(self.lib.mimir_layernorm_bwd(self.handle, _ptr(x), _ptr(dy), _ptr(gamma), _ptr(dx),
                                                _ptr(dgamma), _ptr(dbeta), groups, n, eps,
                                                int(bool(accumulate))))

    def gelu_bwd(self, x, dy, dx, n, accumulate=False):
        self.check(self.lib.mimir_gelu_bwd(self.handle, _ptr(x), _ptr(dy), _ptr(dx), n, int(bool(accumulate))))

    def silu_bwd(self, x, dy, dx, n, accumulate=False):
        self.check(self.lib.mimir_silu_bwd(self.handle, _ptr(x), _ptr(dy), _ptr(dx), n, int(bool(accumulate))))

    def mul_bwd(self, a, b, dy, da, db, n, acc_a=False, acc_b=False):
        self.check(self.lib.mimir_mul_bwd(self.handle, _ptr(a), _ptr(b), _ptr(dy), _ptr(da), _ptr(db), n,
                                          int(bool(acc_a)), int(bool(acc_b))))

    def add_bwd(self, dy, na, nb, da, db, acc_a=False, acc_b=False):
        self.check(self.lib.mimir_add_bwd(self.handle, _ptr(dy), na, nb, _ptr(da), _ptr(db),
                                          int(bool(acc_a)), int(bool(acc_b))))

    def embedding_bwd(self, ids, n_ids, dy, grad_table, table_len, vocab, dim, padding_idx, float_ids=False):
        fn = self.lib.mimir_embedding_f32ids_bwd if float_ids else self.lib.mimir_embedding_bwd
        self.check(fn(self.handle, _ptr(ids), n_ids, _ptr(dy), _ptr(grad_table), table_len, vocab, dim,
                      padding_idx))


class Event:
    """A stream-ordered timing event (``mimir_event``)."""

    def __init__(self, ctx):
        self.ctx = ctx
        h = c_void_p()
        ctx.check(ctx.lib.mimir_event_create(ctx.handle, byref(h)), "mimir_event_create")
        self.handle = h

    def record(self):
        self.ctx.check(self.ctx.lib.mimir_event_record(self.ctx.handle, self.handle))

    def elapsed_ms(self, stop):
        ms = c_float()
        st = self.ctx.lib.mimir_event_elapsed_ms(self.handle, stop.handle, byref(ms))
        if st != OK:
            raise MimirError(st, "mimir_event_elapsed_ms")
        return ms.value

    def close(self):
        if self.handle:
            self.ctx.lib.mimir_event_destroy(self.handle)
            self.handle = None


def rope_table(rows, head_dim, theta=10000.0):
    """Host cos/sin tables [rows x head_dim/2] from mimir_rope_table."""
    lib = _lib.load()
    half = head_dim // 2
    c = np.empty((rows, half), np.float32)
    s = np.empty((rows, half), np.float32)
    st = lib.mimir_rope_table(rows, head_dim, float(theta), c.ctypes.data_as(c_void_p),
                              s.ctypes.data_as(c_void_p))
    if st != OK:
        raise MimirError(st, "mimir_rope_table: invalid argument")
    return c, s


class Store:
    """Device-resident named tensor store + layer runner (mimir_store_*)."""

    def __init__(self, ctx: Context):
        self.ctx = ctx
        h = c_void_p()
        ctx.check(ctx.lib.mimir_store_create(ctx.handle, byref(h)), "mimir_store_create")
        self.handle = h
        self._graphs = weakref.WeakSet()  # StoreGraphs captured on this store

    def close(self):
        """mimir_store_destroy, which also destroys every graph captured on
        this store: their StoreGraph objects are closed with it."""
        if self.handle:
            self.ctx.check(self.ctx.lib.mimir_store_destroy(self.handle), "mimir_store_destroy")
            self.handle = None
        for sg in list(self._graphs):
            sg._destroyed_by_store()
        self._graphs.clear()

    def clear(self):
        self.ctx.check(self.ctx.lib.mimir_store_clear(self.handle))

    def put(self, name, arr):
        a = np.ascontiguousarray(arr)
        dt = _lib.DTYPE_I32 if a.dtype.kind in "iu" else _lib.DTYPE_F32
        a = np.ascontiguousarray(a, np.int32 if dt == _lib.DTYPE_I32 else np.float32).ravel()
        self.ctx.check(self.ctx.lib.mimir_store_put(self.handle, name.encode(), dt, a.ctypes.data_as(c_void_p),
                                                    a.size))

    def info(self, name, dtype=_lib.DTYPE_F32):
        p, n = c_void_p(), ctypes.c_int64()
        self.ctx.check(self.ctx.lib.mimir_store_info(self.handle, name.encode(), dtype, byref(p), byref(n)))
        return p.value, n.value

    def get(self, name, dtype=_lib.DTYPE_F32):
        _, n = self.info(name, dtype)
        out = np.empty(n, np.int32 if dtype == _lib.DTYPE_I32 else np.float32)
        got = ctypes.c_int64()
        self.ctx.check(self.ctx.lib.mimir_store_get(self.handle, name.encode(), dtype,
                                                    out.ctypes.data_as(c_void_p), n, byref(got)))
        return out

    def set_inputs(self, fin=None, iin=None):
        fin = {k: np.ascontiguousarray(v, np.float32).ravel() for k, v in (fin or {}).items()}
        iin = {k: np.ascontiguousarray(v, np.int32).ravel() for k, v in (iin or {}).items()}
        nf, ni = len(fin), len(iin)
        fn = (ctypes.c_char_p * max(1, nf))(*[k.encode() for k in fin])
        fd = (c_void_p * max(1, nf))(*[v.ctypes.data for v in fin.values()])
        fs = (ctypes.c_int64 * max(1, nf))(*[v.size for v in fin.values()])
        inn = (ctypes.c_char_p * max(1, ni))(*[k.encode() for k in iin])
        idd = (c_void_p * max(1, ni))(*[v.ctypes.data for v in iin.values()])
        isz = (ctypes.c_int64 * max(1, ni))(*[v.size for v in iin.values()])
        self.ctx.check(self.ctx.lib.mimir_store_set_inputs(self.handle, fn, fd, fs, nf, inn, idd, isz, ni))

    def set_fusion(self, enable=True):
        """mimir_store_set_fusion: elementwise chains of a run as one kernel."""
        self.ctx.check(self.ctx.lib.mimir_store_set_fusion(self.handle, int(bool(enable))))

    def run(self, graph: "DeviceGraph"):
        self.ctx.check(self.ctx.lib.mimir_store_run(self.handle, graph.c_layers, len(graph.layers)))

    def run_training(self, graph: "DeviceGraph"):
        self.ctx.check(self.ctx.lib.mimir_store_run_training(self.handle, graph.c_layers, len(graph.layers)))

    def backward(self, graph: "DeviceGraph", loss_grad):
        """Model::backwardPass(loss_grad): a host array (the reference's form),
        or a DeviceArray already on the GPU (mimir_store_backward_dev)."""
        if isinstance(loss_grad, DeviceArray):
            self.ctx.check(self.ctx.lib.mimir_store_backward_dev(self.handle, graph.c_layers, len(graph.layers),
                                                                 c_void_p(loss_grad.ptr), loss_grad.size))
            return
        g = np.ascontiguousarray(loss_grad, np.float32).ravel()
        self.ctx.check(self.ctx.lib.mimir_store_backward(self.handle, graph.c_layers, len(graph.layers),
                                                         g.ctypes.data_as(c_void_p), g.size))

    def grad(self, name):
        """The gradient that reached `name` in the last backward, or None."""
        p, n = c_void_p(), ctypes.c_int64()
        st = self.ctx.lib.mimir_store_grad_info(self.handle, name.encode(), byref(p), byref(n))
        if st != 0:
            return None
        out = np.empty(n.value, np.float32)
        got = ctypes.c_int64()
        self.ctx.check(self.ctx.lib.mimir_store_grad_get(self.handle, name.encode(), out.ctypes.data_as(c_void_p),
                                                         n.value, byref(got)))
        return out

    def train_step(self, graph: "DeviceGraph", fin, iin, loss_grad):
        """Model::forwardPassNamed(training=true) then Model::backwardPass on
        the device.  Returns (grads, input_grad): each layer's grad_weights
        after the step (host copies, None for layers without weights) and the
        gradient that reached "__input__" (None if none did)."""
        self.set_inputs(fin, iin)
        self.run_training(graph)
        self.backward(graph, loss_grad)
        return graph.grads(), self.grad("__input__")

    def set_input_ids(self, ids):
        ids = np.ascontiguousarray(ids, np.int32).ravel()
        self.ctx.check(self.ctx.lib.mimir_store_set_input_ids(self.handle, ids.ctypes.data_as(c_void_p), ids.size))

    def run_ids(self, graph: "DeviceGraph", training=True):
        self.ctx.check(self.ctx.lib.mimir_store_run_ids(self.handle, graph.c_layers, len(graph.layers),
                                                        int(bool(training))))

    def forward_ids(self, graph: "DeviceGraph", ids, training=True):
        """Model::forwardPass(const std::vector<int>& ids, training) on the
        device (the reference's default is training=true).  Returns the float
        "x" output (empty for a graph without layers)."""
        self.set_input_ids(ids)
        self.run_ids(graph, training)
        return self.get("x") if graph.layers else np.zeros(0, np.float32)

    def train_step_ids(self, graph: "DeviceGraph", ids, loss_grad):
        """forwardPass(ids, training=true) then Model::backwardPass."""
        self.set_input_ids(ids)
        self.run_ids(graph, True)
        self.backward(graph, loss_grad)
        return graph.grads(), self.grad("__input__")

    def capture(self, graph: "DeviceGraph", fin=None, iin=None):
        """set_inputs(fin, iin), then mimir_store_capture of graph's forward:
        a StoreGraph to replay it."""
        self.set_inputs(fin, iin)
        return StoreGraph(self, graph)

    def forward_named(self, graph: "DeviceGraph", fin=None, iin=None, training=False):
        """Model::forwardPassNamed(fin, iin, training) on the device (the
        training form keeps the backward's snapshots and applies the
        layers' residual merges)."""
        self.set_inputs(fin, iin)
        (self.run_training if training else self.run)(graph)
        return self.get("x")


class StoreGraph:
    """A captured forward (mimir_store_capture): set_input() the tensors bound
    at capture, launch(), get() what the run left bound."""

    def __init__(self, store: "Store", graph: "DeviceGraph"):
        self.store, self.ctx = store, store.ctx
        self.handle = None
        # The captured kernels hold graph's weight and gradient addresses:
        # graph refuses to free them while this graph is open.
        self._graph = graph
        h = c_void_p()
        self.ctx.check(self.ctx.lib.mimir_store_capture(store.handle, graph.c_layers, len(graph.layers), byref(h)))
        self.handle = h
        store._graphs.add(self)
        graph._holders.add(self)

    def _live(self):
        if not self.handle:
            raise MimirError(EINVAL, "StoreGraph: closed (by close() or by closing its Store)")
        return self.handle

    def _release(self):
        if self._graph is not None:
            self._graph._holders.discard(self)
            self._graph = None

    def _destroyed_by_store(self):
        # mimir_store_destroy freed the C graph: only forget the handle.
        self.handle = None
        self._release()

    def set_input(self, name, arr):
        a = np.ascontiguousarray(arr)
        dt = _lib.DTYPE_I32 if a.dtype.kind in "iu" else _lib.DTYPE_F32
        a = np.ascontiguousarray(a, np.int32 if dt == _lib.DTYPE_I32 else np.float32).ravel()
        self.ctx.check(self.ctx.lib.mimir_store_graph_set_input(self._live(), name.encode(), dt,
                                                                a.ctypes.data_as(c_void_p), a.size))

    def launch(self):
        self.ctx.check(self.ctx.lib.mimir_store_graph_launch(self._live()))

    def get(self, name="x", dtype=_lib.DTYPE_F32):
        h = self._live()
        n = ctypes.c_int64()
        self.ctx.check(self.ctx.lib.mimir_store_graph_get(h, name.encode(), dtype, None, 0, byref(n)))
        out = np.empty(n.value, np.int32 if dtype == _lib.DTYPE_I32 else np.float32)
        self.ctx.check(self.ctx.lib.mimir_store_graph_get(h, name.encode(), dtype,
                                                          out.ctypes.data_as(c_void_p), n.value, byref(n)))
        return out

    def close(self):
        """mimir_store_graph_destroy; does nothing once closed, also when its
        Store's close() already destroyed the graph."""
        if self.handle:
            self.ctx.check(self.ctx.lib.mimir_store_graph_destroy(self.handle))
            self.handle = None
            self.store._graphs.discard(self)
        self._release()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def branch_fields(L):
    """(branch_type, merge_op) codes of a layer dict: what Model::push's
    detectBranchType gives its name, unless the dict sets "branch_type" or
    "merge_op" (names of BranchType / MergeOperation) as a caller may set the
    Layer fields afterwards."""
    bt, mop = _lib.detect_branch_type(L.get("name", ""))
    bt, mop = L.get("branch_type", bt), L.get("merge_op", mop)
    return _lib.BRANCH_TYPES.index(bt), _lib.MERGE_OPS.index(mop)


class DeviceGraph:
    """A layer list (dicts with the reference Layer fields and host `weights`)
    with its weight blocks uploaded once to the device, and a zeroed device
    gradient block (Layer::grad_weights) per weighted layer."""

    def __init__(self, ctx: Context, layers):
        self.ctx = ctx
        self.layers = list(layers)
        self._holders = weakref.WeakSet()  # open StoreGraphs whose kernels use these buffers
        self._keep = []
        self.weights = []
        self.grad_bufs = []
        arr = (_lib.Layer_C * max(1, len(self.layers)))()
        for i, L in enumerate(self.layers):
            w = L.get("weights")
            dw = dg = None
            if w is not None and np.asarray(w).size > 0:
                dw = ctx.to_device(np.ascontiguousarray(w, np.float32).ravel())
                dg = ctx.to_device(np.zeros(dw.size, np.float32))
            self.weights.append(dw)
            self.grad_bufs.append(dg)
            names = [n.encode() for n in L.get("inputs", [])]
            cnames = (ctypes.c_char_p * max(1, len(names)))(*names)
            name_b, out_b = L.get("name", "").encode(), L.get("output", "").encode()
            bt, mop = branch_fields(L)
            srcs = list(L.get("branch_sources", []))
            csrcs = (ctypes.c_int32 * max(1, len(srcs)))(*srcs)
            self._keep += [cnames, name_b, out_b, csrcs]
            arr[i] = _lib.Layer_C(
                _lib.LAYER_TYPES.get(L["type"], -1), name_b, cnames, len(names), out_b,
                dw.ptr if dw is not None else None, 0 if dw is None else dw.size,
                float(L.get("eps", 1e-5)), int(L.get("affine", True)), int(L.get("use_bias", True)),
                int(L.get("in_features", 0)), int(L.get("vocab_size", 0)), int(L.get("embed_dim", 0)),
                int(L.get("padding_idx", -1)), int(L.get("seq_len", 0)),
                dg.ptr if dg is not None else None, bt, mop, csrcs, len(srcs),
                int(L.get("num_heads", 8)), int(L.get("head_dim", 0)), int(bool(L.get("causal", False))))
        self.c_layers = arr

    def grads(self):
        """Host copies of the device grad_weights blocks (None where no weights)."""
        return [None if d is None else d.numpy() for d in self.grad_bufs]

    def zero_grads(self):
        for d in self.grad_bufs:
            if d is not None:
                self.ctx.upload(d, np.zeros(d.size, np.float32))

    def close(self):
        """Free the weight and gradient blocks.  Refused (MimirError, EINVAL)
        while a StoreGraph captured from this graph is open: its kernels would
        replay reads of the freed memory."""
        live = [sg for sg in self._holders if sg.handle]
        if live:
            raise MimirError(EINVAL, f"DeviceGraph.close: {len(live)} captured StoreGraph(s) still replay its "
                                     "weights; close them (or their Store) first")
        for d in self.weights + self.grad_bufs:
            if d is not None:
                d.free()
        self.weights = []
        self.grad_bufs = []


class SafeTensors:
    """A SafeTensors checkpoint (mimir_safetensors_*): header parsed on open
    with the reference's checks; tensors read straight into device memory.
    ctx may be None to inspect a file on a machine without a GPU."""

    def __init__(self, ctx, path):
        self.ctx = ctx
        self.lib = _lib.load()
        h = c_void_p()
        st = self.lib.mimir_safetensors_open(ctx.handle if ctx is not None else None, str(path).encode(), byref(h))
        if st != 0:
            msg = self.lib.mimir_safetensors_error(None)
            raise MimirError(st, (msg.decode() if msg else "") or f"cannot open {path}")
        self.handle = h

    def close(self):
        if self.handle:
            self.lib.mimir_safetensors_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def entries(self):
        """{name: (dtype string, shape tuple, nbytes)} in byte order of the names
        (the order in which the reference visits them)."""
        out = {}
        for i in range(self.lib.mimir_safetensors_count(self.handle)):
            name = ctypes.c_char_p()
            dt = ctypes.c_int32()
            shape = (ctypes.c_int64 * 16)()
            nd = ctypes.c_int32()
            nb = ctypes.c_int64()
            if self.lib.mimir_safetensors_entry(self.handle, i, byref(name), byref(dt), shape, 16, byref(nd),
                                                byref(nb)) != 0:
                raise MimirError(1, "mimir_safetensors_entry failed")
            out[name.value.decode()] = (_lib.ST_DTYPES[dt.value], tuple(shape[k] for k in range(nd.value)), nb.value)
        return out

    def read(self, name, dst):
        """Copy tensor `name` into the DeviceArray `dst` (its bytes as stored)."""
        self.ctx.check(self.lib.mimir_safetensors_read(self.handle, name.encode(), _ptr(dst), dst.nbytes))

    def load_graph(self, graph: "DeviceGraph", strict=False):
        """apply_tensors_to_model's weight loop into the graph's device weights."""
        self.ctx.check(self.lib.mimir_safetensors_load_layers(self.handle, graph.c_layers, len(graph.layers),
                                                              int(bool(strict))))
