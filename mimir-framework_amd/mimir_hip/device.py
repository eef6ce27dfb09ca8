"""Device context, buffers and the per-op calls of libmimir_hip.

Everything here is a thin layer over the C ABI: buffers are device memory
owned by a :class:`Context`, ops enqueue on the context's stream and return,
and a non-OK status raises :class:`MimirError` carrying the library's message.
"""
from __future__ import annotations

import ctypes
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

    def embedding(self, ids, n_ids, table, table_len, vocab, dim, padding_idx, y, float_ids=False):
        fn = self.lib.mimir_embedding_f32ids_fwd if float_ids else self.lib.mimir_embedding_fwd
        self.check(fn(self.handle, _ptr(ids), n_ids, _ptr(table), table_len, vocab, dim,
                      padding_idx, _ptr(y)))

    def rope(self, q, q_out, q_heads, k, k_out, k_heads, batch, seq, head_dim, pos_offset,
             cos_tab, sin_tab, table_rows):
        self.check(self.lib.mimir_rope_fwd(self.handle, _ptr(q), _ptr(q_out), q_heads, _ptr(k),
                                           _ptr(k_out), k_heads, batch, seq, head_dim, pos_offset,
                                           _ptr(cos_tab), _ptr(sin_tab), table_rows))


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
