"""Ownership rules of the Python runtime wrappers, on the host.

A captured StoreGraph replays kernels that hold the addresses of its
DeviceGraph's weight and gradient blocks, and mimir_store_destroy frees every
graph captured on the store.  So DeviceGraph.close() refuses while such a
graph is open, Store.close() closes its StoreGraph objects, and a closed
StoreGraph refuses to launch while close() stays safe to repeat.  These rules
live in the wrappers, not in the library; a stand-in for the library records
the calls, so nothing here touches a GPU.
"""
from ctypes import c_void_p

import pytest

from mimir_hip import device as D


class _Lib:
    """Every C entry point returns OK; create/capture hand out fresh handles."""

    def __init__(self):
        self.calls = []
        self._next = 0x1000

    def _out(self, args):
        self._next += 0x10
        args[-1]._obj.value = self._next

    def __getattr__(self, name):
        def call(*args):
            self.calls.append(name)
            if name in ("mimir_store_create", "mimir_store_capture"):
                self._out(args)
            return D.OK
        return call


class _Ctx(D.Context):
    def __init__(self):  # no device: the stand-in library only
        self.lib = _Lib()
        self.handle = c_void_p(0x10)


def _graph(ctx):
    return D.DeviceGraph(ctx, [{"type": "GELU", "name": "act", "inputs": ["x"], "output": "x"}])


def test_device_graph_close_refused_while_a_capture_is_open():
    ctx = _Ctx()
    store, g = D.Store(ctx), _graph(ctx)
    sg = store.capture(g)
    with pytest.raises(D.MimirError, match="still replay"):
        g.close()
    sg.close()
    g.close()  # no open capture left
    assert ctx.lib.calls.count("mimir_store_graph_destroy") == 1


def test_store_close_closes_its_graphs():
    ctx = _Ctx()
    store, g = D.Store(ctx), _graph(ctx)
    sg = store.capture(g)
    store.close()
    assert not sg.handle
    with pytest.raises(D.MimirError, match="closed"):
        sg.launch()
    with pytest.raises(D.MimirError, match="closed"):
        sg.get("x")
    sg.close()
    sg.close()
    # mimir_store_destroy freed the graph: the wrapper must not destroy it again.
    assert ctx.lib.calls.count("mimir_store_graph_destroy") == 0
    g.close()  # the store's graphs are gone, so the weights may go


def test_graph_closed_first_then_store():
    ctx = _Ctx()
    store, g = D.Store(ctx), _graph(ctx)
    a, b = store.capture(g), store.capture(g)
    a.close()
    with pytest.raises(D.MimirError, match="1 captured"):
        g.close()
    store.close()
    g.close()
    assert ctx.lib.calls.count("mimir_store_graph_destroy") == 1
    assert ctx.lib.calls.count("mimir_store_destroy") == 1
