"""mimir_hip -- MI355X (gfx950) backend for Mimir's fused elementwise and
row-reduction layer path, reached through the C ABI of libmimir_hip.so.

``Context`` owns a device and a stream; its op methods take device buffers.
``LayerOps`` mirrors the reference's host-vector op API on top of it.
"""
from ._lib import (EBUSY, EDEVICE, EINVAL, ENOMEM, OK, SOFTMAX_DIV_EPS, SOFTMAX_LOG, SOFTMAX_MUL_INV,
                   HEADER_PATH, LIB_PATH, SIGNATURES, load)
from .device import Context, DeviceArray, DeviceGraph, Event, MimirError, SafeTensors, Store, StoreGraph, rope_table
from .layerops import Layer, LayerOps

__all__ = [
    "Context", "DeviceArray", "DeviceGraph", "Event", "SafeTensors", "Store", "StoreGraph", "MimirError", "Layer", "LayerOps", "rope_table", "load",
    "OK", "EINVAL", "ENOMEM", "EDEVICE", "EBUSY", "SOFTMAX_DIV_EPS", "SOFTMAX_MUL_INV", "SOFTMAX_LOG",
    "LIB_PATH", "HEADER_PATH", "SIGNATURES",
]
