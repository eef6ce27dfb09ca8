"""ctypes binding of libmimir_hip.so (the C ABI declared in include/mimir_hip.h).

Loading fails loudly when the library is not built: there is no CPU fallback
anywhere in this package.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import (POINTER, Structure, c_char_p, c_double, c_float, c_int, c_int32, c_int64, c_size_t,
                    c_void_p)

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_ROOT, "lib", "libmimir_hip.so")
REPO_ROOT = os.path.dirname(PKG_ROOT)
HEADER_PATH = os.path.join(REPO_ROOT, "include", "mimir_hip.h")

OK, EINVAL, ENOMEM, EDEVICE, EBUSY = 0, 1, 2, 3, 4
SOFTMAX_DIV_EPS, SOFTMAX_MUL_INV, SOFTMAX_LOG = 0, 1, 2

_P = c_void_p
_PP = POINTER(c_void_p)

DTYPE_F32, DTYPE_I32 = 0, 1
ST_DTYPES = {0: "F32", 1: "F16", 2: "I32", 3: "I16", 4: "U16", 5: "U8"}  # MIMIR_ST_*
LAYER_TYPES = {"LayerNorm": 1, "RMSNorm": 2, "Softmax": 3, "LogSoftmax": 4, "GELU": 5, "SiLU": 6,
               "Add": 7, "Multiply": 8, "Embedding": 9, "Identity": 10, "Dropout": 11,
               "SelfAttention": 12, "MultiHeadAttention": 13, "CrossAttention": 14}
# The reference's BranchType and MergeOperation (Layers.hpp:59-80), in order.
BRANCH_TYPES = ("NONE", "RESIDUAL", "SKIP_CONNECTION", "DENSE_CONNECTION", "ATTENTION_BRANCH", "MULTI_SCALE",
                "GATE", "SPLIT", "MERGE")
MERGE_OPS = ("ADD", "MULTIPLY", "CONCATENATE", "MAX", "AVERAGE", "GATED", "ATTENTION_WEIGHTED")


def detect_branch_type(name):
    """(branch_type, merge_op) as Layer::detectBranchType (Layers.hpp:260-304)
    sets them from a layer's name; Model::push calls it for every layer
    (Model.cpp:3145).  merge_op keeps its default, ADD, where the reference
    does not set it."""
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
        op = "ADD" if has("add") else "MULTIPLY" if has("mul") else "CONCATENATE" if has("concat") else "ADD"
        return "MERGE", op
    return "NONE", "ADD"


class Layer_C(Structure):
    """struct mimir_layer (include/mimir_hip.h)."""
    _fields_ = [("type", c_int32), ("name", c_char_p), ("inputs", POINTER(c_char_p)),
                ("n_inputs", c_int32), ("output", c_char_p), ("weights", c_void_p),
                ("weights_len", c_int64), ("eps", c_float), ("affine", c_int32), ("use_bias", c_int32),
                ("in_features", c_int32), ("vocab_size", c_int32), ("embed_dim", c_int32),
                ("padding_idx", c_int32), ("seq_len", c_int32), ("grad_weights", c_void_p),
                ("branch_type", c_int32), ("merge_op", c_int32), ("branch_sources", POINTER(c_int32)),
                ("n_branch_sources", c_int32), ("num_heads", c_int32), ("head_dim", c_int32), ("causal", c_int32)]


# name -> (restype, argtypes); mirrors include/mimir_hip.h one to one.
SIGNATURES = {
    "mimir_ctx_create": (c_int, [c_int, _PP]),
    "mimir_ctx_destroy": (c_int, [_P]),
    "mimir_ctx_set_stream": (c_int, [_P, _P]),
    "mimir_ctx_stream": (c_void_p, [_P]),
    "mimir_ctx_set_alloc_limit": (c_int, [_P, c_size_t]),
    "mimir_ctx_set_output_caching": (c_int, [_P, c_int]),
    "mimir_last_error": (c_char_p, [_P]),
    "mimir_malloc": (c_int, [_P, c_size_t, _PP]),
    "mimir_free": (c_int, [_P, _P]),
    "mimir_upload": (c_int, [_P, _P, _P, c_size_t]),
    "mimir_download": (c_int, [_P, _P, _P, c_size_t]),
    "mimir_copy": (c_int, [_P, _P, _P, c_size_t]),
    "mimir_fill_f32": (c_int, [_P, _P, c_int64, c_float]),
    "mimir_sync": (c_int, [_P]),
    "mimir_event_create": (c_int, [_P, _PP]),
    "mimir_event_destroy": (c_int, [_P]),
    "mimir_event_record": (c_int, [_P, _P]),
    "mimir_event_elapsed_ms": (c_int, [_P, _P, POINTER(c_float)]),
    "mimir_layernorm_fwd": (c_int, [_P, _P, _P, _P, _P, c_int64, c_int64, c_float]),
    "mimir_rmsnorm_fwd": (c_int, [_P, _P, _P, c_int64, _P, c_int64, c_int64, c_float]),
    "mimir_add_rmsnorm_fwd": (c_int, [_P, _P, _P, _P, _P, _P, c_int64, c_int64, c_float]),
    "mimir_softmax_fwd": (c_int, [_P, _P, _P, c_int64, c_int64, c_int]),
    "mimir_gelu_fwd": (c_int, [_P, _P, _P, c_int64]),
    "mimir_silu_fwd": (c_int, [_P, _P, _P, c_int64]),
    "mimir_silu_mul_fwd": (c_int, [_P, _P, _P, _P, c_int64]),
    "mimir_gelu_mul_fwd": (c_int, [_P, _P, _P, _P, c_int64]),
    "mimir_add_fwd": (c_int, [_P, _P, c_int64, _P, c_int64, _P]),
    "mimir_mul_fwd": (c_int, [_P, _P, c_int64, _P, c_int64, _P]),
    "mimir_branch_merge_fwd": (c_int, [_P, _P, c_int64, _P, c_int64, _P, c_int]),
    "mimir_embedding_fwd": (c_int, [_P, _P, c_int64, _P, c_int64, c_int32, c_int32, c_int32, _P]),
    "mimir_embedding_f32ids_fwd": (c_int, [_P, _P, c_int64, _P, c_int64, c_int32, c_int32, c_int32,
                                           _P]),
    "mimir_rope_table": (c_int, [c_int64, c_int64, c_double, _P, _P]),
    "mimir_rope_fwd": (c_int, [_P, _P, _P, c_int64, _P, _P, c_int64, c_int64, c_int64, c_int64,
                               c_int64, _P, _P, c_int64]),
    "mimir_attention_fwd": (c_int, [_P, _P, c_int64, _P, _P, c_int64, _P, c_int64, c_int64, c_int64, c_int64,
                                    c_int64, c_int64, c_float, c_int]),
    "mimir_self_attention_fwd": (c_int, [_P, _P, c_int64, c_int64, c_int64, c_int, _P, c_int64, _P]),
    "mimir_cross_attention_fwd": (c_int, [_P, _P, c_int64, _P, c_int64, c_int64, c_int64, c_int, _P, c_int64, _P]),
    "mimir_attention_bwd": (c_int, [_P, _P, c_int64, _P, _P, c_int64, _P, c_int64, _P, c_int64, _P, _P, c_int64,
                                    c_int64, c_int64, c_int64, c_int64, c_int64, c_float, c_int]),
    "mimir_self_attention_bwd": (c_int, [_P, _P, _P, c_int64, c_int64, c_int64, c_int, _P, c_int64, _P, _P, c_int]),
    "mimir_cross_attention_bwd": (c_int, [_P, _P, c_int64, _P, c_int64, _P, c_int64, c_int64, c_int, _P, c_int64, _P,
                                          _P, c_int, _P, c_int]),
    "mimir_layernorm_bwd": (c_int, [_P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_float, c_int]),
    "mimir_layernorm_bwd_noalloc": (c_int, [_P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_float, c_int]),
    "mimir_gelu_bwd": (c_int, [_P, _P, _P, _P, c_int64, c_int]),
    "mimir_silu_bwd": (c_int, [_P, _P, _P, _P, c_int64, c_int]),
    "mimir_mul_bwd": (c_int, [_P, _P, _P, _P, _P, _P, c_int64, c_int, c_int]),
    "mimir_add_bwd": (c_int, [_P, _P, c_int64, c_int64, _P, _P, c_int, c_int]),
    "mimir_embedding_bwd": (c_int, [_P, _P, c_int64, _P, _P, c_int64, c_int32, c_int32, c_int32]),
    "mimir_embedding_f32ids_bwd": (c_int, [_P, _P, c_int64, _P, _P, c_int64, c_int32, c_int32, c_int32]),
    "mimir_store_create": (c_int, [_P, _PP]),
    "mimir_store_destroy": (c_int, [_P]),
    "mimir_store_clear": (c_int, [_P]),
    "mimir_store_put": (c_int, [_P, c_char_p, c_int, _P, c_int64]),
    "mimir_store_info": (c_int, [_P, c_char_p, c_int, _PP, POINTER(c_int64)]),
    "mimir_store_get": (c_int, [_P, c_char_p, c_int, _P, c_int64, POINTER(c_int64)]),
    "mimir_store_set_inputs": (c_int, [_P, POINTER(c_char_p), POINTER(c_void_p), POINTER(c_int64), c_int32,
                                       POINTER(c_char_p), POINTER(c_void_p), POINTER(c_int64), c_int32]),
    "mimir_store_run": (c_int, [_P, POINTER(Layer_C), c_int32]),
    "mimir_store_run_training": (c_int, [_P, POINTER(Layer_C), c_int32]),
    "mimir_store_set_input_ids": (c_int, [_P, _P, c_int64]),
    "mimir_store_run_ids": (c_int, [_P, POINTER(Layer_C), c_int32, c_int]),
    "mimir_safetensors_open": (c_int, [_P, c_char_p, _PP]),
    "mimir_safetensors_close": (c_int, [_P]),
    "mimir_safetensors_count": (c_int64, [_P]),
    "mimir_safetensors_entry": (c_int, [_P, c_int64, POINTER(c_char_p), POINTER(c_int32), POINTER(c_int64), c_int32,
                                        POINTER(c_int32), POINTER(c_int64)]),
    "mimir_safetensors_find": (c_int64, [_P, c_char_p]),
    "mimir_safetensors_error": (c_char_p, [_P]),
    "mimir_safetensors_read": (c_int, [_P, c_char_p, _P, c_size_t]),
    "mimir_safetensors_load_layers": (c_int, [_P, POINTER(Layer_C), c_int32, c_int]),
    "mimir_store_backward": (c_int, [_P, POINTER(Layer_C), c_int32, _P, c_int64]),
    "mimir_store_backward_dev": (c_int, [_P, POINTER(Layer_C), c_int32, _P, c_int64]),
    "mimir_store_grad_info": (c_int, [_P, c_char_p, _PP, POINTER(c_int64)]),
    "mimir_store_grad_get": (c_int, [_P, c_char_p, _P, c_int64, POINTER(c_int64)]),
    "mimir_store_capture": (c_int, [_P, POINTER(Layer_C), c_int32, POINTER(_P)]),
    "mimir_store_set_fusion": (c_int, [_P, c_int]),
    "mimir_store_graph_launch": (c_int, [_P]),
    "mimir_store_graph_set_input": (c_int, [_P, c_char_p, c_int, _P, c_int64]),
    "mimir_store_graph_get": (c_int, [_P, c_char_p, c_int, _P, c_int64, POINTER(c_int64)]),
    "mimir_store_graph_destroy": (c_int, [_P]),
}

_lib = None


def load():
    """Load libmimir_hip.so once; raise if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is not built: run `make -C mimir-framework_amd` "
                "(or __graft_entry__.build()); mimir_hip has no CPU fallback")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib
