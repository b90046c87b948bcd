"""ctypes binding of libdbi_kv.so (include/dbi_kv.h).

The shared library is built in-tree by ``__graft_entry__.build()``. Loading
fails loudly when it is missing: there is no CPU fallback on this path.
"""
from __future__ import annotations

import ctypes
import importlib.util
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libdbi_kv.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "dbi_kv.h")

DBI_OK = 0
DBI_ERR_INVALID = 1
DBI_ERR_UNSUPPORTED = 2
DBI_ERR_NOMEM = 3
DBI_ERR_DEVICE = 4
DBI_ERR_IO = 5
DBI_ERR_FORMAT = 6

DBI_KV_F32 = 0
DBI_KV_INT8 = 1
DBI_W_F32, DBI_W_F16, DBI_W_Q4_0, DBI_W_Q8_0 = 0, 1, 2, 8

EXPORT = {
    "k": 0, "v": 1, "k8": 2, "v8": 3, "k_scale": 4, "v_scale": 5,
    "k_sink": 6, "v_sink": 7, "k_raw": 8,
}


class KvConfig(ctypes.Structure):
    _fields_ = [
        ("n_layers", ctypes.c_uint32),
        ("max_seq", ctypes.c_uint32),
        ("n_kv_heads", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
        ("n_sink", ctypes.c_uint32),
        ("window", ctypes.c_uint32),
        ("dtype", ctypes.c_uint32),
        ("rope_theta", ctypes.c_float),
    ]


_u32 = ctypes.c_uint32
_f32 = ctypes.c_float
_vp = ctypes.c_void_p
_st = ctypes.c_int32


class Weight(ctypes.Structure):
    """dbi_weight: device data and its type (DBI_W_*)."""
    _fields_ = [("data", _vp), ("type", _u32)]


class LayerWeights(ctypes.Structure):
    """dbi_layer_weights (backend::LayerQ's pointers), device memory."""
    _fields_ = [("attn_norm", _vp), ("ffn_norm", _vp),
                ("wq", Weight), ("wk", Weight), ("wv", Weight), ("wo", Weight),
                ("wgate", Weight), ("wup", Weight), ("wdown", Weight),
                ("bq", _vp), ("bk", _vp), ("bv", _vp)]


class OffloadConfig(ctypes.Structure):
    """dbi_offload_config."""
    _fields_ = [("dim", _u32), ("ff", _u32), ("n_heads", _u32), ("rms_eps", _f32),
                ("output_norm", _vp), ("lm_head", Weight), ("vocab", _u32)]

# name -> (restype, argtypes)
SIGNATURES = {
    "dbi_last_error": (ctypes.c_char_p, []),
    "dbi_kv_create": (_st, [ctypes.POINTER(KvConfig), ctypes.POINTER(_vp)]),
    "dbi_kv_destroy": (None, [_vp]),
    "dbi_kv_get_config": (_st, [_vp, ctypes.POINTER(KvConfig)]),
    "dbi_kv_set_stream": (_st, [_vp, _vp]),
    "dbi_kv_sync": (_st, [_vp]),
    "dbi_kv_append": (_st, [_vp, _u32, _u32, _vp, _vp]),
    "dbi_kv_append_n": (_st, [_vp, _u32, _u32, _u32, _vp, _vp]),
    "dbi_kv_append_async": (_st, [_vp, _u32, _u32, _u32, _vp, _vp]),
    "dbi_kv_truncate": (_st, [_vp, _u32]),
    "dbi_kv_n_seen": (_u32, [_vp]),
    "dbi_kv_capacity": (_u32, [_vp]),
    "dbi_kv_slot_for": (_st, [_vp, _u32, ctypes.POINTER(_u32)]),
    "dbi_kv_residents": (_st, [_vp, _vp, _vp, _u32, ctypes.POINTER(_u32)]),
    "dbi_attn_decode": (_st, [_vp, _u32, _u32, _u32, _f32, _vp, _vp]),
    "dbi_attn_decode_async": (_st, [_vp, _u32, _u32, _u32, _f32, _vp, _vp]),
    "dbi_attn_splits": (_st, [_vp, _u32, _u32, _u32, ctypes.POINTER(_u32)]),
    "dbi_kv_decode": (_st, [_vp, _u32, _u32, _vp, _vp, _u32, _f32, _vp, _vp]),
    "dbi_kv_decode_async": (_st, [_vp, _u32, _u32, _vp, _vp, _u32, _f32, _vp, _vp]),
    "dbi_kv_decode_noalloc_async": (_st, [_vp, _u32, _u32, _vp, _vp, _u32, _f32, _vp, _vp]),
    "dbi_attn_chunk": (_st, [_vp, _u32, _u32, _u32, _u32, _f32, _vp, _vp]),
    "dbi_attn_chunk_async": (_st, [_vp, _u32, _u32, _u32, _u32, _f32, _vp, _vp]),
    "dbi_kv_decode_qkv": (_st, [_vp, _u32, _u32, _u32, _f32] + [_vp] * 7),
    "dbi_kv_decode_qkv_async": (_st, [_vp, _u32, _u32, _u32, _f32] + [_vp] * 7),
    "dbi_kv_chunk_qkv": (_st, [_vp, _u32, _u32, _u32, _u32, _f32] + [_vp] * 7),
    "dbi_kv_chunk_qkv_async": (_st, [_vp, _u32, _u32, _u32, _u32, _f32] + [_vp] * 7),
    "dbi_spec_verify_async": (_st, [_vp, _u32, _u32, _vp, _vp, _vp, _vp]),
    "dbi_kv_verify_commit": (_st, [_vp, _u32, _u32, _u32, _vp, _vp, _vp, _vp]),
    "dbi_oproj_residual_async": (_st, [_vp, _u32, _vp, _vp, _vp, _u32, _u32]),
    "dbi_offload_setup": (_st, [_vp, ctypes.POINTER(OffloadConfig), ctypes.POINTER(LayerWeights),
                                _u32]),
    "dbi_decode_token_async": (_st, [_vp, _vp, _u32]),
    "dbi_decode_token_full_async": (_st, [_vp, _vp, _u32, _vp]),
    "dbi_offload_setup_host": (_st, [_vp, ctypes.POINTER(OffloadConfig),
                                     ctypes.POINTER(LayerWeights), _u32]),
    "dbi_decode_token": (_st, [_vp, _vp, _u32]),
    "dbi_decode_token_full": (_st, [_vp, _vp, _u32, _vp]),
    "dbi_kv_prefix_save": (_st, [_vp, ctypes.c_char_p, _vp, _u32]),
    "dbi_kv_prefix_load": (_st, [_vp, ctypes.c_char_p, _vp, _u32, ctypes.POINTER(_u32)]),
    "dbi_kv_export_bytes": (ctypes.c_size_t, [_vp, _u32]),
    "dbi_kv_export": (_st, [_vp, _u32, _u32, _vp, ctypes.c_size_t]),
}


def header_symbols(path: str = HEADER_PATH) -> list[str]:
    """Every function the C-ABI header declares."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dbi_[a-z0-9_]+)\s*\(", text)))


_LIB = None


def load() -> ctypes.CDLL:
    """Loads libdbi_kv.so with typed signatures; raises if it is not built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`")
    # ROCm builds of torch ship their own HIP runtime (soname libamdhip64.so.7,
    # file libamdhip64.so). Loaded after this library, torch would map a second
    # HIP and HSA runtime into the process and find no GPU; loaded first, it
    # lets this library bind to that same runtime by soname.
    if importlib.util.find_spec("torch") is not None:
        import torch  # noqa: F401
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib
