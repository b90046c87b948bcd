"""ctypes binding of the CPU oracle (liboracle_kv.so) -- TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, and only as the checker / the timed CPU baseline. The product
path never imports it.

``OracleKV`` exposes the oracle KV cache with the same method names as
``dbinfer_amd.kv.HipKV`` plus ``export`` returning the reference-layout arrays
(model.cpp:420-455), so parity tests compare the two field by field.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle_kv.so")
REF_OPS_PATH = os.path.join(_HERE, "_ref", "libref_ops.so")

F32 = 0
INT8 = 1
_sz = ctypes.c_size_t
_vp = ctypes.c_void_p


class _Okv(ctypes.Structure):
    _fields_ = [
        ("n_sink_policy", _sz), ("window", _sz), ("dtype", ctypes.c_int),
        ("n_layers", _sz), ("capacity", _sz), ("layer_stride", _sz), ("pos_stride", _sz),
        ("n_kv_heads", _sz), ("head_dim", _sz), ("n_blocks", _sz), ("scale_stride", _sz),
        ("k_group", _sz), ("n_kgroups", _sz), ("k_scale_stride", _sz), ("n_sink", _sz),
        ("n_seen", _sz),
        ("k", ctypes.POINTER(ctypes.c_float)), ("v", ctypes.POINTER(ctypes.c_float)),
        ("k8", ctypes.POINTER(ctypes.c_int8)), ("v8", ctypes.POINTER(ctypes.c_int8)),
        ("k_scale", ctypes.POINTER(ctypes.c_float)), ("v_scale", ctypes.POINTER(ctypes.c_float)),
        ("k_raw", ctypes.POINTER(ctypes.c_float)), ("k_sink", ctypes.POINTER(ctypes.c_float)),
        ("v_sink", ctypes.POINTER(ctypes.c_float)),
    ]


_P = ctypes.POINTER(_Okv)
_SIGS = {
    "okv_create": (_P, [_sz, _sz, _sz, _sz, _sz, _sz, ctypes.c_int]),
    "okv_destroy": (None, [_P]),
    "okv_slot_for": (_sz, [_P, _sz]),
    "okv_append": (None, [_P, _sz, _sz, _vp, _vp]),
    "okv_append_n": (None, [_P, _sz, _sz, _sz, _vp, _vp]),
    "okv_residents": (_sz, [_P, _vp, _vp]),
    "okv_truncate": (None, [_P, _sz]),
    "ok_quant_head": (None, [_vp, _sz, _vp, _vp]),
    "ok_rope": (None, [_vp, _vp, ctypes.c_float, _sz, _sz, _sz]),
    "ok_softmax": (None, [_vp, _vp, _sz]),
    "okv_attend_dense_f32": (None, [_P, _sz, _sz, _sz, ctypes.c_float, _vp, _vp, ctypes.c_int]),
    "okv_attend_dense_int8": (None, [_P, _sz, _sz, _sz, ctypes.c_float, _vp, _vp, ctypes.c_int]),
    "okv_attend_ring": (None, [_P, _sz, _sz, _sz, ctypes.c_float, ctypes.c_float, _vp, _vp, _vp,
                               _vp, ctypes.c_int]),
    "okv_attend_ring_literal": (None, [_P, _sz, _sz, _sz, ctypes.c_float, ctypes.c_float, _vp,
                                       _vp, _vp, _vp]),
    "okv_attend_chunk": (None, [_P, _sz, _sz, _sz, _sz, ctypes.c_float, _vp, _vp,
                                ctypes.c_int]),
    "okv_prefix_save": (ctypes.c_int, [_P, ctypes.c_char_p, _vp, _sz, ctypes.c_char_p, _sz]),
    "okv_prefix_load": (ctypes.c_int, [_P, ctypes.c_char_p, _vp, _sz, ctypes.POINTER(_sz),
                                       ctypes.c_char_p, _sz]),
    "ok_spec_merge": (_sz, [_vp, _sz, _vp, _vp, ctypes.POINTER(_sz)]),
    "ok_argmax": (ctypes.c_int32, [_vp, _sz]),
    "ok_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "ok_oproj_residual": (None, [_vp, ctypes.c_int, _vp, _vp, _sz, _sz]),
    "ok_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
    "ok_quantize_row_q8_0": (None, [_vp, _sz, _vp]),
    "ok_matvec": (None, [_vp, ctypes.c_int, _vp, _vp, _sz, _sz]),
    "ok_rmsnorm": (None, [_vp, _vp, ctypes.c_float, _vp, _sz]),
    "ok_silu": (None, [_vp, _vp, _sz]),
    "okv_decode_layer": (None, [_P, _sz, _vp, ctypes.c_int32, _vp, _sz, _sz, _sz, ctypes.c_float,
                                ctypes.c_float, ctypes.c_int]),
    "ok_logits": (None, [_vp, _vp, _vp, ctypes.c_int, ctypes.c_float, _vp, _sz, _sz]),
}

_LIB = None
_REF = None


def load() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} not built (make -C oracle)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = lib
    return _LIB


def load_ref():
    """The reference's own rope/softmax built from its sources, or None."""
    global _REF
    if _REF is None and os.path.exists(REF_OPS_PATH):
        lib = ctypes.CDLL(REF_OPS_PATH)
        lib.ref_rope.restype = None
        lib.ref_rope.argtypes = [_vp, _vp, ctypes.c_float, _sz, _sz, _sz]
        lib.ref_softmax.restype = None
        lib.ref_softmax.argtypes = [_vp, _vp, _sz]
        if hasattr(lib, "ref_rmsnorm"):
            lib.ref_rmsnorm.restype = None
            lib.ref_rmsnorm.argtypes = [_vp, _vp, ctypes.c_float, _vp, _sz, _sz]
            lib.ref_silu.restype = None
            lib.ref_silu.argtypes = [_vp, _vp, _sz]
        _REF = lib
    return _REF


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def rope(x, positions, theta: float, n_heads: int, seq: int, head_dim: int) -> np.ndarray:
    x = _f32(x).copy()
    p = np.ascontiguousarray(positions, dtype=np.int32)
    load().ok_rope(x.ctypes.data, p.ctypes.data, theta, n_heads, seq, head_dim)
    return x


def softmax(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    load().ok_softmax(x.ctypes.data, out.ctypes.data, x.size)
    return out


def quant_head(x) -> tuple[np.ndarray, np.ndarray]:
    x = _f32(x)
    codes = np.empty(x.size, np.int8)
    scales = np.empty((x.size + 31) // 32, np.float32)
    load().ok_quant_head(x.ctypes.data, x.size, codes.ctypes.data, scales.ctypes.data)
    return codes, scales


def spec_merge(draft, target) -> tuple[int, list[int]]:
    d = np.ascontiguousarray(draft, dtype=np.int32)
    t = np.ascontiguousarray(target, dtype=np.int32)
    out = np.zeros(d.size + 1, np.int32)
    n = _sz()
    acc = load().ok_spec_merge(d.ctypes.data, d.size, t.ctypes.data, out.ctypes.data,
                               ctypes.byref(n))
    return int(acc), out[: n.value].tolist()


def argmax(logits) -> int:
    x = np.ascontiguousarray(logits, dtype=np.float32)
    assert x.size >= 1
    return int(load().ok_argmax(x.ctypes.data, x.size))


def f16_to_f32(h: int) -> float:
    return float(load().ok_f16_to_f32(h))


def f32_to_f16(f: float) -> int:
    return int(load().ok_f32_to_f16(f))


def quantize_row_q8_0(x) -> np.ndarray:
    xa = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(xa.size // 32 * 34, np.uint8)
    load().ok_quantize_row_q8_0(xa.ctypes.data, xa.size, out.ctypes.data)
    return out


def oproj_residual(w, attn, x, q8_0: bool = False):
    """x + w @ attn with the reference's sequential sums. w: float32 or
    float16 [dim][in], or (q8_0) uint8 [dim][in/32*34] Q8_0 blocks."""
    wc = np.ascontiguousarray(w)
    a = np.ascontiguousarray(attn, dtype=np.float32)
    out = np.array(x, dtype=np.float32, copy=True)
    wtype = 8 if q8_0 else (1 if wc.dtype == np.float16 else 0)
    load().ok_oproj_residual(wc.ctypes.data, wtype, a.ctypes.data, out.ctypes.data, out.size,
                             a.size)
    return out


# weight types, numbered as GgmlType (gguf.hpp)
W_F32, W_F16, W_Q4_0, W_Q8_0 = 0, 1, 2, 8


def matvec(w, wtype: int, x, out: int) -> np.ndarray:
    """tensor::matvec_quant of w (fp32 / f16 [out][in], or uint8 Q4_0 / Q8_0
    blocks [out][in/32*18|34]) against x [in]."""
    wc = np.ascontiguousarray(w)
    xa = _f32(x)
    y = np.zeros(out, np.float32)
    load().ok_matvec(wc.ctypes.data, wtype, xa.ctypes.data, y.ctypes.data, out, xa.size)
    return y


def rmsnorm(x, weight, eps: float) -> np.ndarray:
    xa, wa = _f32(x), _f32(weight)
    out = np.zeros_like(xa)
    load().ok_rmsnorm(xa.ctypes.data, wa.ctypes.data, eps, out.ctypes.data, xa.size)
    return out


def silu(x) -> np.ndarray:
    xa = _f32(x)
    out = np.zeros_like(xa)
    load().ok_silu(xa.ctypes.data, out.ctypes.data, xa.size)
    return out


class _OkLayer(ctypes.Structure):
    _fields_ = [("attn_norm", _vp), ("ffn_norm", _vp), ("w", _vp * 7), ("wtype", ctypes.c_int * 7),
                ("bq", _vp), ("bk", _vp), ("bv", _vp)]


def logits(x, output_norm, lm_head, wtype: int, eps: float, vocab: int) -> np.ndarray:
    """Model::forward's tail (model.cpp:914-915)."""
    xa, na = _f32(x), _f32(output_norm)
    lm = np.ascontiguousarray(lm_head)
    out = np.zeros(vocab, np.float32)
    load().ok_logits(xa.ctypes.data, na.ctypes.data, lm.ctypes.data, wtype, eps, out.ctypes.data,
                     xa.size, vocab)
    return out


class OracleError(RuntimeError):
    pass


class OracleKV:
    def __init__(self, n_layers: int, max_seq: int, n_kv_heads: int, head_dim: int,
                 n_sink: int = 0, window: int = 0, dtype: int = F32, rope_theta: float = 1e4):
        self._lib = load()
        self._p = self._lib.okv_create(n_layers, max_seq, n_kv_heads, head_dim, n_sink, window,
                                       dtype)
        if not self._p:
            raise MemoryError("oracle allocation failed")
        self.n_layers, self.n_kv_heads, self.head_dim = n_layers, n_kv_heads, head_dim
        self.n_sink, self.window, self.dtype, self.rope_theta = n_sink, window, dtype, rope_theta
        self.pos_stride = n_kv_heads * head_dim
        self.n_blocks = (head_dim + 31) // 32

    def close(self):
        if getattr(self, "_p", None):
            self._lib.okv_destroy(self._p)
            self._p = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def s(self) -> _Okv:
        return self._p.contents

    @property
    def capacity(self) -> int:
        return int(self.s.capacity)

    @property
    def n_seen(self) -> int:
        return int(self.s.n_seen)

    def truncate(self, n: int) -> None:
        self._lib.okv_truncate(self._p, n)

    def reset(self) -> None:
        self.truncate(0)

    def mark_position(self, pos: int) -> None:
        self.truncate(pos + 1)

    def append(self, layer: int, pos: int, k, v) -> None:
        k, v = _f32(k), _f32(v)
        assert k.size == self.pos_stride and v.size == self.pos_stride
        self._lib.okv_append(self._p, layer, pos, k.ctypes.data, v.ctypes.data)

    def append_n(self, layer: int, pos0: int, k, v) -> None:
        k = _f32(k).reshape(-1, self.pos_stride)
        v = _f32(v).reshape(-1, self.pos_stride)
        assert k.shape == v.shape
        self._lib.okv_append_n(self._p, layer, pos0, k.shape[0], k.ctypes.data, v.ctypes.data)

    def slot_for(self, pos: int) -> int:
        return int(self._lib.okv_slot_for(self._p, pos))

    def residents(self) -> tuple[np.ndarray, np.ndarray]:
        cap = self.capacity
        slot = np.zeros(cap, np.uint64)
        rp = np.zeros(cap, np.int32)
        n = self._lib.okv_residents(self._p, slot.ctypes.data, rp.ctypes.data)
        return slot[:n].astype(np.uint32), rp[:n].copy()

    def attend(self, layer: int, pos: int, q, n_heads: int, scale: float,
               n_threads: int = 1) -> np.ndarray:
        """Dense layouts only (ring attention appends: use attend_ring)."""
        q = _f32(q)
        out = np.empty(n_heads * self.head_dim, np.float32)
        fn = (self._lib.okv_attend_dense_int8 if self.dtype == INT8
              else self._lib.okv_attend_dense_f32)
        fn(self._p, layer, pos, n_heads, scale, q.ctypes.data, out.ctypes.data, n_threads)
        return out

    def attend_ring(self, layer: int, pos: int, q, k, v, n_heads: int, scale: float,
                    n_threads: int = 1, literal: bool = False) -> np.ndarray:
        q, k, v = _f32(q), _f32(k), _f32(v)
        out = np.empty(n_heads * self.head_dim, np.float32)
        if literal:
            self._lib.okv_attend_ring_literal(self._p, layer, pos, n_heads, scale,
                                              self.rope_theta, q.ctypes.data, k.ctypes.data,
                                              v.ctypes.data, out.ctypes.data)
        else:
            self._lib.okv_attend_ring(self._p, layer, pos, n_heads, scale, self.rope_theta,
                                      q.ctypes.data, k.ctypes.data, v.ctypes.data,
                                      out.ctypes.data, n_threads)
        return out

    def attend_chunk(self, layer: int, pos0: int, q, n_heads: int, scale: float,
                     n_threads: int = 1) -> np.ndarray:
        q = _f32(q)
        n = q.size // (n_heads * self.head_dim)
        out = np.empty(q.size, np.float32)
        self._lib.okv_attend_chunk(self._p, layer, pos0, n, n_heads, scale, q.ctypes.data,
                                   out.ctypes.data, n_threads)
        return out

    def decode_layer(self, layer: int, x, pos: int, lw: dict, dim: int, ff: int, n_heads: int,
                     eps: float, n_threads: int = 1) -> np.ndarray:
        """Model::decode_layer (model.cpp:730-787) on a copy of x. lw holds
        attn_norm, ffn_norm, w (7 arrays: q k v o gate up down), wtype (7 ints)
        and optional bq, bk, bv."""
        keep = []

        def ptr(a, dt=None):
            if a is None:
                return None
            a = np.ascontiguousarray(a, dtype=dt) if dt else np.ascontiguousarray(a)
            keep.append(a)
            return a.ctypes.data
        L = _OkLayer()
        L.attn_norm = ptr(lw["attn_norm"], np.float32)
        L.ffn_norm = ptr(lw["ffn_norm"], np.float32)
        for i in range(7):
            L.w[i] = ptr(lw["w"][i])
            L.wtype[i] = int(lw["wtype"][i])
        L.bq = ptr(lw.get("bq"), np.float32)
        L.bk = ptr(lw.get("bk"), np.float32)
        L.bv = ptr(lw.get("bv"), np.float32)
        xa = _f32(x).copy()
        self._lib.okv_decode_layer(self._p, layer, xa.ctypes.data, pos, ctypes.byref(L), dim, ff,
                                   n_heads, eps, self.rope_theta, n_threads)
        return xa

    def save_prefix(self, path: str, tokens) -> None:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        err = ctypes.create_string_buffer(512)
        if self._lib.okv_prefix_save(self._p, path.encode(), t.ctypes.data, t.size, err, 512):
            raise OracleError(err.value.decode())

    def load_prefix(self, path: str, tokens) -> int:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        err = ctypes.create_string_buffer(512)
        n = _sz()
        if self._lib.okv_prefix_load(self._p, path.encode(), t.ctypes.data, t.size,
                                     ctypes.byref(n), err, 512):
            raise OracleError(err.value.decode())
        return int(n.value)

    def export(self, what: str, layer: int) -> np.ndarray:
        """One layer of a storage array, reference layout (copies)."""
        s = self.s
        P, cap, nb = self.pos_stride, self.capacity, self.n_blocks
        if what in ("k", "v"):
            ptr, n, dt = getattr(s, what), cap * P, np.float32
            off = layer * s.layer_stride
        elif what in ("k8", "v8"):
            ptr, n, dt = getattr(s, what), cap * P, np.int8
            off = layer * s.layer_stride
        elif what == "v_scale":
            ptr, n, dt, off = s.v_scale, cap * self.n_kv_heads * nb, np.float32, layer * s.scale_stride
        elif what == "k_scale":
            if s.k_group > 0:
                ptr, n, off = s.k_scale, s.k_scale_stride, layer * s.k_scale_stride
            else:
                ptr, n, off = s.k_scale, cap * self.n_kv_heads * nb, layer * s.scale_stride
            dt = np.float32
        elif what in ("k_sink", "v_sink"):
            ptr, n, dt = getattr(s, what), s.n_sink * P, np.float32
            off = layer * s.n_sink * P
        elif what == "k_raw":
            ptr, n, dt, off = s.k_raw, 32 * P, np.float32, layer * 32 * P
        else:
            raise KeyError(what)
        if not ptr or n == 0:
            raise OracleError(f"{what} not present in this layout")
        addr = ctypes.cast(ptr, ctypes.c_void_p).value + off * np.dtype(dt).itemsize
        buf = (ctypes.c_byte * (n * np.dtype(dt).itemsize)).from_address(addr)
        return np.frombuffer(buf, dtype=dt).copy()
