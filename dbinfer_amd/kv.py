"""Python handle over the C-ABI, named after the reference KVCache API.

``HipKV`` mirrors ``dbinfer::model::KVCache`` (src/model/model.hpp:108-214):
``append``, ``slot_for``, ``residents``, ``n_seen``, ``reset``,
``mark_position``, ``capacity``; plus the attention entry points of
``Model::attend_*`` (model.cpp:567-728) and the chunk attention of
``decode_layer_chunk`` (model.cpp:956-981), and prefix save/load
(model.cpp:1072-1156). Host-array methods take numpy float32 arrays; the
``*_async`` methods take device pointers (e.g. ``torch.Tensor.data_ptr()``).
Every call goes through libdbi_kv.so; failures raise ``DbiError``.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib

F32 = _lib.DBI_KV_F32
INT8 = _lib.DBI_KV_INT8
W_F32 = _lib.DBI_W_F32
W_F16 = _lib.DBI_W_F16
W_Q8_0 = _lib.DBI_W_Q8_0
W_Q4_0 = _lib.DBI_W_Q4_0


class DbiError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"[dbi status {status}] {message}")
        self.status = status
        self.message = message


def _check(lib, st: int) -> None:
    if st != _lib.DBI_OK:
        raise DbiError(st, lib.dbi_last_error().decode())


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


class HipKV:
    """KV cache of one model on the current HIP device."""

    def __init__(self, n_layers: int, max_seq: int, n_kv_heads: int, head_dim: int,
                 n_sink: int = 0, window: int = 0, dtype: int = F32, rope_theta: float = 1e4):
        self._lib = _lib.load()
        cfg = _lib.KvConfig(n_layers, max_seq, n_kv_heads, head_dim, n_sink, window, dtype,
                            rope_theta)
        h = ctypes.c_void_p()
        _check(self._lib, self._lib.dbi_kv_create(ctypes.byref(cfg), ctypes.byref(h)))
        self._h = h
        self.n_layers, self.n_kv_heads, self.head_dim = n_layers, n_kv_heads, head_dim
        self.n_sink, self.window, self.dtype, self.rope_theta = n_sink, window, dtype, rope_theta
        self.pos_stride = n_kv_heads * head_dim
        self.n_blocks = (head_dim + 31) // 32
        self._vocab = 0  # logits length bound by offload_setup (0: no tail)

    # ---- lifetime
    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.dbi_kv_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    # ---- state
    @property
    def capacity(self) -> int:
        return int(self._lib.dbi_kv_capacity(self._h))

    @property
    def n_seen(self) -> int:
        return int(self._lib.dbi_kv_n_seen(self._h))

    def ring(self) -> bool:
        return self.window > 0

    def int8(self) -> bool:
        return self.dtype == INT8

    def truncate(self, n_seen: int) -> None:
        _check(self._lib, self._lib.dbi_kv_truncate(self._h, n_seen))

    def reset(self) -> None:
        self.truncate(0)

    def mark_position(self, pos: int) -> None:
        self.truncate(pos + 1)

    def set_stream(self, stream_ptr: int | None) -> None:
        _check(self._lib, self._lib.dbi_kv_set_stream(self._h, stream_ptr or None))

    def sync(self) -> None:
        _check(self._lib, self._lib.dbi_kv_sync(self._h))

    # ---- append
    def append(self, layer: int, pos: int, k, v) -> None:
        k, v = _f32(k), _f32(v)
        assert k.size == self.pos_stride and v.size == self.pos_stride
        _check(self._lib, self._lib.dbi_kv_append(self._h, layer, pos, _ptr(k), _ptr(v)))

    def append_n(self, layer: int, pos0: int, k, v) -> None:
        k, v = _f32(k), _f32(v)
        n = k.size // self.pos_stride
        assert k.size == n * self.pos_stride and v.size == k.size
        _check(self._lib, self._lib.dbi_kv_append_n(self._h, layer, pos0, n, _ptr(k), _ptr(v)))

    def append_async(self, layer: int, pos0: int, n: int, k_dev: int, v_dev: int) -> None:
        _check(self._lib, self._lib.dbi_kv_append_async(self._h, layer, pos0, n, k_dev, v_dev))

    # ---- ring mapping
    def slot_for(self, pos: int) -> int:
        out = ctypes.c_uint32()
        _check(self._lib, self._lib.dbi_kv_slot_for(self._h, pos, ctypes.byref(out)))
        return int(out.value)

    def residents(self) -> tuple[np.ndarray, np.ndarray]:
        cap = self.capacity
        slot = np.zeros(cap, np.uint32)
        rp = np.zeros(cap, np.int32)
        cnt = ctypes.c_uint32()
        _check(self._lib, self._lib.dbi_kv_residents(self._h, _ptr(slot), _ptr(rp), cap,
                                                     ctypes.byref(cnt)))
        return slot[: cnt.value].copy(), rp[: cnt.value].copy()

    # ---- attention
    def attend(self, layer: int, pos: int, q, n_heads: int, scale: float) -> np.ndarray:
        q = _f32(q)
        assert q.size == n_heads * self.head_dim
        out = np.empty(n_heads * self.head_dim, np.float32)
        _check(self._lib, self._lib.dbi_attn_decode(self._h, layer, pos, n_heads, scale, _ptr(q),
                                                    _ptr(out)))
        return out

    def attend_async(self, layer: int, pos: int, n_heads: int, scale: float, q_dev: int,
                     out_dev: int) -> None:
        _check(self._lib, self._lib.dbi_attn_decode_async(self._h, layer, pos, n_heads, scale,
                                                          q_dev, out_dev))

    def splits(self, pos0: int, rows: int, n_heads: int) -> int:
        """Key splits (partial records per row and kv head) of an attention call."""
        out = ctypes.c_uint32()
        _check(self._lib, self._lib.dbi_attn_splits(self._h, pos0, rows, n_heads,
                                                    ctypes.byref(out)))
        return int(out.value)

    def decode(self, layer: int, pos: int, k, v, q, n_heads: int, scale: float) -> np.ndarray:
        """Fused append of (k, v) at pos + attention of q at pos (one launch)."""
        k, v, q = _f32(k), _f32(v), _f32(q)
        assert k.size == self.pos_stride and v.size == self.pos_stride
        assert q.size == n_heads * self.head_dim
        out = np.empty(n_heads * self.head_dim, np.float32)
        _check(self._lib, self._lib.dbi_kv_decode(self._h, layer, pos, _ptr(k), _ptr(v), n_heads,
                                                  scale, _ptr(q), _ptr(out)))
        return out

    def decode_async(self, layer: int, pos: int, k_dev: int, v_dev: int, n_heads: int,
                     scale: float, q_dev: int, out_dev: int) -> None:
        _check(self._lib, self._lib.dbi_kv_decode_async(self._h, layer, pos, k_dev, v_dev, n_heads,
                                                        scale, q_dev, out_dev))

    def decode_noalloc_async(self, layer: int, pos: int, k_dev: int, v_dev: int, n_heads: int,
                             scale: float, q_dev: int, out_dev: int) -> None:
        """decode_async through the allocation-free entry point (static scratch)."""
        _check(self._lib, self._lib.dbi_kv_decode_noalloc_async(
            self._h, layer, pos, k_dev, v_dev, n_heads, scale, q_dev, out_dev))

    def attend_chunk(self, layer: int, pos0: int, q, n_heads: int, scale: float) -> np.ndarray:
        q = _f32(q)
        n = q.size // (n_heads * self.head_dim)
        assert q.size == n * n_heads * self.head_dim
        out = np.empty(q.size, np.float32)
        _check(self._lib, self._lib.dbi_attn_chunk(self._h, layer, pos0, n, n_heads, scale,
                                                   _ptr(q), _ptr(out)))
        return out

    def attend_chunk_async(self, layer: int, pos0: int, n: int, n_heads: int, scale: float,
                           q_dev: int, out_dev: int) -> None:
        _check(self._lib, self._lib.dbi_attn_chunk_async(self._h, layer, pos0, n, n_heads, scale,
                                                         q_dev, out_dev))

    # ---- q/k/v producer (bias + rope on the device, then append + attention)
    def _biases(self, n_heads, q_bias, k_bias, v_bias):
        out = []
        for b, size in ((q_bias, n_heads * self.head_dim), (k_bias, self.pos_stride),
                        (v_bias, self.pos_stride)):
            if b is None:
                out.append(None)
            else:
                b = _f32(b)
                assert b.size == size
                out.append(b)
        return out

    def decode_qkv(self, layer: int, pos: int, q, k, v, n_heads: int, scale: float,
                   q_bias=None, k_bias=None, v_bias=None) -> np.ndarray:
        """decode_layer's attention half from raw projections (model.cpp:747-771)."""
        q, k, v = _f32(q), _f32(k), _f32(v)
        assert q.size == n_heads * self.head_dim
        assert k.size == self.pos_stride and v.size == self.pos_stride
        bs = self._biases(n_heads, q_bias, k_bias, v_bias)
        out = np.empty(q.size, np.float32)
        _check(self._lib, self._lib.dbi_kv_decode_qkv(
            self._h, layer, pos, n_heads, scale, _ptr(q), _ptr(k), _ptr(v),
            *[None if b is None else _ptr(b) for b in bs], _ptr(out)))
        return out

    def decode_qkv_async(self, layer: int, pos: int, n_heads: int, scale: float, q_dev: int,
                         k_dev: int, v_dev: int, q_bias_dev, k_bias_dev, v_bias_dev,
                         out_dev: int) -> None:
        _check(self._lib, self._lib.dbi_kv_decode_qkv_async(
            self._h, layer, pos, n_heads, scale, q_dev, k_dev, v_dev, q_bias_dev, k_bias_dev,
            v_bias_dev, out_dev))

    def chunk_qkv(self, layer: int, pos0: int, q, k, v, n_heads: int, scale: float,
                  q_bias=None, k_bias=None, v_bias=None) -> np.ndarray:
        """decode_layer_chunk's attention half from raw projections (model.cpp:933-981)."""
        q, k, v = _f32(q), _f32(k), _f32(v)
        n = q.size // (n_heads * self.head_dim)
        assert q.size == n * n_heads * self.head_dim
        assert k.size == n * self.pos_stride and v.size == n * self.pos_stride
        bs = self._biases(n_heads, q_bias, k_bias, v_bias)
        out = np.empty(q.size, np.float32)
        _check(self._lib, self._lib.dbi_kv_chunk_qkv(
            self._h, layer, pos0, n, n_heads, scale, _ptr(q), _ptr(k), _ptr(v),
            *[None if b is None else _ptr(b) for b in bs], _ptr(out)))
        return out

    def chunk_qkv_async(self, layer: int, pos0: int, n: int, n_heads: int, scale: float,
                        q_dev: int, k_dev: int, v_dev: int, q_bias_dev, k_bias_dev,
                        v_bias_dev, out_dev: int) -> None:
        _check(self._lib, self._lib.dbi_kv_chunk_qkv_async(
            self._h, layer, pos0, n, n_heads, scale, q_dev, k_dev, v_dev, q_bias_dev,
            k_bias_dev, v_bias_dev, out_dev))

    # ---- speculative verify round (token side)
    def spec_verify_async(self, k: int, vocab: int, logits_dev: int, draft_dev: int,
                          verified_dev: int, accepted_dev: int) -> None:
        _check(self._lib, self._lib.dbi_spec_verify_async(
            self._h, k, vocab, logits_dev, draft_dev, verified_dev, accepted_dev))

    def verify_commit(self, pos: int, k: int, vocab: int, logits_dev: int, draft):
        """(accepted, merged tokens); the cache keeps pos + accepted + 1 positions."""
        d = np.ascontiguousarray(draft, dtype=np.int32)
        assert d.size == k
        merged = np.zeros(k + 1, np.int32)
        acc = ctypes.c_uint32()
        _check(self._lib, self._lib.dbi_kv_verify_commit(
            self._h, pos, k, vocab, logits_dev, _ptr(d), _ptr(merged), ctypes.byref(acc)))
        return int(acc.value), merged[: acc.value + 1].tolist()

    # ---- output projection + residual (decode_layer's step after attention)
    def oproj_residual_async(self, wtype: int, w_dev: int, attn_dev: int, x_dev: int, dim: int,
                             n_in: int) -> None:
        _check(self._lib, self._lib.dbi_oproj_residual_async(self._h, wtype, w_dev, attn_dev,
                                                             x_dev, dim, n_in))

    # ---- full-layer offload (backend.hpp:133-157)
    def offload_setup(self, dim: int, ff: int, n_heads: int, rms_eps: float, layers: list,
                      output_norm: int | None = None, lm_head: tuple | None = None,
                      vocab: int = 0, host: bool = False) -> None:
        """layers: per block a dict of pointers attn_norm, ffn_norm, bq/bk/bv
        (or None) and (pointer, wtype) tuples wq wk wv wo wgate wup wdown;
        lm_head: (pointer, wtype) or None. Device pointers, or with host=True
        host pointers that the library copies to the device
        (dbi_offload_setup_host)."""
        arr = (_lib.LayerWeights * len(layers))()
        for i, L in enumerate(layers):
            a = arr[i]
            a.attn_norm, a.ffn_norm = L["attn_norm"], L["ffn_norm"]
            for name in ("wq", "wk", "wv", "wo", "wgate", "wup", "wdown"):
                ptr, wt = L[name]
                setattr(a, name, _lib.Weight(ptr, wt))
            a.bq, a.bk, a.bv = L.get("bq"), L.get("bk"), L.get("bv")
        cfg = _lib.OffloadConfig(dim, ff, n_heads, rms_eps, output_norm,
                                 _lib.Weight(*(lm_head if lm_head else (None, 0))), vocab)
        fn = self._lib.dbi_offload_setup_host if host else self._lib.dbi_offload_setup
        _check(self._lib, fn(self._h, ctypes.byref(cfg), arr, len(layers)))
        self._vocab = vocab if lm_head else 0

    def decode_token_async(self, x_dev: int, pos: int) -> None:
        _check(self._lib, self._lib.dbi_decode_token_async(self._h, x_dev, pos))

    def decode_token_full_async(self, x_dev: int, pos: int, logits_dev: int) -> None:
        _check(self._lib, self._lib.dbi_decode_token_full_async(self._h, x_dev, pos, logits_dev))

    def decode_token(self, x, pos: int) -> np.ndarray:
        """Host residual row in, the row after every bound block out."""
        xa = _f32(x).copy()
        _check(self._lib, self._lib.dbi_decode_token(self._h, _ptr(xa), pos))
        return xa

    def decode_token_full(self, x, pos: int, vocab: int) -> np.ndarray:
        # the library writes the vocabulary bound at setup: a buffer of any
        # other size would be overrun or left short
        if vocab != self._vocab:
            raise ValueError(f"vocab {vocab} differs from the {self._vocab} bound at setup")
        xa = _f32(x)
        logits = np.empty(vocab, np.float32)
        _check(self._lib, self._lib.dbi_decode_token_full(self._h, _ptr(xa), pos, _ptr(logits)))
        return logits

    # ---- prefix cache
    def save_prefix(self, path: str, tokens) -> None:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        _check(self._lib, self._lib.dbi_kv_prefix_save(self._h, path.encode(), _ptr(t), t.size))

    def load_prefix(self, path: str, tokens) -> int:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        n = ctypes.c_uint32()
        _check(self._lib, self._lib.dbi_kv_prefix_load(self._h, path.encode(), _ptr(t), t.size,
                                                       ctypes.byref(n)))
        return int(n.value)

    # ---- readback in the reference layout
    def export(self, what: str, layer: int) -> np.ndarray:
        code = _lib.EXPORT[what]
        nbytes = int(self._lib.dbi_kv_export_bytes(self._h, code))
        if nbytes == 0:
            raise DbiError(_lib.DBI_ERR_UNSUPPORTED, f"{what} not present in this layout")
        dt = np.int8 if what in ("k8", "v8") else np.float32
        out = np.empty(nbytes // np.dtype(dt).itemsize, dt)
        _check(self._lib, self._lib.dbi_kv_export(self._h, code, layer, _ptr(out), nbytes))
        return out
