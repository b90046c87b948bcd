"""Prefix cache of the dense int8 cache (DBKVCACH v2, this library's format;
the reference's v1 is dense-fp32-only, model.cpp:1074-1075) and v1 files
loaded into an int8 cache.

Pinned by:
- the file's sections parsed with numpy against the cache's own readback
  (`dbi_kv_export`, the reference layout): codes, scales, raw staging rows
  and sinks of the first len positions, in the documented order;
- load into a fresh cache, then every stored array bit-identical to the
  oracle that appended the same rows, and the next steps (append + attend)
  bit-identical to the cache that was saved;
- a v1 (fp32) file into an int8 cache equals appending the prefix;
- the validation paths (layout mismatch, truncation, mid-group prefixes).
"""
import numpy as np
import pytest

import pyoracle
from dbinfer_amd.kv import F32, INT8, DbiError, HipKV
from helpers import normal

pytestmark = pytest.mark.gpu

NAMES = ["k8", "v8", "k_scale", "v_scale", "k_raw", "k_sink", "v_sink"]


def same_bits(a, b, what):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), what


def filled(L, cap, nkv, hd, n_sink, n, seed):
    g = HipKV(L, cap, nkv, hd, n_sink, 0, INT8, 1e6)
    o = pyoracle.OracleKV(L, cap, nkv, hd, n_sink, 0, INT8, 1e6)
    P = nkv * hd
    K, V = normal(seed, L, n, P), normal(seed + 1, L, n, P)
    K[:, :, 3] *= 8.0
    for l in range(L):
        g.append_n(l, 0, K[l], V[l])
        o.append_n(l, 0, K[l], V[l])
    return g, o, K, V


def parse_v2(path, L, nkv, hd, n_sink):
    b = open(path, "rb").read()
    assert b[:8] == b"DBKVCACH"
    hdr = np.frombuffer(b, "<u4", 7, 8)
    assert hdr[0] == 2 and list(hdr[1:4]) == [L, nkv, hd] and hdr[5] == 1 and hdr[6] == n_sink
    n = int(hdr[4])
    at = 8 + 7 * 4
    toks = np.frombuffer(b, "<i4", n, at)
    at += 4 * n
    P, nb, ngl, w, ns = nkv * hd, hd // 32, -(-n // 32), n % 32, min(n_sink, n)
    out = {"tokens": toks, "len": n}
    for name, dt, shape in [("k8", "i1", (L, n, P)), ("v8", "i1", (L, n, P)),
                            ("v_scale", "<f4", (L, n, nkv * nb)), ("k_scale", "<f4", (L, ngl, P)),
                            ("k_raw", "<f4", (L, w, P)), ("k_sink", "<f4", (L, ns, P)),
                            ("v_sink", "<f4", (L, ns, P))]:
        cnt = int(np.prod(shape))
        out[name] = np.frombuffer(b, dt, cnt, at).reshape(shape)
        at += cnt * np.dtype(dt).itemsize
    assert at == len(b), "file longer than its sections"
    return out


@pytest.mark.parametrize("n,n_sink", [(96, 4), (70, 4), (45, 0), (3, 4)])
def test_int8_prefix_roundtrip(tmp_path, n, n_sink):
    L, cap, nkv, hd = 3, 160, 2, 128
    g, o, K, V = filled(L, cap, nkv, hd, n_sink, n, 800 + n)
    toks = np.arange(5000, 5000 + n, dtype=np.int32)
    path = str(tmp_path / "p.kv")
    g.save_prefix(path, toks)  # len == n_seen: any length
    f = parse_v2(path, L, nkv, hd, n_sink)
    assert np.array_equal(f["tokens"], toks)
    P = nkv * hd
    for l in range(L):
        same_bits(f["k8"][l], g.export("k8", l).reshape(cap, P)[:n], f"file k8 layer {l}")
        same_bits(f["v8"][l], g.export("v8", l).reshape(cap, P)[:n], f"file v8 layer {l}")
        same_bits(f["v_scale"][l], g.export("v_scale", l).reshape(cap, -1)[:n], "file v_scale")
        same_bits(f["k_scale"][l], g.export("k_scale", l).reshape(-1, P)[:-(-n // 32)],
                  "file k_scale")
        same_bits(f["k_raw"][l], g.export("k_raw", l).reshape(32, P)[:n % 32], "file k_raw")
        if n_sink:
            ns = min(n_sink, n)
            same_bits(f["k_sink"][l], g.export("k_sink", l).reshape(n_sink, P)[:ns], "k_sink")
            same_bits(f["v_sink"][l], g.export("v_sink", l).reshape(n_sink, P)[:ns], "v_sink")
    fresh = HipKV(L, cap, nkv, hd, n_sink, 0, INT8, 1e6)
    assert fresh.load_prefix(path, np.concatenate([toks, [7, 8]])) == n
    assert fresh.n_seen == n
    names = NAMES if n_sink else NAMES[:5]
    # continue both caches and the oracle with the same rows, then compare all
    sc = np.float32(1.0) / np.sqrt(np.float32(hd))
    for t in range(n, n + 40):
        k, v, q = normal(900 + t, P), normal(901 + t, P), normal(902 + t, 8 * hd)
        for l in range(L):
            a = fresh.decode(l, t, k, v, q, 8, sc)
            b = g.decode(l, t, k, v, q, 8, sc)
            same_bits(a, b, f"step {t} layer {l} after load vs saved cache")
            o.append(l, t, k, v)
    for l in range(L):
        for name in names:
            same_bits(fresh.export(name, l), o.export(name, l), f"{name} layer {l} vs oracle")
    fresh.close()
    g.close()


def test_v1_prefix_into_int8_cache_equals_appending(tmp_path):
    L, cap, nkv, hd, n = 2, 128, 2, 64, 77
    src = HipKV(L, cap, nkv, hd)  # dense fp32
    P = nkv * hd
    K, V = normal(810, L, n, P), normal(811, L, n, P)
    for l in range(L):
        src.append_n(l, 0, K[l], V[l])
    toks = np.arange(n, dtype=np.int32)
    path = str(tmp_path / "v1.kv")
    src.save_prefix(path, toks)
    q8 = HipKV(L, cap, nkv, hd, 4, 0, INT8, 1e4)
    assert q8.load_prefix(path, toks) == n
    o = pyoracle.OracleKV(L, cap, nkv, hd, 4, 0, INT8, 1e4)
    for l in range(L):
        o.append_n(l, 0, K[l], V[l])
        for name in NAMES:
            same_bits(q8.export(name, l), o.export(name, l), f"{name} layer {l}")
    src.close()
    q8.close()


def test_int8_prefix_errors(tmp_path):
    L, cap, nkv, hd = 2, 96, 2, 64
    g, _, _, _ = filled(L, cap, nkv, hd, 4, 80, 820)
    toks = np.arange(80, dtype=np.int32)
    with pytest.raises(DbiError) as e:  # mid-group, short of n_seen
        g.save_prefix(str(tmp_path / "x.kv"), toks[:50])
    assert "32-token group boundary" in e.value.message
    path = str(tmp_path / "p.kv")
    g.save_prefix(path, toks[:64])  # on a group boundary
    other_sinks = HipKV(L, cap, nkv, hd, 0, 0, INT8, 1e4)
    with pytest.raises(DbiError) as e:
        other_sinks.load_prefix(path, toks)
    assert e.value.message == "kv prefix cache int8 layout does not match this cache"
    fp = HipKV(L, cap, nkv, hd)
    with pytest.raises(DbiError) as e:
        fp.load_prefix(path, toks)
    assert "holds an int8 cache" in e.value.message
    ok = HipKV(L, cap, nkv, hd, 4, 0, INT8, 1e4)
    bad = str(tmp_path / "bad.kv")
    open(bad, "wb").write(open(path, "rb").read()[:-1])
    before = ok.export("k8", 1)
    with pytest.raises(DbiError) as e:
        ok.load_prefix(bad, toks)
    assert e.value.message == "kv prefix cache payload size mismatch"
    assert ok.n_seen == 0
    same_bits(ok.export("k8", 1), before, "untouched after a failed load")
    assert ok.load_prefix(path, toks) == 64
    for h in (g, other_sinks, fp, ok):
        h.close()
