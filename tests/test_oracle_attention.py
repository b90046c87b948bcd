"""Pins the oracle's attention (model.cpp:567-728, 956-981) against
independent float64 formulations.

- dense fp32: textbook softmax attention in float64 (numpy) on the shapes of
  tests/metal_ops_test.cpp:164-170 (nh/nkv 14/2 and 8/8, hd 64/128,
  n_pos 1, 2, 64, 300);
- dense int8: float64 attention over the DEQUANTIZED cache (sinks fp32,
  K = ks[c] * k8, V = vs[b] * v8): pins the fused dequant order and the sink
  split without retyping it;
- ring: float64 attention over the resident keys gathered by slot, each roped
  in float64 at its cache-relative position, q roped at n_res - 1 (the
  reduction of attend_ring to dense attention + rope); and the table-driven
  oracle equals the literal per-query-head form bit for bit;
- chunk: equals per-row decode bit for bit (the reference's invariant,
  tests/chunked_prefill_test.cpp:52);
- head-parallel runs equal 1-thread runs bit for bit.
A dropped term, wrong sign, wrong gqa mapping (h/gqa) or a transposed
operand fails these comparisons.
"""
import numpy as np
import pytest

import pyoracle
from helpers import assert_close, attention64, normal, rope64

SCALE = lambda hd: np.float32(1.0) / np.sqrt(np.float32(hd))  # noqa: E731  model.cpp:757


def fill_dense(kv, L, n, seed):
    P = kv.pos_stride
    K = normal(seed, L, n, P)
    V = normal(seed + 1, L, n, P)
    for l in range(L):
        for p in range(n):
            kv.append(l, p, K[l, p], V[l, p])
    return K, V


@pytest.mark.parametrize("nh,nkv", [(14, 2), (8, 8)])
@pytest.mark.parametrize("hd", [64, 128])
@pytest.mark.parametrize("n_pos", [1, 2, 64, 300])
def test_dense_f32_vs_float64(nh, nkv, hd, n_pos):
    kv = pyoracle.OracleKV(1, 320, nkv, hd, dtype=pyoracle.F32)
    K, V = fill_dense(kv, 1, n_pos, 100 + hd + n_pos)
    q = normal(7, nh * hd)
    got = kv.attend(0, n_pos - 1, q, nh, SCALE(hd)).reshape(nh, hd)
    g = nh // nkv
    for h in range(nh):
        kh = h // g
        want = attention64(q[h * hd:(h + 1) * hd], K[0, :, kh * hd:(kh + 1) * hd],
                           V[0, :, kh * hd:(kh + 1) * hd], float(SCALE(hd)))
        assert_close(got[h], want, atol=2e-6, rtol=2e-5, what=f"head {h}")


def dequant_dense_int8(kv, layer, n):
    nkv, hd = kv.n_kv_heads, kv.head_dim
    k8 = kv.export("k8", layer).reshape(-1, nkv, hd)[:n].astype(np.float64)
    v8 = kv.export("v8", layer).reshape(-1, nkv, hd)[:n].astype(np.float64)
    ks = kv.export("k_scale", layer).reshape(-1, nkv, hd)
    vs = kv.export("v_scale", layer).reshape(-1, nkv, kv.n_blocks)
    Kd = k8 * ks[np.arange(n) // 32]
    Vd = v8 * np.repeat(vs[:n], 32, axis=2)[:, :, :hd]
    ns = min(kv.n_sink, n)
    if ns:
        Kd[:ns] = kv.export("k_sink", layer).reshape(-1, nkv, hd)[:ns]
        Vd[:ns] = kv.export("v_sink", layer).reshape(-1, nkv, hd)[:ns]
    return Kd, Vd


@pytest.mark.parametrize("n_sink", [0, 4])
@pytest.mark.parametrize("nh,nkv,hd,n", [(24, 8, 128, 100), (8, 2, 64, 33), (7, 1, 128, 5)])
def test_dense_int8_vs_dequantized_float64(n_sink, nh, nkv, hd, n):
    kv = pyoracle.OracleKV(1, 128, nkv, hd, n_sink=n_sink, dtype=pyoracle.INT8)
    fill_dense(kv, 1, n, 40 + n)
    q = normal(8, nh * hd)
    got = kv.attend(0, n - 1, q, nh, SCALE(hd)).reshape(nh, hd)
    Kd, Vd = dequant_dense_int8(kv, 0, n)
    g = nh // nkv
    for h in range(nh):
        want = attention64(q[h * hd:(h + 1) * hd], Kd[:, h // g], Vd[:, h // g], float(SCALE(hd)))
        assert_close(got[h], want, atol=2e-6, rtol=2e-5, what=f"head {h}")


def ring_reference64(kv, layer, q, nh, theta):
    """float64 attention over gathered residents with explicit rope."""
    nkv, hd = kv.n_kv_heads, kv.head_dim
    slots, rp = kv.residents()
    if kv.dtype == pyoracle.INT8:
        k8 = kv.export("k8", layer).reshape(-1, nkv, hd).astype(np.float64)
        ks = kv.export("k_scale", layer).reshape(-1, nkv, kv.n_blocks)
        v8 = kv.export("v8", layer).reshape(-1, nkv, hd).astype(np.float64)
        vs = kv.export("v_scale", layer).reshape(-1, nkv, kv.n_blocks)
        K = k8 * np.repeat(ks, 32, axis=2)[:, :, :hd]
        V = v8 * np.repeat(vs, 32, axis=2)[:, :, :hd]
        # the reference dequantizes K in fp32 before roping (model.cpp:689-690)
        K = (k8.astype(np.float32) * np.repeat(ks, 32, axis=2)[:, :, :hd]).astype(np.float64)
    else:
        K = kv.export("k", layer).reshape(-1, nkv, hd).astype(np.float64)
        V = kv.export("v", layer).reshape(-1, nkv, hd).astype(np.float64)
    g = nh // nkv
    n_res = len(slots)
    out = np.zeros((nh, hd))
    for h in range(nh):
        qh = rope64(q[h * hd:(h + 1) * hd], n_res - 1, theta)
        keys = np.stack([rope64(K[s, h // g], r, theta) for s, r in zip(slots, rp)])
        out[h] = attention64(qh, keys, V[slots, h // g], float(SCALE(hd)))
    return out


@pytest.mark.parametrize("dtype", [pyoracle.F32, pyoracle.INT8])
@pytest.mark.parametrize("n_sink,window,steps", [(4, 16, 50), (0, 8, 20), (2, 32, 10)])
def test_ring_vs_float64_and_literal(dtype, n_sink, window, steps):
    nh, nkv, hd, theta = 8, 2, 64, 1e6
    a = pyoracle.OracleKV(1, 0, nkv, hd, n_sink=n_sink, window=window, dtype=dtype,
                          rope_theta=theta)
    b = pyoracle.OracleKV(1, 0, nkv, hd, n_sink=n_sink, window=window, dtype=dtype,
                          rope_theta=theta)
    for t in range(steps):
        q = normal(1000 + t, nh * hd)
        k = normal(2000 + t, nkv * hd)
        v = normal(3000 + t, nkv * hd)
        out = a.attend_ring(0, t, q, k, v, nh, SCALE(hd))
        lit = b.attend_ring(0, t, q, k, v, nh, SCALE(hd), literal=True)
        assert np.array_equal(out.view(np.uint32), lit.view(np.uint32)), f"step {t}"
        if t in (0, steps // 2, steps - 1):
            want = ring_reference64(a, 0, q, nh, theta)
            assert_close(out.reshape(nh, hd), want, atol=5e-6, rtol=5e-5, what=f"step {t}")


@pytest.mark.parametrize("dtype", [pyoracle.F32, pyoracle.INT8])
def test_chunk_equals_per_row_decode(dtype):
    nh, nkv, hd, n0, n = 8, 2, 64, 37, 9
    kv = pyoracle.OracleKV(1, 64, nkv, hd, n_sink=4, dtype=dtype)
    fill_dense(kv, 1, n0 + n, 77)
    q = normal(5, n, nh * hd)
    chunk = kv.attend_chunk(0, n0, q, nh, SCALE(hd)).reshape(n, nh * hd)
    for c in range(n):
        row = kv.attend(0, n0 + c, q[c], nh, SCALE(hd))
        assert np.array_equal(chunk[c].view(np.uint32), row.view(np.uint32))


def test_threads_bitwise_equal():
    nh, nkv, hd = 28, 4, 128
    kv = pyoracle.OracleKV(1, 200, nkv, hd, dtype=pyoracle.F32)
    fill_dense(kv, 1, 200, 3)
    q = normal(4, nh * hd)
    one = kv.attend(0, 199, q, nh, SCALE(hd), n_threads=1)
    many = kv.attend(0, 199, q, nh, SCALE(hd), n_threads=5)
    assert np.array_equal(one.view(np.uint32), many.view(np.uint32))
