"""Pins the oracle's int8 quantization (quant_head model.cpp:303-317,
requantize_kgroup :329-355, append :357-404).

Closed-form checks rather than a retyped formula:
- the block/channel maximum maps to exactly +-127 and the scale equals the
  fp32 quotient max/127;
- every code is the round-half-AWAY-from-zero of x*inv (exact .5 ties are
  built so that round-half-even would fail);
- |x - s*q| <= s/2 (+ fp32 slack) and the reference's own bound
  |x - s*q| <= s + 1e-6 (tests/kv_int8_test.cpp:33-55, LCG seed 0xC0FFEE);
- zero blocks give scale 0 and code 0;
- sinks (pos < n_sink) stay fp32 and are excluded from their group's scale;
- a rollback across a group boundary requantizes the earlier group from the
  staging rows the later group overwrote (model.cpp:359-362, 337-353);
- int8 attention stays within 0.6% relative L2 of fp32 attention
  (tests/kv_int8_test.cpp:115-137, LCG seed 0x1357).
"""
import numpy as np
import pytest

import pyoracle
from helpers import Lcg, normal


def round_half_away(x):
    return np.sign(x) * np.floor(np.abs(x) + 0.5)


def test_quant_head_closed_form():
    x = normal(1, 200) * 3
    x[40:64] = 0.0  # part of block 1 zero
    x[64:96] = 0.0  # block 2 all zero
    codes, scales = pyoracle.quant_head(x)
    for b in range(len(scales)):
        blk = x[b * 32:(b + 1) * 32]
        m = np.float32(np.max(np.abs(blk)))
        assert scales[b] == np.float32(m / np.float32(127.0))
        c = codes[b * 32:(b + 1) * 32]
        if m == 0:
            assert scales[b] == 0 and not c.any()
            continue
        assert np.max(np.abs(c)) == 127
        i = int(np.argmax(np.abs(blk)))
        assert c[i] == np.sign(blk[i]) * 127
        inv = np.float32(1.0) / scales[b]
        assert np.array_equal(c, np.clip(round_half_away(blk * inv), -127, 127).astype(np.int8))
        err = np.abs(blk.astype(np.float64) - scales[b] * c.astype(np.float64))
        assert np.all(err <= scales[b] * 0.5 * (1 + 1e-5) + 1e-12)


def test_quant_ties_round_away_from_zero():
    # max 127 -> scale exactly 1.0, inv 1.0: codes are round(x) with .5 ties
    blk = np.array([127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5] + [0.0] * 24, np.float32)
    codes, scales = pyoracle.quant_head(blk)
    assert scales[0] == 1.0
    assert codes[:8].tolist() == [127, 3, -3, 1, -1, 2, -2, 127]


def test_partial_last_block():
    x = normal(2, 40)  # hd 40: blocks [0,32) and [32,40)
    codes, scales = pyoracle.quant_head(x)
    assert len(scales) == 2
    assert scales[1] == np.float32(np.max(np.abs(x[32:])) / np.float32(127))
    assert np.max(np.abs(codes[32:])) == 127


def test_kv_int8_roundtrip_lcg():
    """tests/kv_int8_test.cpp:33-55"""
    nkv, hd, slots = 3, 40, 5
    rng = Lcg(0xC0FFEE)
    kv = pyoracle.OracleKV(1, slots, nkv, hd, dtype=pyoracle.INT8)
    for s in range(slots):
        k = rng.fill(nkv * hd, 7.0)
        v = rng.fill(nkv * hd, 0.03)
        kv.append(0, s, k, v)
        k8 = kv.export("k8", 0).reshape(slots, nkv, hd)[s]
        ks = kv.export("k_scale", 0).reshape(-1, nkv, hd)[s // 32]
        err = np.abs(k.reshape(nkv, hd) - ks * k8.astype(np.float32))
        assert np.all(err <= ks + 1e-6)


def test_per_channel_group_scale_and_sinks():
    nkv, hd, n_sink = 2, 64, 4
    kv = pyoracle.OracleKV(1, 96, nkv, hd, n_sink=n_sink, dtype=pyoracle.INT8)
    K = normal(3, 70, nkv * hd)
    V = normal(4, 70, nkv * hd)
    K[:, 5] *= 8  # outlier channel
    for p in range(70):
        kv.append(0, p, K[p], V[p])
    k8 = kv.export("k8", 0).reshape(96, nkv * hd)
    ks = kv.export("k_scale", 0).reshape(3, nkv * hd)
    # sinks kept fp32, their int8 slots untouched
    assert np.array_equal(kv.export("k_sink", 0).reshape(n_sink, -1), K[:n_sink])
    assert np.array_equal(kv.export("v_sink", 0).reshape(n_sink, -1), V[:n_sink])
    assert not k8[:n_sink].any()
    # group 0 scale ignores sink rows; full groups use all 32 rows
    assert np.array_equal(ks[0], (np.max(np.abs(K[n_sink:32]), axis=0) / np.float32(127)))
    assert np.array_equal(ks[1], (np.max(np.abs(K[32:64]), axis=0) / np.float32(127)))
    # group 2 holds rows 64..69 so far
    assert np.array_equal(ks[2], (np.max(np.abs(K[64:70]), axis=0) / np.float32(127)))
    inv = np.where(ks[1] > 0, np.float32(1) / ks[1], np.float32(0))
    assert np.array_equal(k8[32:64], np.clip(round_half_away(K[32:64] * inv), -127, 127))
    # per-block V
    vs = kv.export("v_scale", 0).reshape(96, nkv, 2)
    assert vs[10, 1, 0] == np.float32(np.max(np.abs(V[10, 64:96])) / np.float32(127))
    assert not vs[:n_sink].any()


def test_rollback_across_group_aliases_staging_rows():
    """Reference behaviour: k_raw is indexed by pos % 32. After appending into
    group 1 (rows 0..8 now hold pos 32..40), rolling back to pos 30 and
    appending requantizes group 0 from raw rows 0..30, i.e. slots 0..8 are
    re-coded from pos 32..40's keys."""
    nkv, hd = 1, 32
    kv = pyoracle.OracleKV(1, 64, nkv, hd, dtype=pyoracle.INT8)
    K = normal(5, 41, hd)
    V = normal(6, 41, hd)
    for p in range(41):
        kv.append(0, p, K[p], V[p])
    kv.truncate(30)
    knew = normal(7, hd)
    kv.append(0, 30, knew, V[30])
    assert kv.n_seen == 31
    rows = np.concatenate([K[32:41], K[9:30], knew[None]])  # raw rows 0..30
    sc = np.max(np.abs(rows), axis=0) / np.float32(127)
    ks = kv.export("k_scale", 0).reshape(2, hd)
    assert np.array_equal(ks[0], sc)
    inv = np.where(sc > 0, np.float32(1) / sc, np.float32(0))
    k8 = kv.export("k8", 0).reshape(64, hd)
    assert np.array_equal(k8[:31], np.clip(round_half_away(rows * inv), -127, 127))
    # slot 31 keeps its code from before the rollback (not requantized)
    raw = kv.export("k_raw", 0).reshape(32, hd)
    assert np.array_equal(raw[:9], K[32:41]) and np.array_equal(raw[30], knew)


def test_int8_attention_within_fp32_bound():
    """tests/kv_int8_test.cpp:115-137"""
    hd, keys = 64, 48
    rng = Lcg(0x1357)
    q = rng.fill(hd)
    k = rng.fill(keys * hd).reshape(keys, hd)
    v = rng.fill(keys * hd).reshape(keys, hd)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    f = pyoracle.OracleKV(1, keys, 1, hd, dtype=pyoracle.F32)
    i = pyoracle.OracleKV(1, keys, 1, hd, dtype=pyoracle.INT8)
    for p in range(keys):
        f.append(0, p, k[p], v[p])
        i.append(0, p, k[p], v[p])
    ref = f.attend(0, keys - 1, q, 1, scale).astype(np.float64)
    got = i.attend(0, keys - 1, q, 1, scale).astype(np.float64)
    rel = np.sqrt(np.sum((got - ref) ** 2) / np.sum(ref ** 2))
    assert rel <= 0.006


@pytest.mark.parametrize("window,n_sink", [(16, 4), (8, 0)])
def test_ring_int8_per_block_keys(window, n_sink):
    nkv, hd = 2, 64
    kv = pyoracle.OracleKV(1, 0, nkv, hd, n_sink=n_sink, window=window, dtype=pyoracle.INT8)
    K = normal(8, 40, nkv * hd)
    V = normal(9, 40, nkv * hd)
    for p in range(40):
        kv.append(0, p, K[p], V[p])
    k8 = kv.export("k8", 0).reshape(-1, nkv * hd)
    ks = kv.export("k_scale", 0).reshape(-1, nkv * 2)
    for t in range(40 - window, 40):
        s = kv.slot_for(t)
        c, sc = pyoracle.quant_head(K[t][:hd])
        assert np.array_equal(k8[s, :hd], c) and np.array_equal(ks[s, :2], sc)
