"""Pins the oracle's prefix cache (model.cpp:1023-1156), speculative merge
(speculative.cpp:10-23) and greedy argmax (sample.cpp:11-28).

Prefix: the byte layout of DBKVCACH v1 is checked field by field with
struct/numpy (independent of the writer), load(save(x)) restores K/V bitwise
and sets n_seen, and every validation error of model.cpp:1117-1148 is hit in
the reference's order with its message, leaving the cache untouched.
Merge: the direct vectors of tests/speculative_test.cpp:104-133 and the
synthetic oracle-greedy stream property of :136-149.
Argmax: the vectors of tests/sample_test.cpp:38-50; the cases whose answer a
strict-greater scan fixes (NaN in slot 0 or later, signed zeros, infinities);
on NaN-free rows with many ties, numpy's argmax (first occurrence of the
maximum); and on rows with NaNs, the characterisation "the earliest index whose
value equals the maximum of the non-NaN values, or 0 when slot 0 is NaN".
"""
import json
import os
import struct

import numpy as np
import pytest

import pyoracle
from helpers import GOLDEN, normal


def filled(L=3, cap=16, nkv=2, hd=8, n=10, seed=1):
    kv = pyoracle.OracleKV(L, cap, nkv, hd, dtype=pyoracle.F32)
    K = normal(seed, L, n, nkv * hd)
    V = normal(seed + 1, L, n, nkv * hd)
    for l in range(L):
        for p in range(n):
            kv.append(l, p, K[l, p], V[l, p])
    return kv, K, V


def test_prefix_file_layout(tmp_path):
    kv, K, V = filled()
    toks = np.array([40, 1079, 264, 4128, 1614, 13], np.int32)
    path = str(tmp_path / "p.kv")
    kv.save_prefix(path, toks)
    data = open(path, "rb").read()
    assert data[:8] == b"DBKVCACH"
    assert struct.unpack("<5I", data[8:28]) == (1, 3, 2, 8, 6)
    assert np.array_equal(np.frombuffer(data[28:52], "<i4"), toks)
    elems = 3 * 6 * 16
    k = np.frombuffer(data[52:52 + 4 * elems], "<f4").reshape(3, 6, 16)
    v = np.frombuffer(data[52 + 4 * elems:], "<f4").reshape(3, 6, 16)
    assert len(data) == 52 + 8 * elems
    assert np.array_equal(k, K[:, :6]) and np.array_equal(v, V[:, :6])


def test_prefix_round_trip(tmp_path):
    kv, K, V = filled()
    toks = list(range(100, 108))
    path = str(tmp_path / "p.kv")
    kv.save_prefix(path, toks)
    fresh = pyoracle.OracleKV(3, 16, 2, 8, dtype=pyoracle.F32)
    assert fresh.load_prefix(path, toks + [7, 7]) == 8
    assert fresh.n_seen == 8
    for l in range(3):
        assert np.array_equal(fresh.export("k", l).reshape(16, 16)[:8], K[l, :8])
        assert np.array_equal(fresh.export("v", l).reshape(16, 16)[:8], V[l, :8])


def corrupt_cases(good: bytes):
    hdr = bytearray(good)
    bad_magic = bytearray(good)
    bad_magic[3] = ord("X")
    bad_ver = bytearray(good)
    bad_ver[8:12] = struct.pack("<I", 2)
    bad_hp = bytearray(good)
    bad_hp[12:16] = struct.pack("<I", 4)
    zero_len = bytearray(good)
    zero_len[24:28] = struct.pack("<I", 0)
    long_len = bytearray(good)
    long_len[24:28] = struct.pack("<I", 18)
    cap_len = bytearray(good)
    cap_len[24:28] = struct.pack("<I", 17)
    tok = bytearray(good)
    tok[28 + 4 * 2:28 + 4 * 3] = struct.pack("<i", 999)
    return [
        (bytes(hdr[:5]), "kv prefix cache truncated"),
        (bytes(bad_magic), "kv prefix cache bad magic"),
        (bytes(bad_magic[:3]), "kv prefix cache truncated"),
        (bytes(hdr[:10]), "kv prefix cache truncated"),
        (bytes(bad_ver), "kv prefix cache version 2 unsupported"),
        (bytes(hdr[:20]), "kv prefix cache truncated"),
        (bytes(bad_hp), "kv prefix cache hyperparams do not match this model"),
        (bytes(zero_len), "kv prefix cache has a zero-length prefix"),
        (bytes(long_len), "kv prefix is longer than the prompt"),
        (bytes(cap_len), "kv prefix exceeds cache capacity"),
        (bytes(tok), "prompt prefix differs from saved cache at token 2"),
        (bytes(hdr[:40]), "kv prefix cache truncated"),
        (bytes(hdr[:-4]), "kv prefix cache payload size mismatch"),
        (bytes(hdr) + b"\0", "kv prefix cache payload size mismatch"),
    ]


PROMPT = list(range(100, 108)) + [1, 2, 3, 4, 5, 6, 7, 8, 9]  # 17 tokens


def test_prefix_load_errors_leave_cache_untouched(tmp_path):
    kv, K, V = filled()
    path = str(tmp_path / "good.kv")
    kv.save_prefix(path, PROMPT[:8])
    good = open(path, "rb").read()
    target, TK, TV = filled(seed=50, n=5)
    for i, (blob, msg) in enumerate(corrupt_cases(good)):
        p = str(tmp_path / f"bad{i}.kv")
        open(p, "wb").write(blob)
        with pytest.raises(pyoracle.OracleError) as e:
            target.load_prefix(p, PROMPT)
        assert str(e.value) == msg, (i, str(e.value))
        assert target.n_seen == 5
        assert np.array_equal(target.export("k", 0).reshape(16, 16)[:5], TK[0])
    with pytest.raises(pyoracle.OracleError) as e:
        target.load_prefix(str(tmp_path / "missing.kv"), PROMPT)
    assert str(e.value).startswith("cannot open kv prefix cache ")
    with pytest.raises(pyoracle.OracleError) as e:
        target.load_prefix(path, PROMPT[:5])
    assert str(e.value) == "kv prefix is longer than the prompt"


def test_prefix_capacity_check(tmp_path):
    big = pyoracle.OracleKV(3, 32, 2, 8, dtype=pyoracle.F32)
    K = normal(3, 20, 16)
    for l in range(3):
        for p in range(20):
            big.append(l, p, K[p], K[p])
    path = str(tmp_path / "big.kv")
    big.save_prefix(path, list(range(20)))
    small = pyoracle.OracleKV(3, 16, 2, 8, dtype=pyoracle.F32)
    with pytest.raises(pyoracle.OracleError) as e:
        small.load_prefix(path, list(range(20)))
    assert str(e.value) == "kv prefix exceeds cache capacity"


def test_prefix_save_errors(tmp_path):
    kv, _, _ = filled(n=4)
    with pytest.raises(pyoracle.OracleError, match="^kv prefix is empty$"):
        kv.save_prefix(str(tmp_path / "a"), [])
    with pytest.raises(pyoracle.OracleError, match="^cache holds fewer positions than the prefix$"):
        kv.save_prefix(str(tmp_path / "a"), list(range(5)))
    i8 = pyoracle.OracleKV(1, 8, 1, 8, dtype=pyoracle.INT8)
    with pytest.raises(pyoracle.OracleError, match="only the dense fp32 cache"):
        i8.save_prefix(str(tmp_path / "a"), [1])
    ring = pyoracle.OracleKV(1, 0, 1, 8, n_sink=1, window=4)
    with pytest.raises(pyoracle.OracleError, match="only the dense fp32 cache"):
        ring.load_prefix(str(tmp_path / "a"), [1])


CASES = json.load(open(os.path.join(GOLDEN, "spec_merge_cases.json")))["cases"]


@pytest.mark.parametrize("case", CASES)
def test_spec_merge_vectors(case):
    acc, out = pyoracle.spec_merge(case["draft"], case["target"])
    assert acc == case["accepted"] and out == case["out"]


def _oracle(x):
    return (x * 7 + 3) % 101  # tests/speculative_test.cpp:45


@pytest.mark.parametrize("seed", [1, 42, 77])
@pytest.mark.parametrize("k", [1, 4, 8])
@pytest.mark.parametrize("wrong", [0, 2, 3, 1])
def test_spec_stream_equals_greedy(seed, k, wrong):
    """Synthetic verify loop: the merged stream equals greedy decoding whatever
    the draft proposes, and pos advances by accepted + 1 (speculative.cpp:82)."""
    n = 50
    greedy, cur = [], seed
    while len(greedy) < n:
        cur = _oracle(cur)
        greedy.append(cur)
    gen, last, pos, step = [], seed, 0, 0
    while len(gen) < n:
        prop, c = [], last
        for i in range(k):
            c = _oracle(c)
            step += 1
            bad = wrong == 1 or (wrong > 1 and step % wrong == 0)
            prop.append((c + 1) % 101 if bad else c)
            c = prop[-1]
        target, c = [], last
        for i in range(k + 1):
            c = _oracle(c if i == 0 else prop[i - 1])
            target.append(c)
        acc, merged = pyoracle.spec_merge(prop, target)
        if wrong == 0:
            assert acc == k
        if wrong == 1:
            assert acc == 0
        pos += acc + 1
        last = merged[-1]
        gen.extend(merged)
    assert gen[:n] == greedy


ARGMAX = json.load(open(os.path.join(GOLDEN, "argmax_cases.json")))["cases"]


@pytest.mark.parametrize("case", ARGMAX)
def test_argmax_vectors(case):
    assert pyoracle.argmax(case["logits"]) == case["index"]


NAN, INF = float("nan"), float("inf")


@pytest.mark.parametrize("row,want", [
    ([NAN, 1.0, 2.0], 0),        # a NaN best is never replaced
    ([1.0, NAN, 2.0], 2),        # a later NaN is skipped
    ([NAN, NAN, NAN], 0),
    ([-0.0, 0.0, -0.0], 0),      # 0.0 > -0.0 is false: equal values
    ([0.0, -0.0], 0),
    ([-INF, -INF], 0),
    ([-INF, NAN, -1.0], 2),
    ([3.0, INF, INF], 1),
    ([-1.0, -INF, -0.5, NAN], 2),
])
def test_argmax_special_values(row, want):
    assert pyoracle.argmax(row) == want


def _first_max(x):
    if np.isnan(x[0]):
        return 0
    ok = ~np.isnan(x)
    m = x[ok].max()
    return int(np.flatnonzero(ok & (x == m))[0])


@pytest.mark.parametrize("seed", range(6))
def test_argmax_random_rows(seed):
    rng = np.random.default_rng(seed)
    for n in (1, 2, 7, 64, 1000, 4097):
        x = rng.integers(-4, 5, n).astype(np.float32)  # many ties
        assert pyoracle.argmax(x) == int(np.argmax(x))
        y = rng.standard_normal(n).astype(np.float32)
        y[rng.random(n) < 0.1] = np.nan
        assert pyoracle.argmax(y) == _first_max(y)
