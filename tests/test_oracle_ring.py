"""Pins the oracle's ring mapping: slot_for and residents (model.cpp:321-324,
406-418).

Restates tests/kv_ring_test.cpp (payload = token index so the stored value
names the token owning a slot; the 8-case matrix of :90-97, committed as
tests/golden/kv_ring_cases.json) and adds a brute-force check against an
explicit simulation of the StreamingLLM ring (sinks + deque of the most recent
`window` tokens).
"""
import json
import os
from collections import deque

import numpy as np
import pytest

import pyoracle
from helpers import GOLDEN

CASES = json.load(open(os.path.join(GOLDEN, "kv_ring_cases.json")))["cases"]


def fill(n_sink, window, n_seen):
    kv = pyoracle.OracleKV(1, 0, 1, 1, n_sink=n_sink, window=window, dtype=pyoracle.F32)
    for t in range(n_seen):
        kv.append(0, t, np.array([t], np.float32), np.array([t], np.float32))
    return kv


@pytest.mark.parametrize("n_sink,window,n_seen", CASES)
def test_kv_ring_case(n_sink, window, n_seen):
    kv = fill(n_sink, window, n_seen)
    for t in range(n_seen):
        want = t if t < n_sink else n_sink + (t - n_sink) % window
        assert kv.slot_for(t) == want
    slots, rp = kv.residents()
    keys = kv.export("k", 0)
    sinks = min(n_seen, n_sink)
    ws = n_sink
    if n_seen > n_sink and n_seen - n_sink > window:
        ws = n_seen - window
    wlen = n_seen - ws if n_seen > n_sink else 0
    assert len(slots) == sinks + wlen
    for r in range(sinks):  # sinks never evicted
        assert slots[r] == r and rp[r] == r and keys[slots[r]] == r
    for r in range(sinks, len(slots)):  # window holds the most recent tokens
        t = ws + (r - sinks)
        assert keys[slots[r]] == t
        assert rp[r] == n_sink + (t - ws)
    assert list(rp) == list(range(len(slots)))  # rope positions pack to [0, n_res)
    assert len(set(slots.tolist())) == len(slots)  # distinct slots


@pytest.mark.parametrize("n_sink,window", [(4, 8), (0, 5), (1, 4), (3, 1), (7, 16)])
def test_ring_brute_force(n_sink, window):
    """Explicit sinks + deque simulation gives the same resident tokens in the
    same order as the oracle's closed form, at every step."""
    kv = pyoracle.OracleKV(1, 0, 1, 1, n_sink=n_sink, window=window, dtype=pyoracle.F32)
    sinks, win = [], deque(maxlen=window)
    for t in range(3 * (n_sink + window) + 5):
        kv.append(0, t, np.array([t], np.float32), np.array([t], np.float32))
        if len(sinks) < n_sink:
            sinks.append(t)
        else:
            win.append(t)
        slots, rp = kv.residents()
        keys = kv.export("k", 0)
        assert [int(keys[s]) for s in slots] == sinks + list(win)
        assert list(rp) == list(range(len(sinks) + len(win)))


def test_ring_rollback_is_n_seen_only():
    kv = fill(4, 8, 30)
    kv.truncate(20)  # speculative rollback: n_seen moves, storage is not scrubbed
    slots, rp = kv.residents()
    keys = kv.export("k", 0)
    # resident slots are those of tokens 12..19, their bytes still hold the
    # last token written there (20..29): the ring cannot restore evicted rows
    assert list(slots[4:]) == [kv.slot_for(t) for t in range(12, 20)]
    last_writer = {kv.slot_for(t): t for t in range(30)}
    assert [int(keys[s]) for s in slots] == [last_writer[int(s)] for s in slots]
    assert list(rp) == list(range(12))
    kv.append(0, 20, np.array([1000.0], np.float32), np.array([1000.0], np.float32))
    assert kv.n_seen == 21
    assert int(kv.export("k", 0)[kv.slot_for(20)]) == 1000
