"""Pins the oracle's rope and softmax (ops.cpp:19-52).

- against the reference's golden vectors (tests/ops_test.cpp:31-53: theta 1e6,
  head_dim 64, positions 0-5, atol 1e-5);
- bit for bit against the reference's own ops.cpp compiled in oracle/_ref
  (when that build exists in this container);
- against closed forms: rope at position 0 is the identity, rope is a
  rotation (pair norms kept), rope(p) of rope(-p) undoes it; softmax sums to 1
  and is shift-invariant.
"""
import numpy as np
import pytest

import pyoracle
from helpers import load_golden, normal, rope64

POS6 = np.arange(6, dtype=np.int32)


@pytest.mark.parametrize("name,heads", [("rope_q", 14), ("rope_k", 2)])
def test_rope_matches_golden(name, heads):
    x = load_golden(f"{name}_in")
    want = load_golden(f"{name}_out")
    got = pyoracle.rope(x, POS6, 1e6, heads, 6, 64).reshape(want.shape)
    assert np.max(np.abs(got - want)) <= 1e-5


def test_softmax_matches_golden():
    x = load_golden("softmax_in")
    want = load_golden("softmax_out")
    got = np.stack([pyoracle.softmax(r) for r in x])
    assert np.max(np.abs(got - want)) <= 1e-5


def _ref_or_skip():
    ref = pyoracle.load_ref()
    if ref is None:
        pytest.skip("reference ops.cpp build (oracle/_ref) not present")
    return ref


@pytest.mark.parametrize("theta,hd,heads,positions", [
    (1e6, 64, 14, [0, 1, 2, 3, 4, 5]),
    (5e5, 64, 4, [0, 17, 511, 2047]),
    (1e4, 128, 3, [1, 1024, 4095, 32767]),
    (1e6, 128, 2, [4099, 16383]),
])
def test_rope_bitwise_equals_reference_build(theta, hd, heads, positions):
    ref = _ref_or_skip()
    seq = len(positions)
    x = normal(11, heads, seq, hd)
    p = np.array(positions, np.int32)
    want = x.copy()
    ref.ref_rope(want.ctypes.data, p.ctypes.data, theta, heads, seq, hd)
    got = pyoracle.rope(x, p, theta, heads, seq, hd).reshape(x.shape)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("n", [1, 7, 512, 4100])
def test_softmax_bitwise_equals_reference_build(n):
    ref = _ref_or_skip()
    x = normal(5, n) * 4
    want = np.empty_like(x)
    ref.ref_softmax(x.ctypes.data, want.ctypes.data, n)
    assert np.array_equal(pyoracle.softmax(x).view(np.uint32), want.view(np.uint32))


def test_rope_closed_forms():
    hd, theta = 128, 1e6
    x = normal(3, 1, 1, hd)
    # position 0: cos 1, sin 0 -> identity
    assert np.array_equal(pyoracle.rope(x, [0], theta, 1, 1, hd).ravel(), x.ravel())
    # rotation keeps each (j, j + hd/2) pair's norm
    y = pyoracle.rope(x, [777], theta, 1, 1, hd).ravel()
    h = hd // 2
    n0 = np.hypot(x.ravel()[:h], x.ravel()[h:])
    n1 = np.hypot(y[:h], y[h:])
    assert np.allclose(n0, n1, rtol=1e-6, atol=1e-7)
    # matches an independent float64 rotation, and -p undoes +p
    assert np.allclose(y, rope64(x.ravel(), 777, theta), rtol=0, atol=2e-6)
    back = pyoracle.rope(y, [-777], theta, 1, 1, hd).ravel()
    assert np.allclose(back, x.ravel(), atol=2e-6)
    # a transposed pairing (adjacent pairs) would not match the float64 NeoX form
    assert not np.allclose(y[:2], rope64(x.ravel()[:2], 777, theta), atol=1e-3)


def test_softmax_closed_forms():
    x = normal(9, 300) * 3
    s = pyoracle.softmax(x)
    assert abs(float(s.astype(np.float64).sum()) - 1.0) < 1e-5
    assert np.allclose(s, pyoracle.softmax(x + np.float32(50)), rtol=1e-5, atol=1e-8)
    assert int(np.argmax(s)) == int(np.argmax(x))
    one = pyoracle.softmax(np.array([3.5], np.float32))
    assert one[0] == 1.0
