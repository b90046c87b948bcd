"""Pins the oracle's output projection + residual add (model.cpp:773-774 with
tensor::matvec / matvec_f16, matmul.cpp:36-54) and its half conversion
(dequant.cpp:14).

- ok_f16_to_f32: every one of the 65536 half values against numpy's
  float16 -> float32 conversion (a library routine), NaNs by class.
- ok_oproj_residual on small-integer data: every product and partial sum is an
  integer below 2^24, so fp32 arithmetic in any order is exact and equals the
  integer matrix product (numpy int64) plus the residual.
- on N(0,1) data: within the sequential-sum rounding bound of the fp64 dot
  product, |err| <= n * 2^-24 * sum|w_i x_i| + ulp of the residual add.
A planted mistake (a dropped term, a transposed weight, the residual skipped)
fails the integer test exactly.
"""
import numpy as np
import pytest

import pyoracle


def test_f16_all_values():
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([pyoracle.f16_to_f32(int(v)) for v in h], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("dim,n_in", [(1, 8), (7, 64), (64, 256), (33, 1024)])
def test_integer_data_exact(f16, dim, n_in):
    rng = np.random.default_rng(dim * 1000 + n_in)
    w = rng.integers(-8, 9, (dim, n_in))
    a = rng.integers(-8, 9, n_in)
    x = rng.integers(-100, 101, dim).astype(np.float32)
    want = (w.astype(np.int64) @ a.astype(np.int64) + x.astype(np.int64)).astype(np.float32)
    wt = w.astype(np.float16) if f16 else w.astype(np.float32)
    got = pyoracle.oproj_residual(wt, a.astype(np.float32), x)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("f16", [False, True])
def test_random_within_dot_bound(f16):
    rng = np.random.default_rng(7)
    dim, n_in = 96, 4096
    w = rng.standard_normal((dim, n_in)).astype(np.float16 if f16 else np.float32)
    a = rng.standard_normal(n_in).astype(np.float32)
    x = rng.standard_normal(dim).astype(np.float32)
    wf = w.astype(np.float64)
    exact = wf @ a.astype(np.float64) + x
    got = pyoracle.oproj_residual(w, a, x).astype(np.float64)
    bound = n_in * 2.0 ** -24 * (np.abs(wf) @ np.abs(a)) + 2.0 ** -23 * np.abs(exact)
    assert np.all(np.abs(got - exact) <= bound)
