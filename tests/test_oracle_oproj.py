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
    # every NaN half (either sign, any payload) converts to the reference's
    # std::numeric_limits<float>::quiet_NaN(), bits 0x7fc00000 (dequant.cpp:27-29)
    assert nan.sum() == 2 * 1023
    assert np.all(got[nan].view(np.uint32) == 0x7FC00000)


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


def test_f32_to_f16_against_numpy():
    rng = np.random.default_rng(5)
    mags = np.exp(rng.uniform(np.log(1e-9), np.log(7e4), 20000)).astype(np.float32)
    vals = np.concatenate([mags, -mags])
    # halfway cases between adjacent halves (ties to even), subnormal halves,
    # the overflow edge and specials
    h = np.arange(0, 0x7bff, 37, dtype=np.uint16).view(np.float16).astype(np.float64)
    h_next = (np.arange(0, 0x7bff, 37, dtype=np.uint16) + 1).view(np.float16).astype(np.float64)
    ties = ((h + h_next) / 2).astype(np.float32)
    edge = np.array([65504, 65519, 65519.996, 65520, 65536, 1e9, 2.0 ** -24, 2.0 ** -25,
                     2.0 ** -25 * 1.0000001, 2.0 ** -26, 0.0, -0.0, np.inf, -np.inf],
                    np.float32)
    allv = np.concatenate([vals, ties, edge]).astype(np.float32)
    with np.errstate(over="ignore"):  # the overflow edge rounds to infinity
        want = allv.astype(np.float16).view(np.uint16)
    got = np.array([pyoracle.f32_to_f16(float(v)) for v in allv], np.uint16)
    assert np.array_equal(got, want)
    assert pyoracle.f32_to_f16(float("nan")) & 0x7c00 == 0x7c00


def test_quantize_row_q8_0_properties():
    rng = np.random.default_rng(6)
    x = rng.standard_normal(32 * 64).astype(np.float32) * np.repeat(
        np.exp(rng.uniform(-8, 8, 64)), 32).astype(np.float32)
    x[32 * 5: 32 * 6] = 0.0  # an all-zero block: scale 0, codes 0
    q = pyoracle.quantize_row_q8_0(x).reshape(64, 34)
    d_bits = q[:, :2].copy().view(np.uint16).ravel()
    codes = q[:, 2:].view(np.int8).astype(np.int64)
    xb = x.reshape(64, 32)
    amax = np.abs(xb).max(axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    assert np.array_equal(d_bits, d.astype(np.float16).view(np.uint16))
    assert np.all(np.abs(codes) <= 127)
    nz = amax > 0
    assert np.all(np.abs(codes[nz]).max(axis=1) == 127)
    assert np.all(codes[~nz] == 0)
    err = np.abs(xb[nz].astype(np.float64) - codes[nz] * d[nz, None].astype(np.float64))
    assert np.all(err <= 0.5 * d[nz, None] * (1 + 1e-6))


def q8_blocks(codes, scales):
    """Q8_0 rows [dim][nb*34] from int8 codes [dim][nb][32] and f32 scales [dim][nb]."""
    dim, nb, _ = codes.shape
    blk = np.zeros((dim, nb, 34), np.uint8)
    blk[:, :, :2] = scales.astype(np.float16).view(np.uint8).reshape(dim, nb, 2)
    blk[:, :, 2:] = codes.astype(np.int8).view(np.uint8)
    return blk.reshape(dim, nb * 34)


@pytest.mark.parametrize("dim,n_in", [(1, 32), (9, 256), (40, 4096)])
def test_q8_0_integer_data_exact(dim, n_in):
    """Activation blocks whose max is 127 quantize to themselves (d = 1), and
    weight scales of 1 make every term an exact integer."""
    rng = np.random.default_rng(dim + n_in)
    nb = n_in // 32
    a = rng.integers(-127, 128, n_in)
    a[::32] = 127
    codes = rng.integers(-8, 9, (dim, nb, 32))  # |sum| <= 256 * 32 * 8 * 127 < 2^24
    w = q8_blocks(codes, np.ones((dim, nb), np.float32))
    x = rng.integers(-100, 101, dim).astype(np.float32)
    want = (codes.reshape(dim, n_in) @ a + x.astype(np.int64)).astype(np.float32)
    got = pyoracle.oproj_residual(w, a.astype(np.float32), x, q8_0=True)
    assert np.array_equal(got, want)
