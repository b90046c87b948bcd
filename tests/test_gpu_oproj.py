"""Output projection + residual add on the device (`dbi_oproj_residual_async`,
model.cpp:773-774) against the oracle (`ok_oproj_residual`: tensor::matvec /
matvec_f16 sequential sums, then x += proj).

Tolerance: the device sums a row's products in a tree, the reference in
sequence, so the two agree to the rounding of a dot product:
    |a - b| <= 1e-5 + 1e-4 |b| + 2 * n * 2^-24 * sum_i |w_i x_i|
(each order is within n * 2^-24 * sum|w_i x_i| of the exact value). On
small-integer data every partial sum is exact, so there the results must be
bit-identical. Q8_0 (matvec_q8_0_scalar after quantize_row_q8_0): the same
bound over the block terms, sum_b |dw_b * dx_b * sumi_b|; with unit scales
and activation blocks that quantize to themselves, bit-identical.
"""
import numpy as np
import pytest

import pyoracle
from dbinfer_amd.kv import W_F16, W_F32, W_Q4_0, W_Q8_0, DbiError, HipKV
from test_oracle_layer import q4_blocks
from test_oracle_oproj import q8_blocks

pytestmark = pytest.mark.gpu

SHAPES = [(2048, 2048), (3072, 3072), (3584, 3584), (4096, 4096),  # C1/C2, C3, C4, C5
          (5, 8), (70, 520), (1, 4096), (300, 14336)]


@pytest.fixture(scope="module")
def torch():
    return pytest.importorskip("torch")


@pytest.fixture(scope="module")
def kv():
    h = HipKV(1, 64, 1, 64)
    yield h
    h.close()


def run(torch, kv, w, a, x):
    wt = torch.from_numpy(np.ascontiguousarray(w).view(np.uint16) if w.dtype == np.float16
                          else np.ascontiguousarray(w)).cuda()
    at = torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    xt = torch.from_numpy(np.array(x, np.float32)).cuda()
    kv.set_stream(torch.cuda.current_stream().cuda_stream)
    kv.oproj_residual_async(W_F16 if w.dtype == np.float16 else W_F32, wt.data_ptr(),
                            at.data_ptr(), xt.data_ptr(), w.shape[0], w.shape[1])
    torch.cuda.synchronize()
    return xt.cpu().numpy()


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("dim,n_in", SHAPES)
def test_integer_data_bit_exact(torch, kv, f16, dim, n_in):
    rng = np.random.default_rng(dim + n_in)
    w = rng.integers(-8, 9, (dim, n_in)).astype(np.float16 if f16 else np.float32)
    a = rng.integers(-8, 9, n_in).astype(np.float32)
    x = rng.integers(-100, 101, dim).astype(np.float32)
    got = run(torch, kv, w, a, x)
    want = pyoracle.oproj_residual(w, a, x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("dim,n_in", SHAPES)
def test_random_data_within_dot_tolerance(torch, kv, f16, dim, n_in):
    rng = np.random.default_rng(3 * dim + n_in)
    w = (rng.standard_normal((dim, n_in)) * 0.05).astype(np.float16 if f16 else np.float32)
    a = rng.standard_normal(n_in).astype(np.float32)
    x = rng.standard_normal(dim).astype(np.float32)
    got = run(torch, kv, w, a, x).astype(np.float64)
    want = pyoracle.oproj_residual(w, a, x).astype(np.float64)
    mag = np.abs(w.astype(np.float64)) @ np.abs(a.astype(np.float64))
    bound = 1e-5 + 1e-4 * np.abs(want) + 2 * n_in * 2.0 ** -24 * mag
    err = np.abs(got - want)
    assert np.all(err <= bound), f"worst {float((err - bound).max()):.3e}"


def test_oproj_errors(torch, kv):
    w = torch.zeros(64, 64, device="cuda")
    a = torch.zeros(64, device="cuda")
    x = torch.zeros(64, device="cuda")
    for args, msg in [((W_F32, w.data_ptr(), a.data_ptr(), x.data_ptr(), 64, 60), "multiple of 8"),
                      ((W_F32, w.data_ptr(), a.data_ptr(), x.data_ptr(), 0, 64), "dim"),
                      ((6, w.data_ptr(), a.data_ptr(), x.data_ptr(), 64, 64), "fp32, f16"),
                      ((W_F32, w.data_ptr() + 4, a.data_ptr(), x.data_ptr(), 8, 56), "aligned"),
                      ((W_F32, 0, a.data_ptr(), x.data_ptr(), 64, 64), "null")]:
        with pytest.raises(DbiError) as e:
            kv.oproj_residual_async(*args)
        assert msg in e.value.message


def test_oproj_graph_replay(torch):
    """Captured once; each replay reads the attention row written since and
    accumulates into the residual, checked against the oracle every time."""
    dim, n_in = 3072, 3072
    rng = np.random.default_rng(11)
    w = rng.integers(-4, 5, (dim, n_in)).astype(np.float32)
    kv = HipKV(1, 64, 1, 64)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        wt = torch.from_numpy(w).cuda()
        at = torch.zeros(n_in, device="cuda")
        xt = torch.zeros(dim, device="cuda")
        kv.set_stream(s.cuda_stream)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            kv.oproj_residual_async(W_F32, wt.data_ptr(), at.data_ptr(), xt.data_ptr(), dim, n_in)
    torch.cuda.synchronize()
    x = np.zeros(dim, np.float32)
    for rep in range(4):
        a = rng.integers(-4, 5, n_in).astype(np.float32)
        at.copy_(torch.from_numpy(a))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        x = pyoracle.oproj_residual(w, a, x)
        assert np.array_equal(xt.cpu().numpy(), x), f"replay {rep}"
        _ = (at * 2).sum()
    kv.close()


def run_q8(torch, kv, w, a, x, dim, n_in, wtype=W_Q8_0):
    wt = torch.from_numpy(np.ascontiguousarray(w)).cuda()
    at = torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    xt = torch.from_numpy(np.array(x, np.float32)).cuda()
    kv.set_stream(torch.cuda.current_stream().cuda_stream)
    kv.oproj_residual_async(wtype, wt.data_ptr(), at.data_ptr(), xt.data_ptr(), dim, n_in)
    torch.cuda.synchronize()
    return xt.cpu().numpy()


# (70, 8192), (64, 18944) (Qwen2.5-7B's ff) and (2, 32768) below: rows longer
# than one workgroup holds, streamed through the prologue
Q8_SHAPES = [(2048, 2048), (3072, 3072), (3584, 3584), (4096, 4096), (5, 32), (70, 8192),
             (64, 18944), (3, 96)]


@pytest.mark.parametrize("dim,n_in", Q8_SHAPES)
def test_q8_0_integer_data_bit_exact(torch, kv, dim, n_in):
    rng = np.random.default_rng(dim * 7 + n_in)
    nb = n_in // 32
    a = rng.integers(-127, 128, n_in)
    a[::32] = -127  # every activation block's max is 127: d = 1, codes = values
    codes = rng.integers(-8, 9, (dim, nb, 32))  # |sum| <= 256 * 32 * 8 * 127 < 2^24
    w = q8_blocks(codes, np.ones((dim, nb), np.float32))
    x = rng.integers(-100, 101, dim).astype(np.float32)
    got = run_q8(torch, kv, w, a.astype(np.float32), x, dim, n_in)
    want = pyoracle.oproj_residual(w, a.astype(np.float32), x, q8_0=True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("dim,n_in", Q8_SHAPES + [(2, 32768)])  # the largest LDS stage
def test_q8_0_random_within_dot_tolerance(torch, kv, dim, n_in):
    rng = np.random.default_rng(dim * 11 + n_in)
    nb = n_in // 32
    a = rng.standard_normal(n_in).astype(np.float32)
    a[7] = 0.0
    codes = rng.integers(-127, 128, (dim, nb, 32))
    scales = np.exp(rng.uniform(-9, -4, (dim, nb))).astype(np.float32)
    w = q8_blocks(codes, scales)
    x = rng.standard_normal(dim).astype(np.float32)
    got = run_q8(torch, kv, w, a, x, dim, n_in).astype(np.float64)
    want = pyoracle.oproj_residual(w, a, x, q8_0=True).astype(np.float64)
    aq = pyoracle.quantize_row_q8_0(a).reshape(nb, 34)
    dx = aq[:, :2].copy().view(np.float16).astype(np.float64).ravel()
    xc = aq[:, 2:].view(np.int8).astype(np.int64)
    dw = scales.astype(np.float16).astype(np.float64)
    sumi = np.einsum("dbi,bi->db", codes, xc)
    mag = np.abs(dw * dx[None, :] * sumi).sum(axis=1)
    bound = 1e-5 + 1e-4 * np.abs(want) + 2 * nb * 2.0 ** -24 * mag
    err = np.abs(got - want)
    assert np.all(err <= bound), f"worst {float((err - bound).max()):.3e}"


def test_q8_0_errors(torch, kv):
    w = torch.zeros(64 * 34, dtype=torch.uint8, device="cuda")
    a = torch.zeros(64, device="cuda")
    x = torch.zeros(64, device="cuda")
    with pytest.raises(DbiError) as e:
        kv.oproj_residual_async(W_Q8_0, w.data_ptr(), a.data_ptr(), x.data_ptr(), 2, 48)
    assert "multiple of 32" in e.value.message
    with pytest.raises(DbiError) as e:
        kv.oproj_residual_async(W_Q8_0, w.data_ptr() + 2, a.data_ptr(), x.data_ptr(), 2, 32)
    assert "aligned" in e.value.message
    with pytest.raises(DbiError) as e:  # Q5_0 (GgmlType 6) is not served
        kv.oproj_residual_async(6, w.data_ptr(), a.data_ptr(), x.data_ptr(), 2, 32)
    assert "Q4_0 weights only" in e.value.message
    with pytest.raises(DbiError) as e:  # the quantized row must fit the LDS stage
        kv.oproj_residual_async(W_Q8_0, w.data_ptr(), a.data_ptr(), x.data_ptr(), 1, 32800)
    assert "at most 32768" in e.value.message


# ---- Q4_0 (matvec_q4_0_scalar, matmul.cpp:77-99): 18-byte blocks; the block
# sum is an exact integer, so the same dot-product bound holds


@pytest.mark.parametrize("dim,n_in", Q8_SHAPES)
def test_q4_0_integer_data_bit_exact(torch, kv, dim, n_in):
    rng = np.random.default_rng(dim * 13 + n_in)
    nb = n_in // 32
    a = rng.integers(-127, 128, n_in)
    a[::32] = 127  # d = 1: the activation codes are its values
    vals = rng.integers(-8, 8, (dim, nb, 32))
    w = q4_blocks(vals, np.ones((dim, nb), np.float32))
    x = rng.integers(-100, 101, dim).astype(np.float32)
    got = run_q8(torch, kv, w, a.astype(np.float32), x, dim, n_in, W_Q4_0)
    want = (vals.reshape(dim, n_in) @ a + x.astype(np.int64)).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("dim,n_in", Q8_SHAPES + [(2, 32768)])
def test_q4_0_random_within_dot_tolerance(torch, kv, dim, n_in):
    rng = np.random.default_rng(dim * 17 + n_in)
    nb = n_in // 32
    a = rng.standard_normal(n_in).astype(np.float32)
    vals = rng.integers(-8, 8, (dim, nb, 32))
    scales = np.exp(rng.uniform(-7, -2, (dim, nb))).astype(np.float32)
    w = q4_blocks(vals, scales)
    x = rng.standard_normal(dim).astype(np.float32)
    got = run_q8(torch, kv, w, a, x, dim, n_in, W_Q4_0).astype(np.float64)
    want = (x + pyoracle.matvec(w, W_Q4_0, a, dim)).astype(np.float64)
    aq = pyoracle.quantize_row_q8_0(a).reshape(nb, 34)
    dx = aq[:, :2].copy().view(np.float16).astype(np.float64).ravel()
    xc = aq[:, 2:].view(np.int8).astype(np.int64)
    dw = scales.astype(np.float16).astype(np.float64)
    sumi = np.einsum("dbi,bi->db", vals, xc)
    mag = np.abs(dw * dx[None, :] * sumi).sum(axis=1)
    bound = 1e-5 + 1e-4 * np.abs(want) + 2 * nb * 2.0 ** -24 * mag
    err = np.abs(got - want)
    assert np.all(err <= bound), f"worst {float((err - bound).max()):.3e}"
