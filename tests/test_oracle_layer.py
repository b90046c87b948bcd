"""Pins the oracle's pieces of the full decode layer (model.cpp:730-787):

- ok_rmsnorm, ok_silu: bit for bit against the reference's own ops.cpp
  (ops.cpp:7-17, 54-56) compiled in oracle/_ref.
- ok_matvec: fp32 / f16 exact on small-integer data (every partial sum is an
  integer below 2^24); Q8_0 and Q4_0 against an integer restatement written
  from the GGUF block layouts (Q8_0: f16 scale + 32 int8 codes; Q4_0: f16
  scale + 16 bytes, element j the low nibble of byte j and element j + 16
  its high nibble, value - 8) and matvec_q{8,4}_0_scalar's term
  (f16(dw) * f16(dx)) * sumi (matmul.cpp:56-99), summed in sequence. A
  restatement with the nibbles swapped must disagree (the check can fail).
- okv_decode_layer: the layer's wiring (which norm, which buffers, the
  residual adds, dense rope + append vs the ring's attention) against the
  same sequence composed here from the pinned functions, bit for bit, for
  dense fp32, dense int8 and ring caches.
"""
import numpy as np
import pytest

import pyoracle
from pyoracle import W_F16, W_F32, W_Q4_0, W_Q8_0
from helpers import normal


def _ref_or_skip():
    ref = pyoracle.load_ref()
    if ref is None or not hasattr(ref, "ref_rmsnorm"):
        pytest.skip("reference ops.cpp build (oracle/_ref) not present")
    return ref


@pytest.mark.parametrize("dim,eps", [(1, 1e-5), (64, 1e-6), (3584, 1e-6), (4096, 1e-5), (777, 0.0)])
def test_rmsnorm_bitwise_equals_reference_build(dim, eps):
    ref = _ref_or_skip()
    x = normal(dim, dim) * 3.0
    w = normal(dim + 1, dim)
    want = np.zeros(dim, np.float32)
    ref.ref_rmsnorm(x.ctypes.data, w.ctypes.data, eps, want.ctypes.data, 1, dim)
    got = pyoracle.rmsnorm(x, w, eps)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_silu_bitwise_equals_reference_build():
    ref = _ref_or_skip()
    x = np.concatenate([normal(5, 4096) * 6.0,
                        np.array([0.0, -0.0, 88.0, -88.0, 1e-30, -1e-30, 20.0, -104.0],
                                 np.float32)])
    want = np.zeros_like(x)
    ref.ref_silu(x.ctypes.data, want.ctypes.data, x.size)
    assert np.array_equal(pyoracle.silu(x).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("wt", [W_F32, W_F16])
@pytest.mark.parametrize("out,n_in", [(1, 8), (33, 256), (64, 4096)])
def test_matvec_float_types_exact_on_integers(wt, out, n_in):
    rng = np.random.default_rng(out + n_in)
    w = rng.integers(-8, 9, (out, n_in)).astype(np.float16 if wt == W_F16 else np.float32)
    x = rng.integers(-8, 9, n_in).astype(np.float32)
    want = (w.astype(np.int64) @ x.astype(np.int64)).astype(np.float32)
    got = pyoracle.matvec(w.view(np.uint16) if wt == W_F16 else w, wt, x, out)
    assert np.array_equal(got, want)


def q4_blocks(vals, scales):
    """Q4_0 rows [out][nb*18] from values in [-8, 7] [out][nb][32] and f32
    scales [out][nb]: element j the low nibble of byte j, j + 16 the high."""
    out, nb, _ = vals.shape
    blk = np.zeros((out, nb, 18), np.uint8)
    blk[:, :, :2] = scales.astype(np.float16).view(np.uint8).reshape(out, nb, 2)
    n = (vals + 8).astype(np.uint8)
    blk[:, :, 2:] = n[:, :, :16] | (n[:, :, 16:] << 4)
    return blk.reshape(out, nb * 18)


def q8_blocks(codes, scales):
    out, nb, _ = codes.shape
    blk = np.zeros((out, nb, 34), np.uint8)
    blk[:, :, :2] = scales.astype(np.float16).view(np.uint8).reshape(out, nb, 2)
    blk[:, :, 2:] = codes.astype(np.int8).view(np.uint8)
    return blk.reshape(out, nb * 34)


def restated(vals, scales, x, swap=False):
    """sum_b (f16(dw) * f16(dx)) * sumi in sequence, from the activation's
    Q8_0 blocks (ok_quantize_row_q8_0, pinned in test_oracle_oproj)."""
    out, nb, _ = vals.shape
    xq = pyoracle.quantize_row_q8_0(x).reshape(nb, 34)
    dx = xq[:, :2].copy().view(np.float16).astype(np.float32).reshape(nb)
    cx = xq[:, 2:].view(np.int8).astype(np.int64)
    if swap:
        cx = np.concatenate([cx[:, 16:], cx[:, :16]], axis=1)
    dw = scales.astype(np.float16).astype(np.float32)
    y = np.zeros(out, np.float32)
    for o in range(out):
        acc = np.float32(0.0)
        for b in range(nb):
            sumi = int(vals[o, b].astype(np.int64) @ cx[b])
            acc = np.float32(acc + np.float32(np.float32(dw[o, b] * dx[b]) * np.float32(sumi)))
        y[o] = acc
    return y


@pytest.mark.parametrize("wt", [W_Q8_0, W_Q4_0])
@pytest.mark.parametrize("out,n_in", [(1, 32), (9, 256), (20, 1024)])
def test_matvec_quantized_against_integer_restatement(wt, out, n_in):
    rng = np.random.default_rng(7 * out + n_in + wt)
    nb = n_in // 32
    lo, hi = (-8, 8) if wt == W_Q4_0 else (-127, 128)
    vals = rng.integers(lo, hi, (out, nb, 32))
    scales = rng.uniform(0.001, 0.05, (out, nb)).astype(np.float32)
    w = q4_blocks(vals, scales) if wt == W_Q4_0 else q8_blocks(vals, scales)
    x = normal(out + n_in, n_in)
    got = pyoracle.matvec(w, wt, x, out)
    assert np.array_equal(got, restated(vals, scales, x))
    if wt == W_Q4_0:  # the nibble order matters to the check
        assert not np.array_equal(got, restated(vals, scales, x, swap=True))


def layer_weights(rng, dim, ff, nh, nkv, hd, wt, bias):
    """One block's weights; wt is one type for all seven matrices or a list of
    seven (wq wk wv wo wgate wup wdown)."""
    wts = list(wt) if isinstance(wt, (list, tuple)) else [wt] * 7
    it = iter(wts)

    def mat(o, i):
        wt = next(it)
        if wt in (W_F32, W_F16):
            m = (rng.standard_normal((o, i)) * 0.05).astype(np.float32)
            return m.astype(np.float16).view(np.uint16) if wt == W_F16 else m
        # weights of about the float ones' spread (std ~0.05, a matvec gain
        # below 1 at these sizes): uniform codes have std 73 (Q8_0) or 4.6
        # (Q4_0) times the block scale
        nb = i // 32
        lo, hi = (-8, 8) if wt == W_Q4_0 else (-127, 128)
        vals = rng.integers(lo, hi, (o, nb, 32))
        sc = (rng.uniform(0.0003, 0.001, (o, nb)) if wt == W_Q8_0
              else rng.uniform(0.005, 0.016, (o, nb))).astype(np.float32)
        return q4_blocks(vals, sc) if wt == W_Q4_0 else q8_blocks(vals, sc)
    qn, kvn = nh * hd, nkv * hd
    return {
        "attn_norm": (1.0 + 0.1 * rng.standard_normal(dim)).astype(np.float32),
        "ffn_norm": (1.0 + 0.1 * rng.standard_normal(dim)).astype(np.float32),
        "w": [mat(qn, dim), mat(kvn, dim), mat(kvn, dim), mat(dim, qn), mat(ff, dim),
              mat(ff, dim), mat(dim, ff)],
        "wtype": wts,
        "bq": (0.1 * rng.standard_normal(qn)).astype(np.float32) if bias else None,
        "bk": (0.1 * rng.standard_normal(kvn)).astype(np.float32) if bias else None,
        "bv": (0.1 * rng.standard_normal(kvn)).astype(np.float32) if bias else None,
    }


def composed_layer(kv, layer, x, pos, lw, dim, ff, nh, eps):
    """model.cpp:730-787 from the pinned pieces (numpy float32 for the adds)."""
    hd, nkv = kv.head_dim, kv.n_kv_heads
    w, wt = lw["w"], lw["wtype"]
    normed = pyoracle.rmsnorm(x, lw["attn_norm"], eps)
    q = pyoracle.matvec(w[0], wt[0], normed, nh * hd)
    k = pyoracle.matvec(w[1], wt[1], normed, nkv * hd)
    v = pyoracle.matvec(w[2], wt[2], normed, nkv * hd)
    if lw["bq"] is not None:
        q, k, v = q + lw["bq"], k + lw["bk"], v + lw["bv"]
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    if kv.window == 0:
        q = pyoracle.rope(q, [pos], kv.rope_theta, nh, 1, hd)
        k = pyoracle.rope(k, [pos], kv.rope_theta, nkv, 1, hd)
        kv.append(layer, pos, k, v)
        attn = kv.attend(layer, pos, q, nh, scale)
    else:
        attn = kv.attend_ring(layer, pos, q, k, v, nh, scale)
    x = x + pyoracle.matvec(w[3], wt[3], attn, dim)
    normed = pyoracle.rmsnorm(x, lw["ffn_norm"], eps)
    g = pyoracle.matvec(w[4], wt[4], normed, ff)
    u = pyoracle.matvec(w[5], wt[5], normed, ff)
    h = pyoracle.silu(g) * u
    return x + pyoracle.matvec(w[6], wt[6], h, dim)


@pytest.mark.parametrize("layout", ["f32", "int8", "ring"])
@pytest.mark.parametrize("wt,bias", [(W_F32, True), (W_F16, False), (W_Q8_0, True),
                                     (W_Q4_0, False)])
def test_decode_layer_wiring(layout, wt, bias):
    dim, ff, nh, nkv, hd, eps, L = 128, 256, 4, 2, 32, 1e-5, 2
    rng = np.random.default_rng(11 + wt)
    lws = [layer_weights(rng, dim, ff, nh, nkv, hd, wt, bias) for _ in range(L)]
    args = dict(n_sink=2 if layout != "f32" else 0, window=6 if layout == "ring" else 0,
                dtype=pyoracle.INT8 if layout == "int8" else pyoracle.F32, rope_theta=1e4)
    a = pyoracle.OracleKV(L, 16, nkv, hd, **args)
    b = pyoracle.OracleKV(L, 16, nkv, hd, **args)
    for pos in range(10):
        x = normal(100 + pos, dim)
        xa, xb = x.copy(), x.copy()
        for layer in range(L):
            xa = a.decode_layer(layer, xa, pos, lws[layer], dim, ff, nh, eps)
            xb = composed_layer(b, layer, xb, pos, lws[layer], dim, ff, nh, eps)
        assert np.array_equal(xa.view(np.uint32), xb.view(np.uint32)), f"pos {pos}"
        for kv in (a, b):
            kv.mark_position(pos)


@pytest.mark.parametrize("wt", [W_F32, W_F16, W_Q8_0, W_Q4_0])
def test_logits_tail_wiring(wt):
    """ok_logits (Model::forward's tail, model.cpp:914-915) is rmsnorm with
    output_norm, then the lm_head matvec: bit for bit the composition of the
    two pinned functions (rmsnorm against the reference build, the matvec
    against its integer restatement). A tail that skipped the norm, or
    normed with unit weights, gives other bits (the check can fail)."""
    dim, vocab, eps = 256, 300, 1e-5
    rng = np.random.default_rng(23 + wt)
    lm = layer_weights(rng, dim, vocab, 4, 2, 32, wt, False)["w"][4]  # [vocab][dim]
    onorm = (1.0 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    for seed in range(3):
        x = normal(700 + seed, dim) * 2.0
        got = pyoracle.logits(x, onorm, lm, wt, eps, vocab)
        want = pyoracle.matvec(lm, wt, pyoracle.rmsnorm(x, onorm, eps), vocab)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"seed {seed}"
        unnormed = pyoracle.matvec(lm, wt, x, vocab)
        unit = pyoracle.matvec(lm, wt, pyoracle.rmsnorm(x, np.ones(dim, np.float32), eps), vocab)
        assert not np.array_equal(got, unnormed) and not np.array_equal(got, unit)
