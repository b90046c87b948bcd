"""GPU parity of the on-device q/k/v producer (dbi_kv_decode_qkv,
dbi_kv_chunk_qkv): bias + rope on the device, then append + attention.

The oracle side is the reference's host sequence restated with the oracle's
pinned pieces: fp32 bias adds (model.cpp:747-755, 939-947), tensor::rope at
the row's position (ops.cpp:19-38; oracle ok_rope, pinned by the reference's
rope goldens), KVCache::append, then the attention of the layout.

Bars:
- the stored cache (fp32 K/V, int8 codes, scales, raw staging, sinks) is
  bit-identical to the oracle's after the same steps: the device rope
  reproduces the reference's fp64 rope bit for bit;
- the attention output equals, bit for bit, the plain fused step
  (dbi_kv_decode) fed the oracle's roped rows, and is within
  |a - b| <= 1e-5 + 1e-4 |b| of the oracle's attention.
"""
import numpy as np
import pytest

import pyoracle
from dbinfer_amd.kv import F32, INT8, DbiError, HipKV
from helpers import assert_close, normal

pytestmark = pytest.mark.gpu


def scale_of(hd):
    return np.float32(1.0) / np.sqrt(np.float32(hd))


def same_bits(a, b, what):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    if a.dtype == np.float32:
        a, b = a.view(np.uint32), b.view(np.uint32)
    diff = np.nonzero(a != b)[0]
    assert diff.size == 0, f"{what}: {diff.size} differing elements, first at {diff[:5]}"


def store_names(dtype, window, n_sink):
    if dtype == F32:
        return ["k", "v"]
    names = ["k8", "v8", "k_scale", "v_scale"]
    if not window:
        names += ["k_raw"] + (["k_sink", "v_sink"] if n_sink else [])
    return names


def host_produce(q, k, v, qb, kb, vb, pos, nh, nkv, hd, theta, ring):
    """The reference's host sequence between the projections and the cache."""
    q = q + qb if qb is not None else q.copy()
    k = k + kb if kb is not None else k.copy()
    v = v + vb if vb is not None else v.copy()
    if not ring:
        q = pyoracle.rope(q, [pos], theta, nh, 1, hd)
        k = pyoracle.rope(k, [pos], theta, nkv, 1, hd)
    return q, k, v


DECODE_CASES = [
    # dtype, nh, nkv, hd, n_sink, window, theta, steps, bias
    (F32, 32, 8, 128, 0, 0, 1e6, 40, True),     # config 5 shape, Qwen-style biases
    (INT8, 24, 8, 128, 4, 0, 5e5, 70, True),    # config 3 shape: sinks, then groups
    (INT8, 32, 8, 64, 0, 0, 5e5, 40, False),    # no biases (Llama)
    (F32, 32, 4, 64, 0, 0, 1e4, 33, False),     # config 1 shape
    (F32, 28, 4, 128, 4, 24, 1e6, 60, True),    # config 4 ring: biases only, keys stay un-roped
    (INT8, 28, 4, 128, 4, 24, 1e6, 60, True),
    # dense int8, q produced once per workgroup: G = 8 (one rope pair per
    # thread of all 512) and hd 64 with G = 5, both with the steps' own sink
    # rows produced in LDS
    (INT8, 32, 4, 128, 4, 0, 1e6, 40, True),
    (INT8, 40, 8, 64, 4, 0, 1e4, 36, True),
    (INT8, 24, 8, 128, 4, 0, 5e5, 12, False),   # rope only: no bias add on the sink rows
]


@pytest.mark.parametrize("dtype,nh,nkv,hd,n_sink,window,theta,steps,bias", DECODE_CASES)
def test_decode_qkv_matches_oracle(dtype, nh, nkv, hd, n_sink, window, theta, steps, bias):
    cap = 0 if window else steps + 5
    g = HipKV(1, cap, nkv, hd, n_sink, window, dtype, theta)
    sep = HipKV(1, cap, nkv, hd, n_sink, window, dtype, theta)
    o = pyoracle.OracleKV(1, cap, nkv, hd, n_sink, window, dtype, theta)
    P, Q = nkv * hd, nh * hd
    qb = normal(600, Q) if bias else None
    kb = normal(601, P) if bias else None
    vb = normal(602, P) if bias else None
    K, V = normal(603, steps, P), normal(604, steps, P)
    if dtype == INT8:
        K[:, 5] *= 8.0
    sc = scale_of(hd)
    for t in range(steps):
        q = normal(700 + t, Q)
        got = g.decode_qkv(0, t, q, K[t], V[t], nh, sc, qb, kb, vb)
        qr, kr, vr = host_produce(q, K[t], V[t], qb, kb, vb, t, nh, nkv, hd, theta, window > 0)
        ref = sep.decode(0, t, kr, vr, qr, nh, sc)
        if window:
            want = o.attend_ring(0, t, qr, kr, vr, nh, sc)
        else:
            o.append(0, t, kr, vr)
            want = o.attend(0, t, qr, nh, sc)
        same_bits(got, ref, f"producer vs fused step on host-roped rows, step {t}")
        assert_close(got, want, what=f"producer step {t}")
    assert g.n_seen == steps
    for n in store_names(dtype, window, n_sink):
        same_bits(g.export(n, 0), o.export(n, 0), f"store {n} vs oracle")
    g.close()
    sep.close()


def test_decode_qkv_far_positions():
    """Rope table rows near the end of a 16384-position cache (config 5)."""
    nh, nkv, hd, cap, theta = 32, 8, 128, 16384, 1e6
    g = HipKV(1, cap, nkv, hd, 0, 0, INT8, theta)
    o = pyoracle.OracleKV(1, cap, nkv, hd, 0, 0, INT8, theta)
    P, Q = nkv * hd, nh * hd
    start = cap - 40
    K0, V0 = normal(610, start, P), normal(611, start, P)
    g.append_n(0, 0, K0, V0)
    o.append_n(0, 0, K0, V0)
    qb, kb, vb = normal(612, Q), normal(613, P), normal(614, P)
    sc = scale_of(hd)
    for t in range(start, cap):
        q, k, v = normal(620 + t, Q), normal(621 + t, P), normal(622 + t, P)
        got = g.decode_qkv(0, t, q, k, v, nh, sc, qb, kb, vb)
        qr, kr, vr = host_produce(q, k, v, qb, kb, vb, t, nh, nkv, hd, theta, False)
        o.append(0, t, kr, vr)
        if t % 13 == 0 or t == cap - 1:
            assert_close(got, o.attend(0, t, qr, nh, sc), what=f"pos {t}")
    for n in store_names(INT8, 0, 0):
        same_bits(g.export(n, 0), o.export(n, 0), f"store {n}")
    g.close()


CHUNK_CASES = [
    # dtype, nh, nkv, hd, pos0, n, theta, bias
    (F32, 32, 8, 64, 1792, 256, 5e5, False),   # config 2's last prefill chunk (matrix cores)
    (F32, 32, 8, 128, 2043, 5, 1e6, True),     # config 5 verify round
    (INT8, 32, 8, 128, 2043, 5, 1e6, True),
    (INT8, 24, 8, 128, 70, 9, 5e5, False),
    (F32, 14, 2, 64, 3, 100, 1e6, True),       # Qwen2.5-0.5B head counts
]


@pytest.mark.parametrize("dtype,nh,nkv,hd,pos0,n,theta,bias", CHUNK_CASES)
def test_chunk_qkv_matches_oracle(dtype, nh, nkv, hd, pos0, n, theta, bias):
    cap = pos0 + n + 3
    g = HipKV(1, cap, nkv, hd, 4, 0, dtype, theta)
    o = pyoracle.OracleKV(1, cap, nkv, hd, 4, 0, dtype, theta)
    P, Q = nkv * hd, nh * hd
    K0, V0 = normal(630, pos0, P), normal(631, pos0, P)
    if pos0:
        g.append_n(0, 0, K0, V0)
        o.append_n(0, 0, K0, V0)
    qb = normal(632, Q) if bias else None
    kb = normal(633, P) if bias else None
    vb = normal(634, P) if bias else None
    q, k, v = normal(635, n, Q), normal(636, n, P), normal(637, n, P)
    got = g.chunk_qkv(0, pos0, q, k, v, nh, scale_of(hd), qb, kb, vb)
    rows = [host_produce(q[c], k[c], v[c], qb, kb, vb, pos0 + c, nh, nkv, hd, theta, False)
            for c in range(n)]
    qr = np.stack([r[0] for r in rows])
    kr = np.stack([r[1] for r in rows])
    vr = np.stack([r[2] for r in rows])
    o.append_n(0, pos0, kr, vr)
    want = o.attend_chunk(0, pos0, qr, nh, scale_of(hd))
    assert_close(got, want.reshape(got.shape), what=f"chunk qkv pos0 {pos0} n {n}")
    assert g.n_seen == pos0 + n
    for name in store_names(dtype, 0, 4):
        same_bits(g.export(name, 0), o.export(name, 0), f"store {name}")
    g.close()


def test_qkv_async_matches_host_calls():
    """Device-pointer forms on torch tensors equal the host-pointer forms."""
    torch = pytest.importorskip("torch")
    nh, nkv, hd, theta, n = 32, 8, 128, 1e6, 5
    P, Q = nkv * hd, nh * hd
    a = HipKV(1, 64, nkv, hd, 4, 0, INT8, theta)
    b = HipKV(1, 64, nkv, hd, 4, 0, INT8, theta)
    qb, kb, vb = normal(640, Q), normal(641, P), normal(642, P)
    q, k, v = normal(643, n + 1, Q), normal(644, n + 1, P), normal(645, n + 1, P)
    sc = float(scale_of(hd))
    want_c = a.chunk_qkv(0, 0, q[:n], k[:n], v[:n], nh, sc, qb, kb, vb)
    want_d = a.decode_qkv(0, n, q[n], k[n], v[n], nh, sc, qb, kb, vb)
    T = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()  # noqa: E731
    tq, tk, tv, tqb, tkb, tvb = T(q), T(k), T(v), T(qb), T(kb), T(vb)
    out_c = torch.zeros(n, Q, device="cuda")
    out_d = torch.zeros(Q, device="cuda")
    torch.cuda.synchronize()
    b.chunk_qkv_async(0, 0, n, nh, sc, tq.data_ptr(), tk.data_ptr(), tv.data_ptr(),
                      tqb.data_ptr(), tkb.data_ptr(), tvb.data_ptr(), out_c.data_ptr())
    b.decode_qkv_async(0, n, nh, sc, tq[n].data_ptr(), tk[n].data_ptr(), tv[n].data_ptr(),
                       tqb.data_ptr(), tkb.data_ptr(), tvb.data_ptr(), out_d.data_ptr())
    b.sync()
    same_bits(out_c.cpu().numpy().reshape(-1), want_c, "async chunk")
    same_bits(out_d.cpu().numpy(), want_d, "async decode")
    for name in store_names(INT8, 0, 4):
        same_bits(b.export(name, 0), a.export(name, 0), f"store {name}")
    a.close()
    b.close()


def test_decode_qkv_unaligned_inputs_take_the_producer_kernel():
    """Rows that are not 16-byte aligned go through the producer kernel and
    the plain fused step; the result is the same bits as the one-launch path."""
    torch = pytest.importorskip("torch")
    nh, nkv, hd, theta, steps = 24, 8, 128, 5e5, 6
    P, Q = nkv * hd, nh * hd
    a = HipKV(1, 64, nkv, hd, 4, 0, INT8, theta)
    b = HipKV(1, 64, nkv, hd, 4, 0, INT8, theta)
    qb, kb, vb = normal(650, Q), normal(651, P), normal(652, P)
    q, k, v = normal(653, steps, Q), normal(654, steps, P), normal(655, steps, P)
    sc = float(scale_of(hd))
    # one extra float in front of every array: device pointers 4 bytes past alignment
    T = lambda x: torch.from_numpy(np.concatenate([[0.0], x.reshape(-1)]).astype(np.float32)).cuda()  # noqa: E731
    tq, tk, tv, tqb, tkb, tvb = T(q), T(k), T(v), T(qb), T(kb), T(vb)
    out = torch.zeros(Q, device="cuda")
    torch.cuda.synchronize()
    f = 4  # bytes to the first real element
    for t in range(steps):
        want = a.decode_qkv(0, t, q[t], k[t], v[t], nh, sc, qb, kb, vb)
        b.decode_qkv_async(0, t, nh, sc, tq.data_ptr() + f + 4 * Q * t, tk.data_ptr() + f + 4 * P * t,
                           tv.data_ptr() + f + 4 * P * t, tqb.data_ptr() + f, tkb.data_ptr() + f,
                           tvb.data_ptr() + f, out.data_ptr())
        b.sync()
        same_bits(out.cpu().numpy(), want, f"unaligned step {t}")
    for name in store_names(INT8, 0, 4):
        same_bits(b.export(name, 0), a.export(name, 0), f"store {name}")
    a.close()
    b.close()


def test_qkv_errors_leave_state():
    nh, nkv, hd = 8, 2, 64
    P, Q = nkv * hd, nh * hd
    q, k = np.zeros(Q, np.float32), np.zeros(P, np.float32)
    g = HipKV(1, 16, nkv, hd, 0, 0, F32, 0.0)  # dense without a rope base
    with pytest.raises(DbiError):
        g.decode_qkv(0, 0, q, k, k, nh, 0.125)
    assert g.n_seen == 0
    g.close()
    g = HipKV(1, 16, nkv, hd, 0, 0, INT8, 1e4)
    with pytest.raises(DbiError):
        g.decode_qkv(0, 16, q, k, k, nh, 0.125)  # past capacity
    with pytest.raises(DbiError):
        g.chunk_qkv(0, 10, np.zeros((7, Q), np.float32), np.zeros((7, P), np.float32),
                    np.zeros((7, P), np.float32), nh, 0.125)  # rows past capacity
    assert g.n_seen == 0
    g.close()
    r = HipKV(1, 0, nkv, hd, 2, 8, F32, 1e4)
    with pytest.raises(DbiError):  # rings take no chunks
        r.chunk_qkv(0, 0, np.zeros((2, Q), np.float32), np.zeros((2, P), np.float32),
                    np.zeros((2, P), np.float32), nh, 0.125)
    assert r.n_seen == 0
    r.close()
