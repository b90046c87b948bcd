"""GPU parity of the HIP path (through the C-ABI) against the CPU oracle, on
identical seeded inputs fed from one host buffer.

Bar: int8 codes, scales, sinks, raw staging, ring slots/residents and
rollback state bit-exact; fp32 attention |a - b| <= 1e-5 + 1e-4 |b|.
Shapes cover tests/metal_ops_test.cpp:164-170 (nh/nkv 14/2, 8/8; hd 64/128;
n_pos 1, 2, 64, 300) and every gqa factor of the five configs (8, 4, 3, 7, 4).
"""
import numpy as np
import pytest

import pyoracle
from dbinfer_amd.kv import F32, INT8, DbiError, HipKV
from helpers import assert_close, normal

pytestmark = pytest.mark.gpu


def scale_of(hd):
    return np.float32(1.0) / np.sqrt(np.float32(hd))


def pair(L, cap, nkv, hd, n_sink=0, window=0, dtype=F32, theta=1e4):
    return (HipKV(L, cap, nkv, hd, n_sink, window, dtype, theta),
            pyoracle.OracleKV(L, cap, nkv, hd, n_sink, window, dtype, theta))


def same_bits(a, b, what):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    if a.dtype == np.float32:
        a, b = a.view(np.uint32), b.view(np.uint32)
    diff = np.nonzero(a != b)[0]
    assert diff.size == 0, f"{what}: {diff.size} differing elements, first at {diff[:5]}"


def compare_store(g, o, layers, names):
    for l in layers:
        for n in names:
            same_bits(g.export(n, l), o.export(n, l), f"{n} layer {l}")


# ---------------------------------------------------------------- append


@pytest.mark.parametrize("hd", [64, 128, 40])
def test_append_dense_f32(hd):
    g, o = pair(2, 50, 3, hd)
    K, V = normal(1, 2, 50, 3 * hd), normal(2, 2, 50, 3 * hd)
    for l in range(2):
        for p in range(37):
            g.append(l, p, K[l, p], V[l, p])
            o.append(l, p, K[l, p], V[l, p])
        g.append_n(l, 37, K[l, 37:50], V[l, 37:50])
        o.append_n(l, 37, K[l, 37:50], V[l, 37:50])
    assert g.n_seen == o.n_seen == 50
    compare_store(g, o, [0, 1], ["k", "v"])


INT8_DENSE = ["k8", "v8", "k_scale", "v_scale", "k_raw"]


@pytest.mark.parametrize("hd,nkv,n_sink", [(128, 8, 4), (64, 2, 0), (40, 3, 4), (128, 1, 37)])
def test_append_int8_dense_bit_exact(hd, nkv, n_sink):
    L, cap = 2, 130
    g, o = pair(L, cap, nkv, hd, n_sink=n_sink, dtype=INT8)
    P = nkv * hd
    K, V = normal(3, L, cap, P), normal(4, L, cap, P)
    K[:, :, 7] *= 8.0  # outlier channel
    V[:, :, 3] *= 8.0
    K[:, 60, :32] = 0.0  # zero block / zero rows
    names = INT8_DENSE + (["k_sink", "v_sink"] if n_sink else [])
    for l in range(L):
        for p in range(45):  # one by one, crossing a group boundary
            g.append(l, p, K[l, p], V[l, p])
            o.append(l, p, K[l, p], V[l, p])
        compare_store(g, o, [l], names)
        g.append_n(l, 45, K[l, 45:110], V[l, 45:110])  # batch over 3 groups
        o.append_n(l, 45, K[l, 45:110], V[l, 45:110])
        compare_store(g, o, [l], names)


@pytest.mark.parametrize("n_new", [5, 50, 97])
def test_int8_rollback_across_group_boundary(n_new):
    """Rollback then re-append: the staging-row aliasing of the reference
    (k_raw indexed by pos % 32) is reproduced bit for bit. A batch longer
    than a group also overwrites staging rows that its first group still
    reads as they were."""
    L, cap, nkv, hd = 1, 160, 2, 64
    g, o = pair(L, cap, nkv, hd, n_sink=4, dtype=INT8)
    P = nkv * hd
    K, V = normal(5, 80, P), normal(6, 80, P)
    for p in range(41):
        g.append(0, p, K[p], V[p])
        o.append(0, p, K[p], V[p])
    for kv in (g, o):
        kv.truncate(30)
    assert g.n_seen == o.n_seen == 30
    knew, vnew = normal(7, n_new, P), normal(8, n_new, P)
    g.append_n(0, 30, knew, vnew)  # crosses back into group 1
    for r in range(n_new):
        o.append(0, 30 + r, knew[r], vnew[r])
    compare_store(g, o, [0], INT8_DENSE + ["k_sink", "v_sink"])


def test_int8_bulk_append_matches_sequential():
    """One batch of 1000 rows from a group boundary and one from mid-group
    against the oracle's row-by-row appends (31 groups requantized at once)."""
    L, cap, nkv, hd = 1, 2100, 4, 128
    P = nkv * hd
    K, V = normal(9, 2048, P), normal(10, 2048, P)
    K[:, 11] *= 8.0
    for start in (0, 1037):
        g, o = pair(L, cap, nkv, hd, n_sink=4, dtype=INT8)
        if start:
            g.append_n(0, 0, K[:start], V[:start])
            o.append_n(0, 0, K[:start], V[:start])
        g.append_n(0, start, K[start:start + 1000], V[start:start + 1000])
        for r in range(start, start + 1000):
            o.append(0, r, K[r], V[r])
        compare_store(g, o, [0], INT8_DENSE + ["k_sink", "v_sink"])


@pytest.mark.parametrize("dtype", [F32, INT8])
@pytest.mark.parametrize("n_sink,window", [(4, 16), (0, 8), (2, 5)])
def test_ring_append_slots_residents(dtype, n_sink, window):
    nkv, hd = 2, 64
    g, o = pair(1, 0, nkv, hd, n_sink, window, dtype, 1e6)
    P = nkv * hd
    K, V = normal(9, 120, P), normal(10, 120, P)
    names = ["k", "v"] if dtype == F32 else ["k8", "v8", "k_scale", "v_scale"]
    for t in range(60):
        g.append(0, t, K[t], V[t])
        o.append(0, t, K[t], V[t])
        assert g.slot_for(t) == o.slot_for(t)
        gs, gr = g.residents()
        os_, or_ = o.residents()
        same_bits(gs, os_, "slots")
        same_bits(gr, or_, "rope_pos")
    compare_store(g, o, [0], names)
    g.append_n(0, 60, K[60:120], V[60:120])  # batch longer than the window
    o.append_n(0, 60, K[60:120], V[60:120])
    compare_store(g, o, [0], names)
    for kv in (g, o):
        kv.truncate(100)
    same_bits(g.residents()[0], o.residents()[0], "slots after rollback")


# ---------------------------------------------------------------- decode


def fill_both(g, o, L, n, seed, outlier=False):
    P = g.pos_stride
    K, V = normal(seed, L, n, P), normal(seed + 1, L, n, P)
    if outlier:
        ch = np.random.default_rng(seed).choice(P, max(1, P // 100), replace=False)
        K[:, :, ch] *= 8.0
        V[:, :, ch] *= 8.0
    for l in range(L):
        g.append_n(l, 0, K[l], V[l])
        o.append_n(l, 0, K[l], V[l])
    return K, V


@pytest.mark.parametrize("nh,nkv", [(14, 2), (8, 8), (32, 4), (32, 8), (24, 8), (28, 4)])
@pytest.mark.parametrize("hd", [64, 128])
@pytest.mark.parametrize("n_pos", [1, 2, 64, 300])
def test_decode_dense_f32(nh, nkv, hd, n_pos):
    g, o = pair(1, 320, nkv, hd)
    fill_both(g, o, 1, n_pos, 20 + n_pos)
    q = normal(21, nh * hd)
    got = g.attend(0, n_pos - 1, q, nh, scale_of(hd))
    want = o.attend(0, n_pos - 1, q, nh, scale_of(hd))
    assert_close(got, want, what=f"nh{nh} nkv{nkv} hd{hd} n{n_pos}")


@pytest.mark.parametrize("nh,nkv,hd", [(24, 8, 128), (32, 8, 128), (32, 4, 64), (28, 4, 128),
                                       (8, 8, 64)])
@pytest.mark.parametrize("n_sink", [0, 4])
@pytest.mark.parametrize("n_pos", [1, 3, 33, 300, 1000])
def test_decode_dense_int8(nh, nkv, hd, n_sink, n_pos):
    g, o = pair(1, 1024, nkv, hd, n_sink=n_sink, dtype=INT8)
    fill_both(g, o, 1, n_pos, 30 + n_pos, outlier=True)
    q = normal(31, nh * hd)
    got = g.attend(0, n_pos - 1, q, nh, scale_of(hd))
    want = o.attend(0, n_pos - 1, q, nh, scale_of(hd))
    assert_close(got, want, what=f"int8 nh{nh} nkv{nkv} hd{hd} sink{n_sink} n{n_pos}")


@pytest.mark.parametrize("dtype", [F32, INT8])
@pytest.mark.parametrize("nh,nkv,hd,n_sink,window", [(28, 4, 128, 4, 64), (8, 2, 64, 0, 40),
                                                     (32, 8, 128, 4, 100)])
def test_decode_ring_stream(dtype, nh, nkv, hd, n_sink, window):
    """Stream past several wraps with a decode every step (config 4 pattern)."""
    g, o = pair(1, 0, nkv, hd, n_sink, window, dtype, 1e6)
    steps = 3 * (n_sink + window) + 7
    for t in range(steps):
        q = normal(100 + t, nh * hd)
        k = normal(200 + t, nkv * hd)
        v = normal(300 + t, nkv * hd)
        g.append(0, t, k, v)
        got = g.attend(0, t, q, nh, scale_of(hd))
        want = o.attend_ring(0, t, q, k, v, nh, scale_of(hd))
        assert_close(got, want, what=f"ring step {t}")


# ---------------------------------------------------------------- fused decode step


FUSED_CASES = [
    # dtype, nh, nkv, hd, n_sink, window, steps
    (F32, 24, 8, 128, 0, 0, 70),
    (INT8, 24, 8, 128, 4, 0, 70),     # config 3 shape: sinks, then groups
    (INT8, 32, 8, 64, 0, 0, 40),
    (INT8, 28, 4, 128, 37, 0, 45),    # sinks spanning a whole group and more
    (F32, 32, 4, 64, 0, 0, 33),       # config 1 shape (gqa 8, head groups)
    (F32, 28, 4, 128, 4, 24, 70),     # config 4 shape ring, wraps twice
    (INT8, 28, 4, 128, 4, 24, 70),
    (INT8, 8, 2, 64, 0, 20, 50),
]


@pytest.mark.parametrize("dtype,nh,nkv,hd,n_sink,window,steps", FUSED_CASES)
def test_fused_decode_step(dtype, nh, nkv, hd, n_sink, window, steps):
    """dbi_kv_decode (append + attend in one launch) against the oracle's
    append + attend every step, the separate C-ABI path bit for bit, and the
    stored arrays bit-exact at the end."""
    cap = 0 if window else steps + 3
    g, o = pair(1, cap, nkv, hd, n_sink, window, dtype, 1e6)
    sep = HipKV(1, cap, nkv, hd, n_sink, window, dtype, 1e6)
    K = normal(400, steps, nkv * hd)
    V = normal(401, steps, nkv * hd)
    if dtype == INT8:
        K[:, 5] *= 8.0
    sc = scale_of(hd)
    for t in range(steps):
        q = normal(500 + t, nh * hd)
        got = g.decode(0, t, K[t], V[t], q, nh, sc)
        sep.append(0, t, K[t], V[t])
        ref = sep.attend(0, t, q, nh, sc)
        if window:
            want = o.attend_ring(0, t, q, K[t], V[t], nh, sc)
        else:
            o.append(0, t, K[t], V[t])
            want = o.attend(0, t, q, nh, sc)
        assert_close(got, want, what=f"fused step {t}")
        same_bits(got, ref, f"fused vs separate step {t}")
    assert g.n_seen == steps
    if dtype == INT8:
        names = ["k8", "v8", "k_scale", "v_scale"]
        if not window:
            names += ["k_raw"] + (["k_sink", "v_sink"] if n_sink else [])
    else:
        names = ["k", "v"]
    for n in names:
        same_bits(g.export(n, 0), sep.export(n, 0), f"fused store {n} vs separate")
    compare_store(g, o, [0], names)
    sep.close()


def test_fused_decode_rejects_bad_input():
    g = HipKV(1, 16, 2, 64)
    k = np.zeros(128, np.float32)
    q = np.zeros(8 * 64, np.float32)
    with pytest.raises(DbiError):
        g.decode(0, 16, k, k, q, 8, 0.125)  # past capacity
    with pytest.raises(DbiError):
        g.decode(0, 0, k, k, q[: 7 * 64], 7, 0.125)  # n_heads not a multiple of n_kv_heads
    assert g.n_seen == 0
    g.close()


# ---------------------------------------------------------------- chunk


@pytest.mark.parametrize("dtype", [F32, INT8])
@pytest.mark.parametrize("nh,nkv,hd,pos0,n", [
    (32, 8, 64, 0, 64), (32, 8, 64, 256, 100),
    (32, 8, 64, 1792, 256),   # config 2's last prefill chunk (matrix-core path for fp32)
    (32, 8, 128, 300, 128),   # hd 128, gqa 4
    (32, 8, 128, 1500, 64),   # hd 128, 8 key splits
    (24, 8, 128, 300, 100),   # gqa 3 (5 rows per wave, one padding column)
    (28, 4, 128, 1000, 64),   # gqa 7 (2 rows per wave, two padding columns)
    (40, 8, 64, 50, 77),      # gqa 5
    (48, 8, 64, 10, 130),     # gqa 6 (2 rows per wave, four padding columns)
    (16, 16, 128, 40, 130),   # hd 128, gqa 1 (16 rows per wave, 128 per workgroup)
    (8, 8, 64, 5, 70),        # gqa 1
    (16, 8, 128, 17, 77),     # gqa 2, ragged last wave
    (32, 4, 64, 1000, 65),    # gqa 8 (config 1 shape)
    (32, 8, 128, 2047, 5), (24, 8, 128, 70, 9),
    (14, 2, 64, 3, 1)])
def test_chunk_attention(dtype, nh, nkv, hd, pos0, n):
    g, o = pair(1, 2100, nkv, hd, n_sink=4, dtype=dtype)
    fill_both(g, o, 1, pos0 + n, 40 + n)
    q = normal(41, n, nh * hd)
    got = g.attend_chunk(0, pos0, q, nh, scale_of(hd))
    want = o.attend_chunk(0, pos0, q, nh, scale_of(hd))
    assert_close(got, want, what=f"chunk dtype{dtype} pos0 {pos0} n {n}")
    # a second call on the same workspace (split counters at a new epoch)
    again = g.attend_chunk(0, pos0, q, nh, scale_of(hd))
    assert np.array_equal(again, got)


@pytest.mark.parametrize("dtype", [F32, INT8])
@pytest.mark.parametrize("nh,nkv,hd,pos0,n,ns", [
    (32, 8, 128, 0, 3, 4),        # one chunk, one split: direct output; int8: rows see 1..3 sinks
    (16, 8, 128, 17, 2, 4),       # gqa 2: one 16-vector tile
    (40, 8, 64, 33, 6, 4),        # gqa 5: 30 vectors in two tiles
    (28, 4, 128, 4000, 5, 4),     # gqa 7: two row groups (4 + 1)
    (32, 4, 64, 1000, 40, 4),     # gqa 8: ten row groups
    (8, 8, 64, 5, 63, 4),         # gqa 1: two row groups (32 + 31)
    (32, 8, 128, 16379, 5, 4),    # config 5's verify round at 16k (32 splits)
    (32, 8, 128, 4, 6, 9),        # int8: rows see 5..9 sinks (more than the merge holds at once)
    # remainder tiles: 16 vectors + up to 16 / (hd / 32) in (query, block)
    # columns (int8) or up to 4 in 4 x 4 blocks (fp32)
    (32, 8, 128, 2, 5, 4),        # gqa 4, 20 vectors: rows see 3..4 sinks
    (24, 8, 128, 700, 6, 4),      # gqa 3, 18 vectors: a remainder of 2
    (40, 8, 64, 300, 4, 4),       # hd 64, gqa 5, 20 vectors: 4 of 8 remainder columns (fp32: all 4)
    (16, 8, 64, 90, 12, 4),       # hd 64, gqa 2, 24 vectors: the full remainder (fp32: two tiles)
    (28, 4, 128, 4000, 10, 4),    # gqa 7: row groups of 2 rows (14 vectors, one tile)
    (8, 8, 128, 100, 18, 4),      # gqa 1, 18 vectors: remainder of 2 rows
    (16, 8, 128, 500, 10, 4),     # gqa 2, 20 vectors: the full remainder
])
def test_chunk_rows(dtype, nh, nkv, hd, pos0, n, ns):
    """Dense chunks of 2..63 rows (model.cpp:956-981) run on the matrix-core
    rows kernels (fp32; int8 with fp32 sinks and 1% outlier channels x8);
    every row group, split plan and the direct path."""
    g, o = pair(1, pos0 + n + 64, nkv, hd, n_sink=ns, dtype=dtype)
    fill_both(g, o, 1, pos0 + n, 70 + n, outlier=dtype == INT8)
    q = normal(71, n, nh * hd)
    got = g.attend_chunk(0, pos0, q, nh, scale_of(hd))
    want = o.attend_chunk(0, pos0, q, nh, scale_of(hd), n_threads=8)
    assert_close(got, want, what=f"rows dtype {dtype} pos0 {pos0} n {n} gqa {nh // nkv}")
    # a second call on the same workspace (split counters at a new epoch)
    again = g.attend_chunk(0, pos0, q, nh, scale_of(hd))
    assert np.array_equal(again, got)


@pytest.mark.parametrize("dtype", [F32, INT8])
@pytest.mark.parametrize("nh,nkv,hd,pos0,n", [
    (32, 8, 64, 1000, 256),   # fp32: prefill kernel, hd 64
    (24, 8, 128, 300, 100),   # fp32: prefill kernel at gqa 3
    (32, 8, 128, 2000, 5),    # rows kernels (int8: the remainder tile)
])
def test_chunk_attention_rising_scores(dtype, nh, nkv, hd, pos0, n):
    """Scores that climb along the keys (q x 2, K rows scaled by 1 + pos/1024)
    move every row's running maximum from ~7 to ~30 in log2 units, past the
    kernels' lazy reference maximum by more than 8 several times: the
    rescale runs mid-stream and weights near 2^8 enter before it. (Scores
    of several hundred put fp32's own rounding of a score above the 1e-4
    tolerance for every kernel, the exact-product fp32 one included.)"""
    g, o = pair(1, 2100, nkv, hd, n_sink=4, dtype=dtype)
    P = g.pos_stride
    K, V = normal(3100 + n, 1, pos0 + n, P), normal(3101 + n, 1, pos0 + n, P)
    K *= (1.0 + np.arange(pos0 + n, dtype=np.float32) / 1024.0)[None, :, None]
    g.append_n(0, 0, K[0], V[0])
    o.append_n(0, 0, K[0], V[0])
    q = normal(3102 + n, n, nh * hd) * np.float32(2.0)
    got = g.attend_chunk(0, pos0, q, nh, scale_of(hd))
    want = o.attend_chunk(0, pos0, q, nh, scale_of(hd), n_threads=8)
    assert_close(got, want, what=f"rising scores dtype {dtype} hd {hd} n {n}")


# (drawn once with numpy's default_rng(2026); every gqa factor, both head dims)
RANDOM_CHUNKS = [
    (F32, 8, 8, 64, 47, 3), (INT8, 8, 4, 64, 833, 17), (F32, 6, 2, 128, 1147, 17),
    (INT8, 16, 4, 128, 1304, 150), (F32, 40, 8, 64, 1189, 150), (INT8, 12, 2, 64, 1077, 150),
    (F32, 14, 2, 128, 297, 7), (INT8, 48, 6, 128, 1563, 100), (F32, 2, 2, 64, 1048, 64),
    (INT8, 16, 8, 64, 925, 3), (F32, 12, 4, 128, 1082, 150), (INT8, 16, 4, 128, 598, 33),
    (F32, 10, 2, 64, 262, 7), (INT8, 12, 2, 64, 867, 150), (INT8, 24, 8, 128, 1500, 6),
]


@pytest.mark.parametrize("dtype,nh,nkv,hd,pos0,n", RANDOM_CHUNKS)
def test_chunk_attention_random_shapes(dtype, nh, nkv, hd, pos0, n):
    """Chunk calls over mixed shapes: the prefill kernel (fp32, >= 64 rows,
    any gqa), the rows kernels with one or several row groups, and the int8
    remainder tile, each against the oracle."""
    g, o = pair(1, 1900, nkv, hd, n_sink=4, dtype=dtype)
    fill_both(g, o, 1, pos0 + n, 200 + n + pos0 % 97, outlier=dtype == INT8)
    q = normal(201 + n, n, nh * hd)
    got = g.attend_chunk(0, pos0, q, nh, scale_of(hd))
    want = o.attend_chunk(0, pos0, q, nh, scale_of(hd), n_threads=8)
    assert_close(got, want, what=f"random chunk dtype {dtype} {nh}/{nkv} hd {hd} pos0 {pos0} n {n}")


# ---------------------------------------------------------------- long context


@pytest.mark.parametrize("dtype,nh,nkv,hd,n_pos", [
    (INT8, 24, 8, 128, 8192),   # config 3 shape at its context
    (F32, 24, 8, 128, 8192),
    (F32, 32, 8, 128, 16384),   # config 5 shape at its final context
    (F32, 32, 4, 64, 1025),     # config 1 shape
])
def test_decode_long_context(dtype, nh, nkv, hd, n_pos):
    g, o = pair(1, n_pos, nkv, hd, n_sink=4, dtype=dtype)
    fill_both(g, o, 1, n_pos, 50, outlier=dtype == INT8)
    if dtype == INT8:
        compare_store(g, o, [0], INT8_DENSE + ["k_sink", "v_sink"])
    for pos in (n_pos - 1, n_pos // 2 + 5):
        q = normal(51 + pos, nh * hd)
        got = g.attend(0, pos, q, nh, scale_of(hd))
        want = o.attend(0, pos, q, nh, scale_of(hd), n_threads=8)
        assert_close(got, want, what=f"long ctx pos {pos}")


# ---------------------------------------------------------------- prefix + errors


def test_prefix_save_load_matches_oracle(tmp_path):
    L, cap, nkv, hd = 3, 64, 2, 64
    g, o = pair(L, cap, nkv, hd)
    fill_both(g, o, L, 40, 60)
    toks = np.arange(1000, 1030, dtype=np.int32)
    gp, op = str(tmp_path / "g.kv"), str(tmp_path / "o.kv")
    g.save_prefix(gp, toks)
    o.save_prefix(op, toks)
    assert open(gp, "rb").read() == open(op, "rb").read()
    fresh = HipKV(L, cap, nkv, hd)
    assert fresh.load_prefix(op, np.concatenate([toks, [1, 2]])) == 30
    assert fresh.n_seen == 30
    for l in range(L):
        got = fresh.export("k", l).reshape(cap, -1)[:30]
        same_bits(got, o.export("k", l).reshape(cap, -1)[:30], f"k layer {l}")
    # error leaves the GPU cache untouched
    bad = str(tmp_path / "bad.kv")
    open(bad, "wb").write(open(op, "rb").read()[:-4])
    before = fresh.export("v", 1)
    with pytest.raises(DbiError) as e:
        fresh.load_prefix(bad, toks)
    assert e.value.message == "kv prefix cache payload size mismatch"
    assert fresh.n_seen == 30
    same_bits(fresh.export("v", 1), before, "v untouched")
    with pytest.raises(DbiError) as e:
        fresh.load_prefix(op, toks[:10])
    assert e.value.message == "kv prefix is longer than the prompt"


def test_abi_errors_leave_state():
    g = HipKV(2, 16, 2, 64)
    k = normal(1, 128)
    g.append(0, 3, k, k)
    with pytest.raises(DbiError):
        g.append(2, 0, k, k)  # layer out of range
    with pytest.raises(DbiError):
        g.append(0, 16, k, k)  # past capacity
    with pytest.raises(DbiError):
        g.attend(0, 3, normal(2, 3 * 64), 3, 0.125)  # 3 heads over 2 kv heads
    with pytest.raises(DbiError) as e:
        g.attend(0, 3, normal(2, 40 * 64), 40, 0.125)  # gqa 20: no kernel
    assert e.value.status == 2
    with pytest.raises(DbiError):
        g.residents()  # dense cache has no ring mapping
    assert g.n_seen == 4
    ring = HipKV(1, 0, 1, 64, 0, 8, INT8, 1e4)  # rings have no prefix files
    ring.append(0, 0, normal(3, 64), normal(4, 64))
    with pytest.raises(DbiError) as e:
        ring.save_prefix("/tmp/never.kv", [1])
    assert "dense fp32" in e.value.message
