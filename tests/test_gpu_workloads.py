"""Parity of the five benchmark workloads at their real shapes and lengths,
through the C-ABI, against the CPU oracle on the same seeded inputs.

- C4: the ring at window 4096 with 4 sinks (28q/4kv, hd 128), filled past
  three wraps, then fused decode steps across the next wrap. The plan has
  more than 32 key splits, so the merge's second record batch runs
  (model.cpp:321-324, 406-418, 662-728).
- C5: a 2048-token fp32 prefix file at 8 kv heads / hd 128, byte-identical
  to the oracle's (model.cpp:1072-1156), loaded into fp32 and int8 caches,
  then 200 verify rounds: append 5 rows, causal chunk attention over them,
  roll back to len + a + 1 with a ~ U{0..4} (speculative.cpp:25-95,
  rollback at :82; model.cpp:933-981).
- C2: eight 256-row prefill chunks from raw projections (bias-free, rope on
  the device), then decode steps to 4096 (main.cpp:276-296,
  model.cpp:933-981, 996-1021).
- C3: the bench's exact call, the fused int8 step at pos 8191 over a full
  8192-position cache (32 splits), against the oracle's append + attend.

Bars: int8 codes, scales, raw staging rows and sinks bit-exact; fp32 stores
bit-exact; attention |a - b| <= 1e-5 + 1e-4 |b|.
"""
import numpy as np
import pytest

import pyoracle
from dbinfer_amd.kv import F32, INT8, HipKV
from helpers import assert_close, normal

pytestmark = pytest.mark.gpu

INT8_DENSE = ["k8", "v8", "k_scale", "v_scale", "k_raw", "k_sink", "v_sink"]


def scale_of(hd):
    return np.float32(1.0) / np.sqrt(np.float32(hd))


def same_bits(a, b, what):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    if a.dtype == np.float32:
        a, b = a.view(np.uint32), b.view(np.uint32)
    diff = np.nonzero(a != b)[0]
    assert diff.size == 0, f"{what}: {diff.size} differing elements, first at {diff[:5]}"


def compare_store(g, o, layers, names):
    for layer in layers:
        for n in names:
            same_bits(g.export(n, layer), o.export(n, layer), f"{n} layer {layer}")


def outliers(seed, P, rows):
    """1% of channels x8, a seeded choice shared by all rows (config 3)."""
    ch = np.random.default_rng(seed).choice(P, max(1, round(0.01 * P)), replace=False)
    m = np.ones(P, np.float32)
    m[ch] = 8.0
    return rows * m


def rope_rows(x, pos0, theta, heads, hd):
    """tensor::rope of rows [n][heads][hd] at positions pos0.. (ops.cpp:19-38)."""
    n = x.shape[0]
    t = np.ascontiguousarray(x.reshape(n, heads, hd).transpose(1, 0, 2))
    r = pyoracle.rope(t, np.arange(pos0, pos0 + n, dtype=np.int32), theta, heads, n, hd)
    return r.reshape(heads, n, hd).transpose(1, 0, 2).reshape(n, heads * hd)


# ---------------------------------------------------------------- C4


@pytest.mark.parametrize("dtype", [F32, INT8])
def test_c4_ring_window_4096(dtype):
    nh, nkv, hd, s, W, theta = 28, 4, 128, 4, 4096, 1e6
    g = HipKV(1, 0, nkv, hd, s, W, dtype, theta)
    o = pyoracle.OracleKV(1, 0, nkv, hd, s, W, dtype, theta)
    P = nkv * hd
    wrap = s + 3 * W  # slot_for(wrap) == s: the window's fourth wrap starts here
    fill = wrap - 15
    K, V = normal(900, fill, P), normal(901, fill, P)
    if dtype == INT8:
        K, V = outliers(902, P, K), outliers(903, P, V)
    g.append_n(0, 0, K, V)
    o.append_n(0, 0, K, V)
    compare_store(g, o, [0], ["k", "v"] if dtype == F32 else ["k8", "v8", "k_scale", "v_scale"])
    # the full window: 4100 residents over more than 32 splits (second merge batch)
    assert g.splits(fill, 1, nh) > 32
    sc = scale_of(hd)
    for t in range(fill, wrap + 17):
        q = normal(1000 + t, nh * hd)
        k, v = normal(2000 + t, P), normal(3000 + t, P)
        got = g.decode(0, t, k, v, q, nh, sc)
        want = o.attend_ring(0, t, q, k, v, nh, sc, n_threads=8)
        assert_close(got, want, what=f"C4 ring dtype {dtype} step {t}")
    assert g.n_seen == o.n_seen == wrap + 17
    same_bits(g.residents()[0], o.residents()[0], "resident slots")
    same_bits(g.residents()[1], o.residents()[1], "resident rope positions")
    compare_store(g, o, [0], ["k", "v"] if dtype == F32 else ["k8", "v8", "k_scale", "v_scale"])


# ---------------------------------------------------------------- C5


C5_NH, C5_NKV, C5_HD, C5_THETA, C5_PREFIX = 32, 8, 128, 1e6, 2048


@pytest.fixture(scope="module")
def c5_prefix(tmp_path_factory):
    """A 2048-token fp32 prefix of two layers at the C5 shape, saved by the
    device and by the oracle; the files must be byte-identical."""
    L, P = 2, C5_NKV * C5_HD
    cap = C5_PREFIX + 64
    g = HipKV(L, cap, C5_NKV, C5_HD, 0, 0, F32, C5_THETA)
    o = pyoracle.OracleKV(L, cap, C5_NKV, C5_HD, 0, 0, F32, C5_THETA)
    rows = []
    for layer in range(L):
        K, V = normal(1100 + layer, C5_PREFIX, P), normal(1110 + layer, C5_PREFIX, P)
        g.append_n(layer, 0, K, V)
        o.append_n(layer, 0, K, V)
        rows.append((K, V))
    toks = np.arange(7, 7 + C5_PREFIX, dtype=np.int32)
    d = tmp_path_factory.mktemp("c5")
    gp, op = str(d / "gpu.kv"), str(d / "oracle.kv")
    g.save_prefix(gp, toks)
    o.save_prefix(op, toks)
    g.close()
    o.close()
    return gp, op, toks, rows


def test_c5_prefix_file_matches_oracle(c5_prefix):
    gp, op, toks, _ = c5_prefix
    a, b = open(gp, "rb").read(), open(op, "rb").read()
    assert len(a) == len(b) == 28 + 4 * C5_PREFIX + 2 * 2 * C5_PREFIX * C5_NKV * C5_HD * 4
    assert a == b


@pytest.mark.parametrize("dtype", [F32, INT8])
def test_c5_verify_rounds(c5_prefix, dtype):
    """200 verify rounds from the loaded prefix: append 5, attend the 5 rows,
    roll back to len + a + 1. Stores are compared at the end (int8 K-group
    requantization and staging-row aliasing across the rollbacks), outputs
    every 8th round."""
    gp, _, toks, rows = c5_prefix
    L, P, Q = 2, C5_NKV * C5_HD, C5_NH * C5_HD
    rounds, k1 = 200, 5
    cap = C5_PREFIX + rounds * k1 + 64
    n_sink = 4 if dtype == INT8 else 0
    g = HipKV(L, cap, C5_NKV, C5_HD, n_sink, 0, dtype, C5_THETA)
    o = pyoracle.OracleKV(L, cap, C5_NKV, C5_HD, n_sink, 0, dtype, C5_THETA)
    assert g.load_prefix(gp, np.concatenate([toks, [1, 2, 3]])) == C5_PREFIX
    if dtype == F32:
        assert o.load_prefix(gp, toks) == C5_PREFIX
    else:  # a v1 file enters an int8 cache by quantize-on-append
        for layer in range(L):
            o.append_n(layer, 0, rows[layer][0], rows[layer][1])
    assert g.n_seen == o.n_seen == C5_PREFIX
    rng = np.random.default_rng(1200)
    sc = scale_of(C5_HD)
    length = C5_PREFIX
    for r in range(rounds):
        Kn = rng.standard_normal((L, k1, P), dtype=np.float32)
        Vn = rng.standard_normal((L, k1, P), dtype=np.float32)
        check = r % 8 == 0 or r == rounds - 1
        for layer in range(L):
            g.append_n(layer, length, Kn[layer], Vn[layer])
            o.append_n(layer, length, Kn[layer], Vn[layer])
            q = rng.standard_normal((k1, Q), dtype=np.float32)
            got = g.attend_chunk(layer, length, q, C5_NH, sc)
            if check:
                want = o.attend_chunk(layer, length, q, C5_NH, sc, n_threads=8)
                assert_close(got, want, what=f"C5 round {r} layer {layer} dtype {dtype}")
        length += int(rng.integers(0, 5)) + 1
        g.truncate(length)
        o.truncate(length)
    assert g.n_seen == o.n_seen == length
    compare_store(g, o, range(L), ["k", "v"] if dtype == F32 else INT8_DENSE)


# ---------------------------------------------------------------- C2


def test_c2_prefill_chunks_then_decode():
    """Config 2 (32q/8kv, hd 64, theta 5e5): eight 256-row chunks through the
    on-device producer (rope, append, causal chunk attention), then decode
    steps to ctx 4096 from raw projections, outputs checked at sampled
    positions and the whole fp32 store bit-exact at the end."""
    nh, nkv, hd, theta, cap = 32, 8, 64, 5e5, 4096
    P, Q = nkv * hd, nh * hd
    g = HipKV(1, cap, nkv, hd, 0, 0, F32, theta)
    o = pyoracle.OracleKV(1, cap, nkv, hd, 0, 0, F32, theta)
    sc = scale_of(hd)
    rng = np.random.default_rng(1300)
    for c in range(8):
        pos0 = 256 * c
        q = rng.standard_normal((256, Q), dtype=np.float32)
        k = rng.standard_normal((256, P), dtype=np.float32)
        v = rng.standard_normal((256, P), dtype=np.float32)
        assert g.splits(pos0, 256, nh) >= 1
        got = g.chunk_qkv(0, pos0, q, k, v, nh, sc)
        o.append_n(0, pos0, rope_rows(k, pos0, theta, nkv, hd), v)
        want = o.attend_chunk(0, pos0, rope_rows(q, pos0, theta, nh, hd), nh, sc, n_threads=8)
        assert_close(got, want, what=f"C2 prefill chunk {c}")
    checks = {2048, 2049, 2500, 3000, 3333, 4000, 4095}
    for t in range(2048, cap):
        q = rng.standard_normal(Q, dtype=np.float32)
        k = rng.standard_normal(P, dtype=np.float32)
        v = rng.standard_normal(P, dtype=np.float32)
        got = g.decode_qkv(0, t, q, k, v, nh, sc)
        o.append(0, t, pyoracle.rope(k, [t], theta, nkv, 1, hd), v)
        if t in checks:
            want = o.attend(0, t, pyoracle.rope(q, [t], theta, nh, 1, hd), nh, sc, n_threads=8)
            assert_close(got, want, what=f"C2 decode pos {t}")
    assert g.n_seen == o.n_seen == cap
    compare_store(g, o, [0], ["k", "v"])


# ---------------------------------------------------------------- C3 bench call


def test_c3_bench_call_fused_int8_at_8191():
    """The bench's timed call: the fused int8 decode step (append at 8191 +
    attention over 8192 keys with 4 fp32 sinks) on a full config-3 cache."""
    nh, nkv, hd, ctx, s = 24, 8, 128, 8192, 4
    P = nkv * hd
    g = HipKV(1, ctx, nkv, hd, s, 0, INT8, 5e5)
    o = pyoracle.OracleKV(1, ctx, nkv, hd, s, 0, INT8, 5e5)
    K = outliers(1400, P, normal(1401, ctx, P))
    V = outliers(1400, P, normal(1402, ctx, P))
    g.append_n(0, 0, K[:-1], V[:-1])
    o.append_n(0, 0, K[:-1], V[:-1])
    assert g.splits(ctx - 1, 1, nh) > 1
    q = normal(1403, nh * hd)
    sc = scale_of(hd)
    got = g.decode(0, ctx - 1, K[-1], V[-1], q, nh, sc)
    o.append(0, ctx - 1, K[-1], V[-1])
    want = o.attend(0, ctx - 1, q, nh, sc, n_threads=8)
    assert_close(got, want, what="C3 fused int8 step at 8191")
    compare_store(g, o, [0], INT8_DENSE)
    # the same call again (the cache already holds the row): identical bits
    again = g.decode(0, ctx - 1, K[-1], V[-1], q, nh, sc)
    same_bits(again, got, "repeated fused step")
