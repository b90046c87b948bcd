"""The allocation-free decode step (dbi_kv_decode_noalloc_async) against the
fused step it mirrors (dbi_kv_decode_async), through the C-ABI on one GPU:
identical output bits and identical stores on two calls in a row, the
second smaller, over several split plans and layouts, and at the largest
split plan a decode call can have; the oracle checks the result to the
attention tolerance."""
import numpy as np
import pytest

import pyoracle
from dbinfer_amd.kv import F32, INT8, HipKV
from helpers import assert_close

pytestmark = pytest.mark.gpu


def stores(dtype, window, n_sink):
    if dtype == F32:
        return ["k", "v"]
    names = ["k8", "v8", "k_scale", "v_scale"]
    if window:
        return names
    return names + ["k_raw"] + (["k_sink", "v_sink"] if n_sink else [])


CASES = [
    # dtype, nh, nkv, hd, n_sink, window, (ctx of the first call, ctx of the second)
    (INT8, 24, 8, 128, 4, 0, (8192, 700)),   # config 3: 32 splits, then 3
    (F32, 32, 8, 128, 0, 0, (4096, 64)),     # config 5 shape; the second writes directly
    (F32, 28, 4, 128, 4, 4096, (6000, 300)),  # config 4 ring: 52 splits, then fewer
    (INT8, 32, 4, 64, 0, 0, (1025, 40)),     # config 1 shape
]


@pytest.mark.parametrize("dtype,nh,nkv,hd,n_sink,window,ctxs", CASES)
def test_noalloc_decode_matches_decode_async(dtype, nh, nkv, hd, n_sink, window, ctxs):
    torch = pytest.importorskip("torch")
    P, Q = nkv * hd, nh * hd
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    cap = 0 if window else max(ctxs)
    for call, ctx in enumerate(ctxs):
        print(f"noalloc case dtype={dtype} nh={nh} nkv={nkv} hd={hd} window={window} "
              f"call {call} ctx {ctx}", flush=True)
        rng = np.random.default_rng(1500 + ctx)
        K = rng.standard_normal((ctx, P), dtype=np.float32)
        V = rng.standard_normal((ctx, P), dtype=np.float32)
        q = rng.standard_normal(Q, dtype=np.float32)
        ref = HipKV(1, cap, nkv, hd, n_sink, window, dtype, 1e6)
        new = HipKV(1, cap, nkv, hd, n_sink, window, dtype, 1e6)
        o = pyoracle.OracleKV(1, cap, nkv, hd, n_sink, window, dtype, 1e6)
        for kv in (ref, new, o):
            kv.append_n(0, 0, K[:-1], V[:-1])
        stream = torch.cuda.current_stream()
        Kd, Vd, qd = (torch.from_numpy(a).cuda() for a in (K, V, q))
        out_ref = torch.full((Q,), float("nan"), device="cuda")
        out_new = torch.full((Q,), float("nan"), device="cuda")
        for kv in (ref, new):
            kv.set_stream(stream.cuda_stream)
        torch.cuda.synchronize()
        pos = ctx - 1
        ref.decode_async(0, pos, Kd[pos].data_ptr(), Vd[pos].data_ptr(), nh, scale,
                         qd.data_ptr(), out_ref.data_ptr())
        new.decode_noalloc_async(0, pos, Kd[pos].data_ptr(), Vd[pos].data_ptr(), nh, scale,
                                 qd.data_ptr(), out_new.data_ptr())
        torch.cuda.synchronize()
        a, b = out_new.cpu().numpy(), out_ref.cpu().numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"call {call} output bits"
        assert new.n_seen == ref.n_seen == ctx
        for n in stores(dtype, window, n_sink):
            assert np.array_equal(new.export(n, 0).view(np.uint8), ref.export(n, 0).view(np.uint8)), n
        if window:
            want = o.attend_ring(0, pos, q, K[pos], V[pos], nh, np.float32(scale), n_threads=8)
        else:
            o.append(0, pos, K[pos], V[pos])
            want = o.attend(0, pos, q, nh, np.float32(scale), n_threads=8)
        assert_close(a, want, what=f"noalloc call {call} vs oracle")
        for kv in (ref, new, o):
            kv.close()


def test_noalloc_largest_plan():
    """The largest split plan a decode call can have: 4 kv heads x 64 splits
    = 256 workgroups of gqa 8 at hd 128, 1.06 MB of split records, within the
    scratch; bit-identical to dbi_kv_decode_async."""
    torch = pytest.importorskip("torch")
    nh, nkv, hd, ctx = 32, 4, 128, 8192
    P, Q = nkv * hd, nh * hd
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    rng = np.random.default_rng(1600)
    K = rng.standard_normal((ctx, P), dtype=np.float32)
    V = rng.standard_normal((ctx, P), dtype=np.float32)
    q = rng.standard_normal(Q, dtype=np.float32)
    ref = HipKV(1, ctx, nkv, hd)
    new = HipKV(1, ctx, nkv, hd)
    for kv in (ref, new):
        kv.append_n(0, 0, K[:-1], V[:-1])
    assert new.splits(ctx - 1, 1, nh) == 64
    Kd, Vd, qd = (torch.from_numpy(a).cuda() for a in (K, V, q))
    outs = [torch.full((Q,), float("nan"), device="cuda") for _ in range(2)]
    stream = torch.cuda.current_stream()
    for kv in (ref, new):
        kv.set_stream(stream.cuda_stream)
    torch.cuda.synchronize()
    pos = ctx - 1
    ref.decode_async(0, pos, Kd[pos].data_ptr(), Vd[pos].data_ptr(), nh, scale, qd.data_ptr(),
                     outs[0].data_ptr())
    new.decode_noalloc_async(0, pos, Kd[pos].data_ptr(), Vd[pos].data_ptr(), nh, scale,
                             qd.data_ptr(), outs[1].data_ptr())
    torch.cuda.synchronize()
    a, b = outs[1].cpu().numpy(), outs[0].cpu().numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    for kv in (ref, new):
        kv.close()


def test_noalloc_captured_on_fresh_handle():
    """The allocation-free step needs no eager warm-up: on a handle that has
    never attended, a call at config 3's 32-split plan is captured into a HIP
    graph (a workspace growth would be refused under capture), and every
    replay equals dbi_kv_decode_async on a twin handle bit for bit."""
    torch = pytest.importorskip("torch")
    nh, nkv, hd, n_sink, ctx = 24, 8, 128, 4, 8192
    P, Q = nkv * hd, nh * hd
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    rng = np.random.default_rng(1700)
    K = rng.standard_normal((ctx, P), dtype=np.float32)
    V = rng.standard_normal((ctx, P), dtype=np.float32)
    q = rng.standard_normal(Q, dtype=np.float32)
    ref = HipKV(1, ctx, nkv, hd, n_sink, 0, INT8, 1e6)
    new = HipKV(1, ctx, nkv, hd, n_sink, 0, INT8, 1e6)
    for kv in (ref, new):
        kv.append_n(0, 0, K[:-1], V[:-1])
    assert new.splits(ctx - 1, 1, nh) == 32
    Kd, Vd, qd = (torch.from_numpy(a).cuda() for a in (K, V, q))
    out_ref = torch.full((Q,), float("nan"), device="cuda")
    out_new = torch.full((Q,), float("nan"), device="cuda")
    pos = ctx - 1
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    new.set_stream(s.cuda_stream)
    with torch.cuda.graph(graph, stream=s):
        new.decode_noalloc_async(0, pos, Kd[pos].data_ptr(), Vd[pos].data_ptr(), nh, scale,
                                 qd.data_ptr(), out_new.data_ptr())
    torch.cuda.synchronize()
    ref.set_stream(torch.cuda.current_stream().cuda_stream)
    ref.decode_async(0, pos, Kd[pos].data_ptr(), Vd[pos].data_ptr(), nh, scale, qd.data_ptr(),
                     out_ref.data_ptr())
    torch.cuda.synchronize()
    want = out_ref.cpu().numpy().view(np.uint32)
    for rep in range(3):
        out_new.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out_new.cpu().numpy().view(np.uint32), want), f"replay {rep}"
    for n in stores(INT8, 0, n_sink):
        assert np.array_equal(new.export(n, 0).view(np.uint8), ref.export(n, 0).view(np.uint8)), n
    del graph
    for kv in (ref, new):
        kv.close()
