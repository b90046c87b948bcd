"""Graph capture of the decode step (append + attention of every layer), as
bench.py replays it: every replay, with eager work and synchronizations in
between, must give the eager result bit for bit (each launch leaves the
split-K counters ready for the next; no memset node is recorded)."""
import numpy as np
import pytest

from dbinfer_amd.kv import F32, INT8, HipKV

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,n_sink,window", [(INT8, 4, 0), (F32, 0, 0), (INT8, 4, 64),
                                                 (F32, 4, 64)])
def test_graph_replay_matches_eager(dtype, n_sink, window):
    torch = pytest.importorskip("torch")
    L, nh, nkv, hd, ctx = 3, 24, 8, 128, 2000
    pos = ctx - 1
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        g = torch.Generator(device="cuda")
        g.manual_seed(5)
        K = torch.randn(L, ctx, nkv * hd, device="cuda", generator=g)
        V = torch.randn(L, ctx, nkv * hd, device="cuda", generator=g)
        q = torch.randn(L, nh * hd, device="cuda", generator=g)
        kv = HipKV(L, ctx, nkv, hd, n_sink, window, dtype, 1e6)
        kv.set_stream(stream.cuda_stream)
        for l in range(L):
            kv.append_async(l, 0, ctx - 1, K[l].data_ptr(), V[l].data_ptr())
        out = torch.zeros(L, nh * hd, device="cuda")

        def step():
            for l in range(L):
                kv.append_async(l, pos, 1, K[l, pos].data_ptr(), V[l, pos].data_ptr())
                kv.attend_async(l, pos, nh, scale, q[l].data_ptr(), out[l].data_ptr())

        step()
        torch.cuda.synchronize()
        eager = out.clone()
        graph = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream()
        cap.wait_stream(stream)
        with torch.cuda.graph(graph, stream=cap):
            kv.set_stream(cap.cuda_stream)
            step()
        kv.set_stream(stream.cuda_stream)
        torch.cuda.synchronize()
        for r in range(4):
            out.zero_()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"replay {r}"
            # eager work between replays, on the same cache
            other = torch.empty_like(out)
            kv.attend_async(0, pos, nh, scale, q[1].data_ptr(), other[0].data_ptr())
            torch.cuda.synchronize()
        kv.close()


@pytest.mark.parametrize("dtype,n_sink,window,misalign", [
    (INT8, 4, 0, 0), (F32, 0, 0, 0), (INT8, 4, 64, 0), (F32, 4, 64, 0),
    (INT8, 4, 0, 1),  # rows 4 bytes off 16-byte alignment: append kernel, then attention
    (F32, 4, 64, 1),
])
def test_fused_step_graph_matches_separate(dtype, n_sink, window, misalign):
    """The fused decode step (dbi_kv_decode_async, device rows) against the
    separate append + attention calls bit for bit, eager and over graph
    replays (the step is idempotent at a fixed position), and the stored
    arrays equal afterwards."""
    torch = pytest.importorskip("torch")
    L, nh, nkv, hd, ctx = 2, 24, 8, 128, 1500
    P, pos = nkv * hd, ctx - 1
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        g = torch.Generator(device="cuda")
        g.manual_seed(11)
        kflat = torch.randn(L * ctx * P + 1, device="cuda", generator=g)
        vflat = torch.randn(L * ctx * P + 1, device="cuda", generator=g)
        K = kflat[misalign:misalign + L * ctx * P].view(L, ctx, P)
        V = vflat[misalign:misalign + L * ctx * P].view(L, ctx, P)
        q = torch.randn(L, nh * hd, device="cuda", generator=g)
        kv = HipKV(L, ctx, nkv, hd, n_sink, window, dtype, 1e6)
        sep = HipKV(L, ctx, nkv, hd, n_sink, window, dtype, 1e6)
        for h in (kv, sep):
            h.set_stream(stream.cuda_stream)
            for l in range(L):
                h.append_async(l, 0, pos, K[l].data_ptr(), V[l].data_ptr())
        out = torch.zeros(L, nh * hd, device="cuda")
        ref = torch.zeros(L, nh * hd, device="cuda")
        for l in range(L):
            sep.append_async(l, pos, 1, K[l, pos].data_ptr(), V[l, pos].data_ptr())
            sep.attend_async(l, pos, nh, scale, q[l].data_ptr(), ref[l].data_ptr())

        def step():
            for l in range(L):
                kv.decode_async(l, pos, K[l, pos].data_ptr(), V[l, pos].data_ptr(), nh, scale,
                                q[l].data_ptr(), out[l].data_ptr())

        step()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), "eager fused step vs separate calls"
        graph = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream()
        cap.wait_stream(stream)
        with torch.cuda.graph(graph, stream=cap):
            kv.set_stream(cap.cuda_stream)
            step()
        kv.set_stream(stream.cuda_stream)
        torch.cuda.synchronize()
        for r in range(3):
            out.zero_()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, ref), f"replay {r}"
        names = (["k8", "v8", "k_scale", "v_scale"] + ([] if window else ["k_raw"])
                 if dtype == INT8 else ["k", "v"])
        for l in range(L):
            for n in names:
                a, b = kv.export(n, l), sep.export(n, l)
                assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), f"{n} layer {l}"
        kv.close()
        sep.close()


@pytest.mark.parametrize("dtype", [INT8, F32])
def test_split_merge_is_stable_under_load(dtype):
    """The split merge runs in the last workgroup to arrive, reading the other
    splits' records at device coherence. The merge order is fixed, so every
    call must give the same bits whichever workgroup merges: 60 back-to-back
    rounds over 28 layers at the config-3 shape (256 workgroups per call, the
    full-load case) all equal the first round."""
    torch = pytest.importorskip("torch")
    L, nh, nkv, hd, ctx = 28, 24, 8, 128, 4096
    pos = ctx - 1
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        g = torch.Generator(device="cuda")
        g.manual_seed(21)
        K = torch.randn(ctx, nkv * hd, device="cuda", generator=g)
        V = torch.randn(ctx, nkv * hd, device="cuda", generator=g)
        q = torch.randn(L, nh * hd, device="cuda", generator=g)
        kv = HipKV(L, ctx, nkv, hd, 4 if dtype == INT8 else 0, 0, dtype, 1e6)
        kv.set_stream(stream.cuda_stream)
        for l in range(L):
            kv.append_async(l, 0, ctx, K.data_ptr(), V.data_ptr())
        rounds = 60
        out = torch.zeros(rounds, L, nh * hd, device="cuda")
        for r in range(rounds):
            for l in range(L):
                kv.attend_async(l, pos, nh, scale, q[l].data_ptr(), out[r, l].data_ptr())
        torch.cuda.synchronize()
        first = out[0]
        assert torch.isfinite(first).all()
        bad = [r for r in range(1, rounds) if not torch.equal(out[r], first)]
        assert not bad, f"rounds differing from the first: {bad[:10]}"
        kv.close()


@pytest.mark.parametrize("dtype,n_sink,window,bias", [(INT8, 4, 0, False), (F32, 0, 0, True),
                                                      (INT8, 4, 64, True)])
def test_producer_step_graph_replay(dtype, n_sink, window, bias):
    """dbi_kv_decode_qkv_async (raw projections; bias and rope inside the
    attention launch) captured for every layer: each replay, with eager work
    in between, equals the eager step bit for bit."""
    torch = pytest.importorskip("torch")
    L, nh, nkv, hd, ctx = 2, 24, 8, 128, 1200
    P, pos = nkv * hd, ctx - 1
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        g = torch.Generator(device="cuda")
        g.manual_seed(13)
        K = torch.randn(L, ctx, P, device="cuda", generator=g)
        V = torch.randn(L, ctx, P, device="cuda", generator=g)
        q = torch.randn(L, nh * hd, device="cuda", generator=g)
        b = torch.randn(L, nh * hd + 2 * P, device="cuda", generator=g)
        kv = HipKV(L, ctx, nkv, hd, n_sink, window, dtype, 1e6)
        kv.set_stream(stream.cuda_stream)
        for l in range(L):
            kv.append_async(l, 0, pos, K[l].data_ptr(), V[l].data_ptr())
        out = torch.zeros(L, nh * hd, device="cuda")

        def bp(l):
            if not bias:
                return [None] * 3
            return [b[l, :nh * hd].data_ptr(), b[l, nh * hd:nh * hd + P].data_ptr(),
                    b[l, nh * hd + P:].data_ptr()]

        def step():
            for l in range(L):
                kv.decode_qkv_async(l, pos, nh, scale, q[l].data_ptr(), K[l, pos].data_ptr(),
                                    V[l, pos].data_ptr(), *bp(l), out[l].data_ptr())

        step()  # the first producer call builds the rope table (not under capture)
        torch.cuda.synchronize()
        eager = out.clone()
        graph = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream()
        cap.wait_stream(stream)
        with torch.cuda.graph(graph, stream=cap):
            kv.set_stream(cap.cuda_stream)
            step()
        kv.set_stream(stream.cuda_stream)
        torch.cuda.synchronize()
        for r in range(4):
            out.zero_()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"replay {r}"
            other = torch.empty_like(out)
            kv.attend_async(0, pos, nh, scale, q[1].data_ptr(), other[0].data_ptr())
            torch.cuda.synchronize()
        kv.close()


@pytest.mark.parametrize("dtype,nh,nkv,hd,pos0,n", [
    (F32, 32, 8, 64, 1792, 256),   # prefill kernel, 4 key splits and the merge launch
    (F32, 32, 8, 128, 1500, 5),    # fp32 rows kernel and its merge launch
    (INT8, 32, 8, 128, 1500, 5),   # int8 rows kernel: remainder tile, sinks in the merge
])
def test_chunk_graph_replay_matches_eager(dtype, nh, nkv, hd, pos0, n):
    """Chunk calls captured in a graph (the bench's chunk timing): every
    replay, with eager chunk calls on the same workspace in between, gives
    the eager result bit for bit."""
    torch = pytest.importorskip("torch")
    L, cap_pos = 2, pos0 + n
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        g = torch.Generator(device="cuda")
        g.manual_seed(11)
        K = torch.randn(L, cap_pos, nkv * hd, device="cuda", generator=g)
        V = torch.randn(L, cap_pos, nkv * hd, device="cuda", generator=g)
        q = torch.randn(L, n * nh * hd, device="cuda", generator=g)
        q2 = torch.randn(n * nh * hd, device="cuda", generator=g)
        kv = HipKV(L, cap_pos, nkv, hd, 4, 0, dtype, 1e6)
        kv.set_stream(stream.cuda_stream)
        for l in range(L):
            kv.append_async(l, 0, cap_pos, K[l].data_ptr(), V[l].data_ptr())
        out = torch.zeros(L, n * nh * hd, device="cuda")

        def chunk():
            for l in range(L):
                kv.attend_chunk_async(l, pos0, n, nh, scale, q[l].data_ptr(), out[l].data_ptr())

        chunk()
        torch.cuda.synchronize()
        eager = out.clone()
        graph = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream()
        cap.wait_stream(stream)
        with torch.cuda.graph(graph, stream=cap):
            kv.set_stream(cap.cuda_stream)
            chunk()
        kv.set_stream(stream.cuda_stream)
        torch.cuda.synchronize()
        for r in range(4):
            out.zero_()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"replay {r}"
            other = torch.empty_like(q2)
            kv.attend_chunk_async(1, pos0, n, nh, scale, q2.data_ptr(), other.data_ptr())
            torch.cuda.synchronize()
        kv.close()
