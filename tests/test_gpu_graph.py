"""Graph capture of the decode step (append + attention of every layer), as
bench.py replays it: every replay, with eager work and synchronizations in
between, must give the eager result bit for bit (the split-K counters reset
themselves; no memset node is recorded)."""
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
