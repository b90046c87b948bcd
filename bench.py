"""Benchmark of the KV-cache decode hot path on one MI355X.

Workload (BASELINE.json metric, quoted at 8k context): the Llama-3.2-3B
attention shape of config 3 -- 28 layers, 24 query / 8 kv heads, head_dim
128 -- with the dense int8 cache (per-channel K over 32-token groups,
per-block V, 4 fp32 sinks) holding 8192 positions of synthetic N(0,1) keys
and values with 1% outlier channels x8. One step decodes one token through
all 28 layers: per layer, quantize-on-append at position 8191 then GQA decode
attention over the 8192 resident keys (dbi_kv_decode: one kernel, split-K
over the keys, the last split to finish merges). Inputs (q, k, v) are
resident in HBM before the timed region; the step is replayed from a HIP
graph.

The same step over the fp32 cache of that shape (the reference point of
BASELINE.md) is reported beside it. The working sets (529 MB int8, 1.9 GB
fp32) exceed the 256 MB MALL, so each layer's KV is re-read from HBM.

Printed: one JSON line (rank 0) with value = algorithmic HBM GB/s of the
int8 step, the per-layer microseconds, the roofline of the dominant kernel
(int8 decode attention) and the CPU oracle baseline.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "GQA decode attn µs/token/layer + achieved HBM GB/s at 8k ctx, int8 & fp32 KV"
PEAK_GBS = 8000.0  # MI355X HBM3E vendor peak

L, NH, NKV, HD, CTX, NSINK = 28, 24, 8, 128, 8192, 4
POS = CTX - 1


def attn_bytes(dtype: str, n: int = CTX, s: int = NSINK) -> int:
    """Algorithmic HBM bytes of one decode-attention call of one layer."""
    P = NKV * HD
    nb = (HD + 31) // 32
    if dtype == "f32":
        return 2 * n * P * 4
    return (2 * (n - s) * P + -(-n // 32) * P * 4 + (n - s) * NKV * nb * 4 + 2 * s * P * 4)


def make_inputs(torch, seed: int):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    P = NKV * HD
    K = torch.randn(L, CTX, P, device="cuda", generator=g)
    V = torch.randn(L, CTX, P, device="cuda", generator=g)
    # 1% outlier channels x8, a seeded choice per layer shared by K and V
    rng = np.random.default_rng(seed)
    for layer in range(L):
        ch = torch.as_tensor(rng.choice(P, round(0.01 * P), replace=False), device="cuda")
        K[layer, :, ch] *= 8.0
        V[layer, :, ch] *= 8.0
    q = torch.randn(L, NH * HD, device="cuda", generator=g)
    return K, V, q


def build_cache(torch, HipKV, dtype_code, K, V):
    kv = HipKV(L, CTX, NKV, HD, n_sink=NSINK, dtype=dtype_code)
    kv.set_stream(torch.cuda.current_stream().cuda_stream)
    for layer in range(L):
        kv.append_async(layer, 0, CTX, K[layer].data_ptr(), V[layer].data_ptr())
    torch.cuda.synchronize()
    return kv


def step(kv, K, V, q, out, scale, attention_only=False):
    """One decode token through all layers: per layer the fused decode step
    (quantize-on-append at POS + attention, one kernel);
    attention_only leaves the cache as it is and times the attention call."""
    for layer in range(L):
        if attention_only:
            kv.attend_async(layer, POS, NH, scale, q[layer].data_ptr(), out[layer].data_ptr())
        else:
            kv.decode_async(layer, POS, K[layer, POS].data_ptr(), V[layer, POS].data_ptr(), NH,
                            scale, q[layer].data_ptr(), out[layer].data_ptr())


def capture(torch, fn):
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn(s)  # warm-up on the capture stream (workspace allocation happens here)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        fn(s)
    torch.cuda.synchronize()
    return g


def time_graph(torch, g, reps: int) -> float:
    """ms per replay, HIP events on the replay stream."""
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record()
    for _ in range(reps):
        g.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def eager_kernel_us(torch, kv, q, out, scale, reps: int) -> float:
    """Average duration of one decode-attention launch: an event pair around
    every launch on the kernel's own stream, layers rotated."""
    pairs = []
    for r in range(reps):
        for layer in range(L):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            kv.attend_async(layer, POS, NH, scale, q[layer].data_ptr(), out[layer].data_ptr())
            b.record()
            pairs.append((a, b))
    torch.cuda.synchronize()
    return 1000.0 * statistics.median(a.elapsed_time(b) for a, b in pairs)


def kernel_name(name: str, splits: int) -> str:
    """The decode kernel instance a call at POS runs (attention.hip's plan:
    chunks of 32 positions for int8, 16 for fp32, split over 8 waves)."""
    G = NH // NKV
    chunk = 32 if name == "int8" else 16
    per_split = -(-(-(-CTX // chunk)) // splits)
    per_wave = -(-per_split // 8)
    cpw = 1 if per_wave <= 1 else 2 if per_wave <= 2 else 4 if per_wave <= 4 else 0
    if name == "int8":
        return f"attn_i8_kernel<{HD},{G},false,{cpw},1>"
    return f"attn_kernel<{HD},{G},0,false,{cpw}>"


def measure(torch, HipKV, code, name, K, V, q, args, scale):
    kv = build_cache(torch, HipKV, code, K, V)
    out = torch.empty(L, NH * HD, device="cuda")
    res = {}

    def full(s):
        kv.set_stream(s.cuda_stream)
        step(kv, K, V, q, out, scale)

    def attn_only(s):
        kv.set_stream(s.cuda_stream)
        step(kv, K, V, q, out, scale, attention_only=True)

    g_full = capture(torch, full)
    g_attn = capture(torch, attn_only)
    for _ in range(args.warmup):
        g_full.replay()
    torch.cuda.synchronize()
    ms = time_graph(torch, g_full, args.steps)
    res["ms_per_step"] = ms
    res["us_per_token_layer"] = 1000.0 * ms / L
    res["step_gbs"] = attn_bytes(name) * L / (ms * 1e-3) / 1e9
    ms_attn = time_graph(torch, g_attn, args.steps)
    res["attn_us_graph"] = 1000.0 * ms_attn / L
    kv.set_stream(torch.cuda.current_stream().cuda_stream)
    res["attn_us_events"] = eager_kernel_us(torch, kv, q, out, scale, max(2, args.steps // 20))
    res["attn_bytes"] = attn_bytes(name)
    res["kernel"] = kernel_name(name, kv.splits(POS, 1, NH))
    kv.close()
    del g_full, g_attn
    torch.cuda.synchronize()
    return res


def host_threads():
    """(cores this process may run on, threads the CPU baseline uses): every
    core of the job's share. A GPU box allots each GPU a host share and says
    so in OMP_NUM_THREADS (16 per GPU); elsewhere the affinity mask is the
    share."""
    nproc = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS", "")
    share = int(env) if env.isdigit() and int(env) > 0 else nproc
    return nproc, min(nproc, share)


def cpu_baseline(budget_s: float):
    """The CPU oracle (the reference's KVCache::append + attend_dense_int8
    restated, head-parallel like its thread pool; built -O3
    -ffp-contract=off) on the same decode step: per layer, quantize-on-append
    at POS then attention over CTX keys, over CPU_LAYERS layers of a seeded
    cache of the same shape (filling all L layers through the reference's
    per-append group requantization alone takes ~30 s of CPU). Timed on all
    cores of the host share and on 1 core, each the median of >= 5 steps
    (half the budget each); the result is per token and layer."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle  # checker / baseline only

    nproc, threads = host_threads()
    rng = np.random.default_rng(7)
    P = NKV * HD
    nl = CPU_LAYERS
    kv = pyoracle.OracleKV(nl, CTX, NKV, HD, n_sink=NSINK, dtype=pyoracle.INT8)
    t0 = time.perf_counter()
    rows = []
    for layer in range(nl):
        K = rng.standard_normal((CTX, P), dtype=np.float32)
        V = rng.standard_normal((CTX, P), dtype=np.float32)
        ch = rng.choice(P, round(0.01 * P), replace=False)
        K[:, ch] *= 8
        V[:, ch] *= 8
        kv.append_n(layer, 0, K, V)
        rows.append((K[POS].copy(), V[POS].copy()))
    fill_s = time.perf_counter() - t0
    q = rng.standard_normal((nl, NH * HD), dtype=np.float32)
    scale = np.float32(1.0) / np.sqrt(np.float32(HD))
    def timed(n_threads, budget):
        steps = []
        t_end = time.perf_counter() + budget
        while len(steps) < 5 or time.perf_counter() < t_end:
            t = time.perf_counter()
            for layer in range(nl):
                kv.append(layer, POS, rows[layer][0], rows[layer][1])
                kv.attend(layer, POS, q[layer], NH, scale, n_threads=n_threads)
            steps.append(time.perf_counter() - t)
        return statistics.median(steps) / nl, len(steps)

    med, n_all = timed(threads, budget_s / 2)
    med1, n_one = timed(1, budget_s / 2)
    kv.close()
    return {
        "value": round(1e6 * med, 3),
        "unit": "us/token/layer",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle append + attend_dense_int8 decode step at pos {POS} over {nl} of the {L} "
                   f"layers (ctx {CTX}, 24q/8kv, hd 128, 4 sinks), median of {n_all} steps on "
                   f"{threads} threads and of {n_one} on 1 thread, ~{budget_s / 2:.0f}s each; "
                   f"cache filled in {fill_s:.1f}s"),
        "value_1core": round(1e6 * med1, 3),
        "nproc": nproc,
        "gbs_equiv": round(attn_bytes("int8") / med / 1e9, 3),
        "cpu_model": _cpu_model(),
    }


CPU_LAYERS = 4
PROFILE = "profiles/decode_c3_ctx8192_kernels.md"


def _profiled(key):
    """A figure of the committed rocprofv3 summary (PMC counters cannot be read
    in-process): `key: value` lines of PROFILE."""
    try:
        for line in open(os.path.join(ROOT, PROFILE)):
            if line.startswith(key + ":"):
                return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def _profiled_traffic():
    """HBM bytes of one int8 decode-attention call from the FETCH_SIZE/WRITE_SIZE
    passes of PROFILE."""
    t = _profiled("traffic_bytes_per_call_int8")
    return None if t is None else int(t)


# The five benchmark configurations, one decode step (and, where the config has them, the
# prefill chunk / verify round) per config; bench.py --configs
CONFIGS = [
    # name, layers, nh, nkv, hd, dtype, n_sink, window, position decoded, chunk rows
    ("C1 TinyLlama", 22, 32, 4, 64, "f32", 0, 0, 1024, 0),
    ("C2 Llama-3.2-1B", 16, 32, 8, 64, "f32", 0, 0, 4095, 256),
    ("C3 Llama-3.2-3B int8", 28, 24, 8, 128, "int8", 4, 0, 8191, 0),
    ("C3 Llama-3.2-3B fp32", 28, 24, 8, 128, "f32", 0, 0, 8191, 0),
    ("C4 Qwen2.5-7B ring fp32", 28, 28, 4, 128, "f32", 4, 4096, 32767, 0),
    ("C4 Qwen2.5-7B ring int8", 28, 28, 4, 128, "int8", 4, 4096, 32767, 0),
    ("C5 Qwen3-8B fp32", 36, 32, 8, 128, "f32", 0, 0, 16383, 5),
    ("C5 Qwen3-8B int8", 36, 32, 8, 128, "int8", 4, 0, 16383, 5),
]


def config_bytes(dtype, nkv, hd, n, s, ring):
    """Algorithmic HBM bytes of one decode-attention call (n keys or
    residents, s fp32 sinks of the dense int8 layout)."""
    P = nkv * hd
    nb = (hd + 31) // 32
    if dtype == "f32":
        return 2 * n * P * 4
    if ring:
        return 2 * n * P + 2 * n * nkv * nb * 4
    return 2 * (n - s) * P + -(-n // 32) * P * 4 + (n - s) * nkv * nb * 4 + 2 * s * P * 4


def run_configs(torch, HipKV, F32, INT8, args):
    """One JSON line per config: the fused decode step per layer (graph
    replay), its algorithmic GB/s, and the chunk rows of C2 (the last 256-row
    prefill chunk of the 2048-token prompt) and C5 (a 5-row verify round)."""
    for (name, L_, nh, nkv, hd, dt, ns, win, pos, rows) in CONFIGS:
        scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
        P = nkv * hd
        n_fill = pos + 1 if not win else pos + 1
        stream = torch.cuda.Stream()
        res = {"config": name, "layers": L_, "n_heads": nh, "n_kv_heads": nkv, "head_dim": hd,
               "kv": dt + (" ring %d+%d" % (ns, win) if win else (" dense, %d sinks" % ns if ns
                                                                   else " dense"))}
        with torch.cuda.stream(stream):
            g = torch.Generator(device="cuda")
            g.manual_seed(77)
            K = torch.randn(n_fill, P, device="cuda", generator=g)
            V = torch.randn(n_fill, P, device="cuda", generator=g)
            q = torch.randn(L_, max(rows, 1) * nh * hd, device="cuda", generator=g)
            out = torch.empty_like(q)
            kv = HipKV(L_, pos + 1 if not win else 1, nkv, hd, ns, win,
                       INT8 if dt == "int8" else F32, 1e6)
            kv.set_stream(stream.cuda_stream)
            for layer in range(L_):
                kv.append_async(layer, 0, pos, K.data_ptr(), V.data_ptr())
            torch.cuda.synchronize()

            def step(s_):
                kv.set_stream(s_.cuda_stream)
                for layer in range(L_):
                    kv.decode_async(layer, pos, K[pos].data_ptr(), V[pos].data_ptr(), nh, scale,
                                    q[layer].data_ptr(), out[layer].data_ptr())

            gr = capture(torch, step)
            for _ in range(5):
                gr.replay()
            ms = time_graph(torch, gr, args.config_steps)
            n_keys = min(pos + 1, ns + win) if win else pos + 1
            byts = config_bytes(dt, nkv, hd, n_keys, 0 if win else ns, bool(win))
            us = 1000.0 * ms / L_
            res.update({"decode_pos": pos, "keys": n_keys, "us_per_token_layer": round(us, 3),
                        "bytes_per_call": byts, "GBs": round(byts / (us * 1e-6) / 1e9, 1),
                        "frac_of_peak": round(byts / (us * 1e-6) / 1e9 / PEAK_GBS, 4),
                        "working_set_MB": round(L_ * byts / 1e6, 1)})
            del gr
            # the same step from raw projections: bias (Qwen2.5, C4) and rope
            # on the device, then the fused step (dbi_kv_decode_qkv_async)
            bias = torch.randn(nh * hd + 2 * P, device="cuda", generator=g) if win else None
            bp = ([bias[:nh * hd].data_ptr(), bias[nh * hd:nh * hd + P].data_ptr(),
                   bias[nh * hd + P:].data_ptr()] if bias is not None else [None] * 3)

            def pstep(s_):
                kv.set_stream(s_.cuda_stream)
                for layer in range(L_):
                    kv.decode_qkv_async(layer, pos, nh, scale, q[layer].data_ptr(),
                                        K[pos].data_ptr(), V[pos].data_ptr(), *bp,
                                        out[layer].data_ptr())

            gp = capture(torch, pstep)  # its warm-up call builds the rope table
            for _ in range(5):
                gp.replay()
            usp = 1000.0 * time_graph(torch, gp, args.config_steps) / L_
            res.update({"producer_us_per_token_layer": round(usp, 3),
                        "producer_bias": bias is not None})
            del gp
            if name.startswith("C5"):  # fp32: DBKVCACH v1; int8: v2
                res["prefix_io"] = prefix_io(HipKV, INT8 if dt == "int8" else F32, ns, kv, L_,
                                             pos + 1, nkv, hd, 2048)
            if rows:
                pos0 = 1792 if rows == 256 else pos + 1 - rows
                kv.truncate(pos0 + rows)

                def chunk(s_):
                    kv.set_stream(s_.cuda_stream)
                    for layer in range(L_):
                        kv.attend_chunk_async(layer, pos0, rows, nh, scale, q[layer].data_ptr(),
                                              out[layer].data_ptr())

                gc = capture(torch, chunk)
                for _ in range(10):
                    gc.replay()
                msc = time_graph(torch, gc, max(3, args.config_steps))
                usc = 1000.0 * msc / L_
                flops = sum((pos0 + c + 1) * nh * hd * 4 for c in range(rows))
                res.update({"chunk_rows": rows, "chunk_pos0": pos0,
                            "chunk_us_per_layer": round(usc, 2),
                            "chunk_us_per_token_layer": round(usc / rows, 3),
                            "chunk_TFLOPs": round(flops / (usc * 1e-6) / 1e12, 3)})
                del gc
                if rows == 5:
                    res["verify_tokens"] = verify_tokens(torch, kv, rows - 1, g, args)
            kv.close()
            if args.configs_cpu:
                res["cpu"] = config_cpu(K, V, q, name, nh, nkv, hd, dt, ns, win, pos, rows, scale)
            del K, V, q, out
        torch.cuda.synchronize()
        print(json.dumps(res), flush=True)


VOCAB_QWEN3 = 151936


def verify_tokens(torch, kv, k, gen, args):
    """C5's verify round, token side: the argmax of the k+1 logit rows over
    Qwen3's vocabulary and the merge against the draft, one
    dbi_spec_verify_async launch (16 per graph replay); its algorithmic GB/s
    (the logits read once). With --configs-cpu, the oracle's argmax + merge of the
    same rows on the host beside it."""
    vocab = VOCAB_QWEN3
    logits = torch.randn(k + 1, vocab, device="cuda", generator=gen)
    draft = torch.zeros(k, dtype=torch.int32, device="cuda")
    ver = torch.zeros(k + 1, dtype=torch.int32, device="cuda")
    acc = torch.zeros(1, dtype=torch.int32, device="cuda")

    per_graph = 16  # back-to-back calls per replay: the launch of one graph is not timed

    def call(s_):
        kv.set_stream(s_.cuda_stream)
        for _ in range(per_graph):
            kv.spec_verify_async(k, vocab, logits.data_ptr(), draft.data_ptr(), ver.data_ptr(),
                                 acc.data_ptr())

    gv = capture(torch, call)
    for _ in range(5):
        gv.replay()
    us = 1000.0 * time_graph(torch, gv, args.config_steps) / per_graph
    del gv
    byts = (k + 1) * vocab * 4
    res = {"k": k, "vocab": vocab, "us": round(us, 3), "bytes": byts,
           "GBs": round(byts / (us * 1e-6) / 1e9, 1)}
    if args.configs_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import pyoracle  # checker / baseline only

        host = logits.cpu().numpy()
        d = draft.cpu().numpy()
        times = []
        for _ in range(20):
            t = time.perf_counter()
            want = [pyoracle.argmax(r) for r in host]
            pyoracle.spec_merge(d, want)
            times.append(time.perf_counter() - t)
        res["cpu_us"] = round(1e6 * statistics.median(times), 1)
        res["cpu_threads"] = 1
    return res


# (config, dim, n_heads * head_dim) of the output projection after attention
OPROJ_SHAPES = [("C1 TinyLlama", 2048, 2048), ("C3 Llama-3.2-3B", 3072, 3072),
                ("C4 Qwen2.5-7B", 3584, 3584), ("C5 Qwen3-8B", 4096, 4096)]


def run_oproj(torch, HipKV, args):
    """decode_layer's step after attention (model.cpp:773-774): the output
    projection of the attention row plus the residual add, fp32, f16, Q8_0
    and Q4_0 weights, one call per layer with the layer's own weights (graph
    replay), and its GB/s against the HBM peak (the weights are read once)."""
    from dbinfer_amd.kv import W_F16, W_F32, W_Q4_0, W_Q8_0

    kv = HipKV(1, 64, 1, 64)
    for name, dim, n_in in OPROJ_SHAPES:
        L_ = 16  # distinct weight matrices, so no call reads another's from cache
        for wname, wtype, dt, esz in (("f32", W_F32, torch.float32, 4),
                                      ("f16", W_F16, torch.float16, 2),
                                      ("q8_0", W_Q8_0, torch.uint8, 34 / 32),
                                      ("q4_0", W_Q4_0, torch.uint8, 18 / 32)):
            if wtype in (W_Q8_0, W_Q4_0):  # random codes, every block scale 2^-8
                bb = 34 if wtype == W_Q8_0 else 18
                w = torch.randint(0, 256, (L_, dim, n_in // 32, bb), dtype=torch.uint8,
                                  device="cuda")
                w[..., 0] = 0x00
                w[..., 1] = 0x1C
            else:
                w = (torch.randn(L_, dim, n_in, device="cuda") * 0.05).to(dt)
            attn = torch.randn(L_, n_in, device="cuda")
            x = torch.zeros(L_, dim, device="cuda")

            def call(s_):
                kv.set_stream(s_.cuda_stream)
                for layer in range(L_):
                    kv.oproj_residual_async(wtype, w[layer].data_ptr(), attn[layer].data_ptr(),
                                            x[layer].data_ptr(), dim, n_in)

            g = capture(torch, call)
            for _ in range(3):
                g.replay()
            us = 1000.0 * time_graph(torch, g, args.config_steps) / L_
            byts = int(dim * n_in * esz)
            print(json.dumps({"oproj": name, "weights": wname, "dim": dim, "in": n_in,
                              "us": round(us, 3), "weight_bytes": byts,
                              "GBs": round(byts / (us * 1e-6) / 1e9, 1),
                              "frac_of_peak": round(byts / (us * 1e-6) / 1e9 / PEAK_GBS, 4)}),
                  flush=True)
            del g, w, attn, x
    kv.close()


# Full-layer offload shapes: the configs' models, Q8_0
# weights (the reference's offload reads F16 / Q8_0 / Q4_0, backend.hpp:17-18)
LAYER_CONFIGS = [
    # name, layers, dim, ff, nh, nkv, hd, kv dtype, n_sink, position decoded, vocab
    ("Llama-3.2-3B (C3 model), int8 KV at 8k", 28, 3072, 8192, 24, 8, 128, "int8", 4, 8191,
     128256),
    ("Qwen2.5-7B (C4 model), dense fp32 KV at 4k", 28, 3584, 18944, 28, 4, 128, "f32", 0, 4095,
     152064),
]


def q8_weight(torch, out: int, n_in: int, gen):
    """Random Q8_0 blocks [out][n_in/32][34]: codes uniform in [-127, 127],
    every block scale f16(0.5 / sqrt(n_in) / 73), so a matvec's gain stays
    about 1/2 (no overflow through the layers)."""
    w = torch.randint(-127, 128, (out, n_in // 32, 34), dtype=torch.int8, device="cuda",
                      generator=gen).view(torch.uint8)
    sc = torch.full((out, n_in // 32), 0.5 / np.sqrt(n_in) / 73.0, dtype=torch.float16,
                    device="cuda")
    w[..., :2] = sc.view(torch.uint8).view(out, n_in // 32, 2)
    return w


def run_layer(torch, HipKV, F32, INT8, args):
    """The full-layer offload (dbi_decode_token_full_async): every layer of
    one token (rmsnorm, q/k/v, the fused produce + append + attention, o_proj,
    gate/up, silu*up, down) and the lm_head, replayed from a graph; per token
    its time and the algorithmic bytes it streams (the weights once, the
    layer's KV attention bytes) against the HBM peak."""
    from dbinfer_amd.kv import W_Q8_0

    for (name, L_, dim, ff, nh, nkv, hd, dt, ns, pos, vocab) in LAYER_CONFIGS:
        gen = torch.Generator(device="cuda")
        gen.manual_seed(9)
        stream = torch.cuda.Stream()
        with torch.cuda.stream(stream):
            qn, kvn = nh * hd, nkv * hd
            ws, layers = [], []
            for _ in range(L_):
                m = {"wq": q8_weight(torch, qn, dim, gen), "wk": q8_weight(torch, kvn, dim, gen),
                     "wv": q8_weight(torch, kvn, dim, gen), "wo": q8_weight(torch, dim, qn, gen),
                     "wgate": q8_weight(torch, ff, dim, gen), "wup": q8_weight(torch, ff, dim, gen),
                     "wdown": q8_weight(torch, dim, ff, gen)}
                ws.append(m)
            ones = torch.ones(dim, device="cuda")
            for m in ws:
                layers.append({"attn_norm": ones.data_ptr(), "ffn_norm": ones.data_ptr(),
                               **{k: (v.data_ptr(), W_Q8_0) for k, v in m.items()}})
            lm = q8_weight(torch, vocab, dim, gen)
            wbytes = sum(v.numel() for m in ws for v in m.values()) + lm.numel()
            kv = HipKV(L_, pos + 1, nkv, hd, ns, 0, INT8 if dt == "int8" else F32, 1e6)
            kv.set_stream(stream.cuda_stream)
            P = nkv * hd
            K = torch.randn(pos, P, device="cuda", generator=gen)
            V = torch.randn(pos, P, device="cuda", generator=gen)
            for layer in range(L_):
                kv.append_async(layer, 0, pos, K.data_ptr(), V.data_ptr())
            del K, V
            kv.offload_setup(dim, ff, nh, 1e-5, layers, ones.data_ptr(), (lm.data_ptr(), W_Q8_0),
                             vocab)
            x0 = torch.randn(dim, device="cuda", generator=gen)
            x = torch.empty_like(x0)
            logits = torch.empty(vocab, device="cuda")
            torch.cuda.synchronize()

            def step(s_):
                kv.set_stream(s_.cuda_stream)
                x.copy_(x0)
                kv.decode_token_full_async(x.data_ptr(), pos, logits.data_ptr())

            g = capture(torch, step)
            for _ in range(3):
                g.replay()
            ms = time_graph(torch, g, max(5, args.config_steps // 2))
            kvb = L_ * config_bytes(dt, nkv, hd, pos + 1, ns, False)
            tot = wbytes + kvb
            finite = bool(torch.isfinite(logits).all().item())
            print(json.dumps({"layer_offload": name, "layers": L_, "dim": dim, "ff": ff,
                              "n_heads": nh, "n_kv_heads": nkv, "weights": "q8_0",
                              "kv": dt, "pos": pos, "vocab": vocab,
                              "us_per_token": round(1000.0 * ms, 1),
                              "us_per_layer": round(1000.0 * ms / L_, 2),
                              "weight_bytes_per_token": int(wbytes), "kv_bytes_per_token": int(kvb),
                              "GBs": round(tot / (ms * 1e-3) / 1e9, 1),
                              "frac_of_peak": round(tot / (ms * 1e-3) / 1e9 / PEAK_GBS, 4),
                              "logits_finite": finite}), flush=True)
            del g
            kv.close()
            del ws, layers, lm
        torch.cuda.synchronize()


def run_ctx_sweep(torch, HipKV, F32, INT8, args):
    """Config 3's shape over the target context range (8k-32k): one JSON line
    per (context, KV dtype) with the fused decode step and the attention-only
    call per layer (graph replay over all 28 layers), their algorithmic GB/s
    and the fraction of the 8 TB/s HBM peak."""
    scale = float(np.float32(1.0) / np.sqrt(np.float32(HD)))
    P = NKV * HD
    for ctx in (8192, 16384, 32768):
        for name, code in (("int8", INT8), ("f32", F32)):
            stream = torch.cuda.Stream()
            with torch.cuda.stream(stream):
                g = torch.Generator(device="cuda")
                g.manual_seed(ctx)
                kv = HipKV(L, ctx, NKV, HD, n_sink=NSINK, dtype=code)
                kv.set_stream(stream.cuda_stream)
                rows = []
                for layer in range(L):  # one layer's K/V at a time (32k fp32: 268 MB each)
                    K = torch.randn(ctx, P, device="cuda", generator=g)
                    V = torch.randn(ctx, P, device="cuda", generator=g)
                    kv.append_async(layer, 0, ctx, K.data_ptr(), V.data_ptr())
                    rows.append((K[ctx - 1].clone(), V[ctx - 1].clone()))
                    torch.cuda.synchronize()
                    del K, V
                q = torch.randn(L, NH * HD, device="cuda", generator=g)
                out = torch.empty_like(q)
                pos = ctx - 1

                def full(s):
                    kv.set_stream(s.cuda_stream)
                    for layer in range(L):
                        kv.decode_async(layer, pos, rows[layer][0].data_ptr(),
                                        rows[layer][1].data_ptr(), NH, scale,
                                        q[layer].data_ptr(), out[layer].data_ptr())

                def attn(s):
                    kv.set_stream(s.cuda_stream)
                    for layer in range(L):
                        kv.attend_async(layer, pos, NH, scale, q[layer].data_ptr(),
                                        out[layer].data_ptr())

                res = {"sweep": "config 3 shape", "ctx": ctx, "kv": name,
                       "bytes_per_call": attn_bytes(name, ctx)}
                for key, fn in (("step", full), ("attn", attn)):
                    gr = capture(torch, fn)
                    for _ in range(5):
                        gr.replay()
                    us = 1000.0 * time_graph(torch, gr, args.config_steps) / L
                    gbs = attn_bytes(name, ctx) / (us * 1e-6) / 1e9
                    res.update({f"{key}_us_per_layer": round(us, 3), f"{key}_GBs": round(gbs, 1),
                                f"{key}_frac_of_peak": round(gbs / PEAK_GBS, 4)})
                    del gr
                kv.close()
                del rows, q, out
            torch.cuda.synchronize()
            print(json.dumps(res), flush=True)


def prefix_io(HipKV, code, n_sink, kv, L_, cap, nkv, hd, n_tok):
    """Config 5's prefix cache: save the first n_tok positions of every layer
    (fp32: a DBKVCACH v1 file, model.cpp:1023-1156; int8: the v2 file of
    codes, scales and sinks), then load it into a fresh cache of the same
    layout, timed end to end (device pack, PCIe, file)."""
    import tempfile

    tokens = np.arange(n_tok, dtype=np.int32)
    with tempfile.TemporaryDirectory(dir=os.environ.get("TMPDIR", "/tmp")) as d:
        path = os.path.join(d, "prefix.dbkv")
        t = time.perf_counter()
        kv.save_prefix(path, tokens)
        save_s = time.perf_counter() - t
        size = os.path.getsize(path)
        fresh = HipKV(L_, cap, nkv, hd, n_sink, 0, code, 1e6)
        t = time.perf_counter()
        n = fresh.load_prefix(path, tokens)
        load_s = time.perf_counter() - t
        fresh.close()
    assert n == n_tok
    return {"tokens": n_tok, "file_bytes": size, "save_ms": round(1e3 * save_s, 1),
            "load_ms": round(1e3 * load_s, 1), "save_GBs": round(size / save_s / 1e9, 2),
            "load_GBs": round(size / load_s / 1e9, 2)}


def config_cpu(K, V, q, name, nh, nkv, hd, dt, ns, win, pos, rows, scale):
    """The CPU oracle on one layer of the same config (head-parallel on the
    host share, and on 1 core): the decode step (append at pos + attention)
    and, for the chunk configs, the chunk attention; median of >= 5 runs
    (the 256-row chunk: 1)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle  # checker / baseline only

    nproc, threads = host_threads()
    Kh = K.cpu().numpy()
    Vh = V.cpu().numpy()
    qh = q[0].cpu().numpy()
    o = pyoracle.OracleKV(1, pos + 1 if not win else 1, nkv, hd, n_sink=ns, window=win,
                          dtype=pyoracle.INT8 if dt == "int8" else pyoracle.F32, rope_theta=1e6)
    t0 = time.perf_counter()
    o.append_n(0, 0, Kh[:pos], Vh[:pos])
    fill_s = time.perf_counter() - t0

    def med(fn, n=5):
        ts = []
        for _ in range(n):
            t = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t)
        return statistics.median(ts)

    def step_time(n_threads):
        if win:
            return med(lambda: o.attend_ring(0, pos, qh[: nh * hd], Kh[pos], Vh[pos], nh, scale,
                                             n_threads=n_threads))

        def step():
            o.append(0, pos, Kh[pos], Vh[pos])
            o.attend(0, pos, qh[: nh * hd], nh, scale, n_threads=n_threads)
        return med(step)

    step_s = step_time(threads)
    step1_s = step_time(1)
    out = {"us_per_token_layer": round(1e6 * step_s, 1), "threads": threads,
           "us_per_token_layer_1core": round(1e6 * step1_s, 1), "nproc": nproc,
           "cpu_model": _cpu_model(), "fill_s": round(fill_s, 2), "kind": "port"}
    if rows:
        pos0 = 1792 if rows == 256 else pos + 1 - rows
        if dt == "f32" and not win:
            chunk_s = med(lambda: o.attend_chunk(0, pos0, qh[: rows * nh * hd], nh, scale,
                                                 n_threads=threads), 1 if rows > 16 else 5)
            out["chunk_us"] = round(1e6 * chunk_s, 1)
    o.close()
    return out


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--configs", action="store_true",
                    help="instead of the bench line, one JSON line per benchmark config (C1-C5)")
    ap.add_argument("--config-steps", type=int, default=30)
    ap.add_argument("--configs-cpu", action="store_true",
                    help="with --configs: also time the CPU oracle on one layer of each config")
    ap.add_argument("--oproj", action="store_true",
                    help="time the output projection + residual add at the configs' shapes")
    ap.add_argument("--verify", action="store_true",
                    help="time the verify round's token side (argmax + merge) at C5's shape")
    ap.add_argument("--layer", action="store_true",
                    help="time the full-layer offload (decode_token_full) at the configs' models")
    ap.add_argument("--ctx-sweep", action="store_true",
                    help="instead of the bench line, config 3's shape at ctx 8k, 16k, 32k")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB (PMC calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the path shards by kv head with no exchange)", file=sys.stderr)
        sys.exit(2)

    import torch

    from dbinfer_amd.kv import F32, INT8, HipKV

    torch.cuda.set_device(0)
    if args.calibrate_copy_mib:
        n = args.calibrate_copy_mib * (1 << 20) // 4
        src = torch.ones(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration_copy_bytes": n * 4, "launches": 5}))
        return
    if args.configs:
        run_configs(torch, HipKV, F32, INT8, args)
        return
    if args.ctx_sweep:
        run_ctx_sweep(torch, HipKV, F32, INT8, args)
        return
    if args.oproj:
        run_oproj(torch, HipKV, args)
        return
    if args.layer:
        run_layer(torch, HipKV, F32, INT8, args)
        return
    if args.verify:
        # C5's verify round, token side, at k = 4 and 8 (Qwen3's vocabulary)
        kv = HipKV(1, 64, 1, 64)
        gen = torch.Generator(device="cuda")
        gen.manual_seed(5)
        for k in (4, 8):
            print(json.dumps({"config": "C5 verify tokens", **verify_tokens(torch, kv, k, gen,
                                                                             args)}), flush=True)
        kv.close()
        return
    scale = float(np.float32(1.0) / np.sqrt(np.float32(HD)))
    # every launch and event goes on one non-default stream (the kernels'
    # stream), so events bracket exactly the work they time
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        K, V, q = make_inputs(torch, 1234)
        i8 = measure(torch, HipKV, INT8, "int8", K, V, q, args, scale)
        f32 = measure(torch, HipKV, F32, "f32", K, V, q, args, scale)
        del K, V
    torch.cuda.synchronize()

    dom_us = i8["attn_us_graph"]
    achieved = i8["attn_bytes"] / (dom_us * 1e-6) / 1e9
    # the same kernel in the fused step that `value` times (append inside the
    # launch): its fraction with the attention's algorithmic bytes
    fused_us = i8["us_per_token_layer"]
    achieved_fused = i8["attn_bytes"] / (fused_us * 1e-6) / 1e9
    line = {
        "metric": METRIC,
        "value": round(i8["step_gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(i8["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,1) q/K/V, 1% outlier channels x8)",
        "config": {
            "workload": "config 3: Llama-3.2-3B attention shape, dense int8 KV (per-channel K, "
                        "per-block V, 4 fp32 sinks), decode step at ctx 8192 over 28 layers "
                        "(fused append + GQA decode attention per layer, HIP-graph replay)",
            "n_layers": L, "n_heads": NH, "n_kv_heads": NKV, "head_dim": HD, "ctx": CTX,
            "parallelism": "single GPU",
        },
        "us_per_token_layer": round(i8["us_per_token_layer"], 3),
        "attn_us_per_layer": round(dom_us, 3),
        "attn_us_per_layer_events": round(i8["attn_us_events"], 3),
        "fp32": {
            "us_per_token_layer": round(f32["us_per_token_layer"], 3),
            "attn_us_per_layer": round(f32["attn_us_graph"], 3),
            "attn_us_per_layer_events": round(f32["attn_us_events"], 3),
            "step_gbs": round(f32["step_gbs"], 2),
            "attn_gbs": round(f32["attn_bytes"] / (f32["attn_us_graph"] * 1e-6) / 1e9, 2),
            "frac_of_peak": round(f32["attn_bytes"] / (f32["attn_us_graph"] * 1e-6) / 1e9
                                  / PEAK_GBS, 4),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": i8["kernel"] + " (one decode-attention call, attention only)",
            "achieved": round(achieved, 2),
            "peak": PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_GBS, 4),
            "fused_step": {"kernel": i8["kernel"] + " with the append inside (what `value` "
                                                   "times)",
                           "us_per_launch": round(fused_us, 3),
                           "achieved": round(achieved_fused, 2),
                           "frac": round(achieved_fused / PEAK_GBS, 4)},
            "traffic": _profiled_traffic(),
            "traffic_source": PROFILE,
            # the traced duration of the profiled kernel beside the live one: a
            # kernel changed since the profile shows as a disagreement
            "traffic_profiled_us": _profiled("traced_attention_us_int8"),
            "traffic_profile_agrees": (
                None if _profiled("traced_attention_us_int8") is None else
                abs(dom_us - _profiled("traced_attention_us_int8"))
                <= 0.1 * _profiled("traced_attention_us_int8")),
            "bytes_per_launch": i8["attn_bytes"],
        },
        "cpu_baseline": None if args.no_cpu else cpu_baseline(args.cpu_seconds),
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
