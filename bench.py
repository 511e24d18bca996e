"""Benchmark of the int8 W8A8 linear on one MI355X.

Headline workload (the decode GEMV sweep): one step =
one int8 linear (per-token activation quantization + GEMV, bf16 out) for
every M in {1,4,8,16} x (K,N) in {(1024,3072),(3072,1024),(1024,2048),
(1024,151936)}: 16 linears. Every linear owns its own weight copy (656 MB in
total), so a weight is re-read only after >256 MB of other traffic and comes
from HBM, not the Infinity Cache.

  value    = algorithmic bytes of the 16 linears / wall time per step (GB/s),
             bytes per linear = N*K + 4N + 4*M*K + 2*M*N
  roofline = the GEMV kernel alone: its algorithmic bytes (N*K + 4N + M*K + 2*M*N)
             / its average launch duration, timed with HIP events on the stream
             it runs on, vs 8 TB/s
Also reported: each configs[1] shape alone, cold (a graph cycling over
weight copies that exceed the Infinity Cache); configs[0] (one linear,
M=16 K=1024 N=3072, f32 out) on the GPU beside the restated backend-cpu path
on this host; the prefill GEMM sweep (configs[2], each shape timed as one HIP
graph of back-to-back launches) in TOPS vs the 5.0 POPS int8
dense MFMA peak, an MFMA roof probe, and the CPU baselines timed on this host
on bounded samples: the restated backend-cpu decode path (OpenMP) for the
decode sweep, and for prefill (which backend-cpu has no int8 path for) that
GEMV in 32-row chunks plus an OpenMP tiled i32 GEMM.
"""
import argparse
import json
import os
import sys
import time
import traceback

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
DECODE_M = [1, 4, 8, 16]
DECODE_KN = [(1024, 3072), (3072, 1024), (1024, 2048), (1024, 151936)]
PREFILL_M = [512, 2048, 8192]
PREFILL_KN = [(1024, 3072), (3072, 1024), (4096, 11008), (4096, 4096)]


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--prefill-reps", type=int, default=10)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="bound on CPU-baseline work")
    ap.add_argument("--only", default="", help="profiling aid: 'decode', 'gemv', 'shapes', 'config0', 'prefill', "
                    "'quant', 'qwen3', 'dit', 'w4a8', 'moe', 'hbm' or 'copy' only")
    ap.add_argument("--no-quant", action="store_true")
    ap.add_argument("--no-qwen3", action="store_true")
    ap.add_argument("--no-dit", action="store_true")
    ap.add_argument("--no-w4a8", action="store_true")
    ap.add_argument("--no-moe", action="store_true")
    ap.add_argument("--qwen3-batch", type=int, default=0,
                    help="profiling aid: the qwen3 leg at this one batch (f32 KV) only")
    return ap.parse_args()


def gemv_bytes(m, k, n):
    return n * k + 4 * n + m * k + 2 * m * n


def linear_bytes(m, k, n):
    return n * k + 4 * n + 4 * m * k + 2 * m * n


def make_decode_set(torch, dev, gen):
    sets = []
    for m in DECODE_M:
        for k, n in DECODE_KN:
            w = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev, generator=gen)
            sw = torch.empty(n, device=dev).uniform_(0.002, 0.02, generator=gen)
            x = torch.randn(m, k, device=dev, generator=gen)
            sets.append(dict(m=m, k=k, n=n, wq=w.view(torch.int32), sw=sw, x=x,
                             sx=torch.empty(m, device=dev), xq=torch.empty(m, k // 4, dtype=torch.int32, device=dev),
                             out=torch.empty(m, n, dtype=torch.bfloat16, device=dev)))
    return sets


def check_sample(torch, s, out_dtype):
    """Correctness gate before timing: sampled outputs vs the oracle."""
    import numpy as np
    from oracle import oracle as o

    x = s["x"].cpu().numpy()
    sx = o.max_abs_row(x)
    xq = o.quant_pack(x, sx)
    assert (s["sx"].cpu().numpy() == sx).all()
    cols = np.unique(np.random.default_rng(0).integers(0, s["n"], 256))
    wq = s["wq"][torch.from_numpy(cols).to(s["wq"].device)].cpu().numpy().view(np.uint32)
    sw = s["sw"].cpu().numpy()[cols]
    want = o.epilogue(o.acc_exact(xq, wq), sx, sw, None, out_dtype)
    got = s["out"].cpu()
    got = (got.view(torch.int16).numpy().view(np.uint16) if out_dtype == "bf16" else got.numpy())[:, cols]
    assert (got == want).all(), f"bench correctness gate failed at m={s['m']} k={s['k']} n={s['n']}"


def bench_decode(torch, lib, sets, steps, warmup, gemv_only=False):
    """The decode step (16 linears) and, separately, the GEMV kernel alone.
    gemv_only: just the GEMV measurement (the workload profiles/ summarizes
    with rocprofv3, so its kernel average matches roofline.avg_launch_us)."""
    from brain_amd._lib import BH_OUT_BF16, check

    def linear(s):
        # bh_linear_i8: quantization fused into the GEMV where that is faster
        # (small m*K, narrow N), else quantize_rows + GEMV.
        sp = torch.cuda.current_stream().cuda_stream
        check(lib.bh_linear_i8(sp, s["x"].data_ptr(), s["wq"].data_ptr(), s["sw"].data_ptr(), None,
                               s["sx"].data_ptr(), s["xq"].data_ptr(), s["out"].data_ptr(), BH_OUT_BF16,
                               s["m"], s["k"], s["n"]))

    def gemv(s):
        sp = torch.cuda.current_stream().cuda_stream
        check(lib.bh_matmul_i8_gemv(sp, s["xq"].data_ptr(), s["wq"].data_ptr(), s["sx"].data_ptr(),
                                    s["sw"].data_ptr(), None, s["out"].data_ptr(), BH_OUT_BF16, s["m"],
                                    s["k"] // 4, s["n"]))

    def step():
        for s in sets:
            linear(s)

    if gemv_only:
        for s in sets:
            sp = torch.cuda.current_stream().cuda_stream
            check(lib.bh_quantize_rows(sp, s["x"].data_ptr(), s["m"], s["k"], s["sx"].data_ptr(), s["xq"].data_ptr()))
        step_ms = wall = 0.0
    else:
        step_ms, wall = timed_step(torch, step, sets, steps, warmup)
    return gemv_measure(torch, sets, gemv, steps, step_ms, wall)


def timed_step(torch, step, sets, steps, warmup):
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    for s in sets:
        check_sample(torch, s, "bf16")

    # One step = 16 linears (16-32 launches); captured once as a HIP graph so the
    # timed loop measures the GPU, not Python's launch rate.
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for s in sets:
        s["out"].zero_()
    graph.replay()
    torch.cuda.synchronize()
    for s in sets:
        check_sample(torch, s, "bf16")

    stream = torch.cuda.current_stream()
    # Timed region: K graph replays, events at both ends.
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    step_ms = e0.elapsed_time(e1) / steps
    for s in sets:
        check_sample(torch, s, "bf16")
    return step_ms, wall


def gemv_measure(torch, sets, gemv, steps, step_ms, wall):
    stream = torch.cuda.current_stream()

    # GEMV kernel duration: the step's 16 GEMV launches alone (activations
    # already quantized) captured as a second graph and replayed; events on the
    # replay stream bracket the replays, so the per-launch average counts the
    # kernel plus the dispatch gap to the next node. Every weight is re-read
    # only after the other 15 (656 MB in total), so every launch is cold.
    ggraph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(ggraph):
        for s in sets:
            gemv(s)
    ggraph.replay()
    torch.cuda.synchronize()
    reps = max(5, steps // 2)
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(reps):
        ggraph.replay()
    b.record(stream)
    torch.cuda.synchronize()
    mean_us = a.elapsed_time(b) * 1e3 / (reps * len(sets))
    mean_bytes = sum(gemv_bytes(s["m"], s["k"], s["n"]) for s in sets) / len(sets)
    step_bytes = sum(linear_bytes(s["m"], s["k"], s["n"]) for s in sets)
    return dict(step_ms=step_ms, wall=wall, step_bytes=step_bytes, gemv_mean_us=mean_us,
                gemv_mean_bytes=mean_bytes)


def graph_per_launch_us(torch, fns, reps=3):
    """One HIP graph of one launch per callable (each on its own weight
    copy), replayed `reps` times; microseconds per launch from HIP events on
    the replay stream."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for fn in fns:
            fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for fn in fns:
            fn()
    g.replay()
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    cur = torch.cuda.current_stream()
    a.record(cur)
    for _ in range(reps):
        g.replay()
    b.record(cur)
    torch.cuda.synchronize()
    del g
    return a.elapsed_time(b) * 1e3 / (reps * len(fns))


def cold_copies(torch, dev, gen, m, k, n, pool_bytes=512 << 20, max_copies=128):
    """Enough weight copies of one shape that a graph cycling through them
    reads every launch's weights from HBM (together above the 256 MB
    Infinity Cache)."""
    c = max(2, min(max_copies, -(-pool_bytes // (n * k))))
    ws = [torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev, generator=gen).view(torch.int32)
          for _ in range(c)]
    sw = torch.empty(n, device=dev).uniform_(0.002, 0.02, generator=gen)
    return ws, sw


def bench_decode_shapes(torch, lib, dev, gen):
    """Each configs[1] shape alone, cold: a graph of launches cycling over
    weight copies that together exceed the Infinity Cache (the GEMV alone on
    a pre-quantized activation, bf16 out)."""
    from brain_amd._lib import BH_OUT_BF16, check
    rows = []
    for m in DECODE_M:
        for k, n in DECODE_KN:
            ws, sw = cold_copies(torch, dev, gen, m, k, n)
            xq = torch.randint(-127, 128, (m, k), dtype=torch.int8, device=dev, generator=gen).view(torch.int32)
            sx = torch.empty(m, device=dev).uniform_(0.001, 0.05, generator=gen)
            out = torch.empty(m, n, dtype=torch.bfloat16, device=dev)

            def fn(w):
                return lambda: check(lib.bh_matmul_i8_gemv(torch.cuda.current_stream().cuda_stream, xq.data_ptr(),
                                                           w.data_ptr(), sx.data_ptr(), sw.data_ptr(), None,
                                                           out.data_ptr(), BH_OUT_BF16, m, k // 4, n))
            us = graph_per_launch_us(torch, [fn(w) for w in ws])
            gb = gemv_bytes(m, k, n)
            rows.append(dict(m=m, k=k, n=n, copies=len(ws), gemv_us=round(us, 2), gemv_gbs=round(gb / us / 1e3, 1),
                             frac=round(gb / us / 1e3 / HBM_PEAK_GBS, 3)))
            del ws
    return rows


def bench_config0(torch, lib, dev, gen, cpu=True, budget_s=5.0):
    """one int8 linear, M=16, K=1024, N=3072, f32 out (per-token
    quantization inside the call: bh_linear_i8), cold weights on the GPU;
    beside it the restated backend-cpu path (max_abs_row -> quant_pack ->
    matmul_i8_gemv, OpenMP over output columns) on this host, same shape."""
    from brain_amd._lib import BH_OUT_F32, check
    m, k, n = 16, 1024, 3072
    ws, sw = cold_copies(torch, dev, gen, m, k, n)
    x = torch.randn(m, k, device=dev, generator=gen)
    sx = torch.empty(m, device=dev)
    xq = torch.empty(m, k // 4, dtype=torch.int32, device=dev)
    out = torch.empty(m, n, device=dev)

    def fn(w):
        return lambda: check(lib.bh_linear_i8(torch.cuda.current_stream().cuda_stream, x.data_ptr(), w.data_ptr(),
                                              sw.data_ptr(), None, sx.data_ptr(), xq.data_ptr(), out.data_ptr(),
                                              BH_OUT_F32, m, k, n))
    us = graph_per_launch_us(torch, [fn(w) for w in ws])
    byts = linear_bytes(m, k, n) + 2 * m * n  # f32 out: 4 bytes per output
    res = {"workload": "configs[0]: int8 linear M=16 K=1024 N=3072, per-token quant + GEMV, f32 out",
           "gpu_us": round(us, 2), "gpu_gbs": round(byts / us / 1e3, 1), "copies": len(ws)}
    if cpu:
        import numpy as np
        from oracle import oracle as o
        threads = min(len(os.sched_getaffinity(0)), 16)
        wq, swh = o.synth_weights(n, k, 3)
        xh = o.synth_acts(m, k, 4)
        times = []
        t_start = time.perf_counter()
        while len(times) < 5 or (time.perf_counter() - t_start < budget_s and len(times) < 200):
            t0 = time.perf_counter()
            o.cpu_linear_gemv(xh, wq, swh, threads)
            times.append(time.perf_counter() - t0)
        t = sorted(times)[len(times) // 2] * 1e6
        res.update({"cpu_us": round(t, 1), "cpu_gbs": round(byts / t / 1e3, 2), "cpu_cores": threads,
                    "cpu_kind": "port", "cpu_sample": f"the same linear, {len(times)} runs, median",
                    "gpu_vs_cpu": round(t / us, 1)})
        del np
    del ws
    return res


def bench_prefill(torch, lib, dev, gen, reps):
    from brain_amd._lib import BH_OUT_BF16, check

    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    rows = []
    for m in PREFILL_M:
        for k, n in PREFILL_KN:
            xq = torch.randint(-127, 128, (m, k), dtype=torch.int8, device=dev, generator=gen).view(torch.int32)
            wq = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev, generator=gen).view(torch.int32)
            sx = torch.empty(m, device=dev).uniform_(0.001, 0.05, generator=gen)
            sw = torch.empty(n, device=dev).uniform_(0.002, 0.02, generator=gen)
            bias = torch.randn(n, device=dev, generator=gen)
            out = torch.empty(m, n, dtype=torch.bfloat16, device=dev)

            def run(stream_ptr):
                check(lib.bh_matmul_i8_dyn(stream_ptr, xq.data_ptr(), wq.data_ptr(), sx.data_ptr(), sw.data_ptr(),
                                           bias.data_ptr(), out.data_ptr(), BH_OUT_BF16, m, k // 4, n))

            # `reps` back-to-back launches in one HIP graph, so host launch
            # cost stays out of the per-launch time.
            run(sp)
            torch.cuda.synchronize()
            cap = torch.cuda.Stream()
            check(lib.bh_reserve_workspace(cap.cuda_stream, m, k // 4, n))
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=cap):
                for _ in range(reps):
                    run(cap.cuda_stream)
            g.replay()
            torch.cuda.synchronize()
            ts = []
            for _ in range(3):
                a = torch.cuda.Event(enable_timing=True)
                b = torch.cuda.Event(enable_timing=True)
                a.record(stream)
                g.replay()
                b.record(stream)
                ts.append((a, b))
            torch.cuda.synchronize()
            us = 1e3 * sorted(a.elapsed_time(b) for a, b in ts)[1] / reps
            del g
            ops = 2.0 * m * n * k
            byts = m * k + n * k + 2 * m * n + 4 * m + 8 * n
            tops = ops / us / 1e6
            bound = min(INT8_PEAK_TOPS, HBM_PEAK_GBS * ops / byts / 1e3)
            rows.append(dict(m=m, k=k, n=n, us=round(us, 1), tops=round(tops, 1),
                             frac_peak=round(tops / INT8_PEAK_TOPS, 3), frac_bound=round(tops / bound, 3)))
            del xq, wq, out
    tot_ops = sum(2.0 * r["m"] * r["n"] * r["k"] for r in rows)
    tot_us = sum(r["us"] for r in rows)
    return dict(tops=round(tot_ops / tot_us / 1e6, 1), frac_peak=round(tot_ops / tot_us / 1e6 / INT8_PEAK_TOPS, 3),
                shapes=rows)


def mfma_roof(torch, lib, dev):
    from brain_amd._lib import check

    blocks, iters = 256 * 8, 4096
    out = torch.empty(blocks * 256, dtype=torch.int32, device=dev)
    sp = torch.cuda.current_stream().cuda_stream
    check(lib.bh_roof_mfma_i8(sp, blocks, 64, out.data_ptr()))
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    check(lib.bh_roof_mfma_i8(sp, blocks, iters, out.data_ptr()))
    b.record()
    torch.cuda.synchronize()
    ops = blocks * 4 * iters * 4 * 65536.0
    return round(ops / (a.elapsed_time(b) * 1e-3) / 1e12, 1)


def hbm_read_probe(torch, lib, dev, seg_bytes=256 << 20, nseg=4):
    """The streaming-read ceiling on this box (bh_roof_hbm_read: 16-byte
    non-temporal loads): one graph reading `nseg`
    distinct 256 MiB segments in turn (1 GiB, so each read is cold), best over
    five grid sizes."""
    from brain_amd._lib import check
    buf = torch.empty(seg_bytes * nseg // 4, dtype=torch.int32, device=dev).random_(-2**31, 2**31 - 1)
    best = None
    for blocks in (1024, 2048, 4096, 8192, 16384):
        out = torch.empty(blocks * 256, dtype=torch.int32, device=dev)
        fns = [lambda i=i: check(lib.bh_roof_hbm_read(torch.cuda.current_stream().cuda_stream,
                                                       buf.data_ptr() + i * seg_bytes, seg_bytes, blocks,
                                                       out.data_ptr())) for i in range(nseg)]
        us = graph_per_launch_us(torch, fns, reps=3)
        gbs = seg_bytes / (us * 1e-6) / 1e9
        if best is None or gbs > best["gbs"]:
            best = {"gbs": round(gbs, 1), "blocks": blocks, "us_per_256mib": round(us, 1)}
    del buf
    torch.cuda.empty_cache()
    best["frac_of_8tbs"] = round(best["gbs"] / HBM_PEAK_GBS, 4)
    return best


def bench_moe(reps=10, m=16384):
    """moe_linear_gated_i8 at a long-prefill size (m tokens, one expert's
    1024 -> 3072 linear), routed fractions 1/8, 1/4 and 1 (from 8192 rows the
    routed rows are compacted before the GEMM); next to it the dense
    bh_matmul_i8_dyn of all m rows. Each a graph of `reps` launches (warm
    weights)."""
    import torch
    from brain_amd._lib import BH_OUT_F32, check
    import brain_amd
    lib = brain_amd.load()
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    k, n, ne, ei = 1024, 3072, 8, 1
    xq = torch.randint(-127, 128, (m, k), dtype=torch.int8, device=dev, generator=g).view(torch.int32)
    wq = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev, generator=g).view(torch.int32)
    sx = torch.empty(m, device=dev).uniform_(0.001, 0.05, generator=g)
    sw = torch.empty(n, device=dev).uniform_(0.002, 0.02, generator=g)
    out = torch.empty(m, n, device=dev)

    def timed(fn):
        gr = torch.cuda.CUDAGraph()
        st = torch.cuda.Stream()
        with torch.cuda.stream(st):
            fn()  # on the capture stream: its per-stream workspace exists before capture
        torch.cuda.synchronize()
        with torch.cuda.graph(gr, stream=st):
            for _ in range(reps):
                fn()
        gr.replay()
        torch.cuda.synchronize()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        gr.replay()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e3 / reps

    rows = []
    for frac in (0.125, 0.25, 1.0):
        gate = torch.full((m, ne), -1.0, device=dev)
        routed = torch.rand(m, device=dev, generator=g) < frac
        gate[:, ei] = torch.where(routed, 1.0, -1.0)
        us = timed(lambda: check(lib.bh_moe_linear_gated_i8(torch.cuda.current_stream().cuda_stream, xq.data_ptr(),
                                                            wq.data_ptr(), sx.data_ptr(), sw.data_ptr(),
                                                            gate.data_ptr(), ne, ei, out.data_ptr(), m, k // 4, n)))
        mr = int(routed.sum().item())
        rows.append({"routed_rows": mr, "us": round(us, 1), "tops_routed": round(2.0 * mr * k * n / us / 1e6, 1)})
    dense = timed(lambda: check(lib.bh_matmul_i8_dyn(torch.cuda.current_stream().cuda_stream, xq.data_ptr(),
                                                     wq.data_ptr(), sx.data_ptr(), sw.data_ptr(), None,
                                                     out.data_ptr(), BH_OUT_F32, m, k // 4, n)))
    return {"workload": f"moe_linear_gated_i8 M={m} K={k} N={n}, f32 out", "gated": rows,
            "dense_all_rows_us": round(dense, 1)}


def bench_w4a8(reps=20):
    """W4A8 (matmul_q4_gemv / matmul_q4_dyn): the configs[1] decode shapes at
    M = 1 and 16 and two prefill shapes with int4 weights. Decode is measured
    cold, like the int8 per-shape table: one graph of launches cycling over
    weight copies that together exceed the Infinity Cache; GB/s over
    N*K/2 + 4N + M*K + 2*M*N. Prefill: one HIP graph of `reps` launches on one
    weight (as the int8 prefill sweep), TOPS."""
    import torch
    from brain_amd import ops
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    out = {"decode": [], "prefill": []}

    def timed(fn):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn()
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=s):  # the stream whose workspace the warm call sized
            for _ in range(reps):
                fn()
        gr.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        gr.replay()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / reps

    for m, (k, n) in [(m, kn) for kn in DECODE_KN for m in (1, 16)]:
        xq = torch.randint(-127, 128, (m, k), dtype=torch.int8, device=dev, generator=g).view(torch.int32)
        copies = max(2, min(128, -(-(512 << 20) // (n * k // 2))))
        ws = [torch.randint(-2**31, 2**31 - 1, (n, k // 8), dtype=torch.int32, device=dev, generator=g)
              for _ in range(copies)]
        sx = torch.rand(m, device=dev, generator=g)
        sw = torch.rand(n, device=dev, generator=g) * 0.01
        o = torch.empty(m, n, device=dev, dtype=torch.bfloat16)

        def fn(w4):
            return lambda: ops.matmul_q4(xq, w4, sx, sw, None, torch.bfloat16, "auto", out=o)
        us = graph_per_launch_us(torch, [fn(w) for w in ws])
        b = n * k // 2 + 4 * n + m * k + 2 * m * n
        out["decode"].append({"m": m, "k": k, "n": n, "copies": copies, "us": round(us, 2),
                              "gbs": round(b / us / 1e3, 1)})
        del ws
    for m, (k, n) in [(512, (4096, 11008)), (2048, (4096, 4096))]:
        xq = torch.randint(-127, 128, (m, k), dtype=torch.int8, device=dev, generator=g).view(torch.int32)
        w4 = torch.randint(-2**31, 2**31 - 1, (n, k // 8), dtype=torch.int32, device=dev, generator=g)
        sx = torch.rand(m, device=dev, generator=g)
        sw = torch.rand(n, device=dev, generator=g) * 0.01
        o = torch.empty(m, n, device=dev, dtype=torch.bfloat16)
        dt = timed(lambda: ops.matmul_q4(xq, w4, sx, sw, None, torch.bfloat16, "auto", out=o))
        out["prefill"].append({"m": m, "k": k, "n": n, "us": round(dt * 1e6, 2),
                               "tops": round(2 * m * n * k / dt / 1e12, 1)})
    return out


def bench_quant(reps=20):
    """Per-token activation quantization at the configs[2] activation shapes
    (max_abs_rows.wgsl + quant_pack.wgsl, HBM-bound): the single-pass
    bh_quantize_rows (reads the f32 row once) and the reference's two passes
    (bh_max_abs_rows, then bh_quant_pack: the row is read twice), plus the
    bf16 rows of the DiT stack. One HIP graph per shape of at least `reps`
    launches cycling over input copies that together exceed the 256 MB
    Infinity Cache, so every launch reads its rows from HBM. GB/s over the
    algorithmic bytes: f32 reads 4MK per pass, the int8 codes MK, the scales
    4M per write or read."""
    import torch
    from brain_amd import ops
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    out = {"f32": [], "bf16": []}

    def timed(fns):
        n = max(reps, len(fns))
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for fn in fns:
                fn()
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=s):
            for i in range(n):
                fns[i % len(fns)]()
        gr.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        gr.replay()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n

    def ncopies(nbytes):
        return max(2, min(256, -(-(640 << 20) // nbytes)))

    for m in (512, 2048, 8192):
        for k in (1024, 3072, 4096):
            copies = ncopies(4 * m * k)
            xs = [torch.randn(m, k, device=dev, generator=g) for _ in range(copies)]
            sx = torch.empty(m, device=dev)
            xq = torch.empty(m, k // 4, dtype=torch.int32, device=dev)
            one = timed([lambda x=x: ops.quantize_rows(x, sx, xq) for x in xs])
            two = timed([lambda x=x: (ops.max_abs_rows(x, sx), ops.quant_pack(x, sx, xq)) for x in xs])
            b1 = 4 * m * k + m * k + 4 * m
            b2 = 8 * m * k + m * k + 12 * m
            out["f32"].append({"m": m, "k": k, "one_pass_us": round(one * 1e6, 2),
                               "one_pass_gbs": round(b1 / one / 1e9, 1),
                               "one_pass_frac": round(b1 / one / 1e9 / HBM_PEAK_GBS, 3),
                               "two_pass_us": round(two * 1e6, 2), "two_pass_gbs": round(b2 / two / 1e9, 1)})
            del xs
    for m, k in ((1152, 3840), (1152, 10240)):
        copies = ncopies(2 * m * k)
        xs = [torch.randn(m, k, device=dev, generator=g).to(torch.bfloat16) for _ in range(copies)]
        sx = torch.empty(m, device=dev)
        xq = torch.empty(m, k // 4, dtype=torch.int32, device=dev)
        dt = timed([lambda x=x: ops.quantize_rows_bf16(x, sx, xq) for x in xs])
        b = 2 * m * k + m * k + 4 * m
        out["bf16"].append({"m": m, "k": k, "us": round(dt * 1e6, 2), "gbs": round(b / dt / 1e9, 1),
                            "frac": round(b / dt / 1e9 / HBM_PEAK_GBS, 3)})
        del xs
    # Weight quantization (model::int8::quantize_weight, load time): the device
    # kernel over f32 [N, K] (4NK + NK + 4N bytes) and the host quantizer the
    # reference runs at load (rayon over rows), here row-parallel C++.
    import ctypes
    import numpy as np
    from brain_amd import _lib
    out["weights"] = []
    for n, k in ((11008, 4096), (151936, 1024)):
        # Copies that together exceed the Infinity Cache, as above.
        ws = [torch.randn(n, k, device=dev, generator=g) for _ in range(ncopies(4 * n * k))]
        w = ws[0]
        packed = torch.empty(n, k // 4, dtype=torch.int32, device=dev)
        sw = torch.empty(n, device=dev)
        lib = _lib.load()
        dt = timed([lambda wi=wi: _lib.check(lib.bh_quantize_weight_device(ops._stream(), wi.data_ptr(), n, k,
                                                                            packed.data_ptr(), sw.data_ptr()))
                    for wi in ws])
        _lib.check(lib.bh_quantize_weight_device(ops._stream(), w.data_ptr(), n, k, packed.data_ptr(), sw.data_ptr()))
        torch.cuda.synchronize()
        b = 5 * n * k + 4 * n
        row = {"n": n, "k": k, "device_us": round(dt * 1e6, 1), "device_gbs": round(b / dt / 1e9, 1),
               "device_frac": round(b / dt / 1e9 / HBM_PEAK_GBS, 3)}
        if n == 11008:
            wh = w.cpu().numpy()
            ph = np.empty((n, k // 4), np.uint32)
            sh = np.empty(n, np.float32)
            args = (wh.ctypes.data_as(ctypes.c_void_p), n, k, ph.ctypes.data_as(ctypes.c_void_p),
                    sh.ctypes.data_as(ctypes.c_void_p))
            _lib.check(lib.bh_quantize_weight(*args))
            t0 = time.perf_counter()
            for _ in range(3):
                _lib.check(lib.bh_quantize_weight(*args))
            ht = (time.perf_counter() - t0) / 3
            row.update({"host_ms": round(ht * 1e3, 1), "host_gbs": round(b / ht / 1e9, 1),
                        "host_threads": min(int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count(),
                                            os.cpu_count())})
            assert (ph.view(np.int32) == packed.cpu().numpy()).all(), "host and device weight codes differ"
        out["weights"].append(row)
        del w, ws, packed
    return out


def qwen3_weight_bytes(c):
    """int8 weight + scale bytes one decode step streams (every linear + the head)."""
    d, ff, hq, hkv = c["d_model"], c["d_ff"], c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"]
    per_layer = (hq + 2 * hkv) * d + d * hq + 2 * ff * d + d * ff
    rows = c["n_layers"] * (hq + 2 * hkv + d + 2 * ff + d) + c["vocab"]
    return c["n_layers"] * per_layer + c["vocab"] * d + 4 * rows


def qwen3_cpu_baseline(budget_s=8.0, ctx=128):
    """The restated backend-cpu int8 decode of the same architecture (oracle
    or_qwen3_cpu_decode: int8 GEMV per column over OpenMP threads, f32
    norms/RoPE/attention), batch 1 after `ctx` cached positions; as many steps
    as fit the budget after a 1-step estimate."""
    from brain_amd.qwen3 import QWEN3_0_6B
    from oracle import oracle as o
    threads = min(16, os.cpu_count() or 1)
    est = o.qwen3_cpu_decode_seconds(QWEN3_0_6B, threads, ctx, 1)
    steps = max(2, min(64, int(budget_s / max(est, 1e-3))))
    secs = o.qwen3_cpu_decode_seconds(QWEN3_0_6B, threads, ctx, steps)
    return {"value": round(steps / secs, 2), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{steps} greedy int8 decode steps at batch 1 after {ctx} cached positions, random int8 weights"}


def bench_qwen3(prompt_len=128, gen=256, batches=(1, 4, 8), cpu=True, kv8_legs=True):
    """Qwen3-0.6B-architecture int8 decoder, random init, greedy.
    Prefill of a random-id prompt, then `gen` decode steps (one HIP graph
    replay each); tok/s = batch * gen / decode wall time."""
    import numpy as np
    from brain_amd.qwen3 import QWEN3_0_6B, Qwen3Engine
    c = QWEN3_0_6B
    wbytes = qwen3_weight_bytes(c)
    out = {"model": "Qwen3-0.6B architecture (28 layers, d 1024, 16q/8kv heads, hd 128, ff 3072, vocab 151936, tied)",
           "weights": "random init (device, seeded), int8 per-channel", "prompt_len": prompt_len, "decode_steps": gen,
           "int8_weight_mb_per_step": round(wbytes / 1e6, 1)}
    max_seq = prompt_len + gen + 8
    legs = [(b, 0, False) for b in batches]
    if kv8_legs:
        legs += [(max(batches), 1, False), (max(batches), 1, True)]
    for b, kv8, paged in legs:
        cfg = dict(c, kv_int8=kv8)
        if paged:
            # The reference's paged pool: blocks of 32 positions in a pool with
            # spare blocks, each sequence's blocks scattered over it.
            max_bt = -(-max_seq // 32)
            nblk = b * max_bt + 16
            cfg.update(kv_block_size=32, kv_num_blocks=nblk)
        e = Qwen3Engine(cfg, b, max_seq, max_rows=b * prompt_len)
        if paged:
            e.set_block_table(np.random.default_rng(9).permutation(nblk)[:b * max_bt].reshape(b, max_bt))
        e.init_random(7)
        prompts = np.random.default_rng(b).integers(0, c["vocab"], size=(b, prompt_len))
        e.prefill(prompts)
        e.decode(4)                      # graph capture + warm-up
        t0 = time.perf_counter()
        e.prefill(prompts)
        t1 = time.perf_counter()
        toks = e.decode(gen)
        t2 = time.perf_counter()
        assert toks.shape == (gen, b)
        step_s = (t2 - t1) / gen
        avg_ctx = prompt_len + (gen + 1) / 2.0
        kv_bytes = 2 * c["n_layers"] * b * avg_ctx * c["n_kv_heads"] * c["head_dim"] * (1 if kv8 else 4)
        out[f"batch{b}" + ("_kv_int8" if kv8 else "") + ("_paged32" if paged else "")] = {"decode_tok_s": round(b * gen / (t2 - t1), 1), "ms_per_step": round(step_s * 1e3, 4),
                            "prefill_ms": round((t1 - t0) * 1e3, 2),
                            "prefill_tok_s": round(b * prompt_len / (t1 - t0), 1),
                            "step_hbm_gbs": round((wbytes + kv_bytes) / step_s / 1e9, 1)}
        e.close()
    if cpu:
        out["cpu_baseline"] = qwen3_cpu_baseline()
        out["batch1_gpu_vs_cpu"] = round(out["batch1"]["decode_tok_s"] / out["cpu_baseline"]["value"], 1)
    return out


def bench_dit(reps=5):
    """the DiT int8 linear stack (brain_amd.dit), 30 layers at
    M=1152, one HIP graph per step; TOPS over the 4 linears of every layer."""
    import torch
    from brain_amd import dit
    st = dit.DitInt8Stack(device="cuda")
    st.capture()
    st.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        st.replay()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / reps
    ops_step = dit.linear_ops() * st.layers
    out = {"workload": "configs[4]: 30 layers x (quant 3840 -> QKV 3840x11520, out 3840x3840, quant -> FFN up "
                       "3840x10240, quant 10240 -> down 10240x3840), M=1152, bf16 activations",
           "ms_per_step": round(dt * 1e3, 3), "tops": round(ops_step / dt / 1e12, 1),
           "frac_of_int8_peak": round(ops_step / dt / 1e12 / INT8_PEAK_TOPS, 4)}
    assert torch.isfinite(st.x.float()).all()
    del st
    torch.cuda.empty_cache()
    return out


def cpu_baseline(budget_s):
    """The restated backend-cpu decode path (max_abs_row -> quant_pack ->
    matmul_i8_gemv, OpenMP over output columns) on this host, on the same
    16-linear sweep; repeated up to the time budget, median reported."""
    import numpy as np
    from oracle import oracle as o

    threads = min(len(os.sched_getaffinity(0)), 16)
    data = []
    for m in DECODE_M:
        for k, n in DECODE_KN:
            wq, sw = o.synth_weights(n, k, 1000 + m + n) if n * k <= 4 * 1024 * 1024 else _big_weights(n, k)
            data.append((o.synth_acts(m, k, m + k), wq, sw))
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 or (time.perf_counter() - t_start < budget_s and len(times) < 20):
        t0 = time.perf_counter()
        for x, wq, sw in data:
            o.cpu_linear_gemv(x, wq, sw, threads)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s and len(times) >= 1:
            break
    t = sorted(times)[len(times) // 2]
    byts = sum(linear_bytes(m, k, n) for m in DECODE_M for k, n in DECODE_KN)
    return dict(value=round(byts / t / 1e9, 2), unit="GB/s", cores=threads, kind="port",
                sample=f"full 16-linear decode sweep, {len(times)} runs, median {t * 1e3:.1f} ms per sweep",
                step_ms=round(t * 1e3, 2), host=host_cpu())


def host_cpu():
    """The host the CPU baselines ran on: CPU model, logical CPUs, and the
    CPUs this process may use."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0))}


def prefill_cpu_baseline(budget_s):
    """Prefill on the host, where backend-cpu has no int8 path
    (crates/gpu-core/tests/bench_matmul.rs:243-247): the restated decode GEMV
    applied in 32-row chunks ("reference-CPU-equivalent (GEMV-chunked)") and an
    OpenMP tiled i32 GEMM (a stronger host reference), on a bounded row sample
    of the configs[2] shape 512x1024x3072, median of repeated runs."""
    from oracle import oracle as o

    threads = min(len(os.sched_getaffinity(0)), 16)
    k, n = 1024, 3072
    wq, sw = o.synth_weights(n, k, 77)
    out = {}
    for name, rows, fn in (("gemv_chunked", 64, lambda xq, sx: [o.cpu_gemv_packed(xq[r:r + 32], wq, sx[r:r + 32], sw, threads)
                                                             for r in range(0, xq.shape[0], 32)]),
                           ("tiled_i32", 256, lambda xq, sx: o.cpu_gemm_tiled(xq, wq, sx, sw, threads))):
        x = o.synth_acts(rows, k, 5)
        sx = o.max_abs_row(x)
        xq = o.quant_pack(x, sx)
        times = []
        t_start = time.perf_counter()
        while len(times) < 3 or (time.perf_counter() - t_start < budget_s / 2 and len(times) < 15):
            t0 = time.perf_counter()
            fn(xq, sx)
            times.append(time.perf_counter() - t0)
        t = sorted(times)[len(times) // 2]
        out[name] = dict(value=round(2.0 * rows * n * k / t / 1e12, 4), unit="TOPS", cores=threads, kind="port",
                         sample=f"{rows} of the 512 rows of 512x1024x3072, {len(times)} runs, median {t * 1e3:.1f} ms")
    return out


def _big_weights(n, k):
    import numpy as np

    rng = np.random.default_rng(n + k)
    q = rng.integers(-127, 128, (n, k), dtype=np.int8)
    return np.ascontiguousarray(q).view(np.uint32), rng.uniform(0.002, 0.02, n).astype(np.float32)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the int8 linear shards over output channels with no exchange)", file=sys.stderr)
        sys.exit(2)
    import torch

    import brain_amd

    lib = brain_amd.load()
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    res = {}
    if args.only == "copy":
        # Counter calibration: a plain 256 MiB device-to-device copy, 3 times.
        src = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        # ... and the dwordx4 read probe (the GEMV's load width) over the same
        # 256 MiB, 3 times: a second calibration point for FETCH_SIZE.
        from brain_amd._lib import check
        sink = torch.empty(2048 * 256, dtype=torch.int32, device=dev)
        for _ in range(3):
            check(lib.bh_roof_hbm_read(torch.cuda.current_stream().cuda_stream, src.data_ptr(), src.numel() * 4,
                                       2048, sink.data_ptr()))
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": src.numel() * 4, "read_probe_bytes": src.numel() * 4}))
        return
    if args.only == "hbm":
        print(json.dumps({"hbm_read_probe": hbm_read_probe(torch, lib, dev)}))
        return
    if args.only in ("", "decode", "gemv"):
        sets = make_decode_set(torch, dev, gen)
        res["decode"] = bench_decode(torch, lib, sets, args.steps, args.warmup, gemv_only=args.only == "gemv")
        del sets
    def leg(key, fn):
        # A secondary leg that raises is recorded as such, so the line (and
        # the decode measurement it carries) still prints.
        try:
            res[key] = fn()
        except Exception as e:  # noqa: BLE001 - reported in the line and on stderr
            traceback.print_exc()
            res[key] = {"error": f"{type(e).__name__}: {e}"}

    if args.only in ("", "shapes"):
        leg("shapes", lambda: bench_decode_shapes(torch, lib, dev, gen))
    if args.only in ("", "config0"):
        leg("config0", lambda: bench_config0(torch, lib, dev, gen, cpu=not args.no_cpu))
    if args.only in ("", "prefill") and not args.no_prefill:
        leg("prefill", lambda: bench_prefill(torch, lib, dev, gen, args.prefill_reps))
    if args.only in ("", "quant") and not args.no_quant:
        leg("quant", bench_quant)
    if args.only in ("", "qwen3") and not args.no_qwen3:
        if args.qwen3_batch:
            leg("qwen3", lambda: bench_qwen3(batches=(args.qwen3_batch,), cpu=False, kv8_legs=False))
        else:
            leg("qwen3", lambda: bench_qwen3(cpu=not args.no_cpu))
    if args.only in ("", "dit") and not args.no_dit:
        leg("dit", bench_dit)
    if args.only in ("", "w4a8") and not args.no_w4a8:
        leg("w4a8", bench_w4a8)
    if args.only in ("", "moe") and not args.no_moe:
        leg("moe", bench_moe)
    if args.only:
        print(json.dumps(res))
        return
    roof = mfma_roof(torch, lib, dev)
    hbm_roof = hbm_read_probe(torch, lib, dev)
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)
    pcpu = None
    if not args.no_cpu and "prefill" in res and "error" not in res["prefill"]:
        pcpu = prefill_cpu_baseline(min(args.cpu_seconds, 10.0))

    d = res["decode"]
    value = d["step_bytes"] / (d["step_ms"] * 1e-3) / 1e9
    # HBM bytes per GEMV launch from the committed rocprofv3 FETCH_SIZE /
    # WRITE_SIZE runs of this workload (counters cannot be read live here).
    traffic, tsrc = None, {}
    tpath = os.path.join(ROOT, "profiles", "gemv_traffic.txt")
    if os.path.exists(tpath):
        with open(tpath) as f:
            for line in f:
                key, _, val = line.partition(":")
                if key == "traffic_bytes_per_launch":
                    traffic = int(val)
                elif key in ("measured_at_commit", "fetch_factor", "fetch_factor_read_probe", "write_factor"):
                    tsrc[key] = val.strip()
    gemv_gbs = d["gemv_mean_bytes"] / (d["gemv_mean_us"] * 1e-6) / 1e9
    # The same roofline per kernel, from the cold per-shape table: the 12
    # narrow shapes run gemv_i8_kernel, the 4 LM heads gemv_i8_stream_kernel.
    by_kernel = []
    if isinstance(res.get("shapes"), list):
        for name, rows in (("gemv_i8_kernel", [r for r in res["shapes"] if r["n"] < 16384]),
                           ("gemv_i8_stream_kernel", [r for r in res["shapes"] if r["n"] >= 16384])):
            gb = sum(gemv_bytes(r["m"], r["k"], r["n"]) for r in rows) / len(rows)
            us = sum(r["gemv_us"] for r in rows) / len(rows)
            by_kernel.append({"kernel": name, "shapes": len(rows), "avg_algorithmic_bytes": round(gb),
                              "avg_launch_us_cold": round(us, 2), "gbs": round(gb / us / 1e3, 1),
                              "frac": round(gb / us / 1e3 / HBM_PEAK_GBS, 4)})
    line = {
        "metric": "int8 GEMM TOPS & %peak (prefill); GEMV GB/s & %HBM (decode); vs CPU",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(d["step_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8",
        "data": "synthetic (seeded torch RNG: int8 W uniform [-127,127], sw U(0.002,0.02), x N(0,1))",
        "config": {"workload": "configs[1] decode GEMV sweep: 16 int8 linears (quant + GEMV, bf16 out), "
                               "M in {1,4,8,16} x (K,N) in {(1024,3072),(3072,1024),(1024,2048),(1024,151936)}",
                   "weight_pool_mb": round(sum(k * n for k, n in DECODE_KN) * len(DECODE_M) / 1e6, 1),
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(gemv_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gemv_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "gemv_i8_kernel (12 narrow shapes) + gemv_i8_stream_kernel (4 LM heads)",
                     "avg_launch_us": round(d["gemv_mean_us"], 2),
                     "avg_algorithmic_bytes": round(d["gemv_mean_bytes"]),
                     "by_kernel": by_kernel,
                     "traffic_source": dict(tsrc, file="profiles/gemv_traffic.txt",
                                            how="rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of bench.py --only gemv, "
                                                "committed summary, not measured in this run"),
                     "hbm_read_probe": hbm_roof},
        "cpu_baseline": None if cpu is None else {k: cpu[k] for k in ("value", "unit", "cores", "kind", "sample", "host")},
        "decode_shapes_cold": res["shapes"],
        "config0_linear": res["config0"],
        "mfma_roof_probe_tops": roof,
    }
    if "prefill" in res:
        line["prefill"] = res["prefill"]
        if pcpu is not None:  # (the prefill leg succeeded)
            line["prefill_cpu_baseline"] = pcpu
            g = [r for r in res["prefill"]["shapes"] if (r["m"], r["k"], r["n"]) == (512, 1024, 3072)]
            if g:
                line["prefill_gpu_vs_cpu_tiled"] = round(g[0]["tops"] / pcpu["tiled_i32"]["value"], 1)
    if "quant" in res:
        line["activation_quant"] = res["quant"]
    if "qwen3" in res:
        line["qwen3_e2e"] = res["qwen3"]
    if "dit" in res:
        line["dit_stack"] = res["dit"]
    if "w4a8" in res:
        line["w4a8"] = res["w4a8"]
    if "moe" in res:
        line["moe_gated"] = res["moe"]
    if cpu is not None:
        line["gpu_vs_cpu"] = round(value / cpu["value"], 1)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
