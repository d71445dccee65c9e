"""Benchmark of the MI355X weight-only quantized matmul path (one JSON line on stdout).

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A step is one call of the decode GEMV of BASELINE config 0 (W4A16, M=1, K=5120, N=17408, g128 fp16 scales,
bf16 output) on seeded synthetic inputs already resident in HBM. The weights rotate over 8 copies (368 MB,
more than the 256 MB Infinity Cache) so every call streams its weights from HBM. `value` = algorithmic bytes
(N*K/2 + N*(K/128)*2 + M*K*2 + M*N*2 = 46,002,176 B per call) * K / the elapsed time of the K timed steps.
Every secondary figure rotates enough weight copies (or MoE routings) that its working set exceeds the Infinity
Cache and says so (`working_set`, bytes). The K decode launches are captured in one HIP graph and replayed (as a decode loop is served), so the host's
per-call overhead does not starve the GPU. `roofline.achieved` = bytes per call / the stream time per launch
(HIP events on the launch stream before and after the K timed launches); `roofline.read_floor_us` is the same run's
load-only floor of that launch shape (qe_read_probe), `frac_of_read_floor` the GEMV's share of it and `clock_mhz`
the shader clock measured right after the GEMV (qe_clock_probe_mhz): the GEMV time follows the box's clock. The
prefill GEMM (config 2) and the other configs are reported beside it in `secondary`.
The CPU baseline is the oracle's dequantize + fp32 matmul of the same workload on the host cores.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2516.6
INT8_PEAK_TOPS = 5033.2  # dense int8 MFMA, TOP/s


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--copies", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-secondary", action="store_true", help="only the headline GEMV")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--only", choices=["prefill", "w8", "moe", "skinny", "decode", "c2decode"], default=None,
                    help="run one secondary workload alone (profiling); prints its result")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MB",
                    help="time a plain device copy of MB megabytes x 20 (scale for FETCH_SIZE / WRITE_SIZE) and exit")
    ap.add_argument("--read-floor", action="store_true",
                    help="time the m = 1 GEMV's record stream alone (qe_read_probe, same launch shape, no arithmetic) "
                         "on config 0 with the same rotation and graph timing, print it and exit")
    return ap.parse_args()


def gemv_bytes(m, n, k):
    return n * k // 2 + n * (k // 128) * 2 + m * k * 2 + m * n * 2


def read_traffic(name):
    """HBM bytes per launch measured by rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (profiles/<name>): the line
    'hbm_bytes_per_launch: <int>' of the committed summary, else None"""
    p = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(p):
        return None
    for line in open(p):
        if line.startswith("hbm_bytes_per_launch:"):
            return int(line.split(":")[1].strip())
    return None


def time_launches(fn, steps, warmup, nvar, graph=False):
    """fn(i) launches step i on the current stream. Returns (wall ms of the `steps` timed steps bracketed by
    synchronize, stream ms per step from HIP events recorded on the launch stream before and after the timed
    steps). graph=True captures the `steps` launches into one HIP graph and replays it, so host launch overhead
    (ctypes + torch stream lookup, comparable to a 10 us kernel) never starves the GPU: the per-step figure is
    then the kernel's duration plus the dispatch gap between consecutive graph nodes."""
    import torch
    # graph: the warmup runs on the capture stream, as a serving loop warms the stream it captures on (stream-owned
    # workspaces, e.g. the one-pass decode's tail counters, are set up by the eager calls)
    cs = torch.cuda.Stream() if graph else torch.cuda.current_stream()
    cs.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cs):
        for i in range(warmup):
            fn(i % nvar)
    torch.cuda.synchronize()
    run = lambda: [fn(i % nvar) for i in range(steps)]  # noqa: E731
    if graph:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cs):
            run()
        # upload, then untimed replays queued back to back (>= 30 ms of work) so the timed pass starts with the
        # GPU at its working clock: a pass started from idle runs ~15 % slower for its first milliseconds
        g.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        g.replay()
        torch.cuda.synchronize()
        one = max(time.perf_counter() - t0, 1e-4)
        for _ in range(max(2, min(2000, int(0.03 / one)))):
            g.replay()
        # then three single replays, each waited for: the first replay after a long queue of them takes ~40 us more
        # host time (measured at 20 launches of the C0 GEMV: 240-260 us of wall clock against 202-213 us settled;
        # the events inside are the same)
        torch.cuda.synchronize()
        for _ in range(3):
            g.replay()
            torch.cuda.synchronize()
        run = g.replay
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(st)
    run()
    e1.record(st)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    return wall_ms, e0.elapsed_time(e1) / steps


MALL_BYTES = 256 << 20  # MI355X Infinity Cache


def copies_for(bytes_per_copy, minimum):
    """weight copies to rotate so the working set exceeds the Infinity Cache by >= 15 %"""
    return max(minimum, -(-int(1.15 * MALL_BYTES) // int(bytes_per_copy)))


def bench_gemv(args, m=1, n=17408, k=5120, steps=None, warmup=None, invariant=False, mode="w4"):
    """decode GEMV / skinny at m rows. mode "w4": qe_gemv_w4_ex (m <= 16); "matmul": qe_matmul_w4_ex (m <= 64: 16-row
    launches); "h16": the H16 numerics on activations already in the XH layout (qe_gemv_w4h_ex)"""
    import torch
    from qengine_amd import ops, synth
    steps = steps or args.steps
    warmup = warmup or args.warmup
    ncopy = copies_for(gemv_bytes(m, n, k), args.copies)
    if invariant:
        set_config(batch_invariant=1)
    ws = []
    for c in range(ncopy):
        q, s = synth.w4_dev(n, k, seed=100 + c)
        ws.append(ops.repack_w4(q, s))
        del q, s
    x = synth.x_dev(m, k, seed=1)
    y = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    if mode == "h16":
        xh = ops.xh_pack(x)
        fn = lambda i: ops.gemv_w4hx(ws[i], xh, out_bf16=True, y=y)  # noqa: E731
    elif mode == "matmul":
        fn = lambda i: ops.matmul_w4(ws[i], x, out_bf16=True, y=y)  # noqa: E731
    else:
        fn = lambda i: ops.gemv_w4(ws[i], x, out_bf16=True, y=y)  # noqa: E731
    wall_ms, ev_ms = time_launches(fn, steps, warmup, len(ws), graph=True)
    b = gemv_bytes(m, n, k)
    res = dict(m=m, n=n, k=k, bytes=b, ms_per_step=wall_ms / steps, kernel_ms_mean=ev_ms, copies=ncopy,
               working_set=b * ncopy, gbs_wall=b * steps / (wall_ms * 1e-3) / 1e9, gbs_kernel=b / (ev_ms * 1e-3) / 1e9)
    if invariant:
        set_config(batch_invariant=0)
    del ws
    torch.cuda.empty_cache()
    return res


def clock_probe():
    """the shader clock in MHz (qe_clock_probe_mhz: clock64 cycles over 50 us of the constant-rate wall clock)"""
    from qengine_amd import ops
    from qengine_amd.qe import lib
    return round(float(lib().qe_clock_probe_mhz(ops._stream())), 1)


def set_config(**kw):
    from qengine_amd import ops
    ops.set_config(**kw)


def bench_read_floor(args, n=17408, k=5120, steps=None, warmup=None):
    """qe_read_probe: the m = 1 GEMV's launch shape and record loads with no arithmetic, same rotation and timing"""
    import torch
    from qengine_amd import call, ops, synth
    steps = steps or args.steps
    warmup = warmup or args.warmup
    ws = []
    for c in range(args.copies):
        q, s = synth.w4_dev(n, k, seed=100 + c)
        ws.append(ops.repack_w4(q, s))
        del q, s
    sink = torch.zeros(n // 16, dtype=torch.int32, device="cuda")
    fn = lambda i: call("qe_read_probe", ws[i].q, n, k, sink, ops._stream())  # noqa: E731
    wall_ms, ev_ms = time_launches(fn, steps, warmup, len(ws), graph=True)
    rec = n * k // 2
    del ws
    torch.cuda.empty_cache()
    return {"n": n, "k": k, "record_bytes": rec, "us_per_launch": round(ev_ms * 1e3, 3),
            "gbs": round(rec / (ev_ms * 1e-3) / 1e9, 1), "frac_of_peak": round(rec / (ev_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "working_set": rec * args.copies}


def bench_gemm(m, n, k, steps=10, warmup=3, copies=2, h16=False, i8=0):
    """prefill GEMM: TFLOP/s from the kernel's mean duration (events around each launch);
    h16: the fp16-accumulate numerics (qe_gemm_w4h_ex), i8 = G: the W4A8 numerics with activation group G
    (qe_gemm_w4_i8_ex); their activation pre-pass is included in the time"""
    import torch
    from qengine_amd import ops, synth
    ws = []
    for c in range(copies):
        q, s = synth.w4_dev(n, k, seed=300 + c)
        ws.append(ops.repack_w4(q, s))
        del q, s
    x = synth.x_dev(m, k, seed=2)
    y = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    if i8:
        fn = lambda i: ops.gemm_w4_i8(ws[i], x, G=i8, out_bf16=True, y=y)  # noqa: E731
    elif h16:
        fn = lambda i: ops.gemm_w4h(ws[i], x, out_bf16=True, y=y)  # noqa: E731
    else:
        fn = lambda i: ops.gemm_w4(ws[i], x, out_bf16=True, y=y)  # noqa: E731
    old = ops.set_config(gemm_tune=1)  # the first (untimed) call times the candidates once; the timed calls reuse it
    _, ev_ms = time_launches(fn, steps, warmup, len(ws))
    ops.set_config(**old)
    flop = 2.0 * m * n * k
    del ws, x, y
    torch.cuda.empty_cache()
    return {"m": m, "n": n, "k": k, "tflops": round(flop / (ev_ms * 1e-3) / 1e12, 1),
            "pct_bf16_peak": round(100 * flop / (ev_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 1),
            "ms_kernel": round(ev_ms, 4), "working_set": copies * (n * k // 2 + n * k // 64) + m * k * 2 + m * n * 2}


def bench_w8(m, n=8192, k=2048, steps=100, warmup=10, copies=32, w8a8=False):
    """INT8 W8A16 per-channel: GEMV (m = 1) in GB/s, GEMM (m = 4096) in TFLOP/s. w8a8: the
    reference's W8A8 row GEMM of the same matrix (activation pre-pass + int8 GEMM, both timed), against the int8
    peak"""
    import torch
    from qengine_amd import ops
    g = torch.Generator(device="cuda")
    g.manual_seed(400)
    ws = []
    ncopy = copies if m <= 16 else 2
    for c in range(ncopy):
        q = torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda", generator=g)
        s = (torch.randn(n, device="cuda", generator=g).abs() * 0.005).half()
        ws.append(ops.tile_w8(q, s, per_channel=True))
        del q
    from qengine_amd import synth
    x = synth.x_dev(m, k, seed=5)
    y = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    if m <= 16:
        fn = lambda i: ops.gemv_w8(ws[i], x, out_bf16=True, y=y)  # noqa: E731
    elif w8a8:
        fn = lambda i: ops.gemm_w8a8(ws[i], x, out_bf16=True, y=y)  # noqa: E731
    else:
        fn = lambda i: ops.gemm_w8(ws[i], x, out_bf16=True, y=y)  # noqa: E731
    _, ev_ms = time_launches(fn, steps if m <= 16 else 10, warmup, len(ws), graph=m <= 16)
    del ws
    torch.cuda.empty_cache()
    if m <= 16:
        b = n * k + 2 * n + 2 * m * k + 2 * m * n
        return {"m": m, "gbs": round(b / (ev_ms * 1e-3) / 1e9, 1), "pct_hbm": round(100 * b / (ev_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 1),
                "us_kernel": round(ev_ms * 1e3, 2), "bytes": b, "working_set": b * ncopy}
    flop = 2.0 * m * n * k
    r = {"m": m, "tflops": round(flop / (ev_ms * 1e-3) / 1e12, 1),
         "pct_bf16_peak": round(100 * flop / (ev_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 1), "ms_kernel": round(ev_ms, 4),
         "working_set": ncopy * (n * k + 2 * n) + 2 * m * k + 2 * m * n}
    if w8a8:
        r["pct_int8_peak"] = round(100 * flop / (ev_ms * 1e-3) / 1e12 / INT8_PEAK_TOPS, 1)
    return r


def bench_moe(Ts=(1, 16, 4096), E=512, topk=10, H=2048, I=512):
    """MoE layer: route + segment + gate_up + down + combine per call. The routings rotate (64 at
    T = 1, 16 at T = 16, 4 at T = 4096) so the experts hit across the rotation hold far more than the 256 MB
    Infinity Cache (`working_set`: the distinct experts' record bytes over one rotation)."""
    import torch
    from qengine_amd import ops, synth
    g = torch.Generator(device="cuda")
    g.manual_seed(500)
    gq = torch.randint(-2**31, 2**31 - 1, (E, 2 * I, H // 8), dtype=torch.int32, device="cuda", generator=g)
    gs = (torch.randn(E, 2 * I, H // 128, device="cuda", generator=g).abs() * 0.02).half()
    dq = torch.randint(-2**31, 2**31 - 1, (E, H, I // 8), dtype=torch.int32, device="cuda", generator=g)
    ds = (torch.randn(E, H, I // 128, device="cuda", generator=g).abs() * 0.02).half()
    moe = ops.MoE.pack(gq, gs, dq, ds, topk)
    del gq, gs, dq, ds
    torch.cuda.empty_cache()
    res = {}
    per_expert = 256 * H // 2 + 256 * (H // 128) * 2 + H * 64 + H * 2  # one group record
    per_expert *= I // 128
    for T in Ts:
        nrout = 64 if T == 1 else 16 if T <= 16 else 4
        lgs = [torch.randn(T, E, device="cuda", generator=g) for _ in range(nrout)]
        x = synth.x_dev(T, H, seed=6)
        y = torch.empty(T, H, dtype=torch.bfloat16, device="cuda")
        hits, seen = [], set()
        for lg in lgs:
            sel, _ = ops.moe_route(lg, topk)
            u = torch.unique(sel)
            hits.append(int(u.numel()))
            seen.update(u.cpu().tolist())
        fn = lambda i: moe(lgs[i], x, out_bf16=True, out=y)  # noqa: E731
        steps = 100 if T <= 16 else 20
        # decode (T <= 16) replayed from a HIP graph like the GEMV: the five launches of a call cost the host more
        # than the GPU work of a decode step (the layer is graph-safe: tests/test_moe_gpu.py replays it)
        _, ev_ms = time_launches(fn, steps, 5, nrout, graph=T <= 16)
        b = sum(hits) / len(hits) * per_expert + 4 * T * H
        flop = 6.0 * T * topk * H * I
        t_roof = max(b / (HBM_PEAK_GBS * 1e9), flop / (BF16_PEAK_TFLOPS * 1e12))
        res[f"T{T}"] = {"us_layer": round(ev_ms * 1e3, 2), "experts_hit": round(sum(hits) / len(hits), 1),
                        "gbs": round(b / (ev_ms * 1e-3) / 1e9, 1), "tflops": round(flop / (ev_ms * 1e-3) / 1e12, 2),
                        "roofline_frac": round(t_roof / (ev_ms * 1e-3), 3), "routings": nrout,
                        "working_set": len(seen) * per_expert}
        del lgs, x, y
    del moe
    torch.cuda.empty_cache()
    return res


def cpu_baseline(args, m=1, n=17408, k=5120):
    """oracle dequant (bf16_rn((u-8)*s)) + fp32 matmul, same workload shape, host cores, ~cpu_seconds of work"""
    import numpy as np
    import oracle
    from qengine_amd import synth
    cores = len(os.sched_getaffinity(0))
    os.environ["OMP_NUM_THREADS"] = str(cores)
    q, s = synth.w4_host(n, k, seed=100, sdt=1)
    x = synth.x_host(m, k, seed=1)
    reps, t_deq, t_mm = 0, 0.0, 0.0
    t_start = time.perf_counter()
    while reps == 0 or time.perf_counter() - t_start < args.cpu_seconds:
        t0 = time.perf_counter()
        wdq = oracle.dequant_w4(q, s, n, k, 1)
        t1 = time.perf_counter()
        oracle.matmul_bf16(x, wdq, nthreads=cores)
        t2 = time.perf_counter()
        t_deq += t1 - t0
        t_mm += t2 - t1
        reps += 1
    per = (t_deq + t_mm) / reps
    return {"value": round(gemv_bytes(m, n, k) / per / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"{reps} full calls of config 0 (M=1 K=5120 N=17408): oracle dequant_w4 + matmul_bf16 "
                      f"(C, OpenMP {cores} threads); dequant {t_deq / reps * 1e3:.1f} ms + matmul "
                      f"{t_mm / reps * 1e3:.1f} ms per call"}


def cpu_baseline_prefill(rows=8192, n=17408, k=5120):
    """config 2 on the host cores: the oracle's dequantization of the whole matrix and the fp32 matmul
    of `rows` of the 8192 token rows (TFLOP/s of that sample; the rate does not depend on the row count)"""
    import numpy as np  # noqa: F401
    import oracle
    from qengine_amd import synth
    cores = len(os.sched_getaffinity(0))
    q, s = synth.w4_host(n, k, seed=300, sdt=1)
    x = synth.x_host(rows, k, seed=2)
    t0 = time.perf_counter()
    wdq = oracle.dequant_w4(q, s, n, k, 1)
    t1 = time.perf_counter()
    oracle.matmul_bf16(x, wdq, nthreads=cores)
    t2 = time.perf_counter()
    flop = 2.0 * rows * n * k
    return {"value": round(flop / (t2 - t1) / 1e12, 4), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"config 2 (K=5120, N=17408): oracle dequant_w4 of the full matrix ({(t1 - t0) * 1e3:.0f} ms) + "
                      f"matmul_bf16 of {rows} of the 8192 token rows ({(t2 - t1):.2f} s, OpenMP {cores} threads), 1 rep"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: every box of this build has one MI355X and the path has no "
              f"collectives (--gpus {args.gpus} is not supported)", file=sys.stderr)
        sys.exit(2)
    import torch
    from qengine_amd import call
    torch.cuda.set_device(0)
    call("qe_gemv_workspace_init")
    if args.copy_calibration:
        nb = args.copy_calibration << 20
        a = torch.empty(nb, dtype=torch.uint8, device="cuda").fill_(1)
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        for _ in range(20):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_per_launch": nb, "launches": 20}))
        return
    if args.read_floor:
        print(json.dumps({"read_floor": bench_read_floor(args)}))
        return
    if args.only:
        fns = {"prefill": lambda: {"k5120_n17408": bench_gemm(8192, 17408, 5120),
                                   "k17408_n5120": bench_gemm(8192, 5120, 17408),
                                   "h16_k5120_n17408": bench_gemm(8192, 17408, 5120, h16=True),
                                   "w4a8_g64_k5120_n17408": bench_gemm(8192, 17408, 5120, i8=64),
                                   "w4a8_g128_k5120_n17408": bench_gemm(8192, 17408, 5120, i8=128)},
               "w8": lambda: {"m1": bench_w8(1), "m4096": bench_w8(4096), "w8a8_m4096": bench_w8(4096, w8a8=True)},
               "moe": lambda: bench_moe(),
               "skinny": lambda: {f"m{m}_n{n}": (lambda r: {"us": round(r["kernel_ms_mean"] * 1e3, 2),
                                                             "gbs": round(r["gbs_kernel"], 1)})(
                   bench_gemv(args, m=m, n=n, steps=200, warmup=20))
                   for n in (5120, 17408) for m in (1, 2, 4, 8, 16)},
               "decode": lambda: {f"{mode}_m{m}": (lambda r: {"us": round(r["kernel_ms_mean"] * 1e3, 2),
                                                              "gbs": round(r["gbs_kernel"], 1)})(
                   bench_gemv(args, m=m, steps=200, warmup=20, mode=mode))
                   for (m, mode) in [(1, "h16"), (16, "h16"), (32, "matmul"), (48, "matmul"), (64, "matmul")]},
               # decode of C2's second matrix (N = 5120, K = 17408: no even K slicing)
               "c2decode": lambda: {f"m{m}": (lambda r: {"us": round(r["kernel_ms_mean"] * 1e3, 2),
                                                         "gbs": round(r["gbs_kernel"], 1)})(
                   bench_gemv(args, m=m, n=5120, k=17408, steps=200, warmup=20, mode="w4" if m <= 16 else "matmul"))
                   for m in (1, 2, 4, 8, 16, 32)}}
        print(json.dumps({args.only: fns[args.only]()}))
        return

    g = bench_gemv(args)
    clock_mhz = clock_probe()  # right after the GEMV's replays: the shader clock this box ran them at
    floor = bench_read_floor(args, steps=400, warmup=20)
    secondary = {"gemv_c0": {"copies": g["copies"], "working_set": g["working_set"]}, "read_floor_c0": floor}
    if not args.no_secondary:
        gi = bench_gemv(args, steps=400, warmup=20, invariant=True)
        secondary["gemv_c0_batch_invariant"] = {"us_kernel": round(gi["kernel_ms_mean"] * 1e3, 3),
                                                "pct_hbm": round(100 * gi["gbs_kernel"] / HBM_PEAK_GBS, 1),
                                                "working_set": gi["working_set"]}
        for (m, n) in [(2, 5120), (4, 5120), (8, 5120), (16, 5120), (2, 17408), (4, 17408), (8, 17408), (16, 17408)]:
            r = bench_gemv(args, m=m, n=n, steps=200, warmup=20)
            secondary[f"skinny_m{m}_n{n}"] = {"gbs_kernel": round(r["gbs_kernel"], 1),
                                              "pct_hbm": round(100 * r["gbs_kernel"] / HBM_PEAK_GBS, 1),
                                              "us_kernel": round(r["kernel_ms_mean"] * 1e3, 2),
                                              "working_set": r["working_set"]}
        for (m, mode) in [(32, "matmul"), (64, "matmul"), (1, "h16"), (16, "h16")]:
            r = bench_gemv(args, m=m, steps=200, warmup=20, mode=mode)
            key = f"decode_m{m}_n17408" if mode == "matmul" else f"h16_m{m}_n17408"
            secondary[key] = {"gbs_kernel": round(r["gbs_kernel"], 1), "pct_hbm": round(100 * r["gbs_kernel"] / HBM_PEAK_GBS, 1),
                              "us_kernel": round(r["kernel_ms_mean"] * 1e3, 2), "working_set": r["working_set"]}
        # decode of C2's second matrix (K = 17408: 136 groups, no even K slicing)
        for (m, mode) in [(1, "w4"), (32, "matmul")]:
            r = bench_gemv(args, m=m, n=5120, k=17408, steps=200, warmup=20, mode=mode)
            secondary[f"decode_m{m}_n5120_k17408"] = {
                "gbs_kernel": round(r["gbs_kernel"], 1), "pct_hbm": round(100 * r["gbs_kernel"] / HBM_PEAK_GBS, 1),
                "us_kernel": round(r["kernel_ms_mean"] * 1e3, 2), "working_set": r["working_set"]}
        secondary["prefill_k5120_n17408"] = bench_gemm(8192, 17408, 5120)
        secondary["prefill_k17408_n5120"] = bench_gemm(8192, 5120, 17408)
        secondary["prefill_h16_k5120_n17408"] = bench_gemm(8192, 17408, 5120, h16=True)
        secondary["prefill_w4a8_g64_k5120_n17408"] = bench_gemm(8192, 17408, 5120, i8=64)
        secondary["w8_gemv_m1_k2048_n8192"] = bench_w8(1)
        secondary["w8_gemm_m4096_k2048_n8192"] = bench_w8(4096)
        secondary["w8a8_rows_m4096_k2048_n8192"] = bench_w8(4096, w8a8=True)
        secondary["moe_e512_top10_h2048_i512"] = bench_moe()
    cpu = None if args.no_cpu else cpu_baseline(args)
    if not args.no_cpu and not args.no_secondary:
        secondary["cpu_baseline_prefill_k5120_n17408"] = cpu_baseline_prefill()
    achieved = g["gbs_kernel"]
    out = {
        "metric": "W4A16 GEMV GB/s (% HBM peak) at M=1, K=5120, N=17408",
        "value": round(g["gbs_wall"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "w4a16 (int4 g128 weights, bf16 x, fp32 accumulate, bf16 out)",
        "data": "synthetic (seeded: uniform nibbles, fp16 scales |N(0,1)|*0.02, x bf16 N(0,1))",
        "config": {"workload": "BASELINE config 0: W4A16 decode GEMV", "m": 1, "k": 5120, "n": 17408,
                   "group": 128, "scales": "fp16", "out": "bf16", "weight_copies": args.copies,
                   "bytes_per_call": g["bytes"]},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": read_traffic("gemv_w4_c0_m1_traffic.txt"),
                     "kernel_us_mean": round(g["kernel_ms_mean"] * 1e3, 3),
                     # same run: the load-only floor of this launch shape, the GEMV's share of it, the shader clock
                     "read_floor_us": floor["us_per_launch"],
                     "frac_of_read_floor": round(floor["us_per_launch"] / (g["kernel_ms_mean"] * 1e3), 4),
                     "clock_mhz": clock_mhz},
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
