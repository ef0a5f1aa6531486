"""Benchmark of the MI355X Q8_0 linear path (one GPU).

Headline workload: the decode MLP at M=1 --
gate and up Q8_0 projections 2560 -> 9216 with the fused silu(gate)*up
epilogue, then the Q8_0 down projection 9216 -> 2560.  A step is one pass of
that MLP over one synthetic input row, activation quantization included.
Weights are N(0, 0.02) synthesized on the device and packed to q8_0_p4; a
rotating pool of distinct weight copies larger than the 256 MB Infinity Cache
keeps the timing on HBM.  Steps are replayed from a HIP graph so host launch
cost stays out of the timed region.

`value` = whole-step algorithmic bytes / time (GB/s).  `roofline` = the fused
gate/up GEMV (the dominant kernel) timed alone with HIP events on the
library's stream.  `cpu_baseline` = the oracle's C restatement of the
reference's x86 scalar Q8 path (row-parallel OpenMP, so 1 thread at M=1) on a
bounded sample of the same workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
MALL_BYTES = 256 << 20


def p4_bytes(n, k):
    return n * k // 32 * 34


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Timer:
    """HIP events on the library stream around a block of enqueued work."""

    def __init__(self, ctx):
        self.ctx = ctx
        self.e0, self.e1 = ctx.event(), ctx.event()

    def start(self):
        self.ctx.record(self.e0)

    def stop_ms(self):
        self.ctx.record(self.e1)
        return self.ctx.elapsed_ms(self.e0, self.e1)


def graph_of(ctx, fn):
    ctx.sync()
    ctx.graph_begin()
    fn()
    return ctx.graph_end()


def run_graph(ctx, timer, graph, launches):
    ctx.sync()
    timer.start()
    for _ in range(launches):
        ctx.graph_launch(graph)
    ms = timer.stop_ms()
    ctx.sync()
    return ms


def bench_decode_mlp(ctx, q8, steps, warmup, hidden=2560, ffn=9216):
    per_copy = 2 * p4_bytes(ffn, hidden) + p4_bytes(hidden, ffn)
    copies = max(2, -(-int(1.6 * MALL_BYTES) // per_copy))
    log("decode_mlp: %d weight copies x %.1f MB" % (copies, per_copy / 1e6))
    pool = []
    for c in range(copies):
        mats = []
        for i, (n, k) in enumerate([(ffn, hidden), (ffn, hidden), (hidden, ffn)]):
            p4d, _ = ctx.synthesize_p4(seed=1000 + 10 * c + i, rows=n, cols=k)
            mats.append((ctx.register_device_p4(p4d, n, k), p4d))
        pool.append(mats)
    rng = np.random.default_rng(2560)
    x = rng.standard_normal((1, hidden)).astype(np.float32)
    xd, hd, yd = ctx.to_device(x), ctx.alloc(ffn * 4), ctx.alloc(hidden * 4)

    def one_rotation():
        for mats in pool:
            ctx.mlp(xd, mats[0][0], mats[1][0], mats[2][0], yd, h=hd)

    def gateup_rotation():
        for mats in pool:
            ctx.swiglu(xd, mats[0][0], mats[1][0], hd, 1)

    def down_rotation():
        for mats in pool:
            ctx.linear(hd, mats[2][0], yd, 1)

    # fixed cost of one kernel node in graph replay: a 32-element quantize
    tq, ts = ctx.alloc(64), ctx.alloc(64)

    def tiny_rotation():
        for _ in pool:
            ctx.quantize(xd, 1, 32, tq, ts)

    timer = Timer(ctx)
    g_step = graph_of(ctx, one_rotation)
    g_gu = graph_of(ctx, gateup_rotation)
    rounds_w = max(1, -(-warmup // copies))
    rounds = max(1, -(-steps // copies))
    run_graph(ctx, timer, g_step, rounds_w)
    ms = run_graph(ctx, timer, g_step, rounds)
    n_steps = rounds * copies
    step_bytes = (per_copy + hidden * 4 + 2 * ffn * 4 + hidden * 4)
    gb_s = step_bytes * n_steps / (ms * 1e-3) / 1e9

    run_graph(ctx, timer, g_gu, rounds_w)
    ms_gu = run_graph(ctx, timer, g_gu, rounds)
    gu_launch_us = ms_gu * 1e3 / (rounds * copies)
    g_down, g_tiny = graph_of(ctx, down_rotation), graph_of(ctx, tiny_rotation)
    run_graph(ctx, timer, g_down, rounds_w)
    down_launch_us = run_graph(ctx, timer, g_down, rounds) * 1e3 / (rounds * copies)
    run_graph(ctx, timer, g_tiny, rounds_w)
    tiny_launch_us = run_graph(ctx, timer, g_tiny, rounds) * 1e3 / (rounds * copies)
    gu_bytes = 2 * p4_bytes(ffn, hidden) + hidden * 4 + ffn * 4
    gu_gbs = gu_bytes / (gu_launch_us * 1e-6) / 1e9

    # keep one copy's packed bytes for the CPU baseline
    host = [ctx.to_host(m[1], (m[1].nbytes,), np.uint8) for m in pool[0]]
    res = dict(ms=ms, steps=n_steps, gb_s=gb_s, step_bytes=step_bytes,
               copies=copies, pool_bytes=copies * per_copy,
               gu_launch_us=gu_launch_us, gu_bytes=gu_bytes, gu_gbs=gu_gbs,
               down_launch_us=down_launch_us, tiny_launch_us=tiny_launch_us,
               x=x, host_p4=host, hidden=hidden, ffn=ffn)
    for mats in pool:
        for w, p4d in mats:
            ctx.release(w)
            p4d.free()
    return res


def bench_gemv(ctx, n, k, iters=200, residual=False):
    """Config 1: a single Q8_0 GEMV (K = N = 2560) over a rotating pool;
    with `residual`, the same GEMV with the residual add fused
    (llmcp_q8_linear_add, in place on the output row)."""
    per = p4_bytes(n, k)
    copies = max(2, -(-int(1.6 * MALL_BYTES) // per))
    ws = []
    for c in range(copies):
        p4d, _ = ctx.synthesize_p4(seed=5000 + c, rows=n, cols=k)
        ws.append((ctx.register_device_p4(p4d, n, k), p4d))
    x = np.random.default_rng(k).standard_normal((1, k)).astype(np.float32)
    xd, yd = ctx.to_device(x), ctx.alloc(n * 4)

    def rot():
        for w, _ in ws:
            if residual:
                ctx.linear_add(xd, w, yd, yd, 1)
            else:
                ctx.linear(xd, w, yd, 1)

    timer = Timer(ctx)
    g = graph_of(ctx, rot)
    rounds = max(1, iters // copies)
    run_graph(ctx, timer, g, 2)
    ms = run_graph(ctx, timer, g, rounds)
    us = ms * 1e3 / (rounds * copies)
    nbytes = per + k * 4 + n * 4
    for w, p4d in ws:
        ctx.release(w)
        p4d.free()
    return dict(us=us, gb_s=nbytes / (us * 1e-6) / 1e9, bytes=nbytes, copies=copies)


def bench_lm_head(ctx, v=248320, k=2560, iters=20):
    """Config 3: tied lm_head with fused argmax, plus the embedding gather."""
    per = p4_bytes(v, k)
    p4d, _ = ctx.synthesize_p4(seed=77, rows=v, cols=k)
    w = ctx.register_device_p4(p4d, v, k)
    x = np.random.default_rng(v).standard_normal((1, k)).astype(np.float32)
    xd, ld, am = ctx.to_device(x), ctx.alloc(v * 4), ctx.alloc(8)
    timer = Timer(ctx)
    g = graph_of(ctx, lambda: ctx.lm_head(xd, w, ld, 1, argmax=am))
    run_graph(ctx, timer, g, 2)
    ms = run_graph(ctx, timer, g, iters)
    us = ms * 1e3 / iters
    nbytes = per + k * 4 + v * 4
    # eight gathers of 1024 ids per graph (own ids and outputs), so that a
    # graph launch's fixed cost is shared as in a real step
    reps = 8
    rng = np.random.default_rng(1024)
    tds = [ctx.to_device(rng.integers(0, v, 1024).astype(np.int64)) for _ in range(reps)]
    ods = [ctx.alloc(1024 * k * 4) for _ in range(reps)]
    g2 = graph_of(ctx, lambda: [ctx.embedding(tds[i], 1024, w, ods[i]) for i in range(reps)])
    run_graph(ctx, timer, g2, 2)
    ms2 = run_graph(ctx, timer, g2, iters)
    us2 = ms2 * 1e3 / (iters * reps)
    gather_bytes = 1024 * k * 34 // 32 + 1024 * k * 4
    ctx.release(w)
    p4d.free()
    return dict(us=us, gb_s=nbytes / (us * 1e-6) / 1e9, bytes=nbytes,
                gather_us=us2, gather_gb_s=gather_bytes / (us2 * 1e-6) / 1e9)


def bench_gemm(ctx, m, n=9216, k=2560, iters=30):
    """Config 4: the prefill linear as a caller sees it ("op": the tiled Q8_1
    quantizer plus the GEMM kernel) over a rotating pool of weight copies;
    the rates are over the whole op.  The C ABI's dense-layout quantizer is
    timed beside it for reference (the GEMM kernel alone is in the rocprofv3
    summaries)."""
    per = p4_bytes(n, k)
    copies = max(2, -(-int(1.6 * MALL_BYTES) // per)) if m <= 256 else 2
    ws = []
    for c in range(copies):
        p4d, _ = ctx.synthesize_p4(seed=7000 + c, rows=n, cols=k)
        ws.append((ctx.register_device_p4(p4d, n, k), p4d))
    x = np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)
    xd, yd = ctx.to_device(x), ctx.alloc(m * n * 4)
    qd, sd = ctx.alloc(m * k), ctx.alloc(m * k // 32 * 4)
    ctx.linear(xd, ws[0][0], yd, m, mode="prefill")  # first call sizes scratch
    ctx.sync()

    def rot():
        for w, _ in ws:
            ctx.linear(xd, w, yd, m, mode="prefill")

    def qrot():
        for _ in ws:
            ctx.quantize(xd, m, k, qd, sd)

    timer = Timer(ctx)
    g, gq = graph_of(ctx, rot), graph_of(ctx, qrot)
    rounds = max(1, iters // copies)
    run_graph(ctx, timer, g, 1)
    us = run_graph(ctx, timer, g, rounds) * 1e3 / (rounds * copies)
    run_graph(ctx, timer, gq, 1)
    q_us = run_graph(ctx, timer, gq, rounds) * 1e3 / (rounds * copies)
    for w, p4d in ws:
        ctx.release(w)
        p4d.free()
    ops = 2.0 * m * n * k
    return {"op_us": round(us, 2),
            "op_TOPS": round(ops / (us * 1e-6) / 1e12, 1),
            "frac_int8_peak": round(ops / (us * 1e-6) / 1e12 / INT8_PEAK_TOPS, 4),
            "quantize_dense_us": round(q_us, 2),
            "bytes": per + m * k * 4 + m * n * 4}


def bench_sequence(ctx, hidden=2560, ffn=9216, qkv=7680, layers=32, vocab=248320):
    """Config 5: every Q8_0 linear of a 32-layer 4B-class model plus the tied
    lm_head, all resident in HBM, at M=1 (decode) and M=1024 (prefill)."""
    shapes = [("gate", ffn, hidden), ("up", ffn, hidden), ("down", hidden, ffn),
              ("qkv", qkv, hidden), ("o", hidden, hidden), ("a", hidden, hidden),
              ("b", hidden, hidden)]
    layer = []
    total = 0
    for li in range(layers):
        ws = {}
        for j, (name, n, k) in enumerate(shapes):
            p4d, _ = ctx.synthesize_p4(seed=100000 + 16 * li + j, rows=n, cols=k)
            ws[name] = (ctx.register_device_p4(p4d, n, k), p4d)
            total += p4_bytes(n, k)
        layer.append(ws)
    p4d, _ = ctx.synthesize_p4(seed=99, rows=vocab, cols=hidden)
    head = (ctx.register_device_p4(p4d, vocab, hidden), p4d)
    total += p4_bytes(vocab, hidden)
    rng = np.random.default_rng(5)
    out = {"weight_bytes": total, "linears": layers * len(shapes) + 1}
    timer = Timer(ctx)
    for m, mode in ((1, "decode"), (1024, "prefill")):
        x = ctx.to_device(rng.standard_normal((m, hidden)).astype(np.float32))
        h = ctx.to_device(rng.standard_normal((m, ffn)).astype(np.float32))
        yq, yh = ctx.alloc(m * qkv * 4), ctx.alloc(m * ffn * 4)
        y = ctx.alloc(m * hidden * 4)
        logits, am = ctx.alloc(vocab * 4), ctx.alloc(8)

        def step():
            for ws in layer:
                ctx.linear(x, ws["qkv"][0], yq, m, mode=mode)
                for nm in ("o", "a", "b"):
                    ctx.linear(x, ws[nm][0], y, m, mode=mode)
                if m == 1:
                    ctx.mlp(x, ws["gate"][0], ws["up"][0], ws["down"][0], y, h=yh)
                else:
                    ctx.swiglu(x, ws["gate"][0], ws["up"][0], yh, m, mode=mode)
                    ctx.linear(h, ws["down"][0], y, m, mode=mode)
            ctx.lm_head(x, head[0], logits, 1, argmax=am, mode=mode)

        step()  # sizes scratch outside capture
        ctx.sync()
        g = graph_of(ctx, step)
        run_graph(ctx, timer, g, 1)
        reps = 10 if m == 1 else 3
        us = run_graph(ctx, timer, g, reps) * 1e3 / reps
        ops = 2.0 * m * (total - p4_bytes(vocab, hidden)) * 32 / 34 + 2.0 * vocab * hidden
        key = "m%d" % m
        out[key] = {"us": round(us, 1), "GB/s": round(total / (us * 1e-6) / 1e9, 1),
                    "TOPS": round(ops / (us * 1e-6) / 1e12, 2)}
    for ws in layer:
        for w, p4d in ws.values():
            ctx.release(w)
            p4d.free()
    ctx.release(head[0])
    head[1].free()
    return out


def bench_arena(ctx, q8, hidden=2560, ffn=9216, qkv=7680, layers=32, vocab=248320):
    """The whole config-5 model from one LLMCPWGT arena file, as the AOT
    runtime loads it: written once (synthetic weights of the sequence's
    shapes), mapped, uploaded by llmcp_q8_upload_arena (validation, host ->
    HBM copies, device repack), then one decode step run through weight
    descriptors that point into the mapping."""
    import struct
    import tempfile
    shapes = [("gate", ffn, hidden), ("up", ffn, hidden), ("down", hidden, ffn),
              ("qkv", qkv, hidden), ("o", hidden, hidden), ("a", hidden, hidden),
              ("b", hidden, hidden)]
    tensors = []
    for li in range(layers):
        for j, (name, n, k) in enumerate(shapes):
            p4d, _ = ctx.synthesize_p4(seed=200000 + 16 * li + j, rows=n, cols=k)
            tensors.append(("model.layers.%d.%s.weight" % (li, name), n, k,
                            ctx.to_host(p4d, (p4d.nbytes,), np.uint8)))
            p4d.free()
    p4d, _ = ctx.synthesize_p4(seed=199, rows=vocab, cols=hidden)
    tensors.append(("model.embed_tokens.weight", vocab, hidden,
                    ctx.to_host(p4d, (p4d.nbytes,), np.uint8)))
    p4d.free()
    d = "/dev/shm" if os.path.isdir("/dev/shm") else tempfile.gettempdir()
    path = os.path.join(d, "llmcp_q8_bench_arena_%d.bin" % os.getpid())
    try:
        t0 = time.perf_counter()
        q8.write_arena(path, tensors)
        write_s = time.perf_counter() - t0
        del tensors
        f = np.memmap(path, dtype=np.uint8, mode="r")
        ctx.sync()
        t0 = time.perf_counter()
        count = ctx.upload_arena(f)
        ctx.sync()
        upload_s = time.perf_counter() - t0
        arena = struct.unpack_from("<Q", f, 16)[0]
        entries = json.loads(bytes(f[arena:]).decode())["tensors"]
        w = {e["name"]: q8.Weight(ctx, f.ctypes.data + e["offset"], e["shape"][0],
                                  e["shape"][1], owner=f) for e in entries}
        rng = np.random.default_rng(6)
        x = ctx.to_device(rng.standard_normal((1, hidden)).astype(np.float32))
        yq, yh = ctx.alloc(qkv * 4), ctx.alloc(ffn * 4)
        y, logits, am = ctx.alloc(hidden * 4), ctx.alloc(vocab * 4), ctx.alloc(8)

        def step():
            for li in range(layers):
                pre = "model.layers.%d." % li
                ctx.linear(x, w[pre + "qkv.weight"], yq, 1)
                for nm in ("o", "a", "b"):
                    ctx.linear(x, w[pre + nm + ".weight"], y, 1)
                ctx.mlp(x, w[pre + "gate.weight"], w[pre + "up.weight"],
                        w[pre + "down.weight"], y, h=yh)
            ctx.lm_head(x, w["model.embed_tokens.weight"], logits, 1, argmax=am)

        step()
        ctx.sync()
        timer = Timer(ctx)
        g = graph_of(ctx, step)
        run_graph(ctx, timer, g, 1)
        step_us = run_graph(ctx, timer, g, 5) * 1e3 / 5
        for wt in w.values():
            ctx.release(wt)
        nbytes = int(f.nbytes)
        del w, f
    finally:
        if os.path.exists(path):
            os.unlink(path)
    return {"file_bytes": nbytes, "q8_tensors": count, "write_s": round(write_s, 2),
            "upload_s": round(upload_s, 3), "upload_GB/s": round(nbytes / upload_s / 1e9, 2),
            "decode_step_us": round(step_us, 1)}


def cpu_baseline(res, budget_s=12.0):
    """Reference x86 scalar Q8 path (oracle restatement) on the host cores."""
    from oracle import q8_oracle as o
    o.set_threads(int(os.environ.get("OMP_NUM_THREADS", "16")))
    x = res["x"]
    pg, pu, pd = res["host_p4"]
    hidden, ffn = res["hidden"], res["ffn"]
    t0 = time.perf_counter()
    n = 0
    while True:
        h = o.swiglu(x, pg, pu, ffn)              # row-parallel: 1 thread at M=1
        o.linear(h, pd, hidden)
        n += 1
        if time.perf_counter() - t0 > budget_s or n >= 250:
            break
    dt = (time.perf_counter() - t0) / n
    t0 = time.perf_counter()
    m = 0
    while True:
        h = o.swiglu(x, pg, pu, ffn, colpar=True)
        o.linear(h, pd, hidden, colpar=True)
        m += 1
        if time.perf_counter() - t0 > budget_s / 2 or m >= 200:
            break
    dt_col = (time.perf_counter() - t0) / m
    # Config 4's GEMM on the same path: the scalar GEMM is row-parallel over
    # M (Q8Scalar.cpp:84,127), so a 64-row sample on all threads gives its
    # per-row rate, which holds for M = 1024.
    rows = 64
    xg = np.random.default_rng(4).standard_normal((rows, hidden)).astype(np.float32)
    t0 = time.perf_counter()
    k = 0
    while True:
        o.linear(xg, pg, ffn)
        k += 1
        if time.perf_counter() - t0 > budget_s / 4 or k >= 50:
            break
    dt_g = (time.perf_counter() - t0) / k
    gemm_ops = 2.0 * rows * ffn * hidden
    return dict(value=res["step_bytes"] / dt / 1e9, unit="GB/s", cores=1,
                kind="port",
                sample="%d decode-MLP steps (2560->9216 x2 SwiGLU, 9216->2560) on one "
                       "weight copy, scalar epilogue, row-parallel OpenMP as "
                       "Q8Scalar.cpp:84,127 (M=1 -> 1 thread); %.1f ms/step" % (n, dt * 1e3),
                colpar_value=res["step_bytes"] / dt_col / 1e9,
                colpar_threads=o.max_threads(),
                colpar_ms_per_step=dt_col * 1e3,
                gemm={"TOPS": round(gemm_ops / dt_g / 1e12, 4), "threads": o.max_threads(),
                      "sample": "%d-row samples of config 4 (K=2560 -> N=9216), scalar "
                                "epilogue, row-parallel OpenMP; %d calls" % (rows, k),
                      "ms_per_m1024_call": round(dt_g * 1024 / rows * 1e3, 1)})


def copy_calibration(ctx, nbytes=256 << 20, reps=10):
    """A plain device copy of known size (HIP's copy kernel), run under
    rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE to scale the counters."""
    a, b = ctx.alloc(nbytes), ctx.alloc(nbytes)
    q8lib = __import__("llmcp_amd").lib()
    for _ in range(reps):
        q8lib.llmcp_q8_memcpy_d2d(ctx.handle, b.ptr, a.ptr, nbytes)
    ctx.sync()
    a.free()
    b.free()
    return {"copy_bytes": nbytes, "reps": reps}


def load_traffic():
    """HBM bytes per launch of the dominant kernel, from the committed
    rocprofv3 --pmc summary (FETCH_SIZE, WRITE_SIZE, copy-calibrated)."""
    path = os.path.join(ROOT, "profiles", "gemv_gateup_decode_mlp_traffic.json")
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=600)
    ap.add_argument("--warmup", type=int, default=60)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a 256 MiB device copy (counter calibration)")
    ap.add_argument("--arena", action="store_true",
                    help="also load the 32-layer model from a 4.4 GB arena "
                         "file (written to /dev/shm) and time the upload")
    ap.add_argument("--gemm-only", type=int, default=0, metavar="M",
                    help="time only config 4's prefill GEMM at M rows and print "
                         "its figures (a short run for counter collection)")
    ap.add_argument("--platform", choices=("aarch64", "x86"), default="aarch64",
                    help="reference arithmetic to reproduce: the SDOT paths' "
                         "fma epilogue (default) or the x86 scalar path's")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the Q8_0 linear path runs on a single "
              "MI355X in this build (multi-GPU sharding is a design note only); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import llmcp_amd as q8
    ctx = q8.Context(0)
    ctx.set_platform(args.platform)
    if args.copy_calibration:
        copy_calibration(ctx)
    if args.gemm_only:
        r = bench_gemm(ctx, args.gemm_only)
        print(json.dumps({"gemm_m%d_n9216_k2560" % args.gemm_only: r}), flush=True)
        return
    res = bench_decode_mlp(ctx, q8, args.steps, args.warmup)
    extra = {}
    if not args.no_extra:
        c1 = bench_gemv(ctx, 2560, 2560)
        extra["gemv_2560x2560"] = {"us": round(c1["us"], 3), "GB/s": round(c1["gb_s"], 1),
                                   "frac_hbm": round(c1["gb_s"] / HBM_PEAK_GBS, 4)}
        c1a = bench_gemv(ctx, 2560, 2560, residual=True)
        extra["gemv_2560x2560_residual_add"] = {"us": round(c1a["us"], 3)}
        c3 = bench_lm_head(ctx)
        extra["lm_head_248320x2560_argmax"] = {
            "us": round(c3["us"], 2), "GB/s": round(c3["gb_s"], 1),
            "frac_hbm": round(c3["gb_s"] / HBM_PEAK_GBS, 4)}
        extra["embedding_gather_1024"] = {"us": round(c3["gather_us"], 2),
                                          "GB/s": round(c3["gather_gb_s"], 1)}
        for m in (64, 256, 1024):
            extra["gemm_m%d_n9216_k2560" % m] = bench_gemm(ctx, m)
        extra["sequence_32_layers"] = bench_sequence(ctx)
    if args.arena:
        extra["arena_32_layers"] = bench_arena(ctx, q8)
    cpu = None if args.no_cpu else cpu_baseline(res)
    line = {
        "metric": "Q8_0 linear: M=1 GEMV HBM GB/s (% peak); M=1024 GEMM int8 TOPS (% peak)",
        "value": round(res["gb_s"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": res["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(res["ms"] / res["steps"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "decode_mlp_m1 (configs[1]): gate/up 2560->9216 fused "
                               "silu*up, down 9216->2560, Q8_0 N(0,0.02) weights",
                   "hidden": res["hidden"], "ffn": res["ffn"],
                   "step_bytes": res["step_bytes"],
                   "weight_pool_bytes": res["pool_bytes"],
                   "weight_copies": res["copies"],
                   "frac_hbm_peak": round(res["gb_s"] / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(res["gu_gbs"], 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(res["gu_gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": (load_traffic() or {}).get("hbm_bytes_per_launch"),
                     "kernel": "gemv_kernel<2,false,IN_WG,4,4,5,0> (fused gate/up "
                               "SwiGLU, 4-wave workgroups, input row quantized "
                               "per workgroup; timed alone via llmcp_q8_swiglu)",
                     "launch_us": round(res["gu_launch_us"], 3),
                     "algorithmic_bytes": res["gu_bytes"],
                     "down_launch_us": round(res["down_launch_us"], 3),
                     "graph_kernel_floor_us": round(res["tiny_launch_us"], 3)},
        "cpu_baseline": None if cpu is None else {
            k: (round(v, 3) if isinstance(v, float) else v) for k, v in cpu.items()},
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
