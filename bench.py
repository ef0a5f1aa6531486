"""Benchmark of the MI355X Q8_0 linear path (one GPU).

Headline workload: the decode MLP at M=1 --
gate and up Q8_0 projections 2560 -> 9216 with the fused silu(gate)*up
epilogue, then the Q8_0 down projection 9216 -> 2560.  A step is one pass of
that MLP over one synthetic input row, activation quantization included.
Weights are N(0, 0.02) synthesized on the device and packed to q8_0_p4; the
steps cycle through distinct weight copies larger together than the 256 MB
Infinity Cache, which keeps the timing on HBM.  The timed steps (exactly
--steps of them, after exactly --warmup untimed ones) are replayed from one
HIP graph, so host launch cost stays out of the timed region.  The
arithmetic is the selected reference platform's (--platform, default the
aarch64 SDOT paths' fma epilogue).

`value` = whole-step algorithmic bytes / time (GB/s).  `roofline` = the fused
gate/up GEMV (the dominant kernel) timed alone the same way with HIP events
on the library's stream.  `extra` = the other configs (config 1 GEMV, config
3 lm_head + argmax and gather, config 4 GEMMs at M = 64/256/1024, config 5
sequence at M = 1 and 1024, the real model's arena upload and decode step)
and the one-time device repack of each tensor shape.  `cpu_baseline` = the
oracle's C restatement of the reference's x86 scalar Q8 path on bounded
samples of every config, with the host described.

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


# --eager: every timed block runs as plain launches instead of a captured
# graph (for kernel tracers, whose graph replay handling is not needed to
# read per-kernel durations); the printed figures then include launch cost.
EAGER = False


def graph_of(ctx, fn):
    if EAGER:
        return fn
    ctx.sync()
    ctx.graph_begin()
    fn()
    return ctx.graph_end()


def graph_free(ctx, graph):
    if not EAGER:
        ctx.graph_destroy(graph)


def run_graph(ctx, timer, graph, launches):
    ctx.sync()
    timer.start()
    for _ in range(launches):
        if EAGER:
            graph()
        else:
            ctx.graph_launch(graph)
    ms = timer.stop_ms()
    ctx.sync()
    return ms


def bench_decode_mlp(ctx, q8, steps, warmup, hidden=2560, ffn=9216):
    per_copy = 2 * p4_bytes(ffn, hidden) + p4_bytes(hidden, ffn)
    copies = max(2, -(-int(1.6 * MALL_BYTES) // per_copy))
    log("decode_mlp: %d weight copies x %.1f MB" % (copies, per_copy / 1e6))
    pool = []
    repack_ms = {}
    for c in range(copies):
        mats = []
        for i, (n, k) in enumerate([(ffn, hidden), (ffn, hidden), (hidden, ffn)]):
            p4d, _ = ctx.synthesize_p4(seed=1000 + 10 * c + i, rows=n, cols=k)
            w = ctx.register_device_p4(p4d, n, k, time_repack=(c == 0))
            if c == 0:
                repack_ms["%dx%d" % (n, k)] = round(w.repack_ms, 3)
            mats.append((w, p4d))
        pool.append(mats)
    rng = np.random.default_rng(2560)
    x = rng.standard_normal((1, hidden)).astype(np.float32)
    xd, hd, yd = ctx.to_device(x), ctx.alloc(ffn * 4), ctx.alloc(hidden * 4)

    # Graphs of exactly n steps, cycling through the weight copies, so the
    # timed region holds exactly `steps` steps (and the warmup `warmup`).
    def mlp_steps(n):
        return lambda: [ctx.mlp(xd, pool[i % copies][0][0], pool[i % copies][1][0],
                                pool[i % copies][2][0], yd, h=hd) for i in range(n)]

    def gateup_steps(n):
        return lambda: [ctx.swiglu(xd, pool[i % copies][0][0], pool[i % copies][1][0],
                                   hd, 1) for i in range(n)]

    def down_steps(n):
        return lambda: [ctx.linear(hd, pool[i % copies][2][0], yd, 1) for i in range(n)]

    timer = Timer(ctx)

    def timed(make):
        if warmup:
            gw = graph_of(ctx, make(warmup))
            run_graph(ctx, timer, gw, 1)
            graph_free(ctx, gw)
        g = graph_of(ctx, make(steps))
        ms = run_graph(ctx, timer, g, 1)
        graph_free(ctx, g)
        return ms

    ms = timed(mlp_steps)
    step_bytes = (per_copy + hidden * 4 + 2 * ffn * 4 + hidden * 4)
    gb_s = step_bytes * steps / (ms * 1e-3) / 1e9
    gu_launch_us = timed(gateup_steps) * 1e3 / steps
    down_launch_us = timed(down_steps) * 1e3 / steps
    gu_bytes = 2 * p4_bytes(ffn, hidden) + hidden * 4 + ffn * 4
    gu_gbs = gu_bytes / (gu_launch_us * 1e-6) / 1e9
    down_bytes = p4_bytes(hidden, ffn) + ffn * 4 + hidden * 4

    # keep one copy's packed bytes for the CPU baseline
    host = [ctx.to_host(m[1], (m[1].nbytes,), np.uint8) for m in pool[0]]
    res = dict(ms=ms, steps=steps, gb_s=gb_s, step_bytes=step_bytes,
               copies=copies, pool_bytes=copies * per_copy,
               gu_launch_us=gu_launch_us, gu_bytes=gu_bytes, gu_gbs=gu_gbs,
               down_launch_us=down_launch_us, down_bytes=down_bytes,
               repack_ms=repack_ms, x=x, host_p4=host, hidden=hidden, ffn=ffn)
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
        ws.append((ctx.register_device_p4(p4d, n, k, time_repack=(c == 0)), p4d))
    repack_ms = ws[0][0].repack_ms
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
    host_p4 = ctx.to_host(ws[0][1], (per,), np.uint8)
    for w, p4d in ws:
        ctx.release(w)
        p4d.free()
    return dict(us=us, gb_s=nbytes / (us * 1e-6) / 1e9, bytes=nbytes, copies=copies,
                repack_ms=repack_ms, p4=host_p4)


def bench_lm_head(ctx, v=248320, k=2560, iters=20):
    """Config 3: tied lm_head with fused argmax, plus the embedding gather."""
    per = p4_bytes(v, k)
    p4d, _ = ctx.synthesize_p4(seed=77, rows=v, cols=k)
    w = ctx.register_device_p4(p4d, v, k, time_repack=True)
    x = np.random.default_rng(v).standard_normal((1, k)).astype(np.float32)
    xd, ld, am = ctx.to_device(x), ctx.alloc(v * 4), ctx.alloc(8)
    timer = Timer(ctx)
    g = graph_of(ctx, lambda: ctx.lm_head(xd, w, ld, 1, argmax=am))
    run_graph(ctx, timer, g, 2)
    ms = run_graph(ctx, timer, g, iters)
    us = ms * 1e3 / iters
    nbytes = per + k * 4 + v * 4
    # 32 gathers of 1024 ids per graph, each with its own id set and output
    # (together ~690 MB of touched records and outputs, past the 256 MB
    # Infinity Cache, so that the figure is not served from it), so that a
    # graph launch's fixed cost is shared as in a real step
    reps, sets = 32, 32
    rng = np.random.default_rng(1024)
    tds = [ctx.to_device(rng.integers(0, v, 1024).astype(np.int64)) for _ in range(sets)]
    ods = [ctx.alloc(1024 * k * 4) for _ in range(sets)]
    g2 = graph_of(ctx, lambda: [ctx.embedding(tds[i % sets], 1024, w, ods[i % sets])
                                for i in range(reps)])
    run_graph(ctx, timer, g2, 2)
    ms2 = run_graph(ctx, timer, g2, iters)
    us2 = ms2 * 1e3 / (iters * reps)
    gather_bytes = 1024 * k * 34 // 32 + 1024 * k * 4
    host_p4 = ctx.to_host(p4d, (per,), np.uint8)
    ctx.release(w)
    p4d.free()
    return dict(us=us, gb_s=nbytes / (us * 1e-6) / 1e9, bytes=nbytes,
                gather_us=us2, gather_gb_s=gather_bytes / (us2 * 1e-6) / 1e9,
                repack_ms=w.repack_ms, p4=host_p4, x=x)


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

    # as many quantizer launches per graph as the GEMM's smallest rotation
    # would need, so that the graph launch's own cost is shared
    nq = max(16, copies)

    def qrot():
        for _ in range(nq):
            ctx.quantize(xd, m, k, qd, sd)

    timer = Timer(ctx)
    g, gq = graph_of(ctx, rot), graph_of(ctx, qrot)
    rounds = max(1, iters // copies)
    run_graph(ctx, timer, g, 1)
    us = run_graph(ctx, timer, g, rounds) * 1e3 / (rounds * copies)
    run_graph(ctx, timer, gq, 1)
    q_us = run_graph(ctx, timer, gq, rounds) * 1e3 / (rounds * nq)
    for w, p4d in ws:
        ctx.release(w)
        p4d.free()
    ops = 2.0 * m * n * k
    return {"op_us": round(us, 2),
            "op_TOPS": round(ops / (us * 1e-6) / 1e12, 1),
            "frac_int8_peak": round(ops / (us * 1e-6) / 1e12 / INT8_PEAK_TOPS, 4),
            "quantize_dense_us": round(q_us, 2),
            "bytes": per + m * k * 4 + m * n * 4}


def bench_split_k(ctx, n=2560, k=9216, ms=(64, 256)):
    """The SPLIT_K accumulation mode (opt-in, within the north-star
    tolerance) against EXACT on the down projection's shape at few rows,
    where K = 9216 runs 72 serial stages per tile: op times of the same
    calls in both modes (the count of splits is the library's choice)."""
    out = {}
    for m in ms:
        fig = {}
        for mode in ("exact", "split_k"):
            ctx.set_accumulation(mode)
            fig[mode + "_op_us"] = bench_gemm(ctx, m, n=n, k=k, iters=20)["op_us"]
        ctx.set_accumulation("exact")
        fig["speedup"] = round(fig["exact_op_us"] / fig["split_k_op_us"], 2)
        out["m%d" % m] = fig
    return out


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
            ws[name] = (ctx.register_device_p4(p4d, n, k, time_repack=(li == 0)), p4d)
            total += p4_bytes(n, k)
        layer.append(ws)
    qkv_repack_ms = layer[0]["qkv"][0].repack_ms
    qkv_p4 = ctx.to_host(layer[0]["qkv"][1], (p4_bytes(qkv, hidden),), np.uint8)
    p4d, _ = ctx.synthesize_p4(seed=99, rows=vocab, cols=hidden)
    head = (ctx.register_device_p4(p4d, vocab, hidden), p4d)
    total += p4_bytes(vocab, hidden)
    rng = np.random.default_rng(5)
    out = {"weight_bytes": total, "linears": layers * len(shapes) + 1,
           "_qkv_repack_ms": qkv_repack_ms, "_qkv_p4": qkv_p4}
    timer = Timer(ctx)
    for m, mode in ((1, "decode"), (1024, "prefill")):
        x = ctx.to_device(rng.standard_normal((m, hidden)).astype(np.float32))
        h = ctx.to_device(rng.standard_normal((m, ffn)).astype(np.float32))
        yq, yh = ctx.alloc(m * qkv * 4), ctx.alloc(m * ffn * 4)
        y = ctx.alloc(m * hidden * 4)
        logits, am = ctx.alloc(vocab * 4), ctx.alloc(8)

        ya, yb = ctx.alloc(m * hidden * 4), ctx.alloc(m * hidden * 4)

        def step(grouped=False):
            for ws in layer:
                if grouped:
                    # the four linears of one input as one group
                    ctx.linear_group(x, [ws[nm][0] for nm in ("qkv", "o", "a", "b")],
                                     [yq, y, ya, yb], m, mode=mode)
                else:
                    ctx.linear(x, ws["qkv"][0], yq, m, mode=mode)
                    for nm in ("o", "a", "b"):
                        ctx.linear(x, ws[nm][0], y, m, mode=mode)
                if m == 1:
                    ctx.mlp(x, ws["gate"][0], ws["up"][0], ws["down"][0], y, h=yh)
                else:
                    ctx.swiglu(x, ws["gate"][0], ws["up"][0], yh, m, mode=mode)
                    ctx.linear(h, ws["down"][0], y, m, mode=mode)
            ctx.lm_head(x, head[0], logits, 1, argmax=am, mode=mode)

        ops = 2.0 * m * (total - p4_bytes(vocab, hidden)) * 32 / 34 + 2.0 * vocab * hidden
        key = "m%d" % m
        for grouped in (False, True):
            step(grouped)  # sizes scratch outside capture
            ctx.sync()
            g = graph_of(ctx, lambda: step(grouped))
            run_graph(ctx, timer, g, 1)
            reps = 10 if m == 1 else 3
            us = run_graph(ctx, timer, g, reps) * 1e3 / reps
            graph_free(ctx, g)
            fig = {"us": round(us, 1), "GB/s": round(total / (us * 1e-6) / 1e9, 1),
                   "TOPS": round(ops / (us * 1e-6) / 1e12, 2)}
            if grouped:
                out[key]["grouped"] = fig
            else:
                out[key] = fig
    for ws in layer:
        for w, p4d in ws.values():
            ctx.release(w)
            p4d.free()
    ctx.release(head[0])
    head[1].free()
    return out


def bench_norms(ctx, q8, iters=50):
    """The RMSNorm neighbour (llmcp_q8_rmsnorm, gated RMSNorm) at the 4B
    model's shapes in bf16, and the fused RMSNorm + grouped linears against
    the two calls apart.  Each figure is one graph of `iters` calls."""
    rng = np.random.default_rng(12)
    timer = Timer(ctx)

    def timed(fn):
        fn()
        ctx.sync()
        g = graph_of(ctx, lambda: [fn() for _ in range(iters)])
        run_graph(ctx, timer, g, 1)
        us = run_graph(ctx, timer, g, 3) * 1e3 / (3 * iters)
        graph_free(ctx, g)
        return round(us, 2)

    out = {}
    h = 2560
    w = ctx.to_device((rng.standard_normal(h) * 0.1).astype(np.float32).view(np.uint32)
                      .__rshift__(16).astype(np.uint16))
    for m in (1, 1024):
        x = ctx.to_device((rng.standard_normal((m, h)).astype(np.float32).view(np.uint32)
                           >> 16).astype(np.uint16))
        y = ctx.alloc(m * h * 2)
        out["rmsnorm_bf16_m%d_us" % m] = timed(
            lambda: ctx.rmsnorm(x, w, y, m, h, zero_centered=True, dtype="bf16"))
    z = ctx.to_device((rng.standard_normal((1, 4096)).astype(np.float32).view(np.uint32)
                       >> 16).astype(np.uint16))
    gw = ctx.to_device((rng.standard_normal(128) * 0.1 + 1).astype(np.float32))
    gy = ctx.alloc(4096 * 2)
    out["gated_rmsnorm_bf16_m1_4096_us"] = timed(
        lambda: ctx.gated_rmsnorm(z, z, gw, gy, 1, 4096, 128, dtype="bf16"))
    shapes = [(8192, h), (4096, h), (32, h), (32, h)]
    ws = []
    for n, k in shapes:
        d, _ = ctx.synthesize_p4(seed=n + 5, rows=n, cols=k)
        ws.append((ctx.register_device_p4(d, n, k), d))
    ts = [t for t, _ in ws]
    for m in (1, 1024):
        x = ctx.to_device((rng.standard_normal((m, h)).astype(np.float32).view(np.uint32)
                           >> 16).astype(np.uint16))
        nd = ctx.alloc(m * h * 2)
        outs = [ctx.alloc(m * n * 2) for n, _ in shapes]
        mode = "decode" if m == 1 else "prefill"
        fused = timed(lambda: ctx.rmsnorm_linear_group(
            x, w, nd, ts, outs, m, zero_centered=True, mode=mode, dtype="bf16"))

        def apart():
            ctx.rmsnorm(x, w, nd, m, h, zero_centered=True, dtype="bf16")
            ctx.linear_group(nd, ts, outs, m, mode=mode, dtype="bf16")
        out["norm_qkvzab_m%d" % m] = {"fused_us": fused, "separate_us": timed(apart)}
    for t, d in ws:
        ctx.release(t)
        d.free()
    return out


def bench_arena(ctx, q8):
    """The real 4B-class model's arena (426 tensors: Q8_0 matmul weights and
    tied table, BF16/F32 norms and conv/gate parameters; 4.47 GB laid out as
    WeightLayout::build does), written to a file, mapped and uploaded whole
    by llmcp_q8_upload_arena (validation, host -> HBM copies, device repack)
    as the AOT runtime would; then one decode step of all 249 Q8_0 linears
    (every layer's projections and MLP, the last-row lm_head with argmax)
    through weight descriptors that point into the mapping."""
    import tempfile
    from llmcp_amd import model_arena
    t0 = time.perf_counter()
    image, entries = model_arena.build_image(seed=11)
    build_s = time.perf_counter() - t0
    d = "/dev/shm" if os.path.isdir("/dev/shm") else tempfile.gettempdir()
    path = os.path.join(d, "llmcp_q8_bench_arena_%d.bin" % os.getpid())
    try:
        image.tofile(path)
        del image
        f = np.memmap(path, dtype=np.uint8, mode="r")
        ctx.sync()
        t0 = time.perf_counter()
        count = ctx.upload_arena(f)
        ctx.sync()
        upload_s = time.perf_counter() - t0
        w = {e["name"]: q8.Weight(ctx, f.ctypes.data + e["offset"], e["shape"][0],
                                  e["shape"][1], owner=f)
             for e in entries if e["dtype"] == "Q8_0"}
        cfg = model_arena.CONFIG_4B
        hidden, vocab = cfg["hidden"], cfg["vocab"]
        rng = np.random.default_rng(6)
        x = ctx.to_device(rng.standard_normal((1, hidden)).astype(np.float32))
        xv = ctx.to_device(rng.standard_normal((1, 4096)).astype(np.float32))
        out = ctx.alloc(16384 * 4)
        h = ctx.alloc(cfg["intermediate"] * 4)
        logits, am = ctx.alloc(vocab * 4), ctx.alloc(8)
        names = sorted(w)

        outs = [ctx.alloc(8192 * 4) for _ in range(4)]

        # bf16 decode layers as the model builder chains them
        # (ModelBuilder.cpp:219-275, :280-340): input_layernorm fused with
        # the shared-input linears, the gated norm before out_proj (linear
        # attention), out_proj / o_proj with the residual add, the
        # post-attention norm, the SwiGLU pair and down with the residual
        # add.  The mixers' own ops (conv, delta rule, attention) are not
        # Q8 linears and are stood in for by fixed inputs.
        def bf16_of(a):
            return (a.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        xb = ctx.to_device(bf16_of(rng.standard_normal((1, hidden))))
        rb, nb = ctx.alloc(hidden * 2), ctx.alloc(hidden * 2)
        vb = ctx.to_device(bf16_of(rng.standard_normal((1, 4096))))
        gb = ctx.alloc(4096 * 2)
        hb = ctx.alloc(cfg["intermediate"] * 2)
        lnw = ctx.to_device(bf16_of(rng.standard_normal(hidden) * 0.1))
        gnw = ctx.to_device((rng.standard_normal(128) * 0.1 + 1).astype(np.float32))
        outs_b = [ctx.alloc(8192 * 2) for _ in range(4)]

        def layer_step():
            for layer in range(cfg["layers"]):
                pre = "model.language_model.layers.%d." % layer
                mix = [nm for nm in names if nm.startswith(pre) and ".mlp." not in nm]
                shared = [nm for nm in mix if w[nm].cols == hidden]
                ctx.rmsnorm_linear_group(xb, lnw, nb, [w[nm] for nm in shared],
                                         outs_b[:len(shared)], 1, zero_centered=True,
                                         dtype="bf16")
                proj = [nm for nm in mix if w[nm].cols == 4096][0]
                if "linear_attn" in proj:
                    zi = shared.index(pre + "linear_attn.in_proj_z.weight")
                    ctx.gated_rmsnorm(vb, outs_b[zi], gnw, gb, 1, 4096, 128, dtype="bf16")
                    ctx.linear_add(gb, w[proj], xb, rb, 1, dtype="bf16")
                else:
                    ctx.linear_add(vb, w[proj], xb, rb, 1, dtype="bf16")
                ctx.rmsnorm(rb, lnw, nb, 1, hidden, zero_centered=True, dtype="bf16")
                ctx.swiglu(nb, w[pre + "mlp.gate_proj.weight"], w[pre + "mlp.up_proj.weight"],
                           hb, 1, dtype="bf16")
                ctx.linear_add(hb, w[pre + "mlp.down_proj.weight"], rb, xb, 1, dtype="bf16")
            ctx.rmsnorm(xb, lnw, nb, 1, hidden, zero_centered=True, dtype="bf16")
            ctx.lm_head(nb, w["model.language_model.embed_tokens.weight"], logits, 1,
                        argmax=am, dtype="bf16")

        def step(grouped=False):
            for layer in range(cfg["layers"]):
                pre = "model.language_model.layers.%d." % layer
                mix = [nm for nm in names if nm.startswith(pre) and ".mlp." not in nm]
                shared = [nm for nm in mix if w[nm].cols == hidden]  # the normed input's
                for nm in mix:
                    if not grouped or nm not in shared:
                        ctx.linear(xv if w[nm].cols == 4096 else x, w[nm], out, 1)
                if grouped:
                    # qkv/z/a/b (linear attention) or q/k/v (full attention)
                    ctx.linear_group(x, [w[nm] for nm in shared], outs[:len(shared)], 1)
                ctx.mlp(x, w[pre + "mlp.gate_proj.weight"], w[pre + "mlp.up_proj.weight"],
                        w[pre + "mlp.down_proj.weight"], out, h=h)
            ctx.lm_head(x, w["model.language_model.embed_tokens.weight"], logits, 1,
                        argmax=am)

        timer = Timer(ctx)
        step_us = {}
        for grouped in (False, True, "layers"):
            fn = layer_step if grouped == "layers" else (lambda: step(grouped))
            fn()
            ctx.sync()
            g = graph_of(ctx, fn)
            run_graph(ctx, timer, g, 1)
            step_us[grouped] = run_graph(ctx, timer, g, 5) * 1e3 / 5
            graph_free(ctx, g)
        q8_bytes = sum(e["size"] for e in entries if e["dtype"] == "Q8_0")
        for wt in w.values():
            ctx.release(wt)
        nbytes = int(f.nbytes)
        del w, f
    finally:
        if os.path.exists(path):
            os.unlink(path)
    return {"file_bytes": nbytes, "tensors": len(entries), "q8_tensors": count,
            "build_s": round(build_s, 2),
            "upload_s": round(upload_s, 3), "upload_GB/s": round(nbytes / upload_s / 1e9, 2),
            "decode_step_us": round(step_us[False], 1),
            "decode_step_GB/s": round(q8_bytes / (step_us[False] * 1e-6) / 1e9, 1),
            "decode_step_grouped_us": round(step_us[True], 1),
            "decode_step_grouped_GB/s": round(q8_bytes / (step_us[True] * 1e-6) / 1e9, 1),
            "decode_step_bf16_layers_with_norms_us": round(step_us["layers"], 1)}


def host_description():
    """The GPU box's host as the CPU baseline sees it."""
    model = ""
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count()
    return {"nproc": os.cpu_count(), "affinity_cpus": affinity, "model": model}


def _timed(fn, budget_s, max_calls):
    t0 = time.perf_counter()
    n = 0
    while True:
        fn()
        n += 1
        if time.perf_counter() - t0 > budget_s or n >= max_calls:
            return (time.perf_counter() - t0) / n, n


def cpu_baseline(res, c1, c3, seq, budget_s=18.0):
    """The reference's x86 Q8 CPU path (the oracle's C restatement of
    ScalarQ8::emit, Q8Scalar.cpp:65-212, scalar epilogue) on the host cores,
    on bounded samples of each config.  The reference parallelises that path
    over rows only (Q8Scalar.cpp:84,127), so every M = 1 figure runs on one
    thread; the multi-row GEMM runs row-parallel on all threads the box
    allots (OMP_NUM_THREADS, else the process's CPU affinity).  A
    column-parallel variant of the decode MLP on those threads is labelled
    as such."""
    from oracle import q8_oracle as o
    host = host_description()
    threads = int(os.environ.get("OMP_NUM_THREADS") or host["affinity_cpus"] or 1)
    o.set_threads(threads)
    host["omp_max_threads"] = o.max_threads()
    x = res["x"]
    pg, pu, pd = res["host_p4"]
    hidden, ffn = res["hidden"], res["ffn"]

    def mlp():
        o.linear(o.swiglu(x, pg, pu, ffn), pd, hidden)

    dt, n = _timed(mlp, budget_s * 0.3, 250)
    dt_col, m_col = _timed(lambda: o.linear(o.swiglu(x, pg, pu, ffn, colpar=True),
                                            pd, hidden, colpar=True),
                           budget_s * 0.1, 200)
    # config 1: one 2560 x 2560 GEMV (one thread at M = 1)
    x1 = np.random.default_rng(1).standard_normal((1, 2560)).astype(np.float32)
    dt1, n1 = _timed(lambda: o.linear(x1, c1["p4"], 2560), budget_s * 0.08, 500)
    # config 3: the 248320 x 2560 lm_head row and its first-max argmax, and
    # the 1024-id gather
    x3 = c3["x"]
    dt3, n3 = _timed(lambda: o.argmax(o.linear(x3, c3["p4"], 248320)),
                     budget_s * 0.15, 20)
    ids = np.random.default_rng(3).integers(0, 248320, 1024).astype(np.int64)
    dtg, ng = _timed(lambda: o.embedding(ids, c3["p4"], 2560), budget_s * 0.03, 200)
    # config 4: M = 1024 GEMM, row-parallel; a 256-row sample on all threads
    # gives the per-row rate, which a 1024-row call keeps (rows are
    # independent and equal in cost)
    rows = 256
    xg = np.random.default_rng(4).standard_normal((rows, hidden)).astype(np.float32)
    dtg4, ng4 = _timed(lambda: o.linear(xg, pg, ffn), budget_s * 0.12, 20)
    gemm_ops = 2.0 * rows * ffn * hidden
    # config 5: the 32-layer sequence at M = 1 from one-thread times of each
    # shape (the QKV block timed here, the rest above), at M = 1024 from the
    # row-parallel per-row rate
    xq = np.random.default_rng(5).standard_normal((1, 2560)).astype(np.float32)
    dtq, nq = _timed(lambda: o.linear(xq, seq["_qkv_p4"], 7680), budget_s * 0.05, 200)
    t_layer = dtq + 3 * dt1 + dt
    t_seq1 = 32 * t_layer + dt3
    seq_bytes = seq["weight_bytes"]
    seq_ops_layers = 2.0 * (seq_bytes - 248320 * 2560 // 32 * 34) * 32 / 34
    # the GEMM's row-parallel rate on `threads` threads, applied to the
    # sequence's ops
    gemm_rate = gemm_ops / dtg4  # ops/s on all threads
    t_seq1024 = 1024 * seq_ops_layers / gemm_rate + dt3
    c2_bytes = res["step_bytes"]
    return dict(
        value=c2_bytes / dt / 1e9, unit="GB/s", cores=1, kind="port",
        sample="%d decode-MLP steps (2560->9216 x2 SwiGLU, 9216->2560) on one weight "
               "copy, x86 scalar path, row-parallel OpenMP as Q8Scalar.cpp:84,127 "
               "(M=1 -> 1 thread); %.1f ms/step" % (n, dt * 1e3),
        host=host, threads=threads,
        colpar={"GB/s": round(c2_bytes / dt_col / 1e9, 3), "threads": o.max_threads(),
                "ms_per_step": round(dt_col * 1e3, 3), "calls": m_col,
                "note": "column-parallel variant of the same scalar math (not the "
                        "reference's parallelisation)"},
        configs={
            "gemv_2560x2560": {"us": round(dt1 * 1e6, 1), "threads": 1, "calls": n1,
                               "GB/s": round(c1["bytes"] / dt1 / 1e9, 3)},
            "lm_head_248320x2560_argmax": {"us": round(dt3 * 1e6, 1), "threads": 1,
                                           "calls": n3,
                                           "GB/s": round(c3["bytes"] / dt3 / 1e9, 3)},
            "embedding_gather_1024": {"us": round(dtg * 1e6, 1), "threads": 1, "calls": ng},
            "gemm_m1024_n9216_k2560": {"TOPS": round(gemm_ops / dtg4 / 1e12, 4),
                                       "threads": threads,
                                       "ms_per_call": round(dtg4 * 1024 / rows * 1e3, 1),
                                       "sample": "%d-row calls x %d, row-parallel" % (rows, ng4)},
            "sequence_32_layers": {
                "m1_us": round(t_seq1 * 1e6, 1), "m1_threads": 1,
                "m1_GB/s": round(seq_bytes / t_seq1 / 1e9, 3),
                "m1024_ms": round(t_seq1024 * 1e3, 1), "m1024_threads": threads,
                "sample": "sum over the layer's shapes of the one-thread times above "
                          "(QKV 7680x2560 timed %d calls); M=1024 at the GEMM's "
                          "row-parallel rate" % nq},
        })


def bench_peaks(ctx, nbytes=4 << 30):
    """The device's measured peaks (llmcp_q8_microbench_*, the role of the
    reference's microbench/cpu_microbench.cpp for its CPU): streaming read,
    write and copy over a 4 GiB buffer (16x the Infinity Cache; 10 launches
    after one untimed), the int8 MFMA issue rate of independent chains
    without memory traffic, and the ceiling of the prefill GEMM's per-block
    work without its memory stream: the exact epilogue (int8 MFMA, a convert
    and an FMA per element and block), the same with convert-free f16 dots,
    and its MFMAs alone."""
    return {"hbm_read_GB/s": round(ctx.microbench_bandwidth("read", nbytes), 1),
            "hbm_write_GB/s": round(ctx.microbench_bandwidth("write", nbytes), 1),
            "hbm_copy_GB/s": round(ctx.microbench_bandwidth("copy", nbytes), 1),
            "int8_mfma_TOPS": round(ctx.microbench_int8_mfma(), 1),
            "gemm_exact_epilogue_TOPS": round(ctx.microbench_epilogue("exact"), 1),
            "gemm_cvtfree_epilogue_TOPS": round(ctx.microbench_epilogue("cvtfree"), 1),
            "gemm_mfma_only_TOPS": round(ctx.microbench_epilogue("mfma"), 1),
            "buffer_bytes": nbytes,
            "spec": {"hbm_GB/s": HBM_PEAK_GBS, "int8_TOPS": INT8_PEAK_TOPS}}


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
    ap.add_argument("--no-arena", action="store_true",
                    help="skip the real-model arena (4.47 GB file in /dev/shm: "
                         "upload and one decode step through it)")
    ap.add_argument("--gemm-only", type=int, default=0, metavar="M",
                    help="time only config 4's prefill GEMM at M rows and print "
                         "its figures (a short run for counter collection)")
    ap.add_argument("--norm-only", action="store_true",
                    help="time only the RMSNorm neighbour (extra.rmsnorm) and print "
                         "its figures (a short run for kernel traces)")
    ap.add_argument("--eager", action="store_true",
                    help="launch every timed block directly instead of replaying a "
                         "captured graph (for kernel tracers; figures include launch cost)")
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
    global EAGER
    EAGER = args.eager
    ctx = q8.Context(0)
    ctx.set_platform(args.platform)
    if args.copy_calibration:
        copy_calibration(ctx)
    if args.gemm_only:
        r = bench_gemm(ctx, args.gemm_only)
        print(json.dumps({"gemm_m%d_n9216_k2560" % args.gemm_only: r}), flush=True)
        return
    if args.norm_only:
        print(json.dumps({"rmsnorm": bench_norms(ctx, q8)}), flush=True)
        return
    peaks = bench_peaks(ctx)
    res = bench_decode_mlp(ctx, q8, args.steps, args.warmup)
    extra = {"platform": args.platform, "peaks": peaks}
    read_peak, int8_peak = peaks["hbm_read_GB/s"], peaks["int8_mfma_TOPS"]
    repack = dict(res["repack_ms"])
    c1 = c3 = seq = None
    if not args.no_extra:
        c1 = bench_gemv(ctx, 2560, 2560)
        extra["gemv_2560x2560"] = {"us": round(c1["us"], 3), "GB/s": round(c1["gb_s"], 1),
                                   "frac_hbm": round(c1["gb_s"] / HBM_PEAK_GBS, 4),
                                   "frac_hbm_measured": round(c1["gb_s"] / read_peak, 4)}
        repack["2560x2560"] = round(c1["repack_ms"], 3)
        c1a = bench_gemv(ctx, 2560, 2560, residual=True)
        extra["gemv_2560x2560_residual_add"] = {"us": round(c1a["us"], 3)}
        c3 = bench_lm_head(ctx)
        extra["lm_head_248320x2560_argmax"] = {
            "us": round(c3["us"], 2), "GB/s": round(c3["gb_s"], 1),
            "frac_hbm": round(c3["gb_s"] / HBM_PEAK_GBS, 4),
            "frac_hbm_measured": round(c3["gb_s"] / read_peak, 4)}
        repack["248320x2560"] = round(c3["repack_ms"], 3)
        extra["embedding_gather_1024"] = {"us": round(c3["gather_us"], 2),
                                          "GB/s": round(c3["gather_gb_s"], 1)}
        for m in (64, 256, 1024):
            g = bench_gemm(ctx, m)
            g["frac_int8_measured"] = round(g["op_TOPS"] / int8_peak, 4)
            g["frac_exact_epilogue_ceiling"] = round(
                g["op_TOPS"] / peaks["gemm_exact_epilogue_TOPS"], 4)
            extra["gemm_m%d_n9216_k2560" % m] = g
        extra["split_k_n2560_k9216"] = bench_split_k(ctx)
        seq = bench_sequence(ctx)
        repack["7680x2560"] = round(seq["_qkv_repack_ms"], 3)
        extra["sequence_32_layers"] = {k: v for k, v in seq.items() if not k.startswith("_")}
        extra["rmsnorm"] = bench_norms(ctx, q8)
        if not args.no_arena:
            extra["arena_real_model_32_layers"] = bench_arena(ctx, q8)
    # the one-time device repack (unit layout) of one tensor of each shape,
    # timed with HIP events on its own, outside every timed step
    extra["repack_ms"] = repack
    cpu = None if args.no_cpu or c1 is None else cpu_baseline(res, c1, c3, seq)
    fv = 80 if args.platform == "aarch64" else 64
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
                   "frac_hbm_peak": round(res["gb_s"] / HBM_PEAK_GBS, 4),
                   "frac_hbm_measured_peak": round(res["gb_s"] / read_peak, 4)},
        "roofline": {"bound": "hbm", "achieved": round(res["gu_gbs"], 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(res["gu_gbs"] / HBM_PEAK_GBS, 4),
                     "measured_peak": read_peak,
                     "frac_measured": round(res["gu_gbs"] / read_peak, 4),
                     "traffic": (load_traffic() or {}).get("hbm_bytes_per_launch"),
                     "kernel": "gemv_kernel<false,1,4,4,5,%d> (SwiGLU: gate and up "
                               "streamed by the two waves of a pair, 4-wave workgroups, "
                               "input row quantized per workgroup; timed alone via "
                               "llmcp_q8_swiglu, %d launches)"
                               % (fv, res["steps"]),
                     "launch_us": round(res["gu_launch_us"], 3),
                     "algorithmic_bytes": res["gu_bytes"],
                     "down_launch_us": round(res["down_launch_us"], 3),
                     "down_GB/s": round(res["down_bytes"] / res["down_launch_us"] / 1e3, 1)},
        "cpu_baseline": None if cpu is None else {
            k: (round(v, 3) if isinstance(v, float) else v) for k, v in cpu.items()},
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
