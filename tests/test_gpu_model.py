"""Configs[4] on the GPU: the Q8_0 linears of a 4B-class model at their real
shapes, chained as the model builder chains them, against the oracle; and
the real model's mixed BF16 / F32 / Q8_0 arena (426 tensors, 4.47 GB)
uploaded through llmcp_q8_upload_arena and used through descriptors that
point into the file image.

Layer of the chain (ModelBuilder.cpp:205-236, :271-275): the input x feeds
the 7680-wide QKV block and a residual branch r = x + o(x); two more
2560 x 2560 blocks follow, then the MLP (gate/up 9216 x 2560 with silu * up,
down 2560 x 9216) whose output is added to r.  Every row of every step
depends only on the same row of the step before, so at M = 1024 the oracle
follows a sample of rows through the whole chain: two layers (with the
lm_head and the gather) and all 32 layers with distinct weights, in the
pre-norm residual form with the RMSNorms (with the grouped form of each
layer's shared-input linears).  The tied 248320 x 2560
table serves the last-row lm_head (ModelBuilder.cpp:492-513) and a gather of
1024 token ids."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HIDDEN, FFN, QKV, VOCAB = 2560, 9216, 7680, 248320
SHAPES = {"qkv": (QKV, HIDDEN), "o": (HIDDEN, HIDDEN), "a": (HIDDEN, HIDDEN),
          "b": (HIDDEN, HIDDEN), "gate": (FFN, HIDDEN), "up": (FFN, HIDDEN),
          "down": (HIDDEN, FFN)}


def bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


@pytest.fixture(scope="module")
def model(q8):
    """Two layers and the tied table, synthesized on the device (N(0, 0.02)
    weights through the device llmcp-pack), with host copies of the p4
    bytes for the oracle.  Registered per context by the test."""
    with q8.Context(0) as c:
        layers = []
        for li in range(2):
            w = {}
            for j, (name, (n, k)) in enumerate(SHAPES.items()):
                d, _ = c.synthesize_p4(seed=7000 + 16 * li + j, rows=n, cols=k)
                w[name] = c.to_host(d, (d.nbytes,), np.uint8)
                d.free()
            layers.append(w)
        d, _ = c.synthesize_p4(seed=7999, rows=VOCAB, cols=HIDDEN)
        table = c.to_host(d, (d.nbytes,), np.uint8)
        d.free()
    return layers, table


def oracle_layer(oracle, x, w, epi):
    lin = lambda v, name, **kw: oracle.linear(v, w[name], SHAPES[name][0],
                                              epilogue=epi, colpar=True, **kw)
    qkv = lin(x, "qkv")
    r = (lin(x, "o") + x).astype(np.float32)
    b = lin(lin(r, "a"), "b")
    h = oracle.swiglu(b, w["gate"], w["up"], FFN, epilogue=epi, colpar=True)
    y = (lin(h, "down") + r).astype(np.float32)
    return qkv, b, h, y


def gpu_layer(ctx, x, t, m, mode, bufs):
    qkv, r, a, b, h, y = (bufs[k] for k in ("qkv", "r", "a", "b", "h", "y"))
    ctx.linear(x, t["qkv"], qkv, m, mode=mode)
    ctx.linear_add(x, t["o"], x, r, m, mode=mode)
    ctx.linear(r, t["a"], a, m, mode=mode)
    ctx.linear(a, t["b"], b, m, mode=mode)
    ctx.swiglu(b, t["gate"], t["up"], h, m, mode=mode)
    ctx.linear_add(h, t["down"], r, y, m, mode=mode)
    return y


@pytest.mark.parametrize("m,mode", [(1, "decode"), (1024, "prefill")])
def test_config5_two_layer_chain(ctx, oracle, model, m, mode):
    layers, table = model
    regs = [{name: ctx.upload_p4(w[name], *SHAPES[name]) for name in SHAPES}
            for w in layers]
    head = ctx.upload_p4(table, VOCAB, HIDDEN)
    try:
        rng = np.random.default_rng(71 + m)
        x0 = rng.standard_normal((m, HIDDEN)).astype(np.float32)
        rows = np.arange(m) if m == 1 else np.unique(
            np.concatenate([[0, m - 1], rng.choice(m, 6, replace=False)]))
        sizes = {"qkv": QKV, "r": HIDDEN, "a": HIDDEN, "b": HIDDEN, "h": FFN,
                 "y": HIDDEN}
        x = ctx.to_device(x0)
        xr = x0[rows]
        for li, t in enumerate(regs):
            bufs = {k: ctx.alloc(m * n * 4) for k, n in sizes.items()}
            y = gpu_layer(ctx, x, t, m, mode, bufs)
            qkv_ref, b_ref, h_ref, y_ref = oracle_layer(oracle, xr, layers[li], ctx.epilogue)
            got = lambda k, n: ctx.to_host(bufs[k], (m, n), np.float32)[rows]
            assert bits_equal(got("qkv", QKV), qkv_ref), (li, m)
            assert bits_equal(got("b", HIDDEN), b_ref), (li, m)
            assert bits_equal(got("h", FFN), h_ref), (li, m)
            assert bits_equal(got("y", HIDDEN), y_ref), (li, m)
            if m == 1:
                # the fused two-launch MLP on the same input
                ym = ctx.alloc(HIDDEN * 4)
                ctx.mlp(bufs["b"], t["gate"], t["up"], t["down"], ym)
                mlp_ref = oracle.linear(h_ref, layers[li]["down"], HIDDEN,
                                        epilogue=ctx.epilogue, colpar=True)
                assert bits_equal(ctx.to_host(ym, (1, HIDDEN), np.float32), mlp_ref)
            x, xr = y, y_ref
        # last-row lm_head over the tied table, with its argmax
        last = ctx.to_host(x, (m, HIDDEN), np.float32)[m - 1:m]
        assert bits_equal(last, xr[-1:])
        xl = ctx.to_device(last)
        logits, am = ctx.alloc(VOCAB * 4), ctx.alloc(8)
        ctx.lm_head(xl, head, logits, 1, argmax=am, mode=mode)
        ref = oracle.linear(last, table, VOCAB, epilogue=ctx.epilogue, colpar=True)
        assert bits_equal(ctx.to_host(logits, (1, VOCAB), np.float32), ref)
        assert int(ctx.to_host(am, (1,), np.int64)[0]) == oracle.argmax(ref)
        # the embedding gather of 1024 ids from the same table
        ids = rng.integers(0, VOCAB, 1024).astype(np.int64)
        idd, emb = ctx.to_device(ids), ctx.alloc(1024 * HIDDEN * 4)
        ctx.embedding(idd, 1024, head, emb)
        assert bits_equal(ctx.to_host(emb, (1024, HIDDEN), np.float32),
                          oracle.embedding(ids, table, HIDDEN))
        assert ctx.check_flag() == 0
    finally:
        for t in regs:
            for w in t.values():
                ctx.release(w)
        ctx.release(head)


@pytest.fixture(scope="module")
def model32(q8):
    """All 32 layers of config 5 with distinct weights (seeds apart from the
    two-layer fixture's), host copies of their p4 bytes for the oracle."""
    with q8.Context(0) as c:
        layers = []
        for li in range(32):
            w = {}
            for j, (name, (n, k)) in enumerate(SHAPES.items()):
                d, _ = c.synthesize_p4(seed=20000 + 16 * li + j, rows=n, cols=k)
                w[name] = c.to_host(d, (d.nbytes,), np.uint8)
                d.free()
            layers.append(w)
    return layers


@pytest.mark.parametrize("m,mode", [(1, "decode"), (1024, "prefill")])
def test_config5_32_layer_chain(ctx, oracle, model32, m, mode):
    """All 32 layers of configs[4] as one chain, in the model builder's
    pre-norm residual form (ModelBuilder.cpp:205-236, :271-275): xn =
    RMSNorm(x); qkv(xn); r = x + o(xn); rn = RMSNorm(r); h = SwiGLU(b(a(rn)));
    y = r + down(h), each layer's y the next layer's x (the norms keep the
    residual stream finite over 32 layers; without them the SwiGLU squares
    its magnitude every layer).  Every output on the checked rows is
    bit-exact to the oracle (M = 1: the row; M = 1024: first, last and six
    random rows, which depend only on themselves).  At each layer the four
    linears of xn run as one group (the grouped form of the bench's
    sequence) and equal the same four linears one call at a time, over all
    M rows."""
    layers = model32
    regs = [{name: ctx.upload_p4(w[name], *SHAPES[name]) for name in SHAPES}
            for w in layers]
    try:
        rng = np.random.default_rng(171 + m)
        eps = 1e-6
        norms = [(1.0 + 0.1 * rng.standard_normal((2, HIDDEN))).astype(np.float32)
                 for _ in layers]
        x0 = rng.standard_normal((m, HIDDEN)).astype(np.float32)
        rows = np.arange(m) if m == 1 else np.unique(
            np.concatenate([[0, m - 1], rng.choice(m, 6, replace=False)]))
        sizes = {"xn": HIDDEN, "qkv": QKV, "r": HIDDEN, "rn": HIDDEN, "a": HIDDEN,
                 "b": HIDDEN, "h": FFN, "y": HIDDEN}
        bufs = [{k: ctx.alloc(m * n * 4) for k, n in sizes.items()} for _ in range(2)]
        names = ("qkv", "o", "a", "b")
        width = {"qkv": QKV, "o": HIDDEN, "a": HIDDEN, "b": HIDDEN}
        grouped = {nm: ctx.alloc(m * width[nm] * 4) for nm in names}
        single = {nm: ctx.alloc(m * width[nm] * 4) for nm in names}
        x = ctx.to_device(x0)
        xr = x0[rows]
        lin = lambda v, w, name: oracle.linear(v, w[name], SHAPES[name][0],
                                               epilogue=ctx.epilogue, colpar=True)
        for li, t in enumerate(regs):
            bf = bufs[li % 2]
            n1, n2 = ctx.to_device(norms[li][0]), ctx.to_device(norms[li][1])
            ctx.rmsnorm(x, n1, bf["xn"], m, HIDDEN, eps=eps)
            # the grouped form of xn's four linears against single calls
            ctx.linear_group(bf["xn"], [t[nm] for nm in names],
                             [grouped[nm] for nm in names], m, mode=mode)
            for nm in names:
                ctx.linear(bf["xn"], t[nm], single[nm], m, mode=mode)
                assert bits_equal(ctx.to_host(grouped[nm], (m, width[nm]), np.float32),
                                  ctx.to_host(single[nm], (m, width[nm]), np.float32)), (li, nm)
            ctx.linear(bf["xn"], t["qkv"], bf["qkv"], m, mode=mode)
            ctx.linear_add(bf["xn"], t["o"], x, bf["r"], m, mode=mode)
            ctx.rmsnorm(bf["r"], n2, bf["rn"], m, HIDDEN, eps=eps)
            ctx.linear(bf["rn"], t["a"], bf["a"], m, mode=mode)
            ctx.linear(bf["a"], t["b"], bf["b"], m, mode=mode)
            ctx.swiglu(bf["b"], t["gate"], t["up"], bf["h"], m, mode=mode)
            ctx.linear_add(bf["h"], t["down"], bf["r"], bf["y"], m, mode=mode)
            w = layers[li]
            xn = oracle.rmsnorm(xr, norms[li][0], eps)
            qkv = lin(xn, w, "qkv")
            r = (lin(xn, w, "o") + xr).astype(np.float32)
            a = lin(oracle.rmsnorm(r, norms[li][1], eps), w, "a")
            bb = lin(a, w, "b")
            h = oracle.swiglu(bb, w["gate"], w["up"], FFN, epilogue=ctx.epilogue, colpar=True)
            y = (lin(h, w, "down") + r).astype(np.float32)
            got = lambda k, n: ctx.to_host(bf[k], (m, n), np.float32)[rows]
            assert np.all(np.isfinite(y)), li
            assert bits_equal(got("qkv", QKV), qkv), (li, m)
            assert bits_equal(got("r", HIDDEN), r), (li, m)
            assert bits_equal(got("h", FFN), h), (li, m)
            assert bits_equal(got("y", HIDDEN), y), (li, m)
            x, xr = bf["y"], y
    finally:
        for t in regs:
            for w in t.values():
                ctx.release(w)


def test_real_model_arena(q8, oracle):
    """The 32-layer 4B-class arena with the real tensor list and dtypes
    (Q8_0 matmul weights and tied table, BF16 norms / conv / dt_bias, F32
    A_log and gated-norm weights), uploaded whole; one tensor of each Q8_0
    shape is then used through a descriptor into the image, the tied table
    through the lm_head and the embedding gather."""
    from llmcp_amd import model_arena
    image, entries = model_arena.build_image(seed=5)
    assert len(entries) == 426 and image.nbytes > 4.4e9
    assert q8.arena_inspect(image) == (426, 249)
    rng = np.random.default_rng(72)
    with q8.Context(0) as ctx:
        assert ctx.upload_arena(image) == 249
        base = image.ctypes.data
        by_shape = {}
        for e in entries:
            if e["dtype"] == "Q8_0":
                by_shape.setdefault(tuple(e["shape"]), e)
        assert len(by_shape) == 8
        for (n, k), e in sorted(by_shape.items()):
            if n == VOCAB:
                continue
            w = q8.Weight(ctx, base + e["offset"], n, k, owner=image)
            p4 = image[e["offset"]:e["offset"] + e["size"]]
            x = rng.standard_normal((1, k)).astype(np.float32)
            xd, yd = ctx.to_device(x), ctx.alloc(n * 4)
            ctx.linear(xd, w, yd, 1)
            assert bits_equal(ctx.to_host(yd, (1, n), np.float32),
                              oracle.linear(x, p4, n, epilogue=ctx.epilogue,
                                            colpar=True)), (n, k)
        e = by_shape[(VOCAB, HIDDEN)]
        assert e["name"] == "model.language_model.embed_tokens.weight"
        table = q8.Weight(ctx, base + e["offset"], VOCAB, HIDDEN, owner=image)
        p4 = image[e["offset"]:e["offset"] + e["size"]]
        x = rng.standard_normal((1, HIDDEN)).astype(np.float32)
        xd, logits, am = ctx.to_device(x), ctx.alloc(VOCAB * 4), ctx.alloc(8)
        ctx.lm_head(xd, table, logits, 1, argmax=am)
        ref = oracle.linear(x, p4, VOCAB, epilogue=ctx.epilogue, colpar=True)
        assert bits_equal(ctx.to_host(logits, (1, VOCAB), np.float32), ref)
        assert int(ctx.to_host(am, (1,), np.int64)[0]) == oracle.argmax(ref)
        ids = rng.integers(0, VOCAB, 1024).astype(np.int64)
        idd, emb = ctx.to_device(ids), ctx.alloc(1024 * HIDDEN * 2)
        ctx.embedding(idd, 1024, table, emb, dtype="bf16")
        assert np.array_equal(ctx.to_host(emb, (1024, HIDDEN), np.uint16),
                              oracle.f32_to_bf16_bits(oracle.embedding(ids, p4, HIDDEN)))
        assert ctx.check_flag() == 0


LA = {"qkv": (8192, HIDDEN), "z": (4096, HIDDEN), "a": (32, HIDDEN), "b": (32, HIDDEN),
      "out": (HIDDEN, 4096), "gate": (FFN, HIDDEN), "up": (FFN, HIDDEN), "down": (HIDDEN, FFN)}


def test_decode_layers_with_norms_bf16(ctx, oracle, q8):
    """Two linear-attention layers of the real model in bf16 at one row, as
    the model builder chains them around the Q8_0 linears
    (ModelBuilder.cpp:225-236, :259-266, :271-294): input RMSNorm fused with
    the in_proj qkv/z/a/b group; the gated RMSNorm of the value heads (a
    fixed stand-in for the attention core, which is not on this path) with
    z as the gate; out_proj with the residual; the post-attention RMSNorm;
    the SwiGLU; down_proj with the residual.  Every tensor is compared with
    the oracle's composition of the same steps, bit for bit."""
    eps = 1e-6
    rng = np.random.default_rng(505)
    bf = lambda a: oracle.f32_to_bf16_bits(np.asarray(a, np.float32))
    wf = oracle.bf16_bits_to_f32
    layers, regs = [], []
    for li in range(2):
        w = {}
        for j, (name, (n, k)) in enumerate(LA.items()):
            d, _ = ctx.synthesize_p4(seed=9100 + 16 * li + j, rows=n, cols=k)
            w[name] = ctx.to_host(d, (d.nbytes,), np.uint8)
            d.free()
        w["ln"] = bf(rng.standard_normal(HIDDEN) * 0.1)
        w["post"] = bf(rng.standard_normal(HIDDEN) * 0.1)
        w["gn"] = (rng.standard_normal(128) * 0.1 + 1.0).astype(np.float32)
        layers.append(w)
        regs.append({k: ctx.upload_p4(w[k], *LA[k]) for k in LA})
    try:
        x = bf(rng.standard_normal((1, HIDDEN)) * 2.0)
        v = bf(rng.standard_normal((1, 4096)))
        xd, vd = ctx.to_device(x), ctx.to_device(v)
        nd, rd, n2d = ctx.alloc(HIDDEN * 2), ctx.alloc(HIDDEN * 2), ctx.alloc(HIDDEN * 2)
        gd, hd = ctx.alloc(4096 * 2), ctx.alloc(FFN * 2)
        group = ["qkv", "z", "a", "b"]
        outs = [ctx.alloc(LA[k][0] * 2) for k in group]
        epi = ctx.epilogue
        for li, (w, t) in enumerate(zip(layers, regs)):
            lnw, postw, gnw = ctx.to_device(w["ln"]), ctx.to_device(w["post"]), ctx.to_device(w["gn"])
            ctx.rmsnorm_linear_group(xd, lnw, nd, [t[k] for k in group], outs, 1, eps=eps,
                                     zero_centered=True, dtype="bf16")
            ctx.gated_rmsnorm(vd, outs[1], gnw, gd, 1, 4096, 128, eps=eps, dtype="bf16")
            ctx.linear_add(gd, t["out"], xd, rd, 1, dtype="bf16")
            ctx.rmsnorm(rd, postw, n2d, 1, HIDDEN, eps=eps, zero_centered=True, dtype="bf16")
            ctx.swiglu(n2d, t["gate"], t["up"], hd, 1, dtype="bf16")
            ctx.linear_add(hd, t["down"], rd, xd, 1, dtype="bf16")

            normed = oracle.rmsnorm(x, w["ln"], eps, zero_centered=True, out_bf16=True)
            got = lambda d, n: ctx.to_host(d, (1, n), np.uint16)
            assert np.array_equal(got(nd, HIDDEN), normed), li
            ref = {k: bf(oracle.linear(wf(normed), w[k], LA[k][0], epilogue=epi))
                   for k in group}
            for k, o in zip(group, outs):
                assert np.array_equal(got(o, LA[k][0]), ref[k]), (li, k)
            gated = oracle.gated_rmsnorm(v, ref["z"], w["gn"], 128, eps, out_bf16=True)
            assert np.array_equal(got(gd, 4096), gated), li
            lin = bf(oracle.linear(wf(gated), w["out"], HIDDEN, epilogue=epi))
            r = bf(wf(lin) + wf(x))
            assert np.array_equal(got(rd, HIDDEN), r), li
            n2 = oracle.rmsnorm(r, w["post"], eps, zero_centered=True, out_bf16=True)
            assert np.array_equal(got(n2d, HIDDEN), n2), li
            g = bf(oracle.linear(wf(n2), w["gate"], FFN, activation="silu", epilogue=epi))
            u = bf(oracle.linear(wf(n2), w["up"], FFN, epilogue=epi))
            h = bf(wf(g) * wf(u))
            assert np.array_equal(got(hd, FFN), h), li
            down = bf(oracle.linear(wf(h), w["down"], HIDDEN, epilogue=epi))
            x = bf(wf(down) + wf(r))
            assert np.array_equal(got(xd, HIDDEN), x), li
        assert ctx.check_flag() == 0
    finally:
        for t in regs:
            for wt in t.values():
                ctx.release(wt)
