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
follows a sample of rows through the whole chain.  The tied 248320 x 2560
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
