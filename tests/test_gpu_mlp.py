"""The decode MLP (llmcp_q8_mlp[_bf16]: the gate/up SwiGLU GEMV into h, then
the down GEMV of h) at the model's shape, H = 2560, F = 9216, against the
oracle (swiglu then linear, ModelBuilder.cpp:205-216 with FuseSiluMul) bit
for bit: on consecutive calls with new inputs (a stale h would differ), on
24 calls queued back to back without a host synchronization, and on replays
of a captured graph with new inputs copied in between and eager calls on the
same buffers between the replays; and for several rows (the SwiGLU GEMMs and
the down GEMM) in both execution modes and dtypes."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HIDDEN, FFN = 2560, 9216


def bits_equal(a, b):
    a, b = np.asarray(a), np.asarray(b)
    return a.shape == b.shape and a.tobytes() == b.tobytes()


@pytest.fixture(scope="module")
def mlp_weights(ctx, oracle):
    rng = np.random.default_rng(4242)
    ws = [(rng.standard_normal(s) * 0.02).astype(np.float32)
          for s in ((FFN, HIDDEN), (FFN, HIDDEN), (HIDDEN, FFN))]
    p4 = [oracle.pack_q8_0_p4(w) for w in ws]
    t = [ctx.upload_p4(p4[0], FFN, HIDDEN), ctx.upload_p4(p4[1], FFN, HIDDEN),
         ctx.upload_p4(p4[2], HIDDEN, FFN)]
    yield p4, t
    for x in t:
        ctx.release(x)


def reference(oracle, p4, x, dtype, epi):
    if dtype == "f32":
        h = oracle.swiglu(x, p4[0], p4[1], FFN, colpar=True, epilogue=epi)
        return h, oracle.linear(h, p4[2], HIDDEN, colpar=True, epilogue=epi)
    # bf16 tensors: each linear rounded to bf16 before the bf16 multiply,
    # then the down linear of the bf16 h, rounded to bf16
    xf = oracle.bf16_bits_to_f32(x)
    g = oracle.linear(xf, p4[0], FFN, activation="silu", colpar=True, epilogue=epi)
    u = oracle.linear(xf, p4[1], FFN, colpar=True, epilogue=epi)
    gs = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(g))
    ub = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(u))
    h = oracle.f32_to_bf16_bits((gs * ub).astype(np.float32))
    y = oracle.f32_to_bf16_bits(
        oracle.linear(oracle.bf16_bits_to_f32(h), p4[2], HIDDEN, colpar=True, epilogue=epi))
    return h, y


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_mlp_consecutive_calls(ctx, oracle, mlp_weights, dtype):
    p4, (tg, tu, td) = mlp_weights
    esz = 4 if dtype == "f32" else 2
    et = np.float32 if dtype == "f32" else np.uint16
    rng = np.random.default_rng(7 if dtype == "f32" else 8)
    for trial in range(3):
        x = rng.standard_normal((1, HIDDEN)).astype(np.float32)
        if dtype == "bf16":
            x = oracle.f32_to_bf16_bits(x)
        xd, hd = ctx.to_device(x), ctx.alloc(FFN * esz)
        y1, y2 = ctx.alloc(HIDDEN * esz), ctx.alloc(HIDDEN * esz)
        ctx.mlp(xd, tg, tu, td, y1, h=hd, dtype=dtype)
        ctx.mlp(xd, tg, tu, td, y2, dtype=dtype)  # the context's h
        h_ref, y_ref = reference(oracle, p4, x, dtype, ctx.epilogue)
        assert bits_equal(ctx.to_host(hd, (1, FFN), et), h_ref), trial
        assert bits_equal(ctx.to_host(y1, (1, HIDDEN), et), y_ref), trial
        assert bits_equal(ctx.to_host(y2, (1, HIDDEN), et), y_ref), trial


def test_mlp_back_to_back(ctx, oracle, mlp_weights):
    p4, (tg, tu, td) = mlp_weights
    rng = np.random.default_rng(9)
    xs = [rng.standard_normal((1, HIDDEN)).astype(np.float32) for _ in range(3)]
    xds = [ctx.to_device(x) for x in xs]
    yds = [ctx.alloc(HIDDEN * 4) for _ in range(24)]
    for i, yd in enumerate(yds):
        ctx.mlp(xds[i % 3], tg, tu, td, yd)
    refs = [reference(oracle, p4, x, "f32", ctx.epilogue)[1] for x in xs]
    for i, yd in enumerate(yds):
        assert bits_equal(ctx.to_host(yd, (1, HIDDEN), np.float32), refs[i % 3]), i
    assert ctx.check_flag() == 0


def test_mlp_in_a_captured_graph(ctx, oracle, mlp_weights, q8):
    p4, (tg, tu, td) = mlp_weights
    rng = np.random.default_rng(10)
    xd, yd = ctx.alloc(HIDDEN * 4), ctx.alloc(HIDDEN * 4)
    ctx.graph_begin()
    ctx.mlp(xd, tg, tu, td, yd)
    g = ctx.graph_end()
    try:
        for rep in range(4):
            x = rng.standard_normal((1, HIDDEN)).astype(np.float32)
            assert q8.lib().llmcp_q8_memcpy_h2d(ctx.handle, xd.ptr, x.ctypes.data,
                                                x.nbytes) == 0
            ctx.graph_launch(g)
            y = ctx.to_host(yd, (1, HIDDEN), np.float32)
            assert bits_equal(y, reference(oracle, p4, x, "f32", ctx.epilogue)[1]), rep
            ye = ctx.alloc(HIDDEN * 4)  # eager work between replays
            ctx.mlp(xd, tg, tu, td, ye)
            assert bits_equal(ctx.to_host(ye, (1, HIDDEN), np.float32), y), rep
    finally:
        ctx.graph_destroy(g)
    assert ctx.check_flag() == 0


@pytest.mark.parametrize("mode,dtype", [("prefill", "f32"), ("decode", "f32"),
                                        ("prefill", "bf16"), ("decode", "bf16")])
def test_mlp_several_rows(ctx, oracle, mlp_weights, mode, dtype):
    # M = 24: the SwiGLU GEMMs and the down GEMM with the platform's
    # epilogue in either mode; equal to llmcp_q8_swiglu then llmcp_q8_linear
    # and to the oracle, with and without a caller h
    p4, (tg, tu, td) = mlp_weights
    m = 24
    rng = np.random.default_rng(12 if dtype == "f32" else 13)
    x = rng.standard_normal((m, HIDDEN)).astype(np.float32)
    epi = ctx.epilogue
    esz, et = (4, np.float32) if dtype == "f32" else (2, np.uint16)
    if dtype == "f32":
        xh = x
        h_ref = oracle.swiglu(x, p4[0], p4[1], FFN, epilogue=epi)
        y_ref = oracle.linear(h_ref, p4[2], HIDDEN, epilogue=epi)
    else:
        xh = oracle.f32_to_bf16_bits(x)
        xf = oracle.bf16_bits_to_f32(xh)
        g = oracle.f32_to_bf16_bits(oracle.linear(xf, p4[0], FFN, activation="silu", epilogue=epi))
        u = oracle.f32_to_bf16_bits(oracle.linear(xf, p4[1], FFN, epilogue=epi))
        h_ref = oracle.f32_to_bf16_bits(
            (oracle.bf16_bits_to_f32(g) * oracle.bf16_bits_to_f32(u)).astype(np.float32))
        y_ref = oracle.f32_to_bf16_bits(
            oracle.linear(oracle.bf16_bits_to_f32(h_ref), p4[2], HIDDEN, epilogue=epi))
    xd, hd = ctx.to_device(xh), ctx.alloc(m * FFN * esz)
    y1, y2, y3 = (ctx.alloc(m * HIDDEN * esz) for _ in range(3))
    ctx.mlp(xd, tg, tu, td, y1, h=hd, m=m, mode=mode, dtype=dtype)
    assert bits_equal(ctx.to_host(hd, (m, FFN), et), h_ref)
    assert bits_equal(ctx.to_host(y1, (m, HIDDEN), et), y_ref)
    ctx.mlp(xd, tg, tu, td, y2, m=m, mode=mode, dtype=dtype)
    assert bits_equal(ctx.to_host(y2, (m, HIDDEN), et), y_ref)
    h2 = ctx.alloc(m * FFN * esz)
    ctx.swiglu(xd, tg, tu, h2, m, mode=mode, dtype=dtype)
    ctx.linear(h2, td, y3, m, mode=mode, dtype=dtype)
    assert bits_equal(ctx.to_host(y3, (m, HIDDEN), et), y_ref)


def test_swiglu_misaligned_row_declined(ctx, q8, mlp_weights):
    """The one-row SwiGLU (and so the decode MLP) quantizes its row in each
    workgroup from 16 B loads: a row that is not 16 B aligned is declined
    with LLMCP_Q8_DECLINED (the caller falls back), not a HIP error."""
    _, (tg, tu, td) = mlp_weights
    xd, hd, yd = ctx.alloc(HIDDEN * 4 + 16), ctx.alloc(FFN * 4), ctx.alloc(HIDDEN * 4)
    with pytest.raises(q8.Declined):
        ctx.swiglu(xd.ptr + 4, tg, tu, hd, 1)
    with pytest.raises(q8.Declined):
        ctx.mlp(xd.ptr + 4, tg, tu, td, yd, h=hd)
