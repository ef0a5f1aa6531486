"""GPU parity of the linear activations (none, silu, sigmoid, softplus --
LLMCPOps.cpp:74-77) and of bf16 activations in and out (the hook's
f32|bf16 tensors, Q8Decode.cpp:97-98 widening, :126-127 truncf) against the
CPU oracle, bit for bit.  bf16 references: the f32 oracle result on the
exactly widened input, rounded to bf16 (round to nearest even)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def bits_equal(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype == np.uint16 or b.dtype == np.uint16:
        return np.array_equal(a.astype(np.uint16), b.astype(np.uint16))
    return np.array_equal(a.astype(np.float32).view(np.uint32),
                          b.astype(np.float32).view(np.uint32))


def weights(rng, n, k, scale=0.02):
    return (rng.standard_normal((n, k)) * scale).astype(np.float32)


def to_bf16(oracle, x):
    return oracle.f32_to_bf16_bits(np.asarray(x, np.float32))


@pytest.mark.parametrize("act", ["none", "silu", "sigmoid", "softplus"])
@pytest.mark.parametrize("m", [1, 40])
def test_linear_activations(ctx, oracle, act, m):
    rng = np.random.default_rng(300 + m)
    n, k = 264, 1056
    w = weights(rng, n, k, 0.2)  # outputs of a few units: both tails of each act
    x = rng.standard_normal((m, k)).astype(np.float32)
    p4 = oracle.pack_q8_0_p4(w)
    t = ctx.upload_p4(p4, n, k)
    xd, yd = ctx.to_device(x), ctx.alloc(m * n * 4)
    mode = "decode" if m == 1 else "prefill"
    ctx.linear(xd, t, yd, m, activation=act, mode=mode)
    y = ctx.to_host(yd, (m, n), np.float32)
    epi = ctx.epilogue  # GEMV and GEMM: the platform's epilogue
    assert bits_equal(y, oracle.linear(x, p4, n, activation=act, epilogue=epi))
    ctx.release(t)


@pytest.mark.parametrize("m,k,act", [(1, 2560, "none"), (1, 9216, "silu"),
                                     (1, 1056, "softplus"), (37, 2560, "none"),
                                     (64, 1056, "sigmoid")])
def test_linear_bf16(ctx, oracle, m, k, act):
    rng = np.random.default_rng(310 + m + k)
    n = 264
    w = weights(rng, n, k)
    xb = to_bf16(oracle, rng.standard_normal((m, k)))
    p4 = oracle.pack_q8_0_p4(w)
    t = ctx.upload_p4(p4, n, k)
    xd, yd = ctx.to_device(xb), ctx.alloc(m * n * 2)
    mode = "decode" if m == 1 else "prefill"
    ctx.linear(xd, t, yd, m, activation=act, mode=mode, dtype="bf16")
    y = ctx.to_host(yd, (m, n), np.uint16)
    epi = ctx.epilogue
    ref = oracle.linear(oracle.bf16_bits_to_f32(xb), p4, n, activation=act,
                        epilogue=epi)
    assert bits_equal(y, to_bf16(oracle, ref))
    ctx.release(t)


def test_linear_bf16_misaligned_row(ctx, oracle):
    # a row that is not 8-byte aligned takes the separate quantize kernel
    rng = np.random.default_rng(320)
    n, k = 136, 2560
    w = weights(rng, n, k)
    xb = to_bf16(oracle, rng.standard_normal((1, k)))
    p4 = oracle.pack_q8_0_p4(w)
    t = ctx.upload_p4(p4, n, k)
    buf = ctx.alloc(k * 2 + 64)
    from llmcp_amd import lib
    lib().llmcp_q8_memcpy_h2d(ctx.handle, buf.ptr + 2, xb.ctypes.data, k * 2)
    yd = ctx.alloc(n * 2)
    ctx.linear(buf.ptr + 2, t, yd, 1, dtype="bf16")
    y = ctx.to_host(yd, (1, n), np.uint16)
    ref = oracle.linear(oracle.bf16_bits_to_f32(xb), p4, n, epilogue=ctx.epilogue)
    assert bits_equal(y, to_bf16(oracle, ref))
    ctx.release(t)


def swiglu_ref_bf16(oracle, xf, p4g, p4u, n, epi):
    g = to_bf16(oracle, oracle.linear(xf, p4g, n, activation="silu",
                                      epilogue=epi))
    u = to_bf16(oracle, oracle.linear(xf, p4u, n,
                                      epilogue=epi))
    prod = oracle.bf16_bits_to_f32(g) * oracle.bf16_bits_to_f32(u)  # exact in f32
    return to_bf16(oracle, prod)


@pytest.mark.parametrize("m", [1, 33])
def test_swiglu_bf16(ctx, oracle, m):
    rng = np.random.default_rng(330 + m)
    n, k = 1056, 2560
    wg, wu = weights(rng, n, k, 0.05), weights(rng, n, k, 0.05)
    xb = to_bf16(oracle, rng.standard_normal((m, k)))
    p4g, p4u = oracle.pack_q8_0_p4(wg), oracle.pack_q8_0_p4(wu)
    tg, tu = ctx.upload_p4(p4g, n, k), ctx.upload_p4(p4u, n, k)
    xd, hd = ctx.to_device(xb), ctx.alloc(m * n * 2)
    ctx.swiglu(xd, tg, tu, hd, m, mode="decode" if m == 1 else "prefill", dtype="bf16")
    h = ctx.to_host(hd, (m, n), np.uint16)
    assert bits_equal(h, swiglu_ref_bf16(oracle, oracle.bf16_bits_to_f32(xb), p4g, p4u, n, ctx.epilogue))
    ctx.release(tg)
    ctx.release(tu)


def test_mlp_bf16(ctx, oracle):
    rng = np.random.default_rng(340)
    hdim, f = 512, 1056
    wg, wu, wd = weights(rng, f, hdim, 0.05), weights(rng, f, hdim, 0.05), weights(rng, hdim, f)
    xb = to_bf16(oracle, rng.standard_normal((1, hdim)))
    p4g, p4u, p4d = (oracle.pack_q8_0_p4(w) for w in (wg, wu, wd))
    tg, tu, td = ctx.upload_p4(p4g, f, hdim), ctx.upload_p4(p4u, f, hdim), ctx.upload_p4(p4d, hdim, f)
    xd, hd, yd = ctx.to_device(xb), ctx.alloc(f * 2), ctx.alloc(hdim * 2)
    ctx.mlp(xd, tg, tu, td, yd, h=hd, dtype="bf16")
    h = ctx.to_host(hd, (1, f), np.uint16)
    y = ctx.to_host(yd, (1, hdim), np.uint16)
    href = swiglu_ref_bf16(oracle, oracle.bf16_bits_to_f32(xb), p4g, p4u, f, ctx.epilogue)
    assert bits_equal(h, href)
    yref = to_bf16(oracle, oracle.linear(oracle.bf16_bits_to_f32(href), p4d, hdim, epilogue=ctx.epilogue))
    assert bits_equal(y, yref)
    # without a caller buffer for h the result is the same
    y2d = ctx.alloc(hdim * 2)
    ctx.mlp(xd, tg, tu, td, y2d, dtype="bf16")
    assert bits_equal(ctx.to_host(y2d, (1, hdim), np.uint16), yref)
    for t in (tg, tu, td):
        ctx.release(t)


def test_lm_head_bf16_hidden(ctx, oracle):
    rng = np.random.default_rng(350)
    v, k = 16384, 2560
    w = weights(rng, v, k)
    xb = to_bf16(oracle, rng.standard_normal((1, k)))
    p4 = oracle.pack_q8_0_p4(w)
    t = ctx.upload_p4(p4, v, k)
    xd, ld, am = ctx.to_device(xb), ctx.alloc(v * 4), ctx.alloc(8)
    ctx.lm_head(xd, t, ld, 1, argmax=am, dtype="bf16")
    logits = ctx.to_host(ld, (1, v), np.float32)
    ref = oracle.linear(oracle.bf16_bits_to_f32(xb), p4, v, epilogue=ctx.epilogue)
    assert bits_equal(logits, ref)
    assert int(ctx.to_host(am, (1,), np.int64)[0]) == oracle.argmax(ref[0])
    ctx.release(t)


@pytest.mark.parametrize("k", [2560, 9216])
def test_embedding_bf16(ctx, oracle, k):
    rng = np.random.default_rng(360 + k)
    v = 1024
    w = weights(rng, v, k)
    p4 = oracle.pack_q8_0_p4(w)
    t = ctx.upload_p4(p4, v, k)
    tokens = rng.integers(0, v, 300).astype(np.int64)
    td, od = ctx.to_device(tokens), ctx.alloc(tokens.size * k * 2)
    ctx.embedding(td, tokens.size, t, od, dtype="bf16")
    out = ctx.to_host(od, (tokens.size, k), np.uint16)
    assert bits_equal(out, to_bf16(oracle, oracle.embedding(tokens, p4, k)))
    assert ctx.check_flag() == 0
    ctx.release(t)


# bf16 through the persistent GEMM schedule (more tiles than resident
# workgroups: M = 1024, N = 3720, K = 2560), checked on 32 sampled rows.
def _rows(rng, m):
    return np.unique(np.concatenate([[0, m - 1], rng.integers(0, m, 30)]))


def test_linear_bf16_persistent_tiles(ctx, oracle):
    rng = np.random.default_rng(360)
    m, n, k = 1024, 3720, 2560
    w = weights(rng, n, k)
    xb = to_bf16(oracle, rng.standard_normal((m, k)))
    p4 = oracle.pack_q8_0_p4(w)
    t = ctx.upload_p4(p4, n, k)
    xd, yd = ctx.to_device(xb), ctx.alloc(m * n * 2)
    ctx.linear(xd, t, yd, m, activation="silu", mode="prefill", dtype="bf16")
    y = ctx.to_host(yd, (m, n), np.uint16)
    rows = _rows(rng, m)
    ref = oracle.linear(oracle.bf16_bits_to_f32(xb[rows]), p4, n, activation="silu",
                        epilogue=ctx.epilogue)
    assert bits_equal(y[rows], to_bf16(oracle, ref))
    ctx.release(t)


def test_swiglu_bf16_persistent_tiles(ctx, oracle):
    rng = np.random.default_rng(361)
    m, n, k = 1024, 3720, 512
    wg, wu = weights(rng, n, k, 0.05), weights(rng, n, k, 0.05)
    xb = to_bf16(oracle, rng.standard_normal((m, k)))
    p4g, p4u = oracle.pack_q8_0_p4(wg), oracle.pack_q8_0_p4(wu)
    tg, tu = ctx.upload_p4(p4g, n, k), ctx.upload_p4(p4u, n, k)
    xd, hd = ctx.to_device(xb), ctx.alloc(m * n * 2)
    ctx.swiglu(xd, tg, tu, hd, m, mode="prefill", dtype="bf16")
    h = ctx.to_host(hd, (m, n), np.uint16)
    rows = _rows(rng, m)
    ref = swiglu_ref_bf16(oracle, oracle.bf16_bits_to_f32(xb[rows]), p4g, p4u, n, ctx.epilogue)
    assert bits_equal(h[rows], ref)
    ctx.release(tg)
    ctx.release(tu)


# llmcp-matmul-benchmark's Q8 self-check (llmcp-matmul-benchmark.cpp:280-289,
# :331-335; registered as a test at tests/CMakeLists.txt:162-165): every
# record holds scales 0x2008 and q = 127, activations are bf16 1.0, and the
# first bf16 output must equal K.  Run at the registered shape (M = N = K = 64,
# prefill) and on the decode path, for the fixture's K values.
@pytest.mark.parametrize("m,k", [(64, 64), (1, 64), (64, 2560), (1, 2560)])
def test_matmul_benchmark_all_ones_fixture(ctx, oracle, m, k):
    n = 64
    rec = np.array([0x08, 0x20] * 4 + [0x7F] * 128, np.uint8)
    p4 = np.tile(rec, n // 4 * (k // 32))
    t = ctx.upload_p4(p4, n, k)
    xb = np.full((m, k), 0x3F80, np.uint16)  # bf16 1.0
    xd, yd = ctx.to_device(xb), ctx.alloc(m * n * 2)
    ctx.linear(xd, t, yd, m, mode="decode" if m == 1 else "prefill", dtype="bf16")
    y = ctx.to_host(yd, (m, n), np.uint16)
    assert np.all(oracle.bf16_bits_to_f32(y) == np.float32(k))  # first == K
    ref = oracle.linear(np.ones((m, k), np.float32), p4, n,
                        epilogue=ctx.epilogue)
    assert bits_equal(y, to_bf16(oracle, ref))
    ctx.release(t)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_embedding_strided_output(ctx, oracle, dtype):
    # rows that start off 16 B boundaries (output offset by one element,
    # row stride k + 3) take the per-element stores; the padding between
    # rows is left alone
    import ctypes
    import llmcp_amd as q8
    rng = np.random.default_rng(370 + len(dtype))
    v, k, n = 256, 2560, 37
    w = weights(rng, v, k)
    p4 = oracle.pack_q8_0_p4(w)
    t = ctx.upload_p4(p4, v, k)
    tokens = rng.integers(0, v, n).astype(np.int64)
    td = ctx.to_device(tokens)
    el = np.float32 if dtype == "f32" else np.uint16
    ld = k + 3
    sentinel = np.full(n * ld + 1, 0x7FC5 if dtype == "bf16" else np.nan, el)
    if dtype == "f32":
        sentinel = sentinel.view(np.uint32)
        sentinel[:] = 0x7FC00005
        sentinel = sentinel.view(np.float32)
    bd = ctx.to_device(sentinel)
    esz = np.dtype(el).itemsize
    o = q8.f32_memref(bd.ptr + esz, n, k, row_stride=ld)
    ti = q8.i64_memref(td.ptr, n)
    q8.check(ctx._entry("llmcp_q8_embedding", dtype)(
        ctx.handle, ctypes.byref(ti), ctypes.byref(t.memref()), ctypes.byref(o)))
    got = ctx.to_host(bd, (n * ld + 1,), el)
    ref = oracle.embedding(tokens, p4, k)
    if dtype == "bf16":
        ref = to_bf16(oracle, ref)
    rows = np.stack([got[1 + i * ld: 1 + i * ld + k] for i in range(n)])
    assert bits_equal(rows, ref)
    keep = np.ones(n * ld + 1, bool)
    for i in range(n):
        keep[1 + i * ld: 1 + i * ld + k] = False
    assert np.array_equal(got[keep].view(np.uint16 if dtype == "bf16" else np.uint32),
                          sentinel[keep].view(np.uint16 if dtype == "bf16" else np.uint32))
    assert ctx.check_flag() == 0
    ctx.release(t)
