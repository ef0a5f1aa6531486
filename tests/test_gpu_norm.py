"""llmcp_q8_rmsnorm and llmcp_q8_rmsnorm_linear_group: the RMSNorm in front
of the path (DecodeNormalization.cpp:71-154 for decode rows,
LowerToLinalg.cpp:245-300 for prefill -- the same per-row arithmetic) and
its fusion with the linears it feeds (input_layernorm -> in_proj_qkv/z/a/b,
post_attention_layernorm -> gate/up; ModelBuilder.cpp:225-236, :284-294).
Norm outputs must equal the oracle bit for bit; the group's outputs must
equal separate llmcp_q8_linear calls on the normed rows, and the oracle."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def bits(a):
    a = np.asarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a.view(np.uint16)


def same(a, b):
    """Bit equality, with any NaN equal to any NaN (0 * inf has a different
    payload on the GPU and on x86)."""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nan = np.isnan(a)
    return np.array_equal(nan, np.isnan(b)) and np.array_equal(bits(a[~nan]), bits(b[~nan]))


def rows_and_weight(rng, m, h, dtype, oracle, scale=1.0):
    x = (rng.standard_normal((m, h)) * scale).astype(np.float32)
    w = (rng.standard_normal(h) * 0.1 + 1.0).astype(np.float32)
    if dtype == "bf16":
        return oracle.f32_to_bf16_bits(x), oracle.f32_to_bf16_bits(w)
    return x, w


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("m,h", [(1, 2560), (1, 32), (3, 128), (64, 256), (65, 2560),
                                 (200, 96), (1, 9216), (2, 12288), (2, 12320), (1, 16384)])
@pytest.mark.parametrize("zc", [False, True])
def test_rmsnorm_bitwise(ctx, oracle, dtype, m, h, zc):
    rng = np.random.default_rng(m * 7 + h + zc)
    x, w = rows_and_weight(rng, m, h, dtype, oracle, scale=3.0)
    et = np.float32 if dtype == "f32" else np.uint16
    xd, wd = ctx.to_device(x), ctx.to_device(w)
    yd = ctx.alloc(x.nbytes)
    ctx.rmsnorm(xd, wd, yd, m, h, eps=1e-6, zero_centered=zc, dtype=dtype)
    ref = oracle.rmsnorm(x, w, 1e-6, zero_centered=zc, out_bf16=dtype == "bf16")
    assert np.array_equal(bits(ctx.to_host(yd, (m, h), et)), bits(ref))


def test_rmsnorm_edge_rows(ctx, oracle):
    """A zero row (rstd = 1/sqrt(eps)), subnormal and huge values (the sum
    overflows to inf: rstd 0), a row of one large value among tiny ones (the
    serial sum absorbs them), in place (y aliases x)."""
    h = 256
    x = np.zeros((6, h), np.float32)
    x[1] = 1e-40
    x[2] = 3e38
    x[3, :] = 2.0 ** -12
    x[3, 0] = 1.0
    x[4] = np.linspace(-1e-3, 1e-3, h)
    x[5] = np.where(np.arange(h) % 2, 1e19, -1e19)
    w = np.linspace(0.5, 1.5, h).astype(np.float32)
    xd, wd = ctx.to_device(x), ctx.to_device(w)
    for eps in (1e-6, 0.0, 1e-5):
        yd = ctx.to_device(x)
        ctx.rmsnorm(yd, wd, yd, 6, h, eps=eps)
        ref = oracle.rmsnorm(x, w, eps)
        assert same(ctx.to_host(yd, (6, h), np.float32), ref), eps


def stalled_rows(h, dtype, oracle):
    """Rows on which the serial sum stalls, so that any prediction of it from
    the exact sum is far off: once the sum reaches 2^24, adding 1.0 is an
    exact tie that rounds back to 2^24 (its even neighbour), while the exact
    sum keeps growing by 1 per element.  Row 0 stalls from its first element,
    row 1 half way, row 2 stalls and then meets values large enough to move
    the sum again, row 3 is the same after a random prefix."""
    rng = np.random.default_rng(h)
    x = np.ones((4, h), np.float32)
    x[0, 0] = 4096.0
    x[1, : h // 2] = rng.standard_normal(h // 2)
    x[1, h // 2] = 4096.0
    x[2, 0] = 4096.0
    x[2, h // 3 :: 7] = 3.0
    x[3, : h // 4] = rng.standard_normal(h // 4) * 50
    x[3, h // 4] = 4096.0
    w = (rng.standard_normal(h) * 0.1 + 1.0).astype(np.float32)
    if dtype == "bf16":
        return oracle.f32_to_bf16_bits(x), oracle.f32_to_bf16_bits(w)
    return x, w


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("h", [256, 2560, 9216])
def test_rmsnorm_stalled_sums(ctx, oracle, dtype, h):
    """Rows whose serial sum stalls far below the exact one (2^24 where the
    exact sum is 2^24 + i): the speculative sum's first predictions, taken
    from the exact partial sums, are far off, and the second pass has to
    correct them.  The serial sum's value itself is checked against the
    closed form for row 0."""
    x, w = stalled_rows(h, dtype, oracle)
    et = np.float32 if dtype == "f32" else np.uint16
    xd, wd = ctx.to_device(x), ctx.to_device(w)
    yd = ctx.alloc(x.nbytes)
    ctx.rmsnorm(xd, wd, yd, 4, h, eps=1e-6, dtype=dtype)
    ref, rstd = oracle.rmsnorm(x, w, 1e-6, out_bf16=dtype == "bf16", with_rstd=True)
    assert rstd[0] == np.float32(1.0) / np.sqrt(np.float32(2.0 ** 24) / np.float32(h)
                                                  + np.float32(1e-6))
    assert np.array_equal(bits(ctx.to_host(yd, (4, h), et)), bits(ref))


@pytest.mark.parametrize("skew", [64, -40, 20])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("m,h", [(1, 2560), (3, 256), (2, 9216), (1, 12288)])
def test_rmsnorm_fallbacks(ctx, oracle, q8, skew, dtype, m, h):
    """Rows of width <= 12288 run the speculative sum: lanes fold each
    sixteenth of the row from 32 candidate starts around a predicted partial
    sum, and the segments are chained through the candidates whose start is
    the true one.  llmcp_q8_test_ctx_rmsnorm_skew moves the context's
    predictions by
    `skew` f32 steps, so that the true start is found among the first
    pass's candidates instead (f32 rows, whose prediction drift is small) or
    nowhere and the segment is folded again; the results are unchanged."""
    rng = np.random.default_rng(m + h + skew)
    x, w = rows_and_weight(rng, m, h, dtype, oracle, scale=2.0)
    et = np.float32 if dtype == "f32" else np.uint16
    xd, wd = ctx.to_device(x), ctx.to_device(w)
    yd = ctx.alloc(x.nbytes)
    L = q8.lib()
    assert L.llmcp_q8_test_ctx_rmsnorm_skew(ctx.handle, skew) == 0
    try:
        ctx.rmsnorm(xd, wd, yd, m, h, eps=1e-6, zero_centered=True, dtype=dtype)
        got = ctx.to_host(yd, (m, h), et)
    finally:
        L.llmcp_q8_test_ctx_rmsnorm_skew(ctx.handle, 0)
    ref = oracle.rmsnorm(x, w, 1e-6, zero_centered=True, out_bf16=dtype == "bf16")
    assert np.array_equal(bits(got), bits(ref))


@pytest.mark.parametrize("dtype,m,h", [("bf16", 1024, 2560), ("bf16", 1025, 2560),
                                       ("f32", 512, 2560), ("f32", 513, 1024),
                                       ("bf16", 700, 12288)])
def test_rmsnorm_many_rows(ctx, oracle, dtype, m, h):
    """Row counts at the kernels' hand-over: up to 1024 bf16 rows (512 f32)
    run one row per workgroup, more run four rows per workgroup."""
    rng = np.random.default_rng(m + h)
    x, w = rows_and_weight(rng, m, h, dtype, oracle, scale=1.5)
    et = np.float32 if dtype == "f32" else np.uint16
    xd, wd = ctx.to_device(x), ctx.to_device(w)
    yd = ctx.alloc(x.nbytes)
    ctx.rmsnorm(xd, wd, yd, m, h, eps=1e-6, zero_centered=True, dtype=dtype)
    ref = oracle.rmsnorm(x, w, 1e-6, zero_centered=True, out_bf16=dtype == "bf16")
    assert np.array_equal(bits(ctx.to_host(yd, (m, h), et)), bits(ref))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("h", [256, 2560, 12288])
def test_rmsnorm_nan_rows(ctx, oracle, dtype, h):
    """A NaN among the values makes the sum NaN from its segment on (the
    speculative sum's chain falls back there); rows without one are
    unaffected."""
    m = 4
    rng = np.random.default_rng(h)
    x = rng.standard_normal((m, h)).astype(np.float32)
    x[0, 0] = np.nan
    x[1, h // 2 + 3] = np.nan
    x[2, h - 1] = np.nan
    w = (rng.standard_normal(h) * 0.1 + 1.0).astype(np.float32)
    if dtype == "bf16":
        x, w = oracle.f32_to_bf16_bits(x), oracle.f32_to_bf16_bits(w)
    et = np.float32 if dtype == "f32" else np.uint16
    xd, wd = ctx.to_device(x), ctx.to_device(w)
    yd = ctx.alloc(x.nbytes)
    ctx.rmsnorm(xd, wd, yd, m, h, eps=1e-6, dtype=dtype)
    ref = oracle.rmsnorm(x, w, 1e-6, out_bf16=dtype == "bf16")
    got = ctx.to_host(yd, (m, h), et)
    if dtype == "bf16":
        got, ref = oracle.bf16_bits_to_f32(got), oracle.bf16_bits_to_f32(ref)
    assert np.isnan(got[:3]).all()
    assert same(got, ref)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("h", [2560, 16384])
def test_rmsnorm_unaligned_rows(ctx, oracle, dtype, h):
    """Rows that start one element past a vector boundary take the element
    loads (both kernels)."""
    m = 3
    rng = np.random.default_rng(h + 5)
    x, w = rows_and_weight(rng, m, h, dtype, oracle, scale=2.0)
    esz, et = (4, np.float32) if dtype == "f32" else (2, np.uint16)
    flat = np.concatenate([np.zeros(1, x.dtype), x.reshape(-1)])
    xd, wd = ctx.to_device(flat), ctx.to_device(w)
    yd = ctx.alloc(x.nbytes)
    ctx.rmsnorm(xd.ptr + esz, wd, yd, m, h, eps=1e-6, zero_centered=True, dtype=dtype)
    ref = oracle.rmsnorm(x, w, 1e-6, zero_centered=True, out_bf16=dtype == "bf16")
    assert np.array_equal(bits(ctx.to_host(yd, (m, h), et)), bits(ref))


def test_rmsnorm_declines(ctx, q8):
    h = 96
    xd, yd = ctx.alloc(h * 4), ctx.alloc(h * 4)
    wd = ctx.alloc(h * 4 + 16)
    with pytest.raises(q8.Declined):  # width not a multiple of 32
        ctx.rmsnorm(xd, wd, yd, 1, 100)
    L = q8.lib()
    xi, yo = q8.f32_memref(xd.ptr, 1, h), q8.f32_memref(yd.ptr, 1, h)
    wv = q8.i8_memref(wd.ptr + 4, h)  # misaligned weight
    rc = L.llmcp_q8_rmsnorm(ctx.handle, ctypes.byref(xi), ctypes.byref(wv), 1e-6, 0,
                            ctypes.byref(yo))
    assert rc == q8.DECLINED
    wv = q8.i8_memref(wd.ptr, 64)  # weight length != H
    rc = L.llmcp_q8_rmsnorm(ctx.handle, ctypes.byref(xi), ctypes.byref(wv), 1e-6, 0,
                            ctypes.byref(yo))
    assert rc == q8.DECLINED


LINEAR_ATTN = [(8192, 2560), (4096, 2560), (32, 2560), (32, 2560)]
MLP_IN = [(9216, 2560), (9216, 2560)]


@pytest.mark.parametrize("shapes,acts", [
    (LINEAR_ATTN, ["none", "silu", "none", "softplus"]),
    (MLP_IN, ["silu", "none"])])
@pytest.mark.parametrize("m,mode,dtype", [(1, "decode", "bf16"), (1, "decode", "f32"),
                                          (64, "prefill", "bf16"), (97, "prefill", "f32")])
def test_rmsnorm_linear_group(ctx, oracle, shapes, acts, m, mode, dtype):
    rng = np.random.default_rng(m + len(shapes))
    k = shapes[0][1]
    x, w = rows_and_weight(rng, m, k, dtype, oracle, scale=2.0)
    ws = [(rng.standard_normal(s) * 0.02).astype(np.float32) for s in shapes]
    p4 = [oracle.pack_q8_0_p4(a) for a in ws]
    ts = [ctx.upload_p4(p, *s) for p, s in zip(p4, shapes)]
    try:
        esz, et = (4, np.float32) if dtype == "f32" else (2, np.uint16)
        xd, wd = ctx.to_device(x), ctx.to_device(w)
        nd = ctx.alloc(m * k * esz)
        outs = [ctx.alloc(m * n * esz) for n, _ in shapes]
        ctx.rmsnorm_linear_group(xd, wd, nd, ts, outs, m, eps=1e-6, zero_centered=True,
                                 activations=acts, mode=mode, dtype=dtype)
        normed = oracle.rmsnorm(x, w, 1e-6, zero_centered=True, out_bf16=dtype == "bf16")
        assert np.array_equal(bits(ctx.to_host(nd, (m, k), et)), bits(normed))
        nf = normed if dtype == "f32" else oracle.bf16_bits_to_f32(normed)
        for i, ((n, _), t, o) in enumerate(zip(shapes, ts, outs)):
            got = ctx.to_host(o, (m, n), et)
            sep = ctx.alloc(m * n * esz)
            ctx.linear(nd, t, sep, m, activation=acts[i], mode=mode, dtype=dtype)
            assert np.array_equal(bits(got), bits(ctx.to_host(sep, (m, n), et))), i
            rows = np.arange(m) if m <= 4 else np.array([0, m // 2, m - 1])
            ref = oracle.linear(nf[rows], p4[i], n, activation=acts[i],
                                epilogue=ctx.epilogue, colpar=True)
            if dtype == "bf16":
                ref = oracle.f32_to_bf16_bits(ref)
            assert np.array_equal(bits(got[rows]), bits(ref)), i
        assert ctx.check_flag() == 0
    finally:
        for t in ts:
            ctx.release(t)


@pytest.mark.parametrize("m,k,dtype", [(513, 2560, "f32"), (1024, 2560, "f32"),
                                        (1025, 2560, "bf16"), (3, 12320, "f32"),
                                        (2, 16384, "bf16")])
def test_rmsnorm_linear_group_four_row_kernel(ctx, oracle, m, k, dtype):
    """Shapes past the speculative kernel's limits (more than 512 f32 or 1024
    bf16 rows, or rows wider than 12288) take the four-rows RMSNorm kernel,
    whose epilogue writes the tiled Q8_1 that the GEMMs read (QMODE 2, the
    config-4 prefill with its norm): the fused call must equal the norm
    followed by the separate linears bit for bit, and the oracle on sampled
    rows."""
    shapes, acts = [(256, k), (64, k)], ["silu", "none"]
    rng = np.random.default_rng(m + k)
    x, w = rows_and_weight(rng, m, k, dtype, oracle, scale=2.0)
    ws = [(rng.standard_normal(s) * 0.02).astype(np.float32) for s in shapes]
    p4 = [oracle.pack_q8_0_p4(a) for a in ws]
    ts = [ctx.upload_p4(p, *s) for p, s in zip(p4, shapes)]
    try:
        esz, et = (4, np.float32) if dtype == "f32" else (2, np.uint16)
        xd, wd = ctx.to_device(x), ctx.to_device(w)
        nd = ctx.alloc(m * k * esz)
        outs = [ctx.alloc(m * n * esz) for n, _ in shapes]
        ctx.rmsnorm_linear_group(xd, wd, nd, ts, outs, m, eps=1e-6, zero_centered=True,
                                 activations=acts, mode="prefill", dtype=dtype)
        normed = oracle.rmsnorm(x, w, 1e-6, zero_centered=True, out_bf16=dtype == "bf16")
        assert np.array_equal(bits(ctx.to_host(nd, (m, k), et)), bits(normed))
        nf = normed if dtype == "f32" else oracle.bf16_bits_to_f32(normed)
        for i, ((n, _), t, o) in enumerate(zip(shapes, ts, outs)):
            got = ctx.to_host(o, (m, n), et)
            sep = ctx.alloc(m * n * esz)
            ctx.linear(nd, t, sep, m, activation=acts[i], mode="prefill", dtype=dtype)
            assert np.array_equal(bits(got), bits(ctx.to_host(sep, (m, n), et))), i
            rows = np.array([0, m // 2, m - 1])
            ref = oracle.linear(nf[rows], p4[i], n, activation=acts[i],
                                epilogue=ctx.epilogue, colpar=True)
            if dtype == "bf16":
                ref = oracle.f32_to_bf16_bits(ref)
            assert np.array_equal(bits(got[rows]), bits(ref)), i
        assert ctx.check_flag() == 0
    finally:
        for t in ts:
            ctx.release(t)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("m,h,group", [(1, 4096, 128), (5, 4096, 128), (70, 256, 64),
                                       (1, 32, 32), (3, 2048, 2048), (2, 8192, 4096)])
@pytest.mark.parametrize("activated", [False, True])
def test_gated_rmsnorm_bitwise(ctx, oracle, dtype, m, h, group, activated):
    """The linear-attention output norm: 32 value heads of 128 at the real
    shape (ModelBuilder.cpp:259-266), f32 weight; groups of up to 2048 take
    the one-wave-per-group kernel, larger ones the four-rows kernel."""
    rng = np.random.default_rng(m + h + group + activated)
    x = (rng.standard_normal((m, h)) * 2).astype(np.float32)
    z = (rng.standard_normal((m, h)) * 3).astype(np.float32)
    w = (rng.standard_normal(group) * 0.1 + 1).astype(np.float32)
    if dtype == "bf16":
        x, z = oracle.f32_to_bf16_bits(x), oracle.f32_to_bf16_bits(z)
    et = np.float32 if dtype == "f32" else np.uint16
    xd, zd, wd = ctx.to_device(x), ctx.to_device(z), ctx.to_device(w)
    yd = ctx.alloc(x.nbytes)
    ctx.gated_rmsnorm(xd, zd, wd, yd, m, h, group, eps=1e-6, gate_activated=activated,
                      dtype=dtype)
    ref = oracle.gated_rmsnorm(x, z, w, group, 1e-6, gate_activated=activated,
                               out_bf16=dtype == "bf16")
    assert np.array_equal(bits(ctx.to_host(yd, (m, h), et)), bits(ref))


def test_gated_rmsnorm_declines(ctx, q8):
    xd = ctx.alloc(256 * 4)
    wd = ctx.alloc(128 * 4)
    with pytest.raises(q8.Declined):  # group does not divide H
        ctx.gated_rmsnorm(xd, xd, wd, xd, 1, 256, 96)
    with pytest.raises(q8.Declined):  # group not a multiple of 32
        ctx.gated_rmsnorm(xd, xd, wd, xd, 1, 256, 16)


def test_norm_mlir_interface(ctx, oracle, q8):
    """The _mlir_ciface_ entries a lowering hook calls (default context):
    each equals the context entry it wraps, bit for bit."""
    rng = np.random.default_rng(44)
    L = q8.lib()
    h = 2560
    shapes = LINEAR_ATTN
    p4 = [oracle.pack_q8_0_p4((rng.standard_normal(s) * 0.02).astype(np.float32))
          for s in shapes]
    ts = [ctx.upload_p4(p, *s) for p, s in zip(p4, shapes)]
    ref = lambda r: q8.f32_memref(r.ptr, 1, r.nbytes // 2)
    try:
        L.llmcp_q8_set_default_ctx(ctx.handle)
        x, w = rows_and_weight(rng, 1, h, "bf16", oracle, scale=2.0)
        xd, wd = ctx.to_device(x), ctx.to_device(w)
        xi, wv = q8.f32_memref(xd.ptr, 1, h), q8.i8_memref(wd.ptr, h)
        y1, y2 = ctx.alloc(h * 2), ctx.alloc(h * 2)
        ctx.rmsnorm(xd, wd, y1, 1, h, eps=1e-6, zero_centered=True, dtype="bf16")
        yo = q8.f32_memref(y2.ptr, 1, h)
        assert L._mlir_ciface_llmcp_q8_rmsnorm_bf16(ctypes.byref(xi), ctypes.byref(wv), 1e-6, 1,
                                                    ctypes.byref(yo)) == q8.OK, q8.last_error()
        assert np.array_equal(ctx.to_host(y1, (1, h), np.uint16), ctx.to_host(y2, (1, h), np.uint16))
        # f32 rows and weight
        xf, wf = rows_and_weight(rng, 3, h, "f32", oracle)
        xfd, wfd = ctx.to_device(xf), ctx.to_device(wf)
        f1, f2 = ctx.alloc(xf.nbytes), ctx.alloc(xf.nbytes)
        ctx.rmsnorm(xfd, wfd, f1, 3, h)
        xfi, wfv, fo = (q8.f32_memref(xfd.ptr, 3, h), q8.i8_memref(wfd.ptr, h),
                        q8.f32_memref(f2.ptr, 3, h))
        assert L._mlir_ciface_llmcp_q8_rmsnorm(ctypes.byref(xfi), ctypes.byref(wfv), 1e-6, 0,
                                               ctypes.byref(fo)) == q8.OK, q8.last_error()
        assert np.array_equal(bits(ctx.to_host(f1, (3, h), np.float32)),
                              bits(ctx.to_host(f2, (3, h), np.float32)))
        # gated, bf16 and f32
        g = 4096
        gw = ctx.to_device((rng.standard_normal(128) * 0.1 + 1).astype(np.float32))
        gv = q8.i8_memref(gw.ptr, 128)
        for dt, esz, et, fn in (("bf16", 2, np.uint16, L._mlir_ciface_llmcp_q8_gated_rmsnorm_bf16),
                                ("f32", 4, np.float32, L._mlir_ciface_llmcp_q8_gated_rmsnorm)):
            v = (rng.standard_normal((1, g)) * 2).astype(np.float32)
            z = (rng.standard_normal((1, g)) * 3).astype(np.float32)
            if dt == "bf16":
                v, z = oracle.f32_to_bf16_bits(v), oracle.f32_to_bf16_bits(z)
            vd, zd = ctx.to_device(v), ctx.to_device(z)
            o1, o2 = ctx.alloc(g * esz), ctx.alloc(g * esz)
            ctx.gated_rmsnorm(vd, zd, gw, o1, 1, g, 128, dtype=dt)
            vi, zi, oo = (q8.f32_memref(vd.ptr, 1, g), q8.f32_memref(zd.ptr, 1, g),
                          q8.f32_memref(o2.ptr, 1, g))
            assert fn(ctypes.byref(vi), ctypes.byref(zi), ctypes.byref(gv), 128, 1e-6, 0,
                      ctypes.byref(oo)) == q8.OK, q8.last_error()
            assert np.array_equal(bits(ctx.to_host(o1, (1, g), et)),
                                  bits(ctx.to_host(o2, (1, g), et)))
        # the norm feeding qkv/z/a/b (4) and q/k/v-like (3), and the plain groups
        acts = [0, 1, 0, 3]
        for cnt, fn, gfn in ((4, L._mlir_ciface_llmcp_q8_rmsnorm_linear_group4_bf16,
                              L._mlir_ciface_llmcp_q8_linear_group4_bf16),
                             (3, L._mlir_ciface_llmcp_q8_rmsnorm_linear_group3_bf16,
                              L._mlir_ciface_llmcp_q8_linear_group3_bf16)):
            names = ["none", "silu", "none", "softplus"][:cnt]
            nd1, nd2 = ctx.alloc(h * 2), ctx.alloc(h * 2)
            o1 = [ctx.alloc(n * 2) for n, _ in shapes[:cnt]]
            o2 = [ctx.alloc(n * 2) for n, _ in shapes[:cnt]]
            o3 = [ctx.alloc(n * 2) for n, _ in shapes[:cnt]]
            ctx.rmsnorm_linear_group(xd, wd, nd1, ts[:cnt], o1, 1, zero_centered=True,
                                     activations=names, dtype="bf16")
            ws = [t.memref() for t in ts[:cnt]]
            ys = [ref(o) for o in o2]
            ndi = q8.f32_memref(nd2.ptr, 1, h)
            assert fn(ctypes.byref(xi), ctypes.byref(wv), 1e-6, 1, ctypes.byref(ndi),
                      *[ctypes.byref(d) for d in ws], *[ctypes.byref(d) for d in ys],
                      *acts[:cnt], q8.MODE["decode"]) == q8.OK, q8.last_error()
            assert np.array_equal(ctx.to_host(nd1, (1, h), np.uint16),
                                  ctx.to_host(nd2, (1, h), np.uint16))
            ys3 = [ref(o) for o in o3]
            assert gfn(ctypes.byref(ndi), *[ctypes.byref(d) for d in ws],
                       *[ctypes.byref(d) for d in ys3], *acts[:cnt],
                       q8.MODE["decode"]) == q8.OK, q8.last_error()
            for (n, _), a, b, c in zip(shapes[:cnt], o1, o2, o3):
                ra = ctx.to_host(a, (1, n), np.uint16)
                assert np.array_equal(ra, ctx.to_host(b, (1, n), np.uint16))
                assert np.array_equal(ra, ctx.to_host(c, (1, n), np.uint16))
    finally:
        L.llmcp_q8_set_default_ctx(None)
        for t in ts:
            ctx.release(t)
