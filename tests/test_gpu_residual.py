"""llmcp_q8_linear_add: the residual add after out_proj / down
(ModelBuilder.cpp:271, :275) fused into the linear's epilogue.  The oracle
computes the pair as the graph does: the linear (its GEMV or GEMM epilogue
variant), then AddOpLowering's pointwise addf (LowerToLinalg.cpp:359-375) in
f32; on bf16 tensors the linear's result is rounded to bf16 and the add runs
on the widened operands, rounded to bf16 again.  Bit-exact."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def bits_equal(a, b):
    return np.array_equal(np.asarray(a).view(np.uint32 if np.asarray(a).dtype == np.float32 else np.uint16),
                          np.asarray(b).view(np.uint32 if np.asarray(b).dtype == np.float32 else np.uint16))


def to_bf16(oracle, x):
    return oracle.f32_to_bf16_bits(np.asarray(x, np.float32))


def reference(oracle, x, p4, n, r, dtype, epi):
    lin = oracle.linear(x, p4, n, epilogue=epi)
    if dtype == "f32":
        return (lin + r).astype(np.float32)
    widened = oracle.bf16_bits_to_f32(to_bf16(oracle, lin)) + oracle.bf16_bits_to_f32(r)
    return to_bf16(oracle, widened.astype(np.float32))


# (1, 2560, 2560): the GEMV quantizing in-workgroup; (1, 16416, 512): the
# wide GEMV on a pre-quantized row; (1, 264, 9216): the segmented down
# projection; (40, 264, 1056) and (1024, 3720, 2560): the GEMM, single-tile
# and persistent (32 sampled rows checked).
@pytest.mark.parametrize("m,n,k", [(1, 2560, 2560), (1, 16416, 512), (1, 264, 9216),
                                   (40, 264, 1056), (1024, 3720, 2560)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_linear_add(ctx, oracle, m, n, k, dtype):
    rng = np.random.default_rng(500 + m + n + k)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    r = rng.standard_normal((m, n)).astype(np.float32)
    p4 = oracle.pack_q8_0_p4(w)
    t = ctx.upload_p4(p4, n, k)
    if dtype == "bf16":
        x, r = to_bf16(oracle, x), to_bf16(oracle, r)
    xd, rd, yd = ctx.to_device(x), ctx.to_device(r), ctx.alloc(m * n * r.itemsize)
    ctx.linear_add(xd, t, rd, yd, m, mode="decode" if m == 1 else "prefill", dtype=dtype)
    y = ctx.to_host(yd, (m, n), r.dtype)
    rows = np.arange(m) if m <= 64 else np.unique(
        np.concatenate([[0, m - 1], rng.integers(0, m, 30)]))
    xf = oracle.bf16_bits_to_f32(x[rows]) if dtype == "bf16" else x[rows]
    assert bits_equal(y[rows], reference(oracle, xf, p4, n, r[rows], dtype, ctx.epilogue))
    ctx.release(t)


@pytest.mark.parametrize("m", [1, 40])
def test_linear_add_in_place(ctx, oracle, m):
    # residual and output are the same buffer (the residual stream updated
    # in place)
    rng = np.random.default_rng(520 + m)
    n, k = 264, 2560
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    r = rng.standard_normal((m, n)).astype(np.float32)
    p4 = oracle.pack_q8_0_p4(w)
    t = ctx.upload_p4(p4, n, k)
    xd, rd = ctx.to_device(x), ctx.to_device(r)
    ctx.linear_add(xd, t, rd, rd, m, mode="decode" if m == 1 else "prefill")
    assert bits_equal(ctx.to_host(rd, (m, n), np.float32),
                      reference(oracle, x, p4, n, r, "f32", ctx.epilogue))
    ctx.release(t)


def test_linear_add_declines_mismatched_residual(ctx, oracle, q8):
    import ctypes
    rng = np.random.default_rng(530)
    n, k = 264, 512
    p4 = oracle.pack_q8_0_p4((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    t = ctx.upload_p4(p4, n, k)
    xd = ctx.to_device(rng.standard_normal((1, k)).astype(np.float32))
    yd = ctx.alloc(n * 4)
    # a residual of N - 8 columns against an N-column output
    xi, ri, yo = (q8.f32_memref(xd.ptr, 1, k), q8.f32_memref(yd.ptr, 1, n - 8),
                  q8.f32_memref(yd.ptr, 1, n))
    with pytest.raises(q8.Declined):
        q8.check(q8.lib().llmcp_q8_linear_add(ctx.handle, ctypes.byref(xi),
                                              ctypes.byref(t.memref()),
                                              ctypes.byref(ri), ctypes.byref(yo), 1))
    ctx.release(t)
