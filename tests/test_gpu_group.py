"""llmcp_q8_linear_group: linears that share one input -- the model
builder's in_proj_qkv/z/a/b (ModelBuilder.cpp:229-236) and q/k/v (:288-294)
at the 4B-class shapes -- computed with one input quantization (and one
GEMV launch for a row).  Every output must equal the separate
llmcp_q8_linear call's bit for bit, and the oracle's."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LINEAR_ATTN = [(8192, 2560), (4096, 2560), (32, 2560), (32, 2560)]
FULL_ATTN = [(8192, 2560), (1024, 2560), (1024, 2560)]


def bits(a):
    a = np.asarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a.view(np.uint16)


@pytest.mark.parametrize("shapes,acts", [
    (LINEAR_ATTN, ["none", "silu", "none", "softplus"]),
    (FULL_ATTN, ["none", "none", "none"]),
    ([(264, 1056), (136, 1056)], ["sigmoid", "none"])])
@pytest.mark.parametrize("m,mode,dtype", [(1, "decode", "f32"), (1, "decode", "bf16"),
                                          (37, "prefill", "f32"), (2, "decode", "bf16")])
def test_group_matches_separate_linears(ctx, oracle, shapes, acts, m, mode, dtype):
    rng = np.random.default_rng(len(shapes) * 100 + m)
    k = shapes[0][1]
    ws = [(rng.standard_normal(s) * 0.02).astype(np.float32) for s in shapes]
    p4 = [oracle.pack_q8_0_p4(w) for w in ws]
    ts = [ctx.upload_p4(p, *s) for p, s in zip(p4, shapes)]
    try:
        x = rng.standard_normal((m, k)).astype(np.float32)
        esz, et = (4, np.float32) if dtype == "f32" else (2, np.uint16)
        xh = x if dtype == "f32" else oracle.f32_to_bf16_bits(x)
        xd = ctx.to_device(xh)
        outs = [ctx.alloc(m * n * esz) for n, _ in shapes]
        ctx.linear_group(xd, ts, outs, m, activations=acts, mode=mode, dtype=dtype)
        xf = x if dtype == "f32" else oracle.bf16_bits_to_f32(xh)
        for i, ((n, _), t, o) in enumerate(zip(shapes, ts, outs)):
            got = ctx.to_host(o, (m, n), et)
            sep = ctx.alloc(m * n * esz)
            ctx.linear(xd, t, sep, m, activation=acts[i], mode=mode, dtype=dtype)
            assert np.array_equal(bits(got), bits(ctx.to_host(sep, (m, n), et))), i
            ref = oracle.linear(xf, p4[i], n, activation=acts[i],
                                epilogue=ctx.epilogue, colpar=True)
            if dtype == "bf16":
                ref = oracle.f32_to_bf16_bits(ref)
            assert np.array_equal(bits(got), bits(ref)), i
    finally:
        for t in ts:
            ctx.release(t)


def test_group_mlir_interface_and_errors(ctx, oracle, q8):
    rng = np.random.default_rng(9)
    shapes = LINEAR_ATTN
    ws = [(rng.standard_normal(s) * 0.02).astype(np.float32) for s in shapes]
    p4 = [oracle.pack_q8_0_p4(w) for w in ws]
    ts = [ctx.upload_p4(p, *s) for p, s in zip(p4, shapes)]
    L = q8.lib()
    try:
        x = rng.standard_normal((1, 2560)).astype(np.float32)
        xd = ctx.to_device(x)
        outs = [ctx.alloc(n * 4) for n, _ in shapes]
        xi = q8.f32_memref(xd.ptr, 1, 2560)
        wd = [t.memref() for t in ts]
        yd = [q8.f32_memref(o.ptr, 1, n) for o, (n, _) in zip(outs, shapes)]
        L.llmcp_q8_set_default_ctx(ctx.handle)
        rc = L._mlir_ciface_llmcp_q8_linear_group4(
            ctypes.byref(xi), *[ctypes.byref(d) for d in wd], *[ctypes.byref(d) for d in yd],
            0, 1, 0, 0, q8.MODE["decode"])
        assert rc == q8.OK, q8.last_error()
        for i, (n, _) in enumerate(shapes):
            ref = oracle.linear(x, p4[i], n, activation="silu" if i == 1 else "none",
                                epilogue=ctx.epilogue, colpar=True)
            assert np.array_equal(bits(ctx.to_host(outs[i], (1, n), np.float32)), bits(ref))
        rc = L._mlir_ciface_llmcp_q8_linear_group3(
            ctypes.byref(xi), *[ctypes.byref(d) for d in wd[:3]],
            *[ctypes.byref(d) for d in yd[:3]], 0, 0, 0, q8.MODE["prefill"])
        assert rc == q8.OK, q8.last_error()
        # mismatched K is declined; an empty group is an error
        other = ctx.upload_p4(oracle.pack_q8_0_p4(np.zeros((64, 1024), np.float32)), 64, 1024)
        with pytest.raises(q8.Declined):
            ctx.linear_group(xd, [ts[0], other], [outs[0], ctx.alloc(64 * 4)], 1)
        ctx.release(other)
        wp = (ctypes.c_void_p * 1)()
        assert L.llmcp_q8_linear_group(ctx.handle, ctypes.byref(xi), 0, wp, wp, None,
                                       q8.MODE["decode"]) == q8.EINVAL
    finally:
        L.llmcp_q8_set_default_ctx(None)
        for t in ts:
            ctx.release(t)
