"""llmcp_q8_lm_head_noalloc: the lm_head with its scratch in a fixed
per-GPU device array instead of the context's workspace (no allocation on
any path).  Its results must equal llmcp_q8_lm_head's bit for bit, on
consecutive calls (the second with a smaller input, so stale scratch from
the first would show), under graph capture, and it must decline inputs the
fixed scratch cannot hold."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# Each test opens its own context per platform (rather than the session
# fixture) so that, with -x, this file runs after every other GPU test.
PLATFORMS = pytest.mark.parametrize("platform", ["aarch64", "x86"])


@pytest.fixture
def pctx(q8, platform):
    c = q8.Context(0)
    c.set_platform(platform)
    yield c
    c.close()


def call_noalloc(q8, ctx, x, m, w, logits, argmax, mode):
    xi = q8.f32_memref(x.ptr, m, w.cols)
    lo = q8.f32_memref(logits.ptr, m, w.rows)
    return q8.lib().llmcp_q8_lm_head_noalloc(
        ctx.handle, ctypes.byref(xi), ctypes.byref(w.memref()), ctypes.byref(lo),
        argmax.ptr if argmax is not None else None, q8.MODE[mode])


@PLATFORMS
def test_noalloc_matches_lm_head(pctx, oracle, q8):
    ctx = pctx
    rng = np.random.default_rng(77)
    v, k = 20000, 1024  # 5000 lane groups: M = 1 takes the pre-quantized row
    w = (rng.standard_normal((v, k)) * 0.02).astype(np.float32)
    p4 = oracle.pack_q8_0_p4(w)
    t = ctx.upload_p4(p4, v, k)
    try:
        for m, mode in ((24, "prefill"), (1, "decode")):  # second call smaller
            x = rng.standard_normal((m, k)).astype(np.float32)
            xd = ctx.to_device(x)
            la, lb = ctx.alloc(m * v * 4), ctx.alloc(m * v * 4)
            aa, ab = ctx.alloc(8), ctx.alloc(8)
            ctx.lm_head(xd, t, la, m, argmax=aa, mode=mode)
            rc = call_noalloc(q8, ctx, xd, m, t, lb, ab, mode)
            assert rc == q8.OK, q8.last_error()
            ya = ctx.to_host(la, (m, v), np.float32)
            yb = ctx.to_host(lb, (m, v), np.float32)
            assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32)), (m, mode)
            ia = int(ctx.to_host(aa, (1,), np.int64)[0])
            ib = int(ctx.to_host(ab, (1,), np.int64)[0])
            assert ia == ib == oracle.argmax(ya[-1]), (m, mode)
    finally:
        ctx.release(t)


@PLATFORMS
def test_noalloc_under_graph_capture(pctx, oracle, q8):
    ctx = pctx
    rng = np.random.default_rng(78)
    v, k = 20000, 1024
    p4 = oracle.pack_q8_0_p4((rng.standard_normal((v, k)) * 0.02).astype(np.float32))
    t = ctx.upload_p4(p4, v, k)
    try:
        x = rng.standard_normal((1, k)).astype(np.float32)
        xd, ld, am = ctx.to_device(x), ctx.alloc(v * 4), ctx.alloc(8)
        ref, ra = ctx.alloc(v * 4), ctx.alloc(8)
        ctx.lm_head(xd, t, ref, 1, argmax=ra)
        want = ctx.to_host(ref, (1, v), np.float32)
        want_id = int(ctx.to_host(ra, (1,), np.int64)[0])
        ctx.graph_begin()
        rc = call_noalloc(q8, ctx, xd, 1, t, ld, am, "decode")
        g = ctx.graph_end()
        assert rc == q8.OK, q8.last_error()
        try:
            for _ in range(3):  # eager work between the replays
                ctx.lm_head(xd, t, ref, 1, argmax=ra)
                ctx.graph_launch(g)
                got = ctx.to_host(ld, (1, v), np.float32)
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
                assert int(ctx.to_host(am, (1,), np.int64)[0]) == want_id
        finally:
            ctx.graph_destroy(g)
    finally:
        ctx.release(t)


@PLATFORMS
def test_noalloc_declines_oversized_input(pctx, oracle, q8):
    ctx = pctx
    rng = np.random.default_rng(79)
    v, k, m = 64, 1024, 8192  # 8 MiB of quantized rows: past the scratch
    p4 = oracle.pack_q8_0_p4((rng.standard_normal((v, k)) * 0.02).astype(np.float32))
    t = ctx.upload_p4(p4, v, k)
    try:
        xd, ld, am = ctx.alloc(m * k * 4), ctx.alloc(m * v * 4), ctx.alloc(8)
        rc = call_noalloc(q8, ctx, xd, m, t, ld, am, "prefill")
        assert rc == q8.DECLINED
        assert "scratch" in q8.last_error()
    finally:
        ctx.release(t)


def test_noalloc_one_context_per_gpu(oracle, q8):
    """The fixed scratch belongs to the first context that calls the entry
    on a GPU: another context's call is declined (their streams would race
    on the array) until the owner is destroyed."""
    rng = np.random.default_rng(80)
    v, k = 256, 1024
    p4 = oracle.pack_q8_0_p4((rng.standard_normal((v, k)) * 0.02).astype(np.float32))
    a, b = q8.Context(0), q8.Context(0)
    try:
        ta, tb = a.upload_p4(p4, v, k), b.upload_p4(p4, v, k)
        x = rng.standard_normal((1, k)).astype(np.float32)
        xa, la, ma = a.to_device(x), a.alloc(v * 4), a.alloc(8)
        xb, lb, mb = b.to_device(x), b.alloc(v * 4), b.alloc(8)
        assert call_noalloc(q8, a, xa, 1, ta, la, ma, "decode") == q8.OK, q8.last_error()
        assert call_noalloc(q8, b, xb, 1, tb, lb, mb, "decode") == q8.DECLINED
        assert "another context" in q8.last_error()
        want = a.to_host(la, (1, v), np.float32)
        a.release(ta)
        a.close()
        a = None
        assert call_noalloc(q8, b, xb, 1, tb, lb, mb, "decode") == q8.OK, q8.last_error()
        got = b.to_host(lb, (1, v), np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        assert int(b.to_host(mb, (1,), np.int64)[0]) == oracle.argmax(want[0])
        b.release(tb)
    finally:
        if a is not None:
            a.close()
        b.close()
