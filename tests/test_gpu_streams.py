"""Host-side use of the library as a runtime would: two contexts driven from
two host threads at once (ctypes drops the GIL in every call, so the calls
really overlap), and a caller-owned HIP stream adopted with
llmcp_q8_ctx_set_stream, whose work must be ordered with the caller's own
operations on that stream.  Results are checked bit for bit against the
oracle's scalar path (Q8Scalar.cpp:192-199 order)."""
import ctypes
import threading

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def hip_runtime():
    for name in ("libamdhip64.so.7", "/opt/rocm/lib/libamdhip64.so"):
        try:
            return ctypes.CDLL(name)
        except OSError:
            continue
    pytest.fail("libamdhip64 not found")


def test_two_contexts_on_two_threads(q8, oracle):
    rng = np.random.default_rng(31)
    jobs = []
    for n, k in ((2560, 2560), (9216, 2560)):
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        p4 = oracle.pack_q8_0_p4(w)
        xs = [rng.standard_normal((1, k)).astype(np.float32) for _ in range(3)]
        # fresh contexts compute the default platform's (aarch64) fma epilogue
        refs = [oracle.linear(x, p4, n, colpar=True, epilogue="fma") for x in xs]
        jobs.append((n, k, p4, xs, refs))
    errors, done = [], []

    def worker(job):
        n, k, p4, xs, refs = job
        try:
            with q8.Context(0) as c:
                t = c.upload_p4(p4, n, k)
                xds = [c.to_device(x) for x in xs]
                y = c.alloc(n * 4)
                for rep in range(40):
                    c.linear(xds[rep % 3], t, y, 1)
                    got = c.to_host(y, (1, n), np.float32)
                    if got.tobytes() != refs[rep % 3].tobytes():
                        errors.append((n, rep))
                        return
                c.release(t)
            done.append(n)
        except Exception as e:  # reported below, not swallowed
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(j,)) for j in jobs]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=90)
    assert not any(th.is_alive() for th in threads)
    assert not errors, errors
    assert sorted(done) == [2560, 9216]


def test_caller_stream_is_adopted_and_ordered(ctx, oracle, q8):
    L, H = q8.lib(), hip_runtime()
    rng = np.random.default_rng(32)
    n, k = 2560, 2560
    p4 = oracle.pack_q8_0_p4((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    t = ctx.upload_p4(p4, n, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    ref = oracle.linear(x, p4, n, colpar=True, epilogue=ctx.epilogue)
    xd = ctx.to_device(x)
    yd = ctx.to_device(np.full((1, n), np.nan, np.float32))
    stream = ctypes.c_void_p()
    assert H.hipStreamCreate(ctypes.byref(stream)) == 0
    own = L.llmcp_q8_ctx_stream(ctx.handle)
    try:
        assert L.llmcp_q8_ctx_set_stream(ctx.handle, stream) == 0
        assert L.llmcp_q8_ctx_stream(ctx.handle) == stream.value
        ctx.linear(xd, t, yd, 1)
        # the caller's own copy on the same stream must see the GEMV's result
        out = np.empty((1, n), np.float32)
        H.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p]
        assert H.hipMemcpyAsync(out.ctypes.data, ctypes.c_void_p(yd.ptr), out.nbytes,
                                2, stream) == 0  # hipMemcpyDeviceToHost
        assert H.hipStreamSynchronize(stream) == 0
        assert out.tobytes() == ref.tobytes()
    finally:
        assert L.llmcp_q8_ctx_set_stream(ctx.handle, None) == 0
        assert H.hipStreamSynchronize(stream) == 0
        assert H.hipStreamDestroy(stream) == 0
    assert L.llmcp_q8_ctx_stream(ctx.handle) == own
    # the context's own stream works again
    y2 = ctx.alloc(n * 4)
    ctx.linear(xd, t, y2, 1)
    assert ctx.to_host(y2, (1, n), np.float32).tobytes() == ref.tobytes()
    ctx.release(t)
