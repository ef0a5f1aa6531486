"""The C ABI's contract under failure and reuse, on the GPU: the arena
upload is all or nothing (Arena::load replaces the arena only on success,
lib/Runtime/WeightArena.cpp:28-29, :124-130), a captured graph is refused
once memory it references was reallocated, and a caller-owned stream is
ordered after the context's own work."""
import os
import tempfile

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


def unit_bytes(rows, cols):
    # device copy of a q8_0_p4 tensor: rows/4 lane groups x ceil(K/512)
    # units of 2176 B (the unit layout)
    return rows // 4 * ((cols // 32 + 15) // 16) * 2176


def test_arena_upload_is_all_or_nothing(q8, oracle):
    rng = np.random.default_rng(41)
    shapes = [("a", 64, 512), ("b", 128, 512), ("c", 32, 1024)]
    ws = {name: (rng.standard_normal((r, c)) * 0.02).astype(np.float32)
          for name, r, c in shapes}
    p4 = {name: oracle.pack_q8_0_p4(w) for name, w in ws.items()}
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "w.bin")
        q8.write_arena(path, [(n, r, c, p4[n]) for n, r, c in shapes])
        arena = np.fromfile(path, dtype=np.uint8)
    # where each tensor's bytes sit in the file image (the registry keys)
    offsets = {n: bytes(arena).find(p4[n].tobytes()) for n, _, _ in shapes}
    assert all(o >= 64 for o in offsets.values())
    base = arena.ctypes.data
    x = rng.standard_normal((1, 512)).astype(np.float32)
    with q8.Context(0) as ctx:
        # an earlier registration that must survive the failed upload
        keep = ctx.upload_p4(oracle.pack_q8_0_p4(ws["a"]), 64, 512)
        # room for the kept tensor and "a", not for "b": the second staged
        # tensor is refused
        ctx.set_weight_budget(2 * unit_bytes(64, 512) + 1024)
        with pytest.raises(q8.Q8Error) as e:
            ctx.upload_arena(arena)
        assert e.value.code == q8.ENOMEM
        for n, _, _ in shapes:
            assert q8.lib().llmcp_q8_device_bytes(ctx.handle, base + offsets[n]) == 0
        assert q8.lib().llmcp_q8_device_bytes(ctx.handle, keep.key) == unit_bytes(64, 512)
        xd, yd = ctx.to_device(x), ctx.alloc(64 * 4)
        ctx.linear(xd, keep, yd, 1)
        ref = oracle.linear(x, p4["a"], 64, epilogue=ctx.epilogue)
        assert bits_equal(ctx.to_host(yd, (1, 64), np.float32), ref)
        # without the cap every tensor registers, and descriptors into the
        # file image resolve to the device copies
        ctx.set_weight_budget(0)
        assert ctx.upload_arena(arena) == 3
        for n, r, c in shapes:
            assert q8.lib().llmcp_q8_device_bytes(ctx.handle, base + offsets[n]) == unit_bytes(r, c)
        wb = q8.Weight(ctx, base + offsets["b"], 128, 512, owner=arena)
        yb = ctx.alloc(128 * 4)
        ctx.linear(xd, wb, yb, 1)
        assert bits_equal(ctx.to_host(yb, (1, 128), np.float32),
                          oracle.linear(x, p4["b"], 128, epilogue=ctx.epilogue))


def test_graph_refused_after_reallocation(q8, oracle):
    rng = np.random.default_rng(42)
    n, k = 256, 1024
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    p4 = oracle.pack_q8_0_p4(w)
    x = rng.standard_normal((1, k)).astype(np.float32)
    with q8.Context(0) as ctx:
        t = ctx.upload_p4(p4, n, k)
        xd, yd = ctx.to_device(x), ctx.alloc(n * 4)
        ref = oracle.linear(x, p4, n, epilogue=ctx.epilogue)

        def capture():
            ctx.graph_begin()
            ctx.linear(xd, t, yd, 1)
            return ctx.graph_end()

        g = capture()
        ctx.graph_launch(g)
        assert bits_equal(ctx.to_host(yd, (1, n), np.float32), ref)
        # a prefill call grows the workspace (the tiled scratch for 300 rows):
        # the graph may hold the old scratch addresses and is refused
        xm = rng.standard_normal((300, k)).astype(np.float32)
        xmd, ymd = ctx.to_device(xm), ctx.alloc(300 * n * 4)
        ctx.linear(xmd, t, ymd, 300, mode="prefill")
        with pytest.raises(q8.Q8Error) as e:
            ctx.graph_launch(g)
        assert e.value.code == q8.ESTALE
        ctx.graph_destroy(g)
        g = capture()  # captured again: fine
        ctx.linear(ctx.to_device(np.zeros((1, k), np.float32)), t, yd, 1)
        ctx.graph_launch(g)
        assert bits_equal(ctx.to_host(yd, (1, n), np.float32), ref)
        # registering the weight again frees its old device copy
        t = ctx.upload_p4(p4, n, k)
        with pytest.raises(q8.Q8Error) as e:
            ctx.graph_launch(g)
        assert e.value.code == q8.ESTALE
        ctx.graph_destroy(g)
        # a graph from another context is refused too
        with q8.Context(0) as other:
            with pytest.raises(q8.Q8Error) as e:
                g2 = capture()
                other.graph_launch(g2)
            assert e.value.code == q8.EINVAL
            ctx.graph_destroy(g2)


def test_platform_switch_is_per_context(q8, oracle):
    rng = np.random.default_rng(43)
    n, k = 264, 2560
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    p4 = oracle.pack_q8_0_p4(w)
    x = rng.standard_normal((5, k)).astype(np.float32)
    refs = {e: oracle.linear(x, p4, n, epilogue=e) for e in ("fma", "scalar")}
    assert not bits_equal(refs["fma"], refs["scalar"])  # the switch matters here
    with q8.Context(0) as a, q8.Context(0) as b:
        assert a.platform == "aarch64"  # the default
        b.set_platform("x86")
        for c in (a, b):
            t = c.upload_p4(p4, n, k)
            xd = c.to_device(x)
            for m in (1, 5):
                for mode in ("decode", "prefill"):
                    yd = c.alloc(m * n * 4)
                    c.linear(xd, t, yd, m, mode=mode)
                    assert bits_equal(c.to_host(yd, (m, n), np.float32),
                                      refs[c.epilogue][:m]), (c.platform, m, mode)
        with pytest.raises(q8.Q8Error) as e:
            a.set_platform_code(7)
        assert e.value.code == q8.EINVAL


def test_microbench_peaks(q8):
    """The peak microbenchmarks run and report plausible rates (HBM reads
    between 1 and 8 TB/s over a buffer past every cache, int8 MFMA between
    0.5 and 5.1 POPS), and reject bad arguments."""
    c = q8.Context(0)
    try:
        rd = c.microbench_bandwidth("read", 1 << 30, launches=3)
        cp = c.microbench_bandwidth("copy", 1 << 30, launches=3)
        assert 1000.0 < rd < 8000.0, rd
        assert 1000.0 < cp < 8000.0, cp
        tops = c.microbench_int8_mfma(2000)
        assert 500.0 < tops < 5100.0, tops
        # the GEMM's per-block work: the exact epilogue cannot beat its own
        # MFMAs, and both stay below the MFMA issue peak
        exact = c.microbench_epilogue("exact", 2000)
        cvtfree = c.microbench_epilogue("cvtfree", 2000)
        mfma = c.microbench_epilogue("mfma", 2000)
        assert 100.0 < exact < 5100.0 and 100.0 < cvtfree < 5100.0, (exact, cvtfree)
        assert exact < 1.05 * mfma < 1.05 * 5100.0, (exact, mfma)
        with pytest.raises(q8.Q8Error):
            c.microbench_bandwidth("read", 1 << 20)  # below one 64 MiB unit
        with pytest.raises(q8.Q8Error):
            q8.check(q8.lib().llmcp_q8_microbench_int8_mfma(c.handle, 0, None))
        with pytest.raises(q8.Q8Error):
            c.microbench_epilogue("exact", 1)  # below one block pair
        with pytest.raises(q8.Q8Error):
            q8.check(q8.lib().llmcp_q8_microbench_epilogue(c.handle, 3, 100, None))
    finally:
        c.close()


def test_prefill_operands_over_4gib_declined(q8, oracle):
    """The prefill GEMM reads its operands at 32-bit offsets (buffer-addressed
    loads), so a multi-row linear over a weight of 4 GiB or more is declined
    (LLMCP_Q8_DECLINED: the caller's own path runs) before anything is
    launched, also for the lm_head, the grouped linears and the MLP; the
    context stays usable.  The 4.56 GB weight is registered from an
    uninitialised device buffer: no call computes with it."""
    rows, cols = 262144, 16384
    nbytes = rows * cols // 32 * 34
    assert unit_bytes(rows, cols) >= 1 << 32
    rng = np.random.default_rng(47)
    with q8.Context(0) as ctx:
        big = ctx.register_device_p4(ctx.alloc(nbytes), rows, cols)
        x = rng.standard_normal((2, cols)).astype(np.float32)
        xd, yd = ctx.to_device(x), ctx.alloc(2 * rows * 4)
        with pytest.raises(q8.Declined):
            ctx.linear(xd, big, yd, 2, mode="prefill")
        with pytest.raises(q8.Declined):
            ctx.lm_head(xd, big, yd, 2)
        with pytest.raises(q8.Declined):
            ctx.linear_group(xd, [big], [yd], 2)
        ctx.release(big)
        # an ordinary prefill linear on the same context afterwards
        n, k = 64, 512
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        p4 = oracle.pack_q8_0_p4(w)
        t = ctx.upload_p4(p4, n, k)
        xs = rng.standard_normal((3, k)).astype(np.float32)
        xsd, ysd = ctx.to_device(xs), ctx.alloc(3 * n * 4)
        ctx.linear(xsd, t, ysd, 3, mode="prefill")
        assert bits_equal(ctx.to_host(ysd, (3, n), np.float32),
                          oracle.linear(xs, p4, n, epilogue=ctx.epilogue))
