"""GPU parity of the prefill int8-MFMA GEMM (Q8Matmul.cpp / Q8Scalar.cpp
semantics) against the CPU oracle.  Each output element sums its blocks in
order with the selected epilogue, so results are compared bit for bit with
the oracle's matching epilogue and within the north-star tolerance with the
other one."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-4


def bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


def close(a, b):
    err = np.abs(a.astype(np.float64) - b.astype(np.float64))
    return bool(np.all((err <= ATOL) | (err <= RTOL * np.abs(b.astype(np.float64)))))


def gemm(ctx, p4, n, k, x, activation="none"):
    m = x.shape[0]
    t = ctx.upload_p4(p4, n, k)
    xd, yd = ctx.to_device(x), ctx.alloc(m * n * 4)
    ctx.linear(xd, t, yd, m, activation=activation, mode="prefill")
    y = ctx.to_host(yd, (m, n), np.float32)
    ctx.release(t)
    return y


@pytest.mark.parametrize("m,n,k", [(2, 136, 288), (19, 136, 288), (64, 264, 512),
                                   (130, 520, 1056), (256, 1024, 2560),
                                   (33, 136, 4096), (17, 264, 8864)])
def test_gemm_bitwise(ctx, oracle, m, n, k):
    rng = np.random.default_rng(m * 7 + n + k)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[m // 2, 32:64] = 0.0
    p4 = oracle.pack_q8_0_p4(w)
    y = gemm(ctx, p4, n, k, x)
    assert bits_equal(y, oracle.linear(x, p4, n, epilogue=ctx.epilogue))
    assert close(y, oracle.linear(x, p4, n, epilogue=ctx.other_epilogue))


def test_gemm_extreme_input_scales(ctx, oracle):
    # Blocks with subnormal, tiny and huge scales and zero blocks in
    # different rows: the tiled quantizer's exact-reciprocal fix-up.
    rng = np.random.default_rng(11)
    m, n, k = 70, 264, 2560
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[3, 0:32] *= np.float32(1e-41)
    x[5, 64:96] *= np.float32(1e-36)
    x[40, 128:160] *= np.float32(1e37)
    x[69, 2528:2560] *= np.float32(3e-39)
    x[33, :] = 0.0
    p4 = oracle.pack_q8_0_p4(w)
    assert bits_equal(gemm(ctx, p4, n, k, x), oracle.linear(x, p4, n, epilogue=ctx.epilogue))


def test_gemm_exact_operand_boundaries(ctx, oracle):
    # run_numeric.py:690-732 prefill case: M=19, N=136, K=288, exact operands,
    # zero last block of row 0, against a float64 matmul at 1e-5 / 1e-6.
    rng = np.random.default_rng(0)
    m, n, k = 19, 136, 288

    def exact(rows):
        v = rng.integers(-63, 64, size=(rows, k // 32, 32)).astype(np.float64)
        v[:, :, 0] = 127
        e = rng.integers(-6, -4, size=(rows, k // 32, 1))
        return np.ldexp(v, e).reshape(rows, k).astype(np.float32)

    x, w = exact(m), exact(n)
    x[0, -32:] = 0
    y = gemm(ctx, oracle.pack_q8_0_p4(w), n, k, x)
    np.testing.assert_allclose(y, x.astype(np.float64) @ w.astype(np.float64).T,
                               rtol=1e-5, atol=1e-6)


def test_gemm_silu(ctx, oracle):
    rng = np.random.default_rng(3)
    m, n, k = 33, 264, 1024
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    p4 = oracle.pack_q8_0_p4(w)
    y = gemm(ctx, p4, n, k, x, activation="silu")
    assert bits_equal(y, oracle.linear(x, p4, n, activation="silu", epilogue=ctx.epilogue))


@pytest.mark.parametrize("m", [64, 256, 1024])
def test_gemm_config4_rows(ctx, oracle, m):
    # Config 4 (K=2560 -> N=9216, M = 64 / 256 / 1024): full GEMM on the GPU,
    # 24 sampled rows (first, last, random) recomputed by the oracle.
    n, k = 9216, 2560
    p4d, _ = ctx.synthesize_p4(seed=40 + m, rows=n, cols=k)
    t = ctx.register_device_p4(p4d, n, k)
    p4 = ctx.to_host(p4d, (p4d.nbytes,), np.uint8)
    rng = np.random.default_rng(m)
    x = rng.standard_normal((m, k)).astype(np.float32)
    xd, yd = ctx.to_device(x), ctx.alloc(m * n * 4)
    ctx.linear(xd, t, yd, m, mode="prefill")
    y = ctx.to_host(yd, (m, n), np.float32)
    rows = np.unique(np.concatenate([[0, m - 1], rng.integers(0, m, 22)]))
    ref = oracle.linear(x[rows], p4, n, epilogue=ctx.epilogue)
    assert bits_equal(y[rows], ref)
    ctx.release(t)


def test_prefill_swiglu(ctx, oracle):
    # Prefill MLP hidden for M > 1: silu(gate GEMM) * up GEMM, SDOT epilogue.
    rng = np.random.default_rng(5)
    m, n, k = 40, 1056, 512
    wg = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    wu = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    pg, pu = oracle.pack_q8_0_p4(wg), oracle.pack_q8_0_p4(wu)
    tg, tu = ctx.upload_p4(pg, n, k), ctx.upload_p4(pu, n, k)
    xd, hd = ctx.to_device(x), ctx.alloc(m * n * 4)
    ctx.swiglu(xd, tg, tu, hd, m, mode="prefill")
    h = ctx.to_host(hd, (m, n), np.float32)
    assert bits_equal(h, oracle.swiglu(x, pg, pu, n, epilogue=ctx.epilogue))
    ctx.release(tg)
    ctx.release(tu)


def _sampled_rows(rng, m, count=32):
    return np.unique(np.concatenate([[0, m - 1], rng.integers(0, m, count - 2)]))


# More tiles than resident workgroups: with K = 288 and 3872 (1 and 4 blocks
# per lane slot; 288 is a single group of stages) each workgroup runs several
# tiles back to back, its DMA stream crossing from one tile into the next;
# K = 9216 (6 blocks per slot) takes one tile per workgroup in two rounds.
# N = 3720 is 39 column tiles (the schedule's padding ids to 40 are
# skipped).  Every column of 32 sampled rows is checked, which touches each
# column tile in most row tiles.
@pytest.mark.parametrize("k", [288, 3872, 9216])
def test_gemm_persistent_tiles(ctx, oracle, k):
    m, n = 1024, 3720
    rng = np.random.default_rng(900 + k)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    p4 = oracle.pack_q8_0_p4(w)
    y = gemm(ctx, p4, n, k, x)
    rows = _sampled_rows(rng, m)
    assert bits_equal(y[rows], oracle.linear(x[rows], p4, n, epilogue=ctx.epilogue))


def test_prefill_swiglu_persistent_tiles(ctx, oracle):
    m, n, k = 1024, 3720, 512
    rng = np.random.default_rng(950)
    wg = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    wu = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    pg, pu = oracle.pack_q8_0_p4(wg), oracle.pack_q8_0_p4(wu)
    tg, tu = ctx.upload_p4(pg, n, k), ctx.upload_p4(pu, n, k)
    xd, hd = ctx.to_device(x), ctx.alloc(m * n * 4)
    ctx.swiglu(xd, tg, tu, hd, m, mode="prefill")
    h = ctx.to_host(hd, (m, n), np.float32)
    rows = _sampled_rows(rng, m)
    assert bits_equal(h[rows], oracle.swiglu(x[rows], pg, pu, n, epilogue=ctx.epilogue))
    ctx.release(tg)
    ctx.release(tu)
