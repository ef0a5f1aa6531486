"""SPLIT_K accumulation (llmcp_q8_set_accumulation): a multi-row linear
whose tiles underfill the GPU splits K into ranges of whole passes, each a
serial chain of the platform's epilogue, and adds the ranges' partial sums
in order.  Not the reference's summation order, so the f32 outputs are
checked against the oracle (the reference's serial block order) within the
north-star tolerance (relative 1e-5 or absolute 1e-4), and bf16 outputs
within one bf16 step; the per-block int32 dots are the exact ones (the same
MFMAs), repeated calls give the same bits, one split is the EXACT result
bit for bit, and the lm_head stays exact."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-4


def within_tolerance(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    ok = (err <= ATOL) | (err <= RTOL * np.abs(ref))
    return bool(np.all(ok)), float(np.max(err / np.maximum(np.abs(ref), ATOL / RTOL)))


def bf16_within_one_step(got_bits, ref_bits):
    """Two bf16 arrays (uint16 bit patterns) equal or adjacent values."""
    a = got_bits.astype(np.int32)
    b = ref_bits.astype(np.int32)
    # map to a monotonic integer line (sign-magnitude -> two's complement)
    a = np.where(a & 0x8000, -(a & 0x7FFF), a)
    b = np.where(b & 0x8000, -(b & 0x7FFF), b)
    return bool(np.all(np.abs(a - b) <= 1))


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


@pytest.fixture(scope="module", params=["aarch64", "x86"])
def sctx(q8, request):
    c = q8.Context(0)
    c.set_platform(request.param)
    c.set_accumulation("split_k")
    yield c
    c.close()


def sample_rows(m):
    return np.arange(m) if m <= 8 else np.unique(np.array([0, 1, m // 2, m - 2, m - 1]))


# (m, n, k): configs[3] at M = 64 and 256, the model's other K classes
# (K = 9216: segmented layout; K = 4096), odd row counts and N tails;
# (200, 2560, 2560) puts the 128 x 96 workgroups' K splits on one
# workgroup per CU, with the producer waves.
SHAPES = [(64, 9216, 2560), (256, 9216, 2560), (2, 136, 1024), (33, 520, 2560),
          (97, 2560, 9216), (40, 264, 4096), (130, 7680, 2560), (200, 2560, 2560)]


@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("splits", [0, 2, 5])
def test_split_linear_within_tolerance(sctx, oracle, m, n, k, splits):
    rng = np.random.default_rng(m * 13 + n + k + splits)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[m // 2, 32:64] = 0.0
    p4 = oracle.pack_q8_0_p4(w)
    t = sctx.upload_p4(p4, n, k)
    try:
        sctx.set_accumulation("split_k", splits=splits)
        xd, yd, y2 = sctx.to_device(x), sctx.alloc(m * n * 4), sctx.alloc(m * n * 4)
        sctx.linear(xd, t, yd, m, mode="prefill")
        sctx.linear(xd, t, y2, m, mode="prefill")
        y = sctx.to_host(yd, (m, n), np.float32)
        # deterministic: the same bits on a second call
        assert np.array_equal(bits(y), bits(sctx.to_host(y2, (m, n), np.float32)))
        rows = sample_rows(m)
        ref = oracle.linear(x[rows], p4, n, epilogue=sctx.epilogue, colpar=True)
        ok, worst = within_tolerance(y[rows], ref)
        assert ok, (m, n, k, splits, worst)
    finally:
        sctx.set_accumulation("split_k")
        sctx.release(t)


@pytest.mark.parametrize("m,n,k", [(64, 2560, 2560), (24, 520, 9216)])
def test_one_split_is_exact(sctx, q8, oracle, m, n, k):
    """With one split the serial chain is the reference's: bit-exact."""
    rng = np.random.default_rng(m + n + k)
    p4 = oracle.pack_q8_0_p4((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = rng.standard_normal((m, k)).astype(np.float32)
    t = sctx.upload_p4(p4, n, k)
    try:
        sctx.set_accumulation("split_k", splits=1)
        xd, yd = sctx.to_device(x), sctx.alloc(m * n * 4)
        sctx.linear(xd, t, yd, m, mode="prefill")
        y = sctx.to_host(yd, (m, n), np.float32)
        rows = sample_rows(m)
        ref = oracle.linear(x[rows], p4, n, epilogue=sctx.epilogue, colpar=True)
        assert np.array_equal(bits(y[rows]), bits(ref))
    finally:
        sctx.set_accumulation("split_k")
        sctx.release(t)


@pytest.mark.parametrize("act", ["silu", "sigmoid", "softplus"])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_split_activations_and_bf16(sctx, oracle, act, dtype):
    """The reduction applies the epilogue: activation on the summed f32,
    then the bf16 store (within one bf16 step of the reference)."""
    m, n, k = 48, 1024, 2560
    rng = np.random.default_rng(len(act) + len(dtype))
    p4 = oracle.pack_q8_0_p4((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = rng.standard_normal((m, k)).astype(np.float32)
    t = sctx.upload_p4(p4, n, k)
    try:
        rows = sample_rows(m)
        ref = oracle.linear(x[rows], p4, n, activation=act, epilogue=sctx.epilogue,
                            colpar=True)
        if dtype == "f32":
            xd, yd = sctx.to_device(x), sctx.alloc(m * n * 4)
            sctx.linear(xd, t, yd, m, activation=act, mode="prefill")
            ok, worst = within_tolerance(sctx.to_host(yd, (m, n), np.float32)[rows], ref)
            assert ok, worst
        else:
            xb = oracle.f32_to_bf16_bits(x)
            ref = oracle.linear(oracle.bf16_bits_to_f32(xb)[rows], p4, n, activation=act,
                                epilogue=sctx.epilogue, colpar=True)
            xd, yd = sctx.to_device(xb), sctx.alloc(m * n * 2)
            sctx.linear(xd, t, yd, m, activation=act, mode="prefill", dtype="bf16")
            got = sctx.to_host(yd, (m, n), np.uint16)[rows]
            assert bf16_within_one_step(got, oracle.f32_to_bf16_bits(ref))
    finally:
        sctx.release(t)


def test_split_residual_group_and_swiglu(sctx, q8, oracle):
    """The other GEMM users in SPLIT_K mode, each checked as one op against
    the oracle on the same input: linear + residual add (in place), the
    grouped linears, and the SwiGLU (gate with SiLU, up times the gate) as
    configs[1]'s shape at M = 32."""
    rng = np.random.default_rng(5)
    m, h, f = 32, 2560, 9216
    wg, wu = [(rng.standard_normal((f, h)) * 0.02).astype(np.float32) for _ in range(2)]
    pg, pu = oracle.pack_q8_0_p4(wg), oracle.pack_q8_0_p4(wu)
    tg, tu = sctx.upload_p4(pg, f, h), sctx.upload_p4(pu, f, h)
    wo = (rng.standard_normal((h, h)) * 0.02).astype(np.float32)
    po = oracle.pack_q8_0_p4(wo)
    to = sctx.upload_p4(po, h, h)
    try:
        x = rng.standard_normal((m, h)).astype(np.float32)
        r = rng.standard_normal((m, h)).astype(np.float32)
        rows = sample_rows(m)
        xd = sctx.to_device(x)
        # residual add, in place on r
        rd = sctx.to_device(r)
        sctx.linear_add(xd, to, rd, rd, m, mode="prefill")
        got = sctx.to_host(rd, (m, h), np.float32)
        ref = oracle.linear(x[rows], po, h, epilogue=sctx.epilogue, colpar=True) + r[rows]
        ok, worst = within_tolerance(got[rows], ref)
        assert ok, ("residual", worst)
        # grouped linears sharing the input
        outs = [sctx.alloc(m * n * 4) for n in (f, h)]
        sctx.linear_group(xd, [tg, to], outs, m, activations=["silu", "none"], mode="prefill")
        for (p, n, act), o in zip([(pg, f, "silu"), (po, h, "none")], outs):
            ref = oracle.linear(x[rows], p, n, activation=act, epilogue=sctx.epilogue,
                                colpar=True)
            ok, worst = within_tolerance(sctx.to_host(o, (m, n), np.float32)[rows], ref)
            assert ok, ("group", act, worst)
        # SwiGLU: silu(x Wg^T) * (x Wu^T)
        hd = sctx.alloc(m * f * 4)
        sctx.swiglu(xd, tg, tu, hd, m, mode="prefill")
        g = oracle.linear(x[rows], pg, f, activation="silu", epilogue=sctx.epilogue,
                          colpar=True)
        u = oracle.linear(x[rows], pu, f, epilogue=sctx.epilogue, colpar=True)
        ok, worst = within_tolerance(sctx.to_host(hd, (m, f), np.float32)[rows], g * u)
        assert ok, ("swiglu", worst)
    finally:
        for t in (tg, tu, to):
            sctx.release(t)


def test_split_mlp_stages(sctx, oracle):
    """The whole MLP in SPLIT_K mode: h within tolerance of the oracle's
    SwiGLU, and the down projection within tolerance of the oracle applied
    to the h it was given (a Q8_1 rounding tie of h can flip under any
    change of h's last bits, as between the reference's two platforms, so
    the chain is checked one op at a time)."""
    rng = np.random.default_rng(9)
    m, h, f = 16, 2560, 9216
    ws = [(rng.standard_normal(s) * 0.02).astype(np.float32) for s in ((f, h), (f, h), (h, f))]
    ps = [oracle.pack_q8_0_p4(w) for w in ws]
    ts = [sctx.upload_p4(p, *w.shape) for p, w in zip(ps, ws)]
    try:
        x = rng.standard_normal((m, h)).astype(np.float32)
        xd, hd, yd = sctx.to_device(x), sctx.alloc(m * f * 4), sctx.alloc(m * h * 4)
        sctx.mlp(xd, ts[0], ts[1], ts[2], yd, h=hd, m=m, mode="prefill")
        hg = sctx.to_host(hd, (m, f), np.float32)
        rows = sample_rows(m)
        g = oracle.linear(x[rows], ps[0], f, activation="silu", epilogue=sctx.epilogue,
                          colpar=True)
        u = oracle.linear(x[rows], ps[1], f, epilogue=sctx.epilogue, colpar=True)
        ok, worst = within_tolerance(hg[rows], g * u)
        assert ok, ("h", worst)
        ref = oracle.linear(hg[rows], ps[2], h, epilogue=sctx.epilogue, colpar=True)
        ok, worst = within_tolerance(sctx.to_host(yd, (m, h), np.float32)[rows], ref)
        assert ok, ("down", worst)
    finally:
        for t in ts:
            sctx.release(t)


def test_lm_head_stays_exact(sctx, oracle):
    """The lm_head never splits: logits bit-exact and the argmax id the
    reference's, also in SPLIT_K mode."""
    rng = np.random.default_rng(21)
    m, v, k = 24, 4096, 2560
    p4 = oracle.pack_q8_0_p4((rng.standard_normal((v, k)) * 0.02).astype(np.float32))
    x = rng.standard_normal((m, k)).astype(np.float32)
    t = sctx.upload_p4(p4, v, k)
    try:
        sctx.set_accumulation("split_k", splits=5)
        xd, ld, am = sctx.to_device(x), sctx.alloc(m * v * 4), sctx.alloc(8)
        sctx.lm_head(xd, t, ld, m, argmax=am, mode="prefill")
        logits = sctx.to_host(ld, (m, v), np.float32)
        ref = oracle.linear(x[-1:], p4, v, epilogue=sctx.epilogue, colpar=True)
        assert np.array_equal(bits(logits[-1:]), bits(ref))
        assert int(sctx.to_host(am, (1,), np.int64)[0]) == oracle.argmax(ref[0])
    finally:
        sctx.set_accumulation("split_k")
        sctx.release(t)


def test_accumulation_switch(q8):
    c = q8.Context(0)
    try:
        assert c.accumulation == "exact"
        c.set_accumulation("split_k")
        assert c.accumulation == "split_k"
        with pytest.raises(q8.Q8Error):
            q8.check(q8.lib().llmcp_q8_set_accumulation(c.handle, 7))
        assert c.accumulation == "split_k"
        c.set_accumulation("exact")
        assert c.accumulation == "exact"
    finally:
        c.close()
