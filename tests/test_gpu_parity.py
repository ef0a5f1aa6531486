"""GPU parity of the HIP path against the CPU oracle, through the C ABI.

Bars: integer/byte/index work bit-exact (packed bytes, Q8_1 activations,
per-block int32 dots, argmax id, embedding values).  f32 outputs: every
path keeps the reference's block order with the selected platform's
epilogue -- fma on aarch64 (Q8Decode.cpp:192-203), mul+add on x86
(Q8Scalar.cpp:192-199) -- so it is compared bit for bit with the oracle's
matching epilogue and, within the north-star tolerance (max relative error
1e-5 or absolute 1e-4), with the other one.  The session context runs every
test on both platforms (tests/conftest.py).
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
RTOL, ATOL = 1e-5, 1e-4


def close(a, b):
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    err = np.abs(a - b)
    return bool(np.all((err <= ATOL) | (err <= RTOL * np.abs(b))))


def bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


def weights(rng, n, k, scale=0.02):
    return (rng.standard_normal((n, k)) * scale).astype(np.float32)


def run_linear(ctx, oracle, w, x, activation="none", mode="decode"):
    n, k = w.shape
    m = x.shape[0]
    p4 = oracle.pack_q8_0_p4(w)
    wt = ctx.upload_p4(p4, n, k)
    xd = ctx.to_device(x)
    yd = ctx.alloc(m * n * 4)
    ctx.linear(xd, wt, yd, m, activation=activation, mode=mode)
    y = ctx.to_host(yd, (m, n), np.float32)
    ctx.release(wt)
    return y, p4


def test_golden_fixture_rows(ctx, oracle):
    z = np.load(os.path.join(GOLDEN, "q8_small_case.npz"))
    n, k = z["w"].shape
    wt = ctx.upload_p4(z["p4"], n, k)
    for r in range(z["x"].shape[0]):
        xd = ctx.to_device(z["x"][r:r + 1])
        yd = ctx.alloc(n * 4)
        ctx.linear(xd, wt, yd, 1)
        y = ctx.to_host(yd, (1, n), np.float32)
        same, other = ("y_fma", "y_scalar") if ctx.epilogue == "fma" else ("y_scalar", "y_fma")
        assert bits_equal(y, z[same][r:r + 1])
        assert close(y, z[other][r:r + 1])
    ctx.release(wt)


# 4096 / 3872 (8 units of 16 blocks) and 9216 / 8864 (18 units) use the
# segmented unit layout (4 and 6 blocks per lane slot and pass); 3872 and
# 8864 also end in padded blocks.
@pytest.mark.parametrize("k", [32, 288, 512, 1024, 1536, 2048, 2560, 3072,
                               3872, 4096, 5120, 8864, 9216])
def test_gemv_matches_scalar_reference_bitwise(ctx, oracle, k):
    rng = np.random.default_rng(100 + k)
    n = 264 if k != 2560 else 2560
    w = weights(rng, n, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    y, p4 = run_linear(ctx, oracle, w, x)
    ref = oracle.linear(x, p4, n, epilogue=ctx.epilogue)
    assert bits_equal(y, ref), np.max(np.abs(y - ref))
    assert close(y, oracle.linear(x, p4, n, epilogue=ctx.other_epilogue))


# Input rows whose blocks have extreme scales: subnormal (the reciprocal's
# IEEE branch inside the GEMV's in-workgroup quantizer), tiny-normal, huge,
# zero and mixed blocks, for the unrolled (2560, 9216), segmented and runtime
# (3072) pass counts; the M = 1024 prefill path goes through the tiled
# quantizer with the same rows.
@pytest.mark.parametrize("k", [2560, 3072, 9216])
def test_gemv_extreme_input_scales(ctx, oracle, k):
    rng = np.random.default_rng(300 + k)
    n = 264
    w = weights(rng, n, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    x[0, 0:32] *= np.float32(1e-41)     # subnormal values, subnormal scale
    x[0, 64:96] *= np.float32(1e-36)    # scale below 2^-125
    x[0, 65] = np.float32(-1e-36)
    x[0, 128:160] *= np.float32(1e37)   # scale above 2^126 / 127
    x[0, 192:224] = 0.0
    x[0, k - 32:] *= np.float32(3e-39)
    y, p4 = run_linear(ctx, oracle, w, x)
    assert bits_equal(y, oracle.linear(x, p4, n, epilogue=ctx.epilogue))


def test_gemv_exact_operands(ctx, oracle):
    # run_numeric.py:690-732 decode boundary case: N=136, K=288, exact operands,
    # last block of x zero; float64 matmul of the exact values at 1e-5 / 1e-6.
    rng = np.random.default_rng(5)
    n, k = 136, 288
    blocks = k // 32

    def exact(rows):
        v = rng.integers(-63, 64, size=(rows, blocks, 32)).astype(np.float64)
        v[:, :, 0] = 127
        e = rng.integers(-6, -4, size=(rows, blocks, 1))
        return np.ldexp(v, e).reshape(rows, k).astype(np.float32)

    x = exact(1)
    w = exact(n)
    x[0, -32:] = 0
    y, _ = run_linear(ctx, oracle, w, x)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-6)


def test_gemv_silu_activation(ctx, oracle):
    rng = np.random.default_rng(7)
    w = weights(rng, 512, 2560)
    x = rng.standard_normal((1, 2560)).astype(np.float32)
    y, p4 = run_linear(ctx, oracle, w, x, activation="silu")
    assert bits_equal(y, oracle.linear(x, p4, 512, activation="silu", epilogue=ctx.epilogue))


def test_prefill_single_row_uses_same_math(ctx, oracle):
    rng = np.random.default_rng(8)
    w = weights(rng, 128, 1024)
    x = rng.standard_normal((1, 1024)).astype(np.float32)
    y, p4 = run_linear(ctx, oracle, w, x, mode="prefill")
    assert bits_equal(y, oracle.linear(x, p4, 128, epilogue=ctx.epilogue))


def test_decode_and_prefill_rows_share_the_platform_epilogue(ctx, oracle, q8):
    # The reference's decode emitter takes any M (Q8Decode.cpp:236-256) and
    # computes the same per-block epilogue as its prefill GEMM on one
    # platform (fma on aarch64, the scalar path's mul+add for every mode on
    # x86), so decode and prefill rows agree bit for bit with the platform's
    # oracle epilogue.
    rng = np.random.default_rng(9)
    for m, n, k in ((2, 64, 256), (37, 264, 2560), (70, 1032, 9216)):
        w = weights(rng, n, k)
        x = rng.standard_normal((m, k)).astype(np.float32)
        p4 = oracle.pack_q8_0_p4(w)
        t = ctx.upload_p4(p4, n, k)
        xd, yd = ctx.to_device(x), ctx.alloc(m * n * 4)
        ref = oracle.linear(x, p4, n, epilogue=ctx.epilogue)
        for mode in ("decode", "prefill"):
            ctx.linear(xd, t, yd, m, mode=mode)
            y = ctx.to_host(yd, (m, n), np.float32)
            assert bits_equal(y, ref), (m, n, k, mode)
            assert close(y, oracle.linear(x, p4, n, epilogue=ctx.other_epilogue))
        ctx.release(t)


def test_unregistered_weight_is_not_found(ctx, q8):
    xd = ctx.to_device(np.zeros((1, 64), np.float32))
    yd = ctx.alloc(64 * 4)
    fake = q8.Weight(ctx, xd.ptr, 8, 64)
    with pytest.raises(q8.Q8Error) as e:
        ctx.linear(xd, fake, yd, 1)
    assert e.value.code == q8.ENOTFOUND


def test_swiglu_bitwise(ctx, oracle):
    # Decode-MLP gate/up shape (config 2): K=2560 -> N=9216, silu(g) * u.
    rng = np.random.default_rng(10)
    n, k = 9216, 2560
    wg, wu = weights(rng, n, k), weights(rng, n, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    pg, pu = oracle.pack_q8_0_p4(wg), oracle.pack_q8_0_p4(wu)
    tg, tu = ctx.upload_p4(pg, n, k), ctx.upload_p4(pu, n, k)
    xd, hd = ctx.to_device(x), ctx.alloc(n * 4)
    ctx.swiglu(xd, tg, tu, hd, 1)
    h = ctx.to_host(hd, (1, n), np.float32)
    ref = oracle.swiglu(x, pg, pu, n, colpar=True, epilogue=ctx.epilogue)
    assert bits_equal(h, ref)
    ctx.release(tg)
    ctx.release(tu)


def test_decode_mlp_end_to_end(ctx, oracle):
    # Config 2: h = silu(x Wg^T) * (x Wu^T), y = h Wd^T, all Q8_0.  Because each
    # stage is bit-identical, the whole MLP is too.
    rng = np.random.default_rng(11)
    hidden, ffn = 2560, 9216
    wg, wu, wd = weights(rng, ffn, hidden), weights(rng, ffn, hidden), weights(rng, hidden, ffn)
    x = rng.standard_normal((1, hidden)).astype(np.float32)
    pg, pu, pd = (oracle.pack_q8_0_p4(w) for w in (wg, wu, wd))
    tg, tu, td = ctx.upload_p4(pg, ffn, hidden), ctx.upload_p4(pu, ffn, hidden), ctx.upload_p4(pd, hidden, ffn)
    xd, hd, yd = ctx.to_device(x), ctx.alloc(ffn * 4), ctx.alloc(hidden * 4)
    ctx.swiglu(xd, tg, tu, hd, 1)
    ctx.linear(hd, td, yd, 1)
    y = ctx.to_host(yd, (1, hidden), np.float32)
    h_ref = oracle.swiglu(x, pg, pu, ffn, colpar=True, epilogue=ctx.epilogue)
    y_ref = oracle.linear(h_ref, pd, hidden, colpar=True, epilogue=ctx.epilogue)
    assert bits_equal(y, y_ref)
    for t in (tg, tu, td):
        ctx.release(t)


def test_fused_mlp_matches_separate_ops(ctx, oracle):
    # llmcp_q8_mlp: the gate/up GEMV writes h, the down GEMV quantizes it per
    # workgroup; the result must equal swiglu -> linear bit for bit, over
    # repeated calls, with the caller's h buffer or the context's, and for a
    # width that leaves a partial last pass (ffn = 1056 -> 33 blocks).
    rng = np.random.default_rng(21)
    for hidden, ffn in ((2560, 9216), (512, 1056)):
        wg, wu, wd = weights(rng, ffn, hidden), weights(rng, ffn, hidden), weights(rng, hidden, ffn)
        pg, pu, pd = (oracle.pack_q8_0_p4(w) for w in (wg, wu, wd))
        tg, tu, td = ctx.upload_p4(pg, ffn, hidden), ctx.upload_p4(pu, ffn, hidden), ctx.upload_p4(pd, hidden, ffn)
        for trial in range(3):
            x = rng.standard_normal((1, hidden)).astype(np.float32)
            xd, hd, yd = ctx.to_device(x), ctx.alloc(ffn * 4), ctx.alloc(hidden * 4)
            ctx.mlp(xd, tg, tu, td, yd, h=hd)
            h = ctx.to_host(hd, (1, ffn), np.float32)
            y = ctx.to_host(yd, (1, hidden), np.float32)
            h_ref = oracle.swiglu(x, pg, pu, ffn, colpar=True, epilogue=ctx.epilogue)
            y_ref = oracle.linear(h_ref, pd, hidden, colpar=True, epilogue=ctx.epilogue)
            assert bits_equal(h, h_ref)
            assert bits_equal(y, y_ref), (hidden, ffn, trial)
            y2d = ctx.alloc(hidden * 4)
            ctx.mlp(xd, tg, tu, td, y2d)  # internal h buffer
            assert bits_equal(ctx.to_host(y2d, (1, hidden), np.float32), y_ref)
        for t in (tg, tu, td):
            ctx.release(t)


def test_wide_output_uses_prequantized_input(ctx, oracle, q8):
    # N > 16384 quantizes the row once before the GEMV; a misaligned input
    # row takes the same path.  Both must match the reference bit for bit.
    rng = np.random.default_rng(22)
    n, k = 16416, 512
    w = weights(rng, n, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    y, p4 = run_linear(ctx, oracle, w, x)
    assert bits_equal(y, oracle.linear(x, p4, n, epilogue=ctx.epilogue))
    n2 = 264
    w2 = weights(rng, n2, k)
    p42 = oracle.pack_q8_0_p4(w2)
    t = ctx.upload_p4(p42, n2, k)
    xd = ctx.to_device(np.concatenate([[0.0], x.ravel()]).astype(np.float32))
    yd = ctx.alloc(n2 * 4)
    ctx.linear(xd.ptr + 4, t, yd, 1)
    assert bits_equal(ctx.to_host(yd, (1, n2), np.float32), oracle.linear(x, p42, n2, epilogue=ctx.epilogue))
    ctx.release(t)


def test_lm_head_argmax_and_ties(ctx, oracle):
    rng = np.random.default_rng(12)
    v, k = 4096, 2560
    w = weights(rng, v, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    p4 = oracle.pack_q8_0_p4(w)
    ref = oracle.linear(x, p4, v, epilogue=ctx.epilogue)
    best = int(np.argmax(ref))
    # Duplicate the winning row at a lower and a higher index: equal logits,
    # the first maximum must win (std::max_element).
    lo, hi = 17 if best != 17 else 18, v - 3
    w2 = w.copy()
    w2[lo] = w[best]
    w2[hi] = w[best]
    for table, expect in ((w, best), (w2, min(lo, best))):
        p4 = oracle.pack_q8_0_p4(table)
        t = ctx.upload_p4(p4, v, k)
        xd, ld, am = ctx.to_device(x), ctx.alloc(v * 4), ctx.alloc(8)
        for _ in range(3):  # repeated calls reuse and reset the workspace
            ctx.lm_head(xd, t, ld, 1, argmax=am)
            logits = ctx.to_host(ld, (1, v), np.float32)
            idx = int(ctx.to_host(am, (1,), np.int64)[0])
            assert bits_equal(logits, oracle.linear(x, p4, v, epilogue=ctx.epilogue))
            assert idx == oracle.argmax(logits) == expect
        ctx.release(t)


def test_lm_head_argmax_back_to_back(ctx, oracle):
    # Calls queued without a sync in between, alternating two rows whose
    # maxima differ by ~100x: a key left over from one call would win the
    # next one.  4096 x 2560 folds 1024 workgroups into the slots; 248320 rows
    # (test_lm_head_full_vocab) put several workgroups on each slot.
    rng = np.random.default_rng(15)
    v, k = 4096, 2560
    p4 = oracle.pack_q8_0_p4(weights(rng, v, k))
    t = ctx.upload_p4(p4, v, k)
    x1 = rng.standard_normal((1, k)).astype(np.float32)
    x2 = (-0.01 * x1).astype(np.float32)
    xs = [ctx.to_device(x1), ctx.to_device(x2)]
    expect = [oracle.argmax(oracle.linear(x, p4, v, epilogue=ctx.epilogue)) for x in (x1, x2)]
    assert expect[0] != expect[1]
    ld = ctx.alloc(v * 4)
    ams = [ctx.alloc(8) for _ in range(6)]
    for i, am in enumerate(ams):
        ctx.lm_head(xs[i % 2], t, ld, 1, argmax=am)
    got = [int(ctx.to_host(am, (1,), np.int64)[0]) for am in ams]
    assert got == [expect[i % 2] for i in range(6)]
    ctx.release(t)


def test_device_resident_token_loop(ctx, oracle):
    # The decode loop's tail on the device: the embedding gather reads the
    # token id the previous lm_head's argmax wrote, with no host round trip
    # between steps (the 1 MB of logits and the id stay in HBM).  Separate
    # embedding and head tables so the ids keep moving.  Run eagerly, then as
    # one captured step replayed, checking every id against the oracle chain.
    rng = np.random.default_rng(16)
    v, k = 4096, 2560
    pe = oracle.pack_q8_0_p4(weights(rng, v, k))
    pw = oracle.pack_q8_0_p4(weights(rng, v, k))
    te, tw = ctx.upload_p4(pe, v, k), ctx.upload_p4(pw, v, k)
    chain = [7]
    for _ in range(6):
        x = oracle.embedding(np.array(chain[-1:], np.int64), pe, k)
        chain.append(int(oracle.argmax(oracle.linear(x, pw, v, epilogue=ctx.epilogue))))
    assert len(set(chain)) == len(chain)
    xd, ld = ctx.alloc(k * 4), ctx.alloc(v * 4)
    ids = [ctx.to_device(np.array([chain[0]], np.int64))]
    ids += [ctx.alloc(8) for _ in range(6)]
    for i in range(6):
        ctx.embedding(ids[i], 1, te, xd)
        ctx.lm_head(xd, tw, ld, 1, argmax=ids[i + 1])
    got = [int(ctx.to_host(t, (1,), np.int64)[0]) for t in ids]
    assert got == chain
    am = ctx.to_device(np.array([chain[0]], np.int64))
    ctx.graph_begin()
    ctx.embedding(am, 1, te, xd)
    ctx.lm_head(xd, tw, ld, 1, argmax=am)
    g = ctx.graph_end()
    for i in range(6):
        ctx.graph_launch(g)
        assert int(ctx.to_host(am, (1,), np.int64)[0]) == chain[i + 1]
    ctx.graph_destroy(g)
    assert ctx.check_flag() == 0
    ctx.release(te)
    ctx.release(tw)


def test_lm_head_full_vocab(ctx, oracle):
    # Config 3: tied 248320 x 2560 table (0.67 GB of Q8_0), device-synthesized.
    v, k = 248320, 2560
    p4d, _ = ctx.synthesize_p4(seed=3, rows=v, cols=k)
    t = ctx.register_device_p4(p4d, v, k)
    p4 = ctx.to_host(p4d, (p4d.nbytes,), np.uint8)
    rng = np.random.default_rng(13)
    x = rng.standard_normal((1, k)).astype(np.float32)
    xd, ld, am = ctx.to_device(x), ctx.alloc(v * 4), ctx.alloc(8)
    ctx.lm_head(xd, t, ld, 1, argmax=am)
    logits = ctx.to_host(ld, (1, v), np.float32)
    idx = int(ctx.to_host(am, (1,), np.int64)[0])
    ref = oracle.linear(x, p4, v, colpar=True, epilogue=ctx.epilogue)
    assert bits_equal(logits, ref)
    top2 = np.sort(ref.ravel())[-2:]
    assert top2[1] - top2[0] > 1e-4  # the id is meaningful at tolerance level
    assert idx == oracle.argmax(ref)
    ctx.release(t)


@pytest.mark.parametrize("v,k", [(4096, 2560), (1024, 3872), (512, 9216)])
def test_embedding_gather(ctx, oracle, v, k):
    rng = np.random.default_rng(14 + k)
    w = weights(rng, v, k)
    p4 = oracle.pack_q8_0_p4(w)
    t = ctx.upload_p4(p4, v, k)
    tokens = rng.integers(0, v, 1024).astype(np.int64)
    tokens[:4] = [0, v - 1, 3, 4]
    td, od = ctx.to_device(tokens), ctx.alloc(tokens.size * k * 4)
    ctx.embedding(td, tokens.size, t, od)
    out = ctx.to_host(od, (tokens.size, k), np.float32)
    assert bits_equal(out, oracle.embedding(tokens, p4, k))
    assert ctx.check_flag() == 0
    bad = np.array([2, -1, v], np.int64)
    bd, bo = ctx.to_device(bad), ctx.alloc(3 * k * 4)
    ctx.embedding(bd, 3, t, bo)
    out = ctx.to_host(bo, (3, k), np.float32)
    assert bits_equal(out[0], oracle.embedding(bad[:1], p4, k)[0])
    assert np.all(out[1:] == 0) and ctx.check_flag() == 1
    ctx.release(t)


def test_quantize_activations_bitwise(ctx, oracle):
    rng = np.random.default_rng(15)
    m, k = 7, 2560
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[2, 64:96] = 0.0
    x[3, 0] = 127.0
    x[3, 1:8] = [2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 126.5]
    x[3, 8:32] = 0.0
    # scales far from 1: subnormal scale (the reciprocal's IEEE branch),
    # subnormal inputs, and very large magnitudes (the fast branch)
    x[4, 0:32] *= np.float32(1e-36)
    x[4, 32:64] *= np.float32(1e-41)
    x[4, 33] = np.float32(-1e-36)  # keeps 1/scale finite
    x[5, 64:96] *= np.float32(1e37)
    xd, qd, sd = ctx.to_device(x), ctx.alloc(m * k), ctx.alloc(m * k // 32 * 4)
    ctx.quantize(xd, m, k, qd, sd)
    qa, sa = oracle.quantize_act_q8_1(x)
    assert np.array_equal(ctx.to_host(qd, (m, k), np.int8), qa)
    assert bits_equal(ctx.to_host(sd, (m, k // 32), np.float32), sa)


def test_quantizer_division_identities(ctx):
    """The quantizer replaces IEEE division by m*RN(1/127)+FMA correction and
    v_rcp_f32+Newton; the device checks both over every float input."""
    assert ctx.selftest_quantizer() == 0


def test_exp_pinned_over_all_floats(ctx, oracle):
    """The epilogues' exp (f64 Taylor evaluation rounded to f32) against the
    oracle's (host libm exp(double) rounded to f32) over every float input.
    The device lists every input whose exp lies within 2^-46 of a change of
    float rounding; both evaluations are far more accurate than that (the
    device's is measured against the device library's below), so they can
    only disagree on the listed inputs, which are compared one by one."""
    (near, differ, outside, max_ulps), xs, got = ctx.selftest_exp()
    assert outside == 0
    assert max_ulps <= 8  # f64 ulps: the device exp is accurate to ~2^-49
    assert 0 < near == xs.size  # every listed input was returned
    ref = oracle.expf(xs).view(np.uint32)
    bad = np.nonzero(ref != got)[0]
    assert bad.size == 0, (xs[bad][:8], got[bad][:8], ref[bad][:8])
    assert differ <= near


@pytest.mark.parametrize("k", [1056, 3872, 8864])
def test_block_dots_exact(ctx, oracle, k):
    rng = np.random.default_rng(16 + k)
    m, n = 3, 72
    w = weights(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    p4 = oracle.pack_q8_0_p4(w)
    t = ctx.upload_p4(p4, n, k)
    xd, od = ctx.to_device(x), ctx.alloc(m * n * (k // 32) * 4)
    ctx.block_dots(xd, t, od, m)
    got = ctx.to_host(od, (m, n, k // 32), np.int32)
    qa, _ = oracle.quantize_act_q8_1(x)
    assert np.array_equal(got, oracle.block_dots(qa, p4, n))
    ctx.release(t)


def test_device_packer_matches_oracle(ctx, oracle):
    p4d, wd = ctx.synthesize_p4(seed=9, rows=264, cols=2560, keep_f32=True)
    w = ctx.to_host(wd, (264, 2560), np.float32)
    p4 = ctx.to_host(p4d, (p4d.nbytes,), np.uint8)
    assert np.array_equal(p4, oracle.pack_q8_0_p4(w))
    assert abs(float(w.std()) - 0.02) < 0.001 and abs(float(w.mean())) < 0.001


def test_arena_upload_and_descriptor_translation(ctx, oracle, q8, tmp_path):
    # Weights resolved through a descriptor that points into the mapped arena
    # file, as the AOT code's memref.view into the arena does
    # (ModelBuilder.cpp:140-175).
    rng = np.random.default_rng(17)
    wa, wb = weights(rng, 256, 512), weights(rng, 64, 1024)
    pa, pb = oracle.pack_q8_0_p4(wa), oracle.pack_q8_0_p4(wb)
    path = str(tmp_path / "arena.bin")
    q8.write_arena(path, [("blk.0.a", 256, 512, pa), ("blk.0.b", 64, 1024, pb)])
    f = np.fromfile(path, dtype=np.uint8)
    assert ctx.upload_arena(f) == 2
    import json
    import struct
    arena = struct.unpack_from("<Q", f, 16)[0]
    entries = json.loads(bytes(f[arena:]).decode())["tensors"]
    for e, p4 in zip(entries, (pa, pb)):
        n, k = e["shape"]
        wt = q8.Weight(ctx, f.ctypes.data + e["offset"], n, k, owner=f)
        x = rng.standard_normal((1, k)).astype(np.float32)
        xd, yd = ctx.to_device(x), ctx.alloc(n * 4)
        ctx.linear(xd, wt, yd, 1)
        assert bits_equal(ctx.to_host(yd, (1, n), np.float32), oracle.linear(x, p4, n, epilogue=ctx.epilogue))
        ctx.release(wt)


def test_mlir_ciface_entry_uses_default_context(ctx, oracle, q8):
    import ctypes
    rng = np.random.default_rng(18)
    w = weights(rng, 64, 256)
    p4 = oracle.pack_q8_0_p4(w)
    t = ctx.upload_p4(p4, 64, 256)
    x = rng.standard_normal((1, 256)).astype(np.float32)
    xd, yd = ctx.to_device(x), ctx.alloc(64 * 4)
    L = q8.lib()
    L.llmcp_q8_set_default_ctx(ctx.handle)
    xi = q8.f32_memref(xd.ptr, 1, 256)
    yo = q8.f32_memref(yd.ptr, 1, 64)
    rc = L._mlir_ciface_llmcp_q8_linear(ctypes.byref(xi), ctypes.byref(t.memref()),
                                        ctypes.byref(yo), 1, 1)
    assert rc == 0
    ctx.sync()
    assert bits_equal(ctx.to_host(yd, (1, 64), np.float32),
                      oracle.linear(x, p4, 64, activation="silu", epilogue=ctx.epilogue))
    L.llmcp_q8_set_default_ctx(None)
    ctx.release(t)
