"""Seeded random sweeps of the other entry points against the oracle, bit for
bit: the fused SwiGLU (FuseSiluMul, ModelBuilder.cpp:205-216) in decode and
prefill, f32 and bf16; the tied lm_head (LowerToLinalg.cpp:729-765) with the
first-maximum argmax of its last row (llmcp-benchmark.cpp:51-54), where a
duplicated weight row plants an exact tie ahead of the maximum; and the
embedding gather (LowerToLinalg.cpp:435-531) on random ids.  Each case prints
its parameters."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

K_CHOICES = [32, 96, 512, 1056, 2560, 4096, 4128, 9216]


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32 if a.dtype == np.float32 else np.uint16)


def swiglu_cases(count=40, seed=77):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        k = int(rng.choice(K_CHOICES))
        n = 8 * int(rng.integers(1, 400))
        r = rng.random()
        mode, m = (("decode", 1) if r < 0.4 else ("decode", int(rng.integers(2, 40))) if r < 0.5
                   else ("prefill", int(rng.integers(1, 200))))
        if m * n * k * 2 > 2e8:
            continue
        out.append((len(out), m, n, k, mode, "bf16" if rng.random() < 0.4 else "f32"))
    return out


@pytest.mark.parametrize("case", swiglu_cases(), ids=lambda c: "s%02d_m%d_n%d_k%d_%s_%s" % c)
def test_random_swiglu_case(ctx, oracle, case):
    idx, m, n, k, mode, dtype = case
    print("swiglu case", case, flush=True)
    rng = np.random.default_rng(5000 + idx)
    pg = oracle.pack_q8_0_p4((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    pu = oracle.pack_q8_0_p4((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = rng.standard_normal((m, k)).astype(np.float32)
    epi = ctx.epilogue
    tg, tu = ctx.upload_p4(pg, n, k), ctx.upload_p4(pu, n, k)
    try:
        if dtype == "f32":
            ref, xh, et = oracle.swiglu(x, pg, pu, n, epilogue=epi), x, np.float32
        else:
            xh, et = oracle.f32_to_bf16_bits(x), np.uint16
            xf = oracle.bf16_bits_to_f32(xh)
            g = oracle.f32_to_bf16_bits(oracle.linear(xf, pg, n, activation="silu", epilogue=epi))
            u = oracle.f32_to_bf16_bits(oracle.linear(xf, pu, n, epilogue=epi))
            ref = oracle.f32_to_bf16_bits(
                (oracle.bf16_bits_to_f32(g) * oracle.bf16_bits_to_f32(u)).astype(np.float32))
        xd, hd = ctx.to_device(xh), ctx.alloc(m * n * np.dtype(et).itemsize)
        ctx.swiglu(xd, tg, tu, hd, m, mode=mode, dtype=dtype)
        h = ctx.to_host(hd, (m, n), et)
        assert np.array_equal(bits(h), bits(ref)), (case, int(np.sum(bits(h) != bits(ref))))
    finally:
        ctx.release(tg)
        ctx.release(tu)


def lm_cases(count=24, seed=78):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        k = int(rng.choice([512, 1056, 2560, 4096]))
        v = 8 * int(rng.integers(16, 6000))
        r = rng.random()
        mode, m = (("decode", 1) if r < 0.5 else ("decode", int(rng.integers(2, 12))) if r < 0.6
                   else ("prefill", int(rng.integers(1, 40))))
        if m * v * k > 2.5e8:
            continue
        out.append((len(out), m, v, k, mode, "bf16" if rng.random() < 0.4 else "f32",
                    bool(rng.random() < 0.5)))
    return out


@pytest.mark.parametrize("case", lm_cases(), ids=lambda c: "l%02d_m%d_v%d_k%d_%s_%s_tie%d" % c)
def test_random_lm_head_case(ctx, oracle, case):
    idx, m, v, k, mode, dtype, tie = case
    print("lm_head case", case, flush=True)
    rng = np.random.default_rng(6000 + idx)
    w = (rng.standard_normal((v, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    xh = x if dtype == "f32" else oracle.f32_to_bf16_bits(x)
    xf = x if dtype == "f32" else oracle.bf16_bits_to_f32(xh)
    epi = ctx.epilogue
    if tie:
        # copy the winning row to an earlier index: both logits are then
        # bit-identical and the first maximum is the copy
        j = int(oracle.argmax(oracle.linear(xf[-1:], oracle.pack_q8_0_p4(w), v, epilogue=epi)[0]))
        if j > 0:
            w[int(rng.integers(0, j))] = w[j]
    p4 = oracle.pack_q8_0_p4(w)
    ref = oracle.linear(xf, p4, v, epilogue=epi)
    t = ctx.upload_p4(p4, v, k)
    try:
        xd, ld, am = ctx.to_device(xh), ctx.alloc(m * v * 4), ctx.alloc(8)
        ctx.lm_head(xd, t, ld, m, argmax=am, mode=mode, dtype=dtype)
        logits = ctx.to_host(ld, (m, v), np.float32)
        assert np.array_equal(bits(logits), bits(ref)), case
        assert int(ctx.to_host(am, (1,), np.int64)[0]) == oracle.argmax(ref[-1]), case
    finally:
        ctx.release(t)


def embedding_cases(count=16, seed=79):
    rng = np.random.default_rng(seed)
    return [(i, 8 * int(rng.integers(1, 4000)), int(rng.choice(K_CHOICES)),
             int(rng.integers(1, 2000)), "bf16" if rng.random() < 0.4 else "f32")
            for i in range(count)]


@pytest.mark.parametrize("case", embedding_cases(), ids=lambda c: "e%02d_v%d_k%d_n%d_%s" % c)
def test_random_embedding_case(ctx, oracle, case):
    idx, v, k, count, dtype = case
    print("embedding case", case, flush=True)
    rng = np.random.default_rng(7000 + idx)
    p4 = oracle.pack_q8_0_p4((rng.standard_normal((v, k)) * 0.02).astype(np.float32))
    tokens = rng.integers(0, v, count).astype(np.int64)
    ref = oracle.embedding(tokens, p4, k)
    et = np.float32 if dtype == "f32" else np.uint16
    if dtype == "bf16":
        ref = oracle.f32_to_bf16_bits(ref)
    t = ctx.upload_p4(p4, v, k)
    try:
        td, od = ctx.to_device(tokens), ctx.alloc(count * k * np.dtype(et).itemsize)
        ctx.embedding(td, count, t, od, dtype=dtype)
        assert np.array_equal(bits(ctx.to_host(od, (count, k), et)), bits(ref)), case
        assert ctx.check_flag() == 0
    finally:
        ctx.release(t)


def test_lm_head_several_rows(ctx, oracle, q8):
    # M = 8: every row's logits from the GEMM with the platform's epilogue,
    # the argmax of the last row reduced from HBM, with a planted tie; in
    # prefill and in decode mode (the same arithmetic on one platform)
    rng = np.random.default_rng(8100)
    m, v, k = 8, 40000, 1024
    w = (rng.standard_normal((v, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    j = int(oracle.argmax(oracle.linear(x[-1:], oracle.pack_q8_0_p4(w), v, epilogue=ctx.epilogue)[0]))
    w[j // 2] = w[j]
    p4 = oracle.pack_q8_0_p4(w)
    ref = oracle.linear(x, p4, v, epilogue=ctx.epilogue)
    assert oracle.argmax(ref[-1]) == j // 2 or j == 0
    t = ctx.upload_p4(p4, v, k)
    try:
        xd, ld, am = ctx.to_device(x), ctx.alloc(m * v * 4), ctx.alloc(8)
        for mode in ("prefill", "prefill", "decode"):  # slots clear after each call
            ctx.lm_head(xd, t, ld, m, argmax=am, mode=mode)
            assert np.array_equal(bits(ctx.to_host(ld, (m, v), np.float32)), bits(ref))
            assert int(ctx.to_host(am, (1,), np.int64)[0]) == oracle.argmax(ref[-1])
    finally:
        ctx.release(t)


def test_embedding_many_tokens(ctx, oracle):
    # more ids than a 16-bit grid dimension would hold, f32 and bf16 rows
    rng = np.random.default_rng(8200)
    v, k, count = 512, 64, 70000
    p4 = oracle.pack_q8_0_p4((rng.standard_normal((v, k)) * 0.02).astype(np.float32))
    tokens = rng.integers(0, v, count).astype(np.int64)
    ref = oracle.embedding(tokens, p4, k)
    t = ctx.upload_p4(p4, v, k)
    try:
        td = ctx.to_device(tokens)
        od = ctx.alloc(count * k * 4)
        ctx.embedding(td, count, t, od)
        assert np.array_equal(bits(ctx.to_host(od, (count, k), np.float32)), bits(ref))
        ctx.embedding(td, count, t, od, dtype="bf16")
        assert np.array_equal(bits(ctx.to_host(od, (count, k), np.uint16)),
                              bits(oracle.f32_to_bf16_bits(ref)))
        assert ctx.check_flag() == 0
    finally:
        ctx.release(t)
