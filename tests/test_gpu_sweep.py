"""A seeded random sweep of the linear entry points against the oracle, bit
for bit: shapes (N a multiple of 8, K a multiple of 32, including the
unrolled pass counts, the segmented K = 4096 / 9216 layouts and runtime pass
counts), decode (M = 1 the GEMV; M > 1 the GEMM with the scalar epilogue,
Q8Scalar.cpp:192-199) and prefill (M = 1 takes the GEMV, M > 1 the GEMM
with the default FMA epilogue, Q8Matmul.cpp:204-223), f32 and bf16 tensors,
the four activations (MatmulLoweringCommon.cpp:78-103) and the residual add
(LowerToLinalg.cpp:359-375).  Each case prints its parameters, so a failure
names it."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

K_CHOICES = [32, 64, 96, 160, 512, 1024, 1056, 1536, 2048, 2560, 2592, 4096,
             4128, 8864, 9216, 9248]
ACTS = ["none", "silu", "sigmoid", "softplus"]


def make_cases(count=120, seed=2026):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < count:
        k = int(rng.choice(K_CHOICES)) if rng.random() < 0.7 else 32 * int(rng.integers(1, 321))
        n = 8 * int(rng.integers(1, 513))
        r = rng.random()
        if r < 0.35:
            mode, m = "decode", 1
        elif r < 0.45:
            mode, m = "decode", int(rng.integers(2, 65))
        elif r < 0.55:
            mode, m = "prefill", 1
        else:
            mode, m = "prefill", int(rng.integers(2, 301))
        if m * n * k > 2e8:
            continue
        dtype = "bf16" if rng.random() < 0.4 else "f32"
        residual = rng.random() < 0.25
        act = "none" if residual else ACTS[int(rng.integers(0, 4))]
        scale = float(rng.choice([1.0, 1.0, 1e-3, 30.0]))
        cases.append((len(cases), m, n, k, mode, dtype, act, residual, scale))
    return cases


@pytest.mark.parametrize("case", make_cases(), ids=lambda c: "c%03d_m%d_n%d_k%d_%s_%s_%s%s" % (
    c[0], c[1], c[2], c[3], c[4], c[5], c[6], "_res" if c[7] else ""))
def test_random_linear_case(ctx, oracle, case):
    idx, m, n, k, mode, dtype, act, residual, scale = case
    print("sweep case", case, flush=True)
    rng = np.random.default_rng(1000 + idx)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    p4 = oracle.pack_q8_0_p4(w)
    x = (rng.standard_normal((m, k)) * scale).astype(np.float32)
    if m > 2:
        x[m // 2] = 0.0  # an all-zero row: zero scales, zero dots
    epi = ctx.epilogue
    t = ctx.upload_p4(p4, n, k)
    try:
        if dtype == "f32":
            xh, et = x, np.float32
        else:
            xh, et = oracle.f32_to_bf16_bits(x), np.uint16
            x = oracle.bf16_bits_to_f32(xh)
        xd, yd = ctx.to_device(xh), ctx.alloc(m * n * np.dtype(et).itemsize)
        lin = oracle.linear(x, p4, n, activation=act, epilogue=epi)
        if residual:
            rr = rng.standard_normal((m, n)).astype(np.float32)
            if dtype == "f32":
                rh, ref = rr, (lin + rr).astype(np.float32)
            else:
                rh = oracle.f32_to_bf16_bits(rr)
                lb = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(lin))
                ref = oracle.f32_to_bf16_bits(
                    (lb + oracle.bf16_bits_to_f32(rh)).astype(np.float32))
            rd = ctx.to_device(rh)
            ctx.linear_add(xd, t, rd, yd, m, mode=mode, dtype=dtype)
        else:
            ref = lin if dtype == "f32" else oracle.f32_to_bf16_bits(lin)
            ctx.linear(xd, t, yd, m, activation=act, mode=mode, dtype=dtype)
        y = ctx.to_host(yd, (m, n), et)
        if y.tobytes() != np.ascontiguousarray(ref).tobytes():
            bad = np.argwhere(y.view(np.uint32 if et == np.float32 else np.uint16)
                              != np.asarray(ref).view(np.uint32 if et == np.float32 else np.uint16))
            pytest.fail("case %s: %d mismatching outputs, first at %s" % (
                case, len(bad), bad[:3].tolist()))
    finally:
        ctx.release(t)
