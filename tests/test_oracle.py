"""Pins the CPU oracle (oracle/q8_oracle.c) before anything is checked against
it: the reference's own known answers (QuantizationTest.cpp, the
llmcp-matmul-benchmark self-check, run_numeric.py's exact-operand cases) plus
independent mathematics (numpy's IEEE float16, integer brute force, float64
matmul on exactly representable operands).  Each check is chosen so that a
plausible mistake -- wrong tie rule, dropped scale, transposed lane/word,
rounded scale used in the division -- fails it.
"""
import json
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def known():
    with open(os.path.join(GOLDEN, "known_answers.json")) as f:
        return json.load(f)


# ------------------------------------------------------------------ f16 ---

def test_f16_known_answer(oracle):
    # QuantizationTest.cpp:70-74 -- f16(1/127) == 0x2008 (bytes 08 20).
    ka = known()["f16_one_over_127"]
    assert int(oracle.f32_to_f16_bits(np.float32(1.0) / np.float32(127.0))[0]) == int(ka["bits"], 16)


def test_f16_rne_matches_numpy(oracle):
    rng = np.random.default_rng(7)
    mags = np.exp(rng.uniform(np.log(1e-9), np.log(1e6), 400_000)).astype(np.float32)
    signs = rng.choice([-1.0, 1.0], mags.size).astype(np.float32)
    x = mags * signs
    # Exact ties in the normal and subnormal ranges, overflow edges, specials.
    base = np.float32(1.0) + np.float32(2.0 ** -11) * np.arange(1, 64, 2, dtype=np.float32)
    ties = np.concatenate([
        base, -base, base * np.float32(2.0 ** -14), base * np.float32(2.0 ** 10),
        np.float32(2.0 ** -24) * np.arange(1, 64, dtype=np.float32) / np.float32(2.0),
        np.array([65504, 65519.99, 65520, 65536, 2.0 ** -25, 3 * 2.0 ** -26,
                  2.0 ** -14 - 2.0 ** -25, 0.0, -0.0, np.inf, -np.inf,
                  1e-30, -1e-38, 3.4e38], dtype=np.float32),
    ]).astype(np.float32)
    x = np.concatenate([x, ties])
    got = oracle.f32_to_f16_bits(x)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_f16_to_f32_exhaustive(oracle):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_bits_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


# ------------------------------------------------------------- weights ---

def test_quantize_known_answer_bf16_one(oracle):
    # QuantizationTest.cpp:57-80: a bf16 1.0 row of 64 -> scales 08 20 08 20
    # and q = 127 everywhere.
    ka = known()["bf16_one_row_64"]
    d, qs = oracle.quantize_rows_q8_0(np.ones((1, 64), np.float32))
    assert list(d.view(np.uint8).ravel()) == ka["scale_bytes"]
    assert np.all(qs == ka["q"])


def test_quantize_zero_block(oracle):
    # QuantizationTest.cpp:82-89.
    d, qs = oracle.quantize_rows_q8_0(np.zeros((1, 32), np.float32))
    assert d[0, 0] == 0 and np.all(qs == 0)


def test_quantize_round_trip_bound(oracle):
    # QuantizationTest.cpp:42-55: sin(0.1 i) * 2 over 128 values, error < 0.02.
    x = (np.sin(np.arange(128, dtype=np.float32) * np.float32(0.1)) * np.float32(2.0)).astype(np.float32)
    d, qs = oracle.quantize_rows_q8_0(x[None, :])
    deq = oracle.f16_bits_to_f32(d).repeat(32, axis=1) * qs.astype(np.float32)
    assert np.max(np.abs(deq - x)) < 0.02


def test_weight_quant_rounds_half_away_from_zero(oracle):
    # amax = 127 makes scale exactly 1.0, so x/scale == x: halves must go
    # away from zero (std::lround, Quantization.cpp:111), not to even.
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:9] = [2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5, -126.5]
    d, qs = oracle.quantize_rows_q8_0(x[None, :])
    assert d[0, 0] == 0x3C00
    assert list(qs[0, 1:9]) == [3, -3, 1, -1, 2, -2, 127, -127]


def test_weight_quant_divides_by_unrounded_scale(oracle):
    # Quantization.cpp:109-112 divides by the f32 scale amax/127, not by the
    # f16-rounded d.  Find values whose rounding differs between the two.
    amax = np.float32(100.0)
    s32 = amax / np.float32(127.0)
    d16 = np.float32(np.float16(s32))
    assert s32 != d16
    cand = (np.arange(1, 2000, dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    cand = cand[cand < amax]

    def lround(v):
        return np.sign(v) * np.floor(np.abs(v.astype(np.float64)) + 0.5)

    q_true = lround((cand / s32).astype(np.float32))
    q_rounded_scale = lround((cand / d16).astype(np.float32))
    pick = cand[q_true != q_rounded_scale][:31]
    assert pick.size == 31
    x = np.concatenate([[amax], pick]).astype(np.float32)
    _, qs = oracle.quantize_rows_q8_0(x[None, :])
    assert np.array_equal(qs[0, 1:].astype(np.float64), lround((pick / s32).astype(np.float32)))


# --------------------------------------------------------------- layout ---

def exact_int_rows(rng, rows, cols):
    """Rows whose Q8_0 quantization is exact: amax 127 -> scale 1.0."""
    q = rng.integers(-127, 128, size=(rows, cols)).astype(np.float32)
    q[:, ::32] = 127.0
    return q


def test_p4_byte_addresses(oracle):
    # Appendix-A address function, from Q8Scalar.cpp:137-182 and
    # Quantization.cpp:193-210, checked byte by byte.
    rng = np.random.default_rng(1)
    n, k = 16, 96
    w = exact_int_rows(rng, n, k)
    p4 = oracle.pack_q8_0_p4(w)
    assert p4.size == n * (k + k // 32 * 2)
    blocks = k // 32
    for r in range(n):
        g, lane = divmod(r, 4)
        for b in range(blocks):
            rec = (g * blocks + b) * 136
            assert p4[rec + 2 * lane] == 0x00 and p4[rec + 2 * lane + 1] == 0x3C
            for e in range(32):
                off = rec + 8 + (e // 4) * 16 + lane * 4 + (e % 4)
                assert np.int8(p4[off].astype(np.int8)) == int(w[r, 32 * b + e])


def test_p4_matches_reshape_restatement(oracle):
    # An array-reshape restatement of the record: [4 x f16][8 words x 4 lanes x 4 B].
    rng = np.random.default_rng(2)
    n, k = 24, 128
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    p4 = oracle.pack_q8_0_p4(w)
    d, qs = oracle.quantize_rows_q8_0(w)
    blocks = k // 32
    recs = []
    for g in range(n // 4):
        for b in range(blocks):
            scales = d[4 * g:4 * g + 4, b].astype("<u2").view(np.uint8)
            words = qs[4 * g:4 * g + 4, 32 * b:32 * b + 32].reshape(4, 8, 4).transpose(1, 0, 2)
            recs.append(np.concatenate([scales, words.reshape(-1).view(np.uint8)]))
    assert np.array_equal(p4, np.concatenate(recs))
    q2, d2 = oracle.unpack_q8_0_p4(p4, n, k)
    assert np.array_equal(q2, qs) and np.array_equal(d2, d)


def test_pack_rejects_unpackable_shapes(oracle):
    with pytest.raises(ValueError):
        oracle.pack_q8_0_p4(np.zeros((4, 64), np.float32))  # rows % 8
    with pytest.raises(ValueError):
        oracle.pack_q8_0_p4(np.zeros((8, 48), np.float32))  # cols % 32


def test_all_ones_known_answer(oracle):
    # llmcp-matmul-benchmark.cpp:280-289, :331-335: every record holds scales
    # 0x2008 and q = 127; all-ones activations give first == K (bf16 print).
    ka = known()["matmul_benchmark_all_ones"]
    for k in ka["k_values"]:
        n = 16
        rec = np.array([0x08, 0x20] * 4 + [0x7F] * 128, np.uint8)
        p4 = np.tile(rec, n // 4 * (k // 32))
        y = oracle.linear(np.ones((1, k), np.float32), p4, n)
        # bf16 of the output is K exactly, as the reference checks
        bf16 = (y.view(np.uint32) + 0x7FFF + ((y.view(np.uint32) >> 16) & 1)) >> 16
        assert np.all((bf16 << 16).view(np.float32) == np.float32(k))
        # and the f32 value is the closed form: sum of K/32 equal terms
        sa = np.float32(1.0) / np.float32(127.0)
        term = np.float32(32 * 127 * 127) * (sa * np.float32(np.uint16(0x2008).view(np.float16)))
        acc = np.float32(0.0)
        for _ in range(k // 32):
            acc = np.float32(acc + term)
        assert np.all(y == acc)


# ---------------------------------------------------------- activations ---

def test_activation_quant_roundeven_ties(oracle):
    # Q8Decode.cpp:116 uses math.roundeven: with max 127 the scale is 1 and
    # halves go to even (unlike the weight quantizer).
    x = np.zeros((1, 32), np.float32)
    x[0, 0] = 127.0
    x[0, 1:8] = [2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 126.5]
    qa, sa = oracle.quantize_act_q8_1(x)
    assert sa[0, 0] == np.float32(127.0) / np.float32(127.0)
    assert list(qa[0, 1:8]) == [2, 4, -2, -4, 0, 0, 126]


def test_activation_quant_zero_block_and_scale(oracle):
    # run_numeric.py:721,728: a zero activation block -> sa = 0, q = 0.
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 96)).astype(np.float32)
    x[1, 32:64] = 0.0
    qa, sa = oracle.quantize_act_q8_1(x)
    assert sa[1, 1] == 0.0 and np.all(qa[1, 32:64] == 0)
    # sa is the unrounded f32 maxAbs / 127 (not an f16)
    m = np.abs(x.reshape(3, 3, 32)).max(-1)
    assert np.array_equal(sa, (m / np.float32(127.0)).astype(np.float32))
    # every block hits +-127 at its maximum element
    assert np.all(np.abs(qa.reshape(3, 3, 32)).max(-1)[sa > 0] == 127)


# ------------------------------------------------------------ dot, epilogue

def test_block_dots_brute_force(oracle):
    rng = np.random.default_rng(4)
    m, n, k = 3, 16, 160
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    p4 = oracle.pack_q8_0_p4(w)
    qa, _ = oracle.quantize_act_q8_1(x)
    _, qw = oracle.quantize_rows_q8_0(w)
    want = np.einsum("mbi,nbi->mnb", qa.reshape(m, -1, 32).astype(np.int64),
                     qw.reshape(n, -1, 32).astype(np.int64))
    assert np.array_equal(oracle.block_dots(qa, p4, n), want)


def exact_operand(rng, rows, k):
    """run_numeric.py:695-699: integers in [-63,63], element 0 of each block
    127, each block scaled by 2^e with e in {-6,-5} -> exact quantization."""
    blocks = k // 32
    v = rng.integers(-63, 64, size=(rows, blocks, 32)).astype(np.float64)
    v[:, :, 0] = 127
    e = rng.integers(-6, -4, size=(rows, blocks, 1))
    return np.ldexp(v, e).reshape(rows, k).astype(np.float32)


@pytest.mark.parametrize("m", [1, 19])
@pytest.mark.parametrize("epi", ["scalar", "fma"])
def test_exact_operand_linear(oracle, m, epi):
    # run_numeric.py:690-732: M=19 (and the M=1 decode case), N=136, K=288,
    # zero last block of row 0, rel 1e-5 / abs 1e-6 against an f32 matmul.
    rng = np.random.default_rng(5)
    n, k = 136, 288
    x = exact_operand(rng, m, k)
    w = exact_operand(rng, n, k)
    x[0, -32:] = 0
    y = oracle.linear(x, oracle.pack_q8_0_p4(w), n, epilogue=epi)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-6)


def test_scalar_and_fma_epilogues_agree(oracle):
    rng = np.random.default_rng(6)
    x = rng.standard_normal((2, 2560)).astype(np.float32)
    w = (rng.standard_normal((64, 2560)) * 0.02).astype(np.float32)
    p4 = oracle.pack_q8_0_p4(w)
    a = oracle.linear(x, p4, 64, epilogue="scalar")
    b = oracle.linear(x, p4, 64, epilogue="fma")
    np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-4)
    # and both track the float64 product of the dequantized operands
    qa, sa = oracle.quantize_act_q8_1(x)
    d, qw = oracle.quantize_rows_q8_0(w)
    xd = qa.reshape(2, -1, 32) * sa[:, :, None].astype(np.float64)
    wd = qw.reshape(64, -1, 32) * oracle.f16_bits_to_f32(d)[:, :, None].astype(np.float64)
    ref = np.einsum("mbi,nbi->mn", xd, wd)
    np.testing.assert_allclose(a, ref, rtol=1e-5, atol=1e-4)


def test_silu_against_float64(oracle):
    v = np.linspace(-30, 30, 4001).astype(np.float32)
    got = oracle.silu(v).astype(np.float64)
    vd = v.astype(np.float64)
    ref = vd / (1.0 + np.exp(-vd))
    np.testing.assert_allclose(got, ref, rtol=2e-7, atol=1e-30)


def test_linear_silu_applies_activation(oracle):
    rng = np.random.default_rng(8)
    x = rng.standard_normal((1, 256)).astype(np.float32)
    w = (rng.standard_normal((16, 256)) * 0.05).astype(np.float32)
    p4 = oracle.pack_q8_0_p4(w)
    plain = oracle.linear(x, p4, 16)
    act = oracle.linear(x, p4, 16, activation="silu")
    assert np.array_equal(act, oracle.silu(plain))


def test_swiglu_composition(oracle):
    rng = np.random.default_rng(9)
    x = rng.standard_normal((1, 256)).astype(np.float32)
    wg = oracle.pack_q8_0_p4((rng.standard_normal((32, 256)) * 0.05).astype(np.float32))
    wu = oracle.pack_q8_0_p4((rng.standard_normal((32, 256)) * 0.05).astype(np.float32))
    h = oracle.swiglu(x, wg, wu, 32)
    g = oracle.linear(x, wg, 32, activation="silu")
    u = oracle.linear(x, wu, 32)
    assert np.array_equal(h, (g * u).astype(np.float32))


def test_argmax_first_maximum(oracle):
    v = np.array([1.0, 3.0, -2.0, 3.0, 3.0], np.float32)
    assert oracle.argmax(v) == 1  # std::max_element keeps the first maximum
    rng = np.random.default_rng(10)
    for _ in range(20):
        v = rng.integers(0, 5, 100).astype(np.float32)
        assert oracle.argmax(v) == int(np.argmax(v))


def test_embedding_exact(oracle):
    rng = np.random.default_rng(11)
    n, k = 32, 128
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    p4 = oracle.pack_q8_0_p4(w)
    d, qs = oracle.quantize_rows_q8_0(w)
    tokens = np.array([5, 0, 31, 5, 17], np.int64)
    out = oracle.embedding(tokens, p4, k)
    deq = qs.astype(np.float32) * d.view(np.float16).astype(np.float32).repeat(32, axis=1)
    assert np.array_equal(out, deq[tokens])


def test_column_parallel_variant_is_bit_identical(oracle):
    rng = np.random.default_rng(12)
    x = rng.standard_normal((1, 1024)).astype(np.float32)
    p4 = oracle.pack_q8_0_p4((rng.standard_normal((256, 1024)) * 0.02).astype(np.float32))
    a = oracle.linear(x, p4, 256)
    oracle.set_threads(4)
    b = oracle.linear(x, p4, 256, colpar=True)
    oracle.set_threads(1)
    c = oracle.linear(x, p4, 256, colpar=True)
    assert np.array_equal(a, b) and np.array_equal(a, c)


def test_golden_small_case_regression(oracle):
    # Fixture written by tests/golden/make_golden.py from this oracle; keeps the
    # oracle's outputs fixed across changes and feeds the GPU parity tests.
    z = np.load(os.path.join(GOLDEN, "q8_small_case.npz"))
    assert np.array_equal(oracle.pack_q8_0_p4(z["w"]), z["p4"])
    qa, sa = oracle.quantize_act_q8_1(z["x"])
    assert np.array_equal(qa, z["qa"]) and np.array_equal(sa, z["sa"])
    n = z["w"].shape[0]
    assert np.array_equal(oracle.linear(z["x"], z["p4"], n), z["y_scalar"])
    assert np.array_equal(oracle.linear(z["x"], z["p4"], n, epilogue="fma"), z["y_fma"])


def test_f32_to_bf16_matches_torch(oracle):
    # arith.truncf f32 -> bf16 is round to nearest, ties to even; torch's
    # float32 -> bfloat16 conversion is the independent restatement.
    import torch
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    # exact ties (low 16 bits 0x8000) with even and odd kept parts
    ties = (rng.integers(0, 2**16, 20000, dtype=np.uint32) << 16) | 0x8000
    special = np.array([0x00000000, 0x80000000, 0x7f800000, 0xff800000,
                        0x00000001, 0x007fffff, 0x3f808000, 0x3f818000,
                        0x7f7fffff, 0x7f7f8000, 0x3f7fffff], np.uint32)
    allb = np.concatenate([bits, ties, special])
    x = allb.view(np.float32)
    finite = np.isfinite(x) | np.isinf(x)
    got = oracle.f32_to_bf16_bits(x[finite])
    ref = torch.from_numpy(x[finite].copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)
    # NaN stays NaN (quiet)
    nan = oracle.f32_to_bf16_bits(np.array([np.nan], np.float32))[0]
    assert (nan & 0x7f80) == 0x7f80 and (nan & 0x007f) != 0


def test_activations_closed_form(oracle):
    # applyMatmulActivation (MatmulLoweringCommon.cpp:78-103) against float64
    # closed forms; f32 intermediate roundings keep them within a few ulp.
    v = np.concatenate([np.linspace(-30, 30, 6001), [-1e-3, 1e-3, 0.0]]).astype(np.float32)
    d = v.astype(np.float64)
    sig = oracle.sigmoid(v)
    assert np.allclose(sig, 1.0 / (1.0 + np.exp(-d)), rtol=4e-7, atol=1e-30)
    silu = oracle.silu(v)
    assert np.array_equal(silu, (v * sig).astype(np.float32))  # v * sigmoid(v)
    # softplus = math.log1p(math.exp(v)) as the reference compiles it:
    # --convert-math-to-llvm (llmcp-compile.cpp:186) lowers log1p(y) to
    # log(1 + y) with an f32 add.  Closed form: f64 log of the f32 sum.
    sp = oracle.softplus(v)
    e32 = np.exp(d).astype(np.float32)
    s32 = (np.float32(1.0) + e32).astype(np.float32)
    assert np.allclose(sp, np.log(s32.astype(np.float64)), rtol=4e-7, atol=1e-30)
    # where exp(v) < 2^-24 the f32 sum rounds to 1 and the result is 0 (a
    # true log1p would return exp(v)); between, the sum keeps only the
    # leading bits of exp(v)
    tail = oracle.softplus(np.array([-20.0, -17.5, -16.0], np.float32))
    assert tail[0] == 0.0 and tail[1] == 0.0
    assert tail[2] == np.float32(np.log(np.float64(np.float32(1.0) + np.float32(np.exp(-16.0)))))
    assert tail[2] != np.float32(np.log1p(np.exp(-16.0)))
    # softplus overflows where f32 exp does (exp(89) = inf)
    assert np.isinf(oracle.softplus(np.array([89.0], np.float32))[0])
    assert oracle.softplus(np.array([88.0], np.float32))[0] == np.float32(
        np.log(np.float64(np.float32(1.0) + np.float32(np.exp(88.0)))))


# ------------------------------------------------------------- RMSNorm --
# DecodeNormalization.cpp:93-154 / LowerToLinalg.cpp:245-300: the serial sum
# is pinned by numpy's sequential float32 cumsum (its last partial sum), a
# different implementation of the same left-to-right fold.

def _serial_rstd(x, eps):
    s = np.cumsum((x * x).astype(np.float32), dtype=np.float32)[-1]
    mean = np.float32(s) / np.float32(x.size)
    var = np.float32(mean) + np.float32(eps)
    return np.float32(1.0) / np.sqrt(np.float32(var))


@pytest.mark.parametrize("h", [32, 128, 2560])
def test_rmsnorm_sum_is_the_serial_fold(oracle, h):
    rng = np.random.default_rng(h)
    x = (rng.standard_normal((5, h)) * np.array([[1], [1e-3], [30], [1], [1]])).astype(np.float32)
    x[3] = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(x[3]))
    w = rng.standard_normal(h).astype(np.float32)
    y, r = oracle.rmsnorm(x, w, 1e-6, with_rstd=True)
    for i in range(x.shape[0]):
        assert r[i].view(np.uint32) == _serial_rstd(x[i], 1e-6).view(np.uint32), i


def test_rmsnorm_order_changes_the_result(oracle):
    # 1 followed by 4095 squares of 2^-12 (each half an ulp of 1.0): the
    # serial sum stays 1.0 (ties to even); a float64 or pairwise sum does not
    x = np.full(4096, 2.0 ** -12, np.float32)
    x[0] = 1.0
    w = np.ones(4096, np.float32)
    _, r = oracle.rmsnorm(x, w, 0.0, with_rstd=True)
    assert r[0] == np.float32(1.0) / np.sqrt(np.float32(1.0 / 4096))
    s64 = float(np.sum(x.astype(np.float64) ** 2))
    assert np.float32(1.0 / np.sqrt(s64 / 4096)) != r[0]
    assert np.float32(1.0) / np.sqrt(np.float32(np.sum(x * x) / 4096)) != r[0]


def test_rmsnorm_constant_row_closed_form(oracle):
    for c in (0.75, -3.0, 2.0 ** -10):  # squares and their sums exact in f32
        x = np.full((1, 256), c, np.float32)
        w = np.linspace(-2, 2, 256).astype(np.float32)
        eps = 1e-6
        y = oracle.rmsnorm(x, w, eps)[0]
        exact = c / np.sqrt(c * c + eps) * w.astype(np.float64)
        assert np.all(np.abs(y - exact) <= 4 * np.spacing(np.abs(exact).astype(np.float32)) + 1e-30)
        # zero-centered: w + 1
        y1 = oracle.rmsnorm(x, w, eps, zero_centered=True)[0]
        exact1 = c / np.sqrt(c * c + eps) * (w.astype(np.float64) + 1.0)
        assert np.all(np.abs(y1 - exact1) <= 4 * np.spacing(np.abs(exact1).astype(np.float32)) + 1e-30)


def test_rmsnorm_reference_numeric_case(oracle):
    # run_numeric.py:734-749: bf16 x [2, 8], bf16 w, eps 1e-6, bf16 out
    # within (2e-2, 1e-2) of the torch formula, zero-centered and not
    torch = pytest.importorskip("torch")
    torch.manual_seed(0)
    x = torch.randn(2, 8).to(torch.bfloat16)
    w = torch.randn(8).to(torch.bfloat16)
    xf = x.float()
    rstd = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
    xb = x.view(torch.int16).numpy().view(np.uint16)
    wb = w.view(torch.int16).numpy().view(np.uint16)
    for zc, wf in ((True, 1.0 + w.float()), (False, w.float())):
        ref = (xf * rstd * wf).to(torch.bfloat16).float().numpy()
        got = oracle.bf16_bits_to_f32(oracle.rmsnorm(xb, wb, 1e-6, zero_centered=zc,
                                                    out_bf16=True))
        np.testing.assert_allclose(got, ref, rtol=2e-2, atol=1e-2)


def test_gated_rmsnorm_pins(oracle):
    rng = np.random.default_rng(3)
    m, groups, g = 3, 4, 128
    x = rng.standard_normal((m, groups * g)).astype(np.float32)
    z = (rng.standard_normal((m, groups * g)) * 2).astype(np.float32)
    w = (rng.standard_normal(g) * 0.1 + 1).astype(np.float32)
    # an all-ones activated gate reduces to the plain norm of the reshaped
    # rows, whose ((x*1)*w)*rstd differs from (x*rstd)*w only in rounding
    ones = np.ones_like(x)
    yg = oracle.gated_rmsnorm(x, ones, w, g, 1e-6, gate_activated=True)
    _, r = oracle.rmsnorm(x.reshape(-1, g), w, 1e-6, with_rstd=True)
    assert np.array_equal(r, np.array([_serial_rstd(row, 1e-6) for row in x.reshape(-1, g)]))
    expect = ((x.reshape(-1, g) * w) * r[:, None]).reshape(m, -1)
    assert np.array_equal(yg.view(np.uint32), expect.astype(np.float32).view(np.uint32))
    # the gate enters through the oracle's silu (float64 closed form within ulps)
    y = oracle.gated_rmsnorm(x, z, w, g, 1e-6)
    s64 = z.astype(np.float64) / (1 + np.exp(-z.astype(np.float64)))
    ref = (x * s64).reshape(-1, g) * w * r[:, None]
    np.testing.assert_allclose(y, ref.reshape(m, -1), rtol=3e-6, atol=1e-30)
