/*
 * q8_oracle.c -- CPU restatement of llmcp's Q8_0 quantized linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker, never the product:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.  The HIP library in llmcp_amd/ never links or calls it.
 *
 * Every function restates one piece of the reference (paths relative to the
 * reference repository root) in plain C99 with no LLVM dependency.  Build with
 * -ffp-contract=off so the scalar epilogue stays an unfused multiply + add,
 * exactly as the reference's x86 path computes it.
 *
 * How each function is pinned (see tests/test_oracle.py):
 *   f32_to_f16          numpy float16 conversion over >1M inputs incl. ties,
 *                       subnormals, overflow; known answer f16(1/127)=0x2008
 *                       (QuantizationTest.cpp:70-74).
 *   quantize_row_q8_0   known answers of QuantizationTest.cpp:57-89 (bf16 1.0
 *                       -> 08 20 / q=127, zero block) and its round-trip bound
 *                       (:42-55); constructed ties that separate lround from
 *                       roundeven, and division by the unrounded f32 scale.
 *   pack_q8_0_p4        hand-computed byte addresses from the scalar address
 *                       function (Q8Scalar.cpp:137-182) and an array-reshape
 *                       restatement; all-ones known answer output == K
 *                       (llmcp-matmul-benchmark.cpp:280-289, :331-335).
 *   quantize_act_q8_1   constructed roundeven ties, zero block (sa=0, q=0).
 *   block_dots          brute-force int64 einsum.
 *   linear_*            exact-operand construction of run_numeric.py:690-732
 *                       against an float64 matmul at rel 1e-5 / abs 1e-6.
 *   silu/sigmoid/       float64 closed forms within ulp-level tolerance;
 *   softplus            softplus against log(f32(1 + f32(exp v))), the
 *                       lowered log1p, which is 0 where exp(v) < 2^-24 (a
 *                       true log1p there is not), and at the overflow end.
 *   f32_to_bf16         torch's float32 -> bfloat16 conversion (round to
 *                       nearest even) on ties, subnormals, inf and NaN.
 *   argmax              numpy argmax (first maximum), std::max_element rule.
 *   embedding           exact dequantization from the unpacked matrix.
 *   rmsnorm             the serial sum against numpy's sequential float32
 *                       cumsum (the last partial sum), rstd against float32
 *                       1/np.sqrt, constructed rows whose pairwise or float64
 *                       sum differs from the serial one, and the closed form
 *                       of a constant row (y = w * sign(x) within 4 ulp).
 *   gated_rmsnorm       the per-group sums against the plain rmsnorm of the
 *                       reshaped rows, the gate against oracle_silu, and an
 *                       all-ones gate row (activated) against rmsnorm.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK 32            /* kQ8PackedBlockSize, Q8PackedLayout.h:21 */
#define LANES 4          /* kQ8PackedLanes, Q8PackedLayout.h:18 */
#define CHUNK 16         /* kQ8PackedChunkBytes, Q8PackedLayout.h:24 */
#define SCALE_BYTES 8    /* kQ8PackedScaleBytes, Q8PackedLayout.h:27 */
#define RECORD 136       /* kQ8PackedBlockBytes, Q8PackedLayout.h:34 */

/* ------------------------------------------------------------------ f16 -- */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* IEEE-754 binary32 -> binary16, round to nearest, ties to even.
 * Restates floatToHalf (lib/Model/Quantization.cpp:32-37), which uses
 * APFloat::convert(IEEEhalf, rmNearestTiesToEven). */
uint16_t oracle_f32_to_f16(float value) {
  uint32_t x = f2u(value);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xffu) /* inf / nan (quiet) */
    return (uint16_t)(sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0u));
  int32_t e = (int32_t)exp - 127 + 15;
  if (e >= 31)
    return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) { /* f16 subnormal or zero: value = full * 2^(exp-150) */
    if (exp == 0)
      return (uint16_t)sign; /* f32 zero/subnormal is far below f16 range */
    uint32_t full = man | 0x800000u;
    int shift = 14 - e; /* f16 subnormal unit is 2^-24 */
    if (shift > 24)
      return (uint16_t)sign;
    uint32_t m = full >> shift;
    uint32_t rem = full & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (m & 1u)))
      m += 1u; /* may carry into the smallest normal: still correct */
    return (uint16_t)(sign | m);
  }
  uint32_t h = ((uint32_t)e << 10) | (man >> 13);
  uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u)))
    h += 1u; /* carry may overflow into infinity, as RNE requires */
  return (uint16_t)(sign | h);
}

void oracle_f32_to_f16_batch(const float *x, int64_t n, uint16_t *out) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_f32_to_f16(x[i]);
}

/* Exact binary16 -> binary32 (halfToFloat, Quantization.cpp:39-44). */
float oracle_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
  uint32_t man = (uint32_t)h & 0x3ffu;
  if (exp == 0x1fu)
    return u2f(sign | 0x7f800000u | (man << 13));
  if (exp == 0) {
    if (man == 0)
      return u2f(sign);
    float v = (float)man * (1.0f / 16777216.0f); /* man * 2^-24, exact */
    return sign ? -v : v;
  }
  return u2f(sign | ((exp - 15 + 127) << 23) | (man << 13));
}

void oracle_f16_to_f32_batch(const uint16_t *h, int64_t n, float *out) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_f16_to_f32(h[i]);
}

/* bf16 -> f32 widening (bf16ToFloat, Quantization.cpp:25-30). */
float oracle_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* f32 -> bf16 round-to-nearest-even (arith.truncf on the bf16 output path,
 * Q8Scalar.cpp:204-206).  NaN kept quiet. */
uint16_t oracle_f32_to_bf16(float value) {
  uint32_t x = f2u(value);
  if ((x & 0x7fffffffu) > 0x7f800000u)
    return (uint16_t)((x >> 16) | 0x40u);
  uint32_t rounding = 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)((x + rounding) >> 16);
}

void oracle_f32_to_bf16_batch(const float *x, int64_t n, uint16_t *out) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_f32_to_bf16(x[i]);
}

/* ------------------------------------------------------- weight Q8_0 ---- */

/* quantizeRowQ8_0 (lib/Model/Quantization.cpp:92-116), one row of k values:
 * amax = max|x|; amax==0 -> d=0,q=0; else scale = amax/127 (f32),
 * d = f16(scale), q = clamp(lround(x/scale), -127, 127) -- the division uses
 * the unrounded f32 scale and lround rounds halves away from zero. */
void oracle_quantize_row_q8_0(const float *x, int64_t k, uint16_t *d,
                              int8_t *qs) {
  for (int64_t b = 0; b < k / QK; ++b) {
    const float *v = x + b * QK;
    float amax = 0.0f;
    for (int i = 0; i < QK; ++i) {
      float a = fabsf(v[i]);
      amax = amax < a ? a : amax; /* std::max(amax, fabs) */
    }
    if (amax == 0.0f) {
      d[b] = 0;
      memset(qs + b * QK, 0, QK);
      continue;
    }
    float scale = amax / 127.0f;
    d[b] = oracle_f32_to_f16(scale);
    for (int i = 0; i < QK; ++i) {
      long q = lroundf(v[i] / scale);
      if (q < -127) q = -127;
      if (q > 127) q = 127;
      qs[b * QK + i] = (int8_t)q;
    }
  }
}

/* dequantizeQ8_0 (Quantization.cpp:156-163): x = f32(d) * q. */
void oracle_dequantize_row_q8_0(const uint16_t *d, const int8_t *qs, int64_t k,
                                float *out) {
  for (int64_t b = 0; b < k / QK; ++b) {
    float s = oracle_f16_to_f32(d[b]);
    for (int i = 0; i < QK; ++i)
      out[b * QK + i] = s * (float)qs[b * QK + i];
  }
}

/* Byte offset of element (n, k) and of scale (n, block) in the four-column
 * lane layout (Q8Scalar.cpp:137-182, LowerToLinalg.cpp:466-514). */
int64_t oracle_p4_qs_offset(int64_t n, int64_t k, int64_t cols) {
  int64_t blocks = cols / QK;
  int64_t group = n / LANES, lane = n % LANES;
  int64_t block = k / QK, w = k % QK;
  int64_t record = (group * blocks + block) * RECORD;
  return record + SCALE_BYTES + (w / 4) * CHUNK + lane * 4 + (w % 4);
}

int64_t oracle_p4_scale_offset(int64_t n, int64_t block, int64_t cols) {
  int64_t blocks = cols / QK;
  int64_t group = n / LANES, lane = n % LANES;
  return (group * blocks + block) * RECORD + lane * 2;
}

/* quantizeTensorQ8_0Packed (Quantization.cpp:165-214).  Returns 0 on success,
 * -1 when the shape is not packable (isQ8PackedShape, Q8PackedLayout.h:38-42
 * requires rows % 8 and cols % 32; the encoder itself only needs rows % 4). */
int oracle_pack_q8_0_p4(const float *w, int64_t rows, int64_t cols,
                        uint8_t *out) {
  if (rows <= 0 || cols <= 0 || rows % (2 * LANES) || cols % QK)
    return -1;
  int64_t blocks = cols / QK, groups = rows / LANES;
  uint16_t *d = (uint16_t *)malloc(sizeof(uint16_t) * LANES * blocks);
  int8_t *qs = (int8_t *)malloc((size_t)(LANES * cols));
  for (int64_t g = 0; g < groups; ++g) {
    for (int64_t lane = 0; lane < LANES; ++lane)
      oracle_quantize_row_q8_0(w + (g * LANES + lane) * cols, cols,
                               d + lane * blocks, qs + lane * cols);
    for (int64_t b = 0; b < blocks; ++b) {
      uint8_t *rec = out + (g * blocks + b) * RECORD;
      for (int64_t lane = 0; lane < LANES; ++lane)
        memcpy(rec + lane * 2, &d[lane * blocks + b], 2); /* little endian */
      for (int64_t half = 0; half < 2; ++half)
        for (int64_t word = 0; word < 4; ++word) {
          uint8_t *chunk = rec + SCALE_BYTES + (half * 4 + word) * CHUNK;
          for (int64_t lane = 0; lane < LANES; ++lane)
            memcpy(chunk + lane * 4,
                   qs + lane * cols + b * QK + half * 16 + word * 4, 4);
        }
    }
  }
  free(d);
  free(qs);
  return 0;
}

/* Inverse of the layout: recover q[rows][cols] and d[rows][cols/32]. */
void oracle_unpack_q8_0_p4(const uint8_t *p4, int64_t rows, int64_t cols,
                           int8_t *qs, uint16_t *d) {
  int64_t blocks = cols / QK;
  for (int64_t n = 0; n < rows; ++n) {
    for (int64_t b = 0; b < blocks; ++b)
      memcpy(&d[n * blocks + b], p4 + oracle_p4_scale_offset(n, b, cols), 2);
    for (int64_t k = 0; k < cols; ++k)
      qs[n * cols + k] = (int8_t)p4[oracle_p4_qs_offset(n, k, cols)];
  }
}

/* --------------------------------------------------- activation Q8_1 ---- */

/* Activation quantizer, identical in Q8Decode.cpp:83-120,
 * Q8Matmul.cpp:93-141 and Q8Scalar.cpp:83-124: per 32-block
 * sa = maxAbs/127 (f32, stored unrounded), inv = maxAbs==0 ? 0 : 1/sa,
 * q = (int8)(int32)roundeven(x*inv) with no clamp. */
void oracle_quantize_act_q8_1(const float *x, int64_t rows, int64_t cols,
                              int8_t *qa, float *sa) {
  int64_t blocks = cols / QK;
  for (int64_t m = 0; m < rows; ++m)
    for (int64_t b = 0; b < blocks; ++b) {
      const float *v = x + m * cols + b * QK;
      float maxAbs = 0.0f;
      for (int i = 0; i < QK; ++i)
        maxAbs = fmaxf(maxAbs, fabsf(v[i])); /* arith.maxnumf */
      float scale = maxAbs / 127.0f;
      sa[m * blocks + b] = scale;
      float inv = maxAbs == 0.0f ? 0.0f : 1.0f / scale;
      for (int i = 0; i < QK; ++i) {
        float r = nearbyintf(v[i] * inv); /* default mode: ties to even */
        qa[m * cols + b * QK + i] = (int8_t)(int32_t)r;
      }
    }
}

/* ------------------------------------------------------ dot + epilogue -- */

/* Per-block int32 dot I_b[m][n][b] = sum_i qa[m,32b+i] * qw[n,32b+i], read
 * through the packed address function (Q8Scalar.cpp:162-191). */
void oracle_block_dots(const int8_t *qa, const uint8_t *p4, int64_t rows,
                       int64_t n, int64_t cols, int32_t *out) {
  int64_t blocks = cols / QK;
  for (int64_t m = 0; m < rows; ++m)
    for (int64_t c = 0; c < n; ++c)
      for (int64_t b = 0; b < blocks; ++b) {
        int32_t acc = 0;
        for (int64_t i = 0; i < QK; ++i) {
          int64_t k = b * QK + i;
          acc += (int32_t)qa[m * cols + k] *
                 (int32_t)(int8_t)p4[oracle_p4_qs_offset(c, k, cols)];
        }
        out[(m * n + c) * blocks + b] = acc;
      }
}

/* f32 exp used by the silu activation.  math.exp lowers to libm expf in the
 * reference; its last-ulp rounding is below the parity tolerance and is not
 * pinned.  Both this oracle and the HIP kernels evaluate exp in double and
 * round once to f32, so the two agree bit for bit. */
float oracle_expf(float x) { return (float)exp((double)x); }

/* math.log1p as the reference compiles it: --convert-math-to-llvm
 * (tools/llmcp-compile/llmcp-compile.cpp:186) lowers log1p(y) to
 * log(1 + y), the sum an f32 add; the log is evaluated in double and
 * rounded once, like oracle_expf. */
float oracle_log1pf(float x) {
  float s = 1.0f + x;
  return (float)log((double)s);
}

/* applyMatmulActivation (MatmulLoweringCommon.cpp:78-103), one MLIR op at a
 * time in f32: sigmoid = 1/(1+exp(-v)); silu(v) = v * sigmoid(v);
 * softplus(v) = log1p(exp(v)) with log1p lowered as above. */
float oracle_sigmoid(float v) {
  float e = oracle_expf(-v);
  return 1.0f / (1.0f + e);
}

float oracle_silu(float v) {
  float sig = oracle_sigmoid(v);
  return v * sig;
}

float oracle_softplus(float v) {
  float e = oracle_expf(v);
  return oracle_log1pf(e);
}

enum { ACT_NONE = 0, ACT_SILU = 1, ACT_SIGMOID = 2, ACT_SOFTPLUS = 3 };
enum { EPI_SCALAR = 0, EPI_FMA = 1 };

static float activate(float v, int act) {
  switch (act) {
    case ACT_SILU: return oracle_silu(v);
    case ACT_SIGMOID: return oracle_sigmoid(v);
    case ACT_SOFTPLUS: return oracle_softplus(v);
    default: return v;
  }
}

/* One output element over all blocks, in block order b = 0..B-1.
 * EPI_SCALAR: acc = acc + f32(I)*(sa*dw)         (Q8Scalar.cpp:192-199)
 * EPI_FMA:    acc = fma(f32(I), sa*dw, acc)      (Q8Decode.cpp:192-203,
 *                                                 Q8Matmul.cpp:204-223) */
static float dot_row(const int8_t *qa_row, const float *sa_row,
                     const uint8_t *p4, int64_t c, int64_t cols, int epi) {
  int64_t blocks = cols / QK;
  int64_t group = c / LANES, lane = c % LANES;
  float acc = 0.0f;
  for (int64_t b = 0; b < blocks; ++b) {
    const uint8_t *rec = p4 + (group * blocks + b) * RECORD;
    uint16_t dbits = (uint16_t)(rec[lane * 2] | (rec[lane * 2 + 1] << 8));
    float dw = oracle_f16_to_f32(dbits);
    int32_t dot = 0;
    for (int64_t e = 0; e < QK; ++e) {
      int8_t q = (int8_t)rec[SCALE_BYTES + (e / 4) * CHUNK + lane * 4 + e % 4];
      dot += (int32_t)qa_row[b * QK + e] * (int32_t)q;
    }
    float factor = sa_row[b] * dw;
    float dotf = (float)dot;
    if (epi == EPI_FMA) {
      acc = fmaf(dotf, factor, acc);
    } else {
      float contribution = dotf * factor;
      acc = acc + contribution;
    }
  }
  return acc;
}

/* Whole linear y[M,N] = act(x[M,K] . W^T), reference loop nest of
 * ScalarQ8::emit (Q8Scalar.cpp:65-212): quantize every row (parallel over
 * rows, :84), then rows in parallel (:127), columns serial.  With M == 1 the
 * parallel loop has one iteration, so this is single-threaded exactly as the
 * reference's x86 path is. */
void oracle_linear(const float *x, const uint8_t *p4, int64_t rows, int64_t n,
                   int64_t cols, int act, int epi, float *y) {
  int64_t blocks = cols / QK;
  int8_t *qa = (int8_t *)malloc((size_t)(rows * cols));
  float *sa = (float *)malloc(sizeof(float) * (size_t)(rows * blocks));
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < rows; ++m)
    oracle_quantize_act_q8_1(x + m * cols, 1, cols, qa + m * cols,
                             sa + m * blocks);
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < rows; ++m)
    for (int64_t c = 0; c < n; ++c)
      y[m * n + c] = activate(
          dot_row(qa + m * cols, sa + m * blocks, p4, c, cols, epi), act);
  free(qa);
  free(sa);
}

/* Same scalar math, parallel over output columns instead of rows.  Not a
 * reference schedule: a clearly labelled variant so the CPU baseline at M=1
 * can use every core. */
void oracle_linear_colpar(const float *x, const uint8_t *p4, int64_t rows,
                          int64_t n, int64_t cols, int act, int epi,
                          float *y) {
  int64_t blocks = cols / QK;
  int8_t *qa = (int8_t *)malloc((size_t)(rows * cols));
  float *sa = (float *)malloc(sizeof(float) * (size_t)(rows * blocks));
  oracle_quantize_act_q8_1(x, rows, cols, qa, sa);
  for (int64_t m = 0; m < rows; ++m) {
#pragma omp parallel for schedule(static)
    for (int64_t c = 0; c < n; ++c)
      y[m * n + c] = activate(
          dot_row(qa + m * cols, sa + m * blocks, p4, c, cols, epi), act);
  }
  free(qa);
  free(sa);
}

/* SwiGLU MLP hidden: h = silu(linear(x, Wg)) * linear(x, Wu)
 * (FuseLinearActivations.cpp:27-43 + MulOpLowering, LowerToLinalg.cpp:377-393;
 * shape from ModelBuilder.cpp:205-216). */
void oracle_swiglu(const float *x, const uint8_t *wg, const uint8_t *wu,
                   int64_t rows, int64_t n, int64_t cols, int epi, float *h,
                   int colpar) {
  float *u = (float *)malloc(sizeof(float) * (size_t)(rows * n));
  if (colpar) {
    oracle_linear_colpar(x, wg, rows, n, cols, ACT_SILU, epi, h);
    oracle_linear_colpar(x, wu, rows, n, cols, ACT_NONE, epi, u);
  } else {
    oracle_linear(x, wg, rows, n, cols, ACT_SILU, epi, h);
    oracle_linear(x, wu, rows, n, cols, ACT_NONE, epi, u);
  }
  for (int64_t i = 0; i < rows * n; ++i)
    h[i] = h[i] * u[i];
  free(u);
}

/* First index of the maximum: std::max_element with operator<
 * (llmcp-benchmark.cpp:51-54, llmcp-run.cpp:601-604). */
int64_t oracle_argmax(const float *v, int64_t n) {
  int64_t best = 0;
  for (int64_t i = 1; i < n; ++i)
    if (v[best] < v[i])
      best = i;
  return best;
}

/* Q8 embedding gather (emitQ8PackedEmbedding, LowerToLinalg.cpp:435-531):
 * out[t][c] = f32(q(token,c)) * f32(d(token, c/32)), exact in f32. */
void oracle_embedding(const int64_t *tokens, int64_t count, const uint8_t *p4,
                      int64_t cols, float *out) {
  int64_t blocks = cols / QK;
  (void)blocks;
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < count; ++t) {
    int64_t row = tokens[t];
    for (int64_t c = 0; c < cols; ++c) {
      int64_t so = oracle_p4_scale_offset(row, c / QK, cols);
      uint16_t dbits = (uint16_t)(p4[so] | (p4[so + 1] << 8));
      int8_t q = (int8_t)p4[oracle_p4_qs_offset(row, c, cols)];
      out[t * cols + c] = (float)q * oracle_f16_to_f32(dbits);
    }
  }
}

/* RMSNorm of `rows` rows of width h, each row on its own (decode:
 * DecodeNormalization.cpp:71-154 with groupSize = hidden, :160-171; prefill:
 * RmsNormOpLowering, LowerToLinalg.cpp:245-300 -- the same arithmetic):
 *   sum  = 0; for d in 0..h-1: sum = sum + x_d * x_d   (each step rounded)
 *   mean = sum / (float)h;  var = mean + eps
 *   rstd = 1 / sqrt(var)    (math.rsqrt as --convert-math-to-llvm lowers it:
 *                            an IEEE square root, then an IEEE division)
 *   y_d  = (x_d * rstd) * w'_d,  w' = w, or w + 1 when zero-centered.
 * x, w and y are f32 here (bf16 operands are widened exactly by the
 * caller, a bf16 result is rounded by it).  rstd_out (nullable) receives
 * each row's rstd. */
void oracle_rmsnorm(const float *x, int64_t rows, int64_t h, const float *w,
                    float eps, int zero_centered, float *y, float *rstd_out) {
  for (int64_t r = 0; r < rows; ++r) {
    const float *xr = x + r * h;
    float sum = 0.0f;
    for (int64_t d = 0; d < h; ++d) {
      float sq = xr[d] * xr[d];
      sum = sum + sq;
    }
    float mean = sum / (float)h;
    float var = mean + eps;
    float root = sqrtf(var);
    float rstd = 1.0f / root;
    if (rstd_out)
      rstd_out[r] = rstd;
    for (int64_t d = 0; d < h; ++d) {
      float wd = zero_centered ? w[d] + 1.0f : w[d];
      float t = xr[d] * rstd;
      y[r * h + d] = t * wd;
    }
  }
}

/* Gated RMSNorm (DecodeNormalization.cpp:124-147 with gate,
 * GatedRmsNormOpLowering, LowerToLinalg.cpp:574-720): each row splits into
 * groups of g values; per group the serial sum of x*x, rstd as in
 * oracle_rmsnorm with g in place of h, then
 *   y_d = ((x_d * s_d) * w_{d mod g}) * rstd,
 * s = silu(gate) (oracle_silu), or the gate itself when gate_activated. */
void oracle_gated_rmsnorm(const float *x, const float *gate, int64_t rows, int64_t h,
                          int64_t g, const float *w, float eps, int gate_activated,
                          float *y) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c0 = 0; c0 < h; c0 += g) {
      const float *xr = x + r * h + c0;
      const float *gr = gate + r * h + c0;
      float sum = 0.0f;
      for (int64_t d = 0; d < g; ++d) {
        float sq = xr[d] * xr[d];
        sum = sum + sq;
      }
      float mean = sum / (float)g;
      float var = mean + eps;
      float root = sqrtf(var);
      float rstd = 1.0f / root;
      for (int64_t d = 0; d < g; ++d) {
        float s = gate_activated ? gr[d] : oracle_silu(gr[d]);
        float v = xr[d] * s;
        v = v * w[d];
        y[r * h + c0 + d] = v * rstd;
      }
    }
}

int oracle_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void oracle_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0)
    omp_set_num_threads(n);
#else
  (void)n;
#endif
}
