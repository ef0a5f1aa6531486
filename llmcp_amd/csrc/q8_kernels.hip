// q8_kernels.hip -- gfx950 kernels of the Q8_0 linear path: one-time repack,
// synthetic weights + device packer, Q8_1 activation quantizer, the decode
// GEMV family with the scalar epilogue (plain / activations / fused SwiGLU /
// lm_head with fused argmax; the kernel template is in q8_gemv.h, its fma
// twins in q8_gemv_fma.hip), the embedding dequant gather and the exact
// block-dot probe.
//
// Numerics follow the reference's platforms: per output element, blocks are
// visited in order b = 0..B-1 and
//   acc = acc + f32(I_b) * (sa_b * dw_b)      x86 scalar path, Q8Scalar.cpp:192-199
//   acc = fma(f32(I_b), sa_b * dw_b, acc)     SDOT paths, Q8Decode.cpp:192-203
// with the same roundings.  The GEMV keeps that order exactly: the 16 lanes
// that own one row pass the running sum along with a DPP row rotation, so the
// f32 result is bit-identical to the reference.  Build with
// -ffp-contract=off so the compiler does not fuse the scalar form's multiply
// and add.
#include "q8_kernels.h"

#include <math.h>

#include <algorithm>

#include "q8_device.h"

#include "q8_gemv.h"

namespace llmcp_q8 {

// The fma-epilogue GEMVs (q8_gemv_fma.hip).
hipError_t launch_gemv_fma(const GemvArgs &a, const GemvLaunch &l, bool in_wg,
                           hipStream_t s);
hipError_t launch_gemv_group_fma(const GemvGroupArgs &a, const GemvLaunch &l,
                                 hipStream_t s);

namespace {

// ------------------------------------------------------------ repack ---- //

// One thread per (group, padded block, row-in-group).
__global__ void repack_kernel(const uint8_t *__restrict__ p4,
                              uint8_t *__restrict__ out, int64_t groups,
                              int64_t blocks, int64_t passes) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_group = passes * kPassBlocks * kLanes;
  if (t >= groups * per_group) return;
  const int64_t g = t / per_group;
  const int64_t rem = t - g * per_group;
  const int64_t b = rem / kLanes;
  const int r = (int)(rem % kLanes);
  uint32_t w[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  uint16_t scale = 0;
  if (b < blocks) {
    const uint8_t *rec = p4 + (g * blocks + b) * kRecord;
    scale = *(const uint16_t *)(rec + 2 * r);
#pragma unroll
    for (int c = 0; c < 8; ++c)
      w[c] = *(const uint32_t *)(rec + 8 + 16 * c + 4 * r);
  }
  int64_t u;
  int j;
  locate_seg(b, seg_for(passes), u, j);
  uint8_t *pass = out + (g * passes + u) * kPassBytes;
  *(uint4 *)(pass + r * 256 + j * 16) = make_uint4(w[0], w[1], w[2], w[3]);
  *(uint4 *)(pass + 1024 + r * 256 + j * 16) =
      make_uint4(w[4], w[5], w[6], w[7]);
  *(uint16_t *)(pass + kPassQs + 2 * (16 * r + j)) = scale;
}

// ----------------------------------------------- synthetic weights ------ //

__device__ __forceinline__ void philox4x32_10(uint32_t c[4], uint32_t k0,
                                              uint32_t k1) {
#pragma unroll
  for (int i = 0; i < 10; ++i) {
    const uint64_t p0 = (uint64_t)0xD2511F53u * c[0];
    const uint64_t p1 = (uint64_t)0xCD9E8D57u * c[2];
    const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0;
    const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1;
    c[1] = (uint32_t)p1;
    c[3] = (uint32_t)p0;
    c[0] = n0;
    c[2] = n2;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
}

// One thread per pair of elements: Box-Muller on one Philox draw.
__global__ void synth_kernel(uint64_t seed, int64_t count, float stddev,
                             float *__restrict__ w) {
  const int64_t pair = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (2 * pair >= count) return;
  uint32_t c[4] = {(uint32_t)pair, (uint32_t)(pair >> 32), 0x51ed270bu,
                   0x2f2a9e5du};
  philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
  const float u1 = ((float)c[0] + 0.5f) * 2.3283064365386963e-10f;
  const float u2 = (float)c[1] * 2.3283064365386963e-10f;
  const float rad = sqrtf(-2.0f * logf(u1));
  const float ang = 6.283185307179586f * u2;
  w[2 * pair] = stddev * rad * cosf(ang);
  if (2 * pair + 1 < count) w[2 * pair + 1] = stddev * rad * sinf(ang);
}

// Device restatement of quantizeRowQ8_0 + quantizeTensorQ8_0Packed
// (Quantization.cpp:92-116, :165-214).  One thread per (group, block).
__global__ void pack_p4_kernel(const float *__restrict__ w, int64_t groups,
                               int64_t blocks, uint8_t *__restrict__ p4) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= groups * blocks) return;
  const int64_t g = t / blocks, b = t - g * blocks;
  const int64_t cols = blocks * kBlock;
  uint8_t *rec = p4 + t * kRecord;
  for (int r = 0; r < kLanes; ++r) {
    const float *v = w + (g * kLanes + r) * cols + b * kBlock;
    float x[kBlock];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < kBlock; ++i) {
      x[i] = v[i];
      const float a = fabsf(x[i]);
      amax = amax < a ? a : amax;
    }
    uint16_t d = 0;
    int8_t q[kBlock];
    if (amax == 0.0f) {
#pragma unroll
      for (int i = 0; i < kBlock; ++i) q[i] = 0;
    } else {
      const float scale = amax / 127.0f;
      d = float_to_half_bits(scale);
#pragma unroll
      for (int i = 0; i < kBlock; ++i) {
        long v8 = lroundf(x[i] / scale);
        v8 = v8 < -127 ? -127 : (v8 > 127 ? 127 : v8);
        q[i] = (int8_t)v8;
      }
    }
    *(uint16_t *)(rec + 2 * r) = d;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const uint32_t word = (uint32_t)(uint8_t)q[4 * c] |
                            ((uint32_t)(uint8_t)q[4 * c + 1] << 8) |
                            ((uint32_t)(uint8_t)q[4 * c + 2] << 16) |
                            ((uint32_t)(uint8_t)q[4 * c + 3] << 24);
      *(uint32_t *)(rec + 8 + 16 * c + 4 * r) = word;
    }
  }
}


// Exhaustive check of div127 and recip against IEEE division over the
// float bit patterns [lo, hi): one pattern per thread, mismatches counted
// per wave.
__global__ void selftest_quant_kernel(uint32_t lo, uint32_t hi,
                                      unsigned long long *bad) {
  const uint32_t i = lo + blockIdx.x * blockDim.x + threadIdx.x;
  bool miss = false;
  if (i < hi) {
    const float v = __builtin_bit_cast(float, i);
    const float d_ref = v / 127.0f;
    miss = __builtin_bit_cast(uint32_t, div127(v)) !=
           __builtin_bit_cast(uint32_t, d_ref);
    if (v > 0.0f) {
      const float r_ref = 1.0f / v;
      miss |= __builtin_bit_cast(uint32_t, recip(v)) !=
              __builtin_bit_cast(uint32_t, r_ref);
    }
  }
  const unsigned long long mask = __ballot(miss);
  if ((threadIdx.x & 63) == 0 && mask)
    atomicAdd(bad, (unsigned long long)__popcll(mask));
}

// Exhaustive check of exp_f32 over the float bit patterns [lo, hi) (NaN
// inputs skipped).  out[0] counts inputs whose exp y lies within 2^-46
// (relative) of a change of float rounding -- y(1-2^-46) and y(1+2^-46)
// round to different floats -- and the first `cap` of them are stored with
// exp_f32's result bits (out[3] is the append cursor); out[1] counts inputs
// where exp_f32 differs from the math library's exp(double) rounded to
// float, and out[2] those of them outside the first set; out[4] is the
// largest difference between exp_f32's f64 value and the library's
// exp(double), in units of the latter's last place (|v| <= 100).
__global__ void selftest_exp_kernel(uint32_t lo, uint32_t hi,
                                    unsigned long long *out, float *inputs,
                                    uint32_t *results, uint32_t cap) {
  const uint32_t i = lo + blockIdx.x * blockDim.x + threadIdx.x;
  bool near = false, differ = false;
  float v = 0.0f, got = 0.0f;
  if (i < hi) {
    v = __builtin_bit_cast(float, i);
    if (v == v) {
      got = exp_f32(v);
      const float lib = (float)exp((double)v);
      differ = __builtin_bit_cast(uint32_t, got) != __builtin_bit_cast(uint32_t, lib);
      const double y =
          exp_f64_reduced((double)(v > 100.0f ? 100.0f : (v < -110.0f ? -110.0f : v)));
      const float fa = (float)(y * (1.0 - 0x1p-46)), fb = (float)(y * (1.0 + 0x1p-46));
      near = __builtin_bit_cast(uint32_t, fa) != __builtin_bit_cast(uint32_t, fb);
      if (v >= -100.0f && v <= 100.0f) {
        const double yl = exp((double)v);
        int e2;
        (void)frexp(yl, &e2);
        const double ulps = fabs(y - yl) / ldexp(1.0, e2 - 53);
        atomicMax(out + 4, (unsigned long long)ceil(ulps));
      }
    }
  }
  const unsigned long long mn = __ballot(near), md = __ballot(differ),
                           mo = __ballot(differ && !near);
  if ((threadIdx.x & 63) == 0) {
    if (mn) atomicAdd(out, (unsigned long long)__popcll(mn));
    if (md) atomicAdd(out + 1, (unsigned long long)__popcll(md));
    if (mo) atomicAdd(out + 2, (unsigned long long)__popcll(mo));
  }
  if (near) {
    const unsigned long long slot = atomicAdd(out + 3, 1ull);
    if (slot < cap) {
      inputs[slot] = v;
      results[slot] = __builtin_bit_cast(uint32_t, got);
    }
  }
}

// Grid: x covers (row, padded block) in units of 8 blocks per wave.  The
// grid's threads are below 2^32 (the launch checks), so the index math is
// 32-bit (a 64-bit division per thread took the M = 1024, K = 2560
// quantizer from 3.3 to 4.6 us).
__global__ void quantize_kernel(const void *__restrict__ x, int x_bf16,
                                int64_t m, int64_t ldx, int64_t blocks,
                                int8_t *qa, int64_t ldq, float *sa,
                                int64_t lds, int64_t blocks_pad, int aligned) {
  const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t blk_all = t >> 3;  // global (row, block) index
  const int lane = threadIdx.x & 63;
  const uint32_t row_i = blk_all / (uint32_t)blocks_pad;
  const int64_t row = (int64_t)row_i;
  const int64_t blk = (int64_t)(blk_all - row_i * (uint32_t)blocks_pad);
  const bool in_range = row < m;
  const bool valid = in_range && blk < blocks;
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (valid)
    v = load_act4(x, row * ldx + blk * kBlock + (lane & 7) * 4, x_bf16 != 0,
                  aligned != 0);
  int32_t q;
  float s;
  quantize_block8(v, valid, &q, &s);
  if (in_range) {
    *(int32_t *)(qa + row * ldq + blk * kBlock + (lane & 7) * 4) = q;
    if ((lane & 7) == 0) sa[row * lds + blk] = s;
  }
}

// Q8_1 into the GEMM's tiled layout: one wave per 32-row x 1-block tile
// (tile index rt * blocks_pad + b), in four steps of 8 rows: lane l takes
// values 4(l%8) .. +3 of row 32rt + 8c + l/8, so each step reads 8 rows of
// 128 B and writes 256 contiguous bytes of the tile.  quantize_block8 does
// the arithmetic, so the bits match the row kernel.  Rows past m and blocks
// past `blocks` are written as zeros.
template <bool XB, bool AL>
__global__ __launch_bounds__(256) void quantize_tiles_kernel(
    const void *__restrict__ x, int64_t m, int64_t ldx, int32_t blocks,
    int32_t blocks_pad, int64_t tiles, int8_t *__restrict__ qa,
    float *__restrict__ sa) {
  const int lane = threadIdx.x & 63;
  const int64_t tile = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tile >= tiles) return;  // uniform per wave
  const int32_t rt = (int32_t)(tile / blocks_pad);
  const int32_t b = (int32_t)(tile - (int64_t)rt * blocks_pad);
  const int rr = lane >> 3, p = lane & 7;
  // The four loads go out unconditionally (rows past m and padded blocks
  // read a clamped address) and are zeroed only once all are in flight.
  const int32_t bc = b < blocks ? b : blocks - 1;
  float4 v[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int64_t row = (int64_t)rt * 32 + 8 * c + rr;
    const int64_t rc = row < m ? row : m - 1;
    v[c] = load_act4_t<XB, AL>(x, rc * ldx + (int64_t)bc * kBlock + 4 * p);
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int64_t row = (int64_t)rt * 32 + 8 * c + rr;
    if (!(row < m && b < blocks)) v[c] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    int32_t q;
    float s;
    quantize_block8(v[c], true, &q, &s);
    *(int32_t *)(qa + tile * 1024 + (8 * c + rr) * kBlock + 4 * p) = q;
    if (p == 0) sa[tile * 32 + 8 * c + rr] = s;
  }
}


// RMSNorm of up to 4 rows per workgroup, each row on its own as the
// reference reduces it (DecodeNormalization.cpp:93-107 and :124-154 for
// decode rows, LowerToLinalg.cpp:245-300 for prefill: the same arithmetic):
// sum = sum + x*x over the row in index order, each step rounded to f32;
// rstd = 1 / sqrt(sum / H + eps) with an IEEE square root and division
// (math.rsqrt under --convert-math-to-llvm); y = (x * rstd) * w', w' = w, or
// w + 1 when zero-centered; bf16 outputs rounded to nearest even.
//
// The serial sum is one dependent add per element, the critical path: lane
// r of wave 0 folds row r from LDS (four squares per ds_read_b128, rows
// padded by 16 B so the lanes' reads fall in distinct banks), nothing
// else in its instruction stream.  Waves 1-3 load the next 512-column
// chunk of the workgroup's rows and store its squares in the other LDS
// buffer meanwhile.  Then all waves write y and, with QMODE, its Q8_1 (the
// quantizer's arithmetic, quantize_block8, on the values as stored): QMODE
// 1 the dense [m][blocks_pad * 32] layout, QMODE 2 the GEMM's tiled layout
// (blocks past H written as zeros).  Rows past m in the last tile are left
// unwritten, unlike launch_quantize_tiled, which zeroes them: they hold
// whatever the workspace held before.  That is harmless only because every
// consumer of the tiled layout stores results of rows below m alone (the
// GEMM's epilogue checks m < m_rows), which never read those rows.
// Requires h % 32 == 0.
//
// GATED: llmcp.gated_rms_norm, whose groups of h values are the rows here
// (DecodeNormalization.cpp:124-147, GatedRmsNormOpLowering,
// LowerToLinalg.cpp:574-720): the same sum and rstd over x, then
// y = ((x * s) * w) * rstd with s = g * (1 / (1 + exp(-g))) of the gate
// row g, or s = g when the gate is already activated.
constexpr int kNormRows = 4;
constexpr int kNormChunk = 512;

template <bool XB, bool WB, bool YB, int QMODE, bool GATED>
__global__ __launch_bounds__(256) void rmsnorm_kernel(
    const void *__restrict__ x, int64_t ldx, const void *__restrict__ w,
    float eps, int zero_centered, int64_t m, int32_t h, void *__restrict__ y,
    int64_t ldy, int8_t *__restrict__ qa, float *__restrict__ sa,
    int32_t blocks_pad, int aligned, const void *__restrict__ gate, int64_t ldg,
    int gate_activated) {
  static_assert(!GATED || QMODE == 0, "a gated norm writes no Q8_1");
  __shared__ __align__(16) float sq[2][kNormRows][kNormChunk + 4];
  __shared__ float rstd_s[kNormRows];
  const int64_t row0 = (int64_t)blockIdx.x * kNormRows;
  const int rows = (int)min<int64_t>(kNormRows, m - row0);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int chunks = (h + kNormChunk - 1) / kNormChunk;
  // squares of chunk c into buffer b by threads t0.. (nt of them), four
  // consecutive values per thread and step (h % 32 == 0: never a partial
  // vector)
  auto stage = [&](int c, int b, int t0, int nt) __attribute__((always_inline)) {
    const int c0 = c * kNormChunk, cw = min(kNormChunk, h - c0), q = cw / 4;
    for (int e = (int)threadIdx.x - t0; e < rows * q; e += nt) {
      const int r = e / q, j = 4 * (e - r * q);
      const float4 v = load_act4(x, (row0 + r) * ldx + c0 + j, XB, aligned != 0);
      *(float4 *)&sq[b][r][j] = make_float4(v.x * v.x, v.y * v.y, v.z * v.z, v.w * v.w);
    }
  };
  stage(0, 0, 0, 256);
  __syncthreads();
  float sum = 0.0f;
  for (int c = 0; c < chunks; ++c) {
    if (wave == 0) {
      if (lane < rows) {
        const int cw = min(kNormChunk, h - c * kNormChunk);
        const float *q = sq[c & 1][lane];
        // the reads of the next 32 values go out before the adds of these
        // (cw % 64 == 0 except for a final 32), kept in that order by
        // scheduling barriers
        float4 va[8], vb[8];
        auto rd = [&](float4 (&v)[8], int j) __attribute__((always_inline)) {
#pragma unroll
          for (int u = 0; u < 8; ++u) v[u] = *(const float4 *)(q + j + 4 * u);
        };
        auto add = [&](const float4 (&v)[8]) __attribute__((always_inline)) {
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            sum = sum + v[u].x;
            sum = sum + v[u].y;
            sum = sum + v[u].z;
            sum = sum + v[u].w;
          }
        };
        rd(va, 0);
        int j = 0;
        for (; j + 64 <= cw; j += 64) {
          rd(vb, j + 32);
          __builtin_amdgcn_sched_barrier(0);
          add(va);
          __builtin_amdgcn_sched_barrier(0);
          rd(va, j + 64 < cw ? j + 64 : j);
          __builtin_amdgcn_sched_barrier(0);
          add(vb);
          __builtin_amdgcn_sched_barrier(0);
        }
        if (j < cw) add(va);
      }
    } else if (c + 1 < chunks) {
      stage(c + 1, (c + 1) & 1, 64, 192);
    }
    __syncthreads();
  }
  if (wave == 0 && lane < rows) {
    const float mean = sum / (float)h;
    const float var = mean + eps;
    rstd_s[lane] = 1.0f / sqrtf(var);
  }
  __syncthreads();

  // y and its Q8_1: 8 lanes per (row, block), the same trip count in every
  // lane (quantize_block8 works across the wave)
  const int blocks = h / kBlock;
  const int out_rows = rows;
  const int nb = QMODE != 0 ? blocks_pad : blocks;
  const int units = out_rows * nb;
  const int p = threadIdx.x & 7;
  for (int u0 = 0; u0 < units; u0 += 32) {
    const int unit = u0 + (threadIdx.x >> 3);
    const int r = min(unit / nb, max(out_rows - 1, 0));
    const int b = unit - (unit / nb) * nb;
    const int64_t row = row0 + r;
    const bool live = unit < units;
    const bool valid = live && r < rows && b < blocks;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (valid) {
      const float4 xv = load_act4(x, row * ldx + b * kBlock + 4 * p, XB, aligned != 0);
      float4 wv = load_act4(w, (int64_t)b * kBlock + 4 * p, WB, true);
      if (zero_centered) {
        wv.x = wv.x + 1.0f;
        wv.y = wv.y + 1.0f;
        wv.z = wv.z + 1.0f;
        wv.w = wv.w + 1.0f;
      }
      const float rs = rstd_s[r];
      if constexpr (GATED) {
        float4 g = load_act4(gate, row * ldg + b * kBlock + 4 * p, XB, aligned != 0);
        if (!gate_activated) {
          g.x = silu_f32(g.x);
          g.y = silu_f32(g.y);
          g.z = silu_f32(g.z);
          g.w = silu_f32(g.w);
        }
        v.x = ((xv.x * g.x) * wv.x) * rs;
        v.y = ((xv.y * g.y) * wv.y) * rs;
        v.z = ((xv.z * g.z) * wv.z) * rs;
        v.w = ((xv.w * g.w) * wv.w) * rs;
      } else {
        v.x = (xv.x * rs) * wv.x;
        v.y = (xv.y * rs) * wv.y;
        v.z = (xv.z * rs) * wv.z;
        v.w = (xv.w * rs) * wv.w;
      }
      if constexpr (YB) {
        const uint16_t b0 = float_to_bf16(v.x), b1 = float_to_bf16(v.y),
                       b2 = float_to_bf16(v.z), b3 = float_to_bf16(v.w);
        uint16_t *yp = (uint16_t *)y + row * ldy + b * kBlock + 4 * p;
        yp[0] = b0;
        yp[1] = b1;
        yp[2] = b2;
        yp[3] = b3;
        v = make_float4(bf16_to_float(b0), bf16_to_float(b1), bf16_to_float(b2),
                        bf16_to_float(b3));
      } else {
        float *yp = (float *)y + row * ldy + b * kBlock + 4 * p;
        yp[0] = v.x;
        yp[1] = v.y;
        yp[2] = v.z;
        yp[3] = v.w;
      }
    }
    if constexpr (QMODE != 0) {
      int32_t q;
      float sc;
      quantize_block8(v, valid, &q, &sc);
      if (live) {
        if constexpr (QMODE == 1) {
          *(int32_t *)(qa + row * ((int64_t)blocks_pad * kBlock) + b * kBlock + 4 * p) = q;
          if (p == 0) sa[row * blocks_pad + b] = sc;
        } else {
          const int64_t tile = (row >> 5) * blocks_pad + b;
          *(int32_t *)(qa + tile * 1024 + (row & 31) * kBlock + 4 * p) = q;
          if (p == 0) sa[tile * 32 + (row & 31)] = sc;
        }
      }
    }
  }
}

// The serial f32 sum of n squares (n % 4 == 0) from LDS continued from s, in
// order: one dependent add per element, the reads of the next 32 values out
// before the adds of these (kept in that order by scheduling barriers).
__device__ __forceinline__ float fold_serial(const float *q, int n, float s) {
  float4 va[8], vb[8];
  auto rd = [&](float4 (&v)[8], int j) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = *(const float4 *)(q + j + 4 * u);
  };
  auto add = [&](const float4 (&v)[8]) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      s = s + v[u].x;
      s = s + v[u].y;
      s = s + v[u].z;
      s = s + v[u].w;
    }
  };
  const int n32 = n & ~31;
  int j = 0;
  if (n32 > 0) {
    rd(va, 0);
    for (; j + 64 <= n32; j += 64) {
      rd(vb, j + 32);
      __builtin_amdgcn_sched_barrier(0);
      add(va);
      __builtin_amdgcn_sched_barrier(0);
      rd(va, j + 64 < n32 ? j + 64 : j);
      __builtin_amdgcn_sched_barrier(0);
      add(vb);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (j < n32) {
      add(va);
      j += 32;
    }
  }
  for (; j < n; j += 4) {
    const float4 v = *(const float4 *)(q + j);
    s = s + v.x;
    s = s + v.y;
    s = s + v.z;
    s = s + v.w;
  }
  return s;
}

// RMSNorm of one row per workgroup with the serial sum evaluated
// speculatively, for rows of up to kSpecMaxH values.  The result is the
// serial sum itself, bit for bit; only the time depends on the data.
//
// The row's squares go to LDS, split into kSpecSegs segments of whole
// 32-value blocks, segment j owned by half j % 2 of wave j / 2, whose lanes
// fold it serially, exactly as the serial sum would, each from its own
// candidate start: 32 consecutive f32 bit patterns around a prediction of
// the sum where the segment starts (clamped to [+0, +inf]).  The
// predictions come in two passes.  Pass A takes the prefix of the segments'
// sums (f32, any order).  The serial sum drifts from the exact one by its
// rounding errors, but a segment's growth (end - start) from its pass-A
// centre start differs from its growth from the true start by an ulp or two
// at most (the rounding of a step depends on the start only through the
// binade and, at an exact tie, the parity of the sum); so pass B predicts
// each start as the sum of the pass-A growths of the segments before it,
// and folds its candidates around that.  Then the segments are chained in
// order: the true start of segment 0 is +0; the true start of segment j+1
// is the end of segment j from a lane (of pass B, else of pass A) whose
// candidate equals segment j's true start bit for bit, and where no
// candidate does, segment j is folded again from its true start.  Every
// step of the result is thus the serial sum's own step from the same
// operand bits.
//
// x and w are loaded once, each lane four values at a time from its own
// segment, and kept in registers for the epilogue, which is
// rmsnorm_kernel's: y, and with QMODE its Q8_1.  `aligned`: bit 0, rows of x
// start on 4-value boundaries; bit 1, so do rows of y.  Dynamic LDS: 4 * h
// bytes.
constexpr int kSpecSegs = 16;
constexpr int kSpecCands = 32;
constexpr int kSpecThreads = kSpecSegs * kSpecCands;
constexpr int kSpecMaxH = 12288;
// float4s of a segment per lane, at most
constexpr int kSpecRun4 = (kSpecMaxH / 4 / kSpecSegs + kSpecCands - 1) / kSpecCands;
// bf16 rows up to which the one-row-per-workgroup kernel is used (four per
// CU; half as many f32 rows, which hold twice the registers); more rows take
// rmsnorm_kernel, four rows to a workgroup
constexpr int64_t kSpecMaxRows = 1024;

template <bool XB, bool WB, bool YB, int QMODE>
__global__ __launch_bounds__(kSpecThreads) void rmsnorm_spec_kernel(
    const void *__restrict__ x, int64_t ldx, const void *__restrict__ w,
    float eps, int zero_centered, int32_t h, void *__restrict__ y,
    int64_t ldy, int8_t *__restrict__ qa, float *__restrict__ sa,
    int32_t blocks_pad, int aligned, int skew) {
  extern __shared__ __align__(16) float spec_sq[];
  // candidate starts and ends of passes A (0) and B (1)
  __shared__ uint32_t cand_start[2][kSpecSegs][kSpecCands];
  __shared__ uint32_t cand_end[2][kSpecSegs][kSpecCands];
  __shared__ float seg_sum[kSpecSegs];
  __shared__ double seg_grow[kSpecSegs];
  __shared__ uint32_t seg_guess[kSpecSegs];  // pass B's predictions, as bits
  const int64_t row = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63, p = t & 7;
  const int seg = t / kSpecCands, c = t % kSpecCands;
  const int blocks = h / kBlock;
  // the arguments the epilogue needs, in registers from the start: a
  // scalar load still in flight makes every LDS wait a full wait, and the
  // compiler would otherwise issue them just before the folds
  asm volatile("" ::"s"(y), "s"(ldy), "s"(qa), "s"(sa), "s"(eps), "s"(zero_centered));
  // segment j: whole 32-value blocks [lo, hi) with lo = j * blocks / 16, as
  // float4s [8 lo, 8 hi); lane c of its half holds float4s f0 + c + 32 q of
  // x and w in registers (whole blocks in eight consecutive lanes, as the
  // quantizer wants them)
  auto seg4 = [&](int j) __attribute__((always_inline)) {
    return 8 * (int)(((int64_t)j * blocks) / kSpecSegs);
  };
  const int f0 = seg4(seg), l4 = seg4(seg + 1) - f0;
  // float4s per lane in the longest segment (the same in every lane)
  const int r4 = (8 * ((blocks + kSpecSegs - 1) / kSpecSegs) + kSpecCands - 1) / kSpecCands;
  uint4 rx[kSpecRun4], rw[kSpecRun4];
  auto load = [&](auto al) __attribute__((always_inline)) {
    constexpr bool AL = decltype(al)::value;
#pragma unroll
    for (int q = 0; q < kSpecRun4; ++q) {
      if (q < r4) {
        // past the segment: its first float4 again, never used
        const int i = 4 * (f0 + (c + kSpecCands * q < l4 ? c + kSpecCands * q : 0));
        rx[q] = load_raw4<XB, AL>(x, row * ldx + min(i, h - 4));
        rw[q] = load_raw4<WB, true>(w, min(i, h - 4));
      }
    }
  };
  if (aligned & 1)
    load(std::true_type{});
  else
    load(std::false_type{});
  // squares to LDS; the segment's sum in f32, in any order (only pass A's
  // starts come from these sums, and they need only be close)
  float loc = 0.0f;
#pragma unroll
  for (int q = 0; q < kSpecRun4; ++q) {
    if (q < r4 && c + kSpecCands * q < l4) {
      const float4 v = act4_of_raw<XB>(rx[q]);
      const float4 sq = make_float4(v.x * v.x, v.y * v.y, v.z * v.z, v.w * v.w);
      *(float4 *)&spec_sq[4 * (f0 + c + kSpecCands * q)] = sq;
      loc += (sq.x + sq.y) + (sq.z + sq.w);
    }
  }
#pragma unroll
  for (int off = kSpecCands / 2; off > 0; off >>= 1) loc += __shfl_xor(loc, off, kSpecCands);
  if (c == 0) seg_sum[seg] = loc;
  __syncthreads();
  float base = 0.0f;
  {
    float ss[kSpecSegs];
#pragma unroll
    for (int j = 0; j < kSpecSegs; ++j) ss[j] = seg_sum[j];
#pragma unroll
    for (int j = 0; j < kSpecSegs; ++j)
      if (j < seg) base += ss[j];
  }

  // pass A; the segment's growth from its centre candidate
  auto candidates = [&](int pass, float guess) __attribute__((always_inline)) {
    const int cb = (int)min(__float_as_uint(guess), 0x7f800000u) + c - kSpecCands / 2;
    const uint32_t start = (uint32_t)min(max(cb, 0), 0x7f800000);
    const float end = fold_serial(spec_sq + 4 * f0, 4 * l4, __uint_as_float(start));
    cand_start[pass][seg][c] = start;
    cand_end[pass][seg][c] = __float_as_uint(end);
    return end;
  };
  const float end_a = candidates(0, base);
  if (c == kSpecCands / 2)
    seg_grow[seg] = (double)end_a - (double)__uint_as_float(cand_start[0][seg][c]);
  __syncthreads();
  // pass B: the sum of the growths before the segment
  double grown = 0.0;
  {
    double sg[kSpecSegs];
#pragma unroll
    for (int j = 0; j < kSpecSegs; ++j) sg[j] = seg_grow[j];
#pragma unroll
    for (int j = 0; j < kSpecSegs; ++j)
      if (j < seg) grown += sg[j];
  }
  // (skew: a test's offset of the predictions past segment 0, in bits)
  const int gb = min(max((int)min(__float_as_uint((float)grown), 0x7f800000u) +
                             (seg > 0 ? skew : 0), 0), 0x7f800000);
  candidates(1, __uint_as_float((uint32_t)gb));
  if (c == 0) seg_guess[seg] = (uint32_t)gb;
  __syncthreads();

  // the chain (every wave, the same values).  A segment's pass-B candidates
  // start at consecutive bits g - C/2 + i (g: its prediction's bits, C the
  // candidates per segment), so the candidate whose start equals the end of
  // candidate i of segment j is number end - (g' - C/2) of segment j + 1,
  // when in range: nx, in registers (lane l: candidate l % C of segment
  // G r + l / C in register r, G = 64 / C segments per wave); segment 0
  // starts at +0 = candidate C/2 (its prediction is +0).  The walk is then a
  // chain of register reads.
  constexpr int kC = kSpecCands, kG = 64 / kSpecCands, kR = kSpecSegs / kG;
  uint32_t nx[kR], ce_last;
  {
    uint32_t gn[kSpecSegs];
#pragma unroll
    for (int j = 0; j < kSpecSegs; ++j) gn[j] = seg_guess[j];
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      const int j = kG * r + lane / kC;
      const uint32_t en = cand_end[1][j][lane % kC];
      uint32_t g1 = gn[min(kG * r + 1, kSpecSegs - 1)];
#pragma unroll
      for (int k = 1; k < kG; ++k)
        if (lane / kC == k) g1 = gn[min(kG * r + k + 1, kSpecSegs - 1)];
      const uint32_t n = en - (g1 - kC / 2);
      nx[r] = en <= 0x7f800000u && n < (uint32_t)kC ? n : (uint32_t)kC;
    }
    ce_last = cand_end[1][kSpecSegs - 1][lane % kC];
  }
  uint32_t e = 0u;
  int next = 0;  // the first segment not yet chained
  {
    uint32_t idx = kC / 2, bad = seg_guess[0] != 0u ? 1u : 0u;
#pragma unroll
    for (int j = 0; j + 1 < kSpecSegs; ++j) {
      idx = (uint32_t)__builtin_amdgcn_readlane((int)nx[j / kG], kC * (j % kG) + (int)idx);
      bad |= idx / kC;
      idx &= kC - 1u;
    }
    if (!bad) {
      e = (uint32_t)__builtin_amdgcn_readlane((int)ce_last, (int)idx);
      next = kSpecSegs;
    }
  }
  // a segment whose start is not where expected among its pass-B candidates:
  // any candidate of either pass, else fold it again; and the rest
  for (; next < kSpecSegs; ++next) {
    const unsigned long long hit =
        __ballot(lane < 2 * kC && cand_start[lane / kC % 2][next][lane % kC] == e);
    if (hit != 0ull) {
      const int l = __ffsll((long long)hit) - 1;
      e = cand_end[l / kC][next][l % kC];
    } else {
      e = __float_as_uint(fold_serial(spec_sq + 4 * seg4(next),
                                      4 * (seg4(next + 1) - seg4(next)),
                                      __uint_as_float(e)));
    }
  }
  const float sum = __uint_as_float(e);
  const float mean = sum / (float)h;
  const float var = mean + eps;
  const float rs = 1.0f / sqrtf(var);

#pragma unroll
  for (int q = 0; q < kSpecRun4; ++q) {
    const int i4 = f0 + c + kSpecCands * q, i = 4 * i4, b = i4 / 8;
    // whole blocks: the lane's 8-group agrees
    if (q >= r4 || c + kSpecCands * q >= l4) continue;
    const float4 xv = act4_of_raw<XB>(rx[q]);
    float4 wv = act4_of_raw<WB>(rw[q]);
    if (zero_centered) {
      wv.x = wv.x + 1.0f;
      wv.y = wv.y + 1.0f;
      wv.z = wv.z + 1.0f;
      wv.w = wv.w + 1.0f;
    }
    float4 v;
    v.x = (xv.x * rs) * wv.x;
    v.y = (xv.y * rs) * wv.y;
    v.z = (xv.z * rs) * wv.z;
    v.w = (xv.w * rs) * wv.w;
    if constexpr (YB) {
      const uint16_t h0 = float_to_bf16(v.x), h1 = float_to_bf16(v.y),
                     h2 = float_to_bf16(v.z), h3 = float_to_bf16(v.w);
      uint16_t *yp = (uint16_t *)y + row * ldy + i;
      if (aligned & 2) {
        *(uint2 *)yp = make_uint2((uint32_t)h0 | ((uint32_t)h1 << 16),
                                  (uint32_t)h2 | ((uint32_t)h3 << 16));
      } else {
        yp[0] = h0;
        yp[1] = h1;
        yp[2] = h2;
        yp[3] = h3;
      }
      v = make_float4(bf16_to_float(h0), bf16_to_float(h1), bf16_to_float(h2),
                      bf16_to_float(h3));
    } else {
      float *yp = (float *)y + row * ldy + i;
      if (aligned & 2) {
        *(float4 *)yp = v;
      } else {
        yp[0] = v.x;
        yp[1] = v.y;
        yp[2] = v.z;
        yp[3] = v.w;
      }
    }
    if constexpr (QMODE != 0) {
      int32_t qv;
      float sc;
      quantize_block8(v, true, &qv, &sc);
      if constexpr (QMODE == 1) {
        *(int32_t *)(qa + row * ((int64_t)blocks_pad * kBlock) + b * kBlock + 4 * p) = qv;
        if (p == 0) sa[row * blocks_pad + b] = sc;
      } else {
        const int64_t tile = (row >> 5) * blocks_pad + b;
        *(int32_t *)(qa + tile * 1024 + (row & 31) * kBlock + 4 * p) = qv;
        if (p == 0) sa[tile * 32 + (row & 31)] = sc;
      }
    }
  }
  if constexpr (QMODE != 0) {
    // blocks past H up to blocks_pad: zeros, as the quantizer gives them
    for (int b = blocks + t / 8; b < blocks_pad; b += kSpecThreads / 8) {
      if constexpr (QMODE == 1) {
        *(int32_t *)(qa + row * ((int64_t)blocks_pad * kBlock) + b * kBlock + 4 * p) = 0;
        if (p == 0) sa[row * blocks_pad + b] = 0.0f;
      } else {
        const int64_t tile = (row >> 5) * blocks_pad + b;
        *(int32_t *)(qa + tile * 1024 + (row & 31) * kBlock + 4 * p) = 0;
        if (p == 0) sa[tile * 32 + (row & 31)] = 0.0f;
      }
    }
  }
}

// Gated RMSNorm, four groups of g values (g % 32 == 0, g <= kGatedMaxG) per
// 512-thread workgroup, two waves per group: wave j < 4 loads group j's x,
// writes its squares to LDS and folds them serially (every lane the same
// chain, from broadcast reads) into rstd; wave 4 + j meanwhile loads x,
// the gate and the weight and forms p = (x * s) * w, s = silu(gate) or the
// gate; after one barrier it writes y = p * rstd.  The gate's exp runs
// beside the fold instead of after it.  `aligned`: bit 0, x and gate on
// 4-value boundaries; bit 1, y.
constexpr int kGatedMaxG = 2048;
constexpr int kGatedSlots = kGatedMaxG / 256;  // float4s per lane

template <bool XB>
__global__ __launch_bounds__(512) void gated_rmsnorm_kernel(
    const void *__restrict__ x, const void *__restrict__ gate, const float *__restrict__ w,
    int64_t groups, int32_t g, float eps, int gate_activated, void *__restrict__ y,
    int aligned) {
  extern __shared__ __align__(16) float gated_sq[];
  __shared__ float gated_rstd[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, j = wave & 3;
  const int64_t grp = (int64_t)blockIdx.x * 4 + j;
  const bool live = grp < groups;  // uniform per wave
  const int g4 = g / 4, slots = (g4 + 63) / 64;
  asm volatile("" ::"s"(y), "s"(eps), "s"(gate_activated));
  float4 pv[kGatedSlots];
  if (wave < 4) {
    uint4 rx[kGatedSlots];
    auto load = [&](auto al) __attribute__((always_inline)) {
      constexpr bool AL = decltype(al)::value;
#pragma unroll
      for (int k = 0; k < kGatedSlots; ++k)
        if (k < slots) rx[k] = load_raw4<XB, AL>(x, grp * g + 4 * min(lane + 64 * k, g4 - 1));
    };
    if (live) {
      if (aligned & 1)
        load(std::true_type{});
      else
        load(std::false_type{});
      float *sq = gated_sq + j * g;
#pragma unroll
      for (int k = 0; k < kGatedSlots; ++k) {
        if (k < slots && lane + 64 * k < g4) {
          const float4 v = act4_of_raw<XB>(rx[k]);
          *(float4 *)&sq[4 * (lane + 64 * k)] =
              make_float4(v.x * v.x, v.y * v.y, v.z * v.z, v.w * v.w);
        }
      }
      // the wave's own LDS rows, read back in order by the same wave
      __builtin_amdgcn_s_waitcnt(0xc07f);
      __builtin_amdgcn_wave_barrier();
      const float sum = fold_serial(sq, g, 0.0f);
      const float mean = sum / (float)g;
      const float var = mean + eps;
      if (lane == 0) gated_rstd[j] = 1.0f / sqrtf(var);
    }
  } else if (live) {
    uint4 rx[kGatedSlots], rg[kGatedSlots];
    float4 wv[kGatedSlots];
    auto load = [&](auto al) __attribute__((always_inline)) {
      constexpr bool AL = decltype(al)::value;
#pragma unroll
      for (int k = 0; k < kGatedSlots; ++k) {
        if (k < slots) {
          const int i = 4 * min(lane + 64 * k, g4 - 1);
          rx[k] = load_raw4<XB, AL>(x, grp * g + i);
          rg[k] = load_raw4<XB, AL>(gate, grp * g + i);
          wv[k] = *(const float4 *)(w + i);
        }
      }
    };
    if (aligned & 1)
      load(std::true_type{});
    else
      load(std::false_type{});
#pragma unroll
    for (int k = 0; k < kGatedSlots; ++k) {
      if (k < slots) {
        const float4 xv = act4_of_raw<XB>(rx[k]);
        float4 gv = act4_of_raw<XB>(rg[k]);
        if (!gate_activated) {
          gv.x = silu_f32(gv.x);
          gv.y = silu_f32(gv.y);
          gv.z = silu_f32(gv.z);
          gv.w = silu_f32(gv.w);
        }
        pv[k].x = (xv.x * gv.x) * wv[k].x;
        pv[k].y = (xv.y * gv.y) * wv[k].y;
        pv[k].z = (xv.z * gv.z) * wv[k].z;
        pv[k].w = (xv.w * gv.w) * wv[k].w;
      }
    }
  }
  __syncthreads();
  if (wave < 4 || !live) return;
  const float rs = gated_rstd[j];
#pragma unroll
  for (int k = 0; k < kGatedSlots; ++k) {
    if (k < slots && lane + 64 * k < g4) {
      const int i = 4 * (lane + 64 * k);
      float4 v;
      v.x = pv[k].x * rs;
      v.y = pv[k].y * rs;
      v.z = pv[k].z * rs;
      v.w = pv[k].w * rs;
      if constexpr (XB) {
        const uint16_t h0 = float_to_bf16(v.x), h1 = float_to_bf16(v.y),
                       h2 = float_to_bf16(v.z), h3 = float_to_bf16(v.w);
        uint16_t *yp = (uint16_t *)y + grp * g + i;
        if (aligned & 2) {
          *(uint2 *)yp = make_uint2((uint32_t)h0 | ((uint32_t)h1 << 16),
                                    (uint32_t)h2 | ((uint32_t)h3 << 16));
        } else {
          yp[0] = h0;
          yp[1] = h1;
          yp[2] = h2;
          yp[3] = h3;
        }
      } else {
        float *yp = (float *)y + grp * g + i;
        if (aligned & 2) {
          *(float4 *)yp = v;
        } else {
          yp[0] = v.x;
          yp[1] = v.y;
          yp[2] = v.z;
          yp[3] = v.w;
        }
      }
    }
  }
}

// First-maximum argmax of one f32 row already in HBM (the last row of a
// prefill lm_head's logits): the same keys as the GEMV's fused argmax,
// folded into the same slots, so argmax_reduce_kernel finishes it.  A grid
// stride loop over the row, one key per workgroup.
__global__ __launch_bounds__(256) void argmax_row_kernel(
    const float *__restrict__ v, int64_t n, unsigned long long *slots) {
  __shared__ unsigned long long part[4];
  unsigned long long key = 0ull;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * 256)
    key = max_u64(key, argmax_key(v[i], i));
  key = wave_max_u64(key);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = key;
  __syncthreads();
  if (threadIdx.x == 0)
    argmax_fold(slots,
                max_u64(max_u64(part[0], part[1]), max_u64(part[2], part[3])));
}

// Second stage of the fused argmax: one workgroup of 1024 threads takes the
// kArgmaxSlots slots (swapping in 0, so the slots are clear for the next
// call without a memset) and writes the index of the first maximum.  With
// out == nullptr it only clears the slots.
__global__ __launch_bounds__(1024) void argmax_reduce_kernel(
    unsigned long long *slots, int64_t *out) {
  static_assert(kArgmaxSlots % 1024 == 0, "slots per thread");
  __shared__ unsigned long long part[16];
  unsigned long long best = 0ull;
#pragma unroll
  for (int u = 0; u < kArgmaxSlots / 1024; ++u)
    best = max_u64(best, __hip_atomic_exchange(slots + u * 1024 + threadIdx.x,
                                               0ull, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT));
  best = wave_max_u64(best);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x < 64) {
    best = wave_max_u64(threadIdx.x < 16 ? part[threadIdx.x] : 0ull);
    if (threadIdx.x == 0 && out)
      *out = (int64_t)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFull));
  }
}

// ---------------------------------------------------------- embedding -- //

// One thread per (token, V columns) -- LowerToLinalg.cpp:435-531 gathered
// from the unit layout.  out = f32(q) * f32(d), exact.  V = 4 for f32 rows
// (one 4 B word of quants) and 8 for bf16 rows (two words), so that every
// lane stores 16 B and a wave's stores form one contiguous run; the rows
// are written once, so the stores are non-temporal.  (One thread per 16
// columns, 64 B of plain stores per lane, took 6.4 us for 1024 ids of the
// 248320 x 2560 table against 3.8 us for this form.)  Workgroups are
// 256 lanes in two dimensions: x over a row's chunks (64, 128 or 256
// lanes, chosen by the host so that few lanes idle), y over 256 / x
// tokens; the grid's y strides over the tokens past what one resident
// round of workgroups holds.  A
// thread's column offsets are computed once, and no 64-bit division splits
// a flat index.
template <bool BF16>
__global__ __launch_bounds__(256) void embedding_kernel(
    const int64_t *__restrict__ tokens, int64_t count, const uint8_t *__restrict__ t,
    int64_t rows, int64_t passes, int32_t chunks, void *__restrict__ out, int64_t ldo,
    int32_t *err, int aligned) {
  constexpr int V = BF16 ? 8 : 4;
  const int c = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  const int64_t t0 = (int64_t)blockIdx.y * blockDim.y + threadIdx.y;
  const int64_t tstep = (int64_t)gridDim.y * blockDim.y;
  if (c >= chunks) return;
  const int64_t col = (int64_t)c * V;
  const int64_t b = col >> 5;             // block
  const int h = (int)((col >> 4) & 1);    // its 16-value half
  const int off = (int)(col & 15);        // first value within the half
  int64_t u;
  int j;
  locate_seg(b, seg_for(passes), u, j);
  // byte offsets inside a lane group's passes (row r adds r * 256 / 32)
  const int64_t q_off = u * kPassBytes + h * 1024 + j * 16 + off;
  const int64_t d_off = u * kPassBytes + kPassQs + 2 * j;
  typedef unsigned int v4u __attribute__((ext_vector_type(4)));
  for (int64_t ti = t0; ti < count; ti += tstep) {
    const int64_t tok = tokens[ti];
    float v[V];
    if (tok < 0 || tok >= rows) {
#pragma unroll
      for (int e = 0; e < V; ++e) v[e] = 0.0f;
      if (c == 0) atomicOr(err, 1);
    } else {
      const uint8_t *grp = t + (tok >> 2) * passes * kPassBytes;
      const int r = (int)(tok & 3);
      const uint8_t *qp = grp + q_off + r * 256;
      uint32_t w[V / 4];
      if constexpr (BF16) {
        const uint2 q = *(const uint2 *)qp;
        w[0] = q.x;
        w[1] = q.y;
      } else {
        w[0] = *(const uint32_t *)qp;
      }
      const float d = half_bits_to_float(*(const uint16_t *)(grp + d_off + 32 * r));
#pragma unroll
      for (int e = 0; e < V; ++e)
        v[e] = (float)(int8_t)(w[e >> 2] >> (8 * (e & 3))) * d;
    }
    if constexpr (BF16) {
      // truncf to a bf16 result (LowerToLinalg.cpp:435-531)
      uint16_t *o = (uint16_t *)out + ti * ldo + col;
      if (aligned) {
        v4u p;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          p[e] = (uint32_t)float_to_bf16(v[2 * e]) |
                 ((uint32_t)float_to_bf16(v[2 * e + 1]) << 16);
        __builtin_nontemporal_store(p, (v4u *)o);
      } else {
#pragma unroll
        for (int e = 0; e < V; ++e) o[e] = float_to_bf16(v[e]);
      }
    } else {
      float *o = (float *)out + ti * ldo + col;
      if (aligned) {
        const v4u p = {__float_as_uint(v[0]), __float_as_uint(v[1]),
                       __float_as_uint(v[2]), __float_as_uint(v[3])};
        __builtin_nontemporal_store(p, (v4u *)o);
      } else {
#pragma unroll
        for (int e = 0; e < V; ++e) o[e] = v[e];
      }
    }
  }
}

// --------------------------------------------------------- block dots -- //

__global__ void block_dots_kernel(const int8_t *__restrict__ qa, int64_t ldq,
                                  int64_t m, const uint8_t *__restrict__ w,
                                  int64_t rows, int64_t blocks,
                                  int64_t passes, int32_t *__restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= m * rows * blocks) return;
  const int64_t b = t % blocks;
  const int64_t n = (t / blocks) % rows;
  const int64_t mi = t / (blocks * rows);
  const int64_t g = n >> 2;
  const int r = (int)(n & 3);
  int64_t u;
  int j;
  locate_seg(b, seg_for(passes), u, j);
  const uint8_t *pass = w + (g * passes + u) * kPassBytes;
  const uint4 w0 = *(const uint4 *)(pass + r * 256 + j * 16);
  const uint4 w1 = *(const uint4 *)(pass + 1024 + r * 256 + j * 16);
  const int8_t *arow = qa + mi * ldq + b * kBlock;
  uint4 a0, a1;
  __builtin_memcpy(&a0, arow, 16);
  __builtin_memcpy(&a1, arow + 16, 16);
  out[t] = dot8(w1, a1, dot8(w0, a0, 0));
}

}  // namespace

hipError_t launch_repack(const uint8_t *p4, uint8_t *out, int64_t rows,
                         int64_t cols, hipStream_t s) {
  const int64_t groups = rows / kLanes, blocks = cols / kBlock;
  const int64_t passes = passes_for(cols);
  const int64_t threads = groups * passes * kPassBlocks * kLanes;
  hipLaunchKernelGGL(repack_kernel, dim3(grid_for(threads, 256)), dim3(256),
                     0, s, p4, out, groups, blocks, passes);
  return hipGetLastError();
}

hipError_t launch_synth(uint64_t seed, int64_t rows, int64_t cols,
                        float stddev, float *w, hipStream_t s) {
  const int64_t count = rows * cols;
  hipLaunchKernelGGL(synth_kernel, dim3(grid_for((count + 1) / 2, 256)),
                     dim3(256), 0, s, seed, count, stddev, w);
  return hipGetLastError();
}

hipError_t launch_pack_p4(const float *w, int64_t rows, int64_t cols,
                          uint8_t *p4, hipStream_t s) {
  const int64_t groups = rows / kLanes, blocks = cols / kBlock;
  hipLaunchKernelGGL(pack_p4_kernel, dim3(grid_for(groups * blocks, 128)),
                     dim3(128), 0, s, w, groups, blocks, p4);
  return hipGetLastError();
}

hipError_t launch_selftest_quantizer(unsigned long long *bad, hipStream_t s) {
  // every non-negative float up to +inf: 0x00000000 .. 0x7f800000
  const uint32_t lo = 0, hi = 0x7f800001u;
  hipLaunchKernelGGL(selftest_quant_kernel,
                     dim3(grid_for((int64_t)(hi - lo), 256)), dim3(256), 0, s,
                     lo, hi, bad);
  return hipGetLastError();
}

hipError_t launch_selftest_exp(unsigned long long *out, float *inputs,
                               uint32_t *results, uint32_t cap, hipStream_t s) {
  // all bit patterns in two halves (the last one, 0xffffffff, is a NaN)
  const uint32_t bounds[3] = {0u, 0x80000000u, 0xffffffffu};
  for (int h = 0; h < 2; ++h) {
    hipLaunchKernelGGL(selftest_exp_kernel,
                       dim3(grid_for((int64_t)(bounds[h + 1] - bounds[h]), 256)),
                       dim3(256), 0, s, bounds[h], bounds[h + 1], out, inputs,
                       results, cap);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_quantize(const void *x, bool x_bf16, int64_t m, int64_t ldx,
                           int64_t cols, int8_t *qa, int64_t ldq, float *sa,
                           int64_t lds, int64_t blocks_pad, hipStream_t s) {
  const int64_t blocks = cols / kBlock;
  const int64_t threads = m * blocks_pad * 8;
  const int64_t esz = x_bf16 ? 2 : 4;
  const int aligned =
      ((uintptr_t)x % (4 * esz) == 0) && (ldx % 4 == 0) ? 1 : 0;
  const dim3 grid(grid_for(threads, 256));
  // HIP bounds a grid's work-items by 2^32 - 1
  if ((int64_t)grid.x * 256 > 0xFFFFFFFFll) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(quantize_kernel, grid, dim3(256), 0, s, x, x_bf16 ? 1 : 0,
                     m, ldx, blocks, qa, ldq, sa, lds, blocks_pad, aligned);
  return hipGetLastError();
}

hipError_t launch_quantize_tiled(const void *x, bool x_bf16, int64_t m,
                                 int64_t ldx, int64_t cols, int8_t *qa,
                                 float *sa, int64_t blocks_pad, hipStream_t s) {
  const int64_t blocks = cols / kBlock;
  const int64_t tiles = (m + 31) / 32 * blocks_pad;
  const int64_t esz = x_bf16 ? 2 : 4;
  const int aligned =
      ((uintptr_t)x % (4 * esz) == 0) && (ldx % 4 == 0) ? 1 : 0;
  const dim3 grid((unsigned)((tiles + 3) / 4));
  const int32_t nb = (int32_t)blocks, np = (int32_t)blocks_pad;
  if (x_bf16) {
    if (aligned)
      hipLaunchKernelGGL((quantize_tiles_kernel<true, true>), grid, dim3(256), 0, s, x, m, ldx, nb, np, tiles, qa, sa);
    else
      hipLaunchKernelGGL((quantize_tiles_kernel<true, false>), grid, dim3(256), 0, s, x, m, ldx, nb, np, tiles, qa, sa);
  } else {
    if (aligned)
      hipLaunchKernelGGL((quantize_tiles_kernel<false, true>), grid, dim3(256), 0, s, x, m, ldx, nb, np, tiles, qa, sa);
    else
      hipLaunchKernelGGL((quantize_tiles_kernel<false, false>), grid, dim3(256), 0, s, x, m, ldx, nb, np, tiles, qa, sa);
  }
  return hipGetLastError();
}

bool gemv_quantizes_input(int64_t rows, int64_t cols, int nmat) {
  return nmat == 2 || rows / kLanes <= kInLoopQuantMaxGroups || cols <= kInLoopQuantMaxCols;
}


hipError_t launch_gemv(const GemvLaunch &l, hipStream_t s) {
  GemvArgs a;
  a.x = l.x;
  a.qa = l.qa;
  a.sa = l.sa;
  a.w0 = l.w[0];
  a.w1 = l.w[1] ? l.w[1] : l.w[0];
  a.y = l.y;
  a.r = l.residual;
  a.keys = l.keys;
  a.groups = l.rows / kLanes;
  a.blocks = (int32_t)(l.cols / kBlock);
  a.passes = (int32_t)passes_for(l.cols);
  a.act = l.activation;
  const int in = l.x ? IN_WG : IN_PRE;
  if (l.x && (uintptr_t)l.x % (l.x_bf16 ? 8 : 16)) return hipErrorInvalidValue;
  if (l.ngroup > 0) {
    // grouped: the weights' lane groups back to back in one grid
    if (!l.x || l.ngroup > kMaxGroup || l.keys || l.residual)
      return hipErrorInvalidValue;
    GemvGroupArgs ga;
    static_cast<GemvArgs &>(ga) = a;
    ga.nw = l.ngroup;
    int64_t start = 0;
    for (int i = 0; i < kMaxGroup; ++i) {
      const bool used = i < l.ngroup;
      ga.gstart[i] = start;
      ga.wt[i] = used ? l.gw[i] : l.gw[0];
      ga.yt[i] = used ? l.gy[i] : l.gy[0];
      ga.actt[i] = used ? l.gact[i] : 0;
      if (used) start += l.grows[i] / kLanes;
    }
    ga.gstart[kMaxGroup] = start;
    ga.groups = start;
    return l.fma ? launch_gemv_group_fma(ga, l, s) : launch_gemv_group<false>(ga, l, s);
  }
  hipError_t e;
  if (l.fma)
    e = launch_gemv_fma(a, l, in == IN_WG, s);
  else
    e = in == IN_WG ? launch_gemv_in<IN_WG, false>(a, l, s)
                    : launch_gemv_in<IN_PRE, false>(a, l, s);
  if (e != hipSuccess || !l.keys) return e;
  return launch_argmax_reduce(l.keys, l.argmax_out, s);
}


hipError_t launch_argmax_row(const float *v, int64_t n, int64_t *out,
                             unsigned long long *slots, hipStream_t s) {
  if (n <= 0 || n > 0xFFFFFFFFll) return hipErrorInvalidValue;
  const unsigned grid = (unsigned)std::min<int64_t>((n + 255) / 256, 1024);
  hipLaunchKernelGGL(argmax_row_kernel, dim3(grid), dim3(256), 0, s, v, n,
                     slots);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_argmax_reduce(slots, out, s);
}

hipError_t launch_argmax_reduce(unsigned long long *slots, int64_t *out,
                                hipStream_t s) {
  hipLaunchKernelGGL(argmax_reduce_kernel, dim3(1), dim3(1024), 0, s, slots,
                     out);
  return hipGetLastError();
}

hipError_t launch_rmsnorm(const void *x, bool x_bf16, int64_t m, int64_t ldx,
                          int64_t h, const void *w, bool w_bf16, float eps,
                          bool zero_centered, void *y, bool y_bf16, int64_t ldy,
                          int8_t *qa, float *sa, int64_t blocks_pad, int qmode,
                          hipStream_t s, int spec_skew) {
  if (h % kBlock != 0 || m <= 0 || (qmode != 0 && blocks_pad * kBlock < h))
    return hipErrorInvalidValue;
  if ((uintptr_t)w % (w_bf16 ? 8 : 16) != 0) return hipErrorInvalidValue;
  const int64_t esz = x_bf16 ? 2 : 4;
  const int aligned = ((uintptr_t)x % (4 * esz) == 0) && (ldx % 4 == 0) ? 1 : 0;
  const int zc = zero_centered ? 1 : 0;
  const int32_t hh = (int32_t)h, bp = (int32_t)blocks_pad;
  const bool spec = h <= kSpecMaxH && m <= (x_bf16 ? kSpecMaxRows : kSpecMaxRows / 2);
  const int yal = ((uintptr_t)y % (y_bf16 ? 8 : 16) == 0) && (ldy % 4 == 0) ? 1 : 0;
  const dim3 grid((unsigned)(spec ? m : (m + kNormRows - 1) / kNormRows));
  const size_t lds = spec ? (size_t)h * sizeof(float) : 0;
#define LLMCP_NORM(XB, WB, YB, Q)                                                          \
  if (x_bf16 == XB && w_bf16 == WB && y_bf16 == YB && qmode == Q) {                        \
    if (spec)                                                                              \
      hipLaunchKernelGGL((rmsnorm_spec_kernel<XB, WB, YB, Q>), grid, dim3(kSpecThreads), lds, \
                         s, x, ldx, w, eps, zc, hh, y, ldy, qa, sa, bp, aligned | (yal << 1), \
                         spec_skew);                                                       \
    else                                                                                   \
      hipLaunchKernelGGL((rmsnorm_kernel<XB, WB, YB, Q, false>), grid, dim3(256), 0, s, x,  \
                         ldx, w, eps, zc, m, hh, y, ldy, qa, sa, bp, aligned, nullptr, 0, 0); \
    return hipGetLastError();                                                              \
  }
  LLMCP_NORM(false, false, false, 0) LLMCP_NORM(false, false, false, 1)
  LLMCP_NORM(false, false, false, 2) LLMCP_NORM(true, true, true, 0)
  LLMCP_NORM(true, true, true, 1) LLMCP_NORM(true, true, true, 2)
  LLMCP_NORM(false, true, false, 0) LLMCP_NORM(false, true, false, 1)
  LLMCP_NORM(false, true, false, 2) LLMCP_NORM(true, false, true, 0)
  LLMCP_NORM(true, false, true, 1) LLMCP_NORM(true, false, true, 2)
#undef LLMCP_NORM
  return hipErrorInvalidValue;
}

hipError_t launch_gated_rmsnorm(const void *x, const void *gate, bool bf16,
                                int64_t groups, int64_t g, const float *w, float eps,
                                bool gate_activated, void *y, hipStream_t s) {
  if (g % kBlock != 0 || groups <= 0 || (uintptr_t)w % 16 != 0) return hipErrorInvalidValue;
  const int64_t esz = bf16 ? 2 : 4;
  const int aligned = ((uintptr_t)x % (4 * esz) == 0) && ((uintptr_t)gate % (4 * esz) == 0) &&
                              (g % 4 == 0) ? 1 : 0;
  const dim3 grid((unsigned)((groups + kNormRows - 1) / kNormRows));
  const int32_t gg = (int32_t)g;
  const int ga = gate_activated ? 1 : 0;
  if (g <= kGatedMaxG) {
    const int yal = (uintptr_t)y % (4 * esz) == 0 ? 2 : 0;
    const size_t lds = (size_t)4 * g * sizeof(float);
    if (bf16)
      hipLaunchKernelGGL(gated_rmsnorm_kernel<true>, grid, dim3(512), lds, s, x, gate, w,
                         groups, gg, eps, ga, y, aligned | yal);
    else
      hipLaunchKernelGGL(gated_rmsnorm_kernel<false>, grid, dim3(512), lds, s, x, gate, w,
                         groups, gg, eps, ga, y, aligned | yal);
    return hipGetLastError();
  }
  if (bf16)
    hipLaunchKernelGGL((rmsnorm_kernel<true, false, true, 0, true>), grid, dim3(256), 0, s, x, g,
                       w, eps, 0, groups, gg, y, g, nullptr, nullptr, 0, aligned, gate, g, ga);
  else
    hipLaunchKernelGGL((rmsnorm_kernel<false, false, false, 0, true>), grid, dim3(256), 0, s, x,
                       g, w, eps, 0, groups, gg, y, g, nullptr, nullptr, 0, aligned, gate, g, ga);
  return hipGetLastError();
}

hipError_t launch_embedding(const int64_t *tokens, int64_t count,
                            const uint8_t *table, int64_t rows, int64_t cols,
                            void *out, bool out_bf16, int64_t ldo,
                            int32_t *err_flag, hipStream_t s) {
  if (count == 0) return hipSuccess;
  const int64_t chunks = cols / (out_bf16 ? 8 : 4);
  const int aligned = out_bf16
      ? ((uintptr_t)out % 16 == 0) && (ldo % 8 == 0)
      : ((uintptr_t)out % 16 == 0) && (ldo % 4 == 0);
  // a row's chunks over the widest x (256, 128 or 64 lanes) that leaves
  // the fewest lanes idle, 256 / x tokens per workgroup
  int bs = 256;
  for (int cand : {128, 64}) {
    const int64_t waste = (chunks + cand - 1) / cand * cand - chunks;
    if (waste < (chunks + bs - 1) / bs * bs - chunks) bs = cand;
  }
  // At most eight workgroups per CU (32 waves, all resident at once; the
  // y stride hands a thread further tokens): 1024 f32 rows of 2560 values,
  // 2560 workgroups of one token pair each, took 4.51 us against 4.26 with
  // 2045 (and 4.66 with 1020).
  const int by = 256 / bs;
  const int64_t gx = (chunks + bs - 1) / bs;
  const int64_t ty = (count + by - 1) / by;
  int64_t ycap = std::max<int64_t>(1, 8 * (int64_t)cu_count() / gx);
  ycap = std::min<int64_t>(ycap, 65535);
  const dim3 grid((unsigned)gx, (unsigned)std::min(ty, ycap));
  const dim3 block(bs, by);
  if (out_bf16)
    hipLaunchKernelGGL((embedding_kernel<true>), grid, block, 0, s, tokens,
                       count, table, rows, passes_for(cols), (int32_t)chunks, out, ldo,
                       err_flag, aligned ? 1 : 0);
  else
    hipLaunchKernelGGL((embedding_kernel<false>), grid, block, 0, s, tokens,
                       count, table, rows, passes_for(cols), (int32_t)chunks, out, ldo,
                       err_flag, aligned ? 1 : 0);
  return hipGetLastError();
}

hipError_t launch_block_dots(const int8_t *qa, int64_t ldq, int64_t m,
                             const uint8_t *w, int64_t rows, int64_t cols,
                             int32_t *out, hipStream_t s) {
  const int64_t blocks = cols / kBlock;
  const int64_t threads = m * rows * blocks;
  if (threads == 0) return hipSuccess;
  hipLaunchKernelGGL(block_dots_kernel, dim3(grid_for(threads, 256)),
                     dim3(256), 0, s, qa, ldq, m, w, rows, blocks,
                     passes_for(cols), out);
  return hipGetLastError();
}

}  // namespace llmcp_q8