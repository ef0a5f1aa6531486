// q8_kernels.hip -- gfx950 kernels of the Q8_0 linear path: one-time repack,
// synthetic weights + device packer, Q8_1 activation quantizer, the decode
// GEMV family (plain / SiLU / fused SwiGLU / lm_head with fused argmax), the
// embedding dequant gather and the exact block-dot probe.
//
// Numerics follow the reference's x86 scalar path (Q8Scalar.cpp:192-199):
// per output element, blocks are visited in order b = 0..B-1 and
//   acc = acc + f32(I_b) * (sa_b * dw_b)
// with separate roundings.  The GEMV keeps that order exactly: the 16 lanes
// that own one row pass the running sum along with a DPP row rotation, so the
// f32 result is bit-identical to the scalar reference.  Build with
// -ffp-contract=off so the compiler does not fuse the multiply and the add.
#include "q8_kernels.h"

#include <math.h>

namespace llmcp_q8 {
namespace {

__device__ __forceinline__ float half_bits_to_float(uint32_t bits) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

__device__ __forceinline__ uint16_t float_to_half_bits(float v) {
  return __builtin_bit_cast(uint16_t, (_Float16)v);  // v_cvt_f16_f32: RNE
}

// Correctly rounded f32 exp via f64: the same definition the oracle uses.
__device__ __forceinline__ float exp_f32(float v) {
  return (float)exp((double)v);
}

// applyMatmulActivation "silu" (MatmulLoweringCommon.cpp:85-92).
__device__ __forceinline__ float silu(float v) {
  float e = exp_f32(-v);
  float sig = 1.0f / (1.0f + e);
  return v * sig;
}

__device__ __forceinline__ int dot8(const uint4 &w, const uint4 &a, int acc) {
  acc = __builtin_amdgcn_sdot4((int)w.x, (int)a.x, acc, false);
  acc = __builtin_amdgcn_sdot4((int)w.y, (int)a.y, acc, false);
  acc = __builtin_amdgcn_sdot4((int)w.z, (int)a.z, acc, false);
  acc = __builtin_amdgcn_sdot4((int)w.w, (int)a.w, acc, false);
  return acc;
}

// DPP row_ror:1 -- lane i of each 16-lane row receives lane (i-1) mod 16.
__device__ __forceinline__ float row_rotate1(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x121,
                                         0xf, 0xf, false));
}

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
  uint8_t *pass = out + (g * passes + b / kPassBlocks) * kPassBytes;
  const int j = (int)(b % kPassBlocks);
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

// --------------------------------------------- activation quantizer ---- //

// Quantizes 8 blocks per wave instruction: 8 lanes x float4 per block.
// Q8Decode.cpp:83-120: sa = max|x|/127; inv = max==0 ? 0 : 1/sa;
// q = (int8)(int32)roundeven(x*inv).
__device__ __forceinline__ void quantize_block8(float4 v, bool valid,
                                                int lane, int32_t *q_out,
                                                float *s_out) {
  if (!valid) v = make_float4(0.f, 0.f, 0.f, 0.f);
  float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
  m = fmaxf(m, __shfl_xor(m, 1));
  m = fmaxf(m, __shfl_xor(m, 2));
  m = fmaxf(m, __shfl_xor(m, 4));
  const float s = m / 127.0f;
  const float inv = m == 0.0f ? 0.0f : 1.0f / s;
  const int q0 = (int)rintf(v.x * inv), q1 = (int)rintf(v.y * inv);
  const int q2 = (int)rintf(v.z * inv), q3 = (int)rintf(v.w * inv);
  *q_out = (int32_t)((uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) |
                     ((uint32_t)(q2 & 0xff) << 16) |
                     ((uint32_t)(q3 & 0xff) << 24));
  if ((lane & 7) == 0) *s_out = s;
}

__device__ __forceinline__ float4 load_float4(const float *p, bool aligned) {
  if (aligned) return *(const float4 *)p;
  return make_float4(p[0], p[1], p[2], p[3]);
}

// Grid: x covers (row, padded block) in units of 8 blocks per wave.
__global__ void quantize_kernel(const float *__restrict__ x, int64_t m,
                                int64_t ldx, int64_t blocks, int8_t *qa,
                                int64_t ldq, float *sa, int64_t lds,
                                int64_t blocks_pad, int aligned) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t blk_all = t >> 3;  // global (row, block) index
  const int lane = threadIdx.x & 63;
  const int64_t row = blk_all / blocks_pad;
  const int64_t blk = blk_all - row * blocks_pad;
  const bool in_range = row < m;
  const bool valid = in_range && blk < blocks;
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (valid)
    v = load_float4(x + row * ldx + blk * kBlock + (lane & 7) * 4, aligned);
  int32_t q;
  float s;
  quantize_block8(v, valid, lane, &q, &s);
  if (in_range) {
    *(int32_t *)(qa + row * ldq + blk * kBlock + (lane & 7) * 4) = q;
    if ((lane & 7) == 0) sa[row * lds + blk] = s;
  }
}

// --------------------------------------------------------------- GEMV -- //

struct GemvArgs {
  const float *x;    // IN_WAVE / IN_WG: f32 input row, 16 B aligned
  const int8_t *qa;  // IN_PRE: Q8_1 input, padded to passes * 16 blocks
  const float *sa;
  const uint8_t *w0;
  const uint8_t *w1;
  float *y;
  unsigned long long *keys;  // ARGMAX: one (value, index) key per workgroup
  int8_t *qout;              // QOUT: Q8_1 of y, [rows] bytes + [rows/32] scales
  float *sout;
  int64_t groups;
  int32_t blocks;
  int32_t passes;
};

// Where the GEMV's input row comes from.
enum InputMode {
  IN_PRE = 0,   // pre-quantized Q8_1 row in global memory
  IN_WAVE = 1,  // f32 row, each wave quantizes its blocks in the pass loop
  IN_WG = 2     // f32 row, each workgroup quantizes it once into LDS
};

// Total order on (logit, index) whose maximum is the first maximum:
// order-preserving float bits (with -0 folded into +0, which compare equal)
// in the high word, the complemented index in the low word.
__device__ __forceinline__ unsigned long long argmax_key(float v,
                                                         int64_t idx) {
  uint32_t bits = __builtin_bit_cast(uint32_t, v == 0.0f ? 0.0f : v);
  const uint32_t ord = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
  return ((unsigned long long)ord << 32) |
         (unsigned long long)(0xFFFFFFFFu - (uint32_t)idx);
}

__device__ __forceinline__ uint32_t pack4(float a, float b, float c, float d,
                                          float inv) {
  const int q0 = (int)rintf(a * inv), q1 = (int)rintf(b * inv);
  const int q2 = (int)rintf(c * inv), q3 = (int)rintf(d * inv);
  return (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) |
         ((uint32_t)(q2 & 0xff) << 16) | ((uint32_t)(q3 & 0xff) << 24);
}

// Q8_1 of one 32-value block spread over the four lanes j, j+16, j+32, j+48
// (lane 16r + j holds values 8r..8r+7): the same arithmetic as
// Q8Decode.cpp:83-120, then every lane gathers the block's 8 words.
__device__ __forceinline__ void quantize_shared_block(const uint4 &b0,
                                                      const uint4 &b1, int j,
                                                      uint4 &a0, uint4 &a1,
                                                      float &s_out) {
  const float4 v0 = __builtin_bit_cast(float4, b0);
  const float4 v1 = __builtin_bit_cast(float4, b1);
  float m = fmaxf(fmaxf(fmaxf(fabsf(v0.x), fabsf(v0.y)),
                        fmaxf(fabsf(v0.z), fabsf(v0.w))),
                  fmaxf(fmaxf(fabsf(v1.x), fabsf(v1.y)),
                        fmaxf(fabsf(v1.z), fabsf(v1.w))));
  m = fmaxf(m, __shfl_xor(m, 16));
  m = fmaxf(m, __shfl_xor(m, 32));
  const float s = m / 127.0f;
  const float inv = m == 0.0f ? 0.0f : 1.0f / s;
  const uint32_t lo = pack4(v0.x, v0.y, v0.z, v0.w, inv);
  const uint32_t hi = pack4(v1.x, v1.y, v1.z, v1.w, inv);
  a0.x = (uint32_t)__shfl((int)lo, j);
  a0.y = (uint32_t)__shfl((int)hi, j);
  a0.z = (uint32_t)__shfl((int)lo, j + 16);
  a0.w = (uint32_t)__shfl((int)hi, j + 16);
  a1.x = (uint32_t)__shfl((int)lo, j + 32);
  a1.y = (uint32_t)__shfl((int)hi, j + 32);
  a1.z = (uint32_t)__shfl((int)lo, j + 48);
  a1.w = (uint32_t)__shfl((int)hi, j + 48);
  s_out = s;
}

// One wave per lane group (4 rows); lane L = 16r + j owns row 4g+r and the
// blocks 16p + j of every pass p.  Each lane streams its weights (and, for
// IN_PRE / IN_WAVE, its activation block) through a ring of D passes in
// flight.
//   IN    where the input row comes from (InputMode).
//   QOUT  y is also quantized to Q8_1 for the next GEMV.  Needs 8 waves per
//         workgroup: the workgroup owns one 32-row output block and
//         quantizes it through LDS.
//   PC>0  the pass count is a compile-time constant and the pass sequence
//         is fully unrolled, so every wait on the ring is exact.
template <int NMAT, int ACT, bool ARGMAX, int IN, bool QOUT, int D, int PC>
__global__ __launch_bounds__(512) void gemv_kernel(GemvArgs a) {
  extern __shared__ __align__(16) unsigned char lds[];  // IN_WG input row
  __shared__ unsigned long long key_l[8];
  __shared__ float y_l[kBlock];
  __shared__ unsigned count_l;
  if (QOUT && threadIdx.x == 0) count_l = 0;
  const int passes = PC > 0 ? PC : a.passes;
  const int nblk = passes * kPassBlocks;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int waves = blockDim.x >> 6;
  const int64_t g = (int64_t)blockIdx.x * waves + wave;
  const bool active = g < a.groups;
  const int j = lane & 15;
  const int r = lane >> 4;
  int8_t *qa_l = (int8_t *)lds;
  float *sa_l = (float *)(lds + nblk * kBlock);

  const unsigned char *base[NMAT];
  base[0] = a.w0 + g * passes * kPassBytes;
  if (NMAT == 2) base[NMAT - 1] = a.w1 + g * passes * kPassBytes;

  uint4 q0[NMAT][D], q1[NMAT][D], x0[D], x1[D];
  uint32_t sc[NMAT][D];
  float xs[D];
  auto issue = [&](int slot, int p) {
    const int pc = p < passes ? p : passes - 1;
#pragma unroll
    for (int mm = 0; mm < NMAT; ++mm) {
      const unsigned char *pb = base[mm] + (int64_t)pc * kPassBytes;
      q0[mm][slot] = *(const uint4 *)(pb + lane * 16);
      q1[mm][slot] = *(const uint4 *)(pb + 1024 + lane * 16);
      sc[mm][slot] = *(const uint16_t *)(pb + kPassQs + lane * 2);
    }
    // Raw loads only: any use of the loaded values here (even a select)
    // would make the wave wait for them and drain the ring.  Padded blocks
    // (blk >= blocks) are masked in consume().
    const int blk = pc * kPassBlocks + j;
    if (IN == IN_WAVE) {
      const float *xp = a.x + (blk < a.blocks ? blk * kBlock + 8 * r : 0);
      x0[slot] = *(const uint4 *)xp;
      x1[slot] = *(const uint4 *)(xp + 4);
    } else if (IN == IN_PRE) {
      x0[slot] = *(const uint4 *)(a.qa + blk * kBlock);
      x1[slot] = *(const uint4 *)(a.qa + blk * kBlock + 16);
      xs[slot] = a.sa[blk];
    }
  };

  float acc[NMAT];
#pragma unroll
  for (int mm = 0; mm < NMAT; ++mm) acc[mm] = 0.0f;

  // Pass p in ring slot d: exact block dots, scale, then the serial chain
  // over the pass's 16 blocks in block order -- after step t, lane t of each
  // row holds the running sum through block 16p + t; lane 15 carries it
  // into the next pass.
  auto consume = [&](int d, int p) {
    uint4 a0, a1;
    float s_a;
    const int blk = p * kPassBlocks + j;
    const bool valid = blk < a.blocks;  // padded blocks: zero input
    if (IN == IN_WAVE) {
      const uint4 z = make_uint4(0, 0, 0, 0);
      quantize_shared_block(valid ? x0[d] : z, valid ? x1[d] : z, j, a0, a1,
                            s_a);
    } else if (IN == IN_PRE) {
      a0 = x0[d];
      a1 = x1[d];
      s_a = valid ? xs[d] : 0.0f;
    } else {
      a0 = *(const uint4 *)(qa_l + blk * kBlock);
      a1 = *(const uint4 *)(qa_l + blk * kBlock + 16);
      s_a = sa_l[blk];
    }
    float contrib[NMAT];
#pragma unroll
    for (int mm = 0; mm < NMAT; ++mm) {
      int dot = dot8(q0[mm][d], a0, 0);
      dot = dot8(q1[mm][d], a1, dot);
      const float factor = s_a * half_bits_to_float(sc[mm][d]);
      contrib[mm] = (float)dot * factor;
    }
#pragma unroll
    for (int t = 0; t < kPassBlocks; ++t) {
#pragma unroll
      for (int mm = 0; mm < NMAT; ++mm)
        acc[mm] = row_rotate1(acc[mm]) + contrib[mm];
    }
  };

  // sched_barrier(0) pins each refill right after the pass that frees its
  // slot; without it the scheduler sinks the loads toward their uses and
  // only about one pass stays in flight.
  if (active) {
#pragma unroll
    for (int d = 0; d < D; ++d) issue(d, d);
  }
  __builtin_amdgcn_sched_barrier(0);

  if (IN == IN_WG) {
    // Quantize the whole input row into LDS once per workgroup, 8 lanes per
    // block, four blocks' loads in flight per lane (the weight ring above
    // is already on its way).
    constexpr int U = 4;
    const int tasks = nblk * 8;
    for (int t0 = 0; t0 < tasks; t0 += (int)blockDim.x * U) {
      float4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int t = t0 + u * (int)blockDim.x + (int)threadIdx.x;
        const int blk = t >> 3;
        v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (blk < a.blocks) v[u] = *(const float4 *)(a.x + blk * kBlock + (t & 7) * 4);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int t = t0 + u * (int)blockDim.x + (int)threadIdx.x;
        const int blk = t >> 3;
        int32_t q;
        float sq = 0.0f;
        quantize_block8(v[u], blk < a.blocks, lane, &q, &sq);
        if (blk < nblk) {
          ((int32_t *)qa_l)[t] = q;
          if ((t & 7) == 0) sa_l[blk] = sq;
        }
      }
    }
    __syncthreads();
  }

  if (active) {
    if constexpr (PC > 0) {
#pragma unroll
      for (int p = 0; p < PC; ++p) {
        consume(p % D, p);
        __builtin_amdgcn_sched_barrier(0);
        if (p + D < PC) issue(p % D, p + D);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      for (int p0 = 0; p0 < passes; p0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
          if (p0 + d < passes) {
            consume(d, p0 + d);
            __builtin_amdgcn_sched_barrier(0);
            issue(d, p0 + d + D);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
    }
  }

  const int64_t row = g * kLanes + r;
  float y;
  if (NMAT == 2)
    y = silu(acc[0]) * acc[NMAT - 1];
  else
    y = ACT == 1 ? silu(acc[0]) : acc[0];
  const bool owner = active && j == 15;
  if (owner) a.y[row] = y;

  if (QOUT) {
    // The workgroup's 8 waves produced output rows 32*blockIdx.x .. +31.
    // The last wave to finish (LDS arrival count, no barrier, so finished
    // waves leave at once) quantizes that block (Q8Decode.cpp:83-120).
    if (owner) y_l[wave * kLanes + r] = y;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    unsigned arrived = 0;
    if (lane == 0) arrived = atomicAdd(&count_l, 1u);
    arrived = (unsigned)__shfl((int)arrived, 0);
    if (arrived == (unsigned)waves - 1) {
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
      const float v = lane < kBlock ? y_l[lane] : 0.0f;
      float m = fabsf(v);
#pragma unroll
      for (int off = 1; off < 32; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
      const float sq = m / 127.0f;
      const float inv = m == 0.0f ? 0.0f : 1.0f / sq;
      if (lane < kBlock)
        a.qout[(int64_t)blockIdx.x * kBlock + lane] = (int8_t)(int)rintf(v * inv);
      if (lane == 0) a.sout[blockIdx.x] = sq;
    }
  }

  if (ARGMAX) {
    unsigned long long key = owner ? argmax_key(y, row) : 0ull;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const unsigned long long other = __shfl_xor(key, off);
      key = other > key ? other : key;
    }
    if (lane == 0) key_l[wave] = key;
    __syncthreads();
    if (threadIdx.x == 0) {
      unsigned long long best = key_l[0];
      for (int w = 1; w < waves; ++w) best = key_l[w] > best ? key_l[w] : best;
      a.keys[blockIdx.x] = best;
    }
  }
}

// Second stage of the fused argmax: one workgroup reduces the per-workgroup
// keys and writes the index of the first maximum.  Loads are issued 16 deep
// per thread so the pass costs one memory latency.
__global__ __launch_bounds__(1024) void argmax_reduce_kernel(
    const unsigned long long *__restrict__ keys, int64_t n, int64_t *out) {
  __shared__ unsigned long long part[16];
  unsigned long long best = 0ull;
  for (int64_t i0 = 0; i0 < n; i0 += 16 * 1024) {
    unsigned long long k[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int64_t i = i0 + u * 1024 + threadIdx.x;
      k[u] = i < n ? keys[i] : 0ull;
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) best = k[u] > best ? k[u] : best;
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const unsigned long long other = __shfl_xor(best, off);
    best = other > best ? other : best;
  }
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w)
      best = part[w] > best ? part[w] : best;
    *out = (int64_t)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFull));
  }
}

// ---------------------------------------------------------- embedding -- //

// One thread per (token, 16 columns) -- LowerToLinalg.cpp:435-531 gathered
// from the pass layout.  out = f32(q) * f32(d), exact.
__global__ void embedding_kernel(const int64_t *__restrict__ tokens,
                                 int64_t count, const uint8_t *__restrict__ t,
                                 int64_t rows, int64_t passes, int64_t chunks,
                                 float *__restrict__ out, int64_t ldo,
                                 int32_t *err, int aligned) {
  const int64_t c16 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t ti = blockIdx.y;
  if (c16 >= chunks || ti >= count) return;
  const int64_t tok = tokens[ti];
  float v[16];
  if (tok < 0 || tok >= rows) {
#pragma unroll
    for (int e = 0; e < 16; ++e) v[e] = 0.0f;
    if (c16 == 0) atomicOr(err, 1);
  } else {
    const int64_t g = tok >> 2;
    const int r = (int)(tok & 3);
    const int64_t b = c16 >> 1;
    const int h = (int)(c16 & 1);
    const int j = (int)(b % kPassBlocks);
    const uint8_t *pass = t + (g * passes + b / kPassBlocks) * kPassBytes;
    const uint4 q = *(const uint4 *)(pass + h * 1024 + r * 256 + j * 16);
    const float d = half_bits_to_float(
        *(const uint16_t *)(pass + kPassQs + 2 * (16 * r + j)));
    const uint32_t words[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int e = 0; e < 16; ++e)
      v[e] = (float)(int8_t)(words[e >> 2] >> (8 * (e & 3))) * d;
  }
  float *o = out + ti * ldo + c16 * 16;
  if (aligned) {
#pragma unroll
    for (int e = 0; e < 16; e += 4)
      *(float4 *)(o + e) = make_float4(v[e], v[e + 1], v[e + 2], v[e + 3]);
  } else {
#pragma unroll
    for (int e = 0; e < 16; ++e) o[e] = v[e];
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
  const int j = (int)(b % kPassBlocks);
  const uint8_t *pass = w + (g * passes + b / kPassBlocks) * kPassBytes;
  const uint4 w0 = *(const uint4 *)(pass + r * 256 + j * 16);
  const uint4 w1 = *(const uint4 *)(pass + 1024 + r * 256 + j * 16);
  const int8_t *arow = qa + mi * ldq + b * kBlock;
  uint4 a0, a1;
  __builtin_memcpy(&a0, arow, 16);
  __builtin_memcpy(&a1, arow + 16, 16);
  out[t] = dot8(w1, a1, dot8(w0, a0, 0));
}

inline unsigned grid_for(int64_t threads, int block) {
  return (unsigned)((threads + block - 1) / block);
}

template <int NMAT, int ACT, bool ARGMAX, int IN, bool QOUT, int PC>
hipError_t launch_gemv_p(const GemvArgs &args, int waves, hipStream_t s) {
  constexpr int DMAX = NMAT == 2 ? 4 : 12;
  constexpr int D = PC > 0 ? (PC < DMAX ? PC : DMAX) : (NMAT == 2 ? 4 : 8);
  const unsigned grid = (unsigned)((args.groups + waves - 1) / waves);
  const size_t lds = IN == IN_WG ? (size_t)args.passes * kPassBlocks * (kBlock + 4) : 0;
  hipLaunchKernelGGL((gemv_kernel<NMAT, ACT, ARGMAX, IN, QOUT, D, PC>),
                     dim3(grid), dim3(64 * waves), lds, s, args);
  return hipGetLastError();
}

// Pass counts with a fully unrolled kernel: K = 512, 1024, 1536, 2560
// (hidden size), 4096 and 9216 (the MLP down projection).  Others take the
// runtime loop.
template <int NMAT, int ACT, bool ARGMAX, int IN, bool QOUT>
hipError_t launch_gemv_t(const GemvArgs &args, int waves, hipStream_t s) {
  switch (args.passes) {
    case 1: return launch_gemv_p<NMAT, ACT, ARGMAX, IN, QOUT, 1>(args, waves, s);
    case 2: return launch_gemv_p<NMAT, ACT, ARGMAX, IN, QOUT, 2>(args, waves, s);
    case 3: return launch_gemv_p<NMAT, ACT, ARGMAX, IN, QOUT, 3>(args, waves, s);
    case 5: return launch_gemv_p<NMAT, ACT, ARGMAX, IN, QOUT, 5>(args, waves, s);
    case 8: return launch_gemv_p<NMAT, ACT, ARGMAX, IN, QOUT, 8>(args, waves, s);
    case 18: return launch_gemv_p<NMAT, ACT, ARGMAX, IN, QOUT, 18>(args, waves, s);
    default: return launch_gemv_p<NMAT, ACT, ARGMAX, IN, QOUT, 0>(args, waves, s);
  }
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

hipError_t launch_quantize(const float *x, int64_t m, int64_t ldx,
                           int64_t cols, int8_t *qa, int64_t ldq, float *sa,
                           int64_t lds, int64_t blocks_pad, hipStream_t s) {
  const int64_t blocks = cols / kBlock;
  const int64_t threads = m * blocks_pad * 8;
  const int aligned =
      ((uintptr_t)x % 16 == 0) && (ldx % 4 == 0) ? 1 : 0;
  hipLaunchKernelGGL(quantize_kernel, dim3(grid_for(threads, 256)), dim3(256),
                     0, s, x, m, ldx, blocks, qa, ldq, sa, lds, blocks_pad,
                     aligned);
  return hipGetLastError();
}

// Launch shape of a one-row GEMV over `rows` outputs.
//   fused MLP gate/up (quantized output)   8 waves, input quantized per WG
//   wide SwiGLU (>= 2048 groups)           8 waves, input quantized per WG
//   <= kInLoopQuantMaxGroups groups        1 wave,  input quantized per wave
//   wider (lm_head)                        4 waves, pre-quantized input
struct GemvShape {
  int waves;
  int in;
};

static GemvShape gemv_shape(int64_t rows, int nmat, bool qout, bool have_x) {
  const int64_t groups = rows / kLanes;
  if (have_x && (qout || (nmat == 2 && groups >= 2048))) return {8, IN_WG};
  if (have_x) return {1, IN_WAVE};
  return {groups >= 8192 ? 4 : 1, IN_PRE};
}

bool gemv_quantizes_input(int64_t rows, int nmat) {
  return nmat == 2 || rows / kLanes <= kInLoopQuantMaxGroups;
}

int64_t gemv_workgroups(int64_t rows) {
  // Argmax partials are only used by one-matrix GEMVs without QOUT.
  const int64_t groups = rows / kLanes;
  const int w = gemv_quantizes_input(rows, 1) ? 1 : (groups >= 8192 ? 4 : 1);
  return (groups + w - 1) / w;
}

template <int IN>
static hipError_t launch_gemv_in(const GemvArgs &a, const GemvLaunch &l,
                                 int waves, hipStream_t s) {
  if (l.nmat == 2) {
    if (IN == IN_WG && l.qout) return launch_gemv_t<2, 0, false, IN, true>(a, waves, s);
    return launch_gemv_t<2, 0, false, IN, false>(a, waves, s);
  }
  if (IN == IN_WG) return hipErrorInvalidValue;  // one-matrix GEMVs use WAVE/PRE
  if (l.keys) return launch_gemv_t<1, 0, true, IN, false>(a, waves, s);
  if (l.activation == 1) return launch_gemv_t<1, 1, false, IN, false>(a, waves, s);
  return launch_gemv_t<1, 0, false, IN, false>(a, waves, s);
}

hipError_t launch_gemv(const GemvLaunch &l, hipStream_t s) {
  GemvArgs a;
  a.x = l.x;
  a.qa = l.qa;
  a.sa = l.sa;
  a.w0 = l.w[0];
  a.w1 = l.w[1] ? l.w[1] : l.w[0];
  a.y = l.y;
  a.keys = l.keys;
  a.qout = l.qout;
  a.sout = l.sout;
  a.groups = l.rows / kLanes;
  a.blocks = (int32_t)(l.cols / kBlock);
  a.passes = (int32_t)passes_for(l.cols);
  const GemvShape sh = gemv_shape(l.rows, l.nmat, l.qout != nullptr, l.x != nullptr);
  if (l.qout && (sh.in != IN_WG || l.rows % kBlock)) return hipErrorInvalidValue;
  hipError_t e;
  if (sh.in == IN_WG)
    e = launch_gemv_in<IN_WG>(a, l, sh.waves, s);
  else if (sh.in == IN_WAVE)
    e = launch_gemv_in<IN_WAVE>(a, l, sh.waves, s);
  else
    e = launch_gemv_in<IN_PRE>(a, l, sh.waves, s);
  if (e != hipSuccess || !l.keys) return e;
  hipLaunchKernelGGL(argmax_reduce_kernel, dim3(1), dim3(1024), 0, s,
                     (const unsigned long long *)l.keys,
                     (a.groups + sh.waves - 1) / sh.waves, l.argmax_out);
  return hipGetLastError();
}

hipError_t launch_embedding(const int64_t *tokens, int64_t count,
                            const uint8_t *table, int64_t rows, int64_t cols,
                            float *out, int64_t ldo, int32_t *err_flag,
                            hipStream_t s) {
  if (count == 0) return hipSuccess;
  const int64_t chunks = cols / 16;
  const int aligned = ((uintptr_t)out % 16 == 0) && (ldo % 4 == 0) ? 1 : 0;
  hipLaunchKernelGGL(embedding_kernel,
                     dim3(grid_for(chunks, 256), (unsigned)count), dim3(256),
                     0, s, tokens, count, table, rows, passes_for(cols),
                     chunks, out, ldo, err_flag, aligned);
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
