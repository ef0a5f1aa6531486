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

#include <algorithm>

#include "q8_device.h"

namespace llmcp_q8 {
namespace {

__device__ __forceinline__ uint32_t word(const uint4 &v, int k) {
  return k == 0 ? v.x : (k == 1 ? v.y : (k == 2 ? v.z : v.w));
}

__device__ __forceinline__ int dot8(const uint4 &w, const uint4 &a, int acc) {
  acc = __builtin_amdgcn_sdot4((int)w.x, (int)a.x, acc, false);
  acc = __builtin_amdgcn_sdot4((int)w.y, (int)a.y, acc, false);
  acc = __builtin_amdgcn_sdot4((int)w.z, (int)a.z, acc, false);
  acc = __builtin_amdgcn_sdot4((int)w.w, (int)a.w, acc, false);
  return acc;
}

// Lane permutation by DPP control word (quad_perm 0x00-0xFF, row ops above).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                         0xf, 0xf, false));
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

// --------------------------------------------- activation quantizer ---- //

// RN(m / 127) for m >= 0: m * RN(1/127) and one FMA correction.  The
// identity holds for every finite non-negative float (checked exhaustively;
// the device self-test repeats the check); +inf is passed through.
__device__ __forceinline__ float div127(float m) {
  constexpr float c = 1.0f / 127.0f;
  const float q = m * c;
  const float r = __builtin_fmaf(-q, 127.0f, m);
  const float s = __builtin_fmaf(r, c, q);
  return m == __builtin_inff() ? m : s;
}

// recip_in_range / recip_fast (RN(1 / s) on [2^-125, 2^126]): q8_device.h.
__device__ __forceinline__ float recip(float s) {
  return recip_in_range(s) ? recip_fast(s) : 1.0f / s;
}

// Low byte of roundeven(x) for |x| < 2^22: adding 1.5 * 2^23 rounds to an
// integer (round to nearest even) and leaves it, two's complement, in the
// low mantissa bits.  A NaN yields 0, as the integer conversion does.
__device__ __forceinline__ uint32_t round_byte(float x) {
  return __builtin_bit_cast(uint32_t, x + 12582912.0f) & 0xffu;
}

// Quantizes 8 blocks per wave instruction: 8 lanes x float4 per block.
// Q8Decode.cpp:83-120: sa = max|x|/127; inv = max==0 ? 0 : 1/sa;
// q = (int8)(int32)roundeven(x*inv).  The fast form takes the reciprocal
// from recip_fast and returns true in lanes whose scale is outside its
// exact range (extreme magnitudes only); such a block must be redone with
// quantize_block8.
__device__ __forceinline__ bool quantize_block8_fast(float4 v, int32_t *q_out,
                                                     float *s_out) {
  float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
  // max over the 8 lanes of the block with DPP (no LDS round trips): swap
  // neighbours, swap pairs, then mirror each half-row (lane i <-> 7 - i).
  m = fmaxf(m, dpp_f32<0xB1>(m));
  m = fmaxf(m, dpp_f32<0x4E>(m));
  m = fmaxf(m, dpp_f32<0x141>(m));
  const float s = div127(m);
  const bool zero = m == 0.0f;
  const float inv = zero ? 0.0f : recip_fast(s);
  *q_out = (int32_t)(round_byte(v.x * inv) | (round_byte(v.y * inv) << 8) |
                     (round_byte(v.z * inv) << 16) | (round_byte(v.w * inv) << 24));
  *s_out = s;  // the same in all 8 lanes of the block
  return !zero && !recip_in_range(s);
}
__device__ __forceinline__ void quantize_block8(float4 v, bool valid,
                                                int32_t *q_out, float *s_out) {
  if (!valid) v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (__builtin_amdgcn_ballot_w64(quantize_block8_fast(v, q_out, s_out))) {
    // rare: an extreme scale somewhere in the wave
    float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    m = fmaxf(m, dpp_f32<0xB1>(m));
    m = fmaxf(m, dpp_f32<0x4E>(m));
    m = fmaxf(m, dpp_f32<0x141>(m));
    const float s = div127(m);
    const float inv = m == 0.0f ? 0.0f : recip(s);
    *q_out = (int32_t)(round_byte(v.x * inv) | (round_byte(v.y * inv) << 8) |
                       (round_byte(v.z * inv) << 16) | (round_byte(v.w * inv) << 24));
  }
}

// Four consecutive activations as f32: an f32 row (one float4 when 16 B
// aligned) or a bf16 row (widened exactly, one 8 B load when aligned).
__device__ __forceinline__ float4 load_act4(const void *p, int64_t i,
                                            bool bf16, bool aligned) {
  if (bf16) {
    const uint16_t *h = (const uint16_t *)p + i;
    if (aligned) {
      const uint2 w = *(const uint2 *)h;
      return make_float4(bf16_to_float(w.x & 0xffffu), bf16_to_float(w.x >> 16),
                         bf16_to_float(w.y & 0xffffu), bf16_to_float(w.y >> 16));
    }
    return make_float4(bf16_to_float(h[0]), bf16_to_float(h[1]),
                       bf16_to_float(h[2]), bf16_to_float(h[3]));
  }
  const float *f = (const float *)p + i;
  if (aligned) return *(const float4 *)f;
  return make_float4(f[0], f[1], f[2], f[3]);
}

// load_act4 with the row type and alignment fixed at compile time: one
// straight-line load, so several of them stay in flight together.
template <bool BF16, bool ALIGNED>
__device__ __forceinline__ float4 load_act4_t(const void *p, int64_t i) {
  if constexpr (BF16) {
    const uint16_t *h = (const uint16_t *)p + i;
    if constexpr (ALIGNED) {
      const uint2 w = *(const uint2 *)h;
      return make_float4(bf16_to_float(w.x & 0xffffu), bf16_to_float(w.x >> 16),
                         bf16_to_float(w.y & 0xffffu), bf16_to_float(w.y >> 16));
    }
    return make_float4(bf16_to_float(h[0]), bf16_to_float(h[1]),
                       bf16_to_float(h[2]), bf16_to_float(h[3]));
  } else {
    const float *f = (const float *)p + i;
    if constexpr (ALIGNED) return *(const float4 *)f;
    return make_float4(f[0], f[1], f[2], f[3]);
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

// Grid: x covers (row, padded block) in units of 8 blocks per wave.
__global__ void quantize_kernel(const void *__restrict__ x, int x_bf16,
                                int64_t m, int64_t ldx, int64_t blocks,
                                int8_t *qa, int64_t ldq, float *sa,
                                int64_t lds, int64_t blocks_pad, int aligned) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t blk_all = t >> 3;  // global (row, block) index
  const int lane = threadIdx.x & 63;
  const int64_t row = blk_all / blocks_pad;
  const int64_t blk = blk_all - row * blocks_pad;
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

// --------------------------------------------------------------- GEMV -- //

struct GemvArgs {
  const void *x;     // IN_WG: input row, f32 (16 B aligned) or bf16 (8 B)
  const int8_t *qa;  // IN_PRE: Q8_1 input, padded to passes * 16 blocks
  const float *sa;
  const uint8_t *w0;
  const uint8_t *w1;
  void *y;           // output row, f32 or bf16
  const void *r;     // V bit 3: the residual row (y's element type)
  unsigned long long *keys;  // ARGMAX: kArgmaxSlots slots folded into
  int64_t groups;
  int32_t blocks;
  int32_t passes;
  int32_t act;       // llmcp_q8_activation (one-matrix GEMVs)
};

// Where the GEMV's input row comes from.
enum InputMode {
  IN_PRE = 0,  // pre-quantized Q8_1 row in global memory
  IN_WG = 1    // f32 row, each workgroup quantizes it once into LDS
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

__device__ __forceinline__ unsigned long long max_u64(unsigned long long a,
                                                      unsigned long long b) {
  return a > b ? a : b;
}

// DPP move of a 64-bit value (both halves with the same control; lanes with
// no source read 0, the identity of an unsigned max).
template <int CTRL>
__device__ __forceinline__ unsigned long long dpp_u64(unsigned long long v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(
      0, (int)(uint32_t)v, CTRL, 0xf, 0xf, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(
      0, (int)(uint32_t)(v >> 32), CTRL, 0xf, 0xf, false);
  return ((unsigned long long)hi << 32) | lo;
}

// Maximum over the wave, returned in every lane: quad swaps, row shifts by
// 4 and 8 (lane 15 of each row holds the row's maximum), then row_bcast:15
// and row_bcast:31 carry it into lane 63.
__device__ __forceinline__ unsigned long long wave_max_u64(
    unsigned long long v) {
  v = max_u64(v, dpp_u64<0xb1>(v));   // quad_perm [1,0,3,2]
  v = max_u64(v, dpp_u64<0x4e>(v));   // quad_perm [2,3,0,1]
  v = max_u64(v, dpp_u64<0x114>(v));  // row_shr:4
  v = max_u64(v, dpp_u64<0x118>(v));  // row_shr:8
  v = max_u64(v, dpp_u64<0x142>(v));  // row_bcast:15
  v = max_u64(v, dpp_u64<0x143>(v));  // row_bcast:31
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, 63);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), 63);
  return ((unsigned long long)hi << 32) | lo;
}

// Folds a workgroup's best key into slot blockIdx mod kArgmaxSlots.  The
// atomic returns nothing and orders nothing: the reduce kernel that reads
// the slots runs after this kernel has completed.
__device__ __forceinline__ void argmax_fold(unsigned long long *slots,
                                            unsigned long long key) {
  (void)__hip_atomic_fetch_max(slots + (blockIdx.x & (kArgmaxSlots - 1)), key,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Waves per workgroup of an IN_WG GEMV.  The workgroup quantizes the input
// row once (pc * 16 blocks, 8 lanes per block, row_rounds float4 loads per
// lane), so wider workgroups share that work.  Four for every shape: at
// K = 9216 two and eight were 30 % and 13 % slower, at K = 2560 two was 3 %
// slower (one matrix) and three 1 % slower (gate/up).
__host__ __device__ constexpr int wg_waves(int /*nmat*/, int /*pc*/) { return 4; }
__host__ __device__ constexpr int row_rounds(int pc, int w) {
  return (2 * pc + w - 1) / w;
}
// LDS bytes of the quantized row: int8 values + f32 scales per block slot.
__host__ __device__ constexpr int row_slots(int pc, int w) {
  return pc > 0 ? row_rounds(pc, w) * 8 * w : 0;
}

// One wave per lane group (4 rows); lane L = 16r + j owns row 4g+r and the
// blocks 16p + j of every pass p.  W waves per workgroup.  Each lane streams
// its weights (and, for IN_PRE, its activation block) through a ring of D
// passes in flight.
//   IN    where the input row comes from (InputMode).  IN_WG with PC > 0
//         issues the row's loads before the weight ring: loads complete in
//         issue order, so the row is quantized while the ring is in flight.
//   PC>0  the pass count is a compile-time constant and the pass sequence
//         is fully unrolled, so every wait on the ring is exact.
// Per pass, prepare() forms the 16 blocks' contributions and chain() adds
// them in block order; the next pass's prepare() is scheduled together with
// the current chain(), so the dots overlap the serial DPP additions.
// V packs the compile-time variant: bit 0 the input row is bf16 (IN_WG),
// bit 1 the output is bf16, bit 2 a one-matrix GEMV applies a.act, bit 3 a
// one-matrix GEMV adds the residual row a.r to its (rounded) result.
template <int NMAT, bool ARGMAX, int IN, int W, int D, int PC, int V>
__global__ __launch_bounds__(64 * W) void gemv_kernel(GemvArgs a) {
  constexpr bool XB = (V & 1) != 0;
  constexpr bool YB = (V & 2) != 0;
  constexpr bool ACTV = (V & 4) != 0;
  constexpr bool ADD = (V & 8) != 0;
  static_assert(!ADD || (NMAT == 1 && !ARGMAX && !ACTV), "residual add variants");
  extern __shared__ __align__(16) unsigned char lds[];  // IN_WG input row
  __shared__ unsigned long long key_l[W];
  const int passes = PC > 0 ? PC : a.passes;
  const int nblk = passes * kPassBlocks;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t g = (int64_t)blockIdx.x * W + wave;
  const bool active = g < a.groups;
  const int j = lane & 15;
  const int r = lane >> 4;
  // Units (PC or a.passes) of 16 blocks; S of them form one chain pass
  // (seg_for: lane slot j holds S consecutive blocks of the pass).
  constexpr int S = PC > 0 ? seg_for(PC) : 1;
  // Block held by this lane's slot in unit u.
  auto block_of = [&](int u) {
    return (u / S) * (kPassBlocks * S) + S * j + (u % S);
  };
  // IN_WG, compile-time pass count: the row's float4 loads, 8 per block.
  constexpr bool kRowFirst = IN == IN_WG && PC > 0;
  constexpr int XR = kRowFirst ? row_rounds(PC, W) : 1;
  // Block slots in LDS: every task of the unrolled prologue has one (no
  // store is conditional), the runtime prologue covers the padded row.
  const int nslot = kRowFirst ? row_slots(PC, W) : nblk;
  int8_t *qa_l = (int8_t *)lds;
  float *sa_l = (float *)(lds + nslot * kBlock);

  // Raw row words: f32 fills all four, bf16 the first two (4 values).
  uint4 xr[XR];
  if (kRowFirst) {
#pragma unroll
    for (int u = 0; u < XR; ++u) {
      const int t = u * 64 * W + (int)threadIdx.x;
      xr[u] = make_uint4(0, 0, 0, 0);
      if ((t >> 3) < a.blocks) {
        if constexpr (XB) {
          const uint2 w2 = *(const uint2 *)((const uint16_t *)a.x + t * 4);
          xr[u].x = w2.x;
          xr[u].y = w2.y;
        } else {
          xr[u] = *(const uint4 *)((const float *)a.x + t * 4);
        }
      }
    }
  }

  // Waves past the last group stream the last group again (results unused)
  // so that the loads below are unconditional: a branch around them would
  // make the compiler wait for the whole ring at the join.
  const int64_t gl = active ? g : a.groups - 1;
  const unsigned char *base[NMAT];
  base[0] = a.w0 + gl * passes * kPassBytes;
  if (NMAT == 2) base[NMAT - 1] = a.w1 + gl * passes * kPassBytes;

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
    // (blk >= blocks) are masked in prepare().
    if (IN == IN_PRE) {
      const int blk = block_of(pc);
      x0[slot] = *(const uint4 *)(a.qa + blk * kBlock);
      x1[slot] = *(const uint4 *)(a.qa + blk * kBlock + 16);
      xs[slot] = a.sa[blk];
    }
  };

  // sched_barrier(0) pins the ring right after the row loads; without it
  // the scheduler sinks the loads toward their uses and only about one pass
  // stays in flight.
#pragma unroll
  for (int d = 0; d < D; ++d) issue(d, d);
  __builtin_amdgcn_sched_barrier(0);

  if (IN == IN_WG) {
    // Quantize the input row into LDS once per workgroup, 8 lanes per block
    // (blocks past `blocks` become zero).
    if (kRowFirst) {
      // One basic block (no conditional store), so the rounds interleave.
      // Blocks past `blocks` were loaded as zeros.  The fast reciprocal
      // covers every scale but extreme ones; a block with such a scale
      // (flagged per round) is redone exactly after the rounds.
      auto row_value = [&](int u) {
        return XB ? make_float4(bf16_to_float(xr[u].x & 0xffffu),
                                bf16_to_float(xr[u].x >> 16),
                                bf16_to_float(xr[u].y & 0xffffu),
                                bf16_to_float(xr[u].y >> 16))
                  : __builtin_bit_cast(float4, xr[u]);
      };
      bool slow = false;
#pragma unroll
      for (int u = 0; u < XR; ++u) {
        const int t = u * 64 * W + (int)threadIdx.x;
        int32_t q;
        float sq;
        slow |= quantize_block8_fast(row_value(u), &q, &sq);
        ((int32_t *)qa_l)[t] = q;
        sa_l[t >> 3] = sq;
      }
      if (__builtin_amdgcn_ballot_w64(slow)) {
#pragma unroll
        for (int u = 0; u < XR; ++u) {
          const int t = u * 64 * W + (int)threadIdx.x;
          int32_t q;
          float sq;
          quantize_block8(row_value(u), true, &q, &sq);
          ((int32_t *)qa_l)[t] = q;
        }
      }
    } else {
      constexpr int U = 4;
      const int tasks = nblk * 8;
      for (int t0 = 0; t0 < tasks; t0 += 64 * W * U) {
        float4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int t = t0 + u * 64 * W + (int)threadIdx.x;
          v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
          if ((t >> 3) < a.blocks) v[u] = load_act4(a.x, t * 4, XB, true);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int t = t0 + u * 64 * W + (int)threadIdx.x;
          const int blk = t >> 3;
          int32_t q;
          float sq;
          quantize_block8(v[u], blk < a.blocks, &q, &sq);
          if (blk < nblk) {
            ((int32_t *)qa_l)[t] = q;
            if ((t & 7) == 0) sa_l[blk] = sq;
          }
        }
      }
    }
    __syncthreads();
  }

  float acc[NMAT];
#pragma unroll
  for (int mm = 0; mm < NMAT; ++mm) acc[mm] = 0.0f;

  // Contributions of unit u (ring slot d): exact block dots (two
  // independent dot4 chains; integer sums are order-free), then
  // f32(I) * (sa * dw).  Split in three parts so that the next pass's
  // preparation can ride in the current pass's chain (see chain_with).
  struct Next {
    uint4 a0, a1;
    float s_a;
    int d0[NMAT], d1[NMAT];
  };
  auto load_act = [&](int d, int u, Next &n) {
    const int blk = block_of(u);
    if (IN == IN_PRE) {
      n.a0 = x0[d];
      n.a1 = x1[d];
      n.s_a = blk < a.blocks ? xs[d] : 0.0f;  // padded blocks: zero input
    } else {
      n.a0 = *(const uint4 *)(qa_l + blk * kBlock);
      n.a1 = *(const uint4 *)(qa_l + blk * kBlock + 16);
      n.s_a = sa_l[blk];
    }
#pragma unroll
    for (int mm = 0; mm < NMAT; ++mm) n.d0[mm] = n.d1[mm] = 0;
  };
  auto dot_part = [&](int d, int k, Next &n) {
#pragma unroll
    for (int mm = 0; mm < NMAT; ++mm) {
      n.d0[mm] = __builtin_amdgcn_sdot4((int)word(q0[mm][d], k),
                                        (int)word(n.a0, k), n.d0[mm], false);
      n.d1[mm] = __builtin_amdgcn_sdot4((int)word(q1[mm][d], k),
                                        (int)word(n.a1, k), n.d1[mm], false);
    }
  };
  auto finish = [&](int d, Next &n, float (&c)[NMAT]) {
#pragma unroll
    for (int mm = 0; mm < NMAT; ++mm) {
      const int dot = n.d0[mm] + n.d1[mm];
      const float factor = n.s_a * half_bits_to_float(sc[mm][d]);
      c[mm] = (float)dot * factor;
    }
  };
  // All S units of pass p.
  auto prepare = [&](int p, float (&c)[S][NMAT]) {
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const int u = p * S + i;
      Next n;
      load_act(u % D, u, n);
#pragma unroll
      for (int k = 0; k < 4; ++k) dot_part(u % D, k, n);
      finish(u % D, n, c[i]);
    }
  };
  // The serial chain over one pass's 16 lane slots in block order: at step
  // t, slot t takes the running sum from slot t-1 (DPP row rotation) and
  // adds its S blocks in order; after step t, lane t of each row holds the
  // sum through block 16S*p + S*t + S-1, and lane 15 carries it into the
  // next pass.  The next pass's activation reads go out at step 0; its
  // dots and scalings (5 pieces per unit) are spread over steps 4-14, each
  // pinned between chain additions (whose dependent latency they hide) by
  // sched_barrier.  The dots wait for the next pass's weights inside this
  // chain, which costs nothing once the ring has landed.
  auto chain_with = [&](const float (&c)[S][NMAT], bool has_next, int pn,
                        float (&cn)[S][NMAT]) {
    Next n[S];
    if (has_next) {
#pragma unroll
      for (int i = 0; i < S; ++i) load_act((pn * S + i) % D, pn * S + i, n[i]);
    }
#pragma unroll
    for (int t = 0; t < kPassBlocks; ++t) {
#pragma unroll
      for (int mm = 0; mm < NMAT; ++mm)
        acc[mm] = row_rotate1(acc[mm]) + c[0][mm];
#pragma unroll
      for (int i = 1; i < S; ++i) {
#pragma unroll
        for (int mm = 0; mm < NMAT; ++mm) acc[mm] = acc[mm] + c[i][mm];
      }
      if (has_next) {
#pragma unroll
        for (int o = 0; o < 5 * S; ++o) {
          if (4 + (o * 11) / (5 * S) != t) continue;
          const int i = o / 5, k = o % 5;
          const int d = (pn * S + i) % D;
          if (k < 4)
            dot_part(d, k, n[i]);
          else
            finish(d, n[i], cn[i]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  if (active) {
    float cur[S][NMAT], nxt[S][NMAT];
    prepare(0, cur);
    if constexpr (PC > 0) {
      constexpr int NP = PC / S;
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        // refill the slots of this pass's units (prepared already)
#pragma unroll
        for (int i = 0; i < S; ++i) {
          const int u = p * S + i;
          if (u + D < PC) issue(u % D, u + D);
        }
        __builtin_amdgcn_sched_barrier(0);
        chain_with(cur, p + 1 < NP, p + 1, nxt);
#pragma unroll
        for (int i = 0; i < S; ++i)
#pragma unroll
          for (int mm = 0; mm < NMAT; ++mm) cur[i][mm] = nxt[i][mm];
      }
    } else {
      for (int p0 = 0; p0 < passes; p0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
          const int p = p0 + d;
          if (p < passes) {
            issue(d, p + D);
            __builtin_amdgcn_sched_barrier(0);
            chain_with(cur, p + 1 < passes, p + 1, nxt);
#pragma unroll
            for (int mm = 0; mm < NMAT; ++mm) cur[0][mm] = nxt[0][mm];
          }
        }
      }
    }
  }

  const int64_t row = g * kLanes + r;
  // Epilogue (MatmulLoweringCommon.cpp:78-103).  SwiGLU: h = silu(gate) *
  // up; with a bf16 result each linear's output is rounded to bf16 before
  // the bf16 multiply (FuseSiluMul: linear{silu} + mul on bf16 tensors).
  float y;
  if (NMAT == 2) {
    const float gs = silu_f32(acc[0]);
    y = YB ? bf16_to_float(float_to_bf16(gs)) *
                       bf16_to_float(float_to_bf16(acc[NMAT - 1]))
                 : gs * acc[NMAT - 1];
  } else {
    y = ACTV ? activate(acc[0], a.act) : acc[0];
  }
  const bool owner = active && j == 15;
  if (owner) {
    // residual add (AddOpLowering, LowerToLinalg.cpp:359-375): the linear's
    // result as stored, plus r, in f32; bf16 rounds once more
    if constexpr (ADD) {
      if constexpr (YB)
        y = bf16_to_float(float_to_bf16(y)) + bf16_to_float(((const uint16_t *)a.r)[row]);
      else
        y = y + ((const float *)a.r)[row];
    }
    if constexpr (YB)
      ((uint16_t *)a.y)[row] = float_to_bf16(y);
    else
      ((float *)a.y)[row] = y;
  }

  if (ARGMAX) {
    // the key of the value as stored
    const float ys = YB ? bf16_to_float(float_to_bf16(y)) : y;
    unsigned long long key = owner ? argmax_key(ys, row) : 0ull;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const unsigned long long other = __shfl_xor(key, off);
      key = other > key ? other : key;
    }
    if (W == 1) {
      if (lane == 0) argmax_fold(a.keys, key);
    } else {
      if (lane == 0) key_l[wave] = key;
      __syncthreads();
      if (threadIdx.x == 0) {
        unsigned long long best = key_l[0];
#pragma unroll
        for (int w = 1; w < W; ++w) best = key_l[w] > best ? key_l[w] : best;
        argmax_fold(a.keys, best);
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

// One thread per (token, 16 columns), a flat grid over tokens x chunks so
// that every lane has work -- LowerToLinalg.cpp:435-531 gathered from the
// pass layout.  out = f32(q) * f32(d), exact.
__global__ void embedding_kernel(const int64_t *__restrict__ tokens,
                                 int64_t count, const uint8_t *__restrict__ t,
                                 int64_t rows, int64_t passes, int64_t chunks,
                                 void *__restrict__ out, int out_bf16,
                                 int64_t ldo, int32_t *err, int aligned) {
  const int64_t th = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t ti = th / chunks;
  const int64_t c16 = th - ti * chunks;
  if (ti >= count) return;
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
    int64_t u;
    int j;
    locate_seg(b, seg_for(passes), u, j);
    const uint8_t *pass = t + (g * passes + u) * kPassBytes;
    const uint4 q = *(const uint4 *)(pass + h * 1024 + r * 256 + j * 16);
    const float d = half_bits_to_float(
        *(const uint16_t *)(pass + kPassQs + 2 * (16 * r + j)));
    const uint32_t words[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int e = 0; e < 16; ++e)
      v[e] = (float)(int8_t)(words[e >> 2] >> (8 * (e & 3))) * d;
  }
  if (out_bf16) {
    // truncf to a bf16 result (LowerToLinalg.cpp:435-531)
    uint16_t *o = (uint16_t *)out + ti * ldo + c16 * 16;
    uint32_t p[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      p[e] = (uint32_t)float_to_bf16(v[2 * e]) |
             ((uint32_t)float_to_bf16(v[2 * e + 1]) << 16);
    if (aligned) {
      *(uint4 *)o = make_uint4(p[0], p[1], p[2], p[3]);
      *(uint4 *)(o + 8) = make_uint4(p[4], p[5], p[6], p[7]);
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) o[e] = float_to_bf16(v[e]);
    }
    return;
  }
  float *o = (float *)out + ti * ldo + c16 * 16;
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

inline unsigned grid_for(int64_t threads, int block) {
  return (unsigned)((threads + block - 1) / block);
}

// Ring depth: passes in flight per wave.  Two matrices: 4 (72 VGPRs; at
// K = 2560 the fifth pass is issued as the first one is consumed, which
// measured about 1 % faster on the decode MLP than all 5 at once).  One
// matrix from LDS: 4 up to K = 2560 (the 2560 x 2560 GEMV: 3.71 us against
// 3.86 with all 5), else 13 (117 VGPRs; at K = 9216 the down GEMV measured
// 7.46 us against 8.05 with all 18 passes in flight, 7.74 with 12 and
// 7.65-7.82 with 14-16).  One matrix with a pre-quantized row: 12 passes of
// weights + input.
template <int NMAT, int IN, int PC>
constexpr int ring_depth() {
  // at least two passes of units, so the next pass is in flight while the
  // current one chains
  constexpr int two = 2 * seg_for(PC);
  constexpr int base = NMAT == 2 ? 4 : (IN == IN_WG ? (PC <= 5 ? 4 : 13) : 12);
  constexpr int dmax = base > two ? base : two;
  return PC > 0 ? (PC < dmax ? PC : dmax) : (NMAT == 2 ? 4 : 8);
}

template <int NMAT, bool ARGMAX, int IN, int W, int PC, int V>
hipError_t launch_gemv_p(const GemvArgs &args, hipStream_t s) {
  constexpr int D = ring_depth<NMAT, IN, PC>();
  const unsigned grid = (unsigned)((args.groups + W - 1) / W);
  const size_t slots = PC > 0 ? row_slots(PC, W) : (size_t)args.passes * kPassBlocks;
  const size_t lds = IN == IN_WG ? slots * (kBlock + 4) : 0;
  hipLaunchKernelGGL((gemv_kernel<NMAT, ARGMAX, IN, W, D, PC, V>),
                     dim3(grid), dim3(64 * W), lds, s, args);
  return hipGetLastError();
}

// IN_WG takes its workgroup width from wg_waves; IN_PRE (wide outputs)
// runs four waves per workgroup.
template <int NMAT, bool ARGMAX, int IN, int PC, int V>
hipError_t launch_gemv_w(const GemvArgs &args, hipStream_t s) {
  constexpr int W = IN == IN_WG ? wg_waves(NMAT, PC) : 4;
  return launch_gemv_p<NMAT, ARGMAX, IN, W, PC, V>(args, s);
}

// Pass counts with a fully unrolled kernel: K = 512, 1024, 1536, 2560
// (hidden size), 4096 and 9216 (the MLP down projection).  Others take the
// runtime loop.
template <int NMAT, bool ARGMAX, int IN, int V>
hipError_t launch_gemv_t(const GemvArgs &args, hipStream_t s) {
  switch (args.passes) {
    case 1: return launch_gemv_w<NMAT, ARGMAX, IN, 1, V>(args, s);
    case 2: return launch_gemv_w<NMAT, ARGMAX, IN, 2, V>(args, s);
    case 3: return launch_gemv_w<NMAT, ARGMAX, IN, 3, V>(args, s);
    case 5: return launch_gemv_w<NMAT, ARGMAX, IN, 5, V>(args, s);
    case 8: return launch_gemv_w<NMAT, ARGMAX, IN, 8, V>(args, s);
    case 18: return launch_gemv_w<NMAT, ARGMAX, IN, 18, V>(args, s);
    default: return launch_gemv_w<NMAT, ARGMAX, IN, 0, V>(args, s);
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
  hipLaunchKernelGGL(quantize_kernel, dim3(grid_for(threads, 256)), dim3(256),
                     0, s, x, x_bf16 ? 1 : 0, m, ldx, blocks, qa, ldq, sa, lds,
                     blocks_pad, aligned);
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

bool gemv_quantizes_input(int64_t rows, int nmat) {
  return nmat == 2 || rows / kLanes <= kInLoopQuantMaxGroups;
}


// The compile-time variants the C ABI needs (V bits as in gemv_kernel):
// SwiGLU f32 or bf16 in and out; the argmax GEMV (lm_head) with f32 logits
// from an f32 or bf16 row; plain GEMVs with or without an activation, f32 or
// bf16 in and out.  IN_PRE reads an already quantized row (no input type).
template <int IN>
static hipError_t launch_gemv_in(const GemvArgs &a, const GemvLaunch &l,
                                 hipStream_t s) {
  const int xb = (IN == IN_WG && l.x_bf16) ? 1 : 0;
  const int yb = l.y_bf16 ? 2 : 0;
  const int av = (l.nmat == 1 && !l.keys && l.activation != 0) ? 4 : 0;
  const int ad = l.residual ? 8 : 0;
  if (ad && (l.nmat != 1 || l.keys || av)) return hipErrorInvalidValue;
  const int v = xb | yb | av | ad;
  if (l.nmat == 2) {
    if (v == 0) return launch_gemv_t<2, false, IN, 0>(a, s);
    if (v == (IN == IN_WG ? 3 : 2)) return launch_gemv_t<2, false, IN, IN == IN_WG ? 3 : 2>(a, s);
    return hipErrorInvalidValue;
  }
  if (l.keys) {
    if (v == 0) return launch_gemv_t<1, true, IN, 0>(a, s);
    if (IN == IN_WG && v == 1) return launch_gemv_t<1, true, IN, 1>(a, s);
    return hipErrorInvalidValue;
  }
  if (IN == IN_WG) {
    switch (v) {
      case 0: return launch_gemv_t<1, false, IN, 0>(a, s);
      case 3: return launch_gemv_t<1, false, IN, 3>(a, s);
      case 4: return launch_gemv_t<1, false, IN, 4>(a, s);
      case 7: return launch_gemv_t<1, false, IN, 7>(a, s);
      case 8: return launch_gemv_t<1, false, IN, 8>(a, s);
      case 11: return launch_gemv_t<1, false, IN, 11>(a, s);
      default: return hipErrorInvalidValue;
    }
  }
  switch (v) {
    case 0: return launch_gemv_t<1, false, IN, 0>(a, s);
    case 2: return launch_gemv_t<1, false, IN, 2>(a, s);
    case 4: return launch_gemv_t<1, false, IN, 4>(a, s);
    case 6: return launch_gemv_t<1, false, IN, 6>(a, s);
    case 8: return launch_gemv_t<1, false, IN, 8>(a, s);
    case 10: return launch_gemv_t<1, false, IN, 10>(a, s);
    default: return hipErrorInvalidValue;
  }
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
  hipError_t e = in == IN_WG ? launch_gemv_in<IN_WG>(a, l, s)
                             : launch_gemv_in<IN_PRE>(a, l, s);
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

hipError_t launch_embedding(const int64_t *tokens, int64_t count,
                            const uint8_t *table, int64_t rows, int64_t cols,
                            void *out, bool out_bf16, int64_t ldo,
                            int32_t *err_flag, hipStream_t s) {
  if (count == 0) return hipSuccess;
  const int64_t chunks = cols / 16;
  const int aligned = out_bf16
      ? ((uintptr_t)out % 16 == 0) && (ldo % 8 == 0)
      : ((uintptr_t)out % 16 == 0) && (ldo % 4 == 0);
  hipLaunchKernelGGL(embedding_kernel,
                     dim3(grid_for(chunks * count, 256)), dim3(256),
                     0, s, tokens, count, table, rows, passes_for(cols),
                     chunks, out, out_bf16 ? 1 : 0, ldo, err_flag,
                     aligned ? 1 : 0);
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
