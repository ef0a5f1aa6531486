// q8_gemv.h -- the decode GEMV family of the gfx950 Q8_0 linear path and
// the device helpers it shares with the other kernels (block quantizer,
// DPP lane moves, argmax keys).  Included by q8_kernels.hip (scalar
// epilogue variants and every other kernel) and q8_gemv_fma.hip (the fma
// epilogue variants), so the two halves of the GEMV instantiations compile
// in parallel.  The kernels and helpers are in an anonymous namespace: each
// translation unit owns the kernels it instantiates.
#pragma once

#include <math.h>

#include <type_traits>

#include "q8_device.h"
#include "q8_kernels.h"

namespace llmcp_q8 {

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

// Grouped GEMV (V bit 5): the lane groups of up to kMaxGroup weights that
// share the input row, one after another; lane group g belongs to weight i
// when gstart[i] <= g < gstart[i + 1].
struct GemvGroupArgs : GemvArgs {
  int32_t nw;
  int64_t gstart[kMaxGroup + 1];
  const uint8_t *wt[kMaxGroup];
  void *yt[kMaxGroup];
  int32_t actt[kMaxGroup];
};

// Where the GEMV's input row comes from.
enum InputMode {
  IN_PRE = 0,  // pre-quantized Q8_1 row in global memory
  IN_WG = 1    // f32 row, each workgroup quantizes it once into LDS
};

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
// (Written with an "old" operand of 0, which lets the compiler fold the
// move into the consuming add as v_add_f32_dpp.)
__device__ __forceinline__ float row_rotate1(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x121,
                                         0xf, 0xf, false));
}

// 16 B of a weight stream that is read once per call: a non-temporal load
// (measured ~5 % faster than a plain one when streaming 25-675 MB).
__device__ __forceinline__ uint4 load_stream16(const unsigned char *p) {
  typedef unsigned int v4u __attribute__((ext_vector_type(4)));
  const v4u v = __builtin_nontemporal_load((const v4u *)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// DPP move with no "old" value: lanes whose source is out of range receive
// 0 (bound_ctrl), so the destination needs no initialisation.
template <int CTRL>
__device__ __forceinline__ float dpp_mov_f32(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf,
                                      0xf, true));
}

// DPP row_shl:t -- lane i of each 16-lane row receives lane i+t of the row
// (lanes past the row's end receive 0); t = 0 is the value itself.  Lane 0
// of a row thereby reads slot t.  t must be a constant after unrolling.
__device__ __forceinline__ float row_shl(float v, int t) {
  switch (t) {
    case 1: return dpp_mov_f32<0x101>(v);
    case 2: return dpp_mov_f32<0x102>(v);
    case 3: return dpp_mov_f32<0x103>(v);
    case 4: return dpp_mov_f32<0x104>(v);
    case 5: return dpp_mov_f32<0x105>(v);
    case 6: return dpp_mov_f32<0x106>(v);
    case 7: return dpp_mov_f32<0x107>(v);
    case 8: return dpp_mov_f32<0x108>(v);
    case 9: return dpp_mov_f32<0x109>(v);
    case 10: return dpp_mov_f32<0x10A>(v);
    case 11: return dpp_mov_f32<0x10B>(v);
    case 12: return dpp_mov_f32<0x10C>(v);
    case 13: return dpp_mov_f32<0x10D>(v);
    case 14: return dpp_mov_f32<0x10E>(v);
    case 15: return dpp_mov_f32<0x10F>(v);
    default: return v;
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

// The bits of four consecutive values as they come from memory (bf16: two
// dwords of packed halves; f32: four dwords), widened later by act4_of_raw,
// so a batch of loads goes out before the first of them is waited for.
template <bool BF16, bool ALIGNED>
__device__ __forceinline__ uint4 load_raw4(const void *p, int64_t i) {
  if constexpr (BF16) {
    const uint16_t *h = (const uint16_t *)p + i;
    if constexpr (ALIGNED) {
      const uint2 w = *(const uint2 *)h;
      return make_uint4(w.x, w.y, 0u, 0u);
    }
    return make_uint4((uint32_t)h[0] | ((uint32_t)h[1] << 16),
                      (uint32_t)h[2] | ((uint32_t)h[3] << 16), 0u, 0u);
  } else {
    const uint32_t *f = (const uint32_t *)p + i;
    if constexpr (ALIGNED) return *(const uint4 *)f;
    return make_uint4(f[0], f[1], f[2], f[3]);
  }
}

template <bool BF16>
__device__ __forceinline__ float4 act4_of_raw(uint4 r) {
  if constexpr (BF16)
    return make_float4(bf16_to_float(r.x & 0xffffu), bf16_to_float(r.x >> 16),
                       bf16_to_float(r.y & 0xffffu), bf16_to_float(r.y >> 16));
  else
    return make_float4(__uint_as_float(r.x), __uint_as_float(r.y),
                       __uint_as_float(r.z), __uint_as_float(r.w));
}

// --------------------------------------------------------------- GEMV -- //



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

// Waves per workgroup of a one-matrix IN_WG GEMV.  The workgroup quantizes
// the input row once (pc * 16 blocks, 8 lanes per block, row_rounds float4
// loads per lane), so wider workgroups share that work.  Three at K = 9216
// (the down GEMV: 6.94 us against 7.13 with four, 8.8 with six; two and
// eight were 30 % and 13 % slower than four), four elsewhere (at K = 2560
// three measured 3.51 us against 3.42 and two 3 % slower).
__host__ __device__ constexpr int wg_waves(int pc) { return pc == 18 ? 3 : 4; }
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
// bit 1 the output is bf16, bit 2 the GEMV applies a.act, bit 3 it adds the
// residual row a.r to its (rounded) result, bit 4 the fma epilogue, bit 5 a
// grouped GEMV (GemvGroupArgs: each wave takes its weight, output and
// activation from the group table), bit 6 the SwiGLU (gate a.w0, up a.w1).
template <bool ARGMAX, int IN, int W, int D, int PC, int V>
__global__ __launch_bounds__(64 * W) void gemv_kernel(
    std::conditional_t<(V & 32) != 0, GemvGroupArgs, GemvArgs> a) {
  constexpr bool XB = (V & 1) != 0;
  constexpr bool YB = (V & 2) != 0;
  constexpr bool ACTV = (V & 4) != 0;
  constexpr bool ADD = (V & 8) != 0;
  // bit 4: the SDOT paths' epilogue acc = fma(f32(I), sa*dw, acc)
  // (Q8Decode.cpp:192-203); clear: the scalar path's acc + f32(I)*(sa*dw)
  // (Q8Scalar.cpp:192-199).
  constexpr bool FMA = (V & 16) != 0;
  constexpr bool GROUP = (V & 32) != 0;
  // bit 6: SwiGLU by wave pairs.  The even wave of a pair streams the gate
  // matrix, the odd one up, for the same lane group (one wave streaming
  // both measured 7 % slower on the gate/up GEMV); the up wave hands its
  // sums to the gate wave through LDS.
  constexpr bool PAIR = (V & 64) != 0;
  static_assert(!PAIR || (!ARGMAX && !ACTV && !ADD && !GROUP && IN == IN_WG && (W % 2) == 0),
                "SwiGLU variants");
  static_assert(!ADD || (!ARGMAX && !ACTV), "residual add variants");
  static_assert(!GROUP || (!ARGMAX && !ADD && IN == IN_WG), "grouped variants");
  extern __shared__ __align__(16) unsigned char lds[];  // IN_WG input row
  __shared__ unsigned long long key_l[W];
  __shared__ float pair_l[PAIR ? W / 2 : 1][kLanes];
  const int passes = PC > 0 ? PC : a.passes;
  const int nblk = passes * kPassBlocks;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t g = PAIR ? (int64_t)blockIdx.x * (W / 2) + (wave >> 1)
                         : (int64_t)blockIdx.x * W + wave;
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
  // Grouped: the weight of this wave's lane group (wave-uniform) and the
  // lane group's index inside it.
  int widx = 0;
  int64_t lg = gl;
  const uint8_t *w0 = nullptr;
  if constexpr (GROUP) {
#pragma unroll
    for (int i = 1; i < kMaxGroup; ++i)
      if (i < a.nw && gl >= a.gstart[i]) widx = i;
    lg = gl - a.gstart[widx];
    w0 = a.wt[widx];
  } else {
    w0 = (PAIR && (wave & 1)) ? a.w1 : a.w0;
  }
  const unsigned char *base = w0 + lg * passes * kPassBytes;

  uint4 q0[D], q1[D], x0[D], x1[D];
  uint32_t sc[D];
  float xs[D];
  auto issue = [&](int slot, int p) {
    const int pc = p < passes ? p : passes - 1;
    const unsigned char *pb = base + (int64_t)pc * kPassBytes;
    q0[slot] = load_stream16(pb + lane * 16);
    q1[slot] = load_stream16(pb + 1024 + lane * 16);
    sc[slot] = *(const uint16_t *)(pb + kPassQs + lane * 2);
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
  // stays in flight.  With the row quantized in the workgroup, only the
  // first kEarly units go out before the row is quantized and the rest
  // right after: a wave blocks while the memory pipeline accepts its loads,
  // so a whole ring issued first holds up the row's quantization, and with
  // it the chain, until most of the ring has been accepted.  Measured per
  // launch (graph replay, A/B on one box): the down GEMV (K = 9216,
  // 13-unit ring) 7.03-7.09 us with all 13 first, 6.69-6.89 us with 6 (4
  // to 8 alike); K = 2560 (4-unit ring) 3.43-3.44 us with all 4, 3.39 with
  // 3.  The SwiGLU's wave pairs measured the same either way and keep the
  // whole ring first, as do the grouped and argmax variants (not measured).
  constexpr int kEarlyWant =
      (!kRowFirst || PAIR || GROUP || ARGMAX) ? D : PC == 18 ? 6 : PC == 5 ? 3 : D;
  constexpr int kEarly = kEarlyWant < D ? kEarlyWant : D;
#pragma unroll
  for (int d = 0; d < kEarly; ++d) issue(d, d);
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
  // the rest of the ring (all of it went out above unless kEarly < D)
#pragma unroll
  for (int d = kEarly; d < D; ++d) issue(d, d);
  __builtin_amdgcn_sched_barrier(0);

  float acc = 0.0f;

  // Contributions of unit u (ring slot d): exact block dots (two
  // independent dot4 chains; integer sums are order-free), then
  // c = f32(I) * (sa * dw) -- or, for the fma epilogue, the pair
  // (c, cf) = (f32(I), sa * dw) that the chain fuses.  Split in three parts
  // so that the next pass's preparation can ride in the current pass's
  // chain (see chain_with).
  struct Next {
    uint4 a0, a1;
    float s_a;
    int d0, d1;
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
    n.d0 = n.d1 = 0;
  };
  auto dot_part = [&](int d, int k, Next &n) {
    n.d0 = __builtin_amdgcn_sdot4((int)word(q0[d], k), (int)word(n.a0, k), n.d0, false);
    n.d1 = __builtin_amdgcn_sdot4((int)word(q1[d], k), (int)word(n.a1, k), n.d1, false);
  };
  auto finish = [&](int d, Next &n, float &c, float &cf) {
    const int dot = n.d0 + n.d1;
    const float factor = n.s_a * half_bits_to_float(sc[d]);
    if constexpr (FMA) {
      c = (float)dot;
      cf = factor;
    } else {
      c = (float)dot * factor;
      cf = 0.0f;
    }
  };
  // All S units of pass p.
  auto prepare = [&](int p, float (&c)[S], float (&cf)[S]) {
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const int u = p * S + i;
      Next n;
      load_act(u % D, u, n);
#pragma unroll
      for (int k = 0; k < 4; ++k) dot_part(u % D, k, n);
      finish(u % D, n, c[i], cf[i]);
    }
  };
  // The chain's form.  Rotating: the running sum moves one lane per slot
  // (DPP row_ror:1 on the sum, folded into the scalar form's add), so after
  // slot t it sits in lane t and lane 15 ends the pass.  Lane 0: the sum
  // stays in lane 0 of the row and slot t's contribution is brought there
  // by DPP on the source operand (row_shl:t), so the sum never waits on a
  // DPP read; the fma's second factor needs its own DPP move, which does
  // not depend on the sum.  Measured per variant: the fma form with one
  // block per slot runs faster in lane 0 (the rotating fma is a move plus
  // an fma on the sum's path); with segments (S > 1) and for the scalar
  // form the rotating chain is faster.
  constexpr bool LANE0 = FMA && S == 1;
  constexpr int kOwnerSlot = LANE0 ? 0 : 15;
  // One block's step: acc + c (scalar) or fma(c, cf, acc), for slot t;
  // `first` marks the slot's first block (where a rotating chain moves).
  auto step = [&](float acc_in, float c, float cf, int t, bool first) {
    if constexpr (LANE0) {
      return __builtin_fmaf(row_shl(c, t), row_shl(cf, t), acc_in);
    } else if constexpr (FMA) {
      return __builtin_fmaf(c, cf, first ? dpp_mov_f32<0x121>(acc_in) : acc_in);
    } else {
      return (first ? row_rotate1(acc_in) : acc_in) + c;
    }
  };
  // The serial chain over one pass's 16 lane slots in block order: at step
  // t the row's sum takes slot t's S blocks in order, so after step t it
  // holds the sum through block 16S*p + S*t + S-1 and carries it into the
  // next pass.  The next pass's activation reads go out at step 0; its
  // dots and scalings (5 pieces per unit) are spread over steps 4-14, each
  // pinned between chain additions (whose dependent latency they hide) by
  // sched_barrier.  The dots wait for the next pass's weights inside this
  // chain, which costs nothing once the ring has landed.
  auto chain_with = [&](const float (&c)[S], const float (&cf)[S], bool has_next,
                        int pn, float (&cn)[S], float (&cfn)[S]) {
    Next n[S];
    if (has_next) {
#pragma unroll
      for (int i = 0; i < S; ++i) load_act((pn * S + i) % D, pn * S + i, n[i]);
    }
#pragma unroll
    for (int t = 0; t < kPassBlocks; ++t) {
#pragma unroll
      for (int i = 0; i < S; ++i) acc = step(acc, c[i], cf[i], t, i == 0);
      if (has_next) {
#pragma unroll
        for (int o = 0; o < 5 * S; ++o) {
          if (4 + (o * 11) / (5 * S) != t) continue;
          const int i = o / 5, k = o % 5;
          const int d = (pn * S + i) % D;
          if (k < 4)
            dot_part(d, k, n[i]);
          else
            finish(d, n[i], cn[i], cfn[i]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  if (active) {
    float cur[S], nxt[S], curf[S], nxtf[S];
    prepare(0, cur, curf);
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
        chain_with(cur, curf, p + 1 < NP, p + 1, nxt, nxtf);
#pragma unroll
        for (int i = 0; i < S; ++i) {
          cur[i] = nxt[i];
          curf[i] = nxtf[i];
        }
      }
    } else {
      for (int p0 = 0; p0 < passes; p0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
          const int p = p0 + d;
          if (p < passes) {
            issue(d, p + D);
            __builtin_amdgcn_sched_barrier(0);
            chain_with(cur, curf, p + 1 < passes, p + 1, nxt, nxtf);
            cur[0] = nxt[0];
            curf[0] = nxtf[0];
          }
        }
      }
    }
  }

  const int64_t row = lg * kLanes + r;  // lg == g unless grouped (active waves)
  // Epilogue (MatmulLoweringCommon.cpp:78-103).  SwiGLU: h = silu(gate) *
  // up; with a bf16 result each linear's output is rounded to bf16 before
  // the bf16 multiply (FuseSiluMul: linear{silu} + mul on bf16 tensors).
  float y;
  if constexpr (PAIR) {
    // every wave reaches the barrier, active or not
    if (active && (wave & 1) && j == kOwnerSlot) pair_l[wave >> 1][r] = acc;
    __syncthreads();
    const float up = pair_l[wave >> 1][r];
    const float gs = silu_f32(acc);
    y = YB ? bf16_to_float(float_to_bf16(gs)) * bf16_to_float(float_to_bf16(up))
           : gs * up;
  } else {
    int act = a.act;
    if constexpr (GROUP) act = a.actt[widx];
    y = ACTV ? activate(acc, act) : acc;
  }
  void *yout = a.y;
  if constexpr (GROUP) yout = a.yt[widx];
  // the lane holding the sum (PAIR: of the gate wave)
  const bool owner = active && j == kOwnerSlot && !(PAIR && (wave & 1));
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
      ((uint16_t *)yout)[row] = float_to_bf16(y);
    else
      ((float *)yout)[row] = y;
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

inline unsigned grid_for(int64_t threads, int block) {
  return (unsigned)((threads + block - 1) / block);
}

// Ring depth: passes in flight per wave.  From LDS: 4 up to K = 2560 (the
// 2560 x 2560 GEMV: 3.71 us against 3.86 with all 5; the SwiGLU's gate/up
// waves measured the same with 2, 3 or 5), else 13 (117 VGPRs; at K = 9216
// the down GEMV measured 7.46 us against 8.05 with all 18 passes in flight,
// 7.74 with 12 and 7.65-7.82 with 14-16).  With a pre-quantized row: 12
// passes of weights + input.
template <int IN, int PC>
constexpr int ring_depth() {
  // at least two passes of units, so the next pass is in flight while the
  // current one chains
  constexpr int two = 2 * seg_for(PC);
  constexpr int base = IN == IN_WG ? (PC <= 5 ? 4 : 13) : 12;
  constexpr int dmax = base > two ? base : two;
  return PC > 0 ? (PC < dmax ? PC : dmax) : 8;
}

template <bool ARGMAX, int IN, int W, int PC, int V, class A>
hipError_t launch_gemv_p(const A &args, hipStream_t s) {
  constexpr int D = ring_depth<IN, PC>();
  constexpr int GW = (V & 64) != 0 ? W / 2 : W;  // lane groups per workgroup
  const unsigned grid = (unsigned)((args.groups + GW - 1) / GW);
  const size_t slots = PC > 0 ? row_slots(PC, W) : (size_t)args.passes * kPassBlocks;
  const size_t lds = IN == IN_WG ? slots * (kBlock + 4) : 0;
  hipLaunchKernelGGL((gemv_kernel<ARGMAX, IN, W, D, PC, V>),
                     dim3(grid), dim3(64 * W), lds, s, args);
  return hipGetLastError();
}

// One-matrix IN_WG GEMVs take their workgroup width from wg_waves; the
// SwiGLU runs two lane groups per four-wave workgroup (six and eight waves
// measured 10 % and 9 % slower, two 2 % slower); IN_PRE (wide outputs) runs
// four waves per workgroup.
template <bool ARGMAX, int IN, int PC, int V, class A>
hipError_t launch_gemv_w(const A &args, hipStream_t s) {
  constexpr int W = IN == IN_WG ? ((V & 64) != 0 ? 4 : wg_waves(PC)) : 4;
  return launch_gemv_p<ARGMAX, IN, W, PC, V>(args, s);
}

// Pass counts with a fully unrolled kernel: K = 512, 1024, 1536, 2560
// (hidden size), 4096 and 9216 (the MLP down projection).  Others take the
// runtime loop.
template <bool ARGMAX, int IN, int V, class A = GemvArgs>
hipError_t launch_gemv_t(const A &args, hipStream_t s) {
  switch (args.passes) {
    case 1: return launch_gemv_w<ARGMAX, IN, 1, V>(args, s);
    case 2: return launch_gemv_w<ARGMAX, IN, 2, V>(args, s);
    case 3: return launch_gemv_w<ARGMAX, IN, 3, V>(args, s);
    case 5: return launch_gemv_w<ARGMAX, IN, 5, V>(args, s);
    case 8: return launch_gemv_w<ARGMAX, IN, 8, V>(args, s);
    case 18: return launch_gemv_w<ARGMAX, IN, 18, V>(args, s);
    default: return launch_gemv_w<ARGMAX, IN, 0, V>(args, s);
  }
}

// The compile-time variants the C ABI needs (V bits as in gemv_kernel):
// SwiGLU f32 or bf16 in and out; the argmax GEMV (lm_head) with f32 logits
// from an f32 or bf16 row; plain GEMVs with or without an activation, f32 or
// bf16 in and out.  IN_PRE reads an already quantized row (no input type).
template <int IN, bool FMA>
hipError_t launch_gemv_in(const GemvArgs &a, const GemvLaunch &l,
                          hipStream_t s) {
  const int xb = (IN == IN_WG && l.x_bf16) ? 1 : 0;
  const int yb = l.y_bf16 ? 2 : 0;
  const int av = (l.nmat == 1 && !l.keys && l.activation != 0) ? 4 : 0;
  const int ad = l.residual ? 8 : 0;
  if (ad && (l.nmat != 1 || l.keys || av)) return hipErrorInvalidValue;
  const int v = xb | yb | av | ad;
  constexpr int F = FMA ? 16 : 0;
  if (l.nmat == 2) {
    // the SwiGLU quantizes its row in-workgroup (gemv_quantizes_input)
    if constexpr (IN == IN_WG) {
      if (v == 0) return launch_gemv_t<false, IN, (64) | F>(a, s);
      if (v == 3) return launch_gemv_t<false, IN, (3 | 64) | F>(a, s);
    }
    return hipErrorInvalidValue;
  }
  if (l.keys) {
    if (v == 0) return launch_gemv_t<true, IN, (0) | F>(a, s);
    if (IN == IN_WG && v == 1) return launch_gemv_t<true, IN, (1) | F>(a, s);
    return hipErrorInvalidValue;
  }
  if (IN == IN_WG) {
    switch (v) {
      case 0: return launch_gemv_t<false, IN, (0) | F>(a, s);
      case 3: return launch_gemv_t<false, IN, (3) | F>(a, s);
      case 4: return launch_gemv_t<false, IN, (4) | F>(a, s);
      case 7: return launch_gemv_t<false, IN, (7) | F>(a, s);
      case 8: return launch_gemv_t<false, IN, (8) | F>(a, s);
      case 11: return launch_gemv_t<false, IN, (11) | F>(a, s);
      default: return hipErrorInvalidValue;
    }
  }
  switch (v) {
    case 0: return launch_gemv_t<false, IN, (0) | F>(a, s);
    case 2: return launch_gemv_t<false, IN, (2) | F>(a, s);
    case 4: return launch_gemv_t<false, IN, (4) | F>(a, s);
    case 6: return launch_gemv_t<false, IN, (6) | F>(a, s);
    case 8: return launch_gemv_t<false, IN, (8) | F>(a, s);
    case 10: return launch_gemv_t<false, IN, (10) | F>(a, s);
    default: return hipErrorInvalidValue;
  }
}

// Grouped GEMV variants: f32 or bf16 in and out, with or without runtime
// activations (V bit 2 when any weight of the group has one).
template <bool FMA>
hipError_t launch_gemv_group(const GemvGroupArgs &a, const GemvLaunch &l,
                             hipStream_t s) {
  bool any_act = false;
  for (int i = 0; i < l.ngroup; ++i) any_act |= l.gact[i] != 0;
  const int v = (l.x_bf16 ? 1 : 0) | (l.y_bf16 ? 2 : 0) | (any_act ? 4 : 0);
  constexpr int F = (FMA ? 16 : 0) | 32;
  switch (v) {
    case 0: return launch_gemv_t<false, IN_WG, 0 | F>(a, s);
    case 3: return launch_gemv_t<false, IN_WG, 3 | F>(a, s);
    case 4: return launch_gemv_t<false, IN_WG, 4 | F>(a, s);
    case 7: return launch_gemv_t<false, IN_WG, 7 | F>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace
}  // namespace llmcp_q8
