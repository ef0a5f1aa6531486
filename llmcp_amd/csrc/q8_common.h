// q8_common.h -- shared constants and small device helpers for the gfx950
// Q8_0 linear path.
//
// Wire format (arena, "q8_0_p4"): include/llmcp/Support/Q8PackedLayout.h:18-42
//   record(g, b) at (g*B + b)*136 holds [4 x f16 scale][8 chunks x 16 B],
//   chunk c, lane l: bytes q[4g+l][32b + 4c .. 32b + 4c + 3].
//
// Device layout ("unit layout"), produced once per tensor by repack_p4:
//   Per lane group g (4 rows) the B blocks are padded to U = ceil(B/16)
//   units of 16 blocks; unit u of group g is 2176 B at (g*U + u) * 2176:
//     [0, 2048)     qs:  offset h*1024 + r*256 + j*16 holds
//                        q[4g+r][32*b + 16h .. +16]   (h = 0, 1)
//     [2048, 2176)  scales: f16 at 2048 + 2*(16r + j) = d[4g+r][b]
//   for the block b that sits in unit u at lane slot j.  With S = seg_for(U)
//   blocks per slot and pass, pass p covers blocks 16*S*p .. 16*S*(p+1)-1:
//   slot j holds the S consecutive blocks 16Sp + Sj .. 16Sp + Sj + S-1, the
//   i-th of them in unit p*S + i.  (S = 1: unit p holds blocks 16p + j.)
//   Blocks past B are zero (q = 0, d = 0).  When B % 16 == 0 the tensor has
//   exactly the arena's N*K*34/32 bytes.  Wave lane L = 16r + j reads its
//   row-r data of a unit at h*1024 + 16L and 2048 + 2L: every load of a wave
//   is one contiguous, aligned 1024 B (or 128 B) run.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llmcp_q8 {

constexpr int kBlock = 32;           // Q8_0 block size along K
constexpr int kLanes = 4;            // rows per lane group (p4)
constexpr int kRecord = 136;         // p4 record bytes
constexpr int kPassBlocks = 16;      // blocks per pass
constexpr int kPassQs = 2048;        // qs bytes per pass (4 rows x 16 x 32)
constexpr int kPassBytes = 2176;     // qs + 128 B of scales

inline int64_t passes_for(int64_t cols) {
  int64_t blocks = cols / kBlock;
  return (blocks + kPassBlocks - 1) / kPassBlocks;
}

inline int64_t device_bytes_for(int64_t rows, int64_t cols) {
  return rows / kLanes * passes_for(cols) * kPassBytes;
}

// Blocks per slot and pass for a tensor of `units` units.  The serial
// GEMV chain hands its running sum from slot to slot with one DPP step per
// slot and adds a slot's S blocks with plain adds, so S > 1 shortens long
// chains (K = 9216: 18 units, 3 passes of 96 blocks).  Only unit counts the
// GEMV unrolls use S > 1.
__host__ __device__ constexpr int seg_for(int64_t units) {
  return units == 18 ? 6 : (units == 8 ? 4 : 1);
}

// Unit and lane slot of block b for a compile-time S.
template <int S>
__host__ __device__ inline void locate(int64_t b, int64_t &unit, int &slot) {
  const int64_t p = b / (kPassBlocks * S);
  const int rem = (int)(b - p * kPassBlocks * S);
  slot = rem / S;
  unit = p * S + rem % S;
}

// Runtime S: all three mappings, then selects.  (Written branch-free on
// purpose: the branchy form was miscompiled for S = 4 inside the GEMM's
// stage loader, which read unit 0 for blocks 1-3 of a slot.)
__host__ __device__ inline void locate_seg(int64_t b, int seg, int64_t &unit,
                                           int &slot) {
  int64_t u1, u4, u6;
  int s1, s4, s6;
  locate<1>(b, u1, s1);
  locate<4>(b, u4, s4);
  locate<6>(b, u6, s6);
  unit = seg == 6 ? u6 : (seg == 4 ? u4 : u1);
  slot = seg == 6 ? s6 : (seg == 4 ? s4 : s1);
}

}  // namespace llmcp_q8
