// q8_common.h -- shared constants and small device helpers for the gfx950
// Q8_0 linear path.
//
// Wire format (arena, "q8_0_p4"): include/llmcp/Support/Q8PackedLayout.h:18-42
//   record(g, b) at (g*B + b)*136 holds [4 x f16 scale][8 chunks x 16 B],
//   chunk c, lane l: bytes q[4g+l][32b + 4c .. 32b + 4c + 3].
//
// Device layout ("pass layout"), produced once per tensor by repack_p4:
//   Per lane group g (4 rows) the B blocks are cut into P = ceil(B/16)
//   passes of 16 blocks.  Pass p of group g is one 2176 B unit at
//   (g*P + p) * 2176:
//     [0, 2048)     qs:  offset h*1024 + r*256 + j*16 holds
//                        q[4g+r][32*(16p+j) + 16h .. +16]   (h = 0, 1)
//     [2048, 2176)  scales: f16 at 2048 + 2*(16r + j) = d[4g+r][16p+j]
//   Blocks past B are zero (q = 0, d = 0).  When B % 16 == 0 the tensor has
//   exactly the arena's N*K*34/32 bytes.  Wave lane L = 16r + j reads its
//   row-r, block-j data at h*1024 + 16L and 2048 + 2L: every load of a wave
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

}  // namespace llmcp_q8
