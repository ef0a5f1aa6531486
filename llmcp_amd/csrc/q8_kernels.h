// q8_kernels.h -- host-side launchers of the gfx950 kernels (internal; the
// public C ABI is include/llmcp_q8.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "q8_common.h"

namespace llmcp_q8 {

// p4 arena bytes (device) -> pass layout (device), once per tensor.
hipError_t launch_repack(const uint8_t *p4, uint8_t *out, int64_t rows,
                         int64_t cols, hipStream_t s);

// Synthetic N(0, stddev^2) weights from a counter-based generator.
hipError_t launch_synth(uint64_t seed, int64_t rows, int64_t cols,
                        float stddev, float *w, hipStream_t s);

// Device llmcp-pack: f32 [rows, cols] -> p4 bytes (Quantization.cpp:92-214).
hipError_t launch_pack_p4(const float *w, int64_t rows, int64_t cols,
                          uint8_t *p4, hipStream_t s);

// Q8_1 activation quantizer: x [m, cols] f32 or bf16 (row stride ldx
// elements) -> qa [m, ldq] int8 and sa [m, lds] f32, zero-filled up to
// blocks_pad blocks.
hipError_t launch_quantize(const void *x, bool x_bf16, int64_t m, int64_t ldx,
                           int64_t cols, int8_t *qa, int64_t ldq, float *sa,
                           int64_t lds, int64_t blocks_pad, hipStream_t s);

// Exhaustive device check of the quantizer's division identities; adds the
// number of mismatching inputs to *bad.
hipError_t launch_selftest_quantizer(unsigned long long *bad, hipStream_t s);
hipError_t launch_selftest_exp(unsigned long long *out, float *inputs,
                               uint32_t *results, uint32_t cap, hipStream_t s);

// Compute units of the current device (cached per device; 256 if the
// query fails).
int cu_count();

// Most weights one grouped GEMV serves (llmcp_q8_linear_group).
constexpr int kMaxGroup = 8;

struct GemvLaunch {
  const void *x = nullptr;       // input row (f32 16 B / bf16 8 B aligned),
  bool x_bf16 = false;           // quantized once per workgroup into LDS
  const int8_t *qa = nullptr;    // or: Q8_1 input row, padded to passes*16
  const float *sa = nullptr;     //     blocks (used when x is null)
  const uint8_t *w[2] = {nullptr, nullptr};  // unit-layout weights
  void *y = nullptr;             // output [rows], f32 or bf16
  bool y_bf16 = false;
  int64_t rows = 0;              // N
  int64_t cols = 0;              // K
  int nmat = 1;                  // 2 = fused SwiGLU (gate, up)
  int activation = 0;            // llmcp_q8_activation (nmat == 1 only)
  bool fma = false;              // epilogue: fma (SDOT paths) or mul+add
                                 // (x86 scalar path)
  const void *residual = nullptr;      // non-null (one matrix, no activation,
                                       // no argmax): y = r + acc, r [rows] of
                                       // y's element type (may alias y)
  unsigned long long *keys = nullptr;  // non-null: fused argmax into these
  int64_t *argmax_out = nullptr;       // kArgmaxSlots slots, zero on entry
                                       // and left zero
  // ngroup > 0: one launch for ngroup weights that share the input row
  // (same cols; w, y, rows, activation above unused): weight i, gw[i]
  // [grows[i], cols], writes gy[i] with activation gact[i].
  int ngroup = 0;
  const uint8_t *gw[kMaxGroup] = {};
  void *gy[kMaxGroup] = {};
  int64_t grows[kMaxGroup] = {};
  int32_t gact[kMaxGroup] = {};
};

// One-matrix GEMVs with at most this many lane groups quantize the input
// row inside the kernel (once per workgroup); wider ones (every workgroup
// would re-read the row) take a pre-quantized row unless the row is at most
// kInLoopQuantMaxCols wide: the 248320-row lm_head (K = 2560, 15520
// workgroups re-reading a 10 KB row from L2) measured 106.7 us per call
// against 109.9 with the separate quantize launch.  Two-matrix (SwiGLU)
// GEMVs always quantize inside.
constexpr int64_t kInLoopQuantMaxGroups = 4096;
constexpr int64_t kInLoopQuantMaxCols = 2560;
bool gemv_quantizes_input(int64_t rows, int64_t cols, int nmat);

hipError_t launch_gemv(const GemvLaunch &l, hipStream_t s);

// The argmax GEMV folds each workgroup's (value, index) key into one of
// kArgmaxSlots slots with an atomic max; the reduce kernel swaps them back
// to zero.  More slots than this left same-address atomics contending.
constexpr int kArgmaxSlots = 2048;
// Reduces the slots into *out (the first maximum's index) and clears them;
// out == nullptr only clears.
hipError_t launch_argmax_reduce(unsigned long long *slots, int64_t *out,
                                hipStream_t s);

// First-maximum index of the f32 row v[0..n) into *out, through the zeroed
// slots (left zeroed); n < 2^32.
hipError_t launch_argmax_row(const float *v, int64_t n, int64_t *out,
                             unsigned long long *slots, hipStream_t s);

// Prefill GEMM on int8 MFMA.  qa/sa: Q8_1 activations [m, ldq] / [m, lds],
// zero-padded to passes*16 blocks (launch_quantize with blocks_pad).
struct GemmLaunch {
  const int8_t *qa = nullptr;  // tiled Q8_1 input (launch_quantize_tiled)
  const float *sa = nullptr;
  int32_t row_tiles = 0;       // 32-row tiles in qa / sa
  int32_t nblk = 0;            // padded blocks per row (units * 16)
  const uint8_t *w = nullptr;  // unit layout
  int64_t rows = 0;            // N
  int64_t cols = 0;            // K
  int64_t m = 0;               // M
  void *y = nullptr;             // f32 or bf16 [m, ldy]
  bool y_bf16 = false;
  int64_t ldy = 0;
  int activation = 0;            // llmcp_q8_activation
  bool fma = true;             // epilogue: fma (SDOT GEMM) or mul+add (scalar)
  // Non-null: the SwiGLU multiply in the epilogue, y = g * act(acc) with g
  // f32 [m, ldg] (the gate linear's activated output; it may alias y when
  // y is f32).  A bf16 result rounds both factors to bf16 first.
  const float *mul = nullptr;
  int64_t ldg = 0;
  // Non-null (no activation, no mul): the residual add in the epilogue,
  // y = r + acc with r [m, ldr] of y's element type (it may alias y); a bf16
  // result rounds acc to bf16 first and adds in f32.
  const void *add = nullptr;
  int64_t ldr = 0;
  // K splits (1: none, the reference's serial block order bit for bit).
  // splits > 1 (at most passes_for(cols); rows % 4 == 0): each output's
  // blocks run as `splits` serial chains over contiguous ranges of whole
  // passes, each from 0 in the platform's epilogue, stored as f32 partial
  // sums in `part` ([splits][m][rows] floats), which a second kernel adds
  // in split order before the epilogue.  Deterministic; not the reference's
  // summation order, so f32 results agree with it within rounding only.
  int32_t splits = 1;
  float *part = nullptr;
};

hipError_t launch_gemm(const GemmLaunch &l, hipStream_t s);

// K splits for a multi-row linear of [m x cols] by [rows x cols] when
// splitting is allowed: `forced` > 0 (clamped to the pass count), else the
// count measured fastest for the shape class (tiles x splits within one
// workgroup per CU, at most max(3, passes / 3); 1 where the tiles already
// cover the CUs).
int32_t gemm_splits_for(int64_t m, int64_t rows, int64_t cols, int32_t forced);

// Q8_1 activations in the GEMM's tiled layout: the 32 rows x 32 values of
// row tile t and block b are 1 KiB at (t * blocks_pad + b) * 1024 (row r at
// r * 32), their scales 32 floats at (t * blocks_pad + b) * 32.  Rows past m
// in the last tile and blocks past the row's are written as zeros.
hipError_t launch_quantize_tiled(const void *x, bool x_bf16, int64_t m,
                                 int64_t ldx, int64_t cols, int8_t *qa,
                                 float *sa, int64_t blocks_pad, hipStream_t s);

// RMSNorm of m rows of width h (h % 32 == 0) with weight w [h]: y = (x *
// rstd) * (w or w + 1), each row's sum of squares serial in index order.
// x and y share their type (f32 or bf16); w is f32 or bf16.  qmode 1 also
// writes y's Q8_1 in the dense layout (row r at r * blocks_pad * 32, scales
// at r * blocks_pad), qmode 2 in the tiled layout of launch_quantize_tiled.
// spec_skew (tests only; 0 otherwise) offsets the predicted partial sums of
// rows of up to 12288 values, whose serial sum is evaluated speculatively,
// by that many f32 steps, so that the exact fallbacks decide the results;
// the results are the same either way.
hipError_t launch_rmsnorm(const void *x, bool x_bf16, int64_t m, int64_t ldx,
                          int64_t h, const void *w, bool w_bf16, float eps,
                          bool zero_centered, void *y, bool y_bf16, int64_t ldy,
                          int8_t *qa, float *sa, int64_t blocks_pad, int qmode,
                          hipStream_t s, int spec_skew = 0);

// Gated RMSNorm of `groups` dense groups of g values (g % 32 == 0): x, gate
// and y share their type (f32 or bf16), w [g] is f32.
hipError_t launch_gated_rmsnorm(const void *x, const void *gate, bool bf16,
                                int64_t groups, int64_t g, const float *w, float eps,
                                bool gate_activated, void *y, hipStream_t s);

hipError_t launch_embedding(const int64_t *tokens, int64_t count,
                            const uint8_t *table, int64_t rows, int64_t cols,
                            void *out, bool out_bf16, int64_t ldo,
                            int32_t *err_flag, hipStream_t s);

// Peak microbenchmarks (q8_microbench.hip).  launch_stream: kind 0 reads
// `bytes` at src (dst: a 4 B sink, never written in practice), 1 writes
// them at dst, 2 copies src to dst; bytes a multiple of cus * 256 KiB.
hipError_t launch_stream(int kind, const void *src, void *dst, int64_t bytes, int cus,
                         hipStream_t s);
// int8 MFMA chains with no memory traffic; mfma_i8_peak_ops is the number
// of int8 operations one launch performs.
hipError_t launch_mfma_i8_peak(int32_t iterations, int cus, unsigned *sink, hipStream_t s);
double mfma_i8_peak_ops(int32_t iterations, int cus);
// The prefill GEMM's per-block instruction mix on LDS-resident operands
// (mode 0 the exact int8 epilogue, 1 convert-free f16 dots, 2 the MFMAs
// alone), 2 * pairs blocks per wave; epilogue_mix_ops counts 2 * 32^3
// operations per wave and block.
hipError_t launch_epilogue_mix(int mode, int32_t pairs, int cus, unsigned *sink,
                               hipStream_t s);
double epilogue_mix_ops(int32_t pairs, int cus);

hipError_t launch_block_dots(const int8_t *qa, int64_t ldq, int64_t m,
                             const uint8_t *w, int64_t rows, int64_t cols,
                             int32_t *out, hipStream_t s);

}  // namespace llmcp_q8
