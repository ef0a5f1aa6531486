// q8_gemm.hip -- prefill GEMM of the Q8_0 linear path on gfx950 int8 MFMA.
//
// y[M,N] = act( sum_b f32(I_b[m,n]) * (sa[m,b] * dw[n,b]) ), blocks in order
// b = 0..B-1 per output element, I_b the exact int32 dot of one 32-wide
// block.  v_mfma_i32_32x32x32_i8 has K = 32, exactly one Q8 block, so every
// MFMA yields fresh block dots I_b for a 32x32 tile and the per-block scale
// epilogue runs in VALU right after it:
//   EPI_FMA     acc = fma(f32(I), sa*dw, acc)          Q8Matmul.cpp:204-223
//   EPI_SCALAR  acc = acc + f32(I) * (sa*dw)           Q8Scalar.cpp:192-199
// Both match the reference bit for bit; FMA (the reference's own GEMM on its
// SDOT target) costs one VALU op less per element and block.
//
// The activations come from the quantizer's tiled layout (32-row x 1-block
// tiles of 1 KiB, scales [row tile][block][32]), the weights from the unit
// layout; operands reach LDS by direct-to-LDS loads through a ring of
// stage buffers (see gemm_kernel).
#include "q8_kernels.h"

#include <stddef.h>

#include <algorithm>
#include <atomic>
#include <utility>

#include "q8_device.h"

namespace llmcp_q8 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

// ------------------------------------------------- DMA-pipelined GEMM -- //
//
// Workgroup of WM x WN waves, one 32x32 output tile per wave.  K advances
// in stages of four blocks.  A stage's operands travel global -> LDS by
// direct-to-LDS loads (buffer loads with the lds bit: lane l's bytes land
// at base + l * size), NST stage buffers deep, so NST - 1 stages are in flight while
// one is consumed, and no VGPRs hold staged data.  Each load instruction
// reads whole 64-128 B runs, and each LDS piece sits where the MFMA lanes
// read it without bank conflicts:
//   A  (row tile t, block)   the 1 KiB tile of the quantizer's tiled
//                            layout, lane l: row l%32, k half l/32
//   sa (row tile t, 2 blocks) 64 floats: block l/32, row l%32
//   B  (col tile t)          64 runs RI = 32h + (n%32) of 4 blocks x 16 B,
//                            run RI at RI*64, block j at 16*(j ^ (RI/4)%4)
//   dw (col tile t)          f16 pairs holding the stage's scales
// The sa/dw pieces feed one two-block f32 outer-product MFMA per block pair
// (lanes 0-31 block 0, lanes 32-63 block 1) that yields both blocks' scale
// tiles.  Each stage buffer is its own LDS object, so the compiler's wait
// for a wave's own DMA into one buffer does not drain the others; the
// cross-wave hand-off is an explicit vmcnt wait plus s_barrier.
// When the tiles outnumber the resident workgroups, workgroups are
// persistent and the ring runs on from one tile into the next (PERSIST).
// PROD (when the workgroups fit one per CU, not persistent): four more
// waves per workgroup issue all the DMA ops, so the compute waves spend no
// issue slots on them (N = 9216, K = 2560: op 18.4 -> 16.5 us at M = 64 on
// the four-wave 64 x 64 shape, 32.3 -> 31.4 at M = 256 on the twelve-wave
// 128 x 96 one, whose compute waves then fit 128 VGPRs).
constexpr int kStageBlocks = 4;

template <int WM, int WN, int SEG, int NI = WM * WN>
struct GemmStage {
  static constexpr int W = WM * WN;
  // DMA ops of a stage.  16 B per lane (1 KiB per op): the A tiles (row
  // tile, block), the weight chunks (4 per column tile), the activation
  // scales (two row tiles per op: 4 blocks x 32 rows each) and, for S = 1,
  // each column tile's 8 scale blocks of 128 B (the whole unit's scales, so
  // one op instead of scattered 4 B pieces).  4 B per lane: for S > 1 the
  // weight scales of the stage's blocks, which sit in different units.
  static constexpr int CA = WM * kStageBlocks;
  static constexpr int CB = WN * 4;
  static constexpr int CS = (WM + 1) / 2;
  static constexpr int CD16 = SEG == 1 ? WN : 0;
  static constexpr int CD4 = SEG == 1 ? 0 : 2 * WN;
  // Every wave issues the same number of each size (S16, S4),
  // unconditionally: a branch around a DMA, or a branch between DMAs of
  // different sizes, makes the compiler's wait tracking merge states and
  // wait for all loads before the next LDS read.  Where a class does not
  // divide evenly, waves repeat another wave's op (same bytes, same place).
  static constexpr int T16 = CA + CB + CS + CD16;
  static constexpr int T4 = CD4;
  // NI waves issue the ops: the W compute waves, or the producer waves
  static constexpr int S16 = (T16 + NI - 1) / NI;
  static constexpr int S4 = (T4 + NI - 1) / NI;
  static constexpr int OPS = S16 + S4;  // DMA instructions per wave and stage
  __align__(16) int8_t a[WM][kStageBlocks][1024];
  __align__(16) int8_t b[WN][4 * 1024];
  __align__(16) float sa[2 * CS][kStageBlocks][32];
  __align__(16) uint8_t dw16[CD16 > 0 ? WN : 1][1024];
  __align__(16) uint32_t dw4[CD4 > 0 ? WN : 1][2][64];
};

typedef __attribute__((address_space(3))) void lds_void;

// Direct-to-LDS loads (16 B or 4 B per lane), buffer-addressed: the source
// is base (a buffer resource in SGPRs) + a wave-uniform offset (SGPR) + a
// per-lane 32-bit offset (VGPR), so no VALU instruction forms a 64-bit
// address per load (with global_load_lds the M = 1024 op measured 3 %
// slower, M = 256 4 %).  Dword 3 as for every gfx9 raw buffer; the range is
// the whole 4 GiB an unsigned offset reaches (every operand tensor is
// smaller).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void *base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, -1, 0x00020000);
}
__device__ __forceinline__ void bdma16(__amdgpu_buffer_rsrc_t r, uint32_t lane_off,
                                       uint32_t uniform_off, void *lds_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds_base, 16, lane_off, uniform_off,
                                           0, 0);
}
__device__ __forceinline__ void bdma4(__amdgpu_buffer_rsrc_t r, uint32_t lane_off,
                                      uint32_t uniform_off, void *lds_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds_base, 4, lane_off, uniform_off,
                                           0, 0);
}

// s_waitcnt vmcnt(n) (gfx9 encoding; expcnt and lgkmcnt not waited on).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | 0x70 | 0xF00 | ((N >> 4) << 14));
}
// Workgroup barrier without a memory fence: the LDS data it publishes came
// by DMA, whose completion each wave establishes with its own vmcnt wait
// first (a fenced barrier would wait for every load in flight).  The
// signal fences keep the compiler from moving LDS accesses across it.
__device__ __forceinline__ void stage_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// A wave-uniform pointer, made visibly uniform so that an access at
// `uniform + 32-bit lane offset` keeps the per-stage math scalar.
template <class T>
__device__ __forceinline__ const T *uniform_ptr(const T *p) {
  const uint64_t v = (uint64_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const T *)(((uint64_t)hi << 32) | lo);
}

// S = 6 (18 units, passes of 96 blocks): block kb + p of a stage (kb a
// multiple of 4, p < 4) sits at unit 6P + d', slot q + wrap, where
// rem = kb mod 96 = 6q + r (r in {0, 2, 4}), d = r + p, wrap = (d >= 6) and
// d' = d - 6 wrap.  Per lane only (r, p) matter: the kernel keeps the three
// per-lane variants and selects one per stage by the wave-uniform r.
struct Seg6 {
  static __device__ __forceinline__ int wrap(int r, int p) { return r + p >= 6 ? 1 : 0; }
  // byte offset of the block's 16 B piece, relative to unit 6P, slot q
  static __device__ __forceinline__ uint32_t qs(int r, int p) {
    const int w6 = wrap(r, p);
    return (uint32_t)((r + p - 6 * w6) * kPassBytes + w6 * 16);
  }
  // byte offset of the f16 pair holding the block's scale, relative to
  // unit 6P, slot pair (q & ~1)
  static __device__ __forceinline__ uint32_t scale(int r, int q, int p) {
    const int w6 = wrap(r, p);
    return (uint32_t)((r + p - 6 * w6) * kPassBytes + 2 * ((q + w6) & ~1) - 2 * (q & ~1));
  }
};

// The occupancy the LDS allows (12 waves: one workgroup per CU, three waves
// per SIMD; 4 waves: two workgroups per CU) is declared so that the kernel
// stays within 256 VGPRs, which keeps the MFMA results in VGPRs where the
// epilogue reads them (no accumulation-register round trips).
// EPI: activation code in bits 0-1, bf16 output in bit 2, the SwiGLU
// multiply by `mul` (f32) in bit 3, the residual add of `mul` (y's element
// type, no activation) in bit 4 (compile time: the epilogue is inlined for
// every accumulator element).  KSPLIT: the launch splits K (`splits` > 1,
// partial sums, never persistent); without it `splits` and `split_stride`
// are ignored and the stage arithmetic folds as for one split.
template <int WM, int WN, int NST, bool FMA, int SEG, int EPI, bool PERSIST, bool KSPLIT,
          bool PROD>
__global__ __launch_bounds__(64 * (WM * WN + (PROD ? 4 : 0)))
__attribute__((amdgpu_waves_per_eu((WM * WN + (PROD ? 4 : 0) + 3) / 4 > 2
                                       ? (WM * WN + (PROD ? 4 : 0) + 3) / 4 : 2)))
void gemm_kernel(const int8_t *__restrict__ qa, const float *__restrict__ sa,
                 int32_t row_tiles, int32_t nblk, const uint8_t *__restrict__ w,
                 int64_t n_rows, int64_t m_rows, int32_t passes, int32_t m_tiles,
                 int32_t n_tiles, void *y, int64_t ldy, const void *mul,
                 int64_t ldg, int32_t splits_arg, int64_t split_stride) {
  constexpr int W = WM * WN;
  constexpr int P = PROD ? 4 : 0;      // producer waves
  constexpr int NI = PROD ? P : W;     // waves that issue the DMA ops
  typedef GemmStage<WM, WN, SEG, NI> St;
  static_assert(!(KSPLIT && PERSIST), "K splits run one tile per workgroup");
  static_assert(!(PROD && PERSIST), "producer waves serve one tile per workgroup");
  const int32_t splits = KSPLIT ? splits_arg : 1;
  static_assert(NST == 2 || NST == 4, "stage buffers");
  constexpr int BM = 32 * WM, BN = 32 * WN;
  // one LDS object per stage buffer (see above)
  __shared__ St st0, st1, st2, st3, st4;
  auto stage = [&](int i) __attribute__((always_inline)) -> St & {
    return i == 0 ? st0 : i == 1 ? st1 : i == 2 ? st2 : i == 3 ? st3 : st4;
  };

  // XCD-aware tile order: ids with the same (id % 8) share an XCD; each XCD
  // takes whole N-tiles (all their M-tiles and K splits), so a weight tile
  // is fetched into that XCD's L2 once.  Workgroups are persistent:
  // workgroup g takes ids g, g + G, g + 2G, ... (G = gridDim.x, a multiple
  // of 8, so all on one XCD); ids of the padding N-tiles (n_tile >= n_tiles)
  // are skipped.  With splits > 1 (never persistent) each id is one tile's
  // K split: passes [sp * passes / splits, (sp + 1) * passes / splits), its
  // partial sums stored at y + sp * split_stride.
  const int total = (n_tiles + 7) / 8 * 8 * m_tiles * splits;
  const int G = gridDim.x;
  auto tile_of = [&](int id, int &mt, int &nt, int &sp) __attribute__((always_inline)) {
    const int kk = id >> 3;
    if constexpr (KSPLIT) {
      const int per = m_tiles * splits;
      nt = (kk / per) * 8 + (id & 7);
      const int r = kk - (kk / per) * per;
      sp = r / m_tiles;
      mt = r - sp * m_tiles;
    } else {
      nt = (kk / m_tiles) * 8 + (id & 7);
      mt = kk % m_tiles;
      sp = 0;
    }
  };
  auto next_tile = [&](int id) __attribute__((always_inline)) {
    for (; id < total; id += G) {
      int mt, nt, sp;
      tile_of(id, mt, nt, sp);
      if (nt < n_tiles) break;
    }
    return id;
  };
  int id = next_tile(blockIdx.x);
  if (id >= total) return;  // uniform per workgroup
  int m_tile, n_tile, split;
  tile_of(id, m_tile, n_tile, split);
  int64_t m0 = (int64_t)m_tile * BM;
  int64_t n0 = (int64_t)n_tile * BN;
  // this workgroup's stages (four per pass) and the first one's index
  const int pass0 = KSPLIT ? split * passes / splits : 0;
  const int sbase = pass0 * (kPassBlocks / kStageBlocks);
  const int stages = (KSPLIT ? (split + 1) * passes / splits - pass0 : passes) *
                     (kPassBlocks / kStageBlocks);

  const int lane = threadIdx.x & 63;
  // PROD: waves W..W+3 are producers and issue every DMA op (op lists
  // strided over the four of them); the compute waves issue none.
  const int wave_all = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool producer = PROD && wave_all >= W;
  const int wave = producer ? 0 : wave_all;               // compute wave
  const int iw = PROD ? (producer ? wave_all - W : 0) : wave_all;  // issuer
  __builtin_assume(wave >= 0 && wave < W);
  __builtin_assume(iw >= 0 && iw < NI);
  const int wm = wave / WN, wn = wave % WN;
  const int li = lane & 31, lh = lane >> 5;
  const int64_t wrow = (int64_t)passes * kPassBytes;  // bytes per lane group

  // This wave's DMA ops.  Per op: a per-lane byte offset that depends on the
  // tile (a tensor is below 4 GiB), its kind and LDS destination (wave-
  // uniform); the per-stage part of each address is wave-uniform too (plus,
  // for S = 6, a per-lane block offset).
  enum { K_A = 0, K_B = 1, K_SA = 2, K_DW = 3 };
  constexpr int S4N = St::S4 > 0 ? St::S4 : 1;
  int kind[St::S16], abb[St::S16], dst16[St::S16], piece16[St::S16];
  int dst4[S4N], piece4[S4N];
  // S = 6: per-lane block offsets for r = 0, 2, 4 (Seg6), in three arrays
  // indexed only at compile time (a runtime index would put them in scratch)
  uint32_t x16r0[St::S16], x16r2[St::S16], x16r4[St::S16];
  const int q4 = lane >> 2;
#pragma unroll
  for (int u = 0; u < St::S16; ++u) {
    int o = iw + u * NI;
    if (o >= St::T16) o -= St::T16;
    abb[u] = o % kStageBlocks;
    piece16[u] = 0;
    if (o < St::CA) {
      kind[u] = K_A;
      dst16[u] = (int)offsetof(St, a) + o * 1024;
    } else if (o < St::CA + St::CB) {
      kind[u] = K_B;
      const int c = o - St::CA;
      piece16[u] = (lane & 3) ^ ((q4 >> 2) & 3);
      dst16[u] = (int)offsetof(St, b) + c * 1024;
    } else if (o < St::CA + St::CB + St::CS) {
      kind[u] = K_SA;
      dst16[u] = (int)offsetof(St, sa) + (o - St::CA - St::CB) * 1024;
    } else {
      kind[u] = K_DW;
      dst16[u] = (int)offsetof(St, dw16) + (o - St::CA - St::CB - St::CS) * 1024;
    }
  }
  // The wave-uniform part of a 16 B op's source for the stage whose first
  // block is kb at (unit, slot): base + kb * ca + (unit * kPassBytes & um) +
  // (slot * 16 & sm), with the base and coefficients resolved from the
  // op's kind once here, so that a stage costs a few scalar operations per
  // op and no branch on the kind.
  const uint8_t *obase[St::S16];
  uint32_t oca[St::S16], oum[St::S16], osm[St::S16];
#pragma unroll
  for (int u = 0; u < St::S16; ++u) {
    const bool a_ = kind[u] == K_A, b_ = kind[u] == K_B, s_ = kind[u] == K_SA;
    obase[u] = uniform_ptr(a_ ? (const uint8_t *)qa + abb[u] * 1024
                              : s_ ? (const uint8_t *)sa : w);
    oca[u] = a_ ? 1024u : s_ ? 128u : 0u;
    oum[u] = (a_ || s_) ? 0u : ~0u;
    osm[u] = b_ ? ~0u : 0u;
  }
#pragma unroll
  for (int u = 0; u < St::S4; ++u) {
    int o = iw + u * NI;
    if (o >= St::T4) o -= St::T4;
    // S > 1, column tile o/2, block 2(o%2) + lh of the stage, one f16 per
    // dword
    piece4[u] = 2 * (o % 2) + lh;
    dst4[u] = (int)offsetof(St, dw4) + o * 256;
  }
#pragma unroll
  for (int u = 0; u < St::S16; ++u) {
    const bool seg = SEG == 6 && kind[u] == K_B;
    x16r0[u] = seg ? Seg6::qs(0, piece16[u]) : 0u;
    x16r2[u] = seg ? Seg6::qs(2, piece16[u]) : 0u;
    x16r4[u] = seg ? Seg6::qs(4, piece16[u]) : 0u;
  }

  // The tile-dependent per-lane offsets of this wave's ops for the tile at
  // (mt, nn0).
  struct Offsets {
    uint32_t o16[St::S16], o4[S4N];
  };
  auto tile_offsets = [&](int mt, int64_t nn0) __attribute__((always_inline)) {
    Offsets of;
#pragma unroll
    for (int u = 0; u < St::S16; ++u) {
      int o = iw + u * NI;
      if (o >= St::T16) o -= St::T16;
      if (kind[u] == K_A) {
        const int64_t rt = min((int64_t)mt * WM + o / kStageBlocks, (int64_t)row_tiles - 1);
        of.o16[u] = (uint32_t)(rt * nblk * 1024 + li * 32 + lh * 16);
      } else if (kind[u] == K_B) {
        const int c = o - St::CA;
        const int ri = 16 * (c & 3) + q4;
        const int64_t n = min(nn0 + 32 * (c >> 2) + (ri & 31), n_rows - 1);
        const int piece = piece16[u];
        of.o16[u] = (uint32_t)((n >> 2) * wrow + (ri >> 5) * 1024 + (n & 3) * 256 +
                               (SEG == 1 ? piece * 16 : SEG == 4 ? piece * kPassBytes : 0));
      } else if (kind[u] == K_SA) {
        // lanes 0-31: row tile 2c, lanes 32-63: row tile 2c+1 (512 B each)
        const int c = o - St::CA - St::CB;
        const int64_t rt = min((int64_t)mt * WM + 2 * c + lh, (int64_t)row_tiles - 1);
        of.o16[u] = (uint32_t)(rt * nblk * 128 + li * 16);
      } else {
        // column tile c: lane l takes 16 B of group l/8's 128 B scale block
        const int c = o - St::CA - St::CB - St::CS;
        const int64_t ng = min(nn0 + 32 * c + 4 * (lane >> 3), n_rows - 4);
        of.o16[u] = (uint32_t)((ng >> 2) * wrow + kPassQs + (lane & 7) * 16);
      }
    }
#pragma unroll
    for (int u = 0; u < St::S4; ++u) {
      int o = iw + u * NI;
      if (o >= St::T4) o -= St::T4;
      const int64_t n = min(nn0 + 32 * (o / 2) + li, n_rows - 1);
      of.o4[u] = (uint32_t)((n >> 2) * wrow + kPassQs + 32 * (n & 3) +
                            (SEG == 4 ? piece4[u] * kPassBytes : 0));
    }
    return of;
  };

  // Wave-uniform position of a stage's first block in the unit layout:
  // S = 1, 4: its unit and slot; S = 6: unit 6P, slot q and r (Seg6).
  struct StagePos {
    int64_t unit;
    int slot, r;
  };
  auto stage_pos = [&](int kb) __attribute__((always_inline)) {
    StagePos sp;
    if constexpr (SEG == 6) {
      const int pass = kb / 96, rem = kb - 96 * pass;
      sp.unit = 6 * pass;
      sp.slot = rem / 6;
      sp.r = rem - 6 * sp.slot;
    } else {
      locate<SEG>(kb, sp.unit, sp.slot);
      sp.r = 0;
    }
    return sp;
  };

  // Issue DMA op j (j < S16: 16 B class, else 4 B class) of stage s into
  // buffer `buf`: branch-free, the same instruction sequence in every wave.
  auto issue_op = [&](int s, St &buf, auto J, const Offsets &of) __attribute__((always_inline)) {
    constexpr int j = decltype(J)::value;
    const int kb = (sbase + s) * kStageBlocks;  // first block of the stage
    const StagePos sp = stage_pos(kb);
    int8_t *lds_base = (int8_t *)&buf;
    if constexpr (j < St::S16) {
      const int u = j;
      const uint32_t off = (uint32_t)kb * oca[u] + ((uint32_t)sp.unit * kPassBytes & oum[u]) +
                           ((uint32_t)sp.slot * 16u & osm[u]);
      uint32_t extra = 0;
      if constexpr (SEG == 6) {
        // masks, not a select between array elements (which the compiler
        // turns into a load through a selected pointer, forcing the arrays
        // into scratch)
        const uint32_t m0 = sp.r == 0 ? ~0u : 0u, m2 = sp.r == 2 ? ~0u : 0u;
        extra = (x16r0[u] & m0) | (x16r2[u] & m2) | (x16r4[u] & ~(m0 | m2));
      }
      bdma16(buffer_of(obase[u]), of.o16[u] + extra, off, lds_base + dst16[u]);
    } else {
      const int u = j - St::S16;
      const uint32_t soff = (uint32_t)(sp.unit * kPassBytes + 2 * (sp.slot & ~1));
      uint32_t extra = 0;
      if constexpr (SEG == 6) extra = Seg6::scale(sp.r, sp.slot, piece4[u]);
      bdma4(buffer_of(w), of.o4[u] + extra, soff, lds_base + dst4[u]);
    }
  };
  auto issue = [&](int s, St &buf, const Offsets &of) __attribute__((always_inline)) {
    static_for<St::OPS>([&](auto J) __attribute__((always_inline)) { issue_op(s, buf, J, of); });
  };

  float acc[16];
  const v16i zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  // SwiGLU gate values or residuals: this lane's 16, loaded at the start of
  // the last group of stages so that their latency hides behind it (indices
  // clamped, no branch: a branch around a load would disturb the DMA wait
  // tracking).  bf16 residuals are widened exactly.
  float gpre[16];
  auto prefetch_gate = [&]() __attribute__((always_inline)) {
    if constexpr ((EPI & 24) != 0) {
      const int64_t nc = min(n0 + 32 * wn + li, n_rows - 1);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t mc = min(m0 + 32 * wm + 8 * (v >> 2) + 4 * lh + (v & 3), m_rows - 1);
        if constexpr ((EPI & 16) != 0 && (EPI & 4) != 0)
          gpre[v] = bf16_to_float(((const uint16_t *)mul)[mc * ldg + nc]);
        else
          gpre[v] = ((const float *)mul)[mc * ldg + nc];
      }
    }
  };
  const int bsw = (lane >> 2) & 3;  // swizzle of this lane's weight run

  // Scale tiles of blocks kb+2k (lanes 0-31) and kb+2k+1 (lanes 32-63): the
  // LDS reads (read_scales) and, one block later, the f16 half select and
  // the outer-product MFMA (scale_tile).
  typedef float v32f __attribute__((ext_vector_type(32)));
  struct ScaleRaw {
    float fa;
    uint32_t d;
  };
  auto read_scales = [&](int kb, St &buf, int k) __attribute__((always_inline)) -> ScaleRaw {
    ScaleRaw r;
    r.fa = buf.sa[wm][2 * k + lh][li];
    if constexpr (SEG == 1) {
      // this lane's row n = li of column tile wn: group li/4, row li%4; the
      // f16 pair (2k, 2k+1) of the stage's slots
      r.d = ((const uint32_t *)buf.dw16[wn])[(li >> 2) * 32 + (li & 3) * 8 +
                                             ((kb & (kPassBlocks - 1)) >> 1) + k];
    } else {
      r.d = buf.dw4[wn][k][lane];
    }
    return r;
  };
  auto scale_tile = [&](int kb, const ScaleRaw &r, int k) __attribute__((always_inline)) -> v32f {
    uint32_t h;
    if constexpr (SEG == 1) {
      h = lh ? r.d >> 16 : r.d & 0xffffu;  // half lh of the pair
    } else if constexpr (SEG == 4) {
      // the stage's four blocks share one slot
      int64_t ub;
      int sb;
      locate<SEG>(kb, ub, sb);
      h = (sb & 1) ? r.d >> 16 : r.d & 0xffffu;
    } else {
      const StagePos sp = stage_pos(kb);
      h = ((sp.slot + Seg6::wrap(sp.r, 2 * k + lh)) & 1) ? r.d >> 16 : r.d & 0xffffu;
    }
    const float fb = half_bits_to_float(h);
    const v32f z32 = {};
    return __builtin_amdgcn_mfma_f32_32x32x1f32(r.fa, fb, z32, 0, 0, 0);
  };
  // A block's MFMA operands: the A piece (row tile wm) and B piece (column
  // tile wn), read from LDS a block before the MFMA that takes them.
  struct Frag {
    v4i a, b;
  };
  auto read_frag = [&](St &buf, int bb) __attribute__((always_inline)) -> Frag {
    Frag f;
    f.a = *(const v4i *)(buf.a[wm][bb] + lane * 16);
    f.b = *(const v4i *)(buf.b[wn] + lane * 64 + 16 * (bb ^ bsw));
    return f;
  };
  auto dots = [&](const Frag &f) __attribute__((always_inline)) -> v16i {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a, f.b, zero, 0, 0, 0);
  };

  // The block pipeline.  Entering block g (stage s = g / 4, bb = g % 4) a
  // wave holds block g's integer dots (c_cur), its pair's scale tile
  // (f_cur), block g+1's operands (fr) and, for odd g, the raw scales of
  // the pair g+1 starts (sr).  Block g then issues, in this order: block
  // g+1's MFMA, for odd g the next pair's scale MFMA, the LDS reads of block
  // g+2's operands (and, for even g, of the pair at g+2's scales) and its
  // share of the DMA ops; only then its own epilogue, 32 VALU ops that
  // cover the latency of everything just issued.  A scheduling barrier
  // keeps that order.  Block g+2 lies in stage s+1 for bb >= 2, so the
  // hand-off of stage s+1 (vmcnt wait, workgroup barrier) sits in block
  // bb = 2, after that block's MFMA: every LDS read of stage s's buffer
  // (the last at bb = 1, its operands taken by that MFMA) has then been
  // waited on by its wave, so the buffer is free once the barrier is
  // passed.  The DMA of stage s+4 into it starts right there: the first
  // half of its ops goes out in blocks 2 and 3 of stage s, the second half
  // in blocks 0 and 1 of stage s+1, 11-14 blocks before its hand-off.
  // Waves must never pass a hand-off with a read of the freed buffer still
  // outstanding.
  v16i c_cur;
  v32f f_cur;
  Frag fr;
  ScaleRaw sr;
  // Ops j < kHalf of a stage form its first half.  At the hand-off of
  // stage s+1, the ops of stages s+2 and s+3 may still be outstanding.
  constexpr int kHalf = (St::OPS + 1) / 2;
  constexpr int kMidOps = 2 * St::OPS;
  // Stage s reads buffers buf (its own) and buf1 (stage s+1's) and issues
  // the second half of stage sa (into abuf) and the first half of stage sb
  // (into bbuf).
  auto compute = [&](int s, St &buf, St &buf1, int sa, St &abuf, const Offsets &aof, int sb,
                     St &bbuf, const Offsets &bof) __attribute__((always_inline)) {
    const int kb = (sbase + s) * kStageBlocks;
    static_for<kStageBlocks>([&](auto BB) __attribute__((always_inline)) {
      constexpr int bb = decltype(BB)::value;
      v16i c_next = dots(fr);
      v32f f_next;
      if constexpr ((bb & 1) != 0) f_next = scale_tile(bb == 1 ? kb : kb + kStageBlocks, sr, bb == 1 ? 1 : 0);
      // The MFMAs are pure operations: instruction selection would place
      // them next to their first use (the next block's epilogue), which
      // then waits for them.  An empty asm that takes their results keeps
      // them here, ahead of this block's epilogue.
      asm volatile("" ::"v"(c_next));
      if constexpr ((bb & 1) != 0) asm volatile("" ::"v"(f_next));
      if constexpr (bb == 2) {
        if constexpr (!PROD) wait_vmcnt<kMidOps>();
        stage_barrier();
      }
      if constexpr (bb < 2) {
        fr = read_frag(buf, bb + 2);
      } else {
        fr = read_frag(buf1, bb - 2);
      }
      if constexpr (bb == 0) sr = read_scales(kb, buf, 1);
      if constexpr (bb == 2) sr = read_scales(kb + kStageBlocks, buf1, 0);
      if constexpr (!PROD) static_for<St::OPS>([&](auto J) __attribute__((always_inline)) {
        constexpr int j = decltype(J)::value;
        if constexpr (j >= kHalf && bb < 2) {
          if constexpr ((j - kHalf) * 2 / (St::OPS - kHalf) == bb) issue_op(sa, abuf, J, aof);
        }
        if constexpr (j < kHalf && bb >= 2) {
          if constexpr (2 + j * 2 / kHalf == bb) issue_op(sb, bbuf, J, bof);
        }
      });
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float dotf = (float)c_cur[v];
        const float f = f_cur[16 * (bb & 1) + v];
        if (FMA) {
          acc[v] = __builtin_fmaf(dotf, f, acc[v]);
        } else {
          const float contrib = dotf * f;
          acc[v] = acc[v] + contrib;
        }
      }
      // The accumulators are pinned here (an empty asm that reads and
      // writes them), so an epilogue cannot sink below later blocks' MFMAs
      // and pile up their results in registers.
#pragma unroll
      for (int v = 0; v < 16; ++v) asm volatile("" : "+v"(acc[v]));
      __builtin_amdgcn_sched_barrier(0);
      c_cur = c_next;
      if constexpr ((bb & 1) != 0) f_cur = f_next;
    });
  };

  // Every DMA is unconditional: a branch around one makes the compiler's
  // wait tracking merge states and wait for all loads before the next LDS
  // read.  The DMA stream runs on across tiles: the last group of stages
  // issues the next tile's first NST stages, so their latency hides behind
  // that group and this tile's epilogue.  After the last tile they reload
  // the tile's own last stage into buffers nobody reads again.
  static_assert(NST == 4, "the block pipeline runs a ring of four stages");
  static_assert(kPassBlocks / kStageBlocks % NST == 0, "stages per unit");
  const int last = stages - 1;
  Offsets cur = tile_offsets(m_tile, n0);
  auto prologue_dma = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NST - 1; ++i) issue(min(i, last), stage(i), cur);
    static_for<kHalf>([&](auto J) __attribute__((always_inline)) {
      issue_op(min(NST - 1, last), stage(NST - 1), J, cur);
    });
    wait_vmcnt<(NST - 2) * St::OPS + kHalf>();
  };
  if constexpr (PROD) {
    if (producer) {
      // The compute waves' DMA schedule, stage by stage, with the same
      // barriers: the prologue's, then one per stage, after which the
      // buffer of the stage just consumed is free.  Stage s: the second
      // half of stage s+3 (into the buffer freed at stage s-1's barrier),
      // the wait for stage s+1, the barrier, the first half of stage s+4
      // (into stage s's buffer); past the tile's last stage, the last stage
      // again (into buffers nobody reads).  ring() selects the four ring
      // buffers by a runtime index (stage() would also reference the
      // unused fifth, and allocate it).
      auto ring = [&](int i) __attribute__((always_inline)) -> St & {
        return i == 0 ? st0 : i == 1 ? st1 : i == 2 ? st2 : st3;
      };
      prologue_dma();
      stage_barrier();
      for (int s = 0; s < stages; ++s) {
        const int i = s & (NST - 1);
        St &abuf = ring((i + NST - 1) & (NST - 1));
        static_for<St::OPS>([&](auto J) __attribute__((always_inline)) {
          if constexpr (decltype(J)::value >= kHalf) issue_op(min(s + NST - 1, last), abuf, J, cur);
        });
        wait_vmcnt<kMidOps>();
        stage_barrier();
        St &bbuf = ring(i);
        static_for<St::OPS>([&](auto J) __attribute__((always_inline)) {
          if constexpr (decltype(J)::value < kHalf) issue_op(min(s + NST, last), bbuf, J, cur);
        });
      }
      wait_vmcnt<0>();
      return;
    }
  } else {
    prologue_dma();
  }
  // pipeline prologue: stage 0 handed off, block 0's MFMA and its pair's
  // scale tile issued, block 1's operands read
  stage_barrier();
  {
    const Frag f0 = read_frag(stage(0), 0);
    fr = read_frag(stage(0), 1);
    const ScaleRaw r0 = read_scales(sbase * kStageBlocks, stage(0), 0);
    c_cur = dots(f0);
    f_cur = scale_tile(sbase * kStageBlocks, r0, 0);
  }

  for (;;) {
    const int id_next = PERSIST ? next_tile(id + G) : total;
    const bool more = PERSIST && id_next < total;
    // persistent launches have one split: the next tile's is 0 as well
    int m_next = m_tile, n_next = n_tile, split_next = 0;
    if (more) tile_of(id_next, m_next, n_next, split_next);
    (void)split_next;
    Offsets nxt;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;

    // One group of NST stages (static buffer indices).  The last group is
    // peeled off when it differs: with PERSIST the stages it issues past
    // the end are the next tile's, and with the SwiGLU multiply it
    // prefetches the gate values.  Without PERSIST (one tile per
    // workgroup) those stages reload the tile's last stage into buffers
    // nobody reads again.
    auto group = [&](int s0, auto LAST) __attribute__((always_inline)) {
      constexpr bool is_last = decltype(LAST)::value;
      if constexpr (is_last) {
        prefetch_gate();
        if constexpr (PERSIST) nxt = tile_offsets(m_next, (int64_t)n_next * BN);
      }
#pragma unroll
      for (int i = 0; i < NST; ++i) {
        const int s = s0 + i;
        // stage s finishes stage s+3's DMA (into stage s-1's buffer) and
        // starts stage s+4's (into its own)
        St &abuf = stage((i + NST - 1) % NST);
        St &buf1 = stage((i + 1) % NST);
        if (PERSIST && is_last) {
          if (i == 0)
            compute(s, stage(i), buf1, last, abuf, cur, 0, stage(i), nxt);
          else
            compute(s, stage(i), buf1, i - 1, abuf, nxt, i, stage(i), nxt);
        } else {
          compute(s, stage(i), buf1, min(s + NST - 1, last), abuf, cur, min(s + NST, last),
                  stage(i), cur);
        }
      }
    };
    if constexpr (PERSIST || (EPI & 24) != 0) {
      for (int s0 = 0; s0 < stages - NST; s0 += NST) group(s0, std::false_type{});
      group(stages - NST, std::true_type{});
    } else {
      for (int s0 = 0; s0 < stages; s0 += NST) group(s0, std::false_type{});
    }

    const int64_t n = n0 + 32 * wn + li;
    // this split's part of the output (the whole output with one split)
    char *const ys = (char *)y + (int64_t)split * split_stride * ((EPI & 4) != 0 ? 2 : 4);
    // the activation over all 16 values (rows or columns past the end too,
    // whose results are not stored): one straight-line sequence
    activate_array(acc, EPI & 3);
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int64_t m = m0 + 32 * wm + 8 * (v >> 2) + 4 * lh + (v & 3);
      if (m < m_rows && n < n_rows) {
        float o = acc[v];
        if constexpr ((EPI & 8) != 0) {
          // SwiGLU: times the gate's activated output (FuseSiluMul's mul)
          const float g = gpre[v];
          o = (EPI & 4) != 0 ? bf16_to_float(float_to_bf16(g)) * bf16_to_float(float_to_bf16(o))
                             : g * o;
        }
        if constexpr ((EPI & 16) != 0) {
          // residual add (AddOpLowering): the result as stored, plus r, in f32
          o = (EPI & 4) != 0 ? bf16_to_float(float_to_bf16(o)) + gpre[v] : o + gpre[v];
        }
        // non-temporal: the output is written once and not read back here
        // (op time -3 % at M = 256 and 1024)
        if constexpr ((EPI & 4) != 0)
          __builtin_nontemporal_store(float_to_bf16(o), (uint16_t *)ys + m * ldy + n);
        else
          __builtin_nontemporal_store(o, (float *)ys + m * ldy + n);
      }
    }
    if (!more) break;
    id = id_next;
    m_tile = m_next;
    n_tile = n_next;
    m0 = (int64_t)m_tile * BM;
    n0 = (int64_t)n_tile * BN;
    cur = nxt;
  }
  // no DMA may land in LDS after the workgroup has released it
  wait_vmcnt<0>();
}

// The K splits' reduction and the epilogue: y = epi(part[0] + part[1] + ...
// + part[splits - 1]) in that order (a fixed order, so the same inputs give
// the same bits), part [splits][m][n] f32 from gemm_kernel's split
// launches; the epilogue is gemm_kernel's (activation, SwiGLU multiply,
// residual add, bf16 store).  One thread per 4 consecutive outputs of a row
// (n % 4 == 0).
template <int EPI>
__global__ __launch_bounds__(256) void gemm_reduce_kernel(
    const float *__restrict__ part, int32_t splits, int64_t split_stride, int64_t m,
    int64_t n, void *y, int64_t ldy, const void *mul, int64_t ldg) {
  const int64_t nq = n >> 2;
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (q >= m * nq) return;
  const int64_t row = q / nq, c0 = (q - row * nq) * 4;
  const float *p = part + row * n + c0;
  float4 a = *(const float4 *)p;
  for (int32_t i = 1; i < splits; ++i) {
    const float4 t = *(const float4 *)(p + (int64_t)i * split_stride);
    a.x = a.x + t.x;
    a.y = a.y + t.y;
    a.z = a.z + t.z;
    a.w = a.w + t.w;
  }
  float v[4] = {a.x, a.y, a.z, a.w};
  activate_array(v, EPI & 3);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t col = c0 + j;
    float o = v[j];
    if constexpr ((EPI & 8) != 0) {
      const float g = ((const float *)mul)[row * ldg + col];
      o = (EPI & 4) != 0 ? bf16_to_float(float_to_bf16(g)) * bf16_to_float(float_to_bf16(o))
                         : g * o;
    }
    if constexpr ((EPI & 16) != 0) {
      const float r = (EPI & 4) != 0 ? bf16_to_float(((const uint16_t *)mul)[row * ldg + col])
                                     : ((const float *)mul)[row * ldg + col];
      o = (EPI & 4) != 0 ? bf16_to_float(float_to_bf16(o)) + r : o + r;
    }
    if constexpr ((EPI & 4) != 0)
      ((uint16_t *)y)[row * ldy + col] = float_to_bf16(o);
    else
      ((float *)y)[row * ldy + col] = o;
  }
}

}  // namespace

template <int EPI>
static void launch_reduce_e(const GemmLaunch &l, hipStream_t s) {
  const void *mp = (EPI & 16) != 0 ? l.add : (const void *)l.mul;
  const int64_t ld = (EPI & 16) != 0 ? l.ldr : l.ldg;
  const int64_t quads = l.m * (l.rows / 4);
  hipLaunchKernelGGL((gemm_reduce_kernel<EPI>), dim3((unsigned)((quads + 255) / 256)), dim3(256),
                     0, s, l.part, l.splits, l.m * l.rows, l.m, l.rows, l.y, l.ldy, mp, ld);
}

// The epilogue code of a launch: activation in bits 0-1, bf16 output in bit
// 2, the SwiGLU multiply in bit 3, the residual add in bit 4.
static int epi_of(const GemmLaunch &l) {
  if (l.mul) return l.y_bf16 ? 12 : 8;   // the SwiGLU up linear: no activation
  if (l.add) return l.y_bf16 ? 20 : 16;  // linear + residual add: no activation
  return (l.activation & 3) | (l.y_bf16 ? 4 : 0);
}

static void launch_reduce(const GemmLaunch &l, hipStream_t s) {
  switch (epi_of(l)) {
    case 1: return launch_reduce_e<1>(l, s);
    case 2: return launch_reduce_e<2>(l, s);
    case 3: return launch_reduce_e<3>(l, s);
    case 4: return launch_reduce_e<4>(l, s);
    case 5: return launch_reduce_e<5>(l, s);
    case 6: return launch_reduce_e<6>(l, s);
    case 7: return launch_reduce_e<7>(l, s);
    case 8: return launch_reduce_e<8>(l, s);
    case 12: return launch_reduce_e<12>(l, s);
    case 16: return launch_reduce_e<16>(l, s);
    case 20: return launch_reduce_e<20>(l, s);
    default: return launch_reduce_e<0>(l, s);
  }
}

template <int WM, int WN, int NST, bool FMA, int SEG, int EPI>
static void launch_gemm_k(const GemmLaunch &l, int32_t passes, int32_t m_tiles,
                          int32_t n_tiles, unsigned grid, hipStream_t s) {
  // persistent (several tiles per workgroup) only when the tiles outnumber
  // the resident workgroups, and only for the 12-wave shape and S = 1 or 4
  // (with S = 6 the next tile's offsets spill registers)
  constexpr bool kPersist = WM * WN >= 12 && SEG != 6;
  // K splits (never persistent) store f32 partial sums, [splits][m][rows]
  // at l.part, for launch_reduce (EPI 0)
  const int32_t splits = l.splits > 1 ? l.splits : 1;
  const unsigned total = (unsigned)((n_tiles + 7) / 8 * 8 * m_tiles * splits);
  void *const y = splits > 1 ? (void *)l.part : l.y;
  const int64_t ldy = splits > 1 ? l.rows : l.ldy;
  const int64_t stride = splits > 1 ? l.m * l.rows : 0;
  // the epilogue's second operand: the SwiGLU gate or the residual
  const void *mp = (EPI & 16) != 0 ? l.add : (const void *)l.mul;
  const int64_t ld = (EPI & 16) != 0 ? l.ldr : l.ldg;
  // producer waves: when the workgroups fit one per CU (not persistent).
  // With the twelve-wave shape the compute waves are held to 128 VGPRs,
  // which spills inside the stage loop except with S = 1 and no SwiGLU
  // multiply or residual (M = 1024, N = 2560, K = 9216, S = 6, measured 2 %
  // slower with them), so only that form takes them there.
  constexpr bool kProd =
      WM * WN == 4 || (WM * WN == 12 && SEG == 1 && (EPI & 24) == 0);
  const bool prod = kProd && total <= (unsigned)cu_count();
  constexpr int kThreads = 64 * WM * WN, kThreadsP = 64 * (WM * WN + 4);
  if (splits > 1) {
    if constexpr (EPI == 0) {
      if (prod)
        hipLaunchKernelGGL((gemm_kernel<WM, WN, NST, FMA, SEG, 0, false, true, kProd>), dim3(total),
                           dim3(kThreadsP), 0, s, l.qa, l.sa, l.row_tiles, l.nblk,
                           l.w, l.rows, l.m, passes, m_tiles, n_tiles, y, ldy,
                           mp, ld, splits, stride);
      else
        hipLaunchKernelGGL((gemm_kernel<WM, WN, NST, FMA, SEG, 0, false, true, false>), dim3(total),
                           dim3(64 * WM * WN), 0, s, l.qa, l.sa, l.row_tiles, l.nblk,
                           l.w, l.rows, l.m, passes, m_tiles, n_tiles, y, ldy,
                           mp, ld, splits, stride);
    }
  } else if (kPersist && grid < total) {
    hipLaunchKernelGGL((gemm_kernel<WM, WN, NST, FMA, SEG, EPI, kPersist, false, false>), dim3(grid),
                       dim3(kThreads), 0, s, l.qa, l.sa, l.row_tiles, l.nblk,
                       l.w, l.rows, l.m, passes, m_tiles, n_tiles, y, ldy,
                       mp, ld, 1, 0);
  } else if (prod) {
    hipLaunchKernelGGL((gemm_kernel<WM, WN, NST, FMA, SEG, EPI, false, false, kProd>), dim3(total),
                       dim3(kThreadsP), 0, s, l.qa, l.sa, l.row_tiles, l.nblk,
                       l.w, l.rows, l.m, passes, m_tiles, n_tiles, y, ldy,
                       mp, ld, 1, 0);
  } else {
    hipLaunchKernelGGL((gemm_kernel<WM, WN, NST, FMA, SEG, EPI, false, false, false>), dim3(total),
                       dim3(64 * WM * WN), 0, s, l.qa, l.sa, l.row_tiles, l.nblk,
                       l.w, l.rows, l.m, passes, m_tiles, n_tiles, y, ldy,
                       mp, ld, 1, 0);
  }
}

template <int WM, int WN, int NST, bool FMA, int SEG>
static void launch_gemm_e(const GemmLaunch &l, int32_t passes, int32_t m_tiles,
                          int32_t n_tiles, unsigned grid, hipStream_t s) {
  // activation and output type are template arguments: inlined for every
  // accumulator element, runtime switches bloat the kernel and slow it
  // K splits: plain f32 partial sums, then the reduction applies the epilogue
  if (l.splits > 1) {
    launch_gemm_k<WM, WN, NST, FMA, SEG, 0>(l, passes, m_tiles, n_tiles, grid, s);
    return launch_reduce(l, s);
  }
#define LLMCP_GEMM_EPI(E) \
  case E: return launch_gemm_k<WM, WN, NST, FMA, SEG, E>(l, passes, m_tiles, n_tiles, grid, s);
  switch (epi_of(l)) {
    LLMCP_GEMM_EPI(1) LLMCP_GEMM_EPI(2) LLMCP_GEMM_EPI(3) LLMCP_GEMM_EPI(4)
    LLMCP_GEMM_EPI(5) LLMCP_GEMM_EPI(6) LLMCP_GEMM_EPI(7) LLMCP_GEMM_EPI(8)
    LLMCP_GEMM_EPI(12) LLMCP_GEMM_EPI(16) LLMCP_GEMM_EPI(20)
    default: return launch_gemm_k<WM, WN, NST, FMA, SEG, 0>(l, passes, m_tiles, n_tiles, grid, s);
  }
#undef LLMCP_GEMM_EPI
}

int cu_count() {
  static std::atomic<int> cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
            hipSuccess || n <= 0)
      n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

template <int WM, int WN, int NST, bool FMA>
static hipError_t launch_gemm_t(const GemmLaunch &l, hipStream_t s) {
  const int32_t passes = (int32_t)passes_for(l.cols);
  const int32_t m_tiles = (int32_t)((l.m + 32 * WM - 1) / (32 * WM));
  const int32_t n_tiles = (int32_t)((l.rows + 32 * WN - 1) / (32 * WN));
  const int32_t n_tiles8 = (n_tiles + 7) / 8 * 8;
  // persistent workgroups: at most as many as are resident at once (one or
  // two per CU, by LDS), a multiple of 8 so that each stays on its XCD
  const int64_t resident = (int64_t)cu_count() * (WM * WN >= 12 ? 1 : 2) / 8 * 8;
  const unsigned grid =
      (unsigned)std::min<int64_t>((int64_t)n_tiles8 * m_tiles, std::max<int64_t>(8, resident));
  // the weight's unit layout is fixed at registration (seg_for)
  switch (seg_for(passes)) {
    case 6: launch_gemm_e<WM, WN, NST, FMA, 6>(l, passes, m_tiles, n_tiles, grid, s); break;
    case 4: launch_gemm_e<WM, WN, NST, FMA, 4>(l, passes, m_tiles, n_tiles, grid, s); break;
    default: launch_gemm_e<WM, WN, NST, FMA, 1>(l, passes, m_tiles, n_tiles, grid, s);
  }
  return hipGetLastError();
}

// 128 x 96 workgroups (12 waves, one per CU by LDS): at M = 1024, N = 9216
// that is 768 workgroups, three full rounds on 256 CUs.  Up to 64 rows:
// 64 x 64 workgroups (4 waves, two per CU).
static bool small_shape(int64_t m) { return m <= 64; }

template <bool FMA>
static hipError_t launch_gemm_shape(const GemmLaunch &l, hipStream_t s) {
  if (small_shape(l.m)) return launch_gemm_t<2, 2, 4, FMA>(l, s);
  return launch_gemm_t<4, 3, 4, FMA>(l, s);
}

hipError_t launch_gemm(const GemmLaunch &l, hipStream_t s) {
  if (l.splits > 1) {
    if (!l.part || l.splits > passes_for(l.cols) || l.rows % 4 != 0) return hipErrorInvalidValue;
  }
  return l.fma ? launch_gemm_shape<true>(l, s) : launch_gemm_shape<false>(l, s);
}

int32_t gemm_splits_for(int64_t m, int64_t rows, int64_t cols, int32_t forced) {
  const int32_t passes = (int32_t)passes_for(cols);
  if (m <= 1 || passes <= 1) return 1;
  if (forced > 0) return std::min(forced, passes);
  // As many splits as keep tiles x splits within one workgroup per CU, and
  // at most max(3, passes / 3) (three passes per split where K has nine or
  // more).  Measured op time (quantizer, GEMM, reduction) against EXACT,
  // splits in brackets:
  //   N = 2560, K = 9216: M = 64 65.9 -> 26.9 us (6); M = 128 109.8 -> 37.6
  //     (6; 9 splits 50.1); M = 256 109.2 -> 48.7 (4; 6 splits 61.6);
  //     M = 512 107.7 -> 72.8 (2; 3 splits 92.2); M = 1024 127.8, every
  //     split slower.
  //   N = 2560, K = 2560: M = 64 17.5 -> 14.8 (3; 5 splits 14.2);
  //     M = 256 29.1 -> 22.9 (3; 4 splits 23.3).
  //   N = 7680, K = 2560: M = 128 30.1 -> 24.8 (3; 4 splits 36.5);
  //     M = 256 31.9, every split slower.
  //   N = 9216, K = 2560: M = 128 32.4 -> 28.8 (2); M = 16 / 64 / 256
  //     slower split.
  // A second workgroup per CU (the 64-row tiles fit two) shares the CU's
  // operand delivery, so the bound is one per CU for both tile shapes.
  const int64_t tiles = small_shape(m) ? ((m + 63) / 64) * ((rows + 63) / 64)
                                       : ((m + 127) / 128) * ((rows + 95) / 96);
  const int64_t by_cus = (int64_t)cu_count() / tiles;
  const int64_t by_passes = std::max<int64_t>(std::min<int64_t>(passes, 3), passes / 3);
  return (int32_t)std::max<int64_t>(1, std::min(by_cus, by_passes));
}

}  // namespace llmcp_q8
