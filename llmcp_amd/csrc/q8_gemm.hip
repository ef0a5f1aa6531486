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
// direct-to-LDS loads (global_load_lds: lane l's bytes land at base +
// l * size), NST stage buffers deep, so NST - 1 stages are in flight while
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
constexpr int kStageBlocks = 4;

template <int WM, int WN, int SEG>
struct GemmStage {
  static constexpr int DWC = SEG > 1 ? 2 : 1;  // dw pieces per column tile
  static constexpr int CA = WM * kStageBlocks;  // A tiles (1 KiB)
  static constexpr int CS = WM * 2;             // sa pairs (256 B)
  static constexpr int CB = WN * 4;             // weight chunks (1 KiB)
  static constexpr int CD = WN * DWC;           // dw pieces (256 B)
  static constexpr int TOTAL = CA + CS + CB + CD;
  static constexpr int W = WM * WN;
  // DMA instructions per wave and stage: op o goes to wave o % W.
  static constexpr int ops_of(int wave) {
    return TOTAL / W + (wave < TOTAL % W ? 1 : 0);
  }
  __align__(16) int8_t a[WM][kStageBlocks][1024];
  __align__(16) int8_t b[WN][4 * 1024];
  __align__(16) float sa[WM][2][64];
  __align__(16) uint32_t dw[WN][DWC][64];
};

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ void dma16(const void *g, void *lds_base) {
  __builtin_amdgcn_global_load_lds(g, (lds_void *)lds_base, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void *g, void *lds_base) {
  __builtin_amdgcn_global_load_lds(g, (lds_void *)lds_base, 4, 0, 0);
}

// s_waitcnt vmcnt(n) (gfx9 encoding; expcnt and lgkmcnt not waited on).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | 0x70 | 0xF00 | ((N >> 4) << 14));
}
// Waits until at most n of this wave's vector-memory ops are outstanding
// (n wave-uniform, at most NMAX).
template <int NMAX>
__device__ __forceinline__ void wait_vmcnt_dyn(int n) {
  if constexpr (NMAX > 0) {
    if (n >= NMAX) {
      wait_vmcnt<NMAX>();
      return;
    }
    wait_vmcnt_dyn<NMAX - 1>(n);
  } else {
    wait_vmcnt<0>();
  }
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

// Byte offset of block b's slot within its group's units, for the segment
// sizes whose blocks do not sit at a fixed lane offset from the stage's
// first block (S = 6).
template <int SEG>
__device__ __forceinline__ uint32_t block_offset(int b) {
  int64_t unit;
  int slot;
  locate<SEG>(b, unit, slot);
  return (uint32_t)(unit * kPassBytes + slot * 16);
}

// The occupancy the LDS allows (12 waves: one workgroup per CU, three waves
// per SIMD; 4 waves: two workgroups per CU) is declared so that the kernel
// stays within 256 VGPRs, which keeps the MFMA results in VGPRs where the
// epilogue reads them (no accumulation-register round trips).
template <int WM, int WN, int NST, bool FMA, int SEG, int EPI>
__global__ __launch_bounds__(64 * WM * WN)
__attribute__((amdgpu_waves_per_eu(WM * WN >= 12 ? 3 : 2)))
void gemm_kernel(const int8_t *__restrict__ qa, const float *__restrict__ sa,
                 int32_t row_tiles, int32_t nblk, const uint8_t *__restrict__ w,
                 int64_t n_rows, int64_t m_rows, int32_t passes, int32_t m_tiles,
                 int32_t n_tiles, void *__restrict__ y, int64_t ldy) {
  typedef GemmStage<WM, WN, SEG> St;
  static_assert(NST >= 2 && NST <= 5, "stage buffers");
  constexpr int W = WM * WN;
  constexpr int BM = 32 * WM, BN = 32 * WN;
  constexpr int OPS_MAX = St::ops_of(0);
  constexpr int UNIT_S4 = SEG == 4;  // blocks of a stage: one slot, 4 units
  // one LDS object per stage buffer (see above)
  __shared__ St st0, st1, st2, st3, st4;
  auto stage = [&](int i) -> St & {
    return i == 0 ? st0 : i == 1 ? st1 : i == 2 ? st2 : i == 3 ? st3 : st4;
  };

  // XCD-aware tile order: ids with the same (id % 8) share an XCD; each XCD
  // takes whole N-tiles (all their M-tiles), so a weight tile is fetched
  // into that XCD's L2 once.
  const int id = blockIdx.x;
  const int xcd = id & 7;
  const int kk = id >> 3;
  const int n_tile = (kk / m_tiles) * 8 + xcd;
  const int m_tile = kk % m_tiles;
  if (n_tile >= n_tiles) return;  // uniform per workgroup
  const int64_t m0 = (int64_t)m_tile * BM;
  const int64_t n0 = (int64_t)n_tile * BN;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  __builtin_assume(wave >= 0 && wave < W);
  const int wm = wave / WN, wn = wave % WN;
  const int li = lane & 31, lh = lane >> 5;
  const int stages = passes * (kPassBlocks / kStageBlocks);
  const int ops = St::ops_of(wave);
  const int64_t wrow = (int64_t)passes * kPassBytes;  // bytes per lane group

  // Loop-invariant per-lane byte offsets of this wave's DMA ops (a tensor
  // is below 4 GiB); the per-stage part of each address is wave-uniform
  // (plus, for S = 6, a per-lane block offset).
  uint32_t off[OPS_MAX];
  int bpiece[OPS_MAX];  // S = 6: the block of the stage this lane loads
#pragma unroll
  for (int u = 0; u < OPS_MAX; ++u) {
    const int o = wave + u * W;
    off[u] = 0;
    bpiece[u] = 0;
    if (o < St::CA) {
      const int64_t rt = min((int64_t)m_tile * WM + o / kStageBlocks, (int64_t)row_tiles - 1);
      off[u] = (uint32_t)(rt * nblk * 1024 + li * 32 + lh * 16);
    } else if (o < St::CA + St::CS) {
      const int c = o - St::CA;
      const int64_t rt = min((int64_t)m_tile * WM + c / 2, (int64_t)row_tiles - 1);
      off[u] = (uint32_t)((rt * nblk * 32 + lane) * 4);
    } else if (o < St::CA + St::CS + St::CB) {
      const int c = o - St::CA - St::CS;
      const int q = lane >> 2;
      const int ri = 16 * (c & 3) + q;
      const int64_t n = min(n0 + 32 * (c >> 2) + (ri & 31), n_rows - 1);
      const int piece = (lane & 3) ^ ((q >> 2) & 3);
      bpiece[u] = piece;
      off[u] = (uint32_t)((n >> 2) * wrow + (ri >> 5) * 1024 + (n & 3) * 256 +
                          (SEG == 1 ? piece * 16 : SEG == 4 ? piece * kPassBytes : 0));
    } else if (o < St::TOTAL) {
      const int c = o - St::CA - St::CS - St::CB;
      const int64_t n = min(n0 + 32 * (c / St::DWC) + li, n_rows - 1);
      const int j = c % St::DWC;
      // S == 1: lane half lh takes the pair (2lh, 2lh+1) of the stage's 4
      // slots; S > 1: block 2j + lh of the stage, one f16 per dword
      bpiece[u] = 2 * j + lh;
      off[u] = (uint32_t)((n >> 2) * wrow + kPassQs + 32 * (n & 3) +
                          (SEG == 1 ? 4 * lh : SEG == 4 ? (2 * j + lh) * kPassBytes : 0));
    }
  }

  // Issue the DMA of stage s into buffer `buf`.
  auto issue = [&](int s, St &buf) {
    const int kb = s * kStageBlocks;  // first block of the stage
    int64_t unit;
    int slot;
    locate<SEG>(kb, unit, slot);
#pragma unroll
    for (int u = 0; u < OPS_MAX; ++u) {
      const int o = wave + u * W;
      if (o < St::CA) {
        const int bb = o % kStageBlocks;
        dma16(uniform_ptr(qa + (int64_t)(kb + bb) * 1024) + off[u],
              buf.a[o / kStageBlocks][bb]);
      } else if (o < St::CA + St::CS) {
        const int c = o - St::CA;
        dma4(uniform_ptr((const uint8_t *)(sa + (int64_t)(kb + 2 * (c & 1)) * 32)) + off[u],
             buf.sa[c / 2][c & 1]);
      } else if (o < St::CA + St::CS + St::CB) {
        const int c = o - St::CA - St::CS;
        const uint8_t *base = SEG == 6 ? w : uniform_ptr(w + unit * kPassBytes + slot * 16);
        const uint32_t extra = SEG == 6 ? block_offset<SEG>(kb + bpiece[u]) : 0u;
        dma16(base + off[u] + extra, buf.b[c >> 2] + (c & 3) * 1024);
      } else if (o < St::TOTAL) {
        const int c = o - St::CA - St::CS - St::CB;
        const uint8_t *base =
            SEG == 6 ? w : uniform_ptr(w + unit * kPassBytes + 2 * (slot & ~1));
        uint32_t extra = 0;
        if constexpr (SEG == 6) {
          int64_t ub;
          int sb;
          locate<SEG>(kb + bpiece[u], ub, sb);
          extra = (uint32_t)(ub * kPassBytes + 2 * (sb & ~1));
        }
        dma4(base + off[u] + extra, buf.dw[c / St::DWC][c % St::DWC]);
      }
    }
  };

  float acc[16];
#pragma unroll
  for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
  const v16i zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  const int bsw = (lane >> 2) & 3;  // swizzle of this lane's weight run

  auto compute = [&](int s, St &buf) {
    const int kb = s * kStageBlocks;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      // scale tiles of blocks kb+2k (lanes 0-31) and kb+2k+1 (lanes 32-63)
      const float fa = buf.sa[wm][k][lane];
      uint32_t dwp;
      int hi;
      if constexpr (SEG == 1) {
        dwp = buf.dw[wn][0][32 * k + li];
        hi = lh;
      } else {
        dwp = buf.dw[wn][k][lane];
        int64_t ub;
        int sb;
        locate<SEG>(kb + 2 * k + lh, ub, sb);
        hi = sb & 1;
      }
      const float fb = half_bits_to_float(hi ? dwp >> 16 : dwp & 0xffffu);
      typedef float v32f __attribute__((ext_vector_type(32)));
      const v32f z32 = {};
      const v32f fac = __builtin_amdgcn_mfma_f32_32x32x1f32(fa, fb, z32, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int bb = 2 * k + j;
        const v4i af = *(const v4i *)(buf.a[wm][bb] + lane * 16);
        const v4i bf = *(const v4i *)(buf.b[wn] + lane * 64 + 16 * (bb ^ bsw));
        const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bf, zero, 0, 0, 0);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float dotf = (float)c[v];
          const float f = fac[16 * j + v];
          if (FMA) {
            acc[v] = __builtin_fmaf(dotf, f, acc[v]);
          } else {
            const float contrib = dotf * f;
            acc[v] = acc[v] + contrib;
          }
        }
        // One block's MFMA results live at a time: the accumulators are
        // pinned here (an empty asm that reads and writes them), so the
        // epilogue cannot sink below later stages' MFMAs, which would only
        // add registers -- the other waves of the SIMD fill MFMA latency.
#pragma unroll
        for (int v = 0; v < 16; ++v) asm volatile("" : "+v"(acc[v]));
      }
    }
  };

  // Every DMA is unconditional: a branch around one makes the compiler's
  // wait tracking merge states and wait for all loads before the next LDS
  // read.  Stages past the end reload the last stage into a buffer nobody
  // reads again (the stage count, 4 per unit, is a multiple of NST).
  const int last = stages - 1;
#pragma unroll
  for (int i = 0; i < NST - 1; ++i) issue(min(i, last), stage(i));

  for (int s0 = 0; s0 < stages; s0 += NST) {
#pragma unroll
    for (int i = 0; i < NST; ++i) {
      const int s = s0 + i;
      // NST - 2 stages were issued after stage s
      if constexpr (St::TOTAL % W == 0)
        wait_vmcnt<(NST - 2) * OPS_MAX>();
      else
        wait_vmcnt_dyn<(NST - 2) * OPS_MAX>((NST - 2) * ops);
      stage_barrier();
      // every wave is past stage s-1: its buffer takes stage s+NST-1
      issue(min(s + NST - 1, last), stage((i + NST - 1) % NST));
      compute(s, stage(i));
    }
  }
  // no DMA may land in LDS after the workgroup has released it
  wait_vmcnt<0>();

  const int64_t n = n0 + 32 * wn + li;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int64_t m = m0 + 32 * wm + 8 * (v >> 2) + 4 * lh + (v & 3);
    if (m < m_rows && n < n_rows) {
      const float o = activate(acc[v], EPI & 3);
      if constexpr ((EPI & 4) != 0)
        ((uint16_t *)y)[m * ldy + n] = float_to_bf16(o);
      else
        ((float *)y)[m * ldy + n] = o;
    }
  }
}

// SwiGLU multiply of the prefill path: gate (SiLU applied) and up in f32.
// f32: h = g * u in place.  bf16 result: each linear's output rounds to
// bf16 first, then the bf16 multiply (FuseSiluMul on bf16 tensors).
__global__ void mul_kernel(float *__restrict__ g, const float *__restrict__ u,
                           uint16_t *__restrict__ out_bf16, int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  if (out_bf16) {
    const float gb = bf16_to_float(float_to_bf16(g[i]));
    const float ub = bf16_to_float(float_to_bf16(u[i]));
    out_bf16[i] = float_to_bf16(gb * ub);
  } else {
    g[i] = g[i] * u[i];
  }
}

}  // namespace

hipError_t launch_mul(float *g, const float *u, uint16_t *out_bf16,
                      int64_t count, hipStream_t s) {
  if (count == 0) return hipSuccess;
  hipLaunchKernelGGL(mul_kernel, dim3((unsigned)((count + 255) / 256)),
                     dim3(256), 0, s, g, u, out_bf16, count);
  return hipGetLastError();
}

template <int WM, int WN, int NST, bool FMA, int SEG, int EPI>
static void launch_gemm_k(const GemmLaunch &l, int32_t passes, int32_t m_tiles,
                          int32_t n_tiles, unsigned grid, hipStream_t s) {
  hipLaunchKernelGGL((gemm_kernel<WM, WN, NST, FMA, SEG, EPI>), dim3(grid),
                     dim3(64 * WM * WN), 0, s, l.qa, l.sa, l.row_tiles, l.nblk,
                     l.w, l.rows, l.m, passes, m_tiles, n_tiles, l.y, l.ldy);
}

template <int WM, int WN, int NST, bool FMA, int SEG>
static void launch_gemm_e(const GemmLaunch &l, int32_t passes, int32_t m_tiles,
                          int32_t n_tiles, unsigned grid, hipStream_t s) {
  // activation and output type are template arguments: inlined for every
  // accumulator element, runtime switches bloat the kernel and slow it
#define LLMCP_GEMM_EPI(E) \
  case E: return launch_gemm_k<WM, WN, NST, FMA, SEG, E>(l, passes, m_tiles, n_tiles, grid, s);
  switch ((l.activation & 3) | (l.y_bf16 ? 4 : 0)) {
    LLMCP_GEMM_EPI(1) LLMCP_GEMM_EPI(2) LLMCP_GEMM_EPI(3) LLMCP_GEMM_EPI(4)
    LLMCP_GEMM_EPI(5) LLMCP_GEMM_EPI(6) LLMCP_GEMM_EPI(7)
    default: return launch_gemm_k<WM, WN, NST, FMA, SEG, 0>(l, passes, m_tiles, n_tiles, grid, s);
  }
#undef LLMCP_GEMM_EPI
}

template <int WM, int WN, int NST, bool FMA>
static hipError_t launch_gemm_t(const GemmLaunch &l, hipStream_t s) {
  const int32_t passes = (int32_t)passes_for(l.cols);
  const int32_t m_tiles = (int32_t)((l.m + 32 * WM - 1) / (32 * WM));
  const int32_t n_tiles = (int32_t)((l.rows + 32 * WN - 1) / (32 * WN));
  const int32_t n_tiles8 = (n_tiles + 7) / 8 * 8;
  const unsigned grid = (unsigned)(n_tiles8 * m_tiles);
  // the weight's unit layout is fixed at registration (seg_for)
  switch (seg_for(passes)) {
    case 6: launch_gemm_e<WM, WN, NST, FMA, 6>(l, passes, m_tiles, n_tiles, grid, s); break;
    case 4: launch_gemm_e<WM, WN, NST, FMA, 4>(l, passes, m_tiles, n_tiles, grid, s); break;
    default: launch_gemm_e<WM, WN, NST, FMA, 1>(l, passes, m_tiles, n_tiles, grid, s);
  }
  return hipGetLastError();
}

template <bool FMA>
static hipError_t launch_gemm_shape(const GemmLaunch &l, hipStream_t s) {
  // 128 x 96 workgroups (12 waves, one per CU by LDS): at M = 1024, N = 9216
  // that is 768 workgroups, three full rounds on 256 CUs.  Up to 64 rows:
  // 64 x 64 workgroups (4 waves, two per CU).
  if (l.m <= 64) return launch_gemm_t<2, 2, 4, FMA>(l, s);
  return launch_gemm_t<4, 3, 4, FMA>(l, s);
}

hipError_t launch_gemm(const GemmLaunch &l, hipStream_t s) {
  return l.fma ? launch_gemm_shape<true>(l, s) : launch_gemm_shape<false>(l, s);
}

}  // namespace llmcp_q8
