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
// Tiling: workgroup 128(M) x 128(N), four waves in 2x2, each wave 2x2 MFMA
// tiles of 32x32.  A stage is 4 blocks (128 k): A [128 x 128 B], the weight
// tile [128 x 128 B] from the pass layout, 4x128 activation scales and
// 4x128 weight scales (converted to f32 once per workgroup), double
// buffered in LDS.  Workgroups are mapped so the 8 M-tiles of an N-tile run
// on one XCD (workgroup id % 8 selects the XCD): the weight tile is fetched
// into that XCD's L2 once and reused.
#include "q8_kernels.h"

#include "q8_device.h"

namespace llmcp_q8 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int SB = 4;                  // blocks per stage
constexpr int ROW = SB * kBlock + 16;  // LDS row stride (bytes), padded

// Workgroup of WM x WN waves; each wave owns TM x TN tiles of 32x32, so the
// workgroup tile is BM = 32*WM*TM rows of activations by BN = 32*WN*TN
// weight rows.  The per-block scale tile sa (x) dw is formed by an f32 MFMA
// outer product (one exact product, one rounding -- the same value as the
// VALU multiply) whose output layout is the int8 MFMA's, leaving two VALU
// ops per element and block.
// EPI: activation code in bits 0-1, bf16 output in bit 2 (compile time:
// the epilogue is inlined for every accumulator element).
template <int WM, int WN, int TM, int TN, bool FMA, int SEG, int EPI>
__global__ __launch_bounds__(64 * WM * WN) void gemm_kernel(
    const int8_t *__restrict__ qa, int64_t ldq, const float *__restrict__ sa,
    int64_t lds, const uint8_t *__restrict__ w, int64_t n_rows, int64_t m_rows,
    int32_t passes, int32_t m_tiles, int32_t n_tiles, void *__restrict__ y,
    int64_t ldy) {
  constexpr int NT = 64 * WM * WN;
  constexpr int BM = 32 * WM * TM;
  constexpr int BN = 32 * WN * TN;
  __shared__ __align__(16) int8_t a_l[2][BM * ROW];
  __shared__ __align__(16) int8_t b_l[2][BN * ROW];
  __shared__ __align__(16) float sa_l[2][SB][BM];
  __shared__ __align__(16) float dw_l[2][SB][BN];

  // XCD-aware tile order: ids with the same (id % 8) share an XCD; give
  // each XCD whole N-tiles (all their M-tiles).
  const int id = blockIdx.x;
  const int xcd = id & 7;
  const int k = id >> 3;
  const int n_tile = (k / m_tiles) * 8 + xcd;
  const int m_tile = k % m_tiles;
  if (n_tile >= n_tiles) return;  // uniform per workgroup
  const int64_t m0 = (int64_t)m_tile * BM;
  const int64_t n0 = (int64_t)n_tile * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int stages = passes * (kPassBlocks / SB);

  // ---- global -> registers for one stage
  constexpr int AU = BM * 8 / NT;           // 16 B pieces of A per thread
  constexpr int BU = BN * 8 / NT;           // of the weight tile
  constexpr int SU = (SB * BM + NT - 1) / NT;
  constexpr int DU = (SB * BN + NT - 1) / NT;
  uint4 ra[AU], rb[BU];
  float rsa[SU];
  uint32_t rdw[DU];
  auto load_stage = [&](int s) {
    const int kb = s * SB;  // first block of the stage
#pragma unroll
    for (int u = 0; u < AU; ++u) {
      const int idx = u * NT + tid;
      const int64_t m = m0 + (idx >> 3);
      ra[u] = make_uint4(0, 0, 0, 0);
      if (m < m_rows)
        ra[u] = *(const uint4 *)(qa + m * ldq + (int64_t)kb * kBlock + (idx & 7) * 16);
    }
#pragma unroll
    for (int u = 0; u < BU; ++u) {
      const int idx = u * NT + tid;
      const int q = idx & 7;
      const int64_t n = n0 + (idx >> 3);
      rb[u] = make_uint4(0, 0, 0, 0);
      if (n < n_rows) {
        const int b = kb + (q >> 1);
        int64_t unit;
        int slot;
        locate<SEG>(b, unit, slot);  // weight unit layout (q8_common.h)
        const uint8_t *pass =
            w + ((n >> 2) * passes + unit) * (int64_t)kPassBytes;
        rb[u] = *(const uint4 *)(pass + (q & 1) * 1024 + (n & 3) * 256 +
                                 slot * 16);
      }
    }
#pragma unroll
    for (int u = 0; u < SU; ++u) {
      const int idx = u * NT + tid;
      const int bb = idx / BM, row = idx % BM;
      const int64_t m = m0 + row;
      rsa[u] = (idx < SB * BM && m < m_rows) ? sa[m * lds + kb + bb] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < DU; ++u) {
      const int idx = u * NT + tid;
      const int bb = idx / BN, row = idx % BN;
      const int64_t n = n0 + row;
      rdw[u] = 0;
      if (idx < SB * BN && n < n_rows) {
        const int b = kb + bb;
        int64_t unit;
        int slot;
        locate<SEG>(b, unit, slot);
        const uint8_t *pass =
            w + ((n >> 2) * passes + unit) * (int64_t)kPassBytes;
        rdw[u] = *(const uint16_t *)(pass + kPassQs + 2 * (16 * (n & 3) + slot));
      }
    }
  };
  auto store_stage = [&](int buf) {
#pragma unroll
    for (int u = 0; u < AU; ++u) {
      const int idx = u * NT + tid;
      *(uint4 *)(a_l[buf] + (idx >> 3) * ROW + (idx & 7) * 16) = ra[u];
    }
#pragma unroll
    for (int u = 0; u < BU; ++u) {
      const int idx = u * NT + tid;
      const int q = idx & 7;
      *(uint4 *)(b_l[buf] + (idx >> 3) * ROW + (q >> 1) * kBlock + (q & 1) * 16) = rb[u];
    }
#pragma unroll
    for (int u = 0; u < SU; ++u) {
      const int idx = u * NT + tid;
      if (idx < SB * BM) sa_l[buf][idx / BM][idx % BM] = rsa[u];
    }
#pragma unroll
    for (int u = 0; u < DU; ++u) {
      const int idx = u * NT + tid;
      if (idx < SB * BN)
        dw_l[buf][idx / BN][idx % BN] =
            (float)__builtin_bit_cast(_Float16, (uint16_t)rdw[u]);
    }
  };

  float acc[TM][TN][16];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int jn = 0; jn < TN; ++jn)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][jn][v] = 0.0f;

  const int li = lane & 31;   // row (A) / column (B) within a 32x32 tile
  const int lh = lane >> 5;   // k half within the block
  const v16i zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  const v16f zerof = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f,
                      0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const float kmask = lh == 0 ? 1.0f : 0.0f;  // zeroes the k=1 MFMA slice
  const int mrow = 32 * TM * wm;
  const int ncol = 32 * TN * wn;

  load_stage(0);
  store_stage(0);
  __syncthreads();
  for (int s = 0; s < stages; ++s) {
    const int cur = s & 1;
    if (s + 1 < stages) load_stage(s + 1);
    // One block at a time, blocks in order: its MFMA results are consumed
    // by the epilogue before the next block's MFMAs issue.
#pragma unroll 1
    for (int bb = 0; bb < SB; ++bb) {
      v4i af[TM], bf[TN];
#pragma unroll
      for (int t = 0; t < TM; ++t)
        af[t] = *(const v4i *)(a_l[cur] + (mrow + 32 * t + li) * ROW +
                               bb * kBlock + lh * 16);
#pragma unroll
      for (int t = 0; t < TN; ++t)
        bf[t] = *(const v4i *)(b_l[cur] + (ncol + 32 * t + li) * ROW +
                               bb * kBlock + lh * 16);
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) {
        v16i c[TN];
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
          c[tn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[tm], bf[tn], zero,
                                                        0, 0, 0);
        // Scale tiles from the MFMA pipe (an exact product, one rounding,
        // laid out like the int8 result).  TN == 2: one 32x32x1 two-block
        // outer product -- lanes 0-31 feed tile 0, lanes 32-63 tile 1;
        // TN == 1: 32x32x2 with the k=1 slice zeroed.
        const float fa = sa_l[cur][bb][mrow + 32 * tm + li];
        typedef float v32f __attribute__((ext_vector_type(32)));
        v32f fac;
        if constexpr (TN == 2) {
          const float fb = dw_l[cur][bb][ncol + 32 * lh + li];
          const v32f z32 = {};
          fac = __builtin_amdgcn_mfma_f32_32x32x1f32(fa, fb, z32, 0, 0, 0);
        } else {
          const float fb = dw_l[cur][bb][ncol + li] * kmask;
          const v16f f1 = __builtin_amdgcn_mfma_f32_32x32x2f32(fa, fb, zerof, 0, 0, 0);
#pragma unroll
          for (int v = 0; v < 16; ++v) fac[v] = f1[v];
        }
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const float dotf = (float)c[tn][v];
            const float f = fac[16 * tn + v];
            if (FMA) {
              acc[tm][tn][v] = __builtin_fmaf(dotf, f, acc[tm][tn][v]);
            } else {
              const float contrib = dotf * f;
              acc[tm][tn][v] = acc[tm][tn][v] + contrib;
            }
          }
      }
    }
    if (s + 1 < stages) store_stage(cur ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const int64_t n = n0 + ncol + 32 * tn + li;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t m = m0 + mrow + 32 * tm + 8 * (v >> 2) + 4 * lh + (v & 3);
        if (m < m_rows && n < n_rows) {
          const float o = activate(acc[tm][tn][v], EPI & 3);
          if constexpr ((EPI & 4) != 0)
            ((uint16_t *)y)[m * ldy + n] = float_to_bf16(o);
          else
            ((float *)y)[m * ldy + n] = o;
        }
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

template <int WM, int WN, int TM, int TN, bool FMA, int SEG, int EPI>
static void launch_gemm_k(const GemmLaunch &l, int32_t passes, int32_t m_tiles,
                          int32_t n_tiles, unsigned grid, hipStream_t s) {
  hipLaunchKernelGGL((gemm_kernel<WM, WN, TM, TN, FMA, SEG, EPI>), dim3(grid),
                     dim3(64 * WM * WN), 0, s, l.qa, l.ldq, l.sa, l.lds, l.w,
                     l.rows, l.m, passes, m_tiles, n_tiles, l.y, l.ldy);
}

template <int WM, int WN, int TM, int TN, bool FMA, int SEG>
static void launch_gemm_a(const GemmLaunch &l, int32_t passes, int32_t m_tiles,
                          int32_t n_tiles, unsigned grid, hipStream_t s) {
  // activation and output type are template arguments: inlined for every
  // accumulator element, runtime switches bloat the kernel and slow it
#define LLMCP_GEMM_EPI(E) \
  case E: return launch_gemm_k<WM, WN, TM, TN, FMA, SEG, E>(l, passes, m_tiles, n_tiles, grid, s);
  switch ((l.activation & 3) | (l.y_bf16 ? 4 : 0)) {
    LLMCP_GEMM_EPI(1) LLMCP_GEMM_EPI(2) LLMCP_GEMM_EPI(3) LLMCP_GEMM_EPI(4)
    LLMCP_GEMM_EPI(5) LLMCP_GEMM_EPI(6) LLMCP_GEMM_EPI(7)
    default: return launch_gemm_k<WM, WN, TM, TN, FMA, SEG, 0>(l, passes, m_tiles, n_tiles, grid, s);
  }
#undef LLMCP_GEMM_EPI
}

template <int WM, int WN, int TM, int TN, bool FMA>
static hipError_t launch_gemm_t(const GemmLaunch &l, hipStream_t s) {
  constexpr int BM = 32 * WM * TM, BN = 32 * WN * TN;
  const int32_t passes = (int32_t)passes_for(l.cols);
  const int32_t m_tiles = (int32_t)((l.m + BM - 1) / BM);
  const int32_t n_tiles = (int32_t)((l.rows + BN - 1) / BN);
  const int32_t n_tiles8 = (n_tiles + 7) / 8 * 8;
  const unsigned grid = (unsigned)(n_tiles8 * m_tiles);
  // the weight's unit layout is fixed at registration (seg_for)
  switch (seg_for(passes)) {
    case 6: launch_gemm_a<WM, WN, TM, TN, FMA, 6>(l, passes, m_tiles, n_tiles, grid, s); break;
    case 4: launch_gemm_a<WM, WN, TM, TN, FMA, 4>(l, passes, m_tiles, n_tiles, grid, s); break;
    default: launch_gemm_a<WM, WN, TM, TN, FMA, 1>(l, passes, m_tiles, n_tiles, grid, s);
  }
  return hipGetLastError();
}

template <bool FMA>
static hipError_t launch_gemm_shape(const GemmLaunch &l, hipStream_t s) {
  // 8 waves: up to 64 rows a 64x128 workgroup tile of one 32x32 tile per
  // wave (more workgroups share the weight stream); else 128x128 with a
  // 32x64 tile per wave, whose two scale tiles come from one MFMA.
  if (l.m <= 64) return launch_gemm_t<2, 4, 1, 1, FMA>(l, s);
  return launch_gemm_t<4, 2, 1, 2, FMA>(l, s);
}

hipError_t launch_gemm(const GemmLaunch &l, hipStream_t s) {
  return l.fma ? launch_gemm_shape<true>(l, s) : launch_gemm_shape<false>(l, s);
}

}  // namespace llmcp_q8
