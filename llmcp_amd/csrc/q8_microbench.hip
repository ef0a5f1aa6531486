// q8_microbench.hip -- the GPU's own peaks, measured the way the reference's
// microbench measures its CPU (microbench/cpu_microbench.cpp): streaming
// read / write / copy bandwidth over a buffer larger than every cache
// (:480-503), and the int8 dot-product peak from independent accumulator
// chains with no memory traffic (:203-260, the SDOT loop).  The roofline
// fractions of the path's kernels are reported against these as well as
// against the published figures.  A third kernel measures the ceiling of
// the prefill GEMM's exact per-block epilogue (its instruction mix without
// the memory stream), against which the GEMM is also reported.
#include <type_traits>

#include "q8_device.h"
#include "q8_kernels.h"

namespace llmcp_q8 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kStreamThreads = 256;
constexpr int kStreamUnroll = 4;  // 16 B loads in flight per lane and step

// Each lane walks the buffer in steps of gridDim * 256 * 64 B, four
// non-temporal 16 B accesses per step (a wave's four accesses are four
// contiguous 1 KiB runs).  The read kernel folds what it loads into one
// value that it stores only if it equals a constant no fill produces, so
// the loads stay and nothing is written.
__global__ __launch_bounds__(kStreamThreads) void stream_read_kernel(
    const v4i *__restrict__ src, int64_t n16, unsigned *__restrict__ sink) {
  const int64_t stride = (int64_t)gridDim.x * kStreamThreads * kStreamUnroll;
  int64_t i = (int64_t)blockIdx.x * kStreamThreads * kStreamUnroll + threadIdx.x;
  v4i acc = {0, 0, 0, 0};
  for (; i + (kStreamUnroll - 1) * kStreamThreads < n16; i += stride) {
    v4i v[kStreamUnroll];
#pragma unroll
    for (int u = 0; u < kStreamUnroll; ++u)
      v[u] = __builtin_nontemporal_load(src + i + u * kStreamThreads);
#pragma unroll
    for (int u = 0; u < kStreamUnroll; ++u) acc ^= v[u];
  }
  const unsigned x = (unsigned)(acc.x ^ acc.y ^ acc.z ^ acc.w);
  if (x == 0x9e3779b9u) sink[0] = x;
}

__global__ __launch_bounds__(kStreamThreads) void stream_write_kernel(v4i *__restrict__ dst,
                                                                      int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * kStreamThreads * kStreamUnroll;
  int64_t i = (int64_t)blockIdx.x * kStreamThreads * kStreamUnroll + threadIdx.x;
  const v4i v = {(int)i, 1, 2, 3};
  for (; i + (kStreamUnroll - 1) * kStreamThreads < n16; i += stride) {
#pragma unroll
    for (int u = 0; u < kStreamUnroll; ++u)
      __builtin_nontemporal_store(v, dst + i + u * kStreamThreads);
  }
}

__global__ __launch_bounds__(kStreamThreads) void stream_copy_kernel(
    const v4i *__restrict__ src, v4i *__restrict__ dst, int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * kStreamThreads * kStreamUnroll;
  int64_t i = (int64_t)blockIdx.x * kStreamThreads * kStreamUnroll + threadIdx.x;
  for (; i + (kStreamUnroll - 1) * kStreamThreads < n16; i += stride) {
    v4i v[kStreamUnroll];
#pragma unroll
    for (int u = 0; u < kStreamUnroll; ++u)
      v[u] = __builtin_nontemporal_load(src + i + u * kStreamThreads);
#pragma unroll
    for (int u = 0; u < kStreamUnroll; ++u)
      __builtin_nontemporal_store(v[u], dst + i + u * kStreamThreads);
  }
}

// int8 MFMA issue peak: kChains independent accumulators per wave, each
// v_mfma_i32_32x32x32_i8 (32x32x32 multiply-adds) depending only on its own
// chain's previous result, no loads in the loop.  The operands change with
// the lane so that no result is constant; the sums are stored only if they
// equal a constant they never reach.
constexpr int kChains = 8;

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3)))
void mfma_i8_kernel(int32_t iterations, unsigned *__restrict__ sink) {
  const int lane = threadIdx.x & 63;
  const v4i a = {lane, lane * 3 + 1, lane * 5 + 2, lane * 7 + 3};
  const v4i b = {lane ^ 5, 0x01020304, 0x05060708, lane * 11};
  v16i c[kChains];
#pragma unroll
  for (int k = 0; k < kChains; ++k)
    for (int v = 0; v < 16; ++v) c[k][v] = k;
  for (int32_t it = 0; it < iterations; ++it) {
#pragma unroll
    for (int k = 0; k < kChains; ++k) c[k] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c[k], 0, 0, 0);
  }
  int s = 0;
#pragma unroll
  for (int k = 0; k < kChains; ++k)
    for (int v = 0; v < 16; ++v) s ^= c[k][v];
  if ((unsigned)s == 0x9e3779b9u) sink[0] = (unsigned)s;
}

// The prefill GEMM's per-block work on one 32x32 tile, without its memory
// stream: the ceiling of the exact epilogue.  Each wave runs the GEMM's
// block pipeline (the next block's MFMAs issued ahead of this block's
// epilogue, operands read from LDS a block ahead, the two-block f32 scale
// tile every second block) over LDS-resident operands; three waves per
// SIMD, as in the 128 x 96 GEMM tiles.
//   MIX_EXACT    int8 MFMA, 16 converts + 16 FMAs per block (the exact
//                per-block epilogue acc = fma(f32(I), sa * dw, acc))
//   MIX_CVTFREE  two f16 MFMAs per block on integer-valued f16 operands
//                (exact f32 block dots, no convert), 16 FMAs per block;
//                twice the operand bytes
//   MIX_MFMA     the MFMAs of MIX_EXACT alone
enum { MIX_EXACT = 0, MIX_CVTFREE = 1, MIX_MFMA = 2 };
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

template <int MODE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3)))
void epilogue_mix_kernel(int32_t pairs, unsigned *__restrict__ sink) {
  // [block parity][A, B] operands: 1 KiB of int8 or 2 KiB of f16 each
  __shared__ __align__(16) uint8_t opnd[2][2][2048];
  __shared__ float sa_l[2][32];
  __shared__ uint32_t dw_l[64];
  for (int i = threadIdx.x; i < 2 * 2 * 2048 / 4; i += blockDim.x) {
    const uint32_t h = (uint32_t)i * 2654435761u;
    uint32_t v;
    if (MODE == MIX_CVTFREE) {
      // two f16 small integers in [-7, 7]
      const uint32_t lo = __builtin_bit_cast(uint16_t, (_Float16)(float)((int)((h >> 4) % 15u) - 7));
      const uint32_t hi = __builtin_bit_cast(uint16_t, (_Float16)(float)((int)((h >> 12) % 15u) - 7));
      v = lo | hi << 16;
    } else {
      v = (h >> 3) & 0x0f0f0f0fu;
    }
    ((uint32_t *)opnd)[i] = v;
  }
  for (int i = threadIdx.x; i < 64; i += blockDim.x) {
    ((float *)sa_l)[i] = 0.01f + 1e-4f * (float)i;
    dw_l[i] = 0x20082008u + (uint32_t)i;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int li = lane & 31, lh = lane >> 5;
  using Dot = std::conditional_t<MODE == MIX_CVTFREE, v16f, v16i>;
  struct Frag {
    v4i a0, b0, a1, b1;
  };
  // Operands of a block of parity `par`; the offset passes through an
  // empty asm each time so that the reads stay in the loop.
  auto frag = [&](int par) __attribute__((always_inline)) {
    int off = lane * 16;
    asm volatile("" : "+v"(off));
    Frag f;
    f.a0 = *(const v4i *)(opnd[par][0] + off);
    f.b0 = *(const v4i *)(opnd[par][1] + off);
    if (MODE == MIX_CVTFREE) {
      f.a1 = *(const v4i *)(opnd[par][0] + 1024 + off);
      f.b1 = *(const v4i *)(opnd[par][1] + 1024 + off);
    }
    return f;
  };
  auto dots = [&](const Frag &f) __attribute__((always_inline)) -> Dot {
    if constexpr (MODE == MIX_CVTFREE) {
      const v16f z = {};
      const v16f c = __builtin_amdgcn_mfma_f32_32x32x16_f16(
          __builtin_bit_cast(v8h, f.a0), __builtin_bit_cast(v8h, f.b0), z, 0, 0, 0);
      return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, f.a1),
                                                    __builtin_bit_cast(v8h, f.b1), c, 0, 0, 0);
    } else {
      const v16i z = {};
      return __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a0, f.b0, z, 0, 0, 0);
    }
  };
  // scale tile of a block pair: lanes 0-31 the first block, 32-63 the second
  auto scale = [&]() __attribute__((always_inline)) {
    int i = li;
    asm volatile("" : "+v"(i));
    const float fa = sa_l[lh][i];
    const uint32_t d = dw_l[i + 32 * lh];
    const float fb = (float)__builtin_bit_cast(_Float16, (uint16_t)(lh ? d >> 16 : d & 0xffffu));
    const v32f z = {};
    return __builtin_amdgcn_mfma_f32_32x32x1f32(fa, fb, z, 0, 0, 0);
  };
  float acc[16];
#pragma unroll
  for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
  Frag fr = frag(0);
  Dot c_cur = dots(fr);
  v32f f_cur = scale();
  fr = frag(1);
  // four blocks per iteration, so that the two scale tiles in flight
  // alternate between two register sets (no copies)
  for (int32_t p = 0; p < pairs; p += 2) {
    static_for<4>([&](auto BB) __attribute__((always_inline)) {
      constexpr int bb = decltype(BB)::value & 1;
      Dot c_next = dots(fr);
      v32f f_next;
      if constexpr (bb == 1) f_next = scale();
      // pinned here (each element taken by an empty asm), ahead of this
      // block's epilogue
#pragma unroll
      for (int v = 0; v < 16; ++v) asm volatile("" ::"v"(c_next[v]));
      if constexpr (bb == 1) asm volatile("" ::"v"(f_next));
      fr = frag(bb);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (MODE == MIX_MFMA) {
#pragma unroll
        for (int v = 0; v < 16; ++v) asm volatile("" ::"v"(c_cur[v]));
        asm volatile("" ::"v"(f_cur));
      } else {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float d = (float)c_cur[v];  // a convert for int8 dots only
          acc[v] = __builtin_fmaf(d, f_cur[16 * bb + v], acc[v]);
        }
      }
#pragma unroll
      for (int v = 0; v < 16; ++v) asm volatile("" : "+v"(acc[v]));
      __builtin_amdgcn_sched_barrier(0);
      c_cur = c_next;
      if constexpr (bb == 1) f_cur = f_next;
    });
  }
  float s = (float)c_cur[0] + f_cur[0];
#pragma unroll
  for (int v = 0; v < 16; ++v) s += acc[v];
  if (__builtin_bit_cast(uint32_t, s) == 0x7fc00001u) sink[0] = 1u;
}

// three 256-thread workgroups per CU: three waves per SIMD
template <int MODE>
hipError_t launch_mix(int32_t pairs, int cus, unsigned *sink, hipStream_t s) {
  hipLaunchKernelGGL(epilogue_mix_kernel<MODE>, dim3((unsigned)(cus * 3)), dim3(256), 0, s,
                     pairs, sink);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_stream(int kind, const void *src, void *dst, int64_t bytes, int cus,
                         hipStream_t s) {
  const int64_t n16 = bytes / 16;
  const dim3 grid((unsigned)(cus * 16)), block(kStreamThreads);
  switch (kind) {
    case 0:
      hipLaunchKernelGGL(stream_read_kernel, grid, block, 0, s, (const v4i *)src, n16,
                         (unsigned *)dst);
      break;
    case 1:
      hipLaunchKernelGGL(stream_write_kernel, grid, block, 0, s, (v4i *)dst, n16);
      break;
    case 2:
      hipLaunchKernelGGL(stream_copy_kernel, grid, block, 0, s, (const v4i *)src, (v4i *)dst,
                         n16);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_mfma_i8_peak(int32_t iterations, int cus, unsigned *sink, hipStream_t s) {
  // three 256-thread workgroups per CU: three waves per SIMD
  hipLaunchKernelGGL(mfma_i8_kernel, dim3((unsigned)(cus * 3)), dim3(256), 0, s, iterations,
                     sink);
  return hipGetLastError();
}

double mfma_i8_peak_ops(int32_t iterations, int cus) {
  return 2.0 * 32 * 32 * 32 * kChains * (double)iterations * (double)cus * 3 * 4;
}

hipError_t launch_epilogue_mix(int mode, int32_t pairs, int cus, unsigned *sink,
                               hipStream_t s) {
  switch (mode) {
    case MIX_EXACT: return launch_mix<MIX_EXACT>(pairs, cus, sink, s);
    case MIX_CVTFREE: return launch_mix<MIX_CVTFREE>(pairs, cus, sink, s);
    case MIX_MFMA: return launch_mix<MIX_MFMA>(pairs, cus, sink, s);
    default: return hipErrorInvalidValue;
  }
}

double epilogue_mix_ops(int32_t pairs, int cus) {
  // 32 x 32 x 32 multiply-adds per wave and block, two blocks per pair,
  // pairs rounded up to even by the kernel's four-block iterations
  return 2.0 * 32 * 32 * 32 * 2 * (double)((pairs + 1) / 2 * 2) * (double)cus * 3 * 4;
}

}  // namespace llmcp_q8
