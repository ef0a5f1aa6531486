// q8_runtime.cpp -- host side of the MI355X Q8_0 linear path: context,
// weight registry (host/device address -> device-resident repacked tensor),
// LLMCPWGT arena loader, host packer and the C ABI of include/llmcp_q8.h.
//
// Reference interfaces replaced here:
//   lowering hook      MatmulLoweringInternal.h:22-37, MatmulLoweringCommon.cpp:492-508
//   arena loader       lib/Runtime/WeightArena.cpp:27-131, include/llmcp/Support/PackedWeights.h
//   arena writer       lib/Model/WeightPacker.cpp:126-160, :164-274
//   packer             lib/Model/Quantization.cpp:92-116, :165-214
#include <hip/hip_runtime.h>
#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <map>
#include <mutex>
#include <set>
#include <string>
#include <vector>

#include "../../include/llmcp_q8.h"
#include "json_min.h"
#include "q8_kernels.h"

using namespace llmcp_q8;

static_assert(LLMCP_Q8_MAX_GROUP == kMaxGroup, "group size of the C ABI");

namespace {

// A fixed buffer: recording an error never allocates (so it cannot throw).
thread_local char g_last_error[512];

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

// Every entry of the C ABI runs its body through guarded(): a C++ exception
// (std::bad_alloc from the registry, the arena parser or the writer) becomes
// a status code instead of crossing into a C or MLIR caller.
template <class F>
int guarded(F &&body) noexcept {
  try {
    return body();
  } catch (const std::bad_alloc &) {
    return fail(LLMCP_Q8_ENOMEM, "host allocation failed");
  } catch (const std::exception &e) {
    return fail(LLMCP_Q8_EINTERNAL, "internal error: %s", e.what());
  } catch (...) {
    return fail(LLMCP_Q8_EINTERNAL, "internal error: unknown exception");
  }
}

int hip_fail(hipError_t e, const char *what) {
  return fail(LLMCP_Q8_EHIP, "%s: %s", what, hipGetErrorString(e));
}

#define HIP_TRY(expr)                              \
  do {                                             \
    hipError_t e_ = (expr);                        \
    if (e_ != hipSuccess) return hip_fail(e_, #expr); \
  } while (0)

struct Tensor {
  uintptr_t key = 0;       // address callers pass in weight descriptors
  uint64_t key_bytes = 0;  // p4 size: rows * cols * 34 / 32
  uint8_t *dev = nullptr;  // pass layout, device
  uint64_t dev_bytes = 0;
  int64_t rows = 0;
  int64_t cols = 0;
};

}  // namespace

struct llmcp_q8_ctx {
  int device = 0;
  hipStream_t own_stream = nullptr;
  hipStream_t stream = nullptr;
  std::map<uintptr_t, Tensor> registry;  // by key
  int32_t *err_flag = nullptr;
  // Workspace, sized when weights are registered so that decode-time calls
  // (and graph capture) never allocate: the quantized input row, its scales
  // and the lm_head's argmax slots (kArgmaxSlots, zero between calls;
  // keys_dirty when a call may have left them otherwise).
  int8_t *qa = nullptr;
  float *sa = nullptr;
  unsigned long long *keys = nullptr;
  bool keys_dirty = false;
  uint64_t qa_bytes = 0;
  uint64_t sa_bytes = 0;
  // Fused MLP: the SwiGLU output h when the caller passes no buffer for it.
  float *hf = nullptr;
  float *up = nullptr;  // prefill SwiGLU: the up projection
  uint64_t up_bytes = 0;
  uint64_t hf_bytes = 0;
  // Reference platform whose arithmetic every path reproduces
  // (llmcp_q8_platform): aarch64 = fma epilogue everywhere, x86 = mul+add.
  int32_t platform = LLMCP_Q8_PLATFORM_AARCH64;
  // llmcp_q8_accumulation of the multi-row linears; with SPLIT_K the K
  // splits' f32 partial sums live in `part` (grown on demand).
  int32_t accumulation = LLMCP_Q8_ACCUM_EXACT;
  float *part = nullptr;
  uint64_t part_bytes = 0;
  // Tests only (llmcp_q8_test_ctx_gemm_splits): K splits forced on every
  // splittable GEMM of this context in SPLIT_K mode; 0 = chosen by shape.
  int32_t test_splits = 0;
  // Cap on device bytes of registered weights (0: none).
  uint64_t weight_budget = 0;
  uint64_t weight_bytes = 0;
  // Bumped whenever device memory a captured graph may reference is freed
  // (workspace regrowth, a weight released or replaced); graphs captured
  // under an older generation are refused at launch.
  uint64_t generation = 0;
  // Orders work across llmcp_q8_ctx_set_stream.
  hipEvent_t switch_event = nullptr;
  // Tests only (llmcp_q8_test_ctx_rmsnorm_skew): offset of this context's
  // speculative RMSNorm predictions, in f32 steps; 0 otherwise.
  int32_t rmsnorm_skew = 0;
  bool fma() const { return platform == LLMCP_Q8_PLATFORM_AARCH64; }
};

namespace {

llmcp_q8_ctx *g_default_ctx = nullptr;

// Graphs captured through llmcp_q8_graph_end: their context and the
// context's memory generation at capture.
struct GraphInfo {
  llmcp_q8_ctx *ctx;
  uint64_t generation;
};
std::mutex g_graph_mutex;
std::map<void *, GraphInfo> g_graphs;

int set_device(llmcp_q8_ctx *ctx) {
  HIP_TRY(hipSetDevice(ctx->device));
  return LLMCP_Q8_OK;
}

const Tensor *find_tensor(llmcp_q8_ctx *ctx, const void *addr) {
  auto it = ctx->registry.find((uintptr_t)addr);
  if (it == ctx->registry.end()) return nullptr;
  return &it->second;
}

// Weight descriptor -> registered tensor, with the verifier's size rule
// (LLMCPOps.cpp:57-65: size == N * (K + K/16)).
int resolve_weight(llmcp_q8_ctx *ctx, const llmcp_memref_i8_1d *w,
                   const Tensor **out) {
  if (!w || !w->data) return fail(LLMCP_Q8_EINVAL, "null weight descriptor");
  const void *addr = w->data + w->offset;
  const Tensor *t = find_tensor(ctx, addr);
  if (!t)
    return fail(LLMCP_Q8_ENOTFOUND,
                "weight %p is not an uploaded q8_0_p4 tensor", addr);
  if (w->strides[0] != 1 || (uint64_t)w->sizes[0] != t->key_bytes)
    return fail(LLMCP_Q8_DECLINED,
                "q8_0_p4 weight size must be N * (K + (K/32)*2)");
  *out = t;
  return LLMCP_Q8_OK;
}

template <class M>
bool dense_rows(const M *d) {
  return d && d->data && d->strides[1] == 1 && d->sizes[0] >= 0 &&
         d->sizes[1] > 0 && (d->sizes[0] <= 1 || d->strides[0] >= d->sizes[1]);
}

// A row-major [rows, cols] activation view in device memory, f32 or bf16.
struct Rows {
  void *data = nullptr;
  int64_t rows = 0, cols = 0, ld = 0;
  bool bf16 = false;
};

// Device scratch a call uses: the quantized input rows with their scales
// and the argmax slots.  Normally the context's own (grown on demand);
// the no-allocation entry brings a fixed one.
struct Workspace {
  int8_t *qa = nullptr;
  float *sa = nullptr;
  uint64_t qa_bytes = 0;
  uint64_t sa_bytes = 0;
  unsigned long long *keys = nullptr;
  bool *keys_dirty = nullptr;  // the slots may hold keys of a failed call
  bool fixed = false;          // capacities are limits: never grow
};

template <class M>
bool view_of(const M *d, bool bf16, Rows &r) {
  if (!dense_rows(d)) return false;
  r.data = (void *)(d->data + d->offset);
  r.rows = d->sizes[0];
  r.cols = d->sizes[1];
  r.ld = d->sizes[0] <= 1 ? d->sizes[1] : d->strides[0];
  r.bf16 = bf16;
  return true;
}

// A norm's weight vector (dense 1-D memref of f32 or bf16).
struct NormWeight {
  const void *data = nullptr;
  int64_t len = 0;
  bool bf16 = false;
};

template <class D>
static bool norm_weight_of(const D *d, bool bf16, NormWeight &nw) {
  if (!d || !d->data || d->sizes[0] < 0 || (d->sizes[0] > 1 && d->strides[0] != 1))
    return false;
  nw.data = d->data + d->offset;
  nw.len = d->sizes[0];
  nw.bf16 = bf16;
  return true;
}

template <typename T>
int grow(llmcp_q8_ctx *ctx, T *&ptr, uint64_t &have, uint64_t need,
         const char *what) {
  if (need <= have) return LLMCP_Q8_OK;
  if (ptr) {
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    HIP_TRY(hipFree(ptr));
    ++ctx->generation;  // graphs captured earlier may reference ptr
  }
  ptr = nullptr;
  have = 0;
  if (hipMalloc((void **)&ptr, need) != hipSuccess)
    return fail(LLMCP_Q8_ENOMEM, "%s of %llu bytes", what,
                (unsigned long long)need);
  have = need;
  return LLMCP_Q8_OK;
}

int ensure_scratch(llmcp_q8_ctx *ctx, uint64_t qa_bytes, uint64_t sa_bytes) {
  int rc = grow(ctx, ctx->qa, ctx->qa_bytes, qa_bytes, "activation scratch");
  if (!rc) rc = grow(ctx, ctx->sa, ctx->sa_bytes, sa_bytes, "scale scratch");
  return rc;
}

// The context's workspace as a Workspace (after any growth).
Workspace ctx_workspace(llmcp_q8_ctx *ctx) {
  Workspace ws;
  ws.qa = ctx->qa;
  ws.sa = ctx->sa;
  ws.qa_bytes = ctx->qa_bytes;
  ws.sa_bytes = ctx->sa_bytes;
  ws.keys = ctx->keys;
  ws.keys_dirty = &ctx->keys_dirty;
  return ws;
}

// Room for qa_bytes / sa_bytes of quantized input: grows the context's
// workspace, or checks a fixed one.
int reserve(llmcp_q8_ctx *ctx, Workspace &ws, uint64_t qa_bytes,
            uint64_t sa_bytes) {
  if (ws.fixed) {
    if (qa_bytes > ws.qa_bytes || sa_bytes > ws.sa_bytes)
      return fail(LLMCP_Q8_DECLINED,
                  "input needs %llu + %llu bytes of scratch; the fixed "
                  "scratch holds %llu + %llu",
                  (unsigned long long)qa_bytes, (unsigned long long)sa_bytes,
                  (unsigned long long)ws.qa_bytes,
                  (unsigned long long)ws.sa_bytes);
    return LLMCP_Q8_OK;
  }
  int rc = ensure_scratch(ctx, qa_bytes, sa_bytes);
  if (!rc) ws = ctx_workspace(ctx);
  return rc;
}

// ------------------------------------------------ fixed scratch (no alloc) --
// The device scratch of llmcp_q8_lm_head_noalloc: the argmax slots, then the
// quantized input rows' f32 scales and int8 values.  Each GPU the library
// runs on holds its own copy for the life of the process; host code reaches
// it only through the address hipGetSymbolAddress returns for that device
// (g_scratch_ptr), never through the array's name.
constexpr uint64_t kSlotsBytes = (uint64_t)kArgmaxSlots * 8u;
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void *g_scratch_ptr[kMaxDevices];
bool g_scratch_dirty[kMaxDevices];  // the slots may hold a failed call's keys
// The one context per device whose calls may use the fixed scratch (the
// first to call the no-allocation entry there, until it is destroyed):
// two contexts run on different streams, and their calls would race on
// the shared array unordered.
llmcp_q8_ctx *g_scratch_owner[kMaxDevices];

}  // namespace

static __device__ __align__(256) unsigned char scratch[LLMCP_Q8_STATIC_SCRATCH_BYTES];

namespace {

// Resolves this device's copy of `scratch` (the device must be current) and
// zeroes its argmax slots with the reduce kernel in clearing mode (a kernel,
// not a memset).  Once per device; called when a context is created.
int setup_static_scratch(int device, hipStream_t stream) {
  if (device >= kMaxDevices)
    return fail(LLMCP_Q8_EINVAL, "device %d beyond the library's %d", device,
                kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[device]) return LLMCP_Q8_OK;
  void *p = nullptr;
  hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
  e = launch_argmax_reduce((unsigned long long *)p, nullptr, stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  if (e != hipSuccess) return hip_fail(e, "clearing the fixed scratch");
  g_scratch_ptr[device] = p;
  return LLMCP_Q8_OK;
}

// The fixed scratch as a Workspace: slots first, then scales and values in
// the ratio the quantized rows use them (4 B of scale per 32 values).
Workspace static_workspace(int device) {
  Workspace ws;
  unsigned char *base = (unsigned char *)g_scratch_ptr[device];
  const uint64_t rest = (uint64_t)LLMCP_Q8_STATIC_SCRATCH_BYTES - kSlotsBytes;
  ws.keys = (unsigned long long *)base;
  ws.sa_bytes = rest / 9 / 256 * 256;
  ws.sa = (float *)(base + kSlotsBytes);
  ws.qa = (int8_t *)(base + kSlotsBytes + ws.sa_bytes);
  ws.qa_bytes = rest - ws.sa_bytes;
  ws.keys_dirty = &g_scratch_dirty[device];
  ws.fixed = true;
  return ws;
}

// The argmax slots, allocated and zeroed once (before any graph capture).
int ensure_argmax_slots(llmcp_q8_ctx *ctx) {
  if (ctx->keys) return LLMCP_Q8_OK;
  const size_t bytes = (size_t)kArgmaxSlots * sizeof(unsigned long long);
  if (hipMalloc((void **)&ctx->keys, bytes) != hipSuccess) {
    ctx->keys = nullptr;
    return fail(LLMCP_Q8_ENOMEM, "argmax slots of %llu bytes",
                (unsigned long long)bytes);
  }
  HIP_TRY(hipMemsetAsync(ctx->keys, 0, bytes, ctx->stream));
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  return LLMCP_Q8_OK;
}

// Workspace a one-row call against a [rows, cols] weight needs, including
// the f32 buffer for h should its output feed the fused MLP's down GEMV.
int ensure_decode_scratch(llmcp_q8_ctx *ctx, int64_t rows, int64_t cols) {
  const uint64_t nblk = (uint64_t)passes_for(cols) * kPassBlocks;
  int rc = ensure_scratch(ctx, nblk * kBlock, nblk * 4);
  if (!rc) rc = ensure_argmax_slots(ctx);
  if (rc || rows % kBlock) return rc;
  return grow(ctx, ctx->hf, ctx->hf_bytes, (uint64_t)rows * 4, "mlp hidden");
}

// Repacks device p4 bytes into a new device tensor for `key` (not yet
// registered).  The weight budget counts `pending` bytes staged alongside.
int stage_from_device_p4(llmcp_q8_ctx *ctx, const void *key,
                         const uint8_t *dev_p4, int64_t rows, int64_t cols,
                         float *repack_ms, uint64_t pending, Tensor &t) {
  t = Tensor();
  t.key = (uintptr_t)key;
  t.rows = rows;
  t.cols = cols;
  t.key_bytes = (uint64_t)rows * (uint64_t)(cols / kBlock) * 34u;
  t.dev_bytes = (uint64_t)device_bytes_for(rows, cols);
  if (ctx->weight_budget &&
      ctx->weight_bytes + pending + t.dev_bytes > ctx->weight_budget)
    return fail(LLMCP_Q8_ENOMEM,
                "device weight of %llu bytes exceeds the context's weight "
                "budget (%llu of %llu bytes in use)",
                (unsigned long long)t.dev_bytes,
                (unsigned long long)(ctx->weight_bytes + pending),
                (unsigned long long)ctx->weight_budget);
  if (hipMalloc(&t.dev, t.dev_bytes) != hipSuccess) {
    t.dev = nullptr;
    return fail(LLMCP_Q8_ENOMEM, "device weight of %llu bytes",
                (unsigned long long)t.dev_bytes);
  }
  hipEvent_t e0 = nullptr, e1 = nullptr;
  hipError_t err = hipSuccess;
  if (repack_ms) {
    err = hipEventCreate(&e0);
    if (err == hipSuccess) err = hipEventCreate(&e1);
    if (err == hipSuccess) err = hipEventRecord(e0, ctx->stream);
  }
  if (err == hipSuccess)
    err = launch_repack(dev_p4, t.dev, rows, cols, ctx->stream);
  if (err == hipSuccess && repack_ms) {
    err = hipEventRecord(e1, ctx->stream);
    if (err == hipSuccess) err = hipEventSynchronize(e1);
    if (err == hipSuccess) err = hipEventElapsedTime(repack_ms, e0, e1);
  }
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);
  if (err != hipSuccess) {
    (void)hipFree(t.dev);
    t.dev = nullptr;
    return hip_fail(err, "repack");
  }
  return LLMCP_Q8_OK;
}

// Makes staged tensors visible all at once: the new registry is built on
// the side (the only step that can throw) and swapped in; entries they
// replace are freed afterwards.  On failure the staged tensors are freed
// and the registry is unchanged.
int commit_tensors(llmcp_q8_ctx *ctx, std::vector<Tensor> &staged) {
  auto drop_staged = [&] {
    for (Tensor &t : staged) (void)hipFree(t.dev);
    staged.clear();
  };
  // workspace for each tensor's input row (and h for the MLP's down GEMV)
  for (const Tensor &t : staged) {
    int rc = ensure_decode_scratch(ctx, t.rows, t.cols);
    if (rc) {
      drop_staged();
      return rc;
    }
  }
  std::map<uintptr_t, Tensor> next;
  std::vector<uint8_t *> replaced;
  try {
    next = ctx->registry;
    for (const Tensor &t : staged) {
      auto it = next.find(t.key);
      if (it != next.end()) replaced.push_back(it->second.dev);
      next[t.key] = t;
    }
  } catch (...) {
    drop_staged();
    throw;
  }
  if (!replaced.empty()) {
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
      drop_staged();
      return hip_fail(e, "hipStreamSynchronize");
    }
  }
  ctx->registry.swap(next);
  staged.clear();
  uint64_t bytes = 0;
  for (const auto &kv : ctx->registry) bytes += kv.second.dev_bytes;
  ctx->weight_bytes = bytes;
  for (uint8_t *p : replaced) (void)hipFree(p);
  if (!replaced.empty()) ++ctx->generation;
  return LLMCP_Q8_OK;
}

// One tensor: stage and commit.
int register_from_device_p4(llmcp_q8_ctx *ctx, const void *key,
                            const uint8_t *dev_p4, int64_t rows, int64_t cols,
                            float *repack_ms) {
  std::vector<Tensor> staged(1);
  int rc = stage_from_device_p4(ctx, key, dev_p4, rows, cols, repack_ms, 0,
                                staged[0]);
  if (rc) return rc;
  return commit_tensors(ctx, staged);
}

// Host p4 bytes -> device staging copy -> staged tensor.
int stage_from_host_p4(llmcp_q8_ctx *ctx, const void *host_p4, int64_t rows,
                       int64_t cols, float *repack_ms, uint64_t pending,
                       Tensor &t) {
  const uint64_t bytes = (uint64_t)rows * (uint64_t)(cols / kBlock) * 34u;
  uint8_t *staging = nullptr;
  if (hipMalloc(&staging, bytes) != hipSuccess)
    return fail(LLMCP_Q8_ENOMEM, "staging of %llu bytes",
                (unsigned long long)bytes);
  hipError_t e = hipMemcpyAsync(staging, host_p4, bytes, hipMemcpyHostToDevice,
                                ctx->stream);
  int rc = e == hipSuccess ? stage_from_device_p4(ctx, host_p4, staging, rows,
                                                  cols, repack_ms, pending, t)
                           : hip_fail(e, "upload");
  (void)hipStreamSynchronize(ctx->stream);
  (void)hipFree(staging);
  return rc;
}

bool packable(int64_t rows, int64_t cols) {
  // isQ8PackedShape (Q8PackedLayout.h:38-42).
  return rows > 0 && cols > 0 && rows % 8 == 0 && cols % kBlock == 0;
}

uint32_t rd32(const uint8_t *p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
         ((uint32_t)p[3] << 24);
}
uint64_t rd64(const uint8_t *p) {
  return (uint64_t)rd32(p) | ((uint64_t)rd32(p + 4) << 32);
}
void wr32(uint8_t *p, uint32_t v) {
  for (int i = 0; i < 4; ++i) p[i] = (uint8_t)(v >> (8 * i));
}
void wr64(uint8_t *p, uint64_t v) {
  for (int i = 0; i < 8; ++i) p[i] = (uint8_t)(v >> (8 * i));
}

// ---------------------------------------------------- host f16 and pack --

uint16_t host_f32_to_f16(float value) {
  uint32_t x;
  std::memcpy(&x, &value, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t exp = (x >> 23) & 0xffu;
  const uint32_t man = x & 0x7fffffu;
  if (exp == 0xffu)
    return (uint16_t)(sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0u));
  const int32_t e = (int32_t)exp - 112;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (exp == 0) return (uint16_t)sign;
    const uint32_t full = man | 0x800000u;
    const int shift = 14 - e;
    if (shift > 24) return (uint16_t)sign;
    uint32_t m = full >> shift;
    const uint32_t rem = full & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (m & 1u))) ++m;
    return (uint16_t)(sign | m);
  }
  uint32_t h = ((uint32_t)e << 10) | (man >> 13);
  const uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
  return (uint16_t)(sign | h);
}

}  // namespace

// ====================================================================== C ABI

extern "C" {

int32_t llmcp_q8_abi_version(void) { return LLMCP_Q8_ABI_VERSION; }

const char *llmcp_q8_last_error(void) { return g_last_error; }

int llmcp_q8_ctx_create(int device, llmcp_q8_ctx **out) {
  return guarded([&]() -> int {
    if (!out) return fail(LLMCP_Q8_EINVAL, "null output pointer");
    *out = nullptr;
    int count = 0;
    HIP_TRY(hipGetDeviceCount(&count));
    if (device < 0 || device >= count)
      return fail(LLMCP_Q8_EINVAL, "device %d out of range (%d devices)", device,
                  count);
    auto *ctx = new llmcp_q8_ctx();
    ctx->device = device;
    int rc = set_device(ctx);
    if (rc) {
      delete ctx;
      return rc;
    }
    hipError_t e = hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
      delete ctx;
      return hip_fail(e, "hipStreamCreateWithFlags");
    }
    ctx->stream = ctx->own_stream;
    e = hipEventCreateWithFlags(&ctx->switch_event, hipEventDisableTiming);
    if (e != hipSuccess) {
      ctx->switch_event = nullptr;
      llmcp_q8_ctx_destroy(ctx);
      return hip_fail(e, "hipEventCreateWithFlags");
    }
    if (hipMalloc(&ctx->err_flag, sizeof(int32_t)) != hipSuccess) {
      llmcp_q8_ctx_destroy(ctx);
      return fail(LLMCP_Q8_ENOMEM, "context workspace");
    }
    if (hipMemset(ctx->err_flag, 0, sizeof(int32_t)) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess) {
      llmcp_q8_ctx_destroy(ctx);
      return fail(LLMCP_Q8_EHIP, "context workspace init");
    }
    // the device's fixed scratch, for llmcp_q8_lm_head_noalloc
    if ((rc = setup_static_scratch(device, ctx->stream))) {
      llmcp_q8_ctx_destroy(ctx);
      return rc;
    }
    *out = ctx;
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_ctx_destroy(llmcp_q8_ctx *ctx) {
  return guarded([&]() -> int {
    if (!ctx) return LLMCP_Q8_OK;
    (void)hipSetDevice(ctx->device);
    if (ctx->own_stream) (void)hipStreamSynchronize(ctx->own_stream);
    if (ctx->stream && ctx->stream != ctx->own_stream)
      (void)hipStreamSynchronize(ctx->stream);
    for (auto &kv : ctx->registry) (void)hipFree(kv.second.dev);
    if (ctx->err_flag) (void)hipFree(ctx->err_flag);
    if (ctx->qa) (void)hipFree(ctx->qa);
    if (ctx->sa) (void)hipFree(ctx->sa);
    if (ctx->keys) (void)hipFree(ctx->keys);
    if (ctx->hf) (void)hipFree(ctx->hf);
    if (ctx->up) (void)hipFree(ctx->up);
    if (ctx->part) (void)hipFree(ctx->part);
    {
      std::lock_guard<std::mutex> lock(g_graph_mutex);
      for (auto it = g_graphs.begin(); it != g_graphs.end();)
        it = it->second.ctx == ctx ? g_graphs.erase(it) : std::next(it);
    }
    if (ctx->switch_event) (void)hipEventDestroy(ctx->switch_event);
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
    if (g_default_ctx == ctx) g_default_ctx = nullptr;
    if (ctx->device >= 0 && ctx->device < kMaxDevices) {
      // its calls have finished (the streams were synchronized above)
      std::lock_guard<std::mutex> lock(g_scratch_mutex);
      if (g_scratch_owner[ctx->device] == ctx) g_scratch_owner[ctx->device] = nullptr;
    }
    delete ctx;
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_ctx_set_stream(llmcp_q8_ctx *ctx, void *hip_stream) {
  return guarded([&]() -> int {
    if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
    hipStream_t next = hip_stream ? (hipStream_t)hip_stream : ctx->own_stream;
    if (next == ctx->stream) return LLMCP_Q8_OK;
    // Work still queued on the old stream uses the shared workspace: the new
    // stream waits for it before anything is launched there.
    HIP_TRY(hipSetDevice(ctx->device));
    HIP_TRY(hipEventRecord(ctx->switch_event, ctx->stream));
    HIP_TRY(hipStreamWaitEvent(next, ctx->switch_event, 0));
    ctx->stream = next;
    return LLMCP_Q8_OK;
  });
}

void *llmcp_q8_ctx_stream(llmcp_q8_ctx *ctx) {
  return ctx ? (void *)ctx->stream : nullptr;
}

int llmcp_q8_ctx_synchronize(llmcp_q8_ctx *ctx) {
  return guarded([&]() -> int {
    if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_set_default_ctx(llmcp_q8_ctx *ctx) {
  return guarded([&]() -> int {
    g_default_ctx = ctx;
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_set_platform(llmcp_q8_ctx *ctx, int32_t platform) {
  return guarded([&]() -> int {
    if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
    if (platform != LLMCP_Q8_PLATFORM_AARCH64 && platform != LLMCP_Q8_PLATFORM_X86)
      return fail(LLMCP_Q8_EINVAL, "unknown platform %d", platform);
    ctx->platform = platform;
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_set_accumulation(llmcp_q8_ctx *ctx, int32_t mode) {
  return guarded([&]() -> int {
    if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
    if (mode != LLMCP_Q8_ACCUM_EXACT && mode != LLMCP_Q8_ACCUM_SPLIT_K)
      return fail(LLMCP_Q8_EINVAL, "unknown accumulation mode %d", mode);
    ctx->accumulation = mode;
    return LLMCP_Q8_OK;
  });
}

int32_t llmcp_q8_get_accumulation(llmcp_q8_ctx *ctx) {
  return ctx ? ctx->accumulation : -1;
}

// Test hook, declared in no header of the product (no counterpart in the
// reference): forces `splits` K splits (clamped to the pass count; 0 = the
// shape's own choice) on this context's splittable GEMMs in SPLIT_K mode.
int llmcp_q8_test_ctx_gemm_splits(llmcp_q8_ctx *ctx, int32_t splits) {
  if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
  if (splits < 0) return fail(LLMCP_Q8_EINVAL, "negative split count %d", splits);
  ctx->test_splits = splits;
  return LLMCP_Q8_OK;
}

int32_t llmcp_q8_get_platform(llmcp_q8_ctx *ctx) {
  return ctx ? ctx->platform : -1;
}

// Test hook, declared in no header of the product (the tests bind it
// directly; no counterpart in the reference): rows of up to 12288 values
// have their serial sum of squares evaluated speculatively from predicted
// partial sums with exact fallbacks, and this moves the predictions of this
// context's RMSNorm calls by `bits` f32 steps (0 = off) so that the
// fallbacks decide the results.  Results do not change.  The setting is
// per context: no other context's calls see it.
int llmcp_q8_test_ctx_rmsnorm_skew(llmcp_q8_ctx *ctx, int32_t bits) {
  if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
  ctx->rmsnorm_skew = bits;
  return LLMCP_Q8_OK;
}

int llmcp_q8_set_weight_budget(llmcp_q8_ctx *ctx, uint64_t bytes) {
  return guarded([&]() -> int {
    if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
    ctx->weight_budget = bytes;
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_ctx_check(llmcp_q8_ctx *ctx, int32_t *flag) {
  return guarded([&]() -> int {
    if (!ctx || !flag) return fail(LLMCP_Q8_EINVAL, "null argument");
    HIP_TRY(hipSetDevice(ctx->device));
    HIP_TRY(hipMemcpyAsync(flag, ctx->err_flag, sizeof(int32_t),
                           hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipMemsetAsync(ctx->err_flag, 0, sizeof(int32_t), ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_selftest_quantizer(llmcp_q8_ctx *ctx, uint64_t *mismatches) {
  return guarded([&]() -> int {
    if (!ctx || !mismatches) return fail(LLMCP_Q8_EINVAL, "null argument");
    int rc = set_device(ctx);
    if (rc) return rc;
    unsigned long long *bad = nullptr;
    if (hipMalloc(&bad, sizeof(*bad)) != hipSuccess)
      return fail(LLMCP_Q8_ENOMEM, "self-test counter");
    unsigned long long host = 0;
    hipError_t e = hipMemsetAsync(bad, 0, sizeof(*bad), ctx->stream);
    if (e == hipSuccess) e = launch_selftest_quantizer(bad, ctx->stream);
    if (e == hipSuccess)
      e = hipMemcpyAsync(&host, bad, sizeof(host), hipMemcpyDeviceToHost,
                         ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    (void)hipFree(bad);
    if (e != hipSuccess) return hip_fail(e, "quantizer self-test");
    *mismatches = host;
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_selftest_exp(llmcp_q8_ctx *ctx, uint64_t counts[4], float *inputs,
                          uint32_t *results, int64_t cap, int64_t *stored) {
  return guarded([&]() -> int {
    if (!ctx || !counts || !stored || cap < 0 || (cap > 0 && (!inputs || !results)))
      return fail(LLMCP_Q8_EINVAL, "null argument or negative capacity");
    if (cap > (int64_t)1 << 24) return fail(LLMCP_Q8_EINVAL, "capacity above 2^24");
    int rc = set_device(ctx);
    if (rc) return rc;
    unsigned long long *out = nullptr;
    float *din = nullptr;
    uint32_t *dres = nullptr;
    const size_t n = cap > 0 ? (size_t)cap : 1;
    if (hipMalloc(&out, 5 * sizeof(*out)) != hipSuccess ||
        hipMalloc(&din, n * sizeof(float)) != hipSuccess ||
        hipMalloc(&dres, n * sizeof(uint32_t)) != hipSuccess) {
      (void)hipFree(out);
      (void)hipFree(din);
      (void)hipFree(dres);
      return fail(LLMCP_Q8_ENOMEM, "exp self-test buffers");
    }
    unsigned long long host[5] = {0, 0, 0, 0, 0};
    hipError_t e = hipMemsetAsync(out, 0, sizeof(host), ctx->stream);
    if (e == hipSuccess)
      e = launch_selftest_exp(out, din, dres, (uint32_t)cap, ctx->stream);
    if (e == hipSuccess)
      e = hipMemcpyAsync(host, out, sizeof(host), hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    const int64_t k = e == hipSuccess ? (int64_t)std::min<unsigned long long>(host[3], (unsigned long long)cap) : 0;
    if (e == hipSuccess && k > 0)
      e = hipMemcpy(inputs, din, (size_t)k * sizeof(float), hipMemcpyDeviceToHost);
    if (e == hipSuccess && k > 0)
      e = hipMemcpy(results, dres, (size_t)k * sizeof(uint32_t), hipMemcpyDeviceToHost);
    (void)hipFree(out);
    (void)hipFree(din);
    (void)hipFree(dres);
    if (e != hipSuccess) return hip_fail(e, "exp self-test");
    for (int i = 0; i < 3; ++i) counts[i] = host[i];
    counts[3] = host[4];
    *stored = k;
    return LLMCP_Q8_OK;
  });
}

// ------------------------------------------------------------- weights --

int llmcp_q8_upload_p4(llmcp_q8_ctx *ctx, const void *host_p4, int64_t rows,
                       int64_t cols, float *repack_ms) {
  return guarded([&]() -> int {
    if (!ctx || !host_p4) return fail(LLMCP_Q8_EINVAL, "null argument");
    if (!packable(rows, cols))
      return fail(LLMCP_Q8_DECLINED,
                  "packed Q8_0 requires rows %% 8 == 0 and cols %% 32 == 0");
    int rc = set_device(ctx);
    if (rc) return rc;
    std::vector<Tensor> staged(1);
    rc = stage_from_host_p4(ctx, host_p4, rows, cols, repack_ms, 0, staged[0]);
    if (rc) return rc;
    return commit_tensors(ctx, staged);
  });
}

int llmcp_q8_register_device_p4(llmcp_q8_ctx *ctx, const void *dev_p4,
                                int64_t rows, int64_t cols, float *repack_ms) {
  return guarded([&]() -> int {
    if (!ctx || !dev_p4) return fail(LLMCP_Q8_EINVAL, "null argument");
    if (!packable(rows, cols))
      return fail(LLMCP_Q8_DECLINED,
                  "packed Q8_0 requires rows %% 8 == 0 and cols %% 32 == 0");
    int rc = set_device(ctx);
    if (rc) return rc;
    return register_from_device_p4(ctx, dev_p4, (const uint8_t *)dev_p4, rows,
                                   cols, repack_ms);
  });
}

int llmcp_q8_release(llmcp_q8_ctx *ctx, const void *key) {
  return guarded([&]() -> int {
    if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
    auto it = ctx->registry.find((uintptr_t)key);
    if (it == ctx->registry.end())
      return fail(LLMCP_Q8_ENOTFOUND, "no tensor registered at %p", key);
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    HIP_TRY(hipFree(it->second.dev));
    ctx->weight_bytes -= it->second.dev_bytes;
    ctx->registry.erase(it);
    ++ctx->generation;
    return LLMCP_Q8_OK;
  });
}

uint64_t llmcp_q8_device_bytes(llmcp_q8_ctx *ctx, const void *key) {
  if (!ctx) return 0;
  const Tensor *t = find_tensor(ctx, key);
  return t ? t->dev_bytes : 0;
}

}  // extern "C"

namespace {

struct ArenaTensor {
  std::string name;
  std::string dtype;
  const uint8_t *data;
  std::vector<int64_t> shape;
};

// Arena validation follows PackedWeightsHeader::read (PackedWeights.h:36-56)
// and Arena::load (WeightArena.cpp:27-131) rule for rule.
int parse_arena(const void *file, uint64_t file_bytes,
                std::vector<ArenaTensor> &out) {
  if (!file) return fail(LLMCP_Q8_EINVAL, "null argument");
  const uint8_t *f = (const uint8_t *)file;
  if (file_bytes < 64 || std::memcmp(f, "LLMCPWGT", 8) != 0)
    return fail(LLMCP_Q8_EFORMAT,
                "invalid packed weights header; repack weights with llmcp-pack");
  if (rd32(f + 8) != 1 || rd32(f + 12) != 64)
    return fail(LLMCP_Q8_EFORMAT,
                "unsupported packed weights format version or header size");
  const uint64_t arena = rd64(f + 16), moff = rd64(f + 24), mbytes = rd64(f + 32);
  if (arena < 64 || moff != arena || moff > file_bytes || mbytes == 0 ||
      mbytes != file_bytes - moff)
    return fail(LLMCP_Q8_EFORMAT, "invalid packed weights arena or manifest bounds");
  json::Value root;
  json::Parser parser((const char *)f + moff, (size_t)mbytes);
  if (!parser.parse(root) || root.kind != json::Value::Object)
    return fail(LLMCP_Q8_EFORMAT, "invalid embedded weight manifest");
  const json::Value *total = root.get("total_bytes");
  const json::Value *header = root.get("header_bytes");
  const json::Value *mode = root.get("quantization");
  const json::Value *tensors = root.get("tensors");
  if (!total || !total->is_int() || total->i < 0 || (uint64_t)total->i != arena ||
      !header || !header->is_int() || header->i != 64 || !mode ||
      !mode->is_string() || (mode->s != "none" && mode->s != "q8_0") ||
      !tensors || tensors->kind != json::Value::Array || tensors->arr.empty())
    return fail(LLMCP_Q8_EFORMAT, "invalid embedded weight manifest");
  if (mode->s == "q8_0") {
    const json::Value *bs = root.get("block_size");
    const json::Value *ql = root.get("quant_layout");
    if (!bs || !bs->is_int() || bs->i != 32 || !ql || !ql->is_string() ||
        ql->s != "q8_0_p4")
      return fail(LLMCP_Q8_EFORMAT, "invalid embedded weight manifest");
  }
  std::set<std::string> names;
  std::vector<ArenaTensor> result;
  for (const json::Value &e : tensors->arr) {
    const json::Value *name = e.get("name");
    const json::Value *offset = e.get("offset");
    const json::Value *size = e.get("size");
    const json::Value *dtype = e.get("dtype");
    const json::Value *shape = e.get("shape");
    if (e.kind != json::Value::Object || !name || !name->is_string() ||
        name->s.empty() || !offset || !offset->is_int() || offset->i < 64 ||
        offset->i % 64 || !size || !size->is_int() || size->i <= 0 || !dtype ||
        !dtype->is_string() || !shape || shape->kind != json::Value::Array ||
        shape->arr.empty())
      return fail(LLMCP_Q8_EFORMAT, "invalid embedded weight manifest");
    const uint64_t begin = (uint64_t)offset->i, length = (uint64_t)size->i;
    if (begin > arena || length > arena - begin)
      return fail(LLMCP_Q8_EFORMAT, "tensor outside arena: %s", name->s.c_str());
    uint64_t elements = 1;
    std::vector<int64_t> dims;
    for (const json::Value &d : shape->arr) {
      if (!d.is_int() || d.i <= 0 ||
          elements > std::numeric_limits<uint64_t>::max() / (uint64_t)d.i)
        return fail(LLMCP_Q8_EFORMAT, "invalid embedded weight manifest");
      elements *= (uint64_t)d.i;
      dims.push_back(d.i);
    }
    uint64_t unit;
    if (dtype->s == "Q8_0") {
      if (mode->s != "q8_0" || dims.size() != 2 || dims[1] % 32)
        return fail(LLMCP_Q8_EFORMAT, "invalid embedded weight manifest");
      elements /= 32;
      unit = 34;
    } else if (dtype->s == "BF16") {
      unit = 2;
    } else if (dtype->s == "F32") {
      unit = 4;
    } else {
      return fail(LLMCP_Q8_EFORMAT, "invalid embedded weight manifest");
    }
    if (elements > std::numeric_limits<uint64_t>::max() / unit ||
        elements * unit != length)
      return fail(LLMCP_Q8_EFORMAT, "invalid embedded weight manifest");
    if (!names.insert(name->s).second)
      return fail(LLMCP_Q8_EFORMAT, "invalid embedded weight manifest");
    if (dtype->s == "Q8_0" && !packable(dims[0], dims[1]))
      return fail(LLMCP_Q8_EFORMAT, "Q8_0 tensor %s is not a packed shape",
                  name->s.c_str());
    result.push_back({name->s, dtype->s, f + begin, dims});
  }
  out.swap(result);
  return LLMCP_Q8_OK;
}

}  // namespace

extern "C" {

int llmcp_q8_arena_inspect(const void *file, uint64_t file_bytes,
                           int64_t *num_tensors, int64_t *num_q8) {
  return guarded([&]() -> int {
    std::vector<ArenaTensor> tensors;
    int rc = parse_arena(file, file_bytes, tensors);
    if (rc) return rc;
    int64_t q8 = 0;
    for (const ArenaTensor &t : tensors) q8 += t.dtype == "Q8_0";
    if (num_tensors) *num_tensors = (int64_t)tensors.size();
    if (num_q8) *num_q8 = q8;
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_upload_arena(llmcp_q8_ctx *ctx, const void *file,
                          uint64_t file_bytes, int64_t *num_q8) {
  return guarded([&]() -> int {
    if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
    std::vector<ArenaTensor> tensors;
    int rc = parse_arena(file, file_bytes, tensors);
    if (rc) return rc;
    // Validation passed: stage every Q8_0 tensor on the device, then register
    // them all at once.  A failure part-way frees what was staged and leaves
    // the registry as it was (Arena::load builds the new arena aside and
    // replaces the old one only on success, WeightArena.cpp:28-29, :124-130).
    if ((rc = set_device(ctx))) return rc;
    std::vector<Tensor> staged;
    uint64_t pending = 0;
    for (const ArenaTensor &t : tensors) {
      if (t.dtype != "Q8_0") continue;
      Tensor st;
      rc = stage_from_host_p4(ctx, t.data, t.shape[0], t.shape[1], nullptr,
                              pending, st);
      if (!rc) {
        try {
          staged.push_back(st);
        } catch (...) {
          (void)hipFree(st.dev);
          rc = fail(LLMCP_Q8_ENOMEM, "host allocation failed");
        }
      }
      if (rc) {
        for (Tensor &x : staged) (void)hipFree(x.dev);
        return rc;
      }
      pending += st.dev_bytes;
    }
    const int64_t n = (int64_t)staged.size();
    if ((rc = commit_tensors(ctx, staged))) return rc;
    if (num_q8) *num_q8 = n;
    return LLMCP_Q8_OK;
  });
}

// ------------------------------------------------------------------ ops --

// One-row GEMV (decode, or prefill with M == 1).  Narrow outputs quantize
// the input inside the GEMV; wide ones (lm_head) quantize it once first.
// `ws` (nullable): a fixed workspace in place of the context's.
static int gemv_common(llmcp_q8_ctx *ctx, const Rows &x, const Tensor *w0,
                       const Tensor *w1, const Rows &y, int activation,
                       int64_t *argmax_dev, const Rows *residual = nullptr,
                       const Workspace *fixed = nullptr) {
  Workspace ws;
  if (fixed) {
    ws = *fixed;
  } else {
    int rc = ensure_decode_scratch(ctx, w0->rows, w0->cols);
    if (rc) return rc;
    ws = ctx_workspace(ctx);
  }
  GemvLaunch l;
  const bool in_loop = gemv_quantizes_input(w0->rows, w0->cols, w1 ? 2 : 1) &&
                       (uintptr_t)x.data % (x.bf16 ? 8 : 16) == 0;
  if (in_loop) {
    l.x = x.data;
    l.x_bf16 = x.bf16;
  } else if (w1) {
    // the SwiGLU GEMV quantizes its row in each workgroup, from 16 B (8 B)
    // aligned loads
    return fail(LLMCP_Q8_DECLINED, "SwiGLU input row must be %d B aligned", x.bf16 ? 8 : 16);
  } else {
    const int64_t nblk = passes_for(w0->cols) * kPassBlocks;
    int rc = reserve(ctx, ws, (uint64_t)(nblk * kBlock), (uint64_t)(nblk * 4));
    if (rc) return rc;
    hipError_t e = launch_quantize(x.data, x.bf16, 1, w0->cols, w0->cols,
                                   ws.qa, nblk * kBlock, ws.sa, nblk, nblk,
                                   ctx->stream);
    if (e != hipSuccess) return hip_fail(e, "quantize launch");
    l.qa = ws.qa;
    l.sa = ws.sa;
  }
  l.w[0] = w0->dev;
  l.w[1] = w1 ? w1->dev : nullptr;
  l.y = y.data;
  l.y_bf16 = y.bf16;
  l.rows = w0->rows;
  l.cols = w0->cols;
  l.nmat = w1 ? 2 : 1;
  l.activation = activation;
  l.fma = ctx->fma();
  if (residual) l.residual = residual->data;
  if (argmax_dev) {
    l.keys = ws.keys;
    l.argmax_out = argmax_dev;
    // a failed call may have folded keys without the reduce that clears them
    if (*ws.keys_dirty) {
      hipError_t e = launch_argmax_reduce(ws.keys, nullptr, ctx->stream);
      if (e != hipSuccess) return hip_fail(e, "argmax clear launch");
      *ws.keys_dirty = false;
    }
  }
  hipError_t e = launch_gemv(l, ctx->stream);
  if (e != hipSuccess) {
    if (argmax_dev) *ws.keys_dirty = true;
    return hip_fail(e, "gemv launch");
  }
  return LLMCP_Q8_OK;
}

// The prefill GEMM reads its operands at 32-bit offsets from their bases
// (buffer-addressed loads): the weight and the tiled Q8_1 rows must each be
// below 4 GiB, else the call is declined (the caller's CPU path runs).
static int gemm_operands_fit(const Tensor *w, int64_t m) {
  const uint64_t nblk = (uint64_t)passes_for(w->cols) * kPassBlocks;
  const uint64_t rows = (uint64_t)((m + 31) / 32) * 32;
  if (w->dev_bytes > 0xFFFFFFFFull || rows * nblk * kBlock > 0xFFFFFFFFull)
    return fail(LLMCP_Q8_DECLINED,
                "prefill GEMM operands must each be below 4 GiB (weight %llu bytes, "
                "%lld rows of %lld blocks)",
                (unsigned long long)w->dev_bytes, (long long)m, (long long)nblk);
  return LLMCP_Q8_OK;
}

// Q8_1 of the input rows into the workspace (the GEMM's tiled layout; the
// context's scratch grows on first use for a larger M).
static int gemm_quantize(llmcp_q8_ctx *ctx, const Rows &in, const Tensor *w,
                         Workspace &ws) {
  const int64_t m = in.rows;
  if (int rc = gemm_operands_fit(w, m)) return rc;
  const int64_t nblk = passes_for(w->cols) * kPassBlocks;
  const int64_t row_tiles = (m + 31) / 32;  // the tiled layout pads M to 32
  int rc = reserve(ctx, ws, (uint64_t)(row_tiles * 32 * nblk * kBlock),
                   (uint64_t)(row_tiles * 32 * nblk * 4));
  if (rc) return rc;
  hipError_t e = launch_quantize_tiled(in.data, in.bf16, m, in.ld, w->cols,
                                       ws.qa, ws.sa, nblk, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "quantize launch");
  return LLMCP_Q8_OK;
}

// int8-MFMA GEMM of the quantized rows (gemm_quantize) against w.  `mul`
// (nullable, f32 [m, ldg]) turns the epilogue into the SwiGLU multiply.
// Both execution modes take the platform's epilogue: the reference's
// decode and prefill emitters of one platform share it (fma on aarch64,
// Q8Decode.cpp:200-203 and Q8Matmul.cpp:204-223; mul+add in the x86 scalar
// path, Q8Scalar.cpp:192-199, which serves both modes).
// In SPLIT_K mode (and unless `exact`, as for the lm_head) a GEMM whose
// tiles leave the GPU underfilled splits K (gemm_splits_for) and sums the
// splits' partial sums in a second kernel.
static int gemm_launch(llmcp_q8_ctx *ctx, const Workspace &ws, int64_t m,
                       const Tensor *w, const Rows &out, int activation,
                       const float *mul, int64_t ldg,
                       const Rows *residual = nullptr, bool exact = false) {
  if (int rc = gemm_operands_fit(w, m)) return rc;
  const int64_t nblk = passes_for(w->cols) * kPassBlocks;
  GemmLaunch g;
  g.qa = ws.qa;
  g.sa = ws.sa;
  g.row_tiles = (int32_t)((m + 31) / 32);
  g.nblk = (int32_t)nblk;
  g.w = w->dev;
  g.rows = w->rows;
  g.cols = w->cols;
  g.m = m;
  g.y = out.data;
  g.y_bf16 = out.bf16;
  g.ldy = out.ld;
  g.activation = activation;
  g.fma = ctx->fma();
  g.mul = mul;
  g.ldg = ldg;
  if (residual) {
    g.add = residual->data;
    g.ldr = residual->ld;
  }
  if (!exact && ctx->accumulation == LLMCP_Q8_ACCUM_SPLIT_K && !ws.fixed &&
      w->rows % 4 == 0) {
    const int32_t splits = gemm_splits_for(m, w->rows, w->cols, ctx->test_splits);
    if (splits > 1) {
      const uint64_t bytes = (uint64_t)splits * (uint64_t)m * (uint64_t)w->rows * 4u;
      int rc = grow(ctx, ctx->part, ctx->part_bytes, bytes, "split-K partial sums");
      if (rc) return rc;
      g.splits = splits;
      g.part = ctx->part;
    }
  }
  hipError_t e = launch_gemm(g, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "gemm launch");
  return LLMCP_Q8_OK;
}

static int gemm_common(llmcp_q8_ctx *ctx, const Rows &in, const Tensor *w,
                       const Rows &out, int activation,
                       const Workspace *fixed = nullptr, bool exact = false) {
  Workspace ws = fixed ? *fixed : ctx_workspace(ctx);
  int rc = gemm_quantize(ctx, in, w, ws);
  if (rc) return rc;
  return gemm_launch(ctx, ws, in.rows, w, out, activation, nullptr, 0, nullptr, exact);
}

static int check_linear_shapes(const Rows &in, const Tensor *w,
                               const Rows &out) {
  if (in.cols != w->cols)
    return fail(LLMCP_Q8_DECLINED, "input K %lld != weight K %lld",
                (long long)in.cols, (long long)w->cols);
  if (out.cols != w->rows)
    return fail(LLMCP_Q8_DECLINED, "output N %lld != weight N %lld",
                (long long)out.cols, (long long)w->rows);
  if (out.rows != in.rows)
    return fail(LLMCP_Q8_DECLINED, "output outer dimension must match input");
  return LLMCP_Q8_OK;
}

static int check_mode(int32_t mode) {
  if (mode != LLMCP_Q8_DECODE && mode != LLMCP_Q8_PREFILL)
    return fail(LLMCP_Q8_EINVAL, "unknown execution mode %d", mode);
  return LLMCP_Q8_OK;
}

static const char *kDenseMsg = "activations must be row-major memrefs";

static int linear_impl(llmcp_q8_ctx *ctx, const Rows &in,
                       const llmcp_memref_i8_1d *weight, const Rows &out,
                       int32_t activation, int32_t execution_mode) {
  const Tensor *w = nullptr;
  int rc = resolve_weight(ctx, weight, &w);
  if (rc) return rc;
  if ((rc = check_linear_shapes(in, w, out))) return rc;
  if (activation < LLMCP_Q8_ACT_NONE || activation > LLMCP_Q8_ACT_SOFTPLUS)
    return fail(LLMCP_Q8_DECLINED, "unsupported activation %d", activation);
  if ((rc = check_mode(execution_mode))) return rc;
  const int64_t m = in.rows;
  if (m == 0) return LLMCP_Q8_OK;
  if ((rc = set_device(ctx))) return rc;
  // One row (decode, or a one-row prefill such as the last-row lm_head):
  // the GEMV beats a 1/128-full GEMM tile.  Several rows: the GEMM (in
  // either mode, as Q8Decode.cpp:236-256 accepts any M).  Both compute the
  // platform's epilogue in block order.
  if (m == 1) return gemv_common(ctx, in, w, nullptr, out, activation, nullptr);
  return gemm_common(ctx, in, w, out, activation);
}

// llmcp.linear + llmcp.add (ModelBuilder.cpp:271, :275): the residual add
// in the GEMV's or GEMM's epilogue.
static int linear_add_impl(llmcp_q8_ctx *ctx, const Rows &in,
                           const llmcp_memref_i8_1d *weight, const Rows &res,
                           const Rows &out, int32_t execution_mode) {
  const Tensor *w = nullptr;
  int rc = resolve_weight(ctx, weight, &w);
  if (rc) return rc;
  if ((rc = check_linear_shapes(in, w, out))) return rc;
  if (res.rows != out.rows || res.cols != out.cols)
    return fail(LLMCP_Q8_DECLINED, "residual must be [M, N] like the output");
  if ((rc = check_mode(execution_mode))) return rc;
  const int64_t m = in.rows;
  if (m == 0) return LLMCP_Q8_OK;
  if ((rc = set_device(ctx))) return rc;
  if (m == 1)
    return gemv_common(ctx, in, w, nullptr, out, LLMCP_Q8_ACT_NONE, nullptr, &res);
  Workspace ws = ctx_workspace(ctx);
  if ((rc = gemm_quantize(ctx, in, w, ws))) return rc;
  return gemm_launch(ctx, ws, m, w, out, LLMCP_Q8_ACT_NONE, nullptr, 0, &res);
}

// Linears that share one input (the model builder's in_proj_qkv/z/a/b and
// q/k/v, ModelBuilder.cpp:229-236, :288-294): one input quantization and,
// for one row, one GEMV launch over every weight's lane groups.  Results
// equal the separate llmcp_q8_linear calls bit for bit.
static int linear_group_check(llmcp_q8_ctx *ctx, const Rows &in, int32_t count,
                              const llmcp_memref_i8_1d *const *weights,
                              const Rows *outs, const int32_t *acts,
                              int32_t execution_mode, const Tensor **w) {
  if (count < 1 || count > kMaxGroup)
    return fail(LLMCP_Q8_EINVAL, "group of %d linears (1 to %d)", count,
                kMaxGroup);
  for (int32_t i = 0; i < count; ++i) {
    int rc = resolve_weight(ctx, weights[i], &w[i]);
    if (rc) return rc;
    if ((rc = check_linear_shapes(in, w[i], outs[i]))) return rc;
    const int32_t act = acts ? acts[i] : LLMCP_Q8_ACT_NONE;
    if (act < LLMCP_Q8_ACT_NONE || act > LLMCP_Q8_ACT_SOFTPLUS)
      return fail(LLMCP_Q8_DECLINED, "unsupported activation %d", act);
  }
  return check_mode(execution_mode);
}

// The checked group on the current device.  `prequantized`: for several
// rows, the workspace already holds the rows' Q8_1 in the tiled layout
// (written by the RMSNorm that produced them).
static int linear_group_run(llmcp_q8_ctx *ctx, const Rows &in, int32_t count,
                            const Tensor *const *w, const Rows *outs,
                            const int32_t *acts, bool prequantized) {
  const int64_t m = in.rows;
  int rc = LLMCP_Q8_OK;
  auto act_of = [&](int32_t i) { return acts ? acts[i] : LLMCP_Q8_ACT_NONE; };
  if (m > 1) {
    // one quantization of the input rows, then each weight's GEMM (every
    // weight checked before anything is launched)
    for (int32_t i = 0; i < count; ++i)
      if ((rc = gemm_operands_fit(w[i], m))) return rc;
    Workspace ws = ctx_workspace(ctx);
    if (!prequantized && (rc = gemm_quantize(ctx, in, w[0], ws))) return rc;
    for (int32_t i = 0; i < count; ++i)
      if ((rc = gemm_launch(ctx, ws, m, w[i], outs[i], act_of(i), nullptr, 0)))
        return rc;
    return LLMCP_Q8_OK;
  }
  int64_t groups = 0;
  bool same_type = true;
  for (int32_t i = 0; i < count; ++i) {
    groups += w[i]->rows / kLanes;
    same_type &= outs[i].bf16 == outs[0].bf16;
  }
  // One launch when every workgroup can quantize the row itself (aligned
  // row, not wider than one-launch GEMVs quantize in-workgroup); otherwise
  // each weight's GEMV in turn.
  const bool one_launch = same_type && (uintptr_t)in.data % (in.bf16 ? 8 : 16) == 0 &&
                          groups <= kInLoopQuantMaxGroups;
  if (!one_launch || count == 1) {
    for (int32_t i = 0; i < count; ++i)
      if ((rc = gemv_common(ctx, in, w[i], nullptr, outs[i], act_of(i), nullptr)))
        return rc;
    return LLMCP_Q8_OK;
  }
  if ((rc = ensure_decode_scratch(ctx, w[0]->rows, w[0]->cols))) return rc;
  GemvLaunch l;
  l.x = in.data;
  l.x_bf16 = in.bf16;
  l.y_bf16 = outs[0].bf16;
  l.rows = groups * kLanes;
  l.cols = w[0]->cols;
  l.fma = ctx->fma();
  l.ngroup = count;
  for (int32_t i = 0; i < count; ++i) {
    l.gw[i] = w[i]->dev;
    l.gy[i] = outs[i].data;
    l.grows[i] = w[i]->rows;
    l.gact[i] = act_of(i);
  }
  hipError_t e = launch_gemv(l, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "grouped gemv launch");
  return LLMCP_Q8_OK;
}

static int linear_group_impl(llmcp_q8_ctx *ctx, const Rows &in, int32_t count,
                             const llmcp_memref_i8_1d *const *weights,
                             const Rows *outs, const int32_t *acts,
                             int32_t execution_mode) {
  const Tensor *w[kMaxGroup];
  int rc = linear_group_check(ctx, in, count, weights, outs, acts, execution_mode, w);
  if (rc) return rc;
  if (in.rows == 0) return LLMCP_Q8_OK;
  if ((rc = set_device(ctx))) return rc;
  return linear_group_run(ctx, in, count, w, outs, acts, false);
}

// ------------------------------------------------------------- RMSNorm --
// The path's upstream neighbour: llmcp.rms_norm as the reference lowers it
// for decode rows (DecodeNormalization.cpp:71-154, :160-171) and for
// prefill (LowerToLinalg.cpp:245-300), one row at a time with a serial f32
// sum of squares.  Bit-exact; the serial sum bounds it at about one
// dependent add per element (rows run in parallel).


static int check_norm(const Rows &in, const NormWeight &nw, const Rows &out) {
  if (out.rows != in.rows || out.cols != in.cols)
    return fail(LLMCP_Q8_DECLINED, "RMSNorm output must be [M, H] like its input");
  if (nw.len != in.cols)
    return fail(LLMCP_Q8_DECLINED, "RMSNorm weight has %lld values for H = %lld",
                (long long)nw.len, (long long)in.cols);
  if (in.cols % kBlock != 0)
    return fail(LLMCP_Q8_DECLINED, "RMSNorm width %lld is not a multiple of 32",
                (long long)in.cols);
  if ((uintptr_t)nw.data % (nw.bf16 ? 8 : 16) != 0)
    return fail(LLMCP_Q8_DECLINED, "RMSNorm weight must be %d B aligned",
                nw.bf16 ? 8 : 16);
  return LLMCP_Q8_OK;
}

static int rmsnorm_impl(llmcp_q8_ctx *ctx, const Rows &in, const NormWeight &nw,
                        float eps, int32_t zero_centered, const Rows &out) {
  int rc = check_norm(in, nw, out);
  if (rc) return rc;
  if (in.rows == 0) return LLMCP_Q8_OK;
  if ((rc = set_device(ctx))) return rc;
  hipError_t e = launch_rmsnorm(in.data, in.bf16, in.rows, in.ld, in.cols, nw.data,
                                nw.bf16, eps, zero_centered != 0, out.data, out.bf16,
                                out.ld, nullptr, nullptr, 0, 0, ctx->stream, ctx->rmsnorm_skew);
  if (e != hipSuccess) return hip_fail(e, "rmsnorm launch");
  return LLMCP_Q8_OK;
}

// llmcp.gated_rms_norm (the linear-attention output norm in front of
// out_proj, ModelBuilder.cpp:259-266): groups of `group` values per row,
// dense rows only.
static int gated_rmsnorm_impl(llmcp_q8_ctx *ctx, const Rows &in, const Rows &gate,
                              const NormWeight &nw, int64_t group, float eps,
                              int32_t gate_activated, const Rows &out) {
  if (out.rows != in.rows || out.cols != in.cols || gate.rows != in.rows ||
      gate.cols != in.cols)
    return fail(LLMCP_Q8_DECLINED, "gated RMSNorm input, gate and output must share [M, H]");
  if (group <= 0 || group % kBlock != 0 || in.cols % group != 0)
    return fail(LLMCP_Q8_DECLINED, "group size %lld must be a multiple of 32 dividing H",
                (long long)group);
  if (nw.len != group)
    return fail(LLMCP_Q8_DECLINED, "gated RMSNorm weight has %lld values for groups of %lld",
                (long long)nw.len, (long long)group);
  if ((uintptr_t)nw.data % 16 != 0)
    return fail(LLMCP_Q8_DECLINED, "gated RMSNorm weight must be 16 B aligned");
  if ((in.rows > 1 && in.ld != in.cols) || (gate.rows > 1 && gate.ld != gate.cols) ||
      (out.rows > 1 && out.ld != out.cols))
    return fail(LLMCP_Q8_DECLINED, "gated RMSNorm rows must be dense");
  if (in.rows == 0) return LLMCP_Q8_OK;
  int rc = set_device(ctx);
  if (rc) return rc;
  hipError_t e = launch_gated_rmsnorm(in.data, gate.data, in.bf16, in.rows * (in.cols / group),
                                      group, (const float *)nw.data, eps, gate_activated != 0,
                                      out.data, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "gated rmsnorm launch");
  return LLMCP_Q8_OK;
}

// RMSNorm, then linears on the normed rows (the model builder's
// input_layernorm -> in_proj_qkv/z/a/b or q/k/v, post_attention_layernorm
// -> gate/up; ModelBuilder.cpp:225-236, :284-294).  For several rows the
// norm's epilogue writes the rows' Q8_1 for the GEMMs (no separate
// quantization); one row goes through the grouped GEMV, which quantizes
// the normed row in each workgroup.  Bit-exact to llmcp_q8_rmsnorm followed
// by llmcp_q8_linear_group.
static int rmsnorm_group_impl(llmcp_q8_ctx *ctx, const Rows &in, const NormWeight &nw,
                              float eps, int32_t zero_centered, const Rows &normed,
                              int32_t count, const llmcp_memref_i8_1d *const *weights,
                              const Rows *outs, const int32_t *acts,
                              int32_t execution_mode) {
  int rc = check_norm(in, nw, normed);
  if (rc) return rc;
  const Tensor *w[kMaxGroup];
  if ((rc = linear_group_check(ctx, normed, count, weights, outs, acts, execution_mode, w)))
    return rc;
  const int64_t m = in.rows;
  if (m == 0) return LLMCP_Q8_OK;
  if ((rc = set_device(ctx))) return rc;
  if (m == 1) {
    hipError_t e = launch_rmsnorm(in.data, in.bf16, 1, in.ld, in.cols, nw.data, nw.bf16,
                                  eps, zero_centered != 0, normed.data, normed.bf16,
                                  normed.ld, nullptr, nullptr, 0, 0, ctx->stream,
                                  ctx->rmsnorm_skew);
    if (e != hipSuccess) return hip_fail(e, "rmsnorm launch");
    return linear_group_run(ctx, normed, count, w, outs, acts, false);
  }
  for (int32_t i = 0; i < count; ++i)
    if ((rc = gemm_operands_fit(w[i], m))) return rc;
  const int64_t nblk = passes_for(in.cols) * kPassBlocks;
  const int64_t row_tiles = (m + 31) / 32;
  Workspace ws = ctx_workspace(ctx);
  if ((rc = reserve(ctx, ws, (uint64_t)(row_tiles * 32 * nblk * kBlock),
                    (uint64_t)(row_tiles * 32 * nblk * 4))))
    return rc;
  hipError_t e = launch_rmsnorm(in.data, in.bf16, m, in.ld, in.cols, nw.data, nw.bf16, eps,
                                zero_centered != 0, normed.data, normed.bf16, normed.ld,
                                ws.qa, ws.sa, nblk, 2, ctx->stream, ctx->rmsnorm_skew);
  if (e != hipSuccess) return hip_fail(e, "rmsnorm launch");
  return linear_group_run(ctx, normed, count, w, outs, acts, true);
}

static int swiglu_impl(llmcp_q8_ctx *ctx, const Rows &in,
                       const llmcp_memref_i8_1d *w_gate,
                       const llmcp_memref_i8_1d *w_up, const Rows &out,
                       int32_t execution_mode) {
  const Tensor *wg = nullptr, *wu = nullptr;
  int rc = resolve_weight(ctx, w_gate, &wg);
  if (rc) return rc;
  if ((rc = resolve_weight(ctx, w_up, &wu))) return rc;
  if (wg->rows != wu->rows || wg->cols != wu->cols)
    return fail(LLMCP_Q8_DECLINED, "gate and up weights differ in shape");
  if ((rc = check_linear_shapes(in, wg, out))) return rc;
  if ((rc = check_mode(execution_mode))) return rc;
  const int64_t m = in.rows;
  if (m == 0) return LLMCP_Q8_OK;
  if ((rc = set_device(ctx))) return rc;
  if (m == 1) return gemv_common(ctx, in, wg, wu, out, LLMCP_Q8_ACT_NONE, nullptr);
  // Several rows: the input quantized once; the gate GEMM with SiLU, then the up
  // GEMM whose epilogue does the multiply (MulOpLowering,
  // LowerToLinalg.cpp:377-393) with the gate's output.  f32: the gate goes
  // straight into the output and the up GEMM multiplies it in place.  bf16:
  // the gate goes to f32 scratch and the multiply rounds both factors to
  // bf16 first.
  Rows g = out;
  if (out.bf16) {
    rc = grow(ctx, ctx->up, ctx->up_bytes, (uint64_t)(m * wg->rows) * 4,
              "prefill SwiGLU scratch");
    if (rc) return rc;
    g.data = ctx->up;
    g.bf16 = false;
    g.ld = wg->rows;
  }
  Workspace ws = ctx_workspace(ctx);
  if ((rc = gemm_quantize(ctx, in, wg, ws))) return rc;
  if ((rc = gemm_launch(ctx, ws, m, wg, g, LLMCP_Q8_ACT_SILU, nullptr, 0)))
    return rc;
  return gemm_launch(ctx, ws, m, wu, out, LLMCP_Q8_ACT_NONE,
                     (const float *)g.data, g.ld);
}

static int lm_head_impl(llmcp_q8_ctx *ctx, const Rows &in,
                        const llmcp_memref_i8_1d *table, const Rows &logits,
                        int64_t *argmax_dev, int32_t execution_mode,
                        const Workspace *fixed = nullptr) {
  const Tensor *w = nullptr;
  int rc = resolve_weight(ctx, table, &w);
  if (rc) return rc;
  if ((rc = check_linear_shapes(in, w, logits))) return rc;
  if ((rc = check_mode(execution_mode))) return rc;
  const int64_t m = in.rows;
  if (m == 0) return LLMCP_Q8_OK;
  if ((rc = set_device(ctx))) return rc;
  if (m == 1)
    return gemv_common(ctx, in, w, nullptr, logits, LLMCP_Q8_ACT_NONE,
                       argmax_dev, nullptr, fixed);
  // Several rows: the GEMM writes every row's logits, then the first
  // maximum of the last row is reduced from HBM.  Always the serial block
  // order: the argmax id must be the reference's.
  if ((rc = gemm_common(ctx, in, w, logits, LLMCP_Q8_ACT_NONE, fixed, true)))
    return rc;
  if (!argmax_dev) return LLMCP_Q8_OK;
  Workspace ws;
  if (fixed) {
    ws = *fixed;
  } else {
    if ((rc = ensure_argmax_slots(ctx))) return rc;
    ws = ctx_workspace(ctx);
  }
  if (*ws.keys_dirty) {
    hipError_t e = launch_argmax_reduce(ws.keys, nullptr, ctx->stream);
    if (e != hipSuccess) return hip_fail(e, "argmax clear launch");
    *ws.keys_dirty = false;
  }
  hipError_t e = launch_argmax_row((const float *)logits.data + (m - 1) * logits.ld,
                                   logits.cols, argmax_dev, ws.keys, ctx->stream);
  if (e != hipSuccess) {
    *ws.keys_dirty = true;
    return hip_fail(e, "argmax launch");
  }
  return LLMCP_Q8_OK;
}

static int mlp_impl(llmcp_q8_ctx *ctx, const Rows &in,
                    const llmcp_memref_i8_1d *w_gate,
                    const llmcp_memref_i8_1d *w_up,
                    const llmcp_memref_i8_1d *w_down, const Rows *hidden,
                    const Rows &out, int32_t execution_mode) {
  const Tensor *wg = nullptr, *wu = nullptr, *wd = nullptr;
  int rc = resolve_weight(ctx, w_gate, &wg);
  if (!rc) rc = resolve_weight(ctx, w_up, &wu);
  if (!rc) rc = resolve_weight(ctx, w_down, &wd);
  if (rc) return rc;
  if (wg->rows != wu->rows || wg->cols != wu->cols || wd->cols != wg->rows ||
      wd->rows != wg->cols)
    return fail(LLMCP_Q8_DECLINED, "gate/up [F,H] and down [H,F] shapes differ");
  if (wg->rows % kBlock)
    return fail(LLMCP_Q8_DECLINED, "MLP width must be a multiple of 32");
  if (in.cols != wg->cols || out.cols != wd->rows || out.rows != in.rows)
    return fail(LLMCP_Q8_DECLINED, "MLP input/output must be [M, H] row-major");
  if (hidden && (hidden->cols != wg->rows || hidden->rows != in.rows))
    return fail(LLMCP_Q8_DECLINED, "MLP hidden must be [M, F] row-major");
  if ((rc = check_mode(execution_mode))) return rc;
  const int64_t m = in.rows;
  if (m == 0) return LLMCP_Q8_OK;
  if ((rc = set_device(ctx))) return rc;
  if (m > 1) {
    // Several rows: the SwiGLU GEMMs of llmcp_q8_swiglu (gate with SiLU,
    // then up with the multiply in its epilogue) into h, then the GEMM of h,
    // with the platform's epilogue as for llmcp_q8_linear.
    if ((rc = gemm_operands_fit(wg, m)) || (rc = gemm_operands_fit(wd, m))) return rc;
    const int64_t f = wg->rows;
    Rows h;
    if (hidden) {
      h = *hidden;
    } else {
      const uint64_t bytes = (uint64_t)(m * f) * (out.bf16 ? 2 : 4);
      if ((rc = grow(ctx, ctx->hf, ctx->hf_bytes, bytes, "mlp hidden"))) return rc;
      h.data = ctx->hf;
      h.rows = m;
      h.cols = h.ld = f;
      h.bf16 = out.bf16;
    }
    Rows g = h;  // the gate's output: h itself (f32) or f32 scratch (bf16)
    if (h.bf16) {
      if ((rc = grow(ctx, ctx->up, ctx->up_bytes, (uint64_t)(m * f) * 4,
                     "prefill SwiGLU scratch")))
        return rc;
      g.data = ctx->up;
      g.bf16 = false;
      g.ld = f;
    }
    Workspace ws = ctx_workspace(ctx);
    if ((rc = gemm_quantize(ctx, in, wg, ws))) return rc;
    if ((rc = gemm_launch(ctx, ws, m, wg, g, LLMCP_Q8_ACT_SILU, nullptr, 0)))
      return rc;
    if ((rc = gemm_launch(ctx, ws, m, wu, h, LLMCP_Q8_ACT_NONE,
                          (const float *)g.data, g.ld)))
      return rc;
    return gemm_common(ctx, h, wd, out, LLMCP_Q8_ACT_NONE);
  }
  if ((rc = ensure_decode_scratch(ctx, wg->rows, wg->cols))) return rc;
  // Gate/up with the SwiGLU epilogue into h, then the down GEMV, which
  // quantizes h per workgroup (Q8Decode.cpp:83-120) as its input.  h has
  // the output's element type unless the caller passes its own buffer.
  Rows h;
  if (hidden) {
    h = *hidden;
  } else {
    h.data = ctx->hf;
    h.rows = 1;
    h.cols = h.ld = wg->rows;
    h.bf16 = out.bf16;
  }
  rc = gemv_common(ctx, in, wg, wu, h, LLMCP_Q8_ACT_NONE, nullptr);
  if (rc) return rc;
  return gemv_common(ctx, h, wd, nullptr, out, LLMCP_Q8_ACT_NONE, nullptr);
}

static int embedding_impl(llmcp_q8_ctx *ctx, const llmcp_memref_i64_1d *tokens,
                          const llmcp_memref_i8_1d *table, const Rows &out) {
  const Tensor *w = nullptr;
  int rc = resolve_weight(ctx, table, &w);
  if (rc) return rc;
  if (tokens->strides[0] != 1 && tokens->sizes[0] > 1)
    return fail(LLMCP_Q8_DECLINED, "tokens must be contiguous");
  if (out.cols != w->cols || out.rows != tokens->sizes[0])
    return fail(LLMCP_Q8_DECLINED, "embedding output must be [tokens, hidden]");
  // one thread per (token, 4 columns) for f32 rows (8 for bf16) on a
  // one-dimensional grid of 256-thread workgroups; HIP bounds the grid's
  // work-items (workgroups x 256) by 2^32 - 1
  if (tokens->sizes[0] > (1ll << 40) ||
      (tokens->sizes[0] * (w->cols / (out.bf16 ? 8 : 4)) + 255) / 256 * 256 > 0xFFFFFFFFll)
    return fail(LLMCP_Q8_DECLINED, "too many tokens for one launch (%lld)",
                (long long)tokens->sizes[0]);
  if ((rc = set_device(ctx))) return rc;
  hipError_t e = launch_embedding(tokens->data + tokens->offset,
                                  tokens->sizes[0], w->dev, w->rows, w->cols,
                                  out.data, out.bf16, out.ld, ctx->err_flag,
                                  ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "embedding launch");
  return LLMCP_Q8_OK;
}

// ---- public entries: f32 and bf16 activations

int llmcp_q8_linear(llmcp_q8_ctx *ctx, const llmcp_memref_f32_2d *input,
                    const llmcp_memref_i8_1d *weight,
                    llmcp_memref_f32_2d *output, int32_t activation,
                    int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
    Rows in, out;
    if (!view_of(input, false, in) || !view_of(output, false, out))
      return fail(LLMCP_Q8_DECLINED, kDenseMsg);
    return linear_impl(ctx, in, weight, out, activation, execution_mode);
  });
}

int llmcp_q8_linear_bf16(llmcp_q8_ctx *ctx, const llmcp_memref_bf16_2d *input,
                         const llmcp_memref_i8_1d *weight,
                         llmcp_memref_bf16_2d *output, int32_t activation,
                         int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
    Rows in, out;
    if (!view_of(input, true, in) || !view_of(output, true, out))
      return fail(LLMCP_Q8_DECLINED, kDenseMsg);
    return linear_impl(ctx, in, weight, out, activation, execution_mode);
  });
}

int llmcp_q8_linear_add(llmcp_q8_ctx *ctx, const llmcp_memref_f32_2d *input,
                        const llmcp_memref_i8_1d *weight,
                        const llmcp_memref_f32_2d *residual,
                        llmcp_memref_f32_2d *output, int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!ctx || !residual) return fail(LLMCP_Q8_EINVAL, "null argument");
    Rows in, res, out;
    if (!view_of(input, false, in) || !view_of(residual, false, res) ||
        !view_of(output, false, out))
      return fail(LLMCP_Q8_DECLINED, kDenseMsg);
    return linear_add_impl(ctx, in, weight, res, out, execution_mode);
  });
}

int llmcp_q8_linear_add_bf16(llmcp_q8_ctx *ctx,
                             const llmcp_memref_bf16_2d *input,
                             const llmcp_memref_i8_1d *weight,
                             const llmcp_memref_bf16_2d *residual,
                             llmcp_memref_bf16_2d *output,
                             int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!ctx || !residual) return fail(LLMCP_Q8_EINVAL, "null argument");
    Rows in, res, out;
    if (!view_of(input, true, in) || !view_of(residual, true, res) ||
        !view_of(output, true, out))
      return fail(LLMCP_Q8_DECLINED, kDenseMsg);
    return linear_add_impl(ctx, in, weight, res, out, execution_mode);
  });
}

int llmcp_q8_linear_group(llmcp_q8_ctx *ctx, const llmcp_memref_f32_2d *input,
                          int32_t count,
                          const llmcp_memref_i8_1d *const *weights,
                          llmcp_memref_f32_2d *const *outputs,
                          const int32_t *activations, int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!ctx || !weights || !outputs) return fail(LLMCP_Q8_EINVAL, "null argument");
    if (count < 1 || count > kMaxGroup)
      return fail(LLMCP_Q8_EINVAL, "group of %d linears (1 to %d)", count, kMaxGroup);
    Rows in, outs[kMaxGroup];
    if (!view_of(input, false, in)) return fail(LLMCP_Q8_DECLINED, kDenseMsg);
    for (int32_t i = 0; i < count; ++i)
      if (!view_of(outputs[i], false, outs[i]))
        return fail(LLMCP_Q8_DECLINED, kDenseMsg);
    return linear_group_impl(ctx, in, count, weights, outs, activations,
                             execution_mode);
  });
}

int llmcp_q8_linear_group_bf16(llmcp_q8_ctx *ctx,
                               const llmcp_memref_bf16_2d *input, int32_t count,
                               const llmcp_memref_i8_1d *const *weights,
                               llmcp_memref_bf16_2d *const *outputs,
                               const int32_t *activations,
                               int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!ctx || !weights || !outputs) return fail(LLMCP_Q8_EINVAL, "null argument");
    if (count < 1 || count > kMaxGroup)
      return fail(LLMCP_Q8_EINVAL, "group of %d linears (1 to %d)", count, kMaxGroup);
    Rows in, outs[kMaxGroup];
    if (!view_of(input, true, in)) return fail(LLMCP_Q8_DECLINED, kDenseMsg);
    for (int32_t i = 0; i < count; ++i)
      if (!view_of(outputs[i], true, outs[i]))
        return fail(LLMCP_Q8_DECLINED, kDenseMsg);
    return linear_group_impl(ctx, in, count, weights, outs, activations,
                             execution_mode);
  });
}

int llmcp_q8_rmsnorm(llmcp_q8_ctx *ctx, const llmcp_memref_f32_2d *input,
                     const llmcp_memref_f32_1d *weight, float eps,
                     int32_t zero_centered, llmcp_memref_f32_2d *output) {
  return guarded([&]() -> int {
    if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
    Rows in, out;
    NormWeight nw;
    if (!view_of(input, false, in) || !view_of(output, false, out))
      return fail(LLMCP_Q8_DECLINED, kDenseMsg);
    if (!norm_weight_of(weight, false, nw))
      return fail(LLMCP_Q8_DECLINED, "RMSNorm weight must be a dense vector");
    return rmsnorm_impl(ctx, in, nw, eps, zero_centered, out);
  });
}

int llmcp_q8_rmsnorm_bf16(llmcp_q8_ctx *ctx, const llmcp_memref_bf16_2d *input,
                          const llmcp_memref_bf16_1d *weight, float eps,
                          int32_t zero_centered, llmcp_memref_bf16_2d *output) {
  return guarded([&]() -> int {
    if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
    Rows in, out;
    NormWeight nw;
    if (!view_of(input, true, in) || !view_of(output, true, out))
      return fail(LLMCP_Q8_DECLINED, kDenseMsg);
    if (!norm_weight_of(weight, true, nw))
      return fail(LLMCP_Q8_DECLINED, "RMSNorm weight must be a dense vector");
    return rmsnorm_impl(ctx, in, nw, eps, zero_centered, out);
  });
}

int llmcp_q8_gated_rmsnorm(llmcp_q8_ctx *ctx, const llmcp_memref_f32_2d *input,
                           const llmcp_memref_f32_2d *gate,
                           const llmcp_memref_f32_1d *weight, int64_t group_size,
                           float eps, int32_t gate_activated,
                           llmcp_memref_f32_2d *output) {
  return guarded([&]() -> int {
    if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
    Rows in, g, out;
    NormWeight nw;
    if (!view_of(input, false, in) || !view_of(gate, false, g) || !view_of(output, false, out))
      return fail(LLMCP_Q8_DECLINED, kDenseMsg);
    if (!norm_weight_of(weight, false, nw))
      return fail(LLMCP_Q8_DECLINED, "RMSNorm weight must be a dense vector");
    return gated_rmsnorm_impl(ctx, in, g, nw, group_size, eps, gate_activated, out);
  });
}

int llmcp_q8_gated_rmsnorm_bf16(llmcp_q8_ctx *ctx, const llmcp_memref_bf16_2d *input,
                                const llmcp_memref_bf16_2d *gate,
                                const llmcp_memref_f32_1d *weight, int64_t group_size,
                                float eps, int32_t gate_activated,
                                llmcp_memref_bf16_2d *output) {
  return guarded([&]() -> int {
    if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
    Rows in, g, out;
    NormWeight nw;
    if (!view_of(input, true, in) || !view_of(gate, true, g) || !view_of(output, true, out))
      return fail(LLMCP_Q8_DECLINED, kDenseMsg);
    if (!norm_weight_of(weight, false, nw))
      return fail(LLMCP_Q8_DECLINED, "RMSNorm weight must be a dense vector");
    return gated_rmsnorm_impl(ctx, in, g, nw, group_size, eps, gate_activated, out);
  });
}

int llmcp_q8_rmsnorm_linear_group(llmcp_q8_ctx *ctx, const llmcp_memref_f32_2d *input,
                                  const llmcp_memref_f32_1d *norm_weight, float eps,
                                  int32_t zero_centered, llmcp_memref_f32_2d *normed,
                                  int32_t count, const llmcp_memref_i8_1d *const *weights,
                                  llmcp_memref_f32_2d *const *outputs,
                                  const int32_t *activations, int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!ctx || !weights || !outputs) return fail(LLMCP_Q8_EINVAL, "null argument");
    if (count < 1 || count > kMaxGroup)
      return fail(LLMCP_Q8_EINVAL, "group of %d linears (1 to %d)", count, kMaxGroup);
    Rows in, nr, outs[kMaxGroup];
    NormWeight nw;
    if (!view_of(input, false, in) || !view_of(normed, false, nr))
      return fail(LLMCP_Q8_DECLINED, kDenseMsg);
    for (int32_t i = 0; i < count; ++i)
      if (!view_of(outputs[i], false, outs[i])) return fail(LLMCP_Q8_DECLINED, kDenseMsg);
    if (!norm_weight_of(norm_weight, false, nw))
      return fail(LLMCP_Q8_DECLINED, "RMSNorm weight must be a dense vector");
    return rmsnorm_group_impl(ctx, in, nw, eps, zero_centered, nr, count, weights, outs,
                              activations, execution_mode);
  });
}

int llmcp_q8_rmsnorm_linear_group_bf16(
    llmcp_q8_ctx *ctx, const llmcp_memref_bf16_2d *input,
    const llmcp_memref_bf16_1d *norm_weight, float eps, int32_t zero_centered,
    llmcp_memref_bf16_2d *normed, int32_t count, const llmcp_memref_i8_1d *const *weights,
    llmcp_memref_bf16_2d *const *outputs, const int32_t *activations,
    int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!ctx || !weights || !outputs) return fail(LLMCP_Q8_EINVAL, "null argument");
    if (count < 1 || count > kMaxGroup)
      return fail(LLMCP_Q8_EINVAL, "group of %d linears (1 to %d)", count, kMaxGroup);
    Rows in, nr, outs[kMaxGroup];
    NormWeight nw;
    if (!view_of(input, true, in) || !view_of(normed, true, nr))
      return fail(LLMCP_Q8_DECLINED, kDenseMsg);
    for (int32_t i = 0; i < count; ++i)
      if (!view_of(outputs[i], true, outs[i])) return fail(LLMCP_Q8_DECLINED, kDenseMsg);
    if (!norm_weight_of(norm_weight, true, nw))
      return fail(LLMCP_Q8_DECLINED, "RMSNorm weight must be a dense vector");
    return rmsnorm_group_impl(ctx, in, nw, eps, zero_centered, nr, count, weights, outs,
                              activations, execution_mode);
  });
}

int llmcp_q8_swiglu(llmcp_q8_ctx *ctx, const llmcp_memref_f32_2d *input,
                    const llmcp_memref_i8_1d *w_gate,
                    const llmcp_memref_i8_1d *w_up,
                    llmcp_memref_f32_2d *output, int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
    Rows in, out;
    if (!view_of(input, false, in) || !view_of(output, false, out))
      return fail(LLMCP_Q8_DECLINED, kDenseMsg);
    return swiglu_impl(ctx, in, w_gate, w_up, out, execution_mode);
  });
}

int llmcp_q8_swiglu_bf16(llmcp_q8_ctx *ctx, const llmcp_memref_bf16_2d *input,
                         const llmcp_memref_i8_1d *w_gate,
                         const llmcp_memref_i8_1d *w_up,
                         llmcp_memref_bf16_2d *output, int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
    Rows in, out;
    if (!view_of(input, true, in) || !view_of(output, true, out))
      return fail(LLMCP_Q8_DECLINED, kDenseMsg);
    return swiglu_impl(ctx, in, w_gate, w_up, out, execution_mode);
  });
}

int llmcp_q8_lm_head(llmcp_q8_ctx *ctx, const llmcp_memref_f32_2d *hidden,
                     const llmcp_memref_i8_1d *table,
                     llmcp_memref_f32_2d *logits, int64_t *argmax_dev,
                     int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
    Rows in, out;
    if (!view_of(hidden, false, in) || !view_of(logits, false, out))
      return fail(LLMCP_Q8_DECLINED, kDenseMsg);
    return lm_head_impl(ctx, in, table, out, argmax_dev, execution_mode);
  });
}

int llmcp_q8_lm_head_bf16(llmcp_q8_ctx *ctx, const llmcp_memref_bf16_2d *hidden,
                          const llmcp_memref_i8_1d *table,
                          llmcp_memref_f32_2d *logits, int64_t *argmax_dev,
                          int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
    Rows in, out;
    if (!view_of(hidden, true, in) || !view_of(logits, false, out))
      return fail(LLMCP_Q8_DECLINED, kDenseMsg);
    return lm_head_impl(ctx, in, table, out, argmax_dev, execution_mode);
  });
}

// llmcp_q8_lm_head with the device's fixed scratch in place of the
// context's workspace: no allocation on any path (sizes beyond the scratch
// are declined), so it may run under graph capture or where hipMalloc is
// forbidden.
int llmcp_q8_lm_head_noalloc(llmcp_q8_ctx *ctx,
                             const llmcp_memref_f32_2d *hidden,
                             const llmcp_memref_i8_1d *table,
                             llmcp_memref_f32_2d *logits, int64_t *argmax_dev,
                             int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
    Rows in, out;
    if (!view_of(hidden, false, in) || !view_of(logits, false, out))
      return fail(LLMCP_Q8_DECLINED, kDenseMsg);
    if (ctx->device >= kMaxDevices || !g_scratch_ptr[ctx->device])
      return fail(LLMCP_Q8_EINVAL, "no fixed scratch on device %d", ctx->device);
    {
      std::lock_guard<std::mutex> lock(g_scratch_mutex);
      llmcp_q8_ctx *&owner = g_scratch_owner[ctx->device];
      if (!owner) owner = ctx;
      if (owner != ctx)
        return fail(LLMCP_Q8_DECLINED,
                    "the fixed scratch of device %d is in use by another context "
                    "(one context per GPU may call the no-allocation entry)",
                    ctx->device);
    }
    const Workspace ws = static_workspace(ctx->device);
    return lm_head_impl(ctx, in, table, out, argmax_dev, execution_mode, &ws);
  });
}

int llmcp_q8_mlp(llmcp_q8_ctx *ctx, const llmcp_memref_f32_2d *input,
                 const llmcp_memref_i8_1d *w_gate,
                 const llmcp_memref_i8_1d *w_up,
                 const llmcp_memref_i8_1d *w_down, llmcp_memref_f32_2d *hidden,
                 llmcp_memref_f32_2d *output, int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
    Rows in, out, h;
    if (!view_of(input, false, in) || !view_of(output, false, out) ||
        (hidden && !view_of(hidden, false, h)))
      return fail(LLMCP_Q8_DECLINED, kDenseMsg);
    return mlp_impl(ctx, in, w_gate, w_up, w_down, hidden ? &h : nullptr, out,
                    execution_mode);
  });
}

int llmcp_q8_mlp_bf16(llmcp_q8_ctx *ctx, const llmcp_memref_bf16_2d *input,
                      const llmcp_memref_i8_1d *w_gate,
                      const llmcp_memref_i8_1d *w_up,
                      const llmcp_memref_i8_1d *w_down,
                      llmcp_memref_bf16_2d *hidden,
                      llmcp_memref_bf16_2d *output, int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
    Rows in, out, h;
    if (!view_of(input, true, in) || !view_of(output, true, out) ||
        (hidden && !view_of(hidden, true, h)))
      return fail(LLMCP_Q8_DECLINED, kDenseMsg);
    return mlp_impl(ctx, in, w_gate, w_up, w_down, hidden ? &h : nullptr, out,
                    execution_mode);
  });
}

int llmcp_q8_embedding(llmcp_q8_ctx *ctx, const llmcp_memref_i64_1d *tokens,
                       const llmcp_memref_i8_1d *table,
                       llmcp_memref_f32_2d *output) {
  return guarded([&]() -> int {
    if (!ctx || !tokens || !output) return fail(LLMCP_Q8_EINVAL, "null argument");
    Rows out;
    if (!view_of(output, false, out))
      return fail(LLMCP_Q8_DECLINED, "embedding output must be [tokens, hidden]");
    return embedding_impl(ctx, tokens, table, out);
  });
}

int llmcp_q8_embedding_bf16(llmcp_q8_ctx *ctx,
                            const llmcp_memref_i64_1d *tokens,
                            const llmcp_memref_i8_1d *table,
                            llmcp_memref_bf16_2d *output) {
  return guarded([&]() -> int {
    if (!ctx || !tokens || !output) return fail(LLMCP_Q8_EINVAL, "null argument");
    Rows out;
    if (!view_of(output, true, out))
      return fail(LLMCP_Q8_DECLINED, "embedding output must be [tokens, hidden]");
    return embedding_impl(ctx, tokens, table, out);
  });
}

int llmcp_q8_quantize_activations(llmcp_q8_ctx *ctx,
                                  const llmcp_memref_f32_2d *input,
                                  int8_t *qa_dev, float *sa_dev) {
  return guarded([&]() -> int {
    if (!ctx || !qa_dev || !sa_dev) return fail(LLMCP_Q8_EINVAL, "null argument");
    if (!dense_rows(input) || input->sizes[1] % kBlock)
      return fail(LLMCP_Q8_DECLINED, "input must be row-major with K %% 32 == 0");
    int rc = set_device(ctx);
    if (rc) return rc;
    const int64_t m = input->sizes[0], k = input->sizes[1];
    if (m == 0) return LLMCP_Q8_OK;
    // one thread per 4 values on a one-dimensional grid: HIP bounds its
    // work-items by 2^32 - 1
    if (m > (1ll << 40) || m * (k / 4) > 0xFFFFFF00ll)
      return fail(LLMCP_Q8_DECLINED, "too many rows for one launch (%lld)", (long long)m);
    hipError_t e = launch_quantize(input->data + input->offset, false, m,
                                   input->strides[0], k, qa_dev, k, sa_dev,
                                   k / kBlock, k / kBlock, ctx->stream);
    if (e != hipSuccess) return hip_fail(e, "quantize launch");
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_block_dots(llmcp_q8_ctx *ctx, const llmcp_memref_f32_2d *input,
                        const llmcp_memref_i8_1d *weight, int32_t *out_dev) {
  return guarded([&]() -> int {
    if (!ctx || !out_dev) return fail(LLMCP_Q8_EINVAL, "null argument");
    const Tensor *w = nullptr;
    int rc = resolve_weight(ctx, weight, &w);
    if (rc) return rc;
    if (!dense_rows(input) || input->sizes[1] != w->cols)
      return fail(LLMCP_Q8_DECLINED, "input must be row-major [M, K]");
    if ((rc = set_device(ctx))) return rc;
    const int64_t m = input->sizes[0], k = input->sizes[1], b = k / kBlock;
    if (m == 0) return LLMCP_Q8_OK;
    if (m > (1ll << 40) || m * (k / 4) > 0xFFFFFF00ll)
      return fail(LLMCP_Q8_DECLINED, "too many rows for one launch (%lld)", (long long)m);
    if ((rc = ensure_scratch(ctx, (uint64_t)(m * k), (uint64_t)(m * b * 4))))
      return rc;
    hipError_t e = launch_quantize(input->data + input->offset, false, m,
                                   input->strides[0], k, ctx->qa, k, ctx->sa, b,
                                   b, ctx->stream);
    if (e != hipSuccess) return hip_fail(e, "quantize launch");
    e = launch_block_dots(ctx->qa, k, m, w->dev, w->rows, w->cols, out_dev,
                          ctx->stream);
    if (e != hipSuccess) return hip_fail(e, "block dots launch");
    return LLMCP_Q8_OK;
  });
}

// ------------------------------------------------------ offline packing --

int llmcp_q8_pack_p4_host(const float *w, int64_t rows, int64_t cols,
                          uint8_t *out) {
  return guarded([&]() -> int {
    if (!w || !out) return fail(LLMCP_Q8_EINVAL, "null argument");
    if (!packable(rows, cols))
      return fail(LLMCP_Q8_DECLINED,
                  "packed Q8_0 requires rows %% 8 == 0 and cols %% 32 == 0");
    const int64_t blocks = cols / kBlock, groups = rows / kLanes;
  #pragma omp parallel for schedule(static)
    for (int64_t g = 0; g < groups; ++g) {
      for (int64_t b = 0; b < blocks; ++b) {
        uint8_t *rec = out + (g * blocks + b) * kRecord;
        for (int r = 0; r < kLanes; ++r) {
          const float *v = w + (g * kLanes + r) * cols + b * kBlock;
          float amax = 0.0f;
          for (int i = 0; i < kBlock; ++i) amax = std::max(amax, std::fabs(v[i]));
          uint16_t d = 0;
          int8_t q[kBlock] = {0};
          if (amax != 0.0f) {
            const float scale = amax / 127.0f;
            d = host_f32_to_f16(scale);
            for (int i = 0; i < kBlock; ++i) {
              long x = std::lround(v[i] / scale);
              q[i] = (int8_t)std::min(127L, std::max(-127L, x));
            }
          }
          rec[2 * r] = (uint8_t)(d & 0xff);
          rec[2 * r + 1] = (uint8_t)(d >> 8);
          for (int c = 0; c < 8; ++c)
            std::memcpy(rec + 8 + 16 * c + 4 * r, q + 4 * c, 4);
        }
      }
    }
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_synthesize_p4(llmcp_q8_ctx *ctx, uint64_t seed, int64_t rows,
                           int64_t cols, float stddev, float *w_dev,
                           void *p4_dev) {
  return guarded([&]() -> int {
    if (!ctx || !p4_dev) return fail(LLMCP_Q8_EINVAL, "null argument");
    if (!packable(rows, cols))
      return fail(LLMCP_Q8_DECLINED,
                  "packed Q8_0 requires rows %% 8 == 0 and cols %% 32 == 0");
    int rc = set_device(ctx);
    if (rc) return rc;
    float *w = w_dev;
    if (!w && hipMalloc(&w, (size_t)rows * (size_t)cols * 4) != hipSuccess)
      return fail(LLMCP_Q8_ENOMEM, "synthetic weight staging");
    hipError_t e = launch_synth(seed, rows, cols, stddev, w, ctx->stream);
    if (e == hipSuccess)
      e = launch_pack_p4(w, rows, cols, (uint8_t *)p4_dev, ctx->stream);
    if (!w_dev) {
      (void)hipStreamSynchronize(ctx->stream);
      (void)hipFree(w);
    }
    if (e != hipSuccess) return hip_fail(e, "synthesize");
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_write_arena(const char *path, int32_t count,
                         const char *const *names, const int64_t *rows,
                         const int64_t *cols, const void *const *p4) {
  return guarded([&]() -> int {
    if (!path || count <= 0 || !names || !rows || !cols || !p4)
      return fail(LLMCP_Q8_EINVAL, "bad arena writer arguments");
    std::vector<uint64_t> offsets(count), sizes(count);
    uint64_t cursor = 64;
    for (int32_t i = 0; i < count; ++i) {
      if (!names[i] || !names[i][0] || !packable(rows[i], cols[i]))
        return fail(LLMCP_Q8_EINVAL, "tensor %d: bad name or shape", i);
      cursor = (cursor + 63) / 64 * 64;
      offsets[i] = cursor;
      sizes[i] = (uint64_t)rows[i] * (uint64_t)(cols[i] / 32) * 34u;
      cursor += sizes[i];
    }
    const uint64_t arena = (cursor + 63) / 64 * 64;
    std::string m = "{\"model\":\"synthetic\",\"total_bytes\":" +
                    std::to_string(arena) +
                    ",\"header_bytes\":64,\"group_stride\":0,\"num_groups\":0,"
                    "\"alignment\":64,\"quantization\":\"q8_0\",\"block_size\":32,"
                    "\"quant_layout\":\"q8_0_p4\",\"tensors\":[";
    for (int32_t i = 0; i < count; ++i) {
      std::string name;
      for (const char *c = names[i]; *c; ++c) {
        if (*c == '"' || *c == '\\') name += '\\';
        name += *c;
      }
      m += (i ? "," : "");
      m += "{\"name\":\"" + name + "\",\"offset\":" + std::to_string(offsets[i]) +
           ",\"size\":" + std::to_string(sizes[i]) +
           ",\"dtype\":\"Q8_0\",\"source_size\":" +
           std::to_string((uint64_t)rows[i] * (uint64_t)cols[i] * 4u) +
           ",\"shape\":[" + std::to_string(rows[i]) + "," +
           std::to_string(cols[i]) + "]}";
    }
    m += "]}\n";
    FILE *fp = std::fopen(path, "wb");
    if (!fp) return fail(LLMCP_Q8_EIO, "cannot open %s", path);
    std::vector<uint8_t> header(64, 0);
    bool ok = std::fwrite(header.data(), 1, 64, fp) == 64;
    uint64_t pos = 64;
    std::vector<uint8_t> zeros(64, 0);
    for (int32_t i = 0; i < count && ok; ++i) {
      while (ok && pos < offsets[i]) {
        const uint64_t n = std::min<uint64_t>(64, offsets[i] - pos);
        ok = std::fwrite(zeros.data(), 1, n, fp) == n;
        pos += n;
      }
      ok = ok && std::fwrite(p4[i], 1, sizes[i], fp) == sizes[i];
      pos += sizes[i];
    }
    while (ok && pos < arena) {
      const uint64_t n = std::min<uint64_t>(64, arena - pos);
      ok = std::fwrite(zeros.data(), 1, n, fp) == n;
      pos += n;
    }
    ok = ok && std::fwrite(m.data(), 1, m.size(), fp) == m.size();
    // Publish the header last (WeightPacker.cpp:269-272).
    std::memcpy(header.data(), "LLMCPWGT", 8);
    wr32(header.data() + 8, 1);
    wr32(header.data() + 12, 64);
    wr64(header.data() + 16, arena);
    wr64(header.data() + 24, arena);
    wr64(header.data() + 32, m.size());
    ok = ok && std::fflush(fp) == 0 && std::fseek(fp, 0, SEEK_SET) == 0 &&
         std::fwrite(header.data(), 1, 64, fp) == 64;
    ok = (std::fclose(fp) == 0) && ok;
    if (!ok) return fail(LLMCP_Q8_EIO, "short write to %s", path);
    return LLMCP_Q8_OK;
  });
}

// ---------------------------------------------------- MLIR C interface --

int32_t _mlir_ciface_llmcp_q8_linear(llmcp_memref_f32_2d *input,
                                     llmcp_memref_i8_1d *weight,
                                     llmcp_memref_f32_2d *output,
                                     int32_t activation,
                                     int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!g_default_ctx) return fail(LLMCP_Q8_EINVAL, "no default context");
    return llmcp_q8_linear(g_default_ctx, input, weight, output, activation,
                           execution_mode);
  });
}

int32_t _mlir_ciface_llmcp_q8_linear_add(llmcp_memref_f32_2d *input,
                                         llmcp_memref_i8_1d *weight,
                                         llmcp_memref_f32_2d *residual,
                                         llmcp_memref_f32_2d *output,
                                         int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!g_default_ctx) return fail(LLMCP_Q8_EINVAL, "no default context");
    return llmcp_q8_linear_add(g_default_ctx, input, weight, residual, output,
                               execution_mode);
  });
}

int32_t _mlir_ciface_llmcp_q8_linear_add_bf16(llmcp_memref_bf16_2d *input,
                                              llmcp_memref_i8_1d *weight,
                                              llmcp_memref_bf16_2d *residual,
                                              llmcp_memref_bf16_2d *output,
                                              int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!g_default_ctx) return fail(LLMCP_Q8_EINVAL, "no default context");
    return llmcp_q8_linear_add_bf16(g_default_ctx, input, weight, residual,
                                    output, execution_mode);
  });
}

// The model's two shared-input patterns as fixed-arity C-interface entries
// (a lowered func.call passes each memref by descriptor): three linears
// (q/k/v) and four (in_proj_qkv/z/a/b).
int32_t _mlir_ciface_llmcp_q8_linear_group3(
    llmcp_memref_f32_2d *input, llmcp_memref_i8_1d *w0, llmcp_memref_i8_1d *w1,
    llmcp_memref_i8_1d *w2, llmcp_memref_f32_2d *y0, llmcp_memref_f32_2d *y1,
    llmcp_memref_f32_2d *y2, int32_t act0, int32_t act1, int32_t act2,
    int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!g_default_ctx) return fail(LLMCP_Q8_EINVAL, "no default context");
    const llmcp_memref_i8_1d *w[3] = {w0, w1, w2};
    llmcp_memref_f32_2d *y[3] = {y0, y1, y2};
    const int32_t a[3] = {act0, act1, act2};
    return llmcp_q8_linear_group(g_default_ctx, input, 3, w, y, a, execution_mode);
  });
}

int32_t _mlir_ciface_llmcp_q8_linear_group4(
    llmcp_memref_f32_2d *input, llmcp_memref_i8_1d *w0, llmcp_memref_i8_1d *w1,
    llmcp_memref_i8_1d *w2, llmcp_memref_i8_1d *w3, llmcp_memref_f32_2d *y0,
    llmcp_memref_f32_2d *y1, llmcp_memref_f32_2d *y2, llmcp_memref_f32_2d *y3,
    int32_t act0, int32_t act1, int32_t act2, int32_t act3,
    int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!g_default_ctx) return fail(LLMCP_Q8_EINVAL, "no default context");
    const llmcp_memref_i8_1d *w[4] = {w0, w1, w2, w3};
    llmcp_memref_f32_2d *y[4] = {y0, y1, y2, y3};
    const int32_t a[4] = {act0, act1, act2, act3};
    return llmcp_q8_linear_group(g_default_ctx, input, 4, w, y, a, execution_mode);
  });
}

int32_t _mlir_ciface_llmcp_q8_linear_group3_bf16(
    llmcp_memref_bf16_2d *input, llmcp_memref_i8_1d *w0, llmcp_memref_i8_1d *w1,
    llmcp_memref_i8_1d *w2, llmcp_memref_bf16_2d *y0, llmcp_memref_bf16_2d *y1,
    llmcp_memref_bf16_2d *y2, int32_t act0, int32_t act1, int32_t act2,
    int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!g_default_ctx) return fail(LLMCP_Q8_EINVAL, "no default context");
    const llmcp_memref_i8_1d *w[3] = {w0, w1, w2};
    llmcp_memref_bf16_2d *y[3] = {y0, y1, y2};
    const int32_t a[3] = {act0, act1, act2};
    return llmcp_q8_linear_group_bf16(g_default_ctx, input, 3, w, y, a, execution_mode);
  });
}

int32_t _mlir_ciface_llmcp_q8_linear_group4_bf16(
    llmcp_memref_bf16_2d *input, llmcp_memref_i8_1d *w0, llmcp_memref_i8_1d *w1,
    llmcp_memref_i8_1d *w2, llmcp_memref_i8_1d *w3, llmcp_memref_bf16_2d *y0,
    llmcp_memref_bf16_2d *y1, llmcp_memref_bf16_2d *y2, llmcp_memref_bf16_2d *y3,
    int32_t act0, int32_t act1, int32_t act2, int32_t act3,
    int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!g_default_ctx) return fail(LLMCP_Q8_EINVAL, "no default context");
    const llmcp_memref_i8_1d *w[4] = {w0, w1, w2, w3};
    llmcp_memref_bf16_2d *y[4] = {y0, y1, y2, y3};
    const int32_t a[4] = {act0, act1, act2, act3};
    return llmcp_q8_linear_group_bf16(g_default_ctx, input, 4, w, y, a, execution_mode);
  });
}

int32_t _mlir_ciface_llmcp_q8_rmsnorm(llmcp_memref_f32_2d *input, llmcp_memref_f32_1d *weight,
                                      float eps, int32_t zero_centered,
                                      llmcp_memref_f32_2d *output) {
  return guarded([&]() -> int {
    if (!g_default_ctx) return fail(LLMCP_Q8_EINVAL, "no default context");
    return llmcp_q8_rmsnorm(g_default_ctx, input, weight, eps, zero_centered, output);
  });
}

int32_t _mlir_ciface_llmcp_q8_rmsnorm_bf16(llmcp_memref_bf16_2d *input,
                                           llmcp_memref_bf16_1d *weight, float eps,
                                           int32_t zero_centered,
                                           llmcp_memref_bf16_2d *output) {
  return guarded([&]() -> int {
    if (!g_default_ctx) return fail(LLMCP_Q8_EINVAL, "no default context");
    return llmcp_q8_rmsnorm_bf16(g_default_ctx, input, weight, eps, zero_centered, output);
  });
}

int32_t _mlir_ciface_llmcp_q8_gated_rmsnorm(llmcp_memref_f32_2d *input,
                                            llmcp_memref_f32_2d *gate,
                                            llmcp_memref_f32_1d *weight, int64_t group_size,
                                            float eps, int32_t gate_activated,
                                            llmcp_memref_f32_2d *output) {
  return guarded([&]() -> int {
    if (!g_default_ctx) return fail(LLMCP_Q8_EINVAL, "no default context");
    return llmcp_q8_gated_rmsnorm(g_default_ctx, input, gate, weight, group_size, eps,
                                  gate_activated, output);
  });
}

int32_t _mlir_ciface_llmcp_q8_gated_rmsnorm_bf16(llmcp_memref_bf16_2d *input,
                                                 llmcp_memref_bf16_2d *gate,
                                                 llmcp_memref_f32_1d *weight,
                                                 int64_t group_size, float eps,
                                                 int32_t gate_activated,
                                                 llmcp_memref_bf16_2d *output) {
  return guarded([&]() -> int {
    if (!g_default_ctx) return fail(LLMCP_Q8_EINVAL, "no default context");
    return llmcp_q8_gated_rmsnorm_bf16(g_default_ctx, input, gate, weight, group_size, eps,
                                       gate_activated, output);
  });
}

int32_t _mlir_ciface_llmcp_q8_rmsnorm_linear_group3_bf16(
    llmcp_memref_bf16_2d *input, llmcp_memref_bf16_1d *norm_weight, float eps,
    int32_t zero_centered, llmcp_memref_bf16_2d *normed, llmcp_memref_i8_1d *w0,
    llmcp_memref_i8_1d *w1, llmcp_memref_i8_1d *w2, llmcp_memref_bf16_2d *y0,
    llmcp_memref_bf16_2d *y1, llmcp_memref_bf16_2d *y2, int32_t act0, int32_t act1,
    int32_t act2, int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!g_default_ctx) return fail(LLMCP_Q8_EINVAL, "no default context");
    const llmcp_memref_i8_1d *w[3] = {w0, w1, w2};
    llmcp_memref_bf16_2d *y[3] = {y0, y1, y2};
    const int32_t a[3] = {act0, act1, act2};
    return llmcp_q8_rmsnorm_linear_group_bf16(g_default_ctx, input, norm_weight, eps,
                                              zero_centered, normed, 3, w, y, a,
                                              execution_mode);
  });
}

int32_t _mlir_ciface_llmcp_q8_rmsnorm_linear_group4_bf16(
    llmcp_memref_bf16_2d *input, llmcp_memref_bf16_1d *norm_weight, float eps,
    int32_t zero_centered, llmcp_memref_bf16_2d *normed, llmcp_memref_i8_1d *w0,
    llmcp_memref_i8_1d *w1, llmcp_memref_i8_1d *w2, llmcp_memref_i8_1d *w3,
    llmcp_memref_bf16_2d *y0, llmcp_memref_bf16_2d *y1, llmcp_memref_bf16_2d *y2,
    llmcp_memref_bf16_2d *y3, int32_t act0, int32_t act1, int32_t act2, int32_t act3,
    int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!g_default_ctx) return fail(LLMCP_Q8_EINVAL, "no default context");
    const llmcp_memref_i8_1d *w[4] = {w0, w1, w2, w3};
    llmcp_memref_bf16_2d *y[4] = {y0, y1, y2, y3};
    const int32_t a[4] = {act0, act1, act2, act3};
    return llmcp_q8_rmsnorm_linear_group_bf16(g_default_ctx, input, norm_weight, eps,
                                              zero_centered, normed, 4, w, y, a,
                                              execution_mode);
  });
}

int32_t _mlir_ciface_llmcp_q8_swiglu(llmcp_memref_f32_2d *input,
                                     llmcp_memref_i8_1d *w_gate,
                                     llmcp_memref_i8_1d *w_up,
                                     llmcp_memref_f32_2d *output,
                                     int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!g_default_ctx) return fail(LLMCP_Q8_EINVAL, "no default context");
    return llmcp_q8_swiglu(g_default_ctx, input, w_gate, w_up, output,
                           execution_mode);
  });
}

int32_t _mlir_ciface_llmcp_q8_lm_head(llmcp_memref_f32_2d *hidden,
                                      llmcp_memref_i8_1d *table,
                                      llmcp_memref_f32_2d *logits,
                                      llmcp_memref_i64_1d *argmax,
                                      int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!g_default_ctx) return fail(LLMCP_Q8_EINVAL, "no default context");
    int64_t *am = argmax ? argmax->data + argmax->offset : nullptr;
    return llmcp_q8_lm_head(g_default_ctx, hidden, table, logits, am,
                            execution_mode);
  });
}

int32_t _mlir_ciface_llmcp_q8_embedding(llmcp_memref_i64_1d *tokens,
                                        llmcp_memref_i8_1d *table,
                                        llmcp_memref_f32_2d *output) {
  return guarded([&]() -> int {
    if (!g_default_ctx) return fail(LLMCP_Q8_EINVAL, "no default context");
    return llmcp_q8_embedding(g_default_ctx, tokens, table, output);
  });
}

int32_t _mlir_ciface_llmcp_q8_linear_bf16(llmcp_memref_bf16_2d *input,
                                          llmcp_memref_i8_1d *weight,
                                          llmcp_memref_bf16_2d *output,
                                          int32_t activation,
                                          int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!g_default_ctx) return fail(LLMCP_Q8_EINVAL, "no default context");
    return llmcp_q8_linear_bf16(g_default_ctx, input, weight, output, activation,
                                execution_mode);
  });
}

int32_t _mlir_ciface_llmcp_q8_swiglu_bf16(llmcp_memref_bf16_2d *input,
                                          llmcp_memref_i8_1d *w_gate,
                                          llmcp_memref_i8_1d *w_up,
                                          llmcp_memref_bf16_2d *output,
                                          int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!g_default_ctx) return fail(LLMCP_Q8_EINVAL, "no default context");
    return llmcp_q8_swiglu_bf16(g_default_ctx, input, w_gate, w_up, output,
                                execution_mode);
  });
}

int32_t _mlir_ciface_llmcp_q8_lm_head_bf16(llmcp_memref_bf16_2d *hidden,
                                           llmcp_memref_i8_1d *table,
                                           llmcp_memref_f32_2d *logits,
                                           llmcp_memref_i64_1d *argmax,
                                           int32_t execution_mode) {
  return guarded([&]() -> int {
    if (!g_default_ctx) return fail(LLMCP_Q8_EINVAL, "no default context");
    int64_t *am = argmax ? argmax->data + argmax->offset : nullptr;
    return llmcp_q8_lm_head_bf16(g_default_ctx, hidden, table, logits, am,
                                 execution_mode);
  });
}

int32_t _mlir_ciface_llmcp_q8_embedding_bf16(llmcp_memref_i64_1d *tokens,
                                             llmcp_memref_i8_1d *table,
                                             llmcp_memref_bf16_2d *output) {
  return guarded([&]() -> int {
    if (!g_default_ctx) return fail(LLMCP_Q8_EINVAL, "no default context");
    return llmcp_q8_embedding_bf16(g_default_ctx, tokens, table, output);
  });
}

// --------------------------------------------------- device plumbing --

int llmcp_q8_dev_alloc(llmcp_q8_ctx *ctx, uint64_t bytes, void **out) {
  return guarded([&]() -> int {
    if (!ctx || !out) return fail(LLMCP_Q8_EINVAL, "null argument");
    int rc = set_device(ctx);
    if (rc) return rc;
    if (hipMalloc(out, bytes ? bytes : 1) != hipSuccess)
      return fail(LLMCP_Q8_ENOMEM, "hipMalloc of %llu bytes",
                  (unsigned long long)bytes);
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_dev_free(llmcp_q8_ctx *ctx, void *ptr) {
  return guarded([&]() -> int {
    if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
    if (!ptr) return LLMCP_Q8_OK;
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    HIP_TRY(hipFree(ptr));
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_memcpy_h2d(llmcp_q8_ctx *ctx, void *dst, const void *src,
                        uint64_t bytes) {
  return guarded([&]() -> int {
    if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_memcpy_d2h(llmcp_q8_ctx *ctx, void *dst, const void *src,
                        uint64_t bytes) {
  return guarded([&]() -> int {
    if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_memcpy_d2d(llmcp_q8_ctx *ctx, void *dst, const void *src,
                        uint64_t bytes) {
  return guarded([&]() -> int {
    if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_event_create(void **event) {
  return guarded([&]() -> int {
    if (!event) return fail(LLMCP_Q8_EINVAL, "null argument");
    hipEvent_t e;
    HIP_TRY(hipEventCreate(&e));
    *event = (void *)e;
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_event_destroy(void *event) {
  return guarded([&]() -> int {
    if (event) HIP_TRY(hipEventDestroy((hipEvent_t)event));
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_event_record(llmcp_q8_ctx *ctx, void *event) {
  return guarded([&]() -> int {
    if (!ctx || !event) return fail(LLMCP_Q8_EINVAL, "null argument");
    HIP_TRY(hipEventRecord((hipEvent_t)event, ctx->stream));
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_event_elapsed_ms(void *start, void *stop, float *ms) {
  return guarded([&]() -> int {
    if (!start || !stop || !ms) return fail(LLMCP_Q8_EINVAL, "null argument");
    HIP_TRY(hipEventSynchronize((hipEvent_t)stop));
    HIP_TRY(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
    return LLMCP_Q8_OK;
  });
}

// Compute units of the context's device.
static int ctx_cus(llmcp_q8_ctx *ctx) {
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, ctx->device) !=
          hipSuccess || n <= 0)
    n = 256;
  return n;
}

int llmcp_q8_microbench_bandwidth(llmcp_q8_ctx *ctx, int32_t kind, uint64_t bytes,
                                  int32_t launches, double *gb_per_s) {
  return guarded([&]() -> int {
    if (!ctx || !gb_per_s) return fail(LLMCP_Q8_EINVAL, "null argument");
    if (kind < 0 || kind > 2 || launches < 1)
      return fail(LLMCP_Q8_EINVAL, "bandwidth kind %d, %d launches", kind, launches);
    int rc = set_device(ctx);
    if (rc) return rc;
    const int cus = ctx_cus(ctx);
    const uint64_t unit = 64ull << 20;  // a multiple of cus * 256 KiB up to 256 CUs
    const uint64_t half = (kind == 2 ? bytes / 2 : bytes) / unit * unit;
    if (half == 0 || cus > 256)
      return fail(LLMCP_Q8_EINVAL, "bandwidth buffer of %llu bytes on %d CUs",
                  (unsigned long long)bytes, cus);
    void *a = nullptr, *b = nullptr;
    unsigned *sink = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    auto release = [&]() {
      // launches queued before a failure may still use the buffers
      (void)hipStreamSynchronize(ctx->stream);
      if (a) (void)hipFree(a);
      if (b) (void)hipFree(b);
      if (sink) (void)hipFree(sink);
      if (e0) (void)hipEventDestroy(e0);
      if (e1) (void)hipEventDestroy(e1);
    };
    if (hipMalloc(&a, half) != hipSuccess || (kind == 2 && hipMalloc(&b, half) != hipSuccess) ||
        hipMalloc((void **)&sink, 256) != hipSuccess) {
      release();
      return fail(LLMCP_Q8_ENOMEM, "bandwidth buffers of %llu bytes",
                  (unsigned long long)half);
    }
    hipError_t e = hipMemsetAsync(a, 1, half, ctx->stream);
    if (e == hipSuccess) e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    const void *src = a;
    void *dst = kind == 0 ? (void *)sink : kind == 1 ? a : b;
    if (e == hipSuccess) e = launch_stream(kind, src, dst, (int64_t)half, cus, ctx->stream);
    if (e == hipSuccess) e = hipEventRecord(e0, ctx->stream);
    for (int32_t i = 0; i < launches && e == hipSuccess; ++i)
      e = launch_stream(kind, src, dst, (int64_t)half, cus, ctx->stream);
    if (e == hipSuccess) e = hipEventRecord(e1, ctx->stream);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    float ms = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    release();
    if (e != hipSuccess) return hip_fail(e, "bandwidth microbenchmark");
    const double moved = (double)half * (kind == 2 ? 2.0 : 1.0) * launches;
    *gb_per_s = moved / (ms * 1e-3) / 1e9;
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_microbench_int8_mfma(llmcp_q8_ctx *ctx, int32_t iterations, double *tops) {
  return guarded([&]() -> int {
    if (!ctx || !tops) return fail(LLMCP_Q8_EINVAL, "null argument");
    if (iterations < 1) return fail(LLMCP_Q8_EINVAL, "%d iterations", iterations);
    int rc = set_device(ctx);
    if (rc) return rc;
    const int cus = ctx_cus(ctx);
    unsigned *sink = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (hipMalloc((void **)&sink, 256) != hipSuccess)
      return fail(LLMCP_Q8_ENOMEM, "microbenchmark sink");
    hipError_t e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    if (e == hipSuccess) e = launch_mfma_i8_peak(iterations / 8 + 1, cus, sink, ctx->stream);
    if (e == hipSuccess) e = hipEventRecord(e0, ctx->stream);
    if (e == hipSuccess) e = launch_mfma_i8_peak(iterations, cus, sink, ctx->stream);
    if (e == hipSuccess) e = hipEventRecord(e1, ctx->stream);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    float ms = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    (void)hipStreamSynchronize(ctx->stream);  // (after a failure: queued launches)
    (void)hipFree(sink);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (e != hipSuccess) return hip_fail(e, "int8 MFMA microbenchmark");
    *tops = mfma_i8_peak_ops(iterations, cus) / (ms * 1e-3) / 1e12;
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_microbench_epilogue(llmcp_q8_ctx *ctx, int32_t mode, int32_t blocks,
                                 double *tops) {
  return guarded([&]() -> int {
    if (!ctx || !tops) return fail(LLMCP_Q8_EINVAL, "null argument");
    if (mode < 0 || mode > 2 || blocks < 2)
      return fail(LLMCP_Q8_EINVAL, "epilogue mode %d, %d blocks", mode, blocks);
    int rc = set_device(ctx);
    if (rc) return rc;
    const int cus = ctx_cus(ctx);
    const int32_t pairs = blocks / 2;
    unsigned *sink = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (hipMalloc((void **)&sink, 256) != hipSuccess)
      return fail(LLMCP_Q8_ENOMEM, "microbenchmark sink");
    hipError_t e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    if (e == hipSuccess) e = launch_epilogue_mix(mode, pairs / 8 + 1, cus, sink, ctx->stream);
    if (e == hipSuccess) e = hipEventRecord(e0, ctx->stream);
    if (e == hipSuccess) e = launch_epilogue_mix(mode, pairs, cus, sink, ctx->stream);
    if (e == hipSuccess) e = hipEventRecord(e1, ctx->stream);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    float ms = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    (void)hipStreamSynchronize(ctx->stream);  // (after a failure: queued launches)
    (void)hipFree(sink);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (e != hipSuccess) return hip_fail(e, "epilogue microbenchmark");
    *tops = epilogue_mix_ops(pairs, cus) / (ms * 1e-3) / 1e12;
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_graph_begin(llmcp_q8_ctx *ctx) {
  return guarded([&]() -> int {
    if (!ctx) return fail(LLMCP_Q8_EINVAL, "null context");
    HIP_TRY(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_graph_end(llmcp_q8_ctx *ctx, void **graph_exec) {
  return guarded([&]() -> int {
    if (!ctx || !graph_exec) return fail(LLMCP_Q8_EINVAL, "null argument");
    hipGraph_t g = nullptr;
    HIP_TRY(hipStreamEndCapture(ctx->stream, &g));
    hipGraphExec_t ex = nullptr;
    hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
    try {
      std::lock_guard<std::mutex> lock(g_graph_mutex);
      g_graphs[(void *)ex] = {ctx, ctx->generation};
    } catch (...) {
      (void)hipGraphExecDestroy(ex);
      throw;
    }
    *graph_exec = (void *)ex;
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_graph_launch(llmcp_q8_ctx *ctx, void *graph_exec) {
  return guarded([&]() -> int {
    if (!ctx || !graph_exec) return fail(LLMCP_Q8_EINVAL, "null argument");
    {
      std::lock_guard<std::mutex> lock(g_graph_mutex);
      auto it = g_graphs.find(graph_exec);
      if (it == g_graphs.end() || it->second.ctx != ctx)
        return fail(LLMCP_Q8_EINVAL, "graph %p was not captured on this context",
                    graph_exec);
      // Its kernels hold the addresses of the workspace and weights as they
      // were at capture; replaying after one of them was freed would touch
      // freed memory.
      if (it->second.generation != ctx->generation)
        return fail(LLMCP_Q8_ESTALE,
                    "the workspace or a weight was reallocated after this "
                    "graph was captured; capture it again");
    }
    HIP_TRY(hipGraphLaunch((hipGraphExec_t)graph_exec, ctx->stream));
    return LLMCP_Q8_OK;
  });
}

int llmcp_q8_graph_destroy(void *graph_exec) {
  return guarded([&]() -> int {
    if (!graph_exec) return LLMCP_Q8_OK;
    {
      std::lock_guard<std::mutex> lock(g_graph_mutex);
      g_graphs.erase(graph_exec);
    }
    HIP_TRY(hipGraphExecDestroy((hipGraphExec_t)graph_exec));
    return LLMCP_Q8_OK;
  });
}

}  // extern "C"
