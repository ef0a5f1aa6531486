// A C++17 host of the C ABI, written the way llmcp's AOT runtime would use it:
// the library is linked like any C library, the
// weights come from a mapped single-file arena that llmcp_q8_upload_arena
// registers, and the MLIR C-interface entries are called with the runtime's
// own MemRef<T, N> descriptors (include/llmcp/Runtime/AotRuntime.h:52-58),
// the weight descriptor pointing into the mapping as memref.view does
// (ModelBuilder.cpp:170-172).
//
// The data is llmcp-matmul-benchmark's Q8 fixture
// (llmcp-matmul-benchmark.cpp:280-289): every record holds scales 0x2008 and
// q = 127, activations are 1.0, and the first output must equal K
// (:331-335), the check tests/CMakeLists.txt:162-165 runs at M = N = K = 64.
//
//   q8_consumer --cpu DIR   host-only part (packer, arena writer, inspect)
//   q8_consumer --gpu DIR   also the device calls on GPU 0
#include "llmcp_q8.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace {

template <class T, int N>
struct MemRef {  // the AOT runtime's descriptor
  T *base;
  T *data;
  int64_t offset;
  int64_t sizes[N];
  int64_t strides[N];
};
static_assert(sizeof(MemRef<float, 2>) == sizeof(llmcp_memref_f32_2d), "layout");
static_assert(sizeof(MemRef<int8_t, 1>) == sizeof(llmcp_memref_i8_1d), "layout");

int fail(const char *what) {
  std::fprintf(stderr, "FAIL %s: %s\n", what, llmcp_q8_last_error());
  return 1;
}

std::vector<uint8_t> fixture(int64_t n, int64_t k) {
  std::vector<uint8_t> rec(136);
  for (int l = 0; l < 4; ++l) {
    rec[2 * l] = 0x08;
    rec[2 * l + 1] = 0x20;
  }
  std::memset(rec.data() + 8, 127, 128);
  std::vector<uint8_t> p4;
  for (int64_t i = 0; i < n / 4 * (k / 32); ++i) p4.insert(p4.end(), rec.begin(), rec.end());
  return p4;
}

float bf16_to_f32(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

uint16_t f32_to_bf16(float f) {  // round to nearest even (finite values)
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// Offset of a tensor in the arena: the manifest (its file offset is the u64
// at byte 16 of the header) lists {"name":..., "offset":...}.
int64_t tensor_offset(const uint8_t *file, uint64_t size, const std::string &name) {
  uint64_t moff;
  std::memcpy(&moff, file + 16, 8);
  const std::string manifest((const char *)file + moff, size - moff);
  const size_t at = manifest.find("\"name\":\"" + name + "\"");
  if (at == std::string::npos) return -1;
  const size_t o = manifest.find("\"offset\":", at);
  return o == std::string::npos ? -1 : std::atoll(manifest.c_str() + o + 9);
}

}  // namespace

int main(int argc, char **argv) {
  const bool gpu = argc > 1 && std::strcmp(argv[1], "--gpu") == 0;
  const std::string dir = argc > 2 ? argv[2] : "/tmp";
  if (llmcp_q8_abi_version() != LLMCP_Q8_ABI_VERSION) return fail("abi version");

  // Host packer: rows of 1.0 pack to the fixture's records
  // (QuantizationTest.cpp:70-74: f16(1/127) == 0x2008, q = 127).
  std::vector<float> ones(8 * 64, 1.0f);
  std::vector<uint8_t> packed(8 * 64 / 32 * 34);
  if (llmcp_q8_pack_p4_host(ones.data(), 8, 64, packed.data())) return fail("pack");
  if (packed != fixture(8, 64)) return fail("packed bytes differ from the fixture");

  // Arena: the benchmark's 64x64 tensor and a decode-sized 256x2560 one.
  const int64_t rows[2] = {64, 256}, cols[2] = {64, 2560};
  const std::vector<uint8_t> t0 = fixture(rows[0], cols[0]), t1 = fixture(rows[1], cols[1]);
  const char *names[2] = {"bench.q8.weight", "decode.q8.weight"};
  const void *data[2] = {t0.data(), t1.data()};
  const std::string path = dir + "/q8_consumer_arena_" + std::to_string(getpid()) + ".bin";
  if (llmcp_q8_write_arena(path.c_str(), 2, names, rows, cols, data)) return fail("write arena");
  const int fd = open(path.c_str(), O_RDONLY);
  struct stat st;
  if (fd < 0 || fstat(fd, &st) != 0) return fail("open arena");
  const uint64_t fsize = (uint64_t)st.st_size;
  void *map = mmap(nullptr, fsize, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  unlink(path.c_str());
  if (map == MAP_FAILED) return fail("mmap arena");
  const uint8_t *file = (const uint8_t *)map;
  int64_t ntensors = 0, nq8 = 0;
  if (llmcp_q8_arena_inspect(file, fsize, &ntensors, &nq8) || ntensors != 2 || nq8 != 2)
    return fail("arena inspect");
  const int64_t off[2] = {tensor_offset(file, fsize, names[0]), tensor_offset(file, fsize, names[1])};
  if (off[0] < 64 || off[1] < 64) return fail("manifest offsets");
  if (!gpu) {
    munmap(map, fsize);
    std::puts("q8_consumer: host part ok");
    return 0;
  }

  // Device: the runtime's init (AotRuntime.cpp:39-66 + the three calls).
  llmcp_q8_ctx *ctx = nullptr;
  if (llmcp_q8_ctx_create(0, &ctx)) return fail("ctx create");
  int64_t uploaded = 0;
  if (llmcp_q8_upload_arena(ctx, file, fsize, &uploaded) || uploaded != 2) return fail("upload arena");
  if (llmcp_q8_set_default_ctx(ctx)) return fail("default ctx");

  int bad = 0;
  for (int t = 0; t < 2; ++t) {
    const int64_t n = rows[t], k = cols[t];
    MemRef<int8_t, 1> w{(int8_t *)(file + off[t]), (int8_t *)(file + off[t]), 0,
                        {n * (k + k / 16)}, {1}};
    for (const int64_t m : {(int64_t)1, (int64_t)64}) {
      const int32_t mode = m == 1 ? LLMCP_Q8_DECODE : LLMCP_Q8_PREFILL;
      void *xd = nullptr, *yd = nullptr, *rd = nullptr;
      if (llmcp_q8_dev_alloc(ctx, (uint64_t)(m * k * 4), &xd) ||
          llmcp_q8_dev_alloc(ctx, (uint64_t)(m * n * 4), &yd) ||
          llmcp_q8_dev_alloc(ctx, (uint64_t)(m * n * 4), &rd))
        return fail("alloc");
      // bf16: ones in, K out (the benchmark's own check)
      std::vector<uint16_t> xb(m * k, 0x3f80), yb(m * n, 0), rb(m * n, 0x3f80);
      llmcp_q8_memcpy_h2d(ctx, xd, xb.data(), xb.size() * 2);
      MemRef<uint16_t, 2> xm{(uint16_t *)xd, (uint16_t *)xd, 0, {m, k}, {k, 1}};
      MemRef<uint16_t, 2> ym{(uint16_t *)yd, (uint16_t *)yd, 0, {m, n}, {n, 1}};
      if (_mlir_ciface_llmcp_q8_linear_bf16((llmcp_memref_bf16_2d *)&xm, (llmcp_memref_i8_1d *)&w,
                                            (llmcp_memref_bf16_2d *)&ym, LLMCP_Q8_ACT_NONE, mode))
        return fail("linear_bf16");
      llmcp_q8_memcpy_d2h(ctx, yb.data(), yd, yb.size() * 2);
      const float first = bf16_to_f32(yb[0]);  // what the benchmark prints
      for (int64_t i = 0; i < m * n; ++i) bad += bf16_to_f32(yb[i]) != (float)k;
      // bf16 linear + residual of 1.0: K + 1
      llmcp_q8_memcpy_h2d(ctx, rd, rb.data(), rb.size() * 2);
      MemRef<uint16_t, 2> rm{(uint16_t *)rd, (uint16_t *)rd, 0, {m, n}, {n, 1}};
      if (_mlir_ciface_llmcp_q8_linear_add_bf16((llmcp_memref_bf16_2d *)&xm, (llmcp_memref_i8_1d *)&w,
                                                (llmcp_memref_bf16_2d *)&rm,
                                                (llmcp_memref_bf16_2d *)&ym, mode))
        return fail("linear_add_bf16");
      llmcp_q8_memcpy_d2h(ctx, yb.data(), yd, yb.size() * 2);
      for (int64_t i = 0; i < m * n; ++i)
        bad += yb[i] != f32_to_bf16((float)k + 1.0f);
      // f32: ones in; every output is the same sum of K/32 equal terms
      std::vector<float> xf(m * k, 1.0f), yf(m * n, 0.0f);
      llmcp_q8_memcpy_h2d(ctx, xd, xf.data(), xf.size() * 4);
      MemRef<float, 2> xm32{(float *)xd, (float *)xd, 0, {m, k}, {k, 1}};
      MemRef<float, 2> ym32{(float *)yd, (float *)yd, 0, {m, n}, {n, 1}};
      if (_mlir_ciface_llmcp_q8_linear((llmcp_memref_f32_2d *)&xm32, (llmcp_memref_i8_1d *)&w,
                                       (llmcp_memref_f32_2d *)&ym32, LLMCP_Q8_ACT_NONE, mode))
        return fail("linear");
      llmcp_q8_memcpy_d2h(ctx, yf.data(), yd, yf.size() * 4);
      for (int64_t i = 0; i < m * n; ++i)
        bad += yf[i] != yf[0] || bf16_to_f32(f32_to_bf16(yf[i])) != (float)k;
      llmcp_q8_dev_free(ctx, xd);
      llmcp_q8_dev_free(ctx, yd);
      llmcp_q8_dev_free(ctx, rd);
      std::printf("q8_consumer: %lld x %lld, M = %lld: first: %.4f (expected %lld), f32 %.6g\n",
                  (long long)n, (long long)k, (long long)m, (double)first, (long long)k,
                  (double)yf[0]);
    }
  }
  // One device-resident decode step through the C interface: the token id
  // lives in HBM, the embedding gathers its row of the 256 x 2560 table, the
  // tied lm_head scores every row and writes the first-maximum id back in
  // HBM (llmcp-benchmark.cpp:93-101 does the argmax on the host).  On the
  // fixture every row dequantizes to 127 * f16(0x2008) = 131064 / 131072
  // exactly, all logits are equal, and the first maximum is row 0.
  {
    const int64_t v = rows[1], hdim = cols[1];
    MemRef<int8_t, 1> table{(int8_t *)(file + off[1]), (int8_t *)(file + off[1]), 0,
                            {v * (hdim + hdim / 16)}, {1}};
    void *tok = nullptr, *hid = nullptr, *lg = nullptr, *am = nullptr;
    if (llmcp_q8_dev_alloc(ctx, 8, &tok) || llmcp_q8_dev_alloc(ctx, (uint64_t)hdim * 4, &hid) ||
        llmcp_q8_dev_alloc(ctx, (uint64_t)v * 4, &lg) || llmcp_q8_dev_alloc(ctx, 8, &am))
      return fail("alloc");
    const int64_t token = 5, sentinel = -1;
    llmcp_q8_memcpy_h2d(ctx, tok, &token, 8);
    llmcp_q8_memcpy_h2d(ctx, am, &sentinel, 8);
    MemRef<int64_t, 1> tm{(int64_t *)tok, (int64_t *)tok, 0, {1}, {1}};
    MemRef<float, 2> hm{(float *)hid, (float *)hid, 0, {1, hdim}, {hdim, 1}};
    MemRef<float, 2> lm{(float *)lg, (float *)lg, 0, {1, v}, {v, 1}};
    MemRef<int64_t, 1> amm{(int64_t *)am, (int64_t *)am, 0, {1}, {1}};
    if (_mlir_ciface_llmcp_q8_embedding((llmcp_memref_i64_1d *)&tm, (llmcp_memref_i8_1d *)&table,
                                        (llmcp_memref_f32_2d *)&hm))
      return fail("embedding");
    if (_mlir_ciface_llmcp_q8_lm_head((llmcp_memref_f32_2d *)&hm, (llmcp_memref_i8_1d *)&table,
                                      (llmcp_memref_f32_2d *)&lm, (llmcp_memref_i64_1d *)&amm,
                                      LLMCP_Q8_DECODE))
      return fail("lm_head");
    std::vector<float> hv(hdim), lv(v);
    int64_t best = -2;
    llmcp_q8_memcpy_d2h(ctx, hv.data(), hid, (uint64_t)hdim * 4);
    llmcp_q8_memcpy_d2h(ctx, lv.data(), lg, (uint64_t)v * 4);
    llmcp_q8_memcpy_d2h(ctx, &best, am, 8);
    const float row_value = 131064.0f / 131072.0f;
    for (int64_t i = 0; i < hdim; ++i) bad += hv[i] != row_value;
    for (int64_t i = 0; i < v; ++i) bad += lv[i] != lv[0];
    bad += best != 0;
    int32_t flag = -1;
    if (llmcp_q8_ctx_check(ctx, &flag) || flag != 0) return fail("device error flag");
    std::printf("q8_consumer: decode step: token %lld -> row value %.9g, logit %.6g, argmax %lld\n",
                (long long)token, (double)hv[0], (double)lv[0], (long long)best);
    for (void *p : {tok, hid, lg, am}) llmcp_q8_dev_free(ctx, p);
  }
  // The norms in front of the linears, on rows with closed-form results: a
  // row of 2.0 has the serial sum 4 H exactly, so rstd = 1 / sqrt(4) = 0.5
  // (eps 0) and y = (2 * 0.5) * (w + 1) = 1.5 for a zero-centered w of 0.5;
  // the gated norm of groups of 128 twos with an activated gate of 1.0 and a
  // weight of 1.0 gives 1.0.  The fused norm + group on the decode weight
  // must equal a plain linear of the normed row.
  {
    const int64_t hdim = cols[1], n = rows[1];
    MemRef<int8_t, 1> w{(int8_t *)(file + off[1]), (int8_t *)(file + off[1]), 0,
                        {n * (hdim + hdim / 16)}, {1}};
    void *xd = nullptr, *wd = nullptr, *yd = nullptr, *gd = nullptr, *gw = nullptr,
         *o1 = nullptr, *o2 = nullptr;
    if (llmcp_q8_dev_alloc(ctx, (uint64_t)hdim * 2, &xd) ||
        llmcp_q8_dev_alloc(ctx, (uint64_t)hdim * 2, &wd) ||
        llmcp_q8_dev_alloc(ctx, (uint64_t)hdim * 2, &yd) ||
        llmcp_q8_dev_alloc(ctx, (uint64_t)hdim * 2, &gd) ||
        llmcp_q8_dev_alloc(ctx, 128 * 4, &gw) ||
        llmcp_q8_dev_alloc(ctx, (uint64_t)n * 2, &o1) ||
        llmcp_q8_dev_alloc(ctx, (uint64_t)n * 2, &o2))
      return fail("alloc");
    const std::vector<uint16_t> xb(hdim, f32_to_bf16(2.0f)), wb(hdim, f32_to_bf16(0.5f)),
        ones(hdim, f32_to_bf16(1.0f));
    const std::vector<float> gwf(128, 1.0f);
    llmcp_q8_memcpy_h2d(ctx, xd, xb.data(), (uint64_t)hdim * 2);
    llmcp_q8_memcpy_h2d(ctx, wd, wb.data(), (uint64_t)hdim * 2);
    llmcp_q8_memcpy_h2d(ctx, gd, ones.data(), (uint64_t)hdim * 2);
    llmcp_q8_memcpy_h2d(ctx, gw, gwf.data(), 128 * 4);
    MemRef<uint16_t, 2> xm{(uint16_t *)xd, (uint16_t *)xd, 0, {1, hdim}, {hdim, 1}};
    MemRef<uint16_t, 2> ym{(uint16_t *)yd, (uint16_t *)yd, 0, {1, hdim}, {hdim, 1}};
    MemRef<uint16_t, 2> gm{(uint16_t *)gd, (uint16_t *)gd, 0, {1, hdim}, {hdim, 1}};
    MemRef<uint16_t, 1> wm{(uint16_t *)wd, (uint16_t *)wd, 0, {hdim}, {1}};
    MemRef<float, 1> gwm{(float *)gw, (float *)gw, 0, {128}, {1}};
    std::vector<uint16_t> yb(hdim);
    if (llmcp_q8_rmsnorm_bf16(ctx, (llmcp_memref_bf16_2d *)&xm, (llmcp_memref_bf16_1d *)&wm, 0.0f,
                              1, (llmcp_memref_bf16_2d *)&ym))
      return fail("rmsnorm_bf16");
    llmcp_q8_memcpy_d2h(ctx, yb.data(), yd, (uint64_t)hdim * 2);
    for (int64_t i = 0; i < hdim; ++i) bad += yb[i] != f32_to_bf16(1.5f);
    if (llmcp_q8_gated_rmsnorm_bf16(ctx, (llmcp_memref_bf16_2d *)&xm, (llmcp_memref_bf16_2d *)&gm,
                                    (llmcp_memref_f32_1d *)&gwm, 128, 0.0f, 1,
                                    (llmcp_memref_bf16_2d *)&ym))
      return fail("gated_rmsnorm_bf16");
    llmcp_q8_memcpy_d2h(ctx, yb.data(), yd, (uint64_t)hdim * 2);
    for (int64_t i = 0; i < hdim; ++i) bad += yb[i] != f32_to_bf16(1.0f);
    MemRef<uint16_t, 2> om1{(uint16_t *)o1, (uint16_t *)o1, 0, {1, n}, {n, 1}};
    MemRef<uint16_t, 2> om2{(uint16_t *)o2, (uint16_t *)o2, 0, {1, n}, {n, 1}};
    const llmcp_memref_i8_1d *ws[1] = {(const llmcp_memref_i8_1d *)&w};
    llmcp_memref_bf16_2d *os[1] = {(llmcp_memref_bf16_2d *)&om1};
    const int32_t acts[1] = {LLMCP_Q8_ACT_NONE};
    if (llmcp_q8_rmsnorm_linear_group_bf16(ctx, (llmcp_memref_bf16_2d *)&xm,
                                           (llmcp_memref_bf16_1d *)&wm, 0.0f, 1,
                                           (llmcp_memref_bf16_2d *)&ym, 1, ws, os, acts,
                                           LLMCP_Q8_DECODE))
      return fail("rmsnorm_linear_group_bf16");
    if (_mlir_ciface_llmcp_q8_linear_bf16((llmcp_memref_bf16_2d *)&ym, (llmcp_memref_i8_1d *)&w,
                                          (llmcp_memref_bf16_2d *)&om2, LLMCP_Q8_ACT_NONE,
                                          LLMCP_Q8_DECODE))
      return fail("linear_bf16 of the normed row");
    std::vector<uint16_t> r1(n), r2(n);
    llmcp_q8_memcpy_d2h(ctx, yb.data(), yd, (uint64_t)hdim * 2);
    llmcp_q8_memcpy_d2h(ctx, r1.data(), o1, (uint64_t)n * 2);
    llmcp_q8_memcpy_d2h(ctx, r2.data(), o2, (uint64_t)n * 2);
    for (int64_t i = 0; i < hdim; ++i) bad += yb[i] != f32_to_bf16(1.5f);
    for (int64_t i = 0; i < n; ++i) bad += r1[i] != r2[i];
    std::printf("q8_consumer: norms: rmsnorm %.4g, gated 1, group output %.6g\n",
                (double)bf16_to_f32(f32_to_bf16(1.5f)), (double)bf16_to_f32(r1[0]));
    for (void *q : {xd, wd, yd, gd, gw, o1, o2}) llmcp_q8_dev_free(ctx, q);
  }
  // ABI 7: the accumulation switch and the peak microbenchmarks.  In
  // SPLIT_K mode a 64-row linear of the 256 x 2560 weight (4 tiles) splits
  // K; every output is still the same sum of K/32 equal terms, and its
  // bf16 rounding is K.
  {
    const int64_t n = rows[1], k = cols[1], m = 64;
    MemRef<int8_t, 1> w{(int8_t *)(file + off[1]), (int8_t *)(file + off[1]), 0,
                        {n * (k + k / 16)}, {1}};
    if (llmcp_q8_set_accumulation(ctx, LLMCP_Q8_ACCUM_SPLIT_K) ||
        llmcp_q8_get_accumulation(ctx) != LLMCP_Q8_ACCUM_SPLIT_K)
      return fail("set_accumulation");
    void *xd = nullptr, *yd = nullptr;
    if (llmcp_q8_dev_alloc(ctx, (uint64_t)(m * k * 4), &xd) ||
        llmcp_q8_dev_alloc(ctx, (uint64_t)(m * n * 4), &yd))
      return fail("alloc");
    std::vector<float> xf(m * k, 1.0f), yf(m * n, 0.0f);
    llmcp_q8_memcpy_h2d(ctx, xd, xf.data(), xf.size() * 4);
    MemRef<float, 2> xm{(float *)xd, (float *)xd, 0, {m, k}, {k, 1}};
    MemRef<float, 2> ym{(float *)yd, (float *)yd, 0, {m, n}, {n, 1}};
    if (_mlir_ciface_llmcp_q8_linear((llmcp_memref_f32_2d *)&xm, (llmcp_memref_i8_1d *)&w,
                                     (llmcp_memref_f32_2d *)&ym, LLMCP_Q8_ACT_NONE,
                                     LLMCP_Q8_PREFILL))
      return fail("split-K linear");
    llmcp_q8_memcpy_d2h(ctx, yf.data(), yd, yf.size() * 4);
    for (int64_t i = 0; i < m * n; ++i)
      bad += yf[i] != yf[0] || bf16_to_f32(f32_to_bf16(yf[i])) != (float)k;
    if (llmcp_q8_set_accumulation(ctx, LLMCP_Q8_ACCUM_EXACT)) return fail("set_accumulation");
    llmcp_q8_dev_free(ctx, xd);
    llmcp_q8_dev_free(ctx, yd);
    double gbs = 0.0, tops = 0.0, ceiling = 0.0;
    if (llmcp_q8_microbench_bandwidth(ctx, 0, 64ull << 20, 2, &gbs) || !(gbs > 0.0))
      return fail("bandwidth microbenchmark");
    if (llmcp_q8_microbench_int8_mfma(ctx, 200, &tops) || !(tops > 0.0))
      return fail("int8 MFMA microbenchmark");
    if (llmcp_q8_microbench_epilogue(ctx, 0, 200, &ceiling) || !(ceiling > 0.0))
      return fail("epilogue microbenchmark");
    std::printf("q8_consumer: split-K linear %.6g; read %.0f GB/s (64 MiB), int8 MFMA %.0f TOPS, "
                "exact-epilogue ceiling %.0f TOPS (short runs)\n",
                (double)yf[0], gbs, tops, ceiling);
  }
  llmcp_q8_ctx_destroy(ctx);
  munmap(map, fsize);
  if (bad) {
    std::fprintf(stderr, "FAIL %d mismatching outputs\n", bad);
    return 1;
  }
  std::puts("q8_consumer: device part ok");
  return 0;
}
