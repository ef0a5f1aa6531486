/*
 * llmcp_q8.h -- C ABI of the MI355X (gfx950) Q8_0 quantized linear path.
 *
 * This library replaces the loop nests that llmcp's matmul lowering hook
 * emits for `weight_format = "q8_0_p4"`:
 *
 *   emitQ8PackedDecodeMatmul / emitQ8PackedMatmul / emitQ8PackedScalarMatmul
 *     include/llmcp/Dialect/LLMCP/Transforms/MatmulLoweringInternal.h:22-37
 *   dispatched by lowerMatmulInternal
 *     lib/Dialect/LLMCP/Transforms/MatmulLoweringCommon.cpp:492-508
 *
 * The hook would emit `func.call @llmcp_q8_*` with llvm.emit_c_interface, so
 * generated code calls the `_mlir_ciface_llmcp_q8_*` symbols below with
 * memref descriptors laid out as the runtime's MemRef<T,N>
 * (include/llmcp/Runtime/AotRuntime.h:52-58).  Everything is plain C: no
 * torch, no HIP types in signatures (streams travel as `void *`).
 *
 * Conventions
 *  - Every entry returns an int status (LLMCP_Q8_OK == 0).  The reference
 *    hook "declines" by returning a null Value (LowerToLinalg.cpp:161-166,
 *    :745-750); here that is LLMCP_Q8_DECLINED and the caller falls back.
 *    llmcp_q8_last_error() gives a thread-local message for the last failure.
 *    No C++ exception crosses this boundary.
 *  - Activation and output descriptors point to device memory (HBM).  Weight
 *    descriptors may point either into a host arena that was uploaded with
 *    llmcp_q8_upload_arena / llmcp_q8_upload_p4, or at a device p4 buffer
 *    registered with llmcp_q8_register_device_p4; the library translates the
 *    address to its device-resident copy (registry filled at upload).
 *  - Calls are asynchronous on the context's stream.  One host thread drives
 *    one context; calls on one context must not overlap (shared workspace).
 */
#ifndef LLMCP_Q8_H
#define LLMCP_Q8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Version of this C ABI (1: f32 entries; 2: bf16 twins and all four
 * activations; 3: linear + residual add; 4: reference platform switch,
 * weight budget, graph staleness check, grouped linears; 5: RMSNorm, gated
 * RMSNorm and RMSNorm + grouped linears; 6: their MLIR C-interface entries
 * and the bf16 group entries; 7: the accumulation switch).  The model ABI of
 * the AOT library (llmcp_model_abi_version() == 2,
 * include/llmcp/Support/AotAbi.h:12) is not changed by this library. */
#define LLMCP_Q8_ABI_VERSION 7

enum llmcp_q8_status {
  LLMCP_Q8_OK = 0,
  LLMCP_Q8_DECLINED = 1,  /* unsupported shape/format: caller falls back */
  LLMCP_Q8_EINVAL = 2,    /* bad argument (null, inconsistent sizes) */
  LLMCP_Q8_ENOTFOUND = 3, /* weight address not in any uploaded tensor */
  LLMCP_Q8_EHIP = 4,      /* HIP runtime error */
  LLMCP_Q8_EFORMAT = 5,   /* packed-weights header or manifest invalid */
  LLMCP_Q8_EIO = 6,       /* file open/map failure */
  LLMCP_Q8_ENOMEM = 7,    /* device (or host) allocation failed, or the
                             context's weight budget is exceeded */
  LLMCP_Q8_EINTERNAL = 8, /* unexpected internal failure */
  LLMCP_Q8_ESTALE = 9     /* graph captured before memory it uses was
                             reallocated: capture it again */
};

/* The activations llmcp.linear accepts (LLMCPOps.cpp:74-77), applied to the
 * f32 accumulator before the store (applyMatmulActivation,
 * MatmulLoweringCommon.cpp:78-103): silu v/(1+exp(-v)) as v*(1/(1+exp(-v))),
 * sigmoid 1/(1+exp(-v)), softplus math.log1p(exp(v)), which the reference's
 * --convert-math-to-llvm lowers to log(1 + exp(v)) with an f32 add
 * (llmcp-compile.cpp:186). */
enum llmcp_q8_activation {
  LLMCP_Q8_ACT_NONE = 0,
  LLMCP_Q8_ACT_SILU = 1,
  LLMCP_Q8_ACT_SIGMOID = 2,
  LLMCP_Q8_ACT_SOFTPLUS = 3
};

/* The reference platform whose arithmetic every op reproduces bit for bit.
 * The reference lowers q8_0_p4 per target (MatmulLoweringCommon.cpp:492-508):
 * AARCH64 (default)  the SDOT emitters, decode and prefill alike:
 *                    acc = fma(f32(I), sa*dw, acc) per block
 *                    (Q8Decode.cpp:192-203, Q8Matmul.cpp:204-223);
 * X86                the scalar fallback for every mode and M:
 *                    acc = acc + f32(I)*(sa*dw)  (Q8Scalar.cpp:192-199).
 * Blocks are summed in order b = 0..K/32-1 on both; each platform is within
 * the other's 1e-5 relative / 1e-4 absolute tolerance. */
enum llmcp_q8_platform {
  LLMCP_Q8_PLATFORM_X86 = 0,
  LLMCP_Q8_PLATFORM_AARCH64 = 1
};

/* How a context's multi-row linears sum their blocks.  No counterpart in
 * the reference, whose emitters always run one serial chain per output.
 * EXACT (default)  every f32 output is the selected platform's serial
 *                  block-order sum, bit for bit.
 * SPLIT_K          linears of several rows (the GEMM path: linear, linear +
 *                  add, grouped linears, SwiGLU, MLP, RMSNorm + group) whose
 *                  tiles leave CUs idle split K into ranges of whole
 *                  512-value passes, as many as keep one workgroup per CU
 *                  (and at most max(3, passes / 3); a second kernel then
 *                  adds the ranges' partial sums, so shapes that already
 *                  fill the GPU stay unsplit): each range is a serial
 *                  chain of the platform's epilogue, and the ranges' f32
 *                  partial sums are added in range order.  The per-block
 *                  int32 dots are still exact; f32 outputs agree with the
 *                  reference within 1e-5 relative or 1e-4 absolute (bf16
 *                  outputs within one bf16 step); the same inputs give the
 *                  same bits on every call.  One-row calls, the lm_head
 *                  (logits and argmax) and shapes that fill the GPU run as
 *                  in EXACT.  Needs workspace for the partial sums, grown on
 *                  first use like the prefill scratch. */
enum llmcp_q8_accumulation {
  LLMCP_Q8_ACCUM_EXACT = 0,
  LLMCP_Q8_ACCUM_SPLIT_K = 1
};

/* llmcp.execution_mode (LowerToLinalg.cpp:40-52). */
enum llmcp_q8_mode { LLMCP_Q8_PREFILL = 0, LLMCP_Q8_DECODE = 1 };

/* MemRef<T,N> of include/llmcp/Runtime/AotRuntime.h:52-58. */
typedef struct {
  float *base;
  float *data;
  int64_t offset;
  int64_t sizes[2];
  int64_t strides[2];
} llmcp_memref_f32_2d;

/* bf16 activations: the same descriptor with 16-bit elements (raw bf16
 * bits; the real model's hidden state is bf16, ModelBuilder.cpp:72). */
typedef struct {
  uint16_t *base;
  uint16_t *data;
  int64_t offset;
  int64_t sizes[2];
  int64_t strides[2];
} llmcp_memref_bf16_2d;

typedef struct {
  int8_t *base;
  int8_t *data;
  int64_t offset;
  int64_t sizes[1];
  int64_t strides[1];
} llmcp_memref_i8_1d;

typedef struct {
  int64_t *base;
  int64_t *data;
  int64_t offset;
  int64_t sizes[1];
  int64_t strides[1];
} llmcp_memref_i64_1d;

/* Norm weight vectors (memref<Hxf32> / memref<Hxbf16>, the arena's F32 and
 * BF16 tensors). */
typedef struct {
  float *base;
  float *data;
  int64_t offset;
  int64_t sizes[1];
  int64_t strides[1];
} llmcp_memref_f32_1d;

typedef struct {
  uint16_t *base;
  uint16_t *data;
  int64_t offset;
  int64_t sizes[1];
  int64_t strides[1];
} llmcp_memref_bf16_1d;

typedef struct llmcp_q8_ctx llmcp_q8_ctx;

/* ---------------------------------------------------------------- core -- */

int32_t llmcp_q8_abi_version(void);
const char *llmcp_q8_last_error(void);

/* Creates a context on HIP device `device` with its own non-blocking stream
 * (default priority).  Replaces the runtime's per-process state of
 * AotRuntime::init (lib/Runtime/AotRuntime.cpp:39-66). */
int llmcp_q8_ctx_create(int device, llmcp_q8_ctx **out);
int llmcp_q8_ctx_destroy(llmcp_q8_ctx *ctx);
/* Use a caller-owned hipStream_t (NULL restores the context's own stream). */
int llmcp_q8_ctx_set_stream(llmcp_q8_ctx *ctx, void *hip_stream);
void *llmcp_q8_ctx_stream(llmcp_q8_ctx *ctx);
int llmcp_q8_ctx_synchronize(llmcp_q8_ctx *ctx);
/* Selects the reference platform (llmcp_q8_platform) for every later call
 * on the context; llmcp_q8_get_platform returns it (-1 for a null ctx). */
int llmcp_q8_set_platform(llmcp_q8_ctx *ctx, int32_t platform);
int32_t llmcp_q8_get_platform(llmcp_q8_ctx *ctx);
/* Selects the accumulation mode (llmcp_q8_accumulation) for every later
 * call on the context; llmcp_q8_get_accumulation returns it (-1 for a null
 * ctx).  No counterpart in the reference. */
int llmcp_q8_set_accumulation(llmcp_q8_ctx *ctx, int32_t mode);
int32_t llmcp_q8_get_accumulation(llmcp_q8_ctx *ctx);
/* Caps the device bytes of the context's registered weights (0: no cap, the
 * default); a registration past the cap fails with LLMCP_Q8_ENOMEM.  Lets a
 * serving process keep HBM for other state. */
int llmcp_q8_set_weight_budget(llmcp_q8_ctx *ctx, uint64_t bytes);
/* Context used by the _mlir_ciface_* entries (set by the AOT runtime). */
int llmcp_q8_set_default_ctx(llmcp_q8_ctx *ctx);

/* ------------------------------------------------------------- weights -- */

/* Uploads one q8_0_p4 tensor [rows, cols] whose packed bytes live in host
 * memory (e.g. inside a mmapped arena) and repacks it once on the device.
 * Later weight descriptors whose data lies inside [host_p4, host_p4+bytes)
 * resolve to this copy.  Shape rule isQ8PackedShape
 * (include/llmcp/Support/Q8PackedLayout.h:38-42): rows % 8 == 0,
 * cols % 32 == 0.  `repack_ms` (nullable) receives the device repack time. */
int llmcp_q8_upload_p4(llmcp_q8_ctx *ctx, const void *host_p4, int64_t rows,
                       int64_t cols, float *repack_ms);

/* Same for a p4 tensor already in device memory (e.g. written by
 * llmcp_q8_synthesize_p4).  The device buffer is registered under its own
 * address and may be freed by the caller after this call returns. */
int llmcp_q8_register_device_p4(llmcp_q8_ctx *ctx, const void *dev_p4,
                                int64_t rows, int64_t cols, float *repack_ms);

/* Drops the device copy registered under `key` (host or device address). */
int llmcp_q8_release(llmcp_q8_ctx *ctx, const void *key);

/* Validates a mapped LLMCPWGT file (include/llmcp/Support/PackedWeights.h,
 * lib/Runtime/WeightArena.cpp:27-131 rules) and uploads every Q8_0 tensor.
 * `file` is the whole mapping, header first.  Returns the number of Q8_0
 * tensors uploaded through `num_q8` (nullable).  All or nothing: the
 * tensors are staged on the device and registered together only when every
 * one succeeded (Arena::load replaces the arena only on success,
 * WeightArena.cpp:28-29, :124-130); on failure nothing changes. */
int llmcp_q8_upload_arena(llmcp_q8_ctx *ctx, const void *file,
                          uint64_t file_bytes, int64_t *num_q8);

/* Host-only validation of a mapped LLMCPWGT file with the same rules; no
 * device is touched.  Counts all tensors and the Q8_0 ones (nullable). */
int llmcp_q8_arena_inspect(const void *file, uint64_t file_bytes,
                           int64_t *num_tensors, int64_t *num_q8);

/* ------------------------------------------------------------ ops ------- */

/* llmcp.linear with weight_format q8_0_p4 (LowerToLinalg.cpp:143-209):
 * y[M,N] = act(x[M,K] . W[N,K]^T), x quantized per call to Q8_1 blocks.
 * M == 1 runs the GEMV, M > 1 the int8-MFMA GEMM, in either mode (the
 * reference's decode emitter accepts any M, Q8Decode.cpp:236-256); both
 * compute the selected platform's epilogue.  activation:
 * llmcp_q8_activation. */
int llmcp_q8_linear(llmcp_q8_ctx *ctx, const llmcp_memref_f32_2d *input,
                    const llmcp_memref_i8_1d *weight,
                    llmcp_memref_f32_2d *output, int32_t activation,
                    int32_t execution_mode);

/* The same with bf16 input and output (the hook's tensor<MxK x bf16> ->
 * MxN bf16 case): x is widened exactly before Q8_1 quantization
 * (Q8Decode.cpp:97-98) and the activated f32 result is rounded to bf16
 * (arith.truncf, round to nearest even; Q8Decode.cpp:126-127). */
int llmcp_q8_linear_bf16(llmcp_q8_ctx *ctx, const llmcp_memref_bf16_2d *input,
                         const llmcp_memref_i8_1d *weight,
                         llmcp_memref_bf16_2d *output, int32_t activation,
                         int32_t execution_mode);

/* llmcp.linear followed by llmcp.add of a residual, the pair the model
 * builder emits after out_proj and after the MLP's down projection
 * (ModelBuilder.cpp:271, :275; AddOpLowering, LowerToLinalg.cpp:359-375):
 * y[M,N] = r[M,N] + x[M,K] . W[N,K]^T.  The linear's result is formed exactly
 * as llmcp_q8_linear forms it (no activation: the pattern has none), then one
 * f32 addition.  `residual` may be the same memory as `output` (in place);
 * it is a row-major [M, N] device buffer of the output's element type. */
int llmcp_q8_linear_add(llmcp_q8_ctx *ctx, const llmcp_memref_f32_2d *input,
                        const llmcp_memref_i8_1d *weight,
                        const llmcp_memref_f32_2d *residual,
                        llmcp_memref_f32_2d *output, int32_t execution_mode);

/* bf16 in, residual and out: the linear's result is rounded to bf16 first,
 * then the bf16 add as arith.addf on bf16 lowers it (both operands widened to
 * f32, added, rounded to bf16 to nearest even). */
int llmcp_q8_linear_add_bf16(llmcp_q8_ctx *ctx,
                             const llmcp_memref_bf16_2d *input,
                             const llmcp_memref_i8_1d *weight,
                             const llmcp_memref_bf16_2d *residual,
                             llmcp_memref_bf16_2d *output,
                             int32_t execution_mode);

/* Most linears one llmcp_q8_linear_group call takes. */
#define LLMCP_Q8_MAX_GROUP 8

/* Linears that share one input: y_i[M,N_i] = act_i(x[M,K] . W_i[N_i,K]^T)
 * for i < count (1 to LLMCP_Q8_MAX_GROUP), the pattern of the model
 * builder's in_proj_qkv/z/a/b (ModelBuilder.cpp:229-236) and q/k/v
 * (:288-294), which the reference lowers as separate llmcp.linear ops.  The
 * input is quantized once; for one row, one GEMV launch covers every
 * weight (when the row is 16 B aligned, f32 outputs or all bf16, and the
 * weights' rows total at most 16384), else each weight's GEMV follows.
 * Results equal count separate llmcp_q8_linear calls bit for bit.
 * activations (nullable: none) holds llmcp_q8_activation per linear. */
int llmcp_q8_linear_group(llmcp_q8_ctx *ctx, const llmcp_memref_f32_2d *input,
                          int32_t count,
                          const llmcp_memref_i8_1d *const *weights,
                          llmcp_memref_f32_2d *const *outputs,
                          const int32_t *activations, int32_t execution_mode);

/* bf16 input and outputs (as llmcp_q8_linear_bf16 per linear). */
int llmcp_q8_linear_group_bf16(llmcp_q8_ctx *ctx,
                               const llmcp_memref_bf16_2d *input, int32_t count,
                               const llmcp_memref_i8_1d *const *weights,
                               llmcp_memref_bf16_2d *const *outputs,
                               const int32_t *activations,
                               int32_t execution_mode);

/* llmcp.rms_norm over the rows of x [M, H] (H % 32 == 0) with weight w [H],
 * as the reference lowers it for decode rows (DecodeNormalization.cpp:71-154,
 * :160-171) and for prefill (LowerToLinalg.cpp:245-300), bit for bit: per
 * row, sum = sum + x*x in index order in f32, rstd = 1 / sqrt(sum / H + eps)
 * (math.rsqrt as --convert-math-to-llvm lowers it), y = (x * rstd) * w, with
 * w + 1 in place of w when zero_centered; a bf16 y is rounded to nearest
 * even.  eps is the op's f64 attribute as f32.  The serial sum costs about
 * one dependent add per element (rows run in parallel).  The weight must be
 * 16 B aligned (8 B for bf16); declines otherwise. */
int llmcp_q8_rmsnorm(llmcp_q8_ctx *ctx, const llmcp_memref_f32_2d *input,
                     const llmcp_memref_f32_1d *weight, float eps,
                     int32_t zero_centered, llmcp_memref_f32_2d *output);

/* bf16 rows and weight (the real model's hidden state and norm tensors). */
int llmcp_q8_rmsnorm_bf16(llmcp_q8_ctx *ctx, const llmcp_memref_bf16_2d *input,
                          const llmcp_memref_bf16_1d *weight, float eps,
                          int32_t zero_centered, llmcp_memref_bf16_2d *output);

/* llmcp.gated_rms_norm (the linear-attention output norm in front of
 * out_proj, ModelBuilder.cpp:259-266; DecodeNormalization.cpp:124-147 and
 * LowerToLinalg.cpp:574-720): each row of x [M, H] splits into groups of
 * group_size values (a multiple of 32 dividing H); per group the serial sum
 * and rstd of llmcp_q8_rmsnorm, then y = ((x * s) * w) * rstd with
 * s = g * (1 / (1 + exp(-g))) of the gate [M, H], or s = g when
 * gate_activated.  w [group_size] is f32 (the arena's F32 norm weight, 16 B
 * aligned).  Dense rows only. */
int llmcp_q8_gated_rmsnorm(llmcp_q8_ctx *ctx, const llmcp_memref_f32_2d *input,
                           const llmcp_memref_f32_2d *gate,
                           const llmcp_memref_f32_1d *weight, int64_t group_size,
                           float eps, int32_t gate_activated,
                           llmcp_memref_f32_2d *output);

/* bf16 input, gate and output (the real graph's types), f32 weight. */
int llmcp_q8_gated_rmsnorm_bf16(llmcp_q8_ctx *ctx, const llmcp_memref_bf16_2d *input,
                                const llmcp_memref_bf16_2d *gate,
                                const llmcp_memref_f32_1d *weight, int64_t group_size,
                                float eps, int32_t gate_activated,
                                llmcp_memref_bf16_2d *output);

/* The RMSNorm and the linears it feeds (input_layernorm -> in_proj_qkv/z/
 * a/b or q/k/v, post_attention_layernorm -> gate/up; ModelBuilder.cpp:
 * 225-236, :284-294): `normed` receives the norm's rows, then the group runs
 * on them as llmcp_q8_linear_group does.  For several rows the norm also
 * writes the rows' Q8_1 for the GEMMs (the activation quantization fused
 * into the norm's epilogue, no separate quantization); one row goes to the
 * grouped GEMV, which quantizes it inside each workgroup.  Results equal
 * llmcp_q8_rmsnorm followed by llmcp_q8_linear_group bit for bit. */
int llmcp_q8_rmsnorm_linear_group(llmcp_q8_ctx *ctx, const llmcp_memref_f32_2d *input,
                                  const llmcp_memref_f32_1d *norm_weight, float eps,
                                  int32_t zero_centered, llmcp_memref_f32_2d *normed,
                                  int32_t count, const llmcp_memref_i8_1d *const *weights,
                                  llmcp_memref_f32_2d *const *outputs,
                                  const int32_t *activations, int32_t execution_mode);

/* bf16 rows, norm weight, normed rows and outputs. */
int llmcp_q8_rmsnorm_linear_group_bf16(
    llmcp_q8_ctx *ctx, const llmcp_memref_bf16_2d *input,
    const llmcp_memref_bf16_1d *norm_weight, float eps, int32_t zero_centered,
    llmcp_memref_bf16_2d *normed, int32_t count, const llmcp_memref_i8_1d *const *weights,
    llmcp_memref_bf16_2d *const *outputs, const int32_t *activations,
    int32_t execution_mode);

/* Fused SwiGLU hidden: h = silu(x . Wg^T) * (x . Wu^T), the pair
 * `linear{activation=silu}` + `mul` that FuseSiluMul produces
 * (FuseLinearActivations.cpp:27-43, LowerToLinalg.cpp:377-393). */
int llmcp_q8_swiglu(llmcp_q8_ctx *ctx, const llmcp_memref_f32_2d *input,
                    const llmcp_memref_i8_1d *w_gate,
                    const llmcp_memref_i8_1d *w_up,
                    llmcp_memref_f32_2d *output, int32_t execution_mode);

/* bf16 in and out: both linears' results are rounded to bf16 before the
 * bf16 multiply, h = bf16(bf16(silu(g)) * bf16(u)), as the pair
 * linear{silu} + mul computes on bf16 tensors. */
int llmcp_q8_swiglu_bf16(llmcp_q8_ctx *ctx, const llmcp_memref_bf16_2d *input,
                         const llmcp_memref_i8_1d *w_gate,
                         const llmcp_memref_i8_1d *w_up,
                         llmcp_memref_bf16_2d *output, int32_t execution_mode);

/* MLP of one layer, ModelBuilder.cpp:205-216 with FuseSiluMul:
 * h = silu(x . Wg^T) * (x . Wu^T), y = h . Wd^T.  M == 1: two kernels, the
 * fused gate/up GEMV, then the down GEMV (which quantizes h once per
 * workgroup).  M > 1: the SwiGLU GEMMs, then the down GEMM.  `hidden`
 * (nullable) receives h.  Results equal llmcp_q8_swiglu followed by
 * llmcp_q8_linear in the same execution mode. */
int llmcp_q8_mlp(llmcp_q8_ctx *ctx, const llmcp_memref_f32_2d *input,
                 const llmcp_memref_i8_1d *w_gate,
                 const llmcp_memref_i8_1d *w_up,
                 const llmcp_memref_i8_1d *w_down, llmcp_memref_f32_2d *hidden,
                 llmcp_memref_f32_2d *output, int32_t execution_mode);

/* bf16 in, hidden and out (llmcp_q8_swiglu_bf16 then llmcp_q8_linear_bf16). */
int llmcp_q8_mlp_bf16(llmcp_q8_ctx *ctx, const llmcp_memref_bf16_2d *input,
                      const llmcp_memref_i8_1d *w_gate,
                      const llmcp_memref_i8_1d *w_up,
                      const llmcp_memref_i8_1d *w_down,
                      llmcp_memref_bf16_2d *hidden,
                      llmcp_memref_bf16_2d *output, int32_t execution_mode);

/* llmcp.lm_head (LowerToLinalg.cpp:729-765): f32 logits [M,V] over the tied
 * table, plus the first-maximum index of the last row written to
 * `argmax_dev` (device int64, nullable) -- the host std::max_element of
 * llmcp-benchmark.cpp:51-54 on the device: fused into the GEMV for M == 1;
 * for M > 1 the GEMM writes all rows (epilogue as for llmcp_q8_linear) and
 * a reduction reads the last one. */
int llmcp_q8_lm_head(llmcp_q8_ctx *ctx, const llmcp_memref_f32_2d *hidden,
                     const llmcp_memref_i8_1d *table,
                     llmcp_memref_f32_2d *logits, int64_t *argmax_dev,
                     int32_t execution_mode);

/* bf16 hidden state, f32 logits (the AOT ABI's logits are f32,
 * AotRuntime.cpp:87-118). */
int llmcp_q8_lm_head_bf16(llmcp_q8_ctx *ctx, const llmcp_memref_bf16_2d *hidden,
                          const llmcp_memref_i8_1d *table,
                          llmcp_memref_f32_2d *logits, int64_t *argmax_dev,
                          int32_t execution_mode);

/* Size of the per-GPU scratch array of llmcp_q8_lm_head_noalloc: 16 KiB of
 * argmax slots, the rest for the quantized hidden rows (at K = 2560 about
 * 2800 rows; M = 1 needs 2880 bytes). */
#define LLMCP_Q8_STATIC_SCRATCH_BYTES (8u << 20)

/* llmcp_q8_lm_head that allocates nothing.  It has no counterpart in the
 * reference: it is for callers that cannot allocate device memory -- code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  Results equal llmcp_q8_lm_head's.  Its scratch (the quantized
 * hidden rows and the argmax slots) is one file-scope device array of
 * LLMCP_Q8_STATIC_SCRATCH_BYTES that each GPU holds until the process ends,
 * set up when the first context on that GPU is created; a hidden state that
 * needs more returns LLMCP_Q8_DECLINED.  Every call on one GPU shares that
 * array, so one context per GPU may use it: the first context to call this
 * entry on a GPU owns the array until it is destroyed, and calls from any
 * other context on that GPU return LLMCP_Q8_DECLINED.  The owner's calls
 * are ordered on its stream (also across llmcp_q8_ctx_set_stream); calls
 * that overlap in other ways race. */
int llmcp_q8_lm_head_noalloc(llmcp_q8_ctx *ctx,
                             const llmcp_memref_f32_2d *hidden,
                             const llmcp_memref_i8_1d *table,
                             llmcp_memref_f32_2d *logits, int64_t *argmax_dev,
                             int32_t execution_mode);

/* llmcp.embedding with weight_format q8_0_p4 (emitQ8PackedEmbedding,
 * LowerToLinalg.cpp:435-531): out[t, c] = f32(q(token_t, c)) * f32(d).
 * Tokens outside [0, rows) produce a zero row and set the context's
 * error flag (llmcp_q8_ctx_check). */
int llmcp_q8_embedding(llmcp_q8_ctx *ctx, const llmcp_memref_i64_1d *tokens,
                       const llmcp_memref_i8_1d *table,
                       llmcp_memref_f32_2d *output);

/* bf16 result: the exact f32 product rounded to bf16 (the truncf the
 * lowering emits for a bf16 embedding). */
int llmcp_q8_embedding_bf16(llmcp_q8_ctx *ctx,
                            const llmcp_memref_i64_1d *tokens,
                            const llmcp_memref_i8_1d *table,
                            llmcp_memref_bf16_2d *output);

/* Activation quantizer Q8_1 (Q8Decode.cpp:83-120): qa_dev int8 [M,K] and
 * sa_dev f32 [M,K/32], both dense row-major device buffers. */
int llmcp_q8_quantize_activations(llmcp_q8_ctx *ctx,
                                  const llmcp_memref_f32_2d *input,
                                  int8_t *qa_dev, float *sa_dev);

/* Per-block int32 dot products I[m][n][b] (Q8Decode.cpp:166-191) of the
 * Q8_1-quantized input against the registered weight, into out_dev
 * (device int32 [M,N,K/32]).  Exposes the exact integer stage. */
int llmcp_q8_block_dots(llmcp_q8_ctx *ctx, const llmcp_memref_f32_2d *input,
                        const llmcp_memref_i8_1d *weight, int32_t *out_dev);

/* Reads and clears the device error flag (1 = an embedding token was out of
 * range since the last check).  Synchronizes the stream. */
int llmcp_q8_ctx_check(llmcp_q8_ctx *ctx, int32_t *flag);

/* Device self-test of the two floating-point identities the activation
 * quantizer uses in place of IEEE division (no counterpart in the
 * reference; it pins the quantizer's exactness on the running GPU):
 * RN(m/127) by reciprocal-multiply plus one FMA correction for every
 * non-negative float m, and RN(1/s) by v_rcp_f32 plus one Newton step for
 * every positive float s.  Writes the number of inputs where either differs
 * from IEEE division (0 expected).  Synchronous; about 4e9 evaluations. */
int llmcp_q8_selftest_quantizer(llmcp_q8_ctx *ctx, uint64_t *mismatches);

/* Device self-test of the f32 exp inside the silu / sigmoid / softplus
 * epilogues (no counterpart in the reference; it lets a host pin that exp
 * against its own over every float input).  The device evaluates exp for
 * every non-NaN float v.  An exp accurate to 2^-46 can round differently from
 * the correctly rounded value only where exp(v) lies within 2^-46 of a change
 * of float rounding; counts[0] is the number of such inputs, and the first
 * `cap` of them are written to inputs[] with the library's result bits in
 * results[] (*stored of them).  counts[1] is the number of inputs where the
 * library's exp differs from the device math library's exp(double) rounded
 * to float, counts[2] those of them outside the listed set (0 expected), and
 * counts[3] the largest difference between the library's f64 exp and the
 * device math library's, in units in the last place of the latter, over
 * |v| <= 100.  Host buffers; synchronous; about 4e9 evaluations. */
int llmcp_q8_selftest_exp(llmcp_q8_ctx *ctx, uint64_t counts[4], float *inputs,
                          uint32_t *results, int64_t cap, int64_t *stored);

/* ---------------------------------------------------- offline packing -- */

/* quantizeTensorQ8_0Packed (lib/Model/Quantization.cpp:165-214) on the host:
 * [rows, cols] f32 -> rows*cols*34/32 bytes.  OpenMP over lane groups. */
int llmcp_q8_pack_p4_host(const float *w, int64_t rows, int64_t cols,
                          uint8_t *out);

/* Same quantizer on the device for synthetic weights: w[r][c] =
 * stddev * N(0,1) drawn from a counter-based generator keyed by (seed, r*cols+c)
 * and written f32 to w_dev (nullable), then packed into p4_dev. */
int llmcp_q8_synthesize_p4(llmcp_q8_ctx *ctx, uint64_t seed, int64_t rows,
                           int64_t cols, float stddev, float *w_dev,
                           void *p4_dev);

/* Writes a single-file arena (PackedWeights.h layout, manifest of
 * WeightPacker.cpp:126-160) holding the given q8_0_p4 tensors. */
int llmcp_q8_write_arena(const char *path, int32_t count,
                         const char *const *names, const int64_t *rows,
                         const int64_t *cols, const void *const *p4);

/* -------------------------------------------------- MLIR C interface ---- */

/* What the edited lowering hook calls (func.call + llvm.emit_c_interface),
 * on the default context.  Status as above. */
int32_t _mlir_ciface_llmcp_q8_linear(llmcp_memref_f32_2d *input,
                                     llmcp_memref_i8_1d *weight,
                                     llmcp_memref_f32_2d *output,
                                     int32_t activation,
                                     int32_t execution_mode);
/* The group entry in the two arities the model uses (q/k/v, qkv/z/a/b). */
int32_t _mlir_ciface_llmcp_q8_linear_group3(
    llmcp_memref_f32_2d *input, llmcp_memref_i8_1d *w0, llmcp_memref_i8_1d *w1,
    llmcp_memref_i8_1d *w2, llmcp_memref_f32_2d *y0, llmcp_memref_f32_2d *y1,
    llmcp_memref_f32_2d *y2, int32_t act0, int32_t act1, int32_t act2,
    int32_t execution_mode);
int32_t _mlir_ciface_llmcp_q8_linear_group4(
    llmcp_memref_f32_2d *input, llmcp_memref_i8_1d *w0, llmcp_memref_i8_1d *w1,
    llmcp_memref_i8_1d *w2, llmcp_memref_i8_1d *w3, llmcp_memref_f32_2d *y0,
    llmcp_memref_f32_2d *y1, llmcp_memref_f32_2d *y2, llmcp_memref_f32_2d *y3,
    int32_t act0, int32_t act1, int32_t act2, int32_t act3,
    int32_t execution_mode);
/* bf16 twins of the group entries (the real graph's types). */
int32_t _mlir_ciface_llmcp_q8_linear_group3_bf16(
    llmcp_memref_bf16_2d *input, llmcp_memref_i8_1d *w0, llmcp_memref_i8_1d *w1,
    llmcp_memref_i8_1d *w2, llmcp_memref_bf16_2d *y0, llmcp_memref_bf16_2d *y1,
    llmcp_memref_bf16_2d *y2, int32_t act0, int32_t act1, int32_t act2,
    int32_t execution_mode);
int32_t _mlir_ciface_llmcp_q8_linear_group4_bf16(
    llmcp_memref_bf16_2d *input, llmcp_memref_i8_1d *w0, llmcp_memref_i8_1d *w1,
    llmcp_memref_i8_1d *w2, llmcp_memref_i8_1d *w3, llmcp_memref_bf16_2d *y0,
    llmcp_memref_bf16_2d *y1, llmcp_memref_bf16_2d *y2, llmcp_memref_bf16_2d *y3,
    int32_t act0, int32_t act1, int32_t act2, int32_t act3,
    int32_t execution_mode);
/* What the rms_norm / gated_rms_norm patterns call in place of the loop nests
 * of DecodeNormalization.cpp:71-171 and LowerToLinalg.cpp:245-300, :574-720
 * (llmcp_q8_rmsnorm and llmcp_q8_gated_rmsnorm on the default context). */
int32_t _mlir_ciface_llmcp_q8_rmsnorm(llmcp_memref_f32_2d *input, llmcp_memref_f32_1d *weight,
                                      float eps, int32_t zero_centered,
                                      llmcp_memref_f32_2d *output);
int32_t _mlir_ciface_llmcp_q8_rmsnorm_bf16(llmcp_memref_bf16_2d *input,
                                           llmcp_memref_bf16_1d *weight, float eps,
                                           int32_t zero_centered,
                                           llmcp_memref_bf16_2d *output);
int32_t _mlir_ciface_llmcp_q8_gated_rmsnorm(llmcp_memref_f32_2d *input,
                                            llmcp_memref_f32_2d *gate,
                                            llmcp_memref_f32_1d *weight, int64_t group_size,
                                            float eps, int32_t gate_activated,
                                            llmcp_memref_f32_2d *output);
int32_t _mlir_ciface_llmcp_q8_gated_rmsnorm_bf16(llmcp_memref_bf16_2d *input,
                                                 llmcp_memref_bf16_2d *gate,
                                                 llmcp_memref_f32_1d *weight,
                                                 int64_t group_size, float eps,
                                                 int32_t gate_activated,
                                                 llmcp_memref_bf16_2d *output);
/* The norm feeding the q/k/v (3) or qkv/z/a/b (4) group, bf16
 * (llmcp_q8_rmsnorm_linear_group_bf16 on the default context). */
int32_t _mlir_ciface_llmcp_q8_rmsnorm_linear_group3_bf16(
    llmcp_memref_bf16_2d *input, llmcp_memref_bf16_1d *norm_weight, float eps,
    int32_t zero_centered, llmcp_memref_bf16_2d *normed, llmcp_memref_i8_1d *w0,
    llmcp_memref_i8_1d *w1, llmcp_memref_i8_1d *w2, llmcp_memref_bf16_2d *y0,
    llmcp_memref_bf16_2d *y1, llmcp_memref_bf16_2d *y2, int32_t act0, int32_t act1,
    int32_t act2, int32_t execution_mode);
int32_t _mlir_ciface_llmcp_q8_rmsnorm_linear_group4_bf16(
    llmcp_memref_bf16_2d *input, llmcp_memref_bf16_1d *norm_weight, float eps,
    int32_t zero_centered, llmcp_memref_bf16_2d *normed, llmcp_memref_i8_1d *w0,
    llmcp_memref_i8_1d *w1, llmcp_memref_i8_1d *w2, llmcp_memref_i8_1d *w3,
    llmcp_memref_bf16_2d *y0, llmcp_memref_bf16_2d *y1, llmcp_memref_bf16_2d *y2,
    llmcp_memref_bf16_2d *y3, int32_t act0, int32_t act1, int32_t act2, int32_t act3,
    int32_t execution_mode);
int32_t _mlir_ciface_llmcp_q8_swiglu(llmcp_memref_f32_2d *input,
                                     llmcp_memref_i8_1d *w_gate,
                                     llmcp_memref_i8_1d *w_up,
                                     llmcp_memref_f32_2d *output,
                                     int32_t execution_mode);
int32_t _mlir_ciface_llmcp_q8_linear_add(llmcp_memref_f32_2d *input,
                                         llmcp_memref_i8_1d *weight,
                                         llmcp_memref_f32_2d *residual,
                                         llmcp_memref_f32_2d *output,
                                         int32_t execution_mode);
int32_t _mlir_ciface_llmcp_q8_linear_add_bf16(llmcp_memref_bf16_2d *input,
                                              llmcp_memref_i8_1d *weight,
                                              llmcp_memref_bf16_2d *residual,
                                              llmcp_memref_bf16_2d *output,
                                              int32_t execution_mode);
int32_t _mlir_ciface_llmcp_q8_lm_head(llmcp_memref_f32_2d *hidden,
                                      llmcp_memref_i8_1d *table,
                                      llmcp_memref_f32_2d *logits,
                                      llmcp_memref_i64_1d *argmax,
                                      int32_t execution_mode);
int32_t _mlir_ciface_llmcp_q8_embedding(llmcp_memref_i64_1d *tokens,
                                        llmcp_memref_i8_1d *table,
                                        llmcp_memref_f32_2d *output);
int32_t _mlir_ciface_llmcp_q8_linear_bf16(llmcp_memref_bf16_2d *input,
                                          llmcp_memref_i8_1d *weight,
                                          llmcp_memref_bf16_2d *output,
                                          int32_t activation,
                                          int32_t execution_mode);
int32_t _mlir_ciface_llmcp_q8_swiglu_bf16(llmcp_memref_bf16_2d *input,
                                          llmcp_memref_i8_1d *w_gate,
                                          llmcp_memref_i8_1d *w_up,
                                          llmcp_memref_bf16_2d *output,
                                          int32_t execution_mode);
int32_t _mlir_ciface_llmcp_q8_lm_head_bf16(llmcp_memref_bf16_2d *hidden,
                                           llmcp_memref_i8_1d *table,
                                           llmcp_memref_f32_2d *logits,
                                           llmcp_memref_i64_1d *argmax,
                                           int32_t execution_mode);
int32_t _mlir_ciface_llmcp_q8_embedding_bf16(llmcp_memref_i64_1d *tokens,
                                             llmcp_memref_i8_1d *table,
                                             llmcp_memref_bf16_2d *output);

/* ------------------------------------------- device plumbing (host use) -- */
/* Small helpers so hosts without a HIP toolchain (ctypes, cgo) can move data
 * and time work on the context's stream. */

int llmcp_q8_dev_alloc(llmcp_q8_ctx *ctx, uint64_t bytes, void **out);
int llmcp_q8_dev_free(llmcp_q8_ctx *ctx, void *ptr);
int llmcp_q8_memcpy_h2d(llmcp_q8_ctx *ctx, void *dst, const void *src,
                        uint64_t bytes);
int llmcp_q8_memcpy_d2h(llmcp_q8_ctx *ctx, void *dst, const void *src,
                        uint64_t bytes);
int llmcp_q8_memcpy_d2d(llmcp_q8_ctx *ctx, void *dst, const void *src,
                        uint64_t bytes);
int llmcp_q8_event_create(void **event);
int llmcp_q8_event_destroy(void *event);
int llmcp_q8_event_record(llmcp_q8_ctx *ctx, void *event);
int llmcp_q8_event_elapsed_ms(void *start, void *stop, float *ms);
/* Peaks of the device, measured (microbench/cpu_microbench.cpp's role for
 * the reference's CPU: bandwidth read / write / copy, :480-503; the int8
 * dot peak from independent accumulator chains, :203-260).
 * llmcp_q8_microbench_bandwidth: kind 0 read, 1 write, 2 copy over a
 * device buffer of `bytes` (rounded down to a multiple of 64 MiB; copy
 * moves bytes / 2 each way), allocated for the call and freed after;
 * `launches` timed launches after one untimed; *gb_per_s = bytes moved
 * (read plus written) per second / 1e9.  llmcp_q8_microbench_int8_mfma:
 * v_mfma_i32_32x32x32_i8 chains with no memory traffic, three waves per
 * SIMD; *tops = int8 operations (2 per multiply-add) per second / 1e12.
 * llmcp_q8_microbench_epilogue: the prefill GEMM's per-block work on one
 * 32x32 tile without its memory stream, three waves per SIMD, `blocks`
 * blocks per wave (rounded down to even, at least 2): mode 0 the exact
 * epilogue (int8 MFMA, f32 scale tile, a convert and an FMA per element
 * and block), mode 1 the same with two f16 MFMAs per block on
 * integer-valued operands and no convert, mode 2 the MFMAs alone; *tops =
 * the tile's int8 operations (2 * 32^3 per block) per second / 1e12, the
 * ceiling of the GEMM for that epilogue.  All synchronize the context's
 * stream. */
int llmcp_q8_microbench_bandwidth(llmcp_q8_ctx *ctx, int32_t kind, uint64_t bytes,
                                  int32_t launches, double *gb_per_s);
int llmcp_q8_microbench_int8_mfma(llmcp_q8_ctx *ctx, int32_t iterations, double *tops);
int llmcp_q8_microbench_epilogue(llmcp_q8_ctx *ctx, int32_t mode, int32_t blocks,
                                 double *tops);

/* Stream capture into a HIP graph and replay (launch-bound loops).  A graph
 * holds the device addresses of the context's workspace and weights at
 * capture: graph_launch refuses it with LLMCP_Q8_ESTALE once any of them
 * was freed or reallocated (a call that grew the workspace, a weight
 * released or registered again). */
int llmcp_q8_graph_begin(llmcp_q8_ctx *ctx);
int llmcp_q8_graph_end(llmcp_q8_ctx *ctx, void **graph_exec);
int llmcp_q8_graph_launch(llmcp_q8_ctx *ctx, void *graph_exec);
int llmcp_q8_graph_destroy(void *graph_exec);
/* Bytes the device copy of a registered weight occupies (0 if unknown). */
uint64_t llmcp_q8_device_bytes(llmcp_q8_ctx *ctx, const void *key);

#ifdef __cplusplus
}
#endif

#endif /* LLMCP_Q8_H */
