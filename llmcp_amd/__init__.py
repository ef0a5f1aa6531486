"""llmcp_amd -- MI355X (gfx950) Q8_0 quantized linear path of llmcp.

The product is the C-ABI shared library ``libllmcp_q8.so`` (declared in
``include/llmcp_q8.h``).  This module is a thin ctypes front end that mirrors
the reference operators (``llmcp.linear`` / ``llmcp.lm_head`` /
``llmcp.embedding`` with ``weight_format = "q8_0_p4"``) for tests and
benchmarks.  Device memory and streams are plain HIP through the same
library; there is no fallback: if the library is missing, loading fails.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libllmcp_q8.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "llmcp_q8.h")

OK, DECLINED, EINVAL, ENOTFOUND, EHIP, EFORMAT, EIO, ENOMEM, EINTERNAL, ESTALE = range(10)
ACT = {"none": 0, "silu": 1, "sigmoid": 2, "softplus": 3}
DTYPES = ("f32", "bf16")
MODE = {"prefill": 0, "decode": 1}
# Reference platforms (llmcp_q8_platform) and the per-block epilogue each
# computes: fma on aarch64 (SDOT emitters), mul+add on x86 (scalar path).
PLATFORM = {"x86": 0, "aarch64": 1}
ACCUM = {"exact": 0, "split_k": 1}
EPILOGUE = {"x86": "scalar", "aarch64": "fma"}

_lib = None


class Q8Error(RuntimeError):
    def __init__(self, code, message):
        super().__init__("llmcp_q8 status %d: %s" % (code, message))
        self.code = code


class Declined(Q8Error):
    """The hook declined the op (reference: null Value -> caller falls back)."""


class MemRefF32(ctypes.Structure):
    _fields_ = [("base", ctypes.c_void_p), ("data", ctypes.c_void_p),
                ("offset", ctypes.c_int64), ("sizes", ctypes.c_int64 * 2),
                ("strides", ctypes.c_int64 * 2)]


class MemRefI8(ctypes.Structure):
    _fields_ = [("base", ctypes.c_void_p), ("data", ctypes.c_void_p),
                ("offset", ctypes.c_int64), ("sizes", ctypes.c_int64 * 1),
                ("strides", ctypes.c_int64 * 1)]


class MemRefI64(ctypes.Structure):
    _fields_ = [("base", ctypes.c_void_p), ("data", ctypes.c_void_p),
                ("offset", ctypes.c_int64), ("sizes", ctypes.c_int64 * 1),
                ("strides", ctypes.c_int64 * 1)]


EXPORTS = [
    "llmcp_q8_abi_version", "llmcp_q8_last_error", "llmcp_q8_ctx_create",
    "llmcp_q8_ctx_destroy", "llmcp_q8_ctx_set_stream", "llmcp_q8_ctx_stream",
    "llmcp_q8_ctx_synchronize", "llmcp_q8_set_default_ctx",
    "llmcp_q8_set_platform", "llmcp_q8_get_platform", "llmcp_q8_set_weight_budget",
    "llmcp_q8_upload_p4", "llmcp_q8_register_device_p4", "llmcp_q8_release",
    "llmcp_q8_upload_arena", "llmcp_q8_arena_inspect", "llmcp_q8_linear", "llmcp_q8_swiglu",
    "llmcp_q8_lm_head", "llmcp_q8_mlp", "llmcp_q8_embedding", "llmcp_q8_quantize_activations",
    "llmcp_q8_block_dots", "llmcp_q8_ctx_check", "llmcp_q8_pack_p4_host",
    "llmcp_q8_synthesize_p4", "llmcp_q8_write_arena",
    "_mlir_ciface_llmcp_q8_linear", "_mlir_ciface_llmcp_q8_swiglu",
    "_mlir_ciface_llmcp_q8_lm_head", "_mlir_ciface_llmcp_q8_embedding",
    "llmcp_q8_dev_alloc", "llmcp_q8_dev_free", "llmcp_q8_memcpy_h2d",
    "llmcp_q8_memcpy_d2h", "llmcp_q8_memcpy_d2d", "llmcp_q8_event_create",
    "llmcp_q8_event_destroy", "llmcp_q8_event_record",
    "llmcp_q8_event_elapsed_ms", "llmcp_q8_graph_begin", "llmcp_q8_graph_end",
    "llmcp_q8_graph_launch", "llmcp_q8_graph_destroy",
    "llmcp_q8_device_bytes", "llmcp_q8_selftest_quantizer", "llmcp_q8_selftest_exp",
    "llmcp_q8_linear_bf16", "llmcp_q8_swiglu_bf16", "llmcp_q8_mlp_bf16",
    "llmcp_q8_lm_head_bf16", "llmcp_q8_embedding_bf16", "llmcp_q8_lm_head_noalloc",
    "_mlir_ciface_llmcp_q8_linear_bf16", "_mlir_ciface_llmcp_q8_swiglu_bf16",
    "_mlir_ciface_llmcp_q8_lm_head_bf16", "_mlir_ciface_llmcp_q8_embedding_bf16",
    "llmcp_q8_linear_add", "llmcp_q8_linear_add_bf16",
    "_mlir_ciface_llmcp_q8_linear_add", "_mlir_ciface_llmcp_q8_linear_add_bf16",
    "llmcp_q8_linear_group", "llmcp_q8_linear_group_bf16",
    "_mlir_ciface_llmcp_q8_linear_group3", "_mlir_ciface_llmcp_q8_linear_group4",
    "llmcp_q8_rmsnorm", "llmcp_q8_rmsnorm_bf16", "llmcp_q8_rmsnorm_linear_group",
    "llmcp_q8_rmsnorm_linear_group_bf16", "llmcp_q8_gated_rmsnorm",
    "llmcp_q8_gated_rmsnorm_bf16", "llmcp_q8_set_accumulation", "llmcp_q8_get_accumulation",
    "llmcp_q8_microbench_bandwidth", "llmcp_q8_microbench_int8_mfma",
    "llmcp_q8_microbench_epilogue",
    "_mlir_ciface_llmcp_q8_linear_group3_bf16", "_mlir_ciface_llmcp_q8_linear_group4_bf16",
    "_mlir_ciface_llmcp_q8_rmsnorm", "_mlir_ciface_llmcp_q8_rmsnorm_bf16",
    "_mlir_ciface_llmcp_q8_gated_rmsnorm", "_mlir_ciface_llmcp_q8_gated_rmsnorm_bf16",
    "_mlir_ciface_llmcp_q8_rmsnorm_linear_group3_bf16",
    "_mlir_ciface_llmcp_q8_rmsnorm_linear_group4_bf16",
]


def lib():
    """Loads libllmcp_q8.so; raises if it was not built (no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError("libllmcp_q8.so is not built; run "
                          "`python llmcp_amd/build.py` (or __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH)
    P, I, I32, I64, U64 = (ctypes.c_void_p, ctypes.c_int, ctypes.c_int32,
                           ctypes.c_int64, ctypes.c_uint64)
    F = ctypes.POINTER(ctypes.c_float)
    sig = {
        "llmcp_q8_abi_version": (I32, []),
        "llmcp_q8_test_ctx_rmsnorm_skew": (I, [P, I32]),
        "llmcp_q8_test_ctx_gemm_splits": (I, [P, I32]),
        "llmcp_q8_set_accumulation": (I, [P, I32]),
        "llmcp_q8_microbench_bandwidth": (I, [P, I32, U64, I32, ctypes.POINTER(ctypes.c_double)]),
        "llmcp_q8_microbench_int8_mfma": (I, [P, I32, ctypes.POINTER(ctypes.c_double)]),
        "llmcp_q8_microbench_epilogue": (I, [P, I32, I32, ctypes.POINTER(ctypes.c_double)]),
        "llmcp_q8_get_accumulation": (I32, [P]),
        "llmcp_q8_last_error": (ctypes.c_char_p, []),
        "llmcp_q8_ctx_create": (I, [I, ctypes.POINTER(P)]),
        "llmcp_q8_ctx_destroy": (I, [P]),
        "llmcp_q8_ctx_set_stream": (I, [P, P]),
        "llmcp_q8_ctx_stream": (P, [P]),
        "llmcp_q8_ctx_synchronize": (I, [P]),
        "llmcp_q8_set_default_ctx": (I, [P]),
        "llmcp_q8_set_platform": (I, [P, I32]),
        "llmcp_q8_get_platform": (I32, [P]),
        "llmcp_q8_set_weight_budget": (I, [P, U64]),
        "llmcp_q8_upload_p4": (I, [P, P, I64, I64, F]),
        "llmcp_q8_register_device_p4": (I, [P, P, I64, I64, F]),
        "llmcp_q8_release": (I, [P, P]),
        "llmcp_q8_upload_arena": (I, [P, P, U64, ctypes.POINTER(I64)]),
        "llmcp_q8_arena_inspect": (I, [P, U64, ctypes.POINTER(I64),
                                       ctypes.POINTER(I64)]),
        "llmcp_q8_linear": (I, [P, P, P, P, I32, I32]),
        "llmcp_q8_swiglu": (I, [P, P, P, P, P, I32]),
        "llmcp_q8_lm_head": (I, [P, P, P, P, P, I32]),
        "llmcp_q8_mlp": (I, [P, P, P, P, P, P, P, I32]),
        "llmcp_q8_embedding": (I, [P, P, P, P]),
        "llmcp_q8_quantize_activations": (I, [P, P, P, P]),
        "llmcp_q8_block_dots": (I, [P, P, P, P]),
        "llmcp_q8_ctx_check": (I, [P, ctypes.POINTER(I32)]),
        "llmcp_q8_pack_p4_host": (I, [P, I64, I64, P]),
        "llmcp_q8_synthesize_p4": (I, [P, U64, I64, I64, ctypes.c_float, P, P]),
        "llmcp_q8_write_arena": (I, [ctypes.c_char_p, I32, P, P, P, P]),
        "_mlir_ciface_llmcp_q8_linear": (I32, [P, P, P, I32, I32]),
        "_mlir_ciface_llmcp_q8_swiglu": (I32, [P, P, P, P, I32]),
        "_mlir_ciface_llmcp_q8_lm_head": (I32, [P, P, P, P, I32]),
        "_mlir_ciface_llmcp_q8_embedding": (I32, [P, P, P]),
        "llmcp_q8_dev_alloc": (I, [P, U64, ctypes.POINTER(P)]),
        "llmcp_q8_dev_free": (I, [P, P]),
        "llmcp_q8_memcpy_h2d": (I, [P, P, P, U64]),
        "llmcp_q8_memcpy_d2h": (I, [P, P, P, U64]),
        "llmcp_q8_memcpy_d2d": (I, [P, P, P, U64]),
        "llmcp_q8_event_create": (I, [ctypes.POINTER(P)]),
        "llmcp_q8_event_destroy": (I, [P]),
        "llmcp_q8_event_record": (I, [P, P]),
        "llmcp_q8_event_elapsed_ms": (I, [P, P, F]),
        "llmcp_q8_graph_begin": (I, [P]),
        "llmcp_q8_graph_end": (I, [P, ctypes.POINTER(P)]),
        "llmcp_q8_graph_launch": (I, [P, P]),
        "llmcp_q8_graph_destroy": (I, [P]),
        "llmcp_q8_device_bytes": (U64, [P, P]),
        "llmcp_q8_selftest_quantizer": (I, [P, ctypes.POINTER(U64)]),
        "llmcp_q8_selftest_exp": (I, [P, ctypes.POINTER(U64), P, P, ctypes.c_int64,
                                      ctypes.POINTER(ctypes.c_int64)]),
        "llmcp_q8_linear_bf16": (I, [P, P, P, P, I32, I32]),
        "llmcp_q8_swiglu_bf16": (I, [P, P, P, P, P, I32]),
        "llmcp_q8_mlp_bf16": (I, [P, P, P, P, P, P, P, I32]),
        "llmcp_q8_lm_head_bf16": (I, [P, P, P, P, P, I32]),
        "llmcp_q8_lm_head_noalloc": (I, [P, P, P, P, P, I32]),
        "llmcp_q8_embedding_bf16": (I, [P, P, P, P]),
        "_mlir_ciface_llmcp_q8_linear_bf16": (I32, [P, P, P, I32, I32]),
        "_mlir_ciface_llmcp_q8_swiglu_bf16": (I32, [P, P, P, P, I32]),
        "_mlir_ciface_llmcp_q8_lm_head_bf16": (I32, [P, P, P, P, I32]),
        "_mlir_ciface_llmcp_q8_embedding_bf16": (I32, [P, P, P]),
        "llmcp_q8_linear_add": (I, [P, P, P, P, P, I32]),
        "llmcp_q8_linear_add_bf16": (I, [P, P, P, P, P, I32]),
        "_mlir_ciface_llmcp_q8_linear_add": (I32, [P, P, P, P, I32]),
        "_mlir_ciface_llmcp_q8_linear_add_bf16": (I32, [P, P, P, P, I32]),
        "llmcp_q8_linear_group": (I, [P, P, I32, P, P, P, I32]),
        "llmcp_q8_linear_group_bf16": (I, [P, P, I32, P, P, P, I32]),
        "_mlir_ciface_llmcp_q8_linear_group3": (I32, [P] * 7 + [I32] * 4),
        "_mlir_ciface_llmcp_q8_linear_group4": (I32, [P] * 9 + [I32] * 5),
        "llmcp_q8_rmsnorm": (I, [P, P, P, ctypes.c_float, I32, P]),
        "llmcp_q8_rmsnorm_bf16": (I, [P, P, P, ctypes.c_float, I32, P]),
        "llmcp_q8_rmsnorm_linear_group": (I, [P, P, P, ctypes.c_float, I32, P, I32, P, P, P, I32]),
        "llmcp_q8_gated_rmsnorm": (I, [P, P, P, P, I64, ctypes.c_float, I32, P]),
        "llmcp_q8_gated_rmsnorm_bf16": (I, [P, P, P, P, I64, ctypes.c_float, I32, P]),
        "llmcp_q8_rmsnorm_linear_group_bf16": (I, [P, P, P, ctypes.c_float, I32, P, I32, P, P,
                                                   P, I32]),
        "_mlir_ciface_llmcp_q8_linear_group3_bf16": (I32, [P] * 7 + [I32] * 4),
        "_mlir_ciface_llmcp_q8_linear_group4_bf16": (I32, [P] * 9 + [I32] * 5),
        "_mlir_ciface_llmcp_q8_rmsnorm": (I32, [P, P, ctypes.c_float, I32, P]),
        "_mlir_ciface_llmcp_q8_rmsnorm_bf16": (I32, [P, P, ctypes.c_float, I32, P]),
        "_mlir_ciface_llmcp_q8_gated_rmsnorm": (I32, [P, P, P, I64, ctypes.c_float, I32, P]),
        "_mlir_ciface_llmcp_q8_gated_rmsnorm_bf16": (I32, [P, P, P, I64, ctypes.c_float, I32,
                                                           P]),
        "_mlir_ciface_llmcp_q8_rmsnorm_linear_group3_bf16": (
            I32, [P, P, ctypes.c_float, I32, P] + [P] * 6 + [I32] * 4),
        "_mlir_ciface_llmcp_q8_rmsnorm_linear_group4_bf16": (
            I32, [P, P, ctypes.c_float, I32, P] + [P] * 8 + [I32] * 5),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def last_error():
    msg = lib().llmcp_q8_last_error()
    return msg.decode() if msg else ""


def check(rc):
    if rc == OK:
        return
    if rc == DECLINED:
        raise Declined(rc, last_error())
    raise Q8Error(rc, last_error())


def f32_memref(ptr, rows, cols, row_stride=None):
    d = MemRefF32()
    d.base = d.data = ptr
    d.offset = 0
    d.sizes[0], d.sizes[1] = rows, cols
    d.strides[0], d.strides[1] = (cols if row_stride is None else row_stride), 1
    return d


def i8_memref(ptr, nbytes):
    d = MemRefI8()
    d.base = d.data = ptr
    d.offset = 0
    d.sizes[0] = nbytes
    d.strides[0] = 1
    return d


def i64_memref(ptr, count):
    d = MemRefI64()
    d.base = d.data = ptr
    d.offset = 0
    d.sizes[0] = count
    d.strides[0] = 1
    return d


def p4_bytes(rows, cols):
    """Arena size of a q8_0_p4 tensor: N * (K + (K/32)*2) (LLMCPOps.cpp:57-65)."""
    return rows * (cols + cols // 32 * 2)


class DeviceBuffer:
    def __init__(self, ctx, nbytes):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(lib().llmcp_q8_dev_alloc(ctx.handle, self.nbytes, ctypes.byref(p)))
        self.ptr = p.value

    def free(self):
        if self.ptr is not None:
            check(lib().llmcp_q8_dev_free(self.ctx.handle, self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr is not None and self.ctx.handle:
                lib().llmcp_q8_dev_free(self.ctx.handle, self.ptr)
        except Exception:
            pass


class Weight:
    """A q8_0_p4 tensor [rows, cols] known to the library's registry."""

    def __init__(self, ctx, key_ptr, rows, cols, owner=None, repack_ms=None):
        self.ctx, self.key, self.rows, self.cols = ctx, key_ptr, rows, cols
        self.owner = owner  # keeps the host/device bytes alive
        self.repack_ms = repack_ms

    @property
    def nbytes(self):
        return p4_bytes(self.rows, self.cols)

    def memref(self):
        return i8_memref(self.key, self.nbytes)


class Context:
    def __init__(self, device=0):
        h = ctypes.c_void_p()
        check(lib().llmcp_q8_ctx_create(device, ctypes.byref(h)))
        self.handle = h.value

    def close(self):
        if self.handle:
            lib().llmcp_q8_ctx_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def set_platform(self, platform):
        """'aarch64' (SDOT emitters: fma epilogue, the default) or 'x86'
        (scalar path: mul+add) for every later call."""
        check(lib().llmcp_q8_set_platform(self.handle, PLATFORM[platform]))

    def set_accumulation(self, mode, splits=0):
        """'exact' (the serial block order, bit for bit: the default) or
        'split_k' (multi-row GEMMs that underfill the GPU split K, within
        the reference's tolerance) for every later call; `splits` > 0 forces
        that many K splits (a test hook; 0 = chosen by shape)."""
        check(lib().llmcp_q8_set_accumulation(self.handle, ACCUM[mode]))
        check(lib().llmcp_q8_test_ctx_gemm_splits(self.handle, int(splits)))

    @property
    def accumulation(self):
        code = lib().llmcp_q8_get_accumulation(self.handle)
        return {v: k for k, v in ACCUM.items()}.get(code, code)

    def microbench_bandwidth(self, kind, nbytes, launches=10):
        """Measured streaming GB/s: kind 'read', 'write' or 'copy'."""
        out = ctypes.c_double(0.0)
        check(lib().llmcp_q8_microbench_bandwidth(
            self.handle, {"read": 0, "write": 1, "copy": 2}[kind], int(nbytes), int(launches),
            ctypes.byref(out)))
        return out.value

    def microbench_int8_mfma(self, iterations=20000):
        """Measured int8 MFMA TOPS (no memory traffic)."""
        out = ctypes.c_double(0.0)
        check(lib().llmcp_q8_microbench_int8_mfma(self.handle, int(iterations), ctypes.byref(out)))
        return out.value

    def microbench_epilogue(self, mode="exact", blocks=20000):
        """TOPS ceiling of the prefill GEMM's per-block work without its memory
        stream: mode 'exact' (int8 MFMA + convert + FMA), 'cvtfree' (f16
        MFMAs on integer operands + FMA) or 'mfma' (the MFMAs alone)."""
        out = ctypes.c_double(0.0)
        check(lib().llmcp_q8_microbench_epilogue(
            self.handle, {"exact": 0, "cvtfree": 1, "mfma": 2}[mode], int(blocks),
            ctypes.byref(out)))
        return out.value

    def set_platform_code(self, code):
        """llmcp_q8_set_platform with a raw code (tests of the error path)."""
        check(lib().llmcp_q8_set_platform(self.handle, int(code)))

    @property
    def platform(self):
        code = lib().llmcp_q8_get_platform(self.handle)
        return {v: k for k, v in PLATFORM.items()}[code]

    @property
    def epilogue(self):
        """The oracle epilogue this context reproduces bit for bit."""
        return EPILOGUE[self.platform]

    @property
    def other_epilogue(self):
        """The other platform's epilogue (agrees within tolerance)."""
        return "scalar" if self.epilogue == "fma" else "fma"

    def set_weight_budget(self, nbytes):
        """Caps the device bytes of registered weights (0: no cap)."""
        check(lib().llmcp_q8_set_weight_budget(self.handle, int(nbytes)))

    def sync(self):
        check(lib().llmcp_q8_ctx_synchronize(self.handle))

    # ---- memory plumbing
    def alloc(self, nbytes):
        return DeviceBuffer(self, nbytes)

    def to_device(self, array):
        a = np.ascontiguousarray(array)
        buf = self.alloc(max(a.nbytes, 1))
        if a.nbytes:
            check(lib().llmcp_q8_memcpy_h2d(self.handle, buf.ptr,
                                            a.ctypes.data, a.nbytes))
        return buf

    def to_host(self, buf, shape, dtype, offset=0):
        out = np.empty(shape, dtype=dtype)
        if out.nbytes:
            check(lib().llmcp_q8_memcpy_d2h(self.handle, out.ctypes.data,
                                            buf.ptr + offset, out.nbytes))
        return out

    # ---- weights
    def upload_p4(self, host_p4, rows, cols, time_repack=False):
        host = np.ascontiguousarray(host_p4, dtype=np.uint8)
        ms = ctypes.c_float(0.0)
        check(lib().llmcp_q8_upload_p4(self.handle, host.ctypes.data, rows, cols,
                                       ctypes.byref(ms) if time_repack else None))
        return Weight(self, host.ctypes.data, rows, cols, owner=host,
                      repack_ms=ms.value if time_repack else None)

    def register_device_p4(self, buf, rows, cols, time_repack=False):
        ms = ctypes.c_float(0.0)
        check(lib().llmcp_q8_register_device_p4(
            self.handle, buf.ptr, rows, cols,
            ctypes.byref(ms) if time_repack else None))
        return Weight(self, buf.ptr, rows, cols, owner=buf,
                      repack_ms=ms.value if time_repack else None)

    def synthesize_p4(self, seed, rows, cols, stddev=0.02, keep_f32=False):
        """Device-generated N(0, stddev^2) weights packed to q8_0_p4.
        Returns (p4 DeviceBuffer, f32 DeviceBuffer or None)."""
        p4 = self.alloc(p4_bytes(rows, cols))
        w = self.alloc(rows * cols * 4) if keep_f32 else None
        check(lib().llmcp_q8_synthesize_p4(self.handle, seed, rows, cols,
                                           ctypes.c_float(stddev),
                                           w.ptr if w else None, p4.ptr))
        self.sync()
        return p4, w

    def release(self, weight):
        check(lib().llmcp_q8_release(self.handle, weight.key))

    def upload_arena(self, file_bytes):
        n = ctypes.c_int64(0)
        check(lib().llmcp_q8_upload_arena(self.handle, file_bytes.ctypes.data,
                                          file_bytes.nbytes, ctypes.byref(n)))
        return n.value

    # ---- ops (device pointers in, device pointers out).  dtype "bf16"
    # selects the *_bf16 entry: bf16 activations in and out (raw uint16
    # bits; the lm_head keeps f32 logits).  The descriptor layout is the
    # same for both element types.
    @staticmethod
    def _entry(name, dtype):
        if dtype not in DTYPES:
            raise ValueError("dtype must be one of %r" % (DTYPES,))
        return getattr(lib(), name + ("_bf16" if dtype == "bf16" else ""))

    def linear_add(self, x, w, r, y, m, mode="decode", dtype="f32"):
        """y = r + linear(x): the residual add in the linear's epilogue
        (r and y [m, w.rows], same element type; r may be y)."""
        xi = f32_memref(x.ptr if hasattr(x, "ptr") else x, m, w.cols)
        ri = f32_memref(r.ptr if hasattr(r, "ptr") else r, m, w.rows)
        yo = f32_memref(y.ptr if hasattr(y, "ptr") else y, m, w.rows)
        check(self._entry("llmcp_q8_linear_add", dtype)(
            self.handle, ctypes.byref(xi), ctypes.byref(w.memref()),
            ctypes.byref(ri), ctypes.byref(yo), MODE[mode]))

    def linear(self, x, w, y, m, activation="none", mode="decode", dtype="f32"):
        xi = f32_memref(x.ptr if hasattr(x, "ptr") else x, m, w.cols)
        yo = f32_memref(y.ptr if hasattr(y, "ptr") else y, m, w.rows)
        check(self._entry("llmcp_q8_linear", dtype)(
            self.handle, ctypes.byref(xi), ctypes.byref(w.memref()),
            ctypes.byref(yo), ACT[activation], MODE[mode]))

    def linear_group(self, x, weights, outputs, m, activations=None,
                     mode="decode", dtype="f32"):
        """Linears sharing the input x: outputs[i] = act_i(x . W_i^T)."""
        n = len(weights)
        k = weights[0].cols
        xi = f32_memref(x.ptr if hasattr(x, "ptr") else x, m, k)
        ws = [w.memref() for w in weights]
        ys = [f32_memref(y.ptr if hasattr(y, "ptr") else y, m, w.rows)
              for y, w in zip(outputs, weights)]
        wp = (ctypes.c_void_p * n)(*[ctypes.addressof(d) for d in ws])
        yp = (ctypes.c_void_p * n)(*[ctypes.addressof(d) for d in ys])
        acts = (ctypes.c_int32 * n)(*[ACT[a] for a in (activations or ["none"] * n)])
        check(self._entry("llmcp_q8_linear_group", dtype)(
            self.handle, ctypes.byref(xi), n, wp, yp, acts, MODE[mode]))

    def rmsnorm(self, x, w, y, m, h, eps=1e-6, zero_centered=False, dtype="f32"):
        """y = RMSNorm(x) with weight w [h] (x, w and y of dtype)."""
        xi = f32_memref(x.ptr if hasattr(x, "ptr") else x, m, h)
        yo = f32_memref(y.ptr if hasattr(y, "ptr") else y, m, h)
        wv = i8_memref(w.ptr if hasattr(w, "ptr") else w, h)
        check(self._entry("llmcp_q8_rmsnorm", dtype)(
            self.handle, ctypes.byref(xi), ctypes.byref(wv), float(eps),
            1 if zero_centered else 0, ctypes.byref(yo)))

    def gated_rmsnorm(self, x, gate, w, y, m, h, group, eps=1e-6, gate_activated=False,
                      dtype="f32"):
        """y = gated RMSNorm of x [m, h] with gate [m, h] in groups of `group`
        (x, gate and y of dtype; w [group] f32)."""
        xi = f32_memref(x.ptr if hasattr(x, "ptr") else x, m, h)
        gi = f32_memref(gate.ptr if hasattr(gate, "ptr") else gate, m, h)
        yo = f32_memref(y.ptr if hasattr(y, "ptr") else y, m, h)
        wv = i8_memref(w.ptr if hasattr(w, "ptr") else w, group)
        check(self._entry("llmcp_q8_gated_rmsnorm", dtype)(
            self.handle, ctypes.byref(xi), ctypes.byref(gi), ctypes.byref(wv), int(group),
            float(eps), 1 if gate_activated else 0, ctypes.byref(yo)))

    def rmsnorm_linear_group(self, x, norm_w, normed, weights, outputs, m, eps=1e-6,
                             zero_centered=False, activations=None, mode="decode",
                             dtype="f32"):
        """normed = RMSNorm(x); outputs[i] = act_i(normed . W_i^T)."""
        n = len(weights)
        k = weights[0].cols
        xi = f32_memref(x.ptr if hasattr(x, "ptr") else x, m, k)
        no = f32_memref(normed.ptr if hasattr(normed, "ptr") else normed, m, k)
        wv = i8_memref(norm_w.ptr if hasattr(norm_w, "ptr") else norm_w, k)
        ws = [w.memref() for w in weights]
        ys = [f32_memref(y.ptr if hasattr(y, "ptr") else y, m, w.rows)
              for y, w in zip(outputs, weights)]
        wp = (ctypes.c_void_p * n)(*[ctypes.addressof(d) for d in ws])
        yp = (ctypes.c_void_p * n)(*[ctypes.addressof(d) for d in ys])
        acts = (ctypes.c_int32 * n)(*[ACT[a] for a in (activations or ["none"] * n)])
        check(self._entry("llmcp_q8_rmsnorm_linear_group", dtype)(
            self.handle, ctypes.byref(xi), ctypes.byref(wv), float(eps),
            1 if zero_centered else 0, ctypes.byref(no), n, wp, yp, acts, MODE[mode]))

    def swiglu(self, x, wg, wu, h, m, mode="decode", dtype="f32"):
        xi = f32_memref(x.ptr if hasattr(x, "ptr") else x, m, wg.cols)
        ho = f32_memref(h.ptr if hasattr(h, "ptr") else h, m, wg.rows)
        check(self._entry("llmcp_q8_swiglu", dtype)(
            self.handle, ctypes.byref(xi), ctypes.byref(wg.memref()),
            ctypes.byref(wu.memref()), ctypes.byref(ho), MODE[mode]))

    def mlp(self, x, wg, wu, wd, y, h=None, m=1, mode="decode", dtype="f32"):
        xi = f32_memref(x.ptr if hasattr(x, "ptr") else x, m, wg.cols)
        yo = f32_memref(y.ptr if hasattr(y, "ptr") else y, m, wd.rows)
        ho = f32_memref(h.ptr if hasattr(h, "ptr") else h, m, wg.rows) if h is not None else None
        check(self._entry("llmcp_q8_mlp", dtype)(
            self.handle, ctypes.byref(xi), ctypes.byref(wg.memref()),
            ctypes.byref(wu.memref()), ctypes.byref(wd.memref()),
            ctypes.byref(ho) if ho is not None else None,
            ctypes.byref(yo), MODE[mode]))

    def lm_head(self, x, w, logits, m, argmax=None, mode="decode", dtype="f32"):
        xi = f32_memref(x.ptr if hasattr(x, "ptr") else x, m, w.cols)
        lo = f32_memref(logits.ptr if hasattr(logits, "ptr") else logits, m, w.rows)
        am = argmax.ptr if argmax is not None else None
        check(self._entry("llmcp_q8_lm_head", dtype)(
            self.handle, ctypes.byref(xi), ctypes.byref(w.memref()),
            ctypes.byref(lo), am, MODE[mode]))

    def embedding(self, tokens, count, w, out, dtype="f32"):
        t = i64_memref(tokens.ptr, count)
        o = f32_memref(out.ptr, count, w.cols)
        check(self._entry("llmcp_q8_embedding", dtype)(
            self.handle, ctypes.byref(t), ctypes.byref(w.memref()),
            ctypes.byref(o)))

    def quantize(self, x, m, k, qa, sa):
        xi = f32_memref(x.ptr, m, k)
        check(lib().llmcp_q8_quantize_activations(self.handle, ctypes.byref(xi),
                                                  qa.ptr, sa.ptr))

    def block_dots(self, x, w, out, m):
        xi = f32_memref(x.ptr, m, w.cols)
        check(lib().llmcp_q8_block_dots(self.handle, ctypes.byref(xi),
                                        ctypes.byref(w.memref()), out.ptr))

    def check_flag(self):
        f = ctypes.c_int32(0)
        check(lib().llmcp_q8_ctx_check(self.handle, ctypes.byref(f)))
        return f.value

    def selftest_quantizer(self):
        """Mismatches of the quantizer's division identities (0 expected)."""
        n = ctypes.c_uint64(0)
        check(lib().llmcp_q8_selftest_quantizer(self.handle, ctypes.byref(n)))
        return n.value

    def selftest_exp(self, cap=1 << 16):
        """Exhaustive device check of the epilogues' f32 exp: returns
        (counts, inputs, result_bits) -- counts = (inputs near a float
        rounding change, differences from the device math library's
        exp(double), those differences outside the listed inputs, largest
        f64 difference from that library's exp in its ulps)."""
        counts = (ctypes.c_uint64 * 4)()
        xs = np.zeros(cap, np.float32)
        rs = np.zeros(cap, np.uint32)
        k = ctypes.c_int64(0)
        check(lib().llmcp_q8_selftest_exp(self.handle, counts, xs.ctypes.data,
                                          rs.ctypes.data, cap, ctypes.byref(k)))
        return tuple(int(c) for c in counts), xs[:k.value], rs[:k.value]

    # ---- timing
    def event(self):
        e = ctypes.c_void_p()
        check(lib().llmcp_q8_event_create(ctypes.byref(e)))
        return e.value

    def record(self, event):
        check(lib().llmcp_q8_event_record(self.handle, event))

    @staticmethod
    def elapsed_ms(start, stop):
        ms = ctypes.c_float(0.0)
        check(lib().llmcp_q8_event_elapsed_ms(start, stop, ctypes.byref(ms)))
        return ms.value

    def graph_begin(self):
        check(lib().llmcp_q8_graph_begin(self.handle))

    def graph_end(self):
        g = ctypes.c_void_p()
        check(lib().llmcp_q8_graph_end(self.handle, ctypes.byref(g)))
        return g.value

    def graph_launch(self, g):
        check(lib().llmcp_q8_graph_launch(self.handle, g))

    def graph_destroy(self, g):
        check(lib().llmcp_q8_graph_destroy(g))


def pack_p4_host(w):
    """Host llmcp-pack (quantizeTensorQ8_0Packed) of an f32 [N,K] matrix."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    out = np.zeros(p4_bytes(n, k), np.uint8)
    check(lib().llmcp_q8_pack_p4_host(w.ctypes.data, n, k, out.ctypes.data))
    return out


def write_arena(path, tensors):
    """tensors: list of (name, rows, cols, p4 uint8 array)."""
    n = len(tensors)
    names = (ctypes.c_char_p * n)(*[t[0].encode() for t in tensors])
    rows = (ctypes.c_int64 * n)(*[t[1] for t in tensors])
    cols = (ctypes.c_int64 * n)(*[t[2] for t in tensors])
    arrays = [np.ascontiguousarray(t[3], dtype=np.uint8) for t in tensors]
    ptrs = (ctypes.c_void_p * n)(*[a.ctypes.data for a in arrays])
    check(lib().llmcp_q8_write_arena(path.encode(), n, names, rows, cols, ptrs))


def arena_inspect(file_bytes):
    """Validates an LLMCPWGT file image on the host: (tensors, q8 tensors)."""
    buf = np.ascontiguousarray(file_bytes, dtype=np.uint8)
    n, q = ctypes.c_int64(0), ctypes.c_int64(0)
    check(lib().llmcp_q8_arena_inspect(buf.ctypes.data, buf.nbytes,
                                       ctypes.byref(n), ctypes.byref(q)))
    return n.value, q.value
