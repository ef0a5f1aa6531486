"""ctypes front end of oracle/q8_oracle.c -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this module.  Each wrapper restates one reference function;
the C source cites the reference file:line it follows.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libq8oracle.so")

QK = 32
RECORD = 136
ACT = {"none": 0, "silu": 1, "sigmoid": 2, "softplus": 3}
EPI = {"scalar": 0, "fma": 1}

_lib = None


def build():
    """Compile the C oracle in place (make, gcc)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(L):
    P = ctypes.c_void_p
    I64 = ctypes.c_int64
    I = ctypes.c_int
    L.oracle_f32_to_f16.restype = ctypes.c_uint16
    L.oracle_f32_to_f16.argtypes = [ctypes.c_float]
    L.oracle_f16_to_f32.restype = ctypes.c_float
    L.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.oracle_f32_to_f16_batch.argtypes = [P, I64, P]
    L.oracle_f16_to_f32_batch.argtypes = [P, I64, P]
    L.oracle_f32_to_bf16.restype = ctypes.c_uint16
    L.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
    L.oracle_f32_to_bf16_batch.argtypes = [P, I64, P]
    L.oracle_quantize_row_q8_0.argtypes = [P, I64, P, P]
    L.oracle_dequantize_row_q8_0.argtypes = [P, P, I64, P]
    L.oracle_p4_qs_offset.restype = I64
    L.oracle_p4_qs_offset.argtypes = [I64, I64, I64]
    L.oracle_p4_scale_offset.restype = I64
    L.oracle_p4_scale_offset.argtypes = [I64, I64, I64]
    L.oracle_pack_q8_0_p4.restype = I
    L.oracle_pack_q8_0_p4.argtypes = [P, I64, I64, P]
    L.oracle_unpack_q8_0_p4.argtypes = [P, I64, I64, P, P]
    L.oracle_quantize_act_q8_1.argtypes = [P, I64, I64, P, P]
    L.oracle_block_dots.argtypes = [P, P, I64, I64, I64, P]
    L.oracle_expf.restype = ctypes.c_float
    L.oracle_expf.argtypes = [ctypes.c_float]
    for name in ("oracle_silu", "oracle_sigmoid", "oracle_softplus"):
        getattr(L, name).restype = ctypes.c_float
        getattr(L, name).argtypes = [ctypes.c_float]
    L.oracle_linear.argtypes = [P, P, I64, I64, I64, I, I, P]
    L.oracle_linear_colpar.argtypes = [P, P, I64, I64, I64, I, I, P]
    L.oracle_swiglu.argtypes = [P, P, P, I64, I64, I64, I, P, I]
    L.oracle_argmax.restype = I64
    L.oracle_argmax.argtypes = [P, I64]
    L.oracle_embedding.argtypes = [P, I64, P, I64, P]
    L.oracle_max_threads.restype = I
    L.oracle_set_threads.argtypes = [I]
    L.oracle_rmsnorm.argtypes = [P, I64, I64, P, ctypes.c_float, I, P, P]
    L.oracle_gated_rmsnorm.argtypes = [P, P, I64, I64, I64, P, ctypes.c_float, I, P]


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def f32_to_f16_bits(x):
    """floatToHalf (Quantization.cpp:32-37) as uint16 bit patterns."""
    x = _c(np.atleast_1d(x), np.float32)
    out = np.zeros(x.shape, np.uint16)
    lib().oracle_f32_to_f16_batch(_ptr(x), x.size, _ptr(out))
    return out


def f16_bits_to_f32(h):
    """halfToFloat (Quantization.cpp:39-44)."""
    h = _c(np.atleast_1d(h), np.uint16)
    out = np.zeros(h.shape, np.float32)
    lib().oracle_f16_to_f32_batch(_ptr(h), h.size, _ptr(out))
    return out


def quantize_rows_q8_0(w):
    """[N,K] f32 -> (d [N,K/32] uint16 f16 bits, qs [N,K] int8)."""
    w = _c(w, np.float32)
    n, k = w.shape
    d = np.zeros((n, k // QK), np.uint16)
    qs = np.zeros((n, k), np.int8)
    L = lib()
    for r in range(n):
        L.oracle_quantize_row_q8_0(_ptr(w[r]), k, _ptr(d[r]), _ptr(qs[r]))
    return d, qs


def pack_q8_0_p4(w):
    """quantizeTensorQ8_0Packed: [N,K] f32 -> N*K*34/32 bytes (uint8)."""
    w = _c(w, np.float32)
    n, k = w.shape
    out = np.zeros(n * k // QK * 34, np.uint8)
    rc = lib().oracle_pack_q8_0_p4(_ptr(w), n, k, _ptr(out))
    if rc != 0:
        raise ValueError("packed Q8_0 requires rows % 8 == 0 and cols % 32 == 0")
    return out


def unpack_q8_0_p4(p4, n, k):
    p4 = _c(p4, np.uint8)
    qs = np.zeros((n, k), np.int8)
    d = np.zeros((n, k // QK), np.uint16)
    lib().oracle_unpack_q8_0_p4(_ptr(p4), n, k, _ptr(qs), _ptr(d))
    return qs, d


def qs_offset(n, k, cols):
    return lib().oracle_p4_qs_offset(n, k, cols)


def scale_offset(n, b, cols):
    return lib().oracle_p4_scale_offset(n, b, cols)


def quantize_act_q8_1(x):
    """[M,K] f32 -> (qa [M,K] int8, sa [M,K/32] f32)."""
    x = _c(np.atleast_2d(x), np.float32)
    m, k = x.shape
    qa = np.zeros((m, k), np.int8)
    sa = np.zeros((m, k // QK), np.float32)
    lib().oracle_quantize_act_q8_1(_ptr(x), m, k, _ptr(qa), _ptr(sa))
    return qa, sa


def block_dots(qa, p4, n):
    qa = _c(np.atleast_2d(qa), np.int8)
    p4 = _c(p4, np.uint8)
    m, k = qa.shape
    out = np.zeros((m, n, k // QK), np.int32)
    lib().oracle_block_dots(_ptr(qa), _ptr(p4), m, n, k, _ptr(out))
    return out


def _scalar_map(name, v):
    f = getattr(lib(), name)
    v = _c(np.atleast_1d(v), np.float32)
    return np.array([f(float(a)) for a in v.ravel()], np.float32).reshape(v.shape)


def expf(v):
    return _scalar_map("oracle_expf", v)


def silu(v):
    return _scalar_map("oracle_silu", v)


def sigmoid(v):
    return _scalar_map("oracle_sigmoid", v)


def softplus(v):
    return _scalar_map("oracle_softplus", v)


def f32_to_bf16_bits(v):
    """Round to nearest even f32 -> bf16 (raw uint16 bits)."""
    v = _c(np.atleast_1d(v), np.float32)
    out = np.zeros(v.shape, np.uint16)
    lib().oracle_f32_to_bf16_batch(_ptr(v), v.size, _ptr(out))
    return out


def bf16_bits_to_f32(b):
    """Exact bf16 -> f32 widening of raw uint16 bits."""
    b = np.asarray(b, np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def linear(x, p4, n, activation="none", epilogue="scalar", colpar=False):
    """y = act(x . W^T) with W packed q8_0_p4 [n, K]; x [M,K] f32."""
    x = _c(np.atleast_2d(x), np.float32)
    p4 = _c(p4, np.uint8)
    m, k = x.shape
    y = np.zeros((m, n), np.float32)
    fn = lib().oracle_linear_colpar if colpar else lib().oracle_linear
    fn(_ptr(x), _ptr(p4), m, n, k, ACT[activation], EPI[epilogue], _ptr(y))
    return y


def swiglu(x, p4_gate, p4_up, n, epilogue="scalar", colpar=False):
    x = _c(np.atleast_2d(x), np.float32)
    m, k = x.shape
    h = np.zeros((m, n), np.float32)
    lib().oracle_swiglu(_ptr(x), _ptr(_c(p4_gate, np.uint8)),
                        _ptr(_c(p4_up, np.uint8)), m, n, k, EPI[epilogue],
                        _ptr(h), 1 if colpar else 0)
    return h


def argmax(v):
    v = _c(v, np.float32).ravel()
    return int(lib().oracle_argmax(_ptr(v), v.size))


def embedding(tokens, p4, cols):
    t = _c(tokens, np.int64).ravel()
    out = np.zeros((t.size, cols), np.float32)
    lib().oracle_embedding(_ptr(t), t.size, _ptr(_c(p4, np.uint8)), cols,
                           _ptr(out))
    return out


def rmsnorm(x, w, eps, zero_centered=False, out_bf16=False, with_rstd=False):
    """The reference RMSNorm of each row of x [M, H] (f32, or bf16 bit
    patterns as uint16) with weight w [H] (f32 or bf16 bits); the result is
    f32, or its bf16 bits when out_bf16."""
    def widen(a):
        a = np.asarray(a)
        return bf16_bits_to_f32(a) if a.dtype == np.uint16 else a
    x = _c(np.atleast_2d(widen(x)), np.float32)
    w = _c(widen(w).ravel(), np.float32)
    m, h = x.shape
    y = np.zeros((m, h), np.float32)
    r = np.zeros(m, np.float32)
    lib().oracle_rmsnorm(_ptr(x), m, h, _ptr(w), float(np.float32(eps)),
                         1 if zero_centered else 0, _ptr(y), _ptr(r))
    if out_bf16:
        y = f32_to_bf16_bits(y)
    return (y, r) if with_rstd else y


def gated_rmsnorm(x, gate, w, group, eps, gate_activated=False, out_bf16=False):
    """The reference gated RMSNorm of x [M, H] with gate [M, H] (f32, or bf16
    bits as uint16) in groups of `group` values, f32 weight w [group]."""
    def widen(a):
        a = np.asarray(a)
        return bf16_bits_to_f32(a) if a.dtype == np.uint16 else a
    x = _c(np.atleast_2d(widen(x)), np.float32)
    g = _c(np.atleast_2d(widen(gate)), np.float32)
    w = _c(np.asarray(w).ravel(), np.float32)
    m, h = x.shape
    y = np.zeros((m, h), np.float32)
    lib().oracle_gated_rmsnorm(_ptr(x), _ptr(g), m, h, group, _ptr(w),
                               float(np.float32(eps)), 1 if gate_activated else 0, _ptr(y))
    return f32_to_bf16_bits(y) if out_bf16 else y


def max_threads():
    return lib().oracle_max_threads()


def set_threads(n):
    lib().oracle_set_threads(int(n))
