"""ctypes front end of the CPU oracle (oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as
the checker and by bench.py's cpu_baseline leg. The shipped HIP library never
imports or calls it. Each wrapper's reference citation is on the C function in
oracle.h.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")


def build() -> str:
    """Compile oracle.c into liboracle.so (make, in this directory)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    L = ctypes.CDLL(_LIB_PATH)
    i, f, d, sz, ll = (ctypes.c_int, ctypes.c_float, ctypes.c_double,
                       ctypes.c_size_t, ctypes.c_longlong)
    L.orc_fill_xorshift.argtypes = [_f32p, sz, ctypes.c_uint32]
    L.orc_xorshift_stream.argtypes = [_u32p, sz, ctypes.c_uint32]
    L.orc_fill_normal.argtypes = [_f32p, sz, ctypes.c_uint32, f]
    L.orc_gemm_f32seq.argtypes = [i, i, i, i, i, f, _f32p, _f32p, f, _f32p]
    L.orc_gemm_f32seq_mt.argtypes = [i, i, i, i, i, f, _f32p, _f32p, f, _f32p, i]
    L.orc_gemm_f64.argtypes = [i, i, i, i, i, d, _f32p, _f32p, d,
                               ctypes.c_void_p, _f64p]
    L.orc_batched_gemm_f32seq.argtypes = [i, i, i, i, i, i, f, _f32p, ll, _f32p,
                                          ll, f, _f32p, ll]
    L.orc_batched_gemm_f64.argtypes = [i, i, i, i, i, i, d, _f32p, ll, _f32p, ll,
                                       d, ctypes.c_void_p, ll, _f64p]
    L.orc_normwise_f32.argtypes = [_f32p, _f32p, sz, ctypes.POINTER(sz)]
    L.orc_normwise_f32.restype = d
    L.orc_normwise_f64.argtypes = [_f32p, _f64p, sz, ctypes.POINTER(sz)]
    L.orc_normwise_f64.restype = d
    L.orc_attn_fwd_f64.argtypes = [_f32p, i, i, i, i, _f64p, _f64p]
    L.orc_dsum_f64.argtypes = [_f32p, _f32p, i, i, i, i, _f64p]
    L.orc_attn_bwd_f64.argtypes = [_f32p, _f32p, i, i, i, i, _f64p]
    L.orc_attn_fwdbwd_f32.argtypes = [_f32p, _f32p, i, i, i, i, _f32p, _f32p, i]
    L.orc_max_threads.restype = i
    _lib = L
    return L


def _c(a, dtype=np.float32):
    return np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------- fills
def fill_xorshift(n: int, seed: int) -> np.ndarray:
    v = np.empty(n, np.float32)
    lib().orc_fill_xorshift(v, n, seed & 0xFFFFFFFF)
    return v


def xorshift_stream(n: int, seed: int) -> np.ndarray:
    v = np.empty(n, np.uint32)
    lib().orc_xorshift_stream(v, n, seed & 0xFFFFFFFF)
    return v


def fill_normal(n: int, seed: int, std: float = 1.0) -> np.ndarray:
    v = np.empty(n, np.float32)
    lib().orc_fill_normal(v, n, seed & 0xFFFFFFFF, std)
    return v


# ---------------------------------------------------------------- GEMM
def gemm_f32seq(ta, tb, M, N, K, alpha, A, B, beta, C0, threads: int = 1):
    """Returns the new C (a copy); C0 is the C read when beta != 0."""
    C = _c(C0).copy() if C0 is not None else np.zeros(M * N, np.float32)
    C = C.reshape(-1)
    if threads == 1:
        lib().orc_gemm_f32seq(int(ta), int(tb), M, N, K, alpha, _c(A).reshape(-1),
                              _c(B).reshape(-1), beta, C)
    else:
        lib().orc_gemm_f32seq_mt(int(ta), int(tb), M, N, K, alpha,
                                 _c(A).reshape(-1), _c(B).reshape(-1), beta, C,
                                 threads)
    return C.reshape(M, N)


def gemm_f64(ta, tb, M, N, K, alpha, A, B, beta, C0):
    out = np.empty(M * N, np.float64)
    c0 = _c(C0).reshape(-1) if C0 is not None else None
    lib().orc_gemm_f64(int(ta), int(tb), M, N, K, float(alpha),
                       _c(A).reshape(-1), _c(B).reshape(-1), float(beta),
                       c0.ctypes.data if c0 is not None else None, out)
    return out.reshape(M, N)


def batched_gemm_f32seq(ta, tb, batch, M, N, K, alpha, A, sA, B, sB, beta, C0, sC):
    C = _c(C0).reshape(-1).copy()
    lib().orc_batched_gemm_f32seq(int(ta), int(tb), batch, M, N, K, alpha,
                                  _c(A).reshape(-1), sA, _c(B).reshape(-1), sB,
                                  beta, C, sC)
    return C


def batched_gemm_f64(ta, tb, batch, M, N, K, alpha, A, sA, B, sB, beta, C0, sC):
    c0 = _c(C0).reshape(-1)
    out = np.zeros(c0.size, np.float64)
    lib().orc_batched_gemm_f64(int(ta), int(tb), batch, M, N, K, float(alpha),
                               _c(A).reshape(-1), sA, _c(B).reshape(-1), sB,
                               float(beta), c0.ctypes.data, sC, out)
    return out


# ---------------------------------------------------------------- metric
def normwise(got, ref):
    """(max|got-ref| / max|ref|, number of non-finite entries in got)."""
    got = _c(got).reshape(-1)
    bad = ctypes.c_size_t(0)
    if np.asarray(ref).dtype == np.float64:
        r = lib().orc_normwise_f64(got, _c(ref, np.float64).reshape(-1), got.size,
                                   ctypes.byref(bad))
    else:
        r = lib().orc_normwise_f32(got, _c(ref).reshape(-1), got.size,
                                   ctypes.byref(bad))
    return float(r), int(bad.value)


# ---------------------------------------------------------------- attention
def attn_fwd_f64(qkv, B, T, C, NH):
    out = np.empty(B * T * C, np.float64)
    lse = np.empty(B * NH * T, np.float64)
    lib().orc_attn_fwd_f64(_c(qkv).reshape(-1), B, T, C, NH, out, lse)
    return out.reshape(B, T, C), lse.reshape(B, NH, T)


def dsum_f64(dout, out, B, T, C, NH):
    d = np.empty(B * NH * T, np.float64)
    lib().orc_dsum_f64(_c(dout).reshape(-1), _c(out).reshape(-1), B, T, C, NH, d)
    return d.reshape(B, NH, T)


def attn_bwd_f64(qkv, dout, B, T, C, NH):
    d = np.empty(B * T * 3 * C, np.float64)
    lib().orc_attn_bwd_f64(_c(qkv).reshape(-1), _c(dout).reshape(-1), B, T, C, NH, d)
    return d.reshape(B, T, 3 * C)


def attn_fwdbwd_f32(qkv, dout, B, T, C, NH, threads: int = 0):
    out = np.zeros(B * T * C, np.float32)
    dqkv = np.zeros(B * T * 3 * C, np.float32)
    lib().orc_attn_fwdbwd_f32(_c(qkv).reshape(-1), _c(dout).reshape(-1), B, T, C,
                              NH, out, dqkv, threads)
    return out.reshape(B, T, C), dqkv.reshape(B, T, 3 * C)


def max_threads() -> int:
    return int(lib().orc_max_threads())
