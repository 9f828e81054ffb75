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
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_szp = np.ctypeslib.ndpointer(dtype=np.uintp, flags="C_CONTIGUOUS")


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
    L.orc_encoder_fwd.argtypes = [_f64p, _i32p, _f64p, _f64p, i, i, i]
    L.orc_encoder_bwd.argtypes = [_f64p, _f64p, _f64p, _i32p, i, i, i]
    L.orc_layernorm_fwd.argtypes = [_f64p, _f64p, _f64p, _f64p, _f64p, _f64p, i, i]
    L.orc_layernorm_bwd.argtypes = [_f64p, _f64p, _f64p, _f64p, _f64p, _f64p, _f64p,
                                    _f64p, i, i]
    L.orc_gelu_fwd.argtypes = [_f64p, _f64p, sz]
    L.orc_gelu_bwd.argtypes = [_f64p, _f64p, _f64p, sz]
    L.orc_bias_bwd.argtypes = [_f64p, _f64p, i, i]
    L.orc_softmax_xent_fwd.argtypes = [_f64p, _f64p, _f64p, _i32p, i, i, i]
    L.orc_xent_bwd.argtypes = [_f64p, _f64p, _i32p, i, i, i, d]
    L.orc_adamw_f32.argtypes = [_f32p, _f32p, _f32p, _f32p, sz, f, f, f, f, f, i, f]
    L.orc_gpt_param_sizes.argtypes = [_szp, _i32p]
    L.orc_gpt_forward_backward.argtypes = [_i32p, i, i, _f64p, _i32p, _i32p,
                                           ctypes.c_void_p, ctypes.c_void_p,
                                           ctypes.c_void_p]
    L.orc_gpt_forward_backward.restype = d
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
def bf16_rne(x) -> np.ndarray:
    """fp32 -> the nearest bfloat16 (ties to even), returned as fp32 values.
    Finite inputs only. Rounds the 32-bit pattern at bit 16: add 0x7FFF plus
    the lowest kept bit, then clear the low half."""
    u = _c(x).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return r.astype(np.uint32).view(np.float32)


# The largest float that rounds to a finite bfloat16 (bits 0x7F7F7FFF).
BF16_FINITE_MAX = float(np.array(0x7F7F7FFF, np.uint32).view(np.float32))


def bf16x3_split(x):
    """(hi, lo) of the bf16x3 scheme of KERNELS id 10 and gemm()
    (csrc/sgemm_bf16x3.hip split4): hi = bf16(clamp(x, +-BF16_FINITE_MAX)),
    lo = bf16(x - hi). x - hi is exact in fp32 for every finite x (hi holds
    x's leading bits; above BF16_FINITE_MAX hi is bf16's largest finite
    value, within a factor 2 of x); an infinite x gives (+-3.39e38, +-inf)."""
    x = _c(x)
    hi = bf16_rne(np.clip(x, np.float32(-BF16_FINITE_MAX), np.float32(BF16_FINITE_MAX)))
    with np.errstate(invalid="ignore", over="ignore"):
        lo = bf16_rne(x - hi)
    return hi, lo


def gemm_bf16x3_f64(M, N, K, alpha, A, B, beta, C0):
    """What KERNELS id 10 computes, with exact sums: alpha * (Ah Bh + Ah Bl +
    Al Bh) + beta * C0 in fp64 (row-major A M x K, B K x N). Products of two
    bfloat16 are exact in fp64 and the fp64 sums are ~K 2^-53 from exact, so
    the GPU result differs from this only by its fp32 accumulation."""
    Ah, Al = (v.astype(np.float64).reshape(M, K) for v in bf16x3_split(A))
    Bh, Bl = (v.astype(np.float64).reshape(K, N) for v in bf16x3_split(B))
    out = alpha * (Ah @ Bh + Ah @ Bl + Al @ Bh)
    if beta != 0:
        out += beta * _c(C0, np.float64).reshape(M, N)
    return out


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


# ---------------------------------------------------------------- nn ops
def _d(a):
    return np.ascontiguousarray(a, dtype=np.float64).reshape(-1)


def _i(a):
    return np.ascontiguousarray(a, dtype=np.int32).reshape(-1)


def encoder_fwd(tokens, wte, wpe, B, T, C):
    out = np.empty(B * T * C, np.float64)
    lib().orc_encoder_fwd(out, _i(tokens), _d(wte), _d(wpe), B, T, C)
    return out.reshape(B * T, C)


def encoder_bwd(dwte0, dwpe0, dout, tokens, B, T, C):
    dwte, dwpe = _d(dwte0).copy(), _d(dwpe0).copy()
    lib().orc_encoder_bwd(dwte, dwpe, _d(dout), _i(tokens), B, T, C)
    return dwte, dwpe


def layernorm_fwd(inp, w, b, N, C):
    out = np.empty(N * C, np.float64)
    mean = np.empty(N, np.float64)
    rstd = np.empty(N, np.float64)
    lib().orc_layernorm_fwd(out, mean, rstd, _d(inp), _d(w), _d(b), N, C)
    return out.reshape(N, C), mean, rstd


def layernorm_bwd(dinp0, dw0, db0, dout, inp, w, mean, rstd, N, C):
    dinp, dw, db = _d(dinp0).copy(), _d(dw0).copy(), _d(db0).copy()
    lib().orc_layernorm_bwd(dinp, dw, db, _d(dout), _d(inp), _d(w), _d(mean), _d(rstd),
                            N, C)
    return dinp.reshape(N, C), dw, db


def gelu_fwd(x):
    x = _d(x)
    out = np.empty_like(x)
    lib().orc_gelu_fwd(out, x, x.size)
    return out


def gelu_bwd(x, dout):
    x = _d(x)
    out = np.empty_like(x)
    lib().orc_gelu_bwd(out, x, _d(dout), x.size)
    return out


def bias_bwd(dbias0, dout, N, C):
    db = _d(dbias0).copy()
    lib().orc_bias_bwd(db, _d(dout), N, C)
    return db


def softmax_xent_fwd(logits, targets, N, V, Vp):
    probs = np.empty(N * Vp, np.float64)
    losses = np.empty(N, np.float64)
    lib().orc_softmax_xent_fwd(probs, losses, _d(logits), _i(targets), N, V, Vp)
    return probs.reshape(N, Vp), losses


def xent_bwd(probs, targets, N, V, Vp, scale):
    out = np.empty(N * Vp, np.float64)
    lib().orc_xent_bwd(out, _d(probs), _i(targets), N, V, Vp, float(scale))
    return out.reshape(N, Vp)


def adamw_f32(params, grads, m, v, lr, beta1, beta2, eps, wd, step, grad_scale):
    """Returns updated copies (params, m, v)."""
    p = _c(params).reshape(-1).copy()
    mm = _c(m).reshape(-1).copy()
    vv = _c(v).reshape(-1).copy()
    lib().orc_adamw_f32(p, _c(grads).reshape(-1), mm, vv, p.size, lr, beta1, beta2, eps,
                        wd, int(step), grad_scale)
    return p, mm, vv


# ---------------------------------------------------------------- GPT
PARAM_NAMES = ("wte", "wpe", "ln1w", "ln1b", "qkvw", "qkvb", "attprojw", "attprojb",
               "ln2w", "ln2b", "fcw", "fcb", "fcprojw", "fcprojb", "lnfw", "lnfb")


def gpt_param_sizes(cfg):
    """cfg = (max_seq_len, vocab_size, padded_vocab, n_layer, n_head, n_embd)."""
    s = np.zeros(16, np.uintp)
    lib().orc_gpt_param_sizes(s, _i(cfg))
    return [int(x) for x in s]


def gpt_forward_backward(cfg, B, T, params, tokens, targets, grads=True, logits=False):
    """fp64 GPT forward (+ backward). Returns (mean_loss, losses, grads|None,
    logits|None); params is the flat parameter vector (widened to fp64)."""
    p = _d(params)
    n = sum(gpt_param_sizes(cfg))
    assert p.size == n, (p.size, n)
    N = B * T
    losses = np.empty(N, np.float64)
    g = np.empty(n, np.float64) if grads else None
    lg = np.empty(N * cfg[2], np.float64) if logits else None
    loss = lib().orc_gpt_forward_backward(
        _i(cfg), B, T, p, _i(tokens), _i(targets), losses.ctypes.data,
        g.ctypes.data if g is not None else None,
        lg.ctypes.data if lg is not None else None)
    return float(loss), losses, g, (lg.reshape(N, cfg[2]) if lg is not None else None)
