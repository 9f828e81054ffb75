"""Device-memory helpers for the GPU parity tests.

torch is used only to allocate device memory and copy bytes; every
computation under test goes through the C-ABI of lib/libbmb.so.
"""
import numpy as np
import torch

import bmb

GUARD = 64            # floats of canary on each side of an output buffer
CANARY = 0x7FA5A5A5   # a quiet-NaN bit pattern no kernel produces
POISON = 0x7F7F7F7F   # 3.39e38: what the reference test poisons outputs with


def fp32_order_bound(K):
    """Normwise bound for an fp32 result whose products are exact and whose
    only difference from the exact sum is fp32 summation order: a random-walk
    rounding model, 4 * sqrt(K) * 2^-24, plus a few ulp for the alpha/beta
    epilogue. Reduced-precision products (TF32: 2^-11, bf16: 2^-8 relative
    per product) exceed it by orders of magnitude."""
    u = 2.0 ** -24
    return 4.0 * np.sqrt(max(K, 1)) * u + 4.0 * u


def bf16x3_err(got, ta, tb, M, N, K, alpha, A, B, beta, C0):
    """Normwise error of gemm()'s result against the exact value of its
    bf16x3 split (oracle.gemm_bf16x3_f64: three exact bf16 x bf16 products per
    term), with the bound it is held to: fp32 summation of 3K terms
    (fp32_order_bound(3K)). A dropped or doubled cross term, or a truncating
    split, misses it by orders of magnitude."""
    import oracle as O
    Aop = np.ascontiguousarray(A.reshape(K, M).T if ta else A.reshape(M, K))
    Bop = np.ascontiguousarray(B.reshape(N, K).T if tb else B.reshape(K, N))
    want = O.gemm_bf16x3_f64(M, N, K, alpha, Aop, Bop, beta, C0)
    err, bad = O.normwise(np.asarray(got).reshape(M, N), want)
    return (err if bad == 0 else float("inf")), fp32_order_bound(3 * K)


def dev(a):
    """Host numpy array -> device float32 tensor (contiguous copy)."""
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to("cuda")


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def sync(what="kernel"):
    torch.cuda.synchronize()
    bmb.check(what)


class Guarded:
    """A device float32 buffer with canary bands on both sides.

    ptr points at the payload (16-byte aligned); ok() checks the bands."""

    def __init__(self, n, fill=None, poison=False):
        self.n = n
        self.buf = torch.empty(n + 2 * GUARD, dtype=torch.float32, device="cuda")
        self.buf.view(torch.int32).fill_(CANARY - (1 << 32) if CANARY >= 1 << 31 else CANARY)
        payload = self.buf[GUARD:GUARD + n]
        if fill is not None:
            payload.copy_(torch.from_numpy(np.ascontiguousarray(fill, dtype=np.float32).reshape(-1)))
        elif poison:
            payload.view(torch.int32).fill_(POISON)
        self.payload = payload

    @property
    def ptr(self):
        return self.payload.data_ptr()

    def get(self):
        return host(self.payload)

    def ok(self):
        h = host(self.buf.view(torch.int32))
        c = np.int32(np.uint32(CANARY).view(np.int32))
        return bool((h[:GUARD] == c).all() and (h[GUARD + self.n:] == c).all())


# ---- raw device pointers owned by the library (the GPT struct's buffers)
_hip = None


def _hiprt():
    """The HIP runtime already loaded in this process (torch and libbmb share
    one libamdhip64.so.7)."""
    global _hip
    if _hip is None:
        import ctypes
        _hip = ctypes.CDLL("libamdhip64.so.7")
        _hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                   ctypes.c_int]
        _hip.hipMemcpy.restype = ctypes.c_int
    return _hip


def d2h(ptr, n, dtype=np.float32):
    """Copies n elements at device address ptr into a new host array."""
    out = np.empty(n, dtype)
    if n:
        e = _hiprt().hipMemcpy(out.ctypes.data, ptr, out.nbytes, 2)
        assert e == 0, "hipMemcpy D2H failed: %d" % e
    return out


def h2d(ptr, a):
    """Copies host array a to device address ptr."""
    a = np.ascontiguousarray(a)
    if a.size:
        e = _hiprt().hipMemcpy(ptr, a.ctypes.data, a.nbytes, 1)
        assert e == 0, "hipMemcpy H2D failed: %d" % e
