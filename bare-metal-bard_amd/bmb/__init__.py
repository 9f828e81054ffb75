"""ctypes binding of the gfx950 HIP library (lib/libbmb.so).

This is the only way Python reaches the kernels: every call goes through the
C-ABI entry points declared in include/kernels.h, include/gemm.h and
include/flash.h. Pointers are raw device addresses (ints); the caller owns the
memory (tests and bench.py use torch tensors purely as device allocations).

There is no fallback: if the library is missing, lib() raises.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.dirname(_HERE)
LIB_PATH = os.path.join(PKG_DIR, "lib", "libbmb.so")

_lib = None

c_int, c_float, c_double, c_bool = ctypes.c_int, ctypes.c_float, ctypes.c_double, ctypes.c_bool
c_ll, c_vp, c_char_p = ctypes.c_longlong, ctypes.c_void_p, ctypes.c_char_p

SGEMM_FN = ctypes.CFUNCTYPE(None, c_int, c_int, c_int, c_float, c_vp, c_vp, c_float, c_vp)


class KernelEntry(ctypes.Structure):
    """Mirror of `struct KernelEntry` (include/kernels.h)."""
    _fields_ = [("id", c_int), ("name", c_char_p), ("fn", c_vp),
                ("note", c_char_p), ("tol", c_double)]


# Every symbol the C headers declare, with its ctypes signature.
_SIGS = {
    # kernels.h
    "find_kernel": (ctypes.POINTER(KernelEntry), [c_int]),
    "sgemm_naive": (None, [c_int, c_int, c_int, c_float, c_vp, c_vp, c_float, c_vp]),
    "sgemm_coalesced": (None, [c_int, c_int, c_int, c_float, c_vp, c_vp, c_float, c_vp]),
    "sgemm_smem": (None, [c_int, c_int, c_int, c_float, c_vp, c_vp, c_float, c_vp]),
    "sgemm_tile1d": (None, [c_int, c_int, c_int, c_float, c_vp, c_vp, c_float, c_vp]),
    "sgemm_tile2d": (None, [c_int, c_int, c_int, c_float, c_vp, c_vp, c_float, c_vp]),
    "sgemm_vectorized": (None, [c_int, c_int, c_int, c_float, c_vp, c_vp, c_float, c_vp]),
    "sgemm_warptile": (None, [c_int, c_int, c_int, c_float, c_vp, c_vp, c_float, c_vp]),
    "sgemm_doublebuffer": (None, [c_int, c_int, c_int, c_float, c_vp, c_vp, c_float, c_vp]),
    "sgemm_tensorcore": (None, [c_int, c_int, c_int, c_float, c_vp, c_vp, c_float, c_vp]),
    "sgemm_mfma_bf16x3": (None, [c_int, c_int, c_int, c_float, c_vp, c_vp, c_float, c_vp]),
    "bmb_last_error": (c_int, []),
    # gemm.h
    "gemm": (None, [c_bool, c_bool, c_int, c_int, c_int, c_float, c_vp, c_vp,
                    c_float, c_vp, c_vp]),
    "batched_gemm": (None, [c_bool, c_bool, c_int, c_int, c_int, c_int, c_float,
                            c_vp, c_ll, c_vp, c_ll, c_float, c_vp, c_ll, c_vp]),
    # flash.h
    "flash_attention_forward": (None, [c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int]),
    "flash_attention_backward": (None, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_int,
                                        c_int, c_int, c_int]),
    "flash_num_configs": (c_int, []),
    "flash_config_name": (c_char_p, [c_int]),
    "flash_default_config": (c_int, []),
    "flash_attention_forward_cfg": (c_bool, [c_int, c_vp, c_vp, c_vp, c_int, c_int,
                                             c_int, c_int]),
    "flash_num_bwd_configs": (c_int, []),
    "flash_bwd_config_name": (c_char_p, [c_int]),
    "flash_default_bwd_config": (c_int, []),
    "flash_attention_backward_cfg": (c_bool, [c_int, c_vp, c_vp, c_vp, c_vp, c_vp,
                                              c_vp, c_int, c_int, c_int, c_int]),
}
# Data symbols (kernels.h).
DATA_SYMBOLS = ("KERNELS", "NUM_KERNELS")


def build(jobs: int = 8) -> str:
    """Compile every HIP source for gfx950 into lib/libbmb.so (make)."""
    subprocess.run(["make", "-s", "-j%d" % jobs, "-C", PKG_DIR], check=True)
    return LIB_PATH


def lib():
    """Load lib/libbmb.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            "bare-metal-bard_amd: %s is missing; build it first "
            "(python -c 'import __graft_entry__ as g; g.build()')" % LIB_PATH)
    L = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in _SIGS.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def exported_symbols():
    return list(_SIGS) + list(DATA_SYMBOLS)


def last_error() -> int:
    return int(lib().bmb_last_error())


def check(what: str = "launch") -> None:
    e = last_error()
    if e != 0:
        raise RuntimeError("%s failed: hipError %d" % (what, e))


# ------------------------------------------------------------ kernel table
def kernels():
    """List of (id, name, note, tol) from the exported KERNELS table."""
    L = lib()
    n = c_int.in_dll(L, "NUM_KERNELS").value
    table = (KernelEntry * n).in_dll(L, "KERNELS")
    return [(e.id, e.name.decode(), e.note.decode(), e.tol) for e in table]


def find_kernel(kid: int):
    p = lib().find_kernel(kid)
    if not p:
        return None
    e = p.contents
    return {"id": e.id, "name": e.name.decode(), "note": e.note.decode(),
            "tol": e.tol, "fn": SGEMM_FN(e.fn)}


def sgemm(kid: int, M, N, K, alpha, A, B, beta, C) -> None:
    """Calls KERNELS[id].fn (the reference's ke->fn(...), src/bench.cu:265)."""
    ent = find_kernel(kid)
    if ent is None:
        raise KeyError("no kernel with id %d" % kid)
    ent["fn"](M, N, K, alpha, A, B, beta, C)


# ------------------------------------------------------------ gemm.h
def gemm(ta, tb, M, N, K, alpha, A, B, beta, C, stream=0) -> None:
    lib().gemm(bool(ta), bool(tb), M, N, K, alpha, A, B, beta, C, stream or None)


def batched_gemm(ta, tb, batch, M, N, K, alpha, A, sA, B, sB, beta, C, sC,
                 stream=0) -> None:
    lib().batched_gemm(bool(ta), bool(tb), batch, M, N, K, alpha, A, sA, B, sB,
                       beta, C, sC, stream or None)


# ------------------------------------------------------------ flash.h
def flash_forward(out, lse, qkv, B, T, C, NH) -> None:
    lib().flash_attention_forward(out, lse, qkv, B, T, C, NH)


def flash_backward(dqkv, dsum, dout, qkv, out, lse, B, T, C, NH) -> None:
    lib().flash_attention_backward(dqkv, dsum, dout, qkv, out, lse, B, T, C, NH)


def flash_forward_cfg(cfg, out, lse, qkv, B, T, C, NH) -> bool:
    return bool(lib().flash_attention_forward_cfg(cfg, out, lse, qkv, B, T, C, NH))


def flash_backward_cfg(cfg, dqkv, dsum, dout, qkv, out, lse, B, T, C, NH) -> bool:
    return bool(lib().flash_attention_backward_cfg(cfg, dqkv, dsum, dout, qkv, out,
                                                   lse, B, T, C, NH))


def flash_configs():
    L = lib()
    return [L.flash_config_name(i).decode() for i in range(L.flash_num_configs())]


def flash_bwd_configs():
    L = lib()
    return [L.flash_bwd_config_name(i).decode() for i in range(L.flash_num_bwd_configs())]


def flash_default_config() -> int:
    return int(lib().flash_default_config())


def flash_default_bwd_config() -> int:
    return int(lib().flash_default_bwd_config())
