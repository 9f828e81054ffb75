"""ctypes binding of the gfx950 HIP library (lib/libbmb.so).

This is the only way Python reaches the kernels: every call goes through the
C-ABI entry points declared in include/kernels.h, gemm.h, flash.h,
attention.h, nn.h and gpt.h. Pointers are raw device addresses (ints); the
caller owns the memory (tests and bench.py use torch tensors purely as device
allocations), except for the GPT struct, whose buffers gpt_alloc makes.

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


PARAM_NAMES = ("wte", "wpe", "ln1w", "ln1b", "qkvw", "qkvb", "attprojw", "attprojb",
               "ln2w", "ln2b", "fcw", "fcb", "fcprojw", "fcprojb", "lnfw", "lnfb")
ACT_NAMES = ("encoded", "ln1", "ln1_mean", "ln1_rstd", "qkv", "qkvr", "att", "atty",
             "attproj", "lse", "residual2", "ln2", "ln2_mean", "ln2_rstd", "fch", "fch_gelu",
             "fcproj", "residual3", "lnf", "lnf_mean", "lnf_rstd", "logits", "probs", "losses")
GRAD_ACT_NAMES = ("dres", "dln1", "dln2", "datty", "dqkv", "dqkvr", "datt", "dsum", "dfch",
                  "dfch_gelu", "dlogits", "dlnf")
c_size_t = ctypes.c_size_t


class GPTConfig(ctypes.Structure):
    """Mirror of `struct GPTConfig` (include/gpt.h)."""
    _fields_ = [(n, c_int) for n in ("max_seq_len", "vocab_size", "padded_vocab", "n_layer",
                                     "n_head", "n_embd")]


class Parameters(ctypes.Structure):
    _fields_ = [(n, c_vp) for n in PARAM_NAMES]


class Activations(ctypes.Structure):
    _fields_ = [(n, c_vp) for n in ACT_NAMES]


class Gradients(ctypes.Structure):
    _fields_ = [(n, c_vp) for n in GRAD_ACT_NAMES]


class GPT(ctypes.Structure):
    """Mirror of `struct GPT` (include/gpt.h)."""
    _fields_ = [("config", GPTConfig), ("use_flash", c_bool), ("B", c_int), ("T", c_int),
                ("params", Parameters), ("grads", Parameters),
                ("psize", c_size_t * 16), ("num_params", c_size_t),
                ("params_mem", c_vp), ("grads_mem", c_vp), ("m_mem", c_vp), ("v_mem", c_vp),
                ("acts", Activations), ("gr", Gradients),
                ("acts_mem", c_vp), ("grads_act_mem", c_vp),
                ("num_acts", c_size_t), ("num_grad_acts", c_size_t),
                ("d_tokens", c_vp), ("d_targets", c_vp)]


_GPTP = ctypes.POINTER(GPT)

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
    "gemm_noalloc": (c_int, [c_bool, c_bool, c_int, c_int, c_int, c_float, c_vp, c_vp,
                             c_float, c_vp, c_vp]),
    "gemm_set_math": (c_int, [c_int]),
    "gemm_get_math": (c_int, []),
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
    # attention.h
    "attention_forward": (None, [c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int]),
    "attention_backward": (None, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int,
                                  c_int, c_int]),
    # nn.h
    "encoder_forward": (None, [c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int]),
    "encoder_backward": (None, [c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int]),
    "layernorm_forward": (None, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int]),
    "layernorm_backward": (None, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_int,
                                  c_int]),
    "gelu_forward": (None, [c_vp, c_vp, c_int]),
    "gelu_backward": (None, [c_vp, c_vp, c_vp, c_int]),
    "residual_forward": (None, [c_vp, c_vp, c_vp, c_int]),
    "add_inplace": (None, [c_vp, c_vp, c_int]),
    "bias_forward": (None, [c_vp, c_vp, c_int, c_int]),
    "bias_backward": (None, [c_vp, c_vp, c_int, c_int]),
    "softmax_crossentropy_forward": (None, [c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int]),
    "crossentropy_softmax_backward": (None, [c_vp, c_vp, c_vp, c_int, c_int, c_int,
                                             c_float]),
    "adamw_update": (None, [c_vp, c_vp, c_vp, c_vp, c_int, c_float, c_float, c_float,
                            c_float, c_float, c_int, c_float]),
    "grad_global_norm": (c_float, [c_vp, c_int]),
    "zero_buffer": (None, [c_vp, c_size_t]),
    "reduce_mean": (c_float, [c_vp, c_int]),
    # gpt.h
    "param_sizes": (None, [ctypes.POINTER(c_size_t), ctypes.POINTER(GPTConfig)]),
    "gpt_alloc": (None, [_GPTP]),
    "gpt_init": (None, [_GPTP, ctypes.c_uint]),
    "gpt_forward": (c_float, [_GPTP, c_vp, c_vp]),
    "gpt_backward": (None, [_GPTP]),
    "gpt_free": (None, [_GPTP]),
    "gpt_save_checkpoint": (c_int, [_GPTP, c_char_p, c_char_p, c_int]),
    "gpt_load_checkpoint": (c_int, [_GPTP, c_char_p, c_char_p, c_int,
                                    ctypes.POINTER(c_int)]),
}
# Data symbols (kernels.h, gpt.h).
DATA_SYMBOLS = ("KERNELS", "NUM_KERNELS", "PARAM_NAMES")


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


GEMM_MATH_BF16X3, GEMM_MATH_FP32 = 0, 1  # include/gemm.h


def gemm_set_math(math: int) -> int:
    """Selects gemm()'s arithmetic for the process; returns the previous mode."""
    return int(lib().gemm_set_math(int(math)))


def gemm_get_math() -> int:
    return int(lib().gemm_get_math())


class gemm_math:
    """`with bmb.gemm_math(bmb.GEMM_MATH_FP32): ...` runs the block in that
    mode and restores the previous one."""

    def __init__(self, math):
        self.math, self.prev = math, None

    def __enter__(self):
        self.prev = gemm_set_math(self.math)
        if self.prev < 0:
            raise ValueError("unknown gemm math mode %r" % (self.math,))
        return self

    def __exit__(self, *exc):
        gemm_set_math(self.prev)
        return False


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


# ------------------------------------------------------------ attention.h / nn.h
def call(name, *args):
    """Calls the C entry point `name` with raw arguments (device pointers as
    ints); returns its result."""
    return getattr(lib(), name)(*args)


def param_names():
    """PARAM_NAMES as exported by the library (include/gpt.h)."""
    arr = (c_char_p * 16).in_dll(lib(), "PARAM_NAMES")
    return [x.decode() for x in arr]


def param_sizes(cfg):
    s = (c_size_t * 16)()
    c = GPTConfig(*cfg)
    lib().param_sizes(s, ctypes.byref(c))
    return [int(x) for x in s]


class Model:
    """Owns one `struct GPT` (include/gpt.h) and forwards to the C entry points.

    cfg = (max_seq_len, vocab_size, padded_vocab, n_layer, n_head, n_embd).
    tokens/targets are host int32 arrays of B*T ids, as gpt_forward takes them.
    """

    def __init__(self, cfg, B, T, use_flash=True):
        self.g = GPT()
        self.g.config = GPTConfig(*cfg)
        self.g.use_flash = bool(use_flash)
        self.g.B, self.g.T = B, T
        lib().gpt_alloc(ctypes.byref(self.g))
        self._alive = True

    def init(self, seed):
        lib().gpt_init(ctypes.byref(self.g), seed)

    def forward(self, tokens, targets=None):
        import numpy as np
        tok = np.ascontiguousarray(tokens, dtype=np.int32).reshape(-1)
        assert tok.size == self.g.B * self.g.T
        tgt = None
        if targets is not None:
            tgt = np.ascontiguousarray(targets, dtype=np.int32).reshape(-1)
            assert tgt.size == tok.size
        return float(lib().gpt_forward(ctypes.byref(self.g), tok.ctypes.data,
                                       tgt.ctypes.data if tgt is not None else None))

    def backward(self):
        lib().gpt_backward(ctypes.byref(self.g))

    def free(self):
        if self._alive:
            lib().gpt_free(ctypes.byref(self.g))
            self._alive = False

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
