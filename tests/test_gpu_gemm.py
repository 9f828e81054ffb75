"""gemm() and batched_gemm() on the GPU against the CPU oracle.

Mirrors tools/test_gemm.cu: the same 10 shapes x 4 transpose cases with
alpha=0.75, beta=1.25 (test_gemm.cu:51-62,87), the same buffers reinterpreted
for the transposed cases (:81-83), the 4 batched shapes with alpha=0.5,
beta=2 (:123-128,146), normwise error < 1e-4 (:107,170) -- against the fp64
oracle instead of cuBLAS. Also the GPT-2-small training shapes (BT=8192,
C=768) through a row sample.
"""
import numpy as np
import pytest

import bmb
import oracle as O
from gpu_util import Guarded, dev, fp32_order_bound, sync

pytestmark = pytest.mark.gpu

SHAPES = [
    (128, 128, 128), (256, 512, 128), (4096, 384, 384), (4096, 1536, 384),
    (4096, 384, 1536), (384, 384, 4096), (4096, 128, 384), (100, 70, 33),
    (65, 65, 65), (130, 260, 60),
]
TRANS = [(False, False), (True, False), (False, True), (True, True)]


def _tag(t):
    return ("T" if t[0] else "N") + ("T" if t[1] else "N")


@pytest.mark.parametrize("trans", TRANS, ids=_tag)
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "%dx%dx%d" % s)
def test_gemm_shapes(gpu, shape, trans):
    M, N, K = shape
    ta, tb = trans
    A = O.fill_xorshift(M * K, 0x1234)  # stored M x K, or K x M when ta
    B = O.fill_xorshift(K * N, 0x9ABC)
    C0 = O.fill_xorshift(M * N, 0x5555)
    dA, dB = dev(A), dev(B)
    gC = Guarded(M * N, fill=C0)
    print("gemm %s M=%d N=%d K=%d" % (_tag(trans), M, N, K), flush=True)
    bmb.gemm(ta, tb, M, N, K, 0.75, dA.data_ptr(), dB.data_ptr(), 1.25, gC.ptr)
    sync("gemm")
    assert gC.ok()
    ref = O.gemm_f64(ta, tb, M, N, K, 0.75, A, B, 1.25, C0)
    err, bad = O.normwise(gC.get(), ref)
    print("  normwise %.2e" % err)
    assert bad == 0 and err < 1e-4
    assert err < fp32_order_bound(K)  # fp32 products; only the summation order differs


BSHAPES = [(96, 256, 256, 64), (96, 256, 64, 256), (24, 64, 64, 32), (8, 100, 48, 33)]


@pytest.mark.parametrize("trans", TRANS, ids=_tag)
@pytest.mark.parametrize("bshape", BSHAPES, ids=lambda s: "b%d_%dx%dx%d" % s)
def test_batched_gemm(gpu, bshape, trans):
    batch, M, N, K = bshape
    ta, tb = trans
    eA, eB, eC = M * K, K * N, M * N
    A = O.fill_xorshift(eA * batch, 0x2222)
    B = O.fill_xorshift(eB * batch, 0x3333)
    C0 = O.fill_xorshift(eC * batch, 0x4444)
    dA, dB = dev(A), dev(B)
    gC = Guarded(eC * batch, fill=C0)
    print("batched %s batch=%d M=%d N=%d K=%d" % (_tag(trans), batch, M, N, K), flush=True)
    bmb.batched_gemm(ta, tb, batch, M, N, K, 0.5, dA.data_ptr(), eA, dB.data_ptr(), eB,
                     2.0, gC.ptr, eC)
    sync("batched_gemm")
    assert gC.ok()
    ref = O.batched_gemm_f64(ta, tb, batch, M, N, K, 0.5, A, eA, B, eB, 2.0, C0, eC)
    err, bad = O.normwise(gC.get(), ref)
    assert bad == 0 and err < 1e-4


GPT = [  # (M, N, K, ta, tb, beta): forward NT, backward dX = NN, dW = TN (beta 1)
    (8192, 2304, 768, False, True, 0.0), (8192, 768, 768, False, True, 0.0),
    (8192, 3072, 768, False, True, 0.0), (8192, 768, 3072, False, True, 0.0),
    (8192, 50257, 768, False, True, 0.0),
    (8192, 768, 2304, False, False, 0.0), (8192, 768, 3072, False, False, 0.0),
    (2304, 768, 8192, True, False, 1.0), (768, 3072, 8192, True, False, 1.0),
    (50257, 768, 8192, True, False, 1.0),
]


@pytest.mark.parametrize("g", GPT, ids=lambda g: "%dx%dx%d_%s" % (g[0], g[1], g[2], _tag(g[3:5])))
def test_gpt_training_shapes(gpu, g):
    """BASELINE config 3 shapes (weights N(0, 0.02^2), activations N(0, 1)),
    checked on a sample of output rows (rows are independent problems)."""
    M, N, K, ta, tb, beta = g
    A = O.fill_normal(M * K, 0xA11CE, 1.0)
    B = O.fill_normal(K * N, 0xB0B, 0.02)
    C0 = O.fill_normal(M * N, 0xC0C0, 1.0) if beta != 0 else None
    dA, dB = dev(A), dev(B)
    import torch
    dC = dev(C0) if C0 is not None else torch.empty(M * N, device="cuda")
    print("gpt gemm %s M=%d N=%d K=%d beta=%g" % (_tag((ta, tb)), M, N, K, beta), flush=True)
    bmb.gemm(ta, tb, M, N, K, 1.0, dA.data_ptr(), dB.data_ptr(), beta, dC.data_ptr())
    sync("gemm")
    got = dC.cpu().numpy().reshape(M, N)
    rows = np.unique(np.r_[0, 1, 255, 256, M // 2, M - 1, np.random.default_rng(3).integers(0, M, 6)])
    # op(A) restricted to the sampled rows, as a plain M' x K matrix.
    Aop = (A.reshape(K, M).T if ta else A.reshape(M, K))[rows]
    c0 = C0.reshape(M, N)[rows] if C0 is not None else None
    ref = O.gemm_f64(False, tb, len(rows), N, K, 1.0, np.ascontiguousarray(Aop), B, beta, c0)
    err, bad = O.normwise(got[rows], ref)
    print("  normwise %.2e" % err)
    assert bad == 0 and err < 1e-4
