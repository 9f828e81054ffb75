"""SGEMM kernel table on the GPU against the CPU oracle.

Mirrors the verify step of src/bench.cu:259-273 (alpha=0.5, beta=3.0, C
pre-filled, normwise metric, NaN/Inf fail) with the oracle in place of
cuBLAS, plus bit-exactness for the fp32 VALU stages, canary bands around C,
ragged shapes with no fallback, and the beta == 0 write-only contract.
"""
import numpy as np
import pytest

import bmb
import oracle as O
from gpu_util import Guarded, dev, fp32_order_bound, sync

pytestmark = pytest.mark.gpu

SEED_A, SEED_B, SEED_C = 0x12345678, 0x9ABCDEF0, 0x0F0F0F0F  # src/bench.cu:226-228
VALU_IDS = [1, 2, 3, 4, 5, 6, 7, 8]
MFMA_IDS = [9, 10]
SHAPES = [  # (M, N, K)
    (128, 128, 128), (256, 256, 256), (512, 512, 512), (1024, 1024, 1024),
    (1000, 1000, 1000), (100, 70, 33), (65, 65, 65), (130, 260, 60),
    (1, 1, 1), (7, 13, 5), (33, 1, 70), (64, 64, 0),
]


def _inputs(M, N, K):
    A = O.fill_xorshift(M * K, SEED_A).reshape(M, K)
    B = O.fill_xorshift(K * N, SEED_B).reshape(K, N)
    C0 = O.fill_xorshift(M * N, SEED_C).reshape(M, N)
    return A, B, C0


def _run(kid, M, N, K, alpha, beta, A, B, C0):
    dA, dB = dev(A), dev(B)
    gC = Guarded(M * N, fill=C0)
    print("sgemm id=%d M=%d N=%d K=%d alpha=%g beta=%g" % (kid, M, N, K, alpha, beta), flush=True)
    bmb.sgemm(kid, M, N, K, alpha, dA.data_ptr(), dB.data_ptr(), beta, gC.ptr)
    sync("sgemm id %d" % kid)
    assert gC.ok(), "canary band around C overwritten"
    return gC.get().reshape(M, N)


def test_table_contents(gpu):
    ids = [k[0] for k in bmb.kernels()]
    assert ids == list(range(1, 11))
    assert bmb.find_kernel(0) is None and bmb.find_kernel(11) is None


@pytest.mark.parametrize("kid", VALU_IDS)
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "%dx%dx%d" % s)
def test_valu_bit_exact(gpu, kid, shape):
    """fp32 VALU stages equal the sequential-fmaf oracle bit for bit."""
    M, N, K = shape
    A, B, C0 = _inputs(M, N, K)
    got = _run(kid, M, N, K, 0.5, 3.0, A, B, C0)
    want = O.gemm_f32seq(0, 0, M, N, K, 0.5, A, B, 3.0, C0, threads=0)
    assert np.isfinite(got).all()
    assert np.array_equal(got, want), "max |diff| = %g" % np.abs(got - want).max()
    ref = O.gemm_f64(0, 0, M, N, K, 0.5, A, B, 3.0, C0)
    err, bad = O.normwise(got, ref)
    assert bad == 0 and err < bmb.find_kernel(kid)["tol"]


@pytest.mark.parametrize("kid", MFMA_IDS)
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "%dx%dx%d" % s)
def test_mfma_within_tol(gpu, kid, shape):
    M, N, K = shape
    A, B, C0 = _inputs(M, N, K)
    got = _run(kid, M, N, K, 0.5, 3.0, A, B, C0)
    ref = O.gemm_f64(0, 0, M, N, K, 0.5, A, B, 3.0, C0)
    err, bad = O.normwise(got, ref)
    print("id %d %s normwise %.3e" % (kid, shape, err))
    assert bad == 0
    assert err < bmb.find_kernel(kid)["tol"]
    if kid == 9:  # fp32 products: only the summation order differs
        assert err < fp32_order_bound(K)
    if kid == 10:
        _check_bf16x3(got, M, N, K, 0.5, A, B, 3.0, C0)


def _check_bf16x3(got, M, N, K, alpha, A, B, beta, C0):
    """id 10's derived bound: the result is the bf16x3 split's exact value
    (oracle.gemm_bf16x3_f64: three bf16 x bf16 products per term, each exact
    in fp32) up to fp32 accumulation of 3K terms, so it is held to the
    summation-order bound of 3K adds around that value. A dropped or doubled
    cross term or a truncating split misses it by orders of magnitude; the
    split's own error against the exact product (2^-16 |a b| per product at
    most) is printed beside it."""
    want = O.gemm_bf16x3_f64(M, N, K, alpha, A, B, beta, C0)
    err, bad = O.normwise(got, want)
    exact = O.normwise(want.astype(np.float32), O.gemm_f64(0, 0, M, N, K, alpha, A, B, beta, C0))[0]
    print("id 10: normwise %.2e around the bf16x3 value (bound %.2e); split vs exact %.2e"
          % (err, fp32_order_bound(3 * K), exact))
    assert bad == 0 and err < fp32_order_bound(3 * K)


SWEEP_N = [512, 1000, 1024, 1536, 2048, 4096, 4097, 6144, 8192]


@pytest.mark.parametrize("kid", [8, 9, 10])
@pytest.mark.parametrize("n", SWEEP_N)
def test_large_sampled_rows(gpu, kid, n):
    """BASELINE config 2, every size the bench sweeps: alpha = 1, beta = 0.5,
    C pre-filled, the bench's seeds (src/bench.cu:226-228). Rows are
    independent problems, so a row sample of the oracle checks the full-size
    launch (incl. the ragged edge rows of 1000 and 4097)."""
    M = N = K = n
    A, B, C0 = _inputs(M, N, K)
    got = _run(kid, M, N, K, 1.0, 0.5, A, B, C0)
    rows = np.unique(np.r_[0, 1, 127, 128, 255, 256, min(1000, n - 1), n // 2, n - 129, n - 2,
                           n - 1, np.random.default_rng(7).integers(0, n, 8)])
    As = A[rows]
    ref = O.gemm_f64(0, 0, len(rows), N, K, 1.0, As, B, 0.5, C0[rows])
    err, bad = O.normwise(got[rows], ref)
    assert bad == 0 and err < bmb.find_kernel(kid)["tol"]
    if kid == 8:
        want = O.gemm_f32seq(0, 0, len(rows), N, K, 1.0, As, B, 0.5, C0[rows], threads=0)
        assert np.array_equal(got[rows], want)
    if kid == 9:
        assert err < fp32_order_bound(K)
    if kid == 10:
        _check_bf16x3(got[rows], len(rows), N, K, 1.0, As, B, 0.5, C0[rows])


@pytest.mark.parametrize("kid", VALU_IDS + MFMA_IDS)
def test_config1_exact_call(gpu, kid):
    """BASELINE config 1 as the bench times it: N = 1024, alpha = 1, beta = 0
    (C write-only, so it starts as NaN here), the bench's seeds. Its bar is
    normwise 1e-6 against the CPU triple loop, whose fp32 restatement is the
    oracle's sequential fmaf: ids 1-8 equal it bit for bit (error 0). The
    triple loop is itself ~1.5e-6 from the exact product here, so the matrix
    paths, whose summation order differs, are held to their own bounds
    around fp64 instead: id 9 to the fp32 summation bound, id 10 to the
    bf16x3 bound (its split alone is 3.6e-6 from the exact product)."""
    n = 1024
    A, B, _ = _inputs(n, n, n)
    got = _run(kid, n, n, n, 1.0, 0.0, A, B, np.full((n, n), np.nan, np.float32))
    assert np.isfinite(got).all()
    seq = O.gemm_f32seq(0, 0, n, n, n, 1.0, A, B, 0.0, None, threads=0)
    ref = O.gemm_f64(0, 0, n, n, n, 1.0, A, B, 0.0, None)
    err, _ = O.normwise(got, ref)
    e_seq = O.normwise(got, seq)[0]
    print("config 1, id %d: normwise %.2e vs fp64, %.2e vs the CPU triple loop (which is "
          "%.2e from fp64)" % (kid, err, e_seq, O.normwise(seq, ref)[0]))
    assert err < bmb.find_kernel(kid)["tol"]
    if kid in VALU_IDS:
        assert np.array_equal(got, seq) and e_seq <= 1e-6
    elif kid == 9:
        assert err < fp32_order_bound(n)
    else:
        _check_bf16x3(got, n, n, n, 1.0, A, B, 0.0, None)


@pytest.mark.parametrize("kid", [1, 2, 3, 4, 5, 6, 7])
def test_ladder_at_bench_size(gpu, kid):
    """The ladder's fp32 VALU stages at N = 4096 (alpha 1, beta 0.5, C
    pre-filled: the size and call bench.py times them at), bit-exact against
    the sequential-fmaf oracle on a row sample (rows are independent)."""
    n = 4096
    A, B, C0 = _inputs(n, n, n)
    got = _run(kid, n, n, n, 1.0, 0.5, A, B, C0)
    rows = np.unique(np.r_[0, 1, 31, 32, 127, 128, n // 2, n - 33, n - 1,
                           np.random.default_rng(11).integers(0, n, 6)])
    want = O.gemm_f32seq(0, 0, len(rows), n, n, 1.0, A[rows], B, 0.5, C0[rows], threads=0)
    assert np.array_equal(got[rows], want)


@pytest.mark.parametrize("kid", VALU_IDS + MFMA_IDS)
def test_beta_zero_is_write_only(gpu, kid):
    """beta == 0 never reads C: a NaN-filled C gives alpha*A@B."""
    M, N, K = 130, 200, 48
    A, B, _ = _inputs(M, N, K)
    C0 = np.full((M, N), np.nan, np.float32)
    got = _run(kid, M, N, K, 1.25, 0.0, A, B, C0)
    assert np.isfinite(got).all()
    ref = O.gemm_f64(0, 0, M, N, K, 1.25, A, B, 0.0, None)
    err, _ = O.normwise(got, ref)
    assert err < bmb.find_kernel(kid)["tol"]
    if kid in VALU_IDS:
        want = O.gemm_f32seq(0, 0, M, N, K, 1.25, A, B, 0.0, None)
        assert np.array_equal(got, want)


def test_misaligned_pointers(gpu):
    """Pointers off 16-byte alignment take the scalar-load paths."""
    M, N, K = 96, 72, 40
    A, B, C0 = _inputs(M, N, K)
    import torch
    dA = torch.zeros(M * K + 1, dtype=torch.float32, device="cuda")
    dB = torch.zeros(K * N + 1, dtype=torch.float32, device="cuda")
    dC = torch.zeros(M * N + 1, dtype=torch.float32, device="cuda")
    dA[1:].copy_(torch.from_numpy(A.reshape(-1)))
    dB[1:].copy_(torch.from_numpy(B.reshape(-1)))
    for kid in VALU_IDS + MFMA_IDS:
        dC[1:].copy_(torch.from_numpy(C0.reshape(-1)))
        bmb.sgemm(kid, M, N, K, 0.5, dA[1:].data_ptr(), dB[1:].data_ptr(), 3.0, dC[1:].data_ptr())
        sync()
        got = dC[1:].cpu().numpy().reshape(M, N)
        ref = O.gemm_f64(0, 0, M, N, K, 0.5, A, B, 3.0, C0)
        err, bad = O.normwise(got, ref)
        assert bad == 0 and err < bmb.find_kernel(kid)["tol"], kid
        if kid in VALU_IDS:
            assert np.array_equal(got, O.gemm_f32seq(0, 0, M, N, K, 0.5, A, B, 3.0, C0))
