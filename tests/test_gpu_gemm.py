"""gemm() and batched_gemm() on the GPU against the CPU oracle.

Mirrors tools/test_gemm.cu: the same 10 shapes x 4 transpose cases with
alpha=0.75, beta=1.25 (test_gemm.cu:51-62,87), the same buffers reinterpreted
for the transposed cases (:81-83), the 4 batched shapes with alpha=0.5,
beta=2 (:123-128,146), normwise error < 1e-4 (:107,170) -- against the fp64
oracle instead of cuBLAS. Also the GPT-2-small training shapes (BT=8192,
C=768) through a row sample.

gemm() runs on bf16x3 matrix-core products (each fp32 operand split into
bfloat16 hi + lo, three products per term, fp32 accumulation): besides the
reference's 1e-4 it is held to the summation bound around the split's exact
value (gpu_util.bf16x3_err). batched_gemm() keeps fp32 MFMA products and the
fp32 summation-order bound.
"""
import numpy as np
import pytest

import bmb
import oracle as O
from gpu_util import Guarded, bf16x3_err, dev, fp32_order_bound, sync

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
    e3, bound = bf16x3_err(gC.get(), ta, tb, M, N, K, 0.75, A, B, 1.25, C0)
    print("  normwise %.2e; around the bf16x3 value %.2e (bound %.2e)" % (err, e3, bound))
    assert bad == 0 and err < 1e-4
    assert e3 < bound


# Tiles that lie wholly inside C with K one to four k-tiles deep: the
# interior path's unguarded loads and its prefetch index, clamped to the last
# k-tile, on every tile size the planner can pick (4096^2 takes 256x256).
# Small-integer entries (|a|, |b| <= 8, K <= 64) make every fp32 sum exact,
# so the result must equal the exact product bit for bit. 1030 x 771 has rows
# of stored operands that are not whole 16-byte chunks (interior tiles with
# unaligned rows, plus ragged edge tiles). K = 40 and 63 end in a partial
# k-tile: interior tiles guard only that k-tile's loads.
SHORT_K = [(1024, 1024, 16), (512, 768, 32), (2048, 256, 48), (256, 256, 32),
           (4096, 4096, 32), (768, 192, 64), (1030, 771, 48), (1024, 1024, 40),
           (2048, 512, 63), (4096, 4096, 8)]


# off = 1: both operands start one float past a 16-byte boundary, so the
# kernels without aligned 128-bit loads run the same interior tiles with
# 128-bit loads from 4-byte aligned addresses.
@pytest.mark.parametrize("off", [0, 1], ids=["aligned", "off1"])
@pytest.mark.parametrize("trans", TRANS, ids=_tag)
@pytest.mark.parametrize("shape", SHORT_K, ids=lambda s: "%dx%dx%d" % s)
def test_interior_short_k_exact(gpu, shape, trans, off):
    import torch
    M, N, K = shape
    ta, tb = trans
    r = np.random.default_rng(M + 7 * N + 31 * K)
    A = r.integers(-8, 9, M * K).astype(np.float32)
    B = r.integers(-8, 9, K * N).astype(np.float32)
    print("gemm exact %s M=%d N=%d K=%d offset %d" % (_tag(trans), M, N, K, off), flush=True)
    dA = torch.zeros(A.size + off, device="cuda", dtype=torch.float32)
    dB = torch.zeros(B.size + off, device="cuda", dtype=torch.float32)
    dA[off:].copy_(dev(A))  # kept alive until the launch has run
    dB[off:].copy_(dev(B))
    gC = Guarded(M * N, fill=np.full(M * N, np.nan, np.float32))
    bmb.gemm(ta, tb, M, N, K, 1.0, dA[off:].data_ptr(), dB[off:].data_ptr(), 0.0, gC.ptr)
    sync("gemm exact")
    assert gC.ok()
    Am = A.reshape(K, M).T if ta else A.reshape(M, K)
    Bm = B.reshape(N, K).T if tb else B.reshape(K, N)
    ref = (Am.astype(np.float64) @ Bm.astype(np.float64)).astype(np.float32).reshape(-1)
    assert np.array_equal(gC.get(), ref)


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


# Few output tiles and a long K: batched_gemm() never splits K across
# workgroups, so the planner runs such tiles as k-slices of one workgroup
# (2 or 4 slices summed in LDS). Whole tiles with K a multiple of the slices'
# k-tiles, K that leaves the last slice short or empty, tiles shifted back
# at the edges, and problems smaller than one tile.
KSHAPES = [(2, 128, 128, 2048), (3, 100, 70, 3000), (2, 40, 50, 1100), (3, 64, 256, 4160),
           (1, 200, 136, 1000), (2, 64, 64, 72 * 16 + 8)]


@pytest.mark.parametrize("trans", TRANS, ids=_tag)
@pytest.mark.parametrize("bshape", KSHAPES, ids=lambda s: "b%d_%dx%dx%d" % s)
def test_batched_long_k(gpu, bshape, trans):
    """Within fp32_order_bound(K) of the fp64 product (fp32 MFMA products;
    only the summation order differs)."""
    batch, M, N, K = bshape
    ta, tb = trans
    eA, eB, eC = M * K, K * N, M * N
    A = O.fill_xorshift(eA * batch, 0x2468)
    B = O.fill_xorshift(eB * batch, 0x1357)
    C0 = O.fill_xorshift(eC * batch, 0x4444)
    dA, dB = dev(A), dev(B)
    gC = Guarded(eC * batch, fill=C0)
    print("batched long-K %s batch=%d M=%d N=%d K=%d" % (_tag(trans), batch, M, N, K), flush=True)
    bmb.batched_gemm(ta, tb, batch, M, N, K, 0.5, dA.data_ptr(), eA, dB.data_ptr(), eB,
                     2.0, gC.ptr, eC)
    sync("batched_gemm")
    assert gC.ok()
    ref = O.batched_gemm_f64(ta, tb, batch, M, N, K, 0.5, A, eA, B, eB, 2.0, C0, eC)
    err, bad = O.normwise(gC.get(), ref)
    print("  normwise %.2e (bound %.2e)" % (err, fp32_order_bound(K)))
    assert bad == 0 and err < fp32_order_bound(K)


# the 15 GEMMs of the GPT-2-small step (BT = 8192,
# C = 768, V = 50257), i.e. every (layer, pass) that bench.py times. Layer
# (cin, cout): forward y = x w^T is NT (BT, cout, cin); dX = dy w is NN
# (BT, cin, cout); dW += dy^T x is TN (cout, cin, BT) with beta 1
# (src/gpt.cu:256-376).
_LAYERS = [(768, 2304), (768, 768), (768, 3072), (3072, 768), (768, 50257)]
GPT = ([(8192, co, ci, False, True, 0.0) for ci, co in _LAYERS] +
       [(8192, ci, co, False, False, 0.0) for ci, co in _LAYERS] +
       [(co, ci, 8192, True, False, 1.0) for ci, co in _LAYERS])


@pytest.mark.parametrize("g", GPT, ids=lambda g: "%dx%dx%d_%s" % (g[0], g[1], g[2], _tag(g[3:5])))
def test_gpt_training_shapes(gpu, g):
    """BASELINE config 3 shapes (weights N(0, 0.02^2), activations N(0, 1)),
    checked on a sample of output rows (rows are independent problems). The
    ragged LM head at V = 50257 runs split over K in the dX NN case (K =
    50257 ends in a partial k-tile, rows not 16-byte aligned) and over 2-D
    tiles with a ragged edge in the forward and dW."""
    M, N, K, ta, tb, beta = g
    A = O.fill_normal(M * K, 0xA11CE, 1.0)
    B = O.fill_normal(K * N, 0xB0B, 0.02)
    C0 = O.fill_normal(M * N, 0xC0C0, 1.0) if beta != 0 else None
    dA, dB = dev(A), dev(B)
    import torch
    dC = dev(C0) if C0 is not None else torch.empty(M * N, device="cuda", dtype=torch.float32)
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
    e3, bound = bf16x3_err(got[rows], False, tb, len(rows), N, K, 1.0, np.ascontiguousarray(Aop),
                           B, beta, c0)
    print("  normwise %.2e; around the bf16x3 value %.2e (bound %.2e)" % (err, e3, bound))
    assert bad == 0 and err < 1e-4
    assert e3 < bound


# Shapes whose output-tile count is small against their K: gemm() splits K
# into ranges, sums each into a scratch partial and adds the partials in range
# order (deterministic). Odd K leaves a short last range.
SPLIT = [(1000, 1000, 1001), (257, 129, 3000), (96, 160, 777), (1, 1, 4096), (3, 300, 5000),
         (768, 768, 8192)]


@pytest.mark.parametrize("trans", TRANS, ids=_tag)
@pytest.mark.parametrize("shape", SPLIT, ids=lambda s: "%dx%dx%d" % s)
def test_split_k(gpu, shape, trans):
    import torch
    M, N, K = shape
    ta, tb = trans
    A = O.fill_xorshift(M * K, 0x1357)
    B = O.fill_xorshift(K * N, 0x2468)
    C0 = O.fill_xorshift(M * N, 0x9999)
    dA, dB = dev(A), dev(B)
    print("split-k %s M=%d N=%d K=%d" % (_tag(trans), M, N, K), flush=True)
    # beta = 0: C is write-only, so NaN in it must not reach the result
    gC = Guarded(M * N, fill=np.full(M * N, np.nan, np.float32))
    bmb.gemm(ta, tb, M, N, K, 0.75, dA.data_ptr(), dB.data_ptr(), 0.0, gC.ptr)
    sync("gemm beta 0")
    assert gC.ok()
    ref0 = O.gemm_f64(ta, tb, M, N, K, 0.75, A, B, 0.0, None)
    err, bad = O.normwise(gC.get(), ref0)
    assert bad == 0 and err < 1e-4, err
    e3, bound = bf16x3_err(gC.get(), ta, tb, M, N, K, 0.75, A, B, 0.0, None)
    assert e3 < bound, (e3, bound)
    # beta != 0, twice: bit-identical
    outs = []
    for _ in range(2):
        g2 = Guarded(M * N, fill=C0)
        bmb.gemm(ta, tb, M, N, K, 0.75, dA.data_ptr(), dB.data_ptr(), 1.25, g2.ptr)
        sync("gemm")
        assert g2.ok()
        outs.append(g2.get())
    assert np.array_equal(outs[0], outs[1])
    ref = O.gemm_f64(ta, tb, M, N, K, 0.75, A, B, 1.25, C0)
    err, bad = O.normwise(outs[0], ref)
    assert bad == 0 and err < 1e-4, err
    e3, bound = bf16x3_err(outs[0], ta, tb, M, N, K, 0.75, A, B, 1.25, C0)
    assert e3 < bound, (e3, bound)
    # operands one float off 16-byte alignment (the 32-bit load path)
    mA = torch.zeros(A.size + 1, device="cuda", dtype=torch.float32)
    mB = torch.zeros(B.size + 1, device="cuda", dtype=torch.float32)
    mC = torch.zeros(C0.size + 1, device="cuda", dtype=torch.float32)
    mA[1:].copy_(dA)
    mB[1:].copy_(dB)
    mC[1:].copy_(dev(C0))
    bmb.gemm(ta, tb, M, N, K, 0.75, mA[1:].data_ptr(), mB[1:].data_ptr(), 1.25, mC[1:].data_ptr())
    sync("gemm misaligned")
    e3, bound = bf16x3_err(mC[1:].cpu().numpy(), ta, tb, M, N, K, 0.75, A, B, 1.25, C0)
    assert e3 < bound, (e3, bound)


def test_non_null_stream_matches(gpu):
    """gemm() splits K on any stream: its scratch is leased per call and its
    reuse is ordered by an event on the caller's stream. 768 x 768 x 8192 TN
    (the GPT-2 attention-projection dW, split into several K ranges) on a
    torch side stream gives the null stream's bits, twice in a row (the
    second call reuses the first call's buffer), and both are within the
    bf16x3 bound."""
    import torch
    M, N, K = 768, 768, 8192
    A = O.fill_xorshift(M * K, 0x1111)
    B = O.fill_xorshift(K * N, 0x2222)
    C0 = O.fill_xorshift(M * N, 0x3333)
    dA, dB, dC0 = dev(A), dev(B), dev(C0)
    dC = dC0.clone()
    bmb.gemm(True, False, M, N, K, 1.0, dA.data_ptr(), dB.data_ptr(), 0.5, dC.data_ptr())
    sync("gemm on the null stream")
    ref = dC.cpu().numpy().view(np.uint32).copy()
    s = torch.cuda.Stream()
    for i in range(2):
        print("gemm TN %dx%dx%d on a side stream, call %d" % (M, N, K, i), flush=True)
        with torch.cuda.stream(s):
            dC.copy_(dC0)
            bmb.gemm(True, False, M, N, K, 1.0, dA.data_ptr(), dB.data_ptr(), 0.5,
                     dC.data_ptr(), s.cuda_stream)
        s.synchronize()
        bmb.check("gemm on stream")
        got = dC.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), ref)
    e3, bound = bf16x3_err(got, True, False, M, N, K, 1.0, A, B, 0.5, C0)
    assert e3 < bound, (e3, bound)


def test_two_streams_share_scratch_in_order(gpu):
    """Two streams that each run split-K gemm() calls back to back, with no
    ordering between the streams: every call leases the partials buffer the
    other stream's last call returned, so each lease must wait for that
    call's kernels. Each result equals its null-stream bits."""
    import torch
    shapes = [(768, 768, 8192, True), (768, 3072, 8192, True)]
    data = []
    for i, (M, N, K, ta) in enumerate(shapes):
        A = O.fill_xorshift(M * K, 0x7070 + i)
        B = O.fill_xorshift(K * N, 0x8080 + i)
        d = {"A": dev(A), "B": dev(B), "shape": (M, N, K, ta)}
        d["C"] = torch.empty(M * N, device="cuda", dtype=torch.float32)
        bmb.gemm(ta, False, M, N, K, 1.0, d["A"].data_ptr(), d["B"].data_ptr(), 0.0,
                 d["C"].data_ptr())
        sync("reference gemm")
        d["ref"] = d["C"].cpu().numpy().view(np.uint32).copy()
        d["outs"] = [torch.empty(M * N, device="cuda", dtype=torch.float32) for _ in range(4)]
        data.append(d)
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    print("two streams x 4 split-K gemm() calls", flush=True)
    for r in range(4):
        for d, s in zip(data, streams):
            M, N, K, ta = d["shape"]
            bmb.gemm(ta, False, M, N, K, 1.0, d["A"].data_ptr(), d["B"].data_ptr(), 0.0,
                     d["outs"][r].data_ptr(), s.cuda_stream)
    torch.cuda.synchronize()
    bmb.check("gemm on two streams")
    for d in data:
        for o in d["outs"]:
            assert np.array_equal(o.cpu().numpy().view(np.uint32), d["ref"])


def test_null_and_side_stream_share_scratch_in_order(gpu):
    """A lease on the null stream records no event when it returns its
    buffer; a lease on another stream that takes the buffer records one on
    the null stream then and waits for it. Split-K gemm() calls alternate
    between the null stream and a side stream (torch's pool streams do not
    synchronise with the null stream), with no host synchronisation, a large
    shape on the null stream each time so that its reduce is still running
    when the side stream's call is queued. Every result equals its bits from
    calls made one at a time."""
    import torch
    shapes = [(3072, 768, 8192, True), (768, 768, 8192, True)]
    data = []
    for i, (M, N, K, ta) in enumerate(shapes):
        A = O.fill_xorshift(M * K, 0x5150 + i)
        B = O.fill_xorshift(K * N, 0x6160 + i)
        d = {"A": dev(A), "B": dev(B), "shape": (M, N, K, ta)}
        d["C"] = torch.empty(M * N, device="cuda", dtype=torch.float32)
        bmb.gemm(ta, False, M, N, K, 1.0, d["A"].data_ptr(), d["B"].data_ptr(), 0.0,
                 d["C"].data_ptr())
        sync("reference gemm")
        d["ref"] = d["C"].cpu().numpy().view(np.uint32).copy()
        d["outs"] = [torch.empty(M * N, device="cuda", dtype=torch.float32) for _ in range(4)]
        data.append(d)
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    print("null stream and side stream x 4 split-K gemm() calls", flush=True)
    for r in range(4):
        for d, s in zip(data, (0, side.cuda_stream)):
            M, N, K, ta = d["shape"]
            bmb.gemm(ta, False, M, N, K, 1.0, d["A"].data_ptr(), d["B"].data_ptr(), 0.0,
                     d["outs"][r].data_ptr(), s)
    torch.cuda.synchronize()
    bmb.check("gemm on the null and a side stream")
    for d in data:
        for o in d["outs"]:
            assert np.array_equal(o.cpu().numpy().view(np.uint32), d["ref"])


# ---- gemm_set_math(GEMM_MATH_FP32): fp32 matrix-core products, held to the
# fp32 summation bound (the rounding level of the reference's fp32 gemm()).

@pytest.fixture
def fp32_math(gpu):
    with bmb.gemm_math(bmb.GEMM_MATH_FP32):
        assert bmb.gemm_get_math() == bmb.GEMM_MATH_FP32
        yield
    assert bmb.gemm_get_math() == bmb.GEMM_MATH_BF16X3


def test_math_switch_rejects_unknown_modes(gpu):
    assert bmb.gemm_get_math() == bmb.GEMM_MATH_BF16X3
    assert bmb.gemm_set_math(7) == -1
    assert bmb.gemm_get_math() == bmb.GEMM_MATH_BF16X3


@pytest.mark.parametrize("trans", TRANS, ids=_tag)
@pytest.mark.parametrize("shape", SHAPES + SPLIT[:3], ids=lambda s: "%dx%dx%d" % s)
def test_fp32_math_shapes(fp32_math, shape, trans):
    """The reference's 10 shapes x 4 transposes (tools/test_gemm.cu:51-62)
    and three split-K shapes in fp32 mode: within fp32_order_bound(K) of the
    fp64 product, which the bf16x3 default (~1e-6) would miss at every K."""
    M, N, K = shape
    ta, tb = trans
    A = O.fill_xorshift(M * K, 0x1234)
    B = O.fill_xorshift(K * N, 0x9ABC)
    C0 = O.fill_xorshift(M * N, 0x5555)
    dA, dB = dev(A), dev(B)
    gC = Guarded(M * N, fill=C0)
    print("gemm fp32 %s M=%d N=%d K=%d" % (_tag(trans), M, N, K), flush=True)
    bmb.gemm(ta, tb, M, N, K, 0.75, dA.data_ptr(), dB.data_ptr(), 1.25, gC.ptr)
    sync("gemm fp32")
    assert gC.ok()
    err, bad = O.normwise(gC.get(), O.gemm_f64(ta, tb, M, N, K, 0.75, A, B, 1.25, C0))
    print("  normwise %.2e (bound %.2e)" % (err, fp32_order_bound(K)))
    assert bad == 0 and err < fp32_order_bound(K)


@pytest.mark.parametrize("g", GPT, ids=lambda g: "%dx%dx%d_%s" % (g[0], g[1], g[2], _tag(g[3:5])))
def test_fp32_math_gpt_training_shapes(fp32_math, g):
    """BASELINE config 3 at the reference's arithmetic: the 15 GPT-2 GEMMs in
    fp32 mode, row-sampled against fp64, within fp32_order_bound(K)."""
    import torch
    M, N, K, ta, tb, beta = g
    A = O.fill_normal(M * K, 0xA11CE, 1.0)
    B = O.fill_normal(K * N, 0xB0B, 0.02)
    C0 = O.fill_normal(M * N, 0xC0C0, 1.0) if beta != 0 else None
    dA, dB = dev(A), dev(B)
    dC = dev(C0) if C0 is not None else torch.empty(M * N, device="cuda", dtype=torch.float32)
    print("gpt gemm fp32 %s M=%d N=%d K=%d beta=%g" % (_tag((ta, tb)), M, N, K, beta), flush=True)
    bmb.gemm(ta, tb, M, N, K, 1.0, dA.data_ptr(), dB.data_ptr(), beta, dC.data_ptr())
    sync("gemm fp32")
    got = dC.cpu().numpy().reshape(M, N)
    rows = np.unique(np.r_[0, 1, 255, 256, M // 2, M - 1, np.random.default_rng(4).integers(0, M, 6)])
    Aop = (A.reshape(K, M).T if ta else A.reshape(M, K))[rows]
    c0 = C0.reshape(M, N)[rows] if C0 is not None else None
    ref = O.gemm_f64(False, tb, len(rows), N, K, 1.0, np.ascontiguousarray(Aop), B, beta, c0)
    err, bad = O.normwise(got[rows], ref)
    print("  normwise %.2e (bound %.2e)" % (err, fp32_order_bound(K)))
    assert bad == 0 and err < fp32_order_bound(K)


# ---- the top of the fp32 range and infinities (both modes)

@pytest.mark.parametrize("math", [0, 1], ids=["bf16x3", "fp32"])
def test_top_of_range_and_infinities(gpu, math):
    """Finite entries of A up to FLT_MAX (above 0x7F7F7FFF, where a plain
    bfloat16 rounding would give infinity) with B on a 1e-3 scale: the
    result is finite and within the mode's bound of the fp64 product (for
    bf16x3: around the split's exact value). Rows of A holding one +-inf
    each: every entry of such a row is +-inf with the sign of inf * b, or
    NaN where b = 0 (fp32 semantics); the other rows are unaffected."""
    import torch
    M, N, K = 192, 160, 96
    A = O.fill_xorshift(M * K, 0xF00D).reshape(M, K)
    B = (O.fill_xorshift(K * N, 0xBEEF) * np.float32(1e-3)).reshape(K, N)
    big = np.array([0x7F7FFFFF, 0xFF7FFFFF, 0x7F7F8000, 0xFF7F8001, 0x7F7F7FFF, 0x7F700000],
                   np.uint32).view(np.float32)
    r = np.random.default_rng(5)
    A[r.integers(0, M, 40), r.integers(0, K, 40)] = r.choice(big, 40)
    with bmb.gemm_math(math):
        dA, dB = dev(A), dev(B)
        dC = torch.empty(M * N, device="cuda", dtype=torch.float32)
        print("gemm top of range, math %d" % math, flush=True)
        bmb.gemm(False, False, M, N, K, 1.0, dA.data_ptr(), dB.data_ptr(), 0.0, dC.data_ptr())
        sync("gemm top of range")
        got = dC.cpu().numpy().reshape(M, N)
        assert np.isfinite(got).all()
        err, _ = O.normwise(got, O.gemm_f64(False, False, M, N, K, 1.0, A, B, 0.0, None))
        if math == 0:
            e3, bound = bf16x3_err(got, False, False, M, N, K, 1.0, A, B, 0.0, None)
            assert e3 < bound, (e3, bound)
            assert err < 1e-4
        else:
            assert err < fp32_order_bound(K), err
        # infinities: rows 3 and 70 get +inf and -inf
        Ai = A.copy()
        Ai[3, 17], Ai[70, 5] = np.inf, -np.inf
        B0 = B.copy()
        B0[17, :7] = 0.0  # inf * 0 = NaN in those entries of row 3
        dA, dB = dev(Ai), dev(B0)
        bmb.gemm(False, False, M, N, K, 1.0, dA.data_ptr(), dB.data_ptr(), 0.0, dC.data_ptr())
        sync("gemm infinities")
        got = dC.cpu().numpy().reshape(M, N)
    with np.errstate(invalid="ignore", over="ignore"):
        want = Ai.astype(np.float64) @ B0.astype(np.float64)
    for i in (3, 70):
        assert np.array_equal(np.isnan(got[i]), np.isnan(want[i]))
        fin = ~np.isnan(want[i])
        assert np.isinf(got[i][fin]).all()
        assert np.array_equal(np.sign(got[i][fin]), np.sign(want[i][fin]))
    assert np.isnan(got[3, :7]).all()
    rest = np.setdiff1d(np.arange(M), [3, 70])
    assert np.isfinite(got[rest]).all()


# ---- row bands: a tile count just above whole rounds runs as two launches
# (rows [0, m1) on whole rounds of one tile, the rest on its own tile and K
# split; m1 a multiple of 256). 4097^3 takes two bands in both modes' planners
# when K >= 4096; the transposed-A cases run the second band with A offset by
# m1 columns and its full row stride.

@pytest.mark.parametrize("math", [0, 1], ids=["bf16x3", "fp32"])
@pytest.mark.parametrize("trans", TRANS, ids=_tag)
def test_row_bands(gpu, trans, math):
    import torch
    M = N = K = 4097
    ta, tb = trans
    A = O.fill_xorshift(M * K, 0x3131)
    B = O.fill_xorshift(K * N, 0x4141)
    C0 = O.fill_xorshift(M * N, 0x5151)
    with bmb.gemm_math(math):
        dA, dB, dC = dev(A), dev(B), dev(C0)
        print("gemm %s %dx%dx%d math %d" % (_tag(trans), M, N, K, math), flush=True)
        bmb.gemm(ta, tb, M, N, K, 0.75, dA.data_ptr(), dB.data_ptr(), 1.25, dC.data_ptr())
        sync("gemm bands")
    got = dC.cpu().numpy().reshape(M, N)
    # both sides of every 64-row boundary, and the ragged last rows
    rows = np.unique(np.r_[np.arange(0, M, 64), np.arange(63, M, 64), M - 2, M - 1])
    Aop = np.ascontiguousarray((A.reshape(K, M).T if ta else A.reshape(M, K))[rows])
    c0 = C0.reshape(M, N)[rows]
    ref = O.gemm_f64(False, tb, len(rows), N, K, 0.75, Aop, B, 1.25, c0)
    err, bad = O.normwise(got[rows], ref)
    assert bad == 0 and err < 1e-4
    if math == 0:
        e3, bound = bf16x3_err(got[rows], False, tb, len(rows), N, K, 0.75, Aop, B, 1.25, c0)
        assert e3 < bound, (e3, bound)
    else:
        assert err < fp32_order_bound(K), err


# ---- corner plans: C as a block of whole 256 x 256 tiles plus at most 8
# columns right of it and 8 rows below it, the edges on the edge kernels
# (edge_gemm.hip; row-major A and B, BLAS epilogue). The plan trace
# (BMB_GEMM_PLAN_TRACE, read when a shape is first planned) shows that these
# shapes take that plan; the sampled rows include every edge row, and every
# sampled row is checked over all columns (the right edge included). The
# fp32 mode's edges use exact fp32 products, the bf16x3 mode's the bf16x3
# split's three products, each held to its own bound.

# (distinct shapes per mode: plans are memoised per shape; the last has only
# a right edge)
@pytest.mark.parametrize("shape,math", [((4104, 4101, 4099), 0), ((4097, 4100, 4096), 0),
                                        ((4103, 4101, 4099), 1), ((4096, 4100, 4096), 1)],
                         ids=["4104x4101x4099-bf16x3", "4097x4100x4096-bf16x3",
                              "4103x4101x4099-fp32", "4096x4100x4096-fp32"])
def test_corner_edges(gpu, shape, math, capfd, monkeypatch):
    M, N, K = shape
    A = O.fill_xorshift(M * K, 0x6161)
    B = O.fill_xorshift(K * N, 0x7171)
    C0 = O.fill_xorshift(M * N, 0x8181)
    monkeypatch.setenv("BMB_GEMM_PLAN_TRACE", "1")
    with bmb.gemm_math(math):
        dA, dB, dC = dev(A), dev(B), dev(C0)
        print("gemm NN %dx%dx%d math %d" % (M, N, K, math), flush=True)
        bmb.gemm(False, False, M, N, K, 0.75, dA.data_ptr(), dB.data_ptr(), 1.25, dC.data_ptr())
        sync("gemm corner edges")
    err_out = capfd.readouterr().err
    plan = [l for l in err_out.splitlines() if "gemm plan %dx%dx%d:" % (M, N, K) in l]
    assert plan and "edges 1" in plan[0], err_out
    m1 = M // 256 * 256
    got = dC.cpu().numpy().reshape(M, N)
    rows = np.unique(np.r_[0, 1, 255, 256, 2047, 2048, m1 - 1, np.arange(m1, M), M - 1])
    Aop = A.reshape(M, K)[rows]
    c0 = C0.reshape(M, N)[rows]
    ref = O.gemm_f64(False, False, len(rows), N, K, 0.75, Aop, B, 1.25, c0)
    err, bad = O.normwise(got[rows], ref)
    assert bad == 0 and err < 1e-4
    if math == 0:
        e3, bound = bf16x3_err(got[rows], False, False, len(rows), N, K, 0.75, Aop, B, 1.25, c0)
        assert e3 < bound, (e3, bound)
    else:
        assert err < fp32_order_bound(K), err
    # the edge columns alone, over the sampled rows
    n1 = N // 256 * 256
    e_edge, bad = O.normwise(got[rows][:, n1:], ref[:, n1:])
    assert bad == 0 and e_edge < (fp32_order_bound(3 * K) if math == 0 else fp32_order_bound(K))


@pytest.mark.parametrize("math", [0, 1], ids=["bf16x3", "fp32"])
@pytest.mark.parametrize("rm,rn", [(2, 3), (6, 8), (8, 1), (3, 0), (0, 6)],
                         ids=lambda v: str(v))
def test_corner_edge_widths(gpu, rm, rn, math, capfd, monkeypatch):
    """Edge widths 0-8 on a block of whole tiles (K = 4096; the bf16x3
    planner takes the corner plan from a 4096^2 block, the fp32 one already
    from 2048^2): every edge row and column against fp64, the edges' own
    bound, and the plan trace showing the edge kernels ran."""
    base = 4096 if math == 0 else 2048
    M, N, K = base + rm, base + rn, 4096
    A = O.fill_xorshift(M * K, 0x1357)
    B = O.fill_xorshift(K * N, 0x2468)
    C0 = O.fill_xorshift(M * N, 0x3579)
    monkeypatch.setenv("BMB_GEMM_PLAN_TRACE", "1")
    with bmb.gemm_math(math):
        dA, dB, dC = dev(A), dev(B), dev(C0)
        print("gemm NN %dx%dx%d math %d" % (M, N, K, math), flush=True)
        bmb.gemm(False, False, M, N, K, 0.5, dA.data_ptr(), dB.data_ptr(), 2.0, dC.data_ptr())
        sync("gemm corner edge widths")
    err_out = capfd.readouterr().err
    plan = [l for l in err_out.splitlines() if "gemm plan %dx%dx%d:" % (M, N, K) in l]
    assert plan and "edges 1" in plan[0], err_out
    got = dC.cpu().numpy().reshape(M, N)
    rows = np.unique(np.r_[0, 1, 511, 512, 1023, base - 1, np.arange(base, M)])
    ref = O.gemm_f64(False, False, len(rows), N, K, 0.5, A.reshape(M, K)[rows], B, 2.0,
                     C0.reshape(M, N)[rows])
    bound = fp32_order_bound(3 * K) if math == 0 else fp32_order_bound(K)
    err, bad = O.normwise(got[rows], ref)
    assert bad == 0 and err < 1e-4
    if math == 0:
        e3, b3 = bf16x3_err(got[rows], False, False, len(rows), N, K, 0.5,
                            A.reshape(M, K)[rows], B, 2.0, C0.reshape(M, N)[rows])
        assert e3 < b3, (e3, b3)
    else:
        assert err < bound, err
    if rn:
        # the right edge over every row
        refc = O.gemm_f64(False, False, M, rn, K, 0.5, A.reshape(M, K),
                          np.ascontiguousarray(B.reshape(K, N)[:, base:]), 2.0,
                          np.ascontiguousarray(C0.reshape(M, N)[:, base:]))
        ec, bad = O.normwise(got[:, base:], refc)
        assert bad == 0 and ec < bound, ec


# Problems too small to fill the device on whole-K tiles: the bf16x3 planner
# runs them on k-sliced workgroups (64 x 64 or 32 x 32 tiles, 2-8 slices
# whose sums meet in LDS) instead of split-K plus a reduce. The shapes cover
# the unguarded interior loop (K a multiple of slices * 32), ragged tiles
# and K, a last slice with a partial range and one with no data at all.
KS_SHAPES = [(512, 512, 512), (1000, 1000, 1000), (256, 256, 257), (200, 300, 700),
             (64, 64, 4096), (768, 768, 768)]


@pytest.mark.parametrize("trans", TRANS, ids=_tag)
@pytest.mark.parametrize("shape", KS_SHAPES, ids=lambda s: "%dx%dx%d" % s)
def test_k_sliced_tiles(gpu, shape, trans, capfd, monkeypatch):
    M, N, K = shape
    ta, tb = trans
    A = O.fill_xorshift(M * K, 0x4242)
    B = O.fill_xorshift(K * N, 0x5353)
    C0 = O.fill_xorshift(M * N, 0x6464)
    monkeypatch.setenv("BMB_GEMM_PLAN_TRACE", "1")
    dA, dB, dC = dev(A), dev(B), dev(C0)
    print("gemm %s %dx%dx%d" % (_tag(trans), M, N, K), flush=True)
    bmb.gemm(ta, tb, M, N, K, 0.75, dA.data_ptr(), dB.data_ptr(), 1.25, dC.data_ptr())
    sync("gemm k-sliced")
    err_out = capfd.readouterr().err
    # Plans are memoised per shape (not per transpose), so the trace line
    # comes with the first call of a shape, the NN case; the others reuse it.
    plan = [l for l in err_out.splitlines() if "bf16x3 gemm plan %dx%dx%d:" % (M, N, K) in l]
    if trans == (False, False):
        assert plan, err_out
    for line in plan:
        assert any("parts (%d," % t in line for t in (4, 5, 6, 7)), line
    got = dC.cpu().numpy().reshape(M, N)
    ref = O.gemm_f64(ta, tb, M, N, K, 0.75, A, B, 1.25, C0)
    err, bad = O.normwise(got, ref)
    assert bad == 0 and err < 1e-4, err
    e3, bound = bf16x3_err(got, ta, tb, M, N, K, 0.75, A, B, 1.25, C0)
    assert e3 < bound, (e3, bound)


# Shapes drawn at random (fixed seed), run through whatever plan each planner
# picks for them -- whole tiles, k-sliced workgroups, split-K, row bands,
# corner plans -- in both arithmetic modes and all four transposes. C sits
# between canary bands (no write outside it); sampled rows of op(A) against
# fp64: the reference's 1e-4, and each mode's own bound.
def _random_shapes(n, seed):
    r = np.random.default_rng(seed)
    return [(int(r.integers(1, 2600)), int(r.integers(1, 2600)), int(r.integers(1, 5000)))
            for _ in range(n)]


RANDOM_SHAPES = _random_shapes(12, 2024)


@pytest.mark.parametrize("math", [0, 1], ids=["bf16x3", "fp32"])
@pytest.mark.parametrize("trans", TRANS, ids=_tag)
@pytest.mark.parametrize("shape", RANDOM_SHAPES, ids=lambda s: "%dx%dx%d" % s)
def test_random_shapes(gpu, shape, trans, math):
    M, N, K = shape
    ta, tb = trans
    A = O.fill_xorshift(M * K, 0x3131 + M)
    B = O.fill_xorshift(K * N, 0x4141 + N)
    C0 = O.fill_xorshift(M * N, 0x5151 + K)
    with bmb.gemm_math(math):
        dA, dB = dev(A), dev(B)
        gC = Guarded(M * N, fill=C0)
        print("gemm %s %dx%dx%d math %d" % (_tag(trans), M, N, K, math), flush=True)
        bmb.gemm(ta, tb, M, N, K, 0.75, dA.data_ptr(), dB.data_ptr(), 1.25, gC.ptr)
        sync("gemm random shape")
    assert gC.ok()
    rows = np.unique(np.r_[0, M // 2, M - 1, np.random.default_rng(M + N + K).integers(0, M, 9)])
    Aop = np.ascontiguousarray((A.reshape(K, M).T if ta else A.reshape(M, K))[rows])
    c0 = np.ascontiguousarray(C0.reshape(M, N)[rows])
    got = gC.get().reshape(M, N)[rows]
    ref = O.gemm_f64(False, tb, len(rows), N, K, 0.75, Aop, B, 1.25, c0)
    err, bad = O.normwise(got, ref)
    assert bad == 0 and err < 1e-4, err
    if math == 0:
        e3, bound = bf16x3_err(got, False, tb, len(rows), N, K, 0.75, Aop, B, 1.25, c0)
        assert e3 < bound, (e3, bound)
    else:
        assert err < fp32_order_bound(K), (err, fp32_order_bound(K))


def _random_batched(n, seed):
    r = np.random.default_rng(seed)
    return [(int(r.integers(1, 9)), int(r.integers(1, 400)), int(r.integers(1, 400)),
             int(r.integers(1, 3000))) for _ in range(n)]


@pytest.mark.parametrize("trans", TRANS, ids=_tag)
@pytest.mark.parametrize("bshape", _random_batched(8, 77), ids=lambda s: "b%d_%dx%dx%d" % s)
def test_random_batched(gpu, bshape, trans):
    """batched_gemm() on random shapes (fixed seed): whole-K tiles or
    k-sliced workgroups, whatever its planner picks; every problem of the
    batch within fp32_order_bound(K) of fp64, C between canary bands."""
    batch, M, N, K = bshape
    ta, tb = trans
    eA, eB, eC = M * K, K * N, M * N
    A = O.fill_xorshift(eA * batch, 0x6262 + K)
    B = O.fill_xorshift(eB * batch, 0x7272 + M)
    C0 = O.fill_xorshift(eC * batch, 0x8282 + N)
    dA, dB = dev(A), dev(B)
    gC = Guarded(eC * batch, fill=C0)
    print("batched %s batch=%d M=%d N=%d K=%d" % (_tag(trans), batch, M, N, K), flush=True)
    bmb.batched_gemm(ta, tb, batch, M, N, K, 0.5, dA.data_ptr(), eA, dB.data_ptr(), eB,
                     2.0, gC.ptr, eC)
    sync("batched_gemm random")
    assert gC.ok()
    ref = O.batched_gemm_f64(ta, tb, batch, M, N, K, 0.5, A, eA, B, eB, 2.0, C0, eC)
    err, bad = O.normwise(gC.get(), ref)
    assert bad == 0 and err < fp32_order_bound(K), (err, fp32_order_bound(K))
