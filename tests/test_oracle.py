"""Pins the CPU oracle before anything is checked against it.

The reference commits no golden vectors for this path (its tests generate
inputs on the fly and compare GPU against cuBLAS / GPU against GPU), so each
oracle function is pinned by checks it could not pass with a plausible
mistake in it:
  * xorshift32: Marsaglia's published first output for his seed;
  * sequential-fmaf GEMM: brute force with exact rational arithmetic and one
    rounding per fused multiply-add, on inputs whose rounding a separate
    multiply-then-add (or any other k order) would change;
  * fp64 GEMM: numpy's matmul (a library routine) for all transposes/batch;
  * attention: torch's scaled_dot_product_attention in float64 (a library
    routine) and its autograd; closed forms (T=1, K=0, V=const); a directional
    finite difference of the loss (the method of tools/test_grad.cu:8-26);
  * committed fixtures in tests/golden/ (see make_golden.py there).
"""
import math
import os
from fractions import Fraction

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ------------------------------------------------------------ generators
def test_xorshift_known_answer():
    """Marsaglia, 'Xorshift RNGs' (J. Stat. Soft. 2003): y = 2463534242,
    y ^= y<<13; y ^= y>>17; y ^= y<<5 first returns 723471715."""
    assert int(O.xorshift_stream(1, 2463534242)[0]) == 723471715


def test_fill_maps_stream_to_grid():
    """src/bench.cu:59-66: v = ((int)(s % 2000) - 1000) / 1000.0f."""
    s = O.xorshift_stream(1000, 0x12345678).astype(np.int64)
    want = ((s % 2000) - 1000).astype(np.float32) / np.float32(1000.0)
    got = O.fill_xorshift(1000, 0x12345678)
    assert np.array_equal(got, want)
    assert got.min() >= -1.0 and got.max() <= 0.999


def test_fill_normal_moments():
    z = O.fill_normal(200000, 1234).astype(np.float64)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01
    assert np.array_equal(O.fill_normal(10, 5), O.fill_normal(10, 5))


# ------------------------------------------------------------ sequential fmaf
def _round_f32(x: Fraction) -> np.float32:
    """Round an exact rational to the nearest float32, ties to even."""
    c = np.float32(float(x))
    best = None
    for cand in (np.nextafter(c, np.float32(-np.inf)), c, np.nextafter(c, np.float32(np.inf))):
        if not np.isfinite(cand):
            continue
        d = abs(Fraction(float(cand)) - x)
        key = (d, int(np.float32(cand).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, cand)
    return np.float32(best[1])


def _fma32(a, b, c):
    return _round_f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def _brute_gemm(ta, tb, M, N, K, alpha, A, B, beta, C0, fused=True):
    A = A.reshape((K, M) if ta else (M, K))
    B = B.reshape((N, K) if tb else (K, N))
    out = np.empty((M, N), np.float32)
    for i in range(M):
        for j in range(N):
            acc = np.float32(0.0)
            for k in range(K):
                a = A[k, i] if ta else A[i, k]
                b = B[j, k] if tb else B[k, j]
                if fused:
                    acc = _fma32(a, b, acc)
                else:
                    acc = np.float32(np.float32(a * b) + acc)
            if beta == 0.0:
                out[i, j] = np.float32(np.float32(alpha) * acc)
            else:
                out[i, j] = _fma32(np.float32(alpha), acc, np.float32(np.float32(beta) * C0[i, j]))
    return out


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_f32seq_is_sequential_fma(ta, tb):
    rng = np.random.default_rng(11 + 2 * ta + tb)
    M, N, K = 3, 4, 7
    # full-mantissa values over several binades: every rounding step matters
    A = (rng.standard_normal(M * K) * np.exp2(rng.integers(-6, 6, M * K))).astype(np.float32)
    B = (rng.standard_normal(K * N) * np.exp2(rng.integers(-6, 6, K * N))).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    want = _brute_gemm(ta, tb, M, N, K, 0.75, A, B, 1.25, C0)
    got = O.gemm_f32seq(ta, tb, M, N, K, 0.75, A, B, 1.25, C0)
    assert np.array_equal(got, want)
    got_mt = O.gemm_f32seq(ta, tb, M, N, K, 0.75, A, B, 1.25, C0, threads=3)
    assert np.array_equal(got_mt, want)


def test_f32seq_separates_plausible_mistakes():
    """The inputs above do distinguish fused from unfused and from reordered
    accumulation, so the bit-exact test has teeth."""
    rng = np.random.default_rng(5)
    M, N, K = 3, 4, 7
    A = (rng.standard_normal(M * K) * np.exp2(rng.integers(-6, 6, M * K))).astype(np.float32)
    B = (rng.standard_normal(K * N) * np.exp2(rng.integers(-6, 6, K * N))).astype(np.float32)
    fused = _brute_gemm(0, 0, M, N, K, 1.0, A, B, 0.0, None)
    unfused = _brute_gemm(0, 0, M, N, K, 1.0, A, B, 0.0, None, fused=False)
    rev = _brute_gemm(0, 0, M, N, K, 1.0, A.reshape(M, K)[:, ::-1].copy(), B.reshape(K, N)[::-1].copy(),
                      0.0, None)
    assert not np.array_equal(fused, unfused)
    assert not np.array_equal(fused, rev)
    assert np.array_equal(O.gemm_f32seq(0, 0, M, N, K, 1.0, A, B, 0.0, None), fused)


def test_f32seq_beta_zero_never_reads_c():
    A = O.fill_xorshift(6, 1).reshape(2, 3)
    B = O.fill_xorshift(12, 2).reshape(3, 4)
    C0 = np.full((2, 4), np.nan, np.float32)
    out = O.gemm_f32seq(0, 0, 2, 4, 3, 1.0, A, B, 0.0, C0)
    assert np.isfinite(out).all()


def test_f32seq_exact_on_small_integers():
    """Integer-valued products and sums below 2^24 are exact in any order."""
    rng = np.random.default_rng(2)
    M, N, K = 17, 23, 31
    A = rng.integers(-8, 8, (M, K)).astype(np.float32)
    B = rng.integers(-8, 8, (K, N)).astype(np.float32)
    want = (A.astype(np.int64) @ B.astype(np.int64)).astype(np.float32)
    assert np.array_equal(O.gemm_f32seq(0, 0, M, N, K, 1.0, A, B, 0.0, None), want)


# ------------------------------------------------------------ fp64 GEMM
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_f64_matches_numpy(ta, tb):
    rng = np.random.default_rng(3)
    M, N, K = 37, 29, 41
    A = rng.standard_normal(M * K).astype(np.float32)
    B = rng.standard_normal(K * N).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    opA = A.reshape(K, M).T if ta else A.reshape(M, K)
    opB = B.reshape(N, K).T if tb else B.reshape(K, N)
    want = 0.75 * (opA.astype(np.float64) @ opB.astype(np.float64)) + 1.25 * C0.astype(np.float64)
    got = O.gemm_f64(ta, tb, M, N, K, 0.75, A, B, 1.25, C0)
    assert np.allclose(got, want, rtol=1e-13, atol=1e-12)


def test_batched_f64_and_f32seq_match_per_problem():
    rng = np.random.default_rng(4)
    batch, M, N, K = 5, 9, 7, 6
    A = rng.standard_normal(batch * M * K).astype(np.float32)
    B = rng.standard_normal(batch * K * N).astype(np.float32)
    C0 = rng.standard_normal(batch * M * N).astype(np.float32)
    got64 = O.batched_gemm_f64(0, 1, batch, M, N, K, 0.5, A, M * K, B, K * N, 2.0, C0, M * N)
    got32 = O.batched_gemm_f32seq(0, 1, batch, M, N, K, 0.5, A, M * K, B, K * N, 2.0, C0, M * N)
    for z in range(batch):
        a = A[z * M * K:(z + 1) * M * K].reshape(M, K).astype(np.float64)
        b = B[z * K * N:(z + 1) * K * N].reshape(N, K).T.astype(np.float64)
        c = C0[z * M * N:(z + 1) * M * N].reshape(M, N)
        assert np.allclose(got64[z * M * N:(z + 1) * M * N].reshape(M, N), 0.5 * a @ b + 2.0 * c.astype(np.float64),
                           rtol=1e-13, atol=1e-12)
        one = O.gemm_f32seq(0, 1, M, N, K, 0.5, A[z * M * K:(z + 1) * M * K],
                            B[z * K * N:(z + 1) * K * N], 2.0, c)
        assert np.array_equal(got32[z * M * N:(z + 1) * M * N].reshape(M, N), one)


def test_normwise_metric():
    ref = np.array([1.0, -4.0, 2.0], np.float32)
    got = np.array([1.5, -4.0, 2.0], np.float32)
    e, bad = O.normwise(got, ref)
    assert abs(e - 0.125) < 1e-12 and bad == 0
    e, bad = O.normwise(np.array([np.nan, 1, 1], np.float32), ref)
    assert bad == 1


# ------------------------------------------------------------ attention
def _torch_attention(qkv, B, T, C, NH, dout=None):
    torch = pytest.importorskip("torch")
    hs = C // NH
    x = torch.from_numpy(qkv.astype(np.float64)).reshape(B, T, 3, NH, hs)
    q = x[:, :, 0].transpose(1, 2).clone().requires_grad_(True)
    k = x[:, :, 1].transpose(1, 2).clone().requires_grad_(True)
    v = x[:, :, 2].transpose(1, 2).clone().requires_grad_(True)
    y = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True)
    s = (q @ k.transpose(-1, -2)) / math.sqrt(hs)
    mask = torch.ones(T, T, dtype=torch.bool).tril()
    lse = torch.logsumexp(s.masked_fill(~mask, -math.inf), dim=-1)
    out = y.transpose(1, 2).reshape(B, T, C).detach().numpy()
    grads = None
    if dout is not None:
        g = torch.from_numpy(dout.astype(np.float64)).reshape(B, T, NH, hs).transpose(1, 2)
        dq, dk, dv = torch.autograd.grad(y, (q, k, v), g)
        grads = np.concatenate([t.transpose(1, 2).reshape(B, T, C).numpy() for t in (dq, dk, dv)],
                               axis=2)
    return out, lse.detach().numpy(), grads


@pytest.mark.parametrize("shape", [(2, 9, 24, 3), (1, 33, 64, 2), (3, 5, 32, 1)])
def test_attention_matches_torch_sdpa(shape):
    B, T, C, NH = shape
    qkv = O.fill_normal(B * T * 3 * C, 77).reshape(B, T, 3 * C)
    dout = O.fill_normal(B * T * C, 78).reshape(B, T, C)
    ref_o, ref_l, ref_g = _torch_attention(qkv, B, T, C, NH, dout)
    o, l = O.attn_fwd_f64(qkv, B, T, C, NH)
    assert np.allclose(o, ref_o, rtol=1e-12, atol=1e-12)
    assert np.allclose(l, ref_l, rtol=1e-12, atol=1e-12)
    g = O.attn_bwd_f64(qkv, dout, B, T, C, NH)
    assert np.allclose(g, ref_g, rtol=1e-10, atol=1e-11)


def test_attention_closed_forms():
    B, T, C, NH = 1, 6, 8, 2
    hs = C // NH
    qkv = O.fill_normal(B * T * 3 * C, 9).reshape(B, T, 3 * C)
    # T = 1: out = v_0, lse = scale * q.k
    o, l = O.attn_fwd_f64(qkv[:, :1], 1, 1, C, NH)
    for h in range(NH):
        q = qkv[0, 0, h * hs:(h + 1) * hs].astype(np.float64)
        k = qkv[0, 0, C + h * hs:C + (h + 1) * hs].astype(np.float64)
        assert np.allclose(o[0, 0, h * hs:(h + 1) * hs], qkv[0, 0, 2 * C + h * hs:2 * C + (h + 1) * hs])
        assert abs(l[0, h, 0] - q @ k / math.sqrt(hs)) < 1e-12
    # K = 0: uniform weights over j <= i, lse = ln(i + 1)
    z = qkv.copy()
    z[:, :, C:2 * C] = 0
    o, l = O.attn_fwd_f64(z, B, T, C, NH)
    v = z[0, :, 2 * C:].astype(np.float64)
    for i in range(T):
        assert np.allclose(o[0, i], v[:i + 1].mean(axis=0))
        assert np.allclose(l[0, :, i], math.log(i + 1))
    # V = const: out = const
    c = qkv.copy()
    c[:, :, 2 * C:] = 0.375
    o, _ = O.attn_fwd_f64(c, B, T, C, NH)
    assert np.allclose(o, 0.375)


def test_attention_backward_closed_form_k_zero():
    """K = 0 => P_ij = 1/(i+1) for j <= i, so dV_j = sum_{i>=j} dO_i / (i+1)."""
    B, T, C, NH = 1, 7, 8, 1
    qkv = O.fill_normal(B * T * 3 * C, 19).reshape(B, T, 3 * C)
    qkv[:, :, C:2 * C] = 0
    dout = O.fill_normal(B * T * C, 20).reshape(B, T, C)
    g = O.attn_bwd_f64(qkv, dout, B, T, C, NH)
    d = dout[0].astype(np.float64)
    for j in range(T):
        want = sum(d[i] / (i + 1) for i in range(j, T))
        assert np.allclose(g[0, j, 2 * C:], want)


def test_attention_backward_finite_difference():
    """Directional derivative of L = sum(dout * out) along u = g/|g| (the
    method of tools/test_grad.cu:8-26), central difference in fp64."""
    B, T, C, NH = 1, 5, 8, 2
    qkv = O.fill_normal(B * T * 3 * C, 31).reshape(B, T, 3 * C).astype(np.float64)
    dout = O.fill_normal(B * T * C, 32).reshape(B, T, C)
    g = O.attn_bwd_f64(qkv.astype(np.float32), dout, B, T, C, NH)
    # the oracle consumes float32 qkv: evaluate on a float32-representable line
    u = g / np.linalg.norm(g)
    eps = 1e-3

    def loss(x):
        o, _ = O.attn_fwd_f64(x.astype(np.float32), B, T, C, NH)
        return float((o * dout).sum())

    # step along u, rounded to float32 -- use the realised step for the slope
    xp = (qkv + eps * u).astype(np.float32)
    xm = (qkv - eps * u).astype(np.float32)
    fd = (loss(xp) - loss(xm))
    realised = float(((xp.astype(np.float64) - xm.astype(np.float64)) * g).sum())
    assert abs(fd - realised) < 2e-3 * abs(realised)


def test_dsum_matches_numpy():
    B, T, C, NH = 2, 5, 12, 3
    d = O.fill_normal(B * T * C, 1).reshape(B, T, C)
    o = O.fill_normal(B * T * C, 2).reshape(B, T, C)
    got = O.dsum_f64(d, o, B, T, C, NH)
    want = (d.astype(np.float64) * o).reshape(B, T, NH, C // NH).sum(-1).transpose(0, 2, 1)
    assert np.allclose(got, want, rtol=1e-13)


def test_unfused_fp32_close_to_fp64():
    B, T, C, NH = 2, 40, 64, 2
    qkv = O.fill_xorshift(B * T * 3 * C, 4321).reshape(B, T, 3 * C)
    dout = O.fill_xorshift(B * T * C, 8765).reshape(B, T, C)
    o32, g32 = O.attn_fwdbwd_f32(qkv, dout, B, T, C, NH, threads=2)
    o64, _ = O.attn_fwd_f64(qkv, B, T, C, NH)
    g64 = O.attn_bwd_f64(qkv, dout, B, T, C, NH)
    assert O.normwise(o32, o64)[0] < 1e-6
    for s in range(3):
        assert O.normwise(g32[:, :, s * C:(s + 1) * C], g64[:, :, s * C:(s + 1) * C])[0] < 1e-5


# ------------------------------------------------------------ golden fixtures
def _golden(name):
    path = os.path.join(GOLDEN, name)
    if not os.path.exists(path):
        pytest.fail("missing fixture %s (run tests/golden/make_golden.py)" % name)
    return np.load(path, allow_pickle=False)


def test_golden_sgemm():
    z = _golden("sgemm_small.npz")
    M, N, K = (int(x) for x in z["mnk"])
    A, B, C0 = z["A"], z["B"], z["C0"]
    assert np.array_equal(A, O.fill_xorshift(M * K, 0x12345678).reshape(M, K))
    got = O.gemm_f32seq(0, 0, M, N, K, 0.5, A, B, 3.0, C0)
    assert np.array_equal(got, z["C_f32seq"])
    assert np.allclose(O.gemm_f64(0, 0, M, N, K, 0.5, A, B, 3.0, C0), z["C_f64"], rtol=1e-14, atol=1e-14)


def test_golden_attention():
    z = _golden("attention_small.npz")
    B, T, C, NH = (int(x) for x in z["btcnh"])
    o, l = O.attn_fwd_f64(z["qkv"], B, T, C, NH)
    assert np.allclose(o, z["out"], rtol=1e-12, atol=1e-13)
    assert np.allclose(l, z["lse"], rtol=1e-12, atol=1e-13)
    g = O.attn_bwd_f64(z["qkv"], z["dout"], B, T, C, NH)
    assert np.allclose(g, z["dqkv"], rtol=1e-10, atol=1e-12)


def test_bf16_rne_matches_torch():
    """The oracle's fp32 -> bfloat16 rounding (used to restate KERNELS id 10)
    equals torch's conversion, which rounds to nearest even: random values,
    exact ties (the halfway pattern 0x8000 with an even and an odd kept bit),
    carries into the exponent, subnormals, signed zeros."""
    import torch
    r = np.random.default_rng(10)
    x = np.concatenate([
        r.standard_normal(100000).astype(np.float32),
        (r.standard_normal(1000) * 1e-39).astype(np.float32),
        np.array([0x3F808000, 0x3F818000, 0x3F7FFFFF, 0x3FFF8000, 0x80000000, 0,
                  0x00008000, 0x00018000], np.uint32).view(np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(O.bf16_rne(x).view(np.uint32), want.view(np.uint32))
    hi, lo = O.bf16x3_split(x)
    assert np.array_equal((x - hi) + hi, x)  # x - hi is exact in fp32
    big = np.abs(x) > 1e-30
    assert (np.abs(x - hi - lo)[big] <= np.abs(x)[big] * 2.0 ** -16).all()


def test_bf16x3_split_at_the_top_of_the_range():
    """Finite values that round to a bfloat16 infinity (|x| > 0x7F7F7FFF, up
    to FLT_MAX) still split exactly: hi is bf16's largest finite value with
    x's sign, x - hi is exact, and hi + lo is within 2^-16 |x|; at the
    threshold itself hi is x rounded as usual. An infinite x splits into
    (+-0x7F7F, +-inf)."""
    t = np.array([0x7F7F7FFF, 0x7F7F8000, 0x7F7FFFFF, 0x7F7F0000, 0xFF7FFFFF, 0xFF7F8001],
                 np.uint32).view(np.float32)
    hi, lo = O.bf16x3_split(t)
    assert np.isfinite(hi).all() and np.isfinite(lo).all()
    assert (np.abs(hi).view(np.uint32) == 0x7F7F0000).all()
    assert np.array_equal((t - hi) + hi, t)
    assert (np.abs(t.astype(np.float64) - hi - lo) <= np.abs(t) * 2.0 ** -16).all()
    # below the threshold nothing changed: plain round to nearest even
    assert O.bf16_rne(t[:1])[0] == hi[0] and O.BF16_FINITE_MAX == float(t[0])
    inf = np.array([np.inf, -np.inf], np.float32)
    hi, lo = O.bf16x3_split(inf)
    assert (np.abs(hi).view(np.uint32) == 0x7F7F0000).all() and np.array_equal(lo, inf)
    assert np.array_equal(np.sign(hi), np.sign(inf))
