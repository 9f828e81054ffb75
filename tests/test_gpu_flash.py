"""Fused attention on the GPU against the fp64 CPU oracle.

Mirrors tools/test_flash.cu: xorshift inputs (qkv seed 1234, dout seed 99;
ragged shapes 4321/8765), every forward and backward config, outputs poisoned
with 0x7f before the call, normwise error on out and on dq, dk, dv SEPARATELY
with the reference's 1e-5 bar (test_flash.cu:132,226,314), and the ragged
shapes of test_flash.cu:336-340. The oracle is the fp64 textbook attention
and its analytic backward instead of the GPU unfused path.

Besides 1e-5, every config is held to a bar derived from the arithmetic the
reference's kernels use: 4x the error that fp32 arithmetic itself makes on
the same inputs (the oracle's fp32 restatement of src/attention.cu, against
the same fp64 values), per output, with a floor of 2^-21 (a 22-bit operand
alone is 2^-22 from its fp32 value: at T = 1, out = V's representation). The
fp16x3 default kernels carry each operand as 22 significant bits and
measure 1-1.3x that fp32 error; a kernel that dropped a cross term (2^-11)
or four bits (16x) would fail it.
"""
import numpy as np
import pytest

import bmb
import oracle as O
from gpu_util import Guarded, dev, sync

pytestmark = pytest.mark.gpu

TOL = 1e-5
FP32_FACTOR = 4.0      # the derived bar: this many times fp32 arithmetic's own error
FP32_FLOOR = 2.0 ** -21


def _is_h16_bwd(cfg):
    cfg = bmb.flash_default_bwd_config() if cfg is None else cfg
    return "fp16x3" in bmb.flash_bwd_configs()[cfg]


def _run_fwd(qkv, B, T, C, NH, cfg=None):
    NHT = B * NH * T
    d_qkv = dev(qkv)
    out = Guarded(B * T * C, poison=True)
    lse = Guarded(NHT, poison=True)
    print("flash fwd cfg=%s B=%d T=%d C=%d NH=%d" % (cfg, B, T, C, NH), flush=True)
    if cfg is None:
        bmb.flash_forward(out.ptr, lse.ptr, d_qkv.data_ptr(), B, T, C, NH)
    else:
        assert bmb.flash_forward_cfg(cfg, out.ptr, lse.ptr, d_qkv.data_ptr(), B, T, C, NH)
    sync("flash forward")
    assert out.ok() and lse.ok(), "canary overwritten"
    return d_qkv, out, lse


def _run_bwd(d_qkv, out, lse, dout, B, T, C, NH, cfg=None):
    d_dout = dev(dout)
    dqkv = Guarded(B * T * 3 * C, poison=True)
    dsum = Guarded(B * NH * T, poison=True)
    print("flash bwd cfg=%s B=%d T=%d C=%d NH=%d" % (cfg, B, T, C, NH), flush=True)
    args = (dqkv.ptr, dsum.ptr, d_dout.data_ptr(), d_qkv.data_ptr(), out.ptr, lse.ptr,
            B, T, C, NH)
    if cfg is None:
        bmb.flash_backward(*args)
    else:
        assert bmb.flash_backward_cfg(cfg, *args)
    sync("flash backward")
    assert dqkv.ok() and dsum.ok(), "canary overwritten"
    return dqkv.get().reshape(B, T, 3 * C), dsum.get().reshape(B, NH, T)


def _check_grads(got, want, C, h16=True, zero=None):
    """Normwise error of dq, dk, dv separately (test_flash.cu:292-314).

    A slice whose largest |ref| is below 1e-2 of the largest over all three
    is zero in exact arithmetic (T = 1: a one-key softmax has zero gradient,
    so dq = dk = 0 and only dv is non-zero); what the kernel returns there is
    rounding noise of the cancellation dP - D, so it is measured against a
    fraction of the gradient's scale (the largest |ref|), not against zero:
    1e-2 of it for fp32 products, whose noise is ~2^-24 of the scale, and
    the whole scale for the fp16x3 kernels, whose operands carry 22
    significant bits (noise ~2^-22 of the scale). `zero`, if a list, gets
    one flag per slice: whether it is such a slice."""
    gmax = float(np.abs(want).max())
    errs = []
    for s, name in enumerate("qkv"):
        g = got[:, :, s * C:(s + 1) * C]
        w = want[:, :, s * C:(s + 1) * C]
        e, bad = O.normwise(g, w)
        assert bad == 0, "non-finite d%s" % name
        wmax = float(np.abs(w).max()) if w.size else 0.0
        is_zero = wmax < 1e-2 * gmax
        if is_zero:
            e = float(np.abs(g.astype(np.float64) - w).max()) / (gmax if h16 else 1e-2 * gmax)
        if zero is not None:
            zero.append(is_zero)
        errs.append(e)
    return errs


def _fp32_errors(qkv, dout, ref_o, ref_d, B, T, C, NH):
    """The normwise errors (out, dq, dk, dv) that fp32 arithmetic makes on
    these inputs: the oracle's fp32 unfused attention (src/attention.cu
    semantics) against the fp64 values."""
    o32, d32 = O.attn_fwdbwd_f32(qkv, dout, B, T, C, NH)
    eo = O.normwise(o32, ref_o)[0]
    return [eo] + _check_grads(d32, ref_d, C, h16=False)


def _derived_bar(e32):
    return max(FP32_FACTOR * e32, FP32_FLOOR)


def _case(B, T, C, NH, seed_qkv, seed_dout, fcfg=None, bcfg=None):
    qkv = O.fill_xorshift(B * T * 3 * C, seed_qkv).reshape(B, T, 3 * C)
    dout = O.fill_xorshift(B * T * C, seed_dout).reshape(B, T, C)
    d_qkv, out, lse = _run_fwd(qkv, B, T, C, NH, fcfg)
    ref_o, ref_l = O.attn_fwd_f64(qkv, B, T, C, NH)
    o = out.get().reshape(B, T, C)
    eo, bad = O.normwise(o, ref_o)
    assert bad == 0
    el = np.abs(lse.get().reshape(B, NH, T) - ref_l).max()
    dq, ds = _run_bwd(d_qkv, out, lse, dout, B, T, C, NH, bcfg)
    ref_d = O.attn_bwd_f64(qkv, dout, B, T, C, NH)
    zero = []
    eq, ek, ev = _check_grads(dq, ref_d, C, _is_h16_bwd(bcfg), zero)
    ref_ds = O.dsum_f64(dout, o, B, T, C, NH)
    ed = np.abs(ds - ref_ds).max() / max(np.abs(ref_ds).max(), 1e-30)
    e32 = _fp32_errors(qkv, dout, ref_o, ref_d, B, T, C, NH)
    print("B=%d T=%d C=%d NH=%d out %.2e lse %.2e dq %.2e dk %.2e dv %.2e dsum %.2e"
          % (B, T, C, NH, eo, el, eq, ek, ev, ed))
    print("  fp32 arithmetic: out %.2e dq %.2e dk %.2e dv %.2e" % tuple(e32))
    assert eo < TOL and el < 1e-5 and ed < 1e-5
    assert eq < TOL and ek < TOL and ev < TOL
    assert eo < _derived_bar(e32[0]), ("out", eo, e32[0])
    for name, e, e_32, z in zip("qkv", (eq, ek, ev), e32[1:], zero):
        if not z:  # (an exactly-zero slice has no fp32 error to scale)
            assert e < _derived_bar(e_32), ("d" + name, e, e_32)


@pytest.mark.parametrize("shape", [(3, 100, 384, 6), (2, 33, 384, 6), (1, 1, 384, 6),
                                   (2, 129, 256, 8), (5, 200, 128, 4), (2, 70, 256, 2),
                                   (1, 64, 64, 1), (2, 96, 768, 12)],
                         ids=lambda s: "B%dT%dC%dNH%d" % s)
def test_ragged_shapes(gpu, shape):
    """tools/test_flash.cu:336-340 plus hs=128 and tile-aligned cases."""
    _case(*shape, 4321, 8765)


def _random_flash_shapes(n, seed):
    r = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        hs = int(r.choice([32, 64, 128]))
        NH = int(r.integers(1, 9))
        out.append((int(r.integers(1, 5)), int(r.integers(1, 900)), hs * NH, NH))
    return out


@pytest.mark.parametrize("shape", _random_flash_shapes(6, 99), ids=lambda s: "B%dT%dC%dNH%d" % s)
def test_random_shapes(gpu, shape):
    """Default configs on random (B, T, head size, heads), fixed seed: the same
    1e-5 and derived bars against fp64 as every other case."""
    _case(*shape, 2468, 1357)


MAX_CFGS = 10  # more than either table holds; ids past the end are skipped


@pytest.mark.parametrize("cfg", range(MAX_CFGS))
def test_every_forward_config(gpu, cfg):
    if cfg >= len(bmb.flash_configs()):
        pytest.skip("no forward config %d" % cfg)
    _case(2, 256, 384, 6, 1234, 99, fcfg=cfg)
    _case(3, 200, 256, 2, 4321, 8765, fcfg=cfg)  # hs 128, ragged T


def _range_inputs(kind, B, T, C):
    """qkv with magnitudes that a plain fp16 conversion would lose: whole
    inputs far above 65504 or below fp16's normal range, and single key rows
    (one 32-key tile's worth) of K and V scaled up or down by up to 2^40 or
    zeroed, which moves the per-tile and running exponents mid-sequence."""
    qkv = O.fill_xorshift(B * T * 3 * C, 1234).reshape(B, T, 3 * C).astype(np.float64)
    if kind == "big":
        qkv *= 1e4
    elif kind == "small":
        qkv *= 1e-4
    elif kind == "tiny":
        qkv *= 1e-30
    elif kind == "mixed":
        k, v = qkv[:, :, C:2 * C], qkv[:, :, 2 * C:]
        k[:, 40:72] *= 2.0 ** 20     # one tile of loud keys
        v[:, 100:130] *= 2.0 ** 40   # V grows late: the running exponent moves
        v[:, 10:20] *= 2.0 ** -40    # quiet values inside a tile
        v[:, 140:180] = 0.0          # a tile of zero values
        k[:, 200:232] = 0.0          # a tile of zero keys
        qkv[:, 5:9, :C] *= 2.0 ** -30  # quiet queries
    return qkv.astype(np.float32)


@pytest.mark.parametrize("kind", ["big", "small", "tiny", "mixed"])
def test_forward_input_range(gpu, kind):
    """Every forward config against the fp64 oracle on inputs far from unit
    scale. out is held to the reference's normwise 1e-5. lse is a score-sized
    quantity: an fp32 dot product is only exact to ~2^-24 sum_d |q_d k_d|,
    whatever the cancellation, so its error is held to 1e-5 of
    max(1, max_j sum_d |q_id k_jd| / sqrt(hs)) over the query's keys."""
    B, T, C, NH = 2, 257, 256, 4
    hs = C // NH
    qkv = _range_inputs(kind, B, T, C)
    ref_o, ref_l = O.attn_fwd_f64(qkv, B, T, C, NH)
    x = np.abs(qkv.astype(np.float64)).reshape(B, T, 3, NH, hs)
    qa, ka = x[:, :, 0].transpose(0, 2, 1, 3), x[:, :, 1].transpose(0, 2, 1, 3)
    mag = (qa @ ka.transpose(0, 1, 3, 2)) / np.sqrt(hs)        # (B, NH, T, T)
    mag = np.where(np.tril(np.ones((T, T), bool)), mag, 0.0).max(axis=3)
    for cfg in range(len(bmb.flash_configs())):
        _, out, lse = _run_fwd(qkv, B, T, C, NH, cfg)
        eo, bad = O.normwise(out.get().reshape(B, T, C), ref_o)
        el = np.max(np.abs(lse.get().reshape(B, NH, T) - ref_l) / np.maximum(1.0, mag))
        print("%s cfg %d: out %.2e lse %.2e" % (kind, cfg, eo, el))
        assert bad == 0 and eo < TOL and el < 1e-5, (kind, cfg, eo, el)


def _bwd_range_inputs(kind, B, T, C):
    """(qkv, dout) whose magnitudes leave fp16's range while the attention
    stays as well conditioned as at unit scale, so an fp32 backward meets the
    same bar: scores are kept unchanged (Q scaled up exactly as K is scaled
    down), or whole tensors are scaled (every gradient scales with them), or
    single 32-row tiles of V and dO are scaled up, down or zeroed, which
    moves the per-tile and running exponents of the backward mid-sequence."""
    qkv = O.fill_xorshift(B * T * 3 * C, 1234).reshape(B, T, 3 * C).astype(np.float64)
    dout = O.fill_xorshift(B * T * C, 99).reshape(B, T, C).astype(np.float64)
    q, k, v = qkv[:, :, :C], qkv[:, :, C:2 * C], qkv[:, :, 2 * C:]
    if kind == "qk_skew":
        q *= 2.0 ** 20
        k *= 2.0 ** -20
    elif kind == "v_big":
        v *= 1e20
    elif kind == "dout_tiny":
        dout *= 1e-30
    elif kind == "tiles":
        v[:, 100:130] *= 2.0 ** 40   # loud values late: the running exponents move
        v[:, 10:20] *= 2.0 ** -40    # quiet values inside a tile
        v[:, 140:180] = 0.0          # zero values
        dout[:, 64:96] *= 2.0 ** 30  # one tile of loud output gradients
        dout[:, 200:232] = 0.0       # a tile of zero output gradients
        q[:, 5:9] *= 2.0 ** -30      # quiet queries
    return qkv.astype(np.float32), dout.astype(np.float32)


@pytest.mark.parametrize("kind", ["qk_skew", "v_big", "dout_tiny", "tiles"])
def test_backward_input_range(gpu, kind):
    """Every backward config against the fp64 oracle on the inputs of
    _bwd_range_inputs, dq, dk and dv each held to the reference's normwise
    1e-5 (and dsum to 1e-5 of its largest magnitude)."""
    B, T, C, NH = 2, 257, 256, 4
    qkv, dout = _bwd_range_inputs(kind, B, T, C)
    d_qkv, out, lse = _run_fwd(qkv, B, T, C, NH)
    ref_d = O.attn_bwd_f64(qkv, dout, B, T, C, NH)
    ref_ds = O.dsum_f64(dout, out.get().reshape(B, T, C), B, T, C, NH)
    for cfg in range(len(bmb.flash_bwd_configs())):
        dq, ds = _run_bwd(d_qkv, out, lse, dout, B, T, C, NH, cfg)
        # Plain per-slice normwise: no slice is zero in exact arithmetic here,
        # and scaling makes some far smaller than the others on purpose.
        errs = []
        for s in range(3):
            e, bad = O.normwise(dq[:, :, s * C:(s + 1) * C], ref_d[:, :, s * C:(s + 1) * C])
            errs.append(e if bad == 0 else float("inf"))
        eq, ek, ev = errs
        ed = np.abs(ds - ref_ds).max() / max(np.abs(ref_ds).max(), 1e-300)
        print("%s bwd cfg %d: dq %.2e dk %.2e dv %.2e dsum %.2e" % (kind, cfg, eq, ek, ev, ed))
        assert eq < TOL and ek < TOL and ev < TOL and ed < 1e-5, (kind, cfg, eq, ek, ev, ed)


@pytest.mark.parametrize("cfg", range(MAX_CFGS))
def test_every_backward_config(gpu, cfg):
    if cfg >= len(bmb.flash_bwd_configs()):
        pytest.skip("no backward config %d" % cfg)
    _case(2, 256, 384, 6, 1234, 99, bcfg=cfg)
    _case(3, 200, 256, 2, 4321, 8765, bcfg=cfg)  # hs 128, ragged T
    _case(1, 70, 96, 3, 4321, 8765, bcfg=cfg)    # hs 32, B*NH not a multiple of 8


@pytest.mark.parametrize("shape", [(2, 500, 256, 2), (3, 700, 384, 6), (1, 1024, 256, 8),
                                   (1, 2000, 64, 2)],
                         ids=lambda s: "B%dT%dC%dNH%d" % s)
def test_long_blocks_split(gpu, shape):
    """T long enough that the default backward splits its longest dK/dV and
    dQ blocks in two halves accumulated into zeroed rows (ragged T, every
    head size)."""
    _case(*shape, 4321, 8765)


def test_reference_default_shape(gpu):
    """test_flash.cu default: B=16 T=256 C=384 NH=6, seeds 1234 / 99."""
    _case(16, 256, 384, 6, 1234, 99)


def test_benchmark_shape_every_batch(gpu):
    """BASELINE config 4 (B=8, H=12, T=1024, d=64, q/k/v/dO N(0,1)) launched
    in full with the default configs, and all 8 batches (96 heads) checked
    against the fp64 oracle: out, lse and dsum, and dq, dk, dv separately,
    each within 1e-5 and within the derived bar of fp32 arithmetic's own
    error on that batch."""
    B, T, C, NH = 8, 1024, 768, 12
    qkv = O.fill_normal(B * T * 3 * C, 0xBEEF).reshape(B, T, 3 * C)
    dout = O.fill_normal(B * T * C, 0xD0D0).reshape(B, T, C)
    d_qkv, out, lse = _run_fwd(qkv, B, T, C, NH)
    dq, ds = _run_bwd(d_qkv, out, lse, dout, B, T, C, NH)
    o = out.get().reshape(B, T, C)
    l = lse.get().reshape(B, NH, T)
    for b in range(B):
        sl = slice(b, b + 1)
        ref_o, ref_l = O.attn_fwd_f64(qkv[sl], 1, T, C, NH)
        ref_d = O.attn_bwd_f64(qkv[sl], dout[sl], 1, T, C, NH)
        ref_ds = O.dsum_f64(dout[sl], o[sl], 1, T, C, NH)
        eo = O.normwise(o[sl], ref_o)[0]
        el = np.abs(l[sl] - ref_l).max()
        ed = np.abs(ds[sl] - ref_ds).max() / np.abs(ref_ds).max()
        eq, ek, ev = _check_grads(dq[sl], ref_d, C)
        e32 = _fp32_errors(qkv[sl], dout[sl], ref_o, ref_d, 1, T, C, NH)
        print("batch %d: out %.2e lse %.2e dsum %.2e dq %.2e dk %.2e dv %.2e | fp32 %s"
              % (b, eo, el, ed, eq, ek, ev, " ".join("%.2e" % x for x in e32)), flush=True)
        assert eo < TOL and el < 1e-5 and ed < 1e-5
        for e, e_32 in zip((eo, eq, ek, ev), e32):
            assert e < TOL and e < _derived_bar(e_32), (b, e, e_32)


@pytest.mark.parametrize("shape", [(8, 1024, 768, 12), (2, 1000, 256, 4), (4, 256, 384, 6),
                                   (3, 700, 384, 6)], ids=lambda s: "B%dT%dC%dNH%d" % s)
def test_forward_order_matches_formula_order(gpu, shape):
    """The default forward config places its (query block, head) items in a
    host-planned order when the whole grid is resident at once (B*NH a
    multiple of 8); config 2 is the same kernel with the plain formula order.
    Every query row's arithmetic is the same either way, so out and lse must
    match bit for bit on every batch: the plan covers every item once."""
    B, T, C, NH = shape
    qkv = O.fill_normal(B * T * 3 * C, 0xFACE).reshape(B, T, 3 * C)
    names = bmb.flash_configs()
    assert "snake" in names[0] and "snake" not in names[2]
    _, out0, lse0 = _run_fwd(qkv, B, T, C, NH, cfg=0)
    _, out2, lse2 = _run_fwd(qkv, B, T, C, NH, cfg=2)
    assert np.array_equal(out0.get().view(np.uint32), out2.get().view(np.uint32))
    assert np.array_equal(lse0.get().view(np.uint32), lse2.get().view(np.uint32))


@pytest.mark.parametrize("shape", [(8, 1024, 768, 12), (1, 2000, 64, 2), (3, 700, 384, 6)],
                         ids=lambda s: "B%dT%dC%dNH%d" % s)
def test_backward_deterministic(gpu, shape):
    """Two backward calls on the same inputs give the same bits: the halves
    of a split block are the only atomic adds, exactly two onto a zeroed row,
    and the persistent schedule is fixed per shape."""
    B, T, C, NH = shape
    qkv = O.fill_normal(B * T * 3 * C, 0xBEEF).reshape(B, T, 3 * C)
    dout = O.fill_normal(B * T * C, 0xD0D0).reshape(B, T, C)
    d_qkv, out, lse = _run_fwd(qkv, B, T, C, NH)
    first, _ = _run_bwd(d_qkv, out, lse, dout, B, T, C, NH)
    second, _ = _run_bwd(d_qkv, out, lse, dout, B, T, C, NH)
    assert np.array_equal(first.view(np.uint32), second.view(np.uint32))


def test_many_heads_fall_back(gpu):
    """B*NH above 65535 does not fit the persistent backward's work-list
    encoding: the default config declines (nothing launched) and the
    wrapper runs a recompute config instead. The first batches are checked
    against the oracle (it works per (b, h))."""
    B, T, C, NH = 65537, 3, 32, 1
    qkv = O.fill_xorshift(B * T * 3 * C, 4321).reshape(B, T, 3 * C)
    dout = O.fill_xorshift(B * T * C, 8765).reshape(B, T, C)
    d_qkv, out, lse = _run_fwd(qkv, B, T, C, NH)
    import torch
    x = torch.empty(B * T * 3 * C, device="cuda", dtype=torch.float32)
    d_dout = dev(dout)
    assert not bmb.flash_backward_cfg(bmb.flash_default_bwd_config(), x.data_ptr(), x.data_ptr(),
                                      d_dout.data_ptr(), d_qkv.data_ptr(), out.ptr, lse.ptr,
                                      B, T, C, NH)
    dq, _ = _run_bwd(d_qkv, out, lse, dout, B, T, C, NH)
    nb = 4
    ref_o, _ = O.attn_fwd_f64(qkv[:nb], nb, T, C, NH)
    assert O.normwise(out.get().reshape(B, T, C)[:nb], ref_o)[0] < TOL
    ref_d = O.attn_bwd_f64(qkv[:nb], dout[:nb], nb, T, C, NH)
    for e in _check_grads(dq[:nb], ref_d, C, h16=False):  # the fallback is an fp32 config
        assert e < TOL


def test_bad_head_size_rejected(gpu):
    """_cfg returns false and launches nothing for hs outside {32, 64, 128}."""
    import torch
    x = torch.zeros(3 * 2 * 4 * 96, device="cuda", dtype=torch.float32)
    assert not bmb.flash_forward_cfg(0, x.data_ptr(), x.data_ptr(), x.data_ptr(), 2, 4, 96, 2)
    assert not bmb.flash_forward_cfg(99, x.data_ptr(), x.data_ptr(), x.data_ptr(), 2, 4, 128, 2)
    assert not bmb.flash_backward_cfg(-1, x.data_ptr(), x.data_ptr(), x.data_ptr(),
                                      x.data_ptr(), x.data_ptr(), x.data_ptr(), 2, 4, 128, 2)
