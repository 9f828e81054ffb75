"""nn.h on the GPU against the fp64 CPU oracle (oracle/oracle_gpt.c).

Bars, per op (normwise = max|got - ref| / max|ref|):
  * exact fp32 arithmetic (one rounding per output: encoder forward,
    residual, add_inplace, bias forward, the cross-entropy backward) and the
    fp32 AdamW restatement: bit-identical;
  * reductions and transcendental ops (layernorm, gelu, softmax, column
    sums, norms): normwise <= 1e-5 against fp64 -- fp32 rounding of sums
    over at most a few thousand terms plus a few ulp of tanh/exp;
  * every reduction is deterministic: a second call gives the same bits.
Shapes cover the GPT-2 small widths (C = 768, 3C, 4C, Vp = 50304), the
gradient-check config (C = 128, V = 65, Vp = 128) and ragged or odd widths
that take the scalar paths.
"""
import numpy as np
import pytest
import torch

import bmb
import oracle as O
from gpu_util import Guarded, dev, host, sync

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _rng(seed):
    return np.random.default_rng(seed)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _nw(got, ref):
    e, bad = O.normwise(_f32(got), np.asarray(ref, np.float64))
    assert bad == 0, "non-finite output"
    return e


def _itok(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to("cuda")


@pytest.mark.parametrize("B,T,C,V", [(4, 64, 128, 65), (2, 33, 100, 11), (8, 1024, 768, 50304),
                                     (3, 7, 6, 5)])
def test_encoder(gpu, B, T, C, V):
    r = _rng(1)
    wte, wpe = _f32(r.standard_normal((V, C))), _f32(r.standard_normal((T, C)))
    # repeated ids exercise the in-order gathering of the backward
    tok = r.integers(0, min(V, 17), B * T).astype(np.int32)
    print("encoder B=%d T=%d C=%d V=%d" % (B, T, C, V), flush=True)
    out = Guarded(B * T * C, poison=True)
    d_wte, d_wpe, d_tok = dev(wte), dev(wpe), _itok(tok)
    bmb.call("encoder_forward", out.ptr, d_tok.data_ptr(), d_wte.data_ptr(), d_wpe.data_ptr(),
             B, T, C)
    sync("encoder_forward")
    assert out.ok()
    ref = O.encoder_fwd(tok, wte, wpe, B, T, C)
    assert np.array_equal(out.get().reshape(B * T, C), ref.astype(np.float32))

    dout = _f32(r.standard_normal((B * T, C)))
    dwte0, dwpe0 = _f32(r.standard_normal(V * C)), _f32(r.standard_normal(T * C))
    res = []
    for _ in range(2):
        dwte, dwpe = Guarded(V * C, fill=dwte0), Guarded(T * C, fill=dwpe0)
        d_dout = dev(dout)
        bmb.call("encoder_backward", dwte.ptr, dwpe.ptr, d_dout.data_ptr(), d_tok.data_ptr(),
                 B, T, C)
        sync("encoder_backward")
        assert dwte.ok() and dwpe.ok()
        res.append((dwte.get(), dwpe.get()))
    rw, rp = O.encoder_bwd(dwte0, dwpe0, dout, tok, B, T, C)
    assert _nw(res[0][0] - dwte0, rw - dwte0) < TOL
    assert _nw(res[0][1] - dwpe0, rp - dwpe0) < TOL
    assert np.array_equal(res[0][0], res[1][0]) and np.array_equal(res[0][1], res[1][1])


@pytest.mark.parametrize("N,C", [(256, 128), (8192, 768), (37, 1024), (50, 100), (9, 1536),
                                 (5, 4), (3, 1)])
def test_layernorm(gpu, N, C):
    r = _rng(2)
    x = _f32(r.standard_normal((N, C)) * 2 + 0.3)
    w, b = _f32(1 + 0.1 * r.standard_normal(C)), _f32(0.1 * r.standard_normal(C))
    print("layernorm N=%d C=%d" % (N, C), flush=True)
    out, mean, rstd = Guarded(N * C, poison=True), Guarded(N, poison=True), Guarded(N, poison=True)
    dx_, dw_, db_ = dev(x), dev(w), dev(b)
    bmb.call("layernorm_forward", out.ptr, mean.ptr, rstd.ptr, dx_.data_ptr(), dw_.data_ptr(),
             db_.data_ptr(), N, C)
    sync("layernorm_forward")
    assert out.ok() and mean.ok() and rstd.ok()
    ro, rm, rr = O.layernorm_fwd(x, w, b, N, C)
    assert _nw(out.get(), ro) < TOL
    assert np.abs(mean.get() - rm).max() <= TOL * max(np.abs(rm).max(), 1e-3)
    assert _nw(rstd.get(), rr) < TOL

    dy = _f32(r.standard_normal((N, C)))
    d0, w0, b0 = _f32(r.standard_normal((N, C))), _f32(r.standard_normal(C)), _f32(r.standard_normal(C))
    res = []
    for _ in range(2):
        dinp, dw, db = Guarded(N * C, fill=d0), Guarded(C, fill=w0), Guarded(C, fill=b0)
        d_dy = dev(dy)
        bmb.call("layernorm_backward", dinp.ptr, dw.ptr, db.ptr, d_dy.data_ptr(),
                 dx_.data_ptr(), dw_.data_ptr(), mean.ptr, rstd.ptr, N, C)
        sync("layernorm_backward")
        assert dinp.ok() and dw.ok() and db.ok()
        res.append((dinp.get(), dw.get(), db.get()))
    # the oracle backward uses the GPU's saved mean / rstd, as the reference does
    rdi, rdw, rdb = O.layernorm_bwd(d0, w0, b0, dy, x, w, mean.get(), rstd.get(), N, C)
    # dinp's terms are rstd * dout * w; when they cancel exactly (C = 1: xhat = 0
    # and dxhat = its own mean) the error is measured against their scale
    terms = float(np.abs(rstd.get()[:, None] * dy * w[None, :]).max())
    ddi = res[0][0].reshape(N, C).astype(np.float64) - d0
    assert np.abs(ddi - (rdi - d0)).max() < TOL * max(np.abs(rdi - d0).max(), terms)
    assert _nw(res[0][1] - w0, rdw - w0) < TOL
    assert _nw(res[0][2] - b0, rdb - b0) < TOL
    for a, b2 in zip(res[0], res[1]):
        assert np.array_equal(a, b2), "layernorm_backward is not deterministic"


@pytest.mark.parametrize("n", [8192 * 3072, 1000, 1, 7])
def test_gelu(gpu, n):
    r = _rng(3)
    x = _f32(r.standard_normal(n) * 3)
    g = _f32(r.standard_normal(n))
    out, dinp = Guarded(n, poison=True), Guarded(n, poison=True)
    d_x, d_g = dev(x), dev(g)
    bmb.call("gelu_forward", out.ptr, d_x.data_ptr(), n)
    bmb.call("gelu_backward", dinp.ptr, d_x.data_ptr(), d_g.data_ptr(), n)
    sync("gelu")
    assert out.ok() and dinp.ok()
    assert _nw(out.get(), O.gelu_fwd(x)) < TOL
    assert _nw(dinp.get(), O.gelu_bwd(x, g)) < TOL


@pytest.mark.parametrize("n", [8192 * 768, 1001, 3])
def test_residual_and_add_inplace(gpu, n):
    r = _rng(4)
    a, b = _f32(r.standard_normal(n)), _f32(r.standard_normal(n))
    out = Guarded(n, poison=True)
    d_a, d_b = dev(a), dev(b)
    bmb.call("residual_forward", out.ptr, d_a.data_ptr(), d_b.data_ptr(), n)
    dst = Guarded(n, fill=a)
    bmb.call("add_inplace", dst.ptr, d_b.data_ptr(), n)
    sync("residual")
    assert out.ok() and dst.ok()
    assert np.array_equal(out.get(), a + b)
    assert np.array_equal(dst.get(), a + b)


@pytest.mark.parametrize("N,C", [(8192, 2304), (8192, 768), (256, 3072), (33, 101), (1, 5)])
def test_bias(gpu, N, C):
    r = _rng(5)
    x, bias = _f32(r.standard_normal((N, C))), _f32(r.standard_normal(C))
    out = Guarded(N * C, fill=x)
    d_bias = dev(bias)
    bmb.call("bias_forward", out.ptr, d_bias.data_ptr(), N, C)
    sync("bias_forward")
    assert out.ok()
    assert np.array_equal(out.get().reshape(N, C), x + bias[None, :])
    dout = _f32(r.standard_normal((N, C)))
    db0 = _f32(r.standard_normal(C))
    got = []
    for _ in range(2):
        db = Guarded(C, fill=db0)
        d_dout = dev(dout)
        bmb.call("bias_backward", db.ptr, d_dout.data_ptr(), N, C)
        sync("bias_backward")
        assert db.ok()
        got.append(db.get())
    assert _nw(got[0] - db0, O.bias_bwd(db0, dout, N, C) - db0) < TOL
    assert np.array_equal(got[0], got[1])
    # The same dout one float off 16-byte alignment takes the 32-bit-load
    # kernel; every column is summed in the same order, so the bits match.
    import torch
    shifted = torch.empty(N * C + 1, device="cuda", dtype=torch.float32)
    shifted[1:].copy_(dev(dout).reshape(-1))
    db = Guarded(C, fill=db0)
    bmb.call("bias_backward", db.ptr, shifted[1:].data_ptr(), N, C)
    sync("bias_backward misaligned")
    assert db.ok()
    assert np.array_equal(db.get(), got[0])


@pytest.mark.parametrize("N,V,Vp", [(256, 65, 128), (64, 50257, 50304), (17, 3000, 3001),
                                    (5, 70000, 70004), (9, 1, 4), (33, 1000, 1000)])
def test_softmax_crossentropy(gpu, N, V, Vp):
    r = _rng(6)
    logits = _f32(r.standard_normal((N, Vp)) * 3)
    logits[:, V:] = 100.0  # padding must take no probability mass
    tg = r.integers(0, V, N).astype(np.int32)
    if N >= 4 and Vp > V:
        tg[0] = V       # target on a padded column: p = 0 -> loss -ln(1e-30)
    print("softmax_xent N=%d V=%d Vp=%d" % (N, V, Vp), flush=True)
    probs, losses = Guarded(N * Vp, poison=True), Guarded(N, poison=True)
    d_logits, d_tg = dev(logits), _itok(tg)
    bmb.call("softmax_crossentropy_forward", probs.ptr, losses.ptr, d_logits.data_ptr(),
             d_tg.data_ptr(), N, V, Vp)
    sync("softmax_crossentropy_forward")
    assert probs.ok() and losses.ok()
    rp, rl = O.softmax_xent_fwd(logits, tg, N, V, Vp)
    p = probs.get().reshape(N, Vp)
    assert _nw(p, rp) < TOL
    assert np.all(p[:, V:] == 0.0)
    assert np.abs(losses.get() - rl).max() < TOL * max(1.0, np.abs(rl).max())
    # backward, from the GPU's own probs: (p - onehot) * scale is one fp32
    # subtraction and one product per entry -> bit-exact
    scale = np.float32(1.0 / N)
    dl = Guarded(N * Vp, poison=True)
    bmb.call("crossentropy_softmax_backward", dl.ptr, probs.ptr, d_tg.data_ptr(), N, V, Vp,
             float(scale))
    sync("crossentropy_softmax_backward")
    assert dl.ok()
    want = p.copy()
    want[np.arange(N), tg] -= np.float32(1.0)
    want = (want * scale).astype(np.float32)
    want[:, V:] = 0.0
    assert np.array_equal(dl.get().reshape(N, Vp), want)


def test_softmax_crossentropy_bad_targets_give_nan(gpu):
    N, V, Vp = 4, 10, 12
    logits = _f32(_rng(7).standard_normal((N, Vp)))
    tg = np.array([-1, Vp, 3, Vp - 1], np.int32)
    probs, losses = Guarded(N * Vp, poison=True), Guarded(N, poison=True)
    d_logits, d_tg = dev(logits), _itok(tg)
    bmb.call("softmax_crossentropy_forward", probs.ptr, losses.ptr, d_logits.data_ptr(),
             d_tg.data_ptr(), N, V, Vp)
    sync("softmax_crossentropy_forward")
    l = losses.get()
    assert np.isnan(l[0]) and np.isnan(l[1]) and np.isfinite(l[2])
    assert l[3] == pytest.approx(-np.log(np.float32(1e-30)), rel=1e-6)


@pytest.mark.parametrize("n", [124475904, 4097, 1])
def test_adamw_bit_exact(gpu, n):
    r = _rng(8)
    p = _f32(r.standard_normal(n))
    m = _f32(r.standard_normal(n) * 1e-3)
    v = _f32(np.abs(r.standard_normal(n)) * 1e-6)
    g = _f32(r.standard_normal(n) * 1e-2)
    args = (3e-4, 0.9, 0.999, 1e-8, 0.1, 7, 0.75)
    dp, dm, dv = Guarded(n, fill=p), Guarded(n, fill=m), Guarded(n, fill=v)
    dg = dev(g)
    print("adamw n=%d" % n, flush=True)
    bmb.call("adamw_update", dp.ptr, dg.data_ptr(), dm.ptr, dv.ptr, n, *args)
    sync("adamw_update")
    assert dp.ok() and dm.ok() and dv.ok()
    k = min(n, 1 << 20)  # the CPU restatement on a prefix keeps this fast
    wp, wm, wv = O.adamw_f32(p[:k], g[:k], m[:k], v[:k], *args)
    assert np.array_equal(dp.get()[:k], wp)
    assert np.array_equal(dm.get()[:k], wm)
    assert np.array_equal(dv.get()[:k], wv)


@pytest.mark.parametrize("n", [124475904, 1000003, 5, 1])
def test_grad_global_norm_and_reduce_mean(gpu, n):
    x = _f32(_rng(9).standard_normal(n) * 1e-2)
    d = dev(x)
    gn = bmb.call("grad_global_norm", d.data_ptr(), n)
    mean = bmb.call("reduce_mean", d.data_ptr(), n)
    bmb.check("norm")
    xd = x.astype(np.float64)
    assert abs(gn - np.sqrt((xd * xd).sum())) <= 1e-6 * np.sqrt((xd * xd).sum())
    assert abs(mean - xd.mean()) <= 1e-6 * max(abs(xd.mean()), np.abs(xd).max() / np.sqrt(n))
    assert bmb.call("grad_global_norm", d.data_ptr(), n) == gn  # deterministic


@pytest.mark.parametrize("n", [124475904 + 3, 5, 0])
def test_zero_buffer(gpu, n):
    buf = Guarded(n, poison=True) if n else Guarded(1, poison=True)
    bmb.call("zero_buffer", buf.ptr, n)
    sync("zero_buffer")
    assert buf.ok()
    if n:
        assert not np.any(buf.get())
    else:
        assert buf.get().view(np.uint32)[0] == 0x7F7F7F7F  # n = 0 touches nothing
