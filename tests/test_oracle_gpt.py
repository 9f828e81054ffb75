"""Pins the CPU oracle of the transformer building blocks and the GPT model
(oracle/oracle_gpt.c) without a GPU.

Every check is independent of the oracle's own formulas:
  * each op against torch's fp64 functional form and autograd (layer_norm,
    gelu(approximate="tanh"), log_softmax / cross-entropy, embedding,
    optim.AdamW) -- an independent library implementation;
  * the whole GPT forward against a torch fp64 restatement of GPT-2 built from
    torch.nn.functional, and its backward against torch autograd on it;
  * the GPT backward against fp64 central differences of the oracle's own
    loss along each parameter tensor's gradient direction (the method of
    tools/test_grad.cu:8-26, here at fp64 precision);
  * closed forms: a zero token embedding makes every logit zero, so the loss
    is exactly ln V and dlogits = (1/V - onehot) / N; AdamW's first step from
    zero moments moves each parameter by lr * (g/(|g| + eps) + wd * p).
A plausible slip -- a dropped layernorm correction term, a transposed weight,
a missing 1/N, softmax over the padded columns -- fails at least one of these.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O



@pytest.fixture(autouse=True, scope="module")
def _float64_default():
    """torch computes in fp64 for this module's checks; the previous default
    comes back afterwards, so other modules' tensors keep their float32."""
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(prev)


def _rng(seed):
    return np.random.default_rng(seed)


# ------------------------------------------------------------------ ops
def test_layernorm_matches_torch():
    N, C = 37, 48
    r = _rng(1)
    x = r.standard_normal((N, C)) * 3 + 0.5
    w, b = r.standard_normal(C), r.standard_normal(C)
    dy = r.standard_normal((N, C))
    out, mean, rstd = O.layernorm_fwd(x, w, b, N, C)
    xt = torch.tensor(x, requires_grad=True)
    wt = torch.tensor(w, requires_grad=True)
    bt = torch.tensor(b, requires_grad=True)
    yt = F.layer_norm(xt, (C,), wt, bt, eps=1e-5)
    assert np.abs(out - yt.detach().numpy()).max() < 1e-12
    assert np.allclose(mean, x.mean(1), atol=1e-14)
    assert np.allclose(rstd, 1 / np.sqrt(x.var(1) + 1e-5), rtol=1e-13)
    yt.backward(torch.tensor(dy))
    # accumulate onto non-zero buffers (src/nn.cu:106-109 use +=)
    d0, w0, b0 = r.standard_normal((N, C)), r.standard_normal(C), r.standard_normal(C)
    dinp, dw, db = O.layernorm_bwd(d0, w0, b0, dy, x, w, mean, rstd, N, C)
    assert np.abs(dinp - d0 - xt.grad.numpy()).max() < 1e-12
    assert np.abs(dw - w0 - wt.grad.numpy()).max() < 1e-11
    assert np.abs(db - b0 - bt.grad.numpy()).max() < 1e-11


def test_gelu_matches_torch():
    x = np.linspace(-8, 8, 2001)
    g = _rng(2).standard_normal(x.size)
    xt = torch.tensor(x, requires_grad=True)
    yt = F.gelu(xt, approximate="tanh")
    yt.backward(torch.tensor(g))
    assert np.abs(O.gelu_fwd(x) - yt.detach().numpy()).max() < 1e-14
    assert np.abs(O.gelu_bwd(x, g) - xt.grad.numpy()).max() < 1e-13


def test_softmax_xent_matches_torch_and_masks_padding():
    N, V, Vp = 9, 65, 128
    r = _rng(3)
    logits = r.standard_normal((N, Vp)) * 4
    logits[:, V:] = 50.0  # padding columns must not take probability mass
    tg = r.integers(0, V, N).astype(np.int32)
    probs, losses = O.softmax_xent_fwd(logits, tg, N, V, Vp)
    lt = torch.tensor(logits[:, :V], requires_grad=True)
    ls = F.log_softmax(lt, dim=1)
    assert np.abs(probs[:, :V] - ls.exp().detach().numpy()).max() < 1e-14
    assert np.all(probs[:, V:] == 0.0)
    ref_loss = F.nll_loss(ls, torch.tensor(tg, dtype=torch.long), reduction="none")
    assert np.abs(losses - ref_loss.detach().numpy()).max() < 1e-13
    ref_loss.mean().backward()
    d = O.xent_bwd(probs, tg, N, V, Vp, 1.0 / N)
    assert np.abs(d[:, :V] - lt.grad.numpy()).max() < 1e-14
    assert np.all(d[:, V:] == 0.0)
    # targets on padding, and out of range
    tg2 = np.array([V, Vp - 1, -1, Vp] + [0] * (N - 4), np.int32)
    _, l2 = O.softmax_xent_fwd(logits, tg2, N, V, Vp)
    assert l2[0] == pytest.approx(-math.log(1e-30)) and l2[1] == l2[0]
    assert np.isnan(l2[2]) and np.isnan(l2[3])


def test_encoder_matches_torch():
    B, T, C, V = 3, 7, 8, 5
    r = _rng(4)
    wte, wpe = r.standard_normal((V, C)), r.standard_normal((T, C))
    tok = r.integers(0, V, (B, T)).astype(np.int32)
    out = O.encoder_fwd(tok, wte, wpe, B, T, C)
    wt = torch.tensor(wte, requires_grad=True)
    pt = torch.tensor(wpe, requires_grad=True)
    y = F.embedding(torch.tensor(tok, dtype=torch.long), wt) + pt[None]
    assert np.abs(out - y.detach().numpy().reshape(B * T, C)).max() == 0.0
    g = r.standard_normal((B, T, C))
    y.backward(torch.tensor(g))
    dwte, dwpe = O.encoder_bwd(np.ones(V * C), np.zeros(T * C), g, tok, B, T, C)
    assert np.abs(dwte - 1.0 - wt.grad.numpy().reshape(-1)).max() < 1e-14
    assert np.abs(dwpe - pt.grad.numpy().reshape(-1)).max() < 1e-14


def test_bias_bwd_is_column_sum():
    r = _rng(5)
    d = r.standard_normal((11, 6))
    db = O.bias_bwd(np.full(6, 2.0), d, 11, 6)
    assert np.abs(db - 2.0 - d.sum(0)).max() < 1e-14


def test_adamw_first_step_closed_form():
    r = _rng(6)
    n = 1000
    p = r.standard_normal(n).astype(np.float32)
    g = (r.standard_normal(n) * 1e-2).astype(np.float32)
    lr, b1, b2, eps, wd = 1e-3, 0.9, 0.999, 1e-8, 0.1
    p1, m1, v1 = O.adamw_f32(p, g, np.zeros(n, np.float32), np.zeros(n, np.float32),
                             lr, b1, b2, eps, wd, 1, 1.0)
    pd, gd = p.astype(np.float64), g.astype(np.float64)
    want = pd - lr * (gd / (np.abs(gd) + eps) + wd * pd)
    assert np.abs(p1 - want).max() < 4e-7 * np.abs(want).max()
    assert np.abs(m1 - 0.1 * gd).max() <= 1e-7 * np.abs(gd).max()


def test_adamw_matches_torch_optim():
    """Five steps with grad_scale against torch.optim.AdamW in fp64: the same
    update written differently (lr/bc1 * m / (sqrt(v)/sqrt(bc2) + eps))."""
    r = _rng(7)
    n = 4096
    p = r.standard_normal(n).astype(np.float32)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    lr, b1, b2, eps, wd, gs = 3e-3, 0.9, 0.999, 1e-8, 0.1, 0.5
    pt = torch.tensor(p.astype(np.float64), requires_grad=True)
    opt = torch.optim.AdamW([pt], lr=lr, betas=(b1, b2), eps=eps, weight_decay=wd)
    for step in range(1, 6):
        g = (r.standard_normal(n) * 1e-2).astype(np.float32)
        p, m, v = O.adamw_f32(p, g, m, v, lr, b1, b2, eps, wd, step, gs)
        pt.grad = torch.tensor(g.astype(np.float64) * gs)
        opt.step()
    ref = pt.detach().numpy()
    assert np.abs(p - ref).max() < 1e-6 * np.abs(ref).max()


# ------------------------------------------------------------------ GPT
CFG_SMALL = (16, 11, 16, 2, 2, 8)  # T, V, Vp, L, NH, C


def _init_params(cfg, seed, std=0.02):
    sizes = O.gpt_param_sizes(cfg)
    r = _rng(seed)
    p = r.standard_normal(sum(sizes)) * std
    off = np.cumsum([0] + sizes)
    for t in (2, 8, 14):  # layernorm weights near 1
        p[off[t]:off[t + 1]] += 1.0
    return p, sizes, off


def _torch_gpt(cfg, B, T, params, tokens, targets):
    """GPT-2 forward in torch fp64 from torch.nn.functional pieces (the
    architecture of src/gpt.cu:228-300)."""
    maxT, V, Vp, L, NH, C = cfg
    sizes = O.gpt_param_sizes(cfg)
    ts = torch.split(params, sizes)
    wte, wpe = ts[0].view(Vp, C), ts[1].view(maxT, C)
    ln1w, ln1b = ts[2].view(L, C), ts[3].view(L, C)
    qkvw, qkvb = ts[4].view(L, 3 * C, C), ts[5].view(L, 3 * C)
    apw, apb = ts[6].view(L, C, C), ts[7].view(L, C)
    ln2w, ln2b = ts[8].view(L, C), ts[9].view(L, C)
    fcw, fcb = ts[10].view(L, 4 * C, C), ts[11].view(L, 4 * C)
    fpw, fpb = ts[12].view(L, C, 4 * C), ts[13].view(L, C)
    lnfw, lnfb = ts[14], ts[15]
    tok = torch.tensor(tokens, dtype=torch.long).view(B, T)
    x = F.embedding(tok, wte) + wpe[:T][None]
    hs = C // NH
    mask = torch.ones(T, T, dtype=torch.bool).tril()
    for l in range(L):
        h = F.layer_norm(x, (C,), ln1w[l], ln1b[l], eps=1e-5)
        qkv = F.linear(h, qkvw[l], qkvb[l])
        q, k, v = qkv.split(C, dim=2)
        q = q.view(B, T, NH, hs).transpose(1, 2)
        k = k.view(B, T, NH, hs).transpose(1, 2)
        v = v.view(B, T, NH, hs).transpose(1, 2)
        s = (q @ k.transpose(2, 3)) / math.sqrt(hs)
        a = torch.softmax(s.masked_fill(~mask, float("-inf")), dim=-1)
        y = (a @ v).transpose(1, 2).reshape(B, T, C)
        x = x + F.linear(y, apw[l], apb[l])
        h = F.layer_norm(x, (C,), ln2w[l], ln2b[l], eps=1e-5)
        h = F.gelu(F.linear(h, fcw[l], fcb[l]), approximate="tanh")
        x = x + F.linear(h, fpw[l], fpb[l])
    x = F.layer_norm(x, (C,), lnfw, lnfb, eps=1e-5)
    logits = x @ wte.t()
    ls = F.log_softmax(logits[..., :V], dim=-1)
    tg = torch.tensor(targets, dtype=torch.long).view(B, T)
    return F.nll_loss(ls.reshape(B * T, V), tg.reshape(-1)), logits.reshape(B * T, Vp)


@pytest.mark.parametrize("cfg,B,T", [(CFG_SMALL, 2, 16), ((12, 23, 32, 1, 4, 16), 3, 12)])
def test_gpt_matches_torch_autograd(cfg, B, T):
    p, sizes, off = _init_params(cfg, 11, std=0.3)
    r = _rng(12)
    tok = r.integers(0, cfg[1], B * T).astype(np.int32)
    tgt = r.integers(0, cfg[1], B * T).astype(np.int32)
    loss, _, grads, logits = O.gpt_forward_backward(cfg, B, T, p, tok, tgt, logits=True)
    pt = torch.tensor(p, requires_grad=True)
    lt, logt = _torch_gpt(cfg, B, T, pt, tok, tgt)
    lt.backward()
    assert abs(loss - lt.item()) < 1e-12
    assert np.abs(logits - logt.detach().numpy()).max() < 1e-12
    gt = pt.grad.numpy()
    for t, name in enumerate(O.PARAM_NAMES):
        a, b = grads[off[t]:off[t + 1]], gt[off[t]:off[t + 1]]
        scale = max(np.abs(b).max(), 1e-300)
        assert np.abs(a - b).max() <= 1e-10 * scale + 1e-300, name


def test_gpt_directional_derivatives_fp64():
    """tools/test_grad.cu's method in fp64: along u = g/||g|| per tensor,
    (L(p + eps u) - L(p - eps u)) / 2 eps must equal ||g||."""
    cfg, B, T = CFG_SMALL, 2, 16
    p, sizes, off = _init_params(cfg, 21, std=0.3)
    r = _rng(22)
    tok = r.integers(0, cfg[1], B * T).astype(np.int32)
    tgt = r.integers(0, cfg[1], B * T).astype(np.int32)
    _, _, g, _ = O.gpt_forward_backward(cfg, B, T, p, tok, tgt)
    eps = 1e-5
    for t, name in enumerate(O.PARAM_NAMES):
        gt = g[off[t]:off[t + 1]]
        gn = np.linalg.norm(gt)
        if gn < 1e-12:
            continue
        u = np.zeros_like(p)
        u[off[t]:off[t + 1]] = gt / gn
        lp = O.gpt_forward_backward(cfg, B, T, p + eps * u, tok, tgt, grads=False)[0]
        lm = O.gpt_forward_backward(cfg, B, T, p - eps * u, tok, tgt, grads=False)[0]
        num = (lp - lm) / (2 * eps)
        assert abs(num - gn) < 1e-6 * gn, (name, num, gn)


def test_gpt_zero_embedding_gives_ln_v():
    cfg, B, T = CFG_SMALL, 2, 16
    p, sizes, off = _init_params(cfg, 31, std=0.3)
    p[off[0]:off[1]] = 0.0  # wte = 0 -> logits = lnf @ wte^T = 0
    r = _rng(32)
    tok = r.integers(0, cfg[1], B * T).astype(np.int32)
    tgt = r.integers(0, cfg[1], B * T).astype(np.int32)
    loss, losses, _, logits = O.gpt_forward_backward(cfg, B, T, p, tok, tgt, logits=True)
    assert np.all(logits == 0.0)
    assert abs(loss - math.log(cfg[1])) < 1e-15
    assert np.abs(losses - math.log(cfg[1])).max() < 1e-15
