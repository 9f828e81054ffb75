"""Unfused attention (attention.h) on the GPU against the fp64 CPU oracle, and
the fused kernels (flash.h) against it on the same inputs -- the reference's
"vs unfused" check of tools/test_flash.cu, here with the materialised path
itself pinned to fp64.

Bars: out and dq, dk, dv normwise <= 1e-5 (the reference's flash bar,
tools/test_flash.cu:132,226,314); the head permute into qkvr is a copy and is
bit-exact; att rows are probability vectors with exact zeros past the
diagonal; dpreatt may alias datt (src/gpt.cu:371 passes the same buffer).
"""
import numpy as np
import pytest
import torch

import bmb
import oracle as O
from gpu_util import Guarded, dev, sync
from test_gpu_flash import _check_grads

pytestmark = pytest.mark.gpu

TOL = 1e-5
SHAPES = [(2, 64, 128, 4), (4, 256, 384, 6), (3, 100, 384, 6), (1, 1, 64, 2),
          (1, 1024, 768, 12), (1, 1030, 128, 2), (2, 10, 6, 2)]


def _run(B, T, C, NH, alias):
    qkv = O.fill_xorshift(B * T * 3 * C, 4321).reshape(B, T, 3 * C)
    dout = O.fill_xorshift(B * T * C, 8765).reshape(B, T, C)
    print("attention B=%d T=%d C=%d NH=%d alias=%s" % (B, T, C, NH, alias), flush=True)
    d_qkv = dev(qkv)
    out = Guarded(B * T * C, poison=True)
    qkvr = Guarded(4 * B * T * C, poison=True)
    att = Guarded(B * NH * T * T, poison=True)
    bmb.call("attention_forward", out.ptr, qkvr.ptr, att.ptr, d_qkv.data_ptr(), B, T, C, NH)
    sync("attention_forward")
    assert out.ok() and qkvr.ok() and att.ok()
    dqkv = Guarded(B * T * 3 * C, poison=True)
    dqkvr = Guarded(4 * B * T * C, poison=True)
    datt = Guarded(B * NH * T * T, poison=True)
    dpre = datt if alias else Guarded(B * NH * T * T, poison=True)
    d_dout = dev(dout)
    bmb.call("attention_backward", dqkv.ptr, dqkvr.ptr, datt.ptr, dpre.ptr, d_dout.data_ptr(),
             qkvr.ptr, att.ptr, B, T, C, NH)
    sync("attention_backward")
    assert dqkv.ok() and dqkvr.ok() and datt.ok() and dpre.ok()
    return qkv, dout, out.get().reshape(B, T, C), qkvr.get(), att.get(), dqkv.get()


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "B%dT%dC%dNH%d" % s)
def test_unfused_attention_vs_oracle(gpu, shape):
    B, T, C, NH = shape
    hs = C // NH
    qkv, dout, out, qkvr, att, dqkv = _run(B, T, C, NH, alias=True)
    # permute is a copy
    perm = qkv.reshape(B, T, 3, NH, hs).transpose(2, 0, 3, 1, 4).reshape(-1)
    assert np.array_equal(qkvr[:3 * B * T * C], perm)
    # att: probability rows, exact zeros past the diagonal
    A = att.reshape(B, NH, T, T)
    assert np.all(A[:, :, np.triu_indices(T, 1)[0], np.triu_indices(T, 1)[1]] == 0.0)
    assert np.abs(A.astype(np.float64).sum(-1) - 1.0).max() < 1e-5
    ref_o, _ = O.attn_fwd_f64(qkv, B, T, C, NH)
    eo, bad = O.normwise(out, ref_o)
    assert bad == 0 and eo < TOL, eo
    ref_d = O.attn_bwd_f64(qkv, dout, B, T, C, NH)
    errs = _check_grads(dqkv.reshape(B, T, 3 * C), ref_d, C, h16=False)
    print("out %.2e dq %.2e dk %.2e dv %.2e" % (eo, *errs))
    assert max(errs) < TOL


def test_unfused_separate_dpreatt_matches_aliased(gpu):
    r1 = _run(2, 96, 128, 2, alias=True)
    r2 = _run(2, 96, 128, 2, alias=False)
    assert np.array_equal(r1[5], r2[5])


@pytest.mark.parametrize("shape", [(2, 256, 384, 6), (1, 1024, 768, 12), (3, 77, 256, 2)],
                         ids=lambda s: "B%dT%dC%dNH%d" % s)
def test_flash_vs_unfused(gpu, shape):
    """The two GPU paths on the same inputs (the reference's "vs unfused"
    comparison, tools/test_flash.cu:111-132)."""
    B, T, C, NH = shape
    qkv, dout, out_u, _, _, dqkv_u = _run(B, T, C, NH, alias=True)
    d_qkv = dev(qkv)
    out = torch.empty(B * T * C, device="cuda", dtype=torch.float32)
    lse = torch.empty(B * NH * T, device="cuda", dtype=torch.float32)
    dqkv = torch.empty(B * T * 3 * C, device="cuda", dtype=torch.float32)
    dsum = torch.empty(B * NH * T, device="cuda", dtype=torch.float32)
    bmb.flash_forward(out.data_ptr(), lse.data_ptr(), d_qkv.data_ptr(), B, T, C, NH)
    d_dout = dev(dout)
    bmb.flash_backward(dqkv.data_ptr(), dsum.data_ptr(), d_dout.data_ptr(), d_qkv.data_ptr(),
                       out.data_ptr(), lse.data_ptr(), B, T, C, NH)
    sync("flash")
    out_f = out.cpu().numpy()
    # each path against the fp64 oracle first, so a failure names the path
    ref_o, _ = O.attn_fwd_f64(qkv, B, T, C, NH)
    e_f, e_u = O.normwise(out_f, ref_o)[0], O.normwise(out_u, ref_o)[0]
    print("out vs oracle: flash %.2e unfused %.2e" % (e_f, e_u), flush=True)
    assert e_f < TOL and e_u < TOL
    assert O.normwise(out_f, out_u)[0] < TOL
    errs = _check_grads(dqkv.cpu().numpy().reshape(B, T, 3 * C),
                        dqkv_u.reshape(B, T, 3 * C).astype(np.float64), C)
    assert max(errs) < TOL, errs
