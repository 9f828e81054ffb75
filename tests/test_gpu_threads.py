"""Several host threads calling the library at once on one device.

The reference calls gpt_forward/gpt_backward from one host thread per device
(src/train_gpt.cu:400-412), so the replacement must be re-entrant: launch
status, split-K partials, nn partial sums and the flash dS workspace are per
host thread; the per-shape flash plans and per-kernel occupancy tables are
shared and built under a lock on first use. Four threads run a flash forward
+ backward on a shape no other test uses (so the plans are built while the
threads race for them) and a split-K gemm; every thread's results must equal
every other's bit for bit and the oracle to the usual bar. ctypes releases the
GIL during the calls, so they do overlap on the host.
"""
import threading

import numpy as np
import pytest

import bmb
import oracle as O
from gpu_util import dev

pytestmark = pytest.mark.gpu

TOL = 1e-5
NTHREADS = 4


def _work(qkv, dout, A, B, C0, shape, gshape, results, errors, i, barrier):
    import torch
    try:
        Bn, T, C, NH = shape
        M, N, K = gshape
        d_qkv, d_dout = dev(qkv), dev(dout)
        dA, dB, dC = dev(A), dev(B), dev(C0)
        f32 = dict(device="cuda", dtype=torch.float32)
        out, lse = torch.empty(Bn * T * C, **f32), torch.empty(Bn * NH * T, **f32)
        dqkv, dsum = torch.empty(Bn * T * 3 * C, **f32), torch.empty(Bn * NH * T, **f32)
        torch.cuda.synchronize()
        barrier.wait()  # start the library calls together
        bmb.flash_forward(out.data_ptr(), lse.data_ptr(), d_qkv.data_ptr(), Bn, T, C, NH)
        bmb.flash_backward(dqkv.data_ptr(), dsum.data_ptr(), d_dout.data_ptr(), d_qkv.data_ptr(),
                           out.data_ptr(), lse.data_ptr(), Bn, T, C, NH)
        bmb.gemm(False, False, M, N, K, 0.75, dA.data_ptr(), dB.data_ptr(), 1.25, dC.data_ptr())
        torch.cuda.synchronize()
        bmb.check("thread %d" % i)
        results[i] = (out.cpu().numpy(), lse.cpu().numpy(), dqkv.cpu().numpy(), dC.cpu().numpy())
    except Exception as e:  # reported by the main thread
        errors.append((i, repr(e)))


def test_concurrent_host_threads(gpu):
    shape = (2, 777, 256, 4)         # B*NH = 8: planned forward order, persistent backward
    gshape = (257, 129, 3000)        # few output tiles: split-K partials in per-thread scratch
    Bn, T, C, NH = shape
    M, N, K = gshape
    qkv = O.fill_normal(Bn * T * 3 * C, 0x7A7A).reshape(Bn, T, 3 * C)
    dout = O.fill_normal(Bn * T * C, 0x7B7B).reshape(Bn, T, C)
    A = O.fill_xorshift(M * K, 0x1357)
    B = O.fill_xorshift(K * N, 0x2468)
    C0 = O.fill_xorshift(M * N, 0x9999)
    results, errors = [None] * NTHREADS, []
    barrier = threading.Barrier(NTHREADS)
    threads = [threading.Thread(target=_work, args=(qkv, dout, A, B, C0, shape, gshape, results,
                                                    errors, i, barrier))
               for i in range(NTHREADS)]
    print("threads: %d x (flash fwd+bwd B=%d T=%d C=%d NH=%d, gemm %dx%dx%d)"
          % ((NTHREADS,) + shape + gshape), flush=True)
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in threads), "a thread did not finish"
    assert not errors, errors
    for r in results[1:]:
        for a, b in zip(results[0], r):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    out, lse, dqkv, c = results[0]
    ref_o, ref_l = O.attn_fwd_f64(qkv, Bn, T, C, NH)
    assert O.normwise(out.reshape(Bn, T, C), ref_o)[0] < TOL
    assert np.abs(lse.reshape(Bn, NH, T) - ref_l).max() < 1e-5
    ref_d = O.attn_bwd_f64(qkv, dout, Bn, T, C, NH)
    err, bad = O.normwise(dqkv.reshape(Bn, T, 3 * C), ref_d)
    assert bad == 0 and err < TOL
    ref_c = O.gemm_f64(False, False, M, N, K, 0.75, A, B, 1.25, C0)
    err, bad = O.normwise(c, ref_c)
    assert bad == 0 and err < 1e-4
