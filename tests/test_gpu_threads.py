"""Several host threads calling the library at once on one device.

The reference calls gpt_forward/gpt_backward from one host thread per device
(src/train_gpt.cu:400-412), so the replacement must be re-entrant: launch
status is per host thread; split-K partials, nn partial sums and the flash dS
workspace are leased per call from a per-device pool; the per-shape flash
plans and per-kernel occupancy tables are shared and built under a lock on
first use. Four threads run a flash forward
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


def _worker(qkv, dout, A, B, C0, shape, gshape, results, errors, i, barrier):
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
    gshape = (257, 129, 3000)        # few output tiles: split-K partials in leased scratch
    Bn, T, C, NH = shape
    M, N, K = gshape
    qkv = O.fill_normal(Bn * T * 3 * C, 0x7A7A).reshape(Bn, T, 3 * C)
    dout = O.fill_normal(Bn * T * C, 0x7B7B).reshape(Bn, T, C)
    A = O.fill_xorshift(M * K, 0x1357)
    B = O.fill_xorshift(K * N, 0x2468)
    C0 = O.fill_xorshift(M * N, 0x9999)
    results, errors = [None] * NTHREADS, []
    barrier = threading.Barrier(NTHREADS)
    threads = [threading.Thread(target=_worker, args=(qkv, dout, A, B, C0, shape, gshape, results,
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


def _churn(bufs, shapes, norms, i):
    Bn, T, C, NH = shapes["flash"]
    M, N, K = shapes["gemm"]
    Nl, Cl = shapes["ln"]
    b = bufs
    try:
        bmb.gemm(False, False, M, N, K, 1.0, b["A"].data_ptr(), b["B"].data_ptr(), 0.0,
                 b["C"].data_ptr())
        bmb.flash_backward(b["dqkv"].data_ptr(), b["dsum"].data_ptr(), b["dout"].data_ptr(),
                           b["qkv"].data_ptr(), b["out"].data_ptr(), b["lse"].data_ptr(),
                           Bn, T, C, NH)
        bmb.call("layernorm_backward", b["dinp"].data_ptr(), b["dw"].data_ptr(),
                 b["db"].data_ptr(), b["ln_dout"].data_ptr(), b["ln_inp"].data_ptr(),
                 b["ln_w"].data_ptr(), b["mean"].data_ptr(), b["rstd"].data_ptr(), Nl, Cl)
        norms[i] = bmb.call("grad_global_norm", b["A"].data_ptr(), M * K)
        bmb.check("churn thread %d" % i)
    except Exception as e:  # reported by the main thread
        norms[i] = repr(e)


def test_short_lived_threads_do_not_strand_scratch(gpu):
    """The reference trainer starts fresh host threads every step
    (src/train_gpt.cu:400-412,457-459). Each of 50 short-lived threads here
    runs a split-K gemm, the default flash backward (dS workspace), a
    layernorm backward and a gradient norm (nn partial sums) and exits; the
    device's free memory after them must equal what it was after the first
    one (scratch comes back to the pool instead of being stranded per thread:
    at these shapes a thread holds ~37 MB of it, 35 MB of them dS tiles)."""
    import torch
    shapes = {"flash": (4, 1024, 256, 4), "gemm": (257, 129, 3000), "ln": (4096, 768)}
    Bn, T, C, NH = shapes["flash"]
    M, N, K = shapes["gemm"]
    Nl, Cl = shapes["ln"]
    f32 = dict(device="cuda", dtype=torch.float32)
    g = torch.Generator(device="cpu").manual_seed(5)

    def rnd(n):
        return torch.randn(n, generator=g).to(**f32)

    bufs = {"A": rnd(M * K), "B": rnd(K * N), "C": torch.zeros(M * N, **f32),
            "qkv": rnd(Bn * T * 3 * C), "dout": rnd(Bn * T * C),
            "out": torch.empty(Bn * T * C, **f32), "lse": torch.empty(Bn * NH * T, **f32),
            "dqkv": torch.empty(Bn * T * 3 * C, **f32), "dsum": torch.empty(Bn * NH * T, **f32),
            "dinp": torch.zeros(Nl * Cl, **f32), "dw": torch.zeros(Cl, **f32),
            "db": torch.zeros(Cl, **f32), "ln_dout": rnd(Nl * Cl), "ln_inp": rnd(Nl * Cl),
            "ln_w": rnd(Cl), "mean": torch.zeros(Nl, **f32), "rstd": torch.ones(Nl, **f32)}
    bmb.flash_forward(bufs["out"].data_ptr(), bufs["lse"].data_ptr(), bufs["qkv"].data_ptr(),
                      Bn, T, C, NH)
    torch.cuda.synchronize()
    norms = [None] * 51
    print("churn: 51 sequential threads (gemm %dx%dx%d, flash bwd B=%d T=%d C=%d NH=%d, "
          "layernorm bwd %dx%d, grad norm)" % (shapes["gemm"] + shapes["flash"] + shapes["ln"]),
          flush=True)

    def run(i):
        t = threading.Thread(target=_churn, args=(bufs, shapes, norms, i))
        t.start()
        t.join(timeout=60)
        assert not t.is_alive(), "thread %d did not finish" % i
        torch.cuda.synchronize()

    run(0)
    free0 = torch.cuda.mem_get_info()[0]
    for i in range(1, 51):
        run(i)
    free1 = torch.cuda.mem_get_info()[0]
    assert all(isinstance(n, float) for n in norms), [n for n in norms if not isinstance(n, float)]
    assert len(set(norms)) == 1 and np.isfinite(norms[0])
    drift = (free0 - free1) / 2**20
    print("free memory after thread 1: %.1f MiB, after thread 51: %.1f MiB (drift %.1f MiB)"
          % (free0 / 2**20, free1 / 2**20, drift), flush=True)
    assert abs(drift) < 8.0
