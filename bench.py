#!/usr/bin/env python3
"""Headline benchmark: fp32 SGEMM at N=4096 and causal flash fwd+bwd at
B=8, H=12, T=1024, d=64 on one MI355X, through the C-ABI library.

A "step" is one SGEMM C = A@B + 0.5*C at M=N=K=4096 (
alpha=1, beta=0.5, C pre-filled, A/B/C from the reference's xorshift fill)
on the headline kernel (KERNELS id 9, fp32 MFMA). `value` is its GFLOP/s
(2*N^3 per step). The flash fwd+bwd figure and the other ladder stages are
reported in the same JSON line. Inputs are resident in HBM before timing;
each launch is bracketed by HIP events on the null stream, which is the
stream the library launches on (and torch's current stream).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "bare-metal-bard_amd"))

PEAK_FP32_TFLOPS = 157.3     # MI355X fp32 vector (packed) = fp32 matrix peak
PEAK_VALU_SCALAR = 78.6      # 64 fp32 FMA/clk/CU without packed math
PEAK_HBM_GBS = 8000.0
N_SGEMM = 4096
FLASH = dict(B=8, NH=12, T=1024, hs=64)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--kernel", type=int, default=9, help="headline KERNELS id")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-ladder", action="store_true", help="skip ladder stages 1-8, 10")
    ap.add_argument("--only", choices=["sgemm", "flash"], default=None,
                    help="run one workload only (for profiling)")
    ap.add_argument("--flash-sweep", action="store_true",
                    help="also time every forward and backward flash config (as the "
                         "reference's tools/test_flash.cu:198-227,279-319 sweep does)")
    ap.add_argument("--copy-calib", action="store_true",
                    help="first run a plain 256 MiB device-to-device copy 3 times, the "
                         "known-size reference dispatch for rocprofv3 --pmc FETCH_SIZE / "
                         "WRITE_SIZE calibration")
    return ap.parse_args()


def timed(fn, steps, warmup):
    """Per-launch durations (ms) from HIP events on the null stream."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    for a, b in ev:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in ev]


def stats(ms):
    s = sorted(ms)
    return {"avg_ms": sum(s) / len(s), "best_ms": s[0], "median_ms": s[len(s) // 2]}


def load_traffic():
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE and
    WRITE_SIZE, scaled by a copy-kernel calibration), committed under
    profiles/; None until such a measurement exists."""
    p = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(p):
        return {}
    with open(p) as f:
        return json.load(f)


def cpu_sgemm_baseline(A, B, C0, N):
    """The oracle's sequential-fmaf SGEMM (order-preserving, vectorised over
    j, rows split over all host threads) on a row sample of the N=4096 problem
    sized to ~10 s, scaled to GFLOP/s."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    threads = len(os.sched_getaffinity(0))
    threads = min(threads, int(os.environ.get("OMP_NUM_THREADS", threads)))
    rows = 64
    t0 = time.perf_counter()
    O.gemm_f32seq(0, 0, rows, N, N, 1.0, A[:rows], B, 0.5, C0[:rows], threads=threads)
    dt = time.perf_counter() - t0
    rows = int(max(64, min(N, rows * 10.0 / max(dt, 1e-3))))
    t0 = time.perf_counter()
    O.gemm_f32seq(0, 0, rows, N, N, 1.0, A[:rows], B, 0.5, C0[:rows], threads=threads)
    dt = time.perf_counter() - t0
    gf = 2.0 * rows * N * N / dt / 1e9
    return {"value": round(gf, 2), "unit": "GFLOP/s", "cores": threads, "kind": "port",
            "sample": "sequential-fmaf SGEMM (oracle/oracle.c orc_gemm_f32seq_mt), first %d of "
                      "4096 rows of the N=4096 problem, %.1f s" % (rows, dt)}


def cpu_flash_baseline(qkv, dout, B, T, C, NH):
    """Unfused fp32 causal attention fwd+bwd (src/attention.cu semantics,
    oracle orc_attn_fwdbwd_f32, OpenMP over heads) on a head sample."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    threads = len(os.sched_getaffinity(0))
    threads = min(threads, int(os.environ.get("OMP_NUM_THREADS", threads)))
    nb = 1
    t0 = time.perf_counter()
    O.attn_fwdbwd_f32(qkv[:nb], dout[:nb], nb, T, C, NH, threads)
    dt = time.perf_counter() - t0
    hs = C // NH
    pairs = nb * NH * T * (T + 1) / 2
    tf = 14.0 * hs * pairs / dt / 1e12  # fwd 4*d*P + bwd 10*d*P useful flops
    return {"value": round(tf, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": "unfused fp32 attention fwd+bwd, batch 0 of 8 (12 heads, T=1024, d=64), "
                      "%.1f s" % dt}


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (single-GPU tier); "
              "--gpus %d is not supported" % args.gpus, file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    import bmb

    bmb.lib()
    assert torch.cuda.is_available(), "bench.py needs the GPU"
    assert torch.cuda.current_stream().cuda_stream == 0, "events must be on the null stream"
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O  # input generators only, outside the timed region

    if args.copy_calib:
        src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    result = {}
    N = N_SGEMM
    flops = 2.0 * N ** 3
    A = O.fill_xorshift(N * N, 0x12345678).reshape(N, N)
    Bm = O.fill_xorshift(N * N, 0x9ABCDEF0).reshape(N, N)
    C0 = O.fill_xorshift(N * N, 0x0F0F0F0F).reshape(N, N)
    dA = torch.from_numpy(A).cuda()
    dB = torch.from_numpy(Bm).cuda()
    dC = torch.from_numpy(C0).cuda()

    def sg(kid):
        ent = bmb.find_kernel(kid)
        fn = ent["fn"]
        return lambda: fn(N, N, N, 1.0, dA.data_ptr(), dB.data_ptr(), 0.5, dC.data_ptr())

    ladder = {}
    if args.only != "flash":
        ms = timed(sg(args.kernel), args.steps, args.warmup)
        bmb.check("sgemm")
        st = stats(ms)
        result["sgemm"] = st
        if not args.no_ladder and args.only is None:
            for kid in (8, 10, 7, 6, 5, 4, 3):
                k_ms = timed(sg(kid), max(3, args.steps // 4), 2)
                bmb.check("sgemm %d" % kid)
                ks = stats(k_ms)
                ladder[bmb.find_kernel(kid)["name"]] = {
                    "id": kid, "gflops_median": round(flops / ks["median_ms"] / 1e6, 1),
                    "pct_fp32_peak": round(100 * flops / ks["median_ms"] / 1e9 / PEAK_FP32_TFLOPS, 1)}

    flash = None
    if args.only != "sgemm":
        Bf, NH, T, hs = FLASH["B"], FLASH["NH"], FLASH["T"], FLASH["hs"]
        C = NH * hs
        qkv = O.fill_normal(Bf * T * 3 * C, 0xBEEF).reshape(Bf, T, 3 * C)
        dout = O.fill_normal(Bf * T * C, 0xD0D0).reshape(Bf, T, C)
        d_qkv = torch.from_numpy(qkv).cuda()
        d_dout = torch.from_numpy(dout).cuda()
        out = torch.empty(Bf * T * C, device="cuda")
        lse = torch.empty(Bf * NH * T, device="cuda")
        dqkv = torch.empty(Bf * T * 3 * C, device="cuda")
        dsum = torch.empty(Bf * NH * T, device="cuda")
        fwd = lambda: bmb.flash_forward(out.data_ptr(), lse.data_ptr(), d_qkv.data_ptr(),
                                        Bf, T, C, NH)
        bwd = lambda: bmb.flash_backward(dqkv.data_ptr(), dsum.data_ptr(), d_dout.data_ptr(),
                                         d_qkv.data_ptr(), out.data_ptr(), lse.data_ptr(),
                                         Bf, T, C, NH)
        fwd()
        f_ms = timed(fwd, args.steps, args.warmup)
        b_ms = timed(bwd, args.steps, args.warmup)
        bmb.check("flash")
        pairs = Bf * NH * T * (T + 1) / 2
        fwd_fl, bwd_fl = 4.0 * hs * pairs, 10.0 * hs * pairs
        fs, bs = stats(f_ms), stats(b_ms)
        tot = fs["avg_ms"] + bs["avg_ms"]
        flash = {
            "metric": "flash fwd+bwd TFLOP/s @B=8,H=12,T=1024,d=64 (causal, fp32)",
            "value": round((fwd_fl + bwd_fl) / tot / 1e9, 2), "unit": "TFLOP/s",
            "ms_fwd": round(fs["avg_ms"], 4), "ms_bwd": round(bs["avg_ms"], 4),
            "tflops_fwd": round(fwd_fl / fs["avg_ms"] / 1e9, 2),
            "tflops_bwd": round(bwd_fl / bs["avg_ms"] / 1e9, 2),
            "pct_fp32_mfma_peak": round(100 * (fwd_fl + bwd_fl) / tot / 1e9 / PEAK_FP32_TFLOPS, 1),
            "gflop_algorithmic": round((fwd_fl + bwd_fl) / 1e9, 2),
            "tflops_ref_accounting": round(4.5 * fwd_fl / tot / 1e9, 2),
            "fwd_config": bmb.flash_configs()[bmb.flash_default_config()],
            "bwd_config": bmb.flash_bwd_configs()[bmb.flash_default_bwd_config()],
        }
        if args.flash_sweep:
            sweep = {}
            for i, name in enumerate(bmb.flash_configs()):
                f = lambda i=i: bmb.flash_forward_cfg(i, out.data_ptr(), lse.data_ptr(),
                                                      d_qkv.data_ptr(), Bf, T, C, NH)
                ms_ = stats(timed(f, max(3, args.steps // 2), 2))["median_ms"]
                sweep["fwd %d %s" % (i, name)] = round(fwd_fl / ms_ / 1e9, 2)
            fwd()
            for i, name in enumerate(bmb.flash_bwd_configs()):
                f = lambda i=i: bmb.flash_backward_cfg(
                    i, dqkv.data_ptr(), dsum.data_ptr(), d_dout.data_ptr(), d_qkv.data_ptr(),
                    out.data_ptr(), lse.data_ptr(), Bf, T, C, NH)
                ms_ = stats(timed(f, max(3, args.steps // 2), 2))["median_ms"]
                sweep["bwd %d %s" % (i, name)] = round(bwd_fl / ms_ / 1e9, 2)
            bmb.check("flash sweep")
            flash["config_sweep_tflops"] = sweep

    cpu = None
    cpu_flash = None
    if not args.no_cpu:
        if args.only != "flash":
            cpu = cpu_sgemm_baseline(A, Bm, C0, N)
        if flash is not None:
            cpu_flash = cpu_flash_baseline(qkv, dout, Bf, T, C, NH)
            flash["cpu_baseline"] = cpu_flash

    traffic = load_traffic()
    line = {"metric": "SGEMM GFLOP/s @N=4096 fp32 (% peak); flash fwd+bwd TFLOP/s @T=1024,d=64",
            "unit": "GFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "f32", "data": "synthetic (xorshift32 1e-3 grid inputs, seeds of "
                                    "src/bench.cu:226-228; attention N(0,1) Box-Muller)"}
    if "sgemm" in result:
        st = result["sgemm"]
        gfl = flops / st["avg_ms"] / 1e6
        line.update({
            "value": round(gfl, 1), "ms_per_step": round(st["avg_ms"], 4),
            "pct_of_peak": round(100 * gfl / 1e3 / PEAK_FP32_TFLOPS, 1),
            "config": {"workload": "sgemm M=N=K=4096 fp32 row-major alpha=1 beta=0.5, "
                                   "KERNELS id %d (%s)" % (args.kernel,
                                                           bmb.find_kernel(args.kernel)["name"]),
                       "global_batch": 1, "seq_len": None, "parallelism": "single-gpu"},
            "roofline": {"bound": "mfma", "achieved": round(gfl / 1e3, 2),
                         "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(gfl / 1e3 / PEAK_FP32_TFLOPS, 4),
                         "traffic": traffic.get("sgemm_tensorcore_4096")},
            "sgemm_timing_ms": {k: round(v, 4) for k, v in st.items()},
        })
        if ladder:
            line["ladder"] = ladder
    else:
        line.update({"value": None, "ms_per_step": None})
    if flash is not None:
        line["flash"] = flash
    if cpu is not None:
        line["cpu_baseline"] = cpu
    print(json.dumps(line))


if __name__ == "__main__":
    main()
