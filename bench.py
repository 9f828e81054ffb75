#!/usr/bin/env python3
"""Benchmark of the SGEMM ladder and the fused causal attention on one
MI355X, through the C-ABI library (bare-metal-bard_amd/lib/libbmb.so).

A "step" is one SGEMM C = A@B + 0.5*C at M=N=K=4096 (config 2 of the
baseline: alpha=1, beta=0.5, C pre-filled; A, B, C from the reference's
xorshift32 fill, src/bench.cu:59-66,226-228) on the headline kernel, KERNELS
id 9 (fp32 in, fp32 products, fp32 accumulate on v_mfma_f32_32x32x2_f32).
`value` is its GFLOP/s (2*N^3 per step, src/bench.cu:107-110). Inputs are
resident in HBM before timing; W warm-up steps (continued, untimed, until at
least WARM_MIN_MS of warm-up work has run: the GPU's clock takes a few tens
of milliseconds of load to settle at ~2.4 GHz, and a warm-up of a few
milliseconds times the ramp instead), then exactly K steps
bracketed by synchronize on both sides and by a HIP event pair on the null
stream (the stream the library launches on and torch's current stream), so
`ms_per_step` and `roofline.achieved` come from the kernel's own average
duration over the timed region. The flash leg times a step of forward +
backward the same way.

The same JSON line also carries (none of them is `value`):
  * config 1: N=1024, alpha=1, beta=0 for the VALU, MFMA and bf16x3 paths
    (configs 1-3 are timed as bursts of back-to-back launches);
  * config 2: the square sweep N in {512 ... 8192} for the same three paths;
  * the ladder (ids 1-10) at N=4096;
  * config 3: gemm() at the GPT-2-small training shapes (BT=8192, C=768),
    forward NT, backward dX NN (beta 0) and dW TN (beta 1);
  * config 4: flash fwd+bwd at B=8, H=12, T=1024, d=64, with its roofline,
    and (`flash.vs_unfused`) the unfused attention on the same inputs with
    the fused kernels' speedup over it, as tools/test_flash.cu reports;
  * config 5: the full GPT-2-small training step (12L/768/12H, T=1024, B=8,
    V=50257 padded to 50304, fused attention, global-norm clipping, AdamW)
    on synthetic uniform tokens: tokens/s over the timed steps and the loss
    trajectory;
  * cpu_baseline: the oracle's order-preserving SGEMM and unfused attention
    on the host's cores (a bounded sample, reported, not a target);
  * verification: before each timed region, outside it, the result of one
    launch on the same inputs is checked against the CPU oracle, as the
    reference's bench does before timing a kernel (src/bench.cu:259-273):
    sampled rows of every SGEMM (bit-exact for the fp32 VALU ids, within the
    fp32 summation bound for id 9, within the bf16x3 bound for id 10), batch
    0 of the attention (out, lse, dq, dk, dv against fp64), sampled rows of
    every config 3 GEMM in both arithmetic modes, and the GPT step's losses.
    The errors go into the line (`verification`); if any exceeds its bound
    the line is still printed and the bench exits with status 1.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
                       [--only sgemm|flash] [--flash-sweep] [--quick]
       python bench.py --summarize-trace DIR [--region NAME]

Every timed region is wrapped in a roctx range "timed:<region>". Under
`rocprofv3 --kernel-trace --marker-trace --output-format csv -d DIR -- python3
bench.py ...`, `--summarize-trace DIR` then prints, per region, the kernels
dispatched inside it (warm-up excluded) with their count, mean and median
duration: the figures the profiles quote.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "bare-metal-bard_amd"))

PEAK_FP32_TFLOPS = 157.3     # MI355X fp32 vector = fp32 matrix (published)
PEAK_BF16_TFLOPS = 2500.0    # dense bf16 MFMA (published)
# KERNELS id 10 issues three bf16 MFMAs per fp32 product term, so its own
# ceiling is a third of the bf16 peak in fp32-equivalent flops.
BF16X3_CEILING_TFLOPS = PEAK_BF16_TFLOPS / 3
# The default flash kernels carry each fp32 operand as an fp16 hi/lo pair and
# issue three fp16 MFMAs per fp32 product term (fp16 dense peak = bf16's).
PEAK_FP16_TFLOPS = 2500.0
FP16X3_CEILING_TFLOPS = PEAK_FP16_TFLOPS / 3
PEAK_HBM_GBS = 8000.0
N_SGEMM = 4096
SWEEP_N = (512, 1000, 1024, 1536, 2048, 4096, 4097, 6144, 8192)
FLASH = dict(B=8, NH=12, T=1024, hs=64)
GPT = dict(BT=8192, C=768, V=50257)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=25)
    ap.add_argument("--kernel", type=int, default=9, help="headline KERNELS id")
    ap.add_argument("--n", type=int, default=N_SGEMM,
                    help="size of the headline SGEMM (M=N=K; for profiling other sizes)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-telemetry", action="store_true",
                    help="skip the untimed sustained runs that read clock and power (for "
                         "profiling runs, whose per-step kernel totals they would inflate)")
    ap.add_argument("--no-ladder", action="store_true", help="skip the ladder, sweep and GPT shapes")
    ap.add_argument("--quick", action="store_true", help="headline SGEMM and flash only")
    ap.add_argument("--only", choices=["sgemm", "flash", "gpt", "sizes"], default=None,
                    help="run one workload only (for profiling); sizes: KERNELS ids 8, 9 "
                         "and 10 at N = 512, 1024, 4096 and 4097")
    ap.add_argument("--flash-sweep", action="store_true",
                    help="also time every forward and backward flash config (as the "
                         "reference's tools/test_flash.cu:198-227,279-319 sweep does)")
    ap.add_argument("--summarize-trace", metavar="DIR", default=None,
                    help="summarise a rocprofv3 --kernel-trace --marker-trace CSV output "
                         "directory by timed region (no GPU work)")
    ap.add_argument("--region", default=None, help="with --summarize-trace: only this region")
    ap.add_argument("--copy-calib", action="store_true",
                    help="first run a plain 256 MiB device-to-device copy 3 times, the "
                         "known-size reference dispatch for rocprofv3 --pmc FETCH_SIZE / "
                         "WRITE_SIZE calibration")
    return ap.parse_args()


T_START = time.perf_counter()


class _Roctx:
    """roctx ranges around the timed regions (named "timed:<region>"), so that a
    rocprofv3 run with --marker-trace can attribute kernel dispatches to them
    (--summarize-trace). Calls into rocprofiler-sdk's roctx library, which
    does nothing unless a profiler is attached; absent library: no ranges."""

    def __init__(self):
        import ctypes
        self.lib = None
        for name in ("librocprofiler-sdk-roctx.so.1", "librocprofiler-sdk-roctx.so"):
            try:
                lib = ctypes.CDLL(name)
                lib.roctxRangePushA.argtypes = [ctypes.c_char_p]
                lib.roctxRangePushA.restype = ctypes.c_int
                lib.roctxRangePop.restype = ctypes.c_int
                self.lib = lib
                break
            except OSError:
                continue

    def push(self, name):
        if self.lib is not None:
            self.lib.roctxRangePushA(("timed:" + name).encode())

    def pop(self):
        if self.lib is not None:
            self.lib.roctxRangePop()


ROCTX = _Roctx()


def progress(msg):
    """One line on stderr per finished part of the run (the JSON line alone
    goes to stdout)."""
    print("bench.py [%6.1f s] %s" % (time.perf_counter() - T_START, msg), file=sys.stderr,
          flush=True)


def timed(fn, steps, warmup, name="per-launch"):
    """Per-launch durations (ms) from HIP events on the null stream."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    ROCTX.push(name)
    for a, b in ev:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    ROCTX.pop()
    return [a.elapsed_time(b) for a, b in ev]


WARM_MIN_MS = 100.0  # least warm-up work before a timed region
WARM_STEPS_RUN = {}  # warm-up steps actually run, by region name


def timed_steps(fn, steps, warmup, name=None):
    """The contract's timing: `warmup` untimed steps (more, untimed, until
    WARM_MIN_MS of warm-up has run), then exactly `steps` steps bracketed by
    torch.cuda.synchronize() on both sides, with a HIP event pair on the null
    stream (the stream every launch of the library goes to) around the timed
    region. Returns (device ms per step from the events, host wall-clock ms
    per step); the warm-up steps run are kept in WARM_STEPS_RUN[name]."""
    import torch
    torch.cuda.synchronize()
    t0, n = time.perf_counter(), 0
    while n < warmup or (time.perf_counter() - t0) * 1e3 < WARM_MIN_MS:
        fn()
        n += 1
        if n % 8 == 0 or n >= warmup:
            torch.cuda.synchronize()
    if name is not None:
        WARM_STEPS_RUN[name] = n
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ROCTX.push(name or "region")
    t0 = time.perf_counter()
    a.record()
    for _ in range(steps):
        fn()
    b.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    ROCTX.pop()
    return a.elapsed_time(b) / steps, wall


class Telemetry:
    """Clock and power of GPU 0 from amdsmi's metrics table while a `with`
    block runs. The firmware refreshes that table about once a second, so a
    host thread polls it and keeps each refresh (a new energy timestamp);
    result() uses the last two refreshes that both fall inside the block:
    average socket power = energy accumulated between them / their time
    apart, and the per-XCD GFX clocks of the later one. A block shorter than
    about two refreshes has no such pair, and says so."""

    def __init__(self, period=0.02):
        self.period, self.snaps, self.reason = period, [], None
        self.smi = self.h = None
        try:
            import amdsmi
            amdsmi.amdsmi_init()
            hs = amdsmi.amdsmi_get_processor_handles()
            if not hs:
                raise RuntimeError("no GPU handle")
            self.smi, self.h = amdsmi, hs[0]
        except Exception as e:  # not fatal: the figures are reported without it
            self.reason = "amdsmi unavailable: %s" % (repr(e)[:120],)

    def _snap(self):
        smi = self.smi
        e = smi.amdsmi_get_energy_count(self.h)
        m = smi.amdsmi_get_gpu_metrics_info(self.h)
        clks = m.get("current_gfxclks")
        if not isinstance(clks, (list, tuple)):
            clks = [m.get("current_gfxclk")]
        clks = [int(c) for c in clks if isinstance(c, (int, float)) and c < 0xFFFF]
        return (int(e["timestamp"]), int(e["energy_accumulator"]),
                float(e["counter_resolution"]), clks)

    def __enter__(self):
        import threading
        self.snaps, self._stop = [], threading.Event()
        if self.h is not None:
            try:
                self._first_ts = self._snap()[0]  # the refresh current at entry
            except Exception as e:
                self.reason = "amdsmi query failed: %s" % (repr(e)[:120],)
                self.h = None
        if self.h is not None:
            def run():
                last = self._first_ts
                while not self._stop.is_set():
                    try:
                        sn = self._snap()
                    except Exception as e:
                        self.reason = "amdsmi query failed: %s" % (repr(e)[:120],)
                        return
                    if sn[0] != last:
                        self.snaps.append(sn)
                        last = sn[0]
                    self._stop.wait(self.period)
            self._thr = threading.Thread(target=run, daemon=True)
            self._thr.start()
        return self

    def __exit__(self, *exc):
        self._stop.set()
        if self.h is not None:
            self._thr.join()
        return False

    def result(self):
        # The first refresh seen inside the block still averages time before
        # it; a pair of later refreshes covers an interval inside the block.
        if len(self.snaps) < 3:
            return {"available": False,
                    "reason": self.reason or "region shorter than two refreshes (~1 s each) "
                                             "of amdsmi's metrics table"}
        (t0, e0, res, _), (t1, e1, _, clks) = self.snaps[-2], self.snaps[-1]
        dt = (t1 - t0) / 1e9  # ns
        clk = sorted(clks)
        return {"socket_power_w": round((e1 - e0) * res * 1e-6 / dt, 1), "window_s": round(dt, 3),
                "gfx_clk_mhz_per_xcd": clks,
                "gfx_clk_mhz_median": clk[len(clk) // 2] if clk else None,
                "gfx_clk_mhz_max_spec": 2400}


SKIP_TELEMETRY = False  # --no-telemetry


def sustained_telemetry(fn, seconds=3.5):
    """Clock and power under `fn` run back to back for `seconds` (untimed, after
    the timed region): long enough for two refreshes of amdsmi's metrics."""
    import torch
    if SKIP_TELEMETRY:
        return {"available": False, "reason": "--no-telemetry"}
    with Telemetry() as tel:
        t0, n = time.perf_counter(), 0
        while time.perf_counter() - t0 < seconds:
            fn()
            n += 1
            if n % 8 == 0:
                torch.cuda.synchronize()
        torch.cuda.synchronize()
    return tel.result()


def timed_burst(fn, reps, warmup=2, name="burst"):
    """Average duration (ms) of `reps` back-to-back launches between one pair
    of HIP events: the throughput of a kernel in a stream, as the training
    step runs it. Per-launch event pairs add a gap of tens of microseconds
    around each launch, which distorts kernels of a few hundred microseconds.
    Like timed_steps, the warm-up runs at least WARM_MIN_MS of the workload:
    after a switch of workload the clock takes tens of ms to settle (a
    2-launch warm-up put N=4096 SGEMM 7% below its settled rate)."""
    import torch
    torch.cuda.synchronize()
    t0, n = time.perf_counter(), 0
    while n < warmup or (time.perf_counter() - t0) * 1e3 < WARM_MIN_MS:
        fn()
        n += 1
        if n % 8 == 0 or n >= warmup:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ROCTX.push(name)
    a.record()
    for _ in range(reps):
        fn()
    b.record()
    torch.cuda.synchronize()
    ROCTX.pop()
    return a.elapsed_time(b) / reps


def independent_runs(fn, steps, first_ms, runs=3, name="region"):
    """The timed region measured `runs` times in all, each with its own
    warm-up and synchronised ends (the first is the reported one): the
    per-step ms of each run, their median, and the spread (max - min over
    the median), flagged above 3%."""
    ms = [first_ms] + [timed_steps(fn, steps, 2, name + " rerun")[0] for _ in range(runs - 1)]
    s = sorted(ms)
    med = s[len(s) // 2]
    spread = 100.0 * (s[-1] - s[0]) / med
    return {"ms_per_step": [round(x, 4) for x in ms], "median_ms": round(med, 4),
            "spread_pct": round(spread, 2), "spread_over_3pct": spread > 3.0}


def stats(ms):
    s = sorted(ms)
    return {"avg_ms": sum(s) / len(s), "best_ms": s[0], "median_ms": s[len(s) // 2]}


def load_traffic():
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE and
    WRITE_SIZE, scaled by a copy-kernel calibration), committed as
    profiles/traffic.json; {} until such a measurement exists."""
    p = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(p):
        return {}
    with open(p) as f:
        return json.load(f)


def cpu_model():
    """The host CPU's model name (as lscpu prints it), from /proc/cpuinfo."""
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def own_peak(kid):
    """(peak TFLOP/s, its name) a KERNELS id is measured against."""
    if kid == 10:
        return BF16X3_CEILING_TFLOPS, "bf16x3 ceiling = bf16 dense peak / 3"
    return PEAK_FP32_TFLOPS, "fp32 peak (vector = matrix)"


def host_threads():
    n = len(os.sched_getaffinity(0))
    return max(1, min(n, int(os.environ.get("OMP_NUM_THREADS", n))))


def cpu_sgemm_baseline(O, A, B, C0, N):
    """The oracle's sequential-fmaf SGEMM (order-preserving, vectorised over
    j, rows split over the host threads) on a row sample of the N=4096
    problem sized to about 10 s, scaled to GFLOP/s; plus the literal
    single-thread loop at config 1's N=1024 on a row sample."""
    threads = host_threads()
    rows = 64
    t0 = time.perf_counter()
    O.gemm_f32seq(0, 0, rows, N, N, 1.0, A[:rows], B, 0.5, C0[:rows], threads=threads)
    dt = time.perf_counter() - t0
    rows = int(max(64, min(N, rows * 10.0 / max(dt, 1e-3))))
    t0 = time.perf_counter()
    O.gemm_f32seq(0, 0, rows, N, N, 1.0, A[:rows], B, 0.5, C0[:rows], threads=threads)
    dt = time.perf_counter() - t0
    gf = 2.0 * rows * N * N / dt / 1e9
    n1, r1 = 1024, 128
    t0 = time.perf_counter()
    O.gemm_f32seq(0, 0, r1, n1, n1, 1.0, A[:r1, :n1].copy(), B[:n1, :n1].copy(), 0.0, None,
                  threads=1)
    dt1 = time.perf_counter() - t0
    return {"value": round(gf, 2), "unit": "GFLOP/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(), "cpus_online": os.cpu_count(),
            "sample": "sequential-fmaf SGEMM (oracle orc_gemm_f32seq_mt, bit-identical to "
                      "KERNELS ids 1-8), rows 0-%d of the N=4096 alpha=1 beta=0.5 problem, "
                      "%.1f s" % (rows - 1, dt),
            "single_thread_config1": {"value": round(2.0 * r1 * n1 * n1 / dt1 / 1e9, 3),
                                      "unit": "GFLOP/s", "cores": 1,
                                      "sample": "rows 0-%d of N=1024 alpha=1 beta=0, %.2f s"
                                                % (r1 - 1, dt1)}}


def cpu_flash_baseline(O, qkv, dout, B, T, C, NH):
    """Unfused fp32 causal attention fwd+bwd (src/attention.cu semantics,
    oracle orc_attn_fwdbwd_f32, OpenMP over heads) on the first batches of
    the config 4 problem, about 10 s of work."""
    threads = host_threads()
    hs = C // NH
    nb, done, dt = 1, 0, 0.0
    while True:
        t0 = time.perf_counter()
        O.attn_fwdbwd_f32(qkv[done:done + nb], dout[done:done + nb], nb, T, C, NH, threads)
        dt += time.perf_counter() - t0
        done += nb
        if dt > 10.0 or done >= B:
            break
        nb = min(B - done, max(1, int(nb * 2)))
    pairs = done * NH * T * (T + 1) / 2
    tf = 14.0 * hs * pairs / dt / 1e12  # fwd 4*d*P + bwd 10*d*P useful flops
    return {"value": round(tf, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(), "cpus_online": os.cpu_count(),
            "sample": "unfused fp32 attention fwd+bwd (oracle orc_attn_fwdbwd_f32), batches "
                      "0-%d of 8 (12 heads, T=1024, d=64), %.1f s" % (done - 1, dt)}


def sgemm_fn(bmb, kid):
    return bmb.find_kernel(kid)["fn"]


U32 = 2.0 ** -24


def fp32_order_bound(K):
    """Normwise bound (max |err| / max |ref|) for an fp32 result whose
    products are exact and whose only difference from the exact sum is fp32
    summation: a random-walk model, 4 sqrt(K) 2^-24, plus the epilogue."""
    import math
    return 4.0 * math.sqrt(max(K, 1)) * U32 + 4.0 * U32


class Verifier:
    """Results checked against the CPU oracle outside the timed regions;
    `record` keeps each check's error, bound and verdict for the line."""

    def __init__(self, O):
        self.O, self.checks, self.failed = O, {}, []

    def record(self, name, err, bound, kind, ok=None, **extra):
        ok = bool(err <= bound) if ok is None else bool(ok and err <= bound)
        self.checks[name] = dict({"err": float("%.3g" % err), "bound": float("%.3g" % bound),
                                  "kind": kind, "ok": ok}, **extra)
        if not ok:
            self.failed.append(name)
        return ok

    def gemm_rows(self, name, got_rows, A_rows, B, tb, N, K, alpha, beta, C0_rows, math_kind,
                  tol):
        """got_rows = rows of C = alpha op(A) op(B) + beta C0; A_rows are the
        matching rows of op(A) (M' x K), B is stored K x N or N x K (tb).
        math_kind: "seq" (bit-exact against the sequential-fmaf oracle; tb
        false only), "fp32" or "bf16x3". Every kind is also within `tol`
        (normwise against fp64)."""
        import numpy as np
        O = self.O
        M = A_rows.shape[0]
        got_rows = np.asarray(got_rows).reshape(M, N)
        ref = O.gemm_f64(False, tb, M, N, K, alpha, A_rows, B, beta, C0_rows)
        err, bad = O.normwise(got_rows, ref)
        if bad:
            return self.record(name, float("inf"), tol, math_kind + ": non-finite entries")
        if math_kind == "seq":
            want = O.gemm_f32seq(0, 0, M, N, K, alpha, A_rows, B, beta, C0_rows, threads=0)
            same = bool(np.array_equal(got_rows, want))
            return self.record(name, err, tol, "bit-exact vs sequential fmaf, normwise vs fp64",
                               ok=same, bit_exact=same)
        if math_kind == "fp32":
            return self.record(name, err, min(tol, fp32_order_bound(K)),
                               "normwise vs fp64 within the fp32 summation bound")
        Bop = np.ascontiguousarray(B.reshape(N, K).T if tb else B.reshape(K, N))
        want = O.gemm_bf16x3_f64(M, N, K, alpha, A_rows, Bop, beta, C0_rows)
        e3, bad3 = O.normwise(got_rows, want)
        return self.record(name, e3 if not bad3 else float("inf"), fp32_order_bound(3 * K),
                           "normwise around the bf16x3 split's exact value (fp32 summation "
                           "bound of 3K terms); vs fp64 within tol", ok=err <= tol,
                           vs_fp64=float("%.3g" % err), tol=tol)


def sample_rows(n, seed=7, extra=8):
    import numpy as np
    r = np.r_[0, 1, 127, 128, n // 2, n - 2, n - 1,
              np.random.default_rng(seed).integers(0, n, extra)]
    return np.unique(r[(r >= 0) & (r < n)])


def gf(flops, ms):
    return round(flops / ms / 1e6, 1)


def summarize_trace(d, only=None):
    """Kernel dispatches inside each "timed:<region>" roctx range of a
    rocprofv3 CSV output directory (run_kernel_trace.csv and
    run_marker_api_trace.csv, any prefix): count, mean, median, min and max
    duration per kernel, and the region's per-step kernel time when its
    dispatches repeat per step. Markdown on stdout."""
    import csv
    import glob
    import re

    def one(pattern):
        f = sorted(glob.glob(os.path.join(d, "**", pattern), recursive=True))
        if not f:
            sys.exit("bench.py: no %s under %s" % (pattern, d))
        return list(csv.DictReader(open(f[0])))

    kernels = one("*kernel_trace.csv")
    regions = [(m["Function"][len("timed:"):], int(m["Start_Timestamp"]), int(m["End_Timestamp"]))
               for m in one("*marker_api_trace.csv") if m["Function"].startswith("timed:")]

    def short(name):
        name = re.sub(r"\(anonymous namespace\)::", "", name)
        name = re.sub(r"^void ", "", name)
        depth, out = 0, []
        for ch in name:  # drop the parameter list, keep template arguments
            if ch == "(" and depth == 0:
                break
            depth += ch == "<"
            depth -= ch == ">"
            out.append(ch)
        return "".join(out)

    seen = {}
    for rname, t0, t1 in regions:
        if only and rname != only:
            continue
        seen[rname] = seen.get(rname, 0) + 1
        rows = {}
        for k in kernels:
            s, e = int(k["Start_Timestamp"]), int(k["End_Timestamp"])
            if s >= t0 and e <= t1:
                rows.setdefault(short(k["Kernel_Name"]), []).append((e - s) / 1e3)
        print("### region `%s` (occurrence %d): %.3f ms between the range's ends\n"
              % (rname, seen[rname], (t1 - t0) / 1e6))
        print("| kernel | calls | mean us | median us | min us | max us | total ms |")
        print("|---|---:|---:|---:|---:|---:|---:|")
        for name, v in sorted(rows.items(), key=lambda kv: -sum(kv[1])):
            v = sorted(v)
            print("| `%s` | %d | %.1f | %.1f | %.1f | %.1f | %.3f |"
                  % (name, len(v), sum(v) / len(v), v[len(v) // 2], v[0], v[-1], sum(v) / 1e3))
        print()


def main():
    global SKIP_TELEMETRY
    args = parse()
    if args.summarize_trace:
        summarize_trace(args.summarize_trace, args.region)
        return
    SKIP_TELEMETRY = args.no_telemetry
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
    import oracle as O  # input generators and the CPU baseline only, outside the timed region

    extras = not (args.quick or args.no_ladder or args.only)

    if args.copy_calib:
        src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    traffic = load_traffic()
    line = {"metric": "SGEMM GFLOP/s @N=4096 fp32 (% peak); flash fwd+bwd TFLOP/s @T=1024,d=64",
            "value": None, "unit": "GFLOP/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": None, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "f32",
            "data": "synthetic (xorshift32 1e-3 grid inputs with the seeds of "
                    "src/bench.cu:226-228; attention q,k,v,dO N(0,1) by Box-Muller)"}

    N = args.n
    V = Verifier(O)
    A = O.fill_xorshift(N * N, 0x12345678).reshape(N, N)
    Bm = O.fill_xorshift(N * N, 0x9ABCDEF0).reshape(N, N)
    C0 = O.fill_xorshift(N * N, 0x0F0F0F0F).reshape(N, N)
    if args.only in (None, "sgemm"):
        # The problem of size n reads the first n*n floats of each buffer as an
        # n x n row-major matrix; an xorshift stream's first n*n values are the
        # n*n stream, so every size sees the bench's seeded matrices.
        smax = max(max(SWEEP_N), N) if extras else N
        hA = O.fill_xorshift(smax * smax, 0x12345678)
        hB = O.fill_xorshift(smax * smax, 0x9ABCDEF0)
        hC = O.fill_xorshift(smax * smax, 0x0F0F0F0F)
        dA, dB, dC = (torch.from_numpy(h).cuda() for h in (hA, hB, hC))
        dV = torch.empty_like(dC)  # the verification launches' output

        def sq(kid, n, alpha=1.0, beta=0.5):
            fn = sgemm_fn(bmb, kid)
            return lambda: fn(n, n, n, alpha, dA.data_ptr(), dB.data_ptr(), beta, dC.data_ptr())

        def verify_sq(kid, n, alpha=1.0, beta=0.5, extra=8):
            """One launch into a fresh copy of C, sampled rows against the
            oracle (outside every timed region)."""
            dV[:n * n].copy_(torch.from_numpy(hC[:n * n]))
            sgemm_fn(bmb, kid)(n, n, n, alpha, dA.data_ptr(), dB.data_ptr(), beta, dV.data_ptr())
            torch.cuda.synchronize()
            bmb.check("sgemm id %d verification" % kid)
            rows = sample_rows(n, extra=extra)
            got = dV[:n * n].view(n, n)[torch.from_numpy(rows).cuda()].cpu().numpy()
            kind = "seq" if kid <= 8 else ("fp32" if kid == 9 else "bf16x3")
            progress("verified KERNELS id %d at N=%d" % (kid, n))
            return V.gemm_rows("sgemm id%d N=%d alpha=%g beta=%g" % (kid, n, alpha, beta), got,
                               hA[:n * n].reshape(n, n)[rows], hB[:n * n].reshape(n, n), False,
                               n, n, alpha, beta,
                               hC[:n * n].reshape(n, n)[rows] if beta != 0 else None, kind,
                               bmb.find_kernel(kid)["tol"])

        flops = 2.0 * N ** 3
        verify_sq(args.kernel, N)
        ms, wall = timed_steps(sq(args.kernel, N), args.steps, args.warmup, "sgemm")
        st = stats(timed(sq(args.kernel, N), args.steps, 2, "sgemm per-launch"))  # spread
        bmb.check("sgemm")
        g = flops / ms / 1e6
        ent = bmb.find_kernel(args.kernel)
        bytes_alg = 4.0 * (3 * N * N + N * N)  # A, B, C read (beta != 0), C written
        line.update({
            "value": round(g, 1), "ms_per_step": round(ms, 4), "ms_per_step_wall": round(wall, 4),
            "pct_of_peak": round(100 * g / 1e3 / own_peak(args.kernel)[0], 1),
            "config": {"workload": "sgemm M=N=K=%d fp32 row-major alpha=1 beta=0.5, "
                                   "KERNELS id %d (%s)" % (N, args.kernel, ent["name"]),
                       "tol": ent["tol"], "algorithmic_gflop": round(flops / 1e9, 2),
                       "algorithmic_mb": round(bytes_alg / 1e6, 1)},
            "roofline": {"bound": "mfma" if args.kernel >= 9 else "valu",
                         "achieved": round(g / 1e3, 2),
                         "peak": own_peak(args.kernel)[0], "unit": "TFLOP/s",
                         "frac": round(g / 1e3 / own_peak(args.kernel)[0], 4),
                         "peak_is": own_peak(args.kernel)[1],
                         "traffic": traffic.get("sgemm_id%d_%d" % (args.kernel, N))},
            "sgemm_launch_ms": {k: round(v, 4) for k, v in st.items()},
            "independent_runs": independent_runs(sq(args.kernel, N), args.steps, ms,
                                                 name="sgemm"),
            "warmup_steps_run": WARM_STEPS_RUN.get("sgemm"),
            "vendor_fp32_gemm_gflops": vendor_sq(torch, dA, dB, dC, N) if extras else None,
            "device_telemetry_sustained": sustained_telemetry(sq(args.kernel, N)),
        })

        progress("headline SGEMM timed: %.4f ms/step" % ms)
        if extras:
            # Config 1: N=1024, alpha=1, beta=0.
            c1 = {}
            for kid in (8, 9, 10):
                verify_sq(kid, 1024, 1.0, 0.0)
                ms1 = timed_burst(sq(kid, 1024, 1.0, 0.0), 20, 5, name="config1 id%d" % kid)
                c1["id%d %s" % (kid, bmb.find_kernel(kid)["name"])] = gf(2.0 * 1024 ** 3, ms1)
            line["config1_n1024_gflops"] = c1
            line["id10_denominator"] = {
                "bf16x3_ceiling_tflops": round(BF16X3_CEILING_TFLOPS, 1),
                "why": "three bf16 MFMAs per fp32 product term (hi*hi + hi*lo + lo*hi); id 10's "
                       "pct figures below are of this ceiling, ids 1-9 of the 157.3 fp32 peak"}
            # Config 2: square sweep, alpha=1, beta=0.5.
            sweep = {}
            for kid in (8, 9, 10):
                row = {}
                for n in SWEEP_N:
                    verify_sq(kid, n, extra=2)
                    reps = 10 if n <= 4096 else 5
                    row[str(n)] = gf(2.0 * n ** 3, timed_burst(
                        sq(kid, n), reps, name="config2 id%d N=%d" % (kid, n)))
                sweep["id%d %s" % (kid, bmb.find_kernel(kid)["name"])] = row
                progress("config 2 sweep of id %d timed" % kid)
            bmb.check("sgemm sweep")
            line["config2_sweep_gflops"] = sweep
            # The ladder at N=4096.
            ladder = {}
            for kid in range(1, 11):
                if kid not in (8, 9, 10):  # (verified in the sweep at this size)
                    verify_sq(kid, N, extra=2)
                reps, warm = (2, 1) if kid <= 2 else (5, 2)
                s3 = stats(timed(sq(kid, N), reps, warm, "ladder id%d" % kid))
                pk, pk_name = own_peak(kid)
                ladder["id%d %s" % (kid, bmb.find_kernel(kid)["name"])] = {
                    "gflops": gf(flops, s3["median_ms"]),
                    "pct_of_own_peak": round(100 * flops / s3["median_ms"] / 1e9 / pk, 1),
                    "peak_tflops": round(pk, 1)}
            bmb.check("ladder")
            line["ladder_n%d" % N] = ladder
            del dA, dB, dC, dV
            torch.cuda.empty_cache()
            line["config3_gpt_gemm_gflops"] = gpt_shapes(bmb, O, torch, V)

    if args.only == "sizes":
        line["sgemm_sizes_gflops"] = sizes_bench(bmb, O, torch)
    if args.only in (None, "flash"):
        line["flash"] = flash_bench(args, bmb, O, torch, traffic, V)
    if args.only == "gpt" or (args.only is None and not args.quick):
        line["config5_gpt_train_step"] = gpt_step_bench(args, bmb, torch, V)
        if not args.quick:
            with bmb.gemm_math(bmb.GEMM_MATH_FP32):
                line["config5_gpt_train_step_fp32_gemm"] = gpt_step_bench(
                    args, bmb, torch, V, steps=5, warm=2, tag="fp32 GEMM")

    if not args.no_cpu and not args.quick:
        progress("CPU baseline")
        cpu = {}
        if args.only in (None, "sgemm"):
            cpu = cpu_sgemm_baseline(O, A, Bm, C0, N)
        if args.only in (None, "flash"):
            Bf, NH, T, hs = FLASH["B"], FLASH["NH"], FLASH["T"], FLASH["hs"]
            C = NH * hs
            qkv = O.fill_normal(Bf * T * 3 * C, 0xBEEF).reshape(Bf, T, 3 * C)
            dout = O.fill_normal(Bf * T * C, 0xD0D0).reshape(Bf, T, C)
            fl = cpu_flash_baseline(O, qkv, dout, Bf, T, C, NH)
            line["flash"]["cpu_baseline"] = fl
            if not cpu:
                cpu = fl
        line["cpu_baseline"] = cpu
    line["verification"] = {"all_ok": not V.failed, "failed": V.failed, "checks": V.checks}
    print(json.dumps(line))
    if V.failed:
        print("bench.py: verification failed: %s" % ", ".join(V.failed), file=sys.stderr)
        sys.exit(1)


def sizes_bench(bmb, O, torch):
    """KERNELS ids 8 (fp32 VALU), 9 (fp32 MFMA) and 10 (bf16x3) at N = 512,
    1024, 4096 and 4097 with config 2's epilogue (alpha 1, beta 0.5, C
    pre-filled), a burst of launches each: the workload of the rocprofv3
    counter runs for the VALU and bf16x3 paths, for the small shapes, whose
    few output tiles leave most CUs idle, and for the ragged 4097, which the
    MFMA paths run as a corner plan (a 4096^2 block of whole tiles, then the
    edges)."""
    res = {}
    for n in (512, 1024, 4096, 4097):
        dA = torch.from_numpy(O.fill_xorshift(n * n, 0x12345678)).cuda()
        dB = torch.from_numpy(O.fill_xorshift(n * n, 0x9ABCDEF0)).cuda()
        dC = torch.from_numpy(O.fill_xorshift(n * n, 0x0F0F0F0F)).cuda()
        for kid in (8, 9, 10):
            fn = sgemm_fn(bmb, kid)
            run = lambda: fn(n, n, n, 1.0, dA.data_ptr(), dB.data_ptr(), 0.5, dC.data_ptr())
            res["id%d N=%d" % (kid, n)] = gf(2.0 * n ** 3, timed_burst(
                run, 10 if n > 1024 else 50, name="sizes id%d N=%d" % (kid, n)))
        bmb.check("sgemm sizes")
        del dA, dB, dC
    return res


def vendor_sq(torch, dA, dB, dC, N):
    """Context only, not this build's result: the vendor's fp32 GEMM (hipBLASLt
    through torch, TF32 off) on the headline problem, C = A@B + 0.5*C, timed
    like the headline (warm-up, then a burst of 20)."""
    torch.backends.cuda.matmul.allow_tf32 = False
    A = dA[:N * N].view(N, N)
    B = dB[:N * N].view(N, N)
    Cm = dC[:N * N].view(N, N)
    fn = lambda: Cm.addmm_(A, B, beta=0.5)
    timed_steps(fn, 5, 5, "vendor warm-up")
    return gf(2.0 * N ** 3, timed_burst(fn, 20, name="vendor sgemm"))


def gpt_shapes(bmb, O, torch, V):
    """gemm() at the GPT-2-small training shapes
    (src/gpt.cu:256-376), in both of gemm()'s arithmetic modes, each against
    its own ceiling: bf16x3 (the default; 833 TFLOP/s of fp32-equivalent
    work on three bf16 MFMAs per product) and fp32 (gemm_set_math
    GEMM_MATH_FP32: fp32 MFMA products, the reference's arithmetic; 157.3).
    The forward is NT (weights stored out x in), the backward dX is NN with
    beta 0 and dW is TN with beta 1 (accumulate). Activations N(0, 1),
    weights N(0, 0.02^2). Before timing, each GEMM's result is checked on
    sampled rows against the oracle in each mode."""
    import numpy as np
    BT, C, Vv = GPT["BT"], GPT["C"], GPT["V"]
    torch.backends.cuda.matmul.allow_tf32 = False  # the vendor comparison stays fp32
    layers = {"qkv": (C, 3 * C), "attn_proj": (C, C), "mlp_fc": (C, 4 * C),
              "mlp_proj": (4 * C, C), "lm_head": (C, Vv)}
    modes = (("bf16x3", bmb.GEMM_MATH_BF16X3, BF16X3_CEILING_TFLOPS),
             ("fp32", bmb.GEMM_MATH_FP32, PEAK_FP32_TFLOPS))
    res = {"units": "GFLOP/s", "ceilings_tflops": {m[0]: round(m[2], 1) for m in modes},
           "vendor_fp32": "the vendor's fp32 GEMM (hipBLASLt through torch, TF32 off) on the "
                          "same operands: context, not this build's result"}
    f32 = dict(device="cuda", dtype=torch.float32)
    for name, (cin, cout) in layers.items():
        hX = O.fill_normal(BT * cin, 11)
        hW = O.fill_normal(cout * cin, 12, 0.02)
        hDY = O.fill_normal(BT * cout, 13)
        hDW0 = O.fill_normal(cout * cin, 14, 0.02)
        X, W, DY = (torch.from_numpy(h).to(**f32) for h in (hX, hW, hDY))
        Y, DX, DW = torch.empty(BT * cout, **f32), torch.empty(BT * cin, **f32), \
            torch.from_numpy(hDW0).to(**f32)
        fl = 2.0 * BT * cin * cout
        # forward Y[BT,cout] = X[BT,cin] @ W[cout,cin]^T
        fwd = lambda: bmb.gemm(False, True, BT, cout, cin, 1.0, X.data_ptr(), W.data_ptr(),
                               0.0, Y.data_ptr())
        # dX[BT,cin] = dY[BT,cout] @ W[cout,cin]
        dxf = lambda: bmb.gemm(False, False, BT, cin, cout, 1.0, DY.data_ptr(), W.data_ptr(),
                               0.0, DX.data_ptr())
        # dW[cout,cin] += dY^T[cout,BT] @ X[BT,cin]
        dwf = lambda: bmb.gemm(True, False, cout, cin, BT, 1.0, DY.data_ptr(), X.data_ptr(),
                               1.0, DW.data_ptr())
        reps = 3 if name == "lm_head" else 10
        entry = {"shape": "%dx%dx%d" % (BT, cout, cin)}
        rows_bt = sample_rows(BT, seed=3, extra=4)
        rows_co = sample_rows(cout, seed=5, extra=4)
        hXm, hDYm = hX.reshape(BT, cin), hDY.reshape(BT, cout)
        for mname, math, ceil in modes:
            with bmb.gemm_math(math):
                fwd()
                dxf()
                DW.copy_(torch.from_numpy(hDW0))
                dwf()
                torch.cuda.synchronize()
                bmb.check("gemm %s %s" % (name, mname))
                tag = "config3 %s %s" % (name, mname)
                V.gemm_rows(tag + " fwd_NT", Y.view(BT, cout)[rows_bt].cpu().numpy(),
                            hXm[rows_bt], hW, True, cout, cin, 1.0, 0.0, None, mname, 1e-4)
                V.gemm_rows(tag + " dX_NN", DX.view(BT, cin)[rows_bt].cpu().numpy(),
                            hDYm[rows_bt], hW, False, cin, cout, 1.0, 0.0, None, mname, 1e-4)
                V.gemm_rows(tag + " dW_TN_beta1", DW.view(cout, cin)[rows_co].cpu().numpy(),
                            np.ascontiguousarray(hDYm[:, rows_co].T), hX, False, cin, BT, 1.0,
                            1.0, hDW0.reshape(cout, cin)[rows_co], mname, 1e-4)
                g = {"fwd_NT": gf(fl, timed_burst(fwd, reps, name=tag + " fwd_NT")),
                     "dX_NN": gf(fl, timed_burst(dxf, reps, name=tag + " dX_NN")),
                     "dW_TN_beta1": gf(fl, timed_burst(dwf, reps, name=tag + " dW_TN"))}
                bmb.check("gemm " + name)
            g["pct_of_own_ceiling"] = {k: round(v / 1e3 / ceil * 100, 1) for k, v in g.items()}
            entry[mname] = g
        Xm, Wm = X.view(BT, cin), W.view(cout, cin)
        Ym, DYm, DXm = Y.view(BT, cout), DY.view(BT, cout), DX.view(BT, cin)
        entry["vendor_fp32"] = {
            "fwd_NT": gf(fl, timed_burst(lambda: torch.matmul(Xm, Wm.t(), out=Ym), reps,
                                         name="config3 %s vendor fwd_NT" % name)),
            "dX_NN": gf(fl, timed_burst(lambda: torch.matmul(DYm, Wm, out=DXm), reps,
                                        name="config3 %s vendor dX_NN" % name)),
            "dW_TN_beta1": gf(fl, timed_burst(lambda: Wm.addmm_(DYm.t(), Xm), reps,
                                              name="config3 %s vendor dW_TN" % name))}
        res[name] = entry
        progress("config 3 %s verified and timed" % name)
        del X, W, DY, Y, DX, DW, Xm, Wm, Ym, DYm, DXm
    torch.cuda.empty_cache()
    return res


def lr_at(step, warmup, total, lr_max):
    """The trainer's schedule (src/train_gpt.cu:233-238): linear warmup, then
    cosine decay to lr_max / 10."""
    import math
    lr_min = lr_max * 0.1
    if step <= warmup:
        return lr_max * step / warmup
    p = (step - warmup) / max(1, total - warmup)
    return lr_min + 0.5 * (lr_max - lr_min) * (1.0 + math.cos(math.pi * p))


def gpt_step_bench(args, bmb, torch, V, steps=None, warm=None, tag=None):
    """Config 5: one training step = gpt_forward + gpt_backward + global-norm
    clipping + AdamW (src/train_gpt.cu:395-460 at one rank), GPT-2 small,
    B=8, T=1024, random init N(0, 0.02) from gpt_init(1337), synthetic
    i.i.d. uniform token ids in [0, 50257) (a fresh batch every step). Timed
    on the host clock with the device synchronised at both ends; the step
    itself blocks on the loss and the gradient norm, as the trainer's does.
    The linear layers run in gemm()'s current arithmetic mode (bf16x3 by
    default; `tag` names another), attention on the default fp16x3 flash
    kernels. Verified: every loss finite, the first within 1 nat of ln V
    (uniform targets on near-uniform initial logits)."""
    import math
    import numpy as np
    cfg = (1024, 50257, 50304, 12, 12, 768)
    B, T = 8, 1024
    m = bmb.Model(cfg, B, T, use_flash=True)
    m.init(1337)
    n_params = int(m.g.num_params)
    rng = np.random.default_rng(1337)
    warm = min(args.warmup, 3) if warm is None else warm
    steps = args.steps if steps is None else steps
    total = warm + steps
    batches = [(rng.integers(0, cfg[1], B * T).astype(np.int32),
                rng.integers(0, cfg[1], B * T).astype(np.int32)) for _ in range(total)]
    L = bmb.lib()
    losses, norms, times = [], [], []
    for step in range(1, total + 1):
        x, y = batches[step - 1]
        torch.cuda.synchronize()
        if step == warm + 1:
            ROCTX.push("gpt" if tag is None else "gpt-" + tag.replace(" ", "-"))
        t0 = time.perf_counter()
        loss = m.forward(x, y)
        m.backward()
        gn = L.grad_global_norm(m.g.grads_mem, n_params)
        gs = 1.0 / gn if gn > 1.0 else 1.0
        L.adamw_update(m.g.params_mem, m.g.grads_mem, m.g.m_mem, m.g.v_mem, n_params,
                       lr_at(step, 100, 2000, 1e-3), 0.9, 0.999, 1e-8, 0.1, step, gs)
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) * 1e3)
        losses.append(loss)
        norms.append(gn)
    ROCTX.pop()
    bmb.check("gpt step")
    progress("config 5 (%s) timed: %.2f ms/step" % (tag or "bf16x3 GEMM",
                                                    sum(times[warm:]) / max(1, steps)))

    def more_steps():  # untimed training steps for the clock / power reading
        x, y = batches[0]
        m.forward(x, y)
        m.backward()
        g = L.grad_global_norm(m.g.grads_mem, n_params)
        L.adamw_update(m.g.params_mem, m.g.grads_mem, m.g.m_mem, m.g.v_mem, n_params, 1e-4,
                       0.9, 0.999, 1e-8, 0.1, total + 1, 1.0 / g if g > 1.0 else 1.0)
    tel = sustained_telemetry(more_steps) if tag is None else {"available": False,
                                                                "reason": "not measured"}
    # one more step split into its phases, for the breakdown
    x, y = batches[0]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    m.forward(x, y)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    m.backward()
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    gn = L.grad_global_norm(m.g.grads_mem, n_params)
    L.adamw_update(m.g.params_mem, m.g.grads_mem, m.g.m_mem, m.g.v_mem, n_params, 1e-4, 0.9,
                   0.999, 1e-8, 0.1, total + 1, 1.0)
    torch.cuda.synchronize()
    t3 = time.perf_counter()
    m.free()
    timed_ms = times[warm:]
    ms = sum(timed_ms) / len(timed_ms)
    hs = cfg[5] // cfg[4]
    flops = 6.0 * B * T * n_params + 12.0 * cfg[3] * cfg[4] * T * T * hs * B
    lnv = math.log(cfg[1])
    V.record("config5 %s losses finite, first within 1 nat of ln V" % (tag or "bf16x3 GEMM"),
             abs(losses[0] - lnv) if all(math.isfinite(x) for x in losses) else float("inf"),
             1.0, "|loss_first - ln V|; every loss finite")
    gemm_kind = tag or "bf16x3 GEMM"
    return {
        "metric": "GPT-2 small training step tokens/s (%s + fp16x3 attention, fp32 AdamW)"
                  % gemm_kind,
        "compute": "fp32 in/out everywhere; linear layers on %s products (%s), attention on "
                   "the default fp16x3 flash kernels, elementwise ops and AdamW in fp32"
                   % (gemm_kind, "fp32 MFMA" if tag else "three bf16 MFMAs per fp32 product"),
        "value": round(B * T / (ms / 1e3), 1), "unit": "tokens/s",
        "ms_per_step": round(ms, 3), "ms_best": round(min(timed_ms), 3),
        "steps": steps, "warmup": warm,
        "tflops_train_gpt_accounting": round(flops / (ms / 1e3) / 1e12, 2),
        "phase_ms": {"forward": round((t1 - t0) * 1e3, 2), "backward": round((t2 - t1) * 1e3, 2),
                     "norm_clip_adamw": round((t3 - t2) * 1e3, 2)},
        "params": n_params,
        "loss_first": round(losses[0], 5), "loss_last": round(losses[-1], 5),
        "ln_V": round(float(np.log(cfg[1])), 5),
        "grad_norm_first": round(norms[0], 5),
        "device_telemetry_sustained": tel,
        "config": {"workload": "GPT-2 small train step: 12L/768/12H, T=1024, B=8, V=50257 "
                               "(Vp=50304), fused attention, grad clip 1.0, AdamW "
                               "(0.9, 0.999, 1e-8, wd 0.1), lr schedule of train_gpt.cu",
                   "flops_per_step": flops},
    }


def verify_flash(V, O, qkv, dout, out, lse, dqkv, dsum, Bf, T, C, NH):
    """Batch 0 (12 heads) of one forward + backward against the fp64 oracle:
    out, dq, dk, dv normwise (each within the reference's 1e-5,
    tools/test_flash.cu:132,226,314), lse and dsum absolute / relative."""
    import numpy as np
    nb = 1
    o = out.view(Bf, T, C)[:nb].cpu().numpy()
    l = lse.view(Bf, NH, T)[:nb].cpu().numpy()
    d = dqkv.view(Bf, T, 3 * C)[:nb].cpu().numpy()
    ds = dsum.view(Bf, NH, T)[:nb].cpu().numpy()
    ref_o, ref_l = O.attn_fwd_f64(qkv[:nb], nb, T, C, NH)
    ref_d = O.attn_bwd_f64(qkv[:nb], dout[:nb], nb, T, C, NH)
    ref_ds = O.dsum_f64(dout[:nb], o, nb, T, C, NH)
    e, bad = O.normwise(o, ref_o)
    V.record("flash out (batch 0)", e if not bad else float("inf"), 1e-5, "normwise vs fp64")
    V.record("flash lse (batch 0)", float(np.abs(l - ref_l).max()), 1e-5, "max abs vs fp64")
    V.record("flash dsum (batch 0)", float(np.abs(ds - ref_ds).max() / np.abs(ref_ds).max()),
             1e-5, "max abs / max |ref| vs fp64")
    for s_, name in enumerate("qkv"):
        e, bad = O.normwise(d[:, :, s_ * C:(s_ + 1) * C], ref_d[:, :, s_ * C:(s_ + 1) * C])
        V.record("flash d%s (batch 0)" % name, e if not bad else float("inf"), 1e-5,
                 "normwise vs fp64")


def flash_bench(args, bmb, O, torch, traffic, V):
    Bf, NH, T, hs = FLASH["B"], FLASH["NH"], FLASH["T"], FLASH["hs"]
    C = NH * hs
    qkv = O.fill_normal(Bf * T * 3 * C, 0xBEEF).reshape(Bf, T, 3 * C)
    dout = O.fill_normal(Bf * T * C, 0xD0D0).reshape(Bf, T, C)
    d_qkv = torch.from_numpy(qkv).cuda()
    d_dout = torch.from_numpy(dout).cuda()
    out = torch.empty(Bf * T * C, device="cuda", dtype=torch.float32)
    lse = torch.empty(Bf * NH * T, device="cuda", dtype=torch.float32)
    dqkv = torch.empty(Bf * T * 3 * C, device="cuda", dtype=torch.float32)
    dsum = torch.empty(Bf * NH * T, device="cuda", dtype=torch.float32)
    fwd = lambda: bmb.flash_forward(out.data_ptr(), lse.data_ptr(), d_qkv.data_ptr(),
                                    Bf, T, C, NH)
    bwd = lambda: bmb.flash_backward(dqkv.data_ptr(), dsum.data_ptr(), d_dout.data_ptr(),
                                     d_qkv.data_ptr(), out.data_ptr(), lse.data_ptr(),
                                     Bf, T, C, NH)
    def step():
        fwd()
        bwd()

    step()
    torch.cuda.synchronize()
    bmb.check("flash verification")
    verify_flash(V, O, qkv, dout, out, lse, dqkv, dsum, Bf, T, C, NH)
    progress("flash verified")
    tot, wall = timed_steps(step, args.steps, args.warmup, "flash")  # one step = fwd + bwd
    f_ms, _ = timed_steps(fwd, args.steps, 2, "flash-fwd")
    b_ms, _ = timed_steps(bwd, args.steps, 2, "flash-bwd")
    fs = stats(timed(fwd, args.steps, 2, "flash-fwd per-launch"))
    bs = stats(timed(bwd, args.steps, 2, "flash-bwd per-launch"))
    runs = independent_runs(step, args.steps, tot, name="flash")
    bmb.check("flash")
    pairs = Bf * NH * T * (T + 1) / 2
    fwd_fl, bwd_fl = 4.0 * hs * pairs, 10.0 * hs * pairs
    tf = (fwd_fl + bwd_fl) / tot / 1e9
    flash = {
        "metric": "flash fwd+bwd TFLOP/s @B=8,H=12,T=1024,d=64 (causal, fp32 in/out, "
                  "fp16x3 products)",
        "value": round(tf, 2), "unit": "TFLOP/s", "ms_per_step": round(tot, 4),
        "ms_per_step_wall": round(wall, 4),
        "ms_fwd": round(f_ms, 4), "ms_bwd": round(b_ms, 4),
        "launch_ms_fwd_median": round(fs["median_ms"], 4),
        "launch_ms_bwd_median": round(bs["median_ms"], 4),
        "independent_runs": runs,
        "tflops_fwd": round(fwd_fl / f_ms / 1e9, 2),
        "tflops_bwd": round(bwd_fl / b_ms / 1e9, 2),
        "fp16x3_ceiling_tflops": round(FP16X3_CEILING_TFLOPS, 1),
        "gflop_algorithmic": round((fwd_fl + bwd_fl) / 1e9, 2),
        "tflops_ref_accounting": round(4.5 * fwd_fl / tot / 1e9, 2),
        "compute": "fp32 in/out; default kernels split each fp32 operand into an fp16 hi/lo "
                   "pair (exact power-of-two scaling) and accumulate hi*hi + hi*lo + lo*hi "
                   "in fp32 on v_mfma_f32_32x32x16_f16",
        "fwd_config": bmb.flash_configs()[bmb.flash_default_config()],
        "bwd_config": bmb.flash_bwd_configs()[bmb.flash_default_bwd_config()],
        "warmup_steps_run": WARM_STEPS_RUN.get("flash"),
        "device_telemetry_sustained": sustained_telemetry(step),
        # The kernels' own ceiling: fp32-equivalent flops on three fp16 MFMAs
        # per product (the fp32-MFMA configs would be held to 157.3).
        "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": round(FP16X3_CEILING_TFLOPS, 1),
                     "unit": "TFLOP/s", "frac": round(tf / FP16X3_CEILING_TFLOPS, 4),
                     "peak_is": "fp16x3 ceiling = fp16 dense MFMA peak / 3",
                     "traffic": traffic.get("flash_fwd_bwd_b8h12t1024d64")},
    }
    flash["vs_unfused"] = unfused_attention_bench(args, bmb, torch, d_qkv, d_dout, Bf, T, C, NH,
                                                  f_ms, b_ms)
    if args.flash_sweep:
        sweep = {}
        for i, name in enumerate(bmb.flash_configs()):
            f = lambda i=i: bmb.flash_forward_cfg(i, out.data_ptr(), lse.data_ptr(),
                                                  d_qkv.data_ptr(), Bf, T, C, NH)
            ms_ = stats(timed(f, max(3, args.steps // 2), 2, "flash fwd cfg %d" % i))["median_ms"]
            sweep["fwd %d %s" % (i, name)] = round(fwd_fl / ms_ / 1e9, 2)
        fwd()
        for i, name in enumerate(bmb.flash_bwd_configs()):
            f = lambda i=i: bmb.flash_backward_cfg(
                i, dqkv.data_ptr(), dsum.data_ptr(), d_dout.data_ptr(), d_qkv.data_ptr(),
                out.data_ptr(), lse.data_ptr(), Bf, T, C, NH)
            ms_ = stats(timed(f, max(3, args.steps // 2), 2, "flash bwd cfg %d" % i))["median_ms"]
            sweep["bwd %d %s" % (i, name)] = round(bwd_fl / ms_ / 1e9, 2)
        bmb.check("flash sweep")
        flash["config_sweep_tflops"] = sweep
    return flash


def unfused_attention_bench(args, bmb, torch, d_qkv, d_dout, Bf, T, C, NH, f_ms, b_ms):
    """The reference's tools/test_flash.cu reports each fused path against the
    unfused one on the same inputs (:183-192, :270-271): attention_forward
    (3 kernels: permute, QK^T with the full T x T scores, softmax and PV,
    unpermute) and attention_backward (7), timed here on the same q, k, v and
    dO as the flash leg, best and median of a few launches each, and the
    fused forward's and backward's speedup over them (the flash leg's per-step
    times). dpreatt and datt share one buffer, as the reference's harness
    passes them (test_flash.cu:109-110)."""
    f32 = dict(device="cuda", dtype=torch.float32)
    out = torch.empty(Bf * T * C, **f32)
    qkvr = torch.empty(4 * Bf * T * C, **f32)
    att = torch.empty(Bf * NH * T * T, **f32)
    dqkv = torch.empty(Bf * T * 3 * C, **f32)
    dqkvr = torch.empty(4 * Bf * T * C, **f32)
    datt = torch.empty(Bf * NH * T * T, **f32)
    fwd = lambda: bmb.call("attention_forward", out.data_ptr(), qkvr.data_ptr(), att.data_ptr(),
                           d_qkv.data_ptr(), Bf, T, C, NH)
    bwd = lambda: bmb.call("attention_backward", dqkv.data_ptr(), dqkvr.data_ptr(),
                           datt.data_ptr(), datt.data_ptr(), d_dout.data_ptr(), qkvr.data_ptr(),
                           att.data_ptr(), Bf, T, C, NH)
    reps = max(3, args.steps // 4)
    fs = stats(timed(fwd, reps, 2, "unfused attention fwd"))
    bs = stats(timed(bwd, reps, 2, "unfused attention bwd"))
    bmb.check("unfused attention")
    res = {"fwd_best_ms": round(fs["best_ms"], 4), "fwd_median_ms": round(fs["median_ms"], 4),
           "bwd_best_ms": round(bs["best_ms"], 4), "bwd_median_ms": round(bs["median_ms"], 4),
           "fused_fwd_speedup": round(fs["median_ms"] / f_ms, 2),
           "fused_bwd_speedup": round(bs["median_ms"] / b_ms, 2),
           "note": "this build's unfused attention (attention.h: fp32 MFMA batched GEMMs and the "
                   "materialised causal softmax) against its default flash kernels"}
    del out, qkvr, att, dqkv, dqkvr, datt
    torch.cuda.empty_cache()
    return res


if __name__ == "__main__":
    main()
