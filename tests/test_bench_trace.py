"""bench.py --summarize-trace on a synthetic rocprofv3 CSV pair: only the
dispatches that start and end inside a "timed:<region>" range are counted,
per region occurrence, with the warm-up launches before the range left out."""
import csv
import importlib.util
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _write(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)


def test_summarize_trace_counts_timed_dispatches_only(tmp_path, capsys):
    us = 1000  # ns
    k = "void bmb::mfma_gemm_k<false, false, bmb::MfmaTile<256, 256, 32, 2, 4>, true, 0>(int, float)"
    kernels = [
        # warm-up, before the range
        {"Kernel_Name": k, "Start_Timestamp": 0, "End_Timestamp": 900 * us},
        # inside region "sgemm": 3 launches of 10, 20 and 30 us
        {"Kernel_Name": k, "Start_Timestamp": 1000 * us, "End_Timestamp": 1010 * us},
        {"Kernel_Name": k, "Start_Timestamp": 1020 * us, "End_Timestamp": 1040 * us},
        {"Kernel_Name": k, "Start_Timestamp": 1050 * us, "End_Timestamp": 1080 * us},
        # straddles the range's end: not counted
        {"Kernel_Name": k, "Start_Timestamp": 1090 * us, "End_Timestamp": 1200 * us},
        # second occurrence of the region: one launch
        {"Kernel_Name": "flash_fwd_h_k<64, 4, 1>(float*)", "Start_Timestamp": 2000 * us,
         "End_Timestamp": 2005 * us},
    ]
    markers = [
        {"Function": "timed:sgemm", "Start_Timestamp": 995 * us, "End_Timestamp": 1100 * us},
        {"Function": "untimed", "Start_Timestamp": 0, "End_Timestamp": 3000 * us},
        {"Function": "timed:sgemm", "Start_Timestamp": 1999 * us, "End_Timestamp": 2010 * us},
    ]
    _write(tmp_path / "run_kernel_trace.csv", kernels)
    _write(tmp_path / "run_marker_api_trace.csv", markers)
    _bench().summarize_trace(str(tmp_path))
    out = capsys.readouterr().out
    assert out.count("### region `sgemm`") == 2
    first, second = out.split("(occurrence 2)")
    row = [ln for ln in first.splitlines() if "mfma_gemm_k" in ln]
    assert len(row) == 1
    cells = [c.strip() for c in row[0].strip("|").split("|")]
    # kernel | calls | mean | median | min | max | total ms
    assert cells[0] == "`bmb::mfma_gemm_k<false, false, bmb::MfmaTile<256, 256, 32, 2, 4>, true, 0>`"
    assert cells[1:] == ["3", "20.0", "20.0", "10.0", "30.0", "0.060"]
    assert "flash_fwd_h_k<64, 4, 1>" in second and "mfma_gemm_k" not in second
    # a single region
    _bench().summarize_trace(str(tmp_path), "nothing")
    assert "### region" not in capsys.readouterr().out
