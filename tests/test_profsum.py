"""yuuka_amd.profsum: per-kernel summary of a rocprofv3 CSV directory,
restricted to the last N verify steps (each ends with one
accept_finalize_kernel)."""
from __future__ import annotations

import csv

from yuuka_amd import profsum


def _trace(tmp_path, names):
    d = tmp_path / "run" / "host"
    d.mkdir(parents=True)
    with open(d / "run_kernel_trace.csv", "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Grid_Size", "Start_Timestamp", "End_Timestamp"])
        t = 0
        for i, (n, dur) in enumerate(names):
            w.writerow([i + 1, n, 64, t, t + dur])
            t += dur + 100
    return str(tmp_path)


def test_steps_window_and_names(tmp_path):
    fin = "void yk::(anonymous namespace)::accept_finalize_kernel<true>(yk::Args)"
    gemm = "void yk::fgemm_stream_kernel<12, 2, 4, 0, true>(yk::FusedGemmArgs)"
    seq = [(gemm, 99000), (fin, 1000)]            # warm-up step: outside the window
    seq += [(gemm, 10000), (gemm, 20000), (fin, 2000)] * 2
    out = profsum.summarise(profsum.load(_trace(tmp_path, seq)), steps=1)
    rows = {r.split("|")[1].strip(): r.split("|")[2:5] for r in out.splitlines() if r.startswith("| `")}
    assert set(rows) == {"`fgemm_stream_kernel`", "`accept_finalize_kernel`"}
    n, avg, per_step = (x.strip() for x in rows["`fgemm_stream_kernel`"])
    assert (n, avg, per_step) == ("2", "15.00", "30.0")
    assert out.splitlines()[-1].startswith("| total | 3 | | 32.0 |")
