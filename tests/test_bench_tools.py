"""bench.py's profile summarizers on synthetic rocprofv3 outputs: the figures
the committed profiles and the bench line's roofline fields come from.

Each case writes the CSV layout rocprofv3 produces (kernel trace, memory-copy
trace, marker trace, counter collection) for a timeline whose answer is
known by construction, and checks what the summarizer derives from it."""
import csv
import json
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def write_csv(path, fields, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=fields)
        w.writeheader()
        for r in rows:
            w.writerow(r)


def test_union_of_intervals():
    assert bench._union([]) == 0
    assert bench._union([(0, 10), (5, 15), (20, 30)]) == 25
    assert bench._union([(20, 30), (0, 10), (10, 12)]) == 22


@pytest.mark.parametrize("name,info,hit", [
    ("void relx::(anonymous namespace)::k_permute<2, 1, 6, true>(relx::KArgs)",
     {"family": "permute", "win": 2, "wout": 1}, True),
    ("void relx::(anonymous namespace)::k_permute<2, 1, 6, false>(relx::KArgs)",
     {"family": "permute", "win": 2, "wout": 1}, True),
    ("void relx::(anonymous namespace)::k_permute8<2, 1, 6>(relx::KArgs)",
     {"family": "permute", "win": 2, "wout": 1}, True),
    ("void relx::(anonymous namespace)::k_permute_direct8<2, 1, 6>(relx::PermArgs)",
     {"family": "permute", "win": 2, "wout": 1}, True),
    ("void relx::(anonymous namespace)::k_permute_direct<1, 2, 4>(relx::PermArgs)",
     {"family": "permute", "win": 2, "wout": 1}, False),
    ("void relx::(anonymous namespace)::k_interleave1p<4, 2, 4, 2>(unsigned char const*)",
     {"family": "interleave", "win": 4, "wout": 2}, True),
    ("void relx::(anonymous namespace)::k_transpose<4, 4, 1>(relx::KArgs)",
     {"family": "transpose", "win": 1, "wout": 2}, False),
    ("void relx::(anonymous namespace)::k_transpose_b8<1, 2, 4>(relx::KArgs)",
     {"family": "transpose", "win": 1, "wout": 2}, True),
    ("void relx::(anonymous namespace)::k_transpose<1, 2, 4, 128>(relx::KArgs)",
     {"family": "transpose", "win": 1, "wout": 2}, True),
    ("void relx::(anonymous namespace)::k_gather<1, 16, 4, true>(relx::GatherArgs)",
     {"pattern": "k_gather<1, 16, 4, true>"}, True),
])
def test_kernel_pattern(name, info, hit):
    assert bool(bench._kernel_pattern(info).search(name)) == hit


def test_summarize_pmc_scales_by_the_calibration_copy(tmp_path):
    """FETCH_SIZE reads half a copy's bytes on this part: the factor from
    the calibration copy restores them; medians per dispatch."""
    fields = ["Dispatch_Id", "Grid_Size", "Kernel_Name", "Counter_Name", "Counter_Value"]
    cal = 1 << 20
    for counter, d, cal_kib, kib in (("FETCH_SIZE", "f", cal / 2 / 1024, [100.0, 101.0, 500.0]),
                                     ("WRITE_SIZE", "w", cal / 1024, [50.0, 50.0, 50.0])):
        os.makedirs(tmp_path / d)
        rows = [{"Dispatch_Id": 1, "Grid_Size": 4096, "Kernel_Name": "__amd_rocclr_copyBuffer",
                 "Counter_Name": counter, "Counter_Value": cal_kib}]
        rows += [{"Dispatch_Id": 2 + i, "Grid_Size": 1024,
                  "Kernel_Name": "void relx::k_permute_direct8<2, 1, 6>(relx::PermArgs)",
                  "Counter_Name": counter, "Counter_Value": v} for i, v in enumerate(kib)]
        write_csv(tmp_path / d / "x_counter_collection.csv", fields, rows)
    probe = {"calibration_bytes": cal, "kernels": {
        "c5": {"family": "permute", "win": 2, "wout": 1, "algorithmic_bytes": 300 * 1024}}}
    out = bench.summarize_pmc(str(tmp_path / "f"), str(tmp_path / "w"), probe)
    assert out["FETCH_SIZE_calibration_factor"] == 2.0 and out["WRITE_SIZE_calibration_factor"] == 1.0
    c = out["configs"]["c5"]
    assert c["fetch_bytes"] == 2 * 101 * 1024 and c["write_bytes"] == 50 * 1024
    assert c["dispatches"] == 3 and c["traffic_over_algorithmic"] == round(252 / 300, 4)
    assert c["grid_threads"] == 1024


def test_probe_dispatches_are_assigned_in_order(tmp_path, capsys):
    """Two C5 shapes launch the same kernel instance: the trace is split by
    dispatch order (each config's warm-up launches dropped, then the copy of
    its bytes that follows it); kernel rates against 8 TB/s and the copy."""
    us = 1000
    rows, d = [], 0

    def add(name, grid, dur):
        nonlocal d
        d += 1
        rows.append({"Dispatch_Id": d, "Kernel_Name": name, "Grid_Size_X": grid,
                     "Start_Timestamp": 0, "End_Timestamp": int(dur * us)})
    add("__amd_rocclr_copyBuffer", 4096, 50)
    for dur in (20, 10, 10, 12):                       # config a: 1 warm-up + 3
        add("void relx::k_permute_direct8<2, 1, 6>(relx::PermArgs)", 512, dur)
    add("__amd_rocclr_fillBufferAligned", 256, 1)      # the copy's buffer fill
    for dur in (8, 8, 8):
        add("void relx::k_copy16(...)", 768, dur)
    for dur in (30, 40, 40, 40):                       # config b: the same kernel, other grid
        add("void relx::k_permute8<2, 1, 6, false>(relx::KArgs)", 2048, dur)
    for dur in (36, 36):                               # the copy's two forms: the faster counts
        add("void relx::k_copy16<1>(...)", 3072, dur)
    for dur in (44, 44):
        add("void relx::k_copy16<2>(...)", 1536, dur)
    write_csv(tmp_path / "p_kernel_trace.csv", list(rows[0]), rows)
    k = {"family": "permute", "win": 2, "wout": 1, "dispatches": 4, "skip": 1, "copy_bytes": 1}
    probe = {"kernels": {"a": dict(k, algorithmic_bytes=100000),
                         "b": dict(k, algorithmic_bytes=400000)}}
    bench.summarize_stats(str(tmp_path), probe)
    out = capsys.readouterr().out.splitlines()
    a = next(l for l in out if l.startswith("| a |")).split("|")
    b = next(l for l in out if l.startswith("| b |")).split("|")
    assert a[3].strip() == "512" and a[4].strip() == "3" and float(a[5]) == round(32 / 3, 2)
    assert float(a[10]) == 8.0 and float(a[12]) == round((100000 / (32 / 3) / 1e3) / (100000 / 8 / 1e3), 3)
    assert b[3].strip() == "2048" and b[4].strip() == "3" and float(b[5]) == 40.0
    assert float(b[10]) == 36.0


def test_summarize_trace_headline_timeline(tmp_path, capsys):
    """One staged call: two copies [10, 40) and [35, 70) us, kernels
    [30, 40) (under the first copy) and [70, 75) (after the last copy)."""
    us = 1000
    write_csv(tmp_path / "t_marker_api_trace.csv", ["Function", "Start_Timestamp", "End_Timestamp"],
              [{"Function": "relx.h2d.stage chunk=0", "Start_Timestamp": 0, "End_Timestamp": 8 * us},
               {"Function": "relx.h2d.slot_wait chunk=1", "Start_Timestamp": 8 * us,
                "End_Timestamp": 9 * us},
               {"Function": "relx.h2d.stage chunk=1", "Start_Timestamp": 9 * us,
                "End_Timestamp": 30 * us}])
    write_csv(tmp_path / "t_memory_copy_trace.csv", ["Direction", "Start_Timestamp", "End_Timestamp"],
              [{"Direction": "MEMORY_COPY_HOST_TO_DEVICE", "Start_Timestamp": 10 * us,
                "End_Timestamp": 40 * us},
               {"Direction": "MEMORY_COPY_HOST_TO_DEVICE", "Start_Timestamp": 35 * us,
                "End_Timestamp": 70 * us}])
    write_csv(tmp_path / "t_kernel_trace.csv", ["Kernel_Name", "Start_Timestamp", "End_Timestamp"],
              [{"Kernel_Name": "k_permute_direct8<2, 1, 6>", "Start_Timestamp": 30 * us,
                "End_Timestamp": 40 * us},
               {"Kernel_Name": "k_permute_direct8<2, 1, 6>", "Start_Timestamp": 70 * us,
                "End_Timestamp": 75 * us}])
    bench.summarize_trace(str(tmp_path))
    row = [l for l in capsys.readouterr().out.splitlines() if l.startswith("| 0 |")][0]
    cells = [c.strip() for c in row.strip("|").split("|")]
    # span 75 us, first copy after 10 us, 2 copies, busy 60/75, staging 29 us,
    # slot waits 1 us, 2 kernels, 10 of 15 us under a copy, tail 5 us
    assert cells[1] == "pageable (staged)"
    assert cells[2:] == ["0.075", "0.010", "2", "80.0%", "0.03", "0.00", "2", "66.7%", "5.0"]


def test_summarize_report_tables(tmp_path, capsys):
    lines = [{"pinned_h2d_ceiling_GBps": 57.2},
             {"config": "c1", "kernel": "transpose",
              "device": {"ms_per_step": 0.024, "achieved_GBps": 5600.0, "hbm_frac": 0.7},
              "e2e_pageable": {"p50_ms": 1.3, "pcie_frac": 0.9},
              "e2e_pinned": {"p50_ms": 1.2, "pcie_frac": 0.96}},
             {"config": "c4", "kernel": "stream",
              "device": {"ms_per_step": 0.026, "achieved_GBps": 6800.0, "hbm_frac": 0.85},
              "e2e_pageable": {"p50_ms": 6.4, "pcie_frac": 0.96}},
             {"config": "c5_8x1024_d2h", "pinned_d2h_ceiling_GBps": 56.9,
              "pageable": {"p50_ms": 0.75, "effective_GBps": 44.5, "pcie_frac": 0.78, "chunks": 8},
              "pinned": {"p50_ms": 0.65, "effective_GBps": 51.4, "pcie_frac": 0.9, "chunks": 2}},
             {"config": "c1", "N": 128, "e2e_latency_us_p50": 17.1, "e2e_latency_us_p95": 18.7},
             {"hbm_copy_GBps": 5000.0, "vector_copy_GBps": {"16MiB": 4900.0}}]
    path = tmp_path / "report.txt"
    path.write_text("\n".join(json.dumps(l) for l in lines) + "\n")
    bench.summarize_report(str(path))
    out = capsys.readouterr().out
    assert "**57.20 GB/s**" in out and "16MiB 4900 GB/s" in out
    assert "| c1 | transpose | 24.00 | 5600.0 | 0.700 | 1.3 | 0.9 | 1.2 | 0.96 |" in out
    assert "| c4 | stream | 26.00 | 6800.0 | 0.850 | 6.4 | 0.96 | - | - |" in out
    assert "| c5_8x1024_d2h | 0.75 | 44.5 | 0.78 | 0.65 | 51.4 | 0.9 | 8 |" in out
    assert "N=128: 17.1 / 18.7" in out
