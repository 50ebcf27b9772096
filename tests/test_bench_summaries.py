"""bench.py's profile summarizers on synthetic rocprofv3 output (CPU only).

The bench line's roofline.rocprof_mean_us and roofline.traffic are read from
files these summarizers write; a kernel renamed by a new template parameter
must not make them fall silent."""
import csv
import importlib.util
import json
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_tall_mode_reads_both_name_forms(bench):
    assert bench.tall_mode("void ltx25::tall_kernel<0>(ltx25::TallParams)") == 0
    assert bench.tall_mode("void ltx25::tall_kernel<0, false>") == 0
    assert bench.tall_mode("ltx25::tall_kernel<2, true>") == 2
    assert bench.tall_mode("ltx25::tall_kernel<1, false>") == 1
    assert bench.tall_mode("void ltx25::(anonymous namespace)::tall_w8_kernel(ltx25::TallParams)") == 2
    assert bench.tall_mode("ltx25::dequant_kernel<8>") is None
    assert bench.tall_mode("ltx25::mid_kernel<0, false>") is None


def test_kernel_grid_summary_writes_the_roofline_figures(bench, tmp_path, monkeypatch):
    up_grid, down_grid = sorted(bench.FFN_GRIDS, key=lambda g: bench.FFN_GRIDS[g] != "up")
    assert bench.FFN_GRIDS[up_grid] == "up" and bench.FFN_GRIDS[down_grid] == "down"
    rows = []
    t = 1_000_000
    # up 840 us and 842 us, down 770 us and 772 us (ns timestamps), plus an unrelated kernel
    for name, grid, dur_us in [("void ltx25::tall_kernel<0, false>(ltx25::TallParams)", up_grid, 840),
                               ("void ltx25::tall_kernel<0, false>(ltx25::TallParams)", up_grid, 842),
                               ("void ltx25::tall_kernel<0, false>(ltx25::TallParams)", down_grid, 770),
                               ("void ltx25::tall_kernel<0, false>(ltx25::TallParams)", down_grid, 772),
                               ("void ltx25::tall_kernel<2, false>(ltx25::TallParams)", up_grid, 999),
                               ("void ltx25::dequant_kernel<8>(int)", 4194304, 33)] * 4:
        rows.append({"Kernel_Name": name, "Grid_Size": grid, "Start_Timestamp": t,
                     "End_Timestamp": t + dur_us * 1000})
        t += 2_000_000
    trace = tmp_path / "run_kernel_trace.csv"
    with open(trace, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    roof = tmp_path / "roof.json"
    monkeypatch.setattr(bench, "ROOF_JSON", str(roof))
    # a summary of another trace (the audio leg's holds FFN launches too) leaves the figures alone
    bench.kernel_grid_summary(str(trace), str(tmp_path / "audio_kernel_stats.md"), "cmd", "note")
    assert not roof.exists()
    bench.kernel_grid_summary(str(trace), str(tmp_path / "roofline_kernel_stats.md"), "cmd", "note")
    got = json.loads(roof.read_text())
    assert got["up_us"] == pytest.approx(841.0)
    assert got["down_us"] == pytest.approx(771.0)
    assert got["mean_us"] == pytest.approx(806.0)
    flop = 2.0 * 8160 * 4096 * 16384
    assert got["tflops"] == pytest.approx(flop / 806e-6 / 1e12, abs=0.01)
    assert got["frac"] == pytest.approx(got["tflops"] / 2500.0, abs=1e-4)
