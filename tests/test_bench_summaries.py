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


def test_ceilings_summary_carries_rates_and_probe_kernels(bench, tmp_path):
    c = {"ceilings": {
        "read": {"qkv": {"bytes": 1600, "grid": 512, "best_us": 5.0, "best_GBps": 3200.0,
                         "median_GBps": 3000.0}},
        "mfma_stream": {"random_2wave": {"best_ms": 1.0, "TFLOPs": 2100.0,
                                         "frac_bf16_peak": 0.84}}}}
    js = tmp_path / "ceil.json"
    js.write_text("[bench] a log line\n" + json.dumps(c) + "\n")
    rows = [{"Kernel_Name": "ltx25::(anonymous namespace)::stream_read_kernel(int)",
             "Grid_Size_X": 131072, "Start_Timestamp": 0, "End_Timestamp": 5000},
            {"Kernel_Name": "void ltx25::(anonymous namespace)::mfma_stream_kernel<true>(int)",
             "Grid_Size_X": 131072, "Start_Timestamp": 0, "End_Timestamp": 1000000},
            {"Kernel_Name": "ltx25::dequant_kernel<8>(int)", "Grid_Size_X": 64,
             "Start_Timestamp": 0, "End_Timestamp": 1000}]
    trace = tmp_path / "run_kernel_trace.csv"
    with open(trace, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    out = tmp_path / "ceilings.md"
    bench.ceilings_summary(str(js), str(trace), str(out), "the command")
    text = out.read_text()
    assert "| qkv | 1600 | 512 | 5.00 | 3200 | 3000 |" in text
    assert "| random_2wave | 1.000 | 2100 | 0.840 |" in text
    assert "`ltx25::stream_read_kernel` | 131072 | 1 | 5.00" in text
    assert "mfma_stream_kernel<true>" in text
    assert "dequant_kernel" not in text
    assert "the command" in text


def test_skinny_phases_summary_matches_cases_to_trace_runs(bench, tmp_path):
    """Cases map, in order, to consecutive runs of the stamped kernel in the trace (two
    cases of one grid shape stay apart), each run's reductions to its case; the product
    kernel's launches are not counted."""
    ph = {p: 1.0 for p in bench.SKINNY_PHASES}
    def case(name, splits, wg):
        return {"name": name, "K": 2048, "N": 2048, "k_chunk": 0, "splits": splits,
                "workgroups": wg, "clock_GHz": 2.2,
                "span_us_median": 9.0, "wg_start_us_p90": 0.3, "max_workgroups_per_cu": 1,
                "phase_us_median": ph, "phase_us_p90": ph}
    c = {"skinny_phases": {"out k_chunk=plan": case("out", 1, 64),
                           "out k_chunk=512": case("out", 4, 256),
                           "ff_down k_chunk=plan": case("ff_down", 4, 256)}}
    js = tmp_path / "ph.json"
    js.write_text(json.dumps(c) + "\n")
    stamped = "void ltx25::(anonymous namespace)::skinny_kernel<8, {}, true>(ltx25::SParams)"
    rows, t = [], 0
    def add(name, gx, gy, us):
        nonlocal t
        rows.append({"Kernel_Name": name, "Grid_Size_X": gx, "Grid_Size_Y": gy,
                     "Start_Timestamp": t, "End_Timestamp": t + int(us * 1000)})
        t += 100000
    for _ in range(3):
        add(stamped.format("false"), 32768, 1, 10.0)
    add("void ltx25::(anonymous namespace)::skinny_kernel<8, false, false>(ltx25::SParams)",
        32768, 1, 50.0)
    for _ in range(3):
        add(stamped.format("true"), 32768, 4, 8.5)
        add("ltx25::splitk_reduce_kernel(float const*)", 64512, 1, 3.5)
    add("void at::native::fill_kernel(int)", 256, 1, 1.0)
    for _ in range(3):
        add(stamped.format("true"), 32768, 4, 13.5)
        add("ltx25::splitk_reduce_kernel(float const*)", 64512, 1, 4.0)
    trace = tmp_path / "run_kernel_trace.csv"
    with open(trace, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    out = tmp_path / "phases.md"
    bench.skinny_phases_summary(str(js), str(trace), str(out), "the command")
    text = out.read_text()
    assert "| out k_chunk=plan | 1 | 64 |" in text and "| 9.00 | 10.00 | - |" in text
    assert "| out k_chunk=512 | 4 | 256 |" in text and "| 9.00 | 8.50 | 3.50 |" in text
    assert "| ff_down k_chunk=plan | 4 | 256 |" in text and "| 9.00 | 13.50 | 4.00 |" in text
    assert "50.00" not in text and "the command" in text


def test_tall_phases_summary_rows_and_runs(bench, tmp_path):
    """Each case takes the rocprof durations of its own run of the stamped tile; the product
    tile's launches and other kernels split the runs and are not counted."""
    ph = {p: 2.0 for p in bench.TALL_PHASES}
    def case(tiles, clk):
        return {"tiles": tiles, "waves_per_tile": 8, "k_steps": 64, "span_us_median": 880.0,
                "tile_us_p50_p90": [100.0, 110.0], "tiles_per_cu": [8],
                "gap_us_p50_p90": [0.4, 0.7], "k_loop_cycles_per_step": 2318.0,
                "phase_us_median": ph, "phase_us_p90": ph,
                "per_xcc": {str(x): {"tiles_per_call": tiles // 8, "clock_GHz": clk,
                                     "last_end_us": 800.0 + x} for x in range(8)}}
    c = {"tall_phases": {"ffn_up (GELU)": case(2048, 1.7), "int8 N=4096": case(512, 1.4)}}
    js = tmp_path / "tp.json"
    js.write_text(json.dumps(c) + "\n")
    rows, t = [], 0
    def add(name, us):
        nonlocal t
        rows.append({"Kernel_Name": name, "Grid_Size_X": 1048576, "Grid_Size_Y": 1,
                     "Start_Timestamp": t, "End_Timestamp": t + int(us * 1000)})
        t += 2000000
    for _ in range(4):
        add("void ltx25::(anonymous namespace)::tall_kernel<0, false, true>(ltx25::TallParams)", 900.0)
    add("void ltx25::(anonymous namespace)::tall_kernel<0, false, false>(ltx25::TallParams)", 5.0)
    for _ in range(4):
        add("void ltx25::(anonymous namespace)::tall_kernel<1, false, true>(ltx25::TallParams)", 140.0)
    trace = tmp_path / "run_kernel_trace.csv"
    with open(trace, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    out = tmp_path / "tall.md"
    bench.tall_phases_summary(str(js), str(trace), str(out), "the command")
    text = out.read_text()
    assert "| ffn_up (GELU) | 2048 | 8 |" in text and "| 2318 | 880.0 | 900.0 |" in text
    assert "| int8 N=4096 | 512 | 8 |" in text and "| 2318 | 880.0 | 140.0 |" in text
    assert "| ffn_up (GELU) | 1.70 / 800 | 1.70 / 801 |" in text
    assert "5.0" not in text.split("Per XCD")[0].split("|---|")[-1] and "the command" in text
